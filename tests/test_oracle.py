"""The CPU oracle pinned before it is trusted (CPU only).

Each oracle function is held to checks chosen so that a plausible mistake fails one of
them, none of which retypes the oracle's own formula:

==========================  ====================================================================
oracle function             pinned by
==========================  ====================================================================
max_tiles                   the reference's golden values (crates/ops/src/moe/sort.rs:358-368)
moe_sort                    golden maps of crates/nn/tests/moe.rs:297-356; an independent
                            stable-argsort implementation on random routings (live counts,
                            windows, empty experts, skew)
topk_softmax                the exact 3-way tie of moe.rs:95-141; 512 experts / top 10
                            (moe.rs:143-181); scale + map (moe.rs:183-222); the pinned bf16
                            case of tests/python/kernels/moe/test_topk_softmax.py:104-157
                            (golden fixture); float64 brute force on random scores (ids equal
                            unless two float64 probabilities are within a few FP32 ulps);
                            NaN padding rows name no expert; the load counts
router exponential          float64 exp within 2 ulps over the softmax range; exact points
bf16 codec                  torch's bfloat16 conversion (independent implementation)
e4m3 codec                  torch's float8_e4m3fn on all 256 codes and on random values; the
                            exhaustive nearest-even search of moe.rs:568-582; saturation
gather / route / unpermute  float64 brute force of moe.rs:367-477 (`expert_by_hand`) on the
                            reference test's inputs; the window case of moe.rs:479-548
fp8 quantisers              dequantisation error within half an e4m3 step; block maxima at
                            +-448; float64 brute force of the block-scaled products over
                            dequantised values (the format has no reference: parity with the
                            reference is unpinned, the arithmetic is pinned)
moe_layer                   float64 composition of the pieces above on the tiny config;
                            invariance under a redistribution of the experts; the routing options
                            (router bias, slot map, load counts, expert window, live tokens) against
                            a float64 layer written from the reference tests' hand loops
router bias                 float64 brute force of x.W + b with one rounding; a crafted case where
                            rounding before the bias gives another bf16 value
gate (silu, gelu_tanh)      float64 closed forms and torch's gelu(approximate='tanh')
fp32 layer     float64 composition: ids equal, outputs within the reference tests'
                            FP32 tolerance
MX quantisers, products     E2M1 codes by brute force with ties to even; the E8M0 scale by its two
                            defining inequalities; MXFP8 against torch's e4m3 cast; float64 sums
                            of dequantised values (parity with the reference unpinned: NVFP4)
sigmoid_gated_add           the reference's own case (moe.rs:1865-1886); one rounding per type
==========================  ====================================================================
"""

import math

import numpy as np
import pytest

import oracle_lib as O

F32_TOLERANCE = 1e-4  # crates/nn/tests/moe.rs:29-30
BF16_TOLERANCE = 1e-2  # crates/nn/tests/moe.rs:32-34
FLT_EPSILON = float(np.finfo(np.float32).eps)


def assert_close(actual, expected, tolerance):
    """``nn_testing::assert_close`` (crates/nn/testing/src/values.rs:39-51)."""
    actual, expected = np.asarray(actual, np.float64), np.asarray(expected, np.float64)
    assert actual.shape == expected.shape
    bound = tolerance * np.maximum(np.abs(expected), 1.0)
    bad = np.abs(actual - expected) > bound
    assert not bad.any(), f"{bad.sum()} elements beyond the bound; first {np.argwhere(bad)[:3].tolist()}"


# ---- max_tiles ------------------------------------------------------------------------------------


def test_max_tiles_golden_values():
    assert O.max_tiles(2, 2, 4, 128) == 4
    assert O.max_tiles(1024, 8, 128, 128) == 191
    assert O.max_tiles(64, 8, 128, 128) == 131
    assert O.max_tiles(8192, 8, 128, 128) == 639


# ---- moe_sort ---------------------------------------------------------------------------------------


def sort_by_argsort(ids, top, local, offset, live, tile=128):
    """An independent statement: a stable argsort of the held routes by expert."""
    ids = np.asarray(ids, np.int64).reshape(-1)
    routes = np.arange(ids.size)
    live_routes = ids.size if live is None else live * top
    expert = ids - offset
    held = (routes < live_routes) & (expert >= 0) & (expert < local)
    counts = np.bincount(expert[held], minlength=local)
    tiles = -(-counts // tile)
    first_tile = np.concatenate([[0], np.cumsum(tiles)[:-1]])
    order = routes[held][np.argsort(expert[held], kind="stable")]
    e2p = np.where(routes < live_routes, -1, -2)
    rank = np.zeros(ids.size, np.int64)
    for e in range(local):
        members = order[expert[order] == e]
        rank[members] = first_tile[e] * tile + np.arange(members.size)
    e2p[held] = rank[held]
    t2e, t2l = [], []
    for e in range(local):
        for t in range(tiles[e]):
            t2e.append(e)
            t2l.append(min((first_tile[e] + t + 1) * tile, first_tile[e] * tile + counts[e]))
    padded = int(tiles.sum()) * tile
    p2e = np.full(padded, -1)
    p2e[e2p[held]] = routes[held]
    p2t = np.where(p2e >= 0, p2e // top, -1)
    return dict(tile_to_expert=np.array(t2e), tile_to_limit=np.array(t2l), expanded_to_permuted=e2p,
                permuted_to_expanded=p2e, permuted_to_token=p2t, total_padded_tokens=padded,
                num_non_exiting_tiles=int(tiles.sum()))


def assert_sort_matches(got, expected):
    tiles = expected["num_non_exiting_tiles"]
    padded = expected["total_padded_tokens"]
    assert int(got["num_non_exiting_tiles"][0]) == tiles
    assert int(got["total_padded_tokens"][0]) == padded
    np.testing.assert_array_equal(got["tile_to_expert"][:tiles], expected["tile_to_expert"])
    np.testing.assert_array_equal(got["tile_to_limit"][:tiles], expected["tile_to_limit"])
    n = expected["expanded_to_permuted"].size
    np.testing.assert_array_equal(got["expanded_to_permuted"][:n], expected["expanded_to_permuted"])
    np.testing.assert_array_equal(got["permuted_to_expanded"][:padded], expected["permuted_to_expanded"])
    np.testing.assert_array_equal(got["permuted_to_token"][:padded], expected["permuted_to_token"])


def test_sort_golden_tiles_spanning_experts_with_live_count_and_window():
    # crates/nn/tests/moe.rs:297-338
    tokens, top = 150, 2
    ids = np.array([[int(t >= 130), 3 - t % 2] for t in range(tokens)], np.int32)
    got = O.moe_sort(ids, local_experts=3, local_offset=0, live=148)
    assert got["tile_to_expert"][:4].tolist() == [0, 0, 1, 2]
    assert got["tile_to_limit"][:4].tolist() == [128, 130, 274, 458]
    assert got["expanded_to_permuted"][1] == -1, "token 0's second route is expert 3's"
    assert got["expanded_to_permuted"][2 * 148] == -2, "token 148 is not live"
    assert O.max_tiles(tokens, top, 3) == 5
    assert_sort_matches(got, sort_by_argsort(ids, top, 3, 0, 148))
    # Entries past the live tiles and rows keep what the buffers held.
    assert got["tile_to_expert"][4] == -7
    assert (got["permuted_to_expanded"][int(got["total_padded_tokens"][0]):] == -7).all()


def test_sort_golden_window_rebased():
    # crates/nn/tests/moe.rs:340-356
    ids = np.array([3, 1, 2, 0, 2, 3, 1, 1, 0, 2], np.int32).reshape(5, 2)
    got = O.moe_sort(ids, local_experts=2, local_offset=2)
    assert got["tile_to_expert"][:2].tolist() == [0, 1]
    assert_sort_matches(got, sort_by_argsort(ids, 2, 2, 2, None))


@pytest.mark.parametrize("seed", range(6))
def test_sort_matches_an_independent_argsort(seed):
    rng = np.random.default_rng(seed)
    tokens = int(rng.integers(1, 700))
    top = int(rng.integers(1, 9))
    experts = int(rng.integers(top, 160))
    zipf = rng.random() < 0.5
    if zipf:
        p = 1.0 / np.arange(1, experts + 1) ** 1.1
        ids = rng.choice(experts, size=(tokens, top), p=p / p.sum())
    else:
        ids = rng.integers(0, experts, size=(tokens, top))
    offset = int(rng.integers(0, experts))
    local = int(rng.integers(1, experts - offset + 1))
    live = None if rng.random() < 0.5 else int(rng.integers(0, tokens + 1))
    got = O.moe_sort(ids.astype(np.int32), local, offset, live)
    assert_sort_matches(got, sort_by_argsort(ids, top, local, offset, live))


# ---- the router -------------------------------------------------------------------------------------


def route_by_hand(scores, top, renormalize=True):
    """crates/nn/tests/moe.rs:64-93 in float64: one arg-max per pick, the lowest expert among equals."""
    scores = np.asarray(scores, np.float64)
    ids, weights = [], []
    for row in scores:
        shifted = np.exp(row - row.max())
        p = shifted / shifted.sum()
        picked = []
        for _ in range(top):
            best = None
            for e in range(row.size):
                if e in picked:
                    continue
                if best is None or p[e] > p[best]:
                    best = e
            picked.append(best)
        total = sum(p[e] for e in picked)
        ids.append(picked)
        weights.append([p[e] / max(total, FLT_EPSILON) if renormalize else p[e] for e in picked])
    return np.array(ids), np.array(weights)


def test_topk_exact_three_way_tie_resolves_by_ascending_id():
    tokens, experts, top = 4, 6, 3
    scores = O.sequence(tokens * experts, 21).reshape(tokens, experts)
    scores[1] = [0.5, 1.0, 1.0, -1.0, 1.0, 0.2]
    ids, weights = O.topk_softmax(scores, top)
    assert ids[1].tolist() == [1, 2, 4]
    want_ids, want_weights = route_by_hand(scores, top)
    np.testing.assert_array_equal(ids, want_ids)
    assert_close(weights, want_weights, F32_TOLERANCE)
    raw_ids, raw = O.topk_softmax(scores, top, renormalize=False)
    np.testing.assert_array_equal(raw_ids, want_ids)
    assert (raw.sum(axis=1) < 1.0).all()
    assert_close(raw / raw.sum(axis=1, keepdims=True), want_weights, F32_TOLERANCE)


def test_topk_ten_of_five_hundred_and_twelve():
    scores = O.sequence(3 * 512, 77).reshape(3, 512)
    ids, weights = O.topk_softmax(scores, 10)
    want_ids, want_weights = route_by_hand(scores, 10)
    np.testing.assert_array_equal(ids, want_ids)
    assert_close(weights, want_weights, F32_TOLERANCE)


def test_topk_scale_and_map_by_the_expert_s_own_id():
    scores = O.sequence(15, 22).reshape(3, 5)
    scale = np.array([0.5, 2.0, 1.5, 0.25, 3.0], np.float32)
    mapping = np.array([4, 2, 0, 1, 3], np.int32)
    ids, weights = O.topk_softmax(scores, 2, scale=scale, scale_kind=0, mapping=mapping)
    want_ids, want_weights = route_by_hand(scores, 2)
    np.testing.assert_array_equal(ids, mapping[want_ids])
    assert_close(weights, want_weights * scale[want_ids], F32_TOLERANCE)


def test_topk_pinned_bf16_case(golden_topk=None):
    data = np.load(__file__.replace("test_oracle.py", "golden/topk_pinned.npz"))
    ids, weights = O.topk_softmax(data["scores_bf16"], 8, score_kind=1)
    assert ids[0, 1] < ids[0, 2], "the exact tie of row 0 resolves by ascending id"
    np.testing.assert_array_equal(ids, data["ids"])
    # The operator's bound (crates/ops/src/moe/routing.rs:314-324): gamma_E + 4u, relative.
    u = 2.0**-24
    bound = 128 * u / (1 - 128 * u) + 4 * u
    rel = np.abs(weights - data["weights"]) / np.abs(data["weights"])
    assert (rel <= bound).all(), rel.max()


def test_topk_random_scores_agree_with_float64_except_at_float_ties():
    rng = np.random.default_rng(5)
    scores = O.bf16_decode(O.bf16_encode(rng.standard_normal((300, 128)).astype(np.float32)))
    ids, weights = O.topk_softmax(scores, 8)
    want_ids, want_weights = route_by_hand(scores, 8)
    mismatch = np.argwhere(ids != want_ids)
    for row, slot in mismatch:
        # Only probabilities equal to within a few FP32 ulps may order differently.
        x = scores[row].astype(np.float64)
        p = np.exp(x - x.max())
        p /= p.sum()
        a, b = p[ids[row, slot]], p[want_ids[row, slot]]
        assert abs(a - b) <= 8 * 2.0**-24 * max(a, b), (row, slot, a, b)
    assert_close(weights, want_weights, F32_TOLERANCE)


def test_topk_nan_row_names_no_expert_and_load_counts_live_rows():
    scores = O.sequence(5 * 16, 3).reshape(5, 16)
    scores[4] = np.nan
    load = np.zeros(16, np.int64)
    ids, _ = O.topk_softmax(scores, 4, load=load, live=3)
    assert not ((ids[4] >= 0) & (ids[4] < 16)).any()
    want_ids, _ = route_by_hand(scores[:4], 4)
    np.testing.assert_array_equal(ids[:4], want_ids)
    np.testing.assert_array_equal(load, np.bincount(want_ids[:3].ravel(), minlength=16))


def test_router_exponential_is_within_two_ulps_of_exp():
    xs = np.concatenate([np.linspace(-104.0, 0.0, 20011), np.linspace(-1.0, 1.0, 4001), [-87.0, -90.0, -100.0]])
    for x in xs.astype(np.float32):
        got = O.expf(float(x))
        want = math.exp(float(x))
        if want < 2.0**-126:  # subnormal results: absolute half-unit of the subnormal grid
            assert abs(got - want) <= 2.0**-149, (x, got, want)
        else:
            assert abs(got - want) <= 2 * 2.0**-23 * want, (x, got, want)
    assert O.expf(0.0) == 1.0
    assert O.expf(float("-inf")) == 0.0
    assert math.isnan(O.expf(float("nan")))


# ---- codecs -------------------------------------------------------------------------------------------


def test_bf16_codec_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(1)
    values = np.concatenate([rng.standard_normal(20000) * 10.0 ** rng.integers(-30, 30, 20000),
                             [0.0, -0.0, 1.0, 65504.0, 3.0e38, 1e-40, np.inf, -np.inf]]).astype(np.float32)
    want = torch.from_numpy(values).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(O.bf16_encode(values), want)
    np.testing.assert_array_equal(O.bf16_decode(want), torch.from_numpy(want.view(np.int16)).view(torch.bfloat16).float().numpy())


def e4m3_nearest(value):
    """crates/nn/tests/moe.rs:568-582: exhaustive nearest, the even byte of two equally near."""
    best = 0
    for byte in range(1, 0x7F):
        d, kept = abs(O.e4m3_decode(byte) - value), abs(O.e4m3_decode(best) - value)
        if d < kept or (d == kept and byte % 2 == 0):
            best = byte
    return best


def test_e4m3_decode_matches_torch_on_every_code():
    torch = pytest.importorskip("torch")
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = O.e4m3_decode_array(codes)
    nan = np.isnan(want)
    assert (np.isnan(got) == nan).all() and nan.sum() == 2
    np.testing.assert_array_equal(got[~nan], want[~nan])


def test_e4m3_encode_nearest_even_and_saturating():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(2)
    values = np.concatenate([rng.uniform(-448, 448, 4000), rng.standard_normal(4000) * 2.0 ** rng.integers(-12, 6, 4000)])
    values = values.astype(np.float32)
    # exact midpoints between neighbouring codes: ties go to the even code
    grid = O.e4m3_decode_array(np.arange(0, 0x7E, dtype=np.uint8))
    mids = ((grid[:-1].astype(np.float64) + grid[1:]) / 2).astype(np.float32)
    values = np.concatenate([values, mids, -mids])
    got = np.array([O.e4m3_encode(v) for v in values], np.uint8)
    want = torch.from_numpy(values).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(got, want)
    for v in list(mids[::7]) + list(values[:200]):
        code = e4m3_nearest(abs(float(v)))
        assert O.e4m3_encode(abs(float(v))) == code
    assert O.e4m3_encode(500.0) == 0x7E and O.e4m3_encode(-1e9) == 0xFE
    assert O.e4m3_encode(float("inf")) == 0x7E and O.e4m3_encode(464.0) == 0x7E
    assert O.e4m3_encode(2.0**-10) == 0 and O.e4m3_encode(2.0**-9) == 1


# ---- products and the combine --------------------------------------------------------------------------


def silu(x):
    return x / (1.0 + np.exp(-x))


def dense_expert(hidden, intermediate, seed):
    """crates/nn/tests/moe.rs:358-365, in bf16 (the device products read bf16)."""
    def q(v):
        return O.bf16_decode(O.bf16_encode(v))
    return [q(O.sequence(intermediate * hidden, seed)).reshape(intermediate, hidden),
            q(O.sequence(intermediate * hidden, seed + 1)).reshape(intermediate, hidden),
            q(O.sequence(hidden * intermediate, seed + 2)).reshape(hidden, intermediate)]


def expert_by_hand(x, expert):
    up, gate, down = (m.astype(np.float64) for m in expert)
    return down @ (silu(gate @ x) * (up @ x))


def stacks(experts):
    up_gate = np.stack([np.concatenate([e[0], e[1]]) for e in experts])
    down = np.stack([e[2] for e in experts])
    return O.bf16_encode(up_gate), O.bf16_encode(down)


def run_products(x_bits, up_gate_bits, down_bits, ids, weights, local, offset=0, live=None):
    tokens, top = ids.shape
    sort = O.moe_sort(ids, local, offset, live)
    rows = O.max_tiles(tokens, top, local) * 128
    gated = O.gather_gemm(x_bits, up_gate_bits, top, sort, rows, fill=0.0)
    products = O.route_gemm(O.bf16_encode(gated), down_bits, sort, fill=0.0)
    combined = O.moe_unpermute(O.bf16_encode(products), sort["expanded_to_permuted"][: tokens * top].reshape(tokens, top), weights)
    return sort, gated, products, combined


def test_products_and_combine_sum_each_token_s_experts():
    # crates/nn/tests/moe.rs:399-477
    tokens, top, hidden, intermediate = 5, 2, 8, 6
    experts = [dense_expert(hidden, intermediate, 30 + 3 * e) for e in range(4)]
    up_gate, down = stacks(experts)
    x = O.bf16_decode(O.bf16_encode(O.sequence(tokens * hidden, 25))).reshape(tokens, hidden)
    ids = np.array([3, 1, 2, 0, 2, 3, 1, 0, 0, 2], np.int32).reshape(tokens, top)
    weights = O.sequence(tokens * top, 26).reshape(tokens, top)
    sort, gated, products, combined = run_products(O.bf16_encode(x), up_gate, down, ids, weights, 4)
    e2p = sort["expanded_to_permuted"]
    for route in range(tokens * top):
        t, e, row = route // top, ids.reshape(-1)[route], e2p[route]
        up, gate, _ = (m.astype(np.float64) for m in experts[e])
        assert_close(gated[row], silu(gate @ x[t]) * (up @ x[t]), 1e-5)
        g = O.bf16_decode(O.bf16_encode(gated[row])).astype(np.float64)
        assert_close(products[row], experts[e][2].astype(np.float64) @ g, 1e-5)
        assert_close(products[row], expert_by_hand(x[t], experts[e]), BF16_TOLERANCE)
    expected = np.zeros((tokens, hidden))
    for route in range(tokens * top):
        t = route // top
        expected[t] += weights.reshape(-1)[route] * expert_by_hand(x[t], experts[ids.reshape(-1)[route]])
    assert_close(combined, expected, BF16_TOLERANCE)
    # the combine alone, in float64 over the rounded products
    pb = O.bf16_decode(O.bf16_encode(products)).astype(np.float64)
    exact = np.zeros((tokens, hidden))
    for route in range(tokens * top):
        exact[route // top] += weights.reshape(-1)[route] * pb[e2p[route]]
    assert_close(combined, exact, 1e-6)


def test_a_window_computes_its_own_experts_and_skips_the_rest():
    # crates/nn/tests/moe.rs:479-548
    tokens, top, hidden, intermediate = 4, 2, 8, 6
    experts = [dense_expert(hidden, intermediate, 50 + 3 * e) for e in range(4)]
    up_gate, down = stacks(experts[2:])
    x = O.bf16_decode(O.bf16_encode(O.sequence(tokens * hidden, 27))).reshape(tokens, hidden)
    ids = np.array([3, 1, 2, 0, 2, 3, 3, 2], np.int32).reshape(tokens, top)
    weights = O.sequence(tokens * top, 28).reshape(tokens, top)
    _, _, _, combined = run_products(O.bf16_encode(x), up_gate, down, ids, weights, 2, offset=2, live=3)
    expected = np.zeros((tokens, hidden))
    for route in range(tokens * top):
        t = route // top
        if t >= 3 or ids.reshape(-1)[route] < 2:
            continue
        expected[t] += weights.reshape(-1)[route] * expert_by_hand(x[t], experts[ids.reshape(-1)[route]])
    assert_close(combined, expected, BF16_TOLERANCE)
    assert (combined[3] == 0).all()


def test_unpermute_skips_absent_routes_and_reads_the_expanded_layout():
    rng = np.random.default_rng(3)
    tokens, top, hidden = 7, 3, 16
    routes = O.bf16_encode(rng.standard_normal((tokens * top, hidden)).astype(np.float32))
    e2p = rng.permutation(tokens * top).reshape(tokens, top).astype(np.int32)
    e2p[0, :] = -1
    e2p[2, 1] = -2
    w = rng.standard_normal((tokens, top)).astype(np.float32)
    r = O.bf16_decode(routes).astype(np.float64)
    for layout in (0, 1):
        got = O.moe_unpermute(routes, e2p, w, layout=layout)
        want = np.zeros((tokens, hidden))
        for t in range(tokens):
            for k in range(top):
                if e2p[t, k] >= 0:
                    want[t] += w[t, k] * r[e2p[t, k] if layout == 0 else t * top + k]
        assert_close(got, want, 1e-6)
        assert (got[0] == 0).all()


# ---- block-scaled fp8 ------------------------------------------------------------------------------------


def test_row_quantiser_error_and_maxima():
    rng = np.random.default_rng(4)
    x = O.bf16_encode((rng.standard_normal((9, 384)) * 10.0 ** rng.integers(-3, 3, (9, 1))).astype(np.float32))
    x[3, 128:256] = 0  # an all-zero group takes scale 1
    q, s = O.quantize_rows_fp8(x)
    xf = O.bf16_decode(x).astype(np.float64)
    deq = O.e4m3_decode_array(q).astype(np.float64) * np.repeat(s, 128, axis=1)
    step = np.repeat(s, 128, axis=1) * np.maximum(np.abs(xf) / np.repeat(s, 128, axis=1), 2.0**-6) * 2.0**-4
    assert (np.abs(deq - xf) <= step * 1.0001 + 1e-30).all()
    assert s[3, 1] == 1.0 and (q[3, 128:256] == 0).all()
    for r in range(9):
        for g in range(3):
            if s[r, g] != 1.0 or xf[r, g * 128:(g + 1) * 128].any():
                codes = q[r, g * 128:(g + 1) * 128]
                assert ((codes & 0x7F) == 0x7E).any()
                assert ((codes & 0x7F) <= 0x7E).all()


def test_block_quantiser_and_block_scaled_products():
    rng = np.random.default_rng(6)
    experts, hidden, intermediate, tokens, top = 3, 256, 128, 10, 2
    w1 = O.bf16_encode((rng.standard_normal((experts, 2 * intermediate, hidden)) * 0.05).astype(np.float32))
    w2 = O.bf16_encode((rng.standard_normal((experts, hidden, intermediate)) * 0.05).astype(np.float32))
    w1[1, 128:256, 0:128] = O.bf16_encode(np.full((128, 128), 3.0, np.float32))  # one loud block
    q1, s1 = O.quantize_blocks_fp8(w1)
    q2, s2 = O.quantize_blocks_fp8(w2)
    assert s1.shape == (experts, 2, 2) and s2.shape == (experts, 2, 1)
    assert s1[1, 1, 0] == np.float32(3.0) / np.float32(448.0)
    x = O.bf16_encode(rng.standard_normal((tokens, hidden)).astype(np.float32))
    xq, xs = O.quantize_rows_fp8(x)
    ids = rng.integers(0, experts, (tokens, top)).astype(np.int32)
    sort = O.moe_sort(ids, experts)
    rows = O.max_tiles(tokens, top, experts) * 128
    gated = O.gather_gemm_fp8(xq, xs, q1, s1, top, sort, rows, fill=0.0)
    dx = O.e4m3_decode_array(xq).astype(np.float64) * np.repeat(xs, 128, axis=1)
    dw1 = O.e4m3_decode_array(q1).astype(np.float64) * np.repeat(np.repeat(s1, 128, axis=1), 128, axis=2)
    dw2 = O.e4m3_decode_array(q2).astype(np.float64) * np.repeat(np.repeat(s2, 128, axis=1), 128, axis=2)
    e2p = sort["expanded_to_permuted"]
    for route in range(tokens * top):
        t, e, row = route // top, ids.reshape(-1)[route], e2p[route]
        up = dw1[e, :intermediate] @ dx[t]
        gate = dw1[e, intermediate:] @ dx[t]
        assert_close(gated[row], silu(gate) * up, 1e-5)
    gb = O.bf16_encode(gated)
    gq, gs = O.quantize_rows_fp8(gb)
    products = O.route_gemm_fp8(gq, gs, q2, s2, sort, fill=0.0)
    dg = O.e4m3_decode_array(gq).astype(np.float64) * np.repeat(gs, 128, axis=1)
    for route in range(tokens * top):
        e, row = ids.reshape(-1)[route], e2p[route]
        assert_close(products[row], dw2[e] @ dg[row], 1e-5)


# ---- the composed layer ---------------------------------------------------------------------------------------


def tiny_layer(seed=0):
    """T=16, H=256, E=8, top-2, I=128; x ~ N(0,1), weights ~ N(0, 0.02)."""
    T, H, E, K, I = 16, 256, 8, 2, 128
    x = O.bf16_encode(O.normal(T * H, seed * 10 + 1).reshape(T, H))
    router = O.bf16_encode(O.normal(E * H, seed * 10 + 2, 0.02).reshape(E, H))
    up_gate = O.bf16_encode(O.normal(E * 2 * I * H, seed * 10 + 3, 0.02).reshape(E, 2 * I, H))
    down = O.bf16_encode(O.normal(E * H * I, seed * 10 + 4, 0.02).reshape(E, H, I))
    return x, router, up_gate, down, K


def test_layer_is_the_float64_composition():
    x, router, up_gate, down, top = tiny_layer()
    out, ids, weights, _ = O.moe_layer(x, router, up_gate, down, top)
    xf = O.bf16_decode(x).astype(np.float64)
    scores = O.bf16_decode(O.bf16_encode((xf @ O.bf16_decode(router).astype(np.float64).T).astype(np.float32)))
    want_ids, want_weights = route_by_hand(scores, top)
    np.testing.assert_array_equal(ids, want_ids)
    assert_close(weights, want_weights, F32_TOLERANCE)
    w1 = O.bf16_decode(up_gate).astype(np.float64)
    w2 = O.bf16_decode(down).astype(np.float64)
    I = w1.shape[1] // 2
    expected = np.zeros_like(xf)
    for t in range(xf.shape[0]):
        for k in range(top):
            e = want_ids[t, k]
            h = silu(w1[e, I:] @ xf[t]) * (w1[e, :I] @ xf[t])
            expected[t] += want_weights[t, k] * (w2[e] @ h)
    got = O.bf16_decode(out).astype(np.float64)
    rel = np.abs(got - expected).max() / np.abs(expected).max()
    assert rel <= 2e-2 and np.abs(got - expected).mean() <= 1e-3


def test_layer_is_invariant_under_a_redistribution_of_the_experts():
    # crates/nn/tests/moe.rs:1071-1098: where the experts lie does not change the output.
    x, router, up_gate, down, top = tiny_layer(1)
    out, _, _, _ = O.moe_layer(x, router, up_gate, down, top)
    order = np.random.default_rng(0).permutation(router.shape[0])
    moved, _, _, _ = O.moe_layer(x, router[order], up_gate[order], down[order], top)
    # Re-stacking changes which rows share a tile, never a value: bit-identical unless two experts'
    # probabilities are equal (then the tie order by id changes the route order of the sum).
    np.testing.assert_array_equal(out, moved)


def test_sequence_is_the_reference_lcg_shape():
    # The input generator of the reference's tests (values.rs:53-66): 24-bit values in (-1, 1).
    s = O.sequence(1000, 0)
    assert s.min() >= -1.0 and s.max() < 1.0
    assert np.all(np.round((s + 1.0) * 2**23) == (s + 1.0) * 2**23)
    assert not np.array_equal(s, O.sequence(1000, 1))


# ---- the shared expert's join ---------------------------------------------------------------------


def test_sigmoid_gated_add_reference_case():
    """crates/nn/tests/moe.rs:1865-1886: 3 x 4 rows from sequence(.., 90) and sequence(.., 91), gates
    [0.5, -1.5, 2.0], against the closed form target + update / (1 + e^-gate) (float64 here)."""
    rows, width = 3, 4
    target = O.sequence(rows * width, 90).reshape(rows, width)
    update = O.sequence(rows * width, 91).reshape(rows, width)
    gate = np.array([0.5, -1.5, 2.0], dtype=np.float32)
    got = O.sigmoid_gated_add(target, update, gate, 0)
    want = target.astype(np.float64) + update.astype(np.float64) / (1.0 + np.exp(-gate.astype(np.float64)))[:, None]
    # One sigmoid (a few ulps), one product and one sum, in FP32.
    np.testing.assert_allclose(got, want, rtol=0, atol=8 * np.finfo(np.float32).eps * np.abs(want).max())
    # A zero update leaves the target exactly; a gate of -inf adds nothing, +inf adds the update.
    np.testing.assert_array_equal(O.sigmoid_gated_add(target, np.zeros_like(update), gate, 0), target)
    inf_gate = np.array([-np.inf, np.inf, 0.0], dtype=np.float32)
    got = O.sigmoid_gated_add(target, update, inf_gate, 0)
    np.testing.assert_array_equal(got[0], target[0])
    np.testing.assert_array_equal(got[1], target[1] + update[1])
    np.testing.assert_array_equal(got[2], target[2] + np.float32(0.5) * update[2])


def test_sigmoid_gated_add_rounds_once_into_bf16_and_f16():
    """The narrow types: the FP32 sum of the widened operands, rounded once (bf16 bits, f16 bits)."""
    rng = np.random.default_rng(3)
    t = rng.normal(size=(5, 24)).astype(np.float32)
    u = rng.normal(size=(5, 24)).astype(np.float32)
    g = rng.normal(size=5).astype(np.float32)
    tb, ub, gb = O.bf16_encode(t), O.bf16_encode(u), O.bf16_encode(g)
    got = O.sigmoid_gated_add(tb, ub, gb, 1)
    gd = O.bf16_decode(gb).astype(np.float32)
    s = (np.float32(1) / (np.float32(1) + np.exp(-gd).astype(np.float32))).astype(np.float32)
    want = O.bf16_encode(O.bf16_decode(tb) + s[:, None] * O.bf16_decode(ub))
    # One FP32 product and sum differ from numpy's float32 evaluation by at most one bf16 step at a
    # rounding boundary; equal almost everywhere.
    assert np.mean(got == want) > 0.97
    assert np.abs(got.astype(np.int32) - want.astype(np.int32)).max() <= 1
    th, uh, gh = t.astype(np.float16), u.astype(np.float16), g.astype(np.float16)
    got_h = O.sigmoid_gated_add(th.view(np.uint16), uh.view(np.uint16), gh.view(np.uint16), 2).view(np.float16)
    sh = 1.0 / (1.0 + np.exp(-gh.astype(np.float64)))
    want_h = (th.astype(np.float64) + sh[:, None] * uh.astype(np.float64)).astype(np.float16)
    assert np.abs(got_h.astype(np.float64) - want_h.astype(np.float64)).max() <= np.abs(want_h).max() * 2.0 ** -10


# ---- OCP MX (MXFP4 weights x MXFP8 activations) -----------------------------------------------------


def test_e2m1_codec_every_code_and_ties():
    """Every code round-trips; midpoints go to the even code; saturation at 6; signed zero."""
    table = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    for code in range(16):
        want = table[code & 7] * (-1.0 if code & 8 else 1.0)
        assert O.e2m1_decode(code) == want
        assert O.e2m1_encode(want) == code or (code == 8 and O.e2m1_encode(-0.0) == 8)
    ties = {0.25: 0.0, 0.75: 1.0, 1.25: 1.0, 1.75: 2.0, 2.5: 2.0, 3.5: 4.0, 5.0: 4.0}
    for value, want in ties.items():
        assert O.e2m1_decode(O.e2m1_encode(value)) == want, value
        assert O.e2m1_decode(O.e2m1_encode(-value)) == -want, value
    assert O.e2m1_decode(O.e2m1_encode(1e9)) == 6.0 and O.e2m1_decode(O.e2m1_encode(-7.0)) == -6.0
    # Nearest: brute force over a grid against the table.
    for value in np.linspace(-7.0, 7.0, 2801):
        got = O.e2m1_decode(O.e2m1_encode(value))
        best = min(abs(abs(value) - t) for t in table)
        assert abs(abs(got) - abs(value)) == best or abs(value) > 6.0


def test_mx_scale_is_the_smallest_power_without_saturation():
    rng = np.random.default_rng(11)
    for amax in np.concatenate([rng.lognormal(0.0, 8.0, 500), [1.0, 6.0, 448.0, 448.0 * 2 ** -20]]).astype(np.float32):
        for limit in (6.0, 448.0):
            e = O.mx_scale(amax, limit) - 127
            assert amax <= limit * 2.0 ** e, (amax, limit, e)
            assert amax > limit * 2.0 ** (e - 1), (amax, limit, e)
    assert O.mx_scale(0.0, 448.0) == 127 and O.mx_scale(float("inf"), 6.0) == 127
    # Blocks far below 2^-127: the exponent clamps at the smallest E8M0 power (byte 0), never the
    # NaN byte, and that power still holds them.
    for amax in (1.0e-38, 1.0e-40, 2.0 ** -149, 2.0 ** -126):
        for limit in (6.0, 448.0):
            assert O.mx_scale(amax, limit) == 0, (amax, limit)


def test_mxfp8_rows_match_torch_cast_under_the_scale():
    """codes = e4m3(x / 2^(s-127)) by torch's round-to-nearest-even cast, s the smallest power."""
    import torch

    rng = np.random.default_rng(12)
    x = (rng.standard_normal((7, 256)) * np.exp(rng.normal(0, 3, (7, 1)))).astype(np.float32)
    x[2, :32] = 0.0
    bits = O.bf16_encode(x)
    codes, scales = O.quantize_rows_mxfp8(bits)
    values = O.bf16_decode(bits).astype(np.float64)
    for r in range(7):
        for b in range(8):
            block = values[r, b * 32:(b + 1) * 32]
            assert scales[r, b] == O.mx_scale(np.abs(block).max(), 448.0)
            want = torch.from_numpy((block / O.mx_power(scales[r, b])).astype(np.float32)).to(torch.float8_e4m3fn)
            np.testing.assert_array_equal(codes[r, b * 32:(b + 1) * 32], want.view(torch.uint8).numpy())


def test_mxfp4_blocks_round_to_the_nearest_code():
    rng = np.random.default_rng(13)
    w = (rng.standard_normal((2, 4, 64)) * 0.02).astype(np.float32)
    bits = O.bf16_encode(w)
    packed, scales = O.quantize_blocks_mxfp4(bits)
    codes = O.e2m1_unpack(packed)
    values = O.bf16_decode(bits).astype(np.float64)
    table = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])
    for s in range(2):
        for n in range(4):
            for b in range(2):
                block = values[s, n, b * 32:(b + 1) * 32]
                power = O.mx_power(scales[s, n, b])
                assert np.abs(block).max() <= 6.0 * power
                for i, v in enumerate(block):
                    code = codes[s, n, b * 32 + i]
                    got = table[code & 7] * (-1 if code & 8 else 1)
                    assert abs(abs(got) - abs(v) / power) == np.abs(table - abs(v) / power).min()


def test_mx_products_against_float64():
    """FC1 / FC2 over MX operands equal float64 sums of the dequantised values (FP32 rounding)."""
    rng = np.random.default_rng(14)
    tokens, hidden, experts, top, intermediate = 12, 256, 4, 2, 128
    x = O.bf16_encode(rng.standard_normal((tokens, hidden)).astype(np.float32))
    w1 = O.bf16_encode((rng.standard_normal((experts, 2 * intermediate, hidden)) * 0.05).astype(np.float32))
    w2 = O.bf16_encode((rng.standard_normal((experts, hidden, intermediate)) * 0.05).astype(np.float32))
    ids = np.stack([rng.choice(experts, top, replace=False) for _ in range(tokens)]).astype(np.int32)
    sort = O.moe_sort(ids, experts)
    rows = O.max_tiles(tokens, top, experts) * 128
    xq, xs = O.quantize_rows_mxfp8(x)
    q1, s1 = O.quantize_blocks_mxfp4(w1)
    q2, s2 = O.quantize_blocks_mxfp4(w2)
    gated = O.gather_gemm_mx(xq, xs, q1, s1, top, sort, rows, fill=0.0)
    dx = O.e4m3_decode_array(xq) * np.repeat(O.mx_power(xs), 32, axis=1)
    table = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0])
    d1 = table[O.e2m1_unpack(q1)] * np.repeat(O.mx_power(s1), 32, axis=2)
    d2 = table[O.e2m1_unpack(q2)] * np.repeat(O.mx_power(s2), 32, axis=2)
    p2e = sort["permuted_to_expanded"]
    t2e, t2l = sort["tile_to_expert"], sort["tile_to_limit"]
    for t in range(int(sort["num_non_exiting_tiles"][0])):
        for p in range(t * 128, t2l[t]):
            token, e = p2e[p] // top, t2e[t]
            h = d1[e] @ dx[token]
            want = h[intermediate:] / (1 + np.exp(-h[intermediate:])) * h[:intermediate]
            np.testing.assert_allclose(gated[p], want, rtol=1e-4, atol=1e-5 * np.abs(h).max())
    gq, gs = O.quantize_rows_mxfp8(O.bf16_encode(gated))
    products = O.route_gemm_mx(gq, gs, q2, s2, sort, fill=0.0)
    dg = O.e4m3_decode_array(gq) * np.repeat(O.mx_power(gs), 32, axis=1)
    for t in range(int(sort["num_non_exiting_tiles"][0])):
        for p in range(t * 128, t2l[t]):
            want = d2[t2e[t]] @ dg[p]
            np.testing.assert_allclose(products[p], want, rtol=1e-4, atol=1e-5 * np.abs(want).max())


# ---- router bias, the gelu_tanh gate, the f32 path and the layer's routing options ---------------------


def test_router_bias_enters_the_fp32_sum_before_the_one_rounding():
    """Float64 brute force: bf16(x.W + b) within half a bf16 step of the exact value; and a crafted
    case where rounding the product first and adding the bias after gives another bf16 value."""
    rng = np.random.default_rng(3)
    x = O.bf16_encode(rng.standard_normal((40, 256)).astype(np.float32))
    w = O.bf16_encode((rng.standard_normal((24, 256)) * 0.02).astype(np.float32))
    bias = (-1.1 * np.log(np.arange(24) + 1.0)).astype(np.float32)
    got = O.bf16_decode(O.router_gemm(x, w, bias)).astype(np.float64)
    exact = O.bf16_decode(x).astype(np.float64) @ O.bf16_decode(w).astype(np.float64).T + bias
    magnitude = np.abs(O.bf16_decode(x).astype(np.float64)) @ np.abs(O.bf16_decode(w).astype(np.float64)).T
    assert (np.abs(got - exact) <= np.abs(exact) * 2.0**-8 + 2.0**-22 * (magnitude + np.abs(bias))).all()
    # x.W = 1 + 2^-9 (between two bf16 values, 1 and 1 + 2^-7, nearer 1), bias = 2^-8 + 2^-10:
    # once-rounded bf16(1 + 2^-8 + 2^-9 + 2^-10) = 1 + 2^-7; rounded twice, bf16(1 + 2^-8 + 2^-10) = 1.
    xs = O.bf16_encode(np.array([[1.0, 2.0**-9]], np.float32))
    ws = O.bf16_encode(np.array([[1.0, 1.0]], np.float32))
    once = O.bf16_decode(O.router_gemm(xs, ws, np.array([2.0**-8 + 2.0**-10], np.float32)))
    assert once[0, 0] == 1.0 + 2.0**-7
    assert O.bf16_decode(O.router_gemm(xs, ws))[0, 0] == 1.0  # the product alone rounds down
    f32 = O.router_gemm_f32(O.bf16_decode(xs), O.bf16_decode(ws), np.array([2.0**-8 + 2.0**-10], np.float32))
    assert f32[0, 0] == np.float32(1.0 + 2.0**-8 + 2.0**-9 + 2.0**-10)  # f32 scores: no rounding


def test_gelu_tanh_gate_is_pytorch_s_tanh_approximation():
    """crates/nn/src/functional/activation.rs:62-71: 0.5x(1 + tanh(sqrt(2/pi)(x + 0.044715x^3))),
    checked against float64 and torch's gelu(approximate='tanh'); silu against float64."""
    import torch

    xs = np.concatenate([np.linspace(-12, 12, 2001), [0.0, -0.0, 1e-30, -1e-30, 30.0, -30.0]]).astype(np.float32)
    got = np.array([O.gate_activation(float(v), 1) for v in xs], np.float64)
    x64 = xs.astype(np.float64)
    want = 0.5 * x64 * (1 + np.tanh(math.sqrt(2 / math.pi) * (x64 + 0.044715 * x64**3)))
    # FP32 evaluation: a few ulps of the envelope |x| (1 + tanh cancels for large negative x).
    envelope = 8 * 2.0**-24 * np.maximum(np.abs(x64), 2.0**-10)
    assert (np.abs(got - want) <= envelope).all()
    torch_values = torch.nn.functional.gelu(torch.from_numpy(xs), approximate="tanh").numpy().astype(np.float64)
    assert (np.abs(got - torch_values) <= envelope).all()
    got_silu = np.array([O.gate_activation(float(v), 0) for v in xs], np.float64)
    assert (np.abs(got_silu - silu(x64)) <= 4 * 2.0**-24 * np.maximum(np.abs(silu(x64)), 2.0**-10)).all()
    # The two gates are different functions (gelu_tanh(1) = 0.8412, silu(1) = 0.7311).
    assert abs(O.gate_activation(1.0, 1) - 0.8411920) < 1e-6 and abs(O.gate_activation(1.0, 0) - 0.7310586) < 1e-6


def tiny_layer_f32(seed=0):
    """BASELINE configs[0] as stated: fp32, T=16, H=256, E=8, top-2, I=128; x ~ N(0,1), every weight
    ~ N(0, 0.02), from seed 0 (the oracle's SplitMix64 -> Box-Muller normals)."""
    T, H, E, K, I = 16, 256, 8, 2, 128
    x = O.normal(T * H, seed * 10 + 1).reshape(T, H).astype(np.float32)
    router = O.normal(E * H, seed * 10 + 2, 0.02).reshape(E, H).astype(np.float32)
    up_gate = O.normal(E * 2 * I * H, seed * 10 + 3, 0.02).reshape(E, 2 * I, H).astype(np.float32)
    down = O.normal(E * H * I, seed * 10 + 4, 0.02).reshape(E, H, I).astype(np.float32)
    return x, router, up_gate, down, K


def layer_by_hand(x, router, up_gate, down, top, bias=None, mapping=None, window=None, live=None,
                  activation=0, score_round=None):
    """MoE::routed in float64 from the reference's tests' definitions (route_by_hand,
    expert_by_hand of crates/nn/tests/moe.rs:64-93, 367-377): each held route's weighted expert
    output, summed; tokens past the live count give zero."""
    x = np.asarray(x, np.float64)
    scores = x @ np.asarray(router, np.float64).T
    if bias is not None:
        scores = scores + bias
    if score_round is not None:
        scores = score_round(scores)
    ids, weights = route_by_hand(scores, top)
    w1 = np.asarray(up_gate, np.float64)
    w2 = np.asarray(down, np.float64)
    I = w1.shape[1] // 2
    offset, local = (0, w1.shape[0]) if window is None else window
    out = np.zeros_like(x)
    slots = ids if mapping is None else np.asarray(mapping)[ids]
    for t in range(x.shape[0]):
        if live is not None and t >= live:
            continue
        for k in range(top):
            e = slots[t, k] - offset
            if not 0 <= e < local:
                continue
            g = w1[e, I:] @ x[t]
            gate = silu(g) if activation == 0 else 0.5 * g * (1 + np.tanh(math.sqrt(2 / math.pi) * (g + 0.044715 * g**3)))
            out[t] += weights[t, k] * (w2[e] @ (gate * (w1[e, :I] @ x[t])))
    return out, slots, weights


def test_f32_layer_is_the_float64_composition():
    """configs[0] in fp32 (the CPU reference path rounds nothing): ids equal, weights and outputs
    within the reference tests' FP32 tolerance (crates/nn/tests/moe.rs:29-30)."""
    x, router, up_gate, down, top = tiny_layer_f32()
    out, ids, weights, _, scores = O.moe_layer(x, router, up_gate, down, top, scores=True)
    assert out.dtype == np.float32 and scores.dtype == np.float32
    want, want_ids, want_weights = layer_by_hand(x, router, up_gate, down, top)
    np.testing.assert_array_equal(ids, want_ids)
    assert_close(weights, want_weights, F32_TOLERANCE)
    assert_close(scores, x.astype(np.float64) @ router.astype(np.float64).T, F32_TOLERANCE)
    assert_close(out, want, F32_TOLERANCE)
    # gelu_tanh as the gate.
    out_g, _, _, _ = O.moe_layer(x, router, up_gate, down, top, activation=1)
    want_g, _, _ = layer_by_hand(x, router, up_gate, down, top, activation=1)
    assert_close(out_g, want_g, F32_TOLERANCE)
    assert np.abs(want_g - want).max() > 1e-3, "the gates differ on these inputs"


def test_layer_routing_options_are_the_float64_composition():
    """What MoE::routed passes beyond the rows (crates/nn/src/modules/moe.rs:650-671, 770-775): the
    router bias, the slot map, the expert load of the live rows, the live count and the local
    window - each against the float64 composition in bf16."""
    T, H, E, K, I = 48, 256, 16, 4, 128
    rng = np.random.default_rng(7)
    x = O.bf16_encode(rng.standard_normal((T, H)).astype(np.float32))
    router = O.bf16_encode((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
    up_gate = O.bf16_encode((rng.standard_normal((E, 2 * I, H)) * 0.02).astype(np.float32))
    down = O.bf16_encode((rng.standard_normal((E, H, I)) * 0.02).astype(np.float32))
    bias = (-1.1 * np.log(np.arange(E) + 1.0)).astype(np.float32)
    mapping = rng.permutation(E).astype(np.int32)
    window = (4, 9)
    live = 40
    load = np.zeros(E, np.int64)
    out, ids, weights, _, scores = O.moe_layer(
        x, router, up_gate[4:13], down[4:13], K, router_bias=bias, mapping=mapping, load=load, live=live,
        window=window, scores=True)
    xf = O.bf16_decode(x).astype(np.float64)
    rf = O.bf16_decode(router).astype(np.float64)
    np.testing.assert_array_equal(scores, O.router_gemm(x, router, bias))
    bf = lambda v: O.bf16_decode(O.bf16_encode(v.astype(np.float32))).astype(np.float64)  # noqa: E731
    # Score rounding as the layer rounds (the float64 sum rounded once into bf16).
    want, want_ids, want_weights = layer_by_hand(
        xf, rf, O.bf16_decode(up_gate[4:13]), O.bf16_decode(down[4:13]), K, bias=bias, mapping=mapping,
        window=window, live=live, score_round=bf)
    np.testing.assert_array_equal(ids, want_ids)
    assert_close(weights, want_weights, F32_TOLERANCE)
    got = O.bf16_decode(out).astype(np.float64)
    assert (got[live:] == 0).all()
    rel = np.abs(got - want).max() / np.abs(want).max()
    assert rel <= 2e-2 and np.abs(got - want).mean() <= 1e-3, rel
    # The load counts every live route by its router expert (before the map).
    unmapped = np.argsort(mapping)[ids[:live]]
    np.testing.assert_array_equal(load, np.bincount(unmapped.ravel(), minlength=E))
    # The bias skews the routing toward low router experts.
    assert np.bincount(unmapped.ravel(), minlength=E)[:4].sum() > np.bincount(unmapped.ravel(), minlength=E)[-4:].sum()

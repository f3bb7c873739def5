"""topk_softmax and moe_sort on the MI355X against the oracle: bit-exact.

The router's probabilities are computed by the same IEEE operations in the same order on
both sides (the reference kernel's lane order, the library's own exponential), so ids
*and* weights must agree bit for bit; the sort is integer work and must agree bit for bit
on every entry it writes and leave every other entry untouched (buffers are pre-filled
with a sentinel, as tests/python/kernels/moe/test_moe_sort.py:47-50 does).
"""

import ctypes

import numpy as np
import pytest
import torch

import oracle_lib as O
from gpu_helpers import announce, bf16_bits, bf16_values, to_bf16, zipf_bias
from uniserve_moe import ops

pytestmark = pytest.mark.gpu


def route_both(device, scores_host, kind, top, renormalize=True, scale=None, scale_kind=-1, mapping=None,
               live=None, with_load=False):
    """The device router and the oracle on the same host scores."""
    if kind == 1:
        scores = to_bf16(scores_host, device)
    else:
        scores = torch.from_numpy(scores_host).to(device)
    experts = scores.shape[1]
    load = torch.zeros(experts, dtype=torch.int64, device=device) if with_load else None
    dev_scale = None if scale is None else torch.from_numpy(scale).to(device)
    dev_map = None if mapping is None else torch.from_numpy(mapping).to(device)
    dev_live = None if live is None else torch.tensor([live], dtype=torch.int32, device=device)
    ids, weights = ops.topk_softmax(scores, top, renormalize, dev_scale, dev_map, dev_live, load)
    torch.cuda.synchronize()
    host_load = np.zeros(experts, np.int64) if with_load else None
    want_ids, want_weights = O.topk_softmax(scores_host, top, renormalize, score_kind=kind, scale=scale,
                                            scale_kind=scale_kind, mapping=mapping, live=live, load=host_load)
    return (ids.cpu().numpy(), weights.cpu().numpy(), None if load is None else load.cpu().numpy(),
            want_ids, want_weights, host_load)


@pytest.mark.parametrize("experts,top,tokens", [(128, 8, 64), (128, 8, 8192), (8, 2, 16), (512, 10, 37),
                                                 (60, 4, 5), (1024, 32, 9), (1, 1, 3)])
def test_router_is_bit_exact_with_the_oracle(device, experts, top, tokens):
    announce("topk", experts, top, tokens)
    rng = np.random.default_rng(experts * 1000 + top)
    scores = O.bf16_encode((rng.standard_normal((tokens, experts)) * 2.0).astype(np.float32))
    ids, weights, _, want_ids, want_weights, _ = route_both(device, scores, 1, top)
    np.testing.assert_array_equal(ids, want_ids)
    np.testing.assert_array_equal(weights.view(np.uint32), want_weights.view(np.uint32))


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_router_float_scores_without_renormalisation(device, dtype):
    announce("topk float scores", dtype)
    rng = np.random.default_rng(11)
    scores = rng.standard_normal((300, 128)).astype(dtype)
    scores[7, :] = scores[7, 0]  # a whole row tied: ids 0..7 in order
    kind = 0 if dtype == np.float32 else 2
    for renormalize in (True, False):
        ids, weights, _, want_ids, want_weights, _ = route_both(device, scores, kind, 8, renormalize)
        np.testing.assert_array_equal(ids, want_ids)
        np.testing.assert_array_equal(weights.view(np.uint32), want_weights.view(np.uint32))
        assert ids[7].tolist() == list(range(8))


def test_router_scale_map_nan_row_and_load(device):
    announce("topk scale/map/nan/load")
    data = np.load(__file__.replace("test_gpu_router_sort.py", "golden/topk_pinned.npz"))
    scores = data["scores_bf16"].copy()
    scores[-1, :] = 0x7FC0  # a NaN padding row
    experts = scores.shape[1]
    mapping = np.arange(experts - 1, -1, -1, dtype=np.int32)
    scale = np.linspace(0.5, 2.0, experts).astype(np.float32)
    ids, weights, load, want_ids, want_weights, want_load = route_both(
        device, scores, 1, 8, scale=scale, scale_kind=0, mapping=mapping, live=3, with_load=True)
    np.testing.assert_array_equal(ids, want_ids)
    np.testing.assert_array_equal(weights[:-1].view(np.uint32), want_weights[:-1].view(np.uint32))
    np.testing.assert_array_equal(load, want_load)
    assert not ((ids[-1] >= 0) & (ids[-1] < experts)).any(), "the padding row names an expert"
    np.testing.assert_array_equal(ids[:-1], mapping[data["ids"][:-1]])


def test_router_pinned_case(device):
    announce("topk pinned")
    data = np.load(__file__.replace("test_gpu_router_sort.py", "golden/topk_pinned.npz"))
    ids, weights = ops.topk_softmax(to_bf16(data["scores_bf16"], device), 8)
    np.testing.assert_array_equal(ids.cpu().numpy(), data["ids"])
    u = 2.0**-24
    bound = 128 * u / (1 - 128 * u) + 4 * u
    assert (np.abs(weights.cpu().numpy() - data["weights"]) <= bound * data["weights"]).all()


def test_router_code_object_launched_by_name(device):
    """The reference's launch path: load the module, find `uniserve_topk_softmax`, launch its 14
    words on ceil(rows / warps) blocks of warps * 32 threads (crates/ops/src/moe/routing.rs:240-301)."""
    announce("topk code object")
    from uniserve_moe.abi import code_object_path

    hip = ctypes.CDLL("libamdhip64.so")
    module = ctypes.c_void_p()
    assert hip.hipModuleLoad(ctypes.byref(module), str(code_object_path()).encode()) == 0
    function = ctypes.c_void_p()
    assert hip.hipModuleGetFunction(ctypes.byref(function), module, b"uniserve_topk_softmax") == 0
    rng = np.random.default_rng(3)
    rows, experts, top, warps = 45, 128, 8, 4
    host = O.bf16_encode(rng.standard_normal((rows, experts)).astype(np.float32))
    scores = to_bf16(host, device)
    ids = torch.full((rows, top), -1, dtype=torch.int32, device=device)
    weights = torch.zeros((rows, top), dtype=torch.float32, device=device)
    load = torch.zeros(experts, dtype=torch.int64, device=device)
    values = [ctypes.c_void_p(scores.data_ptr()), ctypes.c_int32(1), ctypes.c_int64(experts), ctypes.c_int32(rows),
              ctypes.c_int32(experts), ctypes.c_int32(top), ctypes.c_int32(1), ctypes.c_void_p(0), ctypes.c_int32(-1),
              ctypes.c_void_p(ids.data_ptr()), ctypes.c_void_p(weights.data_ptr()), ctypes.c_void_p(0),
              ctypes.c_void_p(0), ctypes.c_void_p(load.data_ptr())]
    params = (ctypes.c_void_p * len(values))(*[ctypes.cast(ctypes.pointer(v), ctypes.c_void_p) for v in values])
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    grid = (rows + warps - 1) // warps
    status = hip.hipModuleLaunchKernel(function, grid, 1, 1, warps * 32, 1, 1, 0, stream, params, None)
    assert status == 0
    torch.cuda.synchronize()
    hip.hipModuleUnload(module)
    host_load = np.zeros(experts, np.int64)
    want_ids, want_weights = O.topk_softmax(host, top, score_kind=1, load=host_load)
    np.testing.assert_array_equal(ids.cpu().numpy(), want_ids)
    np.testing.assert_array_equal(weights.cpu().numpy().view(np.uint32), want_weights.view(np.uint32))
    np.testing.assert_array_equal(load.cpu().numpy(), host_load)


# ---- moe_sort ------------------------------------------------------------------------------------------


def sort_both(device, ids_host, experts, local=None, live=None):
    tokens, top = ids_host.shape
    start, end = (0, experts) if local is None else local
    ids = torch.from_numpy(ids_host).to(device)
    weights = torch.rand((tokens, top), device=device)
    live_t = None if live is None else torch.tensor([live], dtype=torch.int32, device=device)
    maps = ops.moe_sort(ids, weights, experts, (start, end), live_t)
    torch.cuda.synchronize()
    got = maps.cpu().numpy()
    want = O.moe_sort(ids_host, end - start, start, live)
    return got, want


def assert_sort_equal(got, want, tokens, top):
    names = ["tile_to_expert", "tile_to_limit", "expanded_to_permuted", "permuted_to_expanded",
             "permuted_to_token", "total_padded_tokens", "num_non_exiting_tiles"]
    for row, name in enumerate(names):
        expected = want[name]
        np.testing.assert_array_equal(got[row][: expected.size], expected, err_msg=name)
        # Nothing past what the sort writes is touched.
        assert (got[row][expected.size:] == -7).all(), name


@pytest.mark.parametrize("local,offset,live", [(128, 0, None), (128, 0, 40), (64, 32, None)])
def test_sort_reference_cases(device, local, offset, live):
    """tests/python/kernels/moe/test_moe_sort.py:180-277: T=64, top 8, E=128, tile 128."""
    announce("sort reference case", local, offset, live)
    torch.manual_seed(0)
    ids = torch.randint(0, 128, (64, 8), dtype=torch.int32).numpy()
    got, want = sort_both(device, ids, 128, (offset, offset + local), live)
    assert_sort_equal(got, want, 64, 8)


@pytest.mark.parametrize("tokens,top,experts,skew,live", [
    (8192, 8, 128, "zipf", None), (8192, 8, 128, "uniform", 5000), (4096, 8, 128, "one", None),
    (16, 2, 8, "uniform", None), (1, 8, 128, "uniform", None), (513, 8, 128, "zipf", 513),
    (3000, 6, 60, "uniform", 2999), (700, 1, 1, "one", None), (20000, 4, 300, "zipf", 19000)])
def test_sort_is_bit_exact(device, tokens, top, experts, skew, live):
    announce("sort", tokens, top, experts, skew, live)
    rng = np.random.default_rng(tokens + top + experts)
    if skew == "zipf":
        p = np.exp(zipf_bias(experts).astype(np.float64))
        ids = rng.choice(experts, size=(tokens, top), p=p / p.sum())
    elif skew == "one":
        ids = np.zeros((tokens, top), np.int64)
    else:
        ids = rng.integers(0, experts, (tokens, top))
    got, want = sort_both(device, ids.astype(np.int32), experts, None, live)
    assert_sort_equal(got, want, tokens, top)


@pytest.mark.parametrize("tokens,top,experts,window,live", [
    # The one-launch path (moe_sort_kernel): at most 4096 routes over more experts than the
    # one-workgroup path keeps (> 512 local experts)...
    (500, 8, 640, None, None), (512, 8, 1100, (100, 700), 500), (4096, 1, 860, None, 4000),
    # ...and above 4096 routes over more local experts than the split path's chunks hold (> 1024);
    # those need more LDS than a workgroup has, so the entry refuses them (tested on the CPU).
])
def test_sort_one_launch_path_is_bit_exact(device, tokens, top, experts, window, live):
    announce("sort one-launch path", tokens, top, experts, window, live)
    rng = np.random.default_rng(tokens + experts)
    ids = rng.integers(0, experts, (tokens, top)).astype(np.int32)
    local = None if window is None else (window[0], window[0] + window[1])
    got, want = sort_both(device, ids, experts, local, live)
    assert_sort_equal(got, want, tokens, top)


def test_sort_of_a_window_with_out_of_range_ids(device):
    announce("sort window with foreign ids")
    rng = np.random.default_rng(9)
    ids = rng.integers(-3, 140, (5000, 8)).astype(np.int32)  # ids outside the vocabulary are not held
    got, want = sort_both(device, ids, 140, (20, 100), 4900)
    assert_sort_equal(got, want, 5000, 8)


PREFILL_FRONT = {
    # name: tokens, hidden, experts, top, weights, zipf, window, live, map
    "bf16 30B 8192 zipf": (8192, 2048, 128, 8, "bf16", True, None, None, False),
    "fp8 30B 2048, map + load + live": (2048, 2048, 128, 8, "f8e4m3", False, None, 2000, True),
    "fp8 235B 4096 zipf": (4096, 4096, 128, 8, "f8e4m3", True, None, None, False),
    "mx 30B 2048 window": (2048, 2048, 128, 8, "f4e2m1", False, (8, 112), None, False),
    "bf16 60 experts, 2000 tokens": (2000, 256, 60, 4, "bf16", False, None, 1999, True),
}


@pytest.mark.parametrize("case", list(PREFILL_FRONT))
def test_prefill_front_is_the_separate_operators(device, case):
    """At prefill sizes the layer computes the router scores, topk_softmax and (e4m3, MXFP4) the
    hidden rows' quantisation in one launch. Against the separate operators on the same inputs:
    the scores are the oracle's router within one bf16 step (>= 99% bit for bit: FP32 sums in
    another order), and, given the layer's own scores, the ids, weights and expert load are the
    topk_softmax entry's bit for bit, the seven maps the moe_sort entry's, the hidden codes and
    scales the stand-alone quantiser's, and every held route's row of the route-major scale table
    its token's scales."""
    tokens, hidden, experts, top, wdtype, zipf, window, live, with_map = PREFILL_FRONT[case]
    announce("prefill front", case)
    intermediate = 256
    g = torch.Generator(device=device).manual_seed(17)
    x = (torch.randn((tokens, hidden), generator=g, device=device)).to(torch.bfloat16)
    router = (torch.randn((experts, hidden), generator=g, device=device) * 0.02).to(torch.bfloat16)
    bias = torch.from_numpy(zipf_bias(experts)).to(device) if zipf else None
    local_experts = experts if window is None else window[1]
    up_gate = (torch.randn((local_experts, 2 * intermediate, hidden), generator=g, device=device) * 0.02).to(torch.bfloat16)
    down = (torch.randn((local_experts, hidden, intermediate), generator=g, device=device) * 0.02).to(torch.bfloat16)
    kw = {}
    if wdtype == "f8e4m3":
        q1, s1 = O.quantize_blocks_fp8(bf16_bits(up_gate))
        q2, s2 = O.quantize_blocks_fp8(bf16_bits(down))
    elif wdtype == "f4e2m1":
        q1, s1 = O.quantize_blocks_mxfp4(bf16_bits(up_gate))
        q2, s2 = O.quantize_blocks_mxfp4(bf16_bits(down))
    if wdtype != "bf16":
        d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
        up_gate, down = d(q1), d(q2)
        kw = dict(up_gate_scales=d(s1), down_scales=d(s2))
    rng = np.random.default_rng(5)
    mapping = torch.from_numpy(rng.permutation(experts).astype(np.int32)).to(device) if with_map else None
    load = torch.zeros(experts, dtype=torch.int64, device=device)
    live_t = None if live is None else torch.tensor([live], dtype=torch.int32, device=device)
    layer = ops.MoeLayer(hidden, experts, top, intermediate, tokens, weight_dtype=wdtype)
    layer(x, router, up_gate, down, router_bias=bias, live_tokens=live_t, mapping=mapping, load=load, window=window,
          **kw)
    torch.cuda.synchronize()

    scores = layer.view("scores", torch.bfloat16, (tokens, experts)).clone()
    want_scores = O.router_gemm(bf16_bits(x), bf16_bits(router), None if bias is None else zipf_bias(experts))
    got_bits = bf16_bits(scores)
    assert (got_bits == want_scores).mean() > 0.99
    # Each side's FP32 sum is within n u sum|x w| of the exact one, then rounded once to bf16.
    magnitude = np.abs(bf16_values(x)) @ np.abs(bf16_values(router)).T
    want_values = O.bf16_decode(want_scores).astype(np.float64)
    bound = 2.0**-7 * np.abs(want_values) + 2.0 * hidden * 2.0**-24 * magnitude
    assert (np.abs(bf16_values(scores) - want_values) <= bound).all()

    want_load = torch.zeros(experts, dtype=torch.int64, device=device)
    want_ids, want_weights = ops.topk_softmax(scores, top, True, None, mapping, live_t, want_load)
    ids = layer.view("ids", torch.int32, (tokens, top))
    weights = layer.view("weights", torch.float32, (tokens, top))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(ids.cpu().numpy(), want_ids.cpu().numpy())
    np.testing.assert_array_equal(weights.cpu().numpy().view(np.uint32), want_weights.cpu().numpy().view(np.uint32))
    np.testing.assert_array_equal(load.cpu().numpy(), want_load.cpu().numpy())

    maps = ops.moe_sort(ids, weights, experts, local=None if window is None else (window[0], window[0] + window[1]),
                        live_tokens=live_t)
    torch.cuda.synchronize()
    rows = layer.views.permuted_rows
    lengths = {"tile_to_expert": layer.views.max_tiles, "tile_to_limit": layer.views.max_tiles,
               "expanded_to_permuted": tokens * top, "permuted_to_expanded": rows, "permuted_to_token": rows,
               "total_padded_tokens": 1, "num_non_exiting_tiles": 1}
    padded = int(maps[5][0].item())
    for index, name in enumerate(lengths):
        got = layer.view(name, torch.int32, (lengths[name],)).cpu().numpy()
        want = maps[index][:lengths[name]].cpu().numpy()
        if name in ("permuted_to_expanded", "permuted_to_token"):
            got, want = got[:padded], want[:padded]
        if name in ("tile_to_expert", "tile_to_limit"):
            live_tiles = int(maps[6][0].item())
            got, want = got[:live_tiles], want[:live_tiles]
        np.testing.assert_array_equal(got, want, err_msg=name)

    if wdtype == "bf16":
        return
    quantise = ops.quantize_fp8 if wdtype == "f8e4m3" else ops.quantize_mxfp8
    want_q, want_s = quantise(x)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(layer.view("hidden_q", torch.uint8, (tokens, hidden)).cpu().numpy(),
                                  want_q.cpu().numpy())
    e2p = layer.view("expanded_to_permuted", torch.int32, (tokens * top,)).cpu().numpy()
    held = np.nonzero(e2p >= 0)[0]
    token_of = held // top
    words = hidden // 128
    if wdtype == "f8e4m3":
        token_words = want_s.cpu().numpy().view(np.uint32)  # [tokens, hidden / 128]
        if layer.views.route_scales:
            table = layer.view("hidden_route_s", torch.float32, (words, rows)).cpu().numpy().view(np.uint32).T
            np.testing.assert_array_equal(table[e2p[held]], token_words[token_of])
        else:
            np.testing.assert_array_equal(
                layer.view("hidden_s", torch.float32, (tokens, words)).cpu().numpy().view(np.uint32), token_words)
    else:
        token_words = np.ascontiguousarray(want_s.cpu().numpy()).view(np.uint32).reshape(tokens, words)
        if layer.views.route_scales:
            table = layer.view("hidden_s", torch.int32, (words, rows)).cpu().numpy().view(np.uint32).T
            np.testing.assert_array_equal(table[e2p[held]], token_words[token_of])
        else:
            np.testing.assert_array_equal(
                layer.view("hidden_s", torch.uint8, (tokens, hidden // 32)).cpu().numpy(), want_s.cpu().numpy())

"""The block-scaled e4m3 path and the composed layer on the MI355X against the oracle.

* the activation quantiser writes the oracle's codes and scales bit for bit;
* the e4m3 products agree with the oracle's FP32 evaluation over dequantised values within
  BASELINE's fp8 bar (4e-2 of the peak) - the format has no reference counterpart, so this is
  parity with the oracle's definition, unpinned against the reference;
* the whole layer (router gemm -> topk -> sort -> FC1 -> FC2 -> combine) agrees with the
  oracle's composition: router ids bit-exact, outputs within the bf16 / fp8 bars; at prefill
  size the oracle evaluates a sample of tokens (the layer is per token, so any subset of rows
  is its own smaller call);
* a captured HIP graph of the layer replays to the eager result, bit for bit, across replays
  with eager work between them.
"""

import numpy as np
import pytest
import torch

import oracle_lib as O
from gpu_helpers import announce, assert_bf16_bar, bf16_bits, bf16_values, normal_bf16, sort_on_host, zipf_bias
from uniserve_moe import ops

pytestmark = pytest.mark.gpu


def test_quantiser_is_bit_exact(device):
    announce("quantize fp8")
    x = normal_bf16((333, 2048), 8, device=device)
    x[5] = 0
    x[6, :128] = 1e-30
    q, s = ops.quantize_fp8(x)
    torch.cuda.synchronize()
    want_q, want_s = O.quantize_rows_fp8(bf16_bits(x))
    np.testing.assert_array_equal(q.cpu().numpy(), want_q)
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), want_s.view(np.uint32))
    limit = torch.tensor([100], dtype=torch.int32, device=device)
    q2 = torch.full((333, 2048), 0xAB, dtype=torch.uint8, device=device)
    s2 = torch.full((333, 16), -1.0, device=device)
    call_q, call_s = ops.quantize_fp8(x[:200].contiguous(), row_limit=limit)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(call_q[:100].cpu().numpy(), want_q[:100])
    del q2, s2


def magnitude_groups(rng):
    """128-value groups that pair an amax with every bf16 magnitude not above it (random signs):
    amax over every 4th mantissa of exponents across the range, the smallest subnormals and
    the largest finite values included."""
    exponents = [0, 1, 2, 3, 60, 100, *range(118, 137), 180, 250, 253, 254]
    amaxes = [(e << 7) | m for e in exponents for m in range(0, 128, 4) if (e << 7) | m]
    groups = []
    for a in amaxes:
        v = np.arange(0, a + 1, dtype=np.uint32)
        v = v[v != a]
        pad = (-len(v)) % 127
        v = np.concatenate([v, np.zeros(pad, dtype=np.uint32)]).reshape(-1, 127)
        g = np.concatenate([np.full((len(v), 1), a, dtype=np.uint32), v], axis=1)
        groups.append(g)
    bits = np.concatenate(groups).astype(np.uint16)
    bits |= (rng.integers(0, 2, bits.shape, dtype=np.uint16) << 15)
    rows = -(-len(bits) // 16)
    out = np.zeros((rows * 16, 128), dtype=np.uint16)
    out[:len(bits)] = bits
    return out.reshape(rows, 2048)


def test_quantiser_every_magnitude(device):
    """The division-free quotients of the bf16 quantiser (shared with the FC1 epilogues) against
    IEEE division, for every bf16 magnitude under each of ~1000 group maxima."""
    announce("quantize fp8 every magnitude")
    bits = magnitude_groups(np.random.default_rng(5))
    x = torch.from_numpy(bits.view(np.int16)).to(device).view(torch.bfloat16)
    q, s = ops.quantize_fp8(x)
    torch.cuda.synchronize()
    want_q, want_s = O.quantize_rows_fp8(bits)
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), want_s.view(np.uint32))
    np.testing.assert_array_equal(q.cpu().numpy(), want_q)


def quantized_stacks(device, experts, hidden, intermediate, seed=2):
    up_gate = normal_bf16((experts, 2 * intermediate, hidden), seed, 0.02, device)
    down = normal_bf16((experts, hidden, intermediate), seed + 1, 0.02, device)
    q1, s1 = O.quantize_blocks_fp8(bf16_bits(up_gate))
    q2, s2 = O.quantize_blocks_fp8(bf16_bits(down))
    return q1, s1, q2, s2


@pytest.mark.parametrize("tokens,hidden,experts,top,intermediate,skew", [
    (64, 2048, 128, 8, 768, "uniform"), (1024, 2048, 128, 8, 768, "zipf"), (5, 4096, 16, 8, 1536, "uniform"),
    # the unsplit stream kernel with two 16-row blocks per pass, several passes on hot experts
    (256, 2048, 128, 8, 768, "zipf"),
    # the two-workgroup e4m3 kernels at 235B width (BASELINE configs[4]'s H and I)
    (1024, 4096, 128, 8, 1536, "zipf"),
    # prefill kernels at their smallest shapes: two K stages, one 256-column FC2 slice, ragged tiles
    (600, 256, 8, 2, 256, "zipf"),
    # the split stream kernel with two 16-row blocks per pass and, on the hottest expert, two passes
    (80, 512, 8, 2, 256, "zipf"),
    # three K stages on the two-workgroup FC1; an FC2 neither it nor the 8-wave kernel takes (tiled)
    (300, 384, 16, 4, 384, "uniform")])
def test_fp8_products(device, tokens, hidden, experts, top, intermediate, skew):
    announce("fp8 products", tokens, hidden, experts, top, intermediate, skew)
    rng = np.random.default_rng(tokens)
    if skew == "zipf":
        p = np.exp(zipf_bias(experts).astype(np.float64))
        ids_host = np.stack([rng.choice(experts, size=top, replace=False, p=p / p.sum()) for _ in range(tokens)])
    else:
        ids_host = np.stack([rng.choice(experts, size=top, replace=False) for _ in range(tokens)])
    q1, s1, q2, s2 = quantized_stacks(device, experts, hidden, intermediate)
    x = normal_bf16((tokens, hidden), 1, device=device)
    xq, xs = ops.quantize_fp8(x)
    ids = torch.from_numpy(ids_host.astype(np.int32)).to(device)
    weights = torch.rand((tokens, top), device=device)
    maps = ops.moe_sort(ids, weights, experts)
    rows = ops.permuted_rows(tokens, top, experts)
    d = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    gated = torch.full((rows, intermediate), float("nan"), dtype=torch.bfloat16, device=device)
    ops.gather_gemm_fp8(xq, xs, d(q1), d(s1), top, maps, rows, out=gated)
    padded_t = maps[ops.TOTAL_PADDED_TOKENS][:1]
    gq, gs = ops.quantize_fp8(torch.nan_to_num(gated, 0.0), row_limit=padded_t)
    products = torch.full((rows, hidden), float("nan"), dtype=torch.bfloat16, device=device)
    ops.route_gemm_fp8(gq, gs, d(q2), d(s2), maps, out=products)
    torch.cuda.synchronize()

    sort = sort_on_host(maps, tokens, top)
    padded = int(sort["total_padded_tokens"][0])
    live = sort["permuted_to_expanded"][:padded] >= 0
    want_gated = O.gather_gemm_fp8(xq.cpu().numpy(), xs.cpu().numpy(), q1, s1, top, sort, rows)
    got_gated = bf16_values(gated)
    assert_bf16_bar(got_gated[:padded][live], want_gated[:padded][live], "gather_gemm_fp8", max_rel=4e-2)
    assert np.isnan(got_gated[:padded][~live]).all()
    want_products = O.route_gemm_fp8(gq.cpu().numpy()[:padded], gs.cpu().numpy()[:padded], q2, s2, sort)
    got_products = bf16_values(products)
    assert_bf16_bar(got_products[:padded][live], want_products[:padded][live], "route_gemm_fp8", max_rel=4e-2)


LAYERS = {
    # name: tokens, hidden, experts, top, intermediate, weights, zipf, oracle sample
    "tiny (configs[0] shape, bf16)": (16, 256, 8, 2, 128, "bf16", False, None),
    "30b decode bf16": (64, 2048, 128, 8, 768, "bf16", False, None),
    "30b prefill bf16 zipf": (8192, 2048, 128, 8, 768, "bf16", True, 96),
    "30b decode fp8": (64, 2048, 128, 8, 768, "f8e4m3", False, None),
    "30b prefill fp8 zipf": (8192, 2048, 128, 8, 768, "f8e4m3", True, 96),
    "235b decode fp8 one token": (1, 4096, 128, 8, 1536, "f8e4m3", False, None),
    # the two-workgroup e4m3 kernels at 235B width, route-major scales
    "235b prefill fp8 zipf": (4096, 4096, 128, 8, 1536, "f8e4m3", True, 64),
    # the two-workgroup kernels at their fewest stages (three: e4m3 H = 384, bf16 H = 192), ragged
    # tiles; FC2 of these widths takes the other prefill kernels
    "small prefill fp8, three-stage FC1": (600, 384, 8, 2, 256, "f8e4m3", True, None),
    "small prefill bf16, three-stage FC1": (600, 192, 8, 2, 128, "bf16", True, None),
}


def layer_inputs(device, tokens, hidden, experts, intermediate, seed=0):
    x = normal_bf16((tokens, hidden), seed + 1, device=device)
    router = normal_bf16((experts, hidden), seed + 2, 0.02, device)
    up_gate = normal_bf16((experts, 2 * intermediate, hidden), seed + 3, 0.02, device)
    down = normal_bf16((experts, hidden, intermediate), seed + 4, 0.02, device)
    return x, router, up_gate, down


@pytest.mark.parametrize("case", list(LAYERS))
def test_layer_against_the_oracle(device, case):
    tokens, hidden, experts, top, intermediate, wdtype, zipf, sample = LAYERS[case]
    announce("layer", case)
    x, router, up_gate, down = layer_inputs(device, tokens, hidden, experts, intermediate)
    bias = torch.from_numpy(zipf_bias(experts)).to(device) if zipf else None
    layer = ops.MoeLayer(hidden, experts, top, intermediate, tokens, weight_dtype=wdtype)
    args = {}
    if wdtype == "f8e4m3":
        q1, s1 = O.quantize_blocks_fp8(bf16_bits(up_gate))
        q2, s2 = O.quantize_blocks_fp8(bf16_bits(down))
        up_gate_dev, down_dev = torch.from_numpy(q1).to(device), torch.from_numpy(q2).to(device)
        args = dict(up_gate_scales=torch.from_numpy(s1).to(device), down_scales=torch.from_numpy(s2).to(device))
        host_w = (q1, q2, s1, s2)
    else:
        up_gate_dev, down_dev = up_gate, down
        host_w = (bf16_bits(up_gate), bf16_bits(down), None, None)
    out = layer(x, router, up_gate_dev, down_dev, router_bias=bias, **args)
    torch.cuda.synchronize()
    ids = layer.view("ids", torch.int32, (tokens, top)).cpu().numpy()
    got = bf16_values(out)
    assert np.isfinite(got).all()

    rows = np.arange(tokens) if sample is None else np.random.default_rng(0).choice(tokens, sample, replace=False)
    x_bits = bf16_bits(x)[rows]
    router_bits = bf16_bits(router)
    if zipf:
        # The biased scores against the oracle's router (x . W^T + b in FP32, one rounding):
        # the summation orders differ, so within one bf16 step, and nearly all bit for bit.
        scores = layer.view("scores", torch.bfloat16, (tokens, experts))
        score_bits = bf16_bits(scores)[rows]
        want_scores = O.router_gemm(x_bits, router_bits, zipf_bias(experts))
        s_got = O.bf16_decode(score_bits).astype(np.float64)
        s_want = O.bf16_decode(want_scores).astype(np.float64)
        assert (np.abs(s_got - s_want) <= 2.0**-7 * np.abs(s_want) + 1e-6).all()
        assert (score_bits == want_scores).mean() > 0.99
        # Routing is exact given the scores: the device's ids are the oracle's topk of them.
        want_ids, _ = O.topk_softmax(score_bits, top, score_kind=1)
        np.testing.assert_array_equal(ids[rows], want_ids)
        hist = np.bincount(ids.ravel(), minlength=experts)
        assert hist[0] > 3 * hist[experts // 2], "the Zipf bias skews the routing"
        # Products and combine of the sampled tokens, from the device's routing.
        want = sampled_layer(x_bits, ids[rows], layer.view("weights", torch.float32, (tokens, top)).cpu().numpy()[rows],
                             host_w, experts, top)
    else:
        want_bits, want_ids, want_weights, _ = O.moe_layer(
            x_bits, router_bits, host_w[0], host_w[1], top, up_gate_scales=host_w[2], down_scales=host_w[3])
        np.testing.assert_array_equal(ids[rows], want_ids)
        want = O.bf16_decode(want_bits).astype(np.float64)
    bar = 4e-2 if wdtype == "f8e4m3" else 2e-2
    assert_bf16_bar(got[rows], want, case, max_rel=bar)


def sampled_layer(x_bits, ids, weights, host_w, experts, top):
    """The oracle's products and combine for a sample of tokens with given routes."""
    tokens = x_bits.shape[0]
    w1, w2, s1, s2 = host_w
    sort = O.moe_sort(ids, experts)
    rows = O.max_tiles(tokens, top, experts) * 128
    padded = int(sort["total_padded_tokens"][0])
    if s1 is not None:
        xq, xs = O.quantize_rows_fp8(x_bits)
        gated = O.gather_gemm_fp8(xq, xs, w1, s1, top, sort, rows, fill=0.0)
        gq, gs = O.quantize_rows_fp8(O.bf16_encode(gated))
        products = O.route_gemm_fp8(gq, gs, w2, s2, sort, fill=0.0)
    else:
        gated = O.gather_gemm(x_bits, w1, top, sort, rows, fill=0.0)
        products = O.route_gemm(O.bf16_encode(gated), w2, sort, fill=0.0)
    del padded
    combined = O.moe_unpermute(O.bf16_encode(products), sort["expanded_to_permuted"][: tokens * top].reshape(tokens, top), weights)
    return O.bf16_decode(O.bf16_encode(combined)).astype(np.float64)


@pytest.mark.parametrize("wdtype", ["bf16", "f8e4m3", "f4e2m1"])
def test_layer_live_tokens_leave_padding_rows_zero(device, wdtype):
    """Rows past the live count come out zero and the live rows are the full call's, bit for bit
    (their routes, products and combine do not see the dead rows), for every weight type."""
    announce("layer live tokens", wdtype)
    tokens, hidden, experts, top, intermediate = 64, 2048, 128, 8, 768
    x, router, up_gate, down = layer_inputs(device, tokens, hidden, experts, intermediate, 10)
    args = {}
    if wdtype == "f8e4m3":
        q1, s1 = O.quantize_blocks_fp8(bf16_bits(up_gate))
        q2, s2 = O.quantize_blocks_fp8(bf16_bits(down))
        up_gate, down = torch.from_numpy(q1).to(device), torch.from_numpy(q2).to(device)
        args = dict(up_gate_scales=torch.from_numpy(s1).to(device), down_scales=torch.from_numpy(s2).to(device))
    elif wdtype == "f4e2m1":
        q1, s1 = O.quantize_blocks_mxfp4(bf16_bits(up_gate))
        q2, s2 = O.quantize_blocks_mxfp4(bf16_bits(down))
        up_gate, down = torch.from_numpy(q1).to(device), torch.from_numpy(q2).to(device)
        args = dict(up_gate_scales=torch.from_numpy(s1).to(device), down_scales=torch.from_numpy(s2).to(device))
    layer = ops.MoeLayer(hidden, experts, top, intermediate, tokens, weight_dtype=wdtype)
    full = layer(x, router, up_gate, down, **args).clone()
    live = torch.tensor([40], dtype=torch.int32, device=device)
    part = layer(x, router, up_gate, down, live_tokens=live, **args)
    torch.cuda.synchronize()
    assert (bf16_values(part)[40:] == 0).all()
    np.testing.assert_array_equal(bf16_bits(part)[:40], bf16_bits(full)[:40])


@pytest.mark.parametrize("wdtype", ["bf16", "f8e4m3"])
def test_layer_graph_replays_match_eager(device, wdtype):
    announce("layer graph", wdtype)
    tokens, hidden, experts, top, intermediate = 64, 2048, 128, 8, 768
    x, router, up_gate, down = layer_inputs(device, tokens, hidden, experts, intermediate, 20)
    args = {}
    if wdtype == "f8e4m3":
        q1, s1 = O.quantize_blocks_fp8(bf16_bits(up_gate))
        q2, s2 = O.quantize_blocks_fp8(bf16_bits(down))
        up_gate, down = torch.from_numpy(q1).to(device), torch.from_numpy(q2).to(device)
        args = dict(up_gate_scales=torch.from_numpy(s1).to(device), down_scales=torch.from_numpy(s2).to(device))
    layer = ops.MoeLayer(hidden, experts, top, intermediate, tokens, weight_dtype=wdtype)
    out = torch.empty((tokens, hidden), dtype=torch.bfloat16, device=device)
    layer(x, router, up_gate, down, out=out, **args)
    torch.cuda.synchronize()
    eager = bf16_bits(out).copy()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            layer(x, router, up_gate, down, out=out, **args)
    torch.cuda.synchronize()
    for replay in range(3):
        out.zero_()
        _ = torch.randn(1000, device=device).sum()  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bf16_bits(out), eager, err_msg=f"replay {replay}")


def test_layer_is_deterministic(device):
    announce("layer determinism")
    tokens, hidden, experts, top, intermediate = 2048, 2048, 128, 8, 768
    x, router, up_gate, down = layer_inputs(device, tokens, hidden, experts, intermediate, 30)
    layer = ops.MoeLayer(hidden, experts, top, intermediate, tokens)
    a = bf16_bits(layer(x, router, up_gate, down)).copy()
    b = bf16_bits(layer(x, router, up_gate, down))
    np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("tokens,hidden,intermediate", [(64, 2048, 768), (1, 4096, 1536), (20, 2048, 768)])
def test_decode_front_quantises_like_the_quantiser(device, tokens, hidden, intermediate):
    """At decode sizes the fused front end also quantises the hidden rows for e4m3 layers: its codes
    and scales are the stand-alone quantiser's, bit for bit."""
    announce("front quantisation", tokens, hidden)
    experts, top = 128, 8
    x, router, up_gate, down = layer_inputs(device, tokens, hidden, experts, intermediate, 70 + tokens)
    q1, s1 = O.quantize_blocks_fp8(bf16_bits(up_gate))
    q2, s2 = O.quantize_blocks_fp8(bf16_bits(down))
    layer = ops.MoeLayer(hidden, experts, top, intermediate, tokens, weight_dtype="f8e4m3")
    d = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    layer(x, router, d(q1), d(q2), up_gate_scales=d(s1), down_scales=d(s2))
    want_q, want_s = ops.quantize_fp8(x)
    torch.cuda.synchronize()
    got_q = layer.view("hidden_q", torch.uint8, (tokens, hidden)).cpu().numpy()
    got_s = layer.view("hidden_s", torch.float32, (tokens, hidden // 128)).cpu().numpy()
    np.testing.assert_array_equal(got_q, want_q.cpu().numpy())
    np.testing.assert_array_equal(got_s.view(np.uint32), want_s.cpu().numpy().view(np.uint32))


@pytest.mark.parametrize("tokens,window", [(64, None), (64, (16, 64)), (200, None)])
def test_decode_fc1_quantises_like_the_quantiser(device, tokens, window):
    """At decode sizes (no sort) the e4m3 FC1 also writes the gated rows as FC2's operand: the codes
    and scales of every visible route's row equal the stand-alone quantiser's of the bf16 gated
    rows the same launch leaves, bit for bit (rows scaled by powers of two so that groups span
    many exponents). 200 tokens take two 16-row passes per workgroup."""
    announce("decode e4m3 FC1 quantisation", tokens, window)
    experts, top, hidden, intermediate = 128, 8, 2048, 768
    x, router, up_gate, down = layer_inputs(device, tokens, hidden, experts, intermediate, 130 + tokens)
    x[::3] *= 2.0**20
    x[1::5] *= 2.0**-30
    q1, s1 = O.quantize_blocks_fp8(bf16_bits(up_gate))
    q2, s2 = O.quantize_blocks_fp8(bf16_bits(down))
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    w1, ws1, w2, ws2 = d(q1), d(s1), d(q2), d(s2)
    if window is not None:
        w1, ws1 = w1[window[0]:window[0] + window[1]].contiguous(), ws1[window[0]:window[0] + window[1]].contiguous()
        w2, ws2 = w2[window[0]:window[0] + window[1]].contiguous(), ws2[window[0]:window[0] + window[1]].contiguous()
    layer = ops.MoeLayer(hidden, experts, top, intermediate, tokens, weight_dtype="f8e4m3")
    layer(x, router, w1, w2, up_gate_scales=ws1, down_scales=ws2, window=window)
    routes = tokens * top
    e2p = layer.view("expanded_to_permuted", torch.int32, (routes,)).cpu().numpy()
    visible = np.nonzero(e2p >= 0)[0]
    assert 0 < visible.size and (window is not None or visible.size == routes)
    gated = layer.view("gated", torch.bfloat16, (routes, intermediate)).clone()
    want_q, want_s = ops.quantize_fp8(gated)
    torch.cuda.synchronize()
    got_q = layer.view("gated_q", torch.uint8, (routes, intermediate)).cpu().numpy()
    got_s = layer.view("gated_s", torch.float32, (routes, intermediate // 128)).cpu().numpy()
    np.testing.assert_array_equal(got_q[visible], want_q.cpu().numpy()[visible])
    np.testing.assert_array_equal(got_s[visible].view(np.uint32), want_s.cpu().numpy()[visible].view(np.uint32))


def test_prefill_fc1_quantises_like_the_quantiser(device):
    """At prefill shapes the layer's FC1 writes the gated rows straight in FC2's e4m3 form; codes
    and scales of every live row equal the stand-alone FC1 (bf16 out) followed by quantize_fp8."""
    announce("fused FC1 quantisation")
    tokens, hidden, experts, top, intermediate = 2048, 2048, 128, 8, 768
    x, router, up_gate, down = layer_inputs(device, tokens, hidden, experts, intermediate, 40)
    q1, s1 = O.quantize_blocks_fp8(bf16_bits(up_gate))
    q2, s2 = O.quantize_blocks_fp8(bf16_bits(down))
    w1, w2 = torch.from_numpy(q1).to(device), torch.from_numpy(q2).to(device)
    ws1, ws2 = torch.from_numpy(s1).to(device), torch.from_numpy(s2).to(device)
    layer = ops.MoeLayer(hidden, experts, top, intermediate, tokens, weight_dtype="f8e4m3")
    layer(x, router, w1, w2, up_gate_scales=ws1, down_scales=ws2)
    torch.cuda.synchronize()
    rows = layer.views.permuted_rows
    fused_q = layer.view("gated_q", torch.uint8, (rows, intermediate)).cpu().numpy()
    # Prefill shapes keep both products' activation scales route-major (block by permuted row).
    assert layer.views.route_scales == 1
    fused_s = layer.view("gated_s", torch.float32, (intermediate // 128, rows)).cpu().numpy().T

    class Maps:
        def __getitem__(self, index):
            name = ["tile_to_expert", "tile_to_limit", "expanded_to_permuted", "permuted_to_expanded",
                    "permuted_to_token", "total_padded_tokens", "num_non_exiting_tiles"][index]
            length = {0: layer.views.max_tiles, 1: layer.views.max_tiles, 2: tokens * top, 3: rows, 4: rows,
                      5: 1, 6: 1}[index]
            return layer.view(name, torch.int32, (length,))

    xq = layer.view("hidden_q", torch.uint8, (tokens, hidden))
    xs = layer.view("hidden_s", torch.float32, (tokens, hidden // 128))
    gated = ops.gather_gemm_fp8(xq, xs, w1, ws1, top, Maps(), rows)
    want_q, want_s = ops.quantize_fp8(gated)
    torch.cuda.synchronize()
    p2e = layer.view("permuted_to_expanded", torch.int32, (rows,)).cpu().numpy()
    padded = int(layer.view("total_padded_tokens", torch.int32, (1,)).cpu().numpy()[0])
    live = np.nonzero(p2e[:padded] >= 0)[0]
    assert live.size == tokens * top
    np.testing.assert_array_equal(fused_q[live], want_q.cpu().numpy()[live])
    np.testing.assert_array_equal(fused_s[live].view(np.uint32), want_s.cpu().numpy()[live].view(np.uint32))
    # Each route's row of the route-major hidden scales is its token's row of the quantiser's.
    route_s = layer.view("hidden_route_s", torch.float32, (hidden // 128, rows)).cpu().numpy().T
    tokens_of = p2e[live] // top
    np.testing.assert_array_equal(route_s[live].view(np.uint32), xs.cpu().numpy()[tokens_of].view(np.uint32))


@pytest.mark.parametrize("wdtype,tokens", [("bf16", 64), ("f8e4m3", 64), ("f8e4m3", 2048)])
def test_layer_steps_replay_the_call(device, wdtype, tokens):
    """Every step launched alone over the workspace of a full call, in order, reproduces the call's
    output bit for bit (the step entry launches what the call launches)."""
    announce("layer steps", wdtype, tokens)
    hidden, experts, top, intermediate = 2048, 128, 8, 768
    x, router, up_gate, down = layer_inputs(device, tokens, hidden, experts, intermediate, 50)
    layer = ops.MoeLayer(hidden, experts, top, intermediate, tokens, weight_dtype=wdtype)
    args = {}
    if wdtype == "f8e4m3":
        q1, s1 = O.quantize_blocks_fp8(bf16_bits(up_gate))
        q2, s2 = O.quantize_blocks_fp8(bf16_bits(down))
        up_gate, down = torch.from_numpy(q1).to(device), torch.from_numpy(q2).to(device)
        args = dict(up_gate_scales=torch.from_numpy(s1).to(device), down_scales=torch.from_numpy(s2).to(device))
    out = layer(x, router, up_gate, down, **args)
    want = bf16_bits(out).copy()
    out.zero_()
    layer.view("products", torch.bfloat16, (layer.views.permuted_rows, hidden)).zero_()
    for name in ops.MoeLayer.STEPS:
        layer.step(name)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bf16_bits(out), want)


@pytest.mark.parametrize("wdtype,tokens", [("bf16", 64), ("f8e4m3", 2048)])
def test_layer_is_invariant_under_a_redistribution_of_the_experts(device, wdtype, tokens):
    """crates/nn/tests/moe.rs:1071-1098: the experts stored in another order (router rows and both
    stacks permuted alike) give the same routes and the same output. Experts whose bf16 scores tie
    are picked lower index first, so a redistribution may pick another of equally scored experts
    (checked: the picks that differ score the same) or swap two tied picks. The softmax sums its
    exponentials in lane order, so moving the experts moves the FP32 rounding of the weights by an
    ulp or two; a route's products do not depend on where its expert sits. So: weights within a few
    FP32 ulps, outputs within one bf16 step of their token's peak, and nearly every element bit for bit."""
    announce("layer redistribution", wdtype, tokens)
    hidden, experts, top, intermediate = 2048, 128, 8, 768
    x, router, up_gate, down = layer_inputs(device, tokens, hidden, experts, intermediate, 50)
    args = {}
    if wdtype == "f8e4m3":
        q1, s1 = O.quantize_blocks_fp8(bf16_bits(up_gate))
        q2, s2 = O.quantize_blocks_fp8(bf16_bits(down))
        up_gate, down = torch.from_numpy(q1).to(device), torch.from_numpy(q2).to(device)
        args = dict(up_gate_scales=torch.from_numpy(s1).to(device), down_scales=torch.from_numpy(s2).to(device))
    order = torch.from_numpy(np.random.default_rng(51).permutation(experts)).to(device)
    layer = ops.MoeLayer(hidden, experts, top, intermediate, tokens, weight_dtype=wdtype)
    first = bf16_bits(layer(x, router, up_gate, down, **args)).copy()
    ids = layer.view("ids", torch.int32, (tokens, top)).cpu().numpy().copy()
    scores = bf16_values(layer.view("scores", torch.bfloat16, (tokens, experts)))
    weights = layer.view("weights", torch.float32, (tokens, top)).cpu().numpy().copy()
    moved = {k: v[order].contiguous() for k, v in args.items()}
    second = bf16_bits(layer(x, router[order].contiguous(), up_gate[order].contiguous(), down[order].contiguous(),
                             **moved)).copy()
    moved_ids = order.cpu().numpy()[layer.view("ids", torch.int32, (tokens, top)).cpu().numpy()]
    same_set = (np.sort(moved_ids, axis=1) == np.sort(ids, axis=1)).all(axis=1)
    for t in np.flatnonzero(~same_set):
        gone = sorted(scores[t, e] for e in set(ids[t]) - set(moved_ids[t]))
        came = sorted(scores[t, e] for e in set(moved_ids[t]) - set(ids[t]))
        assert gone == came, (t, gone, came)
    same = (moved_ids == ids).all(axis=1)
    assert same.mean() > 0.5, "most tokens have no tied picks"
    moved_weights = layer.view("weights", torch.float32, (tokens, top)).cpu().numpy()
    np.testing.assert_allclose(moved_weights[same], weights[same], rtol=4 * 2.0 ** -23, atol=0)
    assert (second[same] == first[same]).mean() > 0.999
    a = O.bf16_decode(first[same_set]).astype(np.float64)
    b = O.bf16_decode(second[same_set]).astype(np.float64)
    # One bf16 step of the row's peak: a sum that nearly cancels has no relative bound per element.
    peak = np.maximum(np.abs(a).max(axis=1, keepdims=True), np.abs(b).max(axis=1, keepdims=True))
    assert (np.abs(a - b) <= 2.0 ** -7 * peak).all()

"""MX products on the MI355X against the oracle: MXFP4 weights x MXFP8 activations.

The quantiser is bit-exact with the oracle's rule (tests/test_oracle.py pins that rule against
torch's e4m3 cast and the E2M1 table). The products take the same codes and scales on both sides;
the hardware's block scaling is exact (powers of two) and the FP32 sums differ only in order, so
the gap is the bf16 rounding of the outputs: max |got - want| <= 1e-2 of the peak (and the mean
within BASELINE's 1e-3). Parity unpinned against the reference: it has no MX operator (its four-bit
experts are NVFP4).

Decode-shaped cases (few routes per expert) run the stream kernel; the 512- and 1024-token Zipf
cases and the 8192-token layer run the tiled prefill kernel for both products.
"""

import numpy as np
import pytest
import torch

import oracle_lib as O
from gpu_helpers import announce, assert_bf16_bar, bf16_bits, bf16_values, normal_bf16, sort_on_host, zipf_bias
from uniserve_moe import ops

pytestmark = pytest.mark.gpu


def test_mxfp8_quantiser_is_bit_exact(device):
    announce("quantize mxfp8")
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((300, 512)) * np.exp(rng.normal(0, 4, (300, 1)))).astype(np.float32)
    x[3, :64] = 0.0
    x[7, 5] = 3.0e38
    x[9, 32:64] = 1.0e-39                                 # subnormal block: exponent clamps at -127
    # Blocks whose amax sits on either side of 448 * 2^e (bf16 neighbours of 448, 3.5 and 7 / 2^100).
    x[11, 0:32], x[11, 32], x[11, 64] = 0.25, 448.0, 450.0
    x[11, 96], x[11, 128] = 3.5, 3.515625
    x[12, 0], x[12, 32] = 7.0 * 2.0**-100, 7.25 * 2.0**-100
    bits = O.bf16_encode(x)
    t = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).to(device)
    q, s = ops.quantize_mxfp8(t)
    torch.cuda.synchronize()
    want_q, want_s = O.quantize_rows_mxfp8(bits)
    np.testing.assert_array_equal(s.cpu().numpy(), want_s)
    np.testing.assert_array_equal(q.cpu().numpy(), want_q)
    # A device-side row limit leaves the rows past it untouched.
    q.fill_(0xAB)
    limit = torch.tensor([100], dtype=torch.int32, device=device)
    ops.quantize_mxfp8(t, row_limit=limit)
    call_q, _ = ops.quantize_mxfp8(t, row_limit=limit)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(call_q[:100].cpu().numpy(), want_q[:100])


def mx_stacks(device, experts, hidden, intermediate, seed=2):
    up_gate = normal_bf16((experts, 2 * intermediate, hidden), seed, 0.02, device)
    down = normal_bf16((experts, hidden, intermediate), seed + 1, 0.02, device)
    q1, s1 = O.quantize_blocks_mxfp4(bf16_bits(up_gate))
    q2, s2 = O.quantize_blocks_mxfp4(bf16_bits(down))
    return q1, s1, q2, s2


def test_stage_major_scales_are_the_row_major_bytes_regrouped(device):
    announce("mx stage-major scales")
    rng = np.random.default_rng(3)
    table = rng.integers(0, 256, size=(3, 192, 1536 // 32), dtype=np.uint8)
    got = ops.mx_stage_major_scales(torch.from_numpy(table).to(device)).cpu().numpy()
    want = table.reshape(3, 192, 1536 // 128, 4).transpose(0, 2, 1, 3)
    np.testing.assert_array_equal(got.reshape(3, 1536 // 128, 192, 4), want)


@pytest.mark.parametrize("tokens,hidden,experts,top,intermediate,skew,layout", [
    (64, 2048, 128, 8, 768, "uniform", "row"), (1, 4096, 128, 8, 1536, "uniform", "row"),
    (512, 2048, 128, 8, 768, "zipf", "row"), (1024, 4096, 128, 8, 1536, "zipf", "row"),
    (64, 2048, 128, 8, 768, "uniform", "stage"), (512, 2048, 128, 8, 768, "zipf", "stage"),
    # the tiled kernel at its smallest shapes: two K stages, one weight slice, ragged tiles
    (600, 256, 8, 2, 256, "zipf", "row"),
    # the split stream kernel over several 16-row passes of the hottest expert's tile
    (80, 512, 8, 2, 256, "zipf", "stage")])
def test_mx_products(device, tokens, hidden, experts, top, intermediate, skew, layout):
    announce("mx products", tokens, hidden, experts, top, intermediate, skew, layout)
    rng = np.random.default_rng(tokens + 7)
    if skew == "zipf":
        p = np.exp(zipf_bias(experts).astype(np.float64))
        ids_host = np.stack([rng.choice(experts, size=top, replace=False, p=p / p.sum()) for _ in range(tokens)])
    else:
        ids_host = np.stack([rng.choice(experts, size=top, replace=False) for _ in range(tokens)])
    q1, s1, q2, s2 = mx_stacks(device, experts, hidden, intermediate)
    x = normal_bf16((tokens, hidden), 1, device=device)
    xq, xs = ops.quantize_mxfp8(x)
    ids = torch.from_numpy(ids_host.astype(np.int32)).to(device)
    weights = torch.rand((tokens, top), device=device)
    maps = ops.moe_sort(ids, weights, experts)
    rows = ops.permuted_rows(tokens, top, experts)
    d = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    ws1, ws2 = d(s1), d(s2)
    if layout == "stage":
        ws1, ws2 = ops.mx_stage_major_scales(ws1), ops.mx_stage_major_scales(ws2)
    gated = torch.full((rows, intermediate), float("nan"), dtype=torch.bfloat16, device=device)
    ops.gather_gemm_mx(xq, xs, d(q1), ws1, top, maps, rows, out=gated, scale_layout=layout)
    padded_t = maps[ops.TOTAL_PADDED_TOKENS][:1]
    gq, gs = ops.quantize_mxfp8(torch.nan_to_num(gated, 0.0), row_limit=padded_t)
    products = torch.full((rows, hidden), float("nan"), dtype=torch.bfloat16, device=device)
    ops.route_gemm_mx(gq, gs, d(q2), ws2, maps, out=products, scale_layout=layout)
    torch.cuda.synchronize()

    sort = sort_on_host(maps, tokens, top)
    padded = int(sort["total_padded_tokens"][0])
    live = sort["permuted_to_expanded"][:padded] >= 0
    want_gated = O.gather_gemm_mx(xq.cpu().numpy(), xs.cpu().numpy(), q1, s1, top, sort, rows)
    got_gated = bf16_values(gated)
    assert_bf16_bar(got_gated[:padded][live], want_gated[:padded][live], "gather_gemm_mx", max_rel=1e-2)
    assert np.isnan(got_gated[:padded][~live]).all()
    want_products = O.route_gemm_mx(gq.cpu().numpy()[:padded], gs.cpu().numpy()[:padded], q2, s2, sort)
    got_products = bf16_values(products)
    assert_bf16_bar(got_products[:padded][live], want_products[:padded][live], "route_gemm_mx", max_rel=1e-2)


MX_LAYERS = {
    # name: tokens, hidden, experts, top, intermediate, zipf, oracle sample, weight scale layout
    "30b decode mx": (64, 2048, 128, 8, 768, False, None, "row"),
    "30b prefill mx zipf": (8192, 2048, 128, 8, 768, True, 96, "row"),
    "235b decode mx one token": (1, 4096, 128, 8, 1536, False, None, "row"),
    "30b decode mx stage scales": (64, 2048, 128, 8, 768, False, None, "stage"),
    "30b prefill mx zipf stage scales": (8192, 2048, 128, 8, 768, True, 96, "stage"),
}


def mx_layer_inputs(device, tokens, hidden, experts, intermediate, seed=0):
    x = normal_bf16((tokens, hidden), seed + 1, device=device)
    router = normal_bf16((experts, hidden), seed + 2, 0.02, device)
    q1, s1, q2, s2 = mx_stacks(device, experts, hidden, intermediate, seed + 3)
    return x, router, (q1, s1, q2, s2)


def on(device, host):
    return [torch.from_numpy(a).to(device) for a in host]


@pytest.mark.parametrize("case", list(MX_LAYERS))
def test_mx_layer_against_the_oracle(device, case):
    """The whole layer over MXFP4 stacks against the oracle's composition: router ids bit-exact;
    outputs within 4e-2 of the peak (the gated rows are re-quantised to MXFP8 on both sides from
    bf16 values that may differ in their last bit, which moves a code by one step)."""
    tokens, hidden, experts, top, intermediate, zipf, sample, layout = MX_LAYERS[case]
    announce("mx layer", case)
    x, router, host_w = mx_layer_inputs(device, tokens, hidden, experts, intermediate)
    w1, s1, w2, s2 = on(device, host_w)
    if layout == "stage":
        s1, s2 = ops.mx_stage_major_scales(s1), ops.mx_stage_major_scales(s2)
    bias = torch.from_numpy(zipf_bias(experts)).to(device) if zipf else None
    layer = ops.MoeLayer(hidden, experts, top, intermediate, tokens, weight_dtype="f4e2m1")
    out = layer(x, router, w1, w2, up_gate_scales=s1, down_scales=s2, router_bias=bias, scale_layout=layout)
    # Prefill shapes keep both activation scale tables stage-major by permuted row.
    assert layer.views.route_scales == (1 if tokens >= 4096 else 0)
    torch.cuda.synchronize()
    ids = layer.view("ids", torch.int32, (tokens, top)).cpu().numpy()
    got = bf16_values(out)
    assert np.isfinite(got).all()
    rows = np.arange(tokens) if sample is None else np.random.default_rng(0).choice(tokens, sample, replace=False)
    x_bits = bf16_bits(x)[rows]
    if zipf:
        scores = layer.view("scores", torch.bfloat16, (tokens, experts))
        want_ids, _ = O.topk_softmax(bf16_bits(scores)[rows], top, score_kind=1)
        np.testing.assert_array_equal(ids[rows], want_ids)
        weights = layer.view("weights", torch.float32, (tokens, top)).cpu().numpy()[rows]
        want = sampled_mx_layer(x_bits, ids[rows], weights, host_w, experts, top)
    else:
        want_bits, want_ids, _, _ = O.moe_layer(x_bits, bf16_bits(router), host_w[0], host_w[2], top,
                                                up_gate_scales=host_w[1], down_scales=host_w[3])
        np.testing.assert_array_equal(ids[rows], want_ids)
        want = O.bf16_decode(want_bits).astype(np.float64)
    assert_bf16_bar(got[rows], want, case, max_rel=4e-2)


@pytest.mark.parametrize("tokens,hidden,intermediate", [(64, 2048, 768), (1, 4096, 1536), (20, 2048, 768)])
def test_decode_front_quantises_like_the_mxfp8_quantiser(device, tokens, hidden, intermediate):
    """At decode sizes the fused front end also quantises the hidden rows for MXFP4 layers: its
    codes and E8M0 bytes are the stand-alone MXFP8 quantiser's, bit for bit (a few rows scaled up
    and down by powers of two so that blocks span many exponents)."""
    announce("front mx quantisation", tokens, hidden)
    experts, top = 128, 8
    x, router, host_w = mx_layer_inputs(device, tokens, hidden, experts, intermediate, 90 + tokens)
    x[::3] *= 2.0**40
    x[1::5] *= 2.0**-60
    w1, s1, w2, s2 = on(device, host_w)
    layer = ops.MoeLayer(hidden, experts, top, intermediate, tokens, weight_dtype="f4e2m1")
    layer(x, router, w1, w2, up_gate_scales=s1, down_scales=s2)
    want_q, want_s = ops.quantize_mxfp8(x)
    torch.cuda.synchronize()
    got_q = layer.view("hidden_q", torch.uint8, (tokens, hidden)).cpu().numpy()
    got_s = layer.view("hidden_s", torch.uint8, (tokens, hidden // 32)).cpu().numpy()
    np.testing.assert_array_equal(got_q, want_q.cpu().numpy())
    np.testing.assert_array_equal(got_s, want_s.cpu().numpy())


@pytest.mark.parametrize("tokens,window", [(64, None), (64, (16, 64)), (200, None)])
def test_decode_fc1_quantises_like_the_mxfp8_quantiser(device, tokens, window):
    """At decode sizes (no sort) the MX FC1 also writes the gated rows as FC2's MXFP8 operand: the
    codes and row-major E8M0 bytes of every visible route's row equal the stand-alone MXFP8
    quantiser's of the bf16 gated rows the same launch leaves, bit for bit (rows scaled by powers
    of two so that blocks span many exponents)."""
    announce("decode mx FC1 quantisation", tokens, window)
    experts, top, hidden, intermediate = 128, 8, 2048, 768
    x, router, host_w = mx_layer_inputs(device, tokens, hidden, experts, intermediate, 120 + tokens)
    x[::3] *= 2.0**20
    x[1::5] *= 2.0**-30
    w1, s1, w2, s2 = on(device, host_w)
    if window is not None:
        w1, s1 = w1[window[0]:window[0] + window[1]].contiguous(), s1[window[0]:window[0] + window[1]].contiguous()
        w2, s2 = w2[window[0]:window[0] + window[1]].contiguous(), s2[window[0]:window[0] + window[1]].contiguous()
    layer = ops.MoeLayer(hidden, experts, top, intermediate, tokens, weight_dtype="f4e2m1")
    layer(x, router, w1, w2, up_gate_scales=s1, down_scales=s2, window=window)
    routes = tokens * top
    e2p = layer.view("expanded_to_permuted", torch.int32, (routes,)).cpu().numpy()
    visible = np.nonzero(e2p >= 0)[0]
    assert 0 < visible.size and (window is not None or visible.size == routes)
    gated = layer.view("gated", torch.bfloat16, (routes, intermediate)).clone()
    want_q, want_s = ops.quantize_mxfp8(gated)
    torch.cuda.synchronize()
    got_q = layer.view("gated_q", torch.uint8, (routes, intermediate)).cpu().numpy()
    got_s = layer.view("gated_s", torch.uint8, (routes, intermediate // 32)).cpu().numpy()
    np.testing.assert_array_equal(got_q[visible], want_q.cpu().numpy()[visible])
    np.testing.assert_array_equal(got_s[visible], want_s.cpu().numpy()[visible])


def sampled_mx_layer(x_bits, ids, weights, host_w, experts, top):
    """The oracle's MX products and combine for a sample of tokens with given routes."""
    tokens = x_bits.shape[0]
    w1, s1, w2, s2 = host_w
    sort = O.moe_sort(ids, experts)
    rows = O.max_tiles(tokens, top, experts) * 128
    xq, xs = O.quantize_rows_mxfp8(x_bits)
    gated = O.gather_gemm_mx(xq, xs, w1, s1, top, sort, rows, fill=0.0)
    gq, gs = O.quantize_rows_mxfp8(O.bf16_encode(gated))
    products = O.route_gemm_mx(gq, gs, w2, s2, sort, fill=0.0)
    combined = O.moe_unpermute(O.bf16_encode(products),
                               sort["expanded_to_permuted"][: tokens * top].reshape(tokens, top), weights)
    return O.bf16_decode(O.bf16_encode(combined)).astype(np.float64)


def test_mx_layer_graph_replays_match_eager(device):
    announce("mx layer graph")
    tokens, hidden, experts, top, intermediate = 64, 2048, 128, 8, 768
    x, router, host_w = mx_layer_inputs(device, tokens, hidden, experts, intermediate, 20)
    w1, s1, w2, s2 = on(device, host_w)
    layer = ops.MoeLayer(hidden, experts, top, intermediate, tokens, weight_dtype="f4e2m1")
    out = torch.empty((tokens, hidden), dtype=torch.bfloat16, device=device)
    layer(x, router, w1, w2, out=out, up_gate_scales=s1, down_scales=s2)
    torch.cuda.synchronize()
    eager = bf16_bits(out).copy()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            layer(x, router, w1, w2, out=out, up_gate_scales=s1, down_scales=s2)
    torch.cuda.synchronize()
    for replay in range(3):
        out.zero_()
        _ = torch.randn(1000, device=device).sum()  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bf16_bits(out), eager, err_msg=f"replay {replay}")


def test_device_mxfp4_quantiser_matches_the_oracle(device):
    """The package's stack quantiser, run on the device, writes the oracle's pairs and scales."""
    from uniserve_moe.checkpoint import quantize_blocks_mxfp4

    announce("mxfp4 stack quantiser on device")
    w = normal_bf16((4, 256, 512), 9, 0.02, device)
    pairs, scales = quantize_blocks_mxfp4(w)
    torch.cuda.synchronize()
    want_pairs, want_scales = O.quantize_blocks_mxfp4(bf16_bits(w))
    np.testing.assert_array_equal(scales.cpu().numpy(), want_scales)
    np.testing.assert_array_equal(pairs.cpu().numpy(), want_pairs)


def test_prefill_fc1_quantises_like_the_mxfp8_quantiser(device):
    """At prefill shapes the layer's MX FC1 writes the gated rows straight in FC2's MXFP8 form: codes
    and stage-major E8M0 bytes of every live row equal the stand-alone FC1 (bf16 out) followed by
    the stand-alone MXFP8 quantiser."""
    tokens, hidden, experts, top, intermediate = 4096, 2048, 128, 8, 768
    announce("fused mx FC1 quantisation")
    x, router, host_w = mx_layer_inputs(device, tokens, hidden, experts, intermediate, 33)
    w1, s1, w2, s2 = on(device, host_w)
    s1, s2 = ops.mx_stage_major_scales(s1), ops.mx_stage_major_scales(s2)
    layer = ops.MoeLayer(hidden, experts, top, intermediate, tokens, weight_dtype="f4e2m1")
    layer(x, router, w1, w2, up_gate_scales=s1, down_scales=s2, scale_layout="stage")
    torch.cuda.synchronize()
    assert layer.views.route_scales == 1
    rows = layer.views.permuted_rows

    class Maps:
        def __getitem__(self, index):
            name = ["tile_to_expert", "tile_to_limit", "expanded_to_permuted", "permuted_to_expanded",
                    "permuted_to_token", "total_padded_tokens", "num_non_exiting_tiles"][index]
            length = {0: layer.views.max_tiles, 1: layer.views.max_tiles, 2: tokens * top, 3: rows, 4: rows,
                      5: 1, 6: 1}[index]
            return layer.view(name, torch.int32, (length,))

    xq, xs = ops.quantize_mxfp8(x)
    gated = ops.gather_gemm_mx(xq, xs, w1, s1, top, Maps(), rows, scale_layout="stage")
    want_q, want_s = ops.quantize_mxfp8(gated)
    torch.cuda.synchronize()
    p2e = layer.view("permuted_to_expanded", torch.int32, (rows,)).cpu().numpy()
    padded = int(layer.view("total_padded_tokens", torch.int32, (1,)).cpu().numpy()[0])
    live = np.nonzero(p2e[:padded] >= 0)[0]
    assert live.size == tokens * top
    got_q = layer.view("gated_q", torch.uint8, (rows, intermediate)).cpu().numpy()
    np.testing.assert_array_equal(got_q[live], want_q.cpu().numpy()[live])
    # Stage-major bytes: [intermediate / 128 stages][rows][4 blocks] -> [rows][intermediate / 32].
    table = layer.view("gated_s", torch.uint8, (intermediate // 128, rows, 4)).cpu().numpy()
    got_s = np.ascontiguousarray(table.transpose(1, 0, 2)).reshape(rows, intermediate // 32)
    np.testing.assert_array_equal(got_s[live], want_s.cpu().numpy()[live])

"""What `MoE::routed` passes beyond the rows, and FC1's second gate, on the MI355X.

* The layer call with a slot map, an expert load, a live count and a local window
  (crates/nn/src/modules/moe.rs:650-671, 770-775) against the oracle's layer with the same
  options: ids (slots) bit-exact, load counts exact, outputs within the bf16 / fp8 bars, for
  bf16, e4m3 and MXFP4 stacks at decode and prefill shapes.
* The gelu_tanh gate (crates/ops/src/moe/grouped.rs:53-61) on every FC1 kernel: the stand-alone
  entries against the oracle's FC1 with that gate, and the layer with ``activation="gelu_tanh"``.
* BASELINE configs[0] (the tiny layer, fp32 on the CPU reference path): the HIP layer on the same
  values rounded to bf16 against the oracle's fp32 layer.
"""

import numpy as np
import pytest
import torch

import oracle_lib as O
from gpu_helpers import (announce, assert_bf16_bar, bf16_bits, bf16_values, normal_bf16, sort_on_host,
                         zipf_bias)
from uniserve_moe import ops

pytestmark = pytest.mark.gpu


def quantised(wdtype, up_gate, down, device):
    """Host-quantised stacks (the checker's own quantisers) and the layer's keyword arguments."""
    if wdtype == "bf16":
        return bf16_bits(up_gate), bf16_bits(down), None, None, up_gate, down, {}
    quant = O.quantize_blocks_fp8 if wdtype == "f8e4m3" else O.quantize_blocks_mxfp4
    q1, s1 = quant(bf16_bits(up_gate))
    q2, s2 = quant(bf16_bits(down))
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    return q1, q2, s1, s2, d(q1), d(q2), dict(up_gate_scales=d(s1), down_scales=d(s2))


ROUTED = {
    # name: tokens, hidden, experts, top, intermediate, weights, window, live
    "bf16 decode, map + load + window + live": (64, 2048, 128, 8, 768, "bf16", (32, 48), 50),
    "bf16 prefill, map + load + window": (2048, 2048, 128, 8, 768, "bf16", (16, 96), None),
    "fp8 decode, map + load + window": (64, 2048, 128, 8, 768, "f8e4m3", (40, 64), None),
    "fp8 decode, map + load + window + live": (64, 2048, 128, 8, 768, "f8e4m3", (40, 64), 50),
    "fp8 prefill, map + load + window + live": (2048, 2048, 128, 8, 768, "f8e4m3", (0, 100), 2000),
    "mx decode, map + load + window": (64, 2048, 128, 8, 768, "f4e2m1", (64, 64), None),
    "mx prefill, map + load + window": (2048, 2048, 128, 8, 768, "f4e2m1", (8, 112), None),
    "bf16 decode, every expert, map + load only": (64, 2048, 128, 8, 768, "bf16", None, None),
    "bf16 decode, map + load + window + live": (64, 2048, 128, 8, 768, "bf16", (40, 64), 50),
    "bf16 one token, map + load + window": (1, 2048, 128, 8, 768, "bf16", (32, 64), None),
    # fewer routes than local experts, some experts named twice: the compact expert-major grid
    "bf16 8 tokens, map + load + window + live": (8, 2048, 128, 8, 768, "bf16", (16, 96), 6),
    "fp8 8 tokens, map + load + window": (8, 2048, 128, 8, 768, "f8e4m3", (16, 96), None),
    "mx 8 tokens, map + load + window": (8, 2048, 128, 8, 768, "f4e2m1", (16, 96), None),
    # the expert-split front end (at most 8 tokens) off its usual shape: an expert count that is
    # no multiple of its four experts per workgroup, one or three 512-channel chunks of a narrow
    # row, five of a wide one, top 10
    "fp8 5 tokens, 60 experts, 512 channels": (5, 512, 60, 4, 256, "f8e4m3", None, None),
    "mx 3 tokens, 1536 channels, window + live": (3, 1536, 128, 8, 512, "f4e2m1", (8, 64), 2),
    "bf16 7 tokens, 100 experts, top 10, 2560 channels": (7, 2560, 100, 10, 384, "bf16", None, None),
    # a window of 16 experts: 24 or more routes per local expert, so the decode front end (which
    # still quantises the hidden rows) hands over to the sort and the tiled products
    "fp8 decode, narrow window": (64, 2048, 128, 8, 768, "f8e4m3", (8, 16), None),
    "mx decode, narrow window": (64, 2048, 128, 8, 768, "f4e2m1", (8, 16), None),
    "bf16 decode, narrow window + live": (64, 2048, 128, 8, 768, "bf16", (8, 16), 40),
}


@pytest.mark.parametrize("case", list(ROUTED))
def test_layer_routing_options_against_the_oracle(device, case):
    tokens, hidden, experts, top, intermediate, wdtype, window, live = ROUTED[case]
    announce("layer routing", case)
    x = normal_bf16((tokens, hidden), 61, device=device)
    router = normal_bf16((experts, hidden), 62, 0.02, device)
    local = experts if window is None else window[1]
    offset = 0 if window is None else window[0]
    up_gate = normal_bf16((local, 2 * intermediate, hidden), 63, 0.02, device)
    down = normal_bf16((local, hidden, intermediate), 64, 0.02, device)
    bias = zipf_bias(experts)
    mapping = np.random.default_rng(65).permutation(experts).astype(np.int32)
    w1, w2, s1, s2, up_dev, down_dev, args = quantised(wdtype, up_gate, down, device)

    layer = ops.MoeLayer(hidden, experts, top, intermediate, tokens, weight_dtype=wdtype)
    load = torch.full((experts,), 5, dtype=torch.int64, device=device)  # the load accumulates
    live_t = None if live is None else torch.tensor([live], dtype=torch.int32, device=device)
    out = layer(x, router, up_dev, down_dev, router_bias=torch.from_numpy(bias).to(device), live_tokens=live_t,
                mapping=torch.from_numpy(mapping).to(device), load=load, window=window, **args)
    torch.cuda.synchronize()
    got = bf16_values(out)
    ids = layer.view("ids", torch.int32, (tokens, top)).cpu().numpy()
    scores = bf16_bits(layer.view("scores", torch.bfloat16, (tokens, experts)))
    # Every counter the call's launches meet through (the ticket view) is left zero.
    assert int(layer.workspace[: layer.views.scores].count_nonzero()) == 0

    host_load = np.full(experts, 5, np.int64)
    want_bits, want_ids, _, _, want_scores = O.moe_layer(
        bf16_bits(x), bf16_bits(router), w1, w2, top, up_gate_scales=s1, down_scales=s2, router_bias=bias,
        mapping=mapping, load=host_load, live=live, window=None if window is None else (offset, local), scores=True)
    # The biased scores: one rounding of an FP32 sum (summation orders differ: within a bf16 step).
    s_got, s_want = O.bf16_decode(scores).astype(np.float64), O.bf16_decode(want_scores).astype(np.float64)
    assert (np.abs(s_got - s_want) <= 2.0**-7 * np.abs(s_want) + 1e-6).all()
    assert (scores == want_scores).mean() > 0.99
    np.testing.assert_array_equal(ids, want_ids)
    np.testing.assert_array_equal(load.cpu().numpy(), host_load)
    want = O.bf16_decode(want_bits).astype(np.float64)
    rows = slice(None) if live is None else slice(0, live)
    if live is not None:
        assert (got[live:] == 0).all()
    held = (ids[rows] >= offset) & (ids[rows] < offset + local)
    assert held.any() and (~held).any() if window is not None else held.all()
    assert_bf16_bar(got[rows], want[rows], case, max_rel=2e-2 if wdtype == "bf16" else 4e-2)


GELU_PRODUCTS = {
    # name: tokens, hidden, experts, top, intermediate, weights (the kernel the shape takes)
    "bf16 stream": (64, 2048, 128, 8, 768, "bf16"),
    "bf16 prefill": (2048, 2048, 128, 8, 768, "bf16"),
    "bf16 tiled (odd widths)": (300, 320, 16, 4, 192, "bf16"),
    "fp8 stream": (64, 2048, 128, 8, 768, "f8e4m3"),
    "fp8 two-workgroup": (1024, 2048, 128, 8, 768, "f8e4m3"),
    "fp8 split stream (one token)": (1, 4096, 128, 8, 1536, "f8e4m3"),
    "mx stream": (64, 2048, 128, 8, 768, "f4e2m1"),
    "mx tiled": (1024, 2048, 128, 8, 768, "f4e2m1"),
}


@pytest.mark.parametrize("case", list(GELU_PRODUCTS))
def test_gelu_tanh_fc1_against_the_oracle(device, case):
    tokens, hidden, experts, top, intermediate, wdtype = GELU_PRODUCTS[case]
    announce("gelu_tanh FC1", case)
    rng = np.random.default_rng(tokens + hidden)
    ids_host = np.stack([rng.choice(experts, size=top, replace=False) for _ in range(tokens)]).astype(np.int32)
    x = normal_bf16((tokens, hidden), 71, device=device)
    up_gate = normal_bf16((experts, 2 * intermediate, hidden), 72, 0.02, device)
    ids = torch.from_numpy(ids_host).to(device)
    maps = ops.moe_sort(ids, torch.rand((tokens, top), device=device), experts)
    rows = ops.permuted_rows(tokens, top, experts)
    gated = {}
    for act in ("silu", "gelu_tanh"):
        out = torch.full((rows, intermediate), float("nan"), dtype=torch.bfloat16, device=device)
        if wdtype == "bf16":
            ops.gather_gemm(x, up_gate, top, maps, rows, out=out, activation=act)
        elif wdtype == "f8e4m3":
            xq, xs = ops.quantize_fp8(x)
            q1, s1 = O.quantize_blocks_fp8(bf16_bits(up_gate))
            ops.gather_gemm_fp8(xq, xs, torch.from_numpy(q1).to(device), torch.from_numpy(s1).to(device), top, maps,
                                rows, out=out, activation=act)
        else:
            xq, xs = ops.quantize_mxfp8(x)
            q1, s1 = O.quantize_blocks_mxfp4(bf16_bits(up_gate))
            ops.gather_gemm_mx(xq, xs, torch.from_numpy(q1).to(device), torch.from_numpy(s1).to(device), top, maps,
                               rows, out=out, activation=act)
        gated[act] = out
    torch.cuda.synchronize()
    sort = sort_on_host(maps, tokens, top)
    padded = int(sort["total_padded_tokens"][0])
    live = sort["permuted_to_expanded"][:padded] >= 0
    for act, code in (("silu", 0), ("gelu_tanh", 1)):
        if wdtype == "bf16":
            want = O.gather_gemm(bf16_bits(x), bf16_bits(up_gate), top, sort, rows, activation=code)
        elif wdtype == "f8e4m3":
            want = O.gather_gemm_fp8(xq.cpu().numpy(), xs.cpu().numpy(), q1, s1, top, sort, rows, activation=code)
        else:
            want = O.gather_gemm_mx(xq.cpu().numpy(), xs.cpu().numpy(), q1, s1, top, sort, rows, activation=code)
        got = bf16_values(gated[act])
        assert_bf16_bar(got[:padded][live], want[:padded][live], f"{case} {act}",
                        max_rel=2e-2 if wdtype == "bf16" else 1e-2 if wdtype == "f4e2m1" else 4e-2)
        assert np.isnan(got[:padded][~live]).all()
    # The two gates give different rows (the entry really switches).
    a, b = bf16_values(gated["silu"])[:padded][live], bf16_values(gated["gelu_tanh"])[:padded][live]
    assert (a != b).mean() > 0.5


GELU_LAYERS = {
    # name: weights, tokens, hidden, experts, top, intermediate
    "bf16 decode": ("bf16", 64, 2048, 128, 8, 768),
    "f8e4m3 decode": ("f8e4m3", 64, 2048, 128, 8, 768),
    "f4e2m1 decode": ("f4e2m1", 64, 2048, 128, 8, 768),
    # 128 routes per expert: the prefill products (the two-workgroup kernels, e4m3 FC1 writing
    # FC2's operand through its division-free quantiser)
    "bf16 prefill": ("bf16", 512, 1024, 32, 8, 512),
    "f8e4m3 prefill": ("f8e4m3", 512, 1024, 32, 8, 512),
}


@pytest.mark.parametrize("case", list(GELU_LAYERS))
def test_layer_with_the_gelu_tanh_gate(device, case):
    wdtype, tokens, hidden, experts, top, intermediate = GELU_LAYERS[case]
    announce("layer gelu_tanh", case)
    x = normal_bf16((tokens, hidden), 81, device=device)
    router = normal_bf16((experts, hidden), 82, 0.02, device)
    up_gate = normal_bf16((experts, 2 * intermediate, hidden), 83, 0.02, device)
    down = normal_bf16((experts, hidden, intermediate), 84, 0.02, device)
    w1, w2, s1, s2, up_dev, down_dev, args = quantised(wdtype, up_gate, down, device)
    layer = ops.MoeLayer(hidden, experts, top, intermediate, tokens, weight_dtype=wdtype)
    out = layer(x, router, up_dev, down_dev, activation="gelu_tanh", **args)
    torch.cuda.synchronize()
    want_bits, want_ids, _, _ = O.moe_layer(bf16_bits(x), bf16_bits(router), w1, w2, top, up_gate_scales=s1,
                                            down_scales=s2, activation=1)
    np.testing.assert_array_equal(layer.view("ids", torch.int32, (tokens, top)).cpu().numpy(), want_ids)
    assert_bf16_bar(bf16_values(out), O.bf16_decode(want_bits), f"layer gelu_tanh {case}",
                    max_rel=2e-2 if wdtype == "bf16" else 4e-2)


def test_tiny_config_against_the_fp32_oracle(device):
    """fp32 x, W_r and stacks from the oracle's seeded normals; the oracle runs the
    reference's CPU path in fp32 (nothing rounds), the HIP layer runs on the values rounded to
    bf16. Tokens whose routes agree meet the bf16 bar; a token whose routes differ must be a near
    tie of its fp32 scores within what rounding x and W_r to bf16 can move them."""
    announce("tiny fp32 config")
    T, H, E, K, I = 16, 256, 8, 2, 128
    x = O.normal(T * H, 1).reshape(T, H).astype(np.float32)
    router = O.normal(E * H, 2, 0.02).reshape(E, H).astype(np.float32)
    up_gate = O.normal(E * 2 * I * H, 3, 0.02).reshape(E, 2 * I, H).astype(np.float32)
    down = O.normal(E * H * I, 4, 0.02).reshape(E, H, I).astype(np.float32)
    want, want_ids, _, _, scores = O.moe_layer(x, router, up_gate, down, K, scores=True)
    d = lambda a: torch.from_numpy(a).to(device).to(torch.bfloat16)  # noqa: E731
    layer = ops.MoeLayer(H, E, K, I, T)
    out = layer(d(x), d(router), d(up_gate), d(down))
    torch.cuda.synchronize()
    ids = layer.view("ids", torch.int32, (T, K)).cpu().numpy()
    got = bf16_values(out)
    agree = (ids == want_ids).all(axis=1)
    assert agree.mean() >= 0.75
    magnitude = np.abs(x.astype(np.float64)) @ np.abs(router.astype(np.float64)).T
    for t in np.flatnonzero(~agree):
        dropped = sorted(set(want_ids[t]) - set(ids[t]))
        taken = sorted(set(ids[t]) - set(want_ids[t]))
        for a, b in zip(dropped, taken):
            assert abs(scores[t, a] - scores[t, b]) <= 2.0**-7 * (magnitude[t, a] + magnitude[t, b]), (t, a, b)
    assert_bf16_bar(got[agree], want[agree].astype(np.float64), "tiny fp32 config")


@pytest.mark.parametrize("garbage", [1000, 3])
@pytest.mark.parametrize("tokens", [64, 1])
def test_uncleared_front_counters_fail_loudly_then_clear(device, garbage, tokens):
    """A decode-size call whose workspace counters were not zero before it (a reused buffer): the
    output is NaN, not a quietly wrong result, the counters are cleared, and the next call is
    bit-for-bit the clean one. Garbage past the takers means no workgroup routes; garbage below it
    means a workgroup routes early (on the previous call's scores, here the same ones). The
    workspace still holds the first call's maps, so no kernel reads outside its arrays either way.
    At 64 tokens the front end counts nothing (the words are only checked); at one token the
    expert-split front end counts its workgroups on word 1."""
    hidden, experts, top, intermediate = 2048, 128, 8, 768
    x = normal_bf16((tokens, hidden), 71, device=device)
    router = normal_bf16((experts, hidden), 72, 0.02, device)
    up_gate = normal_bf16((experts, 2 * intermediate, hidden), 73, 0.02, device)
    down = normal_bf16((experts, hidden, intermediate), 74, 0.02, device)
    layer = ops.MoeLayer(hidden, experts, top, intermediate, tokens)
    announce("front counters: clean call", garbage, tokens)
    clean = bf16_bits(layer(x, router, up_gate, down)).copy()
    ticket = layer.view("ticket", torch.int32, (256,))
    words = 1 + (tokens + 15) // 16
    assert (ticket[:words] == 0).all().item()
    ticket[:words] = garbage
    announce("front counters: garbage before the call", garbage, tokens)
    loud = layer(x, router, up_gate, down)
    torch.cuda.synchronize()
    assert torch.isnan(loud.float()).all().item()
    assert (ticket == 0).all().item()
    announce("front counters: the call after", garbage, tokens)
    again = bf16_bits(layer(x, router, up_gate, down))
    assert np.array_equal(again, clean)


@pytest.mark.parametrize("wdtype", ["bf16", "f8e4m3", "f4e2m1"])
def test_prefill_layer_reads_nothing_it_did_not_write(device, wdtype):
    """A prefill-size layer over a workspace whose bytes are all 0x01 (but the front end's counter
    words, which must start at zero) gives the zero workspace's output bit for bit: every
    intermediate is written before it is read, so a reused buffer (the no-alloc scratch, a pool)
    behaves like a fresh one. 0x01 bytes make any unwritten index read a large one."""
    tokens, hidden, experts, top, intermediate = 1024, 2048, 128, 8, 768
    announce("prefill layer over a dirty workspace", wdtype)
    x = normal_bf16((tokens, hidden), 81, device=device)
    router = normal_bf16((experts, hidden), 82, 0.02, device)
    up_gate_bf16 = normal_bf16((experts, 2 * intermediate, hidden), 83, 0.02, device)
    down_bf16 = normal_bf16((experts, hidden, intermediate), 84, 0.02, device)
    _, _, _, _, up_gate, down, kw = quantised(wdtype, up_gate_bf16, down_bf16, device)
    outs = []
    for dirty in (False, True):
        layer = ops.MoeLayer(hidden, experts, top, intermediate, tokens, weight_dtype=wdtype)
        if dirty:
            layer.workspace.fill_(1)
            layer.workspace[:1024].zero_()
        outs.append(bf16_bits(layer(x, router, up_gate, down, **kw)).copy())
    np.testing.assert_array_equal(outs[1], outs[0])

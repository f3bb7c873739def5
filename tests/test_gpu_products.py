"""The grouped products, the combine and the router gemm on the MI355X against the oracle.

Floating point: bf16 outputs against the oracle's FP32 values within BASELINE's bar (max
relative error <= 2e-2 of the peak, mean absolute error <= 1e-3) and within the reference
operator's own bound (``Tolerance::dot`` with the activation envelope,
crates/ops/src/moe/grouped.rs:364-389, :506-523). Rows the operators do not own - a tile's
padding, tiles past ``num_non_exiting_tiles`` - are pre-filled with NaN and must stay NaN:
nothing is written there.
"""

import numpy as np
import pytest
import torch

import oracle_lib as O
from gpu_helpers import (announce, assert_bf16_bar, assert_operator_bound, bf16_bits, bf16_values,
                         normal_bf16, sort_on_host, to_bf16, zipf_bias)
from uniserve_moe import ops

pytestmark = pytest.mark.gpu


def routing(device, tokens, experts, top, skew, seed, emptied=None):
    rng = np.random.default_rng(seed)
    if skew == "zipf":
        p = np.exp(zipf_bias(experts).astype(np.float64))
        ids = np.stack([rng.choice(experts, size=top, replace=False, p=p / p.sum()) for _ in range(tokens)])
    else:
        ids = np.stack([rng.choice(experts, size=top, replace=False) for _ in range(tokens)])
    if emptied is not None:
        ids[ids == emptied] = (emptied + 1) % experts
    return ids.astype(np.int32)


CASES = {
    # name: tokens, hidden, experts, top, intermediate, skew
    "30b decode (stream)": (64, 2048, 128, 8, 768, "uniform"),
    "skewed decode (stream, one-row-block passes over tiles of many rows)": (128, 2048, 128, 8, 768, "zipf"),
    "skewed decode (stream, two-row-block passes over tiles of many rows)": (256, 2048, 128, 8, 768, "zipf"),
    "reference gather shape, emptied expert": (512, 2048, 128, 8, 1536, "uniform"),
    "skewed prefill (tiled)": (1024, 2048, 128, 8, 768, "zipf"),
    "tiny": (16, 256, 8, 2, 128, "uniform"),
    "235b decode one token": (1, 4096, 128, 8, 1536, "uniform"),
    "odd widths (tiled, 64-column slices)": (300, 320, 16, 4, 192, "uniform"),
    "stream, hidden not a multiple of 256 (row-sliced FC1)": (16, 320, 16, 4, 192, "uniform"),
}


@pytest.mark.parametrize("case", list(CASES))
def test_products_and_combine(device, case):
    tokens, hidden, experts, top, intermediate, skew = CASES[case]
    announce("products", case)
    ids_host = routing(device, tokens, experts, top, skew, tokens + hidden,
                       emptied=7 if "emptied" in case else None)
    x = normal_bf16((tokens, hidden), 1, device=device)
    up_gate = normal_bf16((experts, 2 * intermediate, hidden), 2, 0.02, device)
    down = normal_bf16((experts, hidden, intermediate), 3, 0.02, device)
    weights = torch.rand((tokens, top), device=device)
    weights = weights / weights.sum(dim=1, keepdim=True)  # renormalised, as the router writes them
    ids = torch.from_numpy(ids_host).to(device)
    maps = ops.moe_sort(ids, weights, experts)
    rows = ops.permuted_rows(tokens, top, experts)
    gated = torch.full((rows, intermediate), float("nan"), dtype=torch.bfloat16, device=device)
    products = torch.full((rows, hidden), float("nan"), dtype=torch.bfloat16, device=device)
    ops.gather_gemm(x, up_gate, top, maps, rows, out=gated)
    ops.route_gemm(gated, down, maps, out=products)
    combined = ops.moe_unpermute(products, maps[ops.EXPANDED_TO_PERMUTED][: tokens * top], weights)
    torch.cuda.synchronize()

    sort = sort_on_host(maps, tokens, top)
    padded = int(sort["total_padded_tokens"][0])
    live = sort["permuted_to_expanded"][:padded] >= 0
    want_gated = O.gather_gemm(bf16_bits(x), bf16_bits(up_gate), top, sort, rows)
    got_gated = bf16_values(gated)
    assert_bf16_bar(got_gated[:padded][live], want_gated[:padded][live], "gather_gemm")
    assert_operator_bound(got_gated[:padded][live], want_gated[:padded][live], hidden, "gather_gemm")
    assert np.isnan(got_gated[:padded][~live]).all(), "gather_gemm wrote a padding row"
    assert np.isnan(got_gated[padded:]).all(), "gather_gemm wrote past the live tiles"

    # FC2 from the device's own gated rows (the oracle reads the same bf16 inputs).
    gated_bits = bf16_bits(gated)
    gated_bits[padded:] = 0
    gated_bits[:padded][~live] = 0
    want_products = O.route_gemm(gated_bits, bf16_bits(down), sort)
    got_products = bf16_values(products)
    assert_bf16_bar(got_products[:padded][live], want_products[:padded][live], "route_gemm")
    assert_operator_bound(got_products[:padded][live], want_products[:padded][live], intermediate, "route_gemm")
    assert np.isnan(got_products[:padded][~live]).all(), "route_gemm wrote a padding row"

    products_bits = bf16_bits(products)
    want_combined = O.moe_unpermute(products_bits, sort["expanded_to_permuted"].reshape(tokens, top),
                                    weights.cpu().numpy())
    assert_bf16_bar(bf16_values(combined), want_combined, "moe_unpermute")
    assert_operator_bound(bf16_values(combined), want_combined, top, "moe_unpermute", envelope=False)


UNPERMUTE_CASES = ["dropped routes and a token with none", "nothing dropped", "middle routes dropped",
                   "unnamed rows poisoned", "expanded layout"]


@pytest.mark.parametrize("case", UNPERMUTE_CASES)
@pytest.mark.parametrize("scales_dtype", [torch.float32, torch.bfloat16])
def test_unpermute_reference_cases(device, case, scales_dtype):
    """tests/python/kernels/moe/test_moe_unpermute.py:121-265: H=2048, top 8, T=256."""
    announce("unpermute", case, scales_dtype)
    tokens, top, hidden = 256, 8, 2048
    torch.manual_seed(0)
    rows = tokens * top
    routes = (torch.randn(rows, hidden, device=device) * 0.5).to(torch.bfloat16)
    scales = (torch.randn(tokens, top, device=device) * 0.5).to(scales_dtype)
    mapping = torch.randperm(rows, device=device).to(torch.int32).reshape(tokens, top).clone()
    dropped = set()
    if case == "dropped routes and a token with none":
        dropped = {(t, top - 1) for t in range(tokens)} | {(t, 0) for t in range(0, tokens, 3)} | {(0, k) for k in range(top)}
    elif case == "middle routes dropped":
        dropped = {(t, k) for t in range(tokens) for k in range(1, top - 1, 2)}
    elif case == "unnamed rows poisoned":
        dropped = {(t, top - 1) for t in range(tokens)}
    for t, k in dropped:
        mapping[t, k] = -1
    if case == "unnamed rows poisoned":
        named = torch.zeros(rows, dtype=torch.bool, device=device)
        named[mapping[mapping >= 0].long()] = True
        routes[~named] = float("nan")
    layout = 1 if case == "expanded layout" else 0
    before = bf16_bits(routes).copy()
    out = torch.full((tokens, hidden), float("nan"), dtype=torch.bfloat16, device=device)
    ops.moe_unpermute(routes, mapping, scales, out=out, layout=layout)
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(routes), before), "the combine wrote into its inputs"
    want = O.moe_unpermute(bf16_bits(routes), mapping.cpu().numpy(), scales.float().cpu().numpy(), layout)
    got = bf16_values(out)
    empty = (mapping < 0).all(dim=1).cpu().numpy()
    assert (got[empty] == 0).all(), "a token with no route must be exactly zero"
    assert np.isfinite(got).all()
    assert_operator_bound(got[~empty], want[~empty], top, "moe_unpermute", envelope=False)


@pytest.mark.parametrize("tokens,experts,hidden", [(64, 128, 2048), (8192, 128, 2048), (7, 60, 256), (1, 128, 4096)])
def test_router_gemm(device, tokens, experts, hidden):
    announce("router gemm", tokens, experts, hidden)
    x = normal_bf16((tokens, hidden), 5, device=device)
    w = normal_bf16((experts, hidden), 6, 0.02, device)
    scores = ops.router_gemm(x, w)
    torch.cuda.synchronize()
    xh = bf16_values(x)
    wh = bf16_values(w)
    exact = xh @ wh.T
    got = bf16_values(scores)
    # one rounding into bf16 after an FP32 sum: within half a bf16 step plus the sum's bound
    bound = np.abs(exact) * 2.0**-8 + 2 * 2.0**-24 * hidden * (np.abs(xh) @ np.abs(wh).T)
    assert (np.abs(got - exact) <= bound).all()
    if tokens <= 64:
        np.testing.assert_allclose(got, bf16_values(to_bf16(O.router_gemm(bf16_bits(x), bf16_bits(w)), device)),
                                   rtol=2.0**-7, atol=1e-6)

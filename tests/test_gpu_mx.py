"""MX products on the MI355X against the oracle: MXFP4 weights x MXFP8 activations.

The quantiser is bit-exact with the oracle's rule (tests/test_oracle.py pins that rule against
torch's e4m3 cast and the E2M1 table). The products take the same codes and scales on both sides;
the hardware's block scaling is exact (powers of two) and the FP32 sums differ only in order, so
the gap is the bf16 rounding of the outputs: max |got - want| <= 1e-2 of the peak (and the mean
within BASELINE's 1e-3). Parity unpinned against the reference: it has no MX operator (its four-bit
experts are NVFP4).
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


@pytest.mark.parametrize("tokens,hidden,experts,top,intermediate,skew", [
    (64, 2048, 128, 8, 768, "uniform"), (1, 4096, 128, 8, 1536, "uniform"), (512, 2048, 128, 8, 768, "zipf")])
def test_mx_products(device, tokens, hidden, experts, top, intermediate, skew):
    announce("mx products", tokens, hidden, experts, top, intermediate, skew)
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
    gated = torch.full((rows, intermediate), float("nan"), dtype=torch.bfloat16, device=device)
    ops.gather_gemm_mx(xq, xs, d(q1), d(s1), top, maps, rows, out=gated)
    padded_t = maps[ops.TOTAL_PADDED_TOKENS][:1]
    gq, gs = ops.quantize_mxfp8(torch.nan_to_num(gated, 0.0), row_limit=padded_t)
    products = torch.full((rows, hidden), float("nan"), dtype=torch.bfloat16, device=device)
    ops.route_gemm_mx(gq, gs, d(q2), d(s2), maps, out=products)
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

"""Helpers of the GPU parity tests: seeded inputs, host/device moves, the comparison bars."""

import math
import sys

import numpy as np
import torch

import oracle_lib as O


def announce(*what):
    """Names the case before a GPU step, flushed, so a failing run says which case it was."""
    print("[gpu case]", *what, flush=True)
    sys.stdout.flush()


def bf16_bits(tensor):
    """A bf16 device tensor's raw bits as a host uint16 array."""
    return tensor.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def to_bf16(bits, device):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(device)


def bf16_values(tensor):
    return tensor.float().cpu().numpy().astype(np.float64)


def normal_bf16(shape, seed, std=1.0, device="cuda"):
    """Seeded N(0, std) bf16 values, generated on the device by torch."""
    generator = torch.Generator(device=device).manual_seed(seed)
    return (torch.randn(shape, generator=generator, device=device, dtype=torch.float32) * std).to(torch.bfloat16)


def zipf_bias(experts, s=1.1):
    """BASELINE's Zipf(s) skew over expert ids: logit bias -s * ln(e + 1)."""
    return (-s * np.log(np.arange(experts, dtype=np.float64) + 1.0)).astype(np.float32)


def gamma(n, u=2.0**-24):
    t = n * u
    return 1.0 if t >= 1 else t / (1 - t)


def dot_bound(n, out_u=2.0**-8):
    """``Tolerance::dot(n, f32, bf16)`` (crates/ops/src/tolerance.rs:113-137): relative to the peak."""
    return 2.0 * gamma(n) * math.sqrt(n) + out_u


def envelope_atol(n):
    """The grouped products' activation-envelope absolute term (crates/ops/src/moe/grouped.rs:380-388)."""
    return 2.0 * gamma(n) * (8.0 * 8.0 * 2.0)


def assert_bf16_bar(got, want, what, max_rel=2e-2, mean_abs=1e-3):
    """BASELINE's bf16 bar: max |got - want| / max |want| <= 2e-2 and mean |got - want| <= 1e-3."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite values"
    diff = np.abs(got - want)
    peak = max(np.abs(want).max(), 1e-30)
    rel = diff.max() / peak
    mean = diff.mean()
    assert rel <= max_rel and mean <= mean_abs, f"{what}: max rel {rel:.3e}, mean abs {mean:.3e}"
    return rel, mean


def assert_operator_bound(got, want, n, what, envelope=True):
    """The reference operator's own bound: |got - want| <= atol + rtol * peak."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    rtol = dot_bound(n)
    atol = envelope_atol(n) if envelope else 0.0
    peak = np.abs(want).max()
    diff = np.abs(got - want)
    assert (diff <= atol + rtol * peak).all(), f"{what}: max diff {diff.max():.3e} > {atol + rtol * peak:.3e}"


def sort_on_host(maps, tokens, top):
    """The device maps tensor as the oracle's dict."""
    m = maps.cpu().numpy()
    return {
        "tile_to_expert": m[0],
        "tile_to_limit": m[1],
        "expanded_to_permuted": m[2][: tokens * top],
        "permuted_to_expanded": m[3],
        "permuted_to_token": m[4],
        "total_padded_tokens": m[5][:1],
        "num_non_exiting_tiles": m[6][:1],
    }

"""The layer entry that allocates nothing, against the workspace entry (collected last, so that a
failure here cannot hide the other GPU tests).

``uniserve_moe_layer_no_alloc`` runs the same kernels as ``uniserve_moe_layer`` over the library's
per-device scratch instead of a caller workspace, so its output must be the workspace entry's bit
for bit. Two calls in a row on the shared scratch, the second with fewer tokens (the scratch keeps
the first call's contents), then an e4m3 layer.
"""

import ctypes

import numpy as np
import pytest
import torch

from gpu_helpers import announce, bf16_bits, normal_bf16
import oracle_lib as O
from uniserve_moe import ops
from uniserve_moe.abi import ACTIVATION, DTYPE, LayerCall, library

pytestmark = pytest.mark.gpu


def no_alloc(layer, x, router, up_gate, down, **scales):
    """The no-allocation entry, called through the C ABI with the workspace fields left empty."""
    tokens = x.shape[0]
    out = torch.full((tokens, layer.hidden_size), float("nan"), dtype=torch.bfloat16, device=x.device)
    call = LayerCall()
    call.hidden, call.router, call.up_gate, call.down = x.data_ptr(), router.data_ptr(), up_gate.data_ptr(), down.data_ptr()
    s1, s2 = scales.get("up_gate_scales"), scales.get("down_scales")
    call.up_gate_scales = None if s1 is None else s1.data_ptr()
    call.down_scales = None if s2 is None else s2.data_ptr()
    call.out = out.data_ptr()
    call.tokens, call.hidden_size, call.experts = tokens, layer.hidden_size, layer.experts
    call.top, call.intermediate, call.renormalize = layer.top, layer.intermediate, 1
    call.weight_dtype = DTYPE[layer.weight_dtype]
    call.multiprocessors = ops.multiprocessors(x.device)
    call.activation = ACTIVATION["silu"]
    stream = ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)
    status = library().uniserve_moe_layer_no_alloc(ctypes.byref(call), stream)
    assert status == 0, bytes(call.error).split(b"\0", 1)[0].decode()
    return out


def inputs(device, tokens, hidden, experts, intermediate, seed):
    x = normal_bf16((tokens, hidden), seed, device=device)
    router = normal_bf16((experts, hidden), seed + 1, 0.02, device)
    up_gate = normal_bf16((experts, 2 * intermediate, hidden), seed + 2, 0.02, device)
    down = normal_bf16((experts, hidden, intermediate), seed + 3, 0.02, device)
    return x, router, up_gate, down


def test_no_alloc_layer_is_the_workspace_layer_bit_for_bit(device):
    hidden, experts, top, intermediate = 2048, 128, 8, 768
    x, router, up_gate, down = inputs(device, 64, hidden, experts, intermediate, 90)
    want = {}
    for tokens in (64, 16):
        announce("no-alloc reference (workspace entry)", tokens)
        layer = ops.MoeLayer(hidden, experts, top, intermediate, tokens)
        want[tokens] = bf16_bits(layer(x[:tokens].contiguous(), router, up_gate, down)).copy()
    for tokens in (64, 16):  # two calls in a row on the shared scratch, the second smaller
        announce("no-alloc layer", tokens)
        layer = ops.MoeLayer(hidden, experts, top, intermediate, tokens)
        got = no_alloc(layer, x[:tokens].contiguous(), router, up_gate, down)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bf16_bits(got), want[tokens], err_msg=f"{tokens} tokens")


def test_no_alloc_fp8_layer_is_the_workspace_layer_bit_for_bit(device):
    hidden, experts, top, intermediate, tokens = 2048, 128, 8, 768, 1024
    announce("no-alloc fp8 layer", tokens)
    x, router, up_gate, down = inputs(device, tokens, hidden, experts, intermediate, 95)
    q1, s1 = O.quantize_blocks_fp8(bf16_bits(up_gate))
    q2, s2 = O.quantize_blocks_fp8(bf16_bits(down))
    d = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    scales = dict(up_gate_scales=d(s1), down_scales=d(s2))
    layer = ops.MoeLayer(hidden, experts, top, intermediate, tokens, weight_dtype="f8e4m3")
    want = bf16_bits(layer(x, router, d(q1), d(q2), **scales)).copy()
    got = no_alloc(layer, x, router, d(q1), d(q2), **scales)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bf16_bits(got), want)

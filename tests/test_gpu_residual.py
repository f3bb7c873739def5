"""sigmoid_gated_add on the MI355X against the oracle (crates/ops/src/residual.rs:797-898).

The operator's own bound (residual.rs:887-897): the sigmoid's few FP32 ulps, one product and one
sum, rounded once into the target's type, relative to the output's largest magnitude (the sum may
cancel): rtol = 2 u(dtype) + 4 u(f32).
"""

import ctypes

import numpy as np
import pytest
import torch

import oracle_lib as O
from gpu_helpers import announce
from uniserve_moe import ops

pytestmark = pytest.mark.gpu

U = {torch.bfloat16: 2.0**-8, torch.float16: 2.0**-11, torch.float32: 2.0**-24}
KIND = {torch.bfloat16: 1, torch.float16: 2, torch.float32: 0}


def host_bits(t):
    a = t.cpu()
    return a.numpy() if a.dtype == torch.float32 else a.view(torch.int16).numpy().view(np.uint16)


def values(bits, dtype):
    if dtype == torch.float32:
        return bits.astype(np.float64)
    if dtype == torch.float16:
        return bits.view(np.float16).astype(np.float64)
    return O.bf16_decode(bits).astype(np.float64)


CASES = [
    ("reference 3x4 f32", 3, 4, torch.float32),
    ("decode rows bf16", 64, 2048, torch.bfloat16),
    ("prefill rows bf16", 8192, 2048, torch.bfloat16),
    ("odd width f16", 7, 1001, torch.float16),
    ("ragged tail bf16", 5, 2050, torch.bfloat16),
    ("more rows than a grid axis f32", 70000, 8, torch.float32),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_sigmoid_gated_add_against_the_oracle(device, case):
    name, rows, columns, dtype = case
    announce("sigmoid_gated_add", name)
    g = torch.Generator(device="cpu").manual_seed(rows * 131 + columns)
    target = torch.randn((rows, columns), generator=g).to(dtype).to(device)
    update = torch.randn((rows, columns), generator=g).to(dtype).to(device)
    gate = (3.0 * torch.randn((rows, 1), generator=g)).to(dtype).to(device)
    before = host_bits(target)
    alias = target.view(-1)
    out = ops.sigmoid_gated_add_(target, update, gate)
    torch.cuda.synchronize()
    assert out.data_ptr() == target.data_ptr()
    want = O.sigmoid_gated_add(before, host_bits(update), host_bits(gate).reshape(rows), KIND[dtype])
    got_v, want_v = values(host_bits(out), dtype), values(want, dtype)
    bound = (2 * U[dtype] + 4 * 2.0**-24) * np.abs(want_v).max()
    assert np.abs(got_v - want_v).max() <= bound, name
    assert torch.equal(alias.view(rows, columns), out)  # updated in its own storage


def test_sigmoid_gated_add_code_object_launched_by_name(device):
    """The reference's launch words (target, update, gate, columns i32) on (ceil(columns / block), rows)."""
    announce("sigmoid_gated_add code object")
    from uniserve_moe.abi import residual_code_object_path

    hip = ctypes.CDLL("libamdhip64.so")
    module = ctypes.c_void_p()
    assert hip.hipModuleLoad(ctypes.byref(module), str(residual_code_object_path()).encode()) == 0
    function = ctypes.c_void_p()
    assert hip.hipModuleGetFunction(ctypes.byref(function), module, b"uniserve_sigmoid_gated_add_bf16") == 0
    rows, columns, block = 9, 4096 + 16, 2048
    g = torch.Generator(device="cpu").manual_seed(5)
    target = torch.randn((rows, columns), generator=g).to(torch.bfloat16).to(device)
    update = torch.randn((rows, columns), generator=g).to(torch.bfloat16).to(device)
    gate = torch.randn((rows, 1), generator=g).to(torch.bfloat16).to(device)
    before = host_bits(target)
    words = [ctypes.c_void_p(target.data_ptr()), ctypes.c_void_p(update.data_ptr()), ctypes.c_void_p(gate.data_ptr()),
             ctypes.c_int32(columns)]
    params = (ctypes.c_void_p * 4)(*[ctypes.cast(ctypes.pointer(w), ctypes.c_void_p) for w in words])
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    grid = (columns + block - 1) // block
    assert hip.hipModuleLaunchKernel(function, grid, rows, 1, 256, 1, 1, 0, stream, params, None) == 0
    torch.cuda.synchronize()
    hip.hipModuleUnload(module)
    want = values(O.sigmoid_gated_add(before, host_bits(update), host_bits(gate).reshape(rows), 1), torch.bfloat16)
    got = values(host_bits(target), torch.bfloat16)
    assert np.abs(got - want).max() <= (2 * 2.0**-8 + 4 * 2.0**-24) * np.abs(want).max()

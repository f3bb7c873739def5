"""The C ABI without a GPU: layouts, exports and refusals.

* every size and offset a header of ``include/`` asserts is the ctypes mirror's (the
  reference's kernel checks assert the same against its generated headers,
  tests/python/kernels/moe/test_moe_sort.py:87-89);
* the shared object exports every entry the headers declare, and the router's code object
  holds the kernel by its reference name;
* the entries refuse what the reference's entries refuse, with a message in the call's error
  buffer and a nonzero status, before anything is launched
  (crates/ops/kernels/moe_sort/trtllm/src/entry.cpp:26-70, gather_gemm/cute_dsl/src/entry.cpp:18-42,
  moe_unpermute/trtllm/src/entry.cpp:76-107, crates/ops/src/moe/routing.rs:127-238).
"""

import ctypes
import re
from pathlib import Path

import pytest

from uniserve_moe import abi

ROOT = Path(__file__).resolve().parent.parent
HEADERS = sorted((ROOT / "include").glob("*.h"))

MIRRORS = {
    "uniserve_moe_sort_call": abi.SortCall,
    "uniserve_gather_call": abi.GatherCall,
    "uniserve_route_call": abi.RouteCall,
    "uniserve_unpermute_call": abi.UnpermuteCall,
    "UniserveGemmCall": abi.GemmCall,
}


def asserted_layouts():
    sizes, offsets = {}, {}
    for header in HEADERS:
        text = header.read_text()
        for name, size in re.findall(r"static_assert\(sizeof\((\w+)\) == (\d+)", text):
            sizes[name] = int(size)
        for name, field, offset in re.findall(r"static_assert\(offsetof\((\w+), (\w+)\) == (\d+)", text):
            offsets.setdefault(name, {})[field] = int(offset)
    return sizes, offsets


def test_every_asserted_layout_is_the_mirror_s():
    sizes, offsets = asserted_layouts()
    assert set(sizes) == set(MIRRORS)
    for name, mirror in MIRRORS.items():
        assert ctypes.sizeof(mirror) == sizes[name], name
        fields = {f[0] for f in mirror._fields_}
        assert set(offsets[name]) == fields, name
        for field, offset in offsets[name].items():
            assert getattr(mirror, field).offset == offset, (name, field)


def test_reference_layout_sizes():
    # The sizes the reference's generated headers assert: crates/ops/python/src/uniserve_kernels/include/
    # uniserve_moe_sort.h:59, uniserve_gather_gemm.h:43, uniserve_route_gemm.h:41,
    # uniserve_moe_unpermute.h:56, uniserve_gemm.h:71.
    assert ctypes.sizeof(abi.SortCall) == 648
    assert ctypes.sizeof(abi.GatherCall) == 632
    assert ctypes.sizeof(abi.RouteCall) == 616
    assert ctypes.sizeof(abi.UnpermuteCall) == 608
    assert ctypes.sizeof(abi.GemmCall) == 600


def declared_entries():
    names = set()
    for header in HEADERS:
        text = header.read_text()
        names.update(re.findall(r"UNISERVE_EXTERN_C\s+[\w\s\*]+?\b(uniserve_\w+)\s*\(", text))
    return names


def test_the_library_exports_every_declared_entry():
    lib = abi.library()
    names = declared_entries()
    assert {"uniserve_moe_sort", "uniserve_gather_gemm", "uniserve_route_gemm", "uniserve_moe_unpermute",
            "uniserve_gemm", "uniserve_topk_softmax_launch", "uniserve_moe_layer"} <= names
    for name in sorted(names):
        assert hasattr(lib, name), name
    # The router kernel, by the name the reference's operator launches.
    assert hasattr(lib, "uniserve_topk_softmax")
    assert b"uniserve_topk_softmax" in abi.code_object_path().read_bytes()
    for kernel in (b"uniserve_sigmoid_gated_add_bf16", b"uniserve_sigmoid_gated_add_f16", b"uniserve_sigmoid_gated_add_f32"):
        assert hasattr(lib, kernel.decode())
        assert kernel in abi.residual_code_object_path().read_bytes()


def message(call):
    return bytes(call.error).split(b"\0", 1)[0].decode()


def test_sort_refusals():
    lib = abi.library()
    call = abi.SortCall()
    assert lib.uniserve_moe_sort(ctypes.byref(call), None) != 0
    assert "seven metadata buffers" in message(call)
    buffers = (ctypes.c_int32 * 4096)()
    for name in ("ids", "tile_to_expert", "tile_to_limit", "expanded_to_permuted", "permuted_to_expanded",
                 "permuted_to_token", "total_padded_tokens", "num_non_exiting_tiles"):
        setattr(call, name, ctypes.addressof(buffers))
    call.tokens, call.top, call.experts, call.local_experts, call.tile_tokens = 4, 2, 8, 8, 128
    call.scales_dtype = abi.DTYPE["i32"]
    assert lib.uniserve_moe_sort(ctypes.byref(call), None) != 0
    assert "route weights" in message(call)
    call.scales_dtype = abi.DTYPE["f32"]
    call.local_offset = 4
    assert lib.uniserve_moe_sort(ctypes.byref(call), None) != 0
    assert "window" in message(call)
    call.local_offset, call.local_experts, call.experts = 0, 1 << 20, 1 << 20
    assert lib.uniserve_moe_sort(ctypes.byref(call), None) != 0
    assert "LDS" in message(call)
    # The one-launch path keeps (3 + 16 waves) counters per local expert in 64 KB of LDS: 862 at
    # most; more local experts (at any route count) are refused, never launched.
    call.local_experts, call.experts, call.tokens, call.top = 863, 1100, 1024, 8
    assert lib.uniserve_moe_sort(ctypes.byref(call), None) != 0
    assert "LDS" in message(call)
    assert lib.uniserve_moe_sort(None, None) != 0


def test_product_refusals():
    lib = abi.library()
    g = abi.GatherCall()
    g.dtype = abi.DTYPE["f16"]
    assert lib.uniserve_gather_gemm(ctypes.byref(g), None) != 0 and "bf16 only" in message(g)
    g.dtype = abi.DTYPE["bf16"]
    assert lib.uniserve_gather_gemm(ctypes.byref(g), None) != 0 and "needs hidden" in message(g)
    buf = (ctypes.c_uint8 * 64)()
    for name in ("hidden", "weights", "out", "tile_to_expert", "tile_to_limit", "permuted_to_expanded",
                 "num_non_exiting_tiles"):
        setattr(g, name, ctypes.addressof(buf))
    g.width, g.hidden_size, g.multiprocessors, g.tokens, g.top, g.experts = 3, 2048, 256, 4, 2, 8
    assert lib.uniserve_gather_gemm(ctypes.byref(g), None) != 0 and "even" in message(g)
    g.width = 1536
    g.multiprocessors = 0
    assert lib.uniserve_gather_gemm(ctypes.byref(g), None) != 0 and "multiprocessor" in message(g)
    g.multiprocessors = 256
    g.permuted_rows = 4
    assert lib.uniserve_gather_gemm(ctypes.byref(g), None) != 0 and "cannot hold" in message(g)

    # The prefill kernels address gathered hidden rows with 32-bit offsets: a hidden array of
    # exactly 4 GiB passes that check (and meets the next refusal), one row more is refused.
    g.hidden_size, g.permuted_rows = 4096, 4
    g.tokens = (1 << 32) // (4096 * 2)
    assert lib.uniserve_gather_gemm(ctypes.byref(g), None) != 0 and "cannot hold" in message(g)
    g.tokens += 1
    assert lib.uniserve_gather_gemm(ctypes.byref(g), None) != 0 and "below 4 GiB" in message(g)
    for call_type, entry, hidden in ((abi.GatherFp8Call, lib.uniserve_gather_gemm_fp8, 4096),
                                     (abi.GatherMxCall, lib.uniserve_gather_gemm_mx, 4096)):
        c = call_type()
        for name in ("hidden", "hidden_scales", "weights", "weight_scales", "out", "tile_to_expert",
                     "tile_to_limit", "permuted_to_expanded", "num_non_exiting_tiles"):
            setattr(c, name, ctypes.addressof(buf))
        c.out_dtype, c.multiprocessors, c.hidden_size, c.width, c.top, c.experts = abi.DTYPE["bf16"], 256, hidden, 1536, 8, 128
        if hasattr(c, "block_n"):
            c.block_n = c.block_k = 128
        c.permuted_rows, c.tokens = 128, (1 << 32) // hidden
        assert entry(ctypes.byref(c), None) != 0 and "whole 128-row tiles" in message(c)
        c.tokens += 1
        assert entry(ctypes.byref(c), None) != 0 and "below 4 GiB" in message(c)

    # The MXFP4 FC2's stream kernel (few routes per expert) addresses every permuted row from the
    # array's base with 32-bit offsets: rows past 4 GiB are refused before any launch.
    m = abi.RouteMxCall()
    for name in ("rows", "row_scales", "weights", "weight_scales", "out", "tile_to_expert", "tile_to_limit",
                 "permuted_to_expanded", "num_non_exiting_tiles"):
        setattr(m, name, ctypes.addressof(buf))
    m.out_dtype, m.multiprocessors, m.intermediate, m.width, m.experts = abi.DTYPE["bf16"], 256, 1536, 2048, 1 << 16
    m.permuted_rows = 128 * ((1 << 32) // (1536 * 128) + 1)  # just past 4 GiB, far under 24 routes per expert
    assert lib.uniserve_route_gemm_mx(ctypes.byref(m), None) != 0 and "below 4 GiB" in message(m)

    r = abi.RouteCall()
    r.dtype = abi.DTYPE["f32"]
    assert lib.uniserve_route_gemm(ctypes.byref(r), None) != 0 and "bf16 only" in message(r)

    u = abi.UnpermuteCall()
    u.input_dtype, u.output_dtype = abi.DTYPE["bf16"], abi.DTYPE["f32"]
    assert lib.uniserve_moe_unpermute(ctypes.byref(u), None) != 0 and "one input and output" in message(u)
    u.output_dtype = abi.DTYPE["bf16"]
    for name in ("routes", "out", "expanded_to_permuted", "scales"):
        setattr(u, name, ctypes.addressof(buf))
    u.hidden, u.top, u.tokens = 12, 2, 1
    assert lib.uniserve_moe_unpermute(ctypes.byref(u), None) != 0 and "8-element" in message(u)

    q = abi.GemmCall()
    assert lib.uniserve_gemm(ctypes.byref(q), None) != 0 and "needs out" in message(q)


def test_router_refusals():
    lib = abi.library()
    error = ctypes.create_string_buffer(512)
    buf = (ctypes.c_uint8 * 64)()
    p = ctypes.addressof(buf)

    def launch(kind=1, experts=128, top=8, rows=4, stride=128, scale_kind=-1):
        return lib.uniserve_topk_softmax_launch(p, kind, stride, rows, experts, top, 1, None, scale_kind,
                                                p, p, None, None, None, None, error, 512)

    assert launch(kind=7) != 0 and b"routeable" in error.value
    assert launch(experts=0) != 0 and b"at least one expert" in error.value
    assert launch(top=9, experts=8, stride=8) != 0 and b"outside" in error.value
    assert launch(experts=2048, stride=2048) != 0 and b"1024" in error.value
    assert launch(top=33, experts=64, stride=64) != 0 and b"32 picks" in error.value
    assert launch(stride=64) != 0 and b"overlap" in error.value
    assert launch(scale_kind=0) != 0 and b"scale" in error.value
    assert launch(rows=0) == 0  # nothing to route launches nothing


def test_layer_workspace_and_refusals():
    lib = abi.library()
    assert lib.uniserve_moe_max_tiles(64, 8, 128, 128) == 131
    assert lib.uniserve_moe_layer_workspace(64, 2048, 128, 8, 768, abi.DTYPE["bf16"]) > 0
    assert lib.uniserve_moe_layer_workspace(64, 2048, 128, 8, 768, abi.DTYPE["f16"]) == -1
    call = abi.LayerCall()
    assert lib.uniserve_moe_layer(ctypes.byref(call), None) != 0 and "needs hidden" in message(call)
    # The routing fields: a window outside the router's experts and an unknown gate are refused
    # before anything launches (the pointers are never dereferenced).
    p = 1 << 20
    for name in ("hidden", "router", "up_gate", "down", "out", "workspace"):
        setattr(call, name, p)
    call.tokens, call.hidden_size, call.experts, call.top, call.intermediate = 64, 2048, 128, 8, 768
    call.weight_dtype = abi.DTYPE["bf16"]
    call.workspace_bytes = lib.uniserve_moe_layer_workspace(64, 2048, 128, 8, 768, abi.DTYPE["bf16"])
    call.local_offset, call.local_experts = 100, 40
    assert lib.uniserve_moe_layer(ctypes.byref(call), None) != 0 and "window" in message(call)
    call.local_offset, call.local_experts, call.activation = 0, 0, 2
    assert lib.uniserve_moe_layer(ctypes.byref(call), None) != 0 and "silu or gelu_tanh" in message(call)
    # The entry without a workspace refuses extents beyond its scratch before touching a device.
    call.activation, call.tokens, call.weight_dtype = 0, 8192, abi.DTYPE["f8e4m3"]
    assert lib.uniserve_moe_layer_no_alloc(ctypes.byref(call), None) != 0 and "scratch" in message(call)


def test_sigmoid_gated_add_refusals():
    """The operator's refusals (crates/ops/src/residual.rs:820-853), before any launch."""
    lib = abi.library()
    error = ctypes.create_string_buffer(512)
    p = ctypes.c_void_p(16)
    assert lib.uniserve_sigmoid_gated_add_launch(p, p, p, 4, 0, abi.DTYPE["bf16"], None, error, 512) != 0
    assert b"zero elements" in error.value
    assert lib.uniserve_sigmoid_gated_add_launch(p, p, p, 1 << 20, 1 << 12, abi.DTYPE["bf16"], None, error, 512) != 0
    assert b"32-bit" in error.value
    assert lib.uniserve_sigmoid_gated_add_launch(None, p, p, 4, 8, abi.DTYPE["bf16"], None, error, 512) != 0
    assert lib.uniserve_sigmoid_gated_add_launch(p, p, p, 4, 8, abi.DTYPE["f8e4m3"], None, error, 512) != 0
    assert b"bf16, f16 or f32" in error.value
    assert lib.uniserve_sigmoid_gated_add_launch(None, None, None, 0, 8, abi.DTYPE["bf16"], None, error, 512) == 0


# The call structures of this library's own entries (no reference layout to assert against): the
# C compiler's sizes and offsets, read from a program built against include/*.h, are the mirror's.
OWN = {
    "uniserve_quantize_fp8_call": (abi.QuantizeFp8Call, {}),
    "uniserve_gather_fp8_call": (abi.GatherFp8Call, {}),
    "uniserve_route_fp8_call": (abi.RouteFp8Call, {}),
    "uniserve_quantize_mxfp8_call": (abi.QuantizeMxfp8Call, {}),
    "uniserve_gather_mx_call": (abi.GatherMxCall, {}),
    "uniserve_route_mx_call": (abi.RouteMxCall, {}),
    "uniserve_mx_stage_scales_call": (abi.MxStageScalesCall, {"input": "in"}),
    "uniserve_moe_layer_call": (abi.LayerCall, {}),
    "uniserve_moe_layer_views": (abi.LayerViews, {}),
    "uniserve_moe_sort_call": (abi.SortCall, {}),
    "uniserve_gather_call": (abi.GatherCall, {}),
    "uniserve_route_call": (abi.RouteCall, {}),
    "uniserve_unpermute_call": (abi.UnpermuteCall, {}),
}


def test_own_structures_match_the_compiler(tmp_path):
    import shutil
    import subprocess

    compiler = shutil.which("g++") or shutil.which("c++")
    if compiler is None:
        pytest.skip("no host C++ compiler")
    lines = ["#include <cstddef>", "#include <cstdio>"]
    lines += [f'#include "{h.name}"' for h in HEADERS]
    lines.append("int main() {")
    for struct, (mirror, renames) in OWN.items():
        lines.append(f'  std::printf("%s size %zu\\n", "{struct}", sizeof({struct}));')
        for field, _ in mirror._fields_:
            name = renames.get(field, field)
            lines.append(f'  std::printf("%s %s %zu\\n", "{struct}", "{field}", offsetof({struct}, {name}));')
    lines.append("  return 0;\n}")
    source = tmp_path / "layouts.cpp"
    source.write_text("\n".join(lines) + "\n")
    binary = tmp_path / "layouts"
    subprocess.run([compiler, "-std=c++17", "-I", str(ROOT / "include"), str(source), "-o", str(binary)], check=True)
    output = subprocess.run([str(binary)], check=True, capture_output=True, text=True).stdout.split("\n")
    measured = {}
    for line in output:
        if line:
            struct, field, value = line.split()
            measured[(struct, field)] = int(value)
    for struct, (mirror, _) in OWN.items():
        assert ctypes.sizeof(mirror) == measured[(struct, "size")], struct
        for field, _ in mirror._fields_:
            assert getattr(mirror, field).offset == measured[(struct, field)], (struct, field)


def test_a_missing_library_fails_loudly(monkeypatch, tmp_path):
    """No fallback: without the built shared object every operator raises instead of computing
    anything another way."""
    import torch

    from uniserve_moe import ops

    monkeypatch.setattr(abi, "_LIBRARY", None)
    monkeypatch.setattr(abi, "library_path", lambda: tmp_path / "absent.so")
    with pytest.raises(RuntimeError, match="is not built"):
        abi.library()
    with pytest.raises(RuntimeError, match="is not built"):
        ops.quantize_mxfp8(torch.zeros((1, 128), dtype=torch.bfloat16))

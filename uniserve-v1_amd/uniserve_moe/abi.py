"""The call structures and entry points of ``libuniserve_moe_hip.so``, field for field.

Each structure restates one header of ``include/`` (itself the reference's generated
header, e.g. ``crates/ops/python/src/uniserve_kernels/include/uniserve_moe_sort.h``); the
tests compare every size and offset with the header's ``static_assert`` lines.
"""

import ctypes
import os
from pathlib import Path

#: ``uniserve_dtype`` (crates/ops/src/abi.rs:79-92).
# FC1's gate (uniserve_activation); the FC1 entries take it by name, the layer call as a field.
ACTIVATION = {"silu": 0, "gelu_tanh": 1}
ENTRY_SUFFIX = {"silu": "", "gelu_tanh": "_gelu_tanh"}

DTYPE = {
    "u8": 0,
    "i32": 1,
    "i64": 2,
    "f16": 3,
    "bf16": 4,
    "f32": 5,
    "f8e4m3": 6,
    "f4e2m1": 7,
    "i16": 8,
    "u32": 9,
    "f64": 10,
}

LAYOUT_PERMUTED = 0
LAYOUT_EXPANDED = 1

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_ERR = ctypes.c_char * 512


class SortCall(ctypes.Structure):
    """``uniserve_moe_sort_call`` (648 bytes)."""

    _fields_ = [
        ("ids", _P),
        ("scales", _P),
        ("tile_to_expert", _P),
        ("tile_to_limit", _P),
        ("expanded_to_permuted", _P),
        ("permuted_to_expanded", _P),
        ("total_padded_tokens", _P),
        ("num_non_exiting_tiles", _P),
        ("tokens", _I64),
        ("top", _I64),
        ("experts", _I64),
        ("local_experts", _I64),
        ("local_offset", _I64),
        ("tile_tokens", _I64),
        ("scales_dtype", _I64),
        ("error", _ERR),
        ("live_tokens", _P),
        ("permuted_to_token", _P),
    ]


class GatherCall(ctypes.Structure):
    """``uniserve_gather_call`` (632 bytes)."""

    _fields_ = [
        ("hidden", _P),
        ("weights", _P),
        ("out", _P),
        ("tile_to_expert", _P),
        ("tile_to_limit", _P),
        ("permuted_to_expanded", _P),
        ("num_non_exiting_tiles", _P),
        ("tokens", _I64),
        ("permuted_rows", _I64),
        ("width", _I64),
        ("hidden_size", _I64),
        ("experts", _I64),
        ("top", _I64),
        ("dtype", _I64),
        ("multiprocessors", _I64),
        ("error", _ERR),
    ]


class RouteCall(ctypes.Structure):
    """``uniserve_route_call`` (616 bytes)."""

    _fields_ = [
        ("rows", _P),
        ("weights", _P),
        ("out", _P),
        ("tile_to_expert", _P),
        ("tile_to_limit", _P),
        ("permuted_to_expanded", _P),
        ("num_non_exiting_tiles", _P),
        ("permuted_rows", _I64),
        ("width", _I64),
        ("intermediate", _I64),
        ("experts", _I64),
        ("dtype", _I64),
        ("multiprocessors", _I64),
        ("error", _ERR),
    ]


class UnpermuteCall(ctypes.Structure):
    """``uniserve_unpermute_call`` (608 bytes)."""

    _fields_ = [
        ("routes", _P),
        ("out", _P),
        ("expanded_to_permuted", _P),
        ("scales", _P),
        ("tokens", _I64),
        ("top", _I64),
        ("hidden", _I64),
        ("routes_rows", _I64),
        ("input_dtype", _I64),
        ("scales_dtype", _I64),
        ("output_dtype", _I64),
        ("layout", _I64),
        ("error", _ERR),
    ]


class GemmCall(ctypes.Structure):
    """``UniserveGemmCall`` (600 bytes)."""

    _fields_ = [
        ("out", _P),
        ("input", _P),
        ("weight", _P),
        ("bias", _P),
        ("m", _I64),
        ("n", _I64),
        ("k", _I64),
        ("input_row_stride", _I64),
        ("weight_row_stride", _I64),
        ("out_row_stride", _I64),
        ("alpha", ctypes.c_float),
        ("error", _ERR),
    ]


class QuantizeFp8Call(ctypes.Structure):
    """``uniserve_quantize_fp8_call``."""

    _fields_ = [
        ("input", _P),
        ("out", _P),
        ("scales", _P),
        ("row_limit", _P),
        ("rows", _I64),
        ("width", _I64),
        ("input_dtype", _I64),
        ("group", _I64),
        ("error", _ERR),
    ]


class GatherFp8Call(ctypes.Structure):
    """``uniserve_gather_fp8_call``."""

    _fields_ = [
        ("hidden", _P),
        ("hidden_scales", _P),
        ("weights", _P),
        ("weight_scales", _P),
        ("out", _P),
        ("tile_to_expert", _P),
        ("tile_to_limit", _P),
        ("permuted_to_expanded", _P),
        ("num_non_exiting_tiles", _P),
        ("tokens", _I64),
        ("permuted_rows", _I64),
        ("width", _I64),
        ("hidden_size", _I64),
        ("experts", _I64),
        ("top", _I64),
        ("block_n", _I64),
        ("block_k", _I64),
        ("out_dtype", _I64),
        ("multiprocessors", _I64),
        ("error", _ERR),
    ]


class RouteFp8Call(ctypes.Structure):
    """``uniserve_route_fp8_call``."""

    _fields_ = [
        ("rows", _P),
        ("row_scales", _P),
        ("weights", _P),
        ("weight_scales", _P),
        ("out", _P),
        ("tile_to_expert", _P),
        ("tile_to_limit", _P),
        ("permuted_to_expanded", _P),
        ("num_non_exiting_tiles", _P),
        ("permuted_rows", _I64),
        ("width", _I64),
        ("intermediate", _I64),
        ("experts", _I64),
        ("block_n", _I64),
        ("block_k", _I64),
        ("out_dtype", _I64),
        ("multiprocessors", _I64),
        ("error", _ERR),
    ]


class QuantizeMxfp8Call(ctypes.Structure):
    """``uniserve_quantize_mxfp8_call``."""

    _fields_ = [
        ("input", _P),
        ("out", _P),
        ("scales", _P),
        ("row_limit", _P),
        ("rows", _I64),
        ("width", _I64),
        ("input_dtype", _I64),
        ("error", _ERR),
    ]


class GatherMxCall(ctypes.Structure):
    """``uniserve_gather_mx_call``."""

    _fields_ = [
        ("hidden", _P),
        ("hidden_scales", _P),
        ("weights", _P),
        ("weight_scales", _P),
        ("out", _P),
        ("tile_to_expert", _P),
        ("tile_to_limit", _P),
        ("permuted_to_expanded", _P),
        ("num_non_exiting_tiles", _P),
        ("tokens", _I64),
        ("permuted_rows", _I64),
        ("width", _I64),
        ("hidden_size", _I64),
        ("experts", _I64),
        ("top", _I64),
        ("out_dtype", _I64),
        ("multiprocessors", _I64),
        ("weight_scale_layout", _I64),
        ("error", _ERR),
    ]


class RouteMxCall(ctypes.Structure):
    """``uniserve_route_mx_call``."""

    _fields_ = [
        ("rows", _P),
        ("row_scales", _P),
        ("weights", _P),
        ("weight_scales", _P),
        ("out", _P),
        ("tile_to_expert", _P),
        ("tile_to_limit", _P),
        ("permuted_to_expanded", _P),
        ("num_non_exiting_tiles", _P),
        ("permuted_rows", _I64),
        ("width", _I64),
        ("intermediate", _I64),
        ("experts", _I64),
        ("out_dtype", _I64),
        ("multiprocessors", _I64),
        ("weight_scale_layout", _I64),
        ("error", _ERR),
    ]


class MxStageScalesCall(ctypes.Structure):
    """``uniserve_mx_stage_scales_call``."""

    _fields_ = [
        ("input", _P),
        ("out", _P),
        ("stacks", _I64),
        ("rows", _I64),
        ("width", _I64),
        ("error", _ERR),
    ]


class LayerCall(ctypes.Structure):
    """``uniserve_moe_layer_call``."""

    _fields_ = [
        ("hidden", _P),
        ("router", _P),
        ("up_gate", _P),
        ("down", _P),
        ("up_gate_scales", _P),
        ("down_scales", _P),
        ("router_bias", _P),
        ("out", _P),
        ("workspace", _P),
        ("live_tokens", _P),
        ("workspace_bytes", _I64),
        ("tokens", _I64),
        ("hidden_size", _I64),
        ("experts", _I64),
        ("top", _I64),
        ("intermediate", _I64),
        ("renormalize", _I64),
        ("weight_dtype", _I64),
        ("multiprocessors", _I64),
        ("weight_scale_layout", _I64),
        ("error", _ERR),
        ("map", _P),
        ("load", _P),
        ("local_offset", _I64),
        ("local_experts", _I64),
        ("activation", _I64),
    ]


class LayerViews(ctypes.Structure):
    """``uniserve_moe_layer_views``: byte offsets into the layer's workspace."""

    _fields_ = [
        (name, _I64)
        for name in (
            "ticket",
            "scores",
            "ids",
            "weights",
            "tile_to_expert",
            "tile_to_limit",
            "expanded_to_permuted",
            "permuted_to_expanded",
            "permuted_to_token",
            "total_padded_tokens",
            "num_non_exiting_tiles",
            "gated",
            "products",
            "hidden_q",
            "hidden_s",
            "gated_q",
            "gated_s",
            "hidden_route_s",
            "route_scales",
            "max_tiles",
            "permuted_rows",
            "total",
        )
    ]


def max_tiles(tokens, top, local_experts, tile=128):
    """``ops::moe::max_tiles`` (crates/ops/src/moe/mod.rs:63-70)."""
    expanded = tokens * top
    if expanded <= local_experts or tile == 0:
        return expanded
    return (expanded + (tile - 1) * local_experts) // tile


_PACKAGE = Path(__file__).resolve().parent.parent


def library_path():
    """The built shared object, in the package directory (built by its Makefile)."""
    return _PACKAGE / "libuniserve_moe_hip.so"


def code_object_path():
    """The router's standalone code object (``uniserve_topk_softmax`` by name)."""
    return _PACKAGE / "uniserve_topk_softmax.hsaco"


def residual_code_object_path():
    """The shared-expert join's code object (``uniserve_sigmoid_gated_add_{bf16,f16,f32}``)."""
    return _PACKAGE / "uniserve_residual.hsaco"


_LIBRARY = None

_ENTRIES = {
    "uniserve_moe_sort": SortCall,
    "uniserve_gather_gemm": GatherCall,
    "uniserve_gather_gemm_gelu_tanh": GatherCall,
    "uniserve_route_gemm": RouteCall,
    "uniserve_moe_unpermute": UnpermuteCall,
    "uniserve_gemm": GemmCall,
    "uniserve_quantize_fp8": QuantizeFp8Call,
    "uniserve_gather_gemm_fp8": GatherFp8Call,
    "uniserve_gather_gemm_fp8_gelu_tanh": GatherFp8Call,
    "uniserve_route_gemm_fp8": RouteFp8Call,
    "uniserve_moe_layer": LayerCall,
    "uniserve_moe_layer_no_alloc": LayerCall,
    "uniserve_quantize_mxfp8": QuantizeMxfp8Call,
    "uniserve_gather_gemm_mx": GatherMxCall,
    "uniserve_gather_gemm_mx_gelu_tanh": GatherMxCall,
    "uniserve_route_gemm_mx": RouteMxCall,
    "uniserve_mx_stage_major_scales": MxStageScalesCall,
}


def library():
    """The loaded library with its entries' signatures declared; raises when it is absent."""
    global _LIBRARY
    if _LIBRARY is not None:
        return _LIBRARY
    path = library_path()
    if not path.exists():
        raise RuntimeError(
            f"{path} is not built: run `make -C {_PACKAGE}` (or __graft_entry__.build())"
        )
    lib = ctypes.CDLL(os.fspath(path))
    for name, call in _ENTRIES.items():
        entry = getattr(lib, name)
        entry.argtypes = [ctypes.POINTER(call), _P]
        entry.restype = ctypes.c_int32
    lib.uniserve_topk_softmax_launch.argtypes = [
        _P, ctypes.c_int32, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
        ctypes.c_int32, _P, ctypes.c_int32, _P, _P, _P, _P, _P, _P, ctypes.c_char_p, ctypes.c_size_t,
    ]
    lib.uniserve_topk_softmax_launch.restype = ctypes.c_int32
    for name in ("uniserve_moe_layer_workspace",):
        getattr(lib, name).argtypes = [_I64] * 6
        getattr(lib, name).restype = _I64
    lib.uniserve_sigmoid_gated_add_launch.argtypes = [_P, _P, _P, _I64, _I64, ctypes.c_int32, _P, ctypes.c_char_p,
                                                      ctypes.c_size_t]
    lib.uniserve_sigmoid_gated_add_launch.restype = ctypes.c_int32
    lib.uniserve_moe_layer_step.argtypes = [ctypes.POINTER(LayerCall), ctypes.c_int32, _P]
    lib.uniserve_moe_layer_step.restype = ctypes.c_int32
    lib.uniserve_moe_layer_views_of.argtypes = [_I64] * 6 + [ctypes.POINTER(LayerViews)]
    lib.uniserve_moe_layer_views_of.restype = ctypes.c_int32
    lib.uniserve_moe_max_tiles.argtypes = [_I64] * 4
    lib.uniserve_moe_max_tiles.restype = _I64
    _LIBRARY = lib
    return lib

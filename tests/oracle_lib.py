"""numpy bindings of the CPU oracle (``oracle/libmoe_oracle.so``) - test infrastructure.

Only the tests, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg load
this module, and only as the checker.
"""

import ctypes
import os
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
PATH = ROOT / "oracle" / "libmoe_oracle.so"
if not PATH.exists():
    raise RuntimeError(f"{PATH} is not built: run `make -C {PATH.parent}`")
LIB = ctypes.CDLL(os.fspath(PATH))

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32


def _sig(name, args, res=None):
    fn = getattr(LIB, name)
    fn.argtypes = args
    fn.restype = res
    return fn


_sig("oracle_bf16_from_f32", [ctypes.c_float], ctypes.c_uint16)
_sig("oracle_f32_from_bf16", [ctypes.c_uint16], ctypes.c_float)
_sig("oracle_e4m3_from_f32", [ctypes.c_float], ctypes.c_uint8)
_sig("oracle_f32_from_e4m3", [ctypes.c_uint8], ctypes.c_float)
_sig("oracle_expf", [ctypes.c_float], ctypes.c_float)
_sig("oracle_bf16_encode", [_P, _P, _I64])
_sig("oracle_bf16_decode", [_P, _P, _I64])
_sig("oracle_sequence", [_I64, ctypes.c_uint32, _P])
_sig("oracle_normal", [_I64, ctypes.c_uint64, ctypes.c_float, ctypes.c_float, _P])
_sig("oracle_normal_bf16", [_I64, ctypes.c_uint64, ctypes.c_float, _P])
_sig("oracle_max_tiles", [_I64, _I64, _I64, _I64], _I64)
_sig("oracle_topk_softmax", [_P, _I32, _I64, _I32, _I32, _I32, _I32, _P, _I32, _P, _P, _P, _P, _P])
_sig("oracle_moe_sort", [_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P])
_sig("oracle_router_gemm", [_P, _P, _I64, _I64, _I64, _P])
_sig("oracle_router_gemm_ex", [_P, _P, _I32, _P, _I64, _I64, _I64, _I32, _P])
_sig("oracle_gate_activation", [ctypes.c_float, _I32], ctypes.c_float)
_sig("oracle_gather_gemm_ex", [_P, _P, _I32, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _I32, _I32, _P])
_sig("oracle_gather_gemm", [_P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _I32, _P])
_sig("oracle_route_gemm", [_P, _P, _I64, _I64, _I64, _P, _P, _I32, _P])
_sig("oracle_moe_unpermute", [_P, _P, _P, _I64, _I64, _I64, _I64, _I32, _P])
_sig("oracle_quantize_rows_fp8", [_P, _I64, _I64, _I64, _P, _P])
_sig("oracle_quantize_blocks_fp8", [_P, _I64, _I64, _I64, _I64, _P, _P])
_sig("oracle_gather_gemm_fp8", [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _I32, _I32, _P])
_sig("oracle_route_gemm_fp8", [_P, _P, _P, _P, _I64, _I64, _I64, _P, _P, _I32, _P])
_sig("oracle_moe_layer", [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I32, _I32, _P, _P, _P], _I32)
_sig("oracle_threads", [], _I32)


class LayerCall(ctypes.Structure):
    """``oracle_layer_call`` (oracle/moe_oracle.h)."""

    _fields_ = [(name, _P) for name in ("hidden", "router", "router_bias", "up_gate", "up_gate_scales", "down",
                                         "down_scales", "map", "load", "live_tokens")] + \
        [(name, _I64) for name in ("tokens", "hidden_size", "experts", "top", "intermediate", "local_offset",
                                   "local_experts")] + \
        [(name, _I32) for name in ("renormalize", "weight_dtype", "activation", "reserved")] + \
        [(name, _P) for name in ("out", "ids", "weights", "scores")]


_sig("oracle_moe_layer_ex", [ctypes.POINTER(LayerCall)], _I32)
_sig("oracle_sigmoid_gated_add", [_P, _P, _P, _I64, _I64, _I32])
_sig("oracle_f32_from_e2m1", [ctypes.c_uint8], ctypes.c_float)
_sig("oracle_e2m1_from_f32", [ctypes.c_float], ctypes.c_uint8)
_sig("oracle_mx_scale", [ctypes.c_float, ctypes.c_float], ctypes.c_uint8)
_sig("oracle_quantize_rows_mxfp8", [_P, _I64, _I64, _P, _P])
_sig("oracle_quantize_blocks_mxfp4", [_P, _I64, _I64, _I64, _P, _P])
_sig("oracle_gather_gemm_mx", [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _I32, _I32, _P])
_sig("oracle_route_gemm_mx", [_P, _P, _P, _P, _I64, _I64, _I64, _P, _P, _I32, _P])

KINDS = {np.dtype(np.float32): 0, "bf16": 1, np.dtype(np.float16): 2}


def _p(array):
    return None if array is None else array.ctypes.data_as(_P)


def _c(array, dtype):
    return np.ascontiguousarray(array, dtype=dtype)


def bf16_encode(values):
    values = _c(values, np.float32)
    out = np.empty(values.shape, dtype=np.uint16)
    LIB.oracle_bf16_encode(_p(values), _p(out), values.size)
    return out


def bf16_decode(bits):
    bits = _c(bits, np.uint16)
    out = np.empty(bits.shape, dtype=np.float32)
    LIB.oracle_bf16_decode(_p(bits), _p(out), bits.size)
    return out


def expf(x):
    return LIB.oracle_expf(float(x))


def e4m3_encode(value):
    return LIB.oracle_e4m3_from_f32(float(value))


def e4m3_decode(code):
    return LIB.oracle_f32_from_e4m3(int(code))


def e4m3_decode_array(codes):
    table = np.array([LIB.oracle_f32_from_e4m3(c) for c in range(256)], dtype=np.float32)
    return table[np.asarray(codes, dtype=np.uint8)]


def sequence(count, seed):
    out = np.empty(count, dtype=np.float32)
    LIB.oracle_sequence(count, seed, _p(out))
    return out


def normal(count, seed, stddev=1.0, mean=0.0):
    out = np.empty(count, dtype=np.float32)
    LIB.oracle_normal(count, seed, mean, stddev, _p(out))
    return out


def sigmoid_gated_add(target, update, gate, kind):
    """In place on a copy: ``target`` [rows, columns] += sigmoid(gate[rows]) * update; kind 0 f32
    (float32 arrays), 1 bf16 / 2 f16 (uint16 bits). Returns the new target."""
    out = np.array(target, copy=True, order="C")
    update = np.ascontiguousarray(update)
    gate = np.ascontiguousarray(gate)
    rows, columns = out.shape
    LIB.oracle_sigmoid_gated_add(_p(out), _p(update), _p(gate), rows, columns, kind)
    return out


def e2m1_decode(code):
    return LIB.oracle_f32_from_e2m1(int(code))


def e2m1_encode(value):
    return LIB.oracle_e2m1_from_f32(float(value))


def mx_scale(amax, limit):
    return LIB.oracle_mx_scale(float(amax), float(limit))


def mx_power(scales):
    """2^(s - 127) of E8M0 bytes, as float64."""
    return np.ldexp(1.0, np.asarray(scales, dtype=np.int64) - 127)


def quantize_rows_mxfp8(bits):
    """bf16 bits [rows, width] -> (e4m3 codes [rows, width], E8M0 bytes [rows, width / 32])."""
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    rows, width = bits.shape
    out = np.empty((rows, width), dtype=np.uint8)
    scales = np.empty((rows, width // 32), dtype=np.uint8)
    LIB.oracle_quantize_rows_mxfp8(_p(bits), rows, width, _p(out), _p(scales))
    return out, scales


def quantize_blocks_mxfp4(bits):
    """bf16 bits [stacks, n, k] -> (E2M1 pairs [stacks, n, k / 2], E8M0 bytes [stacks, n, k / 32])."""
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    stacks, n, k = bits.shape
    out = np.empty((stacks, n, k // 2), dtype=np.uint8)
    scales = np.empty((stacks, n, k // 32), dtype=np.uint8)
    LIB.oracle_quantize_blocks_mxfp4(_p(bits), stacks, n, k, _p(out), _p(scales))
    return out, scales


def e2m1_unpack(packed):
    """E2M1 pairs [..., k / 2] -> codes [..., k] (low nibble first)."""
    packed = np.asarray(packed, dtype=np.uint8)
    out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 2,), dtype=np.uint8)
    out[..., 0::2] = packed & 15
    out[..., 1::2] = packed >> 4
    return out


def gather_gemm_mx(hq, hs, wq, ws, top, sort, rows, fill=np.nan, activation=0):
    tokens, hidden = hq.shape
    experts, width, _ = wq.shape
    out = np.full((rows, width // 2), fill, dtype=np.float32)
    LIB.oracle_gather_gemm_mx(_p(_c(hq, np.uint8)), _p(_c(hs, np.uint8)), _p(_c(wq, np.uint8)), _p(_c(ws, np.uint8)),
                              tokens, hidden, width // 2, top, 128, _p(sort["tile_to_expert"]),
                              _p(sort["tile_to_limit"]), _p(sort["permuted_to_expanded"]),
                              int(sort["num_non_exiting_tiles"][0]), activation, _p(out))
    return out


def route_gemm_mx(gq, gs, wq, ws, sort, fill=np.nan):
    rows, intermediate = gq.shape
    experts, hidden, _ = wq.shape
    out = np.full((rows, hidden), fill, dtype=np.float32)
    LIB.oracle_route_gemm_mx(_p(_c(gq, np.uint8)), _p(_c(gs, np.uint8)), _p(_c(wq, np.uint8)), _p(_c(ws, np.uint8)),
                             hidden, intermediate, 128, _p(sort["tile_to_expert"]), _p(sort["tile_to_limit"]),
                             int(sort["num_non_exiting_tiles"][0]), _p(out))
    return out


def max_tiles(tokens, top, local_experts, tile=128):
    return LIB.oracle_max_tiles(tokens, top, local_experts, tile)


def topk_softmax(scores, top, renormalize=True, score_kind=None, scale=None, scale_kind=-1,
                 mapping=None, live=None, load=None, experts=None, rows=None):
    """``scores``: float32/float16 array, or uint16 bf16 bits with score_kind=1."""
    scores = np.ascontiguousarray(scores)
    if score_kind is None:
        score_kind = KINDS[scores.dtype]
    rows = scores.shape[0] if rows is None else rows
    experts = scores.shape[1] if experts is None else experts
    ids = np.empty((rows, top), dtype=np.int32)
    weights = np.empty((rows, top), dtype=np.float32)
    live_arr = None if live is None else np.array([live], dtype=np.int32)
    LIB.oracle_topk_softmax(_p(scores), score_kind, scores.shape[1], rows, experts, top,
                            1 if renormalize else 0, _p(scale), scale_kind, _p(ids), _p(weights),
                            _p(None if mapping is None else _c(mapping, np.int32)), _p(live_arr), _p(load))
    return ids, weights


def moe_sort(ids, local_experts, local_offset=0, live=None, tile=128, fill=-7):
    """Device semantics: entries the sort does not write keep ``fill``."""
    ids = _c(ids, np.int32)
    tokens, top = ids.shape
    tiles = max_tiles(tokens, top, local_experts, tile)
    rows = max(tiles * tile, 1)
    out = {
        "tile_to_expert": np.full(max(tiles, 1), fill, np.int32),
        "tile_to_limit": np.full(max(tiles, 1), fill, np.int32),
        "expanded_to_permuted": np.full(max(tokens * top, 1), fill, np.int32),
        "permuted_to_expanded": np.full(rows, fill, np.int32),
        "permuted_to_token": np.full(rows, fill, np.int32),
        "total_padded_tokens": np.full(1, fill, np.int32),
        "num_non_exiting_tiles": np.full(1, fill, np.int32),
    }
    live_arr = None if live is None else np.array([live], dtype=np.int32)
    LIB.oracle_moe_sort(_p(ids), tokens, top, local_experts, local_offset, tile, _p(live_arr),
                        _p(out["tile_to_expert"]), _p(out["tile_to_limit"]),
                        _p(out["expanded_to_permuted"]), _p(out["permuted_to_expanded"]),
                        _p(out["permuted_to_token"]), _p(out["total_padded_tokens"]),
                        _p(out["num_non_exiting_tiles"]))
    return out


def router_gemm(x_bits, w_bits, bias=None):
    """bf16 scores of bf16 rows, the optional f32 bias added to the FP32 sum before rounding."""
    x_bits, w_bits = _c(x_bits, np.uint16), _c(w_bits, np.uint16)
    m, k = x_bits.shape
    n = w_bits.shape[0]
    out = np.empty((m, n), dtype=np.uint16)
    if bias is None:
        LIB.oracle_router_gemm(_p(x_bits), _p(w_bits), m, n, k, _p(out))
    else:
        bias = _c(bias, np.float32)
        LIB.oracle_router_gemm_ex(_p(x_bits), _p(w_bits), 1, _p(bias), m, n, k, 1, _p(out))
    return out


def router_gemm_f32(x, w, bias=None):
    """f32 scores of f32 rows (the CPU reference path): no rounding."""
    x, w = _c(x, np.float32), _c(w, np.float32)
    m, k = x.shape
    n = w.shape[0]
    out = np.empty((m, n), dtype=np.float32)
    LIB.oracle_router_gemm_ex(_p(x), _p(w), 0, _p(None if bias is None else _c(bias, np.float32)), m, n, k, 0, _p(out))
    return out


def gate_activation(g, activation):
    return LIB.oracle_gate_activation(g, activation)


def gather_gemm(hidden_bits, weight_bits, top, sort, rows, fill=np.nan, activation=0):
    """FC1 of bf16 rows (activation 0 silu, 1 gelu_tanh); f32 rows when the inputs are float32."""
    kind = 0 if np.asarray(hidden_bits).dtype == np.float32 else 1
    dtype = np.float32 if kind == 0 else np.uint16
    hidden_bits, weight_bits = _c(hidden_bits, dtype), _c(weight_bits, dtype)
    tokens, hidden = hidden_bits.shape
    intermediate = weight_bits.shape[1] // 2
    out = np.full((rows, intermediate), fill, dtype=np.float32)
    LIB.oracle_gather_gemm_ex(_p(hidden_bits), _p(weight_bits), kind, tokens, hidden, intermediate, top, 128,
                              _p(sort["tile_to_expert"]), _p(sort["tile_to_limit"]),
                              _p(sort["permuted_to_expanded"]), int(sort["num_non_exiting_tiles"][0]), activation,
                              _p(out))
    return out


def route_gemm(rows_bits, weight_bits, sort, fill=np.nan):
    rows_bits, weight_bits = _c(rows_bits, np.uint16), _c(weight_bits, np.uint16)
    rows, intermediate = rows_bits.shape
    hidden = weight_bits.shape[1]
    out = np.full((rows, hidden), fill, dtype=np.float32)
    LIB.oracle_route_gemm(_p(rows_bits), _p(weight_bits), hidden, intermediate, 128,
                          _p(sort["tile_to_expert"]), _p(sort["tile_to_limit"]),
                          int(sort["num_non_exiting_tiles"][0]), _p(out))
    return out


def moe_unpermute(routes_bits, expanded_to_permuted, scales, layout=0):
    routes_bits = _c(routes_bits, np.uint16)
    e2p = _c(expanded_to_permuted, np.int32)
    scales = _c(scales, np.float32)
    tokens, top = scales.shape
    rows, hidden = routes_bits.shape
    out = np.empty((tokens, hidden), dtype=np.float32)
    LIB.oracle_moe_unpermute(_p(routes_bits), _p(e2p), _p(scales), tokens, top, hidden, rows, layout, _p(out))
    return out


def quantize_rows_fp8(bits, group=128):
    bits = _c(bits, np.uint16)
    rows, width = bits.shape
    out = np.empty((rows, width), dtype=np.uint8)
    scales = np.empty((rows, width // group), dtype=np.float32)
    LIB.oracle_quantize_rows_fp8(_p(bits), rows, width, group, _p(out), _p(scales))
    return out, scales


def quantize_blocks_fp8(bits, block=128):
    bits = _c(bits, np.uint16)
    stacks, n, k = bits.shape
    out = np.empty((stacks, n, k), dtype=np.uint8)
    scales = np.empty((stacks, n // block, k // block), dtype=np.float32)
    LIB.oracle_quantize_blocks_fp8(_p(bits), stacks, n, k, block, _p(out), _p(scales))
    return out, scales


def gather_gemm_fp8(hq, hs, wq, ws, top, sort, rows, fill=np.nan, activation=0):
    tokens, hidden = hq.shape
    intermediate = wq.shape[1] // 2
    out = np.full((rows, intermediate), fill, dtype=np.float32)
    LIB.oracle_gather_gemm_fp8(_p(_c(hq, np.uint8)), _p(_c(hs, np.float32)), _p(_c(wq, np.uint8)),
                               _p(_c(ws, np.float32)), tokens, hidden, intermediate, top, 128,
                               _p(sort["tile_to_expert"]), _p(sort["tile_to_limit"]),
                               _p(sort["permuted_to_expanded"]), int(sort["num_non_exiting_tiles"][0]), activation,
                               _p(out))
    return out


def route_gemm_fp8(gq, gs, wq, ws, sort, fill=np.nan):
    rows, intermediate = gq.shape
    hidden = wq.shape[1]
    out = np.full((rows, hidden), fill, dtype=np.float32)
    LIB.oracle_route_gemm_fp8(_p(_c(gq, np.uint8)), _p(_c(gs, np.float32)), _p(_c(wq, np.uint8)),
                              _p(_c(ws, np.float32)), hidden, intermediate, 128,
                              _p(sort["tile_to_expert"]), _p(sort["tile_to_limit"]),
                              int(sort["num_non_exiting_tiles"][0]), _p(out))
    return out


def moe_layer(hidden_bits, router_bits, up_gate, down, top, renormalize=True, up_gate_scales=None,
              down_scales=None, router_bias=None, mapping=None, load=None, live=None, window=None, activation=0,
              scores=False):
    """The composed layer on the CPU; answers (out, ids, weights, threads) and, with ``scores``, the
    router scores last. bf16 bits in and out, or float32 everything (the CPU reference path) when
    ``hidden_bits`` is float32. ``window`` = (local_offset, local_experts): the stacks hold those
    experts only. ``load`` (int64 [experts]) is incremented in place."""
    f32 = np.asarray(hidden_bits).dtype == np.float32
    elem = np.float32 if f32 else np.uint16
    hidden_bits, router_bits = _c(hidden_bits, elem), _c(router_bits, elem)
    tokens, hidden = hidden_bits.shape
    experts = router_bits.shape[0]
    intermediate = up_gate.shape[1] // 2
    # MX stacks: E2M1 pairs with E8M0 byte scales; e4m3: bytes with f32 scales.
    mx = up_gate_scales is not None and np.asarray(up_gate_scales).dtype == np.uint8
    fp8 = up_gate.dtype == np.uint8 and not mx
    out = np.empty((tokens, hidden), dtype=elem)
    ids = np.empty((tokens, top), dtype=np.int32)
    weights = np.empty((tokens, top), dtype=np.float32)
    score_out = np.empty((tokens, experts), dtype=elem)
    keep = []

    def ptr(array, dtype):
        if array is None:
            return None
        array = _c(array, dtype)
        keep.append(array)
        return array.ctypes.data

    if load is not None:
        assert load.dtype == np.int64 and load.flags.c_contiguous
    call = LayerCall()
    call.hidden, call.router = hidden_bits.ctypes.data, router_bits.ctypes.data
    call.router_bias = ptr(router_bias, np.float32)
    call.up_gate = ptr(up_gate, up_gate.dtype)
    call.up_gate_scales = ptr(up_gate_scales, None if up_gate_scales is None else np.asarray(up_gate_scales).dtype)
    call.down = ptr(down, down.dtype)
    call.down_scales = ptr(down_scales, None if down_scales is None else np.asarray(down_scales).dtype)
    call.map = ptr(mapping, np.int32)
    call.load = None if load is None else load.ctypes.data
    call.live_tokens = ptr(None if live is None else np.array([live], np.int32), np.int32)
    call.tokens, call.hidden_size, call.experts, call.top, call.intermediate = tokens, hidden, experts, top, intermediate
    call.local_offset, call.local_experts = (0, 0) if window is None else window
    call.renormalize = 1 if renormalize else 0
    call.weight_dtype = 5 if f32 else 7 if mx else 6 if fp8 else 4
    call.activation = activation
    call.out, call.ids, call.weights, call.scores = out.ctypes.data, ids.ctypes.data, weights.ctypes.data, \
        score_out.ctypes.data
    threads = LIB.oracle_moe_layer_ex(ctypes.byref(call))
    if scores:
        return out, ids, weights, threads, score_out
    return out, ids, weights, threads

"""The MoE operators on torch device tensors, through the library's C entries.

Each function mirrors one of ``nn::functional``'s (crates/nn/src/functional/moe.rs):
the same arguments, the same outputs, the same maps tensor (``[7, permuted rows]`` of
int32, one map per row, ``moe.rs:58-88``). Torch only allocates and orders work on its
current stream; the arithmetic is the HIP library's. A refusal raises with the
entry's message.
"""

import ctypes

import torch

from .abi import (
    ACTIVATION,
    DTYPE,
    ENTRY_SUFFIX,
    LAYOUT_PERMUTED,
    GatherCall,
    GatherFp8Call,
    GemmCall,
    LayerCall,
    LayerViews,
    QuantizeFp8Call,
    MxStageScalesCall,
    QuantizeMxfp8Call,
    GatherMxCall,
    RouteMxCall,
    RouteCall,
    RouteFp8Call,
    SortCall,
    UnpermuteCall,
    library,
    max_tiles,
)

#: Rows of the maps tensor (crates/nn/src/functional/moe.rs:58-88).
TILE_TO_EXPERT, TILE_TO_LIMIT, EXPANDED_TO_PERMUTED, PERMUTED_TO_EXPANDED = 0, 1, 2, 3
PERMUTED_TO_TOKEN, TOTAL_PADDED_TOKENS, NUM_NON_EXITING_TILES = 4, 5, 6
SORT_MAPS = 7
TILE = 128

_TORCH_DTYPE = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}
_SCORE_KIND = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def _stream(device=None):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _ptr(tensor):
    return None if tensor is None else tensor.data_ptr()


def _check(status, call, name):
    if status != 0:
        message = bytes(call.error).split(b"\0", 1)[0].decode(errors="replace")
        raise RuntimeError(f"{name} refused the call ({status}): {message}")


def multiprocessors(device=None):
    return torch.cuda.get_device_properties(device or torch.cuda.current_device()).multi_processor_count


def topk_softmax(scores, top, renormalize=True, scale=None, mapping=None, live=None, load=None):
    """``functional::topk_softmax`` (moe.rs:120-195): ids ``[T, top]`` int32, weights f32."""
    tokens, experts = scores.shape
    ids = torch.empty((tokens, top), dtype=torch.int32, device=scores.device)
    weights = torch.empty((tokens, top), dtype=torch.float32, device=scores.device)
    error = ctypes.create_string_buffer(512)
    status = library().uniserve_topk_softmax_launch(
        _ptr(scores), _SCORE_KIND[scores.dtype], scores.stride(0), tokens, experts, top,
        1 if renormalize else 0, _ptr(scale), -1 if scale is None else _SCORE_KIND[scale.dtype],
        _ptr(ids), _ptr(weights), _ptr(mapping), _ptr(live), _ptr(load), _stream(scores.device),
        error, 512,
    )
    if status != 0:
        raise RuntimeError(f"topk_softmax refused the call: {error.value.decode()}")
    return ids, weights


_ELEMENT = {torch.bfloat16: DTYPE["bf16"], torch.float16: DTYPE["f16"], torch.float32: DTYPE["f32"]}


def sigmoid_gated_add_(target, update, gate):
    """``functional::sigmoid_gated_add_`` (crates/nn/src/functional/moe.rs:1527-1570): ``target``
    ``[rows, columns]`` += sigmoid(``gate`` ``[rows, 1]``) * ``update``, in place; returns ``target``."""
    if target.dim() != 2 or update.shape != target.shape or update.dtype != target.dtype:
        raise ValueError("sigmoid_gated_add_: the update is the target's shape and element type")
    if tuple(gate.shape) != (target.shape[0], 1) or gate.dtype != target.dtype:
        raise ValueError("sigmoid_gated_add_: the gate is one logit per row, of the target's type")
    if not (target.is_contiguous() and update.is_contiguous() and gate.is_contiguous()):
        raise ValueError("sigmoid_gated_add_: a strided view has no rows to update in place")
    error = ctypes.create_string_buffer(512)
    status = library().uniserve_sigmoid_gated_add_launch(
        _ptr(target), _ptr(update), _ptr(gate), target.shape[0], target.shape[1], _ELEMENT[target.dtype],
        _stream(target.device), error, 512)
    if status != 0:
        raise RuntimeError(f"sigmoid_gated_add refused the call: {error.value.decode()}")
    return target


def empty_maps(tokens, top, local_experts, device, fill=-7):
    rows = max_tiles(tokens, top, local_experts, TILE) * TILE
    return torch.full((SORT_MAPS, max(rows, tokens * top, 1)), fill, dtype=torch.int32, device=device)


def moe_sort(ids, weights, experts, local=None, live_tokens=None, maps=None):
    """``functional::moe_sort`` (moe.rs:325-372): the ``[7, rows]`` maps of the routing."""
    tokens, top = ids.shape
    start, end = (0, experts) if local is None else local
    local_experts = end - start
    tiles = max_tiles(tokens, top, local_experts, TILE)
    if maps is None:
        maps = empty_maps(tokens, top, local_experts, ids.device)
    call = SortCall()
    call.ids = ids.data_ptr()
    call.scales = weights.data_ptr()
    call.tile_to_expert = maps[TILE_TO_EXPERT].data_ptr()
    call.tile_to_limit = maps[TILE_TO_LIMIT].data_ptr()
    call.expanded_to_permuted = maps[EXPANDED_TO_PERMUTED].data_ptr()
    call.permuted_to_expanded = maps[PERMUTED_TO_EXPANDED].data_ptr()
    call.permuted_to_token = maps[PERMUTED_TO_TOKEN].data_ptr()
    call.total_padded_tokens = maps[TOTAL_PADDED_TOKENS].data_ptr()
    call.num_non_exiting_tiles = maps[NUM_NON_EXITING_TILES].data_ptr()
    call.tokens, call.top, call.experts = tokens, top, experts
    call.local_experts, call.local_offset, call.tile_tokens = local_experts, start, TILE
    call.scales_dtype = DTYPE[_TORCH_DTYPE[weights.dtype]]
    call.live_tokens = _ptr(live_tokens)
    _check(library().uniserve_moe_sort(ctypes.byref(call), _stream(ids.device)), call, "moe_sort")
    assert tiles * TILE <= maps.shape[1]
    return maps


def permuted_rows(tokens, top, local_experts):
    return max_tiles(tokens, top, local_experts, TILE) * TILE


def gather_gemm(hidden, up_gate, top, maps, rows, out=None, activation="silu"):
    """``functional::gather_gemm`` (moe.rs:476-636): ``[rows, I]`` gated products (bf16), gated by
    ``activation`` ("silu" or "gelu_tanh": the entry of that name)."""
    tokens, width = hidden.shape
    experts, gated, _ = up_gate.shape
    if out is None:
        out = torch.empty((rows, gated // 2), dtype=hidden.dtype, device=hidden.device)
    call = GatherCall()
    call.hidden, call.weights, call.out = hidden.data_ptr(), up_gate.data_ptr(), out.data_ptr()
    call.tile_to_expert = maps[TILE_TO_EXPERT].data_ptr()
    call.tile_to_limit = maps[TILE_TO_LIMIT].data_ptr()
    call.permuted_to_expanded = maps[PERMUTED_TO_EXPANDED].data_ptr()
    call.num_non_exiting_tiles = maps[NUM_NON_EXITING_TILES].data_ptr()
    call.tokens, call.permuted_rows, call.width, call.hidden_size = tokens, rows, gated, width
    call.experts, call.top, call.dtype = experts, top, DTYPE[_TORCH_DTYPE[hidden.dtype]]
    call.multiprocessors = multiprocessors(hidden.device)
    entry = getattr(library(), "uniserve_gather_gemm" + ENTRY_SUFFIX[activation])
    _check(entry(ctypes.byref(call), _stream(hidden.device)), call, "gather_gemm")
    return out


def route_gemm(gated, down, maps, out=None):
    """``functional::route_gemm`` (moe.rs:641-781): ``[rows, H]`` unweighted products."""
    rows, intermediate = gated.shape
    experts, hidden, _ = down.shape
    if out is None:
        out = torch.empty((rows, hidden), dtype=gated.dtype, device=gated.device)
    call = RouteCall()
    call.rows, call.weights, call.out = gated.data_ptr(), down.data_ptr(), out.data_ptr()
    call.tile_to_expert = maps[TILE_TO_EXPERT].data_ptr()
    call.tile_to_limit = maps[TILE_TO_LIMIT].data_ptr()
    call.permuted_to_expanded = maps[PERMUTED_TO_EXPANDED].data_ptr()
    call.num_non_exiting_tiles = maps[NUM_NON_EXITING_TILES].data_ptr()
    call.permuted_rows, call.width, call.intermediate = rows, hidden, intermediate
    call.experts, call.dtype = experts, DTYPE[_TORCH_DTYPE[gated.dtype]]
    call.multiprocessors = multiprocessors(gated.device)
    _check(library().uniserve_route_gemm(ctypes.byref(call), _stream(gated.device)), call, "route_gemm")
    return out


def moe_unpermute(products, expanded_to_permuted, weights, out=None, layout=LAYOUT_PERMUTED):
    """``functional::moe_unpermute`` (moe.rs:1188-1330): ``[T, H]`` weighted sums."""
    rows, hidden = products.shape
    tokens, top = weights.shape
    if out is None:
        out = torch.empty((tokens, hidden), dtype=products.dtype, device=products.device)
    call = UnpermuteCall()
    call.routes, call.out = products.data_ptr(), out.data_ptr()
    call.expanded_to_permuted = expanded_to_permuted.data_ptr()
    call.scales = weights.data_ptr()
    call.tokens, call.top, call.hidden, call.routes_rows = tokens, top, hidden, rows
    call.input_dtype = DTYPE[_TORCH_DTYPE[products.dtype]]
    call.scales_dtype = DTYPE[_TORCH_DTYPE[weights.dtype]]
    call.output_dtype = DTYPE[_TORCH_DTYPE[out.dtype]]
    call.layout = layout
    _check(library().uniserve_moe_unpermute(ctypes.byref(call), _stream(products.device)), call, "moe_unpermute")
    return out


def router_gemm(hidden, router, out=None):
    """The router ``Linear`` as the ``gemm`` module (bf16, nxk, no bias)."""
    tokens, width = hidden.shape
    experts = router.shape[0]
    if out is None:
        out = torch.empty((tokens, experts), dtype=torch.bfloat16, device=hidden.device)
    call = GemmCall()
    call.out, call.input, call.weight, call.bias = out.data_ptr(), hidden.data_ptr(), router.data_ptr(), None
    call.m, call.n, call.k = tokens, experts, width
    call.input_row_stride, call.weight_row_stride, call.out_row_stride = hidden.stride(0), router.stride(0), out.stride(0)
    call.alpha = 1.0
    _check(library().uniserve_gemm(ctypes.byref(call), _stream(hidden.device)), call, "gemm")
    return out


def quantize_fp8(rows_tensor, row_limit=None):
    """Per-row, per-128-channel e4m3 codes (uint8) and FP32 scales."""
    rows, width = rows_tensor.shape
    out = torch.empty((rows, width), dtype=torch.uint8, device=rows_tensor.device)
    scales = torch.empty((rows, width // 128), dtype=torch.float32, device=rows_tensor.device)
    call = QuantizeFp8Call()
    call.input, call.out, call.scales = rows_tensor.data_ptr(), out.data_ptr(), scales.data_ptr()
    call.row_limit = _ptr(row_limit)
    call.rows, call.width, call.group = rows, width, 128
    call.input_dtype = DTYPE[_TORCH_DTYPE[rows_tensor.dtype]]
    _check(library().uniserve_quantize_fp8(ctypes.byref(call), _stream(rows_tensor.device)), call, "quantize_fp8")
    return out, scales


def gather_gemm_fp8(hidden_q, hidden_s, up_gate_q, up_gate_s, top, maps, rows, out=None, activation="silu"):
    tokens, width = hidden_q.shape
    experts, gated, _ = up_gate_q.shape
    if out is None:
        out = torch.empty((rows, gated // 2), dtype=torch.bfloat16, device=hidden_q.device)
    call = GatherFp8Call()
    call.hidden, call.hidden_scales = hidden_q.data_ptr(), hidden_s.data_ptr()
    call.weights, call.weight_scales, call.out = up_gate_q.data_ptr(), up_gate_s.data_ptr(), out.data_ptr()
    call.tile_to_expert = maps[TILE_TO_EXPERT].data_ptr()
    call.tile_to_limit = maps[TILE_TO_LIMIT].data_ptr()
    call.permuted_to_expanded = maps[PERMUTED_TO_EXPANDED].data_ptr()
    call.num_non_exiting_tiles = maps[NUM_NON_EXITING_TILES].data_ptr()
    call.tokens, call.permuted_rows, call.width, call.hidden_size = tokens, rows, gated, width
    call.experts, call.top, call.block_n, call.block_k = experts, top, 128, 128
    call.out_dtype, call.multiprocessors = DTYPE["bf16"], multiprocessors(hidden_q.device)
    entry = getattr(library(), "uniserve_gather_gemm_fp8" + ENTRY_SUFFIX[activation])
    _check(entry(ctypes.byref(call), _stream(hidden_q.device)), call, "gather_gemm_fp8")
    return out


def route_gemm_fp8(gated_q, gated_s, down_q, down_s, maps, out=None):
    rows, intermediate = gated_q.shape
    experts, hidden, _ = down_q.shape
    if out is None:
        out = torch.empty((rows, hidden), dtype=torch.bfloat16, device=gated_q.device)
    call = RouteFp8Call()
    call.rows, call.row_scales = gated_q.data_ptr(), gated_s.data_ptr()
    call.weights, call.weight_scales, call.out = down_q.data_ptr(), down_s.data_ptr(), out.data_ptr()
    call.tile_to_expert = maps[TILE_TO_EXPERT].data_ptr()
    call.tile_to_limit = maps[TILE_TO_LIMIT].data_ptr()
    call.permuted_to_expanded = maps[PERMUTED_TO_EXPANDED].data_ptr()
    call.num_non_exiting_tiles = maps[NUM_NON_EXITING_TILES].data_ptr()
    call.permuted_rows, call.width, call.intermediate = rows, hidden, intermediate
    call.experts, call.block_n, call.block_k = experts, 128, 128
    call.out_dtype, call.multiprocessors = DTYPE["bf16"], multiprocessors(gated_q.device)
    _check(library().uniserve_route_gemm_fp8(ctypes.byref(call), _stream(gated_q.device)), call, "route_gemm_fp8")
    return out


def quantize_mxfp8(rows_tensor, row_limit=None):
    """Per-row, per-32-channel MXFP8: e4m3 codes (uint8) and E8M0 scale bytes (uint8)."""
    rows, width = rows_tensor.shape
    out = torch.empty((rows, width), dtype=torch.uint8, device=rows_tensor.device)
    scales = torch.empty((rows, width // 32), dtype=torch.uint8, device=rows_tensor.device)
    call = QuantizeMxfp8Call()
    call.input, call.out, call.scales = rows_tensor.data_ptr(), out.data_ptr(), scales.data_ptr()
    call.row_limit = _ptr(row_limit)
    call.rows, call.width = rows, width
    call.input_dtype = DTYPE[_TORCH_DTYPE[rows_tensor.dtype]]
    _check(library().uniserve_quantize_mxfp8(ctypes.byref(call), _stream(rows_tensor.device)), call, "quantize_mxfp8")
    return out, scales


MX_SCALE_LAYOUTS = {"row": 0, "stage": 1}


def mx_stage_major_scales(scales):
    """A ``[stacks, rows, K / 32]`` row-major E8M0 table in the stage-major layout (same bytes,
    each 128-element stage's 4-byte words of all rows contiguous), for the prefill kernel."""
    stacks, rows, blocks = scales.shape
    out = torch.empty_like(scales)
    call = MxStageScalesCall()
    call.input, call.out = scales.data_ptr(), out.data_ptr()
    call.stacks, call.rows, call.width = stacks, rows, blocks * 32
    _check(library().uniserve_mx_stage_major_scales(ctypes.byref(call), _stream(scales.device)), call,
           "mx_stage_major_scales")
    return out


def gather_gemm_mx(hidden_q, hidden_s, up_gate_q, up_gate_s, top, maps, rows, out=None, scale_layout="row",
                   activation="silu"):
    """FC1 over MXFP8 tokens and MXFP4 weights (``up_gate_q`` [E, 2I, H / 2] E2M1 pairs; the weight
    scales in ``scale_layout``, "row" or "stage")."""
    tokens, width = hidden_q.shape
    experts, gated, _ = up_gate_q.shape
    if out is None:
        out = torch.empty((rows, gated // 2), dtype=torch.bfloat16, device=hidden_q.device)
    call = GatherMxCall()
    call.hidden, call.hidden_scales = hidden_q.data_ptr(), hidden_s.data_ptr()
    call.weights, call.weight_scales, call.out = up_gate_q.data_ptr(), up_gate_s.data_ptr(), out.data_ptr()
    call.tile_to_expert = maps[TILE_TO_EXPERT].data_ptr()
    call.tile_to_limit = maps[TILE_TO_LIMIT].data_ptr()
    call.permuted_to_expanded = maps[PERMUTED_TO_EXPANDED].data_ptr()
    call.num_non_exiting_tiles = maps[NUM_NON_EXITING_TILES].data_ptr()
    call.tokens, call.permuted_rows, call.width, call.hidden_size = tokens, rows, gated, width
    call.experts, call.top = experts, top
    call.out_dtype, call.multiprocessors = DTYPE["bf16"], multiprocessors(hidden_q.device)
    call.weight_scale_layout = MX_SCALE_LAYOUTS[scale_layout]
    entry = getattr(library(), "uniserve_gather_gemm_mx" + ENTRY_SUFFIX[activation])
    _check(entry(ctypes.byref(call), _stream(hidden_q.device)), call, "gather_gemm_mx")
    return out


def route_gemm_mx(gated_q, gated_s, down_q, down_s, maps, out=None, scale_layout="row"):
    """FC2 over MXFP8 rows and MXFP4 weights (``down_q`` [E, H, I / 2] E2M1 pairs; the weight scales
    in ``scale_layout``)."""
    rows, intermediate = gated_q.shape
    experts, hidden, _ = down_q.shape
    if out is None:
        out = torch.empty((rows, hidden), dtype=torch.bfloat16, device=gated_q.device)
    call = RouteMxCall()
    call.rows, call.row_scales = gated_q.data_ptr(), gated_s.data_ptr()
    call.weights, call.weight_scales, call.out = down_q.data_ptr(), down_s.data_ptr(), out.data_ptr()
    call.tile_to_expert = maps[TILE_TO_EXPERT].data_ptr()
    call.tile_to_limit = maps[TILE_TO_LIMIT].data_ptr()
    call.permuted_to_expanded = maps[PERMUTED_TO_EXPANDED].data_ptr()
    call.num_non_exiting_tiles = maps[NUM_NON_EXITING_TILES].data_ptr()
    call.permuted_rows, call.width, call.intermediate = rows, hidden, intermediate
    call.experts = experts
    call.out_dtype, call.multiprocessors = DTYPE["bf16"], multiprocessors(gated_q.device)
    call.weight_scale_layout = MX_SCALE_LAYOUTS[scale_layout]
    _check(library().uniserve_route_gemm_mx(ctypes.byref(call), _stream(gated_q.device)), call, "route_gemm_mx")
    return out


def layer_views(tokens, hidden, experts, top, intermediate, weight_dtype="bf16"):
    views = LayerViews()
    status = library().uniserve_moe_layer_views_of(tokens, hidden, experts, top, intermediate,
                                                   DTYPE[weight_dtype], ctypes.byref(views))
    if status != 0:
        raise RuntimeError("moe_layer does not serve these extents")
    return views


class MoeLayer:
    """``MoE::routed`` (crates/nn/src/modules/moe.rs:770-795) over one caller-owned workspace."""

    def __init__(self, hidden_size, experts, top, intermediate, max_tokens, weight_dtype="bf16",
                 renormalize=True, device=None):
        self.hidden_size, self.experts, self.top = hidden_size, experts, top
        self.intermediate, self.max_tokens = intermediate, max_tokens
        self.weight_dtype, self.renormalize = weight_dtype, renormalize
        self.device = device or torch.device("cuda")
        self.views = layer_views(max_tokens, hidden_size, experts, top, intermediate, weight_dtype)
        # Zeroed once: the fused front end's counter (the first word) must start at zero, and every
        # call leaves it zero; nothing else needs initialising.
        self.workspace = torch.zeros(self.views.total, dtype=torch.uint8, device=self.device)
        self.call = LayerCall()

    def view(self, name, dtype, shape):
        """An intermediate tensor of the last call, as a view of the workspace."""
        offset = getattr(self.views, name)
        count = 1
        for extent in shape:
            count *= extent
        size = torch.empty((), dtype=dtype).element_size()
        return self.workspace[offset:offset + count * size].view(dtype).view(*shape)

    def __call__(self, hidden, router, up_gate, down, out=None, up_gate_scales=None, down_scales=None,
                 router_bias=None, live_tokens=None, scale_layout="row", mapping=None, load=None, window=None,
                 activation="silu"):
        """``mapping`` (int32 [experts]) names each router expert's slot, ``load`` (int64 [experts])
        counts the live routes by router expert, ``window`` = (local_offset, local_experts) names
        the slots the stacks hold (``up_gate`` [local_experts, ...]); ``activation`` is FC1's gate."""
        tokens = hidden.shape[0]
        if tokens != self.max_tokens:
            raise ValueError("the layer's workspace is laid out for its max_tokens")
        if out is None:
            out = torch.empty((tokens, self.hidden_size), dtype=torch.bfloat16, device=hidden.device)
        call = self.call
        call.hidden, call.router = hidden.data_ptr(), router.data_ptr()
        call.up_gate, call.down = up_gate.data_ptr(), down.data_ptr()
        call.up_gate_scales, call.down_scales = _ptr(up_gate_scales), _ptr(down_scales)
        call.router_bias, call.out = _ptr(router_bias), out.data_ptr()
        call.workspace, call.workspace_bytes = self.workspace.data_ptr(), self.workspace.numel()
        call.live_tokens = _ptr(live_tokens)
        call.tokens, call.hidden_size, call.experts = tokens, self.hidden_size, self.experts
        call.top, call.intermediate = self.top, self.intermediate
        call.renormalize = 1 if self.renormalize else 0
        call.weight_dtype = DTYPE[self.weight_dtype]
        call.multiprocessors = multiprocessors(hidden.device)
        call.weight_scale_layout = MX_SCALE_LAYOUTS[scale_layout]
        call.map, call.load = _ptr(mapping), _ptr(load)
        call.local_offset, call.local_experts = (0, 0) if window is None else window
        call.activation = ACTIVATION[activation]
        _check(library().uniserve_moe_layer(ctypes.byref(call), _stream(hidden.device)), call, "moe_layer")
        return out

    STEPS = ("router", "topk", "sort", "quantize_hidden", "gather", "quantize_gated", "route", "unpermute")

    def step(self, name):
        """Launches one step of the last call again, exactly as the call launched it (same
        arguments, same workspace)."""
        index = self.STEPS.index(name)
        device = self.workspace.device
        _check(library().uniserve_moe_layer_step(ctypes.byref(self.call), index, _stream(device)), self.call,
               "moe_layer_step")

// SPDX-License-Identifier: Apache-2.0
//
// The routed mixture-of-experts layer as one call: what `MoE::routed`
// (crates/nn/src/modules/moe.rs:770-795) issues as six launches, in the same order and with the
// same intermediate tensors - router gemm -> topk_softmax -> moe_sort -> gather_gemm ->
// route_gemm -> moe_unpermute - on one stream, with every intermediate carved from one
// caller-owned workspace so the call allocates nothing and can be captured into a graph.
//
// weight_dtype BF16: `up_gate` [E, 2I, H] (up rows then gate rows) and `down` [E, H, I] in bf16.
// weight_dtype F8E4M3: both stacks e4m3 with FP32 128x128 block scales
// (`up_gate_scales` [E, 2I/128, H/128], `down_scales` [E, H/128, I/128]); the activations are
// quantised per row per 128 channels inside the call.
// weight_dtype F4E2M1 (OCP MXFP4): both stacks E2M1 pairs along K (`up_gate` [E, 2I, H/2],
// `down` [E, H, I/2]) with one E8M0 byte per 32 K elements (`up_gate_scales` [E, 2I, H/32],
// `down_scales` [E, H, I/32], passed through the same pointers as bytes); the activations are
// quantised to MXFP8 inside the call. The output is bf16 in every case.

#pragma once

#include "uniserve_abi.h"

struct uniserve_moe_layer_call {
  const void *hidden;          ///< [tokens, hidden_size] bf16
  const void *router;          ///< [experts, hidden_size] bf16
  const void *up_gate;         ///< [experts, 2 * intermediate, hidden_size]
  const void *down;            ///< [experts, hidden_size, intermediate]
  const float *up_gate_scales; ///< e4m3: f32 block scales; MXFP4: E8M0 bytes
  const float *down_scales;    ///< e4m3: f32 block scales; MXFP4: E8M0 bytes
  const float *router_bias;    ///< [experts] added to the scores before rounding, or null
  void *out;                   ///< [tokens, hidden_size] bf16
  void *workspace;             ///< uniserve_moe_layer_workspace() bytes, 256-byte aligned
  const int32_t *live_tokens;  ///< [1] live token rows, or null
  int64_t workspace_bytes;
  int64_t tokens;
  int64_t hidden_size;
  int64_t experts;
  int64_t top;
  int64_t intermediate;
  int64_t renormalize;
  int64_t weight_dtype;        ///< UNISERVE_DTYPE_BF16, _F8E4M3 or _F4E2M1
  int64_t multiprocessors;
  int64_t weight_scale_layout; ///< MXFP4: uniserve_mx_scale_layout of both scale tables; else 0
  char error[512];
  // What `MoE::select` and `MoE::routed` pass beyond the rows (crates/nn/src/modules/moe.rs:
  // 650-671, 770-775), after `error` so the fields above keep their offsets; zero = absent.
  const int32_t *map;          ///< [experts] slot of each router expert (topk writes map[e]), or null
  int64_t *load;               ///< [experts] each live route counted by router expert, or null
  int64_t local_offset;        ///< first slot of the window this layer's stacks hold
  int64_t local_experts;       ///< slots the stacks hold ([local_experts, ...]); 0 = every expert
  int64_t activation;          ///< FC1's gate: uniserve_activation (0 = silu)
};

/// Workspace bytes the call needs for these extents, or -1 for extents it does not serve. The
/// workspace's first 1024 bytes (the `ticket` view) must be zero before the first call that uses
/// it; every call leaves them zero (the rest needs no initialisation). A call at decode sizes that
/// finds them not zero fails loudly: its output is NaN, and the words are cleared for the next call.
UNISERVE_EXTERN_C int64_t uniserve_moe_layer_workspace(int64_t tokens, int64_t hidden_size,
                                                       int64_t experts, int64_t top,
                                                       int64_t intermediate, int64_t weight_dtype);

/// Offsets (bytes from `workspace`) of the intermediate tensors, for callers that read them:
/// scores, ids, weights, the seven sort maps, gated rows, products. At decode sizes (the fused
/// front end, at most 4096 routes, fewer than 24 per local expert) the layer skips the sort, for
/// every weight type: then expanded_to_permuted holds each route's own index (token * top + k)
/// where the route is live and in the window and -1 elsewhere, the other six maps are not
/// written, and gated rows and products (and the quantised gated rows and their scales) sit at
/// those expanded positions.
struct uniserve_moe_layer_views {
  int64_t ticket;              ///< [256] u32 counters of the fused decode front end (offset 0)
  int64_t scores;              ///< [tokens, experts] bf16
  int64_t ids;                 ///< [tokens, top] i32
  int64_t weights;             ///< [tokens, top] f32
  int64_t tile_to_expert;      ///< [max_tiles] i32
  int64_t tile_to_limit;       ///< [max_tiles] i32
  int64_t expanded_to_permuted;///< [tokens, top] i32
  int64_t permuted_to_expanded;///< [permuted_rows] i32
  int64_t permuted_to_token;   ///< [permuted_rows] i32
  int64_t total_padded_tokens; ///< [1] i32
  int64_t num_non_exiting_tiles;///< [1] i32
  int64_t gated;               ///< [permuted_rows, intermediate] bf16
  int64_t products;            ///< [permuted_rows, hidden_size] bf16
  int64_t hidden_q;            ///< fp8 and MX: [tokens, hidden_size] e4m3
  int64_t hidden_s;            ///< fp8: [tokens, hidden_size / 128] f32; MX: [tokens, hidden_size / 32]
                               ///< E8M0, or with route_scales stage-major by permuted row
                               ///< [hidden_size / 128, permuted_rows, 4]
  int64_t gated_q;             ///< fp8: [permuted_rows, intermediate] e4m3
  int64_t gated_s;             ///< fp8: [permuted_rows, intermediate / 128] f32, or with
                               ///< route_scales [intermediate / 128, permuted_rows];
                               ///< MX: [permuted_rows, intermediate / 32] E8M0, or with route_scales
                               ///< [intermediate / 128, permuted_rows, 4]
  int64_t hidden_route_s;      ///< fp8 with route_scales: [hidden_size / 128, permuted_rows] f32,
                               ///< the scale of each route's token by permuted row; else -1
  int64_t route_scales;        ///< 1 when the fp8 or MX products take their activation scales
                               ///< route-major (prefill shapes), else 0
  int64_t max_tiles;
  int64_t permuted_rows;
  int64_t total;
};

UNISERVE_EXTERN_C int32_t uniserve_moe_layer_views_of(int64_t tokens, int64_t hidden_size,
                                                      int64_t experts, int64_t top,
                                                      int64_t intermediate, int64_t weight_dtype,
                                                      struct uniserve_moe_layer_views *views);

UNISERVE_EXTERN_C int32_t uniserve_moe_layer(const struct uniserve_moe_layer_call *call, void *stream);

/// Bytes of the library's per-device scratch for uniserve_moe_layer_no_alloc: the intermediates
/// of 30B-shaped layers (hidden 2048, intermediate 768, 128 experts, top 8) up to 2991 tokens with
/// e4m3 weights (3887 bf16; 64 tokens take 90-103 MiB), and of 235B-shaped ones (hidden 4096,
/// intermediate 1536) up to 543 tokens with e4m3 weights (943 bf16).
#define UNISERVE_MOE_LAYER_SCRATCH_BYTES (256ll << 20)

/// No counterpart in the reference. For callers that cannot allocate - code under HIP graph
/// capture, tight serving loops, harnesses that forbid hipMalloc: uniserve_moe_layer with the
/// intermediates in a library-owned device array of UNISERVE_MOE_LAYER_SCRATCH_BYTES per GPU
/// (held from the library's load to the process's end) instead of a caller workspace;
/// `workspace` and `workspace_bytes` are ignored, everything else is read as uniserve_moe_layer
/// reads it. Extents whose intermediates (uniserve_moe_layer_workspace) exceed the scratch are
/// refused with a message. Nothing is allocated. The first call on each GPU looks the array's
/// address up (hipGetSymbolAddress, a host-side query) and issues nothing else: the array is
/// zero-initialised storage, so its counter words start at zero, and every call leaves them zero;
/// every other intermediate is written before it is read. Any call, the first included, may be
/// made under stream capture (no memset is ever issued). All calls on
/// one GPU share its array, so calls that overlap on one GPU (concurrent streams or threads) race;
/// serialise them.
UNISERVE_EXTERN_C int32_t uniserve_moe_layer_no_alloc(const struct uniserve_moe_layer_call *call, void *stream);

/// The layer's launches in order. Which step launches what depends on the call's size:
/// - decode sizes (at most 4096 routes over at most 512 local experts, a router of at most 1024
///   experts): ROUTER launches the front end - router scores and topk, plus the sort where the
///   layer does not skip it, plus the hidden rows' e4m3 / MXFP8 quantisation for those weights -
///   and TOPK, SORT and QUANTIZE_HIDDEN launch nothing;
/// - prefill sizes (at most 128 experts, hidden a multiple of 128): ROUTER launches router scores,
///   topk and the hidden rows' quantisation in one kernel (in a call that also runs SORT, the sort's
///   per-chunk counts too, so that SORT launches only its placement), TOPK launches nothing, SORT the sort,
///   and QUANTIZE_HIDDEN only the copy of each token's scales to its routes' rows where the
///   products take them route-major (views.route_scales) and the sort's placement has not made
///   it (the placement makes it for more than 4096 routes, hidden a multiple of 512 up to 4096);
/// - otherwise each step launches its own operator.
/// The quantiser steps launch nothing for bf16 weights, and QUANTIZE_GATED nothing where FC1
/// writes its rows already quantised (e4m3 at prefill sizes; MXFP4 with route-major scales; and, for
/// both e4m3 and MXFP4, at decode sizes where the local experts with routes times intermediate / 64
/// reach 512 - 30B at 64 tokens, not one token - with an intermediate size of whole 128-column
/// groups for e4m3).
enum uniserve_moe_layer_step {
  UNISERVE_MOE_LAYER_ROUTER = 0,
  UNISERVE_MOE_LAYER_TOPK = 1,
  UNISERVE_MOE_LAYER_SORT = 2,
  UNISERVE_MOE_LAYER_QUANTIZE_HIDDEN = 3,
  UNISERVE_MOE_LAYER_GATHER = 4,
  UNISERVE_MOE_LAYER_QUANTIZE_GATED = 5,
  UNISERVE_MOE_LAYER_ROUTE = 6,
  UNISERVE_MOE_LAYER_UNPERMUTE = 7,
};

/// One step of `uniserve_moe_layer` alone, exactly as the full call launches it, over the
/// workspace a full call with the same arguments left (for profiling a step inside the layer;
/// no counterpart in the reference).
UNISERVE_EXTERN_C int32_t uniserve_moe_layer_step(const struct uniserve_moe_layer_call *call, int32_t step,
                                                  void *stream);

/// `ops::moe::max_tiles` (crates/ops/src/moe/mod.rs:63-70): the most tiles `tokens * top` routes
/// over `local_experts` can fill at `tile` rows per tile.
UNISERVE_EXTERN_C int64_t uniserve_moe_max_tiles(int64_t tokens, int64_t top, int64_t local_experts,
                                                 int64_t tile);

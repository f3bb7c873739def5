// SPDX-License-Identifier: Apache-2.0
//
// The routed MoE layer as one call: `MoE::routed` (crates/nn/src/modules/moe.rs:770-795) issues
// router gemm -> topk_softmax -> moe_sort -> gather_gemm -> route_gemm -> moe_unpermute, in that
// order (the order crates/nn/tests/moe.rs:1402-1438 records); this driver issues the same entries
// on one stream over intermediates carved from a caller-owned workspace, so it allocates nothing,
// reads nothing back and can be captured into a HIP graph. With e4m3 weights the activations of
// each product are quantised per row per 128 channels first (two more launches); with MXFP4
// weights they are quantised to MXFP8 (per row per 32 channels, E8M0 scales) the same way.
#include <cstring>
#include <mutex>

#include "common.hpp"
#include "grouped_fp8.hpp"
#include "grouped_mx.hpp"
#include "expert_stream.hpp"
#include "moe_front.hpp"
#include "router_gemm.hpp"
#include "uniserve_gather_gemm.h"
#include "uniserve_moe_fp8.h"
#include "uniserve_moe_layer.h"
#include "uniserve_moe_mx.h"
#include "uniserve_moe_sort.h"
#include "uniserve_moe_unpermute.h"
#include "uniserve_route_gemm.h"
#include "uniserve_topk_softmax.h"

namespace uniserve {
int32_t gather_gemm_bf16(const uniserve_gather_call *call, int32_t activation, void *stream);
}

namespace {

constexpr int64_t kTile = 128;
constexpr int64_t kAlign = 256;

int64_t aligned(int64_t bytes) { return (bytes + kAlign - 1) / kAlign * kAlign; }

bool views_of(int64_t tokens, int64_t hidden, int64_t experts, int64_t top, int64_t intermediate,
              int64_t weight_dtype, uniserve_moe_layer_views *v) {
  if (tokens < 0 || hidden <= 0 || experts <= 0 || top <= 0 || top > experts || intermediate <= 0) return false;
  if (weight_dtype != UNISERVE_DTYPE_BF16 && weight_dtype != UNISERVE_DTYPE_F8E4M3 &&
      weight_dtype != UNISERVE_DTYPE_F4E2M1)
    return false;
  std::memset(v, 0, sizeof(*v));
  v->max_tiles = uniserve_moe_max_tiles(tokens, top, experts, kTile);
  v->permuted_rows = v->max_tiles * kTile;
  int64_t at = 0;
  auto take = [&](int64_t bytes) {
    const int64_t here = at;
    at += aligned(bytes > 0 ? bytes : 1);
    return here;
  };
  v->ticket = take(uniserve::kFrontTicketBytes);  // first: the words a caller zeroes before a workspace's first call
  v->scores = take(tokens * experts * 2);
  v->ids = take(tokens * top * 4);
  v->weights = take(tokens * top * 4);
  v->tile_to_expert = take(v->max_tiles * 4);
  v->tile_to_limit = take(v->max_tiles * 4);
  v->expanded_to_permuted = take(tokens * top * 4);
  v->permuted_to_expanded = take(v->permuted_rows * 4);
  v->permuted_to_token = take(v->permuted_rows * 4);
  v->total_padded_tokens = take(4);
  v->num_non_exiting_tiles = take(4);
  v->gated = take(v->permuted_rows * intermediate * 2);
  v->products = take(v->permuted_rows * hidden * 2);
  if (weight_dtype == UNISERVE_DTYPE_F8E4M3) {
    v->hidden_q = take(tokens * hidden);
    v->hidden_s = take(tokens * (hidden / 128) * 4);
    v->gated_q = take(v->permuted_rows * intermediate);
    v->gated_s = take(v->permuted_rows * (intermediate / 128) * 4);
    v->route_scales = uniserve::fp8_route_scales(tokens, top, experts, hidden, intermediate, v->permuted_rows) ? 1 : 0;
    v->hidden_route_s = v->route_scales ? take(v->permuted_rows * (hidden / 128) * 4) : -1;
  } else if (weight_dtype == UNISERVE_DTYPE_F4E2M1) {
    // Prefill shapes: both activation scale tables stage-major by permuted row.
    v->route_scales = uniserve::mx_route_scales(tokens, top, experts, hidden, intermediate, v->permuted_rows) ? 1 : 0;
    v->hidden_q = take(tokens * hidden);
    v->hidden_s = take((v->route_scales ? v->permuted_rows : tokens) * (hidden / 32));
    v->gated_q = take(v->permuted_rows * intermediate);
    v->gated_s = take(v->permuted_rows * (intermediate / 32));
    v->hidden_route_s = -1;
  } else {
    v->hidden_q = v->hidden_s = v->gated_q = v->gated_s = v->hidden_route_s = -1;
  }
  v->total = at;
  return true;
}

template <class Call>
int32_t forward_error(const uniserve_moe_layer_call *layer, const char *stage, const Call &inner) {
  return ::uniserve::refuse_into(const_cast<char *>(layer->error), "%s: %s", stage, inner.error);
}

}  // namespace

extern "C" int64_t uniserve_moe_max_tiles(int64_t tokens, int64_t top, int64_t local_experts, int64_t tile) {
  const int64_t expanded = tokens * top;
  if (expanded <= local_experts || tile == 0) return expanded;
  return (expanded + (tile - 1) * local_experts) / tile;
}

extern "C" int32_t uniserve_moe_layer_views_of(int64_t tokens, int64_t hidden_size, int64_t experts,
                                               int64_t top, int64_t intermediate, int64_t weight_dtype,
                                               uniserve_moe_layer_views *views) {
  if (views == nullptr) return 1;
  return views_of(tokens, hidden_size, experts, top, intermediate, weight_dtype, views) ? 0 : 1;
}

extern "C" int64_t uniserve_moe_layer_workspace(int64_t tokens, int64_t hidden_size, int64_t experts,
                                                int64_t top, int64_t intermediate, int64_t weight_dtype) {
  uniserve_moe_layer_views v;
  if (!views_of(tokens, hidden_size, experts, top, intermediate, weight_dtype, &v)) return -1;
  return v.total;
}

namespace {

/// moe_sort over the window's experts, as the layer calls it.
/// `counted`: the prefill front end wrote its chunks' counts to `scratch` (only with the two-launch
/// sort: prefill_counts_sort). `words` (two-launch sort only): token_words' `words` 32-bit words per
/// token go to each route's row of route_words ([words, word_rows]) as the placement places it.
int32_t run_sort(const uniserve_moe_layer_call *call, int32_t *ids, float *weights, int32_t *t2e, int32_t *t2l,
                 int32_t *e2p, int32_t *p2e, int32_t *p2t, int32_t *padded, int32_t *tiles, int64_t local_experts,
                 int32_t *scratch, void *stream, bool counted = false, const uint32_t *token_words = nullptr,
                 uint32_t *route_words = nullptr, int64_t words = 0, int64_t word_rows = 0) {
  const int64_t routes = call->tokens * call->top;
  if (scratch != nullptr && uniserve::layer_sort_two_launches(routes, local_experts)) {
    // Above one workgroup's routes: the count, then the scan folded into the placement, with the
    // per-chunk counts in `scratch`.
    uniserve::sort::SortParams p{};
    p.ids = ids;
    p.tile_to_expert = t2e;
    p.tile_to_limit = t2l;
    p.expanded_to_permuted = e2p;
    p.permuted_to_expanded = p2e;
    p.permuted_to_token = p2t;
    p.total_padded_tokens = padded;
    p.num_non_exiting_tiles = tiles;
    p.live_tokens = call->live_tokens;
    p.routes = routes;
    p.top = call->top;
    p.local_experts = static_cast<int32_t>(local_experts);
    p.local_offset = static_cast<int32_t>(call->local_offset);
    p.tile = static_cast<int32_t>(kTile);
    int bits = 0;
    while ((1ll << bits) <= local_experts) ++bits;
    p.key_bits = bits;
    p.token_words = token_words;
    p.route_words = route_words;
    p.words = words;
    p.word_rows = word_rows;
    uniserve::launch_layer_sort(p, scratch, static_cast<hipStream_t>(stream), counted);
    return uniserve::launched(call, "moe_sort");
  }
  uniserve_moe_sort_call sort{};
  sort.ids = ids;
  sort.scales = weights;
  sort.tile_to_expert = t2e;
  sort.tile_to_limit = t2l;
  sort.expanded_to_permuted = e2p;
  sort.permuted_to_expanded = p2e;
  sort.total_padded_tokens = padded;
  sort.num_non_exiting_tiles = tiles;
  sort.tokens = call->tokens;
  sort.top = call->top;
  sort.experts = call->experts;
  sort.local_experts = local_experts;
  sort.local_offset = call->local_offset;
  sort.tile_tokens = kTile;
  sort.scales_dtype = UNISERVE_DTYPE_F32;
  sort.live_tokens = call->live_tokens;
  sort.permuted_to_token = p2t;
  if (uniserve_moe_sort(&sort, stream) != 0) return forward_error(call, "moe_sort", sort);
  return 0;
}

/// MXFP4 experts: quantise the hidden rows to MXFP8, FC1, quantise the live gated rows, FC2.
/// `by_expert` set: the decode products without a sort (rows at expanded positions).
template <class Want>
int32_t run_mx_products(const uniserve_moe_layer_call *call, const uniserve_moe_layer_views &v, char *ws,
                        const Want &want, void *stream, const uniserve::ExpertRouting *by_expert,
                        bool hidden_quantised, bool token_scales_waiting) {
  using namespace uniserve;
  auto at = [&](int64_t offset) { return static_cast<void *>(ws + offset); };
  const auto *t2e = static_cast<const int32_t *>(at(v.tile_to_expert));
  const auto *t2l = static_cast<const int32_t *>(at(v.tile_to_limit));
  const auto *p2e = static_cast<const int32_t *>(at(v.permuted_to_expanded));
  const auto *tiles = static_cast<const int32_t *>(at(v.num_non_exiting_tiles));

  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t scale_rows = v.route_scales ? v.permuted_rows : 0;
  uniserve_quantize_mxfp8_call qx{};
  qx.input = call->hidden;
  qx.out = at(v.hidden_q);
  qx.scales = static_cast<uint8_t *>(at(v.hidden_s));
  qx.rows = call->tokens;
  qx.width = call->hidden_size;
  qx.input_dtype = UNISERVE_DTYPE_BF16;
  if (!want(UNISERVE_MOE_LAYER_QUANTIZE_HIDDEN) || (hidden_quantised && !token_scales_waiting)) {
  } else if (hidden_quantised) {
    // The prefill front end quantised the rows; its token-major scale bytes (parked in the
    // products' rows) go to the routes' rows, one 4-byte word per 128-channel stage.
    launch_scatter_route_words(static_cast<const uint32_t *>(at(v.products)), p2e,
                               static_cast<const int32_t *>(at(v.total_padded_tokens)),
                               static_cast<uint32_t *>(at(v.hidden_s)), scale_rows, call->top,
                               call->hidden_size / 128, s);
    if (int32_t status = launched(call, "scatter of the hidden scales")) return status;
  } else if (scale_rows != 0) {
    // Each token's scale words go to its routes' permuted rows.
    launch_quantize_mxfp8(call->hidden, false, static_cast<uint8_t *>(at(v.hidden_q)), nullptr, nullptr, call->tokens,
                          call->hidden_size, s, static_cast<uint8_t *>(at(v.hidden_s)),
                          static_cast<const int32_t *>(at(v.expanded_to_permuted)), call->top, scale_rows);
    if (int32_t status = launched(call, "quantize_mxfp8")) return status;
  } else if (uniserve_quantize_mxfp8(&qx, stream) != 0) {
    return forward_error(call, "quantize_mxfp8", qx);
  }

  // The call's scale pointers carry E8M0 bytes for MXFP4 stacks.
  uniserve_gather_mx_call fc1{};
  fc1.hidden = at(v.hidden_q);
  fc1.hidden_scales = static_cast<const uint8_t *>(at(v.hidden_s));
  fc1.weights = call->up_gate;
  fc1.weight_scales = reinterpret_cast<const uint8_t *>(call->up_gate_scales);
  fc1.out = at(v.gated);
  fc1.tile_to_expert = t2e;
  fc1.tile_to_limit = t2l;
  fc1.permuted_to_expanded = p2e;
  fc1.num_non_exiting_tiles = tiles;
  fc1.tokens = call->tokens;
  fc1.permuted_rows = v.permuted_rows;
  fc1.width = 2 * call->intermediate;
  fc1.hidden_size = call->hidden_size;
  fc1.experts = call->experts;
  fc1.top = call->top;
  fc1.out_dtype = UNISERVE_DTYPE_BF16;
  fc1.multiprocessors = call->multiprocessors;
  fc1.weight_scale_layout = call->weight_scale_layout;
  // Decode sizes on the unsplit kernel: FC1 also writes FC2's MXFP8 operand (QUANTIZE_GATED then
  // launches nothing).
  const bool fc1_quantizes = by_expert != nullptr && mx_fc1_quantizes_by_expert(*by_expert, 2 * call->intermediate);
  if (!want(UNISERVE_MOE_LAYER_GATHER)) {
  } else if (by_expert != nullptr) {
    gather_gemm_mx_by_expert(&fc1, *by_expert, static_cast<int32_t>(call->activation), stream,
                             fc1_quantizes ? static_cast<uint8_t *>(at(v.gated_q)) : nullptr,
                             fc1_quantizes ? static_cast<uint8_t *>(at(v.gated_s)) : nullptr);
    if (int32_t status = launched(call, "gather_gemm_mx")) return status;
  } else if (gather_gemm_mx(&fc1, scale_rows, static_cast<int32_t>(call->activation), stream,
                            scale_rows != 0 ? static_cast<uint8_t *>(at(v.gated_q)) : nullptr,
                            scale_rows != 0 ? static_cast<uint8_t *>(at(v.gated_s)) : nullptr) != 0) {
    // (Prefill shapes, route-major scales: FC1 writes its rows already as FC2's MXFP8 operand.)
    return forward_error(call, "gather_gemm_mx", fc1);
  }

  uniserve_quantize_mxfp8_call qg{};
  qg.input = at(v.gated);
  qg.out = at(v.gated_q);
  qg.scales = static_cast<uint8_t *>(at(v.gated_s));
  // (Without the sort: every route's row, at its expanded position.)
  qg.row_limit = by_expert != nullptr ? nullptr : static_cast<const int32_t *>(at(v.total_padded_tokens));
  qg.rows = by_expert != nullptr ? by_expert->routes : v.permuted_rows;
  qg.width = call->intermediate;
  qg.input_dtype = UNISERVE_DTYPE_BF16;
  if (!want(UNISERVE_MOE_LAYER_QUANTIZE_GATED) || scale_rows != 0 || fc1_quantizes) {
    // (With route-major scales, or at decode sizes on the unsplit kernel, FC1 wrote the quantised
    // rows itself.)
  } else if (uniserve_quantize_mxfp8(&qg, stream) != 0) {
    return forward_error(call, "quantize_mxfp8", qg);
  }

  uniserve_route_mx_call fc2{};
  fc2.rows = at(v.gated_q);
  fc2.row_scales = static_cast<const uint8_t *>(at(v.gated_s));
  fc2.weights = call->down;
  fc2.weight_scales = reinterpret_cast<const uint8_t *>(call->down_scales);
  fc2.out = at(v.products);
  fc2.tile_to_expert = t2e;
  fc2.tile_to_limit = t2l;
  fc2.permuted_to_expanded = p2e;
  fc2.num_non_exiting_tiles = tiles;
  fc2.permuted_rows = v.permuted_rows;
  fc2.width = call->hidden_size;
  fc2.intermediate = call->intermediate;
  fc2.experts = call->experts;
  fc2.out_dtype = UNISERVE_DTYPE_BF16;
  fc2.multiprocessors = call->multiprocessors;
  fc2.weight_scale_layout = call->weight_scale_layout;
  if (!want(UNISERVE_MOE_LAYER_ROUTE)) {
  } else if (by_expert != nullptr) {
    route_gemm_mx_by_expert(&fc2, *by_expert, stream);
    if (int32_t status = launched(call, "route_gemm_mx")) return status;
  } else if (route_gemm_mx(&fc2, scale_rows, stream) != 0) {
    return forward_error(call, "route_gemm_mx", fc2);
  }
  return 0;
}

/// The layer's launches, all of them (`only` < 0) or the one step `only`, over the workspace
/// `workspace` of `workspace_bytes`.
int32_t run_layer(const uniserve_moe_layer_call *call, int32_t only, void *stream, void *workspace,
                  int64_t workspace_bytes) {
  using namespace uniserve;
  auto want = [&](int32_t step) { return only < 0 || only == step; };
  return guarded(call, [&]() -> int32_t {
    if (call->hidden == nullptr || call->router == nullptr || call->up_gate == nullptr ||
        call->down == nullptr || call->out == nullptr || workspace == nullptr)
      return UNISERVE_REFUSE(call, "moe_layer needs hidden, router, both stacks, out and a workspace");
    const bool fp8 = call->weight_dtype == UNISERVE_DTYPE_F8E4M3;
    const bool mx = call->weight_dtype == UNISERVE_DTYPE_F4E2M1;
    if ((fp8 || mx) && (call->up_gate_scales == nullptr || call->down_scales == nullptr))
      return UNISERVE_REFUSE(call, "moe_layer: quantised stacks need their block scales");
    if (mx && call->weight_scale_layout != UNISERVE_MX_SCALES_ROW_MAJOR &&
        call->weight_scale_layout != UNISERVE_MX_SCALES_STAGE_MAJOR)
      return UNISERVE_REFUSE(call, "moe_layer: no MX scale layout %lld", static_cast<long long>(call->weight_scale_layout));
    if (mx && (call->hidden_size % 256 != 0 || call->intermediate % 256 != 0))
      return UNISERVE_REFUSE(call, "moe_layer: MXFP4 stacks need hidden and intermediate sizes of whole 256-element chunks");
    if (reinterpret_cast<uintptr_t>(workspace) % kAlign != 0)
      return UNISERVE_REFUSE(call, "moe_layer needs a 256-byte aligned workspace");
    uniserve_moe_layer_views v;
    if (!views_of(call->tokens, call->hidden_size, call->experts, call->top, call->intermediate,
                  call->weight_dtype, &v))
      return UNISERVE_REFUSE(call, "moe_layer does not serve these extents or this weight type");
    if (workspace_bytes < v.total)
      return UNISERVE_REFUSE(call, "moe_layer needs %lld workspace bytes, has %lld",
                             static_cast<long long>(v.total), static_cast<long long>(workspace_bytes));
    if (call->activation != UNISERVE_ACTIVATION_SILU && call->activation != UNISERVE_ACTIVATION_GELU_TANH)
      return UNISERVE_REFUSE(call, "moe_layer: FC1 gates with silu or gelu_tanh, not activation %lld",
                             static_cast<long long>(call->activation));
    // The window the stacks hold (the whole router when local_experts is 0). The products are
    // told the router's expert count: they read it for their kernel choice only, and the views
    // above were laid out with it (a window never needs more tiles than every expert).
    const int64_t local_experts = call->local_experts == 0 ? call->experts : call->local_experts;
    if (local_experts < 0 || call->local_offset < 0 || call->local_offset + local_experts > call->experts)
      return UNISERVE_REFUSE(call, "moe_layer's expert window [%lld, %lld + %lld) lies outside the router's %lld experts",
                             static_cast<long long>(call->local_offset), static_cast<long long>(call->local_offset),
                             static_cast<long long>(local_experts), static_cast<long long>(call->experts));
    if (call->tokens == 0) return 0;
    if (call->hidden_size % 64 != 0) return UNISERVE_REFUSE(call, "moe_layer needs a hidden size of whole 64-element steps");
    if (!dma_rows_fit(call->tokens, call->hidden_size * 2))
      return UNISERVE_REFUSE(call, "moe_layer serves hidden rows below 4 GiB (%lld tokens of %lld bytes)",
                             static_cast<long long>(call->tokens), static_cast<long long>(call->hidden_size * 2));
    const int32_t activation = static_cast<int32_t>(call->activation);
    // Decode sizes: no sort - the fused front end routes, and the products' workgroups each serve
    // one local expert, finding its routes in `ids` (rows at expanded positions).
    const int64_t routes = call->tokens * call->top;
    const bool front = front_fits(call->tokens, call->experts, call->hidden_size, call->top, local_experts);
    const bool by_expert = front &&
                           expert_stream_fits(routes, local_experts, call->hidden_size, call->intermediate, true) &&
                           expert_stream_fits(routes, local_experts, call->intermediate, call->hidden_size, false) &&
                           (!mx || (call->hidden_size % 256 == 0 && call->intermediate % 256 == 0));

    // e4m3 and MXFP4 at those sizes: the front end also quantises the hidden rows (QUANTIZE_HIDDEN
    // then launches nothing).
    const bool front_quantizes = front && (fp8 || mx) && !v.route_scales && call->hidden_size % 128 == 0;
    // Prefill sizes: router scores, topk and (e4m3, MXFP4) the hidden rows' quantisation in one
    // launch (ROUTER; TOPK launches nothing). The scales come out token-major; where the products
    // take them route-major, QUANTIZE_HIDDEN copies each token's scales to its routes' rows once
    // the sort has placed them.
    const bool prefill_front =
        !front && prefill_front_fits(call->tokens, call->experts, call->hidden_size, call->top);
    const bool prefill_quantizes = prefill_front && (fp8 || mx);

    char *ws = static_cast<char *>(workspace);
    auto at = [&](int64_t offset) { return static_cast<void *>(ws + offset); };
    const hipStream_t s = static_cast<hipStream_t>(stream);
    int32_t *ids = static_cast<int32_t *>(at(v.ids));
    float *weights = static_cast<float *>(at(v.weights));
    int32_t *t2e = static_cast<int32_t *>(at(v.tile_to_expert));
    int32_t *t2l = static_cast<int32_t *>(at(v.tile_to_limit));
    int32_t *e2p = static_cast<int32_t *>(at(v.expanded_to_permuted));
    int32_t *p2e = static_cast<int32_t *>(at(v.permuted_to_expanded));
    int32_t *p2t = static_cast<int32_t *>(at(v.permuted_to_token));
    int32_t *padded = static_cast<int32_t *>(at(v.total_padded_tokens));
    int32_t *tiles = static_cast<int32_t *>(at(v.num_non_exiting_tiles));
    // The sort's per-chunk counts: the last bytes of the products' rows, which only FC2 writes,
    // later (the MXFP4 prefill front end parks its token-major scales at their start).
    const int64_t products_bytes = v.permuted_rows * call->hidden_size * 2;
    const int64_t sort_bytes = (layer_sort_scratch_bytes(call->tokens, call->top, local_experts) + 255) / 256 * 256;
    int32_t *sort_scratch =
        sort_bytes + call->tokens * (call->hidden_size / 32) <= products_bytes
            ? reinterpret_cast<int32_t *>(static_cast<char *>(at(v.products)) + products_bytes - sort_bytes)
            : nullptr;
    // Prefill e4m3 / MXFP4 with route-major scales: the two-launch sort's placement copies each
    // token's scales (token-major, from the front end) to its routes' rows (QUANTIZE_HIDDEN then
    // launches nothing); the one-workgroup sort leaves the copy to QUANTIZE_HIDDEN.
    const bool sort_scatters = prefill_quantizes && v.route_scales && sort_scratch != nullptr &&
                               layer_sort_two_launches(routes, local_experts) && call->hidden_size % 512 == 0 &&
                               call->hidden_size / 128 <= sort::kMaxRouteWords;

    // Decode sizes: router, topk and sort in one launch (at the ROUTER step; TOPK and SORT launch
    // nothing).
    if (front) {
      if (want(UNISERVE_MOE_LAYER_ROUTER)) {
        FrontParams fp{};
        fp.x = static_cast<const uint16_t *>(call->hidden);
        fp.w = static_cast<const uint16_t *>(call->router);
        fp.bias = call->router_bias;
        fp.scores = static_cast<uint16_t *>(at(v.scores));
        fp.tokens = call->tokens;
        fp.experts = call->experts;
        fp.hidden = call->hidden_size;
        fp.top = static_cast<int32_t>(call->top);
        fp.renormalize = call->renormalize ? 1 : 0;
        fp.map = call->map;
        fp.live = call->live_tokens;
        fp.load = reinterpret_cast<unsigned long long *>(call->load);
        fp.ids = ids;
        fp.weights = weights;
        fp.ticket = static_cast<uint32_t *>(at(v.ticket));
        sort::SortParams &sp = fp.sort;
        sp.ids = ids;
        sp.tile_to_expert = t2e;
        sp.tile_to_limit = t2l;
        sp.expanded_to_permuted = e2p;
        sp.permuted_to_expanded = p2e;
        sp.permuted_to_token = p2t;
        sp.total_padded_tokens = padded;
        sp.num_non_exiting_tiles = tiles;
        sp.live_tokens = call->live_tokens;
        sp.routes = call->tokens * call->top;
        sp.top = call->top;
        sp.local_experts = static_cast<int32_t>(local_experts);
        sp.local_offset = static_cast<int32_t>(call->local_offset);
        sp.tile = static_cast<int32_t>(kTile);
        int bits = 0;
        while ((1ll << bits) <= local_experts) ++bits;
        sp.key_bits = bits;
        fp.sort_routes = by_expert ? 0 : 1;
        if (front_quantizes) {
          fp.hidden_codes = static_cast<uint8_t *>(at(v.hidden_q));
          if (mx) fp.hidden_mx_scales = static_cast<uint8_t *>(at(v.hidden_s));
          else fp.hidden_scales = static_cast<float *>(at(v.hidden_s));
        }
        if (by_expert && local_front_fits(call->tokens, call->experts, call->hidden_size, call->top))
          launch_local_front(fp, s);
        else if (by_expert && split_front_fits(call->tokens, call->experts, call->hidden_size, call->top))
          launch_split_front(fp, s);
        else
          launch_front(fp, s);
        if (int32_t status = launched(call, "router, topk and sort")) return status;
      }
    } else if (prefill_front) {
      // A call that runs both steps lets the front end count the sort's chunks (SORT then launches
      // the placement alone); a SORT step on its own counts again from the ids.
      const bool front_counts = want(UNISERVE_MOE_LAYER_ROUTER) && want(UNISERVE_MOE_LAYER_SORT) &&
                                sort_scratch != nullptr && layer_sort_two_launches(routes, local_experts);
      if (want(UNISERVE_MOE_LAYER_ROUTER)) {
        PrefillFrontParams pp{};
        if (front_counts) {
          pp.chunk_counts = sort_scratch;
          pp.local_offset = static_cast<int32_t>(call->local_offset);
          pp.local_experts = static_cast<int32_t>(local_experts);
        }
        pp.x = static_cast<const uint16_t *>(call->hidden);
        pp.w = static_cast<const uint16_t *>(call->router);
        pp.bias = call->router_bias;
        pp.scores = static_cast<uint16_t *>(at(v.scores));
        pp.tokens = call->tokens;
        pp.experts = call->experts;
        pp.hidden = call->hidden_size;
        pp.top = static_cast<int32_t>(call->top);
        pp.renormalize = call->renormalize ? 1 : 0;
        pp.map = call->map;
        pp.live = call->live_tokens;
        pp.load = reinterpret_cast<unsigned long long *>(call->load);
        pp.ids = ids;
        pp.weights = weights;
        if (fp8) {
          pp.codes = static_cast<uint8_t *>(at(v.hidden_q));
          pp.scales = static_cast<float *>(at(v.hidden_s));
        } else if (mx) {
          // Route-major MX scales: the token-major bytes wait in the products' rows (written only
          // by FC2, later) until QUANTIZE_HIDDEN copies them to the routes' rows.
          pp.codes = static_cast<uint8_t *>(at(v.hidden_q));
          pp.mx_scales = static_cast<uint8_t *>(at(v.route_scales ? v.products : v.hidden_s));
        }
        launch_prefill_front(pp, s);
        if (int32_t status = launched(call, "router and topk")) return status;
      }
      if (want(UNISERVE_MOE_LAYER_SORT)) {
        // The front end's token-major scale words go route-major as the placement places each route.
        const uint32_t *token_words = nullptr;
        uint32_t *route_words = nullptr;
        if (sort_scatters) {
          token_words = static_cast<const uint32_t *>(at(fp8 ? v.hidden_s : v.products));
          route_words = static_cast<uint32_t *>(at(fp8 ? v.hidden_route_s : v.hidden_s));
        }
        if (int32_t status = run_sort(call, ids, weights, t2e, t2l, e2p, p2e, p2t, padded, tiles, local_experts, sort_scratch,
                                      stream, front_counts, token_words, route_words, call->hidden_size / 128,
                                      v.permuted_rows))
          return status;
      }
    } else {
    // 1. Router scores, bf16 (the router Linear's output dtype).
    RouterParams rp{static_cast<const uint16_t *>(call->hidden), static_cast<const uint16_t *>(call->router),
                    static_cast<uint16_t *>(at(v.scores)), call->router_bias, call->tokens, call->experts,
                    call->hidden_size, call->hidden_size, call->hidden_size, call->experts, 1.0f};
    if (want(UNISERVE_MOE_LAYER_ROUTER)) {
      launch_router(rp, s);
      if (int32_t status = launched(call, "router gemm")) return status;
    }

    // 2. topk_softmax over the bf16 scores.
    char message[512] = {0};
    if (want(UNISERVE_MOE_LAYER_TOPK) && uniserve_topk_softmax_launch(at(v.scores), 1, call->experts, static_cast<int32_t>(call->tokens),
                                     static_cast<int32_t>(call->experts), static_cast<int32_t>(call->top),
                                     call->renormalize ? 1 : 0, nullptr, -1, ids, weights, call->map,
                                     reinterpret_cast<const uint32_t *>(call->live_tokens),
                                     call->load, stream,
                                     message, sizeof(message)) != 0)
      return UNISERVE_REFUSE(call, "topk_softmax: %s", message);

    // 3. moe_sort over the window's experts.
    if (want(UNISERVE_MOE_LAYER_SORT)) {
      if (int32_t status = run_sort(call, ids, weights, t2e, t2l, e2p, p2e, p2t, padded, tiles, local_experts, sort_scratch, stream))
        return status;
    }
    }

    // 4-5. The two products.
    if (mx) {
      const ExpertRouting routing{ids, call->live_tokens, routes, call->top, call->local_offset, local_experts};
      if (int32_t status = run_mx_products(call, v, ws, want, stream, by_expert ? &routing : nullptr,
                                                 front_quantizes || prefill_quantizes,
                                                 prefill_quantizes && v.route_scales && !sort_scatters))
        return status;
    } else if (by_expert && !fp8) {
      ExpertStream e{};
      e.ids = ids;
      e.live_tokens = call->live_tokens;
      e.routes = routes;
      e.top = call->top;
      e.local_offset = call->local_offset;
      e.local_experts = local_experts;
      e.activation = activation;
      if (want(UNISERVE_MOE_LAYER_GATHER)) {
        ExpertStream fc1 = e;
        fc1.act = call->hidden;
        fc1.weights = call->up_gate;
        fc1.out = at(v.gated);
        fc1.K = call->hidden_size;
        fc1.n_total = 2 * call->intermediate;
        fc1.out_width = call->intermediate;
        launch_expert_stream(fc1, true, s);
        if (int32_t status = launched(call, "gather_gemm")) return status;
      }
      if (want(UNISERVE_MOE_LAYER_ROUTE)) {
        ExpertStream fc2 = e;
        fc2.act = at(v.gated);
        fc2.weights = call->down;
        fc2.out = at(v.products);
        fc2.K = call->intermediate;
        fc2.n_total = call->hidden_size;
        fc2.out_width = call->hidden_size;
        launch_expert_stream(fc2, false, s);
        if (int32_t status = launched(call, "route_gemm")) return status;
      }
    } else if (!fp8) {
      uniserve_gather_call fc1{};
      fc1.hidden = call->hidden;
      fc1.weights = call->up_gate;
      fc1.out = at(v.gated);
      fc1.tile_to_expert = t2e;
      fc1.tile_to_limit = t2l;
      fc1.permuted_to_expanded = p2e;
      fc1.num_non_exiting_tiles = tiles;
      fc1.tokens = call->tokens;
      fc1.permuted_rows = v.permuted_rows;
      fc1.width = 2 * call->intermediate;
      fc1.hidden_size = call->hidden_size;
      fc1.experts = call->experts;
      fc1.top = call->top;
      fc1.dtype = UNISERVE_DTYPE_BF16;
      fc1.multiprocessors = call->multiprocessors;
      if (want(UNISERVE_MOE_LAYER_GATHER) && gather_gemm_bf16(&fc1, activation, stream) != 0) return forward_error(call, "gather_gemm", fc1);

      uniserve_route_call fc2{};
      fc2.rows = at(v.gated);
      fc2.weights = call->down;
      fc2.out = at(v.products);
      fc2.tile_to_expert = t2e;
      fc2.tile_to_limit = t2l;
      fc2.permuted_to_expanded = p2e;
      fc2.num_non_exiting_tiles = tiles;
      fc2.permuted_rows = v.permuted_rows;
      fc2.width = call->hidden_size;
      fc2.intermediate = call->intermediate;
      fc2.experts = call->experts;
      fc2.dtype = UNISERVE_DTYPE_BF16;
      fc2.multiprocessors = call->multiprocessors;
      if (want(UNISERVE_MOE_LAYER_ROUTE) && uniserve_route_gemm(&fc2, stream) != 0) return forward_error(call, "route_gemm", fc2);
    } else {
      // Prefill shapes: the scales of both products' activations go route-major (block by
      // permuted row), so a tile's scales of one K block are contiguous.
      const int64_t scale_rows = v.route_scales ? v.permuted_rows : 0;
      uniserve_quantize_fp8_call qx{};
      qx.input = call->hidden;
      qx.out = at(v.hidden_q);
      qx.scales = static_cast<float *>(at(v.hidden_s));
      qx.rows = call->tokens;
      qx.width = call->hidden_size;
      qx.input_dtype = UNISERVE_DTYPE_BF16;
      qx.group = 128;
      if (!want(UNISERVE_MOE_LAYER_QUANTIZE_HIDDEN) || front_quantizes || (prefill_quantizes && scale_rows == 0) ||
          sort_scatters) {
      } else if (prefill_quantizes) {
        // The prefill front end quantised the rows; each token's scales go to its routes' rows.
        launch_scatter_route_words(static_cast<const uint32_t *>(at(v.hidden_s)), p2e, padded,
                                   static_cast<uint32_t *>(at(v.hidden_route_s)), scale_rows, call->top,
                                   call->hidden_size / 128, s);
        if (int32_t status = launched(call, "scatter of the hidden scales")) return status;
      } else if (scale_rows != 0) {
        launch_quantize_fp8_routes(static_cast<const uint16_t *>(call->hidden), static_cast<uint8_t *>(at(v.hidden_q)),
                                   static_cast<float *>(at(v.hidden_s)), static_cast<float *>(at(v.hidden_route_s)), e2p,
                                   call->top, scale_rows, call->tokens, call->hidden_size, s);
        if (int32_t status = launched(call, "quantize_fp8")) return status;
      } else if (uniserve_quantize_fp8(&qx, stream) != 0) {
        return forward_error(call, "quantize_fp8", qx);
      }

      if (by_expert) {
        // Decode: expert-major products over rows at expanded positions; the gated quantiser
        // takes every route's row (rows of routes not served are never read).
        GroupedFp8Params e{};
        e.ids = ids;
        e.live_tokens = call->live_tokens;
        e.routes = routes;
        e.local_offset = call->local_offset;
        e.top = call->top;
        e.activation = activation;
        // Where the unsplit kernel serves FC1 it also writes FC2's operand (QUANTIZE_GATED then
        // launches nothing).
        const bool fc1_quantizes = expert_stream_fp8_fc1_quantizes(routes, local_experts, call->intermediate);
        if (want(UNISERVE_MOE_LAYER_GATHER)) {
          GroupedFp8Params fc1 = e;
          if (fc1_quantizes) {
            fc1.out_codes = static_cast<uint8_t *>(at(v.gated_q));
            fc1.out_code_scales = static_cast<float *>(at(v.gated_s));
          }
          fc1.act = static_cast<const uint8_t *>(at(v.hidden_q));
          fc1.act_scales = static_cast<const float *>(at(v.hidden_s));
          fc1.weights = static_cast<const uint8_t *>(call->up_gate);
          fc1.weight_scales = call->up_gate_scales;
          fc1.out = static_cast<uint16_t *>(at(v.gated));
          fc1.K = call->hidden_size;
          fc1.n_total = 2 * call->intermediate;
          fc1.out_width = call->intermediate;
          launch_expert_stream_fp8(fc1, true, local_experts, s);
          if (int32_t status = launched(call, "gather_gemm_fp8")) return status;
        }
        if (want(UNISERVE_MOE_LAYER_QUANTIZE_GATED) && !fc1_quantizes) {
          launch_quantize_fp8(at(v.gated), false, static_cast<uint8_t *>(at(v.gated_q)), static_cast<float *>(at(v.gated_s)),
                              nullptr, routes, call->intermediate, s);
          if (int32_t status = launched(call, "quantize_fp8")) return status;
        }
        if (want(UNISERVE_MOE_LAYER_ROUTE)) {
          GroupedFp8Params fc2 = e;
          fc2.act = static_cast<const uint8_t *>(at(v.gated_q));
          fc2.act_scales = static_cast<const float *>(at(v.gated_s));
          fc2.weights = static_cast<const uint8_t *>(call->down);
          fc2.weight_scales = call->down_scales;
          fc2.out = static_cast<uint16_t *>(at(v.products));
          fc2.K = call->intermediate;
          fc2.n_total = call->hidden_size;
          fc2.out_width = call->hidden_size;
          launch_expert_stream_fp8(fc2, false, local_experts, s);
          if (int32_t status = launched(call, "route_gemm_fp8")) return status;
        }
      } else {
      uniserve_gather_fp8_call fc1{};
      fc1.hidden = at(v.hidden_q);
      fc1.hidden_scales = static_cast<const float *>(at(scale_rows != 0 ? v.hidden_route_s : v.hidden_s));
      fc1.weights = call->up_gate;
      fc1.weight_scales = call->up_gate_scales;
      fc1.out = at(v.gated);
      fc1.tile_to_expert = t2e;
      fc1.tile_to_limit = t2l;
      fc1.permuted_to_expanded = p2e;
      fc1.num_non_exiting_tiles = tiles;
      fc1.tokens = call->tokens;
      fc1.permuted_rows = v.permuted_rows;
      fc1.width = 2 * call->intermediate;
      fc1.hidden_size = call->hidden_size;
      fc1.experts = call->experts;
      fc1.top = call->top;
      fc1.block_n = 128;
      fc1.block_k = 128;
      fc1.out_dtype = UNISERVE_DTYPE_BF16;
      fc1.multiprocessors = call->multiprocessors;
      const bool fused = fp8_fc1_quantizes(call->tokens, call->top, call->experts, call->hidden_size, call->intermediate);
      if (!want(UNISERVE_MOE_LAYER_GATHER)) {
      } else if (fused) {
        // Prefill shapes: FC1 writes the gated rows straight in FC2's e4m3 form.
        if (gather_gemm_fp8(&fc1, static_cast<uint8_t *>(at(v.gated_q)), static_cast<float *>(at(v.gated_s)), scale_rows,
                            activation, stream) != 0)
          return forward_error(call, "gather_gemm_fp8", fc1);
      } else if (gather_gemm_fp8(&fc1, nullptr, nullptr, 0, activation, stream) != 0) {
        return forward_error(call, "gather_gemm_fp8", fc1);
      }

      uniserve_quantize_fp8_call qg{};
      qg.input = at(v.gated);
      qg.out = at(v.gated_q);
      qg.scales = static_cast<float *>(at(v.gated_s));
      qg.row_limit = padded;
      qg.rows = v.permuted_rows;
      qg.width = call->intermediate;
      qg.input_dtype = UNISERVE_DTYPE_BF16;
      qg.group = 128;
      if (want(UNISERVE_MOE_LAYER_QUANTIZE_GATED) && !fused && uniserve_quantize_fp8(&qg, stream) != 0) return forward_error(call, "quantize_fp8", qg);

      uniserve_route_fp8_call fc2{};
      fc2.rows = at(v.gated_q);
      fc2.row_scales = static_cast<const float *>(at(v.gated_s));
      fc2.weights = call->down;
      fc2.weight_scales = call->down_scales;
      fc2.out = at(v.products);
      fc2.tile_to_expert = t2e;
      fc2.tile_to_limit = t2l;
      fc2.permuted_to_expanded = p2e;
      fc2.num_non_exiting_tiles = tiles;
      fc2.permuted_rows = v.permuted_rows;
      fc2.width = call->hidden_size;
      fc2.intermediate = call->intermediate;
      fc2.experts = call->experts;
      fc2.block_n = 128;
      fc2.block_k = 128;
      fc2.out_dtype = UNISERVE_DTYPE_BF16;
      fc2.multiprocessors = call->multiprocessors;
      if (want(UNISERVE_MOE_LAYER_ROUTE) && route_gemm_fp8(&fc2, scale_rows, stream) != 0) return forward_error(call, "route_gemm_fp8", fc2);
      }
    }

    // 6. The weighted combine: permuted layout, or expanded where the products kept rows there.
    uniserve_unpermute_call combine{};
    combine.routes = at(v.products);
    combine.out = call->out;
    combine.expanded_to_permuted = e2p;
    combine.scales = weights;
    combine.tokens = call->tokens;
    combine.top = call->top;
    combine.hidden = call->hidden_size;
    combine.routes_rows = v.permuted_rows;
    combine.input_dtype = UNISERVE_DTYPE_BF16;
    combine.scales_dtype = UNISERVE_DTYPE_F32;
    combine.output_dtype = UNISERVE_DTYPE_BF16;
    combine.layout = by_expert ? UNISERVE_UNPERMUTE_LAYOUT_EXPANDED : UNISERVE_UNPERMUTE_LAYOUT_PERMUTED;
    // After the fused front end the combine also checks that the front end's counters came back to
    // zero (they do unless they were not zero before it: a workspace whose head was not cleared).
    uint32_t *ticket = front ? static_cast<uint32_t *>(at(v.ticket)) : nullptr;
    if (want(UNISERVE_MOE_LAYER_UNPERMUTE) &&
        moe_unpermute_checked(&combine, ticket, front ? front_ticket_words(call->tokens) : 0, stream) != 0)
      return forward_error(call, "moe_unpermute", combine);
    return 0;
  });
}

}  // namespace

extern "C" int32_t uniserve_moe_layer(const uniserve_moe_layer_call *call, void *stream) {
  if (call == nullptr) return 1;
  return run_layer(call, -1, stream, call->workspace, call->workspace_bytes);
}

extern "C" int32_t uniserve_moe_layer_step(const uniserve_moe_layer_call *call, int32_t step, void *stream) {
  if (call == nullptr) return 1;
  if (step < UNISERVE_MOE_LAYER_ROUTER || step > UNISERVE_MOE_LAYER_UNPERMUTE)
    return ::uniserve::refuse_into(const_cast<char *>(call->error), "moe_layer_step: no step %d", step);
  return run_layer(call, step, stream, call->workspace, call->workspace_bytes);
}

// ---- the entry that allocates nothing ------------------------------------------------------------

namespace {

/// The layer's intermediates for callers that pass no workspace: one array per device, held from
/// the library's load to the process's end. Host code never names it in a launch or a copy: the
/// name is a host-side stand-in; the device address comes from hipGetSymbolAddress, per device.
/// It has no initialiser, so it is zero-initialised storage (zero-filled when the code object is
/// loaded on a device): the front end's ticket counters at its head start at zero, and every call
/// leaves them zero. No memset is ever issued, so no call - the first one included - puts a memset
/// node into a graph its caller is capturing.
__device__ __align__(256) unsigned char scratch[UNISERVE_MOE_LAYER_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex scratch_mutex;
void *scratch_address[kMaxDevices] = {};

/// The device address of `scratch` on the current device, looked up once per device (a host-side
/// query: nothing is issued to any stream).
hipError_t scratch_of_current_device(void **address) {
  int device = -1;
  hipError_t status = hipGetDevice(&device);
  if (status != hipSuccess) return status;
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (scratch_address[device] == nullptr) {
    void *ptr = nullptr;
    status = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (status != hipSuccess) return status;
    scratch_address[device] = ptr;
  }
  *address = scratch_address[device];
  return hipSuccess;
}

}  // namespace

extern "C" int32_t uniserve_moe_layer_no_alloc(const uniserve_moe_layer_call *call, void *stream) {
  using namespace uniserve;
  return guarded(call, [&]() -> int32_t {
    uniserve_moe_layer_views v;
    if (!views_of(call->tokens, call->hidden_size, call->experts, call->top, call->intermediate,
                  call->weight_dtype, &v))
      return UNISERVE_REFUSE(call, "moe_layer does not serve these extents or this weight type");
    if (v.total > UNISERVE_MOE_LAYER_SCRATCH_BYTES)
      return UNISERVE_REFUSE(call, "moe_layer_no_alloc: these extents need %lld bytes of intermediates, more than "
                             "the library's %lld-byte scratch; pass a workspace to uniserve_moe_layer instead",
                             static_cast<long long>(v.total), static_cast<long long>(UNISERVE_MOE_LAYER_SCRATCH_BYTES));
    void *address = nullptr;
    const hipError_t status = scratch_of_current_device(&address);
    if (status != hipSuccess)
      return UNISERVE_REFUSE(call, "moe_layer_no_alloc: no scratch address on this device: %s", hipGetErrorString(status));
    return run_layer(call, -1, stream, address, UNISERVE_MOE_LAYER_SCRATCH_BYTES);
  });
}

// SPDX-License-Identifier: Apache-2.0
//
// moe_unpermute on gfx950 (operator: crates/ops/src/moe/combine.rs; reference entry:
// crates/ops/kernels/moe_unpermute/trtllm/src/entry.cpp):
//
//   out[t] = sum_{k visible} scales[t, k] * routes[row(t, k)]
//
// accumulated in FP32 in route order and rounded once into the output type. A route whose map entry
// is negative (or names no row of `routes`) contributes nothing, so a token with no visible route is
// exactly zero. HBM-bound: each lane moves 16 bytes (8 elements) of every route row of its token.
#include "common.hpp"
#include "moe_front.hpp"
#include "uniserve_moe_unpermute.h"

namespace uniserve {
namespace {

// 256 lanes (a 2048-wide bf16 row per workgroup) and non-temporal route loads - every route row is
// read once: 49 us for 8192 tokens x 8 routes x 2048, against 65 with 128 lanes and plain loads.
constexpr int kCombineThreads = 256;
constexpr int kPerLane = 8;
constexpr int kColumnsPerBlock = kCombineThreads * kPerLane;

struct CombineParams {
  const void *routes;
  void *out;
  const int32_t *expanded_to_permuted;
  const void *scales;
  int64_t top;
  int64_t hidden;
  int64_t routes_rows;
  int32_t expanded;
  // Inside the MoE layer after its fused decode front end: the front end's ticket counters, which
  // a correct launch leaves zero (null elsewhere). A nonzero word means the workspace's counters
  // were not zero before the front end ran - then its routing may have run before every score was
  // stored - so the combine writes NaN in place of the output and clears the words, so that the
  // next call routes correctly.
  uint32_t *ticket;
  int32_t ticket_words;
};

template <class Element>
__device__ __forceinline__ float widen(Element value);
template <>
__device__ __forceinline__ float widen<uint16_t>(uint16_t value) { return bf16_to_f32(value); }
template <>
__device__ __forceinline__ float widen<_Float16>(_Float16 value) { return static_cast<float>(value); }
template <>
__device__ __forceinline__ float widen<float>(float value) { return value; }

template <class Element>
__device__ __forceinline__ Element narrow(float value);
template <>
__device__ __forceinline__ uint16_t narrow<uint16_t>(float value) { return f32_to_bf16(value); }
template <>
__device__ __forceinline__ _Float16 narrow<_Float16>(float value) { return static_cast<_Float16>(value); }

/// `Element` is the route/output type (uint16_t = bf16, _Float16 = f16), `Scale` the weights'.
template <class Element, class Scale>
__global__ void __launch_bounds__(kCombineThreads) combine_kernel(CombineParams p) {
  const int64_t token = blockIdx.x;
  const int64_t column = static_cast<int64_t>(blockIdx.y) * kColumnsPerBlock + threadIdx.x * kPerLane;
  const bool in_range = column < p.hidden;
  if (!in_range && p.ticket == nullptr) return;  // with a ticket check every lane meets the barrier
  const Element *routes = static_cast<const Element *>(p.routes);
  const Scale *scales = static_cast<const Scale *>(p.scales);
  // Issued first, used last: the counter check costs no round trip of its own.
  const uint32_t ticket_word =
      p.ticket != nullptr && static_cast<int>(threadIdx.x) < p.ticket_words ? load_device(p.ticket + threadIdx.x) : 0u;
  float sum[kPerLane];
#pragma unroll
  for (int j = 0; j < kPerLane; ++j) sum[j] = 0.0f;
  // Routes in batches of kBatch: the batch's map entries and weights, then its route rows, are
  // loaded before any is used (two round trips per batch, not two per route; one in the expanded
  // layout); the sum still takes the routes in order.
  constexpr int kBatch = 8;
  for (int64_t k0 = 0; k0 < p.top; k0 += kBatch) {
    int32_t entry[kBatch];
    float weight[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t slot = token * p.top + k0 + u;
      const bool exists = k0 + u < p.top;
      entry[u] = exists ? p.expanded_to_permuted[slot] : -1;
      weight[u] = exists ? widen<Scale>(scales[slot]) : 0.0f;
    }
    uint4 packed[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      // Expanded rows sit at known places: loaded beside their map entries (one round trip), an
      // invisible route's row read and then ignored.
      const bool visible = p.expanded ? k0 + u < p.top : entry[u] >= 0 && entry[u] < p.routes_rows;
      const int64_t row = p.expanded ? token * p.top + k0 + u : entry[u];
      if (visible && in_range) {
        const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(routes + row * p.hidden + column));
        packed[u] = uint4{v[0], v[1], v[2], v[3]};
      } else {
        packed[u] = uint4{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      if (entry[u] < 0 || entry[u] >= p.routes_rows) continue;
      const Element *values = reinterpret_cast<const Element *>(&packed[u]);
#pragma unroll
      for (int j = 0; j < kPerLane; ++j) sum[j] = __builtin_fmaf(weight[u], widen<Element>(values[j]), sum[j]);
    }
  }
  if (p.ticket != nullptr && __syncthreads_or(ticket_word != 0u)) {
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) sum[j] = __builtin_nanf("");
    // The last workgroup dispatched clears the words, at its end: every other workgroup was
    // dispatched before it and read them with its first instruction, so none can see them cleared.
    if (blockIdx.x == gridDim.x - 1 && blockIdx.y == gridDim.y - 1 && static_cast<int>(threadIdx.x) < p.ticket_words)
      store_device(p.ticket + threadIdx.x, 0u);
  }
  Element result[kPerLane];
#pragma unroll
  for (int j = 0; j < kPerLane; ++j) result[j] = narrow<Element>(sum[j]);
  if (in_range)
    *reinterpret_cast<uint4 *>(static_cast<Element *>(p.out) + token * p.hidden + column) =
        *reinterpret_cast<const uint4 *>(result);
}

}  // namespace

int32_t moe_unpermute_checked(const uniserve_unpermute_call *call, uint32_t *ticket, int32_t ticket_words,
                              void *stream) {
  return guarded(call, [&]() -> int32_t {
    if (call->input_dtype != call->output_dtype)
      return UNISERVE_REFUSE(call, "moe_unpermute needs one input and output dtype");
    if (call->routes == nullptr || call->out == nullptr || call->expanded_to_permuted == nullptr ||
        call->scales == nullptr)
      return UNISERVE_REFUSE(call, "moe_unpermute needs routes, out, expanded_to_permuted and scales");
    if (call->hidden % 8 != 0 || call->hidden <= 0)
      return UNISERVE_REFUSE(call, "moe_unpermute needs a hidden width of whole 8-element groups");
    if (call->tokens < 0 || call->top <= 0 || call->routes_rows < 0)
      return UNISERVE_REFUSE(call, "moe_unpermute needs non-negative tokens and rows and a positive top");
    if (call->layout != UNISERVE_UNPERMUTE_LAYOUT_PERMUTED && call->layout != UNISERVE_UNPERMUTE_LAYOUT_EXPANDED)
      return UNISERVE_REFUSE(call, "moe_unpermute's layout is neither permuted nor expanded");
    if (call->layout == UNISERVE_UNPERMUTE_LAYOUT_EXPANDED && call->routes_rows < call->tokens * call->top)
      return UNISERVE_REFUSE(call, "moe_unpermute's expanded rows cannot hold every route");
    if (call->tokens == 0) return 0;
    if (call->tokens > 0x7fffffffLL)
      return UNISERVE_REFUSE(call, "moe_unpermute's token count exceeds one grid axis");

    CombineParams p{call->routes, call->out, call->expanded_to_permuted, call->scales,
                    call->top,    call->hidden, call->routes_rows,
                    call->layout == UNISERVE_UNPERMUTE_LAYOUT_EXPANDED ? 1 : 0, ticket, ticket_words};
    if (ticket != nullptr && (ticket_words < 1 || ticket_words > kCombineThreads))
      return UNISERVE_REFUSE(call, "moe_unpermute: %d ticket words to check", ticket_words);
    const dim3 grid(static_cast<uint32_t>(call->tokens),
                    static_cast<uint32_t>(ceil_div<int64_t>(call->hidden, kColumnsPerBlock)));
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (call->input_dtype == UNISERVE_DTYPE_BF16) {
      if (call->scales_dtype == UNISERVE_DTYPE_F32)
        hipLaunchKernelGGL((combine_kernel<uint16_t, float>), grid, dim3(kCombineThreads), 0, s, p);
      else if (call->scales_dtype == UNISERVE_DTYPE_BF16)
        hipLaunchKernelGGL((combine_kernel<uint16_t, uint16_t>), grid, dim3(kCombineThreads), 0, s, p);
      else
        return UNISERVE_REFUSE(call, "moe_unpermute serves bf16 routes with f32 or bf16 scales");
    } else if (call->input_dtype == UNISERVE_DTYPE_F16) {
      if (call->scales_dtype == UNISERVE_DTYPE_F32)
        hipLaunchKernelGGL((combine_kernel<_Float16, float>), grid, dim3(kCombineThreads), 0, s, p);
      else if (call->scales_dtype == UNISERVE_DTYPE_F16)
        hipLaunchKernelGGL((combine_kernel<_Float16, _Float16>), grid, dim3(kCombineThreads), 0, s, p);
      else
        return UNISERVE_REFUSE(call, "moe_unpermute serves f16 routes with f32 or f16 scales");
    } else {
      return UNISERVE_REFUSE(call, "moe_unpermute serves bf16 or f16 routes");
    }
    return launched(call, "moe_unpermute");
  });
}

}  // namespace uniserve

extern "C" int32_t uniserve_moe_unpermute(const uniserve_unpermute_call *call, void *stream) {
  return uniserve::moe_unpermute_checked(call, nullptr, 0, stream);
}

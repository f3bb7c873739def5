// SPDX-License-Identifier: Apache-2.0
//
// topk_softmax on gfx950: the router's FP32 softmax, top-k, renormalisation, scale, map and
// expert-load count (operator: crates/ops/src/moe/routing.rs:1-40; reference kernel:
// crates/ops/kernels/topk_softmax/nvcc/src/topk_softmax.cu).
//
// One token per 32-lane half of a 64-lane wavefront (the routine, topk_route.hpp, keeps the
// reference's FP32 reduction tree so ids are exact). Two tokens per wavefront also keep the
// reference's launch arithmetic: a block of `warps * 32` threads routes `warps` tokens, so a caller
// that computes grid = ceil(rows / warps) from the module's metadata launches this kernel unchanged.
#include "common.hpp"
#include "topk_route.hpp"
#include "uniserve_topk_softmax.h"

#include <cfloat>
#include <climits>

/// The operator's kernel, parameters in the order of
/// crates/ops/kernels/topk_softmax/nvcc/package.toml:35-53. A launch outside 1 <= top <= 32,
/// top <= experts <= 1024 writes nothing (the launcher refuses such calls before they start).
extern "C" __global__ void __launch_bounds__(1024)
uniserve_topk_softmax(const void *scores, int score_kind, int64_t row_stride, int rows, int experts,
                      int top, int renormalize, const void *scale, int scale_kind, int32_t *ids,
                      float *weights, const int32_t *map, const int32_t *live,
                      unsigned long long *load) {
  using namespace uniserve;
  if (experts < 1 || experts > UNISERVE_TOPK_MAX_EXPERTS || top < 1 || top > UNISERVE_TOPK_MAX_TOP ||
      top > experts)
    return;
  const int row = static_cast<int>(blockIdx.x) * static_cast<int>(blockDim.x / topk::kHalf) +
                  static_cast<int>(threadIdx.x / topk::kHalf);
  // Both halves of a wavefront stay convergent through the butterflies: a half past the last row
  // routes row 0 again to take part in its wavefront's exchanges, and stores nothing.
  const bool active = row < rows;
  const int routed = active ? row : 0;
  topk::route_token(scores, score_kind, row_stride, routed, experts, top, renormalize, scale, scale_kind, ids, weights,
                    map, live, load, active);
}

#ifndef UNISERVE_DEVICE_ONLY
extern "C" int32_t uniserve_topk_softmax_launch(
    const void *scores, int32_t score_kind, int64_t row_stride, int32_t rows, int32_t experts,
    int32_t top, int32_t renormalize, const void *scale, int32_t scale_kind, int32_t *ids,
    float *weights, const int32_t *map, const uint32_t *live, int64_t *load, void *stream,
    char *error, size_t error_bytes) {
  auto refuse = [&](const char *message) -> int32_t {
    if (error != nullptr && error_bytes > 0) std::snprintf(error, error_bytes, "%s", message);
    return 1;
  };
  // The refusals of `TopkSoftmax::check` (crates/ops/src/moe/routing.rs:127-238) that the words
  // of the signature can state.
  if (score_kind < 0 || score_kind > 2) return refuse("topk_softmax: scores of this kind are not routeable");
  if (experts < 1) return refuse("topk_softmax: a router selects over at least one expert");
  if (experts > UNISERVE_TOPK_MAX_EXPERTS) return refuse("topk_softmax: more than 1024 experts");
  if (top < 1 || top > experts) return refuse("topk_softmax: top is outside 1..=experts");
  if (top > UNISERVE_TOPK_MAX_TOP) return refuse("topk_softmax: more than 32 picks");
  if (rows < 0) return refuse("topk_softmax: a negative row count");
  if (row_stride < experts) return refuse("topk_softmax: rows overlap (row_stride < experts)");
  if (scale_kind < -1 || scale_kind > 2 || (scale_kind != -1 && scale == nullptr))
    return refuse("topk_softmax: a declared scale needs a pointer of a routeable kind");
  if (rows > 0 && (scores == nullptr || ids == nullptr || weights == nullptr))
    return refuse("topk_softmax: needs scores, ids and weights");
  if (rows == 0) return 0;
  constexpr int kTokensPerBlock = UNISERVE_TOPK_WARPS;
  const dim3 grid((rows + kTokensPerBlock - 1) / kTokensPerBlock);
  hipLaunchKernelGGL(uniserve_topk_softmax, grid, dim3(kTokensPerBlock * 32), 0,
                     static_cast<hipStream_t>(stream), scores, score_kind, row_stride, rows, experts,
                     top, renormalize, scale, scale_kind, ids, weights, map,
                     reinterpret_cast<const int32_t *>(live),
                     reinterpret_cast<unsigned long long *>(load));
  const hipError_t status = hipGetLastError();
  if (status != hipSuccess) return refuse(hipGetErrorString(status));
  return 0;
}
#endif

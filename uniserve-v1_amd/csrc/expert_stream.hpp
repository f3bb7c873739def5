// SPDX-License-Identifier: Apache-2.0
//
// The layer's bf16 decode products without a sort (grouped_gemm.hip): each stream workgroup serves
// one local expert and finds that expert's routes in `ids` itself; rows sit at their expanded
// positions (route t * top + k), so the combine reads them in the expanded layout.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "uniserve_moe_mx.h"

namespace uniserve {

struct ExpertStream {
  const void *act;           ///< FC1: hidden [tokens, K]; FC2: gated rows [routes, K]
  const void *weights;       ///< [local experts, n_total, K] bf16
  void *out;                 ///< [routes, out_width] bf16, rows at expanded positions
  const int32_t *ids;        ///< [routes] expert ids after the slot map
  const int32_t *live_tokens;///< [1] or null
  int64_t routes, top, local_offset, local_experts;
  int64_t K, n_total, out_width;
  int32_t activation;        ///< FC1's gate
};

/// Whether the expert-major stream kernels serve these extents (decode batches: at most 4096
/// routes, fewer than 24 per local expert - with fewer routes than local experts a compact grid over
/// at most 512 of them; FC1 widths of whole 64-column slices, FC2 of whole 128-column ones).
bool expert_stream_fits(int64_t routes, int64_t local_experts, int64_t K, int64_t out_width, bool gated);

/// FC1 (`gated`: the gate of `activation` times the up half) or FC2 over the listed routes.
void launch_expert_stream(const ExpertStream &e, bool gated, hipStream_t stream);

/// The routes the expert-major MXFP4 products serve (their calls' tile maps are not read).
struct ExpertRouting {
  const int32_t *ids;
  const int32_t *live_tokens;
  int64_t routes, top, local_offset, local_experts;
};

/// With `codes` (and `code_scales`), FC1 also writes the gated rows as FC2's MXFP8 operand (codes
/// [routes, width / 2], row-major E8M0 bytes [routes, width / 64]) - only where
/// mx_fc1_quantizes_by_expert holds (the unsplit kernel, whose workgroups own whole 32-column
/// blocks).
bool mx_fc1_quantizes_by_expert(const ExpertRouting &r, int64_t width);
void gather_gemm_mx_by_expert(const uniserve_gather_mx_call *call, const ExpertRouting &r, int32_t activation,
                              void *stream, uint8_t *codes = nullptr, uint8_t *code_scales = nullptr);
void route_gemm_mx_by_expert(const uniserve_route_mx_call *call, const ExpertRouting &r, void *stream);

}  // namespace uniserve

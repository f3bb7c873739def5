// SPDX-License-Identifier: Apache-2.0
//
// route_gemm (FC2): for each live permuted row p of expert e,
//   out[p, :] = W[e] . rows[p]      W: [experts, width = hidden, intermediate]
// FP32 accumulation, one rounding to bf16, live rows only stored, unweighted.
//
// Replaces crates/ops/kernels/route_gemm/cute_dsl/src/entry.cpp (`uniserve_route_gemm`), called
// by `RouteGemm::launch` (crates/ops/src/moe/grouped.rs:469-499). The structure is the
// reference's `RouteCall` (grouped.rs:557-577), field for field.

#pragma once

#include "uniserve_abi.h"

struct uniserve_route_call {
  const void *rows;                     ///< [permuted_rows, intermediate] bf16
  const void *weights;                  ///< [experts, width, intermediate] bf16
  void *out;                            ///< [permuted_rows, width] bf16
  const int32_t *tile_to_expert;
  const int32_t *tile_to_limit;
  const int32_t *permuted_to_expanded;
  const int32_t *num_non_exiting_tiles;
  int64_t permuted_rows;
  int64_t width;
  int64_t intermediate;
  int64_t experts;
  int64_t dtype;
  int64_t multiprocessors;
  char error[512];
};

#ifdef __cplusplus
static_assert(sizeof(uniserve_route_call) == 616, "uniserve_route_call layout");
static_assert(offsetof(uniserve_route_call, rows) == 0, "layout");
static_assert(offsetof(uniserve_route_call, weights) == 8, "layout");
static_assert(offsetof(uniserve_route_call, out) == 16, "layout");
static_assert(offsetof(uniserve_route_call, tile_to_expert) == 24, "layout");
static_assert(offsetof(uniserve_route_call, tile_to_limit) == 32, "layout");
static_assert(offsetof(uniserve_route_call, permuted_to_expanded) == 40, "layout");
static_assert(offsetof(uniserve_route_call, num_non_exiting_tiles) == 48, "layout");
static_assert(offsetof(uniserve_route_call, permuted_rows) == 56, "layout");
static_assert(offsetof(uniserve_route_call, width) == 64, "layout");
static_assert(offsetof(uniserve_route_call, intermediate) == 72, "layout");
static_assert(offsetof(uniserve_route_call, experts) == 80, "layout");
static_assert(offsetof(uniserve_route_call, dtype) == 88, "layout");
static_assert(offsetof(uniserve_route_call, multiprocessors) == 96, "layout");
static_assert(offsetof(uniserve_route_call, error) == 104, "layout");
#endif

UNISERVE_EXTERN_C int32_t uniserve_route_gemm(const struct uniserve_route_call *call, void *stream);

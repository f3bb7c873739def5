// SPDX-License-Identifier: Apache-2.0
//
// moe_unpermute: out[t] = sum over k with a visible row of scales[t,k] * routes[row(t,k)],
// accumulated in FP32 in route order and rounded once; a token with no visible route is 0.
//
// Replaces crates/ops/kernels/moe_unpermute/trtllm/src/entry.cpp (`uniserve_moe_unpermute`),
// called by `MoeUnpermute::launch` (crates/ops/src/moe/combine.rs:194-223). The structure is the
// reference's `combine::Call` (combine.rs:116-135) and the layout enum its `Layout`
// (combine.rs:44-50), field for field.

#pragma once

#include "uniserve_abi.h"

enum uniserve_unpermute_layout
#ifdef __cplusplus
    : int32_t
#endif
{
  /// One row per permuted row; `expanded_to_permuted` names the row of each (token, route).
  UNISERVE_UNPERMUTE_LAYOUT_PERMUTED = 0,
  /// One row per expanded route, `token * top + route`; the map only marks absent routes.
  UNISERVE_UNPERMUTE_LAYOUT_EXPANDED = 1,
};

struct uniserve_unpermute_call {
  const void *routes;                   ///< [routes_rows, hidden] input_dtype
  void *out;                            ///< [tokens, hidden] output_dtype
  const int32_t *expanded_to_permuted;  ///< [tokens, top]; negative = absent
  const void *scales;                   ///< [tokens, top] scales_dtype
  int64_t tokens;
  int64_t top;
  int64_t hidden;
  int64_t routes_rows;
  int64_t input_dtype;
  int64_t scales_dtype;
  int64_t output_dtype;
  int64_t layout;
  char error[512];
};

#ifdef __cplusplus
static_assert(sizeof(uniserve_unpermute_call) == 608, "uniserve_unpermute_call layout");
static_assert(offsetof(uniserve_unpermute_call, routes) == 0, "layout");
static_assert(offsetof(uniserve_unpermute_call, out) == 8, "layout");
static_assert(offsetof(uniserve_unpermute_call, expanded_to_permuted) == 16, "layout");
static_assert(offsetof(uniserve_unpermute_call, scales) == 24, "layout");
static_assert(offsetof(uniserve_unpermute_call, tokens) == 32, "layout");
static_assert(offsetof(uniserve_unpermute_call, top) == 40, "layout");
static_assert(offsetof(uniserve_unpermute_call, hidden) == 48, "layout");
static_assert(offsetof(uniserve_unpermute_call, routes_rows) == 56, "layout");
static_assert(offsetof(uniserve_unpermute_call, input_dtype) == 64, "layout");
static_assert(offsetof(uniserve_unpermute_call, scales_dtype) == 72, "layout");
static_assert(offsetof(uniserve_unpermute_call, output_dtype) == 80, "layout");
static_assert(offsetof(uniserve_unpermute_call, layout) == 88, "layout");
static_assert(offsetof(uniserve_unpermute_call, error) == 96, "layout");
#endif

UNISERVE_EXTERN_C int32_t uniserve_moe_unpermute(const struct uniserve_unpermute_call *call, void *stream);

// SPDX-License-Identifier: Apache-2.0
//
// gather_gemm (FC1): for each live permuted row p of token t and expert e,
//   out[p, :] = act(W[e, I:2I] . x[t]) * (W[e, 0:I] . x[t])
// with FP32 accumulation, the activation on the accumulators and one rounding to bf16; act is
// silu (`uniserve_gather_gemm`) or gelu_tanh (`uniserve_gather_gemm_gelu_tanh`).
//
// Replaces crates/ops/kernels/gather_gemm/cute_dsl/src/entry.cpp:57-59 (`uniserve_gather_gemm`),
// called by `GatherGemm::launch` (crates/ops/src/moe/grouped.rs:326-360). The structure is the
// reference's `GatherCall` (grouped.rs:211-232), field for field.

#pragma once

#include "uniserve_abi.h"

struct uniserve_gather_call {
  const void *hidden;                   ///< [tokens, hidden_size] bf16
  const void *weights;                  ///< [experts, width = 2I, hidden_size] bf16, up rows then gate rows
  void *out;                            ///< [permuted_rows, width / 2] bf16
  const int32_t *tile_to_expert;        ///< [max_tiles]
  const int32_t *tile_to_limit;         ///< [max_tiles]
  const int32_t *permuted_to_expanded;  ///< [permuted_rows]
  const int32_t *num_non_exiting_tiles; ///< [1]
  int64_t tokens;
  int64_t permuted_rows;
  int64_t width;
  int64_t hidden_size;
  int64_t experts;
  int64_t top;
  int64_t dtype;
  int64_t multiprocessors;              ///< compute units of the launching device
  char error[512];
};

#ifdef __cplusplus
static_assert(sizeof(uniserve_gather_call) == 632, "uniserve_gather_call layout");
static_assert(offsetof(uniserve_gather_call, hidden) == 0, "layout");
static_assert(offsetof(uniserve_gather_call, weights) == 8, "layout");
static_assert(offsetof(uniserve_gather_call, out) == 16, "layout");
static_assert(offsetof(uniserve_gather_call, tile_to_expert) == 24, "layout");
static_assert(offsetof(uniserve_gather_call, tile_to_limit) == 32, "layout");
static_assert(offsetof(uniserve_gather_call, permuted_to_expanded) == 40, "layout");
static_assert(offsetof(uniserve_gather_call, num_non_exiting_tiles) == 48, "layout");
static_assert(offsetof(uniserve_gather_call, tokens) == 56, "layout");
static_assert(offsetof(uniserve_gather_call, permuted_rows) == 64, "layout");
static_assert(offsetof(uniserve_gather_call, width) == 72, "layout");
static_assert(offsetof(uniserve_gather_call, hidden_size) == 80, "layout");
static_assert(offsetof(uniserve_gather_call, experts) == 88, "layout");
static_assert(offsetof(uniserve_gather_call, top) == 96, "layout");
static_assert(offsetof(uniserve_gather_call, dtype) == 104, "layout");
static_assert(offsetof(uniserve_gather_call, multiprocessors) == 112, "layout");
static_assert(offsetof(uniserve_gather_call, error) == 120, "layout");
#endif

UNISERVE_EXTERN_C int32_t uniserve_gather_gemm(const struct uniserve_gather_call *call, void *stream);

/// The same call with a gelu_tanh gate: the reference compiles the gate into each FC1 module
/// (`GatherGemmDescriptor::activation`, crates/ops/src/moe/grouped.rs:65-127, descriptors
/// `activation = ["silu", "gelu_tanh"]` in gather_gemm/cute_dsl/package.toml), so a module built
/// for `gelu_tanh` exports this entry under the plain name; here both live in one library.
UNISERVE_EXTERN_C int32_t uniserve_gather_gemm_gelu_tanh(const struct uniserve_gather_call *call, void *stream);

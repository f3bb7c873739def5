// SPDX-License-Identifier: Apache-2.0
//
// moe_sort: groups `tokens x top` route ids by local expert into tiles of `tile_tokens`
// permuted rows and writes the tile tables and the permutation maps.
//
// Replaces the native entry of crates/ops/kernels/moe_sort/trtllm (src/entry.cpp:80-91), called
// by `MoeSort::launch` (crates/ops/src/moe/sort.rs:291-328). The structure is the reference's
// `ops::moe::sort::Call` (sort.rs:173-214), field for field; the assertions below are the
// layout the Rust side lays out.

#pragma once

#include "uniserve_abi.h"

struct uniserve_moe_sort_call {
  const int32_t *ids;              ///< [tokens, top] route ids over the whole vocabulary
  const void *scales;              ///< [tokens, top] route weights; accepted, never read
  int32_t *tile_to_expert;         ///< [max_tiles] local expert of each tile
  int32_t *tile_to_limit;          ///< [max_tiles] exclusive end row of a tile's live rows
  int32_t *expanded_to_permuted;   ///< [tokens, top] permuted row; -1 not held, -2 not live
  int32_t *permuted_to_expanded;   ///< [max_permuted_rows] route of each row; -1 on padding
  int32_t *total_padded_tokens;    ///< [1] rows of the tiles that hold routes
  int32_t *num_non_exiting_tiles;  ///< [1] tiles that hold routes
  int64_t tokens;
  int64_t top;
  int64_t experts;
  int64_t local_experts;
  int64_t local_offset;
  int64_t tile_tokens;
  int64_t scales_dtype;
  char error[512];                 ///< NUL-terminated message on a nonzero return
  const int32_t *live_tokens;      ///< [1] live token rows, or null: every row is live
  int32_t *permuted_to_token;      ///< [max_permuted_rows] token row of each row; -1 on padding
};

#ifdef __cplusplus
static_assert(sizeof(uniserve_moe_sort_call) == 648, "uniserve_moe_sort_call layout");
static_assert(offsetof(uniserve_moe_sort_call, ids) == 0, "layout");
static_assert(offsetof(uniserve_moe_sort_call, scales) == 8, "layout");
static_assert(offsetof(uniserve_moe_sort_call, tile_to_expert) == 16, "layout");
static_assert(offsetof(uniserve_moe_sort_call, tile_to_limit) == 24, "layout");
static_assert(offsetof(uniserve_moe_sort_call, expanded_to_permuted) == 32, "layout");
static_assert(offsetof(uniserve_moe_sort_call, permuted_to_expanded) == 40, "layout");
static_assert(offsetof(uniserve_moe_sort_call, total_padded_tokens) == 48, "layout");
static_assert(offsetof(uniserve_moe_sort_call, num_non_exiting_tiles) == 56, "layout");
static_assert(offsetof(uniserve_moe_sort_call, tokens) == 64, "layout");
static_assert(offsetof(uniserve_moe_sort_call, top) == 72, "layout");
static_assert(offsetof(uniserve_moe_sort_call, experts) == 80, "layout");
static_assert(offsetof(uniserve_moe_sort_call, local_experts) == 88, "layout");
static_assert(offsetof(uniserve_moe_sort_call, local_offset) == 96, "layout");
static_assert(offsetof(uniserve_moe_sort_call, tile_tokens) == 104, "layout");
static_assert(offsetof(uniserve_moe_sort_call, scales_dtype) == 112, "layout");
static_assert(offsetof(uniserve_moe_sort_call, error) == 120, "layout");
static_assert(offsetof(uniserve_moe_sort_call, live_tokens) == 632, "layout");
static_assert(offsetof(uniserve_moe_sort_call, permuted_to_token) == 640, "layout");
#endif

/// Returns 0 after launching on `stream` (a hipStream_t); nonzero with `call->error` set on a
/// refusal. Never allocates, synchronizes or reads device memory on the host.
UNISERVE_EXTERN_C int32_t uniserve_moe_sort(const struct uniserve_moe_sort_call *call, void *stream);

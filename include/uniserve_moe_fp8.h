// SPDX-License-Identifier: Apache-2.0
//
// Block-scaled FP8 (OCP e4m3fn) forms of the two grouped expert products and the activation
// quantiser they read.
//
// The reference has no block-scaled FP8 MoE operator: `crates/nn/src/quantization.rs:241-249`
// refuses checkpoints with 128x128 `weight_scale_inv` blocks, and its FP8 is per-tensor
// (`crates/ops/src/fp8.rs:1-39`, E4M3_MAX = 448). These entries follow the reference's pattern of
// a separate operator per weight representation (the NVFP4 calls, crates/ops/src/moe/grouped.rs:
// 816-869): the dense calls' fields plus the scale tables.
//
// Encoding: value = e4m3(code) * scale. Weights carry one FP32 scale per 128 x 128 block
// (`scale = blockmax / 448`); activations one FP32 scale per row per 128 contiguous channels.

#pragma once

#include "uniserve_abi.h"

/// Rows quantised per 128 contiguous channels: out[r, c] = e4m3(in[r, c] / s[r, c / 128]),
/// s = max(|in[r, group]|) / 448 (1 for an all-zero group), round to nearest even, saturating.
/// Rows at or past `*row_limit` (when given) are left untouched.
struct uniserve_quantize_fp8_call {
  const void *input;          ///< [rows, width] input_dtype (bf16 or f32)
  void *out;                  ///< [rows, width] e4m3
  float *scales;              ///< [rows, width / 128]
  const int32_t *row_limit;   ///< [1] rows to quantise (e.g. a sort's total_padded_tokens), or null
  int64_t rows;
  int64_t width;
  int64_t input_dtype;
  int64_t group;              ///< 128
  char error[512];
};

/// FC1 over e4m3 operands: out[p] = act(gate) * up (act: silu, or gelu_tanh for the `_gelu_tanh`
/// entry) with
///   up = sum_kb (sum_{k in kb} q_x[t,k] q_w[e,n,k]) * s_x[t,kb] * s_w[e,n/128,kb]
/// accumulated in FP32, one rounding into bf16.
struct uniserve_gather_fp8_call {
  const void *hidden;                   ///< [tokens, hidden_size] e4m3
  const float *hidden_scales;           ///< [tokens, hidden_size / 128]
  const void *weights;                  ///< [experts, width = 2I, hidden_size] e4m3, up then gate
  const float *weight_scales;           ///< [experts, width / 128, hidden_size / 128]
  void *out;                            ///< [permuted_rows, width / 2] bf16
  const int32_t *tile_to_expert;
  const int32_t *tile_to_limit;
  const int32_t *permuted_to_expanded;
  const int32_t *num_non_exiting_tiles;
  int64_t tokens;
  int64_t permuted_rows;
  int64_t width;
  int64_t hidden_size;
  int64_t experts;
  int64_t top;
  int64_t block_n;                      ///< 128
  int64_t block_k;                      ///< 128
  int64_t out_dtype;                    ///< bf16
  int64_t multiprocessors;
  char error[512];
};

/// FC2 over e4m3 operands: out[p] = W[e] . rows[p] with the same block-scale rule, bf16 out,
/// live rows only stored.
struct uniserve_route_fp8_call {
  const void *rows;                     ///< [permuted_rows, intermediate] e4m3
  const float *row_scales;              ///< [permuted_rows, intermediate / 128]
  const void *weights;                  ///< [experts, width = hidden, intermediate] e4m3
  const float *weight_scales;           ///< [experts, width / 128, intermediate / 128]
  void *out;                            ///< [permuted_rows, width] bf16
  const int32_t *tile_to_expert;
  const int32_t *tile_to_limit;
  const int32_t *permuted_to_expanded;
  const int32_t *num_non_exiting_tiles;
  int64_t permuted_rows;
  int64_t width;
  int64_t intermediate;
  int64_t experts;
  int64_t block_n;
  int64_t block_k;
  int64_t out_dtype;
  int64_t multiprocessors;
  char error[512];
};

UNISERVE_EXTERN_C int32_t uniserve_quantize_fp8(const struct uniserve_quantize_fp8_call *call, void *stream);
UNISERVE_EXTERN_C int32_t uniserve_gather_gemm_fp8(const struct uniserve_gather_fp8_call *call, void *stream);
UNISERVE_EXTERN_C int32_t uniserve_gather_gemm_fp8_gelu_tanh(const struct uniserve_gather_fp8_call *call, void *stream);
UNISERVE_EXTERN_C int32_t uniserve_route_gemm_fp8(const struct uniserve_route_fp8_call *call, void *stream);

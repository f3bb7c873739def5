// SPDX-License-Identifier: Apache-2.0
//
// OCP microscaling (MX) forms of the two grouped expert products: MXFP4 expert weights times
// MXFP8 activations, and the activation quantiser they read.
//
// The reference's four-bit experts are NVFP4 (`gather_gemm_nvfp4` / `route_gemm_nvfp4`,
// crates/ops/src/moe/grouped.rs:579-1772, with the `nvfp4_quantize` encoder): E2M1 values with
// an E4M3 scale per 16 elements and an FP32 tensor scale. gfx950's matrix cores multiply E2M1 and
// E4M3 operands with a hardware scale per 32 elements in E8M0 (a power of two), which is the OCP
// MX form; these entries are that form, a separate operator per weight representation as the
// reference keeps one (the same call fields plus the scale tables). NVFP4 checkpoints are not read
// by them (their block scales are not powers of two).
//
// Encoding (OCP MX v1.0): a block of 32 consecutive elements along the contraction shares one
// E8M0 scale byte `x` (the power 2^(x - 127); 0xFF is NaN); element i is code_i * 2^(x - 127).
//  * MXFP4 weights: codes E2M1 (1 sign, 2 exponent, 1 mantissa bits: 0, 0.5, 1, 1.5, 2, 3, 4, 6),
//    two per byte along K, the lower K index in the low nibble.
//  * MXFP8 activations: codes OCP e4m3fn bytes.
// The scale of a block is the smallest power of two under which no element saturates:
// 2^ceil(log2(amax / M)), M = 6 (E2M1) or 448 (e4m3); an all-zero block takes 2^0. Codes round
// to nearest, ties to even.

#pragma once

#include "uniserve_abi.h"

/// Layouts of an MXFP4 stack's E8M0 scale table ([stacks, rows, K / 32] bytes either way).
///  * ROW_MAJOR: scale of (stack s, row n, block b) at (s * rows + n) * K/32 + b - the OCP /
///    checkpoint layout.
///  * STAGE_MAJOR: the four blocks of one 128-element stage of a row are one 4-byte word, and a
///    stage's words of all rows are contiguous: (s, n, b) at ((s * K/128 + b / 4) * rows + n) * 4
///    + b % 4. The prefill kernel then fetches a stage's scales of 256 weight rows as one 1 KB run
///    instead of one cache line per row (uniserve_mx_stage_major_scales converts, once, at load).
enum uniserve_mx_scale_layout {
  UNISERVE_MX_SCALES_ROW_MAJOR = 0,
  UNISERVE_MX_SCALES_STAGE_MAJOR = 1,
};

/// Rows quantised per 32 contiguous channels to MXFP8: out[r, c] = e4m3(in[r, c] / 2^(s - 127)),
/// s = scales[r, c / 32]. Rows at or past `*row_limit` (when given) are left untouched.
struct uniserve_quantize_mxfp8_call {
  const void *input;          ///< [rows, width] input_dtype (bf16 or f32)
  void *out;                  ///< [rows, width] e4m3
  uint8_t *scales;            ///< [rows, width / 32] E8M0
  const int32_t *row_limit;   ///< [1] rows to quantise, or null
  int64_t rows;
  int64_t width;              ///< a multiple of 128
  int64_t input_dtype;
  char error[512];
};

/// FC1 over MX operands: out[p] = act(gate) * up (act: silu, or gelu_tanh for the `_gelu_tanh`
/// entry) with
///   up = sum_k e4m3(q_x[t,k]) 2^(s_x[t,k/32]-127) * e2m1(q_w[e,n,k]) 2^(s_w[e,n,k/32]-127)
/// accumulated in FP32, one rounding into bf16.
struct uniserve_gather_mx_call {
  const void *hidden;                   ///< [tokens, hidden_size] e4m3
  const uint8_t *hidden_scales;         ///< [tokens, hidden_size / 32] E8M0
  const void *weights;                  ///< [experts, width = 2I, hidden_size / 2] E2M1 pairs, up then gate
  const uint8_t *weight_scales;         ///< [experts, width, hidden_size / 32] E8M0
  void *out;                            ///< [permuted_rows, width / 2] bf16
  const int32_t *tile_to_expert;
  const int32_t *tile_to_limit;
  const int32_t *permuted_to_expanded;
  const int32_t *num_non_exiting_tiles;
  int64_t tokens;
  int64_t permuted_rows;
  int64_t width;
  int64_t hidden_size;                  ///< a multiple of 256
  int64_t experts;
  int64_t top;
  int64_t out_dtype;                    ///< bf16
  int64_t multiprocessors;
  int64_t weight_scale_layout;          ///< uniserve_mx_scale_layout of weight_scales
  char error[512];
};

/// FC2 over MX operands: out[p] = W[e] . rows[p] with the same rule, bf16 out, live rows only.
struct uniserve_route_mx_call {
  const void *rows;                     ///< [permuted_rows, intermediate] e4m3
  const uint8_t *row_scales;            ///< [permuted_rows, intermediate / 32] E8M0
  const void *weights;                  ///< [experts, width = hidden, intermediate / 2] E2M1 pairs
  const uint8_t *weight_scales;         ///< [experts, width, intermediate / 32] E8M0
  void *out;                            ///< [permuted_rows, width] bf16
  const int32_t *tile_to_expert;
  const int32_t *tile_to_limit;
  const int32_t *permuted_to_expanded;
  const int32_t *num_non_exiting_tiles;
  int64_t permuted_rows;
  int64_t width;
  int64_t intermediate;                 ///< a multiple of 256
  int64_t experts;
  int64_t out_dtype;
  int64_t multiprocessors;
  int64_t weight_scale_layout;          ///< uniserve_mx_scale_layout of weight_scales
  char error[512];
};

/// Converts a ROW_MAJOR scale table to STAGE_MAJOR (see uniserve_mx_scale_layout).
struct uniserve_mx_stage_scales_call {
  const uint8_t *in;                    ///< [stacks, rows, width / 32] E8M0, row-major
  uint8_t *out;                         ///< the same bytes, stage-major
  int64_t stacks;
  int64_t rows;
  int64_t width;                        ///< K, a multiple of 128
  char error[512];
};

UNISERVE_EXTERN_C int32_t uniserve_quantize_mxfp8(const struct uniserve_quantize_mxfp8_call *call, void *stream);
UNISERVE_EXTERN_C int32_t uniserve_gather_gemm_mx(const struct uniserve_gather_mx_call *call, void *stream);
UNISERVE_EXTERN_C int32_t uniserve_gather_gemm_mx_gelu_tanh(const struct uniserve_gather_mx_call *call, void *stream);
UNISERVE_EXTERN_C int32_t uniserve_route_gemm_mx(const struct uniserve_route_mx_call *call, void *stream);
UNISERVE_EXTERN_C int32_t uniserve_mx_stage_major_scales(const struct uniserve_mx_stage_scales_call *call, void *stream);

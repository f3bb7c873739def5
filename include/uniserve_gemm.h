// SPDX-License-Identifier: Apache-2.0
//
// The router's score GEMM, scores[m, n] = alpha * input[m, k] . weight[n, k]^T, FP32 accumulation
// and one rounding into bf16: the `gemm` operator module the MoE block's router `Linear` launches
// (crates/nn/src/modules/moe.rs:656-671 -> crates/ops/kernels/gemm/cublas_lt/src/*.cpp:338,
// `uniserve_gemm`), in the one specialisation the router uses: bf16 input, weight and output, the
// weight stored [n, k] (Hugging Face order, `UNISERVE_WEIGHT_ORDER_NXK`) and no bias. The
// structure is the reference's `UniserveGemmCall`, field for field.

#pragma once

#include "uniserve_abi.h"

enum uniserve_weight_order
#ifdef __cplusplus
    : int32_t
#endif
{
  UNISERVE_WEIGHT_ORDER_KXN = 0,
  UNISERVE_WEIGHT_ORDER_NXK = 1,
};

enum uniserve_epilogue
#ifdef __cplusplus
    : int32_t
#endif
{
  UNISERVE_EPILOGUE_NONE = 0,
  UNISERVE_EPILOGUE_BIAS = 1,
};

typedef struct UniserveGemmCall {
  void *out;                  ///< [m, n] row-major bf16
  const void *input;          ///< [m, k] row-major bf16
  const void *weight;         ///< [n, k] bf16 (nxk)
  const void *bias;           ///< must be null: this module has no bias epilogue
  int64_t m;
  int64_t n;
  int64_t k;
  int64_t input_row_stride;
  int64_t weight_row_stride;
  int64_t out_row_stride;
  float alpha;
  char error[512];
} UniserveGemmCall;

#ifdef __cplusplus
static_assert(sizeof(UniserveGemmCall) == 600, "UniserveGemmCall layout");
static_assert(offsetof(UniserveGemmCall, out) == 0, "layout");
static_assert(offsetof(UniserveGemmCall, input) == 8, "layout");
static_assert(offsetof(UniserveGemmCall, weight) == 16, "layout");
static_assert(offsetof(UniserveGemmCall, bias) == 24, "layout");
static_assert(offsetof(UniserveGemmCall, m) == 32, "layout");
static_assert(offsetof(UniserveGemmCall, n) == 40, "layout");
static_assert(offsetof(UniserveGemmCall, k) == 48, "layout");
static_assert(offsetof(UniserveGemmCall, input_row_stride) == 56, "layout");
static_assert(offsetof(UniserveGemmCall, weight_row_stride) == 64, "layout");
static_assert(offsetof(UniserveGemmCall, out_row_stride) == 72, "layout");
static_assert(offsetof(UniserveGemmCall, alpha) == 80, "layout");
static_assert(offsetof(UniserveGemmCall, error) == 84, "layout");
#endif

UNISERVE_EXTERN_C int32_t uniserve_gemm(UniserveGemmCall *call, void *stream);

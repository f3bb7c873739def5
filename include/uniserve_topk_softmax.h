// SPDX-License-Identifier: Apache-2.0
//
// topk_softmax: the router's FP32 softmax over each token's expert scores, the `top` largest
// probabilities (descending, equal ones in ascending expert id), renormalisation by their sum
// clamped below by FLT_EPSILON, an optional per-expert scale, an optional logical-to-physical
// map and an optional 64-bit expert-load count of live rows.
//
// The reference's operator is a kernel-signature ABI, not a call structure: `TopkSoftmax::launch`
// (crates/ops/src/moe/routing.rs:240-301) loads a module and launches its kernel
// `uniserve_topk_softmax` with the 14 words of crates/ops/kernels/topk_softmax/nvcc/package.toml:35-53
// on a grid of ceil(rows / warps) blocks of warps * 32 threads. This library provides:
//
//  * the device kernel `uniserve_topk_softmax` with that parameter list, in the code object
//    `uniserve_topk_softmax.hsaco` (hipModuleLoad / hipModuleLaunchKernel, the counterpart of the
//    cubin path, kernel.rs `Kernel::launch`): a block of `warps * 32` threads routes `warps`
//    tokens, one 32-lane half of a 64-lane wavefront per token, so the reference's grid
//    arithmetic holds unchanged;
//  * the host launcher below, the same 14 words plus the stream, for callers that link the
//    library instead of loading the code object.
//
// Score and scale kinds (routing.rs:124-131): 0 = f32, 1 = bf16, 2 = f16, -1 = absent.

#pragma once

#include "uniserve_abi.h"

/// Tokens routed by one block of the launcher (and the code object's `num_warps` metadata).
#define UNISERVE_TOPK_WARPS 8
/// Largest expert count and top-k width the kernel serves (package.toml:55-64 bounds).
#define UNISERVE_TOPK_MAX_EXPERTS 1024
#define UNISERVE_TOPK_MAX_TOP 32

/// Launches the router on `stream`. Returns 0, or nonzero with a message copied into `error`
/// (`error_bytes` long, may be null) when the arguments are outside what the kernel serves.
UNISERVE_EXTERN_C int32_t uniserve_topk_softmax_launch(
    const void *scores, int32_t score_kind, int64_t row_stride, int32_t rows, int32_t experts,
    int32_t top, int32_t renormalize, const void *scale, int32_t scale_kind, int32_t *ids,
    float *weights, const int32_t *map, const uint32_t *live, int64_t *load, void *stream,
    char *error, size_t error_bytes);

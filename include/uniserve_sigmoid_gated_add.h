// SPDX-License-Identifier: Apache-2.0
//
// sigmoid_gated_add: a shared expert's join, in place -
//
//   target[r, c] <- target[r, c] + sigmoid(gate[r]) * update[r, c]
//
// with the sigmoid, the product and the sum in FP32 and one rounding into the target's type
// (crates/ops/src/residual.rs:797-898, operator `SigmoidGatedAdd`; the functional form
// `sigmoid_gated_add_`, crates/nn/src/functional/moe.rs:1527-1610). Target, update and gate share one
// element type (bf16, f16 or f32); target and update are contiguous [rows, columns], gate is
// [rows, 1].
//
// Like topk_softmax, the reference's operator is a kernel-signature ABI: its Triton package
// (crates/ops/kernels/sigmoid_gated_add/triton/package.toml) launches `_sigmoid_gated_add_kernel`
// with the words (target, update, gate, columns i32) on a grid of (ceil(columns / block), rows).
// This library provides the device kernels `uniserve_sigmoid_gated_add_{bf16,f16,f32}` with those
// four words, one program per (block of UNISERVE_SIGMOID_GATED_ADD_BLOCK columns, row) - in
// uniserve_topk_softmax.hsaco's sibling code object uniserve_residual.hsaco - and the host launcher
// below.

#pragma once

#include "uniserve_abi.h"

/// Columns one program (one 256-thread workgroup) of the device kernels walks.
#define UNISERVE_SIGMOID_GATED_ADD_BLOCK 2048

/// Launches the join on `stream`; dtype is UNISERVE_DTYPE_BF16, _F16 or _F32. Returns 0, or
/// nonzero with a message in `error` (`error_bytes` long, may be null) for arguments the
/// operator refuses (residual.rs:820-853): zero columns, more than 2^31 - 1 elements, a null
/// pointer for a non-empty call, another element type.
UNISERVE_EXTERN_C int32_t uniserve_sigmoid_gated_add_launch(void *target, const void *update, const void *gate,
                                                            int64_t rows, int64_t columns, int32_t dtype,
                                                            void *stream, char *error, size_t error_bytes);

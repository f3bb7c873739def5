// SPDX-License-Identifier: Apache-2.0
//
// Shared pieces of every MoE operator's C ABI: the element-type numbers the call
// structures carry and the size of their error buffer.
//
// Mirrors crates/ops/src/abi.rs:58-92 (MESSAGE = 512, `ElementType` numbering) and the
// generated crates/ops/python/src/uniserve_kernels/include/uniserve_abi.h, so a Rust caller's
// `#[repr(C)]` structures are read here byte for byte.

#pragma once

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
#define UNISERVE_CONST constexpr static const
#else
#define UNISERVE_CONST static const
#endif

/// Bytes of a call structure's `error` field, the terminating NUL included.
UNISERVE_CONST size_t UNISERVE_MESSAGE = 512;

/// Element-type numbers as the call structures carry them (crates/ops/src/abi.rs:79-92).
enum uniserve_dtype
#ifdef __cplusplus
    : int32_t
#endif
{
  UNISERVE_DTYPE_U8 = 0,
  UNISERVE_DTYPE_I32 = 1,
  UNISERVE_DTYPE_I64 = 2,
  UNISERVE_DTYPE_F16 = 3,
  UNISERVE_DTYPE_BF16 = 4,
  UNISERVE_DTYPE_F32 = 5,
  UNISERVE_DTYPE_F8E4M3 = 6,
  UNISERVE_DTYPE_F4E2M1 = 7,
  UNISERVE_DTYPE_I16 = 8,
  UNISERVE_DTYPE_U32 = 9,
  UNISERVE_DTYPE_F64 = 10,
};

/// FC1's gate, the two a grouped expert product compiles (crates/ops/src/moe/grouped.rs:53-61):
/// silu, and PyTorch's tanh approximation of GELU (crates/nn/src/functional/activation.rs:62-71).
/// The reference compiles the gate into each FC1 module; here the FC1 entries come in one name
/// per gate (`..._gelu_tanh` for the second), and the layer call carries it as a field.
enum uniserve_activation
#ifdef __cplusplus
    : int32_t
#endif
{
  UNISERVE_ACTIVATION_SILU = 0,
  UNISERVE_ACTIVATION_GELU_TANH = 1,
};

#ifdef __cplusplus
#define UNISERVE_EXTERN_C extern "C"
#else
#define UNISERVE_EXTERN_C
#endif

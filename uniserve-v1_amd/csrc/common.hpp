// SPDX-License-Identifier: Apache-2.0
//
// Pieces every kernel file of the MI355X (gfx950) MoE library shares: element conversions, the
// MFMA operand types, wave64 helpers and the refusal convention of the C entries.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <exception>
#include <type_traits>

#include "uniserve_abi.h"

namespace uniserve {

constexpr int kWave = 64;

// ---- refusals ------------------------------------------------------------------------------------

/// Writes a NUL-terminated message into `error` (512 bytes) and answers 1: the entries' way of
/// refusing a call (crates/ops/src/abi.rs:58-70, crates/ops/src/kernel.rs:17-29).
inline int32_t refuse_into(char *error, const char *format, ...) {
  if (error != nullptr) {
    va_list args;
    va_start(args, format);
    std::vsnprintf(error, 512, format, args);
    va_end(args);
  }
  return 1;
}

#define UNISERVE_REFUSE(call, ...) ::uniserve::refuse_into(const_cast<char *>((call)->error), __VA_ARGS__)

/// Runs `body` (which answers an int32 status) and turns any exception into a refusal, so nothing
/// unwinds across the C boundary (the reference's entries do the same:
/// crates/ops/kernels/moe_sort/trtllm/src/entry.cpp:73-91).
template <class Call, class Body>
int32_t guarded(const Call *call, Body body) {
  if (call == nullptr) return 1;
  try {
    return body();
  } catch (std::exception const &thrown) {
    return UNISERVE_REFUSE(call, "%s", thrown.what());
  } catch (...) {
    return UNISERVE_REFUSE(call, "the launch failed without stating why");
  }
}

/// The status of the launch just issued: 0, or a refusal naming the runtime's error.
template <class Call>
int32_t launched(const Call *call, const char *what) {
  const hipError_t status = hipGetLastError();
  if (status == hipSuccess) return 0;
  return UNISERVE_REFUSE(call, "%s could not start: %s", what, hipGetErrorString(status));
}

/// The prefill kernels address gathered activation rows (FC1's token rows) as 32-bit byte offsets
/// from the array's base (the scalar-base form of global_load_lds): an array of `rows` rows of
/// `row_bytes` bytes is served when it lies below 4 GiB. (FC2's rows are addressed from their
/// tile's first row and have no such limit.)
constexpr int64_t kDmaArrayBytes = int64_t{1} << 32;
inline bool dma_rows_fit(int64_t rows, int64_t row_bytes) {
  return rows >= 0 && row_bytes >= 0 && (row_bytes == 0 || rows <= kDmaArrayBytes / row_bytes);
}

// ---- element conversions ---------------------------------------------------------------------------

__device__ __forceinline__ float bf16_to_f32(uint16_t bits) {
  return __uint_as_float(static_cast<uint32_t>(bits) << 16);
}

/// Round to nearest even into bf16 (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16(float value) {
  uint32_t bits = __float_as_uint(value);
  if ((bits & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((bits >> 16) | 0x40u);
  bits += 0x7fffu + ((bits >> 16) & 1u);
  return static_cast<uint16_t>(bits >> 16);
}

/// Two values rounded as f32_to_bf16 does, packed low to high, by gfx950's v_cvt_pk_bf16_f32
/// (identical to f32_to_bf16 on every float, NaNs included - checked exhaustively on the device).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef float floatx2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((floatx2{lo, hi}), bf16x2));
}

/// silu(g) = g / (1 + e^-g), with the hardware exponential (v_exp_f32 on g * -log2 e).
__device__ __forceinline__ float silu(float g) {
  return g / (1.0f + __builtin_amdgcn_exp2f(-g * 1.4426950408889634f));
}

/// FC1's gate. gelu_tanh(g) = 0.5 g (1 + tanh(u)), u = sqrt(2/pi) (g + 0.044715 g^3), written as
/// g / (1 + e^(-2u)) (the identity 1 + tanh(u) = 2 / (1 + e^(-2u))), which does not cancel for
/// large negative g; silu(g) = g / (1 + e^-g). The quotient is taken with the hardware reciprocal
/// (one ulp; the products round the gated values into bf16 next). The choice is uniform over a
/// launch.
template <int kActivation>
__device__ __forceinline__ float gate_of(float g) {
  const float z = kActivation == UNISERVE_ACTIVATION_GELU_TANH ? 1.5957691216057308f * (g + 0.044715f * g * g * g) : g;
  return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-z * 1.4426950408889634f));
}
/// The same with the activation chosen at run time.
__device__ __forceinline__ float gate(float g, int32_t activation) {
  const float z = activation == UNISERVE_ACTIVATION_GELU_TANH ? 1.5957691216057308f * (g + 0.044715f * g * g * g) : g;
  return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-z * 1.4426950408889634f));
}

/// Device-scope loads and stores (relaxed agent-scope atomics: they reach the GPU's coherence point,
/// past the per-XCD L2 slices, with no cache write-back or invalidation) - for values one
/// workgroup hands another inside one launch.
template <class T>
__device__ __forceinline__ T load_device(const T *pointer) {
  return __hip_atomic_load(pointer, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ __forceinline__ void store_device(T *pointer, T value) {
  __hip_atomic_store(pointer, value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- MFMA operands ------------------------------------------------------------------------------------

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef int intx8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

/// D = A . B + C over a 16 x 16 x 32 bf16 block: lane l supplies A row l % 16 and B column
/// l % 16, eight K elements each; D row 4 (l / 16) + i, column l % 16 lands in element i.
__device__ __forceinline__ floatx4 mfma_16x16x32_bf16(u32x4 a, u32x4 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

/// The same block shape over 128 K elements of OCP e4m3 (32 per lane), unscaled.
__device__ __forceinline__ floatx4 mfma_16x16x128_fp8(intx8 a, intx8 b, floatx4 c) {
  // cbsz/blgp 0 = e4m3 for both operands; scale exponents 127 = 2^0.
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

// ---- wave64 helpers --------------------------------------------------------------------------------------

/// The maximum over each 16-lane row of the wavefront, in every lane of the row, by DPP moves:
/// quad_perm [1,0,3,2] and [2,3,0,1] (the quad), row_half_mirror (the other quad of the
/// eight), row_mirror (the other eight); NaNs drop out as in fmaxf.
__device__ __forceinline__ float row16_max(float x) {
  x = __builtin_fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xb1, 0xf, 0xf, false)));
  x = __builtin_fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4e, 0xf, 0xf, false)));
  x = __builtin_fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xf, 0xf, false)));
  x = __builtin_fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xf, 0xf, false)));
  return x;
}

__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x & (kWave - 1)); }

__device__ __forceinline__ uint64_t ballot(bool predicate) { return __ballot(predicate); }

/// The lanes of the wave whose `key` equals this lane's, for keys below 2^bits.
__device__ __forceinline__ uint64_t match_any(uint32_t key, int bits) {
  uint64_t peers = ~0ull;
  for (int bit = 0; bit < bits; ++bit) {
    const bool set = (key >> bit) & 1u;
    const uint64_t mask = ballot(set);
    peers &= set ? mask : ~mask;
  }
  return peers;
}

template <class T>
__host__ __device__ constexpr T ceil_div(T a, T b) {
  return (a + b - 1) / b;
}

}  // namespace uniserve

// SPDX-License-Identifier: Apache-2.0
//
// sigmoid_gated_add on gfx950: target[r] += sigmoid(gate[r]) * update[r], FP32 arithmetic, one
// rounding (operator: crates/ops/src/residual.rs:797-898; reference kernel:
// crates/ops/kernels/sigmoid_gated_add/triton/src/sigmoid_gated_add.py). HBM-bound: two reads and
// one write per element. A 256-thread program owns 2048 columns of one row; a lane moves 8
// consecutive elements with one 16-byte access (32 bytes for f32) when the row allows, else
// element by element.
#include "common.hpp"
#include "uniserve_sigmoid_gated_add.h"

namespace uniserve {
namespace {

constexpr int kThreads = 256;
constexpr int kPerLane = UNISERVE_SIGMOID_GATED_ADD_BLOCK / kThreads;  // 8

template <class T>
__device__ __forceinline__ float widen(T v);
template <>
__device__ __forceinline__ float widen<uint16_t>(uint16_t v) { return bf16_to_f32(v); }
template <>
__device__ __forceinline__ float widen<_Float16>(_Float16 v) { return static_cast<float>(v); }
template <>
__device__ __forceinline__ float widen<float>(float v) { return v; }

template <class T>
__device__ __forceinline__ T narrow(float v);
template <>
__device__ __forceinline__ uint16_t narrow<uint16_t>(float v) { return f32_to_bf16(v); }
template <>
__device__ __forceinline__ _Float16 narrow<_Float16>(float v) { return static_cast<_Float16>(v); }
template <>
__device__ __forceinline__ float narrow<float>(float v) { return v; }

/// 1 / (1 + e^-x) in FP32 (the device library's exponential, within an ulp or two).
__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

template <class T>
__device__ __forceinline__ void join(T *target, const T *update, const T *gate, int32_t columns) {
  const int64_t row = blockIdx.y;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * UNISERVE_SIGMOID_GATED_ADD_BLOCK + threadIdx.x * kPerLane;
  if (first >= columns) return;
  const float g = sigmoid(widen<T>(gate[row]));
  T *t = target + row * columns + first;
  const T *u = update + row * columns + first;
  typedef uint32_t words __attribute__((ext_vector_type(kPerLane * sizeof(T) / 4)));
  const bool whole = first + kPerLane <= columns && columns % kPerLane == 0 &&
                     (reinterpret_cast<uintptr_t>(target) | reinterpret_cast<uintptr_t>(update)) % 16 == 0;
  if (whole) {
    const words tv = *reinterpret_cast<const words *>(t);
    const words uv = *reinterpret_cast<const words *>(u);
    const T *te = reinterpret_cast<const T *>(&tv);
    const T *ue = reinterpret_cast<const T *>(&uv);
    T out[kPerLane];
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) out[j] = narrow<T>(widen<T>(te[j]) + g * widen<T>(ue[j]));
    *reinterpret_cast<words *>(t) = *reinterpret_cast<const words *>(out);
  } else {
    const int64_t count = columns - first < kPerLane ? columns - first : kPerLane;
    for (int64_t j = 0; j < count; ++j) t[j] = narrow<T>(widen<T>(t[j]) + g * widen<T>(u[j]));
  }
}

}  // namespace
}  // namespace uniserve

// The device kernels, the reference's four launch words each (package.toml [launch.types]).
extern "C" __global__ void __launch_bounds__(256)
uniserve_sigmoid_gated_add_bf16(void *target, const void *update, const void *gate, int32_t columns) {
  uniserve::join(static_cast<uint16_t *>(target), static_cast<const uint16_t *>(update),
                 static_cast<const uint16_t *>(gate), columns);
}
extern "C" __global__ void __launch_bounds__(256)
uniserve_sigmoid_gated_add_f16(void *target, const void *update, const void *gate, int32_t columns) {
  uniserve::join(static_cast<_Float16 *>(target), static_cast<const _Float16 *>(update),
                 static_cast<const _Float16 *>(gate), columns);
}
extern "C" __global__ void __launch_bounds__(256)
uniserve_sigmoid_gated_add_f32(void *target, const void *update, const void *gate, int32_t columns) {
  uniserve::join(static_cast<float *>(target), static_cast<const float *>(update),
                 static_cast<const float *>(gate), columns);
}

#ifndef UNISERVE_DEVICE_ONLY
extern "C" int32_t uniserve_sigmoid_gated_add_launch(void *target, const void *update, const void *gate,
                                                     int64_t rows, int64_t columns, int32_t dtype, void *stream,
                                                     char *error, size_t error_bytes) {
  auto refuse = [&](const char *message) -> int32_t {
    if (error != nullptr && error_bytes > 0) std::snprintf(error, error_bytes, "%s", message);
    return 1;
  };
  if (columns <= 0) return refuse("sigmoid_gated_add: a row of zero elements adds nothing");
  if (rows < 0) return refuse("sigmoid_gated_add: a negative row count");
  if (rows * columns > 0x7fffffffLL)
    return refuse("sigmoid_gated_add: the rows span more elements than 32-bit offsets address");
  if (rows == 0) return 0;
  if (target == nullptr || update == nullptr || gate == nullptr)
    return refuse("sigmoid_gated_add needs target, update and gate");
  size_t size;
  decltype(&uniserve_sigmoid_gated_add_bf16) kernel;
  if (dtype == UNISERVE_DTYPE_BF16) {
    size = 2;
    kernel = uniserve_sigmoid_gated_add_bf16;
  } else if (dtype == UNISERVE_DTYPE_F16) {
    size = 2;
    kernel = uniserve_sigmoid_gated_add_f16;
  } else if (dtype == UNISERVE_DTYPE_F32) {
    size = 4;
    kernel = uniserve_sigmoid_gated_add_f32;
  } else {
    return refuse("sigmoid_gated_add serves bf16, f16 or f32");
  }
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int32_t width = static_cast<int32_t>(columns);
  const uint32_t blocks = static_cast<uint32_t>((columns + UNISERVE_SIGMOID_GATED_ADD_BLOCK - 1) / UNISERVE_SIGMOID_GATED_ADD_BLOCK);
  // The reference's grid puts the rows on the second axis; more rows than it holds go in slices.
  constexpr int64_t kRowsPerLaunch = 65535;
  for (int64_t first = 0; first < rows; first += kRowsPerLaunch) {
    const int64_t count = rows - first < kRowsPerLaunch ? rows - first : kRowsPerLaunch;
    const size_t offset = static_cast<size_t>(first * columns) * size;
    hipLaunchKernelGGL(kernel, dim3(blocks, static_cast<uint32_t>(count)), dim3(256), 0, s,
                       static_cast<void *>(static_cast<char *>(target) + offset),
                       static_cast<const void *>(static_cast<const char *>(update) + offset),
                       static_cast<const void *>(static_cast<const char *>(gate) + first * size), width);
  }
  const hipError_t status = hipGetLastError();
  if (status != hipSuccess) return refuse(hipGetErrorString(status));
  return 0;
}
#endif

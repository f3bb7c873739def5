// SPDX-License-Identifier: Apache-2.0
//
// The router score GEMM's launch parameters, shared by its C entry and the layer driver.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace uniserve {

struct RouterParams {
  const uint16_t *x;      ///< [m, k] bf16
  const uint16_t *w;      ///< [n, k] bf16
  uint16_t *out;          ///< [m, n] bf16
  const float *bias;      ///< [n] or null
  int64_t m, n, k;
  int64_t x_stride, w_stride, out_stride;
  float alpha;
};

void launch_router(const RouterParams &p, hipStream_t stream);

}  // namespace uniserve

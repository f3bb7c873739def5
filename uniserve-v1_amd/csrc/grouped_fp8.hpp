// SPDX-License-Identifier: Apache-2.0
//
// Launch parameters of the block-scaled e4m3 grouped products and the activation quantiser,
// shared by their C entries and the layer driver.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace uniserve {

struct GroupedFp8Params {
  const uint8_t *act;           ///< FC1: hidden [tokens, K]; FC2: rows [permuted_rows, K], e4m3
  const float *act_scales;      ///< [rows of act, K / 128]
  const uint8_t *weights;       ///< [experts, n_total, K] e4m3
  const float *weight_scales;   ///< [experts, n_total / 128, K / 128]
  uint16_t *out;                ///< [permuted_rows, out_width] bf16
  const int32_t *tile_to_expert;
  const int32_t *tile_to_limit;
  const int32_t *permuted_to_expanded;
  const int32_t *num_tiles;
  int64_t K;
  int64_t n_total;
  int64_t out_width;
  int64_t top;
};

void launch_quantize_fp8(const void *input, bool input_f32, uint8_t *out, float *scales,
                         const int32_t *row_limit, int64_t rows, int64_t width, hipStream_t stream);
void launch_grouped_fp8(const GroupedFp8Params &p, bool gated, int64_t max_tiles, bool stream_path,
                        hipStream_t stream);
bool fp8_stream_path(int64_t routes, int64_t experts);

}  // namespace uniserve

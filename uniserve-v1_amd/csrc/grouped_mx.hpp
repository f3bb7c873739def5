// SPDX-License-Identifier: Apache-2.0
//
// Library-internal entry points of the MX products (grouped_gemm_mx.hip) for the layer.
#pragma once

#include "common.hpp"
#include "uniserve_moe_mx.h"

namespace uniserve {

/// The MXFP8 quantiser. `scales` (row-major, or null) and/or `stage_scales` (stage-major
/// [width / 128, stage_rows, 4]; with `routes` [rows, top] each row's scales go to the stage rows
/// its routes name instead of the row itself).
void launch_quantize_mxfp8(const void *input, bool input_f32, uint8_t *out, uint8_t *scales, const int32_t *row_limit,
                           int64_t rows, int64_t width, hipStream_t stream, uint8_t *stage_scales = nullptr,
                           const int32_t *routes = nullptr, int64_t top = 0, int64_t stage_rows = 0);

/// Whether both MX products of a layer run on the prefill (tiled) kernel, so both take their
/// activation scales stage-major by permuted row.
bool mx_route_scales(int64_t tokens, int64_t top, int64_t experts, int64_t hidden_size, int64_t intermediate,
                     int64_t permuted_rows);

/// The product entries; with `scale_rows` nonzero the activation scales are stage-major by
/// permuted row ([K / 128, scale_rows, 4], scale_rows >= permuted_rows).
int32_t gather_gemm_mx(const uniserve_gather_mx_call *call, int64_t scale_rows, int32_t activation, void *stream);
int32_t route_gemm_mx(const uniserve_route_mx_call *call, int64_t scale_rows, void *stream);

}  // namespace uniserve

// SPDX-License-Identifier: Apache-2.0
//
// Library-internal entry points of the MX products (grouped_gemm_mx.hip) for the layer.
#pragma once

#include "common.hpp"
#include "grouped_fp8.hpp"
#include "uniserve_moe_mx.h"

namespace uniserve {

/// The E8M0 byte of a block: the smallest power of two 2^e with amax <= limit * 2^e, e in
/// [-127, 127]; an all-zero or infinite block takes 2^0. With amax = ma 2^ea and limit = ml 2^el
/// (mantissas in [0.5, 1), the hardware frexp, exact for subnormals too) the rule is e = ea - el,
/// or one more where ma > ml: every comparison exact, no rounding anywhere.
__device__ __forceinline__ uint32_t mx_scale(float amax, float limit) {
  if (!(amax > 0.0f) || __builtin_isinf(amax)) return 127u;
  int e = __builtin_amdgcn_frexp_expf(amax) - __builtin_amdgcn_frexp_expf(limit);
  if (__builtin_amdgcn_frexp_mantf(amax) > __builtin_amdgcn_frexp_mantf(limit)) ++e;
  e = e < -127 ? -127 : (e > 127 ? 127 : e);  // a subnormal block: 2^-127 already holds it
  return static_cast<uint32_t>(e + 127);
}

/// 2^(byte - 127) for an E8M0 byte in [0, 254] - the block's scale - and its reciprocal, both
/// exact (2^-127 is a subnormal).
__device__ __forceinline__ float e8m0_value(uint32_t byte) { return __builtin_amdgcn_ldexpf(1.0f, static_cast<int>(byte) - 127); }

/// One 32-channel MXFP8 block, four lanes (aligned groups of four lanes of the wavefront) with
/// eight channels each in `v`: writes this lane's eight e4m3 codes to `codes` and returns the
/// block's E8M0 byte (every lane of the block holds it) - the quantiser's arithmetic, shared by
/// every kernel that makes MXFP8 rows.
__device__ __forceinline__ uint32_t mxfp8_eight(const float (&v)[8], uint8_t *codes) {
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[j]));
  amax = __builtin_fmaxf(amax, __shfl_xor(amax, 1, 4));
  amax = __builtin_fmaxf(amax, __shfl_xor(amax, 2, 4));
  const uint32_t scale = mx_scale(amax, 448.0f);
  // The scale is a power of two: v / scale is v times the exact reciprocal, the same number
  // rounded once, and no quotient exceeds 448.
  const float r = e8m0_value(254u - scale);
  uint2 out;
  out.x = e4m3_pair(v[0] * r, v[1] * r) | (e4m3_pair(v[2] * r, v[3] * r) << 16);
  out.y = e4m3_pair(v[4] * r, v[5] * r) | (e4m3_pair(v[6] * r, v[7] * r) << 16);
  *reinterpret_cast<uint2 *>(codes) = out;
  return scale;
}

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
/// `out_codes` (with `out_code_scales`; route-major scales, the tiled kernel only): FC1 writes the
/// gated rows as MXFP8 codes and stage-major E8M0 bytes by permuted row, bit for bit what
/// uniserve_quantize_mxfp8 makes of the bf16 rows, and no bf16 rows.
int32_t gather_gemm_mx(const uniserve_gather_mx_call *call, int64_t scale_rows, int32_t activation, void *stream,
                       uint8_t *out_codes = nullptr, uint8_t *out_code_scales = nullptr);
int32_t route_gemm_mx(const uniserve_route_mx_call *call, int64_t scale_rows, void *stream);

}  // namespace uniserve

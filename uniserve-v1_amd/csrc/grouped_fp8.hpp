// SPDX-License-Identifier: Apache-2.0
//
// Launch parameters of the block-scaled e4m3 grouped products and the activation quantiser,
// shared by their C entries and the layer driver.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.hpp"
#include "uniserve_moe_fp8.h"

namespace uniserve {

// ---- e4m3 encoding ---------------------------------------------------------------------------------------

/// Nearest-even e4m3fn code of `value`, saturating at +-448 (0x7e); NaN -> 0x7f.
__device__ __forceinline__ uint32_t e4m3_encode(float value) {
  const uint32_t bits = __float_as_uint(value);
  const uint32_t sign = (bits >> 24) & 0x80u;
  const float a = __builtin_fabsf(value);
  if (a != a) return sign | 0x7fu;
  if (a >= 448.0f) return sign | 0x7eu;
  if (a < 0.015625f) return sign | static_cast<uint32_t>(__builtin_rintf(a * 512.0f));
  const int e = static_cast<int>((__float_as_uint(a) >> 23) & 0xffu) - 127;
  const float unit = __uint_as_float(static_cast<uint32_t>(127 - e) << 23);  // 2^-e, exact
  int m = static_cast<int>(__builtin_rintf((a * unit - 1.0f) * 8.0f));
  int exponent = e;
  if (m == 8) {
    m = 0;
    exponent += 1;
  }
  uint32_t code = static_cast<uint32_t>(((exponent + 7) << 3) | m);
  if (code > 0x7eu) code = 0x7eu;
  return sign | code;
}

/// The e4m3 codes of a pair of quotients, packed into the low 16 bits. gfx950's conversion rounds
/// to nearest even exactly as e4m3_encode does wherever |q| <= 448 (checked over every such
/// float); anything else (saturation, NaN) takes e4m3_encode.
__device__ __forceinline__ uint32_t e4m3_pair(float q0, float q1) {
  if (__builtin_fabsf(q0) <= 448.0f && __builtin_fabsf(q1) <= 448.0f)
    return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(q0, q1, 0, false)) & 0xffffu;
  return e4m3_encode(q0) | (e4m3_encode(q1) << 8);
}

/// Eight values quantised with one scale: the e4m3 codes of the IEEE quotients v / scale, packed
/// low to high.
__device__ __forceinline__ uint2 e4m3_eight(const float (&v)[8], float scale) {
  uint2 out;
  out.x = e4m3_pair(v[0] / scale, v[1] / scale) | (e4m3_pair(v[2] / scale, v[3] / scale) << 16);
  out.y = e4m3_pair(v[4] / scale, v[5] / scale) | (e4m3_pair(v[6] / scale, v[7] / scale) << 16);
  return out;
}

/// v / scale for a bf16 value v given r = 1 / scale, without a division: q0 = v r, then one
/// correction by the residual v - q0 scale, exact under FMA (Markstein, IBM J. Res. Dev. 34(1),
/// 1990). The result is within an ulp of the IEEE quotient and is not always equal to it, but its
/// e4m3 code is, for scale = amax / 448 over bf16 values |v| <= amax: on the device, every pair of
/// magnitudes with scale in [2^-100, 2^100] gives the code of the IEEE quotient (5.3e8 pairs; the
/// operations are odd in v, and -0 keeps its sign), and the quantiser's GPU test repeats this with
/// both signs for every magnitude under about a thousand maxima.
__device__ __forceinline__ float quotient_bf16(float v, float scale, float r) {
  const float q0 = v * r;
  const float residual = __builtin_fmaf(-q0, scale, v);
  // v = -0 gives q0 = -0 and a residual of +0, whose sum is +0: the sign is v's.
  return __builtin_copysignf(__builtin_fmaf(residual, r, q0), v);
}

/// The e4m3 codes of two non-NaN values, packed into the low 16 bits, as e4m3_encode gives them:
/// magnitudes past 448 (which e4m3_encode saturates) are brought to 448 first, then the hardware
/// conversion (checked against e4m3_encode over every non-NaN float).
__device__ __forceinline__ uint32_t e4m3_pair_saturated(float q0, float q1) {
  const float s0 = __builtin_copysignf(__builtin_fminf(__builtin_fabsf(q0), 448.0f), q0);
  const float s1 = __builtin_copysignf(__builtin_fminf(__builtin_fabsf(q1), 448.0f), q1);
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(s0, s1, 0, false)) & 0xffffu;
}

/// e4m3_eight for bf16 values and a scale amax / 448 of their amax, without division: false (and
/// `out` unset) when a value is NaN or the scale lies outside [2^-100, 2^100]; the caller then
/// takes e4m3_eight.
__device__ __forceinline__ bool e4m3_eight_bf16(const float (&v)[8], float scale, uint2 &out) {
  bool fits = scale >= 0x1p-100f && scale <= 0x1p100f;
#pragma unroll
  for (int j = 0; j < 8; ++j) fits &= !__builtin_isnan(v[j]);
  const float r = 1.0f / scale;
  float q[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) q[j] = quotient_bf16(v[j], scale, r);
  out.x = e4m3_pair_saturated(q[0], q[1]) | (e4m3_pair_saturated(q[2], q[3]) << 16);
  out.y = e4m3_pair_saturated(q[4], q[5]) | (e4m3_pair_saturated(q[6], q[7]) << 16);
  return fits;
}

/// e4m3_eight for bf16 values and a scale amax / 448 of their amax: e4m3_eight_bf16, else by
/// division.
__device__ __forceinline__ uint2 e4m3_eight_of_bf16(const float (&v)[8], float scale) {
  uint2 out;
  if (e4m3_eight_bf16(v, scale, out)) return out;
  return e4m3_eight(v, scale);
}

/// One 128-channel group of a bf16 row as e4m3 codes and its FP32 scale (amax / 448, 1 for an
/// all-zero group), 16 lanes per group (lane `sub` holds channels 8 sub .. 8 sub + 7): the
/// activation quantiser's arithmetic, shared by every kernel that quantises hidden rows. Returns
/// the scale (every lane of the group holds it).
__device__ __forceinline__ float quantize_bf16_group(const uint16_t *group, uint8_t *codes, float *scale_out, int sub) {
  const u32x4 packed = *reinterpret_cast<const u32x4 *>(group + sub * 8);
  float v[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[2 * j] = __uint_as_float(packed[j] << 16);
    v[2 * j + 1] = __uint_as_float(packed[j] & 0xffff0000u);
  }
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[j]));
  amax = row16_max(amax);
  const float scale = amax > 0.0f ? amax / 448.0f : 1.0f;
  *reinterpret_cast<uint2 *>(codes + sub * 8) = e4m3_eight_of_bf16(v, scale);
  if (sub == 0) *scale_out = scale;
  return scale;
}

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
  uint8_t *out_codes;           ///< FC1 only, or null: the gated rows as e4m3 [permuted_rows, out_width]
  float *out_code_scales;       ///< with out_codes: [permuted_rows, out_width / 128]
  int64_t scale_rows;           ///< nonzero (prefill kernel only): act_scales and out_code_scales are
                                ///< route-major, [blocks, scale_rows] by permuted row
  int32_t activation;           ///< FC1's gate: UNISERVE_ACTIVATION_SILU or _GELU_TANH
  // Expert-major stream (decode, no sort): workgroup x serves local expert x, whose rows are the
  // routes naming it in `ids`, at their expanded positions (act rows: FC1 route / top, FC2 route).
  const int32_t *ids;
  const int32_t *live_tokens;
  int64_t routes;
  int64_t local_offset;
  int64_t local_experts;
  int32_t compact;              ///< workgroup x serves the x-th named local expert
};

void launch_quantize_fp8(const void *input, bool input_f32, uint8_t *out, float *scales,
                         const int32_t *row_limit, int64_t rows, int64_t width, hipStream_t stream);
void launch_grouped_fp8(const GroupedFp8Params &p, bool gated, int64_t max_tiles, bool stream_path, bool one_pass,
                        hipStream_t stream);
bool fp8_stream_path(int64_t routes, int64_t experts);
/// The expert-major stream kernel over `local_experts` workgroup columns (p.ids .. set). FC1 with
/// p.out_codes (only where expert_stream_fp8_fc1_quantizes holds: the unsplit kernel) also writes
/// the gated rows as FC2's e4m3 operand (codes [routes, out_width], scales [routes, out_width / 128]).
void launch_expert_stream_fp8(const GroupedFp8Params &p, bool gated, int64_t local_experts, hipStream_t stream);
bool expert_stream_fp8_fc1_quantizes(int64_t routes, int64_t local_experts, int64_t out_width);

/// The quantiser over token rows that also scatters each scale to the permuted rows of the
/// token's routes: route_scales[g, expanded_to_permuted[t, k]] for every held route (k < top).
void launch_quantize_fp8_routes(const uint16_t *input, uint8_t *out, float *scales, float *route_scales,
                                const int32_t *expanded_to_permuted, int64_t top, int64_t route_rows,
                                int64_t rows, int64_t width, hipStream_t stream);

/// Whether FC1 in e4m3 can write its gated rows already quantised for FC2 (the prefill kernel
/// serves the shape), which spares the layer the bf16 round trip and the separate quantiser.
bool fp8_fc1_quantizes(int64_t tokens, int64_t top, int64_t experts, int64_t hidden_size, int64_t intermediate);

/// The gather_gemm_fp8 entry; with `codes` (and `code_scales`) set, the gated rows are written as
/// e4m3 codes and per-128-column scales - bit for bit what uniserve_quantize_fp8 makes of the bf16
/// rows - instead of bf16 (refused unless fp8_fc1_quantizes).
/// With `scale_rows` nonzero, hidden_scales are route-major ([hidden / 128, scale_rows] by permuted
/// row, as launch_quantize_fp8_routes writes them) and so are the code scales written.
/// `activation` is FC1's gate (uniserve_activation).
int32_t gather_gemm_fp8(const uniserve_gather_fp8_call *call, uint8_t *codes, float *code_scales,
                        int64_t scale_rows, int32_t activation, void *stream);

/// Whether the layer's two e4m3 products both run on the prefill kernel, so both can take
/// route-major activation scales: one cache line holds 32 consecutive rows' scales of a block,
/// where row-major scales of gathered token rows cost a line per row.
bool fp8_route_scales(int64_t tokens, int64_t top, int64_t experts, int64_t hidden_size, int64_t intermediate,
                      int64_t permuted_rows);

/// The route_gemm_fp8 entry; with `scale_rows` nonzero the row scales are route-major
/// ([intermediate / 128, scale_rows]; refused unless the prefill kernel serves the shape).
int32_t route_gemm_fp8(const uniserve_route_fp8_call *call, int64_t scale_rows, void *stream);

}  // namespace uniserve

// SPDX-License-Identifier: Apache-2.0
//
// One token's trip through the router, by one workgroup (the decode front end without a sort):
// router scores (crates/nn/src/modules/moe.rs:656-671) and topk_softmax (crates/ops/src/moe/
// routing.rs) for token `token`, and, for e4m3 and MXFP4 layers, the quantisation of its hidden
// row.
//
// The workgroup streams the whole router matrix: wavefront w takes experts w, w + kWaves, ..., one
// or two rows per pass with the next pass's loads in flight, each row as whole 1 KB lines (lane l
// holds channels 512 c + 8 l .. + 7 of chunk c, against the same slice of the token's row, which
// every wavefront keeps in registers). Each lane keeps one FP32 partial sum per expert of its
// wavefront; the sums are reduced across the wavefront by xor butterflies (every expert's the same
// way, so the scores do not depend on kWaves), get the bias and one rounding into bf16, and go to
// the layer's score tensor and to LDS; the first 32-lane half routes the token from there with the
// topk routine, and the id's lane writes the route's expanded_to_permuted entry (the layer skips
// the sort). The first wavefront quantises the hidden row from its registers with the quantisers'
// group routines (codes and scales bit for bit theirs).
#pragma once

#include "common.hpp"
#include "grouped_fp8.hpp"
#include "grouped_mx.hpp"
#include "moe_front.hpp"
#include "topk_route.hpp"

namespace uniserve {
namespace front_token {

constexpr int kChunk = 512;       // channels of one row per wavefront load (64 lanes x 8)
constexpr int kMaxExperts = 128;  // four scores per lane of the routing half

__device__ __forceinline__ float dot8_bf16(const u32x4 &a, const u32x4 &b, float sum) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    sum = __builtin_fmaf(__uint_as_float(a[j] << 16), __uint_as_float(b[j] << 16), sum);
    sum = __builtin_fmaf(__uint_as_float(a[j] & 0xffff0000u), __uint_as_float(b[j] & 0xffff0000u), sum);
  }
  return sum;
}

/// kWaves: the workgroup's wavefronts (every thread calls this); kChunks: at most that many
/// 512-channel chunks per row (4: hidden <= 2048, two router rows per pass; 8: hidden <= 4096,
/// one); kQuant: 0 none, 1 e4m3, 2 MXFP8. `scores`: kMaxExperts bf16 in LDS.
template <int kWaves, int kChunks, int kQuant>
__device__ __forceinline__ void route_one(const FrontParams &p, int64_t token, uint16_t *scores) {
  constexpr int kRows = 8 / kChunks;
  constexpr int kPerWave = kMaxExperts / kWaves;
  constexpr int kPasses = kPerWave / kRows;
  static_assert(kPerWave % kRows == 0, "whole passes");
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  const int lane = lane_id();
  const int chunks = static_cast<int>(p.hidden / kChunk);
  const int experts = static_cast<int>(p.experts);

  u32x4 xs[kChunks];
#pragma unroll
  for (int c = 0; c < kChunks; ++c)
    xs[c] = c < chunks ? *reinterpret_cast<const u32x4 *>(p.x + token * p.hidden + c * kChunk + 8 * lane)
                       : u32x4{0, 0, 0, 0};

  u32x4 w[2][kRows][kChunks];
  float partial[kPerWave];
  auto load_pass = [&](int pass, int buffer) {
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      const int e = wave + (pass * kRows + r) * kWaves;
      const uint16_t *row = p.w + static_cast<int64_t>(e < experts ? e : 0) * p.hidden + 8 * lane;
#pragma unroll
      for (int c = 0; c < kChunks; ++c)
        if (c < chunks) w[buffer][r][c] = *reinterpret_cast<const u32x4 *>(row + c * kChunk);
    }
  };
  load_pass(0, 0);
#pragma unroll
  for (int pass = 0; pass < kPasses; ++pass) {
    if (pass + 1 < kPasses) load_pass(pass + 1, (pass + 1) & 1);
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      float sum = 0.0f;
#pragma unroll
      for (int c = 0; c < kChunks; ++c)
        if (c < chunks) sum = dot8_bf16(w[pass & 1][r][c], xs[c], sum);
      partial[pass * kRows + r] = sum;
    }
  }
#pragma unroll
  for (int offset = 32; offset >= 1; offset /= 2)
#pragma unroll
    for (int i = 0; i < kPerWave; ++i) partial[i] += __shfl_xor(partial[i], offset);
  // Lane i (i < kPerWave) finishes its wavefront's i-th expert.
  float sum = partial[0];
#pragma unroll
  for (int i = 1; i < kPerWave; ++i) sum = lane == i ? partial[i] : sum;
  const int e = wave + lane * kWaves;
  if (lane < kPerWave && e < experts) {
    if (p.bias != nullptr) sum += p.bias[e];
    const uint16_t bits = f32_to_bf16(sum);
    scores[e] = bits;
    p.scores[token * experts + e] = bits;
  }

  // The hidden row's quantisation, first wavefront: lane l's slice of chunk c is channels
  // 512 c + 8 l .. + 7, in 128-channel group 4 c + l / 16 (16 lanes each) or 32-channel block
  // (512 c + 8 l) / 32 (4 lanes each).
  if constexpr (kQuant != 0) {
    if (wave == 0) {
#pragma unroll
      for (int c = 0; c < kChunks; ++c) {
        if (c >= chunks) break;
        float v[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[2 * j] = __uint_as_float(xs[c][j] << 16);
          v[2 * j + 1] = __uint_as_float(xs[c][j] & 0xffff0000u);
        }
        uint8_t *codes = p.hidden_codes + token * p.hidden + c * kChunk + 8 * lane;
        if constexpr (kQuant == 2) {
          const uint32_t scale = mxfp8_eight(v, codes);
          if ((lane & 3) == 0)
            p.hidden_mx_scales[token * (p.hidden / 32) + (c * kChunk + 8 * lane) / 32] = static_cast<uint8_t>(scale);
        } else {
          float amax = 0.0f;
#pragma unroll
          for (int j = 0; j < 8; ++j) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[j]));
          amax = row16_max(amax);
          const float scale = amax > 0.0f ? amax / 448.0f : 1.0f;
          *reinterpret_cast<uint2 *>(codes) = e4m3_eight_of_bf16(v, scale);
          if ((lane & 15) == 0) p.hidden_scales[token * (p.hidden / 128) + 4 * c + lane / 16] = scale;
        }
      }
    }
  }
  __syncthreads();

  // Routing by the first 32-lane half; each pick's lane writes its route's entry.
  if (threadIdx.x < topk::kHalf) {
    const int32_t id = topk::route<kMaxExperts / topk::kHalf, false>(
        scores, 1, experts, static_cast<int>(token), experts, p.top, p.renormalize, nullptr, -1, p.ids, p.weights,
        p.map, p.live, p.load, true, 0);
    const int k = static_cast<int>(threadIdx.x);
    if (k < p.top) {
      const int64_t route = token * p.top + k;
      const int64_t live = (p.live != nullptr ? static_cast<int64_t>(p.live[0]) : p.tokens) * p.top;
      const int64_t local = static_cast<int64_t>(id) - p.sort.local_offset;
      const bool visible = route < live && local >= 0 && local < p.sort.local_experts;
      p.sort.expanded_to_permuted[route] = visible ? static_cast<int32_t>(route) : -1;
    }
  }
}

}  // namespace front_token
}  // namespace uniserve

// SPDX-License-Identifier: Apache-2.0
//
// The router's per-token routine (softmax, top-k, renormalisation, scale, map, load) of the
// topk_softmax kernel.
//
// One token per 32-lane half of a 64-lane wavefront. The probabilities are FP32 reductions whose
// rounding depends on their order, and the selection compares them for equality, so the routine
// keeps the reference's reduction tree exactly (crates/ops/kernels/topk_softmax/nvcc/src/
// topk_softmax.cu:106-199): lane j of a half holds experts j + 32 i, sums its own terms in i
// order, and the halves exchange by xor butterflies over 16, 8, 4, 2, 1 within the half (DPP for
// 1, 2, 4 and 8, the gfx950 row swap for 16).
//
// The exponential is the library's own (`router_expf`) and not the platform's, so that the CPU
// oracle evaluates the identical operations: every probability, and therefore every id, is
// reproducible bit for bit on the host.
#pragma once

#include <cfloat>
#include <climits>

#include "common.hpp"

#pragma clang fp contract(off)

namespace uniserve {
namespace topk {

constexpr int kHalf = 32;

/// Cody-Waite reduction x = n ln2 + r and the degree-7 Taylor polynomial of e^r (Horner, fused
/// multiply-adds), scaled by 2^n in two exact power-of-two steps.
__device__ __forceinline__ float router_expf(float x) {
  if (x != x) return x;
  if (x < -104.0f) return 0.0f;
  if (x > 88.75f) return __builtin_inff();
  const float n = __builtin_rintf(x * 1.44269504088896341f);
  float r = __builtin_fmaf(-n, 0.693145751953125f, x);
  r = __builtin_fmaf(-n, 1.42860682030941723e-6f, r);
  float p = 1.98412698412698413e-4f;
  p = __builtin_fmaf(p, r, 1.38888888888888889e-3f);
  p = __builtin_fmaf(p, r, 8.33333333333333333e-3f);
  p = __builtin_fmaf(p, r, 4.16666666666666667e-2f);
  p = __builtin_fmaf(p, r, 1.66666666666666667e-1f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const int k = static_cast<int>(n);
  const int half = k / 2;
  const float first = __uint_as_float(static_cast<uint32_t>(half + 127) << 23);
  const float second = __uint_as_float(static_cast<uint32_t>(k - half + 127) << 23);
  return (p * first) * second;
}

/// The value of lane (this lane xor kOffset), within each 32-lane half: VALU lane exchanges only
/// (DPP within a 16-lane row, the row swap across rows), no trip through the LDS crossbar.
template <int kOffset>
__device__ __forceinline__ int xor_lane(int value) {
  if constexpr (kOffset == 1) {
    return __builtin_amdgcn_mov_dpp(value, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
  } else if constexpr (kOffset == 2) {
    return __builtin_amdgcn_mov_dpp(value, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
  } else if constexpr (kOffset == 4) {
    // Lanes with bit 2 clear read 4 lanes up (row_shl:4), the others 4 lanes down (row_shr:4);
    // neither leaves its 16-lane row.
    const int up = __builtin_amdgcn_mov_dpp(value, 0x104, 0xF, 0xF, false);
    const int down = __builtin_amdgcn_mov_dpp(value, 0x114, 0xF, 0xF, false);
    return (lane_id() & 4) ? down : up;
  } else if constexpr (kOffset == 8) {
    return __builtin_amdgcn_mov_dpp(value, 0x128, 0xF, 0xF, false);  // row_ror:8 = xor 8 in a row
  } else {
    static_assert(kOffset == 16, "exchanges within a 32-lane half");
    // Swapping the odd rows of one copy with the even rows of another leaves, in each lane, its
    // own row in the first result and its partner row in the second (or the reverse for odd rows).
    const auto swapped = __builtin_amdgcn_permlane16_swap(value, value, false, false);
    return (lane_id() & 16) ? static_cast<int>(swapped[0]) : static_cast<int>(swapped[1]);
  }
}

template <int kOffset>
__device__ __forceinline__ float xor_lane(float value) {
  return __int_as_float(xor_lane<kOffset>(__float_as_int(value)));
}

__device__ __forceinline__ float load_kind(const void *data, int kind, int64_t index) {
  if (kind == 0) return static_cast<const float *>(data)[index];
  if (kind == 2) return static_cast<float>(static_cast<const _Float16 *>(data)[index]);
  return bf16_to_f32(static_cast<const uint16_t *>(data)[index]);
}
/// The same read at device scope (scores another workgroup of the launch stored at device scope).
__device__ __forceinline__ float load_kind_device(const void *data, int kind, int64_t index) {
  if (kind == 0) return load_device(static_cast<const float *>(data) + index);
  const uint16_t bits = load_device(static_cast<const uint16_t *>(data) + index);
  if (kind == 2) return static_cast<float>(__builtin_bit_cast(_Float16, bits));
  return bf16_to_f32(bits);
}

template <int kOffset>
__device__ __forceinline__ void max_step(float &maximum) {
  const float other = xor_lane<kOffset>(maximum);
  maximum = maximum < other ? other : maximum;
}

template <int kOffset>
__device__ __forceinline__ void max_key_step(uint64_t &key) {
  const uint64_t other = (static_cast<uint64_t>(static_cast<uint32_t>(xor_lane<kOffset>(static_cast<int>(key >> 32)))) << 32) |
                         static_cast<uint32_t>(xor_lane<kOffset>(static_cast<int>(static_cast<uint32_t>(key))));
  key = key < other ? other : key;
}

template <int kOffset>
__device__ __forceinline__ void sum_step(float &sum) {
  sum = sum + xor_lane<kOffset>(sum);
}

template <int kOffset>
__device__ __forceinline__ void argmax_step(float &best, int &expert) {
  const float other = xor_lane<kOffset>(best);
  const int other_expert = xor_lane<kOffset>(expert);
  if (other > best || (other == best && other_expert < expert)) {
    best = other;
    expert = other_expert;
  }
}

/// Routes one token with `kIter` scores per lane (the expert count in whole halves, rounded up to
/// a power of two: the extra slots hold -inf and add exact zeros to the sum). kDevice: the scores
/// are read and the ids stored at device scope (scores and ids cross workgroups of one launch).
/// Answers, in lane k < top of an active token, the id it stored (-1 in the other lanes).
template <int kIter, bool kDevice>
__device__ __forceinline__ int32_t route(const void *scores, int score_kind, int64_t row_stride,
                                      int row, int experts, int top, int renormalize,
                                      const void *scale, int scale_kind, int32_t *ids,
                                      float *weights, const int32_t *map, const int32_t *live,
                                      unsigned long long *load, bool active, int score_row) {
  const int lane = static_cast<int>(threadIdx.x) & (kHalf - 1);
  float values[kIter];
#pragma unroll
  for (int it = 0; it < kIter; ++it) {
    const int expert = lane + it * kHalf;
    const int64_t at = static_cast<int64_t>(score_row) * row_stride + expert;
    values[it] = expert < experts ? (kDevice ? load_kind_device(scores, score_kind, at) : load_kind(scores, score_kind, at))
                                  : -__builtin_inff();
  }

  float maximum = values[0];
#pragma unroll
  for (int it = 0; it < kIter; ++it) maximum = maximum > values[it] ? maximum : values[it];
  max_step<16>(maximum);
  max_step<8>(maximum);
  max_step<4>(maximum);
  max_step<2>(maximum);
  max_step<1>(maximum);

  float sum = 0.0f;
#pragma unroll
  for (int it = 0; it < kIter; ++it) {
    values[it] = router_expf(values[it] - maximum);
    sum += values[it];
  }
  sum_step<16>(sum);
  sum_step<8>(sum);
  sum_step<4>(sum);
  sum_step<2>(sum);
  sum_step<1>(sum);
#pragma unroll
  for (int it = 0; it < kIter; ++it) values[it] = values[it] / sum;

  // `top` rounds of a (value, lower id) arg-max; lane j keeps round j's pick. A round's pick is
  // the largest probability among the experts not yet taken, the lowest id among equal ones (the
  // reference's (value, lower id) butterfly, topk_softmax.cu:152-182): the maximum value by a
  // butterfly of max alone, then the lowest expert holding it by one ballot per slot. A candidate
  // is a probability (>= 0, never NaN for a finite row) of an expert of the row not yet taken;
  // the rest stand at -1, below every probability, so a round with no candidate (a row of NaN
  // scores) names no expert: value -1, expert INT_MAX, as in the reference.
  float picked = 0.0f;
  int picked_expert = 0;
  if constexpr (kIter <= 4) {
    // The same selection on 64-bit keys (probability bits, then the complement of the expert id):
    // a candidate's probability is >= 0, so its bits order as the values do, and among equal
    // probabilities the lower id has the larger key - one unsigned maximum per round does the
    // (value, lower id) arg-max. Non-candidates hold key 0, below every candidate's. Each lane
    // sorts its keys once, largest first; a round's offer is the lane's first key not yet taken,
    // and only the lane whose offer won moves on (keys are distinct: the ids are). Half the
    // instructions of a round of the float butterfly and the ballots.
    uint64_t key[kIter];
#pragma unroll
    for (int it = 0; it < kIter; ++it) {
      const int expert = lane + it * kHalf;
      const bool candidate = expert < experts && values[it] >= 0.0f;
      key[it] = candidate ? (static_cast<uint64_t>(__float_as_uint(values[it])) << 32) | (~static_cast<uint32_t>(expert))
                          : 0ull;
    }
    auto order = [&](int a, int b) {  // key[a] >= key[b] afterwards
      const uint64_t x = key[a], y = key[b];
      key[a] = x < y ? y : x;
      key[b] = x < y ? x : y;
    };
    if constexpr (kIter >= 2) order(0, 1);
    if constexpr (kIter == 4) {
      order(2, 3);
      order(0, 2);
      order(1, 3);
      order(1, 2);
    }
    int next = 0;
    for (int j = 0; j < top; ++j) {
      uint64_t offer = 0ull;
#pragma unroll
      for (int it = kIter - 1; it >= 0; --it) offer = next == it ? key[it] : offer;
      uint64_t best = offer;
      max_key_step<16>(best);
      max_key_step<8>(best);
      max_key_step<4>(best);
      max_key_step<2>(best);
      max_key_step<1>(best);
      if (best != 0ull && offer == best) ++next;
      if (lane == j) {
        picked = best != 0ull ? __uint_as_float(static_cast<uint32_t>(best >> 32)) : -1.0f;
        picked_expert = best != 0ull ? static_cast<int>(~static_cast<uint32_t>(best)) : INT_MAX;
      }
    }
  } else {
  uint32_t taken = 0u;
  const uint64_t half_lanes = (lane_id() & kHalf) ? 0xffffffff00000000ull : 0x00000000ffffffffull;
  for (int j = 0; j < top; ++j) {
    float candidate[kIter];
    float best = -1.0f;
#pragma unroll
    for (int it = 0; it < kIter; ++it) {
      const int expert = lane + it * kHalf;
      candidate[it] = (expert < experts && !((taken >> it) & 1u) && values[it] >= 0.0f) ? values[it] : -1.0f;
      best = best < candidate[it] ? candidate[it] : best;
    }
    max_step<16>(best);
    max_step<8>(best);
    max_step<4>(best);
    max_step<2>(best);
    max_step<1>(best);
    int best_expert = INT_MAX;
    if (best >= 0.0f) {
#pragma unroll
      for (int it = kIter - 1; it >= 0; --it) {
        const uint64_t holders = ballot(candidate[it] == best) & half_lanes;
        if (holders != 0) best_expert = it * kHalf + ((__builtin_ctzll(holders)) & (kHalf - 1));
      }
    }
    if (lane == j) {
      picked = best;
      picked_expert = best_expert;
    }
    if (best_expert != INT_MAX && (best_expert & (kHalf - 1)) == lane) taken |= 1u << (best_expert / kHalf);
  }
  }

  float weight = picked;
  if (renormalize) {
    // The butterfly over the next power of two of `top` lanes, lanes past `top` holding zero.
    int width = 1;
    while (width < top) width *= 2;
    float partial = lane < top ? picked : 0.0f;
    if (width > 16) sum_step<16>(partial);
    if (width > 8) sum_step<8>(partial);
    if (width > 4) sum_step<4>(partial);
    if (width > 2) sum_step<2>(partial);
    if (width > 1) sum_step<1>(partial);
    const float total = partial < FLT_EPSILON ? FLT_EPSILON : partial;
    weight = weight / total;
  }
  if (!active || lane >= top) return -1;
  const bool named = picked_expert >= 0 && picked_expert < experts;
  if (scale_kind != -1 && scale != nullptr && named) weight = weight * load_kind(scale, scale_kind, picked_expert);
  const int64_t slot = static_cast<int64_t>(row) * top + lane;
  const int32_t id = (map != nullptr && named) ? map[picked_expert] : picked_expert;
  if constexpr (kDevice) store_device(ids + slot, id);
  else ids[slot] = id;
  weights[slot] = weight;
  if (load != nullptr && named && (live == nullptr || row < live[0])) atomicAdd(load + picked_expert, 1ull);
  return id;
}


/// Routes token `row` (`active` false: take part in the wavefront's exchanges, store nothing),
/// with the per-lane slot count the expert count needs; its scores are row `score_row` of
/// `scores` (-1: row `row`).
template <bool kDevice = false>
__device__ __forceinline__ void route_token(const void *scores, int score_kind, int64_t row_stride, int row,
                                            int experts, int top, int renormalize, const void *scale,
                                            int scale_kind, int32_t *ids, float *weights, const int32_t *map,
                                            const int32_t *live, unsigned long long *load, bool active,
                                            int score_row = -1) {
  if (score_row < 0) score_row = row;
  const int needed = (experts + kHalf - 1) / kHalf;
  if (needed <= 1)
    route<1, kDevice>(scores, score_kind, row_stride, row, experts, top, renormalize, scale, scale_kind, ids, weights, map, live, load, active, score_row);
  else if (needed <= 2)
    route<2, kDevice>(scores, score_kind, row_stride, row, experts, top, renormalize, scale, scale_kind, ids, weights, map, live, load, active, score_row);
  else if (needed <= 4)
    route<4, kDevice>(scores, score_kind, row_stride, row, experts, top, renormalize, scale, scale_kind, ids, weights, map, live, load, active, score_row);
  else if (needed <= 8)
    route<8, kDevice>(scores, score_kind, row_stride, row, experts, top, renormalize, scale, scale_kind, ids, weights, map, live, load, active, score_row);
  else if (needed <= 16)
    route<16, kDevice>(scores, score_kind, row_stride, row, experts, top, renormalize, scale, scale_kind, ids, weights, map, live, load, active, score_row);
  else
    route<32, kDevice>(scores, score_kind, row_stride, row, experts, top, renormalize, scale, scale_kind, ids, weights, map, live, load, active, score_row);
}

}  // namespace topk
}  // namespace uniserve

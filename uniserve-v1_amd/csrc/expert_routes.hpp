// SPDX-License-Identifier: Apache-2.0
//
// The routes of one local expert, found by the workgroup that serves it (decode products without
// a sort): the routes whose id is the expert's, in route order - the order the sort's stable
// placement gives them.
#pragma once

#include "common.hpp"

namespace uniserve {

/// The most routes an expert-major workgroup lists (a decode batch's).
constexpr int kExpertRoutes = 4096;

/// Routes each wavefront of a kWaves-wave workgroup scans (whole chunks of 64).
template <int kWaves>
__host__ __device__ constexpr int64_t routes_per_wave(int64_t routes) {
  return ((routes + kWave - 1) / kWave + kWaves - 1) / kWaves * kWave;
}

/// A wavefront's first 4 x 64 route ids of its stretch (as list_expert_routes scans it), loaded
/// ahead: a kernel that issues its first weight loads between these loads and the scan waits for
/// the ids alone (the wait for a load also waits for every load issued before it).
struct FirstRouteIds {
  int32_t id[4];
};
template <int kWaves>
__device__ __forceinline__ FirstRouteIds load_first_route_ids(const int32_t *ids, int64_t routes) {
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int64_t begin = wave * routes_per_wave<kWaves>(routes);
  FirstRouteIds first;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int64_t route = begin + u * kWave + lane_id();
    first.id[u] = ids[route < routes ? route : 0];  // (the scan drops routes past its stretch)
  }
  return first;
}

/// Lists the live routes (route < live) whose id is `want`: wavefront w ballots routes
/// [w q, (w + 1) q), q = routes_per_wave, into list[w q ..] and counts[w]; counts[kWaves] is the
/// total. Every thread of the workgroup calls it (two barriers); returns the total.
/// `first`, if given: load_first_route_ids' ids, used for the stretch's first 4 x 64 routes.
template <int kWaves>
__device__ __forceinline__ int list_expert_routes(const int32_t *ids, int64_t routes, int64_t live, int32_t want,
                                                  int32_t *list, int32_t *counts,
                                                  const FirstRouteIds *first = nullptr) {
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int lane = lane_id();
  const int64_t per_wave = routes_per_wave<kWaves>(routes);
  const int64_t begin = wave * per_wave;
  const int64_t end = begin + per_wave < routes ? begin + per_wave : routes;
  int32_t *mine = list + wave * per_wave;
  int count = 0;
  for (int64_t c = begin; c < end; c += 4 * kWave) {
    int32_t id[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t route = c + u * kWave + lane;
      const bool held = route < end && route < live;
      if (first != nullptr && c == begin) id[u] = held ? first->id[u] : -1;
      else id[u] = held ? ids[route] : -1;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const bool match = id[u] == want;
      const uint64_t mask = __ballot(match);
      if (match) mine[count + __popcll(mask & ((1ull << lane) - 1))] = static_cast<int32_t>(c + u * kWave + lane);
      count += __popcll(mask);
    }
  }
  if (lane == 0) counts[wave] = count;
  __syncthreads();
  if (threadIdx.x == 0) {
    int total = 0;
    for (int w = 0; w < kWaves; ++w) total += counts[w];
    counts[kWaves] = total;
  }
  __syncthreads();
  return counts[kWaves];
}

/// Local experts a compact grid can tell apart (the fused front end's window bound).
constexpr int kPresentExperts = 512;

/// The n-th smallest local expert that some live route names, or -1 when fewer are named: the
/// workgroup marks the named experts in an LDS bitmap (`bits`, kPresentExperts / 32 words) and
/// every thread counts its way to the n-th mark. Every thread of the workgroup calls it (two
/// barriers) and gets the same answer.
template <int kThreads>
__device__ __forceinline__ int32_t nth_named_expert(const int32_t *ids, int64_t routes, int64_t live, int32_t local_offset,
                                                    int32_t local_experts, int n, uint32_t *bits) {
  constexpr int kWords = kPresentExperts / 32;
  if (threadIdx.x < kWords) bits[threadIdx.x] = 0u;
  __syncthreads();
  const int64_t last = routes < live ? routes : live;
  for (int64_t route = threadIdx.x; route < last; route += kThreads) {
    const int32_t local = ids[route] - local_offset;
    if (local >= 0 && local < local_experts) atomicOr(bits + local / 32, 1u << (local % 32));
  }
  __syncthreads();
  for (int w = 0; w < kWords; ++w) {
    uint32_t word = bits[w];
    const int count = __popc(word);
    if (n >= count) {
      n -= count;
      continue;
    }
    for (; n > 0; --n) word &= word - 1;  // drop the n lowest marks
    return 32 * w + __ffs(static_cast<int>(word)) - 1;
  }
  return -1;
}

/// Row m of the list (m < the total).
template <int kWaves>
__device__ __forceinline__ int64_t listed_route(const int32_t *list, const int32_t *counts, int64_t routes, int m) {
  int w = 0;
  int before = 0;
  while (w + 1 < kWaves && m >= before + counts[w]) before += counts[w++];
  return list[w * routes_per_wave<kWaves>(routes) + (m - before)];
}

}  // namespace uniserve

// SPDX-License-Identifier: Apache-2.0
//
// The sort's parameters and its one-workgroup routine (routes of a decode-sized batch), shared by
// the moe_sort entry (moe_sort.hip) and the layer's fused front end (moe_front.hip).
#pragma once

#include "common.hpp"

namespace uniserve {
namespace sort {

constexpr int kSortThreads = 1024;
constexpr int kSortWaves = kSortThreads / kWave;
constexpr int64_t kChunk = 4096;
constexpr int64_t kMaxLdsBytes = 64 * 1024;

constexpr int kMaxRouteWords = 32;  ///< SortParams::words: a 4096-channel row's 128-channel scales

struct SortParams {
  const int32_t *ids;
  int32_t *tile_to_expert;
  int32_t *tile_to_limit;
  int32_t *expanded_to_permuted;
  int32_t *permuted_to_expanded;
  int32_t *permuted_to_token;
  int32_t *total_padded_tokens;
  int32_t *num_non_exiting_tiles;
  const int32_t *live_tokens;
  int64_t routes;
  int64_t top;
  int32_t local_experts;
  int32_t local_offset;
  int32_t tile;
  int32_t key_bits;  ///< bits of (local expert + 1), the match key
  // Optional, two-launch placement only (the layer's prefill scales): each placed route's row of
  // route_words ([words, word_rows], rows fastest) receives its token's `words` 32-bit words from
  // token_words ([tokens, words], 16-byte aligned rows; words a multiple of 4, at most
  // kMaxRouteWords). Null route_words: nothing.
  const uint32_t *token_words;
  uint32_t *route_words;
  int64_t words;
  int64_t word_rows;
};

/// The local expert of route `route`, or -1 when it is not live or not in the window. kDevice: `ids`
/// read at device scope (stored by other workgroups of the launch).
template <bool kDevice = false>
__device__ __forceinline__ int32_t local_expert(const SortParams &p, int64_t route, int64_t live) {
  if (route >= p.routes || route >= live) return -1;
  const int32_t id = kDevice ? load_device(p.ids + route) : p.ids[route];
  const int64_t local = static_cast<int64_t>(id) - p.local_offset;
  return (local >= 0 && local < p.local_experts) ? static_cast<int32_t>(local) : -1;
}

// ---- the single-workgroup path: up to kChunk routes ---------------------------------------------------
//
// One workgroup, one read of `ids`: wavefront w holds its (at most kSmallGroups) groups of 64
// routes in registers, with their match-any masks, from the count to the placement.
//   1. per-wavefront counts per expert (one LDS update per (wavefront, expert) group);
//   2. thread e sums expert e over the wavefronts, a workgroup scan of the tile counts gives the
//      experts' first rows, and the counts become each wavefront's start rows;
//   3. tile tables and padding rows (a wavefront per expert), then every wavefront places its
//      routes in order.

constexpr int kSmallGroups = static_cast<int>(kChunk / kSortThreads);
constexpr int kSmallMaxExperts = 512;

__host__ __device__ constexpr int64_t small_sort_lds_words(int64_t local_experts) {
  return (kSortWaves + 2) * local_experts + kSortWaves;
}

/// The whole sort by one workgroup of kSortThreads threads; `lds` holds
/// small_sort_lds_words(local experts) words. Without kPadding the padding rows of a tile (past its
/// expert's routes) are left unwritten in permuted_to_expanded and permuted_to_token. kDeviceIds:
/// `ids` read at device scope.
template <bool kPadding, bool kDeviceIds = false>
__device__ __forceinline__ void small_sort(const SortParams &p, int32_t *lds) {
  const int E = p.local_experts;
  int32_t *rows = lds;                          // [kSortWaves][E] counts, then start rows
  int32_t *first_row = rows + kSortWaves * E;   // [E]
  int32_t *total = first_row + E;               // [E]
  int32_t *wave_tiles = total + E;              // [kSortWaves] tiles of each wavefront's experts

  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int lane = lane_id();
  const uint64_t below = (1ull << lane) - 1ull;
  const int64_t live = p.live_tokens == nullptr ? p.routes : static_cast<int64_t>(p.live_tokens[0]) * p.top;
  const int64_t groups = (p.routes + kWave - 1) / kWave;
  const int64_t own = (groups + kSortWaves - 1) / kSortWaves;
  const int64_t first_group = static_cast<int64_t>(wave) * own;

  int32_t e[kSmallGroups];
  uint64_t peers[kSmallGroups];
  bool inside[kSmallGroups];
#pragma unroll
  for (int u = 0; u < kSmallGroups; ++u) {
    const int64_t route = (first_group + u) * kWave + lane;
    inside[u] = u < own && route < p.routes;
    e[u] = inside[u] ? local_expert<kDeviceIds>(p, route, live) : -1;
  }
#pragma unroll
  for (int u = 0; u < kSmallGroups; ++u) peers[u] = match_any(static_cast<uint32_t>(e[u] + 1), p.key_bits);
  for (int i = threadIdx.x; i < kSortWaves * E; i += kSortThreads) rows[i] = 0;
  __syncthreads();

  // 1. This wavefront's counts.
  int32_t *mine = rows + wave * E;
#pragma unroll
  for (int u = 0; u < kSmallGroups; ++u) {
    if (e[u] >= 0 && (peers[u] & below) == 0) mine[e[u]] += __popcll(peers[u]);
    __builtin_amdgcn_wave_barrier();
  }
  __syncthreads();

  // 2. Totals, the scan of the tile counts, the start rows.
  const int ex = static_cast<int>(threadIdx.x);
  int32_t count = 0;
  if (ex < E)
    for (int w = 0; w < kSortWaves; ++w) count += rows[w * E + ex];
  const int32_t tiles = (count + p.tile - 1) / p.tile;
  int32_t inclusive = tiles;
#pragma unroll
  for (int offset = 1; offset < kWave; offset *= 2) {
    const int32_t other = __shfl_up(inclusive, offset);
    if (lane >= offset) inclusive += other;
  }
  if (lane == kWave - 1) wave_tiles[wave] = inclusive;
  __syncthreads();
  int32_t carried = 0;
  for (int w = 0; w < wave; ++w) carried += wave_tiles[w];
  if (ex < E) {
    const int32_t first = (carried + inclusive - tiles) * p.tile;
    first_row[ex] = first;
    total[ex] = count;
    int32_t running = first;
    for (int w = 0; w < kSortWaves; ++w) {
      const int32_t c = rows[w * E + ex];
      rows[w * E + ex] = running;
      running += c;
    }
  }
  if (ex == kSortThreads - 1) {
    p.total_padded_tokens[0] = (carried + inclusive) * p.tile;
    p.num_non_exiting_tiles[0] = carried + inclusive;
  }
  __syncthreads();

  // 3. Tile tables (thread e for expert e) and padding rows (one wavefront per expert); then the
  // placement.
  if (ex < E && count > 0) {
    const int32_t first = (carried + inclusive - tiles) * p.tile;
    const int32_t first_tile = first / p.tile;
    for (int32_t t = 0; t < tiles; ++t) {
      const int32_t end_of_tile = (first_tile + t + 1) * p.tile;
      p.tile_to_expert[first_tile + t] = ex;
      p.tile_to_limit[first_tile + t] = end_of_tile < first + count ? end_of_tile : first + count;
    }
  }
  if constexpr (kPadding) {
    for (int x = wave; x < E; x += kSortWaves) {
      const int32_t n = total[x];
      if (n == 0) continue;
      const int32_t first = first_row[x];
      const int32_t expert_tiles = (n + p.tile - 1) / p.tile;
      for (int32_t row = n + lane; row < expert_tiles * p.tile; row += kWave) {
        p.permuted_to_expanded[first + row] = -1;
        p.permuted_to_token[first + row] = -1;
      }
    }
  }
#pragma unroll
  for (int u = 0; u < kSmallGroups; ++u) {
    const int64_t route = (first_group + u) * kWave + lane;
    if (e[u] >= 0) {
      const int32_t row = mine[e[u]] + __popcll(peers[u] & below);
      p.expanded_to_permuted[route] = row;
      p.permuted_to_expanded[row] = static_cast<int32_t>(route);
      p.permuted_to_token[row] = static_cast<int32_t>(route / p.top);
    } else if (inside[u]) {
      p.expanded_to_permuted[route] = route < live ? -1 : -2;
    }
    __builtin_amdgcn_wave_barrier();
    if (e[u] >= 0 && (peers[u] & below) == 0) mine[e[u]] += __popcll(peers[u]);
    __builtin_amdgcn_wave_barrier();
  }
}

}  // namespace sort

/// The layer's sort above one workgroup's routes, in two launches (count, then the scan folded
/// into the placement) with the per-chunk counts in a scratch table of layer_sort_scratch_bytes
/// that nothing else reads or writes meanwhile; the maps are the moe_sort entry's bit for bit.
/// `counted`: the prefill front end has already written the counts of its chunks of
/// kFrontChunkTokens tokens ([chunks, local experts], the held routes per local expert), and only
/// the placement launches.
constexpr int64_t kFrontChunkTokens = 32;
bool layer_sort_two_launches(int64_t routes, int64_t local_experts);
int64_t layer_sort_scratch_bytes(int64_t tokens, int64_t top, int64_t local_experts);
void launch_layer_sort(const sort::SortParams &p, int32_t *counts, hipStream_t stream, bool counted);

}  // namespace uniserve

// SPDX-License-Identifier: Apache-2.0
//
// moe_sort on gfx950 (operator: crates/ops/src/moe/sort.rs; reference package:
// crates/ops/kernels/moe_sort/trtllm). Groups the held routes of a `tokens x top` routing by local
// expert, each expert's routes in ascending expanded-route order from a tile boundary, and writes
// the tile tables, the three maps and the two counts. Integer work, exact.
//
// Three paths, chosen by the route count R = tokens * top and the local expert count L; none uses
// memory beyond the call's own outputs:
//
//   * small_sort_kernel (R <= 4096, L <= 512; decode): one workgroup reads `ids` once and keeps
//     each wave's routes and match masks in registers from the count to the placement.
//   * sort_count_kernel -> sort_scan_kernel -> sort_place_kernel (R > 4096, L <= 1024; prefill):
//     three launches over 2048-route chunks; the count parks each chunk's per-expert counts in the
//     chunk's own stretch of `expanded_to_permuted`, which only that chunk's placement overwrites.
//   * moe_sort_kernel (the rest: R <= 4096 with 512 < L <= 862; L is capped by 19 counters per
//     expert in 64 KB of LDS, larger windows are refused): one launch; workgroup b owns the chunk
//     [b * kChunk, (b + 1) * kChunk) of the routes and computes everything it needs itself:
//
//   1. count every held route by expert (the totals) and those before its chunk (its base within
//      each expert), reading the whole `ids` vector;
//   2. the tiles per expert and their exclusive scan (workgroup 0 also writes the tile tables, the
//      padding rows and the counts);
//   3. place its chunk: each wavefront owns a contiguous slice, counts it per expert, a scan over
//      the wavefronts turns the counts into starting rows, and the slice is walked again in order.
//
// Routes naming the same expert within one wavefront are found with a ballot per key bit (the
// wave64 form of a match-any), so each (wave, expert) group costs one LDS update and the rank of a
// route within its group is a popcount of the lanes below it - which keeps the order stable.
#include "common.hpp"
#include "sort_small.hpp"
#include "uniserve_moe_sort.h"

namespace uniserve {
namespace {

using namespace sort;

__global__ void __launch_bounds__(kSortThreads) moe_sort_kernel(SortParams p) {
  extern __shared__ int32_t lds[];
  const int E = p.local_experts;
  int32_t *total = lds;                  // [E] held routes per expert
  int32_t *before = total + E;           // [E] held routes per expert before this chunk
  int32_t *first_row = before + E;       // [E] first permuted row of each expert
  int32_t *wave_rows = first_row + E;    // [kSortWaves][E] per-wave counts, then start rows

  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int lane = lane_id();
  const uint64_t below = (1ull << lane) - 1ull;
  const int64_t live = p.live_tokens == nullptr ? p.routes : static_cast<int64_t>(p.live_tokens[0]) * p.top;
  const int64_t chunk_first = static_cast<int64_t>(blockIdx.x) * kChunk;
  const int64_t chunk_past = chunk_first + kChunk < p.routes ? chunk_first + kChunk : p.routes;

  for (int i = threadIdx.x; i < (3 + kSortWaves) * E; i += kSortThreads) lds[i] = 0;
  __syncthreads();

  // 1. Totals and this chunk's bases. kChunk is a multiple of the wavefront, so a group of 64
  //    routes lies wholly before the chunk or not.
  for (int64_t base = static_cast<int64_t>(wave) * kWave; base < p.routes; base += kSortThreads) {
    const int32_t e = local_expert(p, base + lane, live);
    const uint64_t peers = match_any(static_cast<uint32_t>(e + 1), p.key_bits);
    if (e >= 0 && (peers & below) == 0) {
      const int n = __popcll(peers);
      atomicAdd(&total[e], n);
      if (base < chunk_first) atomicAdd(&before[e], n);
    }
  }
  __syncthreads();

  // 2. Each expert's first tile: an exclusive scan of the tile counts by the first wavefront,
  //    64 experts at a time.
  if (wave == 0) {
    int32_t carried = 0;
    for (int first = 0; first < E; first += kWave) {
      const int e = first + lane;
      const int32_t tiles = e < E ? (total[e] + p.tile - 1) / p.tile : 0;
      int32_t inclusive = tiles;
#pragma unroll
      for (int offset = 1; offset < kWave; offset *= 2) {
        const int32_t other = __shfl_up(inclusive, offset);
        if (lane >= offset) inclusive += other;
      }
      if (e < E) first_row[e] = (carried + inclusive - tiles) * p.tile;
      carried += __shfl(inclusive, kWave - 1);
    }
    if (blockIdx.x == 0 && lane == 0) {
      p.total_padded_tokens[0] = carried * p.tile;
      p.num_non_exiting_tiles[0] = carried;
    }
  }
  __syncthreads();

  if (blockIdx.x == 0) {
    // The tile tables and the padding rows of each expert's last tile, one wavefront per expert.
    for (int e = wave; e < E; e += kSortWaves) {
      const int32_t count = total[e];
      if (count == 0) continue;
      const int32_t first = first_row[e];
      const int32_t tiles = (count + p.tile - 1) / p.tile;
      const int32_t first_tile = first / p.tile;
      for (int32_t t = lane; t < tiles; t += kWave) {
        const int32_t end_of_tile = (first_tile + t + 1) * p.tile;
        const int32_t end_of_rows = first + count;
        p.tile_to_expert[first_tile + t] = e;
        p.tile_to_limit[first_tile + t] = end_of_tile < end_of_rows ? end_of_tile : end_of_rows;
      }
      for (int32_t row = count + lane; row < tiles * p.tile; row += kWave) {
        p.permuted_to_expanded[first + row] = -1;
        p.permuted_to_token[first + row] = -1;
      }
    }
  }

  // 3. Place this chunk. Wavefront w owns whole groups of 64 routes, a contiguous slice.
  const int64_t groups = (chunk_past - chunk_first + kWave - 1) / kWave;
  const int64_t own = (groups + kSortWaves - 1) / kSortWaves;
  const int64_t slice_first = chunk_first + static_cast<int64_t>(wave) * own * kWave;
  int64_t slice_past = slice_first + own * kWave;
  if (slice_past > chunk_past) slice_past = chunk_past;
  int32_t *mine = wave_rows + wave * E;

  for (int64_t base = slice_first; base < slice_past; base += kWave) {
    const int64_t route = base + lane;
    const int32_t e = route < slice_past ? local_expert(p, route, live) : -1;
    const uint64_t peers = match_any(static_cast<uint32_t>(e + 1), p.key_bits);
    if (e >= 0 && (peers & below) == 0) mine[e] += __popcll(peers);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += kSortThreads) {
    int32_t running = first_row[e] + before[e];
    for (int w = 0; w < kSortWaves; ++w) {
      const int32_t count = wave_rows[w * E + e];
      wave_rows[w * E + e] = running;
      running += count;
    }
  }
  __syncthreads();

  for (int64_t base = slice_first; base < slice_past; base += kWave) {
    const int64_t route = base + lane;
    const bool inside = route < slice_past;
    const int32_t e = inside ? local_expert(p, route, live) : -1;
    const uint64_t peers = match_any(static_cast<uint32_t>(e + 1), p.key_bits);
    if (e >= 0) {
      const int32_t row = mine[e] + __popcll(peers & below);
      p.expanded_to_permuted[route] = row;
      p.permuted_to_expanded[row] = static_cast<int32_t>(route);
      p.permuted_to_token[row] = static_cast<int32_t>(route / p.top);
    } else if (inside) {
      // -1: a live route of an expert this rank does not hold; -2: a route of a row the batch
      // does not fill (crates/ops/src/moe/sort.rs:15-24).
      p.expanded_to_permuted[route] = route < live ? -1 : -2;
    }
    // Every lane has read its group's start row before the group's first lane advances it.
    __builtin_amdgcn_wave_barrier();
    if (e >= 0 && (peers & below) == 0) mine[e] += __popcll(peers);
    __builtin_amdgcn_wave_barrier();
  }
}

// ---- the single-workgroup path: up to kChunk routes (sort_small.hpp) ------------------------------------

__global__ void __launch_bounds__(kSortThreads) small_sort_kernel(SortParams p) {
  extern __shared__ int32_t lds[];
  small_sort<true>(p, lds);
}

// ---- the split path: more routes than one workgroup places ------------------------------------------
//
// Three launches over chunks of kSplitChunk routes (the last chunk also takes the remainder, so
// every chunk holds at least twice as many routes as there are local experts):
//   count: each chunk's held routes per expert, parked at the head of the chunk's own stretch of
//          `expanded_to_permuted` (which only that chunk's placement overwrites later);
//   scan:  one workgroup turns the parked counts into in-expert offsets, parks the experts' first
//          rows right after them, and writes the tile tables, the padding rows and the two counts;
//   place: each chunk reads its first rows back, then places its routes in order.
// Every launch is wide (one workgroup per chunk) or tiny, instead of one pass that recounts all
// routes per workgroup.

constexpr int kSplitThreads = 512;
constexpr int kSplitWaves = kSplitThreads / kWave;
constexpr int64_t kSplitChunk = 2048;
/// The layer's two-launch sort (counts in a scratch table, no parking) takes smaller chunks: four
/// times the workgroups, each with a quarter of the serial count-and-place walk (30B T=8192: count
/// 6.2 + scan-and-place 17.7 us against 7.3 + 20.0 with 2048-route chunks).
constexpr int64_t kLayerChunk = 512;

template <int64_t kChunkRoutes = kSplitChunk>
__device__ __forceinline__ void split_chunk(const SortParams &p, int64_t *first, int64_t *past) {
  const int64_t chunks = p.routes / kChunkRoutes;
  *first = static_cast<int64_t>(blockIdx.x) * kChunkRoutes;
  *past = static_cast<int64_t>(blockIdx.x) + 1 == chunks ? p.routes : *first + kChunkRoutes;
}

/// Per-wavefront counts of the held routes of [first, past): wavefront w takes the w-th contiguous
/// slice of whole 64-route groups (so a later in-order walk of the slices is stable), counting into
/// its own row of `wave_rows` ([kSplitWaves][E], zero on entry).
__device__ __forceinline__ void split_count(const SortParams &p, int64_t first, int64_t past, int64_t live,
                                            int32_t *wave_rows, int64_t *slice_first, int64_t *slice_past) {
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int lane = lane_id();
  const uint64_t below = (1ull << lane) - 1ull;
  const int64_t groups = (past - first + kWave - 1) / kWave;
  const int64_t own = (groups + kSplitWaves - 1) / kSplitWaves;
  *slice_first = first + static_cast<int64_t>(wave) * own * kWave;
  *slice_past = *slice_first + own * kWave < past ? *slice_first + own * kWave : past;
  int32_t *mine = wave_rows + wave * p.local_experts;
  constexpr int kGroups = 8;  // the wave's ids loads in flight together
  for (int64_t base = *slice_first; base < *slice_past; base += kGroups * kWave) {
    int32_t e[kGroups];
#pragma unroll
    for (int u = 0; u < kGroups; ++u) {
      const int64_t route = base + u * kWave + lane;
      e[u] = route < *slice_past ? local_expert(p, route, live) : -1;
    }
#pragma unroll
    for (int u = 0; u < kGroups; ++u) {
      const uint64_t peers = match_any(static_cast<uint32_t>(e[u] + 1), p.key_bits);
      if (e[u] >= 0 && (peers & below) == 0) mine[e[u]] += __popcll(peers);
      __builtin_amdgcn_wave_barrier();
    }
  }
}

/// `counts` null: each chunk's counts are parked at the head of its stretch of
/// expanded_to_permuted (the entry's three-launch path); else they go to counts[chunk][E].
template <int64_t kChunkRoutes>
__global__ void __launch_bounds__(kSplitThreads) sort_count_kernel(SortParams p, int32_t *counts) {
  extern __shared__ int32_t lds[];
  const int E = p.local_experts;
  int32_t *wave_rows = lds;  // [kSplitWaves][E]
  for (int i = threadIdx.x; i < kSplitWaves * E; i += kSplitThreads) wave_rows[i] = 0;
  __syncthreads();
  const int64_t live = p.live_tokens == nullptr ? p.routes : static_cast<int64_t>(p.live_tokens[0]) * p.top;
  int64_t first, past, slice_first, slice_past;
  split_chunk<kChunkRoutes>(p, &first, &past);
  split_count(p, first, past, live, wave_rows, &slice_first, &slice_past);
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += kSplitThreads) {
    int32_t sum = 0;
    for (int w = 0; w < kSplitWaves; ++w) sum += wave_rows[w * E + e];
    if (counts != nullptr) counts[static_cast<int64_t>(blockIdx.x) * E + e] = sum;
    else p.expanded_to_permuted[first + e] = sum;
  }
}

__global__ void __launch_bounds__(kSortThreads) sort_scan_kernel(SortParams p) {
  extern __shared__ int32_t lds[];
  const int E = p.local_experts;
  int32_t *total = lds;             // [E]
  int32_t *first_row = total + E;   // [E]
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int lane = lane_id();
  const int64_t chunks = p.routes / kSplitChunk;
  constexpr int kBatchChunks = 16;

  // Each expert's running count over the chunks; the parked counts become in-expert offsets.
  for (int e = threadIdx.x; e < E; e += kSortThreads) {
    int32_t running = 0;
    for (int64_t c0 = 0; c0 < chunks; c0 += kBatchChunks) {
      int32_t count[kBatchChunks];
#pragma unroll
      for (int u = 0; u < kBatchChunks; ++u)
        count[u] = c0 + u < chunks ? p.expanded_to_permuted[(c0 + u) * kSplitChunk + e] : 0;
#pragma unroll
      for (int u = 0; u < kBatchChunks; ++u) {
        if (c0 + u < chunks) p.expanded_to_permuted[(c0 + u) * kSplitChunk + e] = running;
        running += count[u];
      }
    }
    total[e] = running;
  }
  __syncthreads();

  // Each expert's first tile: an exclusive scan of the tile counts by the first wavefront.
  if (wave == 0) {
    int32_t carried = 0;
    for (int base = 0; base < E; base += kWave) {
      const int e = base + lane;
      const int32_t tiles = e < E ? (total[e] + p.tile - 1) / p.tile : 0;
      int32_t inclusive = tiles;
#pragma unroll
      for (int offset = 1; offset < kWave; offset *= 2) {
        const int32_t other = __shfl_up(inclusive, offset);
        if (lane >= offset) inclusive += other;
      }
      if (e < E) first_row[e] = (carried + inclusive - tiles) * p.tile;
      carried += __shfl(inclusive, kWave - 1);
    }
    if (lane == 0) {
      p.total_padded_tokens[0] = carried * p.tile;
      p.num_non_exiting_tiles[0] = carried;
    }
  }
  __syncthreads();

  // Tile tables and the padding rows of each expert's last tile, one wavefront per expert.
  for (int e = wave; e < E; e += kSortWaves) {
    const int32_t count = total[e];
    if (count == 0) continue;
    const int32_t first = first_row[e];
    const int32_t tiles = (count + p.tile - 1) / p.tile;
    const int32_t first_tile = first / p.tile;
    for (int32_t t = lane; t < tiles; t += kWave) {
      const int32_t end_of_tile = (first_tile + t + 1) * p.tile;
      const int32_t end_of_rows = first + count;
      p.tile_to_expert[first_tile + t] = e;
      p.tile_to_limit[first_tile + t] = end_of_tile < end_of_rows ? end_of_tile : end_of_rows;
    }
    for (int32_t row = count + lane; row < tiles * p.tile; row += kWave) {
      p.permuted_to_expanded[first + row] = -1;
      p.permuted_to_token[first + row] = -1;
    }
  }

  // Each chunk also gets the experts' first rows, parked right after its offsets (stores only).
  for (int64_t i = threadIdx.x; i < chunks * E; i += kSortThreads) {
    const int64_t c = i / E;
    const int e = static_cast<int>(i - c * E);
    p.expanded_to_permuted[c * kSplitChunk + E + e] = first_row[e];
  }
}

__global__ void __launch_bounds__(kSplitThreads) sort_place_kernel(SortParams p) {
  extern __shared__ int32_t lds[];
  const int E = p.local_experts;
  int32_t *start = lds;              // [E]
  int32_t *wave_rows = start + E;    // [kSplitWaves][E]
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int lane = lane_id();
  const uint64_t below = (1ull << lane) - 1ull;
  const int64_t live = p.live_tokens == nullptr ? p.routes : static_cast<int64_t>(p.live_tokens[0]) * p.top;
  int64_t first, past, slice_first, slice_past;
  split_chunk(p, &first, &past);
  // The chunk's first rows (expert first row plus the chunk's offset, both parked in the chunk's
  // own slots) are read before any of its routes is written over them.
  for (int e = threadIdx.x; e < E; e += kSplitThreads)
    start[e] = p.expanded_to_permuted[first + e] + p.expanded_to_permuted[first + E + e];
  for (int i = threadIdx.x; i < kSplitWaves * E; i += kSplitThreads) wave_rows[i] = 0;
  __syncthreads();
  split_count(p, first, past, live, wave_rows, &slice_first, &slice_past);
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += kSplitThreads) {
    int32_t running = start[e];
    for (int w = 0; w < kSplitWaves; ++w) {
      const int32_t count = wave_rows[w * E + e];
      wave_rows[w * E + e] = running;
      running += count;
    }
  }
  __syncthreads();
  int32_t *mine = wave_rows + wave * E;
  for (int64_t base = slice_first; base < slice_past; base += kWave) {
    const int64_t route = base + lane;
    const bool inside = route < slice_past;
    const int32_t e = inside ? local_expert(p, route, live) : -1;
    const uint64_t peers = match_any(static_cast<uint32_t>(e + 1), p.key_bits);
    if (e >= 0) {
      const int32_t row = mine[e] + __popcll(peers & below);
      p.expanded_to_permuted[route] = row;
      p.permuted_to_expanded[row] = static_cast<int32_t>(route);
      p.permuted_to_token[row] = static_cast<int32_t>(route / p.top);
    } else if (inside) {
      p.expanded_to_permuted[route] = route < live ? -1 : -2;
    }
    __builtin_amdgcn_wave_barrier();
    if (e >= 0 && (peers & below) == 0) mine[e] += __popcll(peers);
    __builtin_amdgcn_wave_barrier();
  }
}

/// The scan folded into the placement (the layer's path: the counts sit in a scratch table that no
/// placement overwrites, so every workgroup reads all of them): each workgroup sums every chunk's
/// counts per expert (the totals) and those of the chunks before its own (its base in each
/// expert), scans the experts' tiles, and places its chunk; workgroup 0 also writes the tile
/// tables, the padding rows and the two counts. Every map entry as the three-launch path writes it.
/// Parts each expert's column of the count table is read in (the workgroup's threads over
/// experts x parts), and the LDS words of the kernel.
__host__ __device__ inline int scan_place_parts(int64_t local_experts) {
  return local_experts >= kSplitThreads ? 1 : static_cast<int>(kSplitThreads / local_experts);
}
inline size_t scan_place_lds_bytes(int64_t local_experts) {
  return static_cast<size_t>((kSplitWaves + 3 + 2 * scan_place_parts(local_experts)) * local_experts) * sizeof(int32_t);
}

/// Chunk b is routes [b chunk_routes, (b + 1) chunk_routes), the last one up to the last route.
__global__ void __launch_bounds__(kSplitThreads) sort_scan_place_kernel(SortParams p, const int32_t *counts,
                                                                        int64_t chunk_routes, int64_t chunks) {
  extern __shared__ int32_t lds[];
  const int E = p.local_experts;
  const int parts = scan_place_parts(E);
  int32_t *start = lds;              // [E] this chunk's first row in each expert
  int32_t *wave_rows = start + E;    // [kSplitWaves][E]
  int32_t *total = wave_rows + kSplitWaves * E;   // [E]
  int32_t *first_row = total + E;                 // [E]
  int32_t *part_total = first_row + E;            // [parts][E]
  int32_t *part_before = part_total + parts * E;  // [parts][E]
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int lane = lane_id();
  const uint64_t below = (1ull << lane) - 1ull;
  const int64_t live = p.live_tokens == nullptr ? p.routes : static_cast<int64_t>(p.live_tokens[0]) * p.top;
  const int64_t own = blockIdx.x;
  constexpr int kBatchChunks = 16;

  // Each expert's column of counts in `parts` contiguous runs of chunks, one thread a run.
  for (int i = threadIdx.x; i < E * parts; i += kSplitThreads) {
    const int e = i % E, part = i / E;
    const int64_t c_begin = chunks * part / parts, c_end = chunks * (part + 1) / parts;
    int32_t running = 0, before = 0;
    for (int64_t c0 = c_begin; c0 < c_end; c0 += kBatchChunks) {
      int32_t count[kBatchChunks];
#pragma unroll
      for (int u = 0; u < kBatchChunks; ++u) count[u] = c0 + u < c_end ? counts[(c0 + u) * E + e] : 0;
#pragma unroll
      for (int u = 0; u < kBatchChunks; ++u) {
        if (c0 + u < own) before += count[u];
        running += count[u];
      }
    }
    part_total[part * E + e] = running;
    part_before[part * E + e] = before;
  }
  for (int i = threadIdx.x; i < kSplitWaves * E; i += kSplitThreads) wave_rows[i] = 0;
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += kSplitThreads) {
    int32_t running = 0, before = 0;
    for (int part = 0; part < parts; ++part) {
      running += part_total[part * E + e];
      before += part_before[part * E + e];
    }
    total[e] = running;
    start[e] = before;
  }
  __syncthreads();

  if (wave == 0) {
    int32_t carried = 0;
    for (int base = 0; base < E; base += kWave) {
      const int e = base + lane;
      const int32_t tiles = e < E ? (total[e] + p.tile - 1) / p.tile : 0;
      int32_t inclusive = tiles;
#pragma unroll
      for (int offset = 1; offset < kWave; offset *= 2) {
        const int32_t other = __shfl_up(inclusive, offset);
        if (lane >= offset) inclusive += other;
      }
      if (e < E) first_row[e] = (carried + inclusive - tiles) * p.tile;
      carried += __shfl(inclusive, kWave - 1);
    }
    if (blockIdx.x == 0 && lane == 0) {
      p.total_padded_tokens[0] = carried * p.tile;
      p.num_non_exiting_tiles[0] = carried;
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += kSplitThreads) start[e] += first_row[e];

  {
    // Tile tables and the padding rows of each expert's last tile, one wavefront per expert, the
    // experts spread over every workgroup's wavefronts (all of them hold the totals and first
    // rows): in workgroup 0 alone this was the launch's tail (30B T=8192 scan-and-place
    // 16.7 -> 11.4 us).
    for (int e = static_cast<int>(blockIdx.x) * kSplitWaves + wave; e < E; e += static_cast<int>(gridDim.x) * kSplitWaves) {
      const int32_t count = total[e];
      if (count == 0) continue;
      const int32_t first = first_row[e];
      const int32_t tiles = (count + p.tile - 1) / p.tile;
      const int32_t first_tile = first / p.tile;
      for (int32_t t = lane; t < tiles; t += kWave) {
        const int32_t end_of_tile = (first_tile + t + 1) * p.tile;
        const int32_t end_of_rows = first + count;
        p.tile_to_expert[first_tile + t] = e;
        p.tile_to_limit[first_tile + t] = end_of_tile < end_of_rows ? end_of_tile : end_of_rows;
      }
      for (int32_t row = count + lane; row < tiles * p.tile; row += kWave) {
        p.permuted_to_expanded[first + row] = -1;
        p.permuted_to_token[first + row] = -1;
      }
    }
  }

  int64_t first, past, slice_first, slice_past;
  first = own * chunk_routes;
  past = own + 1 == chunks ? p.routes : first + chunk_routes;
  split_count(p, first, past, live, wave_rows, &slice_first, &slice_past);
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += kSplitThreads) {
    int32_t running = start[e];
    for (int w = 0; w < kSplitWaves; ++w) {
      const int32_t count = wave_rows[w * E + e];
      wave_rows[w * E + e] = running;
      running += count;
    }
  }
  __syncthreads();
  int32_t *mine = wave_rows + wave * E;
  const int quads = static_cast<int>(p.words / 4);
  for (int64_t base = slice_first; base < slice_past; base += kWave) {
    const int64_t route = base + lane;
    const bool inside = route < slice_past;
    // The route's token words, issued before its id is read (a clamped token past the slice).
    u32x4 token_words[kMaxRouteWords / 4];
    if (p.route_words != nullptr) {
      const u32x4 *from = reinterpret_cast<const u32x4 *>(p.token_words + ((inside ? route : slice_first) / p.top) * p.words);
#pragma unroll
      for (int q = 0; q < kMaxRouteWords / 4; ++q)
        if (q < quads) token_words[q] = from[q];
    }
    const int32_t e = inside ? local_expert(p, route, live) : -1;
    const uint64_t peers = match_any(static_cast<uint32_t>(e + 1), p.key_bits);
    if (e >= 0) {
      const int32_t row = mine[e] + __popcll(peers & below);
      p.expanded_to_permuted[route] = row;
      p.permuted_to_expanded[row] = static_cast<int32_t>(route);
      p.permuted_to_token[row] = static_cast<int32_t>(route / p.top);
      if (p.route_words != nullptr) {
#pragma unroll
        for (int q = 0; q < kMaxRouteWords / 4; ++q)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (q < quads) p.route_words[(4 * q + j) * p.word_rows + row] = token_words[q][j];
      }
    } else if (inside) {
      p.expanded_to_permuted[route] = route < live ? -1 : -2;
    }
    __builtin_amdgcn_wave_barrier();
    if (e >= 0 && (peers & below) == 0) mine[e] += __popcll(peers);
    __builtin_amdgcn_wave_barrier();
  }
}

}  // namespace

bool layer_sort_two_launches(int64_t routes, int64_t local_experts) {
  return routes > sort::kChunk && 2 * local_experts <= kSplitChunk;
}

int64_t layer_sort_scratch_bytes(int64_t tokens, int64_t top, int64_t local_experts) {
  const int64_t counted = tokens * top / kLayerChunk;                 // the count launch's chunks
  const int64_t front = ceil_div<int64_t>(tokens, kFrontChunkTokens);  // the prefill front end's
  return (counted > front ? counted : front) * local_experts * static_cast<int64_t>(sizeof(int32_t));
}

void launch_layer_sort(const sort::SortParams &p, int32_t *counts, hipStream_t stream, bool counted) {
  // The prefill front end counts its own chunks (kFrontChunkTokens tokens each); otherwise the
  // count launch does, over kLayerChunk routes.
  const int64_t chunk_routes = counted ? kFrontChunkTokens * p.top : kLayerChunk;
  const int64_t chunks = counted ? ceil_div<int64_t>(p.routes, chunk_routes) : p.routes / kLayerChunk;
  const size_t count_bytes = kSplitWaves * p.local_experts * sizeof(int32_t);
  if (!counted)
    hipLaunchKernelGGL((sort_count_kernel<kLayerChunk>), dim3(static_cast<uint32_t>(chunks)), dim3(kSplitThreads),
                       count_bytes, stream, p, counts);
  hipLaunchKernelGGL(sort_scan_place_kernel, dim3(static_cast<uint32_t>(chunks)), dim3(kSplitThreads),
                     scan_place_lds_bytes(p.local_experts), stream, p, static_cast<const int32_t *>(counts), chunk_routes,
                     chunks);
}

}  // namespace uniserve

extern "C" int32_t uniserve_moe_sort(const uniserve_moe_sort_call *call, void *stream) {
  using namespace uniserve;
  return guarded(call, [&]() -> int32_t {
    // The refusals of the reference entry (crates/ops/kernels/moe_sort/trtllm/src/entry.cpp:26-70).
    if (call->ids == nullptr || call->tile_to_expert == nullptr || call->tile_to_limit == nullptr ||
        call->expanded_to_permuted == nullptr || call->permuted_to_expanded == nullptr ||
        call->permuted_to_token == nullptr || call->total_padded_tokens == nullptr ||
        call->num_non_exiting_tiles == nullptr)
      return UNISERVE_REFUSE(call, "moe_sort needs the router's ids and all seven metadata buffers");
    if (call->scales_dtype != UNISERVE_DTYPE_F32 && call->scales_dtype != UNISERVE_DTYPE_BF16 &&
        call->scales_dtype != UNISERVE_DTYPE_F16)
      return UNISERVE_REFUSE(call, "moe_sort serves f32, bf16 or fp16 route weights");
    if (call->tokens < 0 || call->top < 0 || call->experts <= 0 || call->local_experts <= 0 ||
        call->tile_tokens <= 0)
      return UNISERVE_REFUSE(call, "moe_sort needs a non-negative route count and positive experts, local experts and tile");
    if (call->local_offset < 0 || call->local_offset + call->local_experts > call->experts)
      return UNISERVE_REFUSE(call, "moe_sort's local expert window lies outside the router's experts");
    if (call->tokens * call->top > 0x7fffffffLL)
      return UNISERVE_REFUSE(call, "moe_sort's expanded routes do not fit the metadata's int32 indexes");
    const int64_t lds_bytes = (3 + kSortWaves) * call->local_experts * static_cast<int64_t>(sizeof(int32_t));
    if (lds_bytes > kMaxLdsBytes)
      return UNISERVE_REFUSE(call, "moe_sort's expert count outgrows one workgroup's LDS (%lld local experts)",
                             static_cast<long long>(call->local_experts));

    SortParams p{};
    p.ids = call->ids;
    p.tile_to_expert = call->tile_to_expert;
    p.tile_to_limit = call->tile_to_limit;
    p.expanded_to_permuted = call->expanded_to_permuted;
    p.permuted_to_expanded = call->permuted_to_expanded;
    p.permuted_to_token = call->permuted_to_token;
    p.total_padded_tokens = call->total_padded_tokens;
    p.num_non_exiting_tiles = call->num_non_exiting_tiles;
    p.live_tokens = call->live_tokens;
    p.routes = call->tokens * call->top;
    p.top = call->top;
    p.local_experts = static_cast<int32_t>(call->local_experts);
    p.local_offset = static_cast<int32_t>(call->local_offset);
    p.tile = static_cast<int32_t>(call->tile_tokens);
    int bits = 0;
    while ((1ll << bits) <= call->local_experts) ++bits;
    p.key_bits = bits;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (p.routes <= kChunk && p.local_experts <= kSmallMaxExperts) {
      const size_t bytes = small_sort_lds_words(call->local_experts) * sizeof(int32_t);
      hipLaunchKernelGGL(small_sort_kernel, dim3(1), dim3(kSortThreads), bytes, s, p);
      return launched(call, "moe_sort");
    }
    if (p.routes <= kChunk || 2 * p.local_experts > kSplitChunk) {
      const int64_t chunks = p.routes == 0 ? 1 : ceil_div<int64_t>(p.routes, kChunk);
      hipLaunchKernelGGL(moe_sort_kernel, dim3(static_cast<uint32_t>(chunks)), dim3(kSortThreads),
                         static_cast<size_t>(lds_bytes), s, p);
      return launched(call, "moe_sort");
    }
    const uint32_t chunks = static_cast<uint32_t>(p.routes / kSplitChunk);
    const size_t count_bytes = kSplitWaves * call->local_experts * sizeof(int32_t);
    hipLaunchKernelGGL((sort_count_kernel<kSplitChunk>), dim3(chunks), dim3(kSplitThreads), count_bytes, s, p, nullptr);
    hipLaunchKernelGGL(sort_scan_kernel, dim3(1), dim3(kSortThreads), 2 * call->local_experts * sizeof(int32_t), s, p);
    hipLaunchKernelGGL(sort_place_kernel, dim3(chunks), dim3(kSplitThreads), count_bytes + call->local_experts * sizeof(int32_t),
                       s, p);
    return launched(call, "moe_sort");
  });
}

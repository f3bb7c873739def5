// SPDX-License-Identifier: Apache-2.0
//
// The two grouped expert products in bf16 on gfx950 MFMA (operators: crates/ops/src/moe/grouped.rs;
// reference packages: crates/ops/kernels/{gather_gemm,route_gemm}/cute_dsl):
//
//   gather_gemm (FC1)  out[p, :I] = silu(W[e, I:2I] . x[t]) * (W[e, :I] . x[t])
//   route_gemm  (FC2)  out[p, :H] = W[e] . rows[p]
//
// for every live permuted row p (below its tile's `tile_to_limit`) of every tile below
// `num_non_exiting_tiles`, e = tile_to_expert[tile], t = permuted_to_expanded[p] / top. FP32
// accumulation, the activation on the accumulators, one rounding into bf16; rows past a tile's
// limit are neither read nor stored.
//
// Three kernels per product, chosen on the host from the expected rows per expert (tokens x top /
// experts), which is all the host knows without reading device memory, and from the shape:
//
//  * `stream` (decode: a few rows per expert). Weight-streaming bound: every touched expert's
//    matrix is read once from HBM and nothing else matters. A workgroup owns one tile and a
//    128-row slice of the expert's weight rows; each wavefront streams its 32 weight rows as whole
//    non-temporal 128-byte lines into registers and regroups them into the MFMA operand layout
//    through its own LDS buffer, the tile's activation rows coming from L2. The weight rows are MFMA
//    operand A and the activation rows operand B (16x16x32 bf16), so each lane ends holding four
//    consecutive output columns of one row - an 8-byte store - and the SiLU pair (up column n,
//    gate column n) meets in one lane. Tiles of more than 32 rows are covered in passes of 32.
//
//  * `prefill` (grouped_prefill.hpp; hundreds of rows per expert): 128 x 512 tiles of 8
//    wavefronts, both operands DMA'd into LDS, for the shapes it serves.
//
//  * `tiled` (prefill shapes the prefill kernel does not serve): a 128 x 128 output tile per
//    workgroup, 64-deep K steps staged through XOR-swizzled LDS (two stages, one barrier per step),
//    four wavefronts of 64 x 64, global loads of step k + 1 in flight during the MFMAs of step k.
//
// The dot products over K use a permutation of K that both operands share, which changes only the
// FP32 summation order.
#include "common.hpp"
#include "grouped_pair.hpp"
#include "expert_routes.hpp"
#include "expert_stream.hpp"
#include "grouped_prefill.hpp"
#include "uniserve_gather_gemm.h"
#include "uniserve_route_gemm.h"

namespace uniserve {
namespace {

constexpr int kTileRows = 128;
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

struct GroupedParams {
  const uint16_t *act;      ///< FC1: hidden [tokens, K]; FC2: rows [permuted_rows, K]
  const uint16_t *weights;  ///< [experts, n_total, K]
  uint16_t *out;            ///< [permuted_rows, out_width]
  const int32_t *tile_to_expert;
  const int32_t *tile_to_limit;
  const int32_t *permuted_to_expanded;
  const int32_t *num_tiles;
  int64_t K;
  int64_t n_total;          ///< weight rows per expert: 2I (FC1) or H (FC2)
  int64_t out_width;        ///< I (FC1) or H (FC2)
  int64_t top;
  int32_t activation;       ///< FC1's gate: UNISERVE_ACTIVATION_SILU or _GELU_TANH
  // Expert-major stream (decode, no sort): workgroup x serves local expert x; its rows are the
  // routes naming it, found in `ids`, in route order, at their expanded positions.
  const int32_t *ids;       ///< [routes] expert ids (after the slot map)
  const int32_t *live_tokens;
  int64_t routes;
  int64_t local_offset;
  int64_t local_experts;
  int32_t compact;          ///< workgroup x serves the x-th named local expert (fewer routes than experts)
};

__device__ __forceinline__ u32x4 load16(const uint16_t *pointer) {
  return *reinterpret_cast<const u32x4 *>(pointer);
}

__device__ __forceinline__ void store_bf16x4(uint16_t *pointer, floatx4 v) {
  uint2 packed;
  packed.x = pack_bf16x2(v[0], v[1]);
  packed.y = pack_bf16x2(v[2], v[3]);
  *reinterpret_cast<uint2 *>(pointer) = packed;
}

// ---- stream kernel (decode) ----------------------------------------------------------------------------

/// Average routes per expert at or below which the stream kernel takes a tile in passes of one
/// 16-row MFMA block instead of two (at 64-token decode: FC2 63.7 against 66.2 us with two, FC1
/// 124 against 125); a tile with more rows re-streams its weights per pass, which at such
/// averages is rare.
constexpr int64_t kOnePassRowsPerExpert = 8;

//
// Grid: (max tiles, weight-row slices). FC1 slices are 64 gated columns (64 up + 64 gate rows),
// FC2 slices 128 output columns; wavefront w takes 16 + 16 of them. Needs K % 128 == 0.
//
// The weight stream is read as whole 128-byte lines: a load instruction covers 8 rows x 128 bytes
// (eight lanes per row), marked non-temporal since every weight line is read once per call - which
// lets HBM run near its streaming rate (loads in the MFMA operand layout consume each line over
// four instructions, and reach about 0.70 of the peak against 0.78). The lines are redistributed
// into the MFMA operand layout (lane l: row l % 16) through an 8 KB LDS buffer per wavefront
// (written and read back by the wave itself, no barrier). A stage is 256 bytes of K per row (two
// lines, 128 bf16): eight line loads per wavefront for its 32 weight rows.
//
// K mapping (the same for weights and activations): step s in 0..3 of a stage, lane group
// g = l / 16 takes the stage's 16-byte chunk 4 s + g, i.e. line s / 2, chunk 4 (s % 2) + g.

/// kPassTiles: rows of a tile one pass covers, in MFMA blocks of 16.
/// kByExpert: workgroup x serves local expert x (grid: local experts x slices) and finds its rows
/// itself - the routes whose id is the expert's, in route order, live ones only (each wavefront
/// ballots a quarter of the routes into a list in LDS) - while its first weight stage is in
/// flight; FC1 reads token route / top and FC2 row `route`, and both write row `route` (the
/// expanded layout). Otherwise the sort's tile tables give the tile's expert and rows.
template <bool kGated, int kPassTiles, bool kByExpert = false>
__global__ void __launch_bounds__(kThreads) stream_kernel(GroupedParams p) {
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int lane = lane_id();
  const int r16 = lane & 15;
  const int g = lane >> 4;
  int64_t expert, first;
  int rows;
  if constexpr (kByExpert) {
    first = 0;
    rows = 0;
    expert = blockIdx.x;
    if (p.compact) {
      __shared__ uint32_t named[kPresentExperts / 32];
      const int64_t live = p.live_tokens != nullptr ? static_cast<int64_t>(p.live_tokens[0]) * p.top : p.routes;
      expert = nth_named_expert<kThreads>(p.ids, p.routes, live, static_cast<int32_t>(p.local_offset),
                                          static_cast<int32_t>(p.local_experts), static_cast<int>(blockIdx.x), named);
      if (expert < 0) return;
    }
  } else {
    const int tile = static_cast<int>(blockIdx.x);
    if (tile >= p.num_tiles[0]) return;
    expert = p.tile_to_expert[tile];
    first = static_cast<int64_t>(tile) * kTileRows;
    rows = p.tile_to_limit[tile] - static_cast<int>(first);
  }

  int64_t n0, n1;
  if constexpr (kGated) {
    n0 = static_cast<int64_t>(blockIdx.y) * 64 + wave * 16;
    n1 = p.out_width + n0;
  } else {
    n0 = static_cast<int64_t>(blockIdx.y) * 128 + wave * 32;
    n1 = n0 + 16;
    if (!kByExpert && n0 >= p.out_width) return;  // (expert-major FC2: whole 128-column slices)
  }
  // Line load i of a stage (i = 0..7): line i / 4 of rows 8 (i % 4) + l / 8 of the wave's 32 (set
  // 0 = rows n0.., set 1 = rows n1..), 16-byte chunk l % 8.
  const uint16_t *line_row[2];
  line_row[0] = p.weights + (expert * p.n_total + n0 + lane / 8) * p.K + (lane & 7) * 8;
  line_row[1] = p.weights + (expert * p.n_total + n1 + lane / 8) * p.K + (lane & 7) * 8;
  // Fragment (set, s): lane l takes row r16 of the set from line load 4 (s / 2) + 2 set + r16 / 8,
  // lane 8 (r16 % 8) + 4 (s % 2) + g - through the wave's own LDS buffer: load i's lane l (row
  // l / 8 of the load, piece l % 8) goes to slot 64 i + 8 r + (piece ^ r), r = l / 8, so the lanes
  // that read one piece of eight rows read eight different bank groups. (Against ds_bpermute from
  // both candidate loads and a select: 30B T=64 FC1 125.3 -> 123.8 us, FC2 66.9 -> 65.7, the layer
  // 213 -> 206.5.)
  const int stages = static_cast<int>(p.K / 128);

  struct Stage {
    u32x4 lines[8];
    u32x4 act[kPassTiles][4];
  };
  auto load_lines = [&](Stage &st, int64_t k) {
    const int64_t offset = k * 128;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int set = (i % 4) / 2;
      const int64_t row_offset = static_cast<int64_t>((i % 4) % 2) * 8 * p.K;
      st.lines[i] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4 *>(line_row[set] + row_offset + offset + (i / 4) * 64));
    }
  };
  Stage even, odd;
  FirstRouteIds first_ids;
  if constexpr (kByExpert) {
    first_ids = load_first_route_ids<kWaves>(p.ids, p.routes);
    load_lines(even, 0);  // no dependence on the routes: out before the scan (after the ids it reads)
  }

  __shared__ u32x4 regroup[kWaves][8 * 64];  // each wave's weight lines of a stage, regrouped
  // Expert-major: the route list (route order), found while the first weight stage is in flight.
  __shared__ int32_t route_list[kByExpert ? kExpertRoutes : 1];
  __shared__ int32_t wave_count[kWaves + 1];
  if constexpr (kByExpert) {
    const int64_t live = p.live_tokens != nullptr ? static_cast<int64_t>(p.live_tokens[0]) * p.top : p.routes;
    rows = list_expert_routes<kWaves>(p.ids, p.routes, live, static_cast<int32_t>(expert + p.local_offset),
                                      route_list, wave_count, &first_ids);
    if (rows == 0) return;
  }
  auto listed = [&](int m) -> int64_t { return listed_route<kWaves>(route_list, wave_count, p.routes, m); };

  for (int pass = 0; pass < rows; pass += 16 * kPassTiles) {
    const uint16_t *a[kPassTiles];
    bool valid[kPassTiles];
#pragma unroll
    for (int ms = 0; ms < kPassTiles; ++ms) {
      const int m = pass + ms * 16 + r16;
      valid[ms] = m < rows;
      int64_t source = first + m;
      if constexpr (kByExpert) {
        source = valid[ms] ? listed(m) : 0;
        if constexpr (kGated) source /= p.top;
      } else if constexpr (kGated) {
        source = valid[ms] ? p.permuted_to_expanded[first + m] / p.top : 0;
      }
      a[ms] = p.act + (valid[ms] ? source : 0) * p.K + g * 8;
    }
    floatx4 acc[2][kPassTiles];
#pragma unroll
    for (int set = 0; set < 2; ++set)
#pragma unroll
      for (int ms = 0; ms < kPassTiles; ++ms) acc[set][ms] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    auto load_act = [&](Stage &st, int64_t k) {
      const int64_t offset = k * 128;
#pragma unroll
      for (int ms = 0; ms < kPassTiles; ++ms)
#pragma unroll
        for (int s = 0; s < 4; ++s)
          st.act[ms][s] = load16(a[ms] + offset + s * 32);  // (rows past the tile: row 0, never stored)
    };
    auto load = [&](Stage &st, int64_t k) {
      load_lines(st, k);
      load_act(st, k);
    };
    auto compute = [&](const Stage &st) {
      {
        const int row = lane >> 3, piece = lane & 7;
#pragma unroll
        for (int i = 0; i < 8; ++i) regroup[wave][i * 64 + row * 8 + (piece ^ row)] = st.lines[i];
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) {
#pragma unroll
        for (int set = 0; set < 2; ++set) {
          const int i = 4 * (s / 2) + 2 * set + (r16 >> 3);
          const int rr = r16 & 7, q = 4 * (s & 1) + g;
          const u32x4 w = regroup[wave][i * 64 + rr * 8 + (q ^ rr)];
#pragma unroll
          for (int ms = 0; ms < kPassTiles; ++ms) acc[set][ms] = mfma_16x16x32_bf16(w, st.act[ms][s], acc[set][ms]);
        }
      }
    };
    if (kByExpert && pass == 0) load_act(even, 0);  // its weight lines went out before the route scan
    else load(even, 0);
    // The steady walk issues both loads unconditionally, so the compiler's wait before each
    // compute counts exactly the other stage's loads still in flight (with the loads under
    // conditions it waited for every load, the prefetched stage's too); the last one or two
    // stages are peeled.
    int k = 0;
    for (; k + 2 < stages; k += 2) {
      load(odd, k + 1);
      compute(even);
      load(even, k + 2);
      compute(odd);
    }
    if (k + 1 < stages) {
      load(odd, k + 1);
      compute(even);
      compute(odd);
    } else {
      compute(even);
    }

#pragma unroll
    for (int ms = 0; ms < kPassTiles; ++ms) {
      const int m = pass + ms * 16 + r16;
      if (m >= rows) continue;
      uint16_t *row = p.out + (kByExpert ? listed(m) : first + m) * p.out_width;
      if constexpr (kGated) {
        floatx4 h;
#pragma unroll
        for (int i = 0; i < 4; ++i) h[i] = gate(acc[1][ms][i], p.activation) * acc[0][ms][i];
        store_bf16x4(row + n0 + 4 * g, h);
      } else {
        store_bf16x4(row + n0 + 4 * g, acc[0][ms]);
        store_bf16x4(row + n1 + 4 * g, acc[1][ms]);
      }
    }
  }
}

// ---- quarter kernel (decode, expert-major) ----------------------------------------------------------------
//
// FC1's gated product with the workgroup's 128 weight rows (64 up + the matching 64 gate rows)
// streamed by every wavefront over its own quarter of K: wavefront q walks K
// lines q K / 256 .. (q + 1) K / 256 - 1 (64 bf16 each) of all 128 rows, one step = one line of 64
// rows (8 instructions of 8 rows x 128 bytes), the two halves of the rows in turn. At any moment
// the workgroup's four wavefronts read four neighbouring stretches of the same rows, which DRAM
// serves from fewer row openings than the row-sliced walk, where each wavefront reads 256 bytes of
// its own rows per stage (a bare kernel reading FC1's weights: 7.2 against 6.3 TB/s). Each
// wavefront holds partial sums of all 128 rows; at the end they meet in LDS and wavefront w adds
// the four in wave order for its output rows (up set w and gate set w + 4: 16 gated columns).
// FC1 from 124 to 120 us at 30B T=64; FC2 (128 rows of one kind) measured 1 us slower, so it keeps
// the row-sliced kernel. Needs K % 256 == 0 and byte offsets of an expert's weights and of the
// activations below 2^32.
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3))) quarter_kernel(GroupedParams p) {
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int lane = lane_id();
  const int r16 = lane & 15;
  const int g = lane >> 4;
  int64_t expert = blockIdx.x;
  if (p.compact) {
    __shared__ uint32_t named[kPresentExperts / 32];
    const int64_t live = p.live_tokens != nullptr ? static_cast<int64_t>(p.live_tokens[0]) * p.top : p.routes;
    expert = nth_named_expert<kThreads>(p.ids, p.routes, live, static_cast<int32_t>(p.local_offset),
                                        static_cast<int32_t>(p.local_experts), static_cast<int>(blockIdx.x), named);
    if (expert < 0) return;
  }
  // Row r (0..127) of the workgroup: up row slice * 64 + r, or gate row I + slice * 64 + r - 64.
  const int64_t slice = blockIdx.y;
  auto weight_row = [&](int r) -> int64_t { return r < 64 ? slice * 64 + r : p.out_width + slice * 64 + (r - 64); };
  const int lines = static_cast<int>(p.K / 64);       // 128-byte lines per row
  const int per_wave = lines / kWaves;                // this wavefront's lines: [wave * per_wave, ..)
  const int steps = 2 * per_wave;                     // (line, half of the rows)
  // Step t: line wave * per_wave + t / 2 of rows 64 (t % 2) + 8 i + l / 8, chunk l % 8. The rows of
  // a half are consecutive, so load i's address is a uniform base (the expert's stack, 8 i rows on,
  // the step's line) plus one 32-bit lane offset per half: few registers per address.
  expert = __builtin_amdgcn_readfirstlane(static_cast<int>(expert));
  const uint8_t *wbase = reinterpret_cast<const uint8_t *>(p.weights + expert * p.n_total * p.K);
  const int64_t row_bytes = p.K * 2;
  uint32_t half_off[2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
    half_off[h] = static_cast<uint32_t>(weight_row(64 * h + lane / 8) * row_bytes + wave * per_wave * 128 + (lane & 7) * 16);
  struct Step {
    u32x4 lines[8];
  };
  auto load_step = [&](Step &st, int t) {
    const int h = t & 1;
    const uint8_t *line = wbase + static_cast<int64_t>(t >> 1) * 128;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      st.lines[i] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4 *>(line + static_cast<int64_t>(i) * 8 * row_bytes + half_off[h]));
  };
  Step even, odd;
  const FirstRouteIds first_ids = load_first_route_ids<kWaves>(p.ids, p.routes);
  load_step(even, 0);  // no dependence on the routes: out before the scan (after the ids it reads)

  __shared__ u32x4 regroup[kWaves][8 * 64];
  __shared__ int32_t route_list[kExpertRoutes];
  __shared__ int32_t wave_count[kWaves + 1];
  const int64_t live = p.live_tokens != nullptr ? static_cast<int64_t>(p.live_tokens[0]) * p.top : p.routes;
  const int rows = list_expert_routes<kWaves>(p.ids, p.routes, live, static_cast<int32_t>(expert + p.local_offset),
                                              route_list, wave_count, &first_ids);
  if (rows == 0) return;
  auto listed = [&](int m) -> int64_t { return listed_route<kWaves>(route_list, wave_count, p.routes, m); };

  for (int pass = 0; pass < rows; pass += 16) {
    const int m = pass + r16;
    const bool valid = m < rows;
    const int64_t source = valid ? listed(m) / p.top : 0;
    // Rows past the expert's routes read row 0 (never stored).
    const uint32_t a_off = static_cast<uint32_t>((source * p.K + static_cast<int64_t>(wave) * per_wave * 64 + g * 8) * 2);
    const uint8_t *act = reinterpret_cast<const uint8_t *>(p.act);
    floatx4 acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    u32x4 x[2][2];  // [line parity][K step of 32]: this lane's 8 elements of each
    auto load_x = [&](int line, u32x4 (&into)[2]) {
      into[0] = *reinterpret_cast<const u32x4 *>(act + static_cast<int64_t>(line) * 128 + a_off);
      into[1] = *reinterpret_cast<const u32x4 *>(act + static_cast<int64_t>(line) * 128 + 64 + a_off);
    };
    auto compute = [&](const Step &st, int t, const u32x4 (&xs)[2]) {
      {
        const int row = lane >> 3, piece = lane & 7;
#pragma unroll
        for (int i = 0; i < 8; ++i) regroup[wave][i * 64 + row * 8 + (piece ^ row)] = st.lines[i];
      }
      const int h = t & 1;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int i = 2 * j + (r16 >> 3), rr = r16 & 7, q = 4 * ks + g;
          const u32x4 w = regroup[wave][i * 64 + rr * 8 + (q ^ rr)];
          acc[4 * h + j] = mfma_16x16x32_bf16(w, xs[ks], acc[4 * h + j]);
        }
    };
    if (pass > 0) load_step(even, 0);
    load_x(0, x[0]);
    // Steps in pairs (both halves of one line); the next pair's loads go out before this pair's
    // computes wait, all unconditionally in the steady walk.
    int t = 0;
    for (; t + 2 < steps; t += 2) {
      load_step(odd, t + 1);
      load_x((t >> 1) + 1, x[1]);
      compute(even, t, x[0]);
      load_step(even, t + 2);
      compute(odd, t + 1, x[0]);
      x[0][0] = x[1][0];
      x[0][1] = x[1][1];
    }
    load_step(odd, t + 1);
    compute(even, t, x[0]);
    compute(odd, t + 1, x[0]);

    // The four quarters' partial sums, added in wave order; each wavefront's go through its own
    // regroup buffer (8 x 64 floatx4, the buffer's size), which it no longer reads.
    auto partial = [&](int w, int j) -> floatx4 & { return reinterpret_cast<floatx4 *>(regroup[w])[j * kWave + lane]; };
#pragma unroll
    for (int j = 0; j < 8; ++j) partial(wave, j) = acc[j];
    __syncthreads();
    floatx4 up = partial(0, wave), gated = partial(0, wave + 4);
#pragma unroll
    for (int w = 1; w < kWaves; ++w) {
      up += partial(w, wave);
      gated += partial(w, wave + 4);
    }
    __syncthreads();  // the next pass regroups over the partial sums
    if (valid) {
      floatx4 hv;
#pragma unroll
      for (int i = 0; i < 4; ++i) hv[i] = gate(gated[i], p.activation) * up[i];
      store_bf16x4(p.out + listed(m) * p.out_width + slice * 64 + wave * 16 + 4 * g, hv);
    }
  }
}

// ---- tiled kernel -----------------------------------------------------------------------------------------

constexpr int kBK = 64;               // K elements per stage: 8 chunks of 16 bytes per row
constexpr int kStageChunks = 128 * 8; // 16-byte chunks per operand per stage

__device__ __forceinline__ int swizzled(int row, int chunk) { return row * 8 + (chunk ^ (row & 7)); }

/// Grid: (max tiles, weight-row slices of 128: FC1 64 up + 64 gate rows, FC2 128 rows).
/// Needs K % 64 == 0.
template <bool kGated>
__global__ void __launch_bounds__(kThreads) tiled_kernel(GroupedParams p) {
  __shared__ u32x4 shared_a[2][kStageChunks];
  __shared__ u32x4 shared_w[2][kStageChunks];
  const int tile = static_cast<int>(blockIdx.x);
  if (tile >= p.num_tiles[0]) return;
  const int64_t expert = p.tile_to_expert[tile];
  const int64_t first = static_cast<int64_t>(tile) * kTileRows;
  const int rows = p.tile_to_limit[tile] - static_cast<int>(first);
  const int t = static_cast<int>(threadIdx.x);
  const int wave = t / kWave;
  const int lane = lane_id();
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int wm = wave & 1;
  const int wn = wave >> 1;
  const int64_t slice = static_cast<int64_t>(blockIdx.y) * (kGated ? 64 : 128);

  // This thread's four rows of each operand and its 16-byte chunk within a stage.
  const int chunk = t & 7;
  const uint16_t *a_row[4];
  const uint16_t *w_row[4];
  bool a_valid[4], w_valid[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = (t >> 3) + 32 * i;
    a_valid[i] = r < rows;
    int64_t source = first + r;
    if constexpr (kGated) source = a_valid[i] ? p.permuted_to_expanded[first + r] / p.top : 0;
    a_row[i] = p.act + (a_valid[i] ? source : 0) * p.K + chunk * 8;
    int64_t n;
    if constexpr (kGated) n = r < 64 ? slice + r : p.out_width + slice + (r - 64);
    else n = slice + r;
    w_valid[i] = kGated ? true : n < p.out_width;
    w_row[i] = p.weights + (expert * p.n_total + (w_valid[i] ? n : 0)) * p.K + chunk * 8;
  }

  u32x4 staged_a[4], staged_w[4];
  auto fetch = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      staged_a[i] = a_valid[i] ? load16(a_row[i] + k0) : u32x4{0, 0, 0, 0};
      staged_w[i] = w_valid[i] ? load16(w_row[i] + k0) : u32x4{0, 0, 0, 0};
    }
  };
  auto deposit = [&](int stage) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = (t >> 3) + 32 * i;
      shared_a[stage][swizzled(r, chunk)] = staged_a[i];
      shared_w[stage][swizzled(r, chunk)] = staged_w[i];
    }
  };

  floatx4 acc[4][4];
#pragma unroll
  for (int ni = 0; ni < 4; ++ni)
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) acc[ni][mi] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  const int steps = static_cast<int>(p.K / kBK);
  fetch(0);
  deposit(0);
  __syncthreads();
  for (int step = 0; step < steps; ++step) {
    const int stage = step & 1;
    if (step + 1 < steps) fetch(static_cast<int64_t>(step + 1) * kBK);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int c = ks * 4 + g;
      u32x4 wf[4], af[4];
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) {
        int r;
        if constexpr (kGated) r = (ni < 2 ? wn * 32 + ni * 16 : 64 + wn * 32 + (ni - 2) * 16) + r16;
        else r = wn * 64 + ni * 16 + r16;
        wf[ni] = shared_w[stage][swizzled(r, c)];
      }
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
        const int r = wm * 64 + mi * 16 + r16;
        af[mi] = shared_a[stage][swizzled(r, c)];
      }
#pragma unroll
      for (int ni = 0; ni < 4; ++ni)
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) acc[ni][mi] = mfma_16x16x32_bf16(wf[ni], af[mi], acc[ni][mi]);
    }
    if (step + 1 < steps) deposit(stage ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
    const int m = wm * 64 + mi * 16 + r16;
    if (m >= rows) continue;
    uint16_t *row = p.out + (first + m) * p.out_width;
    if constexpr (kGated) {
#pragma unroll
      for (int ni = 0; ni < 2; ++ni) {
        floatx4 h;
#pragma unroll
        for (int i = 0; i < 4; ++i) h[i] = gate(acc[ni + 2][mi][i], p.activation) * acc[ni][mi][i];
        store_bf16x4(row + slice + wn * 32 + ni * 16 + 4 * g, h);
      }
    } else {
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) {
        const int64_t col = slice + wn * 64 + ni * 16 + 4 * g;
        if (col < p.out_width) store_bf16x4(row + col, acc[ni][mi]);
      }
    }
  }
}

/// The stream kernel serves batches whose experts average fewer rows than this.
constexpr int64_t kStreamRowsPerExpert = 24;

template <bool kGated>
void launch_grouped(const GroupedParams &p, int64_t max_tiles, bool stream_path, bool one_pass, hipStream_t s) {
  if (!stream_path && (pair_fits<pair::Bf16>(kGated, p.K, p.out_width, 0) || prefill_fits<prefill::Bf16, kGated>(p.K, p.out_width))) {
    PrefillParams q{};
    q.act = reinterpret_cast<const uint8_t *>(p.act);
    q.weights = reinterpret_cast<const uint8_t *>(p.weights);
    q.out = p.out;
    q.tile_to_expert = p.tile_to_expert;
    q.tile_to_limit = p.tile_to_limit;
    q.permuted_to_expanded = p.permuted_to_expanded;
    q.num_tiles = p.num_tiles;
    q.K = p.K;
    q.n_total = p.n_total;
    q.out_width = p.out_width;
    q.top = p.top;
    q.activation = p.activation;
    if (pair_fits<pair::Bf16>(kGated, q.K, q.out_width, 0)) launch_pair<pair::Bf16>(q, kGated, max_tiles, s);
    else launch_prefill<prefill::Bf16, kGated>(q, max_tiles, s);
    return;
  }
  const int64_t slices = kGated ? p.out_width / 64 : ceil_div<int64_t>(p.out_width, 128);
  const dim3 grid(static_cast<uint32_t>(max_tiles), static_cast<uint32_t>(slices));
  if (stream_path && one_pass) hipLaunchKernelGGL((stream_kernel<kGated, 1>), grid, dim3(kThreads), 0, s, p);
  else if (stream_path) hipLaunchKernelGGL((stream_kernel<kGated, 2>), grid, dim3(kThreads), 0, s, p);
  else hipLaunchKernelGGL(tiled_kernel<kGated>, grid, dim3(kThreads), 0, s, p);
}

}  // namespace
}  // namespace uniserve

namespace uniserve {

bool expert_stream_fits(int64_t routes, int64_t local_experts, int64_t K, int64_t out_width, bool gated) {
  // Fewer routes than local experts: a compact grid (a workgroup column per route, each finding
  // the n-th named expert), which tells at most kPresentExperts experts apart.
  return routes >= 1 && routes <= kExpertRoutes && routes < kStreamRowsPerExpert * local_experts &&
         (routes >= local_experts || local_experts <= kPresentExperts) && K % 128 == 0 &&
         (gated ? out_width % 64 == 0 : out_width % 128 == 0) && local_experts <= 0x7fffffffLL;
}

void launch_expert_stream(const ExpertStream &e, bool gated, hipStream_t stream) {
  GroupedParams p{};
  p.act = static_cast<const uint16_t *>(e.act);
  p.weights = static_cast<const uint16_t *>(e.weights);
  p.out = static_cast<uint16_t *>(e.out);
  p.K = e.K;
  p.n_total = e.n_total;
  p.out_width = e.out_width;
  p.top = e.top;
  p.activation = e.activation;
  p.ids = e.ids;
  p.live_tokens = e.live_tokens;
  p.routes = e.routes;
  p.local_offset = e.local_offset;
  p.local_experts = e.local_experts;
  p.compact = e.routes < e.local_experts ? 1 : 0;
  const bool one_pass = e.routes <= kOnePassRowsPerExpert * e.local_experts;
  const int64_t slices = gated ? e.out_width / 64 : e.out_width / 128;
  const dim3 grid(static_cast<uint32_t>(p.compact ? e.routes : e.local_experts), static_cast<uint32_t>(slices));
  constexpr int64_t kOffsetRange = int64_t{1} << 32;  // the quarter kernel's 32-bit byte offsets
  if (gated && e.K % 256 == 0 && e.n_total * e.K * 2 < kOffsetRange && e.routes * e.K * 2 < kOffsetRange) {
    hipLaunchKernelGGL(quarter_kernel, grid, dim3(kThreads), 0, stream, p);
    return;
  }
  if (gated && one_pass) hipLaunchKernelGGL((stream_kernel<true, 1, true>), grid, dim3(kThreads), 0, stream, p);
  else if (gated) hipLaunchKernelGGL((stream_kernel<true, 2, true>), grid, dim3(kThreads), 0, stream, p);
  else if (one_pass) hipLaunchKernelGGL((stream_kernel<false, 1, true>), grid, dim3(kThreads), 0, stream, p);
  else hipLaunchKernelGGL((stream_kernel<false, 2, true>), grid, dim3(kThreads), 0, stream, p);
}

int32_t gather_gemm_bf16(const uniserve_gather_call *call, int32_t activation, void *stream) {
  return guarded(call, [&]() -> int32_t {
    // The refusals of the reference entry (gather_gemm/cute_dsl/src/entry.cpp:18-42) and of
    // `GatherGemm::check` (crates/ops/src/moe/grouped.rs:250-324) the call's words can state.
    if (call->dtype != UNISERVE_DTYPE_BF16) return UNISERVE_REFUSE(call, "gather_gemm serves bf16 only");
    if (call->hidden == nullptr || call->weights == nullptr || call->out == nullptr)
      return UNISERVE_REFUSE(call, "gather_gemm needs hidden, weights and out");
    if (call->tile_to_expert == nullptr || call->tile_to_limit == nullptr ||
        call->permuted_to_expanded == nullptr || call->num_non_exiting_tiles == nullptr)
      return UNISERVE_REFUSE(call, "gather_gemm needs the sort's tile and route maps");
    if (call->width % 2 != 0) return UNISERVE_REFUSE(call, "gather_gemm needs an even 2*intermediate width");
    if (call->multiprocessors <= 0 || call->multiprocessors > INT32_MAX)
      return UNISERVE_REFUSE(call, "gather_gemm needs its device's multiprocessor count");
    if (call->hidden_size <= 0 || call->hidden_size % 64 != 0)
      return UNISERVE_REFUSE(call, "gather_gemm needs a hidden size of whole 64-element steps");
    if (call->width <= 0 || (call->width / 2) % 64 != 0)
      return UNISERVE_REFUSE(call, "gather_gemm needs an intermediate width of whole 64-column blocks");
    if (call->tokens < 0 || call->top <= 0 || call->experts <= 0)
      return UNISERVE_REFUSE(call, "gather_gemm needs non-negative tokens and positive top and experts");
    if (!dma_rows_fit(call->tokens, call->hidden_size * 2))
      return UNISERVE_REFUSE(call, "gather_gemm serves hidden rows below 4 GiB (%lld tokens of %lld bytes)",
                             static_cast<long long>(call->tokens), static_cast<long long>(call->hidden_size * 2));
    if (call->permuted_rows < call->tokens * call->top)
      return UNISERVE_REFUSE(call, "%lld permuted rows cannot hold %lld routes",
                             static_cast<long long>(call->permuted_rows),
                             static_cast<long long>(call->tokens * call->top));
    if (call->permuted_rows % kTileRows != 0)
      return UNISERVE_REFUSE(call, "gather_gemm needs permuted rows of whole 128-row tiles");
    const int64_t max_tiles = call->permuted_rows / kTileRows;
    if (max_tiles == 0) return 0;
    if (max_tiles > 0x7fffffffLL) return UNISERVE_REFUSE(call, "gather_gemm: too many tiles for one grid");

    GroupedParams p{};
    p.act = static_cast<const uint16_t *>(call->hidden);
    p.weights = static_cast<const uint16_t *>(call->weights);
    p.out = static_cast<uint16_t *>(call->out);
    p.tile_to_expert = call->tile_to_expert;
    p.tile_to_limit = call->tile_to_limit;
    p.permuted_to_expanded = call->permuted_to_expanded;
    p.num_tiles = call->num_non_exiting_tiles;
    p.K = call->hidden_size;
    p.n_total = call->width;
    p.out_width = call->width / 2;
    p.top = call->top;
    p.activation = activation;
    const bool stream_path = call->tokens * call->top < kStreamRowsPerExpert * call->experts &&
                             call->hidden_size % 128 == 0;
    launch_grouped<true>(p, max_tiles, stream_path, call->tokens * call->top <= kOnePassRowsPerExpert * call->experts,
                         static_cast<hipStream_t>(stream));
    return launched(call, "gather_gemm");
  });
}

}  // namespace uniserve

extern "C" int32_t uniserve_gather_gemm(const uniserve_gather_call *call, void *stream) {
  return uniserve::gather_gemm_bf16(call, UNISERVE_ACTIVATION_SILU, stream);
}

extern "C" int32_t uniserve_gather_gemm_gelu_tanh(const uniserve_gather_call *call, void *stream) {
  return uniserve::gather_gemm_bf16(call, UNISERVE_ACTIVATION_GELU_TANH, stream);
}

extern "C" int32_t uniserve_route_gemm(const uniserve_route_call *call, void *stream) {
  using namespace uniserve;
  return guarded(call, [&]() -> int32_t {
    if (call->dtype != UNISERVE_DTYPE_BF16) return UNISERVE_REFUSE(call, "route_gemm serves bf16 only");
    if (call->rows == nullptr || call->weights == nullptr || call->out == nullptr)
      return UNISERVE_REFUSE(call, "route_gemm needs rows, weights and out");
    if (call->tile_to_expert == nullptr || call->tile_to_limit == nullptr ||
        call->permuted_to_expanded == nullptr || call->num_non_exiting_tiles == nullptr)
      return UNISERVE_REFUSE(call, "route_gemm needs the sort's tile and route maps");
    if (call->multiprocessors <= 0 || call->multiprocessors > INT32_MAX)
      return UNISERVE_REFUSE(call, "route_gemm needs its device's multiprocessor count");
    if (call->intermediate <= 0 || call->intermediate % 64 != 0)
      return UNISERVE_REFUSE(call, "route_gemm needs an intermediate width of whole 64-element steps");
    if (call->width <= 0 || call->width % 64 != 0)
      return UNISERVE_REFUSE(call, "route_gemm needs a hidden width of whole 64-column blocks");
    if (call->experts <= 0) return UNISERVE_REFUSE(call, "route_gemm needs positive experts");
    if (call->permuted_rows < 0 || call->permuted_rows % kTileRows != 0)
      return UNISERVE_REFUSE(call, "route_gemm needs permuted rows of whole 128-row tiles");
    const int64_t max_tiles = call->permuted_rows / kTileRows;
    if (max_tiles == 0) return 0;
    if (max_tiles > 0x7fffffffLL) return UNISERVE_REFUSE(call, "route_gemm: too many tiles for one grid");

    GroupedParams p{};
    p.act = static_cast<const uint16_t *>(call->rows);
    p.weights = static_cast<const uint16_t *>(call->weights);
    p.out = static_cast<uint16_t *>(call->out);
    p.tile_to_expert = call->tile_to_expert;
    p.tile_to_limit = call->tile_to_limit;
    p.permuted_to_expanded = call->permuted_to_expanded;
    p.num_tiles = call->num_non_exiting_tiles;
    p.K = call->intermediate;
    p.n_total = call->width;
    p.out_width = call->width;
    p.top = 1;
    // The call states no token count: the permuted rows bound the routes, and their expected
    // share per expert is (rows - the padding of one partial tile per expert) / experts.
    const int64_t routes_bound = call->permuted_rows - (kTileRows - 1) * call->experts;
    const bool stream_path = routes_bound < kStreamRowsPerExpert * call->experts &&
                             call->intermediate % 128 == 0;
    launch_grouped<false>(p, max_tiles, stream_path, routes_bound <= kOnePassRowsPerExpert * call->experts,
                          static_cast<hipStream_t>(stream));
    return launched(call, "route_gemm");
  });
}

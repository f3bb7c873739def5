// SPDX-License-Identifier: Apache-2.0
//
// Block-scaled OCP e4m3 forms of the grouped expert products, and the activation quantiser they
// read (no reference counterpart: crates/nn/src/quantization.rs:241-249 refuses 128x128
// block-scaled checkpoints; this is the format BASELINE names, in the call style of the
// reference's NVFP4 operators, crates/ops/src/moe/grouped.rs:816-869).
//
// Values are code * scale with one FP32 scale per 128 x 128 weight block and per 128 channels of an
// activation row. One gfx950 MFMA 16x16x128 (f8f6f4, e4m3 x e4m3) spans exactly one scale block
// along K, so each block's product is formed exactly as the hardware accumulates it and then added
// into the FP32 accumulator times s_w * s_x - the per-block dequantisation never touches the
// operands. Decode shapes run the `stream` kernel; prefill shapes run the two-workgroups-per-CU
// kernel of grouped_dual.hpp, or, where FC1 writes its rows already quantised for FC2, the
// one-workgroup-per-CU kernel of grouped_prefill.hpp; the quantiser's codes are bit-exact with the
// host rule (nearest even, saturating at 448).
#include "common.hpp"
#include "grouped_fp8.hpp"
#include "grouped_dual.hpp"
#include "grouped_pair.hpp"
#include "expert_routes.hpp"
#include "grouped_prefill.hpp"
#include "uniserve_moe_fp8.h"

namespace uniserve {

namespace {

// ---- the activation quantiser -------------------------------------------------------------------------------

constexpr int kQuantThreads = 256;

struct QuantParams {
  const void *input;
  uint8_t *out;
  float *scales;
  const int32_t *row_limit;
  int64_t rows;
  int64_t width;
  int32_t input_f32;
  float *route_scales;                  ///< or null: scales scattered to the routes' permuted rows
  const int32_t *expanded_to_permuted;  ///< with route_scales: [rows, top]
  int64_t top;
  int64_t route_rows;                   ///< with route_scales: its row stride per block
};

/// 16 lanes per 128-channel group, 8 channels each; the grid strides over the groups, stopping at
/// the device-side row limit (the padded rows of a decode batch are a small part of the
/// worst-case rows the host sizes for).
__global__ void __launch_bounds__(kQuantThreads) quantize_kernel(QuantParams p) {
  const int64_t groups_per_row = p.width / 128;
  const int sub = static_cast<int>(threadIdx.x) & 15;
  const int64_t limit = p.row_limit != nullptr ? p.row_limit[0] : p.rows;
  const int64_t last = (limit < p.rows ? limit : p.rows) * groups_per_row;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kQuantThreads / 16;
  for (int64_t group = (static_cast<int64_t>(blockIdx.x) * kQuantThreads + threadIdx.x) / 16; group < last;
       group += stride) {
    const int64_t row = group / groups_per_row;
    const int64_t column = (group % groups_per_row) * 128 + sub * 8;
    float scale;
    if (p.input_f32) {
      const float *src = static_cast<const float *>(p.input) + row * p.width + column;
      const float4 lo = *reinterpret_cast<const float4 *>(src);
      const float4 hi = *reinterpret_cast<const float4 *>(src + 4);
      float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      float amax = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[j]));
      amax = row16_max(amax);
      scale = amax > 0.0f ? amax / 448.0f : 1.0f;
      *reinterpret_cast<uint2 *>(p.out + row * p.width + column) = e4m3_eight(v, scale);
      if (sub == 0) p.scales[row * groups_per_row + column / 128] = scale;
    } else {
      const int64_t group_first = row * p.width + column - sub * 8;
      scale = quantize_bf16_group(static_cast<const uint16_t *>(p.input) + group_first, p.out + group_first,
                                  p.scales + row * groups_per_row + column / 128, sub);
    }
    if (p.route_scales != nullptr) {
      for (int64_t k = sub; k < p.top; k += 16) {
        const int32_t at = p.expanded_to_permuted[row * p.top + k];
        if (at >= 0) p.route_scales[column / 128 * p.route_rows + at] = scale;
      }
    }
  }
}

// ---- grouped products --------------------------------------------------------------------------------------

constexpr int kTileRows = 128;
constexpr int kThreads = 256;

__device__ __forceinline__ void store_bf16x4(uint16_t *pointer, floatx4 v) {
  uint2 packed;
  packed.x = pack_bf16x2(v[0], v[1]);
  packed.y = pack_bf16x2(v[2], v[3]);
  *reinterpret_cast<uint2 *>(pointer) = packed;
}

/// Average routes per expert at or below which the stream kernel takes a tile in passes of one
/// 16-row MFMA block instead of two (fewer registers, more waves per SIMD: at 64-token decode FC1
/// 63.6 against 66.4 us, FC2 35.8 against 39.2; a tile with more rows re-streams its weights per
/// pass, which at such averages is rare).
constexpr int64_t kOnePassRowsPerExpert = 8;

constexpr int64_t kSplitBelow = 512;  // stream workgroups under which K is split over the waves

/// Decode-shaped: as the bf16 stream kernel, one 128-deep scale block per chunk. kSplit: the four
/// wavefronts share one row set and split K (scale block kb goes to wave kb % 4), their partial sums
/// meeting in LDS in wave order - four times the workgroups, for batches whose tiles x slices would
/// leave most of the chip idle (a single token: 8 tiles). Both sets' lines of a block go out
/// together, as in the unsplit form (walking the two sets in turn, half the lines in flight: 235B
/// T=1 FC1 18.5 against 18.3 us, FC2 12.7 against 12.2, the same sums).
/// kPassTiles: rows of a tile one pass covers, in MFMA blocks of 16.
/// kByExpert: workgroup x serves local expert x and lists its rows itself (the routes naming it in
/// `ids`, route order), reading act row route / top (FC1) or route (FC2) and writing row `route`.
/// kRun (expert-major): the workgroup serves kRun consecutive slices one after the other, listing
/// the routes once (grid y = slices / kRun).
/// kWaves (unsplit): the workgroup's wavefronts, 16 gated columns each (FC1). kQuantOut (expert-major
/// FC1, eight waves): the workgroup's 128 gated columns are one whole e4m3 scale group, so it also
/// writes the gated rows as FC2's operand - staged in LDS as the bf16 values the quantiser would
/// read, then quantised by its group routine (codes [routes, out_width] at out_codes, scales
/// [routes, out_width / 128] at out_code_scales).
template <bool kGated, bool kSplit, int kPassTiles, bool kByExpert = false, int kRun = 1, int kWaves = 4,
          bool kQuantOut = false>
__global__ void __launch_bounds__(kWaves * kWave) stream_fp8_kernel(GroupedFp8Params p) {
  static_assert(kRun == 1 || kByExpert, "runs of slices: expert-major");
  static_assert(kWaves == 4 || !kSplit, "the split form: four waves");
  static_assert(!kQuantOut || (kGated && !kSplit && kByExpert && kWaves == 8), "e4m3 out: eight-wave FC1");
  constexpr int kThreads = kWaves * kWave;
  __shared__ floatx4 partial[kSplit ? kWaves - 1 : 1][2][kPassTiles][kWave];
  __shared__ int32_t route_list[kByExpert ? kExpertRoutes : 1];
  __shared__ int32_t route_count[kWaves + 1];
  __shared__ u32x4 regroup[kWaves][4 * 64];  // each wave's weight lines of a block, regrouped
  __shared__ uint16_t gated_tile[kQuantOut ? 16 * kPassTiles * 128 : 1];
  int64_t expert, first;
  int rows = 0;
  if constexpr (kByExpert) {
    expert = blockIdx.x;
    first = 0;
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
  auto listed = [&](int m) -> int64_t {
    return listed_route<kWaves>(route_list, route_count, p.routes, m);
  };
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int lane = lane_id();
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int64_t kb_count = p.K / 128;

  int64_t n0, n1;
  const int row_set = kSplit ? 0 : wave;
  auto slice_rows = [&](int64_t slice) {
    if constexpr (kGated) {
      n0 = slice * (kSplit ? 16 : kWaves * 16) + row_set * 16;
      n1 = p.out_width + n0;
    } else {
      n0 = slice * (kSplit ? 32 : kWaves * 32) + row_set * 32;
      n1 = n0 + 16;
    }
  };
  slice_rows(static_cast<int64_t>(blockIdx.y) * kRun);
  if constexpr (!kGated && !kByExpert) {
    if (n0 >= p.out_width) return;  // (expert-major: whole slices only)
  }
  const int64_t kb_first = kSplit ? wave : 0;
  const int64_t kb_step = kSplit ? kWaves : 1;
  // Weight lines: load i (0..3) of a scale block reads rows 8 (i % 2) + l / 8 of set i / 2 (set 0 =
  // rows n0.., set 1 = rows n1..), 16-byte chunk l % 8 - whole 128-byte lines, non-temporal (each
  // weight line is read once per call). Lane l's MFMA operand (row r16, 32 K bytes of group g:
  // chunks g and g + 4) is gathered from those loads through the wave's own LDS buffer (load i's
  // lane l, row l / 8 of the load and chunk l % 8, at slot 64 i + 8 r + (chunk ^ r), r = l / 8: the
  // lanes reading one chunk of eight rows read eight bank groups); the activations use the same K
  // mapping. (Against ds_bpermute from both candidate loads and a select: 30B T=64 FC2 42 -> 40 us,
  // the layer 131 -> 127.)
  const uint8_t *line_row[2];
  const float *ws0, *ws1;
  auto slice_pointers = [&]() {
    line_row[0] = p.weights + (expert * p.n_total + n0 + lane / 8) * p.K + (lane & 7) * 16;
    line_row[1] = p.weights + (expert * p.n_total + n1 + lane / 8) * p.K + (lane & 7) * 16;
    ws0 = p.weight_scales + (expert * (p.n_total / 128) + n0 / 128) * kb_count;
    ws1 = p.weight_scales + (expert * (p.n_total / 128) + n1 / 128) * kb_count;
  };
  slice_pointers();

  // Expert-major: the first weight block goes out before the route scan (it depends on nothing the
  // routes decide), then the scan lists the expert's rows.
  u32x4 wcur[4], wnext[4];  // the weight lines of alternate blocks
  FirstRouteIds first_ids;
  if constexpr (kByExpert) first_ids = load_first_route_ids<kWaves>(p.ids, p.routes);  // (before the lines)
  if (kByExpert && kb_first < kb_count) {  // (a split wave may own no block)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      wcur[i] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4 *>(line_row[i / 2] + static_cast<int64_t>(i % 2) * 8 * p.K + kb_first * 128));
  }
  if constexpr (kByExpert) {
    const int64_t live = p.live_tokens != nullptr ? static_cast<int64_t>(p.live_tokens[0]) * p.top : p.routes;
    rows = list_expert_routes<kWaves>(p.ids, p.routes, live, static_cast<int32_t>(expert + p.local_offset),
                                      route_list, route_count, &first_ids);
    if (rows == 0) return;
  }

  for (int run = 0; run < kRun; ++run) {
  if (run > 0) {
    slice_rows(static_cast<int64_t>(blockIdx.y) * kRun + run);
    slice_pointers();
  }
  for (int pass = 0; pass < rows; pass += 16 * kPassTiles) {
    const uint8_t *a[kPassTiles];
    const float *as[kPassTiles];
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
      if (!valid[ms]) source = 0;
      a[ms] = p.act + source * p.K + g * 16;
      as[ms] = p.act_scales + source * kb_count;
    }
    floatx4 acc[2][kPassTiles];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int ms = 0; ms < kPassTiles; ++ms) acc[s][ms] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    auto fetch_rest = [&](int64_t kb, intx8 (&x)[kPassTiles], float (&s)[2 + kPassTiles]) {
      s[0] = ws0[kb];
      s[1] = ws1[kb];
#pragma unroll
      for (int ms = 0; ms < kPassTiles; ++ms) {
        const u32x4 lo = *reinterpret_cast<const u32x4 *>(a[ms] + kb * 128);
        const u32x4 hi = *reinterpret_cast<const u32x4 *>(a[ms] + kb * 128 + 64);
        x[ms] = intx8{static_cast<int>(lo[0]), static_cast<int>(lo[1]), static_cast<int>(lo[2]), static_cast<int>(lo[3]),
                      static_cast<int>(hi[0]), static_cast<int>(hi[1]), static_cast<int>(hi[2]), static_cast<int>(hi[3])};
        s[2 + ms] = as[ms][kb];
      }
    };
    auto fetch = [&](int64_t kb, u32x4 (&w)[4], intx8 (&x)[kPassTiles], float (&s)[2 + kPassTiles]) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        w[i] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4 *>(line_row[i / 2] + static_cast<int64_t>(i % 2) * 8 * p.K + kb * 128));
      fetch_rest(kb, x, s);
    };
    auto compute = [&](const u32x4 (&lines)[4], const intx8 (&x)[kPassTiles], const float (&s)[2 + kPassTiles]) {
      intx8 w[2];
      {
        const int row = lane >> 3, piece = lane & 7;
#pragma unroll
        for (int i = 0; i < 4; ++i) regroup[wave][i * 64 + row * 8 + (piece ^ row)] = lines[i];
      }
#pragma unroll
      for (int set = 0; set < 2; ++set) {
        const int i = 2 * set + (r16 >> 3), rr = r16 & 7;
        const u32x4 lo = regroup[wave][i * 64 + rr * 8 + (g ^ rr)];
        const u32x4 hi = regroup[wave][i * 64 + rr * 8 + ((g + 4) ^ rr)];
        w[set] = intx8{static_cast<int>(lo[0]), static_cast<int>(lo[1]), static_cast<int>(lo[2]), static_cast<int>(lo[3]),
                       static_cast<int>(hi[0]), static_cast<int>(hi[1]), static_cast<int>(hi[2]), static_cast<int>(hi[3])};
      }
#pragma unroll
      for (int ms = 0; ms < kPassTiles; ++ms)
#pragma unroll
        for (int set = 0; set < 2; ++set) {
          const floatx4 block = mfma_16x16x128_fp8(w[set], x[ms], floatx4{0.0f, 0.0f, 0.0f, 0.0f});
          const float scale = s[set] * s[2 + ms];
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[set][ms][i] = __builtin_fmaf(block[i], scale, acc[set][ms][i]);
        }
    };
    intx8 acur[kPassTiles], anext[kPassTiles];
    float scur[2 + kPassTiles], snext[2 + kPassTiles];
    if (kb_first < kb_count) {
      if (kByExpert && pass == 0 && run == 0) fetch_rest(kb_first, acur, scur);  // lines out before the scan
      else fetch(kb_first, wcur, acur, scur);
    }
    // The steady walk issues both blocks' loads unconditionally, so the compiler's wait before
    // each compute counts exactly the other block's loads still in flight (with the loads under
    // conditions it waited for every load, the prefetched block's too); the last one or two
    // blocks are peeled.
    int64_t kb = kb_first;
    if (kb < kb_count) {
      for (; kb + 2 * kb_step < kb_count; kb += 2 * kb_step) {
        fetch(kb + kb_step, wnext, anext, snext);
        compute(wcur, acur, scur);
        fetch(kb + 2 * kb_step, wcur, acur, scur);
        compute(wnext, anext, snext);
      }
      if (kb + kb_step < kb_count) {
        fetch(kb + kb_step, wnext, anext, snext);
        compute(wcur, acur, scur);
        compute(wnext, anext, snext);
      } else {
        compute(wcur, acur, scur);
      }
    }
    if constexpr (kSplit) {
      // Waves 1..3 hand their partial sums to wave 0, which adds them in wave order.
      if (wave > 0) {
#pragma unroll
        for (int set = 0; set < 2; ++set)
#pragma unroll
          for (int ms = 0; ms < kPassTiles; ++ms) partial[wave - 1][set][ms][lane] = acc[set][ms];
      }
      __syncthreads();
      if (wave == 0) {
#pragma unroll
        for (int w = 0; w < kWaves - 1; ++w)
#pragma unroll
          for (int set = 0; set < 2; ++set)
#pragma unroll
            for (int ms = 0; ms < kPassTiles; ++ms) acc[set][ms] += partial[w][set][ms][lane];
      }
      __syncthreads();
      if (wave > 0) continue;
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
        if constexpr (kQuantOut) {
          uint2 packed;
          packed.x = pack_bf16x2(h[0], h[1]);
          packed.y = pack_bf16x2(h[2], h[3]);
          *reinterpret_cast<uint2 *>(gated_tile + (ms * 16 + r16) * 128 + wave * 16 + 4 * g) = packed;
        }
      } else {
        store_bf16x4(row + n0 + 4 * g, acc[0][ms]);
        store_bf16x4(row + n1 + 4 * g, acc[1][ms]);
      }
    }
    if constexpr (kQuantOut) {
      // The pass's rows x the workgroup's 128 columns (one e4m3 group), 16 lanes a row.
      __syncthreads();
      const int t = static_cast<int>(threadIdx.x);
      const int r = t / 16, m = pass + r;
      if (r < 16 * kPassTiles && m < rows) {
        const int64_t route = listed(m);
        quantize_bf16_group(gated_tile + r * 128, p.out_codes + route * p.out_width + blockIdx.y * 128,
                            p.out_code_scales + route * (p.out_width / 128) + blockIdx.y, t & 15);
      }
      __syncthreads();
    }
  }
  }
}

/// Prefill-shaped: 128 x 128 tiles, one 128-deep scale block per LDS stage (16 KB per operand).
constexpr int kStageChunks = 128 * 8;  // 16-byte chunks: 128 rows x 128 bytes

__device__ __forceinline__ int swizzled(int row, int chunk) { return row * 8 + (chunk ^ (row & 7)); }

template <bool kGated>
__global__ void __launch_bounds__(kThreads) tiled_fp8_kernel(GroupedFp8Params p) {
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
  const int64_t kb_count = p.K / 128;
  const int64_t nb_count = p.n_total / 128;

  const int chunk = t & 7;
  const uint8_t *a_row[4];
  const uint8_t *w_row[4];
  bool a_valid[4], w_valid[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = (t >> 3) + 32 * i;
    a_valid[i] = r < rows;
    int64_t source = first + r;
    if constexpr (kGated) source = a_valid[i] ? p.permuted_to_expanded[first + r] / p.top : 0;
    a_row[i] = p.act + (a_valid[i] ? source : 0) * p.K + chunk * 16;
    int64_t n;
    if constexpr (kGated) n = r < 64 ? slice + r : p.out_width + slice + (r - 64);
    else n = slice + r;
    w_valid[i] = kGated ? true : n < p.out_width;
    w_row[i] = p.weights + (expert * p.n_total + (w_valid[i] ? n : 0)) * p.K + chunk * 16;
  }
  // The activation scales of this lane's four MFMA rows, and the weight block of each row set.
  const float *row_scale[4];
  bool row_valid[4];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
    const int m = wm * 64 + mi * 16 + r16;
    row_valid[mi] = m < rows;
    int64_t source = first + m;
    if constexpr (kGated) source = row_valid[mi] ? p.permuted_to_expanded[first + m] / p.top : 0;
    row_scale[mi] = p.act_scales + (row_valid[mi] ? source : 0) * kb_count;
  }
  const float *wscale_lo;  // FC1: the up rows; FC2: rows [slice, slice + 128)
  const float *wscale_hi;  // FC1: the gate rows
  if constexpr (kGated) {
    wscale_lo = p.weight_scales + (expert * nb_count + slice / 128) * kb_count;
    wscale_hi = p.weight_scales + (expert * nb_count + (p.out_width + slice) / 128) * kb_count;
  } else {
    wscale_lo = p.weight_scales + (expert * nb_count + slice / 128) * kb_count;
    wscale_hi = wscale_lo;
  }

  u32x4 staged_a[4], staged_w[4];
  auto fetch = [&](int64_t kb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      staged_a[i] = a_valid[i] ? *reinterpret_cast<const u32x4 *>(a_row[i] + kb * 128) : u32x4{0, 0, 0, 0};
      staged_w[i] = w_valid[i] ? *reinterpret_cast<const u32x4 *>(w_row[i] + kb * 128) : u32x4{0, 0, 0, 0};
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

  fetch(0);
  deposit(0);
  __syncthreads();
  for (int64_t kb = 0; kb < kb_count; ++kb) {
    const int stage = static_cast<int>(kb & 1);
    if (kb + 1 < kb_count) fetch(kb + 1);
    float sx[4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) sx[mi] = row_valid[mi] ? row_scale[mi][kb] : 0.0f;
    const float sw_lo = wscale_lo[kb];
    const float sw_hi = wscale_hi[kb];
    // Lane group g takes 16-byte chunks 2g and 2g + 1 of the 128-byte row: 32 K elements.
    intx8 wf[4], af[4];
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) {
      int r;
      if constexpr (kGated) r = (ni < 2 ? wn * 32 + ni * 16 : 64 + wn * 32 + (ni - 2) * 16) + r16;
      else r = wn * 64 + ni * 16 + r16;
      const u32x4 lo = shared_w[stage][swizzled(r, 2 * g)];
      const u32x4 hi = shared_w[stage][swizzled(r, 2 * g + 1)];
      wf[ni] = intx8{static_cast<int>(lo[0]), static_cast<int>(lo[1]), static_cast<int>(lo[2]), static_cast<int>(lo[3]),
                     static_cast<int>(hi[0]), static_cast<int>(hi[1]), static_cast<int>(hi[2]), static_cast<int>(hi[3])};
    }
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
      const int r = wm * 64 + mi * 16 + r16;
      const u32x4 lo = shared_a[stage][swizzled(r, 2 * g)];
      const u32x4 hi = shared_a[stage][swizzled(r, 2 * g + 1)];
      af[mi] = intx8{static_cast<int>(lo[0]), static_cast<int>(lo[1]), static_cast<int>(lo[2]), static_cast<int>(lo[3]),
                     static_cast<int>(hi[0]), static_cast<int>(hi[1]), static_cast<int>(hi[2]), static_cast<int>(hi[3])};
    }
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) {
      const float sw = (kGated ? ni < 2 : true) ? sw_lo : sw_hi;
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
        const floatx4 block = mfma_16x16x128_fp8(wf[ni], af[mi], floatx4{0.0f, 0.0f, 0.0f, 0.0f});
        const float scale = sw * sx[mi];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[ni][mi][i] = __builtin_fmaf(block[i], scale, acc[ni][mi][i]);
      }
    }
    if (kb + 1 < kb_count) deposit(stage ^ 1);
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

constexpr int64_t kStreamRowsPerExpert = 24;

}  // namespace

/// Workgroups for `rows` x `width`: one 16-lane group per 128 channels, at most 2048 workgroups
/// (the kernel strides over the rest).
uint32_t quantize_blocks(int64_t rows, int64_t width) {
  const int64_t blocks = ceil_div<int64_t>(rows * (width / 128) * 16, kQuantThreads);
  return static_cast<uint32_t>(blocks < 2048 ? (blocks > 0 ? blocks : 1) : 2048);
}

void launch_quantize_fp8(const void *input, bool input_f32, uint8_t *out, float *scales,
                         const int32_t *row_limit, int64_t rows, int64_t width, hipStream_t stream) {
  QuantParams p{input, out, scales, row_limit, rows, width, input_f32 ? 1 : 0, nullptr, nullptr, 0, 0};
  hipLaunchKernelGGL(quantize_kernel, dim3(quantize_blocks(rows, width)), dim3(kQuantThreads), 0, stream, p);
}

void launch_quantize_fp8_routes(const uint16_t *input, uint8_t *out, float *scales, float *route_scales,
                                const int32_t *expanded_to_permuted, int64_t top, int64_t route_rows,
                                int64_t rows, int64_t width, hipStream_t stream) {
  QuantParams p{input, out, scales, nullptr, rows, width, 0, route_scales, expanded_to_permuted, top, route_rows};
  hipLaunchKernelGGL(quantize_kernel, dim3(quantize_blocks(rows, width)), dim3(kQuantThreads), 0, stream, p);
}

void launch_grouped_fp8(const GroupedFp8Params &p, bool gated, int64_t max_tiles, bool stream_path, bool one_pass,
                        hipStream_t stream) {
  // The two-workgroup kernel first, then the 8-wave kernels (per-wave weight buffers of 256-K stage
  // pairs, then the shared-stage one), then the generic tiled kernel.
  const bool fits = pair_fits<pair::E4m3>(gated, p.K, p.out_width, p.scale_rows) || dual_fits(gated, p.K, p.out_width, p.out_codes != nullptr) ||
                    (gated ? prefill_fits<prefill::E4m3, true>(p.K, p.out_width)
                           : prefill_fits<prefill::E4m3, false>(p.K, p.out_width));
  if (!stream_path && fits) {
    PrefillParams q{};
    q.act = p.act;
    q.act_scales = p.act_scales;
    q.weights = p.weights;
    q.weight_scales = p.weight_scales;
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
    q.out_codes = p.out_codes;
    q.out_code_scales = p.out_code_scales;
    q.scale_rows = p.scale_rows;
    if (pair_fits<pair::E4m3>(gated, q.K, q.out_width, q.scale_rows)) {
      launch_pair<pair::E4m3>(q, gated, max_tiles, stream);
      return;
    }
    if (dual_fits(gated, q.K, q.out_width, q.out_codes != nullptr)) {
      launch_dual_e4m3(q, gated, max_tiles, stream);
      return;
    }
    if (gated) launch_prefill<prefill::E4m3, true>(q, max_tiles, stream);
    else launch_prefill<prefill::E4m3, false>(q, max_tiles, stream);
    return;
  }
  const int64_t slices = gated ? p.out_width / 64 : ceil_div<int64_t>(p.out_width, 128);
  const dim3 grid(static_cast<uint32_t>(max_tiles), static_cast<uint32_t>(slices));
  if (stream_path) {
    // Fewer workgroups than two per CU of a large part: split K over the waves instead.
    if (max_tiles * slices < kSplitBelow) {
      const int64_t split_slices = gated ? p.out_width / 16 : ceil_div<int64_t>(p.out_width, 32);
      const dim3 split_grid(static_cast<uint32_t>(max_tiles), static_cast<uint32_t>(split_slices));
      if (gated && one_pass) hipLaunchKernelGGL((stream_fp8_kernel<true, true, 1>), split_grid, dim3(kThreads), 0, stream, p);
      else if (gated) hipLaunchKernelGGL((stream_fp8_kernel<true, true, 2>), split_grid, dim3(kThreads), 0, stream, p);
      else if (one_pass) hipLaunchKernelGGL((stream_fp8_kernel<false, true, 1>), split_grid, dim3(kThreads), 0, stream, p);
      else hipLaunchKernelGGL((stream_fp8_kernel<false, true, 2>), split_grid, dim3(kThreads), 0, stream, p);
    } else if (gated) {
      if (one_pass) hipLaunchKernelGGL((stream_fp8_kernel<true, false, 1>), grid, dim3(kThreads), 0, stream, p);
      else hipLaunchKernelGGL((stream_fp8_kernel<true, false, 2>), grid, dim3(kThreads), 0, stream, p);
    } else {
      if (one_pass) hipLaunchKernelGGL((stream_fp8_kernel<false, false, 1>), grid, dim3(kThreads), 0, stream, p);
      else hipLaunchKernelGGL((stream_fp8_kernel<false, false, 2>), grid, dim3(kThreads), 0, stream, p);
    }
  } else {
    if (gated) hipLaunchKernelGGL(tiled_fp8_kernel<true>, grid, dim3(kThreads), 0, stream, p);
    else hipLaunchKernelGGL(tiled_fp8_kernel<false>, grid, dim3(kThreads), 0, stream, p);
  }
}

bool fp8_stream_path(int64_t routes, int64_t experts) { return routes < kStreamRowsPerExpert * experts; }

/// The split FC2 (few routes: 32-row slices, K over the waves): slices served per workgroup, one
/// after the other (a 235B FC2 slice of 32 rows is 48 KB of weights): 235B T=1 FC2 17.7-18.3 ->
/// 15.9 us by events with two (four: 23.2).
constexpr int kSplitFc2Run = 2;

bool expert_stream_fp8_fc1_quantizes(int64_t routes, int64_t local_experts, int64_t out_width) {
  const int64_t served = routes < local_experts ? routes : local_experts;
  return served * (out_width / 64) >= kSplitBelow && out_width % 128 == 0;
}

void launch_expert_stream_fp8(const GroupedFp8Params &params, bool gated, int64_t local_experts, hipStream_t stream) {
  GroupedFp8Params p = params;
  p.local_experts = local_experts;
  p.compact = p.routes < local_experts ? 1 : 0;
  const int64_t columns = p.compact ? p.routes : local_experts;  // workgroup columns
  const bool one_pass = p.routes <= kOnePassRowsPerExpert * local_experts;
  const int64_t slices = gated ? p.out_width / 64 : p.out_width / 128;
  // Workgroups with routes: at most one per route.
  const int64_t served = p.routes < local_experts ? p.routes : local_experts;
  if (served * slices < kSplitBelow) {
    const dim3 grid(static_cast<uint32_t>(columns), static_cast<uint32_t>(gated ? p.out_width / 16 : p.out_width / 32));
    const dim3 run_grid(static_cast<uint32_t>(columns), static_cast<uint32_t>(p.out_width / 32 / kSplitFc2Run));
    const bool runs = !gated && (p.out_width / 32) % kSplitFc2Run == 0;
    if (gated && one_pass) hipLaunchKernelGGL((stream_fp8_kernel<true, true, 1, true>), grid, dim3(kThreads), 0, stream, p);
    else if (gated) hipLaunchKernelGGL((stream_fp8_kernel<true, true, 2, true>), grid, dim3(kThreads), 0, stream, p);
    else if (runs && one_pass) hipLaunchKernelGGL((stream_fp8_kernel<false, true, 1, true, kSplitFc2Run>), run_grid, dim3(kThreads), 0, stream, p);
    else if (runs) hipLaunchKernelGGL((stream_fp8_kernel<false, true, 2, true, kSplitFc2Run>), run_grid, dim3(kThreads), 0, stream, p);
    else if (one_pass) hipLaunchKernelGGL((stream_fp8_kernel<false, true, 1, true>), grid, dim3(kThreads), 0, stream, p);
    else hipLaunchKernelGGL((stream_fp8_kernel<false, true, 2, true>), grid, dim3(kThreads), 0, stream, p);
    return;
  }
  if (gated && p.out_codes != nullptr) {
    // The gated rows also as FC2's operand: eight-wave workgroups of 128 gated columns.
    const dim3 grid(static_cast<uint32_t>(columns), static_cast<uint32_t>(p.out_width / 128));
    if (one_pass)
      hipLaunchKernelGGL((stream_fp8_kernel<true, false, 1, true, 1, 8, true>), grid, dim3(8 * kWave), 0, stream, p);
    else
      hipLaunchKernelGGL((stream_fp8_kernel<true, false, 2, true, 1, 8, true>), grid, dim3(8 * kWave), 0, stream, p);
    return;
  }
  const dim3 grid(static_cast<uint32_t>(columns), static_cast<uint32_t>(slices));
  if (gated && one_pass) hipLaunchKernelGGL((stream_fp8_kernel<true, false, 1, true>), grid, dim3(kThreads), 0, stream, p);
  else if (gated) hipLaunchKernelGGL((stream_fp8_kernel<true, false, 2, true>), grid, dim3(kThreads), 0, stream, p);
  else if (one_pass) hipLaunchKernelGGL((stream_fp8_kernel<false, false, 1, true>), grid, dim3(kThreads), 0, stream, p);
  else hipLaunchKernelGGL((stream_fp8_kernel<false, false, 2, true>), grid, dim3(kThreads), 0, stream, p);
}

}  // namespace uniserve

extern "C" int32_t uniserve_quantize_fp8(const uniserve_quantize_fp8_call *call, void *stream) {
  using namespace uniserve;
  return guarded(call, [&]() -> int32_t {
    if (call->input == nullptr || call->out == nullptr || call->scales == nullptr)
      return UNISERVE_REFUSE(call, "quantize_fp8 needs input, out and scales");
    if (call->group != 128) return UNISERVE_REFUSE(call, "quantize_fp8 quantises groups of 128 channels");
    if (call->width <= 0 || call->width % 128 != 0)
      return UNISERVE_REFUSE(call, "quantize_fp8 needs a width of whole 128-channel groups");
    if (call->input_dtype != UNISERVE_DTYPE_BF16 && call->input_dtype != UNISERVE_DTYPE_F32)
      return UNISERVE_REFUSE(call, "quantize_fp8 reads bf16 or f32 rows");
    if (call->rows < 0) return UNISERVE_REFUSE(call, "quantize_fp8 needs a non-negative row count");
    if (call->rows == 0) return 0;
    launch_quantize_fp8(call->input, call->input_dtype == UNISERVE_DTYPE_F32, static_cast<uint8_t *>(call->out),
                        call->scales, call->row_limit, call->rows, call->width, static_cast<hipStream_t>(stream));
    return launched(call, "quantize_fp8");
  });
}

namespace uniserve {

bool fp8_fc1_quantizes(int64_t tokens, int64_t top, int64_t experts, int64_t hidden_size, int64_t intermediate) {
  return !fp8_stream_path(tokens * top, experts) &&
         (dual_fits(true, hidden_size, intermediate, true) ||
          prefill_fits<prefill::E4m3, true>(hidden_size, intermediate));
}

bool fp8_route_scales(int64_t tokens, int64_t top, int64_t experts, int64_t hidden_size, int64_t intermediate,
                      int64_t permuted_rows) {
  const int64_t routes_bound = permuted_rows - (kTileRows - 1) * experts;
  return fp8_fc1_quantizes(tokens, top, experts, hidden_size, intermediate) &&
         !fp8_stream_path(routes_bound, experts) && prefill_fits<prefill::E4m3, false>(intermediate, hidden_size);
}

int32_t gather_gemm_fp8(const uniserve_gather_fp8_call *call, uint8_t *codes, float *code_scales,
                        int64_t scale_rows, int32_t activation, void *stream) {
  return guarded(call, [&]() -> int32_t {
    if (call->out_dtype != UNISERVE_DTYPE_BF16) return UNISERVE_REFUSE(call, "gather_gemm_fp8 writes bf16 only");
    if (call->block_n != 128 || call->block_k != 128)
      return UNISERVE_REFUSE(call, "gather_gemm_fp8 serves 128 x 128 weight blocks");
    if (call->hidden == nullptr || call->hidden_scales == nullptr || call->weights == nullptr ||
        call->weight_scales == nullptr || call->out == nullptr)
      return UNISERVE_REFUSE(call, "gather_gemm_fp8 needs hidden, weights, their scales and out");
    if (call->tile_to_expert == nullptr || call->tile_to_limit == nullptr ||
        call->permuted_to_expanded == nullptr || call->num_non_exiting_tiles == nullptr)
      return UNISERVE_REFUSE(call, "gather_gemm_fp8 needs the sort's tile and route maps");
    if (call->multiprocessors <= 0) return UNISERVE_REFUSE(call, "gather_gemm_fp8 needs its device's multiprocessor count");
    if (call->hidden_size <= 0 || call->hidden_size % 128 != 0)
      return UNISERVE_REFUSE(call, "gather_gemm_fp8 needs a hidden size of whole 128-element blocks");
    if (call->width <= 0 || call->width % 256 != 0)
      return UNISERVE_REFUSE(call, "gather_gemm_fp8 needs an intermediate width of whole 128-row blocks");
    if (call->tokens < 0 || call->top <= 0 || call->experts <= 0)
      return UNISERVE_REFUSE(call, "gather_gemm_fp8 needs non-negative tokens and positive top and experts");
    if (!dma_rows_fit(call->tokens, call->hidden_size))
      return UNISERVE_REFUSE(call, "gather_gemm_fp8 serves hidden rows below 4 GiB (%lld tokens of %lld bytes)",
                             static_cast<long long>(call->tokens), static_cast<long long>(call->hidden_size));
    if (call->permuted_rows < call->tokens * call->top || call->permuted_rows % kTileRows != 0)
      return UNISERVE_REFUSE(call, "gather_gemm_fp8 needs whole 128-row tiles that hold every route");
    const int64_t max_tiles = call->permuted_rows / kTileRows;
    if (max_tiles == 0) return 0;
    GroupedFp8Params p{};
    p.act = static_cast<const uint8_t *>(call->hidden);
    p.act_scales = call->hidden_scales;
    p.weights = static_cast<const uint8_t *>(call->weights);
    p.weight_scales = call->weight_scales;
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
    if (codes != nullptr) {
      if (!fp8_fc1_quantizes(call->tokens, call->top, call->experts, call->hidden_size, call->width / 2))
        return UNISERVE_REFUSE(call, "gather_gemm_fp8 quantises its output only on the prefill kernel's shapes");
      p.out_codes = codes;
      p.out_code_scales = code_scales;
    }
    if (scale_rows != 0) {
      if (codes == nullptr || scale_rows < call->permuted_rows)
        return UNISERVE_REFUSE(call, "gather_gemm_fp8 takes route-major scales only as it quantises its output");
      p.scale_rows = scale_rows;
    }
    launch_grouped_fp8(p, true, max_tiles, fp8_stream_path(call->tokens * call->top, call->experts),
                       call->tokens * call->top <= kOnePassRowsPerExpert * call->experts,
                       static_cast<hipStream_t>(stream));
    return launched(call, "gather_gemm_fp8");
  });
}

}  // namespace uniserve

extern "C" int32_t uniserve_gather_gemm_fp8(const uniserve_gather_fp8_call *call, void *stream) {
  return uniserve::gather_gemm_fp8(call, nullptr, nullptr, 0, UNISERVE_ACTIVATION_SILU, stream);
}

extern "C" int32_t uniserve_gather_gemm_fp8_gelu_tanh(const uniserve_gather_fp8_call *call, void *stream) {
  return uniserve::gather_gemm_fp8(call, nullptr, nullptr, 0, UNISERVE_ACTIVATION_GELU_TANH, stream);
}

extern "C" int32_t uniserve_route_gemm_fp8(const uniserve_route_fp8_call *call, void *stream) {
  return uniserve::route_gemm_fp8(call, 0, stream);
}

namespace uniserve {

int32_t route_gemm_fp8(const uniserve_route_fp8_call *call, int64_t scale_rows, void *stream) {
  return guarded(call, [&]() -> int32_t {
    if (call->out_dtype != UNISERVE_DTYPE_BF16) return UNISERVE_REFUSE(call, "route_gemm_fp8 writes bf16 only");
    if (call->block_n != 128 || call->block_k != 128)
      return UNISERVE_REFUSE(call, "route_gemm_fp8 serves 128 x 128 weight blocks");
    if (call->rows == nullptr || call->row_scales == nullptr || call->weights == nullptr ||
        call->weight_scales == nullptr || call->out == nullptr)
      return UNISERVE_REFUSE(call, "route_gemm_fp8 needs rows, weights, their scales and out");
    if (call->tile_to_expert == nullptr || call->tile_to_limit == nullptr ||
        call->permuted_to_expanded == nullptr || call->num_non_exiting_tiles == nullptr)
      return UNISERVE_REFUSE(call, "route_gemm_fp8 needs the sort's tile and route maps");
    if (call->multiprocessors <= 0) return UNISERVE_REFUSE(call, "route_gemm_fp8 needs its device's multiprocessor count");
    if (call->intermediate <= 0 || call->intermediate % 128 != 0)
      return UNISERVE_REFUSE(call, "route_gemm_fp8 needs an intermediate width of whole 128-element blocks");
    if (call->width <= 0 || call->width % 128 != 0)
      return UNISERVE_REFUSE(call, "route_gemm_fp8 needs a hidden width of whole 128-row blocks");
    if (call->experts <= 0) return UNISERVE_REFUSE(call, "route_gemm_fp8 needs positive experts");
    if (call->permuted_rows < 0 || call->permuted_rows % kTileRows != 0)
      return UNISERVE_REFUSE(call, "route_gemm_fp8 needs permuted rows of whole 128-row tiles");
    const int64_t max_tiles = call->permuted_rows / kTileRows;
    if (max_tiles == 0) return 0;
    GroupedFp8Params p{};
    p.act = static_cast<const uint8_t *>(call->rows);
    p.act_scales = call->row_scales;
    p.weights = static_cast<const uint8_t *>(call->weights);
    p.weight_scales = call->weight_scales;
    p.out = static_cast<uint16_t *>(call->out);
    p.tile_to_expert = call->tile_to_expert;
    p.tile_to_limit = call->tile_to_limit;
    p.permuted_to_expanded = call->permuted_to_expanded;
    p.num_tiles = call->num_non_exiting_tiles;
    p.K = call->intermediate;
    p.n_total = call->width;
    p.out_width = call->width;
    p.top = 1;
    const int64_t routes_bound = call->permuted_rows - (kTileRows - 1) * call->experts;
    const bool stream_path = fp8_stream_path(routes_bound, call->experts);
    if (scale_rows != 0) {
      if (stream_path || !prefill_fits<prefill::E4m3, false>(p.K, p.out_width) || scale_rows < call->permuted_rows)
        return UNISERVE_REFUSE(call, "route_gemm_fp8 takes route-major scales only on the prefill kernel's shapes");
      p.scale_rows = scale_rows;
    }
    launch_grouped_fp8(p, false, max_tiles, stream_path, routes_bound <= kOnePassRowsPerExpert * call->experts,
                       static_cast<hipStream_t>(stream));
    return launched(call, "route_gemm_fp8");
  });
}

}  // namespace uniserve

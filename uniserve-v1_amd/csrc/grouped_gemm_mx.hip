// SPDX-License-Identifier: Apache-2.0
//
// OCP MX forms of the grouped expert products on gfx950: MXFP4 (E2M1) expert weights times MXFP8
// (e4m3) activations, both with one E8M0 scale per 32 elements along K, and the MXFP8 activation
// quantiser. No reference counterpart (its four-bit experts are NVFP4, crates/ops/src/moe/
// grouped.rs:579-1772, in the same call style).
//
// `v_mfma_scale_f32_16x16x128_f8f6f4` takes an E2M1 A operand (cbsz 4, four registers) and an
// e4m3 B operand (blgp 0, eight registers), plus one E8M0 scale byte per lane for each. Measured on
// this GPU (single-element and scale-doubling probes): lane l = 16 g + r supplies, for row / column
// r, the E2M1 elements K 32 g .. 32 g + 31 (16 bytes, lower K in the low nibble) and the e4m3
// elements K 16 g .. 16 g + 15 and 64 + 16 g .. 64 + 16 g + 15 (two 16-byte pieces); its scale byte
// is that of row / column r's block g (K 32 g .. 32 g + 31), whichever lanes hold the block's data.
// So the hardware applies both MX block scales itself and the products accumulate straight into
// the FP32 accumulator: no per-block scaling on the VALU.
//
// Two product kernels, chosen by routes per expert as for the e4m3 products:
//  * decode shapes: the stream kernel (one tile x a slice of weight rows per workgroup; weights
//    streamed as whole 128-byte lines, non-temporal, and regrouped into the MFMA layout through
//    each wave's own LDS buffer), walking K 256 elements (one 128-byte weight line) at a time;
//  * prefill shapes: the tiled kernel (one 128-row tile x 256 weight rows per workgroup, two
//    workgroups per CU), both operands and both scale tables staged through LDS by DMA in two
//    stages of 128 K.
#include "common.hpp"
#include "grouped_fp8.hpp"
#include "expert_routes.hpp"
#include "expert_stream.hpp"
#include "grouped_mx.hpp"
#include "grouped_prefill.hpp"
#include "uniserve_moe_mx.h"

namespace uniserve {
namespace {

// ---- the MXFP8 quantiser -------------------------------------------------------------------------------

constexpr int kQuantThreads = 256;

struct MxQuantParams {
  const void *input;
  uint8_t *out;
  uint8_t *scales;               ///< row-major [rows, width / 32], or null
  const int32_t *row_limit;
  int64_t rows;
  int64_t width;
  int32_t input_f32;
  uint8_t *stage_scales;         ///< or null: stage-major [width / 128, stage_rows, 4]
  const int32_t *routes;         ///< with stage_scales, or null: row r's scales go to stage rows
                                 ///< routes[r * top + j] (>= 0) instead of row r
  int64_t top;
  int64_t stage_rows;
};

/// Four lanes per 32-channel block, eight channels each; a grid-stride loop that stops at the
/// device-side row limit.
__global__ void __launch_bounds__(kQuantThreads) quantize_mxfp8_kernel(MxQuantParams p) {
  const int64_t blocks_per_row = p.width / 32;
  const int sub = static_cast<int>(threadIdx.x) & 3;
  const int64_t limit = p.row_limit != nullptr ? p.row_limit[0] : p.rows;
  const int64_t last = (limit < p.rows ? limit : p.rows) * blocks_per_row;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kQuantThreads / 4;
  for (int64_t block = (static_cast<int64_t>(blockIdx.x) * kQuantThreads + threadIdx.x) / 4; block < last;
       block += stride) {
    const int64_t row = block / blocks_per_row;
    const int64_t column = (block % blocks_per_row) * 32 + sub * 8;
    float v[8];
    if (p.input_f32) {
      const float *src = static_cast<const float *>(p.input) + row * p.width + column;
      const float4 lo = *reinterpret_cast<const float4 *>(src);
      const float4 hi = *reinterpret_cast<const float4 *>(src + 4);
      v[0] = lo.x; v[1] = lo.y; v[2] = lo.z; v[3] = lo.w;
      v[4] = hi.x; v[5] = hi.y; v[6] = hi.z; v[7] = hi.w;
    } else {
      const u32x4 packed = *reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(p.input) + row * p.width + column);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[2 * j] = __uint_as_float(packed[j] << 16);
        v[2 * j + 1] = __uint_as_float(packed[j] & 0xffff0000u);
      }
    }
    const uint32_t scale = mxfp8_eight(v, p.out + row * p.width + column);
    if (sub == 0 && p.scales != nullptr) p.scales[block] = static_cast<uint8_t>(scale);
    if (p.stage_scales != nullptr) {
      const int64_t b = block % blocks_per_row;
      uint8_t *stage = p.stage_scales + (b / 4) * p.stage_rows * 4 + (b % 4);
      if (p.routes == nullptr) {
        if (sub == 0) stage[row * 4] = static_cast<uint8_t>(scale);
      } else {
        for (int64_t j = sub; j < p.top; j += 4) {
          const int32_t at = p.routes[row * p.top + j];
          if (at >= 0) stage[static_cast<int64_t>(at) * 4] = static_cast<uint8_t>(scale);
        }
      }
    }
  }
}

// ---- the products ----------------------------------------------------------------------------------------------

constexpr int kTileRows = 128;
constexpr int kThreads = 256;
constexpr int kPassTiles = 1;           // 16-token MFMA blocks per pass (one keeps three waves per SIMD)
constexpr int64_t kSplitBelow = 512;    // workgroups under which K is split over the waves

struct MxParams {
  const uint8_t *act;            ///< FC1: [tokens, K] e4m3; FC2: [permuted_rows, K]
  const uint8_t *act_scales;     ///< E8M0, see as_stage / as_row
  const uint8_t *weights;        ///< [experts, n_total, K / 2] E2M1 pairs
  const uint8_t *weight_scales;  ///< E8M0, [experts, n_total, K / 32] bytes in either layout
  uint16_t *out;                 ///< [permuted_rows, out_width] bf16
  const int32_t *tile_to_expert;
  const int32_t *tile_to_limit;
  const int32_t *permuted_to_expanded;
  const int32_t *num_tiles;
  int64_t K;
  int64_t n_total;
  int64_t out_width;
  int64_t top;
  // The 4-byte word of a row's scales of 128-element stage k sits at k * stage + row * row_bytes
  // (row-major: stage 4, row K / 32; stage-major: stage rows * 4, row 4), per expert for weights.
  int64_t ws_stage;
  int64_t ws_row;
  int64_t as_stage;
  int64_t as_row;
  int32_t as_by_route;           ///< activation scale rows are permuted rows, not act rows
  int32_t activation;            ///< FC1's gate: UNISERVE_ACTIVATION_SILU or _GELU_TANH
  // Expert-major stream (decode, no sort): workgroup x serves local expert x (or, compact, the
  // x-th named one), whose rows are the routes naming it in `ids`, at their expanded positions.
  const int32_t *ids;
  const int32_t *live_tokens;
  int64_t routes;
  int64_t local_offset;
  int64_t local_experts;
  int32_t compact;
  // FC1 on the tiled kernel only, or null: the gated rows are written as MXFP8 codes
  // [permuted_rows, out_width] with their E8M0 bytes stage-major by permuted row
  // ([out_width / 128, code_scale_rows, 4]) instead of bf16 rows - FC2's operand.
  uint8_t *out_codes;
  uint8_t *out_code_scales;
  int64_t code_scale_rows;
};

/// Stride words of a scale table with `rows` rows in `layout`.
inline void scale_strides(int64_t layout, int64_t rows, int64_t K, int64_t *stage, int64_t *row) {
  if (layout == UNISERVE_MX_SCALES_STAGE_MAJOR) {
    *stage = rows * 4;
    *row = 4;
  } else {
    *stage = 4;
    *row = K / 32;
  }
}

__device__ __forceinline__ void store_bf16x4(uint16_t *pointer, floatx4 v) {
  uint2 packed;
  packed.x = pack_bf16x2(v[0], v[1]);
  packed.y = pack_bf16x2(v[2], v[3]);
  *reinterpret_cast<uint2 *>(pointer) = packed;
}

/// D += (E2M1 A scaled by 2^(sa - 127)) . (e4m3 B scaled by 2^(sb - 127)) over 128 K; the scales
/// are this lane's bytes (its row and its 32 K elements).
__device__ __forceinline__ floatx4 mfma_mx(const u32x4 &a, const intx8 &b, uint32_t sa, uint32_t sb, floatx4 c) {
  const intx8 a8 = intx8{static_cast<int>(a[0]), static_cast<int>(a[1]), static_cast<int>(a[2]), static_cast<int>(a[3]),
                         0, 0, 0, 0};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a8, b, c, 4, 0, 0, static_cast<int>(sa), 0,
                                                          static_cast<int>(sb));
}

/// One tile x a slice of weight rows per workgroup; each wave owns two sets of 16 weight rows
/// (FC1: 16 up rows and the matching 16 gate rows; FC2: 32 consecutive rows). K walks in 256-element
/// chunks: one 128-byte line of each weight row, i.e. two 16x16x128 MFMAs per set (h = 0, 1).
/// kSplit: the four waves share one row set and split the chunks (chunk c to wave c % 4), their
/// partial sums meeting in LDS in wave order - for batches too small to fill the chip otherwise.
/// kByExpert: the rows are the routes naming the workgroup's local expert (FC1 reads token route /
/// top, FC2 row `route`; both write row `route`), listed by the workgroup while its first weight
/// chunk is in flight. kRun (expert-major): the workgroup serves kRun consecutive slices one after
/// the other, listing the routes once (grid y = slices / kRun).
/// kQuantOut (expert-major FC1, unsplit): the gated rows also leave as FC2's MXFP8 operand - the
/// workgroup's 64 columns are two whole 32-column blocks, staged through LDS as the bf16 values the
/// quantiser would read, then quantised by its routine (codes [routes, out_width] at out_codes,
/// row-major E8M0 bytes [routes, out_width / 32] at out_code_scales).
template <bool kGated, bool kSplit, bool kByExpert = false, int kRun = 1, bool kQuantOut = false>
__global__ void __launch_bounds__(kThreads) stream_mx_kernel(MxParams p) {
  static_assert(!kQuantOut || (kGated && !kSplit && kByExpert && kRun == 1), "MXFP8 out: expert-major FC1");
  __shared__ uint16_t gated_tile[kQuantOut ? 16 * 64 : 1];
  static_assert(kRun == 1 || kByExpert, "runs of slices: expert-major");
  __shared__ floatx4 partial[kSplit ? kThreads / kWave - 1 : 1][2][kPassTiles][kWave];
  __shared__ int32_t route_list[kByExpert ? kExpertRoutes : 1];
  __shared__ int32_t route_count[kThreads / kWave + 1];
  __shared__ u32x4 regroup[kThreads / kWave][4 * 64];  // each wave's weight lines, regrouped
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
    return listed_route<kThreads / kWave>(route_list, route_count, p.routes, m);
  };
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int lane = lane_id();
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int64_t chunks = p.K / 256;
  const int64_t weight_row_bytes = p.K / 2;
  const int64_t scale_row_bytes = p.K / 32;

  int64_t n0, n1;
  const int row_set = kSplit ? 0 : wave;
  auto slice_rows = [&](int64_t slice) {
    if constexpr (kGated) {
      n0 = slice * (kSplit ? 16 : 64) + row_set * 16;
      n1 = p.out_width + n0;
    } else {
      n0 = slice * (kSplit ? 32 : 128) + row_set * 32;
      n1 = n0 + 16;
    }
  };
  slice_rows(static_cast<int64_t>(blockIdx.y) * kRun);
  if constexpr (!kGated && !kByExpert) {
    if (n0 >= p.out_width) return;  // (expert-major: whole slices only)
  }
  const int64_t c_first = kSplit ? wave : 0;
  const int64_t c_step = kSplit ? kThreads / kWave : 1;
  // Weight lines: load i (0..3) of a chunk reads rows 8 (i % 2) + l / 8 of set i / 2, 16-byte piece
  // l % 8 of the row's 128-byte line. Lane l's A operand for MFMA h (row r16, K 128 h + 32 g ..)
  // is piece 4 h + g of row r16, regrouped through LDS. This lane's weight scales: its row r16 of
  // each set, two 4-byte stage words per chunk. Every address is a uniform base (the expert's
  // tables, the activation arrays) plus a 32-bit lane offset, so the loads take the scalar-base
  // form and each address costs one VGPR.
  expert = __builtin_amdgcn_readfirstlane(static_cast<int>(expert));
  const uint8_t *wbase = p.weights + expert * p.n_total * weight_row_bytes;
  const uint8_t *sbase = p.weight_scales + expert * p.n_total * scale_row_bytes;
  uint32_t line_off[2], ws_off[2];
  auto slice_pointers = [&]() {
    line_off[0] = static_cast<uint32_t>((n0 + lane / 8) * weight_row_bytes + (lane & 7) * 16);
    line_off[1] = static_cast<uint32_t>((n1 + lane / 8) * weight_row_bytes + (lane & 7) * 16);
    ws_off[0] = static_cast<uint32_t>((n0 + r16) * p.ws_row);
    ws_off[1] = static_cast<uint32_t>((n1 + r16) * p.ws_row);
  };
  slice_pointers();

  // One chunk's operands: four weight lines, two 8-byte weight-scale words, and per token block
  // 64 activation bytes (two MFMAs' worth: pieces g and g + 4 of each 128-byte half) and an
  // 8-byte activation-scale word.
  struct Chunk {
    u32x4 lines[4];
    uint2 wscale[2];
    intx8 x[kPassTiles][2];
    uint2 xscale[kPassTiles];
  };
  const uint32_t row8 = static_cast<uint32_t>(8 * weight_row_bytes);
  auto fetch_lines = [&](int64_t c, Chunk &d) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      d.lines[i] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4 *>(wbase + (line_off[i / 2] + (i % 2) * row8 + static_cast<uint32_t>(c) * 128u)));
  };
  Chunk cur, next;
  if constexpr (kByExpert) {
    const FirstRouteIds first_ids = load_first_route_ids<kThreads / kWave>(p.ids, p.routes);  // (before the lines)
    if (!kSplit) fetch_lines(c_first, cur);  // it depends on nothing the routes decide
    const int64_t live = p.live_tokens != nullptr ? static_cast<int64_t>(p.live_tokens[0]) * p.top : p.routes;
    rows = list_expert_routes<kThreads / kWave>(p.ids, p.routes, live, static_cast<int32_t>(expert + p.local_offset),
                                                route_list, route_count, &first_ids);
    if (rows == 0) return;
  }

  for (int run = 0; run < kRun; ++run) {
  if (run > 0) {
    slice_rows(static_cast<int64_t>(blockIdx.y) * kRun + run);
    slice_pointers();
  }
  for (int pass = 0; pass < rows; pass += 16 * kPassTiles) {
    uint32_t a_off[kPassTiles];
    uint32_t as_off[kPassTiles];
    const uint32_t as_stage = static_cast<uint32_t>(p.as_stage);
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
      a_off[ms] = static_cast<uint32_t>(source * p.K + g * 16);
      as_off[ms] = static_cast<uint32_t>((p.as_by_route ? first + (valid[ms] ? m : 0) : source) * p.as_row);
    }
    floatx4 acc[2][kPassTiles];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int ms = 0; ms < kPassTiles; ++ms) acc[s][ms] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    auto fetch_rest = [&](int64_t c, Chunk &d) {
#pragma unroll
      for (int s = 0; s < 2; ++s)
        d.wscale[s] = uint2{*reinterpret_cast<const uint32_t *>(sbase + (ws_off[s] + 2u * static_cast<uint32_t>(c) * static_cast<uint32_t>(p.ws_stage))),
                            *reinterpret_cast<const uint32_t *>(sbase + (ws_off[s] + (2u * static_cast<uint32_t>(c) + 1u) * static_cast<uint32_t>(p.ws_stage)))};
#pragma unroll
      for (int ms = 0; ms < kPassTiles; ++ms) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const u32x4 lo = *reinterpret_cast<const u32x4 *>(p.act + (a_off[ms] + static_cast<uint32_t>(c) * 256u + h * 128u));
          const u32x4 hi = *reinterpret_cast<const u32x4 *>(p.act + (a_off[ms] + static_cast<uint32_t>(c) * 256u + h * 128u + 64u));
          d.x[ms][h] = intx8{static_cast<int>(lo[0]), static_cast<int>(lo[1]), static_cast<int>(lo[2]), static_cast<int>(lo[3]),
                             static_cast<int>(hi[0]), static_cast<int>(hi[1]), static_cast<int>(hi[2]), static_cast<int>(hi[3])};
        }
        if constexpr (kByExpert)  // row-major activation scales: the chunk's two words are adjacent
          d.xscale[ms] = *reinterpret_cast<const uint2 *>(p.act_scales + (as_off[ms] + 8u * static_cast<uint32_t>(c)));
        else
          d.xscale[ms] = uint2{*reinterpret_cast<const uint32_t *>(p.act_scales + (as_off[ms] + 2u * static_cast<uint32_t>(c) * as_stage)),
                               *reinterpret_cast<const uint32_t *>(p.act_scales + (as_off[ms] + (2u * static_cast<uint32_t>(c) + 1u) * as_stage))};
      }
    };
    auto fetch = [&](int64_t c, Chunk &d) {
      fetch_lines(c, d);
      fetch_rest(c, d);
    };
    // Byte 4 h + g of an 8-byte scale word: this lane's block of MFMA h.
    auto scale_byte = [&](const uint2 &word, int h) -> uint32_t { return ((h == 0 ? word.x : word.y) >> (8 * g)) & 0xffu; };
    auto compute = [&](const Chunk &d) {
      // The four lines go through the wave's own LDS buffer into the operand layout: load i's lane
      // l (row 8 (i % 2) + l / 8 of set i / 2, piece l % 8) at slot 64 i + 8 r + (piece ^ r), r = l / 8,
      // so the 16 lanes that read one piece of 8 rows read 8 different bank groups.
      {
        const int row = lane >> 3, piece = lane & 7;
#pragma unroll
        for (int i = 0; i < 4; ++i) regroup[wave][i * 64 + row * 8 + (piece ^ row)] = d.lines[i];
      }
#pragma unroll
      for (int set = 0; set < 2; ++set) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int rr = r16 & 7, q = 4 * h + g;
          const u32x4 w = regroup[wave][(2 * set + (r16 >> 3)) * 64 + rr * 8 + (q ^ rr)];
          const uint32_t sw = scale_byte(d.wscale[set], h);
#pragma unroll
          for (int ms = 0; ms < kPassTiles; ++ms)
            acc[set][ms] = mfma_mx(w, d.x[ms][h], sw, scale_byte(d.xscale[ms], h), acc[set][ms]);
        }
      }
    };
    if (kByExpert && !kSplit && pass == 0 && run == 0) fetch_rest(c_first, cur);  // its lines went out before the scan
    else if (c_first < chunks) fetch(c_first, cur);
    // The steady walk issues both chunks' loads unconditionally, so the compiler's wait before
    // each compute counts exactly the other chunk's loads still in flight (with the loads under
    // conditions it waited for every load, the prefetched chunk's too); the last one or two
    // chunks are peeled.
    int64_t c = c_first;
    if (c < chunks) {
      for (; c + 2 * c_step < chunks; c += 2 * c_step) {
        fetch(c + c_step, next);
        // The prefetch goes out before cur's data is waited for: left to itself the scheduler
        // hoists cur's LDS regroup (which waits for cur's lines) above the next chunk's loads (30B
        // T=64 FC1 44 -> 41.6 us, FC2 26.2 -> 24.8; the bf16 and e4m3 stream kernels gain nothing).
        __builtin_amdgcn_sched_barrier(0);
        compute(cur);
        fetch(c + 2 * c_step, cur);
        __builtin_amdgcn_sched_barrier(0);
        compute(next);
      }
      if (c + c_step < chunks) {
        fetch(c + c_step, next);
        __builtin_amdgcn_sched_barrier(0);
        compute(cur);
        compute(next);
      } else {
        compute(cur);
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
        for (int w = 0; w < kThreads / kWave - 1; ++w)
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
        floatx4 v;
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = gate(acc[1][ms][i], p.activation) * acc[0][ms][i];
        store_bf16x4(row + n0 + 4 * g, v);
        if constexpr (kQuantOut) {
          uint2 packed;
          packed.x = pack_bf16x2(v[0], v[1]);
          packed.y = pack_bf16x2(v[2], v[3]);
          *reinterpret_cast<uint2 *>(gated_tile + r16 * 64 + wave * 16 + 4 * g) = packed;
        }
      } else {
        store_bf16x4(row + n0 + 4 * g, acc[0][ms]);
        store_bf16x4(row + n1 + 4 * g, acc[1][ms]);
      }
    }
    if constexpr (kQuantOut) {
      // The tile's 16 rows x two 32-column blocks, four lanes a block (the first two waves).
      __syncthreads();
      const int t = static_cast<int>(threadIdx.x);
      const int r = t / 8, block = (t / 4) & 1, sub = t & 3;
      const int m = pass + r;
      if (t < 128 && m < rows) {
        const u32x4 bits = *reinterpret_cast<const u32x4 *>(gated_tile + r * 64 + block * 32 + sub * 8);
        float v[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[2 * j] = __uint_as_float(bits[j] << 16);
          v[2 * j + 1] = __uint_as_float(bits[j] & 0xffff0000u);
        }
        const int64_t route = listed(m);
        const int64_t column = static_cast<int64_t>(blockIdx.y) * 64 + block * 32;
        const uint32_t scale = mxfp8_eight(v, p.out_codes + route * p.out_width + column + sub * 8);
        if (sub == 0) p.out_code_scales[route * (p.out_width / 32) + column / 32] = static_cast<uint8_t>(scale);
      }
      __syncthreads();
    }
  }
  }
}

// ---- the tiled (prefill) kernel ---------------------------------------------------------------------------
//
// One workgroup of 4 wavefronts owns one 128-row sort tile and 256 weight rows of its expert (FC1:
// 128 up rows and the matching 128 gate rows; FC2: 256 output columns); two workgroups share a CU
// (two waves per SIMD, one from each), so one workgroup's barrier, DMA wait or epilogue is covered
// by the other's MFMAs. Wave (t, w) of the 2 x 2 arrangement multiplies tile rows
// 64 t .. 64 t + 63 (four 16-row token blocks) by slice rows 128 w .. 128 w + 127 (eight 16-row
// weight blocks; FC1: 64 up rows then the 64 gate rows of the same columns): 32 MFMAs of 16x16x128
// per 128-K stage into 32 accumulators of four floats.
//
// A stage holds, per row, 128 e4m3 activation bytes (8 chunks of 16), 64 bytes of E2M1 weight pairs
// (4 chunks) and a 4-byte word of E8M0 scales for each operand (the stage's four 32-element
// blocks). Every byte arrives by DMA (`global_load_lds_dword[x4]`), ten instructions per wave per
// stage, so the loop counts its loads exactly: two stages, stage k + 1 issued while stage k
// multiplies, one barrier per stage. Chunk c of a row sits at c ^ key(row) (activation rows:
// (r >> 1) & 7; weight rows: (r >> 1) & 3, both measured free of bank conflicts for these reads).

constexpr int kSliceRows = 256;                       // weight rows per workgroup

struct MxTiledParams {
  MxParams base;
  int32_t slices;          ///< weight-row slices per tile
  int32_t max_tiles;
  int32_t group;           ///< tiles per group of the numbering
  int32_t groups_per_xcd;
};

/// One stage of kWaves waves: wave w's scale instruction writes 64 words at 64 w (its rows first).
template <int kWaves>
struct MxStage {
  u32x4 act[kTileRows * 8];        // 16 KB
  u32x4 weights[kSliceRows * 4];   // 16 KB
  uint32_t weight_scales[kWaves * kWave];
  uint32_t act_scales[kWaves * kWave];
};

__device__ __forceinline__ int act_slot(int row, int chunk) { return row * 8 + (chunk ^ ((row >> 1) & 7)); }
__device__ __forceinline__ int weight_slot(int row, int chunk) { return row * 4 + (chunk ^ ((row >> 1) & 3)); }

/// One 4-byte DMA per lane from `base` + `offset` into LDS at `lds` + 4 * lane (see `dma16`).
__device__ __forceinline__ void dma4(const void *base, uint32_t offset, uint32_t lds) {
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dword %0, %1\n\t"
      :
      : "v"(offset), "s"(base), "s"(lds)
      : "m0");
}

/// kWaves = 4, kStages = 2: two workgroups per CU. kWaves = 8, kStages = 4: one workgroup per CU
/// with three stages in flight.
template <bool kGated, int kWaves, int kStages>
__global__ void __launch_bounds__(kWaves * kWave, 8 / kWaves) tiled_mx_kernel(MxTiledParams tp) {
  using prefill::dma16;
  using prefill::lds_address;
  constexpr int kThreadsHere = kWaves * kWave;
  constexpr int kRowsPerWave = kSliceRows / (kWaves / 2);  // weight rows of one wave (2 x kWaves/2)
  constexpr int kBlocks = kRowsPerWave / 16;               // its 16-row weight blocks
  constexpr int kCols = kRowsPerWave / 2;                  // FC1: its up (and gate) rows
  constexpr int kActLoads = 16 / kWaves;                   // 8-row activation DMAs per wave
  constexpr int kWeightLoads = 16 / kWaves;                // 16-row weight DMAs per wave
  constexpr int kLoads = kActLoads + kWeightLoads + 2;
  constexpr int kActRows = kTileRows / kWaves;             // rows whose scales a wave brings
  constexpr int kWeightRows = kSliceRows / kWaves;
  const MxParams &p = tp.base;
  __shared__ MxStage<kWaves> ring[kStages];

  // ---- the work item: groups of `group` tiles, slice-major inside a group, dealt to the XCDs in
  // turn (block b runs on XCD b % 8) ----
  const int b = static_cast<int>(blockIdx.x);
  const int span = tp.group * tp.slices;
  const int seq = b >> 3;
  const int group_index = (seq / span) * 8 + (b & 7);
  const int first_tile = group_index * tp.group;
  if (first_tile >= tp.max_tiles) return;
  const int in_group = min(tp.group, tp.max_tiles - first_tile);
  const int within = seq - (seq / span) * span;
  if (within >= in_group * tp.slices) return;
  const int slice = within / in_group;
  const int tile = first_tile + within % in_group;
  if (tile >= p.num_tiles[0]) return;

  const int64_t expert = p.tile_to_expert[tile];
  const int64_t first = static_cast<int64_t>(tile) * kTileRows;
  const int rows = p.tile_to_limit[tile] - static_cast<int>(first);
  const int t = static_cast<int>(threadIdx.x);
  const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
  const int wt = wave & 1;   // token half
  const int ww = wave >> 1;  // weight part
  const int lane = lane_id();
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int stages = static_cast<int>(p.K / 128);
  const int64_t weight_row_bytes = p.K / 2;
  const int64_t scale_row_bytes = p.K / 32;
  const int top = static_cast<int>(p.top);
  // The activation row behind tile row r (FC1 gathers tokens; padding rows read row 0 or the
  // tile's first row).
  auto source_row = [&](int r) -> int64_t {
    if constexpr (kGated) {
      const int expanded = p.permuted_to_expanded[first + r];
      return r < rows ? static_cast<int64_t>(expanded / top) : 0;
    } else {
      return r < rows ? first + r : first;
    }
  };
  // The activation DMA's base: FC2's rows are the tile's own, addressed from the tile's first row,
  // so their 32-bit lane offsets stay under 128 rows whatever the array's size; FC1's gathered
  // token rows are addressed from the array, which the hosts hold below 4 GiB (dma_rows_fit).
  const uint8_t *act_tile = p.act + (kGated ? 0 : first * p.K);
  auto act_row = [&](int r) -> int64_t { return kGated ? source_row(r) : source_row(r) - first; };

  // ---- DMA sources (32-bit lane offsets from wave-uniform bases) ----
  // Activations: wave w's instruction i fills tile rows 8 (kActLoads w + i) + l / 8, lane l
  // bringing logical chunk (l % 8) ^ key(row) into physical chunk l % 8; its scale instruction
  // brings the scale words of tile rows kActRows w + l % kActRows (the other lanes repeat them into
  // the padding).
  uint32_t a_off[kActLoads];
#pragma unroll
  for (int i = 0; i < kActLoads; ++i) {
    const int r = 8 * (kActLoads * wave + i) + lane / 8;
    a_off[i] = static_cast<uint32_t>(act_row(r) * p.K + ((lane & 7) ^ ((r >> 1) & 7)) * 16);
  }
  const int as_r = kActRows * wave + lane % kActRows;
  const uint32_t as_off = static_cast<uint32_t>(
      (p.as_by_route ? first + (as_r < rows ? as_r : 0) : source_row(as_r)) * p.as_row);
  // Weights: slice row j = kRowsPerWave w + jj belongs to wave part w: for FC1 jj < kCols is up row
  // col and jj >= kCols gate row out_width + col, col = slice_col + kCols w + jj % kCols; for FC2
  // row slice_col + j. Wave w's instruction i fills slice rows 16 (kWeightLoads w + i) + l / 4
  // (logical chunk (l % 4) ^ key into physical chunk l % 4, key = (l / 8) % 4); its scale
  // instruction the words of rows kWeightRows w + l % kWeightRows.
  const int64_t slice_col = static_cast<int64_t>(slice) * (kGated ? kSliceRows / 2 : kSliceRows);
  auto weight_row = [&](int j) -> int64_t {
    if constexpr (kGated) {
      const int jj = j % kRowsPerWave;
      const int64_t col = slice_col + kCols * (j / kRowsPerWave) + jj % kCols;
      return jj >= kCols ? p.out_width + col : col;
    } else {
      return slice_col + j;
    }
  };
  const uint8_t *expert_weights = p.weights + expert * p.n_total * weight_row_bytes;
  const uint32_t w_off = static_cast<uint32_t>((lane / 4) * weight_row_bytes + ((lane & 3) ^ ((lane >> 3) & 3)) * 16);
  const uint8_t *expert_scales = p.weight_scales + expert * p.n_total * scale_row_bytes;
  const uint32_t ws_off = static_cast<uint32_t>(weight_row(kWeightRows * wave + lane % kWeightRows) * p.ws_row);

  auto issue = [&](MxStage<kWaves> &st, int k) {
    const uint32_t act_lds = lds_address(st.act + wave * kActLoads * kWave);
#pragma unroll
    for (int i = 0; i < kActLoads; ++i)
      dma16(act_tile + static_cast<int64_t>(k) * 128, a_off[i], __builtin_amdgcn_readfirstlane(act_lds + i * kWave * 16));
    const uint32_t weight_lds = lds_address(st.weights + wave * kWeightLoads * kWave);
#pragma unroll
    for (int i = 0; i < kWeightLoads; ++i)
      dma16(expert_weights + weight_row(16 * (kWeightLoads * wave + i)) * weight_row_bytes + static_cast<int64_t>(k) * 64,
            w_off, __builtin_amdgcn_readfirstlane(weight_lds + i * kWave * 16));
    dma4(expert_scales + static_cast<int64_t>(k) * p.ws_stage, ws_off,
         __builtin_amdgcn_readfirstlane(lds_address(st.weight_scales + wave * kWave)));
    dma4(p.act_scales + static_cast<int64_t>(k) * p.as_stage, as_off,
         __builtin_amdgcn_readfirstlane(lds_address(st.act_scales + wave * kWave)));
  };

  floatx4 acc[4][kBlocks];
#pragma unroll
  for (int tb = 0; tb < 4; ++tb)
#pragma unroll
    for (int jb = 0; jb < kBlocks; ++jb) acc[tb][jb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  auto compute = [&](const MxStage<kWaves> &st) {
    u32x4 wf[kBlocks];
    uint32_t sw[kBlocks];
#pragma unroll
    for (int jb = 0; jb < kBlocks; ++jb) {
      const int row = ww * kRowsPerWave + jb * 16 + r16;
      wf[jb] = st.weights[weight_slot(row, g)];
      sw[jb] = reinterpret_cast<const uint8_t *>(st.weight_scales)[((row / kWeightRows) * kWave + row % kWeightRows) * 4 + g];
    }
    // Every token block's fragment and scale is read before the first MFMA: the reads' latency
    // is paid once per stage, not once per token block.
    intx8 x[4];
    uint32_t sx[4];
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      const int row = wt * 64 + tb * 16 + r16;
      const u32x4 lo = st.act[act_slot(row, g)];
      const u32x4 hi = st.act[act_slot(row, g + 4)];
      x[tb] = intx8{static_cast<int>(lo[0]), static_cast<int>(lo[1]), static_cast<int>(lo[2]), static_cast<int>(lo[3]),
                    static_cast<int>(hi[0]), static_cast<int>(hi[1]), static_cast<int>(hi[2]), static_cast<int>(hi[3])};
      sx[tb] = reinterpret_cast<const uint8_t *>(st.act_scales)[((row / kActRows) * kWave + row % kActRows) * 4 + g];
    }
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
      for (int jb = 0; jb < kBlocks; ++jb) acc[tb][jb] = mfma_mx(wf[jb], x[tb], sw[jb], sx[tb], acc[tb][jb]);
    // Pinned: the compiler would otherwise sink each token block's reads to just before its
    // MFMAs (235B FC1 479 us unpinned, 460 pinned).
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * kBlocks + 12, 0);  // all LDS reads
    __builtin_amdgcn_sched_group_barrier(0x008, 4 * kBlocks, 0);       // then the MFMAs
  };

  // ---- the K loop: at the top of stage k, stages k .. k + kStages - 2 are in flight; once stage k
  // has landed for every wave (own wait - loads complete in issue order - then the barrier, which
  // also retires every wave's reads of stage k - 1), stage k + kStages - 1 is issued into the
  // buffer stage k - 1 used. Issues past the last stage re-read it, so every wait counts the same
  // loads. ----
#pragma unroll
  for (int k = 0; k < kStages - 1; ++k) issue(ring[k], min(k, stages - 1));
  for (int k = 0; k < stages; ++k) {
    prefill::wait_loads_but<(kStages - 2) * kLoads>();
    __syncthreads();
    issue(ring[(k + kStages - 1) % kStages], min(k + kStages - 1, stages - 1));
    compute(ring[k % kStages]);
  }
  prefill::wait_all_loads();
  __syncthreads();  // every wave is done reading the stage buffers

  // ---- epilogue: lane (r16, g) holds, of token block tb and weight block jb, tile row
  // 64 t + 16 tb + r16 and the wave's weight rows 16 jb + 4 g + i in element i. The output tile goes
  // through LDS so the global stores are whole rows; LDS rows are padded by 16 bytes. ----
  constexpr int kOutCols = kGated ? kSliceRows / 2 : kSliceRows;
  constexpr int kOutStride = kOutCols * 2 + 16;
  static_assert(kTileRows * kOutStride <= static_cast<int>(sizeof(ring)), "the output tile fits the stages");
  char *tile_lds = reinterpret_cast<char *>(ring);
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) {
    char *row = tile_lds + (wt * 64 + tb * 16 + r16) * kOutStride;
    if constexpr (kGated) {
#pragma unroll
      for (int jb = 0; jb < kBlocks / 2; ++jb) {
        floatx4 v;
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = gate(acc[tb][jb + kBlocks / 2][i], p.activation) * acc[tb][jb][i];
        store_bf16x4(reinterpret_cast<uint16_t *>(row + (ww * kCols + jb * 16 + 4 * g) * 2), v);
      }
    } else {
#pragma unroll
      for (int jb = 0; jb < kBlocks; ++jb)
        store_bf16x4(reinterpret_cast<uint16_t *>(row + (ww * kRowsPerWave + jb * 16 + 4 * g) * 2), acc[tb][jb]);
    }
  }
  __syncthreads();
  if (kGated && p.out_codes != nullptr) {
    // The gated rows as FC2's MXFP8 operand, straight from the staged bf16 tile (the quantiser's
    // rounding points and encoding: each 32-column block by four lanes, its E8M0 byte from the
    // block's bf16 values): the slice's 128 columns are one 128-element stage, so each row's four
    // scale bytes make its one stage-major word. Live rows only.
    constexpr int kLanesPerRow = kOutCols / 8;  // 16
    const int sub = t % kLanesPerRow;
    uint8_t *stage_scales = p.out_code_scales + (slice_col / 128) * p.code_scale_rows * 4;
    for (int m = t / kLanesPerRow; m < kTileRows; m += kThreadsHere / kLanesPerRow) {
      if (m >= rows) continue;  // a row's lanes are the four lanes of each of its blocks
      const u32x4 packed = *reinterpret_cast<const u32x4 *>(tile_lds + m * kOutStride + sub * 16);
      float v[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[2 * j] = __uint_as_float(packed[j] << 16);
        v[2 * j + 1] = __uint_as_float(packed[j] & 0xffff0000u);
      }
      const uint32_t scale = mxfp8_eight(v, p.out_codes + (first + m) * p.out_width + slice_col + sub * 8);
      if ((sub & 3) == 0) stage_scales[(first + m) * 4 + sub / 4] = static_cast<uint8_t>(scale);
    }
    return;
  }
  constexpr int kPieces = kOutCols / 8;
  for (int index = t; index < kTileRows * kPieces; index += kThreadsHere) {
    const int m = index / kPieces;
    const int c = index - m * kPieces;
    if (m >= rows) continue;
    const u32x4 piece = *reinterpret_cast<const u32x4 *>(tile_lds + m * kOutStride + c * 16);
    *reinterpret_cast<u32x4 *>(p.out + (first + m) * p.out_width + slice_col + c * 8) = piece;
  }
}

/// Whether the tiled kernel serves the shape: whole 128-K stages and whole 256-row weight slices.
bool tiled_fits(bool gated, int64_t K, int64_t out_width) {
  return K % 128 == 0 && K > 0 && out_width % (gated ? kSliceRows / 2 : kSliceRows) == 0;
}

void launch_tiled_mx(const MxParams &p, bool gated, int64_t max_tiles, hipStream_t stream) {
  MxTiledParams tp{};
  tp.base = p;
  tp.slices = static_cast<int32_t>(p.out_width / (gated ? kSliceRows / 2 : kSliceRows));
  tp.max_tiles = static_cast<int32_t>(max_tiles);
  tp.group = 4;  // tiles per group of the work numbering (4 measured best: 235B FC1 475 us against 497 at 16)
  tp.groups_per_xcd = static_cast<int32_t>(ceil_div<int64_t>(ceil_div<int64_t>(max_tiles, tp.group), 8));
  const int64_t blocks = static_cast<int64_t>(tp.groups_per_xcd) * tp.group * tp.slices * 8;
  constexpr int W = 4, S = 2;  // two workgroups per CU (measured better than 8 waves x 4 stages)
  if (gated) hipLaunchKernelGGL((tiled_mx_kernel<true, W, S>), dim3(static_cast<uint32_t>(blocks)), dim3(W * kWave), 0, stream, tp);
  else hipLaunchKernelGGL((tiled_mx_kernel<false, W, S>), dim3(static_cast<uint32_t>(blocks)), dim3(W * kWave), 0, stream, tp);
}

/// Row-major [stacks, rows, width / 32] scale bytes to stage-major: one thread per 4-byte word.
__global__ void __launch_bounds__(256) stage_major_kernel(const uint8_t *in, uint8_t *out, int64_t stacks, int64_t rows,
                                                          int64_t width) {
  const int64_t stages = width / 128;
  const int64_t words = stacks * stages * rows;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t w = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; w < words; w += stride) {
    const int64_t n = w % rows;
    const int64_t k = (w / rows) % stages;
    const int64_t stack = w / (rows * stages);
    const uint32_t word = *reinterpret_cast<const uint32_t *>(in + (stack * rows + n) * (width / 32) + k * 4);
    *reinterpret_cast<uint32_t *>(out + w * 4) = word;
  }
}

void launch_mx(const MxParams &p, bool gated, int64_t max_tiles, hipStream_t stream) {
  const int64_t slices = gated ? p.out_width / 64 : ceil_div<int64_t>(p.out_width, 128);
  if (max_tiles * slices < kSplitBelow) {
    const int64_t split_slices = gated ? p.out_width / 16 : ceil_div<int64_t>(p.out_width, 32);
    const dim3 grid(static_cast<uint32_t>(max_tiles), static_cast<uint32_t>(split_slices));
    if (gated) hipLaunchKernelGGL((stream_mx_kernel<true, true>), grid, dim3(kThreads), 0, stream, p);
    else hipLaunchKernelGGL((stream_mx_kernel<false, true>), grid, dim3(kThreads), 0, stream, p);
    return;
  }
  const dim3 grid(static_cast<uint32_t>(max_tiles), static_cast<uint32_t>(slices));
  if (gated) hipLaunchKernelGGL((stream_mx_kernel<true, false>), grid, dim3(kThreads), 0, stream, p);
  else hipLaunchKernelGGL((stream_mx_kernel<false, false>), grid, dim3(kThreads), 0, stream, p);
}

}  // namespace

void launch_quantize_mxfp8(const void *input, bool input_f32, uint8_t *out, uint8_t *scales, const int32_t *row_limit,
                           int64_t rows, int64_t width, hipStream_t stream, uint8_t *stage_scales,
                           const int32_t *routes, int64_t top, int64_t stage_rows) {
  MxQuantParams p{input, out, scales, row_limit, rows, width, input_f32 ? 1 : 0, stage_scales, routes, top, stage_rows};
  const int64_t blocks = ceil_div<int64_t>(rows * (width / 32) * 4, kQuantThreads);
  const uint32_t grid = static_cast<uint32_t>(blocks < 2048 ? (blocks > 0 ? blocks : 1) : 2048);
  hipLaunchKernelGGL(quantize_mxfp8_kernel, dim3(grid), dim3(kQuantThreads), 0, stream, p);
}

}  // namespace uniserve

extern "C" int32_t uniserve_quantize_mxfp8(const uniserve_quantize_mxfp8_call *call, void *stream) {
  using namespace uniserve;
  return guarded(call, [&]() -> int32_t {
    if (call->input == nullptr || call->out == nullptr || call->scales == nullptr)
      return UNISERVE_REFUSE(call, "quantize_mxfp8 needs input, out and scales");
    if (call->width <= 0 || call->width % 128 != 0)
      return UNISERVE_REFUSE(call, "quantize_mxfp8 needs a width of whole 128-channel groups");
    if (call->input_dtype != UNISERVE_DTYPE_BF16 && call->input_dtype != UNISERVE_DTYPE_F32)
      return UNISERVE_REFUSE(call, "quantize_mxfp8 reads bf16 or f32 rows");
    if (call->rows < 0) return UNISERVE_REFUSE(call, "quantize_mxfp8 needs a non-negative row count");
    if (call->rows == 0) return 0;
    launch_quantize_mxfp8(call->input, call->input_dtype == UNISERVE_DTYPE_F32, static_cast<uint8_t *>(call->out),
                          call->scales, call->row_limit, call->rows, call->width, static_cast<hipStream_t>(stream));
    return launched(call, "quantize_mxfp8");
  });
}

namespace uniserve {

bool mx_route_scales(int64_t tokens, int64_t top, int64_t experts, int64_t hidden_size, int64_t intermediate,
                     int64_t permuted_rows) {
  const int64_t routes_bound = permuted_rows - (kTileRows - 1) * experts;
  return !fp8_stream_path(tokens * top, experts) && tiled_fits(true, hidden_size, intermediate) &&
         !fp8_stream_path(routes_bound, experts) && tiled_fits(false, intermediate, hidden_size);
}

int32_t gather_gemm_mx(const uniserve_gather_mx_call *call, int64_t scale_rows, int32_t activation, void *stream,
                       uint8_t *out_codes, uint8_t *out_code_scales) {
  return guarded(call, [&]() -> int32_t {
    if (call->out_dtype != UNISERVE_DTYPE_BF16) return UNISERVE_REFUSE(call, "gather_gemm_mx writes bf16 only");
    if (call->hidden == nullptr || call->hidden_scales == nullptr || call->weights == nullptr ||
        call->weight_scales == nullptr || call->out == nullptr)
      return UNISERVE_REFUSE(call, "gather_gemm_mx needs hidden, weights, their scales and out");
    if (call->tile_to_expert == nullptr || call->tile_to_limit == nullptr ||
        call->permuted_to_expanded == nullptr || call->num_non_exiting_tiles == nullptr)
      return UNISERVE_REFUSE(call, "gather_gemm_mx needs the sort's tile and route maps");
    if (call->multiprocessors <= 0) return UNISERVE_REFUSE(call, "gather_gemm_mx needs its device's multiprocessor count");
    if (call->hidden_size <= 0 || call->hidden_size % 256 != 0)
      return UNISERVE_REFUSE(call, "gather_gemm_mx needs a hidden size of whole 256-element chunks");
    if (call->width <= 0 || call->width % 128 != 0)
      return UNISERVE_REFUSE(call, "gather_gemm_mx needs an intermediate width of whole 64-column slices");
    if (call->tokens < 0 || call->top <= 0 || call->experts <= 0)
      return UNISERVE_REFUSE(call, "gather_gemm_mx needs non-negative tokens and positive top and experts");
    if (!dma_rows_fit(call->tokens, call->hidden_size))
      return UNISERVE_REFUSE(call, "gather_gemm_mx serves hidden rows below 4 GiB (%lld tokens of %lld bytes)",
                             static_cast<long long>(call->tokens), static_cast<long long>(call->hidden_size));
    if (call->permuted_rows < call->tokens * call->top || call->permuted_rows % kTileRows != 0)
      return UNISERVE_REFUSE(call, "gather_gemm_mx needs whole 128-row tiles that hold every route");
    if (call->weight_scale_layout != UNISERVE_MX_SCALES_ROW_MAJOR && call->weight_scale_layout != UNISERVE_MX_SCALES_STAGE_MAJOR)
      return UNISERVE_REFUSE(call, "gather_gemm_mx: no weight scale layout %lld", static_cast<long long>(call->weight_scale_layout));
    if (scale_rows != 0 && scale_rows < call->permuted_rows)
      return UNISERVE_REFUSE(call, "gather_gemm_mx: route-major scales need a row per permuted row");
    const int64_t max_tiles = call->permuted_rows / kTileRows;
    if (max_tiles == 0) return 0;
    MxParams p{};
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
    scale_strides(call->weight_scale_layout, p.n_total, p.K, &p.ws_stage, &p.ws_row);
    scale_strides(scale_rows != 0 ? UNISERVE_MX_SCALES_STAGE_MAJOR : UNISERVE_MX_SCALES_ROW_MAJOR, scale_rows, p.K,
                  &p.as_stage, &p.as_row);
    p.as_by_route = scale_rows != 0 ? 1 : 0;
    if (!fp8_stream_path(call->tokens * call->top, call->experts) && tiled_fits(true, p.K, p.out_width)) {
      if (out_codes != nullptr) {
        if (scale_rows == 0) return UNISERVE_REFUSE(call, "gather_gemm_mx: quantised rows need route-major scales");
        p.out_codes = out_codes;
        p.out_code_scales = out_code_scales;
        p.code_scale_rows = scale_rows;
      }
      launch_tiled_mx(p, true, max_tiles, static_cast<hipStream_t>(stream));
    } else {
      if (out_codes != nullptr) return UNISERVE_REFUSE(call, "gather_gemm_mx: quantised rows only on the tiled kernel");
      launch_mx(p, true, max_tiles, static_cast<hipStream_t>(stream));
    }
    return launched(call, "gather_gemm_mx");
  });
}

int32_t route_gemm_mx(const uniserve_route_mx_call *call, int64_t scale_rows, void *stream) {
  return guarded(call, [&]() -> int32_t {
    if (call->out_dtype != UNISERVE_DTYPE_BF16) return UNISERVE_REFUSE(call, "route_gemm_mx writes bf16 only");
    if (call->rows == nullptr || call->row_scales == nullptr || call->weights == nullptr ||
        call->weight_scales == nullptr || call->out == nullptr)
      return UNISERVE_REFUSE(call, "route_gemm_mx needs rows, weights, their scales and out");
    if (call->tile_to_expert == nullptr || call->tile_to_limit == nullptr ||
        call->permuted_to_expanded == nullptr || call->num_non_exiting_tiles == nullptr)
      return UNISERVE_REFUSE(call, "route_gemm_mx needs the sort's tile and route maps");
    if (call->multiprocessors <= 0) return UNISERVE_REFUSE(call, "route_gemm_mx needs its device's multiprocessor count");
    if (call->intermediate <= 0 || call->intermediate % 256 != 0)
      return UNISERVE_REFUSE(call, "route_gemm_mx needs an intermediate width of whole 256-element chunks");
    if (call->width <= 0 || call->width % 32 != 0)
      return UNISERVE_REFUSE(call, "route_gemm_mx needs a hidden width of whole 32-row sets");
    if (call->experts <= 0) return UNISERVE_REFUSE(call, "route_gemm_mx needs positive experts");
    if (call->permuted_rows < 0 || call->permuted_rows % kTileRows != 0)
      return UNISERVE_REFUSE(call, "route_gemm_mx needs permuted rows of whole 128-row tiles");
    if (call->weight_scale_layout != UNISERVE_MX_SCALES_ROW_MAJOR && call->weight_scale_layout != UNISERVE_MX_SCALES_STAGE_MAJOR)
      return UNISERVE_REFUSE(call, "route_gemm_mx: no weight scale layout %lld", static_cast<long long>(call->weight_scale_layout));
    if (scale_rows != 0 && scale_rows < call->permuted_rows)
      return UNISERVE_REFUSE(call, "route_gemm_mx: route-major scales need a row per permuted row");
    const int64_t max_tiles = call->permuted_rows / kTileRows;
    if (max_tiles == 0) return 0;
    MxParams p{};
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
    scale_strides(call->weight_scale_layout, p.n_total, p.K, &p.ws_stage, &p.ws_row);
    scale_strides(scale_rows != 0 ? UNISERVE_MX_SCALES_STAGE_MAJOR : UNISERVE_MX_SCALES_ROW_MAJOR, scale_rows, p.K,
                  &p.as_stage, &p.as_row);
    p.as_by_route = scale_rows != 0 ? 1 : 0;
    // No token count in the call: the permuted rows less one partial tile per expert bound the routes.
    const int64_t routes_bound = call->permuted_rows - (kTileRows - 1) * call->experts;
    if (!fp8_stream_path(routes_bound, call->experts) && tiled_fits(false, p.K, p.out_width)) {
      launch_tiled_mx(p, false, max_tiles, static_cast<hipStream_t>(stream));
    } else {
      // The stream kernel addresses every permuted row from the arrays' bases (32-bit offsets; the
      // scales, K / 32 bytes a row, take fewer bytes than the codes).
      if (!dma_rows_fit(call->permuted_rows, p.K))
        return UNISERVE_REFUSE(call, "route_gemm_mx serves rows below 4 GiB on its stream kernel (%lld rows of %lld bytes)",
                               static_cast<long long>(call->permuted_rows), static_cast<long long>(p.K));
      launch_mx(p, false, max_tiles, static_cast<hipStream_t>(stream));
    }
    return launched(call, "route_gemm_mx");
  });
}

namespace {

/// FC2 (expert-major, unsplit): 128-row slices served per workgroup, one after the other. An
/// MXFP4 FC2 slice is 48 KB of weights at 768 channels, too short a life for a workgroup: 30B
/// T=64 FC2 31.5 us with one slice each, 30.0 with two, 28.0 with four, 36.3 with eight (FC1's
/// 128 KB slices: 43.7 us alone, 49 in runs of two or four; the e4m3 FC2's 96 KB ones: 34.5 us
/// alone, 36.0 and 36.4 in runs of two and four).
constexpr int kFc2Run = 4;
/// The split FC2 (few routes: 32-row slices, K over the waves) likewise, two slices per workgroup:
/// 235B T=1 FC2 14.2 -> 11.6 us by events (four: 15.9, eight: 23.2).
constexpr int kSplitFc2Run = 2;

void launch_expert_mx(MxParams p, bool gated, const ExpertRouting &r, hipStream_t stream) {
  p.ids = r.ids;
  p.live_tokens = r.live_tokens;
  p.routes = r.routes;
  p.local_offset = r.local_offset;
  p.local_experts = r.local_experts;
  p.compact = r.routes < r.local_experts ? 1 : 0;
  const int64_t columns = p.compact ? r.routes : r.local_experts;
  const int64_t slices = gated ? p.out_width / 64 : p.out_width / 128;
  const int64_t served = r.routes < r.local_experts ? r.routes : r.local_experts;
  if (served * slices < kSplitBelow) {
    const dim3 grid(static_cast<uint32_t>(columns), static_cast<uint32_t>(gated ? p.out_width / 16 : p.out_width / 32));
    if (gated) {
      hipLaunchKernelGGL((stream_mx_kernel<true, true, true>), grid, dim3(kThreads), 0, stream, p);
    } else if ((p.out_width / 32) % kSplitFc2Run == 0) {
      const dim3 run_grid(static_cast<uint32_t>(columns), static_cast<uint32_t>(p.out_width / 32 / kSplitFc2Run));
      hipLaunchKernelGGL((stream_mx_kernel<false, true, true, kSplitFc2Run>), run_grid, dim3(kThreads), 0, stream, p);
    } else {
      hipLaunchKernelGGL((stream_mx_kernel<false, true, true>), grid, dim3(kThreads), 0, stream, p);
    }
    return;
  }
  if (gated && p.out_codes != nullptr) {
    const dim3 grid(static_cast<uint32_t>(columns), static_cast<uint32_t>(slices));
    hipLaunchKernelGGL((stream_mx_kernel<true, false, true, 1, true>), grid, dim3(kThreads), 0, stream, p);
  } else if (gated) {
    const dim3 grid(static_cast<uint32_t>(columns), static_cast<uint32_t>(slices));
    hipLaunchKernelGGL((stream_mx_kernel<true, false, true>), grid, dim3(kThreads), 0, stream, p);
  } else if (slices % kFc2Run == 0) {
    const dim3 grid(static_cast<uint32_t>(columns), static_cast<uint32_t>(slices / kFc2Run));
    hipLaunchKernelGGL((stream_mx_kernel<false, false, true, kFc2Run>), grid, dim3(kThreads), 0, stream, p);
  } else {
    const dim3 grid(static_cast<uint32_t>(columns), static_cast<uint32_t>(slices));
    hipLaunchKernelGGL((stream_mx_kernel<false, false, true>), grid, dim3(kThreads), 0, stream, p);
  }
}

}  // namespace

bool mx_fc1_quantizes_by_expert(const ExpertRouting &r, int64_t width) {
  const int64_t served = r.routes < r.local_experts ? r.routes : r.local_experts;
  return served * (width / 2 / 64) >= kSplitBelow;
}

void gather_gemm_mx_by_expert(const uniserve_gather_mx_call *call, const ExpertRouting &r, int32_t activation,
                              void *stream, uint8_t *codes, uint8_t *code_scales) {
  MxParams p{};
  p.act = static_cast<const uint8_t *>(call->hidden);
  p.act_scales = call->hidden_scales;
  p.weights = static_cast<const uint8_t *>(call->weights);
  p.weight_scales = call->weight_scales;
  p.out = static_cast<uint16_t *>(call->out);
  p.K = call->hidden_size;
  p.n_total = call->width;
  p.out_width = call->width / 2;
  p.top = call->top;
  p.activation = activation;
  p.out_codes = codes;
  p.out_code_scales = code_scales;
  scale_strides(call->weight_scale_layout, p.n_total, p.K, &p.ws_stage, &p.ws_row);
  scale_strides(UNISERVE_MX_SCALES_ROW_MAJOR, 0, p.K, &p.as_stage, &p.as_row);
  launch_expert_mx(p, true, r, static_cast<hipStream_t>(stream));
}

void route_gemm_mx_by_expert(const uniserve_route_mx_call *call, const ExpertRouting &r, void *stream) {
  MxParams p{};
  p.act = static_cast<const uint8_t *>(call->rows);
  p.act_scales = call->row_scales;
  p.weights = static_cast<const uint8_t *>(call->weights);
  p.weight_scales = call->weight_scales;
  p.out = static_cast<uint16_t *>(call->out);
  p.K = call->intermediate;
  p.n_total = call->width;
  p.out_width = call->width;
  p.top = r.top;
  scale_strides(call->weight_scale_layout, p.n_total, p.K, &p.ws_stage, &p.ws_row);
  scale_strides(UNISERVE_MX_SCALES_ROW_MAJOR, 0, p.K, &p.as_stage, &p.as_row);
  launch_expert_mx(p, false, r, static_cast<hipStream_t>(stream));
}

}  // namespace uniserve

extern "C" int32_t uniserve_gather_gemm_mx(const uniserve_gather_mx_call *call, void *stream) {
  return uniserve::gather_gemm_mx(call, 0, UNISERVE_ACTIVATION_SILU, stream);
}

extern "C" int32_t uniserve_gather_gemm_mx_gelu_tanh(const uniserve_gather_mx_call *call, void *stream) {
  return uniserve::gather_gemm_mx(call, 0, UNISERVE_ACTIVATION_GELU_TANH, stream);
}

extern "C" int32_t uniserve_route_gemm_mx(const uniserve_route_mx_call *call, void *stream) {
  return uniserve::route_gemm_mx(call, 0, stream);
}

extern "C" int32_t uniserve_mx_stage_major_scales(const uniserve_mx_stage_scales_call *call, void *stream) {
  using namespace uniserve;
  return guarded(call, [&]() -> int32_t {
    if (call->in == nullptr || call->out == nullptr) return UNISERVE_REFUSE(call, "mx_stage_major_scales needs in and out");
    if (call->in == call->out) return UNISERVE_REFUSE(call, "mx_stage_major_scales does not convert in place");
    if (call->stacks < 0 || call->rows < 0 || call->width <= 0 || call->width % 128 != 0)
      return UNISERVE_REFUSE(call, "mx_stage_major_scales needs non-negative extents and a width of whole 128-element stages");
    const int64_t words = call->stacks * call->rows * (call->width / 128);
    if (words == 0) return 0;
    const int64_t blocks = ceil_div<int64_t>(words, 256);
    hipLaunchKernelGGL(stage_major_kernel, dim3(static_cast<uint32_t>(blocks < 4096 ? blocks : 4096)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), call->in, call->out, call->stacks, call->rows, call->width);
    return launched(call, "mx_stage_major_scales");
  });
}

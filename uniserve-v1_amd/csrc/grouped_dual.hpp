// SPDX-License-Identifier: Apache-2.0
//
// The prefill-shaped e4m3 products (FC1 with SiLU, or FC2) on gfx950 with 128 x 128 FP32 block
// scales, as two independent workgroups per CU.
//
// One workgroup of 4 wavefronts owns one 128-row sort tile and 128 weight rows of its expert (FC1:
// 64 up rows and the matching 64 gate rows; FC2: 128 output columns); two workgroups share a CU, so
// each SIMD runs two waves from different workgroups: one workgroup's barrier, DMA wait or
// epilogue is covered by the other's MFMAs, and one wave's scaling FMAs by the other's MFMAs (a
// wave issues its VALU and MFMA instructions one after the other). Wave (t, w) of the 2 x 2 arrangement multiplies tile
// rows 64 t .. 64 t + 63 (four 16-row token blocks) by slice rows of four 16-row weight blocks
// (FC1: 32 up rows and the 32 gate rows of the same columns; FC2: 64 consecutive rows).
//
// One 16x16x128 MFMA spans one 128-element scale block along K: its FP32 result is added into the
// accumulator times s_w * s_x (the weight block's scale, wave-uniform, times the token row's scale
// of that block), so the operands are never dequantised.
//
// A stage holds 128 K of every row: 128 e4m3 activation bytes and 128 e4m3 weight bytes (8 chunks of
// 16, chunk c at c ^ ((r >> 1) & 7), free of bank conflicts for the fragment reads) and one FP32
// activation scale per tile row. Every byte arrives by DMA (`global_load_lds_dword[x4]`), nine
// instructions per wave per stage, so the loop counts its loads exactly: two stages, stage k + 1
// issued while stage k multiplies, one barrier per stage.
#pragma once

#include "common.hpp"
#include "grouped_fp8.hpp"
#include "grouped_prefill.hpp"

namespace uniserve {
namespace dual {

constexpr int kRows = 128;           // tile rows
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * kWave;
constexpr int kSliceRows = 128;      // weight rows per workgroup

struct Stage {
  u32x4 act[kRows * 8];              // 16 KB
  u32x4 weights[kSliceRows * 8];     // 16 KB
  float act_scales[kWaves * kWave];  // tile row r at 64 (r / 32) + r % 32
};

__device__ __forceinline__ int slot(int row, int chunk) { return row * 8 + (chunk ^ ((row >> 1) & 7)); }
__device__ __forceinline__ int scale_slot(int row) { return (row >> 5) * kWave + (row & 31); }

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

/// Lane (r, g)'s e4m3 operand of a 16x16x128 MFMA: K 16 g .. 16 g + 15 and 64 + 16 g .. of its row.
__device__ __forceinline__ intx8 fragment(const u32x4 *rows, int row, int g) {
  const u32x4 lo = rows[slot(row, g)];
  const u32x4 hi = rows[slot(row, g + 4)];
  return intx8{static_cast<int>(lo[0]), static_cast<int>(lo[1]), static_cast<int>(lo[2]), static_cast<int>(lo[3]),
               static_cast<int>(hi[0]), static_cast<int>(hi[1]), static_cast<int>(hi[2]), static_cast<int>(hi[3])};
}

/// A workgroup covers its columns in sweeps through one continuous stage pipeline, each sweep's
/// results but the last parked in registers as bf16: FC1 64 columns (one sweep), or with kQuantize
/// 128 columns in two sweeps of 64, written as FC2's e4m3 operand - codes and one scale per 128
/// columns, the rounding points and encoding of uniserve_quantize_fp8 over the bf16 values; FC2 256
/// columns in two sweeps of 128, which halves the per-item prologue and epilogue of its short K.
template <bool kGated, bool kQuantize>
__global__ void __launch_bounds__(kThreads, 2) e4m3_kernel(PrefillParams p) {
  static_assert(kGated || !kQuantize, "only FC1 quantises its output");
  constexpr int kSweeps = (kQuantize || !kGated) ? 2 : 1;
  constexpr int kSweepCols = kGated ? kSliceRows / 2 : kSliceRows;  // output columns per sweep
  using prefill::dma16;
  using prefill::lds_address;
  __shared__ Stage ring[2];

  // ---- the work item: groups of `group` tiles, slice-major inside a group, dealt to the XCDs in
  // turn (block b runs on XCD b % 8) ----
  const int b = static_cast<int>(blockIdx.x);
  const int span = p.group * p.slices;
  const int seq = b >> 3;
  const int group_index = (seq / span) * 8 + (b & 7);
  const int first_tile = group_index * p.group;
  if (first_tile >= p.max_tiles) return;
  const int in_group = min(p.group, p.max_tiles - first_tile);
  const int within = seq - (seq / span) * span;
  if (within >= in_group * p.slices) return;
  const int slice = within / in_group;
  const int tile = first_tile + within % in_group;
  if (tile >= p.num_tiles[0]) return;

  const int64_t expert = p.tile_to_expert[tile];
  const int64_t first = static_cast<int64_t>(tile) * kRows;
  const int rows = p.tile_to_limit[tile] - static_cast<int>(first);
  const int t = static_cast<int>(threadIdx.x);
  const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
  const int wt = wave & 1;   // token half
  const int ww = wave >> 1;  // weight half
  const int lane = lane_id();
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int stages = static_cast<int>(p.K / 128);
  const int kb_count = stages;
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
  // Wave w's instruction i fills rows 32 w + 8 i + l / 8 of both the activation and the weight
  // stage, lane l bringing logical chunk (l % 8) ^ key(row) into physical chunk l % 8; its scale
  // instruction brings the scales of tile rows 32 w + l % 32 (lanes 32.. repeat them into the
  // padding). Slice row j is, for FC1, up row slice_col + j (j < 64) or gate row out_width +
  // slice_col + j - 64; for FC2, row slice_col + j.
  const int64_t slice_col = static_cast<int64_t>(slice) * kSweeps * kSweepCols;
  auto weight_row = [&](int j) -> int64_t {
    if constexpr (kGated) return j < 64 ? slice_col + j : p.out_width + slice_col + j - 64;
    else return slice_col + j;
  };
  uint32_t a_off[4];
  uint32_t w_first[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 32 * wave + 8 * i + lane / 8;
    a_off[i] = static_cast<uint32_t>(act_row(r) * p.K + ((lane & 7) ^ ((r >> 1) & 7)) * 16);
    w_first[i] = static_cast<uint32_t>(weight_row(32 * wave + 8 * i));
  }
  // key(32 w + 8 i + l / 8) = (l / 16) % 4 + 4 (i % 2): one lane offset per instruction parity.
  uint32_t w_lane[2];
#pragma unroll
  for (int parity = 0; parity < 2; ++parity)
    w_lane[parity] = static_cast<uint32_t>((lane / 8) * p.K + ((lane & 7) ^ (((lane >> 4) & 3) + 4 * parity)) * 16);
  const uint8_t *expert_weights = p.weights + expert * p.n_total * p.K;
  // Activation scales: route-major ([K / 128, scale_rows] by permuted row) or row-major by
  // source row ([rows of act, K / 128]).
  const int scale_r = 32 * wave + (lane & 31);
  const uint32_t as_off = p.scale_rows != 0 ? static_cast<uint32_t>((first + (scale_r < rows ? scale_r : 0)) * 4)
                                            : static_cast<uint32_t>(source_row(scale_r) * kb_count * 4);
  const int64_t as_stage = p.scale_rows != 0 ? p.scale_rows * 4 : 4;
  // Weight block scales ([experts, n_total / 128, K / 128]): the wave's up and gate blocks (FC1; the
  // same for both sweeps, which share one 128-column block) or its blocks of sweeps 0 and 1 (FC2),
  // wave-uniform. Lane k holds stage k's (K / 128 <= 64), read into a scalar per stage, so the loop
  // issues no vector loads of its own besides the counted DMA.
  const int64_t blocks_n = p.n_total / 128;
  const float *sw_first =
      p.weight_scales + (expert * blocks_n + weight_row(kGated ? 0 : 64 * ww) / 128) * kb_count;
  const float *sw_second =
      p.weight_scales + (expert * blocks_n + (kGated ? weight_row(64) : weight_row(64 * ww) + kSweepCols) / 128) * kb_count;
  const int sw_lane = lane < stages ? lane : 0;
  const int sw_first_lanes = __float_as_int(sw_first[sw_lane]);
  const int sw_second_lanes = __float_as_int(sw_second[sw_lane]);
  // Used here, so the compiler waits for these loads before the first DMA is issued.
  float s_first_k = __int_as_float(__builtin_amdgcn_readlane(sw_first_lanes, 0));
  float s_second_k = __int_as_float(__builtin_amdgcn_readlane(sw_second_lanes, 0));

  // Virtual stage v: sweep v / stages (its weight rows kSweepCols columns on), K stage v % stages.
  auto issue = [&](Stage &st, int v) {
    const int sweep = kSweeps == 1 ? 0 : v / stages;
    const int k = v - sweep * stages;
    const uint8_t *sweep_weights = expert_weights + static_cast<int64_t>(sweep) * kSweepCols * p.K;
    const uint32_t act_lds = lds_address(st.act + wave * 4 * kWave);
    const uint32_t weight_lds = lds_address(st.weights + wave * 4 * kWave);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      dma16(act_tile + static_cast<int64_t>(k) * 128, a_off[i], __builtin_amdgcn_readfirstlane(act_lds + i * kWave * 16));
#pragma unroll
    for (int i = 0; i < 4; ++i)
      dma16(sweep_weights + static_cast<int64_t>(w_first[i]) * p.K + static_cast<int64_t>(k) * 128, w_lane[i & 1],
            __builtin_amdgcn_readfirstlane(weight_lds + i * kWave * 16));
    dma4(reinterpret_cast<const uint8_t *>(p.act_scales) + k * as_stage, as_off,
         __builtin_amdgcn_readfirstlane(lds_address(st.act_scales + wave * kWave)));
  };

  floatx4 acc[4][4];
#pragma unroll
  for (int tb = 0; tb < 4; ++tb)
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) acc[tb][jb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  // The wave's slice rows of weight block jb: FC1 jb 0, 1 up and 2, 3 gate (32 w + 16 (jb % 2)
  // .. of each half); FC2 64 w + 16 jb ..
  auto slice_row = [&](int jb) {
    if constexpr (kGated) return (jb >> 1) * 64 + ww * 32 + (jb & 1) * 16 + r16;
    else return ww * 64 + jb * 16 + r16;
  };
  auto compute = [&](const Stage &st, int k, int sweep) {
    const float s_first = k == 0 ? s_first_k : __int_as_float(__builtin_amdgcn_readlane(sw_first_lanes, k));
    const float s_second = k == 0 ? s_second_k : __int_as_float(__builtin_amdgcn_readlane(sw_second_lanes, k));
    intx8 wf[4];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) wf[jb] = fragment(st.weights, slice_row(jb), g);
    // Token block tb's MFMAs go out before block tb - 1's scaling, so the FMAs never wait on the
    // MFMA that feeds them and the other wave's MFMAs fill the VALU's turns.
    floatx4 block[2][4];
    float scale[2][2];
#pragma unroll
    for (int tb = 0; tb <= 4; ++tb) {
      if (tb < 4) {
        const int row = wt * 64 + tb * 16 + r16;
        const intx8 x = fragment(st.act, row, g);
        const float sx = st.act_scales[scale_slot(row)];
        scale[tb & 1][0] = sx * s_first;
        scale[tb & 1][1] = sx * s_second;
#pragma unroll
        for (int jb = 0; jb < 4; ++jb)
          // cbsz/blgp 0: e4m3 x e4m3; scale exponents 127 = 2^0 (the block scales are applied below).
          block[tb & 1][jb] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wf[jb], x, floatx4{0.0f, 0.0f, 0.0f, 0.0f},
                                                                              0, 0, 0, 127, 0, 127);
      }
      if (tb > 0) {
        const int pb = (tb - 1) & 1;
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
          const float s = scale[pb][kGated ? (jb >> 1) : sweep];
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[tb - 1][jb][e] = __builtin_fmaf(block[pb][jb][e], s, acc[tb - 1][jb][e]);
        }
      }
    }
  };

  // ---- the K loop: at the top of stage k only stage k is in flight; once it has landed for every
  // wave (own wait, then the barrier, which also retires every wave's reads of stage k - 1), stage
  // k + 1 is issued into the other buffer. The issue past the last stage re-reads it, so every wait
  // counts the same loads. ----
  // The first sweep's results, bf16: token block tb, weight block jb (FC1: up blocks 0, 1).
  uint2 parked[4][4];
  const int total = kSweeps * stages;
  issue(ring[0], 0);
  for (int v = 0; v < total; ++v) {
    prefill::wait_all_loads();
    __syncthreads();
    issue(ring[(v + 1) & 1], min(v + 1, total - 1));
    const int sweep = kSweeps == 1 ? 0 : v / stages;
    compute(ring[v & 1], v - sweep * stages, sweep);
    if constexpr (!kGated) {
      if (v == stages - 1) {
#pragma unroll
        for (int tb = 0; tb < 4; ++tb)
#pragma unroll
          for (int jb = 0; jb < 4; ++jb) {
            parked[tb][jb] = uint2{pack_bf16x2(acc[tb][jb][0], acc[tb][jb][1]), pack_bf16x2(acc[tb][jb][2], acc[tb][jb][3])};
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[tb][jb][i] = 0.0f;
          }
      }
    }
    if constexpr (kQuantize) {
      if (v == stages - 1) {
#pragma unroll
        for (int tb = 0; tb < 4; ++tb)
#pragma unroll
          for (int jb = 0; jb < 2; ++jb) {
            float g4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) g4[i] = gate(acc[tb][jb + 2][i], p.activation) * acc[tb][jb][i];
            parked[tb][jb] = uint2{pack_bf16x2(g4[0], g4[1]), pack_bf16x2(g4[2], g4[3])};
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[tb][jb][i] = acc[tb][jb + 2][i] = 0.0f;
          }
      }
    }
  }
  prefill::wait_all_loads();
  __syncthreads();  // every wave is done reading the stage buffers

  // ---- epilogue: lane (r16, g) holds, of token block tb and weight block jb, tile row
  // 64 t + 16 tb + r16 and the block's rows 4 g + i in element i. The output tile goes through LDS
  // so the global stores are whole rows; LDS rows are padded by 16 bytes. ----
  constexpr int kOutCols = kSweeps * kSweepCols;
  constexpr int kOutStride = kOutCols * 2 + 16;
  static_assert(kRows * kOutStride <= static_cast<int>(sizeof(ring)), "the output tile fits the stages");
  char *tile_lds = reinterpret_cast<char *>(ring);
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) {
    char *row = tile_lds + (wt * 64 + tb * 16 + r16) * kOutStride;
    if constexpr (kGated) {
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        floatx4 v;
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = gate(acc[tb][jb + 2][i], p.activation) * acc[tb][jb][i];
        uint2 packed;
        packed.x = pack_bf16x2(v[0], v[1]);
        packed.y = pack_bf16x2(v[2], v[3]);
        *reinterpret_cast<uint2 *>(row + ((kSweeps - 1) * 64 + ww * 32 + jb * 16 + 4 * g) * 2) = packed;
        if constexpr (kQuantize) *reinterpret_cast<uint2 *>(row + (ww * 32 + jb * 16 + 4 * g) * 2) = parked[tb][jb];
      }
    } else {
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) {
        uint2 packed;
        packed.x = pack_bf16x2(acc[tb][jb][0], acc[tb][jb][1]);
        packed.y = pack_bf16x2(acc[tb][jb][2], acc[tb][jb][3]);
        *reinterpret_cast<uint2 *>(row + (kSweepCols + ww * 64 + jb * 16 + 4 * g) * 2) = packed;
        *reinterpret_cast<uint2 *>(row + (ww * 64 + jb * 16 + 4 * g) * 2) = parked[tb][jb];
      }
    }
  }
  __syncthreads();
  if constexpr (kQuantize) {
    // Each row's 128 columns are quantised by 16 lanes from the bf16 values in LDS: amax of the
    // bf16 values, s = amax / 448 (1 for an all-zero group), code = e4m3(v / s); live rows only.
    const int sub = t & 15;
    const int64_t groups_per_row = p.out_width / 128;
    for (int m = t / 16; m < kRows; m += kThreads / 16) {
      const u32x4 piece = *reinterpret_cast<const u32x4 *>(tile_lds + m * kOutStride + sub * 16);
      float v[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[2 * j] = __uint_as_float(piece[j] << 16);
        v[2 * j + 1] = __uint_as_float(piece[j] & 0xffff0000u);
      }
      float amax = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[j]));
      amax = row16_max(amax);
      if (m >= rows) continue;
      const float scale = amax > 0.0f ? amax / 448.0f : 1.0f;
      *reinterpret_cast<uint2 *>(p.out_codes + (first + m) * p.out_width + slice_col + sub * 8) = e4m3_eight_of_bf16(v, scale);
      if (sub == 0) {
        const int64_t at = p.scale_rows != 0 ? slice_col / 128 * p.scale_rows + first + m
                                             : (first + m) * groups_per_row + slice_col / 128;
        p.out_code_scales[at] = scale;
      }
    }
    return;
  }
  constexpr int kPieces = kOutCols / 8;
  for (int index = t; index < kRows * kPieces; index += kThreads) {
    const int m = index / kPieces;
    const int c = index - m * kPieces;
    if (m >= rows) continue;
    const u32x4 piece = *reinterpret_cast<const u32x4 *>(tile_lds + m * kOutStride + c * 16);
    *reinterpret_cast<u32x4 *>(p.out + (first + m) * p.out_width + slice_col + c * 8) = piece;
  }
}

}  // namespace dual

/// Output columns per workgroup: FC1 64, FC1 writing e4m3 codes 128, FC2 256.
inline int64_t dual_columns(bool gated, bool quantize) { return gated ? (quantize ? 128 : 64) : 256; }

/// Whether the dual-workgroup e4m3 kernel serves the shape: whole 128-K stages (at most 64 of
/// them) and whole slices of dual_columns.
inline bool dual_fits(bool gated, int64_t K, int64_t out_width, bool quantize = false) {
  return K % 128 == 0 && K > 0 && K / 128 <= kWave && out_width % dual_columns(gated, quantize) == 0;
}

/// Launches the dual-workgroup e4m3 product over `max_tiles` tiles (tiles past `num_tiles` exit at
/// once); with `p.out_codes` set (FC1 only) the gated rows are written as e4m3 codes and scales.
/// `group`: tiles per group of the work numbering (4 measured best: 235B FC1 765 us against 792 at 16).
inline void launch_dual_e4m3(PrefillParams p, bool gated, int64_t max_tiles, hipStream_t stream, int group = 4) {
  const bool quantize = gated && p.out_codes != nullptr;
  p.slices = static_cast<int32_t>(p.out_width / dual_columns(gated, quantize));
  p.max_tiles = static_cast<int32_t>(max_tiles);
  p.group = group;
  p.groups_per_xcd = static_cast<int32_t>(ceil_div<int64_t>(ceil_div<int64_t>(max_tiles, group), 8));
  const dim3 grid(static_cast<uint32_t>(static_cast<int64_t>(p.groups_per_xcd) * group * p.slices * 8));
  if (quantize) hipLaunchKernelGGL((dual::e4m3_kernel<true, true>), grid, dim3(dual::kThreads), 0, stream, p);
  else if (gated) hipLaunchKernelGGL((dual::e4m3_kernel<true, false>), grid, dim3(dual::kThreads), 0, stream, p);
  else hipLaunchKernelGGL((dual::e4m3_kernel<false, false>), grid, dim3(dual::kThreads), 0, stream, p);
}

}  // namespace uniserve

// SPDX-License-Identifier: Apache-2.0
//
// The prefill-shaped grouped products (FC1 with its gate, or FC2) on gfx950, two workgroups per CU,
// in e4m3 with 128 x 128 FP32 block scales or in bf16.
//
// A workgroup of four wavefronts owns one 128-row sort tile and 256 weight rows of its expert (FC1:
// 128 up rows and the matching 128 gate rows; FC2: 256 output columns). K is walked in stages of
// 128 bytes per row (128 e4m3 or 64 bf16 elements; an e4m3 stage is one scale block).
//
// Wavefront w multiplies all 128 tile rows (eight 16-row token blocks) by its own 64 weight rows
// (four 16-row blocks; FC1: 32 up rows and the 32 gate rows of the same columns):
//   * e4m3: one v_mfma_scale_f32_16x16x128_f8f6f4 per (token block, weight block) and stage, whose
//     result is added into the accumulator times s_w * s_x (the weight block's scale, uniform over
//     the wave, times the token row's scale of that block);
//   * bf16: two v_mfma_f32_16x16x32_bf16 per (token block, weight block) and stage, accumulating
//     directly.
//
// The operands arrive by DMA (`global_load_lds_dwordx4`), the activation scales by plain loads
// issued as inline assembly, all invisible to the compiler, so the loop counts its loads itself and
// waits with exact vmcnt values:
//   * each wavefront's 64 weight rows go to a buffer of its own (8 KB), read into registers at the
//     top of stage k and refilled with stage k + 1 right after; no wavefront waits on another's
//     weights;
//   * the activation rows of the tile (gathered token rows for FC1) go through a three-stage ring
//     shared by the workgroup (48 KB), one barrier per stage;
//   * e4m3: each lane's activation scales (eight token rows per stage, route-major by permuted
//     row) go to registers, one stage ahead.
// That is 80 KB per workgroup: two per CU, so one workgroup's prologue, barriers and epilogue run
// under the other's MFMAs. A stage's loads go out spread over its first token blocks, so that no
// wave stalls long on a full memory queue with its MFMAs unissued.
#pragma once

#include <type_traits>

#include "common.hpp"
#include "grouped_fp8.hpp"
#include "grouped_prefill.hpp"

namespace uniserve {
namespace pair {

constexpr int kRows = 128;                   // tile rows
constexpr int kWaveRows = 64;                // weight rows per wavefront
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * kWave;
constexpr int kSliceRows = kWaves * kWaveRows;
constexpr int kActStages = 3;
constexpr int kTokenBlocks = kRows / 16;
constexpr int kWeightLoads = kWaveRows / 8;  // 16-byte DMA instructions per wave per stage (8 rows each)
constexpr int kActLoads = kRows / 8 / kWaves;

/// Block-scaled e4m3: 128 elements per stage.
struct E4m3 {
  static constexpr bool kScaled = true;
  static constexpr int kElementBytes = 1;
};
/// bf16: 64 elements per stage.
struct Bf16 {
  static constexpr bool kScaled = false;
  static constexpr int kElementBytes = 2;
};

struct Shared {
  u32x4 weights[kWaves][kWaveRows * 8];  // each wavefront's own rows
  u32x4 act[kActStages][kRows * 8];      // chunk c of row r at slot(r, c)
};

__device__ __forceinline__ int slot(int row, int chunk) { return row * 8 + (chunk ^ ((row >> 1) & 7)); }

/// Lane (r, g)'s operand bytes of `row` in a stage: 16 g .. 16 g + 15 (lo) and 64 + 16 g .. (hi).
/// e4m3: the two halves of one 16x16x128 operand (K 16 g .. and 64 + 16 g ..); bf16: the operands
/// of the stage's two 16x16x32 MFMAs (K 8 g .. 8 g + 7 of elements 0..31 and of 32..63).
struct Fragment {
  u32x4 lo, hi;
};
__device__ __forceinline__ Fragment fragment(const u32x4 *rows, int row, int g) {
  return Fragment{rows[slot(row, g)], rows[slot(row, g + 4)]};
}
__device__ __forceinline__ intx8 joined(const Fragment &f) {
  return intx8{static_cast<int>(f.lo[0]), static_cast<int>(f.lo[1]), static_cast<int>(f.lo[2]), static_cast<int>(f.lo[3]),
               static_cast<int>(f.hi[0]), static_cast<int>(f.hi[1]), static_cast<int>(f.hi[2]), static_cast<int>(f.hi[3])};
}

/// The activation scales of this lane's token blocks 4 h .. 4 h + 3 at one K stage: four 4-byte
/// loads from `base` + `offset` + 64 tb, issued as inline assembly like the DMA so that the loop's
/// own waits count them; `wait_loads_and_scales` is the only place their registers become
/// readable.
template <int kHalf>
__device__ __forceinline__ void load_scales_half(float (&out)[kTokenBlocks], const void *base, uint32_t offset) {
  asm volatile(
      "global_load_dword %0, %4, %5 offset:%6\n\t"
      "global_load_dword %1, %4, %5 offset:%7\n\t"
      "global_load_dword %2, %4, %5 offset:%8\n\t"
      "global_load_dword %3, %4, %5 offset:%9\n\t"
      : "=&v"(out[4 * kHalf]), "=&v"(out[4 * kHalf + 1]), "=&v"(out[4 * kHalf + 2]), "=&v"(out[4 * kHalf + 3])
      : "v"(offset), "s"(base), "n"(256 * kHalf), "n"(256 * kHalf + 64), "n"(256 * kHalf + 128), "n"(256 * kHalf + 192));
}

/// Waits until at most N vector-memory loads of this wave are outstanding (they complete in issue
/// order), declaring the scale registers written by the wait: the compiler cannot read them, or
/// move a read of them, before it. The loads and this wait sit in one straight stretch of a loop
/// iteration, so no control-flow merge makes the compiler copy the registers in between.
template <int N>
__device__ __forceinline__ void wait_loads_and_scales(float (&s)[kTokenBlocks]) {
  static_assert(N >= 0 && N < 16, "vmcnt's low bits");
  asm volatile("s_waitcnt vmcnt(%8)"
               : "+v"(s[0]), "+v"(s[1]), "+v"(s[2]), "+v"(s[3]), "+v"(s[4]), "+v"(s[5]), "+v"(s[6]), "+v"(s[7])
               : "n"(N));
}

/// The epilogue's output tile in LDS (bf16 rows, padded by 8 bytes), or the operand buffers.
template <bool kGated>
constexpr int out_stride() {
  return (kGated ? kSliceRows / 2 : kSliceRows) * 2 + 8;
}
template <bool kGated>
constexpr int lds_bytes() {
  return static_cast<int>(sizeof(Shared)) > kRows * out_stride<kGated>() ? static_cast<int>(sizeof(Shared))
                                                                          : kRows * out_stride<kGated>();
}

/// e4m3 needs route-major activation scales (p.scale_rows >= the tiles' rows).
template <class F, bool kGated>
__global__ void __launch_bounds__(kThreads, 2) pair_kernel(PrefillParams p) {
  using prefill::dma16;
  using prefill::dma16_after_lds_reads;
  using prefill::lds_address;
  static_assert(lds_bytes<kGated>() * 2 <= 160 * 1024, "two workgroups fit the CU's LDS");
  __shared__ __align__(16) char lds[lds_bytes<kGated>()];
  Shared &sh = *reinterpret_cast<Shared *>(lds);

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
  const int lane = lane_id();
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int64_t row_bytes = p.K * F::kElementBytes;
  const int stages = static_cast<int>(row_bytes / 128);
  const int top = static_cast<int>(p.top);
  // The activation row behind tile row r: FC1 gathers token permuted_to_expanded / top (padding
  // rows read row 0), FC2 reads its own permuted row (padding rows read the tile's first row).
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
  const uint8_t *act_tile = p.act + (kGated ? 0 : first * row_bytes);
  auto act_row = [&](int r) -> int64_t { return kGated ? source_row(r) : source_row(r) - first; };

  // ---- sources (32-bit lane offsets from wave-uniform bases) ----
  // Activations: wave w brings tile rows kActLoads * 8 w .., instruction i rows
  // kActLoads * 8 w + 8 i + l / 8, lane l the logical chunk (l % 8) ^ key(row) into physical
  // chunk l % 8.
  uint32_t a_off[kActLoads];
#pragma unroll
  for (int i = 0; i < kActLoads; ++i) {
    const int r = kActLoads * 8 * wave + 8 * i + lane / 8;
    a_off[i] = static_cast<uint32_t>(act_row(r) * row_bytes + ((lane & 7) ^ ((r >> 1) & 7)) * 16);
  }
  // Weights: the wave's 64 rows. FC1 rows 0..31 are up rows slice_col + 32 w .., rows 32..63 the
  // gate rows of the same columns; FC2 rows are 64 consecutive output columns. Instruction i
  // fills rows 8 i + l / 8; key(8 i + l / 8) = (l / 16) % 4 + 4 (i % 2).
  const int64_t slice_col = static_cast<int64_t>(slice) * (kGated ? kSliceRows / 2 : kSliceRows);
  const int64_t wave_col = slice_col + wave * (kGated ? kWaveRows / 2 : kWaveRows);
  auto weight_row = [&](int j) -> int64_t {  // weight row of the wave's row j
    if constexpr (kGated) return j < 32 ? wave_col + j : p.out_width + wave_col + (j - 32);
    else return wave_col + j;
  };
  const uint8_t *w_base[2];
  w_base[0] = p.weights + (expert * p.n_total + weight_row(0)) * row_bytes;
  w_base[1] = p.weights + (expert * p.n_total + weight_row(32)) * row_bytes;
  const uint32_t w_lane = static_cast<uint32_t>((lane / 8) * row_bytes);
  const uint32_t w_chunk = static_cast<uint32_t>((lane & 7) ^ ((lane >> 4) & 3));

  // e4m3 scales. Activations ([K / 128, scale_rows] by permuted row): tile row 16 tb + r16 of
  // stage k at k * scale_rows + first + 16 tb + r16 (padding rows read the scales of rows past the
  // tile's routes, inside the table, and their products are never stored). Weight blocks
  // ([experts, n_total / 128, K / 128]): the wave's rows 0..31 and 32..63 each lie in one 128-row
  // block (FC1: the up and the gate block; FC2: the same block); lane k holds stage k's
  // (K / 128 <= 64), read into a scalar per stage.
  const uint32_t sx_off = static_cast<uint32_t>((first + r16) * 4);
  const int64_t sx_stage = p.scale_rows * 4;
  const uint8_t *scale_table = reinterpret_cast<const uint8_t *>(p.act_scales);
  int sw_lanes[2] = {0, 0};
  if constexpr (F::kScaled) {
    const int64_t blocks_n = p.n_total / 128;
    const int sw_lane = lane < stages ? lane : 0;
    sw_lanes[0] = __float_as_int(p.weight_scales[(expert * blocks_n + weight_row(0) / 128) * stages + sw_lane]);
    sw_lanes[1] = __float_as_int(p.weight_scales[(expert * blocks_n + weight_row(32) / 128) * stages + sw_lane]);
    // Consumed here, so the compiler's wait for these loads comes before the first DMA is issued
    // (a wait after it would count the DMA too).
    asm volatile("" ::"v"(sw_lanes[0]), "v"(sw_lanes[1]));
  }

  // Weights of stage k, the h-th of `parts` equal runs of the eight instructions; `after_reads`:
  // the wave just read its rows of the buffer, and the first DMA waits for those LDS reads
  // (lgkmcnt 0) before it may overwrite them.
  auto issue_weights = [&](int k, int h, bool after_reads, int parts = 2) {
    const uint32_t weight_lds = lds_address(sh.weights[wave]);
#pragma unroll
    for (int j = 0; j < kWeightLoads / parts; ++j) {
      const int i = h * (kWeightLoads / parts) + j;
      const uint8_t *base = w_base[i / 4] + static_cast<int64_t>(k) * 128 + static_cast<int64_t>(i % 4) * 8 * row_bytes;
      const uint32_t lane_offset = w_lane + ((w_chunk ^ static_cast<uint32_t>(4 * (i & 1))) << 4);
      const uint32_t dst = __builtin_amdgcn_readfirstlane(weight_lds + i * kWave * 16);
      if (i == 0 && after_reads) dma16_after_lds_reads(base, lane_offset, dst);
      else dma16(base, lane_offset, dst);
    }
  };
  // Activations of stage k, instructions kActLoads / 2 h ..
  auto issue_act = [&](int k, int h) {
    const uint32_t act_lds = lds_address(sh.act[k % kActStages] + wave * kActLoads * kWave);
#pragma unroll
    for (int j = 0; j < kActLoads / 2; ++j) {
      const int i = h * (kActLoads / 2) + j;
      dma16(act_tile + static_cast<int64_t>(k) * 128, a_off[i], __builtin_amdgcn_readfirstlane(act_lds + i * kWave * 16));
    }
  };

  floatx4 acc[kTokenBlocks][4];
#pragma unroll
  for (int tb = 0; tb < kTokenBlocks; ++tb)
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) acc[tb][jb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  // ---- the K loop. Prefetched during stage k: the wave's weights of stage k + 1 (it has read
  // stage k's into registers at the top), the scales of stage k + 1 and the activations of stage
  // k + 2 (into the slot stage k - 1 used: every wavefront has passed the barrier after reading
  // it); past the last stage, the last stage again (cache-resident: into buffers nobody reads, or,
  // in the second-to-last stage, over the last stage's activation rows with the same bytes), so
  // that every wait counts alike. They go out in that order - weights, scales, activations. At the
  // end of stage k everything up to the scales of stage k + 1 has landed (the wait that makes the
  // scale registers readable), at the top of stage k + 1 everything but the activations, then
  // the barrier for the other wavefronts' activation rows. (At least three stages: pair_fits.) ----
  constexpr int kLast = kActLoads;  // loads of the farthest group
  float sx[kTokenBlocks];
  issue_act(0, 0);
  issue_act(0, 1);
  issue_weights(0, 0, false);
  issue_weights(0, 1, false);
  if constexpr (F::kScaled) {
    load_scales_half<0>(sx, scale_table, sx_off);
    load_scales_half<1>(sx, scale_table, sx_off);
  }
  issue_act(1, 0);
  issue_act(1, 1);
  if constexpr (F::kScaled) wait_loads_and_scales<kLast>(sx);
  for (int k = 0; k < stages; ++k) {
    prefill::wait_loads_but<kLast>();
    __syncthreads();
    const u32x4 *act = sh.act[k % kActStages];
    Fragment wf[4];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) wf[jb] = fragment(sh.weights[wave], jb * 16 + r16, g);
    const int act_next = min(k + 2, stages - 1);
    const int next = min(k + 1, stages - 1);
    // The loads issued before token block tb's MFMAs: two weight instructions before each of the
    // first four blocks, then the scales, then the activations.
    auto issue_part = [&](int tb) {
      if (tb < 4) issue_weights(next, tb, tb == 0, 4);
      constexpr int kActAt = F::kScaled ? 6 : 4;
      if constexpr (F::kScaled) {
        if (tb == 4) load_scales_half<0>(sx, scale_table + next * sx_stage, sx_off);
        if (tb == 5) load_scales_half<1>(sx, scale_table + next * sx_stage, sx_off);
      }
      if (tb == kActAt) issue_act(act_next, 0);
      if (tb == kActAt + 1) issue_act(act_next, 1);
    };

    if constexpr (F::kScaled) {
      const float sw0 = __int_as_float(__builtin_amdgcn_readlane(sw_lanes[0], k));
      const float sw1 = __int_as_float(__builtin_amdgcn_readlane(sw_lanes[1], k));
      float sc[kTokenBlocks][2];
#pragma unroll
      for (int tb = 0; tb < kTokenBlocks; ++tb) {
        sc[tb][0] = sx[tb] * sw0;
        sc[tb][1] = sx[tb] * sw1;
      }
      intx8 w8[4];
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) w8[jb] = joined(wf[jb]);
      auto scale_into = [&](floatx4 &into, const floatx4 &result, float s) {
#pragma unroll
        for (int e = 0; e < 4; ++e) into[e] = __builtin_fmaf(result[e], s, into[e]);
      };
      // The stage's 32 MFMAs in (token block, weight block) order; after issuing MFMA n the wave
      // scales the result of MFMA n - 2 (done by then: the matrix pipe runs one MFMA at a time),
      // and the next token block's activation fragment is read three MFMAs before its first use.
      // cbsz/blgp 0: e4m3 x e4m3; scale exponents 127 = 2^0 (the block scales are applied after).
      intx8 x = joined(fragment(act, r16, g)), x_next;
      floatx4 result[3];
#pragma unroll
      for (int n = 0; n < kTokenBlocks * 4; ++n) {
        const int tb = n / 4, jb = n % 4;
        if (jb == 0) issue_part(tb);
        result[n % 3] =
            __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(w8[jb], x, floatx4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0, 127, 0, 127);
        if (jb == 0 && tb + 1 < kTokenBlocks) x_next = joined(fragment(act, (tb + 1) * 16 + r16, g));
        if (n >= 2) {
          const int m = n - 2;
          scale_into(acc[m / 4][m % 4], result[m % 3], sc[m / 4][(m % 4) / 2]);
        }
        if (jb == 3 && tb + 1 < kTokenBlocks) x = x_next;
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // the MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // then four VALU (the scaling)
      }
#pragma unroll
      for (int m = kTokenBlocks * 4 - 2; m < kTokenBlocks * 4; ++m)
        scale_into(acc[m / 4][m % 4], result[m % 3], sc[m / 4][(m % 4) / 2]);
      wait_loads_and_scales<kLast>(sx);
    } else {
      // Per token block: the four weight blocks' MFMAs over the stage's first 32 elements, then
      // over its last 32 (each accumulator's two MFMAs four apart); the next token block's
      // activation fragment is read after the first.
      Fragment x = fragment(act, r16, g), x_next;
#pragma unroll
      for (int tb = 0; tb < kTokenBlocks; ++tb) {
        issue_part(tb);
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
          acc[tb][jb] = mfma_16x16x32_bf16(wf[jb].lo, x.lo, acc[tb][jb]);
          if (jb == 0 && tb + 1 < kTokenBlocks) x_next = fragment(act, (tb + 1) * 16 + r16, g);
        }
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) acc[tb][jb] = mfma_16x16x32_bf16(wf[jb].hi, x.hi, acc[tb][jb]);
        if (tb + 1 < kTokenBlocks) x = x_next;
      }
    }
  }
  prefill::wait_all_loads();
  if (!(kGated && p.out_codes != nullptr)) {
    // Each wave stages its own columns of one token block at a time in its own weight buffer (no
    // other wave reads it, and its last loads have landed), then stores whole 16-byte pieces.
    constexpr int kWaveCols = kGated ? kWaveRows / 2 : kWaveRows;  // bf16 columns of this wave
    constexpr int kRowBytes = kWaveCols * 2;
    constexpr int kStride = kRowBytes + 16;
    constexpr int kPiecesPerRow = kRowBytes / 16;
    char *stage = reinterpret_cast<char *>(sh.weights[wave]);
    uint16_t *out_cols = p.out + slice_col + wave * kWaveCols;
#pragma unroll
    for (int tb = 0; tb < kTokenBlocks; ++tb) {
      char *row = stage + r16 * kStride;
      if constexpr (kGated) {
        auto gated = [&](auto activation) {
#pragma unroll
          for (int jb = 0; jb < 2; ++jb) {
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = gate_of<decltype(activation)::value>(acc[tb][jb + 2][e]) * acc[tb][jb][e];
            uint2 packed;
            packed.x = pack_bf16x2(v[0], v[1]);
            packed.y = pack_bf16x2(v[2], v[3]);
            *reinterpret_cast<uint2 *>(row + (jb * 16 + 4 * g) * 2) = packed;
          }
        };
        if (p.activation == UNISERVE_ACTIVATION_GELU_TANH) gated(std::integral_constant<int, UNISERVE_ACTIVATION_GELU_TANH>{});
        else gated(std::integral_constant<int, UNISERVE_ACTIVATION_SILU>{});
      } else {
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
          uint2 packed;
          packed.x = pack_bf16x2(acc[tb][jb][0], acc[tb][jb][1]);
          packed.y = pack_bf16x2(acc[tb][jb][2], acc[tb][jb][3]);
          *reinterpret_cast<uint2 *>(row + (jb * 16 + 4 * g) * 2) = packed;
        }
      }
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int piece = lane; piece < 16 * kPiecesPerRow; piece += kWave) {
        const int r = piece / kPiecesPerRow;
        const int c = piece - r * kPiecesPerRow;
        const u32x4 v = *reinterpret_cast<const u32x4 *>(stage + r * kStride + c * 16);
        const int m = tb * 16 + r;
        if (m < rows) *reinterpret_cast<u32x4 *>(out_cols + (first + m) * p.out_width + c * 8) = v;
      }
      __builtin_amdgcn_wave_barrier();
    }
    return;
  }
  if constexpr (kGated) {
    __syncthreads();  // every wave is done with the operand buffers

    // ---- e4m3 FC1 written as FC2's operand: lane (r16, g) holds, of token block tb and weight
    // block jb, tile row 16 tb + r16 and the wave's weight rows 16 jb + 4 g + e in element e. The
    // gated bf16 tile goes through LDS, where 16 lanes take each (row, 128-column group). ----
    constexpr int kOutCols = kSliceRows / 2;
    constexpr int kOutStride = out_stride<kGated>();
#pragma unroll
    for (int tb = 0; tb < kTokenBlocks; ++tb) {
      char *row = lds + (tb * 16 + r16) * kOutStride;
      // The activation is uniform over the launch: one branch, each side with its gate inlined.
      auto gated = [&](auto activation) {
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) {
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = gate_of<decltype(activation)::value>(acc[tb][jb + 2][e]) * acc[tb][jb][e];
          uint2 packed;
          packed.x = pack_bf16x2(v[0], v[1]);
          packed.y = pack_bf16x2(v[2], v[3]);
          *reinterpret_cast<uint2 *>(row + (wave * 32 + jb * 16 + 4 * g) * 2) = packed;
        }
      };
      if (p.activation == UNISERVE_ACTIVATION_GELU_TANH) gated(std::integral_constant<int, UNISERVE_ACTIVATION_GELU_TANH>{});
      else gated(std::integral_constant<int, UNISERVE_ACTIVATION_SILU>{});
    }
    __syncthreads();
    // Written as the FC2 operand: each (row, 128-column group) quantised by 16 lanes (one DPP
    // row) from the bf16 values (the stand-alone quantiser's rounding points and encoding: amax of
    // the bf16 values, s = amax / 448, code = e4m3(v / s)); live rows only. Every lane's passes
    // are independent: their LDS reads, reductions and encodings interleave.
    constexpr int kGroups = kOutCols / 128;
    constexpr int kPasses = kRows * kGroups / (kThreads / 16);
    static_assert(kRows * kGroups % (kThreads / 16) == 0, "whole passes");
    const int sub = t & 15;
    const int64_t groups_per_row = p.out_width / 128;
    float v[kPasses][8];
    float amax[kPasses];
#pragma unroll
    for (int pass = 0; pass < kPasses; ++pass) {
      const int index = t / 16 + pass * (kThreads / 16);
      const int m = index / kGroups;
      const int group = index - m * kGroups;
      const u32x4 piece = *reinterpret_cast<const u32x4 *>(lds + m * kOutStride + (group * 128 + sub * 8) * 2);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[pass][2 * j] = __uint_as_float(piece[j] << 16);
        v[pass][2 * j + 1] = __uint_as_float(piece[j] & 0xffff0000u);
      }
      amax[pass] = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) amax[pass] = __builtin_fmaxf(amax[pass], __builtin_fabsf(v[pass][j]));
    }
#pragma unroll
    for (int pass = 0; pass < kPasses; ++pass) amax[pass] = row16_max(amax[pass]);
    // Every pass without division (e4m3_eight_bf16); the rare (row, group)s it leaves - a NaN,
    // a scale outside its range - are encoded by division afterwards, from the staged tile, in
    // one copy of that code.
    uint32_t redo = 0;
#pragma unroll
    for (int pass = 0; pass < kPasses; ++pass) {
      const int index = t / 16 + pass * (kThreads / 16);
      const int m = index / kGroups;
      const int group = index - m * kGroups;
      if (m >= rows) continue;
      const float scale = amax[pass] > 0.0f ? amax[pass] / 448.0f : 1.0f;
      const int64_t column = slice_col + group * 128 + sub * 8;
      uint2 codes;
      if (!e4m3_eight_bf16(v[pass], scale, codes)) redo |= 1u << pass;
      *reinterpret_cast<uint2 *>(p.out_codes + (first + m) * p.out_width + column) = codes;
      if (sub == 0) {
        const int64_t at = p.scale_rows != 0 ? column / 128 * p.scale_rows + first + m
                                             : (first + m) * groups_per_row + column / 128;
        p.out_code_scales[at] = scale;
      }
    }
#pragma unroll 1
    for (int pass = 0; pass < kPasses; ++pass) {
      if (__ballot((redo >> pass) & 1u) == 0) continue;  // uniform: the whole wavefront redoes it
      const int index = t / 16 + pass * (kThreads / 16);
      const int m = index / kGroups;
      const int group = index - m * kGroups;
      const u32x4 piece = *reinterpret_cast<const u32x4 *>(lds + m * kOutStride + (group * 128 + sub * 8) * 2);
      float w[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        w[2 * j] = __uint_as_float(piece[j] << 16);
        w[2 * j + 1] = __uint_as_float(piece[j] & 0xffff0000u);
      }
      float wmax = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) wmax = __builtin_fmaxf(wmax, __builtin_fabsf(w[j]));
      wmax = row16_max(wmax);
      if (m >= rows || ((redo >> pass) & 1u) == 0) continue;
      const float scale = wmax > 0.0f ? wmax / 448.0f : 1.0f;
      const int64_t column = slice_col + group * 128 + sub * 8;
      *reinterpret_cast<uint2 *>(p.out_codes + (first + m) * p.out_width + column) = e4m3_eight(w, scale);
    }
  }
}

}  // namespace pair

/// Whether the two-workgroup kernel serves the shape: whole 128-byte stages (at least three; e4m3:
/// at most 64, and route-major activation scales), whole slices (FC1 128 output columns, FC2 256).
template <class F>
inline bool pair_fits(bool gated, int64_t K, int64_t out_width, int64_t scale_rows) {
  const int64_t columns = gated ? pair::kSliceRows / 2 : pair::kSliceRows;
  const int64_t row_bytes = K * F::kElementBytes;
  if (row_bytes % 128 != 0 || row_bytes / 128 < 3 || out_width % columns != 0) return false;
  if constexpr (F::kScaled) return row_bytes / 128 <= kWave && scale_rows != 0;
  return true;
}

/// Launches it over `max_tiles` tiles (tiles past `num_tiles` exit at once); with `p.out_codes`
/// set (e4m3 FC1 only) the gated rows are written as e4m3 codes and scales.
#ifndef UNISERVE_PAIR_GROUP
#define UNISERVE_PAIR_GROUP 4
#endif
template <class F>
inline void launch_pair(PrefillParams p, bool gated, int64_t max_tiles, hipStream_t stream, int group = UNISERVE_PAIR_GROUP) {
  const int64_t columns = gated ? pair::kSliceRows / 2 : pair::kSliceRows;
  p.slices = static_cast<int32_t>(p.out_width / columns);
  p.max_tiles = static_cast<int32_t>(max_tiles);
  p.group = group;
  p.groups_per_xcd = static_cast<int32_t>(ceil_div<int64_t>(ceil_div<int64_t>(max_tiles, group), 8));
  const dim3 grid(static_cast<uint32_t>(static_cast<int64_t>(p.groups_per_xcd) * group * p.slices * 8));
  const dim3 block(static_cast<uint32_t>(pair::kThreads));
  if (gated) hipLaunchKernelGGL((pair::pair_kernel<F, true>), grid, block, 0, stream, p);
  else hipLaunchKernelGGL((pair::pair_kernel<F, false>), grid, block, 0, stream, p);
}

}  // namespace uniserve

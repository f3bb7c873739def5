// SPDX-License-Identifier: Apache-2.0
//
// The prefill-shaped grouped products (FC1 with SiLU, or FC2) on gfx950, in bf16 or in 128 x 128
// block-scaled OCP e4m3.
//
// One workgroup (8 wavefronts, two per SIMD) owns one 128-row sort tile and a 512-row slice of its
// expert's weight rows (FC1: 256 up rows and the matching 256 gate rows; FC2: 512 output columns).
// K is walked in stages of 128 bytes per row (64 bf16 or 128 e4m3 elements: one scale block).
//
//  * Both operands travel HBM/L2 -> LDS by `global_load_lds_dwordx4`: eight lanes cover one
//    128-byte row, so every load is fully coalesced (rows gathered by the sort's maps for FC1).
//    Two LDS stages of 80 KB (16 KB activations + 64 KB weights), one barrier per stage. The
//    activation rows of stage k + 1 fly while stage k multiplies. bf16 weight rows fly two stages:
//    a wave reads only its own weight rows, so it refills them with stage k + 2 as soon as it holds
//    stage k's in registers.
//  * LDS rows are 8 chunks of 16 bytes, chunk c of row r stored at c ^ key(r) with
//    key(r) = (r >> 1) & 7: a DMA instruction writes 8 whole rows, and a 16-lane group of an MFMA
//    fragment read (16 consecutive rows, one logical chunk) hits all 64 banks once - rows of one
//    parity see 8 distinct chunks. The key repeats every 16 rows, so the fragment reads of every
//    32-row block share one address per chunk, up to an immediate offset.
//  * Wavefront w multiplies all 128 activation rows by its own 64 weight rows with 32x32 MFMAs
//    (weights as operand A, activations as operand B): a lane ends with four consecutive output
//    columns of one token row (an 8-byte store), and SiLU's up column n and gate column n meet in
//    one lane.
//  * e4m3: one 32x32x64 MFMA pair spans one scale block; its FP32 block result is added into the
//    accumulator times s_w * s_x (weight block scale, a wave-uniform scalar, times the row's
//    activation scale). Two waves per SIMD keep the MFMA pipe busy while the other wave's VALU
//    applies its scales. bf16: the MFMA accumulates directly.
//
// Both operands share one permutation of K inside a stage (lane half h holds bytes 64 h .. 64 h + 63
// of the stage's 128, its steps in order), which changes only the FP32 summation order.
//
// Work items (tile, slice) come in groups of `group` consecutive tiles, slice-major inside a group;
// the groups are dealt to the 8 XCDs in turn (block b runs on XCD b % 8; group g on XCD g % 8), and
// each XCD runs its groups in order. The workgroups resident on one XCD at a time share a few
// weight slices and activation tiles in that XCD's L2, and every XCD gets a like share of the
// experts with few tiles, whose weights stream from HBM with no reuse (a contiguous range of tiles
// per XCD would leave some XCDs all single-tile experts and others one heavy expert).
#pragma once

#include "common.hpp"
#include "grouped_fp8.hpp"

namespace uniserve {

struct PrefillParams {
  const uint8_t *act;            ///< FC1: [tokens, K]; FC2: [permuted_rows, K]
  const float *act_scales;       ///< e4m3: [rows of act, K / 128]
  const uint8_t *weights;        ///< [experts, n_total, K]
  const float *weight_scales;    ///< e4m3: [experts, n_total / 128, K / 128]
  uint16_t *out;                 ///< [permuted_rows, out_width] bf16
  const int32_t *tile_to_expert;
  const int32_t *tile_to_limit;
  const int32_t *permuted_to_expanded;
  const int32_t *num_tiles;
  int64_t K;                     ///< elements
  int64_t n_total;               ///< weight rows per expert: 2 I (FC1) or H (FC2)
  int64_t out_width;             ///< I (FC1) or H (FC2)
  int64_t top;
  int32_t slices;                ///< weight-row slices per tile
  int32_t max_tiles;
  int32_t group;                 ///< tiles per work group of the numbering
  int32_t groups_per_xcd;        ///< groups of tiles each XCD runs
  uint8_t *out_codes;            ///< FC1 only, or null: write the gated rows as e4m3 codes
  float *out_code_scales;        ///< with out_codes: [permuted_rows, out_width / 128]
  int64_t scale_rows;            ///< nonzero: act_scales are [K / 128, scale_rows] and out_code_scales
                                 ///< [out_width / 128, scale_rows], both indexed by permuted row
  int32_t activation;            ///< FC1's gate: UNISERVE_ACTIVATION_SILU or _GELU_TANH
};

namespace prefill {

constexpr int kRows = 128;                       // activation rows per tile
constexpr int kWaveRows = 64;                    // weight rows per wavefront
constexpr int kChunks = 8;                       // 16-byte chunks per 128-byte stage row
constexpr int kActChunks = kRows * kChunks;
constexpr int kWeightLoads = kWaveRows * kChunks / kWave;     // 8 (the wave's own rows)

typedef float floatx16 __attribute__((ext_vector_type(16)));

/// bf16: 4 MFMA steps of 16 bytes per stage; eight wavefronts over 512 weight rows, two 80 KB
/// LDS stages (measured faster than four wavefronts over 256 rows with three 48 KB stages).
struct Bf16 {
  static constexpr int kSteps = 4;
  static constexpr int kPieces = 1;  // 16-byte pieces per lane per step
  static constexpr bool kScaled = false;
  static constexpr int kWaves = 8;
  static constexpr int kStages = 2;
};

/// e4m3: 2 MFMA steps of 32 bytes per stage; eight wavefronts (two per SIMD: one wave's MFMAs
/// cover the other's scaling) over 512 weight rows, two 80 KB LDS stages.
struct E4m3 {
  static constexpr int kSteps = 2;
  static constexpr int kPieces = 2;
  static constexpr bool kScaled = true;
  static constexpr int kWaves = 8;
  static constexpr int kStages = 2;
};

/// Weight rows of a slice, and the output columns one workgroup covers.
template <class F>
constexpr int weight_rows() {
  return F::kWaves * kWaveRows;
}
template <class F, bool kGated>
constexpr int slice_width() {
  return kGated ? weight_rows<F>() / 2 : weight_rows<F>();
}

__device__ __forceinline__ int key(int row) { return (row >> 1) & 7; }
__device__ __forceinline__ int slot(int row, int chunk) { return row * kChunks + (chunk ^ key(row)); }

template <class F>
struct Operand {
  u32x4 piece[F::kPieces];
};

template <class F>
__device__ __forceinline__ floatx16 mma(const Operand<F> &w, const Operand<F> &a, floatx16 c) {
  if constexpr (F::kScaled) {
    const intx8 wa = __builtin_bit_cast(intx8, w);
    const intx8 aa = __builtin_bit_cast(intx8, a);
    // cbsz/blgp 0: e4m3 x e4m3; scale exponents 127 = 2^0 (the block scales are applied after).
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wa, aa, c, 0, 0, 0, 127, 0, 127);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, w.piece[0]),
                                                   __builtin_bit_cast(bf16x8, a.piece[0]), c, 0, 0, 0);
  }
}

template <class F>
struct Stage {
  u32x4 act[kActChunks];
  u32x4 weights[weight_rows<F>() * kChunks];
};

/// One 16-byte DMA per lane from `base` + `offset` (base wave-uniform, in SGPRs) into LDS at
/// `lds` + 16 * lane (`lds` wave-uniform). Issued as inline assembly so the compiler does not
/// count it: the K loop waits for these loads itself, once per stage, before its barrier. No
/// memory clobber: the barriers order it against the LDS reads, and the global memory it reads
/// is never written by the kernel (so the weight scales can stay scalar loads).
__device__ __forceinline__ void dma16(const void *base, uint32_t offset, uint32_t lds) {
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %1\n\t"
      :
      : "v"(offset), "s"(base), "s"(lds)
      : "m0");
}

/// `dma16` preceded by a wait for this wave's outstanding LDS reads, so the DMA cannot overwrite
/// LDS that an earlier `ds_read` of the wave has not read yet.
__device__ __forceinline__ void dma16_after_lds_reads(const void *base, uint32_t offset, uint32_t lds) {
  asm volatile(
      "s_waitcnt lgkmcnt(0)\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %1\n\t"
      :
      : "v"(offset), "s"(base), "s"(lds)
      : "m0");
}

/// Waits until at most N vector-memory loads of this wave are outstanding (they complete in
/// issue order); the other counters untouched.
template <int N>
__device__ __forceinline__ void wait_loads_but() {
  static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
  __builtin_amdgcn_s_waitcnt(0x0f70 | (N & 15) | ((N >> 4) << 14));
}

/// Waits until every vector-memory load of this wave has landed (vmcnt 0; the other counters
/// untouched). The compiler sees the wait, so it knows its own loads issued before are complete.
__device__ __forceinline__ void wait_all_loads() { __builtin_amdgcn_s_waitcnt(0x0f70); }


__device__ __forceinline__ uint32_t lds_address(const void *pointer) {
  typedef const __attribute__((address_space(3))) char *lds_pointer;
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_pointer)pointer));
}

template <class F, bool kGated>
__global__ void __launch_bounds__(F::kWaves * kWave) prefill_kernel(PrefillParams p) {
  constexpr int NS = F::kSteps;
  constexpr int NP = F::kPieces;
  constexpr int kThreads = F::kWaves * kWave;
  constexpr int kActLoads = kActChunks / kWave / F::kWaves;  // DMA instructions per wave per stage
  // The DMA is invisible to the compiler, so one array of stages is as good as separate objects.
  __shared__ Stage<F> ring[F::kStages];

  // ---- the work item ----
  const int b = static_cast<int>(blockIdx.x);
  const int span = p.group * p.slices;        // work items of one group of tiles
  const int seq = b >> 3;                      // this block's place in its XCD's sequence
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
  const int h = lane >> 5;
  const int r32 = lane & 31;
  const int64_t row_bytes = p.K * (F::kScaled ? 1 : 2);
  const int stages = static_cast<int>(row_bytes / 128);
  // The activation row behind tile row r: FC1 gathers token permuted_to_expanded / top (the maps
  // are read unconditionally - they span every tile - and padding rows take row 0), FC2 reads its
  // own permuted row (padding rows read the tile's first row).
  const int top = static_cast<int>(p.top);
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

  // ---- DMA sources: instruction i of this wave fills 8 whole LDS rows; lane l brings logical
  // chunk (l % 8) ^ key(row) of row 8 i' + l / 8, landing in physical chunk l % 8 ----
  // 32-bit lane offsets from wave-uniform bases keep the addresses in one VGPR each (the DMA's
  // scalar-base form).
  uint32_t a_off[kActLoads];
#pragma unroll
  for (int i = 0; i < kActLoads; ++i) {
    const int r = (wave * kActLoads + i) * 8 + lane / 8;
    const int64_t source = act_row(r);
    a_off[i] = static_cast<uint32_t>(source * row_bytes + ((lane & 7) ^ key(r)) * 16);
  }
  // This wave's 64 weight rows (LDS rows 64 w ..): FC1 rows 0..31 are up rows, 32..63 the gate
  // rows of the same 32 output columns; FC2 rows are 64 consecutive output columns.
  const int64_t slice_col = static_cast<int64_t>(slice) * slice_width<F, kGated>();
  const int64_t wave_col = slice_col + wave * (kGated ? 32 : 64);
  auto weight_row = [&](int j) -> int64_t {  // first weight row of 32-row block j of this wave
    if constexpr (kGated) return j == 0 ? wave_col : p.out_width + wave_col;
    else return wave_col + 32 * j;
  };
  bool block_live[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) block_live[j] = kGated || weight_row(j) < p.out_width;
  // Row r = 8 i + l / 8 of the wave's 64 (i = 0..7; block r / 32): key(64 w + r) =
  // 4 (i % 2) + (l / 16) % 4, so lane l's chunk is (l % 8) ^ ((l / 16) % 4) ^ 4 (i % 2) - one lane
  // offset plus a wave-uniform base per i.
  const uint8_t *w_block[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
    w_block[j] = p.weights + (expert * p.n_total + (block_live[j] ? weight_row(j) : 0)) * row_bytes;
  const uint32_t w_lane = static_cast<uint32_t>((lane / 8) * row_bytes);
  const uint32_t w_chunk = static_cast<uint32_t>((lane & 7) ^ ((lane >> 4) & 3));
  auto issue_act = [&](Stage<F> &st, int k) {
    const int64_t offset = static_cast<int64_t>(k) * 128;
    const uint32_t act_lds = lds_address(st.act + wave * kActLoads * kWave);
#pragma unroll
    for (int i = 0; i < kActLoads; ++i)
      dma16(act_tile + offset, a_off[i], __builtin_amdgcn_readfirstlane(act_lds + i * kWave * 16));
  };
  // `after_reads`: the wave's own weight rows of `st` were just read into registers; the first
  // DMA waits for those LDS reads (lgkmcnt 0) before it may overwrite them.
  auto issue_weights = [&](Stage<F> &st, int k, bool after_reads) {
    const int64_t offset = static_cast<int64_t>(k) * 128;
    const uint32_t weight_lds = lds_address(st.weights + wave * kWaveRows * kChunks);
#pragma unroll
    for (int i = 0; i < kWeightLoads; ++i) {
      const uint8_t *base = w_block[i / 4] + offset + (i % 4) * 8 * row_bytes;
      const uint32_t lane_offset = w_lane + ((w_chunk ^ static_cast<uint32_t>(4 * (i & 1))) << 4);
      const uint32_t lds = __builtin_amdgcn_readfirstlane(weight_lds + i * 8 * kChunks * 16);
      if (i == 0 && after_reads) dma16_after_lds_reads(base, lane_offset, lds);
      else dma16(base, lane_offset, lds);
    }
  };

  // ---- e4m3 scales: the activation scales of this lane's four token rows (prefetched a stage
  // ahead) and the weight blocks' scales (wave-uniform) ----
  const int kb_count = static_cast<int>(p.K / 128);
  // The activation scales of this lane's four tile rows: by permuted row, block-major (a stage's
  // 128 scales are one contiguous run: one cache line per 32 lanes), or row-major by source row
  // (FC1 gathers them from token rows). Padding rows take the tile's first row.
  int sx_row[4];
  const int64_t sx_block_stride = p.scale_rows != 0 ? p.scale_rows : 1;
  const float *sw_src[2];
  if constexpr (F::kScaled) {
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
      const int r = mi * 32 + r32;
      sx_row[mi] = p.scale_rows != 0 ? static_cast<int>(first) + (r < rows ? r : 0)
                                     : static_cast<int>(source_row(r)) * kb_count;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
      sw_src[j] = p.weight_scales + (expert * (p.n_total / 128) + (block_live[j] ? weight_row(j) : 0) / 128) * kb_count;
  }

  floatx16 acc[4][2];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[mi][j][e] = 0.0f;

  float sx[2][4];
  float sw[2][2];
  auto load_scales = [&](int buffer, int k) {
    if constexpr (F::kScaled) {
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) sx[buffer][mi] = (p.act_scales + k * sx_block_stride)[sx_row[mi]];
      sw[buffer][0] = sw_src[0][k];
      sw[buffer][1] = sw_src[1][k];
    }
  };

  auto compute = [&](const Stage<F> &st, int sb, auto &&after_weight_reads) {
    // The wave's weight fragments for the whole stage, then one 32-row activation block at a time.
    Operand<F> wf[2][NS];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int q = 0; q < NP; ++q)
          wf[j][s].piece[q] = st.weights[slot(wave * kWaveRows + j * 32 + r32, 4 * h + s * NP + q)];
    after_weight_reads();
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
      Operand<F> af[NS];
#pragma unroll
      for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int q = 0; q < NP; ++q) af[s].piece[q] = st.act[slot(mi * 32 + r32, 4 * h + s * NP + q)];
      if constexpr (F::kScaled) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          floatx16 block = {};
#pragma unroll
          for (int s = 0; s < NS; ++s) block = mma<F>(wf[j][s], af[s], block);
          const float scale = sw[sb][j] * sx[sb][mi];
#pragma unroll
          for (int e = 0; e < 16; ++e) acc[mi][j][e] = __builtin_fmaf(block[e], scale, acc[mi][j][e]);
        }
        // Bound the live fragments and block results to one activation block (the register
        // budget at two waves per SIMD); the SIMD's other wave covers the latencies.
        __builtin_amdgcn_sched_barrier(0);
      } else {
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
          for (int j = 0; j < 2; ++j) acc[mi][j] = mma<F>(wf[j][s], af[s], acc[mi][j]);
      }
    }
  };

  // ---- the K loop (an even number of stages) ----
  auto nothing = [] {};
  if constexpr (F::kScaled) {
    // e4m3: stage k + 1's DMA and activation scales fly while stage k multiplies. Each wave waits
    // for its own loads, then the barrier for every wave, so the stage is complete and the other
    // buffer is free to refill. (The scale loads are compiler-visible: the compiler waits for all
    // loads before their use, so nothing may stay in flight across a stage here.) The DMA of the
    // last stage re-reads it (unconditional issue keeps the waits exact).
    issue_act(ring[0], 0);
    issue_weights(ring[0], 0, false);
    load_scales(0, 0);
    for (int k = 0; k < stages; k += 2) {
      wait_all_loads();
      __syncthreads();
      issue_act(ring[1], k + 1);
      issue_weights(ring[1], k + 1, false);
      load_scales(1, k + 1);
      compute(ring[0], 0, nothing);
      wait_all_loads();
      __syncthreads();
      issue_act(ring[0], min(k + 2, stages - 1));
      issue_weights(ring[0], min(k + 2, stages - 1), false);
      load_scales(0, min(k + 2, stages - 1));
      compute(ring[1], 1, nothing);
    }
  } else {
    // bf16: a wave's weight rows are read by that wave alone, and it holds a stage's weight
    // fragments in registers before it multiplies. So it refills its own rows of the buffer with
    // stage k + 2 as soon as it has read stage k's - two stages of cover for 80% of the bytes,
    // with no barrier in between. The shared activation rows refill after each barrier (stage
    // k + 1 while k multiplies). At each barrier every load but the wave's latest weight refill
    // has landed. Loads past the last stage re-read it, keeping the counts exact.
    issue_act(ring[0], 0);
    issue_weights(ring[0], 0, false);
    issue_weights(ring[1], min(1, stages - 1), false);
    for (int k = 0; k < stages; k += 2) {
      wait_loads_but<kWeightLoads>();
      __syncthreads();
      issue_act(ring[1], k + 1);
      compute(ring[0], 0, [&] { issue_weights(ring[0], min(k + 2, stages - 1), true); });
      wait_loads_but<kWeightLoads>();
      __syncthreads();
      issue_act(ring[0], min(k + 2, stages - 1));
      compute(ring[1], 1, [&] { issue_weights(ring[1], min(k + 3, stages - 1), true); });
    }
  }
  // The last refills re-read the final stage; they land before the epilogue reuses the LDS.
  wait_all_loads();

  // ---- epilogue: the output tile goes through LDS so the global stores are whole rows. Lane holds
  // token row 32 mi + lane % 32 and, of block j, weight rows 8 q + 4 h + i in element 4 q + i.
  // LDS rows are padded to kOutStride bytes (8 more than a multiple of 256), so the
  // 32 rows one 8-byte write instruction touches fall on distinct banks. Rows 0..63 live in the
  // first stage buffer, rows 64..127 in the second. ----
  constexpr int kOutCols = slice_width<F, kGated>();
  constexpr int kOutStride = kOutCols * 2 + 8;
  static_assert(64 * kOutStride <= static_cast<int>(sizeof(Stage<F>)), "the output tile fits the stage buffers");
  auto out_row = [&](int m) -> char * {
    return (m < 64 ? reinterpret_cast<char *>(&ring[0]) : reinterpret_cast<char *>(&ring[1])) + (m & 63) * kOutStride;
  };
  __syncthreads();  // every wave is done reading the stage buffers
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
    char *row = out_row(mi * 32 + r32);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if constexpr (kGated) {
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = gate(acc[mi][1][4 * q + i], p.activation) * acc[mi][0][4 * q + i];
        uint2 packed;
        packed.x = pack_bf16x2(v[0], v[1]);
        packed.y = pack_bf16x2(v[2], v[3]);
        *reinterpret_cast<uint2 *>(row + (wave * 32 + 8 * q + 4 * h) * 2) = packed;
      } else {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          uint2 packed;
          packed.x = pack_bf16x2(acc[mi][j][4 * q], acc[mi][j][4 * q + 1]);
          packed.y = pack_bf16x2(acc[mi][j][4 * q + 2], acc[mi][j][4 * q + 3]);
          *reinterpret_cast<uint2 *>(row + (wave * 64 + j * 32 + 8 * q + 4 * h) * 2) = packed;
        }
      }
    }
  }
  __syncthreads();
  if (kGated && p.out_codes != nullptr) {
    // Write-out as the FC2 operand: each (row, 128-column group) is quantised by 16 lanes from the
    // bf16 values in LDS (the same rounding points and encoding as the stand-alone quantiser:
    // amax of the bf16 values, s = amax / 448, code = e4m3(v / s)), live rows only.
    constexpr int kGroups = kOutCols / 128;
    const int sub = t & 15;
    const int64_t groups_per_row = p.out_width / 128;
    for (int index = t / 16; index < kRows * kGroups; index += kThreads / 16) {
      const int m = index / kGroups;
      const int group = index - m * kGroups;
      const u32x4 piece = *reinterpret_cast<const u32x4 *>(out_row(m) + (group * 128 + sub * 8) * 2);
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
      const int64_t column = slice_col + group * 128 + sub * 8;
      *reinterpret_cast<uint2 *>(p.out_codes + (first + m) * p.out_width + column) = e4m3_eight_of_bf16(v, scale);
      if (sub == 0) {
        const int64_t at = p.scale_rows != 0 ? column / 128 * p.scale_rows + first + m
                                             : (first + m) * groups_per_row + column / 128;
        p.out_code_scales[at] = scale;
      }
    }
    return;
  }
  // Write-out: 16-byte pieces, consecutive lanes along a row; live rows and columns only.
  constexpr int kPieces = kOutCols / 8;
  const int64_t live_cols = min(static_cast<int64_t>(kOutCols), p.out_width - slice_col);
  for (int index = t; index < kRows * kPieces; index += kThreads) {
    const int m = index / kPieces;
    const int c = index - m * kPieces;
    if (m >= rows || c * 8 >= live_cols) continue;
    const u32x4 piece = *reinterpret_cast<const u32x4 *>(out_row(m) + c * 16);
    *reinterpret_cast<u32x4 *>(p.out + (first + m) * p.out_width + slice_col + c * 8) = piece;
  }
}

}  // namespace prefill

/// Whether the prefill kernel serves this shape: an even number of 128-byte K stages, FC1 widths
/// of whole 256-column slices, FC2 widths of whole 32-row blocks (e4m3: whole 128-row scale blocks);
/// FC2 widths that are a multiple of 8 columns keep the epilogue's 16-byte pieces whole.
template <class F, bool kGated>
inline bool prefill_fits(int64_t K, int64_t out_width) {
  const int64_t row_bytes = K * (F::kScaled ? 1 : 2);
  if (row_bytes % 256 != 0 || row_bytes == 0) return false;
  if (kGated) return out_width % prefill::slice_width<F, kGated>() == 0;
  return out_width % (F::kScaled ? 128 : 32) == 0;
}

/// Launches the prefill product over `max_tiles` tiles (tiles past `num_tiles` exit at once).
template <class F, bool kGated>
inline void launch_prefill(PrefillParams p, int64_t max_tiles, hipStream_t stream, int group = 16) {
  p.slices = static_cast<int32_t>(ceil_div<int64_t>(p.out_width, prefill::slice_width<F, kGated>()));
  p.max_tiles = static_cast<int32_t>(max_tiles);
  p.group = group;
  p.groups_per_xcd = static_cast<int32_t>(ceil_div<int64_t>(ceil_div<int64_t>(max_tiles, group), 8));
  const int64_t blocks = static_cast<int64_t>(p.groups_per_xcd) * group * p.slices * 8;
  hipLaunchKernelGGL((prefill::prefill_kernel<F, kGated>), dim3(static_cast<uint32_t>(blocks)),
                     dim3(F::kWaves * kWave), 0, stream, p);
}

}  // namespace uniserve

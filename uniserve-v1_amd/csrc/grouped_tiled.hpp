// SPDX-License-Identifier: Apache-2.0
//
// The prefill-shaped bf16 grouped product (FC1 with SiLU, or FC2) on gfx950.
//
// One workgroup (4 wavefronts) owns one 128-row sort tile and a 256-row slice of its expert's
// weight rows (FC1: 128 up rows and the matching 128 gate rows; FC2: 256 output columns), and
// walks K in stages of 64 elements (128 bytes) per row:
//
//  * operands travel HBM -> LDS by `global_load_lds_dwordx4` (no VGPR staging), three stages in
//    flight; the wait for a stage is an explicit `s_waitcnt vmcnt` on the loads of the stages
//    behind it, so the next two stages keep streaming while the MFMAs consume the current one;
//  * LDS rows are 8 chunks of 16 bytes, chunk c of row r stored at c ^ key(r) with
//    key(r) = (r ^ (r >> 3)) & 7, which keeps a 16-row MFMA fragment read free of bank conflicts
//    on 8- and 16-lane LDS issue groups;
//  * each wavefront computes 64 rows x 128 weight rows with 32x32x16 MFMAs (2 x 4 blocks, 128
//    accumulators), weights as MFMA operand A and activations as operand B, so a lane ends with
//    four consecutive output columns of one row and SiLU's up/gate pair in the same lane.
//
// Workgroups are numbered XCD-major: consecutive work items (the slices of one tile, then the
// next tiles of the same expert) run on the same XCD and share its L2.
#pragma once

#include "common.hpp"

namespace uniserve {

struct TiledParams {
  const void *act;            ///< FC1: [tokens, K]; FC2: [permuted_rows, K]; bf16
  const void *weights;        ///< [experts, n_total, K] bf16
  uint16_t *out;              ///< [permuted_rows, out_width] bf16
  const int32_t *tile_to_expert;
  const int32_t *tile_to_limit;
  const int32_t *permuted_to_expanded;
  const int32_t *num_tiles;
  int64_t K;                  ///< elements
  int64_t n_total;
  int64_t out_width;
  int64_t top;
  int32_t slices;             ///< weight-row slices per tile
  int32_t work;               ///< max_tiles * slices
};

namespace tiled {

constexpr int kThreads = 256;
constexpr int kRows = 128;           // activation rows per tile
constexpr int kWeightRows = 256;     // weight rows per slice
constexpr int kChunks = 8;           // 16-byte chunks per row per stage
constexpr int kStages = 3;
constexpr int kActChunks = kRows * kChunks;          // 1024 chunks = 16 KB
constexpr int kWeightChunks = kWeightRows * kChunks; // 2048 chunks = 32 KB
constexpr int kStageChunks = kActChunks + kWeightChunks;
constexpr int kActLoads = kActChunks / kWave / 4;        // DMA instructions per wave per stage: 4
constexpr int kWeightLoads = kWeightChunks / kWave / 4;  // 8

__device__ __forceinline__ int key(int row) { return (row ^ (row >> 3)) & 7; }
__device__ __forceinline__ int slot(int row, int chunk) { return row * kChunks + (chunk ^ key(row)); }

/// One 16-byte DMA from global memory into LDS at `lds` + 16 * lane (`lds` wave-uniform). The
/// compiler does not see it as a load, so the waits for it are `wait_loads` and nothing else.
__device__ __forceinline__ void dma16(const void *src, uint32_t lds) {
  asm volatile(
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, off\n\t"
      :
      : "v"(src), "s"(lds)
      : "memory", "m0");
}

template <int kOutstanding>
__device__ __forceinline__ void wait_loads() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kOutstanding) : "memory");
}

__device__ __forceinline__ uint32_t lds_address(const void *p) {
  typedef const __attribute__((address_space(3))) char *lds_pointer;
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_pointer)p));
}

template <bool kGated>
__global__ void __launch_bounds__(kThreads, 1) tiled_kernel(TiledParams p) {
  __shared__ u32x4 stages[kStages][kStageChunks];
  constexpr int kLoadsPerStage = kActLoads + kWeightLoads;

  // XCD-major work numbering: block b runs on XCD b % 8.
  const int per_xcd = (p.work + 7) / 8;
  const int b = static_cast<int>(blockIdx.x);
  const int w_index = (b % 8) * per_xcd + b / 8;
  if (w_index >= p.work) return;
  const int tile = w_index / p.slices;
  const int slice = w_index % p.slices;
  if (tile >= p.num_tiles[0]) return;

  const int64_t expert = p.tile_to_expert[tile];
  const int64_t first = static_cast<int64_t>(tile) * kRows;
  const int rows = p.tile_to_limit[tile] - static_cast<int>(first);
  const int t = static_cast<int>(threadIdx.x);
  const int wave = t / kWave;
  const int lane = lane_id();
  const int wm = wave & 1;
  const int wn = wave >> 1;
  const int64_t row_bytes = p.K * 2;
  const int64_t n_base = static_cast<int64_t>(slice) * (kGated ? 128 : 256);

  // This lane's DMA sources: LDS chunk (64 j + lane) holds row 8 j + lane / 8, logical chunk
  // (lane % 8) ^ key(row).
  const char *act = static_cast<const char *>(p.act);
  const char *wts = static_cast<const char *>(p.weights);
  const char *a_src[kActLoads];
  const char *w_src[kWeightLoads];
#pragma unroll
  for (int i = 0; i < kActLoads; ++i) {
    const int j = wave * kActLoads + i;
    const int r = 8 * j + lane / 8;
    const int c = (lane & 7) ^ key(r);
    int64_t source = 0;
    if (r < rows) {
      if constexpr (kGated) source = p.permuted_to_expanded[first + r] / p.top;
      else source = first + r;
    }
    a_src[i] = act + source * row_bytes + c * 16;
  }
#pragma unroll
  for (int i = 0; i < kWeightLoads; ++i) {
    const int j = wave * kWeightLoads + i;
    const int r = 8 * j + lane / 8;
    const int c = (lane & 7) ^ key(r);
    int64_t n;
    if constexpr (kGated) n = r < 128 ? n_base + r : p.out_width + n_base + (r - 128);
    else n = n_base + r < p.out_width ? n_base + r : 0;
    w_src[i] = wts + (expert * p.n_total + n) * row_bytes + c * 16;
  }
  const uint32_t lds_base = lds_address(&stages[0][0]);
  auto issue = [&](int stage_index, int64_t k_bytes) {
    const uint32_t base = lds_base + static_cast<uint32_t>(stage_index * kStageChunks * 16);
#pragma unroll
    for (int i = 0; i < kActLoads; ++i)
      dma16(a_src[i] + k_bytes, __builtin_amdgcn_readfirstlane(base + ((wave * kActLoads + i) * kWave) * 16));
#pragma unroll
    for (int i = 0; i < kWeightLoads; ++i)
      dma16(w_src[i] + k_bytes,
            __builtin_amdgcn_readfirstlane(base + (kActChunks + (wave * kWeightLoads + i) * kWave) * 16));
  };


  // Accumulators: 2 x 4 blocks of 32 x 32 (rows wm * 64 + 32 mi, weight blocks of 32 rows).
  typedef float floatx16 __attribute__((ext_vector_type(16)));
  floatx16 acc16[2][4];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc16[mi][ni][i] = 0.0f;

  // First LDS weight row of each of the wave's four 32-row MFMA blocks (FC1: the first two are
  // up rows, the other two the matching gate rows).
  auto weight_row = [&](int ni) {
    if constexpr (kGated) return ni < 2 ? wn * 64 + ni * 32 : 128 + wn * 64 + (ni - 2) * 32;
    else return wn * 128 + ni * 32;
  };

  const int steps = static_cast<int>(row_bytes / 128);
  issue(0, 0);
  if (steps > 1) issue(1, 128);
  for (int step = 0; step < steps; ++step) {
    const int stage_index = step % kStages;
    if (step + 1 < steps) wait_loads<kLoadsPerStage>();
    else wait_loads<0>();
    __syncthreads();
    if (step + 2 < steps) issue((step + 2) % kStages, static_cast<int64_t>(step + 2) * 128);
    const u32x4 *act_stage = stages[stage_index];
    const u32x4 *w_stage = stages[stage_index] + kActChunks;
    {
      // 32x32x16 MFMAs: lane l supplies row l % 32 and K elements 8 (l / 32) .. + 8 of the
      // 16-element step, i.e. 16-byte chunk 2 s + l / 32 of the stage's 128-byte row segment.
      const int h = lane >> 5;
      const int r32 = lane & 31;
      // Fragments of step s + 1 are read before the MFMAs of step s issue.
      u32x4 af[2][2], wf[2][4];
      auto read = [&](int s, int buffer) {
        const int c = 2 * s + h;
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) af[buffer][mi] = act_stage[slot(wm * 64 + mi * 32 + r32, c)];
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) wf[buffer][ni] = w_stage[slot(weight_row(ni) + r32, c)];
      };
      read(0, 0);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        if (s + 1 < 4) read(s + 1, (s + 1) & 1);
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
          for (int ni = 0; ni < 4; ++ni)
            acc16[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                __builtin_bit_cast(bf16x8, wf[s & 1][ni]), __builtin_bit_cast(bf16x8, af[s & 1][mi]), acc16[mi][ni], 0, 0, 0);
      }
    }
  }

  {
    // Lane l holds token row wm * 64 + 32 mi + l % 32 and, of each 32-row weight block, rows
    // 8 q + 4 (l / 32) + i for element 4 q + i.
    const int h = lane >> 5;
    const int r32 = lane & 31;
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) {
      const int m = wm * 64 + mi * 32 + r32;
      if (m >= rows) continue;
      uint16_t *row = p.out + (first + m) * p.out_width;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if constexpr (kGated) {
#pragma unroll
          for (int ni = 0; ni < 2; ++ni) {
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = silu(acc16[mi][ni + 2][4 * q + i]) * acc16[mi][ni][4 * q + i];
            uint2 packed;
            packed.x = pack_bf16x2(v[0], v[1]);
            packed.y = pack_bf16x2(v[2], v[3]);
            *reinterpret_cast<uint2 *>(row + n_base + wn * 64 + ni * 32 + 8 * q + 4 * h) = packed;
          }
        } else {
#pragma unroll
          for (int ni = 0; ni < 4; ++ni) {
            const int64_t col = n_base + wn * 128 + ni * 32 + 8 * q + 4 * h;
            if (col >= p.out_width) continue;
            uint2 packed;
            packed.x = pack_bf16x2(acc16[mi][ni][4 * q], acc16[mi][ni][4 * q + 1]);
            packed.y = pack_bf16x2(acc16[mi][ni][4 * q + 2], acc16[mi][ni][4 * q + 3]);
            *reinterpret_cast<uint2 *>(row + col) = packed;
          }
        }
      }
    }
  }
}

}  // namespace tiled

/// Launches the tiled product over `max_tiles` tiles. FC1 needs out_width % 128 == 0; FC2 any
/// out_width % 64 == 0; K * element size % 128 == 0 (bf16 K % 64, e4m3 K % 128).
template <bool kGated>
inline void launch_tiled(TiledParams p, int64_t max_tiles, hipStream_t stream) {
  p.slices = static_cast<int32_t>(kGated ? p.out_width / 128 : ceil_div<int64_t>(p.out_width, 256));
  p.work = static_cast<int32_t>(max_tiles * p.slices);
  const int blocks = (p.work + 7) / 8 * 8;
  hipLaunchKernelGGL((tiled::tiled_kernel<kGated>), dim3(blocks), dim3(tiled::kThreads), 0, stream, p);
}

}  // namespace uniserve

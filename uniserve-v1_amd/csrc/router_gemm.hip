// SPDX-License-Identifier: Apache-2.0
//
// The router's scores on gfx950 MFMA: scores[m, n] = alpha * x[m, :] . W[n, :] (+ bias[n]), FP32
// accumulation and one rounding into bf16 - the router `Linear` of the MoE block
// (crates/nn/src/modules/moe.rs:656-671), which the reference runs as its cuBLASLt `gemm` module
// (crates/ops/kernels/gemm/cublas_lt, entry `uniserve_gemm`).
//
// Two kernels. Batches large enough to fill the chip with 64 x 64 output tiles take 64-deep K
// steps through two XOR-swizzled LDS buffers, their loads eight steps ahead in registers. Smaller ones (decode: 64 tokens x 128 experts is two such
// tiles) use 16 x 16 tiles whose contraction is split over the eight wavefronts of a workgroup:
// each wave loads its K steps straight into registers, eight steps in flight, and the partial
// sums meet in LDS in wave order. In both, weight rows are MFMA operand A and token rows
// operand B, so each lane holds four consecutive expert scores of one token.
#include "common.hpp"
#include "router_gemm.hpp"
#include "uniserve_gemm.h"

namespace uniserve {
namespace {

constexpr int kRouterThreads = 256;
constexpr int kBM = 64, kBN = 64, kBK = 64;
constexpr int kDepth = 8;  // K steps whose loads are in flight

__device__ __forceinline__ int swizzled(int row, int chunk) { return row * 8 + (chunk ^ (row & 7)); }

/// kBMTile: tokens per workgroup (64: four waves of 16 tokens x 64 experts; 32: waves of 16
/// tokens x 32 experts, twice the workgroups for the same batch).
template <int kBMTile>
__global__ void __launch_bounds__(kRouterThreads) router_kernel(RouterParams p) {
  constexpr int kXLoads = kBMTile / 32;           // x rows per thread and step
  constexpr int kColBlocks = kBMTile == 64 ? 4 : 2;  // 16-expert blocks per wave
  __shared__ u32x4 shared_x[2][kBMTile * 8];
  __shared__ u32x4 shared_w[2][kBN * 8];
  const int t = static_cast<int>(threadIdx.x);
  const int wave = t / kWave;
  const int lane = lane_id();
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int64_t m0 = static_cast<int64_t>(blockIdx.x) * kBMTile;
  const int64_t n0 = static_cast<int64_t>(blockIdx.y) * kBN;
  // The wave's 16 tokens and first expert of the tile.
  const int wave_m = kBMTile == 64 ? wave * 16 : (wave & 1) * 16;
  const int wave_n = kBMTile == 64 ? 0 : (wave >> 1) * 32;

  const int chunk = t & 7;
  const uint16_t *x_row[2];
  const uint16_t *w_row[2];
  bool x_valid[2], w_valid[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = (t >> 3) + 32 * i;
    x_valid[i] = i < kXLoads && m0 + r < p.m;
    w_valid[i] = n0 + r < p.n;
    x_row[i] = p.x + (x_valid[i] ? m0 + r : 0) * p.x_stride + chunk * 8;
    w_row[i] = p.w + (w_valid[i] ? n0 + r : 0) * p.w_stride + chunk * 8;
  }
  floatx4 acc[kColBlocks];
#pragma unroll
  for (int ni = 0; ni < kColBlocks; ++ni) acc[ni] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  // The K steps' global loads run kDepth steps ahead in registers (the MFMA work of a step is far
  // shorter than a load's latency); each step goes through one of two LDS buffers, one barrier
  // per step.
  const int64_t steps = p.k / kBK;
  u32x4 rx[kDepth][kXLoads], rw[kDepth][2];
  auto load = [&](int d, int64_t step) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      if (i < kXLoads)
        rx[d][i] = x_valid[i] ? *reinterpret_cast<const u32x4 *>(x_row[i] + step * kBK) : u32x4{0, 0, 0, 0};
      rw[d][i] = w_valid[i] ? *reinterpret_cast<const u32x4 *>(w_row[i] + step * kBK) : u32x4{0, 0, 0, 0};
    }
  };
#pragma unroll
  for (int d = 0; d < kDepth; ++d)
    if (d < steps) load(d, d);
  for (int64_t k0 = 0; k0 < steps; k0 += kDepth) {
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
      const int64_t k = k0 + d;
      if (k >= steps) break;
      const int buffer = static_cast<int>(k & 1);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int r = (t >> 3) + 32 * i;
        if (i < kXLoads) shared_x[buffer][swizzled(r, chunk)] = rx[d][i];
        shared_w[buffer][swizzled(r, chunk)] = rw[d][i];
      }
      __syncthreads();
      if (k + kDepth < steps) load(d, k + kDepth);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int c = ks * 4 + g;
        const u32x4 xf = shared_x[buffer][swizzled(wave_m + r16, c)];
#pragma unroll
        for (int ni = 0; ni < kColBlocks; ++ni) {
          const u32x4 wf = shared_w[buffer][swizzled(wave_n + ni * 16 + r16, c)];
          acc[ni] = mfma_16x16x32_bf16(wf, xf, acc[ni]);
        }
      }
    }
  }

  const int64_t m = m0 + wave_m + r16;
  if (m >= p.m) return;
#pragma unroll
  for (int ni = 0; ni < kColBlocks; ++ni) {
    const int64_t n = n0 + wave_n + ni * 16 + 4 * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (n + i >= p.n) continue;
      float v = p.alpha * acc[ni][i];
      if (p.bias != nullptr) v += p.bias[n + i];
      p.out[m * p.out_stride + n + i] = f32_to_bf16(v);
    }
  }
}

constexpr int kSkinnyWaves = 8;
constexpr int kSkinnyUnroll = 8;  // a hidden size of 2048 is one batch of loads per wavefront

__global__ void __launch_bounds__(kSkinnyWaves * kWave) skinny_router_kernel(RouterParams p) {
  __shared__ floatx4 partial[kSkinnyWaves][kWave];
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int lane = lane_id();
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int64_t m = static_cast<int64_t>(blockIdx.x) * 16 + r16;
  const int64_t n = static_cast<int64_t>(blockIdx.y) * 16 + r16;
  // Rows past the edge read row 0 and are never stored.
  const uint16_t *x_row = p.x + (m < p.m ? m : 0) * p.x_stride + g * 8;
  const uint16_t *w_row = p.w + (n < p.n ? n : 0) * p.w_stride + g * 8;

  floatx4 acc = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  const int64_t steps = p.k / 32;
  for (int64_t s = wave; s < steps; s += kSkinnyWaves * kSkinnyUnroll) {
    u32x4 xv[kSkinnyUnroll], wv[kSkinnyUnroll];
#pragma unroll
    for (int u = 0; u < kSkinnyUnroll; ++u) {
      const int64_t step = s + u * kSkinnyWaves;
      if (step < steps) {
        xv[u] = *reinterpret_cast<const u32x4 *>(x_row + step * 32);
        wv[u] = *reinterpret_cast<const u32x4 *>(w_row + step * 32);
      } else {
        xv[u] = u32x4{0, 0, 0, 0};
        wv[u] = u32x4{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int u = 0; u < kSkinnyUnroll; ++u) acc = mfma_16x16x32_bf16(wv[u], xv[u], acc);
  }
  partial[wave][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  floatx4 total = partial[0][lane];
#pragma unroll
  for (int w = 1; w < kSkinnyWaves; ++w) total += partial[w][lane];

  // Lane l holds token r16 and experts 4 g .. 4 g + 3 of the tile.
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 16 + r16;
  if (row >= p.m) return;
  const int64_t col = static_cast<int64_t>(blockIdx.y) * 16 + 4 * g;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (col + i >= p.n) continue;
    float v = p.alpha * total[i];
    if (p.bias != nullptr) v += p.bias[col + i];
    p.out[row * p.out_stride + col + i] = f32_to_bf16(v);
  }
}

}  // namespace

void launch_router(const RouterParams &p, hipStream_t stream) {
  // Fewer 64 x 64 tiles than a quarter of the CUs: the split-contraction kernel.
  const int64_t wide_tiles = ceil_div<int64_t>(p.m, kBM) * ceil_div<int64_t>(p.n, kBN);
  if (wide_tiles < 64 && p.k % 32 == 0) {
    const dim3 grid(static_cast<uint32_t>(ceil_div<int64_t>(p.m, 16)), static_cast<uint32_t>(ceil_div<int64_t>(p.n, 16)));
    hipLaunchKernelGGL(skinny_router_kernel, grid, dim3(kSkinnyWaves * kWave), 0, stream, p);
    return;
  }
#ifndef UNISERVE_ROUTER_BM
#define UNISERVE_ROUTER_BM 32
#endif
  constexpr int kTileM = UNISERVE_ROUTER_BM;
  const dim3 grid(static_cast<uint32_t>(ceil_div<int64_t>(p.m, kTileM)),
                  static_cast<uint32_t>(ceil_div<int64_t>(p.n, kBN)));
  hipLaunchKernelGGL(router_kernel<kTileM>, grid, dim3(kRouterThreads), 0, stream, p);
}

}  // namespace uniserve

extern "C" int32_t uniserve_gemm(UniserveGemmCall *call, void *stream) {
  using namespace uniserve;
  return guarded(call, [&]() -> int32_t {
    if (call->out == nullptr || call->input == nullptr || call->weight == nullptr)
      return UNISERVE_REFUSE(call, "gemm needs out, input and weight");
    if (call->bias != nullptr)
      return UNISERVE_REFUSE(call, "gemm: this module is compiled without a bias epilogue");
    if (call->m < 0 || call->n <= 0 || call->k <= 0)
      return UNISERVE_REFUSE(call, "gemm needs non-negative m and positive n and k");
    if (call->k % 64 != 0) return UNISERVE_REFUSE(call, "gemm needs a contraction of whole 64-element steps");
    if (call->input_row_stride < call->k || call->weight_row_stride < call->k || call->out_row_stride < call->n)
      return UNISERVE_REFUSE(call, "gemm's row strides are shorter than its rows");
    if (call->input_row_stride % 8 != 0 || call->weight_row_stride % 8 != 0)
      return UNISERVE_REFUSE(call, "gemm needs 16-byte aligned input and weight rows");
    if (call->m == 0) return 0;
    RouterParams p{static_cast<const uint16_t *>(call->input), static_cast<const uint16_t *>(call->weight),
                   static_cast<uint16_t *>(call->out), nullptr, call->m, call->n, call->k,
                   call->input_row_stride, call->weight_row_stride, call->out_row_stride, call->alpha};
    launch_router(p, static_cast<hipStream_t>(stream));
    return launched(call, "gemm");
  });
}

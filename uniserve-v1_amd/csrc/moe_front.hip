// SPDX-License-Identifier: Apache-2.0
//
// The MoE layer's front end at decode sizes in one launch: the router scores
// (crates/nn/src/modules/moe.rs:656-671), topk_softmax (crates/ops/src/moe/routing.rs) and
// moe_sort (crates/ops/src/moe/sort.rs) - what MoE::routed issues as three launches
// (moe.rs:770-775), each of which at 64 tokens is a few microseconds of latency and little work.
//
// Every workgroup computes one 16-token x 16-expert tile of scores, its contraction split over 16
// wavefronts (partial sums added in wavefront order, the bias added to the FP32 sum, one rounding
// into bf16), and stores it. Then two rounds of tickets - agent-scope atomic counters; the scores
// and ids that cross workgroups are stored and read at device scope (past the per-XCD L2 slices),
// and a workgroup counts only after its stores have completed, so a taker of a round's last ticket
// reads everything the round's other workgroups stored, with no cache write-back or invalidation:
//   * the last of a token block's workgroups routes that block's 16 tokens (the topk routine of
//     topk_route.hpp, one token per 32-lane half: ids and weights bit for bit those of the
//     topk_softmax kernel) - the routing is spread over the token blocks' CUs, since on one CU its
//     VALU work is the front end's longest step;
//   * the last of the token blocks sorts every route (the one-workgroup sort of sort_small.hpp:
//     every map entry the layer reads bit for bit the moe_sort entry's; the padding rows of the two
//     permuted maps, which the layer never reads, are not written).
// Each last taker resets its counter, so every launch leaves the counters zero.
#include "common.hpp"
#include "grouped_fp8.hpp"
#include "grouped_mx.hpp"
#include "moe_front.hpp"
#include "sort_small.hpp"
#include "topk_route.hpp"
#include "front_token.hpp"

namespace uniserve {
namespace {

constexpr int kThreads = sort::kSortThreads;  // the sort's workgroup: 16 wavefronts
constexpr int kWaves = kThreads / kWave;
constexpr int kUnroll = 4;                    // K steps of 32 whose loads a wavefront keeps in flight
constexpr int kTile = 16;

/// Takes a ticket of `counter` for one of `takers` workgroups; answers, to every thread, whether it
/// was the last (then the counter is reset).
///
/// Ordering. What crosses workgroups - the scores and the ids - is stored and read only with
/// relaxed agent-scope atomics (store_device / load_device). On gfx950 those are emitted with the
/// sc1 bit: a store is written through the XCD's L2 to the memory-side coherence point and counts
/// in vmcnt until that write is acknowledged there; a load bypasses the XCD's L2 and is served from
/// the coherence point. So no L2 write-back (release) or invalidation (acquire) is needed - those
/// exist for ordinary cached accesses, which this hand-off does not use. What remains is order:
///   * publisher: every thread waits vmcnt(0) (its device-scope stores acknowledged), then the
///     workgroup barrier, then thread 0's fetch_add - the ticket is taken only after every store of
///     the workgroup has reached the coherence point;
///   * taker: the ticket answer reaches the other threads through LDS behind a barrier, and their
///     device-scope loads are issued after it.
/// The language's memory model does not promise that order for relaxed atomics to different
/// addresses, so it is pinned for the compiler with a full signal fence on each side of the
/// ticket (no instruction emitted; no memory access moves across it), on top of the hardware
/// wait. Release/acquire at agent scope would give the same order with an L2 write-back and
/// invalidate per ticket; measured, the front end took 20.0 us that way against 17.8.
__device__ __forceinline__ bool last_ticket(uint32_t *counter, uint32_t takers, int32_t *flag) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this thread's device-scope stores acknowledged
  __syncthreads();
  if (threadIdx.x == 0) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const uint32_t taken = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = taken + 1 == takers;
    if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = last ? 1 : 0;
  }
  __syncthreads();
  const bool last = *flag != 0;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  return last;
}

__global__ void __launch_bounds__(kThreads) front_kernel(FrontParams p) {
  extern __shared__ __align__(16) int32_t front_lds[];
  __shared__ int32_t flag;
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int lane = lane_id();
  const int r16 = lane & 15;
  const int g = lane >> 4;

  // 1. One tile of scores. Lane l: token row l % 16 (operand B) and expert row l % 16 (operand A),
  // eight K elements at 8 (l / 16); rows past the edge read row 0 and are never stored.
  const int64_t m = static_cast<int64_t>(blockIdx.x) * kTile + r16;
  const int64_t n = static_cast<int64_t>(blockIdx.y) * kTile + r16;
  // Wave 0's lanes add the bias of experts 4 (l / 16) .. + 3 of the tile: loaded now, with the
  // operands, rather than after the reduction.
  float bias[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (wave == 0 && p.bias != nullptr) {
    const int64_t col = static_cast<int64_t>(blockIdx.y) * kTile + 4 * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) bias[i] = col + i < p.experts ? p.bias[col + i] : 0.0f;
  }
  const uint16_t *x_row = p.x + (m < p.tokens ? m : 0) * p.hidden + g * 8;
  const uint16_t *w_row = p.w + (n < p.experts ? n : 0) * p.hidden + g * 8;
  floatx4 acc = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  const int64_t steps = p.hidden / 32;
  for (int64_t s = wave; s < steps; s += kWaves * kUnroll) {
    u32x4 xv[kUnroll], wv[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t step = s + u * kWaves;
      if (step < steps) {
        xv[u] = *reinterpret_cast<const u32x4 *>(x_row + step * 32);
        wv[u] = *reinterpret_cast<const u32x4 *>(w_row + step * 32);
      } else {
        xv[u] = u32x4{0, 0, 0, 0};
        wv[u] = u32x4{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc = mfma_16x16x32_bf16(wv[u], xv[u], acc);
  }
  floatx4 *partial = reinterpret_cast<floatx4 *>(front_lds);
  partial[wave * kWave + lane] = acc;
  __syncthreads();
  if (wave == 0) {
    floatx4 total = partial[lane];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) total += partial[w * kWave + lane];
    // Lane l holds token l % 16 and experts 4 (l / 16) .. + 3 of the tile.
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kTile + r16;
    const int64_t col = static_cast<int64_t>(blockIdx.y) * kTile + 4 * g;
    if (row < p.tokens) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (col + i >= p.experts) continue;
        float v = total[i];
        if (p.bias != nullptr) v += bias[i];
        store_device(p.scores + row * p.experts + col + i, f32_to_bf16(v));
      }
    }
  }
  __syncthreads();

  // e4m3 and MXFP4 layers: the hidden rows' quantisation, off the routing's path - each workgroup's
  // share of its token block's 128-channel groups (group g to expert block g % expert blocks), or
  // 32-channel MXFP8 blocks, done once the workgroup has nothing else to do (the quantisers'
  // arithmetic: codes bit for bit their own).
  auto quantize_share = [&]() __attribute__((always_inline)) {
    if (p.hidden_codes == nullptr) return;
    if (p.hidden_mx_scales != nullptr) {
      // MXFP8: blocks of 32 channels, four lanes each (block b to expert block b % expert blocks).
      const int64_t blocks_per_row = p.hidden / 32;
      const int64_t block_blocks = kTile * blocks_per_row;
      const int64_t step = static_cast<int64_t>(kThreads / 4) * gridDim.y;
      const int sub = static_cast<int>(threadIdx.x & 3);
      for (int64_t b = blockIdx.y + static_cast<int64_t>(threadIdx.x / 4) * gridDim.y; b < block_blocks; b += step) {
        const int64_t row = static_cast<int64_t>(blockIdx.x) * kTile + b / blocks_per_row;
        if (row >= p.tokens) continue;
        const int64_t column = (b % blocks_per_row) * 32 + sub * 8;
        const u32x4 packed = *reinterpret_cast<const u32x4 *>(p.x + row * p.hidden + column);
        float v[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[2 * j] = __uint_as_float(packed[j] << 16);
          v[2 * j + 1] = __uint_as_float(packed[j] & 0xffff0000u);
        }
        const uint32_t scale = mxfp8_eight(v, p.hidden_codes + row * p.hidden + column);
        if (sub == 0) p.hidden_mx_scales[row * blocks_per_row + b % blocks_per_row] = static_cast<uint8_t>(scale);
      }
      return;
    }
    const int64_t groups_per_row = p.hidden / 128;
    const int64_t block_groups = kTile * groups_per_row;
    const int64_t step = static_cast<int64_t>(kThreads / 16) * gridDim.y;
    for (int64_t g = blockIdx.y + static_cast<int64_t>(threadIdx.x / 16) * gridDim.y; g < block_groups; g += step) {
      const int64_t row = static_cast<int64_t>(blockIdx.x) * kTile + g / groups_per_row;
      if (row >= p.tokens) continue;
      const int64_t column = (g % groups_per_row) * 128;
      quantize_bf16_group(p.x + row * p.hidden + column, p.hidden_codes + row * p.hidden + column,
                          p.hidden_scales + row * groups_per_row + g % groups_per_row, static_cast<int>(threadIdx.x & 15));
    }
  };

  // 2. The last of the token block's tiles routes its tokens, one per 32-lane half.
  if (!last_ticket(p.ticket + 1 + blockIdx.x, gridDim.y, &flag)) {
    quantize_share();
    return;
  }
  const int half = static_cast<int>(threadIdx.x) / topk::kHalf;
  if (half < kTile) {
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kTile + half;
    const bool active = row < p.tokens;
    topk::route_token<true>(p.scores, 1, p.experts, static_cast<int>(active ? row : 0), static_cast<int>(p.experts), p.top,
                      p.renormalize, nullptr, -1, p.ids, p.weights, p.map, p.live, p.load, active);
  }
  __syncthreads();
  if (!p.sort_routes) {
    // No sort: each route of the block is visible at its own expanded index, or not at all.
    const int64_t live = (p.live != nullptr ? static_cast<int64_t>(p.live[0]) : p.tokens) * p.top;
    const int64_t block_first = static_cast<int64_t>(blockIdx.x) * kTile * p.top;
    for (int64_t i = threadIdx.x; i < kTile * p.top; i += kThreads) {
      const int64_t route = block_first + i;
      if (route >= p.tokens * p.top) break;
      const int64_t local = static_cast<int64_t>(load_device(p.ids + route)) - p.sort.local_offset;
      const bool visible = route < live && local >= 0 && local < p.sort.local_experts;
      p.sort.expanded_to_permuted[route] = visible ? static_cast<int32_t>(route) : -1;
    }
    quantize_share();
    return;
  }

  // 3. The last of the token blocks sorts every route.
  if (!last_ticket(p.ticket, gridDim.x, &flag)) {
    quantize_share();
    return;
  }
  sort::small_sort<false, true>(p.sort, front_lds);
  quantize_share();
}

// ---- the front end without a sort: one workgroup per token ------------------------------------------
//
// Where the layer skips the sort (the expert-major products find their routes themselves), nothing
// crosses workgroups: each 16-wavefront workgroup takes one token through front_token::route_one
// (front_token.hpp). No tickets, no device-scope hand-offs.

/// kChunks: at most that many 512-channel chunks per row (4: hidden <= 2048; 8: hidden <= 4096);
/// kQuant: 0 none, 1 e4m3, 2 MXFP8.
template <int kChunks, int kQuant>
__global__ void __launch_bounds__(kThreads) local_front_kernel(FrontParams p) {
  __shared__ uint16_t scores[front_token::kMaxExperts];
  front_token::route_one<kWaves, kChunks, kQuant>(p, blockIdx.x, scores);
}

// ---- the front end for a few tokens without a sort: experts split over workgroups -------------------
//
// A one-token step is latency-bound: the tile-split kernel above gives the router's 16-expert
// tiles to eight workgroups (128 KB each at 4096 channels) and a workgroup per token would stream
// the whole matrix alone. Here each wavefront owns one expert (its row in registers, whole 1 KB
// lines: lane l holds channels 512 c + 8 l .. + 7 of chunk c, as in front_token.hpp) and takes the
// tokens one after another: the dot product in FP32, an xor-butterfly reduction, the bias, one
// rounding into bf16, a device-scope store. Each workgroup then quantises its share of the hidden
// rows (e4m3 / MXFP8), and the last workgroup to take the ticket routes every token, one per
// 32-lane half, writing the ids, weights and each route's expanded_to_permuted entry from the id
// the routine answers.

constexpr int kSplitThreads = 256;
constexpr int kSplitWaves = kSplitThreads / kWave;  // experts per workgroup
constexpr int64_t kSplitMaxTokens = kSplitThreads / topk::kHalf;

template <int kChunks, int kQuant>
__global__ void __launch_bounds__(kSplitThreads) split_front_kernel(FrontParams p) {
  __shared__ int32_t flag;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  const int lane = lane_id();
  const int chunks = static_cast<int>(p.hidden / front_token::kChunk);
  const int64_t expert = static_cast<int64_t>(blockIdx.x) * kSplitWaves + wave;
  const bool named = expert < p.experts;

  u32x4 w[kChunks];
  const uint16_t *row = p.w + (named ? expert : 0) * p.hidden + 8 * lane;
#pragma unroll
  for (int c = 0; c < kChunks; ++c)
    if (c < chunks) w[c] = *reinterpret_cast<const u32x4 *>(row + c * front_token::kChunk);
  const float bias = named && p.bias != nullptr ? p.bias[expert] : 0.0f;
  for (int64_t t = 0; t < p.tokens; ++t) {
    const uint16_t *x = p.x + t * p.hidden + 8 * lane;
    float sum = 0.0f;
#pragma unroll
    for (int c = 0; c < kChunks; ++c)
      if (c < chunks) sum = front_token::dot8_bf16(w[c], *reinterpret_cast<const u32x4 *>(x + c * front_token::kChunk), sum);
#pragma unroll
    for (int offset = 32; offset >= 1; offset /= 2) sum += __shfl_xor(sum, offset);
    if (lane == 0 && named) {
      if (p.bias != nullptr) sum += bias;
      store_device(p.scores + t * p.experts + expert, f32_to_bf16(sum));
    }
  }

  // This workgroup's share of the hidden rows' quantisation (the quantisers' routines).
  if constexpr (kQuant == 1) {
    const int64_t per_row = p.hidden / 128;
    const int64_t groups = p.tokens * per_row;
    const int64_t stride = static_cast<int64_t>(kSplitThreads / 16) * gridDim.x;
    for (int64_t g = blockIdx.x + static_cast<int64_t>(threadIdx.x / 16) * gridDim.x; g < groups; g += stride) {
      const int64_t t = g / per_row, column = (g % per_row) * 128;
      quantize_bf16_group(p.x + t * p.hidden + column, p.hidden_codes + t * p.hidden + column,
                          p.hidden_scales + t * per_row + g % per_row, static_cast<int>(threadIdx.x & 15));
    }
  } else if constexpr (kQuant == 2) {
    const int64_t per_row = p.hidden / 32;
    const int64_t blocks = p.tokens * per_row;
    const int64_t stride = static_cast<int64_t>(kSplitThreads / 4) * gridDim.x;
    const int sub = static_cast<int>(threadIdx.x & 3);
    for (int64_t b = blockIdx.x + static_cast<int64_t>(threadIdx.x / 4) * gridDim.x; b < blocks; b += stride) {
      const int64_t t = b / per_row, column = (b % per_row) * 32 + sub * 8;
      const u32x4 packed = *reinterpret_cast<const u32x4 *>(p.x + t * p.hidden + column);
      float v[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[2 * j] = __uint_as_float(packed[j] << 16);
        v[2 * j + 1] = __uint_as_float(packed[j] & 0xffff0000u);
      }
      const uint32_t scale = mxfp8_eight(v, p.hidden_codes + t * p.hidden + column);
      if (sub == 0) p.hidden_mx_scales[t * per_row + b % per_row] = static_cast<uint8_t>(scale);
    }
  }

  // The last workgroup routes every token, one per 32-lane half.
  if (!last_ticket(p.ticket + 1, gridDim.x, &flag)) return;
  const int half = static_cast<int>(threadIdx.x) / topk::kHalf;
  if (half >= p.tokens) return;
  const int32_t id = topk::route<front_token::kMaxExperts / topk::kHalf, true>(
      p.scores, 1, p.experts, half, static_cast<int>(p.experts), p.top, p.renormalize, nullptr, -1, p.ids,
      p.weights, p.map, p.live, p.load, true, half);
  const int k = static_cast<int>(threadIdx.x) & (topk::kHalf - 1);
  if (k < p.top) {
    const int64_t route = static_cast<int64_t>(half) * p.top + k;
    const int64_t live = (p.live != nullptr ? static_cast<int64_t>(p.live[0]) : p.tokens) * p.top;
    const int64_t local = static_cast<int64_t>(id) - p.sort.local_offset;
    const bool visible = route < live && local >= 0 && local < p.sort.local_experts;
    p.sort.expanded_to_permuted[route] = visible ? static_cast<int32_t>(route) : -1;
  }
}

}  // namespace

bool split_front_fits(int64_t tokens, int64_t experts, int64_t hidden, int64_t top) {
  return tokens >= 1 && tokens <= kSplitMaxTokens && experts >= 1 && experts <= front_token::kMaxExperts &&
         hidden % front_token::kChunk == 0 && hidden / front_token::kChunk <= 8 && top >= 1 &&
         top <= topk::kHalf && top <= experts;
}

void launch_split_front(const FrontParams &p, hipStream_t stream) {
  const dim3 grid(static_cast<uint32_t>(ceil_div<int64_t>(p.experts, kSplitWaves)));
  const int quant = p.hidden_codes == nullptr ? 0 : (p.hidden_mx_scales != nullptr ? 2 : 1);
  const bool narrow = p.hidden <= 4 * front_token::kChunk;
  auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, dim3(kSplitThreads), 0, stream, p); };
  if (narrow && quant == 0) go(split_front_kernel<4, 0>);
  else if (narrow && quant == 1) go(split_front_kernel<4, 1>);
  else if (narrow) go(split_front_kernel<4, 2>);
  else if (quant == 0) go(split_front_kernel<8, 0>);
  else if (quant == 1) go(split_front_kernel<8, 1>);
  else go(split_front_kernel<8, 2>);
}

constexpr int64_t kLocalMinTokens = 32;

bool local_front_fits(int64_t tokens, int64_t experts, int64_t hidden, int64_t top) {
  // Each workgroup streams the whole router matrix: for a few tokens the tile-split front end,
  // whose workgroups read a share each, is the faster (235B, one token: 16 us against 18).
  return tokens >= kLocalMinTokens && tokens <= 0x7fffffffLL && experts >= 1 &&
         experts <= front_token::kMaxExperts && hidden % front_token::kChunk == 0 &&
         hidden / front_token::kChunk <= 8 && top >= 1 && top <= topk::kHalf && top <= experts;
}

void launch_local_front(const FrontParams &p, hipStream_t stream) {
  const dim3 grid(static_cast<uint32_t>(p.tokens));
  const int quant = p.hidden_codes == nullptr ? 0 : (p.hidden_mx_scales != nullptr ? 2 : 1);
  const bool narrow = p.hidden <= 4 * front_token::kChunk;
  auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, dim3(kThreads), 0, stream, p); };
  if (narrow && quant == 0) go(local_front_kernel<4, 0>);
  else if (narrow && quant == 1) go(local_front_kernel<4, 1>);
  else if (narrow) go(local_front_kernel<4, 2>);
  else if (quant == 0) go(local_front_kernel<8, 0>);
  else if (quant == 1) go(local_front_kernel<8, 1>);
  else go(local_front_kernel<8, 2>);
}

bool front_fits(int64_t tokens, int64_t experts, int64_t hidden, int64_t top, int64_t local_experts) {
  const int64_t wide_tiles = ceil_div<int64_t>(tokens, 64) * ceil_div<int64_t>(experts, 64);
  return tokens > 0 && ceil_div<int64_t>(tokens, kTile) <= kFrontTokenBlocks && wide_tiles < 64 &&
         hidden % 32 == 0 && experts <= 1024 && top >= 1 && top <= 32 && top <= experts &&
         tokens * top <= sort::kChunk && local_experts >= 1 && local_experts <= sort::kSmallMaxExperts;
}

void launch_front(const FrontParams &p, hipStream_t stream) {
  const int64_t router_bytes = static_cast<int64_t>(kThreads) * sizeof(floatx4);
  const int64_t sort_bytes = sort::small_sort_lds_words(p.sort.local_experts) * static_cast<int64_t>(sizeof(int32_t));
  const size_t lds = static_cast<size_t>(router_bytes > sort_bytes ? router_bytes : sort_bytes);
  const dim3 grid(static_cast<uint32_t>(ceil_div<int64_t>(p.tokens, kTile)),
                  static_cast<uint32_t>(ceil_div<int64_t>(p.experts, kTile)));
  hipLaunchKernelGGL(front_kernel, grid, dim3(kThreads), lds, stream, p);
}

}  // namespace uniserve

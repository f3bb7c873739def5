// SPDX-License-Identifier: Apache-2.0
//
// The MoE layer's front end at prefill sizes in one launch: the router scores
// (crates/nn/src/modules/moe.rs:656-671), topk_softmax (crates/ops/src/moe/routing.rs) and, for
// e4m3 and MXFP4 stacks, the quantisation of the hidden rows - what MoE::routed issues as separate
// launches (moe.rs:770-775), each of which re-reads the hidden rows or the scores.
//
// A workgroup of sixteen wavefronts owns 32 tokens and every expert (at most 128): it streams the
// tokens' hidden rows and the whole router matrix through LDS in stages of 128 channels (a
// four-slot ring filled by global_load_lds, 40 KB a stage, three stages ahead), multiplies them
// with v_mfma_f32_16x16x32_bf16 (wavefront w: expert block w % 8, token block w / 8), and, while a
// stage's hidden rows are in LDS, quantises them (one 128-channel e4m3 group, or four 32-channel
// MXFP8 blocks, per row and stage) with the stand-alone quantisers' arithmetic. The scores get the
// bias in FP32 and one rounding into bf16, go to the layer's score tensor and to LDS, and the
// workgroup routes its 32 tokens from there, one per 32-lane half, with the topk_softmax routine
// (topk_route.hpp): ids and weights bit for bit those of the topk_softmax kernel over the same
// scores.
//
// The router matrix is read once per 32 tokens (from L2); at 8192 tokens that is one workgroup per
// CU, each streaming 512 KB of router rows and 128 KB of hidden rows.
#include "common.hpp"
#include "grouped_fp8.hpp"
#include "grouped_mx.hpp"
#include "grouped_prefill.hpp"
#include "moe_front.hpp"
#include "topk_route.hpp"

namespace uniserve {
namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / kWave;
constexpr int kTokens = 32;             // tokens per workgroup: one per 32-lane half
static_assert(kTokens == kFrontChunkTokens, "the sort's chunks are the workgroups' tokens");
constexpr int kExperts = 128;           // router rows the LDS holds
constexpr int kRowBytes = 256;          // 128 bf16 channels per row and stage
constexpr int kSlots = 4;               // stages in flight: three ahead of the one being read
constexpr int kWeightLoads = kExperts * kRowBytes / (kWave * 16) / kWaves;  // 2 per wave
constexpr int kLoads = kWeightLoads + 1;                                    // and one of hidden rows
constexpr int kQuantWaves = kTokens * 16 / kWave;                           // 8: 16 lanes per row

struct Slot {
  u32x4 w[kExperts * 16];  // 16 chunks of 16 bytes per row: chunk c of row r at r * 16 + (c ^ (r % 16))
  u32x4 x[kTokens * 16];
};
static_assert(sizeof(Slot) * kSlots <= 160 * 1024, "the ring fits the CU's LDS");

__device__ __forceinline__ int chunk_slot(int row, int chunk) { return row * 16 + (chunk ^ (row & 15)); }

/// s_waitcnt vmcnt(n) for the few counts the loop needs (n even, 6 <= n <= 12).
__device__ __forceinline__ void wait_vm(int n) {
  if (n <= 6) prefill::wait_loads_but<6>();
  else if (n == 8) prefill::wait_loads_but<8>();
  else if (n == 10) prefill::wait_loads_but<10>();
  else prefill::wait_loads_but<12>();
}

/// kQuant: 0 none, 1 e4m3 (codes and an FP32 scale per 128 channels), 2 MXFP8 (codes and an E8M0
/// byte per 32 channels).
template <int kQuant>
__global__ void __launch_bounds__(kThreads) prefill_front_kernel(PrefillFrontParams p) {
  using prefill::dma16;
  using prefill::lds_address;
  __shared__ __align__(16) char lds[sizeof(Slot) * kSlots];
  Slot *ring = reinterpret_cast<Slot *>(lds);

  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  const int lane = lane_id();
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int64_t token0 = static_cast<int64_t>(blockIdx.x) * kTokens;
  const int64_t row_bytes = p.hidden * 2;
  const int stages = static_cast<int>(p.hidden / 128);
  const int experts = static_cast<int>(p.experts);
  // Each workgroup walks the channels from its own starting stage, so that the workgroups running
  // together read different router lines.
  const int rotation = static_cast<int>(blockIdx.x % static_cast<uint32_t>(stages));

  // ---- DMA sources: one instruction fills 4 rows (64 lanes x 16 bytes); lane l lands in
  // physical chunk l % 16 of row 4 i + l / 16 and brings logical chunk (l % 16) ^ (row % 16).
  // Wave w brings router rows 8 w .. 8 w + 7 and hidden rows 4 (w % 8) .. + 3 (waves w and w + 8
  // bring the same hidden rows, the same bytes to the same place). Router rows past the experts
  // and hidden rows past the tokens repeat the last one. ----
  uint32_t w_off[kWeightLoads];
#pragma unroll
  for (int i = 0; i < kWeightLoads; ++i) {
    const int row = (wave * kWeightLoads + i) * 4 + lane / 16;
    const int source = row < experts ? row : experts - 1;
    w_off[i] = static_cast<uint32_t>(source * row_bytes + (((lane & 15) ^ (row & 15)) * 16));
  }
  const int x_row = (wave & 7) * 4 + lane / 16;
  const int64_t x_source = token0 + x_row < p.tokens ? token0 + x_row : p.tokens - 1;
  const uint32_t x_off = static_cast<uint32_t>((x_source - token0) * row_bytes + (((lane & 15) ^ (x_row & 15)) * 16));
  const uint8_t *w_base = reinterpret_cast<const uint8_t *>(p.w);
  const uint8_t *x_base = reinterpret_cast<const uint8_t *>(p.x) + token0 * row_bytes;

  // Stage k (k-th of the walk, channels 128 kk ..) into slot k % kSlots; stages past the last
  // load the last again (into a slot no stage reads), so every stage issues kLoads loads.
  auto channel_stage = [&](int k) {
    const int kk = k + rotation;
    return kk >= stages ? kk - stages : kk;
  };
  auto issue = [&](int k) {
    const int slot = k % kSlots;
    const int kk = channel_stage(k < stages ? k : stages - 1);
#pragma unroll
    for (int i = 0; i < kWeightLoads; ++i)
      dma16(w_base + static_cast<int64_t>(kk) * kRowBytes, w_off[i],
            __builtin_amdgcn_readfirstlane(lds_address(ring[slot].w + (wave * kWeightLoads + i) * kWave)));
    dma16(x_base + static_cast<int64_t>(kk) * kRowBytes, x_off,
          __builtin_amdgcn_readfirstlane(lds_address(ring[slot].x + (wave & 7) * kWave)));
  };

  // ---- the hidden rows' quantisation of one stage, waves 0..7 (16 lanes per row): exactly two
  // stores per wave, every row included (rows past the tokens hold the last token's row and write
  // its codes and scales again, the same bytes), so the loop's waits can count them ----
  constexpr int kStores = kQuant != 0 ? 2 : 0;
  const int stores = wave < kQuantWaves ? kStores : 0;
  auto quantize_stage = [&](int k) {
    if constexpr (kQuant == 0) return;
    if (wave >= kQuantWaves) return;
    const int kk = channel_stage(k);
    const u32x4 *xs = ring[k % kSlots].x;
    const int t = static_cast<int>(threadIdx.x);
    const int row = t / 16;
    const int sub = t & 15;  // channels 8 sub .. 8 sub + 7 of the stage
    const u32x4 packed = xs[chunk_slot(row, sub)];
    float v[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = __uint_as_float(packed[j] << 16);
      v[2 * j + 1] = __uint_as_float(packed[j] & 0xffff0000u);
    }
    const int64_t token = token0 + row < p.tokens ? token0 + row : p.tokens - 1;
    uint8_t *codes = p.codes + token * p.hidden + static_cast<int64_t>(kk) * 128 + sub * 8;
    if constexpr (kQuant == 2) {
      const uint32_t scale = mxfp8_eight(v, codes);  // four lanes per 32-channel block
      if ((sub & 3) == 0) p.mx_scales[token * (p.hidden / 32) + kk * 4 + sub / 4] = static_cast<uint8_t>(scale);
    } else {
      float amax = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[j]));
      amax = row16_max(amax);
      const float scale = amax > 0.0f ? amax / 448.0f : 1.0f;
      *reinterpret_cast<uint2 *>(codes) = e4m3_eight_of_bf16(v, scale);
      if (sub == 0) p.scales[token * (p.hidden / 128) + kk] = scale;
    }
  };

  // ---- the scores: wavefront w takes expert block w % 8 (rows 16 (w % 8) ..) and token block
  // w / 8; lane (r16, g) of an MFMA reads router row 16 (w % 8) + r16 and hidden row
  // 16 (w / 8) + r16 at channels 8 g .. 8 g + 7 of each 32-channel step ----
  const int eb = wave & 7;
  const int tb = wave >> 3;
  const bool has_block = eb * 16 < experts;
  floatx4 acc = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  issue(0);
  issue(1);
  issue(2);
  for (int k = 0; k < stages; ++k) {
    // Issued since stage k's loads: stages k + 1 and k + 2 (kLoads loads each) and the stores of
    // the last min(k, 3) stages.
    wait_vm(2 * kLoads + stores * (k < 3 ? k : 3));
    __syncthreads();
    issue(k + 3);
    // No memory access of the stage moves above its loads: the waits count this stage's stores
    // as issued after them.
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const int slot = k % kSlots;
    if (has_block) {
      const int w_row = eb * 16 + r16;
      const int x_row_mma = tb * 16 + r16;
#pragma unroll
      for (int step = 0; step < 4; ++step) {
        const int chunk = step * 4 + g;
        const u32x4 a = ring[slot].w[chunk_slot(w_row, chunk)];
        const u32x4 b = ring[slot].x[chunk_slot(x_row_mma, chunk)];
        acc = mfma_16x16x32_bf16(a, b, acc);
      }
    }
    quantize_stage(k);
  }
  prefill::wait_all_loads();
  __syncthreads();  // the ring is free: the scores tile goes over it, the chunk's counts after it
  int32_t *held = reinterpret_cast<int32_t *>(lds + kTokens * kExperts * 2);
  if (p.chunk_counts != nullptr && static_cast<int>(threadIdx.x) < p.local_experts) held[threadIdx.x] = 0;

  // Lane (r16, g) holds token 16 tb + r16 and experts 16 eb + 4 g .. + 3.
  uint16_t *scores = reinterpret_cast<uint16_t *>(lds);
  if (has_block) {
    const int local = tb * 16 + r16;
    const int64_t token = token0 + local;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int expert = eb * 16 + 4 * g + e;
      if (expert >= experts) continue;
      float value = acc[e];
      if (p.bias != nullptr) value += p.bias[expert];
      const uint16_t bits = f32_to_bf16(value);
      scores[local * experts + expert] = bits;
      if (token < p.tokens) p.scores[token * experts + expert] = bits;
    }
  }
  __syncthreads();

  // ---- routing: one token per 32-lane half, from the LDS copy of the scores ----
  const int local = static_cast<int>(threadIdx.x) / topk::kHalf;
  const int64_t token = token0 + local;
  const bool active = token < p.tokens;
  // Four slots per lane whatever the expert count (at most 128): the slots past it hold -inf and
  // add exact zeros, so the picks and weights are those of the smallest slot count.
  const int32_t id = topk::route<kExperts / topk::kHalf, false>(
      scores, 1, experts, static_cast<int>(active ? token : 0), experts, p.top, p.renormalize, nullptr, -1, p.ids,
      p.weights, p.map, p.live, p.load, active, local);

  // The sort's count of this chunk of tokens: lane k < top of an active token holds route
  // token * top + k's id (the one stored).
  if (p.chunk_counts != nullptr) {
    const int k = static_cast<int>(threadIdx.x) & (topk::kHalf - 1);
    const int64_t live = (p.live != nullptr ? static_cast<int64_t>(p.live[0]) : p.tokens) * p.top;
    const int64_t slot = static_cast<int64_t>(id) - p.local_offset;
    if (active && k < p.top && token * p.top + k < live && slot >= 0 && slot < p.local_experts)
      atomicAdd(held + slot, 1);
    __syncthreads();
    if (static_cast<int>(threadIdx.x) < p.local_experts)
      p.chunk_counts[static_cast<int64_t>(blockIdx.x) * p.local_experts + threadIdx.x] = held[threadIdx.x];
  }
}

/// One thread per (permuted row, word), rows fastest: the stores of a word run along the rows.
/// Only the rows the sort wrote are read (below its total_padded_tokens): the rest of
/// permuted_to_expanded holds whatever the buffer held before.
__global__ void __launch_bounds__(256) scatter_route_words_kernel(const uint32_t *from, const int32_t *p2e,
                                                                 const int32_t *padded, uint32_t *to, int64_t rows,
                                                                 int64_t top, int64_t words) {
  const int64_t index = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (index >= rows * words) return;
  const int64_t word = index / rows;
  const int64_t row = index - word * rows;
  if (row >= padded[0]) return;
  const int32_t route = p2e[row];
  if (route < 0) return;
  to[word * rows + row] = from[(route / top) * words + word];
}

}  // namespace

void launch_scatter_route_words(const uint32_t *from, const int32_t *permuted_to_expanded, const int32_t *padded,
                                uint32_t *to, int64_t rows, int64_t top, int64_t words, hipStream_t stream) {
  const int64_t threads = rows * words;
  if (threads == 0) return;
  hipLaunchKernelGGL(scatter_route_words_kernel, dim3(static_cast<uint32_t>(ceil_div<int64_t>(threads, 256))), dim3(256), 0,
                     stream, from, permuted_to_expanded, padded, to, rows, top, words);
}

bool prefill_front_fits(int64_t tokens, int64_t experts, int64_t hidden, int64_t top) {
  return tokens > 0 && experts >= 1 && experts <= kExperts && hidden % 128 == 0 && hidden >= 128 &&
         hidden * 2 * kExperts <= (int64_t{1} << 31) && top >= 1 && top <= 32 && top <= experts &&
         ceil_div<int64_t>(tokens, kTokens) <= 0x7fffffffLL;
}

void launch_prefill_front(const PrefillFrontParams &p, hipStream_t stream) {
  const dim3 grid(static_cast<uint32_t>(ceil_div<int64_t>(p.tokens, kTokens)));
  if (p.codes == nullptr) hipLaunchKernelGGL((prefill_front_kernel<0>), grid, dim3(kThreads), 0, stream, p);
  else if (p.mx_scales != nullptr) hipLaunchKernelGGL((prefill_front_kernel<2>), grid, dim3(kThreads), 0, stream, p);
  else hipLaunchKernelGGL((prefill_front_kernel<1>), grid, dim3(kThreads), 0, stream, p);
}

}  // namespace uniserve

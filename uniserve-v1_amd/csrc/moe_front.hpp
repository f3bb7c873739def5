// SPDX-License-Identifier: Apache-2.0
//
// The layer's fused front end at decode sizes: router scores, topk_softmax and moe_sort in one
// launch (moe_front.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "sort_small.hpp"
#include "uniserve_moe_unpermute.h"

namespace uniserve {

/// Token blocks (16 tokens each) the front end's counters cover: one counter per block and one for
/// the sort, kFrontTicketBytes in all.
constexpr int64_t kFrontTokenBlocks = 255;
constexpr int64_t kFrontTicketBytes = (1 + kFrontTokenBlocks) * 4;

struct FrontParams {
  const uint16_t *x;        ///< [tokens, hidden] bf16
  const uint16_t *w;        ///< [experts, hidden] bf16 router
  const float *bias;        ///< [experts] or null
  uint16_t *scores;         ///< [tokens, experts] bf16
  int64_t tokens, experts, hidden;
  int32_t top, renormalize;
  const int32_t *map;       ///< [experts] or null
  const int32_t *live;      ///< [1] or null
  unsigned long long *load; ///< [experts] or null
  int32_t *ids;             ///< [tokens, top]
  float *weights;           ///< [tokens, top]
  uint32_t *ticket;         ///< [1 + kFrontTokenBlocks] counters, zero before the launch and after it
  sort::SortParams sort;    ///< the sort over `ids` (its ids pointer is `ids`)
  /// 0: no sort - the routing workgroups write sort.expanded_to_permuted as each route's own
  /// expanded index where it is live and in the window, -1 elsewhere (for products that find their
  /// routes themselves and keep rows at expanded positions), and nothing else of the sort's.
  int32_t sort_routes;
  /// Or null: the hidden rows as e4m3 codes [tokens, hidden] with a scale per 128 channels
  /// [tokens, hidden / 128] - the activation quantiser's output, made by this launch.
  uint8_t *hidden_codes;
  float *hidden_scales;
  /// With hidden_codes and instead of hidden_scales: MXFP8 blocks of 32 channels, their E8M0
  /// bytes [tokens, hidden / 32] - the MXFP8 quantiser's output.
  uint8_t *hidden_mx_scales;
};

/// Whether one launch serves these extents: the router's split-contraction tiles, a router of at
/// most 1024 experts picking at most 32, and a sort one workgroup does (<= 4096 routes over
/// <= 512 local experts).
bool front_fits(int64_t tokens, int64_t experts, int64_t hidden, int64_t top, int64_t local_experts);

void launch_front(const FrontParams &p, hipStream_t stream);

/// The same front end where the layer skips the sort (sort_routes 0), one workgroup per token and
/// no hand-off between workgroups: at least 32 tokens, at most 128 experts, the hidden size in
/// whole 512-channel chunks up to 4096.
bool local_front_fits(int64_t tokens, int64_t experts, int64_t hidden, int64_t top);
void launch_local_front(const FrontParams &p, hipStream_t stream);

/// The same for at most 8 tokens: one expert per wavefront across ceil(experts / 4) workgroups,
/// the last of which (counter word 1 of `ticket`) routes every token. At most 128 experts, the
/// hidden size in whole 512-channel chunks up to 4096.
bool split_front_fits(int64_t tokens, int64_t experts, int64_t hidden, int64_t top);
void launch_split_front(const FrontParams &p, hipStream_t stream);

/// The front end at prefill sizes (front_prefill.hip): router scores, topk and (with `codes`) the
/// hidden rows' quantisation in one launch, one workgroup per 32 tokens.
struct PrefillFrontParams {
  const uint16_t *x;        ///< [tokens, hidden] bf16
  const uint16_t *w;        ///< [experts, hidden] bf16 router
  const float *bias;        ///< [experts] or null
  uint16_t *scores;         ///< [tokens, experts] bf16
  int64_t tokens, experts, hidden;
  int32_t top, renormalize;
  const int32_t *map;       ///< [experts] or null
  const int32_t *live;      ///< [1] or null
  unsigned long long *load; ///< [experts] or null
  int32_t *ids;             ///< [tokens, top]
  float *weights;           ///< [tokens, top]
  /// Or null: the hidden rows as e4m3 codes [tokens, hidden] with FP32 scales [tokens, hidden / 128]
  /// (`scales`), or as MXFP8 codes with E8M0 bytes [tokens, hidden / 32] (`mx_scales`).
  uint8_t *codes;
  float *scales;
  uint8_t *mx_scales;
  /// Or null: each workgroup's held routes per local expert ([workgroups, local_experts]; a route
  /// is held when it is live and its id lies in [local_offset, local_offset + local_experts)) -
  /// the sort's count of the workgroup's 32 tokens (kFrontChunkTokens).
  int32_t *chunk_counts;
  int32_t local_offset, local_experts;
};

/// Whether one launch serves these extents: at most 128 experts picking at most 32, whole
/// 128-channel stages.
bool prefill_front_fits(int64_t tokens, int64_t experts, int64_t hidden, int64_t top);

void launch_prefill_front(const PrefillFrontParams &p, hipStream_t stream);

/// Each route's copy of its token's `words` 4-byte scale words: token-major `from` ([tokens,
/// words]) to route-major `to` ([words, rows] by permuted row), for the rows below the sort's
/// total_padded_tokens (`padded`, on the device) whose permuted_to_expanded names a route; padding
/// rows and rows past them are left alone.
void launch_scatter_route_words(const uint32_t *from, const int32_t *permuted_to_expanded, const int32_t *padded,
                                uint32_t *to, int64_t rows, int64_t top, int64_t words, hipStream_t stream);

/// Counter words a launch over `tokens` tokens uses: the sort's and one per token block.
inline int32_t front_ticket_words(int64_t tokens) { return static_cast<int32_t>(1 + (tokens + 15) / 16); }

/// uniserve_moe_unpermute that also checks the front end's `ticket_words` counters at `ticket`
/// (moe_unpermute.hip): nonzero words - counters that were not zero before the front end ran -
/// turn the output into NaN and are cleared.
int32_t moe_unpermute_checked(const uniserve_unpermute_call *call, uint32_t *ticket, int32_t ticket_words,
                              void *stream);

}  // namespace uniserve

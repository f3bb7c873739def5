/* SPDX-License-Identifier: Apache-2.0
 *
 * CPU oracle of the fused-MoE hot path. TEST INFRASTRUCTURE ONLY: the parity tests, the smoke
 * check and the bench's CPU-baseline leg link this library as the checker. Nothing in the product
 * library calls it, and the product fails loudly rather than falling back to it.
 *
 * Every function restates the reference's algorithm (file:line cited at each definition in
 * moe_oracle.c) in plain C on host memory. Elements: bf16 and e4m3 are passed as their raw bits
 * (uint16_t / uint8_t); maps are int32 with the device sentinels (-1 absent / padding, -2 not
 * live).
 */
#ifndef UNISERVE_MOE_ORACLE_H
#define UNISERVE_MOE_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- element codecs ------------------------------------------------------------------------ */
uint16_t oracle_bf16_from_f32(float value);
float oracle_f32_from_bf16(uint16_t bits);
uint16_t oracle_f16_from_f32(float value);
float oracle_f32_from_f16(uint16_t bits);
uint8_t oracle_e4m3_from_f32(float value);
float oracle_f32_from_e4m3(uint8_t code);
float oracle_expf(float x);
void oracle_bf16_encode(const float *in, uint16_t *out, int64_t count);
void oracle_bf16_decode(const uint16_t *in, float *out, int64_t count);

/* ---- inputs ---------------------------------------------------------------------------------- */
void oracle_sequence(int64_t count, uint32_t seed, float *out);
void oracle_normal(int64_t count, uint64_t seed, float mean, float stddev, float *out);
void oracle_normal_bf16(int64_t count, uint64_t seed, float stddev, uint16_t *out);

/* ---- the operators ----------------------------------------------------------------------------- */
int64_t oracle_max_tiles(int64_t tokens, int64_t top, int64_t local_experts, int64_t tile);

void oracle_topk_softmax(const void *scores, int32_t score_kind, int64_t row_stride, int32_t rows,
                         int32_t experts, int32_t top, int32_t renormalize, const void *scale,
                         int32_t scale_kind, int32_t *ids, float *weights, const int32_t *map,
                         const int32_t *live, int64_t *load);

void oracle_moe_sort(const int32_t *ids, int64_t tokens, int64_t top, int64_t local_experts,
                     int64_t local_offset, int64_t tile, const int32_t *live_tokens,
                     int32_t *tile_to_expert, int32_t *tile_to_limit,
                     int32_t *expanded_to_permuted, int32_t *permuted_to_expanded,
                     int32_t *permuted_to_token, int32_t *total_padded_tokens,
                     int32_t *num_non_exiting_tiles);

void oracle_router_gemm(const uint16_t *x, const uint16_t *weight, int64_t m, int64_t n, int64_t k,
                        uint16_t *out);
/* kind / out_kind: 0 f32, 1 bf16 bits; bias [n] f32 or NULL, added to the FP32 sum before rounding. */
void oracle_router_gemm_ex(const void *x, const void *weight, int32_t kind, const float *bias,
                           int64_t m, int64_t n, int64_t k, int32_t out_kind, void *out);
/* FC1's gate: activation 0 silu, 1 gelu_tanh. */
float oracle_gate_activation(float g, int32_t activation);
void oracle_gather_gemm_ex(const void *hidden, const void *weights, int32_t kind, int64_t tokens,
                           int64_t hidden_size, int64_t intermediate, int64_t top, int64_t tile,
                           const int32_t *tile_to_expert, const int32_t *tile_to_limit,
                           const int32_t *permuted_to_expanded, int32_t num_tiles, int32_t activation,
                           float *out);
void oracle_route_gemm_ex(const void *rows, const void *weights, int32_t kind, int64_t hidden_size,
                          int64_t intermediate, int64_t tile, const int32_t *tile_to_expert,
                          const int32_t *tile_to_limit, int32_t num_tiles, float *out);
void oracle_moe_unpermute_ex(const void *routes, int32_t kind, const int32_t *expanded_to_permuted,
                             const float *scales, int64_t tokens, int64_t top, int64_t hidden,
                             int64_t routes_rows, int32_t layout, float *out);

void oracle_gather_gemm(const uint16_t *hidden, const uint16_t *weights, int64_t tokens,
                        int64_t hidden_size, int64_t intermediate, int64_t top, int64_t tile,
                        const int32_t *tile_to_expert, const int32_t *tile_to_limit,
                        const int32_t *permuted_to_expanded, int32_t num_tiles, float *out);

void oracle_route_gemm(const uint16_t *rows, const uint16_t *weights, int64_t hidden_size,
                       int64_t intermediate, int64_t tile, const int32_t *tile_to_expert,
                       const int32_t *tile_to_limit, int32_t num_tiles, float *out);

void oracle_moe_unpermute(const uint16_t *routes, const int32_t *expanded_to_permuted,
                          const float *scales, int64_t tokens, int64_t top, int64_t hidden,
                          int64_t routes_rows, int32_t layout, float *out);

/* ---- the shared expert's join ---------------------------------------------------------------- */
/* kind: 0 f32, 1 bf16, 2 f16 (raw bits); target updated in place. */
void oracle_sigmoid_gated_add(void *target, const void *update, const void *gate, int64_t rows,
                              int64_t columns, int32_t kind);

/* ---- block-scaled fp8 ---------------------------------------------------------------------- */
void oracle_quantize_rows_fp8(const uint16_t *in_bf16, int64_t rows, int64_t width, int64_t group,
                              uint8_t *out, float *scales);
void oracle_quantize_blocks_fp8(const uint16_t *in_bf16, int64_t stacks, int64_t n, int64_t k,
                                int64_t block, uint8_t *out, float *scales);
void oracle_gather_gemm_fp8(const uint8_t *hidden, const float *hidden_scales,
                            const uint8_t *weights, const float *weight_scales, int64_t tokens,
                            int64_t hidden_size, int64_t intermediate, int64_t top, int64_t tile,
                            const int32_t *tile_to_expert, const int32_t *tile_to_limit,
                            const int32_t *permuted_to_expanded, int32_t num_tiles, int32_t activation,
                            float *out);
void oracle_route_gemm_fp8(const uint8_t *rows, const float *row_scales, const uint8_t *weights,
                           const float *weight_scales, int64_t hidden_size, int64_t intermediate,
                           int64_t tile, const int32_t *tile_to_expert,
                           const int32_t *tile_to_limit, int32_t num_tiles, float *out);

/* ---- OCP MX: MXFP4 weights x MXFP8 activations ------------------------------------------------ */
float oracle_f32_from_e2m1(uint8_t code);
uint8_t oracle_e2m1_from_f32(float value);
uint8_t oracle_mx_scale(float amax, float limit);
void oracle_quantize_rows_mxfp8(const uint16_t *in_bf16, int64_t rows, int64_t width, uint8_t *out,
                                uint8_t *scales);
void oracle_quantize_blocks_mxfp4(const uint16_t *in_bf16, int64_t stacks, int64_t n, int64_t k,
                                  uint8_t *out, uint8_t *scales);
void oracle_gather_gemm_mx(const uint8_t *hidden, const uint8_t *hidden_scales, const uint8_t *weights,
                           const uint8_t *weight_scales, int64_t tokens, int64_t hidden_size,
                           int64_t intermediate, int64_t top, int64_t tile, const int32_t *tile_to_expert,
                           const int32_t *tile_to_limit, const int32_t *permuted_to_expanded,
                           int32_t num_tiles, int32_t activation, float *out);
void oracle_route_gemm_mx(const uint8_t *rows, const uint8_t *row_scales, const uint8_t *weights,
                          const uint8_t *weight_scales, int64_t hidden_size, int64_t intermediate, int64_t tile,
                          const int32_t *tile_to_expert, const int32_t *tile_to_limit, int32_t num_tiles,
                          float *out);

/* ---- the composed layer (the bench's CPU baseline) -------------------------------------------- */
/* weight_dtype 4 = bf16 (up_gate / down are uint16_t bf16), 6 = e4m3 (uint8_t + f32 scales),
 * 7 = MX (E2M1 pairs + E8M0 scale bytes passed through the scale pointers).
 * out is bf16 [tokens, hidden]. Returns the number of OpenMP threads used. */
int32_t oracle_moe_layer(const uint16_t *hidden, const uint16_t *router, const void *up_gate,
                         const float *up_gate_scales, const void *down, const float *down_scales,
                         int64_t tokens, int64_t hidden_size, int64_t experts, int64_t top,
                         int64_t intermediate, int32_t renormalize, int32_t weight_dtype,
                         uint16_t *out, int32_t *ids_out, float *weights_out);

/* The composed layer with everything MoE::routed passes (crates/nn/src/modules/moe.rs:650-795).
 * weight_dtype 5 = f32 (hidden, router, up_gate, down, out all f32: the CPU reference path),
 * 4 = bf16, 6 = e4m3, 7 = MX as above (hidden, router and out bf16 bits). The stacks hold the
 * window's experts [local_experts, ...]; local_experts 0 means every expert. Optional (NULL):
 * router_bias [experts] f32, map [experts], load [experts] (incremented), live_tokens [1],
 * ids / weights / scores outputs (scores in the hidden rows' element type). */
typedef struct oracle_layer_call {
  const void *hidden;
  const void *router;
  const float *router_bias;
  const void *up_gate;
  const void *up_gate_scales;
  const void *down;
  const void *down_scales;
  const int32_t *map;
  int64_t *load;
  const int32_t *live_tokens;
  int64_t tokens;
  int64_t hidden_size;
  int64_t experts;
  int64_t top;
  int64_t intermediate;
  int64_t local_offset;
  int64_t local_experts;
  int32_t renormalize;
  int32_t weight_dtype;
  int32_t activation;
  int32_t reserved;
  void *out;
  int32_t *ids;
  float *weights;
  void *scores;
} oracle_layer_call;
int32_t oracle_moe_layer_ex(const oracle_layer_call *call);
int32_t oracle_threads(void);

#ifdef __cplusplus
}
#endif

#endif

/* SPDX-License-Identifier: Apache-2.0
 *
 * CPU oracle of the fused-MoE hot path - TEST INFRASTRUCTURE, never shipped or called by the
 * product library. Each function cites the reference code it restates. Which of them are pinned
 * by which checks (golden vectors of the reference's tests, closed forms, brute force,
 * independent implementations) is listed in tests/test_oracle.py; a function no check pins says
 * "parity unpinned" at its definition.
 *
 * Compiled with -ffp-contract=off: every fused multiply-add is an explicit fmaf, so the router's
 * arithmetic is the same sequence of IEEE operations as the device kernel's.
 */
#include "moe_oracle.h"

#include <float.h>
#include <limits.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- element codecs ---------------------------------------------------------------------------- */

static uint32_t bits_of(float value) {
  uint32_t bits;
  memcpy(&bits, &value, 4);
  return bits;
}

static float float_of(uint32_t bits) {
  float value;
  memcpy(&value, &bits, 4);
  return value;
}

/* bf16 = the high half of an FP32, rounded to nearest even (the tensor library's rounding,
 * crates/nn/testing/src/values.rs:5-9 -> ops::values::encode). */
uint16_t oracle_bf16_from_f32(float value) {
  uint32_t bits = bits_of(value);
  if ((bits & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((bits >> 16) | 0x40u);
  bits += 0x7fffu + ((bits >> 16) & 1u);
  return (uint16_t)(bits >> 16);
}

float oracle_f32_from_bf16(uint16_t bits) { return float_of((uint32_t)bits << 16); }

/* IEEE binary16, round to nearest even (for f16 router scores, routing.rs:124-131). */
uint16_t oracle_f16_from_f32(float value) {
  uint32_t bits = bits_of(value);
  uint32_t sign = (bits >> 16) & 0x8000u;
  float a = fabsf(value);
  if (a != a) return (uint16_t)(sign | 0x7e00u);
  if (a >= 65520.0f) return (uint16_t)(sign | 0x7c00u);
  if (a < 6.103515625e-05f) { /* subnormal: units of 2^-24 */
    float q = rintf(a * 16777216.0f);
    return (uint16_t)(sign | (uint32_t)q);
  }
  int exponent;
  float mantissa = frexpf(a, &exponent); /* a = m * 2^e, m in [0.5, 1) */
  float scaled = rintf((mantissa * 2.0f - 1.0f) * 1024.0f);
  uint32_t e = (uint32_t)(exponent - 1 + 15);
  uint32_t m = (uint32_t)scaled;
  if (m == 1024u) { m = 0; e += 1; }
  return (uint16_t)(sign | (e << 10) | m);
}

float oracle_f32_from_f16(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  float magnitude;
  if (e == 0) magnitude = ldexpf((float)m, -24);
  else if (e == 31) magnitude = m ? NAN : INFINITY;
  else magnitude = ldexpf((float)(m | 0x400u), (int)e - 25);
  return float_of(bits_of(magnitude) | sign);
}

/* OCP e4m3fn: bias 7, three mantissa bits, no infinities, 0x7f/0xff NaN, largest finite 448.
 * Nearest even, saturating at 448: the rule crates/nn/src/quantization/dynamic.rs:9 states and
 * `e4m3_nearest` (crates/nn/tests/moe.rs:568-582) spells out by exhaustive search. */
uint8_t oracle_e4m3_from_f32(float value) {
  uint8_t sign = signbit(value) ? 0x80u : 0u;
  float a = fabsf(value);
  if (a != a) return (uint8_t)(sign | 0x7fu);
  if (a >= 448.0f) return (uint8_t)(sign | 0x7eu);
  if (a < 0.015625f) { /* below 2^-6: subnormal steps of 2^-9 (8 steps reach 2^-6 = code 8) */
    float q = rintf(a * 512.0f);
    return (uint8_t)(sign | (uint8_t)q);
  }
  int exponent;
  float mantissa = frexpf(a, &exponent); /* a = m * 2^exponent, m in [0.5, 1) */
  int e = exponent - 1;                  /* a = (2m) * 2^e, 2m in [1, 2) */
  float steps = rintf((mantissa * 2.0f - 1.0f) * 8.0f);
  int m = (int)steps;
  if (m == 8) { m = 0; e += 1; }
  int code = ((e + 7) << 3) | m;
  if (code > 0x7e) code = 0x7e;
  return (uint8_t)(sign | (uint8_t)code);
}

/* `e4m3_value` (crates/nn/tests/moe.rs:550-565) and NaN for 0x7f/0xff. */
float oracle_f32_from_e4m3(uint8_t code) {
  int exponent = (code >> 3) & 0xf, mantissa = code & 7;
  float magnitude;
  if ((code & 0x7f) == 0x7f) return NAN;
  if (exponent == 0) magnitude = ldexpf((float)mantissa, -9);
  else magnitude = ldexpf((float)(8 + mantissa), exponent - 10);
  return (code & 0x80) ? -magnitude : magnitude;
}

/* The 256 e4m3 values, decoded once when the library loads (the products read them per element). */
static float e4m3_values[256];

__attribute__((constructor)) static void fill_e4m3_values(void) {
  for (int code = 0; code < 256; ++code) e4m3_values[code] = oracle_f32_from_e4m3((uint8_t)code);
}

void oracle_bf16_encode(const float *in, uint16_t *out, int64_t count) {
  for (int64_t i = 0; i < count; ++i) out[i] = oracle_bf16_from_f32(in[i]);
}

void oracle_bf16_decode(const uint16_t *in, float *out, int64_t count) {
  for (int64_t i = 0; i < count; ++i) out[i] = oracle_f32_from_bf16(in[i]);
}

/* The router's exponential: Cody-Waite reduction x = n ln2 + r, |r| <= ln2/2, and the degree-7
 * Taylor polynomial of e^r in Horner form with fused multiply-adds, scaled by 2^n in two exact
 * power-of-two steps. Its truncation error is below r^8/8! < 6e-9 relative, under half an FP32
 * unit. The device kernel evaluates the same operations in the same order (the reference's kernel
 * calls CUDA's expf, topk_softmax.cu:126, whose steps are not restated here), so the oracle's
 * probabilities are the kernel's bit for bit. */
float oracle_expf(float x) {
  if (x != x) return x;
  if (x < -104.0f) return 0.0f;
  if (x > 88.75f) return INFINITY;
  const float n = rintf(x * 1.44269504088896341f);
  float r = fmaf(-n, 0.693145751953125f, x);
  r = fmaf(-n, 1.42860682030941723e-6f, r);
  float p = 1.98412698412698413e-4f; /* 1/7! */
  p = fmaf(p, r, 1.38888888888888889e-3f);
  p = fmaf(p, r, 8.33333333333333333e-3f);
  p = fmaf(p, r, 4.16666666666666667e-2f);
  p = fmaf(p, r, 1.66666666666666667e-1f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const int k = (int)n;
  const int half = k / 2;
  const float first = float_of((uint32_t)(half + 127) << 23);
  const float second = float_of((uint32_t)(k - half + 127) << 23);
  return (p * first) * second;
}

/* ---- inputs ------------------------------------------------------------------------------------ */

/* nn_testing::sequence (crates/nn/testing/src/values.rs:53-66): a 32-bit LCG with Numerical
 * Recipes' constants seeded 0x9e3779b9 * (seed + 1); value = (state >> 8) / 2^23 - 1. */
void oracle_sequence(int64_t count, uint32_t seed, float *out) {
  uint32_t state = 0x9e3779b9u * (seed + 1u);
  for (int64_t i = 0; i < count; ++i) {
    state = state * 1664525u + 1013904223u;
    out[i] = (float)(state >> 8) / (float)(1u << 23) - 1.0f;
  }
}

static uint64_t splitmix64(uint64_t x) {
  x += 0x9e3779b97f4a7c15ull;
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
  return x ^ (x >> 31);
}

/* Seeded N(mean, stddev): SplitMix64 of (seed, pair index) -> Box-Muller. Counter-based, so
 * element i does not depend on how the range is split between threads. */
void oracle_normal(int64_t count, uint64_t seed, float mean, float stddev, float *out) {
  const int64_t pairs = (count + 1) / 2;
#pragma omp parallel for schedule(static)
  for (int64_t j = 0; j < pairs; ++j) {
    uint64_t a = splitmix64(seed * 0x100000001b3ull + 2u * (uint64_t)j);
    uint64_t b = splitmix64(a ^ 0x632be59bd9b4e019ull);
    double u1 = ((double)(a >> 11) + 1.0) * 0x1.0p-53; /* (0, 1] */
    double u2 = (double)(b >> 11) * 0x1.0p-53;
    double radius = sqrt(-2.0 * log(u1));
    double angle = 6.283185307179586476925 * u2;
    out[2 * j] = (float)(mean + stddev * radius * cos(angle));
    if (2 * j + 1 < count) out[2 * j + 1] = (float)(mean + stddev * radius * sin(angle));
  }
}

void oracle_normal_bf16(int64_t count, uint64_t seed, float stddev, uint16_t *out) {
  const int64_t block = 1 << 16;
  float *buffer = (float *)malloc((size_t)block * sizeof(float));
  for (int64_t first = 0; first < count; first += block) {
    int64_t n = count - first < block ? count - first : block;
    /* element i of the whole range: generate the block's pairs from their global indices */
    const int64_t pairs = (n + 1) / 2;
    for (int64_t j = 0; j < pairs; ++j) {
      int64_t global = first / 2 + j;
      uint64_t a = splitmix64(seed * 0x100000001b3ull + 2u * (uint64_t)global);
      uint64_t b = splitmix64(a ^ 0x632be59bd9b4e019ull);
      double u1 = ((double)(a >> 11) + 1.0) * 0x1.0p-53;
      double u2 = (double)(b >> 11) * 0x1.0p-53;
      double radius = sqrt(-2.0 * log(u1));
      double angle = 6.283185307179586476925 * u2;
      buffer[2 * j] = (float)(stddev * radius * cos(angle));
      if (2 * j + 1 < n) buffer[2 * j + 1] = (float)(stddev * radius * sin(angle));
    }
    for (int64_t i = 0; i < n; ++i) out[first + i] = oracle_bf16_from_f32(buffer[i]);
  }
  free(buffer);
}

/* ---- max_tiles --------------------------------------------------------------------------------- */

/* ops::moe::max_tiles (crates/ops/src/moe/mod.rs:63-70). */
int64_t oracle_max_tiles(int64_t tokens, int64_t top, int64_t local_experts, int64_t tile) {
  const int64_t expanded = tokens * top;
  if (expanded <= local_experts || tile == 0) return expanded;
  return (expanded + (tile - 1) * local_experts) / tile;
}

/* ---- topk_softmax ------------------------------------------------------------------------------ */

static float load_kind(const void *data, int32_t kind, int64_t index) {
  if (kind == 0) return ((const float *)data)[index];
  if (kind == 2) return oracle_f32_from_f16(((const uint16_t *)data)[index]);
  return oracle_f32_from_bf16(((const uint16_t *)data)[index]);
}

#define LANES 32
#define MAX_ITER 32 /* 1024 experts / 32 lanes */
#define MAX_PICKS 32

/* The router's arithmetic in the order the reference device kernel evaluates it, lane by lane
 * of one 32-lane group (crates/ops/kernels/topk_softmax/nvcc/src/topk_softmax.cu:102-214):
 * lane l holds experts l + 32 i (-inf past the row), takes its maximum, xor-butterflies it over
 * 16..1, sums exp(v - max) in i order, xor-butterflies the sum, divides; then `top` rounds of a
 * (value, lower id) arg-max butterfly; renormalises by the xor butterfly over the next power of
 * two of `top` picks (zeros past `top`), clamped at FLT_EPSILON; scales; maps; counts the load.
 * The CPU formula of the same operator is crates/nn/src/functional/moe.rs:197-262 (the same
 * selection rule: descending probability, equal ones in ascending id). */
void oracle_topk_softmax(const void *scores, int32_t score_kind, int64_t row_stride, int32_t rows,
                         int32_t experts, int32_t top, int32_t renormalize, const void *scale,
                         int32_t scale_kind, int32_t *ids, float *weights, const int32_t *map,
                         const int32_t *live, int64_t *load) {
  const int iterations = (experts + LANES - 1) / LANES;
  int width = 1;
  while (width < top) width *= 2;
  for (int32_t row = 0; row < rows; ++row) {
    float values[LANES][MAX_ITER];
    float lane_max[LANES], next[LANES];
    for (int lane = 0; lane < LANES; ++lane) {
      for (int it = 0; it < iterations; ++it) {
        const int expert = lane + it * LANES;
        values[lane][it] = expert < experts
                               ? load_kind(scores, score_kind, (int64_t)row * row_stride + expert)
                               : -INFINITY;
      }
      float m = values[lane][0];
      for (int it = 0; it < iterations; ++it) m = m > values[lane][it] ? m : values[lane][it];
      lane_max[lane] = m;
    }
    for (int offset = LANES / 2; offset > 0; offset /= 2) {
      for (int lane = 0; lane < LANES; ++lane) {
        const float other = lane_max[lane ^ offset];
        next[lane] = lane_max[lane] < other ? other : lane_max[lane];
      }
      memcpy(lane_max, next, sizeof(next));
    }
    float sums[LANES];
    for (int lane = 0; lane < LANES; ++lane) {
      float sum = 0.0f;
      for (int it = 0; it < iterations; ++it) {
        values[lane][it] = oracle_expf(values[lane][it] - lane_max[lane]);
        sum += values[lane][it];
      }
      sums[lane] = sum;
    }
    for (int offset = LANES / 2; offset > 0; offset /= 2) {
      for (int lane = 0; lane < LANES; ++lane) next[lane] = sums[lane] + sums[lane ^ offset];
      memcpy(sums, next, sizeof(next));
    }
    for (int lane = 0; lane < LANES; ++lane)
      for (int it = 0; it < iterations; ++it) values[lane][it] = values[lane][it] / sums[lane];

    float top_value[MAX_PICKS];
    int top_expert[MAX_PICKS];
    uint32_t taken[LANES];
    memset(taken, 0, sizeof(taken));
    for (int j = 0; j < width; ++j) {
      if (j >= top) {
        top_value[j] = 0.0f;
        top_expert[j] = 0;
        continue;
      }
      float best[LANES];
      int best_expert[LANES];
      for (int lane = 0; lane < LANES; ++lane) {
        best[lane] = -1.0f;
        best_expert[lane] = INT_MAX;
        for (int it = 0; it < iterations; ++it) {
          const int expert = lane + it * LANES;
          if (expert < experts && !((taken[lane] >> it) & 1u) && values[lane][it] > best[lane]) {
            best[lane] = values[lane][it];
            best_expert[lane] = expert;
          }
        }
      }
      for (int offset = LANES / 2; offset > 0; offset /= 2) {
        float nb[LANES];
        int ne[LANES];
        for (int lane = 0; lane < LANES; ++lane) {
          const float other = best[lane ^ offset];
          const int other_expert = best_expert[lane ^ offset];
          nb[lane] = best[lane];
          ne[lane] = best_expert[lane];
          if (other > best[lane] || (other == best[lane] && other_expert < best_expert[lane])) {
            nb[lane] = other;
            ne[lane] = other_expert;
          }
        }
        memcpy(best, nb, sizeof(nb));
        memcpy(best_expert, ne, sizeof(ne));
      }
      top_value[j] = best[0];
      top_expert[j] = best_expert[0];
      /* No expert named (a row of NaN scores): nothing is marked taken. */
      if (best_expert[0] >= 0 && best_expert[0] < experts)
        taken[best_expert[0] % LANES] |= 1u << (best_expert[0] / LANES);
    }

    float total = 0.0f;
    if (renormalize) {
      float partial[MAX_PICKS], summed[MAX_PICKS];
      for (int j = 0; j < width; ++j) partial[j] = top_value[j];
      for (int offset = width / 2; offset > 0; offset /= 2) {
        for (int j = 0; j < width; ++j) summed[j] = partial[j] + partial[j ^ offset];
        memcpy(partial, summed, sizeof(float) * (size_t)width);
      }
      total = partial[0] < FLT_EPSILON ? FLT_EPSILON : partial[0];
    }
    for (int slot = 0; slot < top; ++slot) {
      float weight = top_value[slot];
      const int expert = top_expert[slot];
      const int named = expert >= 0 && expert < experts;
      if (renormalize) weight = weight / total;
      if (scale_kind != -1 && scale != NULL && named) weight = weight * load_kind(scale, scale_kind, expert);
      ids[(int64_t)row * top + slot] = (map != NULL && named) ? map[expert] : expert;
      weights[(int64_t)row * top + slot] = weight;
      if (load != NULL && named && (live == NULL || row < live[0])) load[expert] += 1;
    }
  }
}

/* ---- moe_sort ---------------------------------------------------------------------------------- */

/* The routing order of TensorRT-LLM's pipeline as the reference states it
 * (crates/ops/kernels/moe_sort/trtllm/src/routing.cu:1-30, crates/nn/src/functional/moe.rs:
 * 1791-1905 `sort_formula`, crates/nn/tests/moe.rs:224-276 `sort_by_hand`): held routes grouped
 * by local expert in the window's order, each expert's routes in ascending expanded-route order
 * from a tile boundary, empty experts taking no tile. Writes what the device writes: every
 * route's entry (-1 not held, -2 not live), the live tiles' tables and the live tiles' rows
 * (-1 on padding), and the two counts; every other entry is left as it was. */
void oracle_moe_sort(const int32_t *ids, int64_t tokens, int64_t top, int64_t local_experts,
                     int64_t local_offset, int64_t tile, const int32_t *live_tokens,
                     int32_t *tile_to_expert, int32_t *tile_to_limit,
                     int32_t *expanded_to_permuted, int32_t *permuted_to_expanded,
                     int32_t *permuted_to_token, int32_t *total_padded_tokens,
                     int32_t *num_non_exiting_tiles) {
  const int64_t routes = tokens * top;
  const int64_t live = live_tokens ? (int64_t)live_tokens[0] * top : routes;
  int64_t *count = (int64_t *)calloc((size_t)local_experts, sizeof(int64_t));
  int64_t *first_tile = (int64_t *)calloc((size_t)local_experts, sizeof(int64_t));
  int64_t *filled = (int64_t *)calloc((size_t)local_experts, sizeof(int64_t));
  for (int64_t r = 0; r < routes && r < live; ++r) {
    const int64_t e = (int64_t)ids[r] - local_offset;
    if (e >= 0 && e < local_experts) count[e] += 1;
  }
  int64_t tiles = 0;
  for (int64_t e = 0; e < local_experts; ++e) {
    first_tile[e] = tiles;
    tiles += (count[e] + tile - 1) / tile;
  }
  for (int64_t e = 0; e < local_experts; ++e) {
    const int64_t n = (count[e] + tile - 1) / tile;
    const int64_t first_row = first_tile[e] * tile;
    for (int64_t t = 0; t < n; ++t) {
      const int64_t end_of_tile = (first_tile[e] + t + 1) * tile;
      const int64_t end_of_rows = first_row + count[e];
      tile_to_expert[first_tile[e] + t] = (int32_t)e;
      tile_to_limit[first_tile[e] + t] = (int32_t)(end_of_tile < end_of_rows ? end_of_tile : end_of_rows);
    }
    for (int64_t row = count[e]; row < n * tile; ++row) {
      permuted_to_expanded[first_row + row] = -1;
      permuted_to_token[first_row + row] = -1;
    }
  }
  for (int64_t r = 0; r < routes; ++r) {
    if (r >= live) {
      expanded_to_permuted[r] = -2;
      continue;
    }
    const int64_t e = (int64_t)ids[r] - local_offset;
    if (e < 0 || e >= local_experts) {
      expanded_to_permuted[r] = -1;
      continue;
    }
    const int64_t row = first_tile[e] * tile + filled[e]++;
    expanded_to_permuted[r] = (int32_t)row;
    permuted_to_expanded[row] = (int32_t)r;
    permuted_to_token[row] = (int32_t)(r / top);
  }
  total_padded_tokens[0] = (int32_t)(tiles * tile);
  num_non_exiting_tiles[0] = (int32_t)tiles;
  free(count);
  free(first_tile);
  free(filled);
}

/* ---- products ---------------------------------------------------------------------------------- */

/* A dot product of FP32 rows in eight interleaved partial sums (a fixed order; the reference's
 * CPU matmul, the `gemm` crate, sums in its own blocked order, which the operators' tolerance
 * covers: crates/ops/src/tolerance.rs:113-137). */
static float dot(const float *a, const float *b, int64_t n) {
  float partial[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int64_t i = 0;
  for (; i + 8 <= n; i += 8)
    for (int j = 0; j < 8; ++j) partial[j] += a[i + j] * b[i + j];
  float sum = 0.0f;
  for (int j = 0; j < 8; ++j) sum += partial[j];
  for (; i < n; ++i) sum += a[i] * b[i];
  return sum;
}

static float silu(float x) { return x / (1.0f + expf(-x)); }

/* The gate of FC1: silu (Qwen3) or PyTorch's gelu_pytorch_tanh, 0.5 g (1 + tanh(sqrt(2/pi)
 * (g + 0.044715 g^3))), evaluated in FP32 (crates/nn/src/functional/activation.rs:62-82; the
 * grouped products gate with these two only, crates/ops/src/moe/grouped.rs:53-61). */
static float gate_activation(float g, int32_t activation) {
  if (activation == 1) return 0.5f * g * (1.0f + tanhf(0.7978845608028654f * (g + 0.044715f * g * g * g)));
  return silu(g);
}

float oracle_gate_activation(float g, int32_t activation) { return gate_activation(g, activation); }

/* `n` elements of kind `kind` (0 f32, 1 bf16, 2 f16) from `data` at element `offset`, widened. */
static void widen_row(const void *data, int32_t kind, int64_t offset, int64_t n, float *out) {
  if (kind == 0) memcpy(out, (const float *)data + offset, (size_t)n * sizeof(float));
  else if (kind == 1) oracle_bf16_decode((const uint16_t *)data + offset, out, n);
  else
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_f32_from_f16(((const uint16_t *)data)[offset + i]);
}

/* The router Linear (crates/nn/src/modules/moe.rs:656-671 -> `Linear::forward`,
 * crates/nn/src/modules/linear.rs:653-669 -> `gemm`): out = x . W^T (+ bias) with FP32
 * accumulation, the bias added to the FP32 sum, and one rounding into the output's element type
 * (`out_kind` 1: bf16 bits; 0: f32, no rounding). Elements of x and W are of kind `kind`. */
void oracle_router_gemm_ex(const void *x, const void *weight, int32_t kind, const float *bias,
                           int64_t m, int64_t n, int64_t k, int32_t out_kind, void *out) {
  float *wf = (float *)malloc((size_t)(n * k) * sizeof(float));
  widen_row(weight, kind, 0, n * k, wf);
#pragma omp parallel
  {
    float *xf = (float *)malloc((size_t)k * sizeof(float));
#pragma omp for schedule(static)
    for (int64_t i = 0; i < m; ++i) {
      widen_row(x, kind, i * k, k, xf);
      for (int64_t j = 0; j < n; ++j) {
        float value = dot(xf, wf + j * k, k);
        if (bias != NULL) value += bias[j];
        if (out_kind == 0) ((float *)out)[i * n + j] = value;
        else ((uint16_t *)out)[i * n + j] = oracle_bf16_from_f32(value);
      }
    }
    free(xf);
  }
  free(wf);
}

void oracle_router_gemm(const uint16_t *x, const uint16_t *weight, int64_t m, int64_t n, int64_t k,
                        uint16_t *out) {
  oracle_router_gemm_ex(x, weight, 1, NULL, m, n, k, 1, out);
}

/* gather_gemm's CPU formula (crates/nn/src/functional/moe.rs:554-578): per live permuted row p
 * of tile t (rows below tile_to_limit[t]), token = permuted_to_expanded[p] / top, expert =
 * tile_to_expert[t]; up = W[e, 0:I] . x[token], gate = W[e, I:2I] . x[token] in FP32;
 * out[p, :] = silu(gate) * up in FP32 (the rounding into bf16 is the caller's). The per-row
 * weight gather of the reference (`index_select(&expert)`, moe.rs:570) is evaluated per tile:
 * the same sums, grouped by expert. Rows the formula does not name are left untouched. */
void oracle_gather_gemm_ex(const void *hidden, const void *weights, int32_t kind, int64_t tokens,
                           int64_t hidden_size, int64_t intermediate, int64_t top, int64_t tile,
                           const int32_t *tile_to_expert, const int32_t *tile_to_limit,
                           const int32_t *permuted_to_expanded, int32_t num_tiles, int32_t activation,
                           float *out) {
  (void)tokens;
  const int64_t width = 2 * intermediate;
#pragma omp parallel
  {
    float *w = (float *)malloc((size_t)hidden_size * sizeof(float));
    float *x = (float *)malloc((size_t)(tile * hidden_size) * sizeof(float));
    float *up = (float *)malloc((size_t)(tile * intermediate) * sizeof(float));
#pragma omp for schedule(dynamic, 1)
    for (int32_t t = 0; t < num_tiles; ++t) {
      const int64_t e = tile_to_expert[t];
      const int64_t first = (int64_t)t * tile;
      const int64_t rows = tile_to_limit[t] - first;
      for (int64_t r = 0; r < rows; ++r)
        widen_row(hidden, kind, (permuted_to_expanded[first + r] / top) * hidden_size, hidden_size,
                  x + r * hidden_size);
      for (int64_t n = 0; n < width; ++n) {
        widen_row(weights, kind, (e * width + n) * hidden_size, hidden_size, w);
        for (int64_t r = 0; r < rows; ++r) {
          const float value = dot(x + r * hidden_size, w, hidden_size);
          if (n < intermediate) up[r * intermediate + n] = value;
          else out[(first + r) * intermediate + (n - intermediate)] =
                   gate_activation(value, activation) * up[r * intermediate + (n - intermediate)];
        }
      }
    }
    free(w);
    free(x);
    free(up);
  }
}

void oracle_gather_gemm(const uint16_t *hidden, const uint16_t *weights, int64_t tokens,
                        int64_t hidden_size, int64_t intermediate, int64_t top, int64_t tile,
                        const int32_t *tile_to_expert, const int32_t *tile_to_limit,
                        const int32_t *permuted_to_expanded, int32_t num_tiles, float *out) {
  oracle_gather_gemm_ex(hidden, weights, 1, tokens, hidden_size, intermediate, top, tile, tile_to_expert,
                        tile_to_limit, permuted_to_expanded, num_tiles, 0, out);
}

/* route_gemm's CPU formula (crates/nn/src/functional/moe.rs:706-723): out[p, :] =
 * W[e] . rows[p] in FP32 for the live rows of every live tile. */
void oracle_route_gemm_ex(const void *rows, const void *weights, int32_t kind, int64_t hidden_size,
                          int64_t intermediate, int64_t tile, const int32_t *tile_to_expert,
                          const int32_t *tile_to_limit, int32_t num_tiles, float *out) {
#pragma omp parallel
  {
    float *w = (float *)malloc((size_t)intermediate * sizeof(float));
    float *x = (float *)malloc((size_t)(tile * intermediate) * sizeof(float));
#pragma omp for schedule(dynamic, 1)
    for (int32_t t = 0; t < num_tiles; ++t) {
      const int64_t e = tile_to_expert[t];
      const int64_t first = (int64_t)t * tile;
      const int64_t count = tile_to_limit[t] - first;
      widen_row(rows, kind, first * intermediate, count * intermediate, x);
      for (int64_t n = 0; n < hidden_size; ++n) {
        widen_row(weights, kind, (e * hidden_size + n) * intermediate, intermediate, w);
        for (int64_t r = 0; r < count; ++r)
          out[(first + r) * hidden_size + n] = dot(x + r * intermediate, w, intermediate);
      }
    }
    free(w);
    free(x);
  }
}

void oracle_route_gemm(const uint16_t *rows, const uint16_t *weights, int64_t hidden_size,
                       int64_t intermediate, int64_t tile, const int32_t *tile_to_expert,
                       const int32_t *tile_to_limit, int32_t num_tiles, float *out) {
  oracle_route_gemm_ex(rows, weights, 1, hidden_size, intermediate, tile, tile_to_expert, tile_to_limit,
                       num_tiles, out);
}

/* moe_unpermute (crates/ops/src/moe/combine.rs:1-17, CPU formula crates/nn/src/functional/moe.rs:
 * 1258-1291): out[t] = sum over k in route order of scales[t,k] * routes[row] in FP32, a route
 * whose map entry is negative (or past the routes' rows) contributing nothing; row =
 * expanded_to_permuted[t,k] in the permuted layout, t * top + k in the expanded one. */
void oracle_moe_unpermute_ex(const void *routes, int32_t kind, const int32_t *expanded_to_permuted,
                             const float *scales, int64_t tokens, int64_t top, int64_t hidden,
                             int64_t routes_rows, int32_t layout, float *out) {
#pragma omp parallel
  {
    float *row_values = (float *)malloc((size_t)hidden * sizeof(float));
#pragma omp for schedule(static)
    for (int64_t t = 0; t < tokens; ++t) {
      float *sum = out + t * hidden;
      for (int64_t h = 0; h < hidden; ++h) sum[h] = 0.0f;
      for (int64_t k = 0; k < top; ++k) {
        const int64_t entry = expanded_to_permuted[t * top + k];
        if (entry < 0 || entry >= routes_rows) continue;
        const int64_t row = layout == 1 ? t * top + k : entry;
        const float w = scales[t * top + k];
        widen_row(routes, kind, row * hidden, hidden, row_values);
        for (int64_t h = 0; h < hidden; ++h) sum[h] += w * row_values[h];
      }
    }
    free(row_values);
  }
}

void oracle_moe_unpermute(const uint16_t *routes, const int32_t *expanded_to_permuted,
                          const float *scales, int64_t tokens, int64_t top, int64_t hidden,
                          int64_t routes_rows, int32_t layout, float *out) {
  oracle_moe_unpermute_ex(routes, 1, expanded_to_permuted, scales, tokens, top, hidden, routes_rows, layout, out);
}

/* sigmoid_gated_add (crates/ops/src/residual.rs:808-811; CPU form crates/nn/src/functional/moe.rs:1589-1600):
 * target[r, c] = round(target[r, c] + sigmoid(gate[r]) * update[r, c]), FP32 arithmetic, elements of
 * `kind` (0 f32, 1 bf16, 2 f16) as raw bits. */
static float widen_kind(const void *data, int32_t kind, int64_t index) {
  if (kind == 0) return ((const float *)data)[index];
  if (kind == 2) return oracle_f32_from_f16(((const uint16_t *)data)[index]);
  return oracle_f32_from_bf16(((const uint16_t *)data)[index]);
}

void oracle_sigmoid_gated_add(void *target, const void *update, const void *gate, int64_t rows,
                              int64_t columns, int32_t kind) {
  for (int64_t r = 0; r < rows; ++r) {
    const float g = 1.0f / (1.0f + expf(-widen_kind(gate, kind, r)));
    for (int64_t c = 0; c < columns; ++c) {
      const int64_t i = r * columns + c;
      const float sum = widen_kind(target, kind, i) + g * widen_kind(update, kind, i);
      if (kind == 0) ((float *)target)[i] = sum;
      else if (kind == 2) ((uint16_t *)target)[i] = oracle_f16_from_f32(sum);
      else ((uint16_t *)target)[i] = oracle_bf16_from_f32(sum);
    }
  }
}

/* ---- block-scaled fp8 (no reference counterpart: parity unpinned against the reference;
 *      crates/nn/src/quantization.rs:241-249 refuses this format) ------------------------------ */

static float group_scale(float amax) { return amax > 0.0f ? amax / 448.0f : 1.0f; }

/* Per row, per `group` contiguous channels: s = max|x| / 448 (1 for an all-zero group),
 * q = e4m3(x / s), nearest even, saturating. */
void oracle_quantize_rows_fp8(const uint16_t *in_bf16, int64_t rows, int64_t width, int64_t group,
                              uint8_t *out, float *scales) {
  const int64_t groups = width / group;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t g = 0; g < groups; ++g) {
      const uint16_t *x = in_bf16 + r * width + g * group;
      float amax = 0.0f;
      for (int64_t i = 0; i < group; ++i) {
        const float a = fabsf(oracle_f32_from_bf16(x[i]));
        amax = a > amax ? a : amax;
      }
      const float s = group_scale(amax);
      scales[r * groups + g] = s;
      for (int64_t i = 0; i < group; ++i)
        out[r * width + g * group + i] = oracle_e4m3_from_f32(oracle_f32_from_bf16(x[i]) / s);
    }
  }
}

/* Per `block` x `block` block of each [n, k] matrix: the same rule over the block's maximum. */
void oracle_quantize_blocks_fp8(const uint16_t *in_bf16, int64_t stacks, int64_t n, int64_t k,
                                int64_t block, uint8_t *out, float *scales) {
  const int64_t bn = n / block, bk = k / block;
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t s = 0; s < stacks; ++s) {
    for (int64_t i = 0; i < bn; ++i) {
      for (int64_t j = 0; j < bk; ++j) {
        float amax = 0.0f;
        for (int64_t r = 0; r < block; ++r)
          for (int64_t c = 0; c < block; ++c) {
            const float a = fabsf(oracle_f32_from_bf16(in_bf16[(s * n + i * block + r) * k + j * block + c]));
            amax = a > amax ? a : amax;
          }
        const float scale = group_scale(amax);
        scales[(s * bn + i) * bk + j] = scale;
        for (int64_t r = 0; r < block; ++r)
          for (int64_t c = 0; c < block; ++c) {
            const int64_t at = (s * n + i * block + r) * k + j * block + c;
            out[at] = oracle_e4m3_from_f32(oracle_f32_from_bf16(in_bf16[at]) / scale);
          }
      }
    }
  }
}

/* Dot of two e4m3 rows under per-128 block scales: sum_b (sum_{k in b} qa*qb) * sa[b] * sb[b],
 * each block's inner sum exact in FP32 (products of two e4m3 values have at most 8 significant
 * bits and 128 of them stay far inside FP32's range and precision only approximately; the
 * order is fixed). */
static float dot_fp8(const uint8_t *a, const float *sa, const uint8_t *b, const float *sb,
                     int64_t k, int64_t block) {
  float total = 0.0f;
  for (int64_t kb = 0; kb < k / block; ++kb) {
    float partial = 0.0f;
    for (int64_t i = 0; i < block; ++i)
      partial += e4m3_values[a[kb * block + i]] * e4m3_values[b[kb * block + i]];
    total += partial * (sa[kb] * sb[kb]);
  }
  return total;
}

void oracle_gather_gemm_fp8(const uint8_t *hidden, const float *hidden_scales,
                            const uint8_t *weights, const float *weight_scales, int64_t tokens,
                            int64_t hidden_size, int64_t intermediate, int64_t top, int64_t tile,
                            const int32_t *tile_to_expert, const int32_t *tile_to_limit,
                            const int32_t *permuted_to_expanded, int32_t num_tiles, int32_t activation,
                            float *out) {
  (void)tokens;
  const int64_t width = 2 * intermediate, kb = hidden_size / 128, nb = width / 128;
#pragma omp parallel
  {
    float *sb = (float *)malloc((size_t)kb * sizeof(float));
#pragma omp for schedule(dynamic, 1)
    for (int32_t t = 0; t < num_tiles; ++t) {
      const int64_t e = tile_to_expert[t];
      const int64_t first = (int64_t)t * tile;
      for (int64_t p = first; p < tile_to_limit[t]; ++p) {
        const int64_t token = permuted_to_expanded[p] / top;
        for (int64_t n = 0; n < intermediate; ++n) {
          float v[2];
          for (int half = 0; half < 2; ++half) {
            const int64_t row = n + half * intermediate;
            for (int64_t b = 0; b < kb; ++b) sb[b] = weight_scales[(e * nb + row / 128) * kb + b];
            v[half] = dot_fp8(hidden + token * hidden_size, hidden_scales + token * kb,
                              weights + (e * width + row) * hidden_size, sb, hidden_size, 128);
          }
          out[p * intermediate + n] = gate_activation(v[1], activation) * v[0];
        }
      }
    }
    free(sb);
  }
}

void oracle_route_gemm_fp8(const uint8_t *rows, const float *row_scales, const uint8_t *weights,
                           const float *weight_scales, int64_t hidden_size, int64_t intermediate,
                           int64_t tile, const int32_t *tile_to_expert,
                           const int32_t *tile_to_limit, int32_t num_tiles, float *out) {
  const int64_t kb = intermediate / 128, nb = hidden_size / 128;
#pragma omp parallel
  {
    float *sb = (float *)malloc((size_t)kb * sizeof(float));
#pragma omp for schedule(dynamic, 1)
    for (int32_t t = 0; t < num_tiles; ++t) {
      const int64_t e = tile_to_expert[t];
      const int64_t first = (int64_t)t * tile;
      for (int64_t p = first; p < tile_to_limit[t]; ++p)
        for (int64_t n = 0; n < hidden_size; ++n) {
          for (int64_t b = 0; b < kb; ++b) sb[b] = weight_scales[(e * nb + n / 128) * kb + b];
          out[p * hidden_size + n] = dot_fp8(rows + p * intermediate, row_scales + p * kb,
                                             weights + (e * hidden_size + n) * intermediate, sb,
                                             intermediate, 128);
        }
    }
    free(sb);
  }
}

/* ---- OCP MX: MXFP4 weights x MXFP8 activations (no reference counterpart: the reference's
 *      four-bit experts are NVFP4, crates/ops/src/moe/grouped.rs:579-1772; parity unpinned
 *      against the reference) --------------------------------------------------------------- */

/* E2M1: sign, two exponent bits (bias 1), one mantissa bit: magnitudes 0, 0.5, 1, 1.5, 2, 3, 4, 6. */
float oracle_f32_from_e2m1(uint8_t code) {
  static const float magnitude[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  const float m = magnitude[code & 7];
  return (code & 8) ? -m : m;
}

/* Nearest E2M1 code, ties to the even code (even mantissa bit), saturating at 6; NaN -> 0. */
uint8_t oracle_e2m1_from_f32(float value) {
  if (value != value) return 0;
  const uint8_t sign = signbit(value) ? 8 : 0;
  const float a = fabsf(value);
  uint8_t best = 7;
  if (a < 6.0f) {
    /* The two neighbours in the table; midpoints go to the even code. */
    for (uint8_t c = 0; c < 7; ++c) {
      const float lo = oracle_f32_from_e2m1(c), hi = oracle_f32_from_e2m1((uint8_t)(c + 1));
      if (a >= lo && a <= hi) {
        const float mid = 0.5f * (lo + hi);
        if (a < mid) best = c;
        else if (a > mid) best = (uint8_t)(c + 1);
        else best = (c & 1) ? (uint8_t)(c + 1) : c;
        break;
      }
    }
  }
  return (uint8_t)(sign | best);
}

/* The E8M0 scale byte of a block: the smallest power of two 2^e with amax <= limit * 2^e (no
 * element saturates), e clamped to [-127, 127]; an all-zero (or non-finite) block takes 2^0. */
uint8_t oracle_mx_scale(float amax, float limit) {
  if (!(amax > 0.0f) || isinf(amax)) return 127;
  int e;
  frexpf(amax / limit, &e);                      /* amax / limit in [2^(e-1), 2^e) */
  while (e > -127 && amax <= ldexpf(limit, e - 1)) --e;
  while (e < 127 && amax > ldexpf(limit, e)) ++e;
  if (e < -127) e = -127;                        /* a subnormal block: 2^-127 already holds it */
  return (uint8_t)(e + 127);
}

static float mx_power(uint8_t x) { return ldexpf(1.0f, (int)x - 127); }

/* Per row, per 32 channels: s = oracle_mx_scale(amax, 448), q = e4m3(x / 2^(s-127)). */
void oracle_quantize_rows_mxfp8(const uint16_t *in_bf16, int64_t rows, int64_t width, uint8_t *out,
                                uint8_t *scales) {
  const int64_t blocks = width / 32;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t b = 0; b < blocks; ++b) {
      const uint16_t *x = in_bf16 + r * width + b * 32;
      float amax = 0.0f;
      for (int64_t i = 0; i < 32; ++i) {
        const float a = fabsf(oracle_f32_from_bf16(x[i]));
        amax = a > amax ? a : amax;
      }
      const uint8_t s = oracle_mx_scale(amax, 448.0f);
      scales[r * blocks + b] = s;
      const float power = mx_power(s);
      for (int64_t i = 0; i < 32; ++i) out[r * width + b * 32 + i] = oracle_e4m3_from_f32(oracle_f32_from_bf16(x[i]) / power);
    }
  }
}

/* [stacks, n, k] bf16 -> E2M1 pairs [stacks, n, k / 2] (low nibble = lower k) and E8M0 scales
 * [stacks, n, k / 32], s = oracle_mx_scale(amax, 6). */
void oracle_quantize_blocks_mxfp4(const uint16_t *in_bf16, int64_t stacks, int64_t n, int64_t k,
                                  uint8_t *out, uint8_t *scales) {
  const int64_t blocks = k / 32;
#pragma omp parallel for schedule(static)
  for (int64_t row = 0; row < stacks * n; ++row) {
    for (int64_t b = 0; b < blocks; ++b) {
      const uint16_t *x = in_bf16 + row * k + b * 32;
      float amax = 0.0f;
      for (int64_t i = 0; i < 32; ++i) {
        const float a = fabsf(oracle_f32_from_bf16(x[i]));
        amax = a > amax ? a : amax;
      }
      const uint8_t s = oracle_mx_scale(amax, 6.0f);
      scales[row * blocks + b] = s;
      const float power = mx_power(s);
      for (int64_t i = 0; i < 32; i += 2) {
        const uint8_t lo = oracle_e2m1_from_f32(oracle_f32_from_bf16(x[i]) / power);
        const uint8_t hi = oracle_e2m1_from_f32(oracle_f32_from_bf16(x[i + 1]) / power);
        out[row * (k / 2) + (b * 32 + i) / 2] = (uint8_t)(lo | (hi << 4));
      }
    }
  }
}

/* Dot of an MXFP8 row and an MXFP4 row over k: per 32-block the FP32 sum of code products (in
 * order), times both blocks' powers of two; the blocks summed in order. */
static float dot_mx(const uint8_t *a, const uint8_t *sa, const uint8_t *w, const uint8_t *sw, int64_t k) {
  float total = 0.0f;
  for (int64_t b = 0; b < k / 32; ++b) {
    float partial = 0.0f;
    for (int64_t i = 0; i < 32; ++i) {
      const int64_t at = b * 32 + i;
      const uint8_t code = (uint8_t)((w[at / 2] >> (4 * (at & 1))) & 15);
      partial += e4m3_values[a[at]] * oracle_f32_from_e2m1(code);
    }
    total += partial * (mx_power(sa[b]) * mx_power(sw[b]));
  }
  return total;
}

void oracle_gather_gemm_mx(const uint8_t *hidden, const uint8_t *hidden_scales, const uint8_t *weights,
                           const uint8_t *weight_scales, int64_t tokens, int64_t hidden_size,
                           int64_t intermediate, int64_t top, int64_t tile, const int32_t *tile_to_expert,
                           const int32_t *tile_to_limit, const int32_t *permuted_to_expanded,
                           int32_t num_tiles, int32_t activation, float *out) {
  (void)tokens;
  const int64_t width = 2 * intermediate, kb = hidden_size / 32;
#pragma omp parallel for schedule(dynamic, 1)
  for (int32_t t = 0; t < num_tiles; ++t) {
    const int64_t e = tile_to_expert[t];
    for (int64_t p = (int64_t)t * tile; p < tile_to_limit[t]; ++p) {
      const int64_t token = permuted_to_expanded[p] / top;
      for (int64_t n = 0; n < intermediate; ++n) {
        float v[2];
        for (int half = 0; half < 2; ++half) {
          const int64_t row = e * width + n + half * intermediate;
          v[half] = dot_mx(hidden + token * hidden_size, hidden_scales + token * kb, weights + row * (hidden_size / 2),
                           weight_scales + row * kb, hidden_size);
        }
        out[p * intermediate + n] = gate_activation(v[1], activation) * v[0];
      }
    }
  }
}

void oracle_route_gemm_mx(const uint8_t *rows, const uint8_t *row_scales, const uint8_t *weights,
                          const uint8_t *weight_scales, int64_t hidden_size, int64_t intermediate, int64_t tile,
                          const int32_t *tile_to_expert, const int32_t *tile_to_limit, int32_t num_tiles,
                          float *out) {
  const int64_t kb = intermediate / 32;
#pragma omp parallel for schedule(dynamic, 1)
  for (int32_t t = 0; t < num_tiles; ++t) {
    const int64_t e = tile_to_expert[t];
    for (int64_t p = (int64_t)t * tile; p < tile_to_limit[t]; ++p)
      for (int64_t n = 0; n < hidden_size; ++n) {
        const int64_t row = e * hidden_size + n;
        out[p * hidden_size + n] = dot_mx(rows + p * intermediate, row_scales + p * kb,
                                          weights + row * (intermediate / 2), weight_scales + row * kb, intermediate);
      }
  }
}

/* ---- the composed layer ------------------------------------------------------------------------ */

int32_t oracle_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* MoE::routed (crates/nn/src/modules/moe.rs:770-795) on the CPU, `MoE::select` (:656-671)
 * included: router gemm (+ bias, scores in the hidden rows' element type) -> topk (the slot map,
 * the live rows' load) -> sort (over the local window, live rows only) -> FC1 -> FC2 -> combine.
 * Rounding points are the reference's: for bf16 rows the scores, the gated rows and the products
 * round into bf16, the combine sums in FP32 and rounds once; for f32 rows (weight_dtype 5,
 * the CPU reference path of crates/nn/src/functional/moe.rs:554-578, 706-723, 1258-1291) nothing
 * rounds. For e4m3 weights (6) the activations of each product are quantised per row per 128
 * channels first; for MX weights (7: E2M1 codes, E8M0 scale bytes) per row per 32 channels to
 * MXFP8. The stacks hold the window's experts only: [local_experts, ...]. */
int32_t oracle_moe_layer_ex(const oracle_layer_call *c) {
  const int64_t tile = 128, tokens = c->tokens, hidden_size = c->hidden_size, experts = c->experts;
  const int64_t top = c->top, intermediate = c->intermediate;
  const int64_t local_experts = c->local_experts > 0 ? c->local_experts : experts;
  const int32_t f32 = c->weight_dtype == 5, kind = f32 ? 0 : 1;
  const int64_t tiles = oracle_max_tiles(tokens, top, local_experts, tile);
  const int64_t rows = tiles * tile;
  void *scores = malloc((size_t)(tokens * experts) * (f32 ? 4 : 2));
  int32_t *ids = (int32_t *)malloc((size_t)(tokens * top) * 4);
  float *weights = (float *)malloc((size_t)(tokens * top) * 4);
  int32_t *t2e = (int32_t *)calloc((size_t)tiles + 1, 4), *t2l = (int32_t *)calloc((size_t)tiles + 1, 4);
  int32_t *e2p = (int32_t *)malloc((size_t)(tokens * top) * 4);
  int32_t *p2e = (int32_t *)malloc((size_t)rows * 4), *p2t = (int32_t *)malloc((size_t)rows * 4);
  int32_t padded = 0, live_tiles = 0;
  float *gated = (float *)calloc((size_t)(rows * intermediate), 4);
  uint16_t *gated_bf16 = (uint16_t *)malloc((size_t)(rows * intermediate) * 2);
  float *products = (float *)calloc((size_t)(rows * hidden_size), 4);
  uint16_t *products_bf16 = (uint16_t *)malloc((size_t)(rows * hidden_size) * 2);
  float *combined = (float *)malloc((size_t)(tokens * hidden_size) * 4);
  const uint16_t *hidden = (const uint16_t *)c->hidden;

  oracle_router_gemm_ex(c->hidden, c->router, kind, c->router_bias, tokens, experts, hidden_size, kind, scores);
  oracle_topk_softmax(scores, kind, experts, (int32_t)tokens, (int32_t)experts, (int32_t)top, c->renormalize,
                      NULL, -1, ids, weights, c->map, c->live_tokens, c->load);
  oracle_moe_sort(ids, tokens, top, local_experts, c->local_offset, tile, c->live_tokens, t2e, t2l, e2p, p2e, p2t,
                  &padded, &live_tiles);
  if (c->weight_dtype == 6) {
    uint8_t *xq = (uint8_t *)malloc((size_t)(tokens * hidden_size));
    float *xs = (float *)malloc((size_t)(tokens * hidden_size / 128) * 4);
    oracle_quantize_rows_fp8(hidden, tokens, hidden_size, 128, xq, xs);
    oracle_gather_gemm_fp8(xq, xs, (const uint8_t *)c->up_gate, (const float *)c->up_gate_scales, tokens,
                           hidden_size, intermediate, top, tile, t2e, t2l, p2e, live_tiles, c->activation, gated);
    oracle_bf16_encode(gated, gated_bf16, (int64_t)padded * intermediate);
    uint8_t *gq = (uint8_t *)malloc((size_t)(rows * intermediate));
    float *gs = (float *)malloc((size_t)(rows * intermediate / 128) * 4);
    oracle_quantize_rows_fp8(gated_bf16, padded, intermediate, 128, gq, gs);
    oracle_route_gemm_fp8(gq, gs, (const uint8_t *)c->down, (const float *)c->down_scales, hidden_size,
                          intermediate, tile, t2e, t2l, live_tiles, products);
    free(xq); free(xs); free(gq); free(gs);
  } else if (c->weight_dtype == 7) {
    uint8_t *xq = (uint8_t *)malloc((size_t)(tokens * hidden_size));
    uint8_t *xs = (uint8_t *)malloc((size_t)(tokens * hidden_size / 32));
    oracle_quantize_rows_mxfp8(hidden, tokens, hidden_size, xq, xs);
    oracle_gather_gemm_mx(xq, xs, (const uint8_t *)c->up_gate, (const uint8_t *)c->up_gate_scales, tokens,
                          hidden_size, intermediate, top, tile, t2e, t2l, p2e, live_tiles, c->activation, gated);
    oracle_bf16_encode(gated, gated_bf16, (int64_t)padded * intermediate);
    uint8_t *gq = (uint8_t *)malloc((size_t)(rows * intermediate));
    uint8_t *gs = (uint8_t *)malloc((size_t)(rows * intermediate / 32));
    oracle_quantize_rows_mxfp8(gated_bf16, padded, intermediate, gq, gs);
    oracle_route_gemm_mx(gq, gs, (const uint8_t *)c->down, (const uint8_t *)c->down_scales, hidden_size,
                         intermediate, tile, t2e, t2l, live_tiles, products);
    free(xq); free(xs); free(gq); free(gs);
  } else if (f32) {
    oracle_gather_gemm_ex(c->hidden, c->up_gate, 0, tokens, hidden_size, intermediate, top, tile, t2e, t2l, p2e,
                          live_tiles, c->activation, gated);
    oracle_route_gemm_ex(gated, c->down, 0, hidden_size, intermediate, tile, t2e, t2l, live_tiles, products);
  } else {
    oracle_gather_gemm_ex(c->hidden, c->up_gate, 1, tokens, hidden_size, intermediate, top, tile, t2e, t2l, p2e,
                          live_tiles, c->activation, gated);
    oracle_bf16_encode(gated, gated_bf16, (int64_t)padded * intermediate);
    oracle_route_gemm_ex(gated_bf16, c->down, 1, hidden_size, intermediate, tile, t2e, t2l, live_tiles, products);
  }
  if (f32) {
    oracle_moe_unpermute_ex(products, 0, e2p, weights, tokens, top, hidden_size, rows, 0, (float *)c->out);
  } else {
    oracle_bf16_encode(products, products_bf16, (int64_t)padded * hidden_size);
    oracle_moe_unpermute_ex(products_bf16, 1, e2p, weights, tokens, top, hidden_size, rows, 0, combined);
    oracle_bf16_encode(combined, (uint16_t *)c->out, tokens * hidden_size);
  }
  if (c->ids) memcpy(c->ids, ids, (size_t)(tokens * top) * 4);
  if (c->weights) memcpy(c->weights, weights, (size_t)(tokens * top) * 4);
  if (c->scores) memcpy(c->scores, scores, (size_t)(tokens * experts) * (f32 ? 4 : 2));
  free(scores); free(ids); free(weights); free(t2e); free(t2l); free(e2p); free(p2e); free(p2t);
  free(gated); free(gated_bf16); free(products); free(products_bf16); free(combined);
  return oracle_threads();
}

/* The plain call: bf16 rows, every expert, no bias, map, load or live count, silu. */
int32_t oracle_moe_layer(const uint16_t *hidden, const uint16_t *router, const void *up_gate,
                         const float *up_gate_scales, const void *down, const float *down_scales,
                         int64_t tokens, int64_t hidden_size, int64_t experts, int64_t top,
                         int64_t intermediate, int32_t renormalize, int32_t weight_dtype,
                         uint16_t *out, int32_t *ids_out, float *weights_out) {
  oracle_layer_call c;
  memset(&c, 0, sizeof(c));
  c.hidden = hidden;
  c.router = router;
  c.up_gate = up_gate;
  c.up_gate_scales = up_gate_scales;
  c.down = down;
  c.down_scales = down_scales;
  c.tokens = tokens;
  c.hidden_size = hidden_size;
  c.experts = experts;
  c.top = top;
  c.intermediate = intermediate;
  c.renormalize = renormalize;
  c.weight_dtype = weight_dtype;
  c.out = out;
  c.ids = ids_out;
  c.weights = weights_out;
  return oracle_moe_layer_ex(&c);
}

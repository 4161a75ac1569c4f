/*
 * CPU baseline of one int4 MoE decode layer (benchmark configuration 2), timed by bench.py's
 * cpu_baseline leg beside the GPU figures.  TEST / MEASUREMENT INFRASTRUCTURE ONLY: never
 * linked into the product library.
 *
 * The reference has no CPU implementation of this path (its CUDA kernels are the
 * implementation, kernels/drama.cu:369-599; tools/reference.py:331-351 is a torch restatement),
 * so this is a plain-C restatement of the same semantics written for speed on host cores, the
 * "dequant-then-fp32-dot" form of the baseline plan:
 *   xn = RMSNorm(x; nw), logits = R . xn (bf16 router rows, row E = shared gate),
 *   softmax over the E expert logits, top-k (probability desc, index asc), weights renormalised,
 *   act[k][j] = silu(G_e[j] . xn) * (U_e[j] . xn) with w = q * scale + min per group of 64,
 *   act[topk][j] the same with the int8 shared expert (w = q * s),
 *   y[n] = res[n] + sigmoid(sgate) (SD[n] . act[topk]) + sum_k wts[k] (D_e[n] . act[k]).
 * Every weight is dequantised to fp32 and multiplied in fp32 (8 partial sums per dot, which
 * the compiler keeps in vector registers); OpenMP splits each projection over output rows.
 * Accuracy: fp32 throughout (the value oracle, or_moe_decode, accumulates in fp64); the tests
 * compare this baseline with the oracle within 1e-3 + 1e-3 |ref| (tests/test_oracle_moe.py).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "moe_oracle.h"

#define HOT __attribute__((target_clones("arch=haswell", "default")))

static inline float bf(uint16_t h) {
  union {
    uint32_t u;
    float f;
  } v = {(uint32_t)h << 16};
  return v.f;
}

static inline float scale_of(const void* s, int kind, size_t i) {
  if (kind == OR_F32) return ((const float*)s)[i];
  const uint16_t h = ((const uint16_t*)s)[i];
  return kind == OR_BF16 ? bf(h) : or_f16_to_f32(h);
}

/* fp32 dot of a bf16 row with x */
HOT static float dot_bf16(const uint16_t* w, const float* x, int K) {
  float acc[8] = {0};
  for (int k = 0; k < K; k += 8)
    for (int t = 0; t < 8; ++t) acc[t] += bf(w[k + t]) * x[k + t];
  return ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
}

/* fp32 dot of an int4 (scale, min) group-64 row with x: each weight dequantised, then multiplied */
HOT static float dot_q4(const uint8_t* q, const void* sm, int kind, size_t g0, const float* x, int K) {
  float acc[8] = {0};
  for (int g = 0; g < K / 64; ++g) {
    const float s = scale_of(sm, kind, 2 * (g0 + g)), m = scale_of(sm, kind, 2 * (g0 + g) + 1);
    const uint8_t* qg = q + g * 32;
    const float* xg = x + g * 64;
    for (int c = 0; c < 32; c += 4)
      for (int t = 0; t < 4; ++t) {
        const uint8_t b = qg[c + t];
        acc[2 * t] += ((float)(b & 15) * s + m) * xg[2 * (c + t)];
        acc[2 * t + 1] += ((float)(b >> 4) * s + m) * xg[2 * (c + t) + 1];
      }
  }
  return ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
}

/* fp32 dot of an int8 row (scale per `group` inputs) with x */
HOT static float dot_q8(const int8_t* q, const void* s, int kind, size_t s0, int group, const float* x, int K) {
  float acc[8] = {0};
  for (int g0 = 0; g0 < K; g0 += group) {
    const float sc = scale_of(s, kind, s0 + (size_t)(g0 / group));
    for (int k = g0; k < g0 + group; k += 8)
      for (int t = 0; t < 8; ++t) acc[t] += ((float)q[k + t] * sc) * x[k + t];
  }
  return ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
}

static float silu_f(float g) { return g / (1.f + expf(-g)); }

/* One decode layer on the host: routing out (idx, wts), y = res + MoE(RMSNorm(x)).  Only the
 * int4 experts (W->kind == 0) are supported; h % 64 == 0, i % 64 == 0, e <= 256, topk <= 32.
 * y may alias x and res.  Returns 0, or -1 for an unsupported shape. */
int or_cpu_layer_f32(const or_moe_weights* W, const uint16_t* router, const float* nw, float eps, const float* x,
                     const float* res, float* y, int E, int H, int I, int topk, int* idx, float* wts) {
  if (W->kind != 0 || H % 64 || I % 64 || E > 256 || E < 1 || topk < 1 || topk > 32 || topk > E) return -1;
  float* xn = (float*)malloc(sizeof(float) * (size_t)H);
  float* logits = (float*)malloc(sizeof(float) * (size_t)(E + 1));
  float* act = (float*)malloc(sizeof(float) * (size_t)(topk + 1) * I);
  float* out = (float*)malloc(sizeof(float) * (size_t)H);
  double ss = 0.0;
  for (int k = 0; k < H; ++k) ss += (double)x[k] * x[k];
  const float inv = 1.f / sqrtf((float)(ss / H) + eps);
  for (int k = 0; k < H; ++k) xn[k] = x[k] * inv * (nw ? nw[k] : 1.f);
#pragma omp parallel for schedule(static)
  for (int r = 0; r <= E; ++r) logits[r] = dot_bf16(router + (size_t)r * H, xn, H);
  or_softmax_topk(logits, E, topk, idx, wts);
  const float sg = 1.f / (1.f + expf(-logits[E]));
  const size_t gu_row = (size_t)(H / 2), gu_grp = (size_t)(H / 64), d_row = (size_t)(I / 2), d_grp = (size_t)(I / 64);
#pragma omp parallel for schedule(static) collapse(2)
  for (int k = 0; k <= topk; ++k)
    for (int j = 0; j < I; ++j) {
      float g, u;
      if (k < topk) {
        const size_t e = (size_t)idx[k];
        const size_t rg = e * 2 * I + j, ru = e * 2 * I + I + j;
        g = dot_q4(W->gu_q + rg * gu_row, W->gu_s, W->sc_kind, rg * gu_grp, xn, H);
        u = dot_q4(W->gu_q + ru * gu_row, W->gu_s, W->sc_kind, ru * gu_grp, xn, H);
      } else {
        const int grp = W->sh_group_gu;
        g = dot_q8(W->sgu_q + (size_t)j * H, W->sgu_s, W->sh_kind, (size_t)j * (H / grp), grp, xn, H);
        u = dot_q8(W->sgu_q + (size_t)(I + j) * H, W->sgu_s, W->sh_kind, (size_t)(I + j) * (H / grp), grp, xn, H);
      }
      act[(size_t)k * I + j] = silu_f(g) * u;
    }
#pragma omp parallel for schedule(static)
  for (int n = 0; n < H; ++n) {
    const int grp = W->sh_group_d;
    float acc = sg * dot_q8(W->sd_q + (size_t)n * I, W->sd_s, W->sh_kind, (size_t)n * (I / grp), grp,
                            act + (size_t)topk * I, I);
    for (int k = 0; k < topk; ++k) {
      const size_t r = (size_t)idx[k] * H + n;
      acc += wts[k] * dot_q4(W->d_q + r * d_row, W->d_s, W->sc_kind, r * d_grp, act + (size_t)k * I, I);
    }
    out[n] = res[n] + acc;
  }
  memcpy(y, out, sizeof(float) * (size_t)H);
  free(out);
  free(act);
  free(logits);
  free(xn);
  return 0;
}

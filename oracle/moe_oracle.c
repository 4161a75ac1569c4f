/*
 * CPU oracle for the drama-rs routed-expert MoE path.  TEST INFRASTRUCTURE ONLY: loaded by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the product.
 *
 * Compile with -ffp-contract=off: every fused multiply-add below is an explicit fmaf and
 * every other operation rounds on its own, so the canonical fp32 functions are reproducible
 * bit for bit by the gfx950 kernels.
 *
 * Parity status per function (how each one is pinned, see tests/test_oracle_*.py):
 *   or_dequant_q4       KAT of src/apple.rs:206-227 + closed forms (nibble 0 -> min, 15 -> 15s+min)
 *   or_dequant_q8       KAT of src/apple.rs:191-203
 *   or_quant_q8         KAT of src/convert/mod.rs:624-635 (half-even, 127 -> scale 1.0)
 *   or_fp8e4m3_to_f32   KAT of src/convert/mod.rs:614-621 + closed form over all 256 codes
 *   or_exp              against libm exp in double (<= 2 ulp), special values
 *   or_rmsnorm_canon,
 *   or_dot_bf16_canon   against float64 sums (tight bound) and exact small-integer cases
 *   or_softmax_topk     one-hot, all-equal (ties -> lowest indices), E == topk, brute-force sort,
 *                       weights against float64 softmax
 *   or_moe_group        histogram / exclusive scan / stable-permutation invariants, brute force
 *   or_moe_decode       dense float64 matmul restatement (numpy), single-expert == SwiGLU MLP,
 *                       expert-storage permutation invariance, zero expert
 *   or_moe_prefill_*    row-wise agreement with or_moe_decode_rows on bf16-rounded inputs
 */
#include "moe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------------------------ */
/* conversions */

static inline uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

float or_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t or_f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40); /* quiet NaN */
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float or_f16_to_f32(uint16_t h) {
  const uint32_t s = (uint32_t)(h >> 15) << 31;
  const int e = (h >> 10) & 31;
  const uint32_t m = h & 1023;
  if (e == 31) return u2f(s | 0x7f800000u | (m << 13));
  if (e == 0) {
    const float v = (float)m * 5.9604644775390625e-08f; /* m * 2^-24, exact */
    return s ? -v : v;
  }
  return u2f(s | ((uint32_t)(e - 15 + 127) << 23) | (m << 13));
}

uint16_t or_f32_to_f16(float f) {
  const uint32_t u = f2u(f);
  const uint16_t s = (uint16_t)((u >> 16) & 0x8000);
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return s | 0x7e00;
  if (a >= 0x477ff000u) return s | 0x7c00; /* >= 65520 rounds to inf */
  if (a < 0x38800000u) {                   /* below 2^-14: subnormal half */
    /* value * 2^24 rounded to nearest even integer gives the subnormal mantissa */
    const double v = (double)u2f(a) * 16777216.0;
    double r = nearbyint(v);
    return s | (uint16_t)r;
  }
  uint32_t e = (a >> 23) - 127 + 15;
  uint32_t m = a & 0x7fffffu;
  uint32_t h = (e << 10) | (m >> 13);
  const uint32_t rem = m & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1; /* carries into exponent correctly */
  return s | (uint16_t)h;
}

/* OCP e4m3 ("e4m3fn"): bias 7, no infinities, S.1111.111 is NaN, max 448.
 * Follows the table of src/convert/mod.rs:126-140. */
float or_fp8e4m3_to_f32(uint8_t v) {
  const int sign = (v >> 7) & 1, e = (v >> 3) & 15, m = v & 7;
  float mag;
  if (e == 15 && m == 7)
    mag = NAN;
  else if (e == 0)
    mag = ldexpf((float)m, -9);
  else
    mag = ldexpf(1.0f + (float)m / 8.0f, e - 7);
  return sign ? -mag : mag;
}

/* round-to-nearest-even encode with saturation to +-448 (the OCP "satfinite" convention) */
uint8_t or_f32_to_fp8e4m3(float f) {
  if (f != f) return 0x7f;
  const uint8_t s = signbit(f) ? 0x80 : 0;
  float a = fabsf(f);
  if (a >= 448.0f) return s | 0x7e;
  /* enumerate: find the nearest of the 127 finite magnitudes, ties to even mantissa */
  int best = 0;
  float bd = INFINITY;
  for (int c = 0; c < 0x7f; ++c) {
    const float d = fabsf(or_fp8e4m3_to_f32((uint8_t)c) - a);
    if (d < bd || (d == bd && (c & 1) == 0)) bd = d, best = c;
  }
  return s | (uint8_t)best;
}

/* exp(x): Cody-Waite reduction x = k ln2 + r with k = rint(x log2 e), then the degree-8
 * Taylor polynomial of e^r on |r| <= ln2/2 in Horner form, then r-scaling by 2^k.  Results
 * that would fall below 2^-125 return 0 and large inputs return +inf, so no subnormal is ever
 * produced.  The kernels evaluate the same sequence of fp32 operations. */
float or_exp(float x) {
  if (x != x) return x;
  if (x < -86.5f) return 0.0f;
  if (x > 88.0f) return INFINITY;
  const float k = rintf(x * 1.44269504088896341f);
  float r = fmaf(-k, 0.693145751953125f, x);
  r = fmaf(-k, 1.428606765330187e-06f, r);
  float p = 2.48015873e-05f;
  p = fmaf(p, r, 1.98412698e-04f);
  p = fmaf(p, r, 1.38888889e-03f);
  p = fmaf(p, r, 8.33333333e-03f);
  p = fmaf(p, r, 4.16666667e-02f);
  p = fmaf(p, r, 1.66666667e-01f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const int ki = (int)k;
  return p * u2f((uint32_t)(ki + 127) << 23);
}

void or_exp_array(const float* x, float* y, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = or_exp(x[i]);
}

/* ------------------------------------------------------------------------------------------ */
/* canonical fp32 reductions: 64 lanes, lane-strided chunks, then the ascending xor butterfly
 * (step o = 1, 2, 4, ..., 32 combines a[l] and a[l ^ o]) */

static float tree64(float* a) {
  float b[64];
  for (int o = 1; o <= 32; o <<= 1) {
    for (int l = 0; l < 64; ++l) b[l] = a[l] + a[l ^ o];
    memcpy(a, b, sizeof b);
  }
  return a[0];
}

/* 1/sqrt(t): bit-pattern seed 0x5f3759df - bits/2, then three Newton steps
 * y = y * (1.5 - (0.5 t) * (y * y)), each operation rounded on its own. */
static float canon_rsqrt(float t) {
  float y = u2f(0x5f3759dfu - (f2u(t) >> 1));
  const float h = 0.5f * t;
  for (int i = 0; i < 3; ++i) {
    const float yy = y * y;
    const float hyy = h * yy;
    const float c = 1.5f - hyy;
    y = y * c;
  }
  return y;
}

/* RMSNorm (kernels/drama.cu:180-200 semantics; the reference's rsqrtf becomes the
 * reproducible canon_rsqrt): lane l accumulates x^2 over float4 indices c = l + 64 j
 * (components in order) with fmaf, butterfly sum, t = ss * (1/K) + eps, inv = rsqrt(t),
 * xn = (x * inv) * nw. */
void or_rmsnorm_canon(const float* x, const float* nw, float eps, int K, float* xn) {
  if (!nw) {
    memcpy(xn, x, sizeof(float) * (size_t)K);
    return;
  }
  float a[64];
  for (int l = 0; l < 64; ++l) {
    float s = 0.f;
    for (int c = l; c < K / 4; c += 64)
      for (int t = 0; t < 4; ++t) s = fmaf(x[4 * c + t], x[4 * c + t], s);
    a[l] = s;
  }
  const float ss = tree64(a);
  const float t = ss * (1.0f / (float)K) + eps;
  const float inv = canon_rsqrt(t);
  for (int i = 0; i < K; ++i) xn[i] = (x[i] * inv) * nw[i];
}

/* bf16 row dot (kernels/drama.cu:104-132 semantics): lane l owns 8-element chunks
 * c = l + 64 j and accumulates w * x with fmaf in element order, then the butterfly. */
float or_dot_bf16_canon(const uint16_t* w, const float* x, int K) {
  float a[64];
  for (int l = 0; l < 64; ++l) {
    float s = 0.f;
    for (int c = l; c < K / 8; c += 64)
      for (int t = 0; t < 8; ++t) s = fmaf(or_bf16_to_f32(w[8 * c + t]), x[8 * c + t], s);
    a[l] = s;
  }
  return tree64(a);
}

void or_router_logits(const uint16_t* W, const float* xn, int rows, int K, float* logits) {
  for (int r = 0; r < rows; ++r) logits[r] = or_dot_bf16_canon(W + (size_t)r * K, xn, K);
}

/* Top-k selection key of a logit: an int in the float order of the logit (negative values
 * have their magnitude bits flipped, so -0 sorts just below +0); NaN logits rank below
 * every number, picked experts below those. */
#define KEY_PAD INT32_MIN
#define KEY_PICKED (INT32_MIN + 1)
#define KEY_NAN (INT32_MIN + 2)
static int32_t logit_key(float v) {
  if (v != v) return KEY_NAN;
  const int32_t i = (int32_t)f2u(v);
  return i >= 0 ? i : i ^ 0x7fffffff;
}

/* Top-k of E logits with softmax-renormalised weights (kernels/drama.cu:322-367,398-431;
 * selection on the logits as src/mlx/engine.rs:249-258 does -- exp is monotone, so the
 * logit order is the probability order).  Selection: k rounds of (key desc, index asc).
 * m = max of the non-NaN logits; z: lane l sums exp(l - m) over experts l + 64 j in order,
 * then the butterfly; p_k = exp(l_k - m) / z; total = sum of p_k in pick order;
 * wts_k = p_k / total. */
int or_softmax_topk(const float* l, int E, int topk, int* idx, float* wts) {
  if (E < 1 || E > 256 || topk < 1 || topk > E || topk > 32) return -1;
  float m = -INFINITY;
  for (int e = 0; e < E; ++e) m = l[e] > m ? l[e] : m;
  float a[64];
  for (int ln = 0; ln < 64; ++ln) {
    float s = 0.f;
    for (int j = 0; j < 4; ++j) {
      const int e = ln + 64 * j;
      s = s + (e < E ? or_exp(l[e] - m) : 0.f);
    }
    a[ln] = s;
  }
  const float z = tree64(a);
  int32_t key[256];
  for (int e = 0; e < E; ++e) key[e] = logit_key(l[e]);
  float total = 0.f;
  for (int k = 0; k < topk; ++k) {
    int bi = 0;
    int32_t bk = KEY_PAD;
    for (int e = 0; e < E; ++e)
      if (key[e] > bk) bk = key[e], bi = e; /* strict > keeps the lowest index on ties */
    idx[k] = bi;
    key[bi] = KEY_PICKED;
    wts[k] = or_exp(l[bi] - m) / z;
    total = total + wts[k];
  }
  for (int k = 0; k < topk; ++k) wts[k] = wts[k] / total;
  return 0;
}

int or_router_topk(const uint16_t* W, const float* x, const float* nw, float eps, float* logits, int E,
                   int topk, int K, int* idx, float* wts, float* sgate) {
  if (K % 8 != 0) return -1;
  float* xn = (float*)malloc(sizeof(float) * (size_t)K);
  or_rmsnorm_canon(x, nw, eps, K, xn);
  or_router_logits(W, xn, E + 1, K, logits);
  free(xn);
  const int rc = or_softmax_topk(logits, E, topk, idx, wts);
  if (rc) return rc;
  *sgate = logits[E];
  return 0;
}

int or_moe_topk(const float* logits, int rows, int E, int topk, int stride, int* idx, float* wts,
                float* sgate) {
  for (int r = 0; r < rows; ++r) {
    const float* l = logits + (size_t)r * stride;
    const int rc = or_softmax_topk(l, E, topk, idx + (size_t)r * topk, wts + (size_t)r * topk);
    if (rc) return rc;
    sgate[r] = l[E];
  }
  return 0;
}

/* C[M, N] = A[M, K] . W[N, K]^T with A, W bf16 and the canonical dot per element. */
int or_router_logits_rows(const uint16_t* A, const uint16_t* W, float* C, int M, int N, int K) {
  if (K % 8 != 0) return -1;
#pragma omp parallel for schedule(static)
  for (int m = 0; m < M; ++m) {
    float* x = (float*)malloc(sizeof(float) * (size_t)K);
    for (int k = 0; k < K; ++k) x[k] = or_bf16_to_f32(A[(size_t)m * K + k]);
    for (int n = 0; n < N; ++n) C[(size_t)m * N + n] = or_dot_bf16_canon(W + (size_t)n * K, x, K);
    free(x);
  }
  return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* grouping: counting sort of (row, k) pairs by expert, stable in the pair index
 * (kernels/drama.cu:744-778 computes the same counts/offsets; its within-expert order comes
 * from atomics and is unspecified, the stable order is the refinement both sides use). */
int or_moe_group(const int* idx, int n, int E, int* counts, int* offsets, int* slot_of) {
  if (E <= 0 || n < 0) return -1;
  for (int e = 0; e < E; ++e) counts[e] = 0;
  for (int i = 0; i < n; ++i) {
    if (idx[i] < 0 || idx[i] >= E) return -1;
    counts[idx[i]]++;
  }
  int acc = 0;
  for (int e = 0; e < E; ++e) offsets[e] = acc, acc += counts[e];
  int* fill = (int*)calloc((size_t)E, sizeof(int));
  for (int i = 0; i < n; ++i) slot_of[i] = offsets[idx[i]] + fill[idx[i]]++;
  free(fill);
  return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* dequantisation */

static inline float scale_val(const void* s, int kind, size_t i) {
  if (kind == OR_F32) return ((const float*)s)[i];
  const uint16_t h = ((const uint16_t*)s)[i];
  return kind == OR_BF16 ? or_bf16_to_f32(h) : or_f16_to_f32(h);
}

/* w = q * scale + min, per 64-group (tools/reference.py:29-35). */
static void row_q4(const uint8_t* q, const uint16_t* sm, int kind, size_t row, int K, float* w) {
  const uint8_t* qr = q + row * (size_t)(K / 2);
  const size_t g0 = row * (size_t)(K / 64);
  for (int k = 0; k < K; ++k) {
    const int nib = (k & 1) ? (qr[k >> 1] >> 4) : (qr[k >> 1] & 15);
    const size_t g = g0 + (size_t)(k / 64);
    const float sc = scale_val(sm, kind, 2 * g), mn = scale_val(sm, kind, 2 * g + 1);
    w[k] = (float)nib * sc + mn;
  }
}

static void row_q8(const int8_t* q, const uint16_t* s, int kind, int group, size_t row, int K, float* w) {
  const int8_t* qr = q + row * (size_t)K;
  const size_t g0 = row * (size_t)(K / group);
  for (int k = 0; k < K; ++k) w[k] = (float)qr[k] * scale_val(s, kind, g0 + (size_t)(k / group));
}

static void row_fp8(const uint8_t* w8, const void* s, int kind, size_t row, int K, float* w) {
  const uint8_t* r = w8 + row * (size_t)K;
  const size_t b0 = (row >> 7) * (size_t)(K / 128);
  for (int k = 0; k < K; ++k) w[k] = or_fp8e4m3_to_f32(r[k]) * scale_val(s, kind, b0 + (size_t)(k >> 7));
}

void or_dequant_q4(const uint8_t* q, const uint16_t* sm, int sm_kind, int N, int K, float* w) {
  for (int n = 0; n < N; ++n) row_q4(q, sm, sm_kind, (size_t)n, K, w + (size_t)n * K);
}

void or_dequant_q8(const int8_t* q, const uint16_t* s, int s_kind, int group, int N, int K, float* w) {
  for (int n = 0; n < N; ++n) row_q8(q, s, s_kind, group, (size_t)n, K, w + (size_t)n * K);
}

void or_dequant_fp8(const uint8_t* w8, const void* s, int s_kind, int N, int K, float* w) {
  for (int n = 0; n < N; ++n) row_fp8(w8, s, s_kind, (size_t)n, K, w + (size_t)n * K);
}

/* tools/convert.py:33-41 / src/convert/mod.rs:80-103: scale = f16(amax / 127) (>= 1e-12),
 * q = round-half-even(w / scale) clamped to +-127, one f16 scale per 128 inputs. */
void or_quant_q8(const float* w, int N, int K, int8_t* q, uint16_t* s) {
  for (int n = 0; n < N; ++n)
    for (int g = 0; g < K / 128; ++g) {
      const float* x = w + (size_t)n * K + g * 128;
      float amax = 0.f;
      for (int i = 0; i < 128; ++i) amax = fabsf(x[i]) > amax ? fabsf(x[i]) : amax;
      if (amax < 1e-12f) amax = 1e-12f;
      float sc = or_f16_to_f32(or_f32_to_f16(amax / 127.0f));
      if (sc < 1e-12f) sc = 1e-12f;
      for (int i = 0; i < 128; ++i) {
        float v = nearbyintf(x[i] / sc);
        v = v > 127.f ? 127.f : v < -127.f ? -127.f : v;
        q[(size_t)n * K + g * 128 + i] = (int8_t)v;
      }
      s[(size_t)n * (K / 128) + g] = or_f32_to_f16(sc);
    }
}

/* ------------------------------------------------------------------------------------------ */
/* value functions: dequantise, accumulate in double */

static double dotd(const float* w, const float* x, int K) {
  double s = 0.0;
  for (int k = 0; k < K; ++k) s += (double)w[k] * (double)x[k];
  return s;
}

static double silud(double g) { return g / (1.0 + exp(-g)); }
static double sigmoidd(double g) { return 1.0 / (1.0 + exp(-g)); }

void or_gemv_q4(const uint8_t* q, const uint16_t* sm, int sm_kind, const float* x, int N, int K, float* y) {
#pragma omp parallel
  {
    float* w = (float*)malloc(sizeof(float) * (size_t)K);
#pragma omp for schedule(static)
    for (int n = 0; n < N; ++n) {
      row_q4(q, sm, sm_kind, (size_t)n, K, w);
      y[n] = (float)dotd(w, x, K);
    }
    free(w);
  }
}

void or_gemv_q8(const int8_t* q, const uint16_t* s, int s_kind, int group, const float* x, int N, int K,
                float* y) {
#pragma omp parallel
  {
    float* w = (float*)malloc(sizeof(float) * (size_t)K);
#pragma omp for schedule(static)
    for (int n = 0; n < N; ++n) {
      row_q8(q, s, s_kind, group, (size_t)n, K, w);
      y[n] = (float)dotd(w, x, K);
    }
    free(w);
  }
}

/* Row `row` of routed expert e of a [E, N, K] weight, dequantised. */
static void expert_row(const or_moe_weights* W, int which_down, int e, int row, int N, int K, float* out) {
  const uint8_t* q = which_down ? W->d_q : W->gu_q;
  const void* s = which_down ? W->d_s : W->gu_s;
  if (W->kind == 0) {
    row_q4(q + (size_t)e * N * (K / 2), (const uint16_t*)s + (size_t)e * N * (K / 64) * 2, W->sc_kind,
           (size_t)row, K, out);
  } else {
    const size_t so = (size_t)e * (N / 128) * (K / 128);
    const void* se = W->sc_kind == OR_F32 ? (const void*)((const float*)s + so)
                                          : (const void*)((const uint16_t*)s + so);
    row_fp8(q + (size_t)e * N * K, se, W->sc_kind, (size_t)row, K, out);
  }
}

/* One decode token (kernels/drama.cu:470-599, tools/reference.py:331-351):
 *   xn = rmsnorm(x) (or x), act[k][j] = silu(G_e[j] xn) * (U_e[j] xn) for e = idx[k],
 *   act[topk][j] the same with the int8 shared expert,
 *   y[n] = res[n] + sigmoid(sgate) * (SD[n] act[topk]) + sum_k wts[k] (D_e[n] act[k]).
 * act keeps fp32 values as the GPU does.  y may alias x and res. */
int or_moe_decode(const or_moe_weights* W, const float* x, const int* idx, const float* wts,
                  const float* sgate, const float* res, float* act, float* y, int H, int I, int topk,
                  const float* nw, float eps) {
  float* xn = (float*)malloc(sizeof(float) * (size_t)H);
  or_rmsnorm_canon(x, nw, eps, H, xn);
#pragma omp parallel
  {
    float* wg = (float*)malloc(sizeof(float) * (size_t)H);
    float* wu = (float*)malloc(sizeof(float) * (size_t)H);
#pragma omp for schedule(static) collapse(2)
    for (int k = 0; k <= topk; ++k)
      for (int j = 0; j < I; ++j) {
        if (k < topk) {
          expert_row(W, 0, idx[k], j, 2 * I, H, wg);
          expert_row(W, 0, idx[k], I + j, 2 * I, H, wu);
        } else {
          row_q8(W->sgu_q, W->sgu_s, W->sh_kind, W->sh_group_gu, (size_t)j, H, wg);
          row_q8(W->sgu_q, W->sgu_s, W->sh_kind, W->sh_group_gu, (size_t)(I + j), H, wu);
        }
        const double g = dotd(wg, xn, H), u = dotd(wu, xn, H);
        act[(size_t)k * I + j] = (float)(silud(g) * u);
      }
    free(wg);
    free(wu);
  }
  free(xn);
  float* out = (float*)malloc(sizeof(float) * (size_t)H);
  const double sg = sigmoidd((double)sgate[0]);
#pragma omp parallel
  {
    float* wd = (float*)malloc(sizeof(float) * (size_t)I);
#pragma omp for schedule(static)
    for (int n = 0; n < H; ++n) {
      row_q8(W->sd_q, W->sd_s, W->sh_kind, W->sh_group_d, (size_t)n, I, wd);
      double acc = sg * dotd(wd, act + (size_t)topk * I, I);
      for (int k = 0; k < topk; ++k) {
        expert_row(W, 1, idx[k], n, H, I, wd);
        acc += (double)wts[k] * dotd(wd, act + (size_t)k * I, I);
      }
      out[n] = (float)((double)res[n] + acc);
    }
    free(wd);
  }
  memcpy(y, out, sizeof(float) * (size_t)H);
  free(out);
  return 0;
}

/* Routed + shared MoE output (without residual) for `rows` already-normalised fp32 rows,
 * keeping act in fp32: the batched form of or_moe_decode. */
int or_moe_decode_rows(const or_moe_weights* W, const float* xn_rows, int rows, const int* idx,
                       const float* wts, const float* sgate, float* y, int H, int I, int topk) {
  float* act = (float*)malloc(sizeof(float) * (size_t)(topk + 1) * I);
  float* zero = (float*)calloc((size_t)H, sizeof(float));
  for (int r = 0; r < rows; ++r) {
    or_moe_decode(W, xn_rows + (size_t)r * H, idx + (size_t)r * topk, wts + (size_t)r * topk, sgate + r,
                  zero, act, y + (size_t)r * H, H, I, topk, NULL, 0.f);
  }
  free(zero);
  free(act);
  return 0;
}

/* dr_moe_prefill semantics (kernels/drama.cu:799-968): for each expert e and each slot t in
 * [offsets[e], offsets[e] + counts[e]): act[t] = bf16(silu(G_e xp[t]) * (U_e xp[t])),
 * yp[t] = D_e act[t] (fp32). */
int or_moe_prefill_experts(const or_moe_weights* W, const uint16_t* xp, const int* offsets,
                           const int* counts, int E, uint16_t* act, float* yp, int H, int I) {
  for (int e = 0; e < E; ++e) {
    const int cnt = counts[e], off = offsets[e];
    if (cnt == 0) continue;
#pragma omp parallel
    {
      float* w = (float*)malloc(sizeof(float) * (size_t)H);
      float* x = (float*)malloc(sizeof(float) * (size_t)H * cnt);
      float* a = (float*)malloc(sizeof(float) * (size_t)I * cnt);
      for (int t = 0; t < cnt; ++t)
        for (int k = 0; k < H; ++k) x[(size_t)t * H + k] = or_bf16_to_f32(xp[(size_t)(off + t) * H + k]);
      double* g = (double*)malloc(sizeof(double) * (size_t)cnt);
#pragma omp for schedule(static)
      for (int j = 0; j < I; ++j) {
        expert_row(W, 0, e, j, 2 * I, H, w);
        for (int t = 0; t < cnt; ++t) g[t] = dotd(w, x + (size_t)t * H, H);
        expert_row(W, 0, e, I + j, 2 * I, H, w);
        for (int t = 0; t < cnt; ++t) {
          const double u = dotd(w, x + (size_t)t * H, H);
          act[(size_t)(off + t) * I + j] = or_f32_to_bf16((float)(silud(g[t]) * u));
        }
      }
      /* implicit barrier: act complete before down */
      for (int t = 0; t < cnt; ++t)
        for (int j = 0; j < I; ++j) a[(size_t)t * I + j] = or_bf16_to_f32(act[(size_t)(off + t) * I + j]);
#pragma omp for schedule(static)
      for (int n = 0; n < H; ++n) {
        expert_row(W, 1, e, n, H, I, w);
        for (int t = 0; t < cnt; ++t) yp[(size_t)(off + t) * H + n] = (float)dotd(w, a + (size_t)t * I, I);
      }
      free(g);
      free(a);
      free(x);
      free(w);
    }
  }
  return 0;
}

/* Prefill shared expert (src/engine.rs:560-562): act = bf16(silu(SG hn) * (SU hn)),
 * out = SD act in fp32.  The weights are used exactly dequantised (the reference rounds the
 * dequantised int8 weights to bf16 before its GEMM; this restatement does not). */
int or_shared_prefill(const or_moe_weights* W, const uint16_t* hn_b, int rows, uint16_t* act, float* out,
                      int H, int I) {
#pragma omp parallel
  {
    float* wg = (float*)malloc(sizeof(float) * (size_t)H);
    float* wu = (float*)malloc(sizeof(float) * (size_t)H);
    float* x = (float*)malloc(sizeof(float) * (size_t)H);
#pragma omp for schedule(static)
    for (int r = 0; r < rows; ++r) {
      for (int k = 0; k < H; ++k) x[k] = or_bf16_to_f32(hn_b[(size_t)r * H + k]);
      for (int j = 0; j < I; ++j) {
        row_q8(W->sgu_q, W->sgu_s, W->sh_kind, W->sh_group_gu, (size_t)j, H, wg);
        row_q8(W->sgu_q, W->sgu_s, W->sh_kind, W->sh_group_gu, (size_t)(I + j), H, wu);
        const double g = dotd(wg, x, H), u = dotd(wu, x, H);
        act[(size_t)r * I + j] = or_f32_to_bf16((float)(silud(g) * u));
      }
    }
#pragma omp barrier
#pragma omp for schedule(static)
    for (int r = 0; r < rows; ++r) {
      float* a = x;
      for (int j = 0; j < I; ++j) a[j] = or_bf16_to_f32(act[(size_t)r * I + j]);
      for (int n = 0; n < H; ++n) {
        row_q8(W->sd_q, W->sd_s, W->sh_kind, W->sh_group_d, (size_t)n, I, wg);
        out[(size_t)r * H + n] = (float)dotd(wg, a, I);
      }
    }
    free(x);
    free(wu);
    free(wg);
  }
  return 0;
}

/* Engine::moe_prefill (src/engine.rs:544-604) over `rows` bf16 normalised rows hn_b, with the
 * routing already computed (idx/wts/sgate, e.g. by or_moe_topk on or_router_logits_rows):
 * x[r] += sigmoid(sgate[r]) * shared[r] + sum_k wts[r, k] * yp[slot_of[r, k]]. */
int or_moe_prefill_layer(const or_moe_weights* W, const uint16_t* hn_b, int rows, const int* idx,
                         const float* wts, const float* sgate, float* x, int H, int I, int topk) {
  const int n = rows * topk;
  const int E = 256;
  int* counts = (int*)malloc(sizeof(int) * E);
  int* offsets = (int*)malloc(sizeof(int) * E);
  int* slot_of = (int*)malloc(sizeof(int) * (size_t)n);
  int rc = or_moe_group(idx, n, E, counts, offsets, slot_of);
  if (rc) {
    free(counts), free(offsets), free(slot_of);
    return rc;
  }
  uint16_t* xp = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)n * H);
  for (int i = 0; i < n; ++i) memcpy(xp + (size_t)slot_of[i] * H, hn_b + (size_t)(i / topk) * H, 2 * (size_t)H);
  uint16_t* act = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)n * I);
  float* yp = (float*)malloc(sizeof(float) * (size_t)n * H);
  or_moe_prefill_experts(W, xp, offsets, counts, E, act, yp, H, I);
  uint16_t* sact = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)rows * I);
  float* sh = (float*)malloc(sizeof(float) * (size_t)rows * H);
  or_shared_prefill(W, hn_b, rows, sact, sh, H, I);
  for (int r = 0; r < rows; ++r) {
    const double sg = sigmoidd((double)sgate[r]);
    for (int c = 0; c < H; ++c) {
      double acc = sg * sh[(size_t)r * H + c];
      for (int k = 0; k < topk; ++k)
        acc += (double)wts[r * topk + k] * yp[(size_t)slot_of[r * topk + k] * H + c];
      x[(size_t)r * H + c] = (float)((double)x[(size_t)r * H + c] + acc);
    }
  }
  free(sh), free(sact), free(yp), free(act), free(xp), free(counts), free(offsets), free(slot_of);
  return 0;
}

int or_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void or_set_threads(int n) {
#ifdef _OPENMP
  omp_set_num_threads(n);
#else
  (void)n;
#endif
}

// Canonical fp32 router arithmetic shared by the router kernels and the fused decode step
// (reference semantics: kernels/drama.cu:178-200,317-461).
//
// Every function fixes its operation order, so the CPU oracle reproduces logits, softmax
// probabilities and therefore the selected experts bit for bit:
//   RMSNorm  lane l accumulates x^2 over float4 indices l + 64 j with fmaf, 64-lane xor
//            butterfly, t = ss * (1 / K) + eps, inv = canon_rsqrt(t), xn = (x * inv) * nw
//   dot      lane l owns 8-element chunks l + 64 j, fmaf in element order, xor butterfly
//   top-k    k rounds of (logit desc, index asc), NaN logits last (the logit order is the
//            probability order; selecting on logits needs no exp or division per expert)
//   softmax  m = max logit, ex = exp(l - m) with canon_exp, lane l sums experts l + 64 j in
//            order, xor butterfly = z; p_k = ex_k / z (correctly rounded) for the picks;
//            total = sum of picked p in pick order; wts = p / total
// No expression in here may be contracted into an fma: every body switches contraction off
// and no header math helper is used.
#pragma once
#include "common.hpp"

namespace drm {

// exp: Cody-Waite reduction with k = rint(x log2 e), ln 2 split in a 16-bit head and a tail,
// degree-8 Taylor polynomial of e^r in Horner form with fma, scaling by 2^k through the
// exponent field.  Inputs below -86.5 give 0 and above 88 give +inf, so no subnormal result
// is ever formed.  Accuracy: within 2 ulp of exp on the range that matters (x <= 0).
DEV float canon_exp(float x) {
#pragma clang fp contract(off)
  if (x != x) return x;
  if (x < -86.5f) return 0.0f;
  if (x > 88.0f) return __builtin_inff();
  const float k = __builtin_rintf(x * 1.44269504088896341f);
  float r = __builtin_fmaf(-k, 0.693145751953125f, x);
  r = __builtin_fmaf(-k, 1.428606765330187e-06f, r);
  float p = 2.48015873e-05f;
  p = __builtin_fmaf(p, r, 1.98412698e-04f);
  p = __builtin_fmaf(p, r, 1.38888889e-03f);
  p = __builtin_fmaf(p, r, 8.33333333e-03f);
  p = __builtin_fmaf(p, r, 4.16666667e-02f);
  p = __builtin_fmaf(p, r, 1.66666667e-01f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const int ki = (int)k;
  return p * __uint_as_float((uint32_t)(ki + 127) << 23);
}

// 1 / sqrt(t) for t > 0 from plain multiplies and subtractions only, so every step rounds
// the same way on any IEEE machine: seed from the exponent/mantissa bit pattern
// (0x5f3759df - bits / 2), then three Newton steps y = y * (1.5 - (0.5 t) * (y * y)).
// Relative error <= 2e-7.
DEV float canon_rsqrt(float t) {
#pragma clang fp contract(off)
  float y = __uint_as_float(0x5f3759dfu - (__float_as_uint(t) >> 1));
  const float h = 0.5f * t;
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const float yy = y * y;
    const float hyy = h * yy;
    const float c = 1.5f - hyy;
    y = y * c;
  }
  return y;
}

// Canonical RMSNorm scale from the lane's float4 values xr[j] = x4[lane + 64 j], j < NRM
// (K = 256 NRM); every lane gets the same bits.
template <int NRM>
DEV float canon_rms_inv_regs(const float4 (&xr)[NRM], float eps) {
#pragma clang fp contract(off)
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NRM; ++j) {
    ss = __builtin_fmaf(xr[j].x, xr[j].x, ss);
    ss = __builtin_fmaf(xr[j].y, xr[j].y, ss);
    ss = __builtin_fmaf(xr[j].z, xr[j].z, ss);
    ss = __builtin_fmaf(xr[j].w, xr[j].w, ss);
  }
  ss = wave_sum(ss);
  const float t = ss * (1.0f / (float)(NRM * 256)) + eps;
  return canon_rsqrt(t);
}

// xn = (x * inv) * nw, element by element
DEV float4 canon_norm4(float4 a, float inv, float4 n) {
#pragma clang fp contract(off)
  return make_float4((a.x * inv) * n.x, (a.y * inv) * n.y, (a.z * inv) * n.z, (a.w * inv) * n.w);
}

// One logit row: w[j] = the row's bf16 chunk lane + 64 j, (a[j], b[j]) = the matching 8
// normalised inputs.  Returns the wave total (same bits on every lane).
template <int NCH>
DEV float canon_row_dot(const uint4 (&w)[NCH], const float4 (&a)[NCH], const float4 (&b)[NCH]) {
#pragma clang fp contract(off)
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    acc = __builtin_fmaf(bf16_lo(w[j].x), a[j].x, acc);
    acc = __builtin_fmaf(bf16_hi(w[j].x), a[j].y, acc);
    acc = __builtin_fmaf(bf16_lo(w[j].y), a[j].z, acc);
    acc = __builtin_fmaf(bf16_hi(w[j].y), a[j].w, acc);
    acc = __builtin_fmaf(bf16_lo(w[j].z), b[j].x, acc);
    acc = __builtin_fmaf(bf16_hi(w[j].z), b[j].y, acc);
    acc = __builtin_fmaf(bf16_lo(w[j].w), b[j].z, acc);
    acc = __builtin_fmaf(bf16_hi(w[j].w), b[j].w, acc);
  }
  return wave_sum(acc);
}

// Top-k selection key of a logit: an int whose order is the float order of the logit
// (negative values have their magnitude bits flipped, so -0 sorts just below +0); a NaN
// logit gets KEY_NAN, below every number; picked experts KEY_PICKED, padding KEY_PAD.
constexpr int KEY_PAD = -2147483647 - 1, KEY_PICKED = KEY_PAD + 1, KEY_NAN = KEY_PAD + 2;
DEV int canon_logit_key(float v) {
  const int i = __float_as_int(v);
  return v != v ? KEY_NAN : (i >= 0 ? i : i ^ 0x7fffffff);
}

template <int O>
DEV int xmax_step_i(int v) {
  float a, b;
  xchg<O>(__int_as_float(v), a, b);
  return max(__float_as_int(a), __float_as_int(b));
}
DEV int wave_max_i(int v) {
  v = xmax_step_i<1>(v);
  v = xmax_step_i<2>(v);
  v = xmax_step_i<4>(v);
  v = xmax_step_i<8>(v);
  v = xmax_step_i<16>(v);
  return xmax_step_i<32>(v);
}

// Top-k selection over E <= 256 logits by one wave: k rounds of (logit desc, index asc)
// on canon_logit_key.  Lane k < topk receives the expert of pick k.  Expert e = 4 lane + j
// lives in lane e / 4, so among equal keys the lowest index is in the lowest lane holding the
// key, and within a lane in the lowest slot.  Each lane first sorts its four (key, slot) pairs
// by (key desc, slot asc); a round then takes the wave maximum of the lane heads, the lowest
// lane whose head equals it wins, and that lane drops its head (KEY_PICKED moves in behind).
// Every pick is a distinct expert below E.
DEV int canon_select_topk(const float* __restrict__ l, int E, int topk) {
  const int lane = lane_id();
  int key[4], slot[4] = {0, 1, 2, 3};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = 4 * lane + j;
    key[j] = e < E ? canon_logit_key(l[e]) : KEY_PAD;
  }
  auto cex = [&](int a, int b) {
    const bool sw = key[b] > key[a] || (key[b] == key[a] && slot[b] < slot[a]);
    const int ka = key[a], kb = key[b], sa = slot[a], sb = slot[b];
    key[a] = sw ? kb : ka, key[b] = sw ? ka : kb;
    slot[a] = sw ? sb : sa, slot[b] = sw ? sa : sb;
  };
  cex(0, 1), cex(2, 3), cex(0, 2), cex(1, 3), cex(1, 2);
  int slots = slot[0] | slot[1] << 2 | slot[2] << 4 | slot[3] << 6;  // slot order, 2 bits each
  int id = 0;
  for (int k = 0; k < topk; ++k) {
    const int kb = wave_max_i(key[0]);
    const int ls = (int)__builtin_ctzll(__ballot(key[0] == kb));
    const int js = __builtin_amdgcn_readlane(slots, ls) & 3;
    const bool win = lane == ls;
    key[0] = win ? key[1] : key[0];
    key[1] = win ? key[2] : key[1];
    key[2] = win ? key[3] : key[2];
    key[3] = win ? KEY_PICKED : key[3];
    slots = win ? slots >> 2 : slots;
    id = lane == k ? 4 * ls + js : id;
  }
  return id;
}

// The same selection in two phases for topk <= 8 and E <= 256, spread over four waves.
// Phase 1, wave w (w < 4): the top-8 of experts [64 w, 64 w + 64) (one per lane), in pick
// order; lane r < 8 returns pick r as (key, expert), candidate c = 8 w + r.  The top-k of the
// 32 candidates is the top-k of all E experts (each group contributes at most 8); phase 2,
// canon_merge_rank32, orders them.
DEV void canon_select_group8(const float* __restrict__ l, int E, int w, int* cand_key, int* cand_e) {
  const int lane = lane_id();
  const int e = 64 * w + lane;
  int key = e < E ? canon_logit_key(l[e]) : KEY_PAD;
  int ck = KEY_PAD, ce = 0;
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int kb = wave_max_i(key);
    const int ls = (int)__builtin_ctzll(__ballot(key == kb));
    if (lane == ls) key = KEY_PICKED;
    if (lane == r) ck = kb, ce = 64 * w + ls;
  }
  *cand_key = ck;
  *cand_e = ce;
}

// Candidate (key, expert) as one integer ordered like the selection: larger key first, lower
// expert first among equal keys.
DEV uint64_t canon_cand64(int key, int e) {
  return ((uint64_t)((uint32_t)key ^ 0x80000000u) << 32) | (uint32_t)(0xffffffffu - (uint32_t)e);
}
DEV int canon_cand64_expert(uint64_t c) { return (int)(0xffffffffu - (uint32_t)c); }

// Phase 2, the merge of the 32 candidates, computed as ranks without rounds: candidate c
// (held by lanes c and c + 32, c < 32) is pick #{d : cand[d] > cand[c]} in the canon_cand64
// order (key desc, expert asc), the order in which k rounds of "largest key, lowest slot
// among equals" would pick them: within a group equal keys are picked in index order and the
// groups are in index order, so a lower slot holds the lower expert.  Valid candidates are
// distinct experts, so their ranks are distinct; padding candidates may repeat an expert but
// rank behind at least topk valid ones whenever E >= topk.  Lanes c and c + 32 count 16
// candidates each; every lane returns the full rank of candidate lane % 32.  All 64 lanes
// must be active.
DEV int canon_merge_rank32(const uint64_t* __restrict__ cand) {
  const int lane = lane_id();
  const uint64_t me = cand[lane & 31];
  const uint64_t* h = cand + 16 * (lane >> 5);
  int c[4] = {0, 0, 0, 0};
#pragma unroll
  for (int j = 0; j < 16; ++j) c[j & 3] += h[j] > me;
  float a, b;
  xchg<32>(__int_as_float((c[0] + c[1]) + (c[2] + c[3])), a, b);
  return __float_as_int(a) + __float_as_int(b);
}

// Pick k < topk <= 8 of the 32 group candidates, by rank (canon_merge_rank32): the candidate
// of rank k is written to sel[k] and read back by lane k.  One wave, all lanes active.
DEV int merge_picks(const uint64_t* cand, int* sel, int topk) {
  const int lane = lane_id();
  const int rk = canon_merge_rank32(cand);
  if (lane < 32 && rk < topk) sel[rk] = canon_cand64_expert(cand[lane]);
  return lane < topk ? sel[lane] : 0;
}

// Softmax denominator: m = max of the non-NaN logits, z = sum of canon_exp(l - m) with lane
// l summing experts l + 64 j in order, then the xor butterfly.  Same bits on every lane.
DEV float canon_softmax_z(const float* __restrict__ l, int E, float* m_out) {
#pragma clang fp contract(off)
  const int lane = lane_id();
  float v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = lane + WAVE * j;
    v[j] = e < E ? l[e] : -__builtin_inff();
  }
  const float m = wave_max(fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])));
  float z = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = lane + WAVE * j;
    z = z + (e < E ? canon_exp(v[j] - m) : 0.f);
  }
  *m_out = m;
  return wave_sum(z);
}

// Renormalised weight of the pick held by this lane (lane k < topk holds pick k, logit lk):
// p_k = canon_exp(lk - m) / z, total = sum of p_k in pick order, w_k = p_k / total.
DEV float canon_topk_weight(float lk, float m, float z, int topk) {
#pragma clang fp contract(off)
  const float p = canon_exp(lk - m) / z;
  float total = 0.f;
  for (int k = 0; k < topk; ++k) total = total + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), k));
  return p / total;
}

// Softmax + top-k of one row by one wave; lane k < topk receives pick k and its weight.
DEV void canon_softmax_topk(const float* __restrict__ l, int E, int topk, int* my_idx, float* my_w) {
  const int id = canon_select_topk(l, E, topk);
  float m;
  const float z = canon_softmax_z(l, E, &m);
  *my_idx = id;
  *my_w = canon_topk_weight(l[lane_id() < topk ? id : 0], m, z, topk);
}

}  // namespace drm

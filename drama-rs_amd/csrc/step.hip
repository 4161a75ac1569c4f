// Fused batch-1 decode step: router, top-k, gate_up + SiLU*up, down + weighted combine and
// the int8 shared expert of n_layers MoE layers in ONE persistent launch, with int4 or
// block-FP8 routed experts.  It computes exactly what the engine's per-layer chain
// dr_router_topk -> dr_moe_decode (or dr_moe_decode_fp8) computes (reference:
// src/engine.rs:1001-1007 recording kernels/drama.cu:369-461,470-742 per layer), with routing
// bit-exact to the canonical router order of canon.hpp.
//
// Why one launch: a layer streams ~18 MB, 2.3 us at the HBM roofline, while each dependent
// launch costs ~1.5 us on MI355X before its first load issues.  Here 256 workgroups (one per
// CU, 8 waves each) stay resident for the whole step and hand data to each other through
// three all-to-all exchanges per layer: the 257 router logits, the 9 x 512 activations and
// the 2048-float residual stream.  Each exchange is a "low latency" slot array: every value
// travels in a 64-bit word with a tag (fp32 bits + 32-bit tag; by default the routed
// activations two fp32 per word, each rounded to 21 mantissa bits with a 2-bit phase in its
// two low mantissa bits, which halves the largest exchange), written with one cache-bypassing
// (device-scope) store and read with device-scope loads until every word carries the tag of
// the current phase.  A 64-bit access is single-copy atomic (and each 32-bit half of a packed
// activation word carries its own phase), so a reader never sees a value without its tag and
// no separate flag, fence or counter is needed: one memory hop per exchange.  Tags are epoch * 4096 + 3 layer + phase + 1, with the epoch read from sync[0] at
// launch and advanced by the launch's last act, so slots never need clearing between calls.
//
// Work map (g = global wave, 0..2047): router row g/8 on wave 0 of every block (row 256, the
// shared-expert gate, on block 0 wave 1); routed gate_up pairs j, j+1 of expert slot g/256
// with j = 2g mod 512; shared gate_up pair g/4 on waves 2 and 6; down output row g.  Every
// wave polls one eighth of each exchange.  A wave's loads return in order, so weight loads
// are placed where no poll has to wait for them: the routed gate_up and down rows right
// after top-k (needed next anyway), the next layer's router and shared gate_up rows right
// after the activation poll, so they stream in during the down phase and the exchanges.
//
// Every wait is bounded: after ~0.2 s without progress the block writes sync[1] = 1 and
// returns, and a launch that finds sync[1] != 0 returns at once, so the grid always drains.
#include <atomic>

#include "canon.hpp"
#include "drama_moe.h"

using namespace drm;

namespace {

constexpr int ST_H = 2048, ST_I = 512, ST_TOPK = 8, ST_MAXE = 256;
constexpr int ST_NB = 256, ST_WPB = 8, ST_NT = ST_WPB * 64, ST_NP = 8;  // every wave polls a share
constexpr uint32_t ST_TAG_STRIDE = 4096;
constexpr int ST_MAXL = (ST_TAG_STRIDE - 1) / 3;
// When each wave polls an exchange for the first time, in 10 ns ticks of s_memrealtime after
// a point every wave of the block passes together (so the waves that reach an exchange early,
// like the non-router waves at the logits, do not poll before the data can be there): the
// logits after the layer start, the activations after top-k, the residual after the
// activation barrier.  A poll that comes too early costs a whole extra round trip, and early
// polls slow the exchange for everybody; the offsets (kOffL, kOffAct, kOffX of the weight-format
// policies below) were measured on MI355X
// (configuration 3: 13.9 us/layer with per-wave delays counted from each wave's own arrival,
// 11.9 us/layer with these; 10 ticks earlier than the activation offset already costs 0.3 us).
constexpr uint32_t ST_DLY_ROUND = 15;  // between poll rounds (15: 9.93, 20: 9.95, 30: 10.5 us/layer); the first-poll offsets are per format
constexpr uint64_t ST_DEFER_SIBLING = 55;  // ticks after the layer start at which waves 4 and 5 begin the norm
constexpr uint64_t ST_TIMEOUT_TICKS = 20000000;  // default wait limit; s_memrealtime runs at 100 MHz: 0.2 s

// slot arrays (64-bit words) inside the caller's ll buffer
// The activation region holds the 4096 routed activations either one fp32 per word (A32) or
// two fp32 per word with the phase in their two low mantissa bits, then the 512 shared ones
// (one fp32 per word).
constexpr int LL_LOG = 0, LL_ACT = 264, LL_X = LL_ACT + ST_TOPK * ST_I + ST_I, LL_WORDS = LL_X + ST_H;
static_assert(LL_WORDS == DR_STEP_LL_WORDS, "slot layout");
static_assert(kErrStepTimeout == DR_ERR_STEP_TIMEOUT && kErrPrefillWait == DR_ERR_PREFILL_WAIT &&
                  kErrRouteWait == DR_ERR_ROUTE_WAIT,
              "error codes");

// Phase timestamps for development builds (-DST_TRACE): thread 0 of each block stores the
// 100 MHz clock at points 0..7, 9 and 11..14 of each layer (poll rounds at 8, 10 and 15) into
// words LL_WORDS.. of a larger ll buffer.
#ifdef ST_TRACE
#define ST_PUT(pt, v) \
  if (threadIdx.x == 0) ll[LL_WORDS + ((size_t)l * 16 + (pt)) * ST_NB + blockIdx.x] = (v)
#define ST_MARK(pt) ST_PUT(pt, __builtin_amdgcn_s_memrealtime())
#define ST_MARKW(pt, w) \
  if (threadIdx.x == 64 * (w)) ll[LL_WORDS + ((size_t)l * 16 + (pt)) * ST_NB + blockIdx.x] = __builtin_amdgcn_s_memrealtime()
#else
#define ST_MARKW(pt, w)
#define ST_PUT(pt, v)
#define ST_MARK(pt)
#endif

DEV void ll_put(uint64_t* p, float v, uint32_t tag) {
  __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
DEV uint64_t ll_get(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Two activations in one word, each an fp32 whose two low mantissa bits carry the phase t2:
// the value rounded to 21 mantissa bits (relative error <= 2^-22; infinities and NaNs are
// not rounded, and an infinity comes out as a NaN), then t2 in bits 0-1.  Every 32-bit half
// carries its own phase, so the word needs no single-copy atomicity beyond 32 bits.  t2 is
// the running count of layers of all launches on this ll / sync pair plus one, mod 4
// (sync[2] holds the count): a slot always holds the previous layer's value, whose t2 differs
// by one, or zero (t2 0) before the first call.
DEV uint32_t enc_t2(float v, uint32_t t2) {
  const uint32_t u = __float_as_uint(v);
  return (((u & 0x7f800000u) == 0x7f800000u ? u : u + 2u) & ~3u) | t2;
}
DEV void ll_put2(uint64_t* p, float a, float b, uint32_t t2) {
  const uint64_t w = ((uint64_t)enc_t2(b, t2) << 32) | (uint64_t)enc_t2(a, t2);
  __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
DEV float2 ll_val2(uint64_t w) {
  return make_float2(__uint_as_float((uint32_t)w & ~3u), __uint_as_float((uint32_t)(w >> 32) & ~3u));
}

DEV void wait_until(uint64_t t) {
  while (__builtin_amdgcn_s_memrealtime() < t) __builtin_amdgcn_s_sleep(1);
}
DEV void wait_ticks(uint32_t n) { wait_until(__builtin_amdgcn_s_memrealtime() + n); }

// LDS float4 slots: int4 rows give lane l the 32 inputs [32 l, 32 l + 32) -> slot i * 64 + l
DEV int slot_q4(int f) { return (f & ~511) + (f & 7) * 64 + ((f & 511) >> 3); }

// Wave share of an exchange: wave p of NP owns, in lane l, the words base[l + 64 r] of rows
// r = p + NP i, i < N.  It reads them first at s_memrealtime first_poll, reloads the words
// whose tag is not yet the phase's until all are current, then hands each to spec.store.  Returns the rounds taken, 0 after ~0.2 s (the
// caller aborts).
template <int N, int NP, class Spec>
DEV uint32_t poll_wave(const uint64_t* base, int p, const Spec& sp, uint32_t* sync, uint64_t first_poll,
                       uint64_t tmo) {
  const int lane = lane_id();
  wait_until(first_poll);
  const uint64_t* b = base + lane + 64 * p;
  uint64_t v[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int r = p + NP * i;
    v[i] = sp.valid(r, lane + 64 * r) ? ll_get(b + 64 * NP * i) : sp.ready(r);
  }
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  uint32_t it = 1;
  for (;; ++it) {
    bool good = true;
#pragma unroll
    for (int i = 0; i < N; ++i) good &= sp.ok(p + NP * i, v[i]);
    if (__ballot(!good) == 0) break;
    if ((it & 63) == 0 && __builtin_amdgcn_s_memrealtime() - t0 > tmo) {
      if (lane == 0) __hip_atomic_store(sync + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return 0;
    }
    wait_ticks(ST_DLY_ROUND);
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (!sp.ok(p + NP * i, v[i])) v[i] = ll_get(b + 64 * NP * i);
  }
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int r = p + NP * i;
    if (sp.valid(r, lane + 64 * r)) sp.store(r, lane + 64 * r, v[i]);
    sp.post(r, v[i]);  // whole wave
  }
  return it;
}

// one fp32 value per word: logits (words 0..E) and the residual stream (2048 words)
struct Spec32 {
  uint32_t tag;
  int n;
  float* dst;
  DEV bool valid(int, int w) const { return w < n; }
  DEV uint64_t ready(int) const { return (uint64_t)tag << 32; }
  DEV bool ok(int, uint64_t v) const { return (uint32_t)(v >> 32) == tag; }
  DEV void store(int, int w, uint64_t v) const { dst[w] = __uint_as_float((uint32_t)v); }
  DEV void post(int, uint64_t) const {}
};

// activations, routed then shared, stored into the down slots of the weight format F.
// A32: words 0..4095 hold routed element w (fp32, 32-bit tag), rows i < 64; otherwise words
// 0..2047 hold routed elements 2w (low half) and 2w + 1 (high half) with the in-band phase t2,
// rows i < 32.  The 512 shared elements follow, one fp32 per word (32-bit tag), in the last 8
// rows.
template <class F, bool A32>
struct SpecAct {
  static constexpr int kRouted = A32 ? 64 : 32, kRows = kRouted + 8, kSharedWord = kRouted * 64;
  uint32_t tag, t2;
  float* dst;   // as4 as floats
  float* sums;  // [0, 128): sums of the 32-element routed chunks (int4), [128, 192): of the 8-element shared chunks
  DEV bool valid(int r, int) const { return r < kRows; }
  DEV uint64_t ready(int i) const {
    return !A32 && i < kRouted ? ((uint64_t)t2 << 32) | t2 : (uint64_t)tag << 32;
  }
  DEV bool ok(int i, uint64_t v) const {
    return !A32 && i < kRouted ? (v & 0x300000003ull) == (((uint64_t)t2 << 32) | t2) : (uint32_t)(v >> 32) == tag;
  }
  DEV void store(int i, int w, uint64_t v) const {
    if (i < kRouted) {
      if constexpr (A32) {
        F::act_pair(dst, w >> 1)[w & 1] = __uint_as_float((uint32_t)v);
      } else {
        const float2 p = ll_val2(v);
        float* d = F::act_pair(dst, w);
        d[0] = p.x, d[1] = p.y;
      }
    } else {
      const int e = w - kSharedWord;
      dst[(1024 + ((e >> 2) & 1) * 64 + (e >> 3)) * 4 + (e & 3)] = __uint_as_float((uint32_t)v);
    }
  }
  // chunk sums for the down dots' min terms: an int4 routed chunk is 32 (A32) or 16
  // consecutive words (lanes) of one row, a shared chunk 8 consecutive words
  DEV void post(int r, uint64_t v) const {
    const int lane = lane_id();
    if (r < kRouted) {
      if constexpr (F::kMinTerm) {
        if constexpr (A32) {
          float t = __uint_as_float((uint32_t)v);
          t = xsum_step<1>(t), t = xsum_step<2>(t), t = xsum_step<4>(t), t = xsum_step<8>(t), t = xsum_step<16>(t);
          if ((lane & 31) == 0) sums[2 * r + (lane >> 5)] = t;
        } else {
          const float2 p = ll_val2(v);
          float t = p.x + p.y;
          t = xsum_step<1>(t), t = xsum_step<2>(t), t = xsum_step<4>(t), t = xsum_step<8>(t);
          if ((lane & 15) == 0) sums[4 * r + (lane >> 4)] = t;
        }
      }
    } else {
      float t = __uint_as_float((uint32_t)v);
      t = xsum_step<1>(t), t = xsum_step<2>(t), t = xsum_step<4>(t);
      if ((lane & 7) == 0) sums[128 + 8 * (r - kRouted) + (lane >> 3)] = t;
    }
  }
};

// Routed-expert weight formats of the step.  Each gives the lane slots of the normalised
// input (xslot), the two (gate, up) pairs rj, rj + 1 of one expert per wave (load_gu, then
// gate_up: the activations of both pairs), output row n of the 8 experts' down projections
// (load_dn, then down: the weighted sum of the 8 dots, without the shared expert) and where
// routed activation word w lands in the down slots (act_pair).
//
// int4 (scale, min) groups of 64: a 1024-byte gate_up row is one 16-byte load per lane,
// lane l holding inputs [32 l, 32 l + 32); a 256-byte down row is 16 chunks, lane l holding
// chunk l & 15 of experts l >> 4 and 4 + (l >> 4).
template <class SC>
struct StepQ4 {
  static constexpr bool kMinTerm = true;
  // gate_up loads issued straight from the merge's ranks, before the picks go through LDS
  // (10.87 -> 10.68 us/layer; the FP8 policy measured 11.2 -> 14.4 with it and keeps the LDS path)
  static constexpr bool kEarlyGu = true;
  // first-poll offsets (measured; kOffX: 195 -> 12.3, 215-235 -> 11.6-11.8, 285 -> 12.2 us/layer)
  // (kOffL: 185 before the router waves had their SIMDs to themselves; 115 -> 11.8, 130 -> 11.4,
  // 140-160 -> 11.15-11.2 us/layer)
  // (kOffX, with the in-band activation phase and kOffActIb 375-385: 175 -> 11.0, 185-195 -> 10.85-10.95,
  // 215 -> 11.1 us/layer)
  // (retuned after the start-up and exchange changes, as a grid over kOffX x kOffActIb: kOffX 150 ->
  // 10.44, 160-175 -> 10.02-10.07, 190 -> 10.23, 205 -> 10.39 us/layer; with kOffActIb 330: kOffX 165
  // -> 9.93-9.95; kOffActIb 310 -> 10.43, 320 -> 10.14, 330-340 -> 9.94-9.96, 360 -> 10.20)
  // (retuned for the integer-digit gate_up dots, whose pairs are done ~0.4 us sooner: kOffActIb 330 ->
  // 10.11, 310 -> 9.88, 290-300 -> 9.85 with kOffX 165, 9.68-9.70 with kOffX 180 (170 -> 9.75, 195 -> 9.84,
  // 210 -> 9.96); kOffL 125 -> 9.64, 130 -> 9.57, 135 -> 9.59, 140 -> 9.64, 155 -> 9.78 us/layer;
  // on a second box with kOffActIb 295: kOffX 180 -> 9.50-9.54, 172 -> 9.44-9.50, 165 -> 9.41-9.46,
  // 160 -> 9.41-9.43, the first box flat over 170-185: 165 sits inside both plateaus)
  static constexpr uint32_t kOffL = 130, kOffAct = 300, kOffX = 165;
  static constexpr uint32_t kOffXA32 = 235;  // residual offset with the full-fp32 activation exchange
                                             // (190 -> 11.95, 215 -> 11.6-11.7, 235 -> 11.5 us/layer)
  // with the in-band activation phase (measured: 330 -> 12.7, 355 -> 11.8, 370-380 -> 11.4,
  // 400 -> 11.5 us/layer); full-fp32 activations with the integer-digit dots: kOffAct 355 -> 11.06,
  // 340 -> 10.85, 320 -> 10.73, 300 -> 10.55-10.61, 285 -> 10.70, 270 -> 11.10 us/layer
  static constexpr uint32_t kOffActIb = 295;  // (335-350 with the early gate_up loads: 10.7 us/layer)
  DEV static int xslot(int f) { return slot_q4(f); }
  struct GU {
    uint4 wg[2], wu[2];
    uint32_t sg[2], su[2];
  };
  DEV static void load_gu(const dr_decode_layer& Ly, size_t ek, int rj, int lane, GU& g) {
    constexpr int H = ST_H, I = ST_I;
    const uint8_t* q = Ly.gu_q + ek * (2 * I) * (H / 2) + lane * 16;
    const uint32_t* sm = reinterpret_cast<const uint32_t*>(Ly.gu_s) + ek * (2 * I) * (H / 64) + (lane >> 1);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int j = rj + p;
      g.wg[p] = ld16(q + (size_t)j * (H / 2));
      g.wu[p] = ld16(q + (size_t)(I + j) * (H / 2));
      g.sg[p] = ld4(sm + (size_t)j * (H / 64));
      g.su[p] = ld4(sm + (size_t)(I + j) * (H / 64));
    }
  }
  // x of lane l's chunk as the fixed-point digits of q4_digits_stage (stage_xq): each weight
  // word is six exact v_dot8 sums, w x = s (q - 8) x + (m + 8 s) x
  DEV static void gate_up(const GU& g, const float4* xq4, const float* s_xsum, int lane, float (&av)[2]) {
    uint32_t dg[24];
    q4_digits_load(reinterpret_cast<const uint32_t*>(xq4), lane, dg);
    const float xsum = s_xsum[lane], xsc = s_xsum[64 + lane];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const float dgv = q4_dot_digits(g.wg[p], dg), duv = q4_dot_digits(g.wu[p], dg);
      const float2 a = SC::pair(g.sg[p]), b = SC::pair(g.su[p]);
      const float gv = wave_sum(a.x * (dgv * xsc) + __builtin_fmaf(8.f, a.x, a.y) * xsum);
      const float uv = wave_sum(b.x * (duv * xsc) + __builtin_fmaf(8.f, b.x, b.y) * xsum);
      av[p] = silu(gv) * uv;
    }
  }
  struct DN {
    uint4 qa, qb;
    uint32_t sa, sb;
  };
  DEV static void load_dn(const dr_decode_layer& Ly, int my_idx, int n, int lane, DN& d) {
    constexpr int H = ST_H, I = ST_I;
    const int ka = lane >> 4, cc = lane & 15;
    const size_t ea = (size_t)__shfl(my_idx, ka), eb = (size_t)__shfl(my_idx, 4 + ka);
    const uint32_t* dsm = reinterpret_cast<const uint32_t*>(Ly.d_s);
    d.qa = ld16(Ly.d_q + (ea * H + n) * (I / 2) + cc * 16);
    d.qb = ld16(Ly.d_q + (eb * H + n) * (I / 2) + cc * 16);
    d.sa = ld4(dsm + (ea * H + n) * (I / 64) + (cc >> 1));
    d.sb = ld4(dsm + (eb * H + n) * (I / 64) + (cc >> 1));
  }
  DEV static float down(const DN& d, const float4* as4, const float* s_asum, float my_w, int lane) {
    const int ka = lane >> 4;
    const float wa = __shfl(my_w, ka), wb = __shfl(my_w, 4 + ka);
    float xa[32], xb[32];
    const float suma = s_asum[lane], sumb = s_asum[64 + lane];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 v = as4[i * 64 + lane], w = as4[512 + i * 64 + lane];
      xa[4 * i] = v.x, xa[4 * i + 1] = v.y, xa[4 * i + 2] = v.z, xa[4 * i + 3] = v.w;
      xb[4 * i] = w.x, xb[4 * i + 1] = w.y, xb[4 * i + 2] = w.z, xb[4 * i + 3] = w.w;
    }
    float da = 0.f, db = 0.f;
    da = dot8_q4(d.qa.x, xa + 0, da), db = dot8_q4(d.qb.x, xb + 0, db);
    da = dot8_q4(d.qa.y, xa + 8, da), db = dot8_q4(d.qb.y, xb + 8, db);
    da = dot8_q4(d.qa.z, xa + 16, da), db = dot8_q4(d.qb.z, xb + 16, db);
    da = dot8_q4(d.qa.w, xa + 24, da), db = dot8_q4(d.qb.w, xb + 24, db);
    const float2 pa = SC::pair(d.sa), pb = SC::pair(d.sb);
    return wa * (pa.x * da + pa.y * suma) + wb * (pb.x * db + pb.y * sumb);
  }
  DEV static float* act_pair(float* as4f, int w) { return as4f + slot_q4(w >> 1) * 4 + (w & 1) * 2; }
};

// Block-FP8 (e4m3, one scale per 128 x 128 block, f32 for SF = 0, bf16 for SF = 1): a
// 2048-byte gate_up row is two 16-byte loads per lane (bytes [16 l, 16 l + 16) and
// [1024 + 16 l, ...), the int8 shared layout); a 512-byte down row is 32 chunks, lane l
// holding chunk l & 31 of experts 2 i + (l >> 5), i < 4.  Every 16-byte chunk lies in one
// scale block.
template <int SF>
struct StepFP8 {
  static constexpr bool kMinTerm = false;
  static constexpr bool kEarlyGu = false;
  // first-poll offsets (measured; kOffAct: twice the gate_up bytes of int4; kOffX: 165-175 ->
  // 11.4-11.6, 205 -> 12.0, 245 -> 12.3 us/layer)
  // (kOffL: 135-160 -> 11.36-11.41, 185 -> 11.66 us/layer)
  // (retuned with the int4 policy's changes: kOffActIb 445 -> 10.83, 485 -> 11.23 us/layer against 11.04
  // at 465; kOffL 135 -> 10.87, 165 -> 11.18; kOffX 140 -> 10.89, 170 -> 11.16; together kOffL 135,
  // kOffX 140, kOffActIb 430: 10.55-10.7; kOffX 125 -> 10.96, kOffL 120 with kOffX 125 -> 11.28)
  static constexpr uint32_t kOffL = 135, kOffAct = 430, kOffX = 140;
  static constexpr uint32_t kOffXA32 = 165;
  // in-band activation phase: 400 -> 12.6, 430 -> 11.8, 460-470 -> 11.7, 510 -> 12.0 us/layer
  static constexpr uint32_t kOffActIb = 430;
  DEV static int xslot(int f) { return (f & ~255) + (f & 3) * 64 + ((f & 255) >> 2); }
  struct GU {
    uint4 g[2][2], u[2][2];
    uint32_t sg[2][2], su[2][2];  // raw scale bits
  };
  DEV static void load_gu(const dr_decode_layer& Ly, size_t ek, int rj, int lane, GU& g) {
    constexpr int H = ST_H, I = ST_I;
    const uint8_t* w = Ly.gu_q + ek * (2 * I) * H + lane * 16;
    const size_t sb = ek * (size_t)(2 * I / 128) * (H / 128) + (lane >> 3);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int j = rj + p;
      g.g[p][0] = ld16(w + (size_t)j * H), g.g[p][1] = ld16(w + (size_t)j * H + 1024);
      g.u[p][0] = ld16(w + (size_t)(I + j) * H), g.u[p][1] = ld16(w + (size_t)(I + j) * H + 1024);
      g.sg[p][0] = blk_raw<SF>(Ly.gu_s, sb + (size_t)(j >> 7) * (H / 128));
      g.sg[p][1] = blk_raw<SF>(Ly.gu_s, sb + (size_t)(j >> 7) * (H / 128) + 8);
      g.su[p][0] = blk_raw<SF>(Ly.gu_s, sb + (size_t)((I + j) >> 7) * (H / 128));
      g.su[p][1] = blk_raw<SF>(Ly.gu_s, sb + (size_t)((I + j) >> 7) * (H / 128) + 8);
    }
  }
  DEV static void gate_up(const GU& g, const float4* xq4, const float*, int lane, float (&av)[2]) {
    float xa[16], xb[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 v = xq4[i * 64 + lane], w = xq4[256 + i * 64 + lane];
      xa[4 * i] = v.x, xa[4 * i + 1] = v.y, xa[4 * i + 2] = v.z, xa[4 * i + 3] = v.w;
      xb[4 * i] = w.x, xb[4 * i + 1] = w.y, xb[4 * i + 2] = w.z, xb[4 * i + 3] = w.w;
    }
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const float gv = wave_sum(blk_cvt<SF>(g.sg[p][0]) * dot16_fp8(g.g[p][0], xa, 0.f) +
                                blk_cvt<SF>(g.sg[p][1]) * dot16_fp8(g.g[p][1], xb, 0.f));
      const float uv = wave_sum(blk_cvt<SF>(g.su[p][0]) * dot16_fp8(g.u[p][0], xa, 0.f) +
                                blk_cvt<SF>(g.su[p][1]) * dot16_fp8(g.u[p][1], xb, 0.f));
      av[p] = silu(gv) * uv;
    }
  }
  struct DN {
    uint4 q[4];
    uint32_t sc[4];  // raw scale bits
  };
  DEV static void load_dn(const dr_decode_layer& Ly, int my_idx, int n, int lane, DN& d) {
    constexpr int H = ST_H, I = ST_I;
    const int half = lane >> 5, cc = lane & 31;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const size_t e = (size_t)__shfl(my_idx, 2 * i + half);
      d.q[i] = ld16(Ly.d_q + (e * H + n) * I + cc * 16);
      d.sc[i] = blk_raw<SF>(Ly.d_s, (e * (H / 128) + (n >> 7)) * (I / 128) + (cc >> 3));
    }
  }
  DEV static float down(const DN& d, const float4* as4, const float*, float my_w, int lane) {
    const int half = lane >> 5;
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float xa[16];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const float4 v = as4[256 * i + t * 64 + lane];
        xa[4 * t] = v.x, xa[4 * t + 1] = v.y, xa[4 * t + 2] = v.z, xa[4 * t + 3] = v.w;
      }
      acc += __shfl(my_w, 2 * i + half) * blk_cvt<SF>(d.sc[i]) * dot16_fp8(d.q[i], xa, 0.f);
    }
    return acc;
  }
  // routed element m (even) of expert slot k -> float 4 (256 (k >> 1) + 64 t + 32 (k & 1) + m / 16) + m % 4
  DEV static float* act_pair(float* as4f, int w) {
    const int k = w >> 8, m = 2 * (w & 255);
    return as4f + (256 * (k >> 1) + ((m & 15) >> 2) * 64 + (k & 1) * 32 + (m >> 4)) * 4 + (m & 3);
  }
};

struct RouterRow {
  uint4 w[4];
};
struct SharedPair {
  uint4 g0, g1, u0, u1;
  uint32_t sg0, sg1, su0, su1;  // raw scale bits (SH::cvt at use)
};

template <class SH>
DEV void load_shared_pair(const dr_decode_layer& Ly, int j, int lane, SharedPair& s) {
  constexpr int H = ST_H, I = ST_I;
  const int8_t* rg = Ly.sgu_q + (size_t)j * H + lane * 16;
  const int8_t* ru = Ly.sgu_q + (size_t)(I + j) * H + lane * 16;
  s.g0 = ld16(rg), s.g1 = ld16(rg + 1024), s.u0 = ld16(ru), s.u1 = ld16(ru + 1024);
  s.sg0 = SH::raw(Ly.sgu_s, j, lane * 16, H), s.sg1 = SH::raw(Ly.sgu_s, j, 1024 + lane * 16, H);
  s.su0 = SH::raw(Ly.sgu_s, I + j, lane * 16, H), s.su1 = SH::raw(Ly.sgu_s, I + j, 1024 + lane * 16, H);
}

template <class F, class SH, bool A32>
__global__ void __launch_bounds__(ST_NT, 1)
    k_decode_step(const dr_decode_layer* __restrict__ layers, int L, float* x, int E, float eps,
                  uint64_t* __restrict__ ll, uint32_t* __restrict__ sync, int* __restrict__ idx_out,
                  float* __restrict__ wts_out, float* __restrict__ sgate_out, float* __restrict__ xs_out,
                  uint32_t* __restrict__ err, uint64_t tmo, const char* __restrict__ pf, size_t pf_bytes) {
  constexpr int H = ST_H, I = ST_I;
  __shared__ float4 xr4[H / 4];                        // residual stream x (raw)
  __shared__ float4 nws[H / 4];                        // RMSNorm weight of the layer
  __shared__ float4 xq4[H / 4];                        // normalised x in the F::xslot lane slots
  __shared__ float4 as4[(ST_TOPK + 1) * I / 4];        // activations in the down lane slots
  __shared__ float lg[ST_MAXE + 1];
  __shared__ int s_sel[ST_WPB][ST_TOPK];  // every wave's copy of the picks
  __shared__ float s_asum[192];  // activation chunk sums (see SpecAct::post)
  __shared__ float s_xsum[128];  // int4: sums of the 32-input chunks of xn (lane l's chunk), then their 2^-S
  __shared__ uint64_t s_cand[32];  // per-group top 8 (canon_cand64)
  __shared__ int s_abort;
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  // A block that gives up (a bounded wait expired, or an earlier call did and sync was not
  // reset) poisons the whole output with NaN and raises DR_ERR_STEP_TIMEOUT, so a failed call
  // can never pass for a result.
  auto give_up = [&]() {
    const float q = __builtin_nanf("");
    reinterpret_cast<float4*>(x)[tid] = make_float4(q, q, q, q);
    if (tid == 0) raise_err(err, kErrStepTimeout);
  };
  // Start-up: the loads that need nothing else go out at once (the sync words, x, the first
  // layer's record), the first layer's weights as soon as its record is in, and whether an
  // earlier call gave up is checked only at the start-up barrier: a launch pays one dependent
  // round trip (record, then weights) before its first layer, not three (sync word, barrier,
  // record, weights; measured: first layer starts 2.75 -> 2.5 us after the launch's first wave,
  // one-layer launches 13.0 -> 12.75 us)
  const uint32_t gave_up = __hip_atomic_load(sync + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const float4 xv = reinterpret_cast<const float4*>(x)[tid];
  const int pw = wave;  // every wave polls rows pw + 8 i of each exchange
  const bool poller = true;
  const int g = blockIdx.x * ST_WPB + wave;
  const uint32_t epoch = __hip_atomic_load(sync, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint32_t tag0 = epoch * ST_TAG_STRIDE + 1;
  const uint32_t lbase_in = __hip_atomic_load(sync + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // sync[3]: the activation transport of the previous launch on this ll / sync pair (0 none, 1
  // packed, 2 fp32 with tags).  After the other transport, words that launch left in the packed
  // routed slots could pass for current ones (a tagged word's tag and value bits can carry the
  // phase), so this launch clears those slots before its first exchange and restarts the phase
  // count at a multiple of 4: the first layer's phase is then 1, which no cleared word carries.
  constexpr uint32_t kTransport = A32 ? 2u : 1u;
  const uint32_t prev_transport = __hip_atomic_load(sync + 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const bool switched = prev_transport != 0 && prev_transport != kTransport;
  const uint32_t lbase = switched ? (lbase_in + 3u) & ~3u : lbase_in;

  const bool is_router = (wave == 0 && (int)blockIdx.x <= E) || (wave == 1 && blockIdx.x == 0 && E == ST_MAXE);
  const int rrow = wave == 0 ? (int)blockIdx.x : ST_MAXE;
  const bool is_shared = (wave & 3) == 2;
  const int sj = g >> 2;               // shared gate_up pair
  const int rk = g >> 8;               // routed expert slot of the gate_up pairs
  const int rj = (2 * g) & (I - 1);    // first of the two gate_up pairs
  const int n = g;                     // down output row

  RouterRow rw;
  SharedPair sp;
  float4 nwv = make_float4(1.f, 1.f, 1.f, 1.f);
  if (tid == 0) s_abort = 0;
  // layer records travel in scalar registers (read with scalar loads a layer ahead): staged
  // in LDS or read through a generic pointer they would turn every weight load into a flat
  // load, whose waits also drain the LDS counter
  dr_decode_layer Ly = layers[0];
  {
    const dr_decode_layer& L0 = Ly;
    if (is_router) {
      const uint16_t* wr = L0.router + (size_t)rrow * H;
#pragma unroll
      for (int j = 0; j < 4; ++j) rw.w[j] = ld16(wr + (size_t)(lane + 64 * j) * 8);
    }
    if (is_shared) load_shared_pair<SH>(L0, sj, lane, sp);
    if (L0.nw) nwv = ldf4(L0.nw + 4 * tid);
    nws[tid] = nwv;
    xr4[tid] = xv;
  }
  if (switched && tid < 2048 / ST_NB) {
    // complete before the start-up barrier, so before this block's first logit is published:
    // every block reads all logits before any activation is published or polled
    __hip_atomic_store(ll + LL_ACT + blockIdx.x * (2048 / ST_NB) + tid, 0ull, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  }
  if (__syncthreads_or(gave_up != 0)) {
    give_up();
    return;
  }

  dr_decode_layer Ln = Ly;
  for (int l = 0; l < L; ++l) {
    const uint32_t tA = tag0 + 3 * l, tB = tA + 1, tC = tA + 2, t2 = (lbase + l + 1) & 3u;
    ST_MARK(0);
    const uint64_t t_layer = __builtin_amdgcn_s_memrealtime();
    float res;  // x[n], read now: the poller overwrites xr4 during the down phase

    // ---- RMSNorm (canonical, every wave) and the router row; the poller collects logits
    {
      res = reinterpret_cast<const float*>(xr4)[n];
      // waves 4 and 5 share SIMDs 0 and 1 with the router waves (wave 0, and wave 1 of block 0):
      // they start their norm once the router rows are out (measured: the logits can then be
      // polled 0.4 us earlier, 11.5 -> 11.15 us/layer)
      if (wave == 4 || wave == 5) wait_until(t_layer + ST_DEFER_SIBLING);
      float4 xr[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) xr[j] = xr4[lane + 64 * j];
      const float inv = Ly.nw ? canon_rms_inv_regs<8>(xr, eps) : 1.f;
      // this thread's part of the normalised x as gate_up reads it (int4: the chunk sums, scales
      // and fixed-point digits; FP8: the floats in their lane slots); the router waves do it after
      // their router row
      auto stage_xq = [&]() {
        const float4 xn = canon_norm4(xr4[tid], inv, nwv);
        if constexpr (!F::kMinTerm) xq4[F::xslot(tid)] = xn;
        if constexpr (F::kMinTerm)  // threads 8c .. 8c + 7 hold chunk c
          q4_digits_stage(xn, tid >> 3, tid & 7, reinterpret_cast<uint32_t*>(xq4), s_xsum, s_xsum + 64);
      };
      if (!is_router) stage_xq();
      if (is_router) {
        float4 a[4], b[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int c = lane + 64 * j;
          a[j] = canon_norm4(xr4[2 * c], inv, nws[2 * c]);
          b[j] = canon_norm4(xr4[2 * c + 1], inv, nws[2 * c + 1]);
        }
        const float acc = canon_row_dot<4>(rw.w, a, b);
        if (lane == 0) ll_put(ll + LL_LOG + rrow, acc, tA);
        stage_xq();
      }
      // shared gate_up pair (waves 2 and 6): needs only the normalised x, so it runs here,
      // inside the logits exchange, instead of after top-k
      if (is_shared) {
        float xa[16], xb[16], sa = 0.f, sb = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int f = 4 * lane + i;
          const float4 v = canon_norm4(xr4[f], inv, nws[f]), w = canon_norm4(xr4[256 + f], inv, nws[256 + f]);
          xa[4 * i] = v.x, xa[4 * i + 1] = v.y, xa[4 * i + 2] = v.z, xa[4 * i + 3] = v.w;
          xb[4 * i] = w.x, xb[4 * i + 1] = w.y, xb[4 * i + 2] = w.z, xb[4 * i + 3] = w.w;
          sa += (v.x + v.y) + (v.z + v.w);
          sb += (w.x + w.y) + (w.z + w.w);
        }
        float ga = 0.f, gb = 0.f, ua = 0.f, ub = 0.f;
        const uint32_t gw0[4] = {sp.g0.x, sp.g0.y, sp.g0.z, sp.g0.w}, gw1[4] = {sp.g1.x, sp.g1.y, sp.g1.z, sp.g1.w};
        const uint32_t uw0[4] = {sp.u0.x, sp.u0.y, sp.u0.z, sp.u0.w}, uw1[4] = {sp.u1.x, sp.u1.y, sp.u1.z, sp.u1.w};
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          ga = dot4_u8b(gw0[d], xa + 4 * d, ga), gb = dot4_u8b(gw1[d], xb + 4 * d, gb);
          ua = dot4_u8b(uw0[d], xa + 4 * d, ua), ub = dot4_u8b(uw1[d], xb + 4 * d, ub);
        }
        const float gv = wave_sum(SH::cvt(sp.sg0) * (ga - 128.f * sa) + SH::cvt(sp.sg1) * (gb - 128.f * sb));
        const float uv = wave_sum(SH::cvt(sp.su0) * (ua - 128.f * sa) + SH::cvt(sp.su1) * (ub - 128.f * sb));
        if (lane == 0) ll_put(ll + LL_ACT + SpecAct<F, A32>::kSharedWord + sj, silu(gv) * uv, tB);
      }
      ST_MARK(1);
    }
    if (poller) {
      const uint32_t r = poll_wave<1, ST_NP>(ll + LL_LOG, pw, Spec32{tA, E + 1, lg}, sync, t_layer + F::kOffL, tmo);
      if (!r && lane == 0) s_abort = 1;
      ST_PUT(8, r);
    }
    // ---- top-k, first half: wave w < 4 has just polled (and stored) the logits of experts
    // [64 w, 64 w + 64), so it selects their top 8 before the barrier
    if (wave < 4) {
      int ck, ce;
      canon_select_group8(lg, E, wave, &ck, &ce);
      if (lane < 8) s_cand[wave * 8 + lane] = canon_cand64(ck, ce);
    }
    __syncthreads();
    ST_MARK(2);
    if (s_abort) {
      give_up();
      return;
    }

    // ---- top-k, second half: the 32 candidates ranked by every wave (no second barrier);
    // lane k < 8 of each wave's s_sel row receives pick k
    typename F::GU gu;
    int my_idx;
    {
      const int rk8 = canon_merge_rank32(s_cand);
      const int my_e = canon_cand64_expert(s_cand[lane & 31]);
      // the next layer's record: a scalar load, issued ahead of the gate_up loads (behind them
      // its return, which the LDS reads below wait for too, queues behind the weight stream);
      // read at the activation barrier it would cost a round trip on the way to the residual
      // publish, and at the layer start its wait would hold up the router's LDS reads
      Ln = layers[l + 1 < L ? l + 1 : l];
      if constexpr (F::kEarlyGu) {
        // ---- routed weight loads: gate_up pairs of expert slot rk, whose expert the lane
        // holding the candidate of rank rk hands over (no LDS round trip before the loads)
        const uint64_t hit = __ballot(lane < 32 && rk8 == rk);
        const size_t ek = (size_t)__builtin_amdgcn_readlane(my_e, hit ? (int)__builtin_ctzll(hit) : 0);
        F::load_gu(Ly, ek, rj, lane, gu);
      }
      if (lane < 32 && rk8 < ST_TOPK) s_sel[wave][rk8] = my_e;
      my_idx = s_sel[wave][lane & (ST_TOPK - 1)];
    }

    {
      ST_MARK(3);
      const uint64_t t_topk = __builtin_amdgcn_s_memrealtime();
      if constexpr (!F::kEarlyGu) F::load_gu(Ly, (size_t)__builtin_amdgcn_readlane(my_idx, rk), rj, lane, gu);
      // routing weights, needed only by the down phase: every wave computes the softmax
      // denominator and its pick weights while its gate_up loads are in flight
      __builtin_amdgcn_sched_barrier(0);
      float my_w;
      {
        float m;
        const float z = canon_softmax_z(lg, E, &m);
        my_w = canon_topk_weight(lg[my_idx], m, z, ST_TOPK);
      }

      // ---- gate_up: two routed pairs per wave
      {
        float av[2];
        F::gate_up(gu, xq4, s_xsum, lane, av);
        if (lane == 0) {
          if constexpr (A32) {
            ll_put(ll + LL_ACT + rk * I + rj, av[0], tB);
            ll_put(ll + LL_ACT + rk * I + rj + 1, av[1], tB);
          } else {
            ll_put2(ll + LL_ACT + ((rk * I + rj) >> 1), av[0], av[1], t2);
          }
        }
      }
      ST_MARK(4);
      // down rows (8 experts + shared): issued after the gate_up stores so the gate_up stream
      // has the bandwidth to itself, and well before the activation poll, whose reads return
      // behind them
      typename F::DN dn;
      F::load_dn(Ly, my_idx, n, lane, dn);
      const uint2 qs = ld8(Ly.sd_q + (size_t)n * I + lane * 8);
      const uint32_t ssr = SH::raw(Ly.sd_s, n, lane * 8, I);

      // ---- activation exchange, collected by the poller
      ST_MARKW(14, 2);
      if (poller) {
        ST_MARKW(12, 7);
        const uint32_t r = poll_wave<SpecAct<F, A32>::kRows / ST_NP, ST_NP>(
            ll + LL_ACT, pw, SpecAct<F, A32>{tB, t2, reinterpret_cast<float*>(as4), s_asum}, sync, t_topk + (A32 ? F::kOffAct : F::kOffActIb), tmo);
        if (!r && lane == 0) s_abort = 1;
        ST_MARKW(13, 7);
#ifdef ST_TRACE
        if (threadIdx.x == 448) ll[LL_WORDS + ((size_t)l * 16 + 15) * ST_NB + blockIdx.x] = r;
#endif
      }
      __syncthreads();
      ST_MARK(5);
      const uint64_t t_act = __builtin_amdgcn_s_memrealtime();
      if (s_abort) {
      give_up();
      return;
    }


      ST_MARK(9);
      const float sgv = sigmoid(lg[E]);
      if (blockIdx.x == 0 && wave == 0) {
        if (idx_out && lane < ST_TOPK) idx_out[l * ST_TOPK + lane] = my_idx;
        if (wts_out && lane < ST_TOPK) wts_out[l * ST_TOPK + lane] = my_w;
        if (sgate_out && lane == 0) sgate_out[l] = lg[E];
      }

      // ---- down row n: 8 experts + shared, weighted, plus the residual
      float xc[8];
      const float sumc = s_asum[128 + lane];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const float4 v = as4[1024 + i * 64 + lane];
        xc[4 * i] = v.x, xc[4 * i + 1] = v.y, xc[4 * i + 2] = v.z, xc[4 * i + 3] = v.w;
      }
      float dc = dot4_u8b(qs.x, xc, 0.f);
      dc = dot4_u8b(qs.y, xc + 4, dc);
      float acc = F::down(dn, as4, s_asum, my_w, lane) + sgv * SH::cvt(ssr) * (dc - 128.f * sumc);
      acc = wave_sum(acc);
      ST_MARK(11);
      if (lane == 0) {
        const float y = res + acc;
        if (l + 1 < L) ll_put(ll + LL_X + n, y, tC);
        else x[n] = y;
        if (xs_out) xs_out[(size_t)l * H + n] = y;
      }
      // ---- next layer's known weights: issued after the residual publish (issued before it,
      // the compiler's wait for a spilled address ahead of the publish would wait for them
      // too) and after the activation poll (a wave's loads return in order, so loads issued
      // before a poll would delay it)
      if (l + 1 < L) {
        if (is_router) {
          const uint16_t* wr = Ln.router + (size_t)rrow * H;
#pragma unroll
          for (int j = 0; j < 4; ++j) rw.w[j] = ld16(wr + (size_t)(lane + 64 * j) * 8);
        }
        if (is_shared) load_shared_pair<SH>(Ln, sj, lane, sp);
        nwv = Ln.nw ? ldf4(Ln.nw + 4 * tid) : make_float4(1.f, 1.f, 1.f, 1.f);
      }
      ST_MARK(6);
      // ---- residual exchange for the next layer (every wave read its x[n] at the layer start)
      if (poller && l + 1 < L) {
        const uint32_t r = poll_wave<4, ST_NP>(ll + LL_X, pw, Spec32{tC, H, reinterpret_cast<float*>(xr4)}, sync, t_act + (A32 ? F::kOffXA32 : F::kOffX), tmo);
        if (!r && lane == 0) s_abort = 1;
        ST_PUT(10, r);
      }
      // the next layer's norm weight, stored after the poll (its load returns ahead of the
      // poll's reads anyway); the router rows read nws after the barrier below
      nws[tid] = nwv;
    }
    __syncthreads();
    ST_MARK(7);
    if (s_abort) {
      give_up();
      return;
    }
    Ly = Ln;
  }
  if (blockIdx.x == 0 && tid == 0) {
    __hip_atomic_store(sync + 2, lbase + (uint32_t)L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(sync + 3, kTransport, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(sync, epoch + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // the caller's next-op range [pf, pf + pf_bytes) warmed in the memory-side cache, each block
  // its share, after the outputs are stored.  (Issued during the last layer instead, the warm
  // loads' registers stay allocated across the layer loop: 10.25 -> 11.2 us/layer.)
  warm_range(pf, pf_bytes);
}

// The grid needs all ST_NB workgroups resident at once; checked once per device.
int step_grid_ok(const void* kernel) {
  static std::atomic<int> ok[64];  // 0 unknown, 1 yes, -1 no (launchers may run on several threads)
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (ok[dev].load(std::memory_order_relaxed) == 0) {
    int cus = 0, per = 0;
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, ST_NT, 0);
    ok[dev].store((cus * per >= ST_NB) ? 1 : -1, std::memory_order_relaxed);
  }
  return ok[dev].load(std::memory_order_relaxed) == 1;
}

std::atomic<uint64_t> g_wait_ticks{ST_TIMEOUT_TICKS};

// Transport of the routed activations: two fp32 per word with the phase in their two low
// mantissa bits (default: half the words of the other form) or fp32 with a 32-bit tag per word;
// dr_step_set_act_exchange selects it for later launches.
std::atomic<int> g_act_bits{30};

template <class F, class SH, bool A32>
int launch_step_as(const dr_decode_layer* layers, int L, float* x, int E, float eps, uint64_t* ll, uint32_t* sync,
                   int* idx_out, float* wts_out, float* sgate_out, float* xs_out, const char* pf, size_t pf_bytes,
                   hipStream_t st, bool noalloc) {
  const void* k = reinterpret_cast<const void*>(&k_decode_step<F, SH, A32>);
  if (!step_grid_ok(k)) return -1;
  // the no-allocation entry point only reads the error word's address (set up when the library
  // was loaded); the others set it up on first use
  uint32_t* err = noalloc ? err_word_noalloc() : err_word();
  if (err_pending() == DR_ERR_STEP_TIMEOUT) return DR_ERR_STEP_TIMEOUT;  // until dr_last_error clears it
  hipLaunchKernelGGL((k_decode_step<F, SH, A32>), dim3(ST_NB), dim3(ST_NT), 0, st, layers, L, x, E, eps, ll, sync,
                     idx_out, wts_out, sgate_out, xs_out, err, g_wait_ticks.load(std::memory_order_relaxed),
                     pf_bytes ? pf : nullptr, pf ? pf_bytes : 0);
  return 0;
}

template <class F, class SH>
int launch_step(const dr_decode_layer* layers, int L, float* x, int E, int H, int I, int topk, float eps,
                uint64_t* ll, uint32_t* sync, int* idx_out, float* wts_out, float* sgate_out, float* xs_out,
                const char* pf, size_t pf_bytes, hipStream_t st, bool noalloc = false) {
  if (H != ST_H || I != ST_I || topk != ST_TOPK || E < ST_TOPK || E > ST_MAXE || L < 1 || L > ST_MAXL) return -1;
  if (!layers || !x || !ll || !sync) return -1;
  if (g_act_bits.load(std::memory_order_relaxed) == 30)
    return launch_step_as<F, SH, false>(layers, L, x, E, eps, ll, sync, idx_out, wts_out, sgate_out, xs_out, pf,
                                        pf_bytes, st, noalloc);
  return launch_step_as<F, SH, true>(layers, L, x, E, eps, ll, sync, idx_out, wts_out, sgate_out, xs_out, pf, pf_bytes,
                                     st, noalloc);
}

constexpr int ST_SCRATCH_WORDS = LL_WORDS + 2;  // ll, then sync[4] as two 64-bit words

}  // namespace

// ---- The entry point that allocates nothing (for callers that cannot allocate: code under
// graph capture, serving loops, harnesses that forbid hipMalloc).  Its exchange buffer and sync
// words are a file-scope device array, one copy per GPU, held until the process ends
// (ST_SCRATCH_WORDS x 8 = 55,376 bytes).  Host code never passes the array's name: its address
// on each device comes from hipGetSymbolAddress, looked up once per device with that device
// current.  Calls that overlap on one GPU share the array and race; stream-order them.
static __device__ __align__(256) uint64_t scratch[ST_SCRATCH_WORDS];

namespace {

__global__ void __launch_bounds__(256) k_zero_scratch(uint64_t* __restrict__ p, int n) {
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) p[i] = 0;
}

uint64_t* scratch_ptr() {
  static std::atomic<uint64_t*> ptrs[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  uint64_t* p = ptrs[dev].load(std::memory_order_acquire);
  if (!p) {
    void* q = nullptr;
    if (hipGetSymbolAddress(&q, HIP_SYMBOL(scratch)) != hipSuccess || !q) {
      (void)hipGetLastError();
      return nullptr;
    }
    p = static_cast<uint64_t*>(q);
    ptrs[dev].store(p, std::memory_order_release);
  }
  return p;
}

}  // namespace

API int dr_moe_decode_step_bf16s_noalloc(const dr_decode_layer* layers, int n_layers, float* x, int E, int H, int I,
                                         int topk, float eps, int* idx_out, float* wts_out, float* sgate_out,
                                         float* xs_out, const char* pf, size_t pf_bytes, dr_stream_t st) {
  if (H != ST_H || I != ST_I || topk != ST_TOPK || E < ST_TOPK || E > ST_MAXE || n_layers < 1 || n_layers > ST_MAXL ||
      !layers || !x)
    return -1;
  uint64_t* p = scratch_ptr();
  if (!p) return (int)hipErrorInvalidSymbol;
  // every call starts from cleared slots and sync words (a fill kernel: graph-capturable)
  hipLaunchKernelGGL(k_zero_scratch, dim3(28), dim3(256), 0, (hipStream_t)st, p, ST_SCRATCH_WORDS);
  return launch_step<StepQ4<ScaleBF16>, Q8RowBF16>(layers, n_layers, x, E, H, I, topk, eps, p,
                                                   reinterpret_cast<uint32_t*>(p + LL_WORDS), idx_out, wts_out,
                                                   sgate_out, xs_out, pf, pf_bytes, (hipStream_t)st, true);
}

API int dr_step_set_act_exchange(int bits) {
  if (bits != 0 && bits != 32 && bits != 30) return -1;
  g_act_bits.store(bits ? bits : 30, std::memory_order_relaxed);
  return 0;
}

API int dr_step_set_wait_limit(uint32_t us) {
  g_wait_ticks.store(us ? (uint64_t)us * 100u : ST_TIMEOUT_TICKS, std::memory_order_relaxed);
  return 0;
}

API int dr_moe_decode_step(const dr_decode_layer* layers, int n_layers, float* x, int E, int H, int I, int topk,
                           float eps, uint64_t* ll, uint32_t* sync, int* idx_out, float* wts_out, float* sgate_out,
                           float* xs_out, const char* pf, size_t pf_bytes, dr_stream_t st) {
  return launch_step<StepQ4<ScaleF16>, Q8G128F16>(layers, n_layers, x, E, H, I, topk, eps, ll, sync, idx_out, wts_out,
                                          sgate_out, xs_out, pf, pf_bytes, (hipStream_t)st);
}

API int dr_moe_decode_step_bf16s(const dr_decode_layer* layers, int n_layers, float* x, int E, int H, int I,
                                 int topk, float eps, uint64_t* ll, uint32_t* sync, int* idx_out, float* wts_out,
                                 float* sgate_out, float* xs_out, const char* pf, size_t pf_bytes, dr_stream_t st) {
  return launch_step<StepQ4<ScaleBF16>, Q8RowBF16>(layers, n_layers, x, E, H, I, topk, eps, ll, sync, idx_out, wts_out,
                                           sgate_out, xs_out, pf, pf_bytes, (hipStream_t)st);
}

API int dr_moe_decode_step_fp8(const dr_decode_layer* layers, int n_layers, float* x, int E, int H, int I, int topk,
                               float eps, uint64_t* ll, uint32_t* sync, int* idx_out, float* wts_out,
                               float* sgate_out, float* xs_out, const char* pf, size_t pf_bytes, dr_stream_t st) {
  return launch_step<StepFP8<0>, Q8G128F16>(layers, n_layers, x, E, H, I, topk, eps, ll, sync, idx_out, wts_out,
                                           sgate_out, xs_out, pf, pf_bytes, (hipStream_t)st);
}

API int dr_moe_decode_step_fp8_bf16s(const dr_decode_layer* layers, int n_layers, float* x, int E, int H, int I,
                                     int topk, float eps, uint64_t* ll, uint32_t* sync, int* idx_out, float* wts_out,
                                     float* sgate_out, float* xs_out, const char* pf, size_t pf_bytes, dr_stream_t st) {
  return launch_step<StepFP8<1>, Q8RowBF16>(layers, n_layers, x, E, H, I, topk, eps, ll, sync, idx_out, wts_out,
                                           sgate_out, xs_out, pf, pf_bytes, (hipStream_t)st);
}

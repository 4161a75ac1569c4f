// Batch-1 decode MoE with int4 routed experts (reference: kernels/drama.cu:470-599,
// src/ffi.rs:42-46) and the single int4 GEMV of benchmark configuration 1.
//
// gfx950 mapping.  A K = 2048 int4 row is 1024 bytes: exactly one 16-byte load per lane of a
// wave64, so lane l always owns elements [32 l, 32 l + 32) and half of group l / 2.  gate_up
// stages its 32 normalised inputs once per block in LDS as 24-bit fixed-point digits
// (q4_digits_stage, read back with conflict-free 16-byte reads), so each weight word is six
// exact v_dot8 sums; each lane folds scale and min into its partial dot,
// s 2^-S sum((q - 8) X) + (m + 8 s) sum(x), and one 64-lane butterfly finishes the row.
//
// Down projection: one output row n gathers 8 expert rows of 256 bytes plus the 512-byte
// int8 shared row.  Lane l owns chunk (l & 15) of experts (l >> 4) and 4 + (l >> 4) and 8
// bytes of the shared row, so one row costs 2 x 16 + 8 bytes of loads per lane and the lane's
// 72 activations stay in registers across rows.
#include <type_traits>

#include "common.hpp"

using namespace drm;

namespace {

constexpr int DEC_H = 2048, DEC_I = 512, DEC_TOPK = 8;

// gate_up of B decode rows.  Routed units are (row b, pick k, pair j), j fastest; the NBR
// routed blocks' waves walk them spaced by the grid (wave g takes units g, g + NW, ..., so
// waves running side by side read neighbouring rows of one expert), keeping D units in flight
// and loading unit p + D once unit p is computed.  The shared-expert blocks, dispatched first
// (PPWS pairs per wave, int8 rows read as two 1024-byte halves), serve all B rows with one read
// of their weights.  x (and the norm weight) are requested before the weights, so the staging
// overlaps the weight fetch (a wave's loads return in order).
template <class SC, class SH, int WPB, int NBR, int D, int PPWS, int B>
__global__ void __launch_bounds__(WPB * 64)
    k_moe_gate_up_q4(const uint8_t* __restrict__ Q, const uint32_t* __restrict__ SM, const int8_t* __restrict__ shq,
                     const uint16_t* __restrict__ shs, const float* x, const int* __restrict__ idx,
                     float* __restrict__ act, const float* nw, float eps) {
  constexpr int H = DEC_H, I = DEC_I, NT = WPB * 64, NW = NBR * WPB, PPW = B * DEC_TOPK * I / NW;
  constexpr int NBS = I / (WPB * PPWS);
  static_assert(PPW * NW == B * DEC_TOPK * I && D <= PPW, "units split evenly over the routed waves");
  __shared__ float4 xs[B * H / 4];
  const int lane = lane_id(), wave = wave_id();
  if ((int)blockIdx.x >= NBS) {
    const int g = (blockIdx.x - NBS) * WPB + wave;
    XStage<H, NT, B, SlotQ4D> xst;
    xst.load(x, nw);
    uint4 wg[D], wu[D];
    uint32_t sg[D], su[D];
    auto issue = [&](int p, int d) {
      const int u = g + NW * p, b = u / (DEC_TOPK * I), k = (u / I) % DEC_TOPK, j = u % I;
      const size_t e = (size_t)idx[b * DEC_TOPK + k];
      const uint8_t* q = Q + (e * (2 * I) + j) * (H / 2) + lane * 16;
      const uint32_t* sm = SM + (e * (2 * I) + j) * (H / 64) + (lane >> 1);
      wg[d] = ld16(q), wu[d] = ld16(q + (size_t)I * (H / 2));
      sg[d] = ld4(sm), su[d] = ld4(sm + (size_t)I * (H / 64));
      __builtin_amdgcn_sched_barrier(0);
    };
#pragma unroll
    for (int p = 0; p < D; ++p) issue(p, p);
    xst.finish(nw != nullptr, eps, xs);
#pragma unroll
    for (int p = 0; p < PPW; ++p) {
      const int d = p % D;
      const int u = g + NW * p, b = u / (DEC_TOPK * I), k = (u / I) % DEC_TOPK, j = u % I;
      // row b of x as fixed-point digits (XStage with SlotQ4D): w . x = s (q - 8) . x + (m + 8 s) sum x
      const float* rb = reinterpret_cast<const float*>(xs + b * (H / 4));
      uint32_t dg[24];
      q4_digits_load(reinterpret_cast<const uint32_t*>(rb), lane, dg);
      const float xsum = rb[1536 + lane], xsc = rb[1600 + lane];
      opaque(wg[d]), opaque(wu[d]);
      const float qg = q4_dot_digits(wg[d], dg), qu = q4_dot_digits(wu[d], dg);
      const float2 pa = SC::pair(sg[d]), pb = SC::pair(su[d]);
      if (p + D < PPW) issue(p + D, d);
      const float gv = wave_sum(pa.x * (qg * xsc) + __builtin_fmaf(8.f, pa.x, pa.y) * xsum);
      const float uv = wave_sum(pb.x * (qu * xsc) + __builtin_fmaf(8.f, pb.x, pb.y) * xsum);
      if (lane == 0) act[(size_t)b * (DEC_TOPK + 1) * I + k * I + j] = silu(gv) * uv;
    }
  } else {
    const int j0 = (blockIdx.x * WPB + wave) * PPWS;
    XStage<H, NT, B, SlotQ8H> xst;
    xst.load(x, nw);
    uint4 g0[PPWS], g1[PPWS], u0[PPWS], u1[PPWS];
    float sg0[PPWS], sg1[PPWS], su0[PPWS], su1[PPWS];
#pragma unroll
    for (int p = 0; p < PPWS; ++p) {
      const int8_t* rg = shq + (size_t)(j0 + p) * H + lane * 16;
      const int8_t* ru = shq + (size_t)(I + j0 + p) * H + lane * 16;
      g0[p] = ld16(rg), g1[p] = ld16(rg + 1024), u0[p] = ld16(ru), u1[p] = ld16(ru + 1024);
    }
#pragma unroll
    for (int p = 0; p < PPWS; ++p) {
      const int j = j0 + p;
      sg0[p] = SH::scale(shs, j, lane * 16, H), sg1[p] = SH::scale(shs, j, 1024 + lane * 16, H);
      su0[p] = SH::scale(shs, I + j, lane * 16, H), su1[p] = SH::scale(shs, I + j, 1024 + lane * 16, H);
    }
    xst.finish(nw != nullptr, eps, xs);
#pragma unroll 1
    for (int r = 0; r < B; ++r) {
      float xa[16], xb[16], sa = 0.f, sb = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 v = xs[r * (H / 4) + i * 64 + lane], w = xs[r * (H / 4) + 256 + i * 64 + lane];
        xa[4 * i] = v.x, xa[4 * i + 1] = v.y, xa[4 * i + 2] = v.z, xa[4 * i + 3] = v.w;
        xb[4 * i] = w.x, xb[4 * i + 1] = w.y, xb[4 * i + 2] = w.z, xb[4 * i + 3] = w.w;
        sa += (v.x + v.y) + (v.z + v.w);
        sb += (w.x + w.y) + (w.z + w.w);
      }
#pragma unroll
      for (int p = 0; p < PPWS; ++p) {
        // converted per row, not hoisted out of the row loop
        opaque(g0[p]), opaque(g1[p]), opaque(u0[p]), opaque(u1[p]);
        float ga = 0.f, gb = 0.f, ua = 0.f, ub = 0.f;
        const uint32_t gw0[4] = {g0[p].x, g0[p].y, g0[p].z, g0[p].w}, gw1[4] = {g1[p].x, g1[p].y, g1[p].z, g1[p].w};
        const uint32_t uw0[4] = {u0[p].x, u0[p].y, u0[p].z, u0[p].w}, uw1[4] = {u1[p].x, u1[p].y, u1[p].z, u1[p].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          ga = dot4_u8b(gw0[q], xa + 4 * q, ga), gb = dot4_u8b(gw1[q], xb + 4 * q, gb);
          ua = dot4_u8b(uw0[q], xa + 4 * q, ua), ub = dot4_u8b(uw1[q], xb + 4 * q, ub);
        }
        const float gv = wave_sum(sg0[p] * (ga - 128.f * sa) + sg1[p] * (gb - 128.f * sb));
        const float uv = wave_sum(su0[p] * (ua - 128.f * sa) + su1[p] * (ub - 128.f * sb));
        if (lane == 0) act[(size_t)r * (DEC_TOPK + 1) * I + DEC_TOPK * I + j0 + p] = silu(gv) * uv;
      }
    }
  }
}

// down of decode row blockIdx.y: wave w of block b owns output rows n0 .. n0 + RPW - 1; lane l
// holds chunk (l & 15) of experts (l >> 4) and 4 + (l >> 4) and 8 bytes of the int8 shared row.
// The row's activations are requested first and staged in LDS while the weights stream in.
template <class SC, class SH, int WPB, int RPW>
__global__ void __launch_bounds__(WPB * 64)
    k_moe_down_q4(const uint8_t* __restrict__ Q, const uint32_t* __restrict__ SM, const int8_t* __restrict__ shq,
                  const uint16_t* __restrict__ shs, const float* act, const int* __restrict__ idx,
                  const float* __restrict__ wts, const float* __restrict__ sgate, const float* res, float* y,
                  uint16_t* yb, const char* pf, size_t pf_bytes) {
  constexpr int H = DEC_H, I = DEC_I, AW = (DEC_TOPK + 1) * I / 4, NT = WPB * 64, NA = 1024 / NT;
  __shared__ float4 as[AW];
  const int lane = lane_id(), wave = wave_id();
  const int ka = lane >> 4, cc = lane & 15, b = blockIdx.y;
  const int n0 = (blockIdx.x * WPB + wave) * RPW;
  act += (size_t)b * (DEC_TOPK + 1) * I, idx += b * DEC_TOPK, wts += b * DEC_TOPK;
  // pick indices and weights with scalar loads, then the activations, then the weights
  size_t ea, eb;
  float wa, wb;
  {
    int ia[4], ib[4];
    float fa[4], fb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ia[i] = idx[i], ib[i] = idx[4 + i], fa[i] = wts[i], fb[i] = wts[4 + i];
    int sa_ = ia[0], sb_ = ib[0];
    float ta = fa[0], tb = fb[0];
#pragma unroll
    for (int i = 1; i < 4; ++i) {
      sa_ = ka == i ? ia[i] : sa_, sb_ = ka == i ? ib[i] : sb_;
      ta = ka == i ? fa[i] : ta, tb = ka == i ? fb[i] : tb;
    }
    ea = (size_t)sa_, eb = (size_t)sb_, wa = ta, wb = tb;
  }
  const float sgv = sigmoid(sgate[b]);
  const float4* a4 = reinterpret_cast<const float4*>(act);
  float4 av[NA + 1];
#pragma unroll
  for (int t = 0; t < NA; ++t) av[t] = ldf4(a4 + threadIdx.x + NT * t);
  av[NA] = ldf4(a4 + 1024 + (threadIdx.x & 127));
  issue_fence();
  uint4 qa[RPW], qb[RPW];
  uint32_t sa[RPW], sb[RPW], ssr[RPW];
  uint2 qs[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const size_t n = (size_t)(n0 + r);
    qa[r] = ld16(Q + (ea * H + n) * (I / 2) + cc * 16);
    qb[r] = ld16(Q + (eb * H + n) * (I / 2) + cc * 16);
    sa[r] = ld4(SM + (ea * H + n) * (I / 64) + (cc >> 1));
    sb[r] = ld4(SM + (eb * H + n) * (I / 64) + (cc >> 1));
    qs[r] = ld8(shq + n * I + lane * 8);
    ssr[r] = SH::raw(shs, n, lane * 8, I);
    __builtin_amdgcn_sched_barrier(0);
  }
  // routed part as two 512-float4 halves with the 8-per-lane swizzle, shared part (128 float4)
  // with 2 per lane
#pragma unroll
  for (int t = 0; t < NA; ++t) {
    const int f = threadIdx.x + NT * t;
    as[(f & ~511) + (f & 7) * 64 + ((f & 511) >> 3)] = av[t];
  }
  if ((int)threadIdx.x < 128) {
    const int f = threadIdx.x;
    as[1024 + (f & 1) * 64 + (f >> 1)] = av[NA];
  }
  __syncthreads();
  float xa[32], xb[32], xc[8];
  float suma = 0.f, sumb = 0.f, sumc = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float4 v = as[i * 64 + lane], w = as[512 + i * 64 + lane];
    xa[4 * i] = v.x, xa[4 * i + 1] = v.y, xa[4 * i + 2] = v.z, xa[4 * i + 3] = v.w;
    xb[4 * i] = w.x, xb[4 * i + 1] = w.y, xb[4 * i + 2] = w.z, xb[4 * i + 3] = w.w;
    suma += (v.x + v.y) + (v.z + v.w);
    sumb += (w.x + w.y) + (w.z + w.w);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float4 v = as[1024 + i * 64 + lane];
    xc[4 * i] = v.x, xc[4 * i + 1] = v.y, xc[4 * i + 2] = v.z, xc[4 * i + 3] = v.w;
    sumc += (v.x + v.y) + (v.z + v.w);
  }
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    float da = 0.f, db = 0.f;
    da = dot8_q4(qa[r].x, xa + 0, da), db = dot8_q4(qb[r].x, xb + 0, db);
    da = dot8_q4(qa[r].y, xa + 8, da), db = dot8_q4(qb[r].y, xb + 8, db);
    da = dot8_q4(qa[r].z, xa + 16, da), db = dot8_q4(qb[r].z, xb + 16, db);
    da = dot8_q4(qa[r].w, xa + 24, da), db = dot8_q4(qb[r].w, xb + 24, db);
    float dc = dot4_u8b(qs[r].x, xc, 0.f);
    dc = dot4_u8b(qs[r].y, xc + 4, dc);
    const float2 pa = SC::pair(sa[r]), pb = SC::pair(sb[r]);
    float acc = wa * (pa.x * da + pa.y * suma) + wb * (pb.x * db + pb.y * sumb) +
                sgv * SH::cvt(ssr[r]) * (dc - 128.f * sumc);
    acc = wave_sum(acc);
    const size_t n = (size_t)b * H + n0 + r;
    if (lane == 0) {
      const float out = res[n] + acc;
      y[n] = out;
      if (yb) yb[n] = to_bf16(out);
    }
  }
  warm_range(pf, pf_bytes);
}

// Launch shapes: batch 1 (the engine's per-layer chain) uses 256-thread blocks, many of them;
// B > 1 uses 512-thread blocks, two per CU (as the FP8 kernels).
template <class SC, class SH, int B>
void launch_decode_b(const uint8_t* gu_q, const void* gu_sm, const uint8_t* d_q, const void* d_sm,
                     const int8_t* sgu_q, const uint16_t* sgu_s, const int8_t* sd_q, const uint16_t* sd_s,
                     const float* x, const int* idx, const float* wts, const float* sgate, const float* res, float* act,
                     float* y, uint16_t* yb, const float* nw, float eps, const char* pf, size_t pf_bytes,
                     hipStream_t st) {
  constexpr int GW = B == 1 ? 4 : 8, GB = 512, GD = 2, GS = B == 1 ? 1 : 2, DW = B == 1 ? 4 : 8, DR = 2;
  constexpr int NB = GB + DEC_I / (GW * GS);
  hipLaunchKernelGGL((k_moe_gate_up_q4<SC, SH, GW, GB, GD, GS, B>), dim3(NB), dim3(GW * 64), 0, st, gu_q,
                     (const uint32_t*)gu_sm, sgu_q, sgu_s, x, idx, act, nw, eps);
  hipLaunchKernelGGL((k_moe_down_q4<SC, SH, DW, DR>), dim3(DEC_H / (DW * DR), B), dim3(DW * 64), 0, st, d_q,
                     (const uint32_t*)d_sm, sd_q, sd_s, act, idx, wts, sgate, res, y, yb, pf, pf_bytes);
}

// rows independent decode rows (x, res, y: [rows, H]; idx, wts: [rows, topk]; act: rows x
// (topk + 1) x I), launched 4 rows at a time
template <class SC, class SH>
int launch_decode(const uint8_t* gu_q, const void* gu_sm, const uint8_t* d_q, const void* d_sm, const int8_t* sgu_q,
                  const uint16_t* sgu_s, const int8_t* sd_q, const uint16_t* sd_s, const float* x, const int* idx,
                  const float* wts, const float* sgate, const float* res, float* act, float* y, uint16_t* yb, int H,
                  int I, int topk, const float* nw, float eps, const char* pf, size_t pf_bytes, hipStream_t st,
                  int rows = 1) {
  if (H != DEC_H || I != DEC_I || topk != DEC_TOPK || rows < 1 || rows > 64) return -1;
  for (int r0 = 0; r0 < rows; r0 += 4) {
    const int b = rows - r0 < 4 ? rows - r0 : 4;
    const size_t xo = (size_t)r0 * H, ko = (size_t)r0 * topk, ao = (size_t)r0 * (topk + 1) * I;
    auto go = [&](auto kb) {
      constexpr int KB = decltype(kb)::value;
      launch_decode_b<SC, SH, KB>(gu_q, gu_sm, d_q, d_sm, sgu_q, sgu_s, sd_q, sd_s, x + xo, idx + ko, wts + ko,
                                  sgate + r0, res + xo, act + ao, y + xo, yb ? yb + xo : nullptr, nw, eps,
                                  r0 + b == rows ? pf : nullptr, pf_bytes, st);
    };
    if (b == 1) go(std::integral_constant<int, 1>{});
    else if (b == 2) go(std::integral_constant<int, 2>{});
    else if (b == 3) go(std::integral_constant<int, 3>{});
    else go(std::integral_constant<int, 4>{});
  }
  return 0;
}

// ---- single int4 GEMV (configuration 1) ------------------------------------------------------
// One output row per wave, so a 1024-row GEMV spreads over 256 blocks (every CU).  The first
// 2048-input segment of the row is requested before x is staged, so the weight fetch and the
// x staging share one memory round trip.
constexpr int GV_WPB = 4, GV_RPW = 1;

template <class SC>
__global__ void __launch_bounds__(256)
    k_gemv_q4(const uint8_t* __restrict__ Q, const uint32_t* __restrict__ SM, const uint16_t* __restrict__ x,
              float* __restrict__ y, uint16_t* __restrict__ yb, int N, int K) {
  extern __shared__ float4 xsd[];
  const int lane = lane_id(), wave = wave_id();
  const int row0 = (blockIdx.x * GV_WPB + wave) * GV_RPW;
  uint4 w[GV_RPW];
  uint32_t s[GV_RPW];
  auto fetch = [&](int seg) {
#pragma unroll
    for (int r = 0; r < GV_RPW; ++r) {
      const int row = row0 + r < N ? row0 + r : N - 1;
      w[r] = ld16(Q + (size_t)row * (K / 2) + seg * 1024 + lane * 16);
      s[r] = SM[(size_t)row * (K / 64) + seg * 32 + (lane >> 1)];
    }
  };
  fetch(0);
  // stage x (bf16) as fp32 float4 with the lane-major swizzle per 2048-element segment
  for (int f = threadIdx.x; f < K / 4; f += blockDim.x) {
    const uint2 v = ld8(x + (size_t)f * 4);
    xsd[(f & ~511) + (f & 7) * 64 + ((f & 511) >> 3)] = make_float4(bf16_lo(v.x), bf16_hi(v.x), bf16_lo(v.y), bf16_hi(v.y));
  }
  __syncthreads();
  float acc[GV_RPW];
#pragma unroll
  for (int r = 0; r < GV_RPW; ++r) acc[r] = 0.f;
  for (int seg = 0; seg < K / 2048; ++seg) {
    if (seg) fetch(seg);
    float xv[32], xsum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 v = xsd[seg * 512 + i * 64 + lane];
      xv[4 * i] = v.x, xv[4 * i + 1] = v.y, xv[4 * i + 2] = v.z, xv[4 * i + 3] = v.w;
      xsum += (v.x + v.y) + (v.z + v.w);
    }
#pragma unroll
    for (int r = 0; r < GV_RPW; ++r) {
      float q = 0.f;
      q = dot8_q4(w[r].x, xv, q);
      q = dot8_q4(w[r].y, xv + 8, q);
      q = dot8_q4(w[r].z, xv + 16, q);
      q = dot8_q4(w[r].w, xv + 24, q);
      const float2 p = SC::pair(s[r]);
      acc[r] += p.x * q + p.y * xsum;
    }
  }
#pragma unroll
  for (int r = 0; r < GV_RPW; ++r) {
    const float v = wave_sum(acc[r]);
    const int row = row0 + r;
    if (lane == 0 && row < N) {
      y[row] = v;
      if (yb) yb[row] = to_bf16(v);
    }
  }
}

}  // namespace

API int dr_moe_decode(const uint8_t* gu_q, const uint16_t* gu_sm, const uint8_t* d_q, const uint16_t* d_sm,
                      const int8_t* sgu_q, const uint16_t* sgu_s, const int8_t* sd_q, const uint16_t* sd_s,
                      const float* x, const int* idx, const float* wts, const float* sgate, const float* res, float* act,
                      float* y, int H, int I, int topk, const float* nw, float eps, const char* pf, size_t pf_bytes,
                      hipStream_t st) {
  return launch_decode<ScaleF16, Q8G128F16>(gu_q, gu_sm, d_q, d_sm, sgu_q, sgu_s, sd_q, sd_s, x, idx, wts, sgate, res,
                                            act, y, nullptr, H, I, topk, nw, eps, pf, pf_bytes, st);
}

API int dr_moe_decode_bf16s(const uint8_t* gu_q, const uint16_t* gu_sm, const uint8_t* d_q, const uint16_t* d_sm,
                            const int8_t* sgu_q, const uint16_t* sgu_s, const int8_t* sd_q, const uint16_t* sd_s,
                            const float* x, const int* idx, const float* wts, const float* sgate, const float* res,
                            float* act, float* y, uint16_t* yb, int H, int I, int topk, const float* nw, float eps,
                            const char* pf, size_t pf_bytes, hipStream_t st) {
  return launch_decode<ScaleBF16, Q8RowBF16>(gu_q, gu_sm, d_q, d_sm, sgu_q, sgu_s, sd_q, sd_s, x, idx, wts, sgate,
                                             res, act, y, yb, H, I, topk, nw, eps, pf, pf_bytes, st);
}

API int dr_moe_decode_rows(const uint8_t* gu_q, const uint16_t* gu_sm, const uint8_t* d_q, const uint16_t* d_sm,
                           const int8_t* sgu_q, const uint16_t* sgu_s, const int8_t* sd_q, const uint16_t* sd_s,
                           const float* x, const int* idx, const float* wts, const float* sgate, const float* res,
                           float* act, float* y, int rows, int H, int I, int topk, const float* nw, float eps,
                           hipStream_t st) {
  return launch_decode<ScaleF16, Q8G128F16>(gu_q, gu_sm, d_q, d_sm, sgu_q, sgu_s, sd_q, sd_s, x, idx, wts, sgate, res,
                                            act, y, nullptr, H, I, topk, nw, eps, nullptr, 0, st, rows);
}

API int dr_moe_decode_rows_bf16s(const uint8_t* gu_q, const uint16_t* gu_sm, const uint8_t* d_q, const uint16_t* d_sm,
                                 const int8_t* sgu_q, const uint16_t* sgu_s, const int8_t* sd_q, const uint16_t* sd_s,
                                 const float* x, const int* idx, const float* wts, const float* sgate, const float* res,
                                 float* act, float* y, uint16_t* yb, int rows, int H, int I, int topk, const float* nw,
                                 float eps, hipStream_t st) {
  return launch_decode<ScaleBF16, Q8RowBF16>(gu_q, gu_sm, d_q, d_sm, sgu_q, sgu_s, sd_q, sd_s, x, idx, wts, sgate,
                                             res, act, y, yb, H, I, topk, nw, eps, nullptr, 0, st, rows);
}

API int dr_gemv_q4_bf16s(const uint8_t* q, const uint16_t* sm, const uint16_t* x, float* y, uint16_t* yb, int N, int K,
                         hipStream_t st) {
  if (K % 2048 != 0 || K <= 0 || K > 8192 || N <= 0) return -1;
  const int rows_per_block = GV_WPB * GV_RPW;
  hipLaunchKernelGGL(k_gemv_q4<ScaleBF16>, dim3((N + rows_per_block - 1) / rows_per_block), dim3(256),
                     (size_t)K * sizeof(float), st, q, (const uint32_t*)sm, x, y, yb, N, K);
  return 0;
}

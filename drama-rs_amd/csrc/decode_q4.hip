// Batch-1 decode MoE with int4 routed experts (reference: kernels/drama.cu:470-599,
// src/ffi.rs:42-46) and the single int4 GEMV of benchmark configuration 1.
//
// gfx950 mapping.  A K = 2048 int4 row is 1024 bytes: exactly one 16-byte load per lane of a
// wave64, so lane l always owns elements [32 l, 32 l + 32) and half of group l / 2.  Its 32
// normalised inputs therefore live in registers for every row the wave touches; they are
// staged once per block through LDS in a lane-major swizzle (slot = i * 64 + lane) so the
// 16-byte LDS reads are conflict free.  Each lane folds scale and min into its partial dot:
// s * sum(q x) + m * sum(x), and one 64-lane butterfly finishes the row.
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
constexpr int GU_WPB = 4, GU_PPW = 2;  // routed gate_up: waves per block, (gate, up) pairs per wave
constexpr int GU_NB_ROUTED = DEC_TOPK * DEC_I / (GU_WPB * GU_PPW);
constexpr int GU_NB_SHARED = DEC_I / GU_WPB;  // one shared pair per wave
constexpr int DN_WPB = 4, DN_RPW = 2;         // down: waves per block, output rows per wave

// Block-wide RMSNorm of x (H floats) into LDS, float4 f stored at slot(f).  Fast rsqrt: the
// decode values are compared with a tolerance, only the router needs the canonical order.
template <int H, class Slot>
DEV void stage_xn(const float* __restrict__ x, const float* __restrict__ nw, float eps, float4* xs, Slot slot) {
  __shared__ float red[4];
  const float4* x4 = reinterpret_cast<const float4*>(x);
  constexpr int PER = H / 4 / 256;
  float4 v[PER], w[PER];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) v[i] = x4[threadIdx.x + 256 * i];
  if (nw) {
    const float4* n4 = reinterpret_cast<const float4*>(nw);
#pragma unroll
    for (int i = 0; i < PER; ++i) w[i] = n4[threadIdx.x + 256 * i];
#pragma unroll
    for (int i = 0; i < PER; ++i) ss += v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w;
    ss = wave_sum(ss);
    if (lane_id() == 0) red[wave_id()] = ss;
    __syncthreads();
    const float inv = rsqrtf((red[0] + red[1] + red[2] + red[3]) / (float)H + eps);
#pragma unroll
    for (int i = 0; i < PER; ++i)
      v[i] = make_float4(v[i].x * inv * w[i].x, v[i].y * inv * w[i].y, v[i].z * inv * w[i].z, v[i].w * inv * w[i].w);
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) xs[slot(threadIdx.x + 256 * i)] = v[i];
  __syncthreads();
}

// lane slices of 8 float4 (32 floats) per lane: f -> (f & 7) * 64 + (f >> 3) within 512-float4 parts
struct SlotQ4 {
  DEV int operator()(int f) const { return (f & ~511) + (f & 7) * 64 + ((f & 511) >> 3); }
};
// int8 K = 2048 rows read as bytes [16 l, 16 l + 16) and [1024 + 16 l, ...): 4 float4 per lane per half
struct SlotQ8H {
  DEV int operator()(int f) const { return (f & ~255) + (f & 3) * 64 + ((f & 255) >> 2); }
};

// B decode rows (B = 1: the engine's batch-1 call): routed blocks serve row blockIdx.y, the
// shared-expert blocks of row 0 serve every row with one read of their weights.  Row r uses
// x + r H, idx + r topk and act + r (topk + 1) I.
template <class SC, class SH, int B>
__global__ void __launch_bounds__(256)
    k_moe_gate_up_q4(const uint8_t* __restrict__ Q, const uint32_t* __restrict__ SM, const int8_t* __restrict__ shq,
                     const uint16_t* __restrict__ shs, const float* __restrict__ x, const int* __restrict__ idx,
                     float* __restrict__ act, const float* __restrict__ nw, float eps) {
  constexpr int H = DEC_H, I = DEC_I;
  __shared__ float4 xs[H / 4];
  const int lane = lane_id(), wave = wave_id();
  if (blockIdx.x < GU_NB_ROUTED) {
    const int row = B > 1 ? (int)blockIdx.y : 0;
    x += (size_t)row * H, idx += row * DEC_TOPK, act += (size_t)row * (DEC_TOPK + 1) * I;
    constexpr int BPE = GU_NB_ROUTED / DEC_TOPK;  // blocks per expert
    const int k = blockIdx.x / BPE, jb = blockIdx.x % BPE;
    const size_t e = (size_t)idx[k];
    const uint8_t* q = Q + e * (2 * I) * (H / 2) + lane * 16;
    const uint32_t* sm = SM + e * (2 * I) * (H / 64) + (lane >> 1);
    uint4 wg[GU_PPW], wu[GU_PPW];
    uint32_t sg[GU_PPW], su[GU_PPW];
#pragma unroll
    for (int p = 0; p < GU_PPW; ++p) {
      const int j = (jb * GU_WPB + wave) * GU_PPW + p;
      wg[p] = ld16(q + (size_t)j * (H / 2));
      wu[p] = ld16(q + (size_t)(I + j) * (H / 2));
      sg[p] = sm[(size_t)j * (H / 64)];
      su[p] = sm[(size_t)(I + j) * (H / 64)];
    }
    stage_xn<H>(x, nw, eps, xs, SlotQ4{});
    float xv[32], xsum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 v = xs[i * 64 + lane];
      xv[4 * i] = v.x, xv[4 * i + 1] = v.y, xv[4 * i + 2] = v.z, xv[4 * i + 3] = v.w;
      xsum += (v.x + v.y) + (v.z + v.w);
    }
#pragma unroll
    for (int p = 0; p < GU_PPW; ++p) {
      float qg = 0.f, qu = 0.f;
      qg = dot8_q4(wg[p].x, xv + 0, qg), qu = dot8_q4(wu[p].x, xv + 0, qu);
      qg = dot8_q4(wg[p].y, xv + 8, qg), qu = dot8_q4(wu[p].y, xv + 8, qu);
      qg = dot8_q4(wg[p].z, xv + 16, qg), qu = dot8_q4(wu[p].z, xv + 16, qu);
      qg = dot8_q4(wg[p].w, xv + 24, qg), qu = dot8_q4(wu[p].w, xv + 24, qu);
      const float2 a = SC::pair(sg[p]), b = SC::pair(su[p]);
      const float g = wave_sum(a.x * qg + a.y * xsum);
      const float u = wave_sum(b.x * qu + b.y * xsum);
      const int j = (jb * GU_WPB + wave) * GU_PPW + p;
      if (lane == 0) act[k * I + j] = silu(g) * u;
    }
  } else {
    // shared expert, int8 [2I, H]: lane reads bytes [16 l, 16 l + 16) and [1024 + 16 l, ...)
    if (B > 1 && blockIdx.y != 0) return;
    const int j = (blockIdx.x - GU_NB_ROUTED) * GU_WPB + wave;
    const int8_t* rg = shq + (size_t)j * H + lane * 16;
    const int8_t* ru = shq + (size_t)(I + j) * H + lane * 16;
    const uint4 g0 = ld16(rg), g1 = ld16(rg + 1024), u0 = ld16(ru), u1 = ld16(ru + 1024);
    const float sg0 = SH::scale(shs, j, lane * 16, H), sg1 = SH::scale(shs, j, 1024 + lane * 16, H);
    const float su0 = SH::scale(shs, I + j, lane * 16, H), su1 = SH::scale(shs, I + j, 1024 + lane * 16, H);
    for (int row = 0; row < B; ++row) {
    if (row) __syncthreads();  // every wave has read the previous row's inputs
    stage_xn<H>(x + (size_t)row * H, nw, eps, xs, SlotQ8H{});
    float xa[16], xb[16], sa = 0.f, sb = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 v = xs[i * 64 + lane], w = xs[256 + i * 64 + lane];
      xa[4 * i] = v.x, xa[4 * i + 1] = v.y, xa[4 * i + 2] = v.z, xa[4 * i + 3] = v.w;
      xb[4 * i] = w.x, xb[4 * i + 1] = w.y, xb[4 * i + 2] = w.z, xb[4 * i + 3] = w.w;
      sa += (v.x + v.y) + (v.z + v.w);
      sb += (w.x + w.y) + (w.z + w.w);
    }
    float ga = 0.f, gb = 0.f, ua = 0.f, ub = 0.f;
    const uint32_t gw0[4] = {g0.x, g0.y, g0.z, g0.w}, gw1[4] = {g1.x, g1.y, g1.z, g1.w};
    const uint32_t uw0[4] = {u0.x, u0.y, u0.z, u0.w}, uw1[4] = {u1.x, u1.y, u1.z, u1.w};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      ga = dot4_u8b(gw0[d], xa + 4 * d, ga), gb = dot4_u8b(gw1[d], xb + 4 * d, gb);
      ua = dot4_u8b(uw0[d], xa + 4 * d, ua), ub = dot4_u8b(uw1[d], xb + 4 * d, ub);
    }
    const float g = wave_sum(sg0 * (ga - 128.f * sa) + sg1 * (gb - 128.f * sb));
    const float u = wave_sum(su0 * (ua - 128.f * sa) + su1 * (ub - 128.f * sb));
    if (lane == 0) act[(size_t)row * (DEC_TOPK + 1) * I + DEC_TOPK * I + j] = silu(g) * u;
    }
  }
}

// B decode rows: each wave owns output rows n0, n0 + 1 of every row r (routed rows of row r's
// experts, one read of the shared rows for all B), the activations of all rows staged in LDS.
template <class SC, class SH, int B>
__global__ void __launch_bounds__(256)
    k_moe_down_q4(const uint8_t* __restrict__ Q, const uint32_t* __restrict__ SM, const int8_t* __restrict__ shq,
                  const uint16_t* __restrict__ shs, const float* __restrict__ act, const int* __restrict__ idx,
                  const float* __restrict__ wts, const float* __restrict__ sgate, const float* res, float* y,
                  uint16_t* yb, const char* pf, size_t pf_bytes) {
  constexpr int H = DEC_H, I = DEC_I, AW = (DEC_TOPK + 1) * I / 4;  // act float4 per row
  __shared__ float4 as[B * AW];
  const int lane = lane_id(), wave = wave_id();
  const int ka = lane >> 4, cc = lane & 15;
  const int n0 = (blockIdx.x * DN_WPB + wave) * DN_RPW;
  uint4 qa[B][DN_RPW], qb[B][DN_RPW];
  uint32_t sa[B][DN_RPW], sb[B][DN_RPW];
  uint2 qs[DN_RPW];
  float ss[DN_RPW];
#pragma unroll
  for (int b = 0; b < B; ++b) {
    const size_t ea = (size_t)idx[b * DEC_TOPK + ka], eb = (size_t)idx[b * DEC_TOPK + 4 + ka];
#pragma unroll
    for (int r = 0; r < DN_RPW; ++r) {
      const size_t n = (size_t)(n0 + r);
      qa[b][r] = ld16(Q + (ea * H + n) * (I / 2) + cc * 16);
      qb[b][r] = ld16(Q + (eb * H + n) * (I / 2) + cc * 16);
      sa[b][r] = ld4(SM + (ea * H + n) * (I / 64) + (cc >> 1));
      sb[b][r] = ld4(SM + (eb * H + n) * (I / 64) + (cc >> 1));
    }
  }
#pragma unroll
  for (int r = 0; r < DN_RPW; ++r) {
    const size_t n = (size_t)(n0 + r);
    qs[r] = ld8(shq + n * I + lane * 8);
    ss[r] = SH::scale(shs, n, lane * 8, I);
  }
  // stage act: routed part as two 512-float4 halves with the 8-per-lane swizzle, shared part
  // (128 float4) with 2 per lane
#pragma unroll
  for (int b = 0; b < B; ++b) {
    const float4* a4 = reinterpret_cast<const float4*>(act + (size_t)b * (DEC_TOPK + 1) * I);
    float4* ab = as + b * AW;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int f = threadIdx.x + 256 * i;
      ab[(f & ~511) + (f & 7) * 64 + ((f & 511) >> 3)] = a4[f];
    }
    if (threadIdx.x < 128) {
      const int f = threadIdx.x;
      ab[1024 + (f & 1) * 64 + (f >> 1)] = a4[1024 + f];
    }
  }
  __syncthreads();
#pragma unroll
  for (int b = 0; b < B; ++b) {
    const float4* ab = as + b * AW;
    float xa[32], xb[32], xc[8];
    float suma = 0.f, sumb = 0.f, sumc = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 v = ab[i * 64 + lane], w = ab[512 + i * 64 + lane];
      xa[4 * i] = v.x, xa[4 * i + 1] = v.y, xa[4 * i + 2] = v.z, xa[4 * i + 3] = v.w;
      xb[4 * i] = w.x, xb[4 * i + 1] = w.y, xb[4 * i + 2] = w.z, xb[4 * i + 3] = w.w;
      suma += (v.x + v.y) + (v.z + v.w);
      sumb += (w.x + w.y) + (w.z + w.w);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const float4 v = ab[1024 + i * 64 + lane];
      xc[4 * i] = v.x, xc[4 * i + 1] = v.y, xc[4 * i + 2] = v.z, xc[4 * i + 3] = v.w;
      sumc += (v.x + v.y) + (v.z + v.w);
    }
    const float wa = wts[b * DEC_TOPK + ka], wb = wts[b * DEC_TOPK + 4 + ka];
    const float sgv = sigmoid(sgate[b]);
#pragma unroll
    for (int r = 0; r < DN_RPW; ++r) {
      float da = 0.f, db = 0.f;
      da = dot8_q4(qa[b][r].x, xa + 0, da), db = dot8_q4(qb[b][r].x, xb + 0, db);
      da = dot8_q4(qa[b][r].y, xa + 8, da), db = dot8_q4(qb[b][r].y, xb + 8, db);
      da = dot8_q4(qa[b][r].z, xa + 16, da), db = dot8_q4(qb[b][r].z, xb + 16, db);
      da = dot8_q4(qa[b][r].w, xa + 24, da), db = dot8_q4(qb[b][r].w, xb + 24, db);
      float dc = dot4_u8b(qs[r].x, xc, 0.f);
      dc = dot4_u8b(qs[r].y, xc + 4, dc);
      const float2 pa = SC::pair(sa[b][r]), pb = SC::pair(sb[b][r]);
      float acc = wa * (pa.x * da + pa.y * suma) + wb * (pb.x * db + pb.y * sumb) + sgv * ss[r] * (dc - 128.f * sumc);
      acc = wave_sum(acc);
      const size_t n = (size_t)b * H + n0 + r;
      if (lane == 0) {
        const float out = res[n] + acc;
        y[n] = out;
        if (yb) yb[n] = to_bf16(out);
      }
    }
  }
  warm_range(pf, pf_bytes);
}

template <class SC, class SH, int B>
void launch_decode_b(const uint8_t* gu_q, const void* gu_sm, const uint8_t* d_q, const void* d_sm,
                     const int8_t* sgu_q, const uint16_t* sgu_s, const int8_t* sd_q, const uint16_t* sd_s,
                     const float* x, const int* idx, const float* wts, const float* sgate, const float* res, float* act,
                     float* y, uint16_t* yb, const float* nw, float eps, const char* pf, size_t pf_bytes,
                     hipStream_t st) {
  hipLaunchKernelGGL((k_moe_gate_up_q4<SC, SH, B>), dim3(GU_NB_ROUTED + GU_NB_SHARED, B), dim3(256), 0, st, gu_q,
                     (const uint32_t*)gu_sm, sgu_q, sgu_s, x, idx, act, nw, eps);
  hipLaunchKernelGGL((k_moe_down_q4<SC, SH, B>), dim3(DEC_H / (DN_WPB * DN_RPW)), dim3(256), 0, st, d_q,
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

// Device helpers shared by the gfx950 kernels of the MoE path.
//
// Everything here is written for CDNA4 wave64: a "wave" is 64 lanes, reductions are xor
// butterflies over 64 lanes.  Half-precision values travel as raw 16-bit patterns.
#pragma once
#include <type_traits>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#define DEV __device__ __forceinline__
#define API extern "C" __attribute__((visibility("default")))

namespace drm {

constexpr int WAVE = 64;

// Library error word: one host-mapped pinned word shared by every device, written by a kernel
// whose bounded wait gave up (system-scope store) and read by the host without synchronising
// (dr_last_error, dr_stream_sync, the launchers).  err_word() returns its device address,
// nullptr if it could not be set up; err_pending() the current code (0 = none).
// Codes (the header's DR_ERR_STEP_TIMEOUT / DR_ERR_PREFILL_WAIT / DR_ERR_ROUTE_WAIT).
constexpr uint32_t kErrStepTimeout = 9001, kErrPrefillWait = 9002, kErrRouteWait = 9003;
uint32_t* err_word();
uint32_t* err_word_noalloc();  // the address if already set up (at library load), else nullptr; never allocates
uint32_t err_pending();

DEV void raise_err(uint32_t* err, uint32_t code) {
  if (err) __hip_atomic_store(err, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Loads from global memory, explicitly in the global address space: a pointer read out of a
// table (rather than passed as a kernel argument) is otherwise generic, and generic (flat)
// loads count against both the vector-memory and the LDS counters, so every wait for an LDS
// value would also wait for all weight loads in flight.
typedef uint32_t gu32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t gu32x2 __attribute__((ext_vector_type(2)));
template <class T>
DEV T gld(const void* p) {
  return *(const __attribute__((address_space(1))) T*)p;
}
DEV uint4 ld16(const void* p) {
  const gu32x4 v = gld<gu32x4>(p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
DEV uint2 ld8(const void* p) {
  const gu32x2 v = gld<gu32x2>(p);
  return make_uint2(v.x, v.y);
}
// Keeps the loads issued before this point ahead of those issued after it (a compiler memory
// barrier, which also stops loads from being sunk towards their first use, and a scheduling
// barrier).  A wave's loads return in order, so staging loads issued first do not wait for
// the weight loads behind them.
DEV void issue_fence() {
  __builtin_amdgcn_sched_barrier(0);
}
DEV float4 ldf4(const void* p) {
  const gu32x4 v = gld<gu32x4>(p);
  return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}
DEV uint32_t ld4(const void* p) { return gld<uint32_t>(p); }
DEV uint32_t ld2(const void* p) { return gld<uint16_t>(p); }

DEV float bf16f(uint32_t h) { return __uint_as_float(h << 16); }
DEV float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
DEV float bf16_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }
DEV float f16f(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

// Round-to-nearest-even fp32 -> bf16 bits (NaN stays NaN).
DEV uint16_t to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Cross-lane exchange for the ascending xor butterfly o = 1, 2, 4, 8, 16, 32.
//   o = 1, 2: DPP quad_perm, the exact xor partner;
//   o = 4, 8: DPP row_half_mirror / row_mirror (lane 7 - i, 15 - i); after the lower steps every
//             quad (octet) holds one value, so the mirrored lane carries the xor partner's bits;
//   o = 16, 32: v_permlane16_swap / v_permlane32_swap of the value with itself, which hands
//             every lane both halves (lo, hi) of the pair.
// Every combine is a commutative op on the two halves, so all 64 lanes end with identical bits
// and the result is one fixed tree: step o combines a[l] and a[l ^ o].  All lanes must be active.
template <int O>
DEV void xchg(float v, float& lo, float& hi) {
  if constexpr (O == 1 || O == 2 || O == 4 || O == 8) {
    constexpr int ctrl = O == 1 ? 0xB1 : O == 2 ? 0x4E : O == 4 ? 0x141 : 0x140;
    lo = v;
    // bound_ctrl set: with full row and bank masks every lane has a valid source, so it changes
    // no value, and it lets the compiler fold the move into the combining instruction
    hi = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), ctrl, 0xF, 0xF, true));
  } else if constexpr (O == 16) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    lo = __uint_as_float(r[0]), hi = __uint_as_float(r[1]);
  } else {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    lo = __uint_as_float(r[0]), hi = __uint_as_float(r[1]);
  }
}

template <int O>
DEV float xsum_step(float v) {
  float a, b;
  xchg<O>(v, a, b);
  return a + b;
}

// Sum over the wave with the ascending xor tree (see xchg); every lane gets the same bits.
DEV float wave_sum(float v) {
  v = xsum_step<1>(v);
  v = xsum_step<2>(v);
  v = xsum_step<4>(v);
  v = xsum_step<8>(v);
  v = xsum_step<16>(v);
  return xsum_step<32>(v);
}

template <int O>
DEV float xmax_step(float v) {
  float a, b;
  xchg<O>(v, a, b);
  return fmaxf(a, b);
}

DEV float wave_max(float v) {
  v = xmax_step<1>(v);
  v = xmax_step<2>(v);
  v = xmax_step<4>(v);
  v = xmax_step<8>(v);
  v = xmax_step<16>(v);
  return xmax_step<32>(v);
}

// (value, index) pair of the wave maximum: larger value first, lower index on ties.
template <int O>
DEV void xarg_step(float& v, int& i) {
  float va, vb, ia, ib;
  xchg<O>(v, va, vb);
  xchg<O>(__int_as_float(i), ia, ib);
  const int a = __float_as_int(ia), b = __float_as_int(ib);
  const bool take_b = vb > va || (vb == va && b < a);
  v = take_b ? vb : va;
  i = take_b ? b : a;
}

DEV void wave_argmax(float& v, int& i) {
  xarg_step<1>(v, i);
  xarg_step<2>(v, i);
  xarg_step<4>(v, i);
  xarg_step<8>(v, i);
  xarg_step<16>(v, i);
  xarg_step<32>(v, i);
}

// Workgroup barrier that orders LDS only: global loads in flight stay in flight across it.
DEV void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Block-FP8 helpers: one scale per 128 x 128 block, f32 (SF = 0, the reference's scale_inv)
// or bf16 (SF = 1); e4m3 bytes convert to f32 exactly with v_cvt_pk_f32_fp8.
template <int SF>
DEV uint32_t blk_raw(const void* S, size_t i) {
  return SF ? ld2(reinterpret_cast<const uint16_t*>(S) + i) : ld4(reinterpret_cast<const float*>(S) + i);
}
template <int SF>
DEV float blk_cvt(uint32_t r) {
  return SF ? bf16f(r) : __uint_as_float(r);
}
template <int SF>
DEV float blk_scale(const void* S, size_t i) {
  return blk_cvt<SF>(blk_raw<SF>(S, i));
}

// sum_{i<16} e4m3(w bytes) * x[i]
DEV float dot16_fp8(const uint4& w, const float* x, float acc) {
  const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(ww[d], false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(ww[d], true);
    acc = __builtin_fmaf(lo[0], x[4 * d + 0], acc);
    acc = __builtin_fmaf(lo[1], x[4 * d + 1], acc);
    acc = __builtin_fmaf(hi[0], x[4 * d + 2], acc);
    acc = __builtin_fmaf(hi[1], x[4 * d + 3], acc);
  }
  return acc;
}

DEV int lane_id() { return (int)(threadIdx.x & (WAVE - 1)); }
DEV int wave_id() { return (int)(threadIdx.x >> 6); }

// Fast activations (tolerance paths only).
DEV float silu(float x) { return x / (1.f + __expf(-x)); }
DEV float sigmoid(float x) { return 1.f / (1.f + __expf(-x)); }

// int4 group scale/min pairs: one 32-bit word holds (scale, min) as two halves.
struct ScaleF16 {
  static DEV float2 pair(uint32_t w) { return make_float2(f16f(w & 0xffffu), f16f(w >> 16)); }
};
struct ScaleBF16 {
  static DEV float2 pair(uint32_t w) { return make_float2(bf16_lo(w), bf16_hi(w)); }
};

// int8 scale of element k of row n for a K-wide int8 matrix.
// raw() loads the scale's bits, cvt() converts them (so a load can be issued long before use).
struct Q8G128F16 {  // reference layout: f16 scale per 128 inputs, s [N, K/128]
  static DEV uint32_t raw(const uint16_t* s, size_t n, int k, int K) { return ld2(s + n * (K / 128) + (k >> 7)); }
  static DEV float cvt(uint32_t r) { return f16f(r); }
  static DEV float scale(const uint16_t* s, size_t n, int k, int K) { return cvt(raw(s, n, k, K)); }
  static constexpr bool per_row = false;
};
struct Q8RowBF16 {  // per-output-channel bf16 scale, s [N]
  static DEV uint32_t raw(const uint16_t* s, size_t n, int, int) { return ld2(s + n); }
  static DEV float cvt(uint32_t r) { return bf16f(r); }
  static DEV float scale(const uint16_t* s, size_t n, int k, int K) { return cvt(raw(s, n, k, K)); }
  static constexpr bool per_row = true;
};

// Sum of 8 int4 nibbles of w times x[0..7] (x[i] pairs with nibble i = bits 4i..4i+3).
// Masks the even and the odd nibbles into bytes so each value converts with one
// v_cvt_f32_ubyteN.
DEV float dot8_q4(uint32_t w, const float* x, float acc) {
  const uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
  acc = __builtin_fmaf((float)(lo & 0xff), x[0], acc);
  acc = __builtin_fmaf((float)(hi & 0xff), x[1], acc);
  acc = __builtin_fmaf((float)((lo >> 8) & 0xff), x[2], acc);
  acc = __builtin_fmaf((float)((hi >> 8) & 0xff), x[3], acc);
  acc = __builtin_fmaf((float)((lo >> 16) & 0xff), x[4], acc);
  acc = __builtin_fmaf((float)((hi >> 16) & 0xff), x[5], acc);
  acc = __builtin_fmaf((float)(lo >> 24), x[6], acc);
  acc = __builtin_fmaf((float)(hi >> 24), x[7], acc);
  return acc;
}

// ---- int4 dots against fixed-point digits of x ---------------------------------------------
// A 32-input chunk c of x (the chunk lane c of an int4 row dot owns) is written as 24-bit fixed
// point X = x 2^S, S per chunk from its largest exponent e (every |x| < 2^e, S = 22 - e, so
// |X| <= 2^22), in six balanced base-16 digits: V = (X + 0x888888) ^ 0x888888 has digit k of X
// as the int4 nibble k.  Digit k of the 8 inputs of group g of the chunk is one word (nibble i =
// input 8 g + i, as the weight words), at word ((j >> 2) * 64 + c) * 4 + (j & 3), j = 6 g + k,
// so lane c reads its 24 words as six 16-byte LDS reads with no bank conflicts.  A weight word
// xor 0x88888888 holds q - 8 as int4 nibbles, and sum (q - 8) X is six exact v_dot8 sums;
// q4_dot_digits returns it as a float (one rounding) and the caller forms
// w . x = s 2^-S sum (q - 8) X + (m + 8 s) sum x.
// Staging: the 8 threads of a chunk (consecutive lanes, part = lane & 7, thread part holding
// inputs 4 part .. 4 part + 3 as xn) each call q4_digits_stage; it also leaves the chunk's sum
// in csum[c] and 2^-S in cscale[c].
DEV void q4_digits_stage(float4 xn, int c, int part, uint32_t* xd, float* csum, float* cscale) {
  float t = (xn.x + xn.y) + (xn.z + xn.w);
  t = xsum_step<1>(t), t = xsum_step<2>(t), t = xsum_step<4>(t);
  float mx = fmaxf(fmaxf(fabsf(xn.x), fabsf(xn.y)), fmaxf(fabsf(xn.z), fabsf(xn.w)));
  mx = xmax_step<1>(mx), mx = xmax_step<2>(mx), mx = xmax_step<4>(mx);
  const int e = (int)((__float_as_uint(mx) >> 23) & 0xff) - 126;
  const int sh = 22 - e;
  if (part == 0) csum[c] = t, cscale[c] = __builtin_ldexpf(1.f, -sh);
  const float xv4[4] = {xn.x, xn.y, xn.z, xn.w};
  uint32_t V[4];
#pragma unroll
  for (int t4 = 0; t4 < 4; ++t4) V[t4] = ((uint32_t)__float2int_rn(__builtin_ldexpf(xv4[t4], sh)) + 0x888888u) ^ 0x888888u;
  // this thread holds inputs 4 h .. 4 h + 3 of group gi: half h of each digit word
  uint16_t* xh = reinterpret_cast<uint16_t*>(xd);
  const int gi = part >> 1, h = part & 1;
#pragma unroll
  for (int k = 0; k < 6; ++k) {
    const uint32_t hw = ((V[0] >> (4 * k)) & 15u) | (((V[1] >> (4 * k)) & 15u) << 4) |
                        (((V[2] >> (4 * k)) & 15u) << 8) | (((V[3] >> (4 * k)) & 15u) << 12);
    const int j = gi * 6 + k;
    xh[(((j >> 2) * 64 + c) * 4 + (j & 3)) * 2 + h] = (uint16_t)hw;
  }
}
DEV void q4_digits_load(const uint32_t* xd, int lane, uint32_t (&dg)[24]) {
  const uint4* xd4 = reinterpret_cast<const uint4*>(xd);
#pragma unroll
  for (int j = 0; j < 6; ++j) {
    const uint4 v = xd4[j * 64 + lane];
    dg[4 * j] = v.x, dg[4 * j + 1] = v.y, dg[4 * j + 2] = v.z, dg[4 * j + 3] = v.w;
  }
}
// sum over the lane's 32 inputs of (q - 8) X for the weight words w (inputs 8 g .. 8 g + 7 in w[g])
DEV float q4_dot_digits(const uint4& w, const uint32_t (&dg)[24]) {
  const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
  int a[6] = {0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int q = (int)(ww[g] ^ 0x88888888u);
#pragma unroll
    for (int k = 0; k < 6; ++k) a[k] = __builtin_amdgcn_sdot8(q, (int)dg[6 * g + k], a[k], false);
  }
  float d = (float)a[5];
#pragma unroll
  for (int k = 4; k >= 0; --k) d = __builtin_fmaf(d, 16.f, (float)a[k]);
  return d;
}

// Sum of 4 int8 values of w times x[0..3], computed as sum((b ^ 0x80) x) - 128 sum(x): the
// caller subtracts 128 * sum(x) once per row slice.
DEV float dot4_u8b(uint32_t w, const float* x, float acc) {
  const uint32_t u = w ^ 0x80808080u;
  acc = __builtin_fmaf((float)(u & 0xff), x[0], acc);
  acc = __builtin_fmaf((float)((u >> 8) & 0xff), x[1], acc);
  acc = __builtin_fmaf((float)((u >> 16) & 0xff), x[2], acc);
  acc = __builtin_fmaf((float)(u >> 24), x[3], acc);
  return acc;
}



// Touch [pf, pf + bytes) so the data sits in the memory-side cache (MALL) for the next
// kernel.  Each block takes an equal share; the loaded words are folded into a register
// that an empty asm statement consumes, so the loads stay live.
DEV void warm_range(const char* pf, size_t bytes) {
  if (!pf || !bytes) return;
  const size_t nb = (size_t)gridDim.x * gridDim.y;
  const size_t b = (size_t)blockIdx.y * gridDim.x + blockIdx.x;
  const size_t per = ((bytes + nb - 1) / nb + 255) & ~(size_t)255;
  const size_t b0 = b * per, b1 = b0 + per < bytes ? b0 + per : bytes;
  uint32_t acc = 0;
  for (size_t o = b0 + threadIdx.x * 64; o + 16 <= b1; o += (size_t)blockDim.x * 64) acc ^= ld16(pf + o).x;
  asm volatile("" ::"v"(acc));
}

// LDS layouts of staged inputs.  SlotQ8H (float4 f -> slot): lane l reads the 16 inputs
// [16 l, 16 l + 16) of each 1024-input half as 4 float4.  SlotQ4D: the row as the int4 dots'
// fixed-point digits (q4_digits_stage; H = 2048): lane l's 32-input chunk as 24 digit words in
// the first 6 KB of the row's 8 KB, then the 64 chunk sums and the 64 scales 2^-S.
struct SlotQ4D {};
struct SlotQ8H {
  DEV int operator()(int f) const { return (f & ~255) + (f & 3) * 64 + ((f & 255) >> 2); }
};

// Stage NR rows of RMSNorm(x) (nw == nullptr: x itself) in LDS, float4 f of a row at
// Slot{}(f) (SlotQ8H: the 16-element lane chunks of byte rows read as two 1024-byte halves), or
// as the digits of SlotQ4D.  load() issues the global loads unconditionally and ahead of everything issued after
// it (loads return in order, so weight loads issued later do not delay the staging);
// finish() reduces (partial sums added in wave order), normalises and writes LDS.  Every
// thread of the block calls both.
template <int H, int NT, int NR, class Slot>
struct XStage {
  static constexpr int NWV = NT / WAVE, PER = H / 4 / NT;
  float4 v[NR][PER], w[PER];
  DEV void load(const float* x, const float* nw) {
    const float4* x4 = reinterpret_cast<const float4*>(x);
    const float4* n4 = reinterpret_cast<const float4*>(nw ? nw : x);
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
      for (int i = 0; i < PER; ++i) v[r][i] = ldf4(x4 + r * (H / 4) + threadIdx.x + NT * i);
#pragma unroll
    for (int i = 0; i < PER; ++i) w[i] = ldf4(n4 + threadIdx.x + NT * i);
    issue_fence();
  }
  DEV void finish(bool norm, float eps, float4* xs) {
    __shared__ float red[NR][NWV];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < PER; ++i)
        ss += v[r][i].x * v[r][i].x + v[r][i].y * v[r][i].y + v[r][i].z * v[r][i].z + v[r][i].w * v[r][i].w;
      ss = wave_sum(ss);
      if (lane_id() == 0) red[r][wave_id()] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      float t = red[r][0];
#pragma unroll
      for (int q = 1; q < NWV; ++q) t += red[r][q];
      // without a norm weight: x * 1 * 1 == x exactly
      const float inv = norm ? rsqrtf(t / (float)H + eps) : 1.f;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const float wx = norm ? w[i].x : 1.f, wy = norm ? w[i].y : 1.f, wz = norm ? w[i].z : 1.f,
                    ww = norm ? w[i].w : 1.f;
        v[r][i] = make_float4(v[r][i].x * inv * wx, v[r][i].y * inv * wy, v[r][i].z * inv * wz, v[r][i].w * inv * ww);
      }
    }
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int f = threadIdx.x + NT * i;
        if constexpr (std::is_same<Slot, SlotQ4D>::value) {
          float* rb = reinterpret_cast<float*>(xs + r * (H / 4));
          q4_digits_stage(v[r][i], f >> 3, f & 7, reinterpret_cast<uint32_t*>(rb), rb + 1536, rb + 1600);
        } else {
          xs[r * (H / 4) + Slot{}(f)] = v[r][i];
        }
      }
    __syncthreads();
  }
};

// Keeps weight registers opaque at this point, so the compiler cannot convert them to float
// earlier (ahead of the input staging, or once outside a loop over rows): expanded to fp32,
// every 16 bytes of weights would hold 16 registers.
DEV void opaque(uint4& w) {
  uint32_t a = w.x, b = w.y, c = w.z, d = w.w;
  asm volatile("" : "+v"(a), "+v"(b), "+v"(c), "+v"(d));
  w = make_uint4(a, b, c, d);
}
template <int PPW>
DEV void pin_weights(uint4 (&g0)[PPW], uint4 (&g1)[PPW], uint4 (&u0)[PPW], uint4 (&u1)[PPW]) {
#pragma unroll
  for (int p = 0; p < PPW; ++p) opaque(g0[p]), opaque(g1[p]), opaque(u0[p]), opaque(u1[p]);
}

}  // namespace drm

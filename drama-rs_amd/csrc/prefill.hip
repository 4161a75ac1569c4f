// Prefill expert-grouped GEMM on the CDNA4 matrix cores (reference: kernels/drama.cu:799-1109,
// src/ffi.rs:52-54,60-63) and the fused int8 shared-expert prefill (src/engine.rs:560-562).
//
// Rows of xp are sorted by expert; expert e owns rows [offsets[e], offsets[e] + counts[e]).
// gate_up: act[t] = bf16(silu(G_e . x_t) * (U_e . x_t)); down: y[t] = D_e . act_t (fp32).
//
// One wave owns a 16-row tile of weight rows (for gate_up: 16 gate rows and the 16 matching
// up rows) and computes it against up to 64 tokens of its expert with
// v_mfma_f32_16x16x32_bf16: A = weights (16 x 32), B = tokens (32 x 16), D = 16 x 16 fp32.
// Weights are dequantised exactly in registers: an int4 nibble q becomes the bf16 value
// 128 + q (bit pattern 0x4300 | q), an int8 or fp8 value converts to bf16 exactly.  Each MFMA
// stays inside one scale group, so per group g the fp32 product sum acc_g is rescaled:
//   int4:  out += s_g acc_g + (m_g - 128 s_g) X_g,  X_g = sum of the group's inputs
//   int8 / fp8:  out += s_g acc_g  (one scale per 128 inputs, or one per row at the end)
// which is w = q s + m applied after exact integer x bf16 products: the same values as
// dequantise-then-fp32, accumulated in fp32.
//
// Lane l of a wave holds, for MFMA step s (two per 64-wide group G), weight row (l % 16) and
// the 8 inputs k = 64 G + 16 (l / 16) + 8 s + perm(t), t = 0..7, where perm = 0 4 1 5 2 6 3 7
// is the order in which the nibble masking (w >> 4 j) & 0x000f000f produces bf16 pairs.  The
// token tile in LDS is stored in the same permuted order, so each B fragment is one 16-byte
// LDS read.
#include "common.hpp"

using namespace drm;

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int PF_WPB = 8;     // waves per block
constexpr int PF_TOK = 64;    // tokens per pass (4 token tiles of 16)
constexpr int PF_KC = 256;    // inputs per LDS chunk (4 groups of 64)
constexpr int PF_MAXE = 256;  // experts

DEV f32x4 mfma(const uint4& a, const uint4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
                                                 0);
}

// ---- weight formats: per lane and 64-wide group, two MFMA A fragments -------------------------

// int4, (scale, min) pairs per 64 inputs; SC = ScaleF16 | ScaleBF16
template <class SC>
struct FmtQ4 {
  static constexpr bool has_min = true;
  static constexpr int scale_group = 64;  // inputs per scale
  static DEV size_t row_bytes(int K) { return (size_t)K / 2; }
  // fragment bytes of (row, group G) for lane group g: 8 bytes = 16 nibbles
  static DEV void load(const uint8_t* row, int G, int g, uint2& raw) { raw = ld8(row + G * 32 + g * 8); }
  static DEV void convert(const uint2& raw, uint4& a0, uint4& a1) {
    const uint32_t m = 0x000f000fu, b = 0x43004300u;
    a0 = make_uint4((raw.x & m) | b, ((raw.x >> 4) & m) | b, ((raw.x >> 8) & m) | b, ((raw.x >> 12) & m) | b);
    a1 = make_uint4((raw.y & m) | b, ((raw.y >> 4) & m) | b, ((raw.y >> 8) & m) | b, ((raw.y >> 12) & m) | b);
  }
  // (scale, min) of row n, group G
  static DEV float2 scale(const void* S, size_t n, int G, int K) {
    return SC::pair(reinterpret_cast<const uint32_t*>(S)[n * (K / 64) + G]);
  }
};

// element order inside an 8-element fragment: perm = 0 4 1 5 2 6 3 7
// int8: 16 bytes per lane and group; bytes k..k+15 of the group slice, reordered
template <class SH>
struct FmtQ8 {
  static constexpr bool has_min = false;
  static constexpr int scale_group = SH::per_row ? 0 : 128;
  static DEV size_t row_bytes(int K) { return (size_t)K; }
  static DEV void load(const uint8_t* row, int G, int g, uint4& raw) { raw = ld16(row + G * 64 + g * 16); }
  static DEV uint32_t pk(int a, int b) {  // two int8 values -> bf16 pair (exact: |v| <= 127)
    return (__float_as_uint((float)b) & 0xffff0000u) | (__float_as_uint((float)a) >> 16);
  }
  static DEV int sb(uint32_t w, int i) { return (int)(int8_t)(w >> (8 * i)); }
  // 8 bytes (two words) -> fragment in perm order: slots (e0,e4) (e1,e5) (e2,e6) (e3,e7)
  static DEV uint4 frag(uint32_t lo, uint32_t hi) {
    return make_uint4(pk(sb(lo, 0), sb(hi, 0)), pk(sb(lo, 1), sb(hi, 1)), pk(sb(lo, 2), sb(hi, 2)), pk(sb(lo, 3), sb(hi, 3)));
  }
  static DEV void convert(const uint4& raw, uint4& a0, uint4& a1) {
    a0 = frag(raw.x, raw.y);
    a1 = frag(raw.z, raw.w);
  }
  static DEV float2 scale(const void* S, size_t n, int G, int K) {
    return make_float2(SH::scale(reinterpret_cast<const uint16_t*>(S), n, G * 64, K), 0.f);
  }
};

// fp8 e4m3 (OCP), one scale per 128 x 128 block; SF: 0 = f32 scales, 1 = bf16 scales
template <int SF>
struct FmtFP8 {
  static constexpr bool has_min = false;
  static constexpr int scale_group = 128;
  static DEV size_t row_bytes(int K) { return (size_t)K; }
  static DEV void load(const uint8_t* row, int G, int g, uint4& raw) { raw = ld16(row + G * 64 + g * 16); }
  static DEV uint32_t pk(float a, float b) { return (__float_as_uint(b) & 0xffff0000u) | (__float_as_uint(a) >> 16); }
  // e4m3 -> f32 is exact, and every e4m3 value is a bf16 value
  static DEV uint4 frag(uint32_t lo, uint32_t hi) {
    const float l0 = __builtin_amdgcn_cvt_f32_fp8(lo, 0), l1 = __builtin_amdgcn_cvt_f32_fp8(lo, 1);
    const float l2 = __builtin_amdgcn_cvt_f32_fp8(lo, 2), l3 = __builtin_amdgcn_cvt_f32_fp8(lo, 3);
    const float h0 = __builtin_amdgcn_cvt_f32_fp8(hi, 0), h1 = __builtin_amdgcn_cvt_f32_fp8(hi, 1);
    const float h2 = __builtin_amdgcn_cvt_f32_fp8(hi, 2), h3 = __builtin_amdgcn_cvt_f32_fp8(hi, 3);
    return make_uint4(pk(l0, h0), pk(l1, h1), pk(l2, h2), pk(l3, h3));
  }
  static DEV void convert(const uint4& raw, uint4& a0, uint4& a1) {
    a0 = frag(raw.x, raw.y);
    a1 = frag(raw.z, raw.w);
  }
  // scale of row n, 64-group G: block (n / 128, G / 2); S points at this expert's blocks
  static DEV float2 scale(const void* S, size_t n, int G, int K) {
    const size_t i = (n >> 7) * (size_t)(K / 128) + (G >> 1);
    return make_float2(SF ? bf16f(reinterpret_cast<const uint16_t*>(S)[i]) : reinterpret_cast<const float*>(S)[i], 0.f);
  }
};

template <class F>
struct Raw;
template <class SC>
struct Raw<FmtQ4<SC>> {
  using T = uint2;
};
template <class SH>
struct Raw<FmtQ8<SH>> {
  using T = uint4;
};
template <int SF>
struct Raw<FmtFP8<SF>> {
  using T = uint4;
};

// Stage tokens [t0, t0 + 64) x inputs [kc, kc + PF_KC) of a bf16 row matrix into LDS in the
// permuted fragment order, zero-filling tokens >= ntok; xsum[t][gi] = sum of the 64 inputs
// of group gi for token t (fp32).
DEV void stage_tokens(const uint16_t* __restrict__ X, size_t row0, int ntok, int K, int kc, uint4* xs, float* xsum) {
  constexpr int BLK = PF_TOK * PF_KC / 8;  // 16-byte blocks
  for (int b = threadIdx.x; b < BLK; b += PF_WPB * 64) {
    const int t = b / (PF_KC / 8), r = b % (PF_KC / 8);
    uint4 v = make_uint4(0, 0, 0, 0);
    if (t < ntok) v = ld16(X + (row0 + t) * (size_t)K + kc + r * 8);
    // (e0 e1)(e2 e3)(e4 e5)(e6 e7) -> (e0 e4)(e1 e5)(e2 e6)(e3 e7)
    const uint4 p = make_uint4(__builtin_amdgcn_perm(v.z, v.x, 0x05040100u), __builtin_amdgcn_perm(v.z, v.x, 0x07060302u),
                               __builtin_amdgcn_perm(v.w, v.y, 0x05040100u), __builtin_amdgcn_perm(v.w, v.y, 0x07060302u));
    xs[b] = p;
    float s = (bf16_lo(v.x) + bf16_hi(v.x)) + (bf16_lo(v.y) + bf16_hi(v.y)) + (bf16_lo(v.z) + bf16_hi(v.z)) +
              (bf16_lo(v.w) + bf16_hi(v.w));
    // the 8 blocks of one (token, group) are 8 consecutive threads
    s = xsum_step<1>(s);
    s = xsum_step<2>(s);
    s = xsum_step<4>(s);
    if ((r & 7) == 0) xsum[t * (PF_KC / 64) + (r >> 3)] = s;
  }
}

// MODE 0: gate_up (pairs of rows j, I + j; writes bf16 silu(g) u)   MODE 1: down (writes f32)
template <class F, int MODE>
__global__ void __launch_bounds__(PF_WPB * 64)
    k_grouped(const uint8_t* __restrict__ Wq, const void* __restrict__ Ws, const uint16_t* __restrict__ X,
              const int* __restrict__ offsets, const int* __restrict__ counts, void* __restrict__ out, int N, int K,
              size_t expert_q_bytes, size_t expert_s_elems, int s_elem_bytes, int fixed_rows) {
  __shared__ uint4 xs[PF_TOK * PF_KC / 8];
  __shared__ float xsum[PF_TOK * (PF_KC / 64)];
  // grouped: block x = expert; single matrix (fixed_rows >= 0): block x = 64-token pass
  const int e = fixed_rows >= 0 ? 0 : blockIdx.x;
  const int cnt = fixed_rows >= 0 ? min(PF_TOK, fixed_rows - (int)blockIdx.x * PF_TOK) : counts[e];
  if (cnt <= 0) return;
  const size_t off = fixed_rows >= 0 ? (size_t)blockIdx.x * PF_TOK : (size_t)offsets[e];
  const int lane = lane_id(), wave = wave_id();
  const int g = lane >> 4, c16 = lane & 15;
  const int tile = blockIdx.y * PF_WPB + wave;  // 16-row tile of output rows
  const int rows_out = MODE == 0 ? N / 2 : N;   // gate_up: N = 2I weight rows, I outputs
  const bool active = tile * 16 < rows_out;
  const int r0 = tile * 16;
  const uint8_t* wq = Wq + (size_t)e * expert_q_bytes;
  const char* ws = reinterpret_cast<const char*>(Ws) + (size_t)e * expert_s_elems * s_elem_bytes;
  const size_t rb = F::row_bytes(K);
  const uint8_t* rowA = wq + (size_t)(r0 + c16) * rb;                          // gate / down row
  const uint8_t* rowB = wq + (size_t)((MODE == 0 ? N / 2 : 0) + r0 + c16) * rb;  // up row (gate_up)
  for (int p0 = 0; p0 < cnt; p0 += PF_TOK) {
    const int ntok = min(PF_TOK, cnt - p0);
    const int ntiles = (ntok + 15) / 16;
    f32x4 totA[4], totB[4], accA[4], accB[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) totA[t] = totB[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int kc = 0; kc < K; kc += PF_KC) {
      // weights of this chunk first, so their latency overlaps the token staging
      typename Raw<F>::T rawA[PF_KC / 64], rawB[PF_KC / 64];
      if (active) {
#pragma unroll
        for (int gi = 0; gi < PF_KC / 64; ++gi) {
          F::load(rowA, kc / 64 + gi, g, rawA[gi]);
          if (MODE == 0) F::load(rowB, kc / 64 + gi, g, rawB[gi]);
        }
      }
      __syncthreads();
      stage_tokens(X, off + p0, ntok, K, kc, xs, xsum);
      __syncthreads();
      if (!active) continue;
#pragma unroll
      for (int gi = 0; gi < PF_KC / 64; ++gi) {
        const int G = kc / 64 + gi;
        uint4 a0, a1, b0, b1;
        F::convert(rawA[gi], a0, a1);
        if (MODE == 0) F::convert(rawB[gi], b0, b1);
        // scales of the 4 output rows this lane holds in D: r0 + 4 g + i
        float2 sA[4], sB[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sA[i] = F::scale(ws, (size_t)(r0 + 4 * g + i), G, K);
          if (MODE == 0) sB[i] = F::scale(ws, (size_t)(N / 2 + r0 + 4 * g + i), G, K);
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          if (t >= ntiles) break;
          const int xrow = t * 16 + c16;
          const uint4 x0 = xs[xrow * (PF_KC / 8) + gi * 8 + 2 * g];
          const uint4 x1 = xs[xrow * (PF_KC / 8) + gi * 8 + 2 * g + 1];
          const f32x4 z = {0.f, 0.f, 0.f, 0.f};
          if (F::scale_group == 64 || F::scale_group == 128) {
            accA[t] = mfma(a1, x1, mfma(a0, x0, z));
            if (MODE == 0) accB[t] = mfma(b1, x1, mfma(b0, x0, z));
            const float X_g = F::has_min ? xsum[xrow * (PF_KC / 64) + gi] : 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              if (F::has_min) {
                totA[t][i] += sA[i].x * accA[t][i] + (sA[i].y - 128.f * sA[i].x) * X_g;
                if (MODE == 0) totB[t][i] += sB[i].x * accB[t][i] + (sB[i].y - 128.f * sB[i].x) * X_g;
              } else {
                totA[t][i] += sA[i].x * accA[t][i];
                if (MODE == 0) totB[t][i] += sB[i].x * accB[t][i];
              }
            }
          } else {  // one scale per row: accumulate raw sums, scale at the end
            totA[t] = mfma(a1, x1, mfma(a0, x0, totA[t]));
            if (MODE == 0) totB[t] = mfma(b1, x1, mfma(b0, x0, totB[t]));
          }
        }
      }
    }
    if (!active) continue;
    float rsA[4] = {1.f, 1.f, 1.f, 1.f}, rsB[4] = {1.f, 1.f, 1.f, 1.f};
    if (F::scale_group == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        rsA[i] = F::scale(ws, (size_t)(r0 + 4 * g + i), 0, K).x;
        if (MODE == 0) rsB[i] = F::scale(ws, (size_t)(N / 2 + r0 + 4 * g + i), 0, K).x;
      }
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if (t >= ntiles) break;
      const int tok = p0 + t * 16 + c16;
      if (tok >= cnt) continue;
      if (MODE == 0) {
        uint16_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float gv = totA[t][i] * rsA[i], uv = totB[t][i] * rsB[i];
          o[i] = to_bf16(silu(gv) * uv);
        }
        uint16_t* act = reinterpret_cast<uint16_t*>(out) + (off + tok) * (size_t)(N / 2) + r0 + 4 * g;
        *reinterpret_cast<uint2*>(act) = make_uint2(o[0] | ((uint32_t)o[1] << 16), o[2] | ((uint32_t)o[3] << 16));
      } else {
        float* y = reinterpret_cast<float*>(out) + (off + tok) * (size_t)N + r0 + 4 * g;
        *reinterpret_cast<float4*>(y) =
            make_float4(totA[t][0] * rsA[0], totA[t][1] * rsA[1], totA[t][2] * rsA[2], totA[t][3] * rsA[3]);
      }
    }
  }
}

// grid x: experts (grouped) or 64-token passes (fixed_rows >= 0); grid y: 16-row tiles / PF_WPB
template <class F>
void launch_grouped(const uint8_t* wq, const void* ws, const uint16_t* X, const int* offsets, const int* counts,
                    void* out, int E, int N, int K, int mode, size_t eq, size_t es, int sb, int fixed_rows,
                    hipStream_t st) {
  const int rows_out = mode == 0 ? N / 2 : N;
  const int gx = fixed_rows >= 0 ? (fixed_rows + PF_TOK - 1) / PF_TOK : E;
  const dim3 grid(gx, (rows_out / 16 + PF_WPB - 1) / PF_WPB);
  if (mode == 0)
    hipLaunchKernelGGL((k_grouped<F, 0>), grid, dim3(PF_WPB * 64), 0, st, wq, ws, X, offsets, counts, out, N, K, eq, es,
                       sb, fixed_rows);
  else
    hipLaunchKernelGGL((k_grouped<F, 1>), grid, dim3(PF_WPB * 64), 0, st, wq, ws, X, offsets, counts, out, N, K, eq, es,
                       sb, fixed_rows);
}

// gate_up then down for all experts of a grouped batch
template <class F>
int moe_prefill(const uint8_t* gu_q, const void* gu_s, const uint8_t* d_q, const void* d_s, const uint16_t* xp,
                const int* offsets, const int* counts, uint16_t* act, float* y, int E, int H, int I, size_t gu_q_b,
                size_t gu_s_e, size_t d_q_b, size_t d_s_e, int sb, hipStream_t st) {
  if (H != 2048 || I != 512 || E < 1 || E > PF_MAXE) return -1;
  launch_grouped<F>(gu_q, gu_s, xp, offsets, counts, act, E, 2 * I, H, 0, gu_q_b, gu_s_e, sb, -1, st);
  launch_grouped<F>(d_q, d_s, act, offsets, counts, y, E, H, I, 1, d_q_b, d_s_e, sb, -1, st);
  return 0;
}

// Shared expert over all rows: act = bf16(silu(SG hn) * (SU hn)), out = SD act (fp32).
template <class SH>
int shared_prefill(const int8_t* sgu_q, const uint16_t* sgu_s, const int8_t* sd_q, const uint16_t* sd_s, const uint16_t* hn,
                   int rows, uint16_t* act, float* out, int H, int I, hipStream_t st) {
  if (H % PF_KC != 0 || I % PF_KC != 0 || I % 16 != 0 || rows < 0) return -1;
  if (rows == 0) return 0;
  launch_grouped<FmtQ8<SH>>((const uint8_t*)sgu_q, sgu_s, hn, nullptr, nullptr, act, 1, 2 * I, H, 0, 0, 0, 2, rows, st);
  launch_grouped<FmtQ8<SH>>((const uint8_t*)sd_q, sd_s, act, nullptr, nullptr, out, 1, H, I, 1, 0, 0, 2, rows, st);
  return 0;
}

}  // namespace

API int dr_moe_prefill(const uint8_t* gu_q, const uint16_t* gu_sm, const uint8_t* d_q, const uint16_t* d_sm,
                       const uint16_t* xp, const int* offsets, const int* counts, uint16_t* act, float* y, int E, int H,
                       int I, hipStream_t st) {
  return moe_prefill<FmtQ4<ScaleF16>>(gu_q, gu_sm, d_q, d_sm, xp, offsets, counts, act, y, E, H, I,
                                      (size_t)2 * I * (H / 2), (size_t)2 * I * (H / 64) * 2, (size_t)H * (I / 2),
                                      (size_t)H * (I / 64) * 2, 2, st);
}

API int dr_moe_prefill_bf16s(const uint8_t* gu_q, const uint16_t* gu_sm, const uint8_t* d_q, const uint16_t* d_sm,
                             const uint16_t* xp, const int* offsets, const int* counts, uint16_t* act, float* y, int E,
                             int H, int I, hipStream_t st) {
  return moe_prefill<FmtQ4<ScaleBF16>>(gu_q, gu_sm, d_q, d_sm, xp, offsets, counts, act, y, E, H, I,
                                       (size_t)2 * I * (H / 2), (size_t)2 * I * (H / 64) * 2, (size_t)H * (I / 2),
                                       (size_t)H * (I / 64) * 2, 2, st);
}

API int dr_moe_prefill_fp8(const uint8_t* gu_w, const float* gu_s, const uint8_t* d_w, const float* d_s,
                           const uint16_t* xp, const int* offsets, const int* counts, uint16_t* act, float* y, int E,
                           int H, int I, hipStream_t st) {
  return moe_prefill<FmtFP8<0>>(gu_w, gu_s, d_w, d_s, xp, offsets, counts, act, y, E, H, I, (size_t)2 * I * H,
                                (size_t)(2 * I / 128) * (H / 128), (size_t)H * I, (size_t)(H / 128) * (I / 128), 4, st);
}

API int dr_moe_prefill_fp8_bf16s(const uint8_t* gu_w, const uint16_t* gu_s, const uint8_t* d_w, const uint16_t* d_s,
                                 const uint16_t* xp, const int* offsets, const int* counts, uint16_t* act, float* y,
                                 int E, int H, int I, hipStream_t st) {
  return moe_prefill<FmtFP8<1>>(gu_w, gu_s, d_w, d_s, xp, offsets, counts, act, y, E, H, I, (size_t)2 * I * H,
                                (size_t)(2 * I / 128) * (H / 128), (size_t)H * I, (size_t)(H / 128) * (I / 128), 2, st);
}

API int dr_moe_shared_prefill(const int8_t* sgu_q, const uint16_t* sgu_s, const int8_t* sd_q, const uint16_t* sd_s,
                              const uint16_t* hn, int rows, uint16_t* act, float* out, int H, int I, hipStream_t st) {
  return shared_prefill<Q8G128F16>(sgu_q, sgu_s, sd_q, sd_s, hn, rows, act, out, H, I, st);
}

API int dr_moe_shared_prefill_bf16s(const int8_t* sgu_q, const uint16_t* sgu_s, const int8_t* sd_q, const uint16_t* sd_s,
                                    const uint16_t* hn, int rows, uint16_t* act, float* out, int H, int I,
                                    hipStream_t st) {
  return shared_prefill<Q8RowBF16>(sgu_q, sgu_s, sd_q, sd_s, hn, rows, act, out, H, I, st);
}

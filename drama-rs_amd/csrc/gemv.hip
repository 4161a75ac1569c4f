// Dense decode GEMVs around the MoE (reference: kernels/drama.cu:216-315, src/ffi.rs:33-40):
// int8 with f16 scales per 128 inputs, the int8 SwiGLU pair form, bf16, and int8 with one bf16
// scale per row (the lm_head / projection layout of benchmark configuration 5).
//
// Lane l owns 16-byte chunks c = l + 64 j of a row (16 int8 or 8 bf16 inputs each), so its
// slice of the normalised input is fixed for every row of the wave and lives in registers,
// staged once per block through LDS with a lane-major swizzle.  int8 values enter the fp32 FMA
// as (byte ^ 0x80) via v_cvt_f32_ubyte, with 128 * sum(x) subtracted once per chunk.
// K = 512 rows are 8 bytes per lane.
#include <algorithm>
#include <atomic>

#include "common.hpp"

using namespace drm;

namespace {

constexpr int GV8_WPB = 8, GV8_RPW = 4;

// xn (RMSNorm(x; nw) or x) of K floats into LDS, float4 f of part p = f / (4 * 64 * CPL)...
// layout: element slice of lane l for chunk j: float4 index F = (B/4)(l + 64 j) + i, i < B/4,
// where B = inputs per chunk (16 for int8, 8 for bf16); stored at slot j * (B/4) * 64 + i * 64 + l.
template <int B>
DEV void stage_x_lanes(const float* __restrict__ x, const float* __restrict__ nw, float eps, int K, float4* xs) {
  __shared__ float red[GV8_WPB];
  const float4* x4 = reinterpret_cast<const float4*>(x);
  constexpr int Q = B / 4;  // float4 per chunk
  float inv = 1.f;
  if (nw) {
    float ss = 0.f;
    for (int f = threadIdx.x; f < K / 4; f += blockDim.x) {
      const float4 v = x4[f];
      ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    ss = wave_sum(ss);
    if (lane_id() == 0) red[wave_id()] = ss;
    __syncthreads();
    float t = 0.f;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) t += red[w];
    inv = rsqrtf(t / (float)K + eps);
  }
  const float4* n4 = reinterpret_cast<const float4*>(nw);
  for (int f = threadIdx.x; f < K / 4; f += blockDim.x) {
    float4 v = x4[f];
    if (nw) {
      const float4 w = n4[f];
      v = make_float4(v.x * inv * w.x, v.y * inv * w.y, v.z * inv * w.z, v.w * inv * w.w);
    }
    const int c = f / Q, i = f % Q, l = c & 63, j = c >> 6;
    xs[j * Q * 64 + i * 64 + l] = v;
  }
  __syncthreads();
}

// int8 row dot over CPL 16-byte chunks per lane (K = 1024 CPL), from the lane's loaded chunks
// w (load_q8); S: scale functor
template <int CPL>
DEV void load_q8(const int8_t* __restrict__ row, uint4 (&w)[CPL]) {
  const int lane = lane_id();
#pragma unroll
  for (int j = 0; j < CPL; ++j) w[j] = ld16(row + (size_t)(lane + 64 * j) * 16);
}
template <int CPL, class SCL>
DEV float row_dot_q8(const uint4 (&w)[CPL], const float (*xv)[16], const float* xsum, SCL scl) {
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    float d = dot4_u8b(w[j].x, xv[j], 0.f);
    d = dot4_u8b(w[j].y, xv[j] + 4, d);
    d = dot4_u8b(w[j].z, xv[j] + 8, d);
    d = dot4_u8b(w[j].w, xv[j] + 12, d);
    acc += scl(j) * (d - 128.f * xsum[j]);
  }
  return acc;
}

// MODE 0: y = W xn (+ res);  MODE 1: swiglu pair rows;  SK 0: f16 per 128 (reference), 1: bf16 per row
template <int CPL, int MODE, int SK, bool PRE_OK>
__global__ void __launch_bounds__(GV8_WPB * 64)
    k_gemv_q8(const int8_t* __restrict__ W, const uint16_t* __restrict__ S, const float* __restrict__ x, const float* res,
              float* y, int N, const float* __restrict__ nw, float eps, const char* pf, size_t pf_bytes) {
  constexpr int K = 1024 * CPL;
  constexpr int NR = MODE == 1 ? 2 : 1;  // rows per output: the gate and up rows of a pair
  __shared__ float4 xs[K / 4];
  const int lane = lane_id(), wave = wave_id();
  const int row0 = (blockIdx.x * GV8_WPB + wave) * GV8_RPW;
  // PRE_OK (small N, where a block's latency is not hidden by other blocks): every weight load
  // of the wave first, so they stream while x is staged (up to 4 chunks per row and lane);
  // otherwise each row loads before its dot and more blocks fit on a CU
  constexpr bool PRE = PRE_OK && CPL * NR <= 4;
  uint4 w[GV8_RPW][NR][CPL];
  auto load_row = [&](int r) {
    const int n = row0 + r < N ? row0 + r : N - 1;
#pragma unroll
    for (int h = 0; h < NR; ++h) load_q8<CPL>(W + (size_t)(n + h * N) * K, w[r][h]);
  };
  if constexpr (PRE) {
#pragma unroll
    for (int r = 0; r < GV8_RPW; ++r) load_row(r);
  }
  stage_x_lanes<16>(x, nw, eps, K, xs);
  float xv[CPL][16], xsum[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    xsum[j] = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 v = xs[j * 256 + i * 64 + lane];
      xv[j][4 * i] = v.x, xv[j][4 * i + 1] = v.y, xv[j][4 * i + 2] = v.z, xv[j][4 * i + 3] = v.w;
      xsum[j] += (v.x + v.y) + (v.z + v.w);
    }
  }
#pragma unroll
  for (int r = 0; r < GV8_RPW; ++r) {
    const int n = row0 + r;
    if (n >= N) break;
    if constexpr (!PRE) load_row(r);
    auto scl_of = [&](size_t row) {
      return [=](int j) {
        if (SK == 1) return bf16f(S[row]);
        return f16f(S[row * (K / 128) + (size_t)((lane + 64 * j) * 16) / 128]);
      };
    };
    if (MODE == 0) {
      float d = wave_sum(row_dot_q8<CPL>(w[r][0], xv, xsum, scl_of((size_t)n)));
      if (lane == 0) y[n] = d + (res ? res[n] : 0.f);
    } else {
      const float g = wave_sum(row_dot_q8<CPL>(w[r][0], xv, xsum, scl_of((size_t)n)));
      const float u = wave_sum(row_dot_q8<CPL>(w[r][NR - 1], xv, xsum, scl_of((size_t)(N + n))));
      if (lane == 0) y[n] = silu(g) * u;
    }
  }
  warm_range(pf, pf_bytes);
}

// Large-N form of MODE 0 (the lm_head): a grid of GV8_PB blocks per CU stages x once and each
// wave walks tiles of GV8_RPW rows spaced by the grid, the next tile's loads issued before the
// current tile's dots (two tiles of weight chunks in registers).  Same arithmetic per row as
// k_gemv_q8.
constexpr int GV8_PB = 4;  // measured: 2 -> 51.0 us, 3 -> 55, 4 -> 50.5 (lm_head 151936 x 2048)
template <int CPL, int SK>
__global__ void __launch_bounds__(GV8_WPB * 64)
    k_gemv_q8_walk(const int8_t* __restrict__ W, const uint16_t* __restrict__ S, const float* __restrict__ x,
                   const float* res, float* y, int N, const float* __restrict__ nw, float eps, const char* pf,
                   size_t pf_bytes) {
  constexpr int K = 1024 * CPL;
  __shared__ float4 xs[K / 4];
  const int lane = lane_id(), wave = wave_id();
  // tiles of GV8_RPW rows, wave after wave, spaced by the grid (waves running side by side
  // read neighbouring rows: measured faster than a contiguous share per wave)
  const int step = gridDim.x * GV8_WPB * GV8_RPW, end = N;
  int base = (blockIdx.x * GV8_WPB + wave) * GV8_RPW;
  uint4 w[2][GV8_RPW][CPL];
  auto load_tile = [&](int b, uint4 (&tl)[GV8_RPW][CPL]) {
#pragma unroll
    for (int r = 0; r < GV8_RPW; ++r) {
      const int n = b + r < end ? b + r : end - 1;
      load_q8<CPL>(W + (size_t)n * K, tl[r]);
    }
  };
  if (base < end) load_tile(base, w[0]);
  stage_x_lanes<16>(x, nw, eps, K, xs);
  float xv[CPL][16], xsum[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    xsum[j] = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 v = xs[j * 256 + i * 64 + lane];
      xv[j][4 * i] = v.x, xv[j][4 * i + 1] = v.y, xv[j][4 * i + 2] = v.z, xv[j][4 * i + 3] = v.w;
      xsum[j] += (v.x + v.y) + (v.z + v.w);
    }
  }
  auto dots = [&](int b, const uint4 (&tl)[GV8_RPW][CPL]) {
#pragma unroll
    for (int r = 0; r < GV8_RPW; ++r) {
      const int n = b + r;
      if (n >= end) break;
      const float d = wave_sum(row_dot_q8<CPL>(tl[r], xv, xsum, [&](int j) {
        if (SK == 1) return bf16f(S[n]);
        return f16f(S[(size_t)n * (K / 128) + (size_t)((lane + 64 * j) * 16) / 128]);
      }));
      if (lane == 0) y[n] = d + (res ? res[n] : 0.f);
    }
  };
  for (; base < end; base += step) {
    // two register tiles alternate; the loop is unrolled by hand so both stay in registers
    if (base + step < end) load_tile(base + step, w[1]);
    dots(base, w[0]);
    base += step;
    if (base >= end) break;
    if (base + step < end) load_tile(base + step, w[0]);
    dots(base, w[1]);
  }
  warm_range(pf, pf_bytes);
}

// K = 512 int8 rows: 8 bytes per lane (one f16 scale group of 128 covers lanes 16 g .. 16 g + 15)
template <int MODE, int SK>
__global__ void __launch_bounds__(GV8_WPB * 64)
    k_gemv_q8_k512(const int8_t* __restrict__ W, const uint16_t* __restrict__ S, const float* __restrict__ x,
                   const float* res, float* y, int N, const float* __restrict__ nw, float eps, const char* pf,
                   size_t pf_bytes) {
  constexpr int K = 512;
  __shared__ float4 xs[K / 4];
  const int lane = lane_id(), wave = wave_id();
  stage_x_lanes<8>(x, nw, eps, K, xs);
  float xv[8];
  const float4 a = xs[lane], b = xs[64 + lane];
  xv[0] = a.x, xv[1] = a.y, xv[2] = a.z, xv[3] = a.w, xv[4] = b.x, xv[5] = b.y, xv[6] = b.z, xv[7] = b.w;
  const float xsum = (a.x + a.y) + (a.z + a.w) + (b.x + b.y) + (b.z + b.w);
  const int row0 = (blockIdx.x * GV8_WPB + wave) * GV8_RPW;
  auto dot = [&](size_t row) {
    const uint2 w = ld8(W + row * K + lane * 8);
    float d = dot4_u8b(w.x, xv, 0.f);
    d = dot4_u8b(w.y, xv + 4, d);
    const float s = SK == 1 ? bf16f(S[row]) : f16f(S[row * (K / 128) + lane / 16]);
    return s * (d - 128.f * xsum);
  };
#pragma unroll
  for (int r = 0; r < GV8_RPW; ++r) {
    const int n = row0 + r;
    if (n >= N) break;
    if (MODE == 0) {
      const float d = wave_sum(dot((size_t)n));
      if (lane == 0) y[n] = d + (res ? res[n] : 0.f);
    } else {
      const float g = wave_sum(dot((size_t)n)), u = wave_sum(dot((size_t)(N + n)));
      if (lane == 0) y[n] = silu(g) * u;
    }
  }
  warm_range(pf, pf_bytes);
}

template <int CPL>
__global__ void __launch_bounds__(GV8_WPB * 64)
    k_gemv_bf16(const uint16_t* __restrict__ W, const float* __restrict__ x, float* __restrict__ y, int N,
                const float* __restrict__ nw, float eps, const char* pf, size_t pf_bytes) {
  constexpr int K = 512 * CPL;  // 8 bf16 per 16-byte chunk
  __shared__ float4 xs[K / 4];
  const int lane = lane_id(), wave = wave_id();
  stage_x_lanes<8>(x, nw, eps, K, xs);
  float xv[CPL][8];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const float4 a = xs[j * 128 + lane], b = xs[j * 128 + 64 + lane];
    xv[j][0] = a.x, xv[j][1] = a.y, xv[j][2] = a.z, xv[j][3] = a.w;
    xv[j][4] = b.x, xv[j][5] = b.y, xv[j][6] = b.z, xv[j][7] = b.w;
  }
  const int row0 = (blockIdx.x * GV8_WPB + wave) * GV8_RPW;
#pragma unroll
  for (int r = 0; r < GV8_RPW; ++r) {
    const int n = row0 + r;
    if (n >= N) break;
    uint4 w[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) w[j] = ld16(W + (size_t)n * K + (size_t)(lane + 64 * j) * 8);
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      acc = __builtin_fmaf(bf16_lo(w[j].x), xv[j][0], acc);
      acc = __builtin_fmaf(bf16_hi(w[j].x), xv[j][1], acc);
      acc = __builtin_fmaf(bf16_lo(w[j].y), xv[j][2], acc);
      acc = __builtin_fmaf(bf16_hi(w[j].y), xv[j][3], acc);
      acc = __builtin_fmaf(bf16_lo(w[j].z), xv[j][4], acc);
      acc = __builtin_fmaf(bf16_hi(w[j].z), xv[j][5], acc);
      acc = __builtin_fmaf(bf16_lo(w[j].w), xv[j][6], acc);
      acc = __builtin_fmaf(bf16_hi(w[j].w), xv[j][7], acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) y[n] = acc;
  }
  warm_range(pf, pf_bytes);
}

int blocks_for(int rows) { return (rows + GV8_WPB * GV8_RPW - 1) / (GV8_WPB * GV8_RPW); }

template <int MODE, int SK>
int launch_q8(const int8_t* W, const uint16_t* S, const float* x, const float* res, float* y, int N, int K,
              const float* nw, float eps, const char* pf, size_t pf_bytes, hipStream_t st) {
  if (N <= 0) return N == 0 ? 0 : -1;
  const dim3 g(blocks_for(N)), b(GV8_WPB * 64);
  const bool small = N <= 16384;  // at most ~2 blocks per CU
  if (MODE == 0 && !small && (K == 1024 || K == 2048)) {
    static std::atomic<int> cus{0};
    if (cus.load(std::memory_order_relaxed) == 0) {
      int dev = 0, c = 0;
      (void)hipGetDevice(&dev);
      (void)hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev);
      cus.store(c > 0 ? c : 256, std::memory_order_relaxed);
    }
    const dim3 gw(std::min<int>(blocks_for(N), GV8_PB * cus.load(std::memory_order_relaxed)));
    if (K == 1024) hipLaunchKernelGGL((k_gemv_q8_walk<1, SK>), gw, b, 0, st, W, S, x, res, y, N, nw, eps, pf, pf_bytes);
    else hipLaunchKernelGGL((k_gemv_q8_walk<2, SK>), gw, b, 0, st, W, S, x, res, y, N, nw, eps, pf, pf_bytes);
    return 0;
  }
  switch (K) {
    case 512: hipLaunchKernelGGL((k_gemv_q8_k512<MODE, SK>), g, b, 0, st, W, S, x, res, y, N, nw, eps, pf, pf_bytes); break;
    case 1024: if (small) hipLaunchKernelGGL((k_gemv_q8<1, MODE, SK, true>), g, b, 0, st, W, S, x, res, y, N, nw, eps, pf, pf_bytes);
      else hipLaunchKernelGGL((k_gemv_q8<1, MODE, SK, false>), g, b, 0, st, W, S, x, res, y, N, nw, eps, pf, pf_bytes);
      break;
    case 2048: if (small) hipLaunchKernelGGL((k_gemv_q8<2, MODE, SK, true>), g, b, 0, st, W, S, x, res, y, N, nw, eps, pf, pf_bytes);
      else hipLaunchKernelGGL((k_gemv_q8<2, MODE, SK, false>), g, b, 0, st, W, S, x, res, y, N, nw, eps, pf, pf_bytes);
      break;
    case 4096: if (small) hipLaunchKernelGGL((k_gemv_q8<4, MODE, SK, true>), g, b, 0, st, W, S, x, res, y, N, nw, eps, pf, pf_bytes);
      else hipLaunchKernelGGL((k_gemv_q8<4, MODE, SK, false>), g, b, 0, st, W, S, x, res, y, N, nw, eps, pf, pf_bytes);
      break;
    case 6144: hipLaunchKernelGGL((k_gemv_q8<6, MODE, SK, false>), g, b, 0, st, W, S, x, res, y, N, nw, eps, pf, pf_bytes); break;
    default: return -1;
  }
  return 0;
}

}  // namespace

API int dr_gemv_q8(const int8_t* W, const uint16_t* S, const float* x, const float* res, float* y, int N, int K,
                   const float* nw, float eps, const char* pf, size_t pf_bytes, hipStream_t st) {
  return launch_q8<0, 0>(W, S, x, res, y, N, K, nw, eps, pf, pf_bytes, st);
}

API int dr_gemv_q8_swiglu(const int8_t* W, const uint16_t* S, const float* x, float* y, int I, int K, const float* nw,
                          float eps, const char* pf, size_t pf_bytes, hipStream_t st) {
  return launch_q8<1, 0>(W, S, x, nullptr, y, I, K, nw, eps, pf, pf_bytes, st);
}

API int dr_gemv_q8_bf16s(const int8_t* W, const uint16_t* S, const float* x, const float* res, float* y, int N, int K,
                         const float* nw, float eps, hipStream_t st) {
  return launch_q8<0, 1>(W, S, x, res, y, N, K, nw, eps, nullptr, 0, st);
}

API int dr_gemv_bf16(const uint16_t* W, const float* x, float* y, int N, int K, const float* nw, float eps,
                     const char* pf, size_t pf_bytes, hipStream_t st) {
  if (N <= 0) return N == 0 ? 0 : -1;
  const dim3 g(blocks_for(N)), b(GV8_WPB * 64);
  switch (K) {
    case 2048: hipLaunchKernelGGL(k_gemv_bf16<4>, g, b, 0, st, W, x, y, N, nw, eps, pf, pf_bytes); break;
    case 4096: hipLaunchKernelGGL(k_gemv_bf16<8>, g, b, 0, st, W, x, y, N, nw, eps, pf, pf_bytes); break;
    default: return -1;
  }
  return 0;
}

// Router: logits, softmax and top-k (reference: kernels/drama.cu:317-468, src/ffi.rs:41,55-59)
// plus the bf16 GEMM dr_gemm that the prefill router uses (src/engine.rs:554).
//
// These kernels follow the canonical fp32 operation order of canon.hpp (RMSNorm, row dot,
// softmax, top-k), so the CPU oracle reproduces the logits, the softmax probabilities and
// hence the selected experts bit for bit.
#include "router_rows.hpp"

#pragma clang fp contract(off)

using namespace drm;

namespace {

// Decode router for B rows (B <= 8) in one launch of router blocks (router_rows.hpp).
template <int B>
__global__ void __launch_bounds__(RT_WPB * 64)
    k_router_topk_rows(const uint16_t* __restrict__ W, const float* __restrict__ x, const float* __restrict__ nw,
                       float eps, float* __restrict__ logits, int E, int topk, int* __restrict__ idx,
                       float* __restrict__ wts, float* __restrict__ sgate, uint32_t* __restrict__ counter) {
  __shared__ float4 xs[B][2048 / 4];
  router_rows_block<B>(blockIdx.x, gridDim.x, W, x, nw, eps, logits, E, topk, idx, wts, sgate, counter, nullptr, 0u,
                       xs);
}

// One row per block.  topk <= 8: waves 0..3 each pick the top 8 of 64 experts and wave 4
// computes the softmax denominator, then wave 0 ranks the 32 candidates (the same selection
// and weights as canon_softmax_topk, in less than half the time); topk > 8: wave 0 alone.
__global__ void __launch_bounds__(320)
    k_moe_topk(const float* __restrict__ logits, int E, int topk, int stride, int* __restrict__ idx,
               float* __restrict__ wts, float* __restrict__ sgate) {
  const int r = blockIdx.x, lane = lane_id(), wave = wave_id();
  const float* l = logits + (size_t)r * stride;
  __shared__ float lg[257];
  __shared__ uint64_t s_cand[32];
  __shared__ int s_sel[8];
  __shared__ float s_mz[2];
  if ((int)threadIdx.x <= E) lg[threadIdx.x] = l[threadIdx.x];
  __syncthreads();
  if (wave == 0 && lane == 0) sgate[r] = lg[E];
  if (topk <= 8) {
    if (wave < 4) {
      int ck, ce;
      canon_select_group8(lg, E, wave, &ck, &ce);
      if (lane < 8) s_cand[wave * 8 + lane] = canon_cand64(ck, ce);
    } else {
      float m;
      const float z = canon_softmax_z(lg, E, &m);
      if (lane == 0) s_mz[0] = m, s_mz[1] = z;
    }
    __syncthreads();
    if (wave != 0) return;
    const int id = merge_picks(s_cand, s_sel, topk);
    const float w = canon_topk_weight(lg[lane < topk ? id : 0], s_mz[0], s_mz[1], topk);
    if (lane < topk) idx[(size_t)r * topk + lane] = id, wts[(size_t)r * topk + lane] = w;
  } else {
    if (wave != 0) return;
    int my_idx;
    float my_w;
    canon_softmax_topk(lg, E, topk, &my_idx, &my_w);
    if (lane < topk) idx[(size_t)r * topk + lane] = my_idx, wts[(size_t)r * topk + lane] = my_w;
  }
}

// The same canonical GEMM for few rows of A (M <= GR_MAXM, decode batches): one wave per W
// row, which it loads once and dots with every A row (4 at a time, all loads issued first);
// 8 waves per block.  Every dot has the canonical order, so C equals k_gemm_tile's bits.
constexpr int GR_MAXM = 16;
template <int NCH>
__global__ void __launch_bounds__(512)
    k_gemm_rows(const uint16_t* __restrict__ A, const uint16_t* __restrict__ W, float* __restrict__ C, int M,
                int N, int K, float beta) {
  const int lane = lane_id();
  const int n = blockIdx.x * 8 + wave_id();
  if (n >= N) return;
  const int KC = K / 8;
  uint4 w[NCH];
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int c = lane + WAVE * j;
    w[j] = c < KC ? ld16(W + (size_t)n * K + (size_t)c * 8) : make_uint4(0, 0, 0, 0);
  }
  for (int m0 = 0; m0 < M; m0 += 4) {
    uint4 av[4][NCH];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = m0 + r < M ? m0 + r : M - 1;
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        const int c = lane + WAVE * j;
        av[r][j] = c < KC ? ld16(A + (size_t)m * K + (size_t)c * 8) : make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        if (lane + WAVE * j < KC) {
          const uint4 a = av[r][j], b = w[j];
          acc = __builtin_fmaf(bf16_lo(b.x), bf16_lo(a.x), acc);
          acc = __builtin_fmaf(bf16_hi(b.x), bf16_hi(a.x), acc);
          acc = __builtin_fmaf(bf16_lo(b.y), bf16_lo(a.y), acc);
          acc = __builtin_fmaf(bf16_hi(b.y), bf16_hi(a.y), acc);
          acc = __builtin_fmaf(bf16_lo(b.z), bf16_lo(a.z), acc);
          acc = __builtin_fmaf(bf16_hi(b.z), bf16_hi(a.z), acc);
          acc = __builtin_fmaf(bf16_lo(b.w), bf16_lo(a.w), acc);
          acc = __builtin_fmaf(bf16_hi(b.w), bf16_hi(a.w), acc);
        }
      }
      acc = wave_sum(acc);
      const int m = m0 + r;
      if (lane == 0 && m < M) {
        float* c = C + (size_t)m * N + n;
        *c = beta == 0.f ? acc : acc + beta * *c;
      }
    }
  }
}

// The same canonical GEMM, one wave per 8 x 8 tile of C (4 tiles per block, no LDS): lane l
// accumulates all 64 dots over its chunks l + 64 j in element order (the canonical lane sums),
// then one reduce-scatter over the ascending xor tree finishes them together.  Step o pairs
// lane l with l ^ o exactly as the canonical butterfly does, and each pair of lanes splits its
// list of partial sums: the lane with bit o clear keeps the first half (adding its partner's
// copy of it), the other the second half, so after the six steps lane l holds output
// bitrev6(l) with the canonical tree's bits (a + b = b + a).  Exchanges: DPP quad_perm (o = 1,
// 2) and row_ror (o = 4: by 12 for the lanes whose partner is l + 4, by 4 for l - 4; o = 8: by
// 8), v_permlane16_swap / v_permlane32_swap (o = 16, 32; the swap itself hands each lane the
// half it keeps).  A and W chunks of the next j are requested before the current j's FMAs.
// Measured at 300 x 257 x 2048 with 8 x 8 tiles: 12.0 us (a 2 x 8 per-wave kernel with one butterfly
// per dot: 16.8 us); 4 x 8 tiles (twice the waves, more conversions per FMA) 13.9 us.
template <int O, int V>
DEV void rs_step(float (&v)[64]) {
  const int lane = lane_id();
#pragma unroll
  for (int k = 0; k < V / 2; ++k) {
    const float x = v[k], y = v[k + V / 2];
    if constexpr (O >= 16) {
      const auto r = O == 16 ? __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(y), false, false)
                             : __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
      v[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    } else {
      constexpr int cx = O == 1 ? 0xB1 : O == 2 ? 0x4E : O == 4 ? 0x12C : 0x128;
      constexpr int cy = O == 1 ? 0xB1 : O == 2 ? 0x4E : O == 4 ? 0x124 : 0x128;
      const float px = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), cx, 0xF, 0xF, true));
      const float py = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(y), cy, 0xF, 0xF, true));
      v[k] = (lane & O) ? y + py : x + px;
    }
  }
}

// Tiles of TM x TN outputs (at most 8 x 8: the 64 reduce-scatter slots; the unused slots stay
// zero and are never stored).  8 x 5 balances 300 x 257 best over the 1024 SIMDs: measured 9.5-9.8
// us against 10.7-11.2 for 8 x 8 (1254 tiles, a fifth of the SIMDs running two), 9.8 for 8 x 6,
// 10.1-10.3 for 8 x 7 and 12.1 for 8 x 4 (more A loads per FMA), with identical bits.
constexpr int GT_TM = 8, GT_TN = 5;
template <int NCH, int TM = GT_TM, int TN = GT_TN>
__global__ void __launch_bounds__(256)
    k_gemm_tile(const uint16_t* __restrict__ A, const uint16_t* __restrict__ W, float* __restrict__ C, int M, int N,
                int K, float beta) {
#pragma clang fp contract(off)
  static_assert(TM >= 1 && TM <= 8 && TN >= 1 && TN <= 8, "tile of at most 8 x 8 (64 reduce-scatter slots)");
  const int lane = lane_id();
  const int tn = (N + TN - 1) / TN;
  const int tile = blockIdx.x * 4 + wave_id();
  const int m0 = (tile / tn) * TM, n0 = (tile % tn) * TN;
  if (m0 >= M) return;
  const int KC = K / 8;
  const uint16_t* ap[8];
  const uint16_t* wp[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    ap[r] = A + (size_t)(m0 + r < M ? m0 + r : M - 1) * K + (size_t)lane * 8;
    wp[r] = W + (size_t)(n0 + r < N ? n0 + r : N - 1) * K + (size_t)lane * 8;
  }
  (void)ap, (void)wp;
  float acc[64];
#pragma unroll
  for (int i = 0; i < 64; ++i) acc[i] = 0.f;
  uint4 ac[2][8], wc[2][8];
  auto load = [&](int j, int b) {
    const bool in = lane + WAVE * j < KC;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      if (r < TM) ac[b][r] = in ? ld16(ap[r] + (size_t)j * WAVE * 8) : make_uint4(0, 0, 0, 0);
      if (r < TN) wc[b][r] = in ? ld16(wp[r] + (size_t)j * WAVE * 8) : make_uint4(0, 0, 0, 0);
    }
  };
  load(0, 0);
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int b = j & 1;
    if (j + 1 < NCH) load(j + 1, b ^ 1);
    if (lane + WAVE * j < KC) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float a[8], w[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          if (r < TM) {
            const uint32_t aw = e < 2 ? ac[b][r].x : e < 4 ? ac[b][r].y : e < 6 ? ac[b][r].z : ac[b][r].w;
            a[r] = (e & 1) ? bf16_hi(aw) : bf16_lo(aw);
          }
          if (r < TN) {
            const uint32_t ww = e < 2 ? wc[b][r].x : e < 4 ? wc[b][r].y : e < 6 ? wc[b][r].z : wc[b][r].w;
            w[r] = (e & 1) ? bf16_hi(ww) : bf16_lo(ww);
          }
        }
#pragma unroll
        for (int m = 0; m < TM; ++m)
#pragma unroll
          for (int n = 0; n < TN; ++n) acc[8 * m + n] = __builtin_fmaf(w[n], a[m], acc[8 * m + n]);
      }
    }
  }
  rs_step<1, 64>(acc);
  rs_step<2, 32>(acc);
  rs_step<4, 16>(acc);
  rs_step<8, 8>(acc);
  rs_step<16, 4>(acc);
  rs_step<32, 2>(acc);
  const int i = (int)(__builtin_bitreverse32((uint32_t)lane) >> 26);
  const int m = m0 + (i >> 3), n = n0 + (i & 7);
  if ((i >> 3) < TM && (i & 7) < TN && m < M && n < N) {
    float* c = C + (size_t)m * N + n;
    *c = beta == 0.f ? acc[0] : acc[0] + beta * *c;
  }
}

template <int NCH>
void launch_gemm(const uint16_t* A, const uint16_t* W, float* C, int M, int N, int K, float beta, hipStream_t st) {
  if (M <= GR_MAXM) {
    hipLaunchKernelGGL(k_gemm_rows<NCH>, dim3((N + 7) / 8), dim3(512), 0, st, A, W, C, M, N, K, beta);
    return;
  }
  const int tiles = ((M + GT_TM - 1) / GT_TM) * ((N + GT_TN - 1) / GT_TN);
  hipLaunchKernelGGL(k_gemm_tile<NCH>, dim3((tiles + 3) / 4), dim3(256), 0, st, A, W, C, M, N, K, beta);
}

}  // namespace

hipStream_t gemm_handle_stream(void* h);

API int dr_router_topk(const uint16_t* W, const float* x, const float* nw, float eps, float* logits, int E, int topk,
                       int K, int* idx, float* wts, float* sgate, uint32_t* counter, const char*, const char*,
                       const char*, const char*, size_t, size_t, size_t, size_t, hipStream_t st) {
  if (K != 2048 || E > 256 || E < 1 || topk > 32 || topk < 1 || topk > E) return -1;
  // the one-row case of the small-batch router (its one-wave top-k measured 0.3 us shorter per
  // call than four group selections and a rank merge, with the same picks)
  hipLaunchKernelGGL(k_router_topk_rows<1>, dim3((E + RT_WPB) / RT_WPB), dim3(RT_WPB * 64), 0, st, W, x, nw, eps, logits,
                     E, topk, idx, wts, sgate, counter);
  return 0;
}

API int dr_router_topk_rows(const uint16_t* W, const float* x, const float* nw, float eps, float* logits, int E,
                            int topk, int K, int rows, int* idx, float* wts, float* sgate, uint32_t* counter,
                            hipStream_t st) {
  if (K != 2048 || E > 256 || E < 1 || topk > 32 || topk < 1 || topk > E || rows < 1 || rows > 8) return -1;
  const dim3 g((E + RT_WPB) / RT_WPB), b(RT_WPB * 64);
  switch (rows) {
#define RT_ROWS(n) \
  case n: hipLaunchKernelGGL(k_router_topk_rows<n>, g, b, 0, st, W, x, nw, eps, logits, E, topk, idx, wts, sgate, counter); break;
    RT_ROWS(1) RT_ROWS(2) RT_ROWS(3) RT_ROWS(4) RT_ROWS(5) RT_ROWS(6) RT_ROWS(7) RT_ROWS(8)
#undef RT_ROWS
  }
  return 0;
}

API int dr_moe_topk(const float* logits, int rows, int E, int topk, int stride, int* idx, float* wts, float* sgate,
                    hipStream_t st) {
  if (E > 256 || E < 1 || topk > 32 || topk < 1 || topk > E || stride < E + 1) return -1;
  if (rows <= 0) return 0;
  hipLaunchKernelGGL(k_moe_topk, dim3(rows), dim3(320), 0, st, logits, E, topk, stride, idx, wts, sgate);
  return 0;
}

API int dr_gemm(void* h, const uint16_t* A, const uint16_t* W, float* C, int M, int N, int K, float beta) {
  if (K % 8 != 0 || K <= 0 || M < 0 || N < 0) return -1;
  if (M == 0 || N == 0) return 0;
  hipStream_t st = gemm_handle_stream(h);
  const int kc = K / 8;
  if (kc <= 64) launch_gemm<1>(A, W, C, M, N, K, beta, st);
  else if (kc <= 128) launch_gemm<2>(A, W, C, M, N, K, beta, st);
  else if (kc <= 256) launch_gemm<4>(A, W, C, M, N, K, beta, st);
  else if (kc <= 512) launch_gemm<8>(A, W, C, M, N, K, beta, st);
  else return -1;
  return 0;
}

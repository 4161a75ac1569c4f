// Prefill grouping of (row, k) pairs by expert (reference: kernels/drama.cu:744-797,
// src/engine.rs:564-575) and the weighted combine.
//
// dr_moe_group is one workgroup of 16 waves: a stable counting sort in three phases, each wave's
// expert ids loaded once, all at the start (one memory round trip).
//   1. wave w takes chunks of 128 pairs; for each 64-pair half it finds, with 8 ballots over
//      the expert-id bits, the lanes that share its expert: the rank within the chunk is the
//      count of lower such lanes, the chunk count goes to a [chunk][expert] table in LDS;
//   2. four threads per expert scan its column over the chunks (exclusive, 16 chunks each,
//      the four in different waves so each wave reads whole table rows, then combined
//      through LDS), giving each chunk's base and the expert's total; a block scan over
//      experts gives the offsets;
//   3. slot = offsets[e] + base[chunk][e] + rank.
// The order within an expert is ascending pair index (the reference's atomics give an
// unspecified order; this is one of its possible outcomes, and the CPU oracle's).
#include "canon.hpp"

using namespace drm;

namespace {

constexpr int GR_THREADS = 1024, GR_WAVES = GR_THREADS / 64, GR_CHUNK = 128, GR_MAXN = 8192;
constexpr int GR_MAXCH = GR_MAXN / GR_CHUNK;  // 64 chunks

// mask of lanes whose 8-bit key equals this lane's
DEV uint64_t match8(uint32_t key, bool valid) {
  uint64_t m = __ballot(valid);
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    const bool bit = (key >> b) & 1u;
    const uint64_t bal = __ballot(bit && valid);
    m &= bit ? bal : ~bal;
  }
  return m;
}

// The counting sort of one workgroup of GR_THREADS threads over pairs 0..n-1 whose expert ids
// ld(i) returns.  mode 0: compute counts/offsets and slots; mode 1 (dr_moe_permute): offsets
// given, fill holds the pairs of each expert already placed by earlier segments and is advanced
// by this one.  row_of_slot (nullable): the inverse map slot -> pair i / topk.
template <class Ld>
DEV void group_block(const Ld& ld, int n, int E, int* __restrict__ counts, int* __restrict__ offsets,
                     int* __restrict__ slot_of, int mode, int* __restrict__ fill, int* __restrict__ row_of_slot,
                     int topk) {
  __shared__ uint16_t tab[GR_MAXCH][256];  // per-chunk count, then per-chunk base
  __shared__ uint8_t rank[GR_MAXN];
  __shared__ int s_off[256], s_tot[256];
  __shared__ int s_wsum[GR_WAVES];
  const int lane = lane_id(), wave = wave_id();
  const int nch = (n + GR_CHUNK - 1) / GR_CHUNK;
  // every expert id this wave handles (chunks wave + 16 cc, both halves), requested at once:
  // one memory round trip instead of one per chunk half and pass
  constexpr int NKEY = GR_MAXCH / GR_WAVES * 2;
  uint32_t keys[NKEY];
#pragma unroll
  for (int j = 0; j < NKEY; ++j) {
    const int i = (wave + GR_WAVES * (j >> 1)) * GR_CHUNK + (j & 1) * 64 + lane;
    keys[j] = i < n ? (uint32_t)ld(i) & 255u : 0u;  // ids must be < E <= 256
  }
  // every row is cleared, so the scan below reads and writes all GR_MAXCH rows without a
  // bounds test (a test per read would make each read wait for the one before it)
#pragma unroll
  for (int i = threadIdx.x; i < GR_MAXCH * 64; i += GR_THREADS) reinterpret_cast<uint64_t*>(&tab[0][0])[i] = 0;
  __syncthreads();
#pragma unroll
  for (int j = 0; j < NKEY; ++j) {
    const int c = wave + GR_WAVES * (j >> 1), h = j & 1;
    if (c < nch) {
      const int i = c * GR_CHUNK + h * 64 + lane;
      const bool valid = i < n;
      const uint32_t key = keys[j];
      const uint64_t m = match8(key, valid);
      const uint64_t lower = lane ? (~0ull >> (64 - lane)) : 0ull;
      const int r = __popcll(m & lower);
      // earlier half's count of the same key: read from the table (written below by the leader)
      __builtin_amdgcn_wave_barrier();
      const int prev = valid ? (int)tab[c][key] : 0;
      __builtin_amdgcn_wave_barrier();
      if (valid) rank[i] = (uint8_t)(prev + r);
      const bool leader = valid && r == 0;
      if (leader) tab[c][key] = (uint16_t)(prev + __popcll(m));
      __builtin_amdgcn_wave_barrier();
    }
  }
  __syncthreads();
  // phase 2: per-expert exclusive scan over chunks.  Wave w takes quarter q = w / 4 of the
  // chunks (16 q .. 16 q + 15) for the 64 experts 64 (w % 4) ..: each of its reads is one
  // contiguous table row (no bank conflicts), the quarter is skipped as a whole when it lies
  // past nch, and the four quarters of an expert are combined through s_part
  {
    static_assert(GR_THREADS == 4 * 256 && GR_MAXCH == 4 * 16, "four chunk quarters of 256 experts");
    __shared__ int s_part[4][256];
    const int e = threadIdx.x & 255, q = threadIdx.x >> 8;
    const bool any = 16 * q < nch;  // the same for the whole wave
    int v[16], loc = 0;
    if (any) {
#pragma unroll
      for (int t = 0; t < 16; ++t) v[t] = tab[16 * q + t][e];  // rows past nch hold zeros
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const int c = v[t];
        v[t] = loc;
        loc += c;
      }
    }
    s_part[q][e] = loc;
    __syncthreads();
    int base = 0, tot = 0;
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      const int p = s_part[qq][e];
      base += qq < q ? p : 0;
      tot += p;
    }
    if (any) {
#pragma unroll
      for (int t = 0; t < 16; ++t) tab[16 * q + t][e] = (uint16_t)(v[t] + base);  // rows past nch unused
    }
    if (q == 0) s_tot[e] = tot;
  }
  __syncthreads();
  int total = 0;
  if (threadIdx.x < 256) total = s_tot[threadIdx.x];
  // block-wide exclusive scan of totals over experts 0..255 (waves 0..3)
  if (threadIdx.x < 256) {
    int v = total;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int t = __shfl_up(v, o, 64);
      if (lane >= o) v += t;
    }
    if (lane == 63) s_wsum[wave] = v;
    s_off[threadIdx.x] = v - total;  // exclusive within the wave
  }
  __syncthreads();
  if (threadIdx.x < 256) {
    int base = 0;
    for (int w = 0; w < wave; ++w) base += s_wsum[w];
    const int e = threadIdx.x;
    if (mode == 0) {
      s_off[e] = s_off[e] + base;
      if (e < E) counts[e] = total, offsets[e] = s_off[e];
    } else if (total > 0) {
      // only experts that occur in this segment are touched (offsets/fill have the caller's E
      // entries); fill carries the pairs of earlier segments, so slots stay stable across them
      const int f = fill[e];
      s_off[e] = offsets[e] + f;
      fill[e] = f + total;
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < NKEY; ++j) {
    // c < GR_MAXCH and i < GR_MAXN for every j, so the LDS reads need no bounds test and all
    // of them are issued before the first store; pairs past n are not stored
    const int c = wave + GR_WAVES * (j >> 1), i = c * GR_CHUNK + (j & 1) * 64 + lane;
    const int e = (int)keys[j];
    const int slot = s_off[e] + (int)tab[c][e] + (int)rank[i];
    if (i < n) {
      slot_of[i] = slot;
      if (row_of_slot) row_of_slot[slot] = i / topk;
    }
  }
}

__global__ void __launch_bounds__(GR_THREADS)
    k_group(const int* __restrict__ idx, int n, int E, int* __restrict__ counts, int* __restrict__ offsets,
            int* __restrict__ slot_of, int mode, int* __restrict__ fill, int* __restrict__ row_of_slot, int topk) {
  group_block([&](int i) { return idx[i]; }, n, E, counts, offsets, slot_of, mode, fill, row_of_slot, topk);
}

// Prefill top-k and grouping in one launch.  Each block of 16 waves takes 3 rows (waves 5 s ..
// 5 s + 4 for row 3 b + s: four 64-expert group selections and the softmax denominator, then the
// rank merge, as k_moe_topk), publishes idx with cache-bypassing stores and counts itself in
// once they have completed; the last block runs the stable counting sort of dr_moe_group over
// all rows * topk pairs (reading idx back with cache-bypassing loads), writes counts, offsets,
// slot_of and the inverse map row_of_slot, and resets the counter.
constexpr int TG_ROWS = 3;
__global__ void __launch_bounds__(GR_THREADS)
    k_moe_topk_group(const float* __restrict__ logits, int rows, int E, int topk, int stride, int* __restrict__ idx,
                     float* __restrict__ wts, float* __restrict__ sgate, int* __restrict__ counts,
                     int* __restrict__ offsets, int* __restrict__ slot_of, int* __restrict__ row_of_slot,
                     uint32_t* __restrict__ counter) {
  __shared__ float lg[TG_ROWS][257];
  __shared__ uint64_t s_cand[TG_ROWS][32];
  __shared__ int s_sel[TG_ROWS][8];
  __shared__ float s_mz[TG_ROWS][2];
  __shared__ int s_last;
  const int lane = lane_id(), wave = wave_id();
  const int sub = wave / 5, w5 = wave % 5, r = blockIdx.x * TG_ROWS + sub;
  const bool active = sub < TG_ROWS && r < rows;
  for (int i = threadIdx.x; i < TG_ROWS * (E + 1); i += GR_THREADS) {
    const int s = i / (E + 1), e = i - s * (E + 1), rr = blockIdx.x * TG_ROWS + s;
    if (rr < rows) lg[s][e] = logits[(size_t)rr * stride + e];
  }
  __syncthreads();
  if (active && topk <= 8) {
    if (w5 < 4) {
      int ck, ce;
      canon_select_group8(lg[sub], E, w5, &ck, &ce);
      if (lane < 8) s_cand[sub][w5 * 8 + lane] = canon_cand64(ck, ce);
    } else {
      float m;
      const float z = canon_softmax_z(lg[sub], E, &m);
      if (lane == 0) s_mz[sub][0] = m, s_mz[sub][1] = z;
    }
  }
  __syncthreads();
  if (active && w5 == 0) {
    int id;
    float w;
    if (topk <= 8) {
      id = merge_picks(s_cand[sub], s_sel[sub], topk);
      w = canon_topk_weight(lg[sub][lane < topk ? id : 0], s_mz[sub][0], s_mz[sub][1], topk);
    } else {
      canon_softmax_topk(lg[sub], E, topk, &id, &w);
    }
    if (lane < topk) {
      __hip_atomic_store(idx + (size_t)r * topk + lane, id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      wts[(size_t)r * topk + lane] = w;
    }
    if (lane == 0) sgate[r] = lg[sub][E];
  }
  // Hand-over to the last block.  The idx words are the only data handed over, and they are
  // stored with agent-scope atomic stores (written through to the device-coherent level, not
  // left in this XCD's L2); s_waitcnt(0) waits until those stores are acknowledged, the barrier
  // orders every wave's acknowledgement before thread 0's count, and the last block reads idx
  // with agent-scope atomic loads (not served from a possibly stale L2 line).  A release /
  // acquire pair on the count would instead write back and invalidate the whole L2 of each
  // block's XCD: measured 12.1 -> 14.4 us for this kernel at 300 rows.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0)
    s_last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
  __syncthreads();
  if (!s_last) return;
  group_block([&](int i) { return __hip_atomic_load(idx + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); },
              rows * topk, E, counts, offsets, slot_of, 0, nullptr, row_of_slot, topk);
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// xp[slot_of[i]] = x[i / topk]: 16 bytes per thread, one pair per 256-thread block.
__global__ void __launch_bounds__(256)
    k_gather_rows(const int* __restrict__ slot_of, int topk, const uint16_t* __restrict__ x, uint16_t* __restrict__ xp,
                  int H) {
  const int i = blockIdx.x;
  const int slot = slot_of[i];
  const uint4* src = reinterpret_cast<const uint4*>(x + (size_t)(i / topk) * H);
  uint4* dst = reinterpret_cast<uint4*>(xp + (size_t)slot * H);
  for (int c = threadIdx.x; c < H / 8; c += blockDim.x) dst[c] = src[c];
}

__global__ void k_count(const int* __restrict__ idx, int n, int* __restrict__ counts) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) atomicAdd(counts + idx[i], 1);
}

// x[r, c] += sigmoid(sgate[r]) * shared[r, c] + sum_k wts[r, k] * y[slot_of[r, k], c], k ascending.
// Block = one row and 1024 columns (one float4 per thread); TK > 0: topk fixed at compile time,
// so all TK row loads of a thread are in flight together.
template <int TK>
__global__ void __launch_bounds__(256)
    k_combine(float* __restrict__ x, const float* __restrict__ y, const int* __restrict__ slot_of,
              const float* __restrict__ wts, const float* __restrict__ sgate, const float* __restrict__ shared,
              int topk, int H) {
  const int r = blockIdx.x, c = (blockIdx.y * 256 + threadIdx.x) * 4;
  if (c >= H) return;
  const int K = TK > 0 ? TK : topk;
  const float sg = sigmoid(sgate[r]);
  const float4 sh = *reinterpret_cast<const float4*>(shared + (size_t)r * H + c);
  float4 acc = make_float4(sg * sh.x, sg * sh.y, sg * sh.z, sg * sh.w);
#pragma unroll
  for (int k = 0; k < (TK > 0 ? TK : 32); ++k) {
    if (TK == 0 && k >= K) break;
    const float w = wts[r * K + k];
    const float4 v = *reinterpret_cast<const float4*>(y + (size_t)slot_of[r * K + k] * H + c);
    acc.x += w * v.x, acc.y += w * v.y, acc.z += w * v.z, acc.w += w * v.w;
  }
  float4* xo = reinterpret_cast<float4*>(x + (size_t)r * H + c);
  float4 o = *xo;
  o.x += acc.x, o.y += acc.y, o.z += acc.z, o.w += acc.w;
  *xo = o;
}

__global__ void k_dequant_q8(const int8_t* __restrict__ W, const uint16_t* __restrict__ S, uint16_t* __restrict__ out,
                             size_t n, int K) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const size_t row = i / K, col = i % K;
  out[i] = to_bf16((float)W[i] * f16f(S[row * (K / 128) + col / 128]));
}

__global__ void k_f32_to_bf16(const float* __restrict__ x, uint16_t* __restrict__ y, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = to_bf16(x[i]);
}

__global__ void k_swiglu_rows(const float* __restrict__ h, uint16_t* __restrict__ y, int rows, int I) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)rows * I) return;
  const size_t r = i / I, j = i % I;
  y[i] = to_bf16(silu(h[r * 2 * I + j]) * h[r * 2 * I + I + j]);
}

}  // namespace

API int dr_moe_group(const int* idx, int n, int E, int* counts, int* offsets, int* slot_of, hipStream_t st) {
  if (n < 0 || n > GR_MAXN || E < 1 || E > 256) return -1;
  hipLaunchKernelGGL(k_group, dim3(1), dim3(GR_THREADS), 0, st, idx, n, E, counts, offsets, slot_of, 0, nullptr,
                     nullptr, 1);
  return 0;
}

API int dr_moe_group_rows(const int* idx, int rows, int topk, int E, int* counts, int* offsets, int* slot_of,
                         int* row_of_slot, hipStream_t st) {
  if (rows < 0 || topk < 1 || (long long)rows * topk > GR_MAXN || E < 1 || E > 256 || !row_of_slot) return -1;
  hipLaunchKernelGGL(k_group, dim3(1), dim3(GR_THREADS), 0, st, idx, rows * topk, E, counts, offsets, slot_of, 0,
                     nullptr, row_of_slot, topk);
  return 0;
}

API int dr_moe_topk_group(const float* logits, int rows, int E, int topk, int stride, int* idx, float* wts,
                         float* sgate, int* counts, int* offsets, int* slot_of, int* row_of_slot, uint32_t* counter,
                         hipStream_t st) {
  if (E > 256 || E < 1 || topk > 32 || topk < 1 || topk > E || stride < E + 1 || rows < 0 ||
      (long long)rows * topk > GR_MAXN || !counter)
    return -1;
  if (rows == 0) return 0;
  hipLaunchKernelGGL(k_moe_topk_group, dim3((rows + TG_ROWS - 1) / TG_ROWS), dim3(GR_THREADS), 0, st, logits, rows, E,
                     topk, stride, idx, wts, sgate, counts, offsets, slot_of, row_of_slot, counter);
  return 0;
}

API int dr_moe_gather_rows(const int* slot_of, int rows, int topk, const uint16_t* x, uint16_t* xp, int H,
                           hipStream_t st) {
  if (H % 8 != 0 || rows < 0 || topk < 1) return -1;
  if (rows == 0) return 0;
  hipLaunchKernelGGL(k_gather_rows, dim3(rows * topk), dim3(256), 0, st, slot_of, topk, x, xp, H);
  return 0;
}

API int dr_moe_count(const int* idx, int n, int* counts, hipStream_t st) {
  if (n < 0) return -1;
  if (n == 0) return 0;
  hipLaunchKernelGGL(k_count, dim3((n + 255) / 256), dim3(256), 0, st, idx, n, counts);
  return 0;
}

API int dr_moe_permute(const int* idx, int rows, int topk, const int* offsets, int* fill, int* slot_of,
                       const uint16_t* x, uint16_t* xp, int H, hipStream_t st) {
  if (rows < 0 || topk < 1 || H % 8 != 0) return -1;
  const long long nl = (long long)rows * topk;
  if (nl > (1ll << 30)) return -1;
  const int n = (int)nl;
  if (n == 0) return 0;
  // segments of GR_MAXN pairs in stream order; fill (zero on entry) is the running base
  for (int s0 = 0; s0 < n; s0 += GR_MAXN) {
    const int m = n - s0 < GR_MAXN ? n - s0 : GR_MAXN;
    hipLaunchKernelGGL(k_group, dim3(1), dim3(GR_THREADS), 0, st, idx + s0, m, 256, nullptr,
                       const_cast<int*>(offsets), slot_of + s0, 1, fill, nullptr, 1);
  }
  hipLaunchKernelGGL(k_gather_rows, dim3(n), dim3(256), 0, st, slot_of, topk, x, xp, H);
  return 0;
}

API int dr_moe_combine(float* x, const float* y, const int* slot_of, const float* wts, const float* sgate,
                       const float* shared, int rows, int topk, int H, hipStream_t st) {
  if (topk < 1 || topk > 32 || H % 4 != 0) return -1;
  if (rows <= 0) return 0;
  const dim3 grid(rows, (H / 4 + 255) / 256);
  if (topk == 8)
    hipLaunchKernelGGL(k_combine<8>, grid, dim3(256), 0, st, x, y, slot_of, wts, sgate, shared, topk, H);
  else
    hipLaunchKernelGGL(k_combine<0>, grid, dim3(256), 0, st, x, y, slot_of, wts, sgate, shared, topk, H);
  return 0;
}

API int dr_dequant_q8(const int8_t* W, const uint16_t* S, uint16_t* out, int N, int K, hipStream_t st) {
  if (K % 128 != 0) return -1;
  const size_t n = (size_t)N * K;
  if (n == 0) return 0;
  hipLaunchKernelGGL(k_dequant_q8, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, W, S, out, n, K);
  return 0;
}

API int dr_f32_to_bf16(const float* x, uint16_t* y, size_t n, hipStream_t st) {
  if (n == 0) return 0;
  hipLaunchKernelGGL(k_f32_to_bf16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, y, n);
  return 0;
}

API int dr_swiglu_rows(const float* h, uint16_t* y, int rows, int I, hipStream_t st) {
  const size_t n = (size_t)rows * I;
  if (n == 0) return 0;
  hipLaunchKernelGGL(k_swiglu_rows, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, h, y, rows, I);
  return 0;
}

// Decode router for B rows (B <= 8) as one block's work: shared by dr_router_topk (B = 1),
// dr_router_topk_rows (a launch of router blocks only) and the fused small-batch FP8 kernel
// (router blocks ahead of the gate_up blocks in one launch).  Reference semantics:
// kernels/drama.cu:317-461 per row.
//
// Block blk of nblk: wave w computes logit row RT_WPB blk + w for every row, its weight row
// loaded once.  The rows of x are staged in LDS, wave r < B computes row r's canonical RMSNorm
// scale, and the block normalises the staged rows in place (canon_norm4 is elementwise, so the
// values equal those of the canonical norm in registers).  Every logit has the canonical order
// of canon.hpp, so each row's logits, picks and weights equal the CPU oracle's on that row.
// Logits are published with cache-bypassing (sc1) stores; each block counts itself in once its
// stores completed, and the last block loads the logits of all rows at once and
// spreads the per-row work over its waves: for topk <= 8 and 2 B <= RT_WPB one wave selects
// each row's top-k over all its experts (canon_select_topk) beside the B softmax
// denominators; above 4 rows the 4 B group selections come first and one rank merge per row
// replaces the row selection; the picks go out at once, then the weights follow; for topk > 8
// one wave per row does both.  It writes idx, wts and sgate, and (tags != nullptr) also
// publishes them as tagged words
// (tag << 32) | value bits with cache-bypassing stores, for blocks of the same launch to poll:
// row r's experts at tags[r topk ..] (and, for B topk <= 32, in RR_REPS replicas), its
// weights at tags[(B + r) topk ..], its shared-expert gate logit at tags[2 B topk + r].
// It resets the counter.  Every thread returns normally (no early exit), so callers may add
// work after it.
#pragma once
#include "canon.hpp"

namespace drm {

constexpr int RT_WPB = 8;  // router waves (= logit rows) per block
// Replicas of the tagged experts for pollers (replica r of word i at tags[RR_WORD0 + 32 r + i],
// one replica per 256 bytes, B topk <= 32): hundreds of pollers on one cache line serialise.
constexpr int RR_REPS = 16, RR_WORD0 = 128;

template <int B>
DEV void router_rows_block(int blk, int nblk, const uint16_t* __restrict__ W, const float* __restrict__ x,
                           const float* __restrict__ nw, float eps, float* __restrict__ logits, int E, int topk,
                           int* __restrict__ idx, float* __restrict__ wts, float* __restrict__ sgate,
                           uint32_t* __restrict__ counter, uint64_t* __restrict__ tags, uint32_t tag,
                           float4 (*xs)[2048 / 4]) {
#pragma clang fp contract(off)
  constexpr int K = 2048, NCH = K / 8 / WAVE, NRM = K / 4 / WAVE, NT = RT_WPB * 64;
  __shared__ float s_inv[B];
  __shared__ int s_last;
  const int lane = lane_id(), wave = wave_id();
  const int row = blk * RT_WPB + wave;
  uint4 w[NCH];
  if (row <= E) {
    const uint16_t* wr = W + (size_t)row * K;
#pragma unroll
    for (int j = 0; j < NCH; ++j) w[j] = ld16(wr + (size_t)(lane + WAVE * j) * 8);
  }
  const float4* x4 = reinterpret_cast<const float4*>(x);
  const float4* n4 = reinterpret_cast<const float4*>(nw);
  float4 nv[K / 4 / NT];
  if (nw) {
#pragma unroll
    for (int i = 0; i < K / 4 / NT; ++i) nv[i] = n4[threadIdx.x + NT * i];
  }
#pragma unroll
  for (int i = threadIdx.x; i < B * K / 4; i += NT) xs[i / (K / 4)][i % (K / 4)] = x4[i];
  __syncthreads();
  if (nw) {
    if (wave < B) {
      float4 xr[NRM];
#pragma unroll
      for (int j = 0; j < NRM; ++j) xr[j] = xs[wave][lane + WAVE * j];
      const float inv = canon_rms_inv_regs<NRM>(xr, eps);
      if (lane == 0) s_inv[wave] = inv;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < B; ++r)
#pragma unroll
      for (int i = 0; i < K / 4 / NT; ++i) {
        const int c = threadIdx.x + NT * i;
        xs[r][c] = canon_norm4(xs[r][c], s_inv[r], nv[i]);
      }
    __syncthreads();
  }
  if (row <= E) {
#pragma unroll
    for (int r = 0; r < B; ++r) {
      float4 xa[NCH], xb[NCH];
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        const int c = lane + WAVE * j;
        xa[j] = xs[r][2 * c], xb[j] = xs[r][2 * c + 1];
      }
      const float acc = canon_row_dot<NCH>(w, xa, xb);
      if (lane == 0) __hip_atomic_store(logits + (size_t)r * (E + 1) + row, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0)
    s_last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)nblk - 1;
  __syncthreads();
  if (!s_last) return;
  __shared__ float lg[B][257];
  __shared__ uint64_t s_cand[B][32];
  __shared__ int s_sel[B][8];
  __shared__ float s_mz[B][2];
  {
    // every row's logits requested at once (one round trip), then stored
    constexpr int NL = (B * 257 + NT - 1) / NT;
    float v[NL];
#pragma unroll
    for (int t = 0; t < NL; ++t) {
      const int i = threadIdx.x + NT * t;
      v[t] = i < B * (E + 1) ? __hip_atomic_load(logits + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.f;
    }
#pragma unroll
    for (int t = 0; t < NL; ++t) {
      const int i = threadIdx.x + NT * t;
      if (i < B * (E + 1)) {
        const int r = i / (E + 1);
        lg[r][i - r * (E + 1)] = v[t];
      }
    }
  }
  __syncthreads();
  auto publish = [&](int r, int id, float wt) {
    if (lane < topk) {
      idx[r * topk + lane] = id, wts[r * topk + lane] = wt;
      if (tags) {
        __hip_atomic_store(tags + r * topk + lane, ((uint64_t)tag << 32) | (uint32_t)id, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(tags + (B + r) * topk + lane, ((uint64_t)tag << 32) | __float_as_uint(wt),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  };
  if (topk <= 8) {
    // the 4 B group selections first, then each row's rank merge (its picks are published at
    // once: the gate_up blocks of the fused launch wait for them) beside the B softmax
    // denominators, then the weights
    constexpr bool kRowWave = 2 * B <= RT_WPB;  // one wave selects a whole row (8 rounds over 256)
    if constexpr (!kRowWave) {
      for (int t = wave; t < 4 * B; t += RT_WPB) {
        int ck, ce;
        canon_select_group8(lg[t >> 2], E, t & 3, &ck, &ce);
        if (lane < 8) s_cand[t >> 2][(t & 3) * 8 + lane] = canon_cand64(ck, ce);
      }
      __syncthreads();
    }
    for (int t = wave; t < 2 * B; t += RT_WPB) {
      if (t < B) {
        int id;
        if constexpr (kRowWave) {
          id = canon_select_topk(lg[t], E, topk);
          if (lane < topk) s_sel[t][lane] = id;
        } else {
          id = merge_picks(s_cand[t], s_sel[t], topk);
        }
        if (lane < topk) {
          idx[t * topk + lane] = id;
          if (tags) {
            const uint64_t v = ((uint64_t)tag << 32) | (uint32_t)id;
            __hip_atomic_store(tags + t * topk + lane, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (B * topk <= 32) {
#pragma unroll
              for (int rp = 0; rp < RR_REPS; ++rp)
                __hip_atomic_store(tags + RR_WORD0 + 32 * rp + t * topk + lane, v, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            }
          }
        }
      } else {
        float m;
        const float z = canon_softmax_z(lg[t - B], E, &m);
        if (lane == 0) s_mz[t - B][0] = m, s_mz[t - B][1] = z;
      }
    }
    __syncthreads();
    for (int r = wave; r < B; r += RT_WPB) {
      const int id = lane < topk ? s_sel[r][lane] : 0;
      const float wt = canon_topk_weight(lg[r][id], s_mz[r][0], s_mz[r][1], topk);
      if (lane < topk) {
        wts[r * topk + lane] = wt;
        if (tags)
          __hip_atomic_store(tags + (B + r) * topk + lane, ((uint64_t)tag << 32) | __float_as_uint(wt),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  } else {
    for (int r = wave; r < B; r += RT_WPB) {
      int my_idx;
      float my_w;
      canon_softmax_topk(lg[r], E, topk, &my_idx, &my_w);
      publish(r, my_idx, my_w);
    }
  }
  if ((int)threadIdx.x < B) {
    sgate[threadIdx.x] = lg[threadIdx.x][E];
    if (tags)
      __hip_atomic_store(tags + 2 * B * topk + threadIdx.x, ((uint64_t)tag << 32) | __float_as_uint(lg[threadIdx.x][E]),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace drm

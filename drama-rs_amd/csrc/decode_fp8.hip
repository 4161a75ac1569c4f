// Batch-1 decode MoE with block-FP8 (OCP e4m3) routed experts (reference:
// kernels/drama.cu:602-742, src/ffi.rs:47-51).  Same structure as the int4 decode:
//   gate_up: a 2048-byte e4m3 row is two 16-byte loads per lane (bytes [16 l, 16 l + 16) and
//            [1024 + 16 l, ...)), the layout of the int8 shared rows, so routed and shared
//            blocks stage x̂ identically; e4m3 -> f32 with v_cvt_pk_f32_fp8 (exact);
//   down:    one output row gathers 8 expert rows of 512 bytes: 4 loads per lane, load i
//            covering experts 2 i (lanes 0-31) and 2 i + 1 (lanes 32-63), plus 8 bytes of the
//            int8 shared row.
// One scale per 128 x 128 block (f32 scale_inv in the reference layout, bf16 in the
// benchmark configuration); every 16-element lane chunk lies inside one block.
#include <type_traits>

#include "router_rows.hpp"

using namespace drm;

namespace {

constexpr int H8 = 2048, I8 = 512, TOPK8 = 8;

DEV float dot16_u8b(const uint4& w, const float* x, float acc) {
  acc = dot4_u8b(w.x, x, acc);
  acc = dot4_u8b(w.y, x + 4, acc);
  acc = dot4_u8b(w.z, x + 8, acc);
  return dot4_u8b(w.w, x + 12, acc);
}

DEV void unpack16(const float4* xs, int lane, float (&xa)[16], float (&xb)[16], float& sa, float& sb) {
  sa = 0.f, sb = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 v = xs[i * 64 + lane], w = xs[256 + i * 64 + lane];
    xa[4 * i] = v.x, xa[4 * i + 1] = v.y, xa[4 * i + 2] = v.z, xa[4 * i + 3] = v.w;
    xb[4 * i] = w.x, xb[4 * i + 1] = w.y, xb[4 * i + 2] = w.z, xb[4 * i + 3] = w.w;
    sa += (v.x + v.y) + (v.z + v.w);
    sb += (w.x + w.y) + (w.z + w.w);
  }
}

// gate_up of B decode rows.  Routed units are (row b, pick k, pair j), j fastest; the routed
// waves walk them spaced by the grid (wave g of NW takes units g, g + NW, ..., so waves running
// side by side read neighbouring rows of one expert), keeping D units in flight and loading
// unit p + D once unit p is computed.  The shared expert's pairs (PPWS per wave, all loaded at
// once) serve all B rows with one read of their weights.  Both read x̂ staged in LDS by XStage.
template <int SF, int D, int B, int NW>
struct RoutedFP8 {
  static constexpr int H = H8, I = I8, PPW = B * TOPK8 * I / NW;
  static_assert(PPW * NW == B * TOPK8 * I && D <= PPW, "units split evenly over the routed waves");
  uint4 g0[D], g1[D], u0[D], u1[D];
  uint32_t sr[D][4];
  template <class Picks>
  DEV void issue(const uint8_t* __restrict__ W, const void* __restrict__ S, const Picks& picks, int g, int p, int d) {
    const int lane = lane_id();
    const int u = g + NW * p, b = u / (TOPK8 * I), k = (u / I) % TOPK8, j = u % I;
    const size_t e = (size_t)picks.get(b * TOPK8 + k);
    const uint8_t* rg = W + (e * (2 * I) + j) * H + lane * 16;
    const uint8_t* ru = rg + (size_t)I * H;
    g0[d] = ld16(rg), g1[d] = ld16(rg + 1024), u0[d] = ld16(ru), u1[d] = ld16(ru + 1024);
    const size_t sb = e * (size_t)(2 * I / 128) * (H / 128);
    sr[d][0] = blk_raw<SF>(S, sb + (size_t)(j >> 7) * (H / 128) + (lane >> 3));
    sr[d][1] = blk_raw<SF>(S, sb + (size_t)(j >> 7) * (H / 128) + 8 + (lane >> 3));
    sr[d][2] = blk_raw<SF>(S, sb + (size_t)((I + j) >> 7) * (H / 128) + (lane >> 3));
    sr[d][3] = blk_raw<SF>(S, sb + (size_t)((I + j) >> 7) * (H / 128) + 8 + (lane >> 3));
    __builtin_amdgcn_sched_barrier(0);
  }
  // units 0 .. D - 1 issued, x̂ staged
  template <class Picks>
  DEV void run(const uint8_t* __restrict__ W, const void* __restrict__ S, const Picks& picks, int g,
               const float4* xs, float* __restrict__ act) {
    const int lane = lane_id();
#pragma unroll
    for (int p = 0; p < PPW; ++p) {
      const int d = p % D;
      const int u = g + NW * p, b = u / (TOPK8 * I), k = (u / I) % TOPK8, j = u % I;
      float xa[16], xb[16], sa, sbm;
      unpack16(xs + b * (H / 4), lane, xa, xb, sa, sbm);
      opaque(g0[d]), opaque(g1[d]), opaque(u0[d]), opaque(u1[d]);
      float gv = blk_cvt<SF>(sr[d][0]) * dot16_fp8(g0[d], xa, 0.f) + blk_cvt<SF>(sr[d][1]) * dot16_fp8(g1[d], xb, 0.f);
      float uv = blk_cvt<SF>(sr[d][2]) * dot16_fp8(u0[d], xa, 0.f) + blk_cvt<SF>(sr[d][3]) * dot16_fp8(u1[d], xb, 0.f);
      if (p + D < PPW) issue(W, S, picks, g, p + D, d);
      gv = wave_sum(gv);
      uv = wave_sum(uv);
      if (lane == 0) act[(size_t)b * (TOPK8 + 1) * I + k * I + j] = silu(gv) * uv;
    }
  }
};

template <class SH, int PPWS, int B>
struct SharedFP8 {
  static constexpr int H = H8, I = I8;
  uint4 g0[PPWS], g1[PPWS], u0[PPWS], u1[PPWS];
  float sg0[PPWS], sg1[PPWS], su0[PPWS], su1[PPWS];
  DEV void load(const int8_t* __restrict__ shq, const uint16_t* __restrict__ shs, int j0) {
    const int lane = lane_id();
#pragma unroll
    for (int p = 0; p < PPWS; ++p) {
      const uint8_t* rg = reinterpret_cast<const uint8_t*>(shq) + (size_t)(j0 + p) * H + lane * 16;
      const uint8_t* ru = reinterpret_cast<const uint8_t*>(shq) + (size_t)(I + j0 + p) * H + lane * 16;
      g0[p] = ld16(rg), g1[p] = ld16(rg + 1024), u0[p] = ld16(ru), u1[p] = ld16(ru + 1024);
    }
#pragma unroll
    for (int p = 0; p < PPWS; ++p) {
      const int j = j0 + p;
      sg0[p] = SH::scale(shs, j, lane * 16, H), sg1[p] = SH::scale(shs, j, 1024 + lane * 16, H);
      su0[p] = SH::scale(shs, I + j, lane * 16, H), su1[p] = SH::scale(shs, I + j, 1024 + lane * 16, H);
    }
  }
  DEV void run(const float4* xs, float* __restrict__ act, int j0) {
    const int lane = lane_id();
#pragma unroll 1
    for (int r = 0; r < B; ++r) {
      pin_weights(g0, g1, u0, u1);  // converted per row, not hoisted out of the row loop
      float xa[16], xb[16], sa, sbm;
      unpack16(xs + r * (H / 4), lane, xa, xb, sa, sbm);
      float* ar = act + (size_t)r * (TOPK8 + 1) * I + TOPK8 * I + j0;
#pragma unroll
      for (int p = 0; p < PPWS; ++p) {
        float g = sg0[p] * (dot16_u8b(g0[p], xa, 0.f) - 128.f * sa) + sg1[p] * (dot16_u8b(g1[p], xb, 0.f) - 128.f * sbm);
        float u = su0[p] * (dot16_u8b(u0[p], xa, 0.f) - 128.f * sa) + su1[p] * (dot16_u8b(u1[p], xb, 0.f) - 128.f * sbm);
        g = wave_sum(g);
        u = wave_sum(u);
        if (lane == 0) ar[p] = silu(g) * u;
      }
    }
  }
};

// Block blk of the gate_up grid: NBS shared-expert blocks first, then the NBR routed blocks.
// x (and the norm weight) are requested before the weights, so the staging overlaps the
// fetch; a routed block's picks come from Picks (wait() by every thread, get(i) = pick i).
template <int SF, class SH, int WPB, int NBR, int D, int PPWS, int B, class Picks>
DEV void gate_up_fp8_block(int blk, const uint8_t* __restrict__ W, const void* __restrict__ S,
                           const int8_t* __restrict__ shq, const uint16_t* __restrict__ shs, const float* x,
                           const Picks& picks, float* __restrict__ act, const float* nw, float eps, float4* xs) {
  constexpr int NT = WPB * 64, NW = NBR * WPB;
  constexpr int NBS = I8 / (WPB * PPWS);  // shared-expert blocks, dispatched first
  const int wave = wave_id();
  XStage<H8, NT, B, SlotQ8H> xst;
  xst.load(x, nw);
  if (blk >= NBS) {
    const int g = (blk - NBS) * WPB + wave;
    picks.wait();
    RoutedFP8<SF, D, B, NW> ru;
#pragma unroll
    for (int p = 0; p < D; ++p) ru.issue(W, S, picks, g, p, p);
    xst.finish(nw != nullptr, eps, xs);
    ru.run(W, S, picks, g, xs, act);
  } else {
    const int j0 = (blk * WPB + wave) * PPWS;
    SharedFP8<SH, PPWS, B> sh;
    sh.load(shq, shs, j0);
    xst.finish(nw != nullptr, eps, xs);
    sh.run(xs, act, j0);
  }
}

struct PicksGlobal {
  const int* idx;
  DEV void wait() const {}
  DEV int get(int i) const { return idx[i]; }
};

template <int SF, class SH, int WPB, int NBR, int D, int PPWS, int B>
__global__ void __launch_bounds__(WPB * 64) __attribute__((amdgpu_waves_per_eu(WPB == 8 ? 4 : 1)))
    k_moe_gate_up_fp8(const uint8_t* __restrict__ W, const void* __restrict__ S, const int8_t* __restrict__ shq,
                      const uint16_t* __restrict__ shs, const float* x, const int* __restrict__ idx,
                      float* __restrict__ act, const float* nw, float eps) {
  __shared__ float4 xs[B * H8 / 4];
  gate_up_fp8_block<SF, SH, WPB, NBR, D, PPWS, B>(blockIdx.x, W, S, shq, shs, x, PicksGlobal{idx}, act, nw, eps, xs);
}

// The picks of the fused router + gate_up launch: wave 0 of the block polls its replica of the
// B * 8 tagged words (tag << 32) | expert that the router's last block publishes, until every
// tag is the
// launch's (bounded: on time-out DR_ERR_ROUTE_WAIT is raised and expert 0 is used), and leaves
// the experts in LDS for the block.
template <int B>
struct PicksTagged {
  const uint64_t* tags;
  uint32_t tag;
  int* s_idx;
  uint32_t* err;
  DEV void wait() const {
    constexpr int n = B * TOPK8;
    if (wave_id() == 0) {
      const int lane = lane_id();
      // this block's replica of the experts (router_rows.hpp)
      const uint64_t* rep = tags + RR_WORD0 + 32 * (blockIdx.x % RR_REPS);
      uint64_t v = (uint64_t)tag << 32;
      for (int it = 0;; ++it) {
        if (lane < n) v = __hip_atomic_load(rep + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (__ballot((uint32_t)(v >> 32) != tag) == 0) break;
        if (it == (1 << 20)) {
          if (lane == 0) raise_err(err, kErrRouteWait);
          v = (uint64_t)tag << 32;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
      if (lane < n) s_idx[lane] = (int)(uint32_t)v;
    }
    __syncthreads();
  }
  DEV int get(int i) const { return s_idx[i]; }
};

// The launch's finished-block count without one hot address (hundreds of same-address
// atomics serialise): block c of nb adds itself to group counter c % RC_G, each on its own
// 128-byte line in the tags buffer after the picks, and the block that fills its group adds
// one to a top counter; the block that fills the top is the launch's last.  Counters start at
// zero and the last block resets them.
constexpr int RC_G = 16, RC_DONE = RR_WORD0 + 32 * RR_REPS, RC_WORDS = RC_DONE + 16 * RC_G;
static_assert(RC_WORDS == 896, "the tags buffer size the header states");
static_assert(RR_WORD0 >= 4 * (2 * TOPK8 + 1) && 4 * TOPK8 <= 32, "picks, then their replicas, then the counters");
DEV uint32_t* rc_ctr(uint64_t* tags, int base, int g) { return reinterpret_cast<uint32_t*>(tags + base + 16 * g); }
DEV uint32_t rc_n(int nb, int g) { return (uint32_t)(nb / RC_G + (g < nb % RC_G ? 1 : 0)); }
// one thread per block; true for the block that completes the count
DEV bool rc_add(uint64_t* tags, int base, uint32_t* top, int c, int nb) {
  const int g = c % RC_G;
  if (__hip_atomic_fetch_add(rc_ctr(tags, base, g), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != rc_n(nb, g) - 1u)
    return false;
  return __hip_atomic_fetch_add(top, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)RC_G - 1u;
}
// one wave
DEV void rc_reset(uint64_t* tags, int base) {
  if (lane_id() < RC_G) __hip_atomic_store(rc_ctr(tags, base, lane_id()), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// End of a launch, wave 0 of every block: the block that completes the done count resets the
// done counters and counter[2] and advances the tag in counter[1].  Every block read the tag
// at its start, before it counted.
DEV void launch_done(uint64_t* tags, uint32_t* counter, int blk, int nb, uint32_t tag) {
  const int lane = lane_id();
  bool last = false;
  if (lane == 0) last = rc_add(tags, RC_DONE, counter + 2, blk, nb);
  if (!__ballot(last)) return;
  rc_reset(tags, RC_DONE);
  if (lane == 0) {
    __hip_atomic_store(counter + 2, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(counter + 1, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Router, top-k and gate_up of B decode rows in one launch of RG_BLOCKS blocks, one per
// routed gate_up slice: every wave takes B units (RoutedFP8, D in flight) once the picks are
// there.  Before that, blocks [0, NRB) run the router of router_rows.hpp (its last block
// publishes the picks as tagged words) and blocks [NRB, NRB + RG_NBS) the shared expert's
// pairs (which need no picks), so the router's and the shared expert's time is spent while the
// picks are awaited, and no block waits for a free slot (two blocks per CU hold the grid).
// Wave 0 of each block polls the picks.  counter: [0] the router's arrivals (reset by its last
// block), [1] the tag of the previous launch, [2] the top of the finished-block count
// (launch_done), whose last block advances [1], so every launch tags its picks afresh.
constexpr int RG_BLOCKS = 512, RG_PPWS = 2, RG_NBS = I8 / (8 * RG_PPWS);
constexpr uint64_t RG_X_DELAY = 300;  // measured: 3 µs ahead of the router rows 8.1 -> 7.8 µs, launch -1 µs
template <int SF, class SH, int D, int B>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4)))
    k_moe_route_gate_up_fp8(const uint16_t* __restrict__ RW, float* __restrict__ logits, int E,
                            int* __restrict__ idx, float* __restrict__ wts, float* __restrict__ sgate,
                            uint32_t* __restrict__ counter, uint64_t* __restrict__ tags, uint32_t* err,
                            const uint8_t* __restrict__ W, const void* __restrict__ S,
                            const int8_t* __restrict__ shq, const uint16_t* __restrict__ shs, const float* x,
                            float* __restrict__ act, const float* nw, float eps) {
  __shared__ float4 xs[B * H8 / 4];
  __shared__ int s_idx[B * TOPK8];
  __shared__ uint32_t s_tag;
  if (threadIdx.x == 0) s_tag = __hip_atomic_load(counter + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
  __syncthreads();
  const uint32_t tag = s_tag;
  const int blk = blockIdx.x, wave = wave_id();
  const int nrb = (E + RT_WPB) / RT_WPB;
  if (blk < nrb) {
    router_rows_block<B>(blk, nrb, RW, x, nw, eps, logits, E, TOPK8, idx, wts, sgate, counter, tags, tag,
                         reinterpret_cast<float4(*)[H8 / 4]>(xs));
    __syncthreads();  // the router's staging in xs is done with
  }
  const bool shared = blk >= nrb && blk < nrb + RG_NBS;
  if (blk >= nrb + RG_NBS) {
    // the routed-only blocks request their x RG_X_DELAY ticks (10 ns) late: their units wait
    // for the picks anyway, and their 32 KB each would otherwise queue ahead of the router's
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while (__builtin_amdgcn_s_memrealtime() - t0 < RG_X_DELAY) __builtin_amdgcn_s_sleep(8);
  }
  XStage<H8, 512, B, SlotQ8H> xst;
  xst.load(x, nw);
  const int j0 = ((blk - nrb) * 8 + wave) * RG_PPWS;
  if (shared) {
    SharedFP8<SH, RG_PPWS, B> sh;
    sh.load(shq, shs, j0);
    xst.finish(nw != nullptr, eps, xs);
    sh.run(xs, act, j0);
  } else {
    xst.finish(nw != nullptr, eps, xs);
  }
  const PicksTagged<B> picks{tags, tag, s_idx, err};
  picks.wait();
  const int g = blk * 8 + wave;
  RoutedFP8<SF, D, B, RG_BLOCKS * 8> ru;
#pragma unroll
  for (int p = 0; p < D; ++p) ru.issue(W, S, picks, g, p, p);
  ru.run(W, S, picks, g, xs, act);
  if (wave == 0) launch_done(tags, counter, blk, RG_BLOCKS, tag);
}

// The down weights of output rows n0 .. n0 + RPW - 1: per row the 8 routed expert rows of
// 512 bytes (load i: experts 2 i on lanes 0-31, 2 i + 1 on lanes 32-63, e[i] per lane) and 8
// bytes of the int8 shared row per lane.
template <int SF, class SH, int RPW>
struct DownFP8 {
  uint4 q[RPW][4];
  uint32_t sc[RPW][4];
  uint2 qs[RPW];
  uint32_t ssr[RPW];
  DEV void issue(const uint8_t* __restrict__ W, const void* __restrict__ S, const int8_t* __restrict__ shq,
                 const uint16_t* __restrict__ shs, const size_t (&e)[4], int n0) {
    constexpr int H = H8, I = I8;
    const int lane = lane_id(), cc = lane & 31;
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const size_t n = (size_t)(n0 + r);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        q[r][i] = ld16(W + (e[i] * H + n) * I + cc * 16);
        sc[r][i] = blk_raw<SF>(S, (e[i] * (H / 128) + (n >> 7)) * (I / 128) + (cc >> 3));
      }
      qs[r] = ld8(shq + n * I + lane * 8);
      ssr[r] = SH::raw(shs, n, lane * 8, I);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // as: the row's activations staged by stage_slot (routed part in lane slices, shared part at
  // 1024); w[i] the pick weight of e[i]; y[n] = res[n] + routed + sigmoid(gate) * shared
  DEV void finish(const float4* as, const float (&w)[4], float sgv, const float* res, float* y, uint16_t* yb,
                  size_t nb) const {
    const int lane = lane_id();
    float xa[4][16], xc[8], sumc = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const float4 v = as[256 * i + t * 64 + lane];
        xa[i][4 * t] = v.x, xa[i][4 * t + 1] = v.y, xa[i][4 * t + 2] = v.z, xa[i][4 * t + 3] = v.w;
      }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const float4 v = as[1024 + t * 64 + lane];
      xc[4 * t] = v.x, xc[4 * t + 1] = v.y, xc[4 * t + 2] = v.z, xc[4 * t + 3] = v.w;
      sumc += (v.x + v.y) + (v.z + v.w);
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) acc += w[i] * blk_cvt<SF>(sc[r][i]) * dot16_fp8(q[r][i], xa[i], 0.f);
      float dc = dot4_u8b(qs[r].x, xc, 0.f);
      dc = dot4_u8b(qs[r].y, xc + 4, dc);
      acc += sgv * SH::cvt(ssr[r]) * (dc - 128.f * sumc);
      acc = wave_sum(acc);
      const size_t n = nb + r;
      if (lane == 0) {
        const float out = res[n] + acc;
        y[n] = out;
        if (yb) yb[n] = to_bf16(out);
      }
    }
  }
};
// LDS slot of activation float4 f of a row ((TOPK8 + 1) * I / 4 of them): the routed part in
// the lane slices DownFP8 reads (load i = act[1024 i + 16 l .. + 16) -> 4 float4 per part of
// 256), the shared part's 8 floats per lane at 1024 + t * 64 + l
DEV int down_slot(int f) {
  return f < 1024 ? (f & ~255) + (f & 3) * 64 + ((f & 255) >> 2) : 1024 + ((f - 1024) & 1) * 64 + ((f - 1024) >> 1);
}

// down of decode row blockIdx.y: wave w of block b owns output rows n0 .. n0 + RPW - 1
// (DownFP8); the row's activations are requested first and staged in LDS.
template <int SF, class SH, int WPB, int RPW>
__global__ void __launch_bounds__(WPB * 64)
    k_moe_down_fp8(const uint8_t* __restrict__ W, const void* __restrict__ S, const int8_t* __restrict__ shq,
                   const uint16_t* __restrict__ shs, const float* act, const int* __restrict__ idx,
                   const float* __restrict__ wts, const float* __restrict__ sgate, const float* res, float* y,
                   uint16_t* yb, const char* pf, size_t pf_bytes) {
  constexpr int H = H8, I = I8, AW = (TOPK8 + 1) * I / 4, NT = WPB * 64;
  __shared__ float4 as[AW];
  const int lane = lane_id(), wave = wave_id();
  const int half = lane >> 5, b = blockIdx.y;
  const int n0 = (blockIdx.x * WPB + wave) * RPW;
  act += (size_t)b * (TOPK8 + 1) * I, idx += b * TOPK8, wts += b * TOPK8;
  // pick indices with scalar loads, then the activations (requested before the weights, so
  // the staging overlaps the weight fetch), then the weights row by row
  size_t e[4];
  float w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ea = idx[2 * i], eb = idx[2 * i + 1];
    const float wa = wts[2 * i], wb = wts[2 * i + 1];
    e[i] = (size_t)(half ? eb : ea);
    w[i] = half ? wb : wa;
  }
  const float sgv = sigmoid(sgate[b]);
  constexpr int NA = 1024 / NT;
  const float4* a4 = reinterpret_cast<const float4*>(act);
  float4 av[NA + 1];
#pragma unroll
  for (int t = 0; t < NA; ++t) av[t] = ldf4(a4 + threadIdx.x + NT * t);
  av[NA] = ldf4(a4 + 1024 + (threadIdx.x & 127));
  issue_fence();
  DownFP8<SF, SH, RPW> dn;
  dn.issue(W, S, shq, shs, e, n0);
#pragma unroll
  for (int t = 0; t < NA; ++t) as[down_slot(threadIdx.x + NT * t)] = av[t];
  if ((int)threadIdx.x < 128) as[down_slot(1024 + threadIdx.x)] = av[NA];
  __syncthreads();
  dn.finish(as, w, sgv, res, y, yb, (size_t)b * H + n0);
  warm_range(pf, pf_bytes);
}

// Launch shapes: batch 1 (the engine's per-layer chain) uses small blocks, many of them.
// B > 1 uses 512-thread blocks, two per CU: gate_up walks B * 8 * 512 / 4096 units per wave
// with 2 in flight (measured at B = 4: 37.8 us for the three launches, against 39.1 with one
// block of 3 in flight per CU and 43.0 with 4 in flight, whose registers spill).
template <int SF, class SH, int B>
void launch_decode_fp8_b(const uint8_t* gu_w, const void* gu_s, const uint8_t* d_w, const void* d_s,
                         const int8_t* sgu_q, const uint16_t* sgu_s, const int8_t* sd_q, const uint16_t* sd_s,
                         const float* x, const int* idx, const float* wts, const float* sgate, const float* res,
                         float* act, float* y, uint16_t* yb, const float* nw, float eps, const char* pf,
                         size_t pf_bytes, hipStream_t st) {
  constexpr int GW = B == 1 ? 4 : 8, GB = B == 1 ? 1024 : 512, GD = B == 1 ? 1 : 2;
  constexpr int GS = B == 1 ? 1 : 2, DW = B == 1 ? 4 : 8, DR = 2;
  constexpr int NB = GB + I8 / (GW * GS);
  hipLaunchKernelGGL((k_moe_gate_up_fp8<SF, SH, GW, GB, GD, GS, B>), dim3(NB), dim3(GW * 64), 0, st, gu_w, gu_s, sgu_q,
                     sgu_s, x, idx, act, nw, eps);
  hipLaunchKernelGGL((k_moe_down_fp8<SF, SH, DW, DR>), dim3(H8 / (DW * DR), B), dim3(DW * 64), 0, st, d_w, d_s, sd_q,
                     sd_s, act, idx, wts, sgate, res, y, yb, pf, pf_bytes);
}

// rows independent decode rows (x, res, y: [rows, H]; idx, wts: [rows, topk]; act: rows x
// (topk + 1) x I), launched 4 rows at a time
template <int SF, class SH>
int launch_decode_fp8(const uint8_t* gu_w, const void* gu_s, const uint8_t* d_w, const void* d_s, const int8_t* sgu_q,
                      const uint16_t* sgu_s, const int8_t* sd_q, const uint16_t* sd_s, const float* x, const int* idx,
                      const float* wts, const float* sgate, const float* res, float* act, float* y, uint16_t* yb, int H,
                      int I, int topk, const float* nw, float eps, const char* pf, size_t pf_bytes, hipStream_t st,
                      int rows = 1) {
  if (H != H8 || I != I8 || topk != TOPK8 || rows < 1 || rows > 64) return -1;
  for (int r0 = 0; r0 < rows; r0 += 4) {
    const int b = rows - r0 < 4 ? rows - r0 : 4;
    const size_t xo = (size_t)r0 * H, ko = (size_t)r0 * topk, ao = (size_t)r0 * (topk + 1) * I;
    auto go = [&](auto kb) {
      constexpr int KB = decltype(kb)::value;
      launch_decode_fp8_b<SF, SH, KB>(gu_w, gu_s, d_w, d_s, sgu_q, sgu_s, sd_q, sd_s, x + xo, idx + ko, wts + ko,
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

// The small-batch path with the router in the gate_up launch, rows in chunks of four (each
// chunk's logits and picks at its row offset; every launch tags its picks afresh in the same
// tags words), then down.
template <int SF, class SH>
int launch_decode_routed_fp8(const uint16_t* rw, float* logits, int E, int* idx, float* wts, float* sgate,
                             uint32_t* counter, uint64_t* tags, const uint8_t* gu_w, const void* gu_s,
                             const uint8_t* d_w, const void* d_s, const int8_t* sgu_q, const uint16_t* sgu_s,
                             const int8_t* sd_q, const uint16_t* sd_s, const float* x, const float* res, float* act,
                             float* y, uint16_t* yb, int rows, int H, int I, int topk, const float* nw, float eps,
                             hipStream_t st) {
  if (H != H8 || I != I8 || topk != TOPK8 || rows < 1 || rows > 64 || E < TOPK8 || E > 256) return -1;
  if (!rw || !logits || !idx || !wts || !sgate || !counter || !tags) return -1;
  uint32_t* err = err_word();
  for (int r0 = 0; r0 < rows; r0 += 4) {
    const int b = rows - r0 < 4 ? rows - r0 : 4;
    const size_t xo = (size_t)r0 * H, ko = (size_t)r0 * topk, ao = (size_t)r0 * (topk + 1) * I;
    float* lg = logits + (size_t)r0 * (E + 1);
    auto go = [&](auto kb) {
      constexpr int KB = decltype(kb)::value, D = KB < 2 ? KB : 2, DW = KB == 1 ? 4 : 8, DR = 2;
      hipLaunchKernelGGL((k_moe_route_gate_up_fp8<SF, SH, D, KB>), dim3(RG_BLOCKS), dim3(512), 0, st,
                         rw, lg, E, idx + ko, wts + ko, sgate + r0, counter, tags, err, gu_w, gu_s, sgu_q, sgu_s,
                         x + xo, act + ao, nw, eps);
      hipLaunchKernelGGL((k_moe_down_fp8<SF, SH, DW, DR>), dim3(H8 / (DW * DR), KB), dim3(DW * 64), 0, st, d_w, d_s,
                         sd_q, sd_s, act + ao, idx + ko, wts + ko, sgate + r0, res + xo, y + xo,
                         yb ? yb + xo : nullptr, nullptr, (size_t)0);
    };
    if (b == 1) go(std::integral_constant<int, 1>{});
    else if (b == 2) go(std::integral_constant<int, 2>{});
    else if (b == 3) go(std::integral_constant<int, 3>{});
    else go(std::integral_constant<int, 4>{});
  }
  return 0;
}

}  // namespace

API int dr_moe_decode_fp8(const uint8_t* gu_w, const float* gu_s, const uint8_t* d_w, const float* d_s,
                          const int8_t* sgu_q, const uint16_t* sgu_s, const int8_t* sd_q, const uint16_t* sd_s,
                          const float* x, const int* idx, const float* wts, const float* sgate, const float* res,
                          float* act, float* y, int H, int I, int topk, const float* nw, float eps, const char* pf,
                          size_t pf_bytes, hipStream_t st) {
  return launch_decode_fp8<0, Q8G128F16>(gu_w, gu_s, d_w, d_s, sgu_q, sgu_s, sd_q, sd_s, x, idx, wts, sgate, res, act,
                                         y, nullptr, H, I, topk, nw, eps, pf, pf_bytes, st);
}

API int dr_moe_decode_fp8_bf16s(const uint8_t* gu_w, const uint16_t* gu_s, const uint8_t* d_w, const uint16_t* d_s,
                                const int8_t* sgu_q, const uint16_t* sgu_s, const int8_t* sd_q, const uint16_t* sd_s,
                                const float* x, const int* idx, const float* wts, const float* sgate, const float* res,
                                float* act, float* y, uint16_t* yb, int H, int I, int topk, const float* nw, float eps,
                                const char* pf, size_t pf_bytes, hipStream_t st) {
  return launch_decode_fp8<1, Q8RowBF16>(gu_w, gu_s, d_w, d_s, sgu_q, sgu_s, sd_q, sd_s, x, idx, wts, sgate, res, act,
                                         y, yb, H, I, topk, nw, eps, pf, pf_bytes, st);
}

API int dr_moe_decode_rows_fp8(const uint8_t* gu_w, const float* gu_s, const uint8_t* d_w, const float* d_s,
                               const int8_t* sgu_q, const uint16_t* sgu_s, const int8_t* sd_q, const uint16_t* sd_s,
                               const float* x, const int* idx, const float* wts, const float* sgate, const float* res,
                               float* act, float* y, int rows, int H, int I, int topk, const float* nw, float eps,
                               hipStream_t st) {
  return launch_decode_fp8<0, Q8G128F16>(gu_w, gu_s, d_w, d_s, sgu_q, sgu_s, sd_q, sd_s, x, idx, wts, sgate, res, act,
                                         y, nullptr, H, I, topk, nw, eps, nullptr, 0, st, rows);
}

API int dr_moe_decode_rows_fp8_bf16s(const uint8_t* gu_w, const uint16_t* gu_s, const uint8_t* d_w,
                                     const uint16_t* d_s, const int8_t* sgu_q, const uint16_t* sgu_s,
                                     const int8_t* sd_q, const uint16_t* sd_s, const float* x, const int* idx,
                                     const float* wts, const float* sgate, const float* res, float* act, float* y,
                                     uint16_t* yb, int rows, int H, int I, int topk, const float* nw, float eps,
                                     hipStream_t st) {
  return launch_decode_fp8<1, Q8RowBF16>(gu_w, gu_s, d_w, d_s, sgu_q, sgu_s, sd_q, sd_s, x, idx, wts, sgate, res, act,
                                         y, yb, H, I, topk, nw, eps, nullptr, 0, st, rows);
}

API int dr_moe_decode_rows_routed_fp8(const uint16_t* router_w, const float* nw, float eps, int E,
                                      const uint8_t* gu_w, const float* gu_s, const uint8_t* d_w, const float* d_s,
                                      const int8_t* sgu_q, const uint16_t* sgu_s, const int8_t* sd_q,
                                      const uint16_t* sd_s, const float* x, float* logits, int* idx, float* wts,
                                      float* sgate, uint32_t* counter, uint64_t* tags, const float* res, float* act,
                                      float* y, int rows, int H, int I, int topk, hipStream_t st) {
  return launch_decode_routed_fp8<0, Q8G128F16>(router_w, logits, E, idx, wts, sgate, counter, tags, gu_w, gu_s, d_w,
                                                d_s, sgu_q, sgu_s, sd_q, sd_s, x, res, act, y, nullptr, rows, H, I,
                                                topk, nw, eps, st);
}

API int dr_moe_decode_rows_routed_fp8_bf16s(const uint16_t* router_w, const float* nw, float eps, int E,
                                            const uint8_t* gu_w, const uint16_t* gu_s, const uint8_t* d_w,
                                            const uint16_t* d_s, const int8_t* sgu_q, const uint16_t* sgu_s,
                                            const int8_t* sd_q, const uint16_t* sd_s, const float* x, float* logits,
                                            int* idx, float* wts, float* sgate, uint32_t* counter, uint64_t* tags,
                                            const float* res, float* act, float* y, uint16_t* yb, int rows, int H,
                                            int I, int topk, hipStream_t st) {
  return launch_decode_routed_fp8<1, Q8RowBF16>(router_w, logits, E, idx, wts, sgate, counter, tags, gu_w, gu_s, d_w,
                                                d_s, sgu_q, sgu_s, sd_q, sd_s, x, res, act, y, yb, rows, H, I, topk,
                                                nw, eps, st);
}


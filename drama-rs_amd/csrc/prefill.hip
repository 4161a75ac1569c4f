// Prefill expert-grouped GEMM on the CDNA4 matrix cores (reference: kernels/drama.cu:799-1109,
// src/ffi.rs:52-54,60-63) and the fused int8 shared-expert prefill (src/engine.rs:560-562).
//
// Rows of xp are sorted by expert; expert e owns rows [offsets[e], offsets[e] + counts[e]).
// gate_up: act[t] = bf16(silu(G_e . x_t) * (U_e . x_t)); down: y[t] = D_e . act_t (fp32).
//
// k_grouped (the routed experts): a wave owns a 16-row tile of weight rows and computes it
// against a 16-token pass of its expert with v_mfma_f32_16x16x32_bf16: A = tokens (16 x 32),
// B = weights (32 x 16), D = 16 x 16 fp32, so the four D values of a lane share one weight row.
// Weights are dequantised exactly in registers: an int4 nibble q becomes the bf16 value
// 128 + q (bit pattern 0x4300 | q), an int8 or fp8 value converts to bf16 exactly.  Each MFMA
// stays inside one scale group, so per group g the fp32 product sum acc_g is rescaled:
//   int4:  out += s_g acc_g + (m_g - 128 s_g) X_g,  X_g = sum of the group's inputs
//   int8 / fp8:  out += s_g acc_g  (one scale per 128 inputs, or one per row at the end)
// which is w = q s + m applied after exact integer x bf16 products: the same values as
// dequantise-then-fp32, accumulated in fp32.
//
// Fragment order: an MFMA lane holds 8 inputs in the order 0 4 1 5 2 6 3 7 of an 8-input
// chunk, the order in which the nibble masking (w >> 4 j) & 0x000f000f (and the int8 / fp8
// byte pairing) produces bf16 pairs; token tiles in LDS are stored in the same permuted
// order, 16-byte chunk b of token t at b ^ (t % 16), so the 16 token rows of one read spread
// over all banks and each A fragment is one 16-byte LDS read.  The per-kernel comments give
// the lane -> input mapping of each weight format.
#include <mutex>

#include "common.hpp"

using namespace drm;

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int PF_WPB = 8;     // waves per block (k_grouped_ks)
constexpr int PF_GWPB = 8;    // waves per block (k_grouped)
// 16-row tiles per wave and item (k_grouped).  Measured: 2 (one token tile serving both) is
// level with 1 at 300 prefill rows and 20% slower at 4 decode rows (fewer, larger items)
constexpr int PF_GRPW = 1;
constexpr int PF_TOK = 16;    // tokens per pass (one MFMA tile)
constexpr int PF_MAXE = 256;  // experts
constexpr int PF_DEPTH = 4;   // 4-group weight steps in flight per wave (k_grouped)

DEV f32x4 mfma(const uint4& a, const uint4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
                                                 0);
}

// ---- weight formats: per lane and 64-wide group, two MFMA A fragments -------------------------

// int4, (scale, min) pairs per 64 inputs; SC = ScaleF16 | ScaleBF16
template <class SC>
struct FmtQ4 {
  static constexpr bool q8 = false;
  static constexpr bool has_min = true;
  static constexpr bool paired = true;  // k_grouped: 16-byte loads covering two groups per row
  static constexpr bool packable = true;  // has a tile-step layout (dr_moe_pack_q4)
  static constexpr int scale_group = 64;  // inputs per scale
  static DEV size_t row_bytes(int K) { return (size_t)K / 2; }
  // fragment bytes of (row, group G) for lane group g: 8 bytes = 16 nibbles
  static DEV void load(const uint8_t* row, int G, int g, uint2& raw) { raw = ld8(row + G * 32 + g * 8); }
  static DEV void convert(const uint2& raw, uint4& a0, uint4& a1) {
    const uint32_t m = 0x000f000fu, b = 0x43004300u;
    a0 = make_uint4((raw.x & m) | b, ((raw.x >> 4) & m) | b, ((raw.x >> 8) & m) | b, ((raw.x >> 12) & m) | b);
    a1 = make_uint4((raw.y & m) | b, ((raw.y >> 4) & m) | b, ((raw.y >> 8) & m) | b, ((raw.y >> 12) & m) | b);
  }
  // (scale, min) of row n, group G: raw word, then decoded
  static DEV uint32_t scale_raw(const void* S, size_t n, int G, int K) {
    return reinterpret_cast<const uint32_t*>(S)[n * (K / 64) + G];
  }
  static DEV float2 scale_val(uint32_t w) { return SC::pair(w); }
  static DEV float2 scale(const void* S, size_t n, int G, int K) { return scale_val(scale_raw(S, n, G, K)); }
};

// element order inside an 8-element fragment: perm = 0 4 1 5 2 6 3 7
// int8: 16 bytes per lane and group; bytes k..k+15 of the group slice, reordered
template <class SH>
struct FmtQ8 {
  using Scale = SH;
  static constexpr bool q8 = true;
  static constexpr bool has_min = false;
  static constexpr bool paired = false;
  static constexpr bool packable = false;
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
  static DEV uint32_t scale_raw(const void* S, size_t n, int G, int K) {
    return __float_as_uint(SH::scale(reinterpret_cast<const uint16_t*>(S), n, G * 64, K));
  }
  static DEV float2 scale_val(uint32_t w) { return make_float2(__uint_as_float(w), 0.f); }
  static DEV float2 scale(const void* S, size_t n, int G, int K) { return scale_val(scale_raw(S, n, G, K)); }
};

// fp8 e4m3 (OCP), one scale per 128 x 128 block; SF: 0 = f32 scales, 1 = bf16 scales
template <int SF>
struct FmtFP8 {
  static constexpr bool q8 = false;
  static constexpr bool has_min = false;
  static constexpr bool paired = false;
  static constexpr bool packable = true;  // has a tile-step layout (dr_moe_pack_fp8)
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
  static DEV uint32_t scale_raw(const void* S, size_t n, int G, int K) {
    const size_t i = (n >> 7) * (size_t)(K / 128) + (G >> 1);
    return SF ? (uint32_t)reinterpret_cast<const uint16_t*>(S)[i] << 16 : reinterpret_cast<const uint32_t*>(S)[i];
  }
  static DEV float2 scale_val(uint32_t w) { return make_float2(__uint_as_float(w), 0.f); }
  static DEV float2 scale(const void* S, size_t n, int G, int K) { return scale_val(scale_raw(S, n, G, K)); }
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

// Spin until an LDS counter reaches target (acquire); bounded, so a broken protocol ends the
// wait instead of hanging the GPU, and then raises DR_ERR_PREFILL_WAIT in the library error
// word (the results of the launch are wrong; dr_stream_sync and dr_last_error report it).
DEV void lds_wait_ge(const uint32_t* c, uint32_t target, uint32_t* err) {
  for (int it = 0; it < (1 << 22); ++it) {
    if (__hip_atomic_load(c, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= target) return;
    __builtin_amdgcn_s_sleep(1);
  }
  if (lane_id() == 0) raise_err(err, kErrPrefillWait);
}
DEV void lds_count(uint32_t* c) {
  if (lane_id() == 0) __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Token tile of tokens [row0, row0 + ntok) x all K inputs of a bf16 row matrix, staged into LDS
// in the permuted fragment order: 16-byte block r of token t at t * K / 8 + (r ^ t), the xor
// spreading the 16 tokens of one read over distinct LDS banks; rows beyond ntok are zero.
// Split in two so the caller can issue its first weight loads between the token loads and
// the LDS stores: the stores wait only for the token loads issued before those weight loads.
template <int K, int NT>
struct TokTile {
  static constexpr int NB = PF_TOK * K / 8 / NT;  // 16-byte blocks per thread (NT threads)
  static_assert(NB >= 1 && NB * NT == PF_TOK * K / 8, "token tile split");
  uint4 v[NB];
  // rows [row0, row0 + ntok) through a buffer resource bounded at the last row: the lanes of
  // rows past ntok read zeros without a memory access (and the code stays branch-free, which
  // keeps the load counter exact)
  DEV void load(const uint16_t* __restrict__ X, size_t row0, int ntok) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(X + row0 * (size_t)K), 0, ntok * K * 2, 0x00020000);
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int b = threadIdx.x + i * NT, t = b / (K / 8), r = b % (K / 8);
      v[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, (t * K + r * 8) * 2, 0, 0));
    }
  }
  // The same tile with its rows gathered through a slot -> row map: token t of the pass is row
  // rmap[row0 + t] of X (x_rows rows).  The 16 indices come with scalar loads (their wait does
  // not queue behind the weight loads in flight), rows past ntok read zeros.  K / 8 = NT / 2:
  // thread b's blocks belong to tokens 2 i and 2 i + 1.
  DEV void load_rows(const uint16_t* __restrict__ X, int x_rows, const int* __restrict__ rmap, size_t row0,
                     int ntok) {
    static_assert(NT == 2 * (K / 8), "two tokens per block index");
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(X), 0, x_rows * K * 2, 0x00020000);
    const __attribute__((address_space(4))) int* rp =
        (const __attribute__((address_space(4))) int*)(rmap + row0);
    int rr[PF_TOK];
#pragma unroll
    for (int t = 0; t < PF_TOK; ++t) rr[t] = rp[t];
    const bool hi = threadIdx.x >= NT / 2;
    const int r = threadIdx.x % (K / 8);
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int t = 2 * i + (hi ? 1 : 0);
      const int row = hi ? rr[2 * i + 1] : rr[2 * i];
      const uint32_t off = t < ntok ? (uint32_t)((row * K + r * 8) * 2) : 0x7ffffff0u;
      v[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
    }
  }
  // with_sums: also the fp32 sum of every 64-input group of every token, at float index
  // PF_TOK K / 2 + 16 G + t (after the tile), for the min term of the int4 format
  DEV void store(uint4* xs, bool with_sums) const {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int b = threadIdx.x + i * NT, t = b / (K / 8);
      if (with_sums) {
        // 8 chunks of a group sit in 8 consecutive lanes (K / 8 and the stride are multiples of 8)
        float sum = 0.f;
        const uint32_t wv[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) sum += __uint_as_float(wv[k] << 16) + __uint_as_float(wv[k] & 0xffff0000u);
        sum = xsum_step<4>(xsum_step<2>(xsum_step<1>(sum)));
        const int r = b % (K / 8);
        if ((r & 7) == 0) reinterpret_cast<float*>(xs + PF_TOK * K / 8)[16 * (r >> 3) + t] = sum;
      }
      // (e0 e1)(e2 e3)(e4 e5)(e6 e7) -> (e0 e4)(e1 e5)(e2 e6)(e3 e7)
      xs[b ^ (t & 15)] =
          make_uint4(__builtin_amdgcn_perm(v[i].z, v[i].x, 0x05040100u), __builtin_amdgcn_perm(v[i].z, v[i].x, 0x07060302u),
                     __builtin_amdgcn_perm(v[i].w, v[i].y, 0x05040100u), __builtin_amdgcn_perm(v[i].w, v[i].y, 0x07060302u));
    }
  }
};

// per-lane weight data of 4 consecutive 64-input groups: raw fragments and (scale, min) pairs.
// Unpaired formats: raw[i] = this lane's fragment bytes of group G0 + i.  Paired (int4): the
// four lanes of a row read the 64 bytes of groups (G0 + 2 p, G0 + 2 p + 1) as 16 bytes each,
// raw[p] = bytes 16 g of that span: lanes g = 0, 1 hold the first group, g = 2, 3 the second
// (one 64-byte run per row per load: half the cache-line requests of 8-byte loads); all four
// (scale, min) words of the step come in one 16-byte load.
template <class F, bool P = F::paired>
struct Step {
  typename Raw<F>::T raw[4];
  uint32_t sc[4];
};
template <class F>
struct Step<F, true> {
  uint4 raw[2];
  uint4 sc;
};

template <class F>
DEV void load_step(const uint8_t* row, const void* ws, size_t n, int G0, int g, int K, Step<F>& s) {
  if constexpr (F::paired) {
    s.raw[0] = ld16(row + G0 * 32 + g * 16);
    s.raw[1] = ld16(row + G0 * 32 + 64 + g * 16);
    s.sc = ld16(reinterpret_cast<const uint32_t*>(ws) + n * (size_t)(K / 64) + G0);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) F::load(row, G0 + i, g, s.raw[i]);
    if (F::scale_group != 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) s.sc[i] = F::scale_raw(ws, n, G0 + i, K);
    }
  }
}

// nibbles of one 32-bit word -> bf16 fragment 128 + q in the order 0 4 1 5 2 6 3 7 with
// m = 0x000f000f, b = 0x43004300; m = b = 0 gives the zero fragment (a lane left out)
DEV uint4 q4_frag(uint32_t w, uint32_t m, uint32_t b) {
  return make_uint4((w & m) | b, ((w >> 4) & m) | b, ((w >> 8) & m) | b, ((w >> 12) & m) | b);
}

// MODE 0: gate_up (row pairs j, I + j; writes bf16 silu(g) u)   MODE 1: down (writes f32)
//
// Work items: (expert e, 16-token pass p < ceil(counts[e] / 16), row block yb).  A persistent
// grid of resident blocks walks them (item = blockIdx.x, + gridDim.x, ...).  Each wave owns one
// 16-row tile of an item: down, rows (yb PF_GWPB + w) 16; gate_up, waves 0 .. W/2 - 1 gate
// rows (W/2 yb + w) 16 and the other half the matching up rows (W waves per block), the up results handed to the gate waves
// through LDS at the item boundary.  A wave streams its tile as a sequence of 4-group steps
// against the item's token tile in LDS; the ring of DEPTH steps in flight runs on across
// items (the next item's first steps are fetched during the current item's last ones, its
// tokens just before them), and the tokens are stored into the second of two LDS tile buffers
// at the boundary, so one barrier per item is the only gap.  MFMA operands: A = tokens (lane: token l % 16),
// B = weights (lane: row l % 16), so D[token 4 (l / 16) + i][row l % 16] sits in lane l: one
// weight row per lane, one (scale, min) pair per group.  The group input sums X_g come from an
// MFMA against bf16 ones (int4: staged with the tokens).
// PK (int4 only): the weights are in the tile-step layout of dr_moe_pack_q4, so each step of a
// wave is one contiguous 2048-byte block (two 1024-byte wave loads) and 256 bytes of scales,
// where the reference layout gives 16 rows x 128 bytes 1 KB apart.
template <class F, int MODE, int K, bool GATHER, bool PK = false>
__global__ void __launch_bounds__(PF_GWPB * 64)
    k_grouped(const uint8_t* __restrict__ Wq, const void* __restrict__ Ws, const uint16_t* __restrict__ X,
              const int* __restrict__ offsets, const int* __restrict__ counts, void* __restrict__ out, int N,
              size_t expert_q_bytes, size_t expert_s_elems, int s_elem_bytes, int E, uint32_t* __restrict__ err,
              const int* __restrict__ rmap, int x_rows) {
  extern __shared__ uint4 xs[];  // two tile buffers of BUF blocks, the item table, the up hand-over
  constexpr int BUF = PF_TOK * K / 8 + (F::paired ? (K / 64) * PF_TOK / 4 : 0);
  constexpr int WR = MODE == 0 ? PF_GWPB / 2 : PF_GWPB;  // row tiles per item (per row set)
  const int lane = lane_id(), wave = wave_id();
  const int g = lane >> 4, c16 = lane & 15;
  const int YB = (MODE == 0 ? N / 2 : N) / (16 * WR * PF_GRPW);  // row blocks per expert
  // per lane: pass counts of experts 4 lane + j and their inclusive prefix over all experts;
  // (end of passes, count, offset) of each kept in LDS; every wave writes the same values and
  // each lane reads back only its own entries, so no barrier is needed
  uint4* tbl = xs + 2 * BUF;
  f32x4* ups = reinterpret_cast<f32x4*>(tbl + 192);  // [2][PF_GRPW][WR][64] up results (gate_up)
  int n_pass;
  {
    int cl[4], ol[4], pl[4], psum = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = 4 * lane + j;
      cl[j] = e < E ? counts[e] : 0;
      ol[j] = e < E ? offsets[e] : 0;
      pl[j] = (cl[j] + PF_TOK - 1) / PF_TOK;
      psum += pl[j];
    }
    int incl = psum;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int t = __shfl_up(incl, o);
      if (lane >= o) incl += t;
    }
    n_pass = __builtin_amdgcn_readfirstlane(__shfl(incl, 63));  // wave-uniform, in a scalar register
    int end = incl - psum, ends[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) end += pl[j], ends[j] = end;
    tbl[lane] = make_uint4(ends[0], ends[1], ends[2], ends[3]);
    tbl[64 + lane] = make_uint4(cl[0], cl[1], cl[2], cl[3]);
    tbl[128 + lane] = make_uint4(ol[0], ol[1], ol[2], ol[3]);
  }
  const int n_items = n_pass * YB;
  struct Item {
    const uint8_t* wq;
    const char* ws;
    size_t row0;  // first token row of the pass
    int ntok, yb;
    bool valid;
  };
  if (n_pass == 0) return;
  // Item i -> (flat pass q, row block yb).  Blocks run on XCD blockIdx % 8, each XCD with its
  // own L2: where the grid allows, the YB row blocks of a pass go to blocks of one XCD in the
  // same round of gridDim.x items, so its token tile is fetched into that L2 once (round r,
  // block b = x + 8 j: q = (8 r + x) EPR + j / YB, yb = j % YB with EPR passes per XCD and
  // round).  Otherwise q = i % n_pass, yb = i / n_pass.  Indices past the last pass are
  // invalid; they map to pass 0, row block 0 (loaded, never computed).
  const int G = gridDim.x, EPR = (G / 8) / YB;
  const bool xcd_map = G % 8 == 0 && EPR > 0 && (G / 8) % YB == 0;
  auto item_at = [&](int i) {
    Item it;
    int q, yb;
    if (xcd_map) {
      const int rnd = i / G, b = i - rnd * G, j = b >> 3;
      q = (rnd * 8 + (b & 7)) * EPR + j / YB;
      yb = j % YB;
      it.valid = q < n_pass;
    } else {
      it.valid = i < n_items;
      q = i % n_pass;
      yb = i / n_pass;
    }
    if (!it.valid) q = 0, yb = 0;
    it.yb = yb;
    const uint4 en = tbl[lane], cn = tbl[64 + lane], of = tbl[128 + lane];
    const int ev[4] = {(int)en.x, (int)en.y, (int)en.z, (int)en.w}, cv[4] = {(int)cn.x, (int)cn.y, (int)cn.z, (int)cn.w};
    const int ov[4] = {(int)of.x, (int)of.y, (int)of.z, (int)of.w};
    int me = 0, mp = 0, mc = 0, mo = 0;
    bool found = false;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int p = (cv[j] + PF_TOK - 1) / PF_TOK;
      const bool in = q < ev[j] && q >= ev[j] - p;
      me = in ? 4 * lane + j : me;
      mp = in ? q - (ev[j] - p) : mp;
      mc = in ? cv[j] : mc;
      mo = in ? ov[j] : mo;
      found = found || in;
    }
    const uint64_t bal = __ballot(found);
    const int src = bal ? __builtin_ctzll(bal) : 0;
    const int e = __builtin_amdgcn_readlane(me, src), pass = __builtin_amdgcn_readlane(mp, src);
    const int cnt = __builtin_amdgcn_readlane(mc, src), o0 = __builtin_amdgcn_readlane(mo, src);
    it.wq = Wq + (size_t)e * expert_q_bytes;
    it.ws = reinterpret_cast<const char*>(Ws) + (size_t)e * expert_s_elems * s_elem_bytes;
    it.row0 = (size_t)o0 + (size_t)pass * PF_TOK;
    it.ntok = min(PF_TOK, cnt - pass * PF_TOK);
    return it;
  };
  const size_t rb = F::row_bytes(K);
  constexpr int SPT = K / 256;         // 4-group steps per tile
  constexpr int NS = PF_GRPW * SPT;    // per item
  constexpr int DEPTH = PF_DEPTH < NS ? PF_DEPTH : NS;
  static_assert(NS % DEPTH == 0, "the ring of steps must divide an item");
  const bool up = MODE == 0 && wave >= WR;  // gate_up: this wave computes up rows
  const int wt = wave % WR;
  // weight row of this lane in item it (gate_up: the up row of an up wave)
  auto row_of = [&](const Item& it, int t) {
    return (size_t)(up ? N / 2 : 0) + (size_t)(((it.yb * PF_GRPW + t) * WR + wt) * 16 + c16);
  };
  auto fetch = [&](const Item& it, int s, Step<F>& st) {
    const size_t n = row_of(it, s / SPT);
    if constexpr (PK && F::paired) {
      // int4 block (tile n / 16, step): lane l's 16 bytes of each half are what load_step reads
      const size_t blk = (n >> 4) * SPT + (size_t)(s % SPT);
      const uint8_t* tb = it.wq + blk * 2048;
      st.raw[0] = ld16(tb + lane * 16);
      st.raw[1] = ld16(tb + 1024 + lane * 16);
      st.sc = ld16(reinterpret_cast<const uint8_t*>(it.ws) + blk * 256 + c16 * 16);
    } else if constexpr (PK) {
      // fp8 block (tile n / 16, step): 1024 bytes per group, lane l's 16 bytes of group i at
      // i 1024 + 16 l (the block scales keep their layout)
      static_assert(F::packable, "no tile-step layout for this format");
      const size_t blk = (n >> 4) * SPT + (size_t)(s % SPT);
      const uint8_t* tb = it.wq + blk * 4096;
      const int G0 = (s % SPT) * 4;
#pragma unroll
      for (int i = 0; i < 4; ++i) st.raw[i] = ld16(tb + i * 1024 + lane * 16);
#pragma unroll
      for (int i = 0; i < 4; ++i) st.sc[i] = F::scale_raw(it.ws, n, G0 + i, K);
    } else {
      load_step<F>(it.wq + n * rb, it.ws, n, (s % SPT) * 4, g, K, st);
    }
  };
  const uint4 ones = make_uint4(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);
  // the int4 conversion constants live in VGPRs: v_and_or_b32 (VOP3) takes no literal
  // operands on this architecture and at most one scalar one, so with literals the
  // conversion would cost two instructions per dword instead of one
  uint32_t q_mask = 0x000f000fu, q_bias = 0x43004300u;
  asm volatile("" : "+v"(q_mask), "+v"(q_bias));

  Item cur = item_at(blockIdx.x);
  if (!cur.valid) return;
  Item nxt = item_at(blockIdx.x + gridDim.x);
  Step<F> ring[DEPTH];  // steps in flight
  TokTile<K, PF_GWPB * 64> tt;
  // Waves synchronise per item through LDS counters instead of a block barrier, so they may
  // drift by up to half an item: n_stored = 8 (k + 1) once every wave stored its part of item
  // k's tile; n_done = 8 (k + 1) once every wave finished computing item k; (gate_up) n_up /
  // n_gate count the up results handed over and read, 4 per item.
  __shared__ uint32_t n_stored, n_done, n_up, n_gate;
  if (threadIdx.x == 0) n_stored = 0, n_done = 0, n_up = 0, n_gate = 0;
  {
    if constexpr (GATHER) tt.load_rows(X, x_rows, rmap, cur.row0, cur.ntok);
    else tt.load(X, cur.row0, cur.ntok);
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) fetch(cur, d, ring[d]);
    __builtin_amdgcn_sched_barrier(0);
    tt.store(xs, F::paired);
  }
  lds_barrier();
  __builtin_amdgcn_sched_barrier(0);
  // gate_up: the gate waves finish item k - 1 after the boundary barrier, with the up results
  // the up waves left in ups[(k - 1) & 1]
  struct Pending {
    f32x4 t[PF_GRPW];
    size_t row0;
    int ntok, col[PF_GRPW];
    bool valid;
  } pend;
  pend.valid = false;
  auto finish_gate = [&](const Pending& pd, int k1) {
    lds_wait_ge(&n_up, (uint32_t)(WR * (k1 + 1)), err);
#pragma unroll
    for (int t = 0; t < PF_GRPW; ++t) {
      const f32x4 u = ups[(((k1 & 1) * PF_GRPW + t) * WR + wt) * 64 + lane];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tok = 4 * g + r;
        if (tok >= pd.ntok) break;
        reinterpret_cast<uint16_t*>(out)[(pd.row0 + tok) * (size_t)(N / 2) + pd.col[t]] =
            to_bf16(silu(pd.t[t][r]) * u[r]);
      }
    }
    lds_count(&n_gate);
  };
  int k = 0;
  for (;; ++k) {
    if (MODE == 0 && !up && pend.valid) finish_gate(pend, k - 1);  // (at mid-item: measured slower)
    const uint4* xb = xs + (k & 1) * BUF;
    const uint4* xrow = xb + (size_t)c16 * (K / 8);
    // int4 pairs: first 8-input token block of this lane's swapped words (see compute)
    const int tb = 4 * (g & 1) + 2 * (g >> 1);
    // token block (16 P + j) ^ c16 = 16 P + (j ^ c16) for j < 16: per-lane bases for the j this
    // lane reads, so 16 P becomes the LDS instruction's immediate offset (no address arithmetic
    // per read)
    const uint4* xj0 = xrow + ((tb) ^ c16);
    const uint4* xj1 = xrow + ((tb + 1) ^ c16);
    const uint4* xj8 = xrow + ((tb + 8) ^ c16);
    const uint4* xj9 = xrow + ((tb + 9) ^ c16);
    const uint4* xu0 = xrow + ((2 * g) ^ c16);
    const uint4* xu1 = xrow + ((2 * g + 1) ^ c16);
    const uint4* xu8 = xrow + ((8 + 2 * g) ^ c16);
    const uint4* xu9 = xrow + ((9 + 2 * g) ^ c16);
    f32x4 tA = {0.f, 0.f, 0.f, 0.f};
    auto compute = [&](const Step<F>& sa, int G0) {
      if constexpr (F::paired) {
        // min term of the step's four groups as one fp32 MFMA: A = group sums X[token c16][G0 + g],
        // B = (m - 128 s)[row c16][G0 + g] (this lane's scale word g)
        {
          const float xg = reinterpret_cast<const float*>(xb + PF_TOK * K / 8)[(G0 + g) * 16 + c16];
          // (selecting among decoded floats: a select among the step's words becomes an indexed
          // access that sends the whole ring to scratch memory)
          const float2 p0 = F::scale_val(sa.sc.x), p1 = F::scale_val(sa.sc.y);
          const float2 p2 = F::scale_val(sa.sc.z), p3 = F::scale_val(sa.sc.w);
          const float c0 = p0.y - 128.f * p0.x, c1 = p1.y - 128.f * p1.x;
          const float c2 = p2.y - 128.f * p2.x, c3 = p3.y - 128.f * p3.x;
          const float cg = g & 2 ? (g & 1 ? c3 : c2) : (g & 1 ? c1 : c0);
          // accumulated straight into tA, step by step: the min terms cancel most of the 128 q
          // offset of the products, and summing them apart would lose that cancellation's bits
          tA = __builtin_amdgcn_mfma_f32_16x16x4f32(xg, cg, tA, 0, 0, 0);
        }
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
          const int P = G0 / 2 + pp;
          // Lane (c16, g) holds nibbles [32 g, 32 g + 32) of the pair's 128 (g < 2: group A,
          // g >= 2: group B), word j its inputs + 8 j.  Swapping words 2, 3 of lanes 0..31 with
          // words 0, 1 of lanes 32..63 (same weight row c16) leaves every lane with two words of
          // each group: fa0 / fa1 hold group A inputs 8 tb .. 8 tb + 15 and fb0 / fb1 the same of
          // group B (tb = 4 (g & 1) + 2 (g >> 1), in 8-input blocks), so each group takes two
          // full MFMAs against token blocks tb, tb + 1 (A) and tb + 8, tb + 9 (B).
          const auto s02 = __builtin_amdgcn_permlane32_swap(sa.raw[pp].x, sa.raw[pp].z, false, false);
          const auto s13 = __builtin_amdgcn_permlane32_swap(sa.raw[pp].y, sa.raw[pp].w, false, false);
          const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
          const f32x4 ua = mfma(xj1[16 * P], q4_frag(s13[0], q_mask, q_bias),
                                mfma(xj0[16 * P], q4_frag(s02[0], q_mask, q_bias), z4));
          const f32x4 ub = mfma(xj9[16 * P], q4_frag(s13[1], q_mask, q_bias),
                                mfma(xj8[16 * P], q4_frag(s02[1], q_mask, q_bias), z4));
          const uint32_t sw[4] = {sa.sc.x, sa.sc.y, sa.sc.z, sa.sc.w};
          const float sca = F::scale_val(sw[2 * pp]).x, scb = F::scale_val(sw[2 * pp + 1]).x;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            tA[r] = __builtin_fmaf(sca, ua[r], tA[r]);
            tA[r] = __builtin_fmaf(scb, ub[r], tA[r]);
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int G = G0 + i;
          // (G * 8 + 2 g + j) ^ c16 = 16 (G >> 1) + ((8 (G & 1) + 2 g + j) ^ c16)
          const uint4 x0 = (G & 1 ? xu8 : xu0)[16 * (G >> 1)], x1 = (G & 1 ? xu9 : xu1)[16 * (G >> 1)];
          const f32x4 z = {0.f, 0.f, 0.f, 0.f};
          uint4 a0, a1;
          F::convert(sa.raw[i], a0, a1);
          if (F::scale_group == 0) {
            tA = mfma(x1, a1, mfma(x0, a0, tA));
          } else {
            const f32x4 accA = mfma(x1, a1, mfma(x0, a0, z));
            f32x4 xg = z;
            if (F::has_min) xg = mfma(x1, ones, mfma(x0, ones, z));
            const float2 pa = F::scale_val(sa.sc[i]);
            const float ca = pa.y - 128.f * pa.x;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              tA[r] = __builtin_fmaf(pa.x, accA[r], tA[r]);
              if (F::has_min) tA[r] = __builtin_fmaf(ca, xg[r], tA[r]);
            }
          }
        }
      }
      // the sums are materialised here, each step: otherwise the compiler sinks the scale
      // loads and rescaling into the (conditional) stores at the end of the item, which
      // costs one more memory round trip and keeps every group's raw sums live
      asm volatile("" : "+v"(tA));
    };
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int b = i % DEPTH;
      compute(ring[b], (i % SPT) * 4);
      // the next item's tokens go out after step 0 (ahead of that step's weight fetch) and are
      // stored into the other tile buffer at mid-item, once every wave finished item k - 1
      // (the buffer's previous tile); after the block's last item nxt is the first item again
      // (loads and stores no one uses): branch-free, so the load counter stays exact
      if (i == 0) {
        if constexpr (GATHER) tt.load_rows(X, x_rows, rmap, nxt.row0, nxt.ntok);
        else tt.load(X, nxt.row0, nxt.ntok);
      }
      if (i + DEPTH < NS) {
        fetch(cur, i + DEPTH, ring[b]);
      } else {
        fetch(nxt, i + DEPTH - NS, ring[b]);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (i == (NS == 2 ? 1 : NS / 2 - 1)) {  // measured: step 3 of 8 (1, 2 and 5 slower)
        lds_wait_ge(&n_done, (uint32_t)(PF_GWPB * k), err);
        tt.store(xs + ((k + 1) & 1) * BUF, F::paired);
        lds_count(&n_stored);
        __builtin_amdgcn_sched_barrier(0);
      }
      if ((i + 1) % SPT != 0) continue;
      // end of tile t: per-row scale, then down stores y; gate_up up waves leave u in LDS,
      // gate waves keep g until the boundary
      const int t = i / SPT;
      const size_t n = row_of(cur, t);
      const float rs = F::scale_group == 0 ? F::scale(cur.ws, n, 0, K).x : 1.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) tA[r] *= rs;
      if (MODE == 1) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int tok = 4 * g + r;
          if (tok >= cur.ntok) break;
          reinterpret_cast<float*>(out)[(cur.row0 + tok) * (size_t)N + n] = tA[r];
        }
      } else if (up) {
        // ups[k & 1] held item k - 2, which every gate wave has read
        lds_wait_ge(&n_gate, (uint32_t)(WR * (k > 0 ? k - 1 : 0)), err);
        ups[(((k & 1) * PF_GRPW + t) * WR + wt) * 64 + lane] = tA;
        lds_count(&n_up);
      } else {
        pend.t[t] = tA, pend.col[t] = (int)n;
        pend.row0 = cur.row0, pend.ntok = cur.ntok, pend.valid = true;
      }
      tA = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    lds_count(&n_done);  // this wave is done with tile k (its LDS reads have returned)
    if (!nxt.valid) break;
    cur = nxt;
    nxt = item_at(blockIdx.x + (k + 2) * gridDim.x);
    // the next tile is complete once every wave stored its part
    lds_wait_ge(&n_stored, (uint32_t)(PF_GWPB * (k + 1)), err);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (MODE == 0 && !up && pend.valid) finish_gate(pend, k);  // the last item
  // no wave may leave while others still count on its LDS (the counters live in it)
  lds_barrier();
}


// K-split variant, used for the shared expert (one weight set over all rows; for the grouped
// experts it measured slower than k_grouped).  Block = one 16-row tile of weight rows (gate_up:
// 16 gate + 16 up rows) of one expert; wave w owns the input groups [GPW w, GPW (w + 1)) of
// every row, so each wave issues all loads of the tile at once.  The weights stay in registers
// for every 16-token tile of the expert (tiles blockIdx.z, + gridDim.z, ...); a wave reads its
// slice of the 16 tokens straight from global memory (no LDS staging; the next tile's slice is
// loaded while the current one is used), runs the exact-dequant MFMA steps, and the eight
// partial 16 x 16 tiles are summed through LDS in wave order.
template <class F>
struct Wts {
  typename Raw<F>::T a, b;
  uint32_t sa, sb;
};

template <class F, int MODE, int K>
DEV void load_tile(const uint8_t* wq, const char* ws, size_t rb, int half, int r0, int G0, int g, int c16,
                   Wts<F> (&w)[K / 64 / PF_WPB]) {
  constexpr int GPW = K / 64 / PF_WPB;
  const size_t nA = (size_t)(r0 + c16), nB = (size_t)(half + r0 + c16);
#pragma unroll
  for (int i = 0; i < GPW; ++i) {
    F::load(wq + nA * rb, G0 + i, g, w[i].a);
    if (MODE == 0) F::load(wq + nB * rb, G0 + i, g, w[i].b);
    if (F::scale_group != 0) {
      w[i].sa = F::scale_raw(ws, nA, G0 + i, K);
      if (MODE == 0) w[i].sb = F::scale_raw(ws, nB, G0 + i, K);
    }
  }
}

template <class F, int MODE, int K>
__global__ void __launch_bounds__(PF_WPB * 64)
    k_grouped_ks(const uint8_t* __restrict__ Wq, const void* __restrict__ Ws, const uint16_t* __restrict__ X,
                 const int* __restrict__ offsets, const int* __restrict__ counts, void* __restrict__ out, int N,
                 size_t expert_q_bytes, size_t expert_s_elems, int s_elem_bytes, int fixed_rows) {
  constexpr int NG = K / 64, GPW = NG / PF_WPB;
  static_assert(GPW * PF_WPB == NG, "groups per wave");
  __shared__ float red[PF_WPB][8][64];
  const int e = fixed_rows >= 0 ? 0 : blockIdx.x;
  const int cnt = fixed_rows >= 0 ? fixed_rows : counts[e];
  const int tiles = (cnt + PF_TOK - 1) / PF_TOK;
  if ((int)blockIdx.z >= tiles) return;
  const size_t off = fixed_rows >= 0 ? 0 : (size_t)offsets[e];
  const int lane = lane_id(), wave = wave_id();
  const int g = lane >> 4, c16 = lane & 15;
  const int half = MODE == 0 ? N / 2 : 0;
  const uint8_t* wq = Wq + (size_t)e * expert_q_bytes;
  const char* ws = reinterpret_cast<const char*>(Ws) + (size_t)e * expert_s_elems * s_elem_bytes;
  const size_t rb = F::row_bytes(K);
  const int G0 = wave * GPW;
  const uint4 ones = make_uint4(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  Wts<F> cur[GPW];
  load_tile<F, MODE, K>(wq, ws, rb, half, blockIdx.y * 16, G0, g, c16, cur);
  {
    const int r0 = blockIdx.y * 16;
    // this lane's token row (MFMA A row c16) of a tile, its 16 inputs 64 G + 16 g .. + 15 per
    // group; the next tile's rows are loaded before the current one is used (rows past the
    // end load the last row and are zeroed: straight-line code keeps the load counter exact)
    auto load_x = [&](int tile, uint4 (&x0)[GPW], uint4 (&x1)[GPW]) {
      const int tok = tile * PF_TOK + c16;
      const uint16_t* xr = X + (off + (size_t)(tok < cnt ? tok : cnt - 1)) * K;
#pragma unroll
      for (int i = 0; i < GPW; ++i) {
        const int k0 = 64 * (G0 + i) + 16 * g;
        x0[i] = ld16(xr + k0), x1[i] = ld16(xr + k0 + 8);
      }
    };
    auto perm_x = [&](int tile, uint4 (&x0)[GPW], uint4 (&x1)[GPW]) {
      const bool live = tile * PF_TOK + c16 < cnt;
#pragma unroll
      for (int i = 0; i < GPW; ++i) {
        const uint4 v0 = live ? x0[i] : make_uint4(0, 0, 0, 0), v1 = live ? x1[i] : make_uint4(0, 0, 0, 0);
        // (e0 e1)(e2 e3)(e4 e5)(e6 e7) -> (e0 e4)(e1 e5)(e2 e6)(e3 e7)
        x0[i] = make_uint4(__builtin_amdgcn_perm(v0.z, v0.x, 0x05040100u), __builtin_amdgcn_perm(v0.z, v0.x, 0x07060302u),
                           __builtin_amdgcn_perm(v0.w, v0.y, 0x05040100u), __builtin_amdgcn_perm(v0.w, v0.y, 0x07060302u));
        x1[i] = make_uint4(__builtin_amdgcn_perm(v1.z, v1.x, 0x05040100u), __builtin_amdgcn_perm(v1.z, v1.x, 0x07060302u),
                           __builtin_amdgcn_perm(v1.w, v1.y, 0x05040100u), __builtin_amdgcn_perm(v1.w, v1.y, 0x07060302u));
      }
    };
    uint4 nx0[GPW], nx1[GPW];
    load_x(blockIdx.z, nx0, nx1);
    for (int tile = blockIdx.z; tile < tiles; tile += gridDim.z) {
      uint4 x0[GPW], x1[GPW];
#pragma unroll
      for (int i = 0; i < GPW; ++i) x0[i] = nx0[i], x1[i] = nx1[i];
      const int nt = tile + gridDim.z;
      load_x(nt < tiles ? nt : tile, nx0, nx1);
      perm_x(tile, x0, x1);
      f32x4 tA = z, tB = z;
#pragma unroll
      for (int i = 0; i < GPW; ++i) {
        uint4 a0, a1;
        F::convert(cur[i].a, a0, a1);
        if (F::scale_group == 0) {
          tA = mfma(x1[i], a1, mfma(x0[i], a0, tA));
          if (MODE == 0) {
            uint4 b0, b1;
            F::convert(cur[i].b, b0, b1);
            tB = mfma(x1[i], b1, mfma(x0[i], b0, tB));
          }
        } else {
          const f32x4 accA = mfma(x1[i], a1, mfma(x0[i], a0, z));
          f32x4 xg = z;
          if (F::has_min) xg = mfma(x1[i], ones, mfma(x0[i], ones, z));
          const float2 pa = F::scale_val(cur[i].sa);
          const float ca = pa.y - 128.f * pa.x;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            tA[r] = __builtin_fmaf(pa.x, accA[r], tA[r]);
            if (F::has_min) tA[r] = __builtin_fmaf(ca, xg[r], tA[r]);
          }
          if (MODE == 0) {
            uint4 b0, b1;
            F::convert(cur[i].b, b0, b1);
            const f32x4 accB = mfma(x1[i], b1, mfma(x0[i], b0, z));
            const float2 pb = F::scale_val(cur[i].sb);
            const float cb = pb.y - 128.f * pb.x;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              tB[r] = __builtin_fmaf(pb.x, accB[r], tB[r]);
              if (F::has_min) tB[r] = __builtin_fmaf(cb, xg[r], tB[r]);
            }
          }
        }
      }
      // sum the eight K slices in wave order; lane (token 4 g + r, row c16) of every wave
      __syncthreads();
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        red[wave][r][lane] = tA[r];
        if (MODE == 0) red[wave][4 + r][lane] = tB[r];
      }
      __syncthreads();
      const int ll = threadIdx.x & 63, rr = threadIdx.x >> 6;
      if (rr < 4) {
        float a = 0.f, b = 0.f;
#pragma unroll
        for (int w = 0; w < PF_WPB; ++w) {
          a += red[w][rr][ll];
          if (MODE == 0) b += red[w][4 + rr][ll];
        }
        const int tk = tile * PF_TOK + 4 * (ll >> 4) + rr, row = ll & 15;
        if (tk < cnt) {
          float rsA = 1.f, rsB = 1.f;
          if (F::scale_group == 0) {
            rsA = F::scale(ws, (size_t)(r0 + row), 0, K).x;
            if (MODE == 0) rsB = F::scale(ws, (size_t)(half + r0 + row), 0, K).x;
          }
          const size_t slot = off + tk;
          if (MODE == 0)
            reinterpret_cast<uint16_t*>(out)[slot * (size_t)(N / 2) + r0 + row] = to_bf16(silu(a * rsA) * (b * rsB));
          else
            reinterpret_cast<float*>(out)[slot * (size_t)N + r0 + row] = a * rsA;
        }
      }
    }
  }
}

// Shared-expert down projection over all prefill rows (one int8 weight set, dense, y = D act):
// a weight-stationary MFMA GEMM.  Block = 4 waves, 32 token rows x 32 weight rows.  The block's 32 rows (all K) are staged once in LDS
// (padded rows), then wave w streams half the inputs (K half w / 2) of the 16 token rows
// 16 (w % 2) .. of the block straight from global memory, DQ_D 64-input groups ahead, against
// both 16-row weight tiles (no barrier in the K loop); the two halves are summed through LDS.  Exact dequant as in k_grouped (int8 -> bf16 exactly; scale per row at the end,
// or per 128 inputs for the reference layout).
constexpr int DQ_TM = 32, DQ_D = 8;

template <class SH, int K>
__global__ void __launch_bounds__(256)
    k_dense_q8(const uint8_t* __restrict__ Wq, const uint16_t* __restrict__ Ws, const uint16_t* __restrict__ X,
               float* __restrict__ out, int rows, int N) {
  using F = FmtQ8<SH>;
  constexpr int WROW = K + 16, NG = K / 64, NW = 32 * K / 16 / 256;  // LDS row bytes, groups, fill loads
  constexpr int NH = NG / 2;  // groups per K half
  constexpr int D = DQ_D < NH ? DQ_D : NH;  // groups in flight
  static_assert(NH % D == 0 && NW >= 1, "shape");
  extern __shared__ uint4 dq_lds[];
  uint8_t* wl = reinterpret_cast<uint8_t*>(dq_lds);
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const int g = lane >> 4, c16 = lane & 15;
  const int t0 = blockIdx.x * DQ_TM;
  auto wrow = [&](int i) { return (size_t)(blockIdx.y * 32 + i); };
  // this lane's token row (MFMA A row c16 of wave w's tile), read through a buffer resource
  // bounded at the last row: rows past it read zeros without a fetch
  const int ntok = min(DQ_TM, rows - t0);
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(X + (size_t)t0 * K), 0, ntok * K * 2, 0x00020000);
  const int tok = (wave & 1) * 16 + c16, kh = wave >> 1;
  auto xload = [&](int G, uint4& v0, uint4& v1) {
    const int off = (tok * K + 64 * G + 16 * g) * 2;
    v0 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
    v1 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xr, off + 16, 0, 0));
  };
  // weights: NW 16-byte pieces per thread, all loads first, then the LDS stores
  {
    uint4 wv[NW];
#pragma unroll
    for (int q = 0; q < NW; ++q) {
      const int p = tid + 256 * q, r = p / (K / 16), b = p % (K / 16);
      wv[q] = ld16(Wq + wrow(r) * (size_t)K + b * 16);
    }
#pragma unroll
    for (int q = 0; q < NW; ++q) {
      const int p = tid + 256 * q, r = p / (K / 16), b = p % (K / 16);
      *reinterpret_cast<uint4*>(wl + r * WROW + b * 16) = wv[q];
    }
  }
  uint4 xa[D], xb[D];
#pragma unroll
  for (int d = 0; d < D; ++d) xload(kh * NH + d, xa[d], xb[d]);
  __syncthreads();
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  f32x4 tA = z, tB = z, cA = z, cB = z;
#pragma unroll 1
  for (int G0 = kh * NH; G0 < (kh + 1) * NH; G0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int G = G0 + d;
      // (e0 e1)(e2 e3)(e4 e5)(e6 e7) -> (e0 e4)(e1 e5)(e2 e6)(e3 e7): the fragment order of FmtQ8
      const uint4 v0 = xa[d], v1 = xb[d];
      const uint4 x0 = make_uint4(__builtin_amdgcn_perm(v0.z, v0.x, 0x05040100u), __builtin_amdgcn_perm(v0.z, v0.x, 0x07060302u),
                                  __builtin_amdgcn_perm(v0.w, v0.y, 0x05040100u), __builtin_amdgcn_perm(v0.w, v0.y, 0x07060302u));
      const uint4 x1 = make_uint4(__builtin_amdgcn_perm(v1.z, v1.x, 0x05040100u), __builtin_amdgcn_perm(v1.z, v1.x, 0x07060302u),
                                  __builtin_amdgcn_perm(v1.w, v1.y, 0x05040100u), __builtin_amdgcn_perm(v1.w, v1.y, 0x07060302u));
      if (G + D < (kh + 1) * NH) xload(G + D, xa[d], xb[d]);
      uint4 a0, a1, b0, b1;
      F::convert(*reinterpret_cast<const uint4*>(wl + c16 * WROW + G * 64 + g * 16), a0, a1);
      F::convert(*reinterpret_cast<const uint4*>(wl + (16 + c16) * WROW + G * 64 + g * 16), b0, b1);
      cA = mfma(x1, a1, mfma(x0, a0, cA));
      cB = mfma(x1, b1, mfma(x0, b0, cB));
      if (!SH::per_row && (G & 1)) {
        // per 128 inputs: scale the pair of groups, restart
        const float sa = SH::scale(Ws, wrow(c16), G * 64, K), sb = SH::scale(Ws, wrow(16 + c16), G * 64, K);
#pragma unroll
        for (int r = 0; r < 4; ++r) tA[r] = __builtin_fmaf(sa, cA[r], tA[r]), tB[r] = __builtin_fmaf(sb, cB[r], tB[r]);
        cA = z, cB = z;
      }
    }
  }
  float sa = 1.f, sb = 1.f;
  if (SH::per_row) {
    tA = cA, tB = cB;
    sa = SH::scale(Ws, wrow(c16), 0, K), sb = SH::scale(Ws, wrow(16 + c16), 0, K);
  }
  // the upper K half hands its sums to the lower one (LDS after the weights)
  f32x4* red = reinterpret_cast<f32x4*>(wl + 32 * WROW);
  if (kh == 1) red[((wave & 1) * 2) * 64 + lane] = tA, red[((wave & 1) * 2 + 1) * 64 + lane] = tB;
  __syncthreads();
  if (kh == 1) return;
  {
    const f32x4 ua = red[((wave & 1) * 2) * 64 + lane], ub = red[((wave & 1) * 2 + 1) * 64 + lane];
#pragma unroll
    for (int r = 0; r < 4; ++r) tA[r] += ua[r], tB[r] += ub[r];
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = (wave & 1) * 16 + 4 * g + r;
    if (t >= ntok) break;
    float* y = out + (size_t)(t0 + t) * N + blockIdx.y * 32;
    y[c16] = tA[r] * sa;
    y[16 + c16] = tB[r] * sb;
  }
}

// blocks of a kernel resident on the whole current device at once (occupancy x CUs), cached
// per (kernel, device); launchers may be called from several host threads
inline int resident_blocks(const void* kern, int threads, size_t lds) {
  static std::mutex mu;
  static const void* keys[64];
  static int devs[64], vals[64], n = 0;
  int dev = 0;
  (void)hipGetDevice(&dev);
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < n; ++i)
    if (keys[i] == kern && devs[i] == dev) return vals[i];
  int cus = 0, per = 0;
  (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kern, threads, lds);
  const int v = (per > 0 ? per : 1) * (cus > 0 ? cus : 256);
  if (n < 64) keys[n] = kern, devs[n] = dev, vals[n] = v, ++n;
  return v;
}

template <class F>
void launch_grouped(const uint8_t* wq, const void* ws, const uint16_t* X, const int* offsets, const int* counts,
                    void* out, int E, int N, int K, int mode, size_t eq, size_t es, int sb, int fixed_rows,
                    hipStream_t st, const int* rmap = nullptr, int x_rows = 0, bool packed = false) {
  const int rows_out = mode == 0 ? N / 2 : N;
  if (fixed_rows >= 0) {
    // one weight set over all rows (the shared expert).  gate_up: the K-split kernel, one
    // 16-row tile per block, token tiles over grid z (z = 4, 16, 32 and the dense kernel measured
    // slower); down: the dense weight-stationary kernel (6.6 against 10.2 us at 300 rows)
    if (mode == 0) {
      const int tiles = (fixed_rows + PF_TOK - 1) / PF_TOK;
      const dim3 grid(1, rows_out / 16, tiles < 8 ? tiles : 8);
      hipLaunchKernelGGL((k_grouped_ks<F, 0, 2048>), grid, dim3(PF_WPB * 64), 0, st, wq, ws, X, offsets, counts, out,
                         N, eq, es, sb, fixed_rows);
    } else if constexpr (F::q8) {  // fixed_rows is the int8 shared expert's mode only
      const dim3 grid((fixed_rows + DQ_TM - 1) / DQ_TM, N / 32);
      hipLaunchKernelGGL((k_dense_q8<typename F::Scale, 512>), grid, dim3(256), 32 * (512 + 16) + 4096, st, wq,
                         reinterpret_cast<const uint16_t*>(ws), X, reinterpret_cast<float*>(out), fixed_rows, N);
    }
    return;
  }
  // grouped experts: a persistent grid of as many blocks as are resident at once, walking the
  // work items (expert, token pass, row block) the kernel derives from counts
  const size_t lds = 2 * ((size_t)PF_TOK * K * 2 + (F::paired ? (size_t)(K / 64) * PF_TOK * 4 : 0)) + 192 * 16 +
                     (mode == 0 ? 2 * PF_GRPW * (PF_GWPB / 2) * 64 * 16 : 0);
  auto kern = mode == 1 ? k_grouped<F, 1, 512, false> : rmap ? k_grouped<F, 0, 2048, true> : k_grouped<F, 0, 2048, false>;
  if constexpr (F::packable) {
    if (packed)
      kern = mode == 1 ? k_grouped<F, 1, 512, false, true>
                       : rmap ? k_grouped<F, 0, 2048, true, true> : k_grouped<F, 0, 2048, false, true>;
  }
  int grid = resident_blocks((const void*)kern, PF_GWPB * 64, lds);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(PF_GWPB * 64), lds, st, wq, ws, X, offsets, counts, out, N, eq, es, sb, E,
                     err_word(), rmap, x_rows);
}

// gate_up then down for all experts of a grouped batch; with rmap, the gate_up token rows are
// read from X (x_rows rows) through the slot -> row map instead of from a gathered xp
template <class F>
int moe_prefill(const uint8_t* gu_q, const void* gu_s, const uint8_t* d_q, const void* d_s, const uint16_t* xp,
                const int* offsets, const int* counts, uint16_t* act, float* y, int E, int H, int I, size_t gu_q_b,
                size_t gu_s_e, size_t d_q_b, size_t d_s_e, int sb, hipStream_t st, const int* rmap = nullptr,
                int x_rows = 0, bool packed = false) {
  if (H != 2048 || I != 512 || E < 1 || E > PF_MAXE) return -1;
  if (rmap && (x_rows < 1 || (long long)x_rows * H * 2 > 0x7fffffffll)) return -1;
  launch_grouped<F>(gu_q, gu_s, xp, offsets, counts, act, E, 2 * I, H, 0, gu_q_b, gu_s_e, sb, -1, st, rmap, x_rows,
                    packed);
  launch_grouped<F>(d_q, d_s, act, offsets, counts, y, E, H, I, 1, d_q_b, d_s_e, sb, -1, st, nullptr, 0, packed);
  return 0;
}

// Shared expert over all rows: act = bf16(silu(SG hn) * (SU hn)), out = SD act (fp32).
template <class SH>
int shared_prefill(const int8_t* sgu_q, const uint16_t* sgu_s, const int8_t* sd_q, const uint16_t* sd_s, const uint16_t* hn,
                   int rows, uint16_t* act, float* out, int H, int I, hipStream_t st) {
  if (H != 2048 || I != 512 || rows < 0) return -1;
  if (rows == 0) return 0;
  launch_grouped<FmtQ8<SH>>((const uint8_t*)sgu_q, sgu_s, hn, nullptr, nullptr, act, 1, 2 * I, H, 0, 0, 0, 2, rows, st);
  launch_grouped<FmtQ8<SH>>((const uint8_t*)sd_q, sd_s, act, nullptr, nullptr, out, 1, H, I, 1, 0, 0, 2, rows, st);
  return 0;
}

// int4 experts [e][n][k / 2] with (scale, min) words [e][n][k / 64] -> the tile-step layout of
// k_grouped<..., PK>: for tile t (rows 16 t .. 16 t + 15) and step st (inputs 256 st ..
// 256 st + 255), block t * (k / 256) + st holds 2048 bytes, byte p 1024 + 16 l + b = byte
// 128 st + 64 p + 16 (l >> 4) + b of row 16 t + (l & 15), and 256 bytes of scales, word
// 4 r + w = scale word 4 st + w of row 16 t + r.  One thread per 16 bytes of either.
__global__ void __launch_bounds__(256)
    k_pack_q4(const uint8_t* __restrict__ q, const uint32_t* __restrict__ sm, uint8_t* __restrict__ qo,
              uint32_t* __restrict__ so, int n, int k, size_t nq, size_t ns) {
  const size_t c = (size_t)blockIdx.x * 256 + threadIdx.x;
  const int spt = k / 256;
  if (c < nq) {
    const size_t per_e = (size_t)n * (k / 2) / 16;
    const size_t e = c / per_e, r = c % per_e, blk = r / 128;
    const int p = (int)((r % 128) / 64), l = (int)(r % 64);
    const size_t t = blk / spt, stp = blk % spt;
    const size_t row = 16 * t + (l & 15);
    const size_t src = e * per_e * 16 + row * (k / 2) + stp * 128 + p * 64 + (l >> 4) * 16;
    *reinterpret_cast<uint4*>(qo + c * 16) = *reinterpret_cast<const uint4*>(q + src);
  } else if (c < nq + ns) {
    const size_t cs = c - nq;
    const size_t per_e = (size_t)n * (k / 64) / 4;
    const size_t e = cs / per_e, r = cs % per_e, blk = r / 16;
    const size_t t = blk / spt, stp = blk % spt, row = 16 * t + r % 16;
    const size_t src = e * per_e * 4 + row * (k / 64) + stp * 4;
    *reinterpret_cast<uint4*>(so + cs * 4) = *reinterpret_cast<const uint4*>(sm + src);
  }
}

// e4m3 experts [e][n][k] -> the tile-step layout of k_grouped<FmtFP8, ..., PK>: block t * (k / 256)
// + st of 4096 bytes (tile t of 16 rows, step st of 256 inputs), byte i 1024 + 16 l + b = byte
// 256 st + 64 i + 16 (l >> 4) + b of row 16 t + (l & 15).  One thread per 16 bytes.
__global__ void __launch_bounds__(256)
    k_pack_fp8(const uint8_t* __restrict__ q, uint8_t* __restrict__ qo, int n, int k, size_t nq) {
  const size_t c = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= nq) return;
  const int spt = k / 256;
  const size_t per_e = (size_t)n * k / 16;
  const size_t e = c / per_e, r = c % per_e, blk = r / 256;
  const int i = (int)((r % 256) / 64), l = (int)(r % 64);
  const size_t t = blk / spt, stp = blk % spt;
  const size_t row = 16 * t + (l & 15);
  const size_t src = e * per_e * 16 + row * k + stp * 256 + i * 64 + (l >> 4) * 16;
  *reinterpret_cast<uint4*>(qo + c * 16) = *reinterpret_cast<const uint4*>(q + src);
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

API int dr_moe_prefill_rows(const uint8_t* gu_q, const uint16_t* gu_sm, const uint8_t* d_q, const uint16_t* d_sm,
                            const uint16_t* x, int x_rows, const int* row_of_slot, const int* offsets,
                            const int* counts, uint16_t* act, float* y, int E, int H, int I, hipStream_t st) {
  if (!row_of_slot) return -1;
  return moe_prefill<FmtQ4<ScaleF16>>(gu_q, gu_sm, d_q, d_sm, x, offsets, counts, act, y, E, H, I,
                                      (size_t)2 * I * (H / 2), (size_t)2 * I * (H / 64) * 2, (size_t)H * (I / 2),
                                      (size_t)H * (I / 64) * 2, 2, st, row_of_slot, x_rows);
}

API int dr_moe_prefill_rows_bf16s(const uint8_t* gu_q, const uint16_t* gu_sm, const uint8_t* d_q, const uint16_t* d_sm,
                                  const uint16_t* x, int x_rows, const int* row_of_slot, const int* offsets,
                                  const int* counts, uint16_t* act, float* y, int E, int H, int I, hipStream_t st) {
  if (!row_of_slot) return -1;
  return moe_prefill<FmtQ4<ScaleBF16>>(gu_q, gu_sm, d_q, d_sm, x, offsets, counts, act, y, E, H, I,
                                       (size_t)2 * I * (H / 2), (size_t)2 * I * (H / 64) * 2, (size_t)H * (I / 2),
                                       (size_t)H * (I / 64) * 2, 2, st, row_of_slot, x_rows);
}

API int dr_moe_prefill_rows_fp8(const uint8_t* gu_w, const float* gu_s, const uint8_t* d_w, const float* d_s,
                                const uint16_t* x, int x_rows, const int* row_of_slot, const int* offsets,
                                const int* counts, uint16_t* act, float* y, int E, int H, int I, hipStream_t st) {
  if (!row_of_slot) return -1;
  return moe_prefill<FmtFP8<0>>(gu_w, gu_s, d_w, d_s, x, offsets, counts, act, y, E, H, I, (size_t)2 * I * H,
                                (size_t)(2 * I / 128) * (H / 128), (size_t)H * I, (size_t)(H / 128) * (I / 128), 4, st,
                                row_of_slot, x_rows);
}

API int dr_moe_prefill_rows_fp8_bf16s(const uint8_t* gu_w, const uint16_t* gu_s, const uint8_t* d_w,
                                      const uint16_t* d_s, const uint16_t* x, int x_rows, const int* row_of_slot,
                                      const int* offsets, const int* counts, uint16_t* act, float* y, int E, int H,
                                      int I, hipStream_t st) {
  if (!row_of_slot) return -1;
  return moe_prefill<FmtFP8<1>>(gu_w, gu_s, d_w, d_s, x, offsets, counts, act, y, E, H, I, (size_t)2 * I * H,
                                (size_t)(2 * I / 128) * (H / 128), (size_t)H * I, (size_t)(H / 128) * (I / 128), 2, st,
                                row_of_slot, x_rows);
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

// [a, a + na) and [b, b + nb) share a byte
static bool overlaps(const void* a, size_t na, const void* b, size_t nb) {
  const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return x < y + nb && y < x + na;
}

API int dr_moe_pack_q4(const uint8_t* q, const uint16_t* sm, int e, int n, int k, uint8_t* q_out, uint16_t* sm_out,
                       hipStream_t st) {
  if (e < 1 || n < 16 || n % 16 || k < 256 || k % 256 || !q || !sm || !q_out || !sm_out) return -1;
  const size_t nq = (size_t)e * n * (k / 2) / 16, ns = (size_t)e * n * (k / 64) / 4;
  const size_t qb = nq * 16, sb = ns * 16;  // bytes of the weights and of the scale words
  if (overlaps(q_out, qb, q, qb) || overlaps(q_out, qb, sm, sb) || overlaps(sm_out, sb, q, qb) ||
      overlaps(sm_out, sb, sm, sb) || overlaps(q_out, qb, sm_out, sb))
    return -1;
  const size_t blocks = (nq + ns + 255) / 256;
  hipLaunchKernelGGL(k_pack_q4, dim3((unsigned)blocks), dim3(256), 0, st, q, reinterpret_cast<const uint32_t*>(sm),
                     q_out, reinterpret_cast<uint32_t*>(sm_out), n, k, nq, ns);
  return 0;
}

API int dr_moe_prefill_rows_packed(const uint8_t* gu_q, const uint16_t* gu_sm, const uint8_t* d_q,
                                   const uint16_t* d_sm, const uint16_t* x, int x_rows, const int* row_of_slot,
                                   const int* offsets, const int* counts, uint16_t* act, float* y, int E, int H, int I,
                                   hipStream_t st) {
  if (!row_of_slot) return -1;
  return moe_prefill<FmtQ4<ScaleF16>>(gu_q, gu_sm, d_q, d_sm, x, offsets, counts, act, y, E, H, I,
                                      (size_t)2 * I * (H / 2), (size_t)2 * I * (H / 64) * 2, (size_t)H * (I / 2),
                                      (size_t)H * (I / 64) * 2, 2, st, row_of_slot, x_rows, true);
}

API int dr_moe_prefill_rows_packed_bf16s(const uint8_t* gu_q, const uint16_t* gu_sm, const uint8_t* d_q,
                                         const uint16_t* d_sm, const uint16_t* x, int x_rows, const int* row_of_slot,
                                         const int* offsets, const int* counts, uint16_t* act, float* y, int E, int H,
                                         int I, hipStream_t st) {
  if (!row_of_slot) return -1;
  return moe_prefill<FmtQ4<ScaleBF16>>(gu_q, gu_sm, d_q, d_sm, x, offsets, counts, act, y, E, H, I,
                                       (size_t)2 * I * (H / 2), (size_t)2 * I * (H / 64) * 2, (size_t)H * (I / 2),
                                       (size_t)H * (I / 64) * 2, 2, st, row_of_slot, x_rows, true);
}

API int dr_moe_pack_fp8(const uint8_t* q, int e, int n, int k, uint8_t* q_out, hipStream_t st) {
  if (e < 1 || n < 16 || n % 16 || k < 256 || k % 256 || !q || !q_out) return -1;
  const size_t nq = (size_t)e * n * k / 16;
  if (overlaps(q_out, nq * 16, q, nq * 16)) return -1;
  hipLaunchKernelGGL(k_pack_fp8, dim3((unsigned)((nq + 255) / 256)), dim3(256), 0, st, q, q_out, n, k, nq);
  return 0;
}

API int dr_moe_prefill_rows_packed_fp8(const uint8_t* gu_w, const float* gu_s, const uint8_t* d_w, const float* d_s,
                                       const uint16_t* x, int x_rows, const int* row_of_slot, const int* offsets,
                                       const int* counts, uint16_t* act, float* y, int E, int H, int I,
                                       hipStream_t st) {
  if (!row_of_slot) return -1;
  return moe_prefill<FmtFP8<0>>(gu_w, gu_s, d_w, d_s, x, offsets, counts, act, y, E, H, I, (size_t)2 * I * H,
                                (size_t)(2 * I / 128) * (H / 128), (size_t)H * I, (size_t)(H / 128) * (I / 128), 4, st,
                                row_of_slot, x_rows, true);
}

API int dr_moe_prefill_rows_packed_fp8_bf16s(const uint8_t* gu_w, const uint16_t* gu_s, const uint8_t* d_w,
                                             const uint16_t* d_s, const uint16_t* x, int x_rows,
                                             const int* row_of_slot, const int* offsets, const int* counts,
                                             uint16_t* act, float* y, int E, int H, int I, hipStream_t st) {
  if (!row_of_slot) return -1;
  return moe_prefill<FmtFP8<1>>(gu_w, gu_s, d_w, d_s, x, offsets, counts, act, y, E, H, I, (size_t)2 * I * H,
                                (size_t)(2 * I / 128) * (H / 128), (size_t)H * I, (size_t)(H / 128) * (I / 128), 2, st,
                                row_of_slot, x_rows, true);
}

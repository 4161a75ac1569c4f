/*
 * drama_moe.h -- C ABI of libdramamoe.so, the gfx950 (MI355X) routed-expert MoE path.
 *
 * The symbols, argument order and argument meaning of the first two sections are those of
 * the Rust bindings in apiplant/drama-rs src/ffi.rs (declarations at the lines cited), so the
 * reference engine (src/engine.rs) links against this library in place of its CUDA
 * libdramakernels.a.  Streams are hipStream_t, passed as an opaque pointer exactly like the
 * reference's `Stream = *mut c_void` (src/ffi.rs:7).
 *
 * Conventions (src/gpu.rs:146-163):
 *   - launchers return 0 on success and -1 for an unsupported shape; they never allocate,
 *     free or synchronise, and read routing/indices from device memory so they can be
 *     captured in a graph;
 *   - runtime wrappers return the raw HIP error code (0 = success), mapped by dr_error_string;
 *   - every buffer is caller owned; scratch sizes are stated per entry point.
 *
 * Weight layouts (src/model.rs:16-43,99-111, tools/convert.py:92-110):
 *   int4 experts: q u8 [E, N, K/2], nibble (k & 1) of byte k/2 is element k, low nibble first;
 *                 sm [E, N, K/64, 2] = (scale, min) per group of 64, w = q * scale + min.
 *   int8 dense:   q i8 [N, K], w = q * s; s f16 [N, K/128] (reference) or bf16 [N] (_bf16s).
 *   fp8 experts:  OCP e4m3 [E, N, K], scale per 128x128 block [E, N/128, K/128].
 * The *_bf16s entry points (third section) take the same arguments with bf16 instead of f16
 * scale encodings and per-output-channel int8 scales: the formats of the synthetic
 * benchmark configurations.  They have no counterpart in the reference.
 */
#ifndef DRAMA_MOE_H
#define DRAMA_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Library error codes (beside -1 and the raw HIP codes): a kernel whose bounded wait gave up
 * sets a process-wide error word; dr_stream_sync reports it after the wait, the fused-step
 * launchers refuse to start while it is set, and dr_last_error returns and clears it. */
#define DR_ERR_STEP_TIMEOUT 9001 /* fused step: workgroups not co-resident within the wait limit */
#define DR_ERR_PREFILL_WAIT 9002 /* prefill grouped GEMM: an LDS hand-off between waves timed out */
#define DR_ERR_ROUTE_WAIT 9003 /* fused small-batch router + experts: the picks did not arrive in time */

typedef void* dr_stream_t;     /* hipStream_t */
typedef void* dr_graph_exec_t; /* hipGraphExec_t */
typedef uint16_t dr_bf16;      /* raw bf16 bits */
typedef uint16_t dr_half;      /* raw IEEE binary16 bits */

/* ===================================================================================== */
/* Runtime wrappers -- src/ffi.rs:13-31, defined in kernels/drama.cu:1995-2044            */
/* ===================================================================================== */

const char* dr_error_string(int e);                               /* src/ffi.rs:13 */
int dr_last_error(void);                                          /* src/ffi.rs:14 (+ library errors, cleared) */
int dr_malloc(void** p, size_t n);                                /* src/ffi.rs:15 */
int dr_free(void* p);                                             /* src/ffi.rs:16 */
int dr_host_alloc(void** p, size_t n);                            /* src/ffi.rs:17 */
int dr_host_free(void* p);                                        /* src/ffi.rs:18 */
int dr_h2d(void* d, const void* h, size_t n, dr_stream_t st);     /* src/ffi.rs:19 */
int dr_d2h(void* h, const void* d, size_t n, dr_stream_t st);     /* src/ffi.rs:20 */
int dr_d2d(void* d, const void* s, size_t n, dr_stream_t st);     /* src/ffi.rs:21 */
/* src/ffi.rs:22.  Implemented with a fill kernel (not hipMemsetAsync) so it is safe inside
 * graph capture. */
int dr_memset(void* d, int v, size_t n, dr_stream_t st);
int dr_stream_create(dr_stream_t* s);                             /* src/ffi.rs:23, non-blocking */
int dr_stream_sync(dr_stream_t s);                                /* src/ffi.rs:24 (+ pending library error) */
int dr_device_sync(void);                                         /* kernels/drama.cu:2012 */
int dr_mem_info(size_t* free_b, size_t* total_b);                 /* src/ffi.rs:25 */
int dr_graph_begin(dr_stream_t s);                                /* src/ffi.rs:26, thread-local capture */
int dr_graph_end(dr_stream_t s, dr_graph_exec_t* exec);           /* src/ffi.rs:27 */
int dr_graph_launch(dr_graph_exec_t exec, dr_stream_t s);         /* src/ffi.rs:28 */
int dr_graph_destroy(dr_graph_exec_t exec);                       /* src/ffi.rs:29 */
/* src/ffi.rs:30.  The name is kept for the engine; the handle only records the stream for
 * dr_gemm, which is this library's own kernel (no BLAS). */
int dr_cublas_create(void** h, dr_stream_t s);
/* src/ffi.rs:31.  C[M, N] (row-major f32) = A[M, K] (bf16) . W[N, K]^T (bf16) + beta * C.
 * Every element is accumulated in the canonical fp32 order of the router (lane-strided
 * 8-element chunks, fmaf in element order, 64-lane xor butterfly), so prefill router logits
 * are reproducible bit for bit.  K % 8 == 0. */
int dr_gemm(void* h, const dr_bf16* A, const dr_bf16* W, float* C, int M, int N, int K, float beta);

/* ===================================================================================== */
/* MoE launchers -- src/ffi.rs:41-73                                                       */
/* ===================================================================================== */

/* src/ffi.rs:55-59, kernels/drama.cu:369-461.  Router logits over E+1 bf16 rows (row E is
 * the shared-expert gate) of RMSNorm(x; nw) (x as is when nw is NULL), softmax over E,
 * top-k by (p desc, index asc), wts renormalised to sum 1, sgate = logits[E].  counter (>= 4
 * bytes) must be 0 on entry and is 0 again on exit.  The prefetch arguments are accepted and
 * ignored (the reference disables them too, src/engine.rs:18,976).
 * Unsupported: K != 2048, E > 256, topk > 32, topk > E -> -1. */
int dr_router_topk(const dr_bf16* w, const float* x, const float* nw, float eps, float* logits, int e,
                   int topk, int k, int* idx, float* wts, float* sgate, uint32_t* counter,
                   const char* gu_q, const char* gu_sm, const char* d_q, const char* d_sm, size_t gu_q_b,
                   size_t gu_sm_b, size_t d_q_b, size_t d_sm_b, dr_stream_t st);

/* src/ffi.rs:41, kernels/drama.cu:320-367,463-468.  Row-wise softmax/top-k of prefill router
 * logits with row stride `stride` (>= E + 1), sgate[r] = logits[r, E].  E > 256 -> -1. */
int dr_moe_topk(const float* logits, int rows, int e, int topk, int stride, int* idx, float* wts,
                float* sgate, dr_stream_t st);

/* src/ffi.rs:42-46, kernels/drama.cu:470-599.  One decode token:
 *   xn = RMSNorm(x; nw), act[k][j] = silu(G_e[j] . xn) * (U_e[j] . xn) for e = idx[k],
 *   act[topk][j] the same with the int8 shared expert,
 *   y[n] = res[n] + sigmoid(sgate) * (SD[n] . act[topk]) + sum_k wts[k] (D_e[n] . act[k]).
 * act is scratch of (topk + 1) * i floats.  x, res and y may alias (the engine passes one
 * buffer for all three).  pf/pf_bytes: a range the kernel warms in the memory-side cache
 * after its own work (the next op's weights).  Unsupported: h != 2048, i != 512, topk != 8. */
int dr_moe_decode(const uint8_t* gu_q, const dr_half* gu_sm, const uint8_t* d_q, const dr_half* d_sm,
                  const int8_t* sgu_q, const dr_half* sgu_s, const int8_t* sd_q, const dr_half* sd_s,
                  const float* x, const int* idx, const float* wts, const float* sgate, const float* res,
                  float* act, float* y, int h, int i, int topk, const float* nw, float eps, const char* pf,
                  size_t pf_bytes, dr_stream_t st);

/* src/ffi.rs:47-51, kernels/drama.cu:602-742.  As dr_moe_decode with block-FP8 e4m3 experts:
 * gu_w [E, 2I, H], gu_s f32 [E, 2I/128, H/128]; d_w [E, H, I], d_s f32 [E, H/128, I/128]. */
int dr_moe_decode_fp8(const uint8_t* gu_w, const float* gu_s, const uint8_t* d_w, const float* d_s,
                      const int8_t* sgu_q, const dr_half* sgu_s, const int8_t* sd_q, const dr_half* sd_s,
                      const float* x, const int* idx, const float* wts, const float* sgate, const float* res,
                      float* act, float* y, int h, int i, int topk, const float* nw, float eps,
                      const char* pf, size_t pf_bytes, dr_stream_t st);

/* src/ffi.rs:52-54, kernels/drama.cu:970-1109.  FP8 counterpart of dr_moe_prefill. */
int dr_moe_prefill_fp8(const uint8_t* gu_w, const float* gu_s, const uint8_t* d_w, const float* d_s,
                       const dr_bf16* xp, const int* offsets, const int* counts, dr_bf16* act, float* y, int e,
                       int h, int i, dr_stream_t st);

/* src/ffi.rs:60-63, kernels/drama.cu:799-968.  Expert-grouped prefill: rows of xp are
 * sorted by expert (expert e owns rows [offsets[e], offsets[e] + counts[e])):
 *   act[t] = bf16(silu(G_e . xp[t]) * (U_e . xp[t])),  y[t] = D_e . act[t] (f32).
 * Unsupported: h != 2048, i != 512, e > 256. */
int dr_moe_prefill(const uint8_t* gu_q, const dr_half* gu_sm, const uint8_t* d_q, const dr_half* d_sm,
                   const dr_bf16* xp, const int* offsets, const int* counts, dr_bf16* act, float* y, int e,
                   int h, int i, dr_stream_t st);

/* src/ffi.rs:64, kernels/drama.cu:744-753.  counts[idx[i]] += 1 for i < n (caller zeroes). */
int dr_moe_count(const int* idx, int n, int* counts, dr_stream_t st);

/* src/ffi.rs:65-68, kernels/drama.cu:755-778.  Scatter bf16 rows of x into expert order:
 * pair i = (row i / topk, k) goes to slot offsets[e] + (number of pairs j < i routed to e),
 * slot_of[i] = slot, xp[slot] = x[i / topk].  The within-expert order is stable in the pair
 * index (the reference's order comes from atomics and is unspecified; this is one of the
 * orders it can produce).  fill must be zero on entry and ends equal to the per-expert
 * counts, as in the reference; only the entries of experts that occur in idx are read or
 * written, so offsets/fill may hold just the model's E entries.  Pairs are grouped 8192 at a
 * time in stream order (any rows * topk up to 2^30).  Unsupported: h % 8 != 0 -> -1. */
int dr_moe_permute(const int* idx, int rows, int topk, const int* offsets, int* fill, int* slot_of,
                   const dr_bf16* x, dr_bf16* xp, int h, dr_stream_t st);

/* src/ffi.rs:69-72, kernels/drama.cu:780-797.
 * x[r] += sigmoid(sgate[r]) * shared[r] + sum_k wts[r, k] * y[slot_of[r, k]] (k ascending). */
int dr_moe_combine(float* x, const float* y, const int* slot_of, const float* wts, const float* sgate,
                   const float* shared, int rows, int topk, int h, dr_stream_t st);

/* src/ffi.rs:74, kernels/drama.cu:1114-1134.  out = bf16(q * s), s f16 per 128 inputs. */
int dr_dequant_q8(const int8_t* w, const dr_half* s, dr_bf16* out, int n, int k, dr_stream_t st);
/* src/ffi.rs:75, kernels/drama.cu:1156-1164. */
int dr_f32_to_bf16(const float* x, dr_bf16* y, size_t n, dr_stream_t st);
/* src/ffi.rs:76, kernels/drama.cu:1166-1180.  y[r, j] = bf16(silu(h[r, j]) * h[r, i + j]). */
int dr_swiglu_rows(const float* h, dr_bf16* y, int rows, int i, dr_stream_t st);

/* src/ffi.rs:33-40, kernels/drama.cu:216-315: the dense decode GEMVs around the MoE.
 * y[n] = W[n] . xn (+ res[n]) with xn = RMSNorm(x; nw); y may alias res. */
int dr_gemv_q8(const int8_t* w, const dr_half* s, const float* x, const float* res, float* y, int n, int k,
               const float* nw, float eps, const char* pf, size_t pf_bytes, dr_stream_t st);
/* y[j] = silu(W[j] . xn) * (W[i + j] . xn) for j < i. */
int dr_gemv_q8_swiglu(const int8_t* w, const dr_half* s, const float* x, float* y, int i, int k,
                      const float* nw, float eps, const char* pf, size_t pf_bytes, dr_stream_t st);
int dr_gemv_bf16(const dr_bf16* w, const float* x, float* y, int n, int k, const float* nw, float eps,
                 const char* pf, size_t pf_bytes, dr_stream_t st);

/* ===================================================================================== */
/* Extensions: no counterpart in src/ffi.rs                                                */
/* ===================================================================================== */

/* Releases a handle of dr_cublas_create (NULL is a no-op).  The reference keeps its BLAS handle
 * for the engine's lifetime and has no counterpart; for callers that create handles per stream. */
int dr_cublas_destroy(void* h);

/* Device-side grouping in one launch: counts (histogram), offsets (exclusive scan) and
 * slot_of (stable counting sort of the n pairs by expert), replacing dr_moe_count + the host
 * scan of src/engine.rs:564-575, so a prefill layer needs no host round trip.
 * Unsupported: n > 8192, e > 256 -> -1. */
int dr_moe_group(const int* idx, int n, int e, int* counts, int* offsets, int* slot_of, dr_stream_t st);

/* xp[slot_of[i]] = x[i / topk] for i < rows * topk: the copy half of dr_moe_permute for a
 * grouping computed by dr_moe_group. */
int dr_moe_gather_rows(const int* slot_of, int rows, int topk, const dr_bf16* x, dr_bf16* xp, int h,
                       dr_stream_t st);

/* Prefill top-k and grouping in one launch: dr_moe_topk (same idx, wts and sgate bits) followed
 * by dr_moe_group over the rows * topk pairs (same counts, offsets and slot_of), plus the inverse
 * map row_of_slot[slot] = pair / topk, the token row each grouped slot takes its input from.
 * counter (>= 4 bytes) must be 0 on entry and is 0 again on exit.  row_of_slot needs
 * rows * topk + 16 entries (dr_moe_prefill_rows reads the map 16 entries at a time).
 * Unsupported: rows * topk > 8192, e > 256, topk > 32, topk > e, stride < e + 1 -> -1. */
int dr_moe_topk_group(const float* logits, int rows, int e, int topk, int stride, int* idx, float* wts,
                      float* sgate, int* counts, int* offsets, int* slot_of, int* row_of_slot, uint32_t* counter,
                      dr_stream_t st);

/* dr_moe_group of rows * topk pairs plus row_of_slot as in dr_moe_topk_group (for a routing
 * that does not come from dr_moe_topk_group).  Unsupported: rows * topk > 8192, e > 256 -> -1. */
int dr_moe_group_rows(const int* idx, int rows, int topk, int e, int* counts, int* offsets, int* slot_of,
                      int* row_of_slot, dr_stream_t st);

/* dr_moe_prefill with the gate_up inputs read straight from the x_rows token rows of x through
 * row_of_slot (from dr_moe_topk_group) instead of from a gathered xp: the same act and y bits as
 * dr_moe_gather_rows followed by dr_moe_prefill, one launch and the xp copy fewer.  Formats as
 * dr_moe_prefill, dr_moe_prefill_bf16s, dr_moe_prefill_fp8 and dr_moe_prefill_fp8_bf16s. */
int dr_moe_prefill_rows(const uint8_t* gu_q, const dr_half* gu_sm, const uint8_t* d_q, const dr_half* d_sm,
                        const dr_bf16* x, int x_rows, const int* row_of_slot, const int* offsets, const int* counts,
                        dr_bf16* act, float* y, int e, int h, int i, dr_stream_t st);
int dr_moe_prefill_rows_bf16s(const uint8_t* gu_q, const dr_bf16* gu_sm, const uint8_t* d_q, const dr_bf16* d_sm,
                              const dr_bf16* x, int x_rows, const int* row_of_slot, const int* offsets,
                              const int* counts, dr_bf16* act, float* y, int e, int h, int i, dr_stream_t st);
int dr_moe_prefill_rows_fp8(const uint8_t* gu_w, const float* gu_s, const uint8_t* d_w, const float* d_s,
                            const dr_bf16* x, int x_rows, const int* row_of_slot, const int* offsets,
                            const int* counts, dr_bf16* act, float* y, int e, int h, int i, dr_stream_t st);
int dr_moe_prefill_rows_fp8_bf16s(const uint8_t* gu_w, const dr_bf16* gu_s, const uint8_t* d_w,
                                  const dr_bf16* d_s, const dr_bf16* x, int x_rows, const int* row_of_slot,
                                  const int* offsets, const int* counts, dr_bf16* act, float* y, int e, int h,
                                  int i, dr_stream_t st);

/* A second, prefill-only copy of int4 experts in the tile-step layout the grouped MFMA kernel
 * streams best: e matrices [n, k/2] (q) with their (scale, min) pairs [n, k/64] (sm, f16 or bf16
 * pairs, copied as they are) -> q_out, sm_out of the same sizes, where each 16-row tile's
 * 256-input step is one contiguous 2048-byte block (byte p*1024 + 16 l + b of block
 * t*(k/256) + s = byte 128 s + 64 p + 16 (l >> 4) + b of row 16 t + (l & 15)) followed in
 * sm_out by 256 bytes of its scale words (word 4 r + w = word 4 s + w of row 16 t + r).
 * Pack gu_q/gu_sm with n = 2i, k = h and d_q/d_sm with n = h, k = i.  The layout costs a second
 * copy of the routed experts (16.9 GiB for configuration 3's 40 layers, 6% of an MI355X's HBM)
 * and changes no result.  Unsupported: n % 16, k % 256, or outputs overlapping the inputs (no
 * in-place packing) -> -1.  No reference counterpart. */
int dr_moe_pack_q4(const uint8_t* q, const uint16_t* sm, int e, int n, int k, uint8_t* q_out, uint16_t* sm_out,
                   dr_stream_t st);
/* dr_moe_prefill_rows / dr_moe_prefill_rows_bf16s with the expert weights packed by
 * dr_moe_pack_q4: the same act and y bits, ~6% less time at configuration 4. */
int dr_moe_prefill_rows_packed(const uint8_t* gu_q, const dr_half* gu_sm, const uint8_t* d_q, const dr_half* d_sm,
                               const dr_bf16* x, int x_rows, const int* row_of_slot, const int* offsets,
                               const int* counts, dr_bf16* act, float* y, int e, int h, int i, dr_stream_t st);
int dr_moe_prefill_rows_packed_bf16s(const uint8_t* gu_q, const dr_bf16* gu_sm, const uint8_t* d_q,
                                     const dr_bf16* d_sm, const dr_bf16* x, int x_rows, const int* row_of_slot,
                                     const int* offsets, const int* counts, dr_bf16* act, float* y, int e, int h,
                                     int i, dr_stream_t st);
/* FP8 counterpart of dr_moe_pack_q4: e4m3 experts [e][n][k] -> q_out in the tile-step layout,
 * block t (k / 256) + s of 4096 bytes (t: 16-row tile, s: 256-input step), byte
 * 1024 p + 16 l + b = byte 256 s + 64 p + 16 (l >> 4) + b of row 16 t + (l & 15).  The 128x128
 * block scales keep their layout and are passed unchanged.  Unsupported: n % 16, k % 256, or
 * q_out overlapping q -> -1.
 * No reference counterpart. */
int dr_moe_pack_fp8(const uint8_t* q, int e, int n, int k, uint8_t* q_out, dr_stream_t st);
/* dr_moe_prefill_rows_fp8 / dr_moe_prefill_rows_fp8_bf16s with the expert weights packed by
 * dr_moe_pack_fp8: the same act and y bits. */
int dr_moe_prefill_rows_packed_fp8(const uint8_t* gu_w, const float* gu_s, const uint8_t* d_w, const float* d_s,
                                   const dr_bf16* x, int x_rows, const int* row_of_slot, const int* offsets,
                                   const int* counts, dr_bf16* act, float* y, int e, int h, int i, dr_stream_t st);
int dr_moe_prefill_rows_packed_fp8_bf16s(const uint8_t* gu_w, const dr_bf16* gu_s, const uint8_t* d_w,
                                         const dr_bf16* d_s, const dr_bf16* x, int x_rows, const int* row_of_slot,
                                         const int* offsets, const int* counts, dr_bf16* act, float* y, int e,
                                         int h, int i, dr_stream_t st);

/* Prefill shared expert fused: act = bf16(silu(SG . hn) * (SU . hn)), out = SD . act (f32),
 * int8 weights dequantised in registers (replaces dr_dequant_q8 + dr_gemm + dr_swiglu_rows +
 * dr_dequant_q8 + dr_gemm of src/engine.rs:560-562).  act: scratch of rows * i bf16. */
int dr_moe_shared_prefill(const int8_t* sgu_q, const dr_half* sgu_s, const int8_t* sd_q, const dr_half* sd_s,
                          const dr_bf16* hn, int rows, dr_bf16* act, float* out, int h, int i, dr_stream_t st);

/* Configuration formats (bf16 scales, per-channel int8 scales).  Same semantics as the
 * entry point named without the suffix; yb (nullable) also receives y rounded to bf16. */
int dr_moe_decode_bf16s(const uint8_t* gu_q, const dr_bf16* gu_sm, const uint8_t* d_q, const dr_bf16* d_sm,
                        const int8_t* sgu_q, const dr_bf16* sgu_s, const int8_t* sd_q, const dr_bf16* sd_s,
                        const float* x, const int* idx, const float* wts, const float* sgate, const float* res,
                        float* act, float* y, dr_bf16* yb, int h, int i, int topk, const float* nw, float eps,
                        const char* pf, size_t pf_bytes, dr_stream_t st);
int dr_moe_decode_fp8_bf16s(const uint8_t* gu_w, const dr_bf16* gu_s, const uint8_t* d_w, const dr_bf16* d_s,
                            const int8_t* sgu_q, const dr_bf16* sgu_s, const int8_t* sd_q, const dr_bf16* sd_s,
                            const float* x, const int* idx, const float* wts, const float* sgate,
                            const float* res, float* act, float* y, dr_bf16* yb, int h, int i, int topk,
                            const float* nw, float eps, const char* pf, size_t pf_bytes, dr_stream_t st);
int dr_moe_prefill_bf16s(const uint8_t* gu_q, const dr_bf16* gu_sm, const uint8_t* d_q, const dr_bf16* d_sm,
                         const dr_bf16* xp, const int* offsets, const int* counts, dr_bf16* act, float* y,
                         int e, int h, int i, dr_stream_t st);
int dr_moe_prefill_fp8_bf16s(const uint8_t* gu_w, const dr_bf16* gu_s, const uint8_t* d_w, const dr_bf16* d_s,
                             const dr_bf16* xp, const int* offsets, const int* counts, dr_bf16* act, float* y,
                             int e, int h, int i, dr_stream_t st);
int dr_moe_shared_prefill_bf16s(const int8_t* sgu_q, const dr_bf16* sgu_s, const int8_t* sd_q,
                                const dr_bf16* sd_s, const dr_bf16* hn, int rows, dr_bf16* act, float* out, int h,
                                int i, dr_stream_t st);

/* Small decode batches (a few tokens decoded together, e.g. benchmark configuration 5's
 * batch 4): the batch-1 chain dr_router_topk -> dr_moe_decode(_fp8) for `rows` independent
 * rows in three launches instead of a prefill-style grouping.  Row r uses x + r k (f32),
 * logits + r (e + 1), idx/wts + r topk, sgate + r; the experts of each row are streamed once
 * per row and the shared expert once for up to four rows.  Routing of each row is bit-exact
 * with dr_router_topk on that row.  No reference counterpart (the engine decodes one token
 * per step).  dr_router_topk_rows: rows <= 8, counter as in dr_router_topk. */
int dr_router_topk_rows(const dr_bf16* w, const float* x, const float* nw, float eps, float* logits, int e,
                        int topk, int k, int rows, int* idx, float* wts, float* sgate, uint32_t* counter,
                        dr_stream_t st);
/* x, res, y [rows, h] (y may alias x and res), act scratch rows x (topk + 1) x i floats;
 * 1 <= rows <= 64.  Same weights and formats as dr_moe_decode / dr_moe_decode_bf16s /
 * dr_moe_decode_fp8 / dr_moe_decode_fp8_bf16s. */
int dr_moe_decode_rows(const uint8_t* gu_q, const dr_half* gu_sm, const uint8_t* d_q, const dr_half* d_sm,
                       const int8_t* sgu_q, const dr_half* sgu_s, const int8_t* sd_q, const dr_half* sd_s,
                       const float* x, const int* idx, const float* wts, const float* sgate, const float* res,
                       float* act, float* y, int rows, int h, int i, int topk, const float* nw, float eps,
                       dr_stream_t st);
int dr_moe_decode_rows_bf16s(const uint8_t* gu_q, const dr_bf16* gu_sm, const uint8_t* d_q, const dr_bf16* d_sm,
                             const int8_t* sgu_q, const dr_bf16* sgu_s, const int8_t* sd_q, const dr_bf16* sd_s,
                             const float* x, const int* idx, const float* wts, const float* sgate, const float* res,
                             float* act, float* y, dr_bf16* yb, int rows, int h, int i, int topk, const float* nw,
                             float eps, dr_stream_t st);
int dr_moe_decode_rows_fp8(const uint8_t* gu_w, const float* gu_s, const uint8_t* d_w, const float* d_s,
                           const int8_t* sgu_q, const dr_half* sgu_s, const int8_t* sd_q, const dr_half* sd_s,
                           const float* x, const int* idx, const float* wts, const float* sgate, const float* res,
                           float* act, float* y, int rows, int h, int i, int topk, const float* nw, float eps,
                           dr_stream_t st);
int dr_moe_decode_rows_fp8_bf16s(const uint8_t* gu_w, const dr_bf16* gu_s, const uint8_t* d_w, const dr_bf16* d_s,
                                 const int8_t* sgu_q, const dr_bf16* sgu_s, const int8_t* sd_q, const dr_bf16* sd_s,
                                 const float* x, const int* idx, const float* wts, const float* sgate,
                                 const float* res, float* act, float* y, dr_bf16* yb, int rows, int h, int i,
                                 int topk, const float* nw, float eps, dr_stream_t st);
/* The FP8 small-batch path with the router in the gate_up launch: dr_router_topk_rows followed
 * by dr_moe_decode_rows_fp8(_bf16s) on the same arguments, with the same results bit for bit
 * (routing bit-exact per row), in two launches per four rows instead of three.  The router's
 * blocks come first in the gate_up launch; the gate_up blocks request their rows of x and
 * then wait for the picks, which the router's last block publishes as tagged 64-bit words;
 * down follows as in dr_moe_decode_rows_fp8.  counter: 4 words, zero before the first call
 * and then owned by the library (word 1 holds the tag of the last launch); tags: 896 words
 * (the picks and the launch's block count), zero before the first call and then owned by the
 * library; logits rows (e + 1) floats; idx / wts / sgate as dr_router_topk_rows; act rows x
 * (topk + 1) x i floats; y may alias x and res.  e in [topk, 256], topk = 8,
 * 1 <= rows <= 64.  Calls that share counter or tags must not overlap.  A gate_up block that
 * sees no picks within its wait limit raises DR_ERR_ROUTE_WAIT (the outputs are then wrong).
 * No reference counterpart (the engine decodes one token per step). */
int dr_moe_decode_rows_routed_fp8(const dr_bf16* router_w, const float* nw, float eps, int e, const uint8_t* gu_w,
                                  const float* gu_s, const uint8_t* d_w, const float* d_s, const int8_t* sgu_q,
                                  const dr_half* sgu_s, const int8_t* sd_q, const dr_half* sd_s, const float* x,
                                  float* logits, int* idx, float* wts, float* sgate, uint32_t* counter,
                                  uint64_t* tags, const float* res, float* act, float* y, int rows, int h, int i,
                                  int topk, dr_stream_t st);
int dr_moe_decode_rows_routed_fp8_bf16s(const dr_bf16* router_w, const float* nw, float eps, int e,
                                        const uint8_t* gu_w, const dr_bf16* gu_s, const uint8_t* d_w,
                                        const dr_bf16* d_s, const int8_t* sgu_q, const dr_bf16* sgu_s,
                                        const int8_t* sd_q, const dr_bf16* sd_s, const float* x, float* logits,
                                        int* idx, float* wts, float* sgate, uint32_t* counter, uint64_t* tags,
                                        const float* res, float* act, float* y, dr_bf16* yb, int rows, int h,
                                        int i, int topk, dr_stream_t st);

/* Single int4 GEMV (benchmark configuration 1): y[n] = sum_k (q[n,k] scale + min) x[k] with
 * x bf16, bf16 (scale, min) pairs per 64-group, fp32 accumulation; y f32 and (nullable) yb
 * bf16.  Unsupported: k % 2048 != 0 or k > 8192 -> -1. */
int dr_gemv_q4_bf16s(const uint8_t* q, const dr_bf16* sm, const dr_bf16* x, float* y, dr_bf16* yb, int n, int k,
                     dr_stream_t st);

/* int8 GEMV with a per-row bf16 scale (lm_head / projections of configuration 5):
 * y[n] = s[n] * sum_k q[n, k] xn[k] (+ res[n]), xn = RMSNorm(x; nw). */
int dr_gemv_q8_bf16s(const int8_t* w, const dr_bf16* s, const float* x, const float* res, float* y, int n,
                     int k, const float* nw, float eps, dr_stream_t st);

/* ===================================================================================== */
/* Fused multi-layer decode step (persistent kernel) -- no single reference symbol: it    */
/* replaces the per-layer chain dr_router_topk + dr_moe_decode that src/engine.rs:1001-   */
/* 1007 records for every MoE layer of a decode step (src/ffi.rs:41-46).                  */
/* ===================================================================================== */

/* Per-layer weight pointers, an array of n_layers of these in DEVICE memory.  Formats as in
 * dr_moe_decode (reference: f16 scales, int8 group 128) or dr_moe_decode_bf16s (bf16 scales,
 * per-channel int8 scales); router is the bf16 [E+1, H] matrix whose row E is the
 * shared-expert gate; nw is the RMSNorm weight (+1 folded in) or NULL for no norm. */
typedef struct dr_decode_layer {
  const dr_bf16* router;
  const float* nw;
  const uint8_t* gu_q;
  const void* gu_s;
  const uint8_t* d_q;
  const void* d_s;
  const int8_t* sgu_q;
  const uint16_t* sgu_s;
  const int8_t* sd_q;
  const uint16_t* sd_s;
} dr_decode_layer;

/* 64-bit words of the exchange buffer `ll` of dr_moe_decode_step*. */
#define DR_STEP_LL_WORDS 6920

/* One token through n_layers MoE layers in one launch (h = 2048, i = 512, topk = 8,
 * 8 <= e <= 256, 1 <= n_layers <= 1365):  for each layer, x = x + MoE(RMSNorm(x)) with the
 * same router, top-k, expert and shared-expert arithmetic as dr_router_topk followed by
 * dr_moe_decode(x, res = x, y = x); routing is bit-exact with that chain.
 *   x         f32 [h], read at launch and overwritten with the last layer's output;
 *   ll        u64 [DR_STEP_LL_WORDS] exchange buffer, sync u32 [4]: both zeroed once by the
 *             caller before the first call and then left alone (a call advances sync[0] and
 *             sync[2], and records its activation transport in sync[3]);
 *             sync[1] != 0 reports that a call timed out waiting for its workgroups: that call
 *             leaves NaN in x (every block that gives up overwrites all of x with NaN; a block
 *             that completed its last layer may still store its own rows afterwards) and raises
 *             DR_ERR_STEP_TIMEOUT,
 *             which dr_stream_sync reports and dr_last_error returns and clears; until then the
 *             step launchers return DR_ERR_STEP_TIMEOUT, and calls made before the caller zeroes
 *             sync and ll again give up at once (NaN x, the error raised again);
 *   idx_out i32 [n_layers*8], wts_out f32 [n_layers*8], sgate_out f32 [n_layers],
 *   xs_out f32 [n_layers*h]: optional (NULL) per-layer routing and layer outputs;
 *   pf/pf_bytes: a range the step warms in the memory-side cache after its last layer (the
 *             next op's weights, as dr_moe_decode's pf; the prefetch chain of
 *             src/engine.rs:674-708), NULL / 0 for none.
 * Needs 256 co-resident workgroups of 512 threads (one MI355X); returns -1 otherwise.  Calls
 * sharing one ll/sync pair must be stream ordered. */
int dr_moe_decode_step(const dr_decode_layer* layers, int n_layers, float* x, int e, int h, int i, int topk,
                       float eps, uint64_t* ll, uint32_t* sync, int* idx_out, float* wts_out, float* sgate_out,
                       float* xs_out, const char* pf, size_t pf_bytes, dr_stream_t st);
int dr_moe_decode_step_bf16s(const dr_decode_layer* layers, int n_layers, float* x, int e, int h, int i,
                             int topk, float eps, uint64_t* ll, uint32_t* sync, int* idx_out, float* wts_out,
                             float* sgate_out, float* xs_out, const char* pf, size_t pf_bytes, dr_stream_t st);
/* Transport of the routed activations between the fused step's workgroups, for later launches.
 * 30 (default; 0 restores it) packs two fp32 per slot with the exchange phase in the two low
 * mantissa bits of each: the activations reach the down projection rounded to 21 mantissa bits
 * (relative error <= 2^-22, an order below the fp32 rounding of the 2048-term dots that produce
 * them), with half the exchange traffic.  32 carries every activation as a full fp32 with a
 * 32-bit phase tag, as the reference's act buffer (kernels/drama.cu:493,516).  Other values ->
 * -1.  The step keeps a running layer count in sync[2]. */
int dr_step_set_act_exchange(int bits);

/* Wait limit of the fused step's exchanges in microseconds (0 restores the default, 200000).
 * A call whose workgroups are not all resident within the limit (another kernel holding CUs)
 * gives up: x becomes NaN, sync[1] is set and DR_ERR_STEP_TIMEOUT is raised.  For tests that
 * force that path from the host. */
int dr_step_set_wait_limit(uint32_t us);

/* The same step with block-FP8 routed experts: per layer gu_q/d_q are the e4m3 weights and
 * gu_s/d_s their 128 x 128 block scales of dr_moe_decode_fp8 (f32 scale_inv, int8 shared
 * scales f16 per 128) or of dr_moe_decode_fp8_bf16s (bf16 block scales, bf16 per-channel
 * shared scales); everything else as dr_moe_decode_step.  No reference counterpart: the
 * reference decodes FP8 layers with dr_router_topk + dr_moe_decode_fp8 per layer
 * (kernels/drama.cu:602-742), which these replace for a whole stack of layers. */
int dr_moe_decode_step_fp8(const dr_decode_layer* layers, int n_layers, float* x, int e, int h, int i, int topk,
                           float eps, uint64_t* ll, uint32_t* sync, int* idx_out, float* wts_out, float* sgate_out,
                           float* xs_out, const char* pf, size_t pf_bytes, dr_stream_t st);
int dr_moe_decode_step_fp8_bf16s(const dr_decode_layer* layers, int n_layers, float* x, int e, int h, int i,
                                 int topk, float eps, uint64_t* ll, uint32_t* sync, int* idx_out, float* wts_out,
                                 float* sgate_out, float* xs_out, const char* pf, size_t pf_bytes, dr_stream_t st);

/* ===================================================================================== */
/* Entry point that allocates nothing -- no counterpart in the reference.                 */
/* ===================================================================================== */

/* dr_moe_decode_step_bf16s without the caller's ll/sync buffers, for callers that cannot
 * allocate (code under graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The exchange buffer and sync words are a file-scope device array of 55,376 bytes, one per
 * GPU, held until the process ends; each call clears it first (a fill kernel on st) and calls
 * no allocator.  Calls that overlap on one GPU share the array and race: stream-order them.
 * Same shapes and limits as dr_moe_decode_step_bf16s (n_layers <= 1365, else -1). */
int dr_moe_decode_step_bf16s_noalloc(const dr_decode_layer* layers, int n_layers, float* x, int e, int h, int i,
                                     int topk, float eps, int* idx_out, float* wts_out, float* sgate_out,
                                     float* xs_out, const char* pf, size_t pf_bytes, dr_stream_t st);

#ifdef __cplusplus
}
#endif
#endif

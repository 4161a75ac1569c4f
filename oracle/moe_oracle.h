/*
 * CPU oracle for the drama-rs routed-expert MoE path.  TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C restatement of the reference algorithm (apiplant/drama-rs,
 * kernels/drama.cu, tools/reference.py, tools/convert.py).  Only the test suite,
 * __graft_entry__.smoke() and the cpu_baseline leg of bench.py may load it, and only as
 * the checker or the timed CPU baseline.  The product library (libdramamoe.so) never
 * links, includes or calls anything here.
 *
 * Two kinds of functions:
 *   - bit-exact contract functions (router logits, RMSNorm, softmax/top-k, grouping):
 *     they fix one canonical fp32 operation order that the gfx950 kernels follow too,
 *     so routing indices and weights can be compared bit for bit;
 *   - value functions (dequant, GEMV, decode layer, prefill layer): dequantise then
 *     accumulate in double, the "dequant-then-fp32" semantics of tools/reference.py:331-351
 *     evaluated more accurately than fp32, so GPU results are compared with a tolerance.
 *
 * Layouts follow the reference: int4 q u8 [N, K/2] (low nibble = even k), scale/min
 * pairs [N, K/64, 2] (src/model.rs:31-43, tools/convert.py:92-110); int8 q i8 [N, K] with
 * one scale per `group` inputs of a row (src/model.rs:16-29); fp8 e4m3 [N, K] with one
 * scale per 128x128 block (kernels/drama.cu:602-604).  Half-precision values are passed as
 * raw uint16_t bits.
 */
#ifndef DRAMA_MOE_ORACLE_H
#define DRAMA_MOE_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* scale encodings */
enum { OR_F16 = 0, OR_BF16 = 1, OR_F32 = 2 };

/* ---- scalar conversions (IEEE round-to-nearest-even) ---- */
float or_bf16_to_f32(uint16_t h);
uint16_t or_f32_to_bf16(float f);
float or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);
float or_fp8e4m3_to_f32(uint8_t v);
uint8_t or_f32_to_fp8e4m3(float f);
float or_exp(float x);
void or_exp_array(const float* x, float* y, size_t n);

/* ---- bit-exact router contract ---- */
void or_rmsnorm_canon(const float* x, const float* nw, float eps, int K, float* xn);
float or_dot_bf16_canon(const uint16_t* w, const float* x, int K);
void or_router_logits(const uint16_t* W, const float* xn, int rows, int K, float* logits);
int or_softmax_topk(const float* l, int E, int topk, int* idx, float* wts);
int or_router_topk(const uint16_t* W, const float* x, const float* nw, float eps, float* logits, int E,
                   int topk, int K, int* idx, float* wts, float* sgate);
int or_moe_topk(const float* logits, int rows, int E, int topk, int stride, int* idx, float* wts,
                float* sgate);
int or_router_logits_rows(const uint16_t* A, const uint16_t* W, float* C, int M, int N, int K);

/* ---- grouping (stable counting sort) ---- */
int or_moe_group(const int* idx, int n, int E, int* counts, int* offsets, int* slot_of);

/* ---- dequantisation ---- */
void or_dequant_q4(const uint8_t* q, const uint16_t* sm, int sm_kind, int N, int K, float* w);
void or_dequant_q8(const int8_t* q, const uint16_t* s, int s_kind, int group, int N, int K, float* w);
void or_dequant_fp8(const uint8_t* w8, const void* s, int s_kind, int N, int K, float* w);
void or_quant_q8(const float* w, int N, int K, int8_t* q, uint16_t* s);

/* ---- value functions ---- */
void or_gemv_q4(const uint8_t* q, const uint16_t* sm, int sm_kind, const float* x, int N, int K, float* y);
void or_gemv_q8(const int8_t* q, const uint16_t* s, int s_kind, int group, const float* x, int N, int K,
                float* y);

/* Weight formats of one MoE layer.  kind: 0 = int4 (group 64), 1 = fp8 e4m3 (128x128 blocks).
 * For int4, sc points at the [E, N, K/64, 2] scale/min pairs, sc_kind OR_F16 | OR_BF16.
 * For fp8, sc points at [E, N/128, K/128] block scales, sc_kind OR_F32 | OR_BF16.
 * The shared expert is int8 with one scale per sh_group inputs (128, or K for per-channel). */
typedef struct {
  int kind;
  const uint8_t* gu_q;
  const void* gu_s;
  const uint8_t* d_q;
  const void* d_s;
  int sc_kind;
  const int8_t* sgu_q;
  const uint16_t* sgu_s;
  const int8_t* sd_q;
  const uint16_t* sd_s;
  int sh_kind;
  int sh_group_gu; /* group along K = H for shared gate_up (128 or H) */
  int sh_group_d;  /* group along K = I for shared down (128 or I) */
} or_moe_weights;

/* fp32 host baseline of one int4 decode layer (cpu_baseline.c; bench.py's cpu_baseline leg) */
int or_cpu_layer_f32(const or_moe_weights* w, const uint16_t* router, const float* nw, float eps, const float* x,
                     const float* res, float* y, int E, int H, int I, int topk, int* idx, float* wts);
int or_moe_decode(const or_moe_weights* w, const float* x, const int* idx, const float* wts,
                  const float* sgate, const float* res, float* act, float* y, int H, int I, int topk,
                  const float* nw, float eps);
int or_moe_decode_rows(const or_moe_weights* w, const float* xn_rows, int rows, const int* idx,
                       const float* wts, const float* sgate, float* y, int H, int I, int topk);
int or_moe_prefill_layer(const or_moe_weights* w, const uint16_t* hn_b, int rows, const int* idx,
                         const float* wts, const float* sgate, float* x, int H, int I, int topk);
int or_moe_prefill_experts(const or_moe_weights* w, const uint16_t* xp, const int* offsets,
                           const int* counts, int E, uint16_t* act, float* yp, int H, int I);
int or_shared_prefill(const or_moe_weights* w, const uint16_t* hn_b, int rows, uint16_t* act, float* out,
                      int H, int I);

int or_num_threads(void);
void or_set_threads(int n);

#ifdef __cplusplus
}
#endif
#endif

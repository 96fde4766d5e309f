/* wzy_oracle.h -- CPU oracle for the MI355X decode path.  TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's arithmetic (liaoyangr8-ai/wzy-flash-serve) for every
 * function on the per-token decode path.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, and only as the checker (or, for cpu_moe_pool.cpp, as the timed
 * CPU baseline); the product library never links it.
 *
 * Conventions: shapes are runtime arguments; reductions accumulate in double and round once (the
 * reference accumulates in fp32 in a device-specific order, so float parity is tolerance based);
 * every rounding step that changes a discrete result (int8 quantisation, fp16/bf16 rounding,
 * e2m1/e4m3 decode, tie rules) is restated exactly as the reference does it.
 *
 * Pinning (see tests/test_oracle_*.py): e2m1/e4m3/fp16/bf16 decodes against torch/numpy dtype
 * conversions and the OCP MX spec values; NVFP4 GEMVs against a float64 dequantise-then-matmul
 * formulation; top-k/argmax against numpy sorts; GDN against the delta-rule closed forms; QSA
 * selection against brute-force sorting with the restated tie rule.
 */
#ifndef WZY_ORACLE_H
#define WZY_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- formats (src/wzy_stage_v2.cuh:181-195) ---- */
int orc_e2m1x2(int code);                 /* 2*value of an e2m1 nibble as int */
float orc_ue4m3_half(int code);           /* unsigned e4m3 (sign ignored) * 0.5 */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);         /* round to nearest even */
float orc_bf16_to_f32(uint16_t h);
size_t orc_blob_bytes(int D, int F);      /* reference expert blob size (PER) */

/* ---- activation quantisation (src/wzy_kernels_v2.cuh:58-107) ---- */
void orc_quant_act(const float* x, int cols, int T, int8_t* q32, float* s32, int8_t* q16, float* s16);

/* ---- dense GEMVs ---- */
/* Q8_0 (src/wzy_kernels_v2.cuh:120-159) */
void orc_gemv_q8(const int8_t* codes, const uint16_t* scales, const int8_t* xq, const float* xs, float* y,
                 int rows, int cols, int T);
/* bf16 x fp32 (src/wzy_kernels_v2.cuh:307-337) */
void orc_gemv_bf16(const uint16_t* W, const float* x, float* y, int rows, int cols, int T);

/* ---- router (src/wzy_kernels_v2.cuh:989-1090) ----
 * probs_out [T x E] (optional) receives the fp32 softmax probabilities the selection ran on. */
void orc_router_topk(const float* logits, int E, int K, int T, int* ids, float* wts, float* probs_out);

/* ---- NVFP4 experts, reference blob layout ---- */
/* gate/up + SwiGLU + per-16 requant for one routed entry (src/wzy_kernels_v2.cuh:1583-1721).
 * act_out (optional) receives the fp32 SwiGLU activation before requantisation. */
void orc_expert_gate_up(const uint8_t* blob, int D, int F, const int8_t* xq16, const float* xs16, int8_t* aq16,
                        float* as16, float* act_out);
/* down projection of one routed entry (src/wzy_kernels_v2.cuh:1725-1834) */
void orc_expert_down(const uint8_t* blob, int D, int F, const int8_t* aq16, const float* as16, float* out);

typedef struct orc_moe_weights {
    int n_embd, n_ff, n_exp, top_k;
    const uint16_t* router;              /* bf16 [E x D] */
    const uint16_t* sgate;               /* bf16 [D] */
    const uint8_t* const* blobs;         /* E pointers to reference-layout blobs (NULL = not materialised) */
    const int8_t* sh_gate_q; const uint16_t* sh_gate_s;
    const int8_t* sh_up_q;   const uint16_t* sh_up_s;
    const int8_t* sh_down_q; const uint16_t* sh_down_s;
} orc_moe_weights;

/* Full MoE block (src/wzy_stage_v2.cuh:697-724): returns 0, or -1 if a routed blob is NULL.
 * logits_out [T x E], sg_out [T] optional. */
int orc_moe_block(const orc_moe_weights* w, const float* x, int T, float* comb, int* ids, float* wts,
                  float* logits_out, float* sg_out);

/* ---- logit reductions (src/wzy_kernels_v2.cuh:1873-1984) ---- */
void orc_row_argmax(const float* logits, int nvocab, int T, int* out);
void orc_row_top16(const float* logits, int nvocab, int T, int* greedy, float* top_v, int* top_i);

/* ---- CPU baseline: restatement of the reference CpuMoePool (oracle/cpu_moe_pool.cpp) ----
 * All T*K routed entries are treated as cold.  Returns 0 on success. */
typedef struct orc_cpu_pool orc_cpu_pool;
orc_cpu_pool* orc_cpu_pool_create(int n_threads, int D, int F);
void orc_cpu_pool_destroy(orc_cpu_pool* p);
int orc_cpu_pool_threads(const orc_cpu_pool* p);
/* Routed-expert output sum_k w_k * expert_k(x) for T rows (no shared expert), like
 * CpuMoePool::run (src/wzy_cpu_moe.cuh:590-614); xq16/xs16 are per-16 activations [T x D]. */
int orc_cpu_pool_run(orc_cpu_pool* p, const uint8_t* const* blobs, const int* ids, const float* wts, int T, int K,
                     const int8_t* xq16, const float* xs16, float* out);

#ifdef __cplusplus
}
#endif
#endif /* WZY_ORACLE_H */

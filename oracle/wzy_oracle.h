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
/* Same, fetching blobs that w->blobs does not hold (or all, when w->blobs is NULL) from blob_fn. */
typedef const uint8_t* (*orc_blob_fn)(void* ctx, int layer, int expert);
int orc_moe_block_fn(const orc_moe_weights* w, const float* x, int T, float* comb, int* ids, float* wts,
                     float* logits_out, float* sg_out, orc_blob_fn blob_fn, void* blob_ctx, int layer);

/* Prefill MoE block with bf16 numerics (see orc_core.c); needs every routed blob in w->blobs.
 * Returns 0, or -1 if a routed blob is NULL. */
int orc_moe_prefill(const orc_moe_weights* w, const float* x, int T, float* comb, int* ids, float* wts);
/* Same, fetching blobs that w->blobs does not hold from blob_fn (layer `layer`); logits_out [T x E]
 * (optional) receives the router logits. */
int orc_moe_prefill_fn(const orc_moe_weights* w, const float* x, int T, float* comb, int* ids, float* wts,
                       float* logits_out, orc_blob_fn blob_fn, void* blob_ctx, int layer);

/* ---- hyper-connection read (src/wzy_kernels_v2.cuh:409-454,632-827): see orc_layers.c ---- */
void orc_hc_read(const float* R_in, const float* emb_rows, const float* bo, const float* inj_prev, const float* norm_w,
                 const int8_t* down_q, const uint16_t* down_s, const uint16_t* inj_w, const int8_t* up_q,
                 const uint16_t* up_s, int D, int HC, int HCLR, float eps, int T, float* R_out, float* nsc, float* lo,
                 float* inj, float* mixed);

/* ---- GDN (src/wzy_kernels_v2.cuh:833-984); state S[h][i][j] ---- */
void orc_gdn_step(const float* qkv_raw, const float* z, const float* ab_raw, const float* dt, const float* ssm_a,
                  const float* conv_w, float* conv_hist, float* state, const float* gamma, float eps, float* y, int hk,
                  int hv, int T);
void orc_gdn_recurrence(const float* q, const float* k, const float* v, const float* decay, const float* beta,
                        const float* z, const float* gamma, float eps, float* state, float* y, int hk, int hv, int T);

/* ---- QSA (src/wzy_qsa_256k.cuh, src/wzy_qsa_wmma.cuh) ---- */
void orc_rope_tables(int ctx, int n_rot, float theta, float* cos_tab, float* sin_tab);
void orc_head_norm_rope(float* p, int hd, const float* gamma, const float* cos_tab, const float* sin_tab, int pos,
                        int n_rot, float eps);
void orc_kv_quant_row(const float* x, int n, int8_t* q, uint16_t* s);
void orc_indexer_append(const float* raw, const float* gamma, const float* cos_tab, const float* sin_tab, int pos,
                        int dim, int blk, int n_rot, float eps, float* tail, float* dead, uint16_t* pooled);
void orc_indexer_append_f32(const float* raw, const float* gamma, const float* cos_tab, const float* sin_tab, int pos,
                            int dim, int blk, int n_rot, float eps, float* tail, float* dead, uint16_t* pooled,
                            float* key_out);
void orc_block_scores(const uint16_t* pooled, const float* dead, const float* q_idx, int n_kv, int heads, int dim,
                      int blk, float* scores);
int orc_topk_select(const float* scores, int n_kv, int blk, int topk, int* sel);
void orc_attend(const float* qg, const int8_t* kq, const uint16_t* ks, const int8_t* vq, const uint16_t* vs,
                const int* sel, int n, int qh, int kvh, int hd, float* out);

/* ---- whole decode window (StageGpu::record_forward with the head, src/wzy_stage_v2.cuh:476-857) ---- */
typedef struct orc_layer {
    int qsa;
    const float* hc_norm[2];
    const int8_t* hc_down_q[2]; const uint16_t* hc_down_s[2];
    const int8_t* hc_up_q[2];   const uint16_t* hc_up_s[2];
    const uint16_t* hc_inj[2];
    /* GDN */
    const int8_t* qkv_q;   const uint16_t* qkv_s;
    const int8_t* wgate_q; const uint16_t* wgate_s;
    const int8_t* wout_q;  const uint16_t* wout_s;
    const uint16_t* alpha; const uint16_t* beta;
    const float* ssm_a; const float* dt; const float* conv_w; const float* ssm_norm;
    float* conv_hist; float* ssm;                       /* state, updated */
    /* QSA */
    const int8_t* wq_q; const uint16_t* wq_s; const int8_t* wk_q; const uint16_t* wk_s;
    const int8_t* wv_q; const uint16_t* wv_s; const int8_t* wo_q; const uint16_t* wo_s;
    const float* q_norm; const float* k_norm;
    const uint16_t* idx_q; const uint16_t* idx_k; const float* idx_qn; const float* idx_kn;
    int8_t* kq; uint16_t* ks; int8_t* vq; uint16_t* vs;  /* KV store [ctx_max x kvd], updated */
    float* idx_tail; float* idx_dead; uint16_t* idx_pooled;  /* indexer state, updated */
    /* MoE (expert blobs come from the model's blob_fn) */
    const uint16_t* router; const uint16_t* sgate;
    const int8_t* sh_gate_q; const uint16_t* sh_gate_s; const int8_t* sh_up_q; const uint16_t* sh_up_s;
    const int8_t* sh_down_q; const uint16_t* sh_down_s;
} orc_layer;

/* PLE weights, table access and state of a model whose layer 1 carries the per-layer embedding
 * (orc_ple.c; NULL in orc_model: no PLE, the BASELINE synthetic model) */
typedef const uint8_t* (*orc_ple_row_fn)(void* ctx, uint32_t row);   /* the table row's head bytes */
typedef struct orc_ple_w {
    orc_ple_row_fn row; void* row_ctx;      /* fp8 table rows (16 heads x head bytes per token) */
    float scale; int eos;                   /* table scale (strata.ple.scale), end-of-sequence id */
    const uint16_t* wk; const uint16_t* wv; /* bf16 [HC*D x D], [D x D] */
    const float* norm_q; const float* norm_k; const float* norm_c;   /* [HC*D] */
    const float* conv_w;                    /* [HC*D x 4] */
    float* hist;                            /* [HC*D x 9] state */
    int* tok_hist;                          /* [ctx_max] token of each cell, written by every window */
} orc_ple_w;

typedef struct orc_model {
    int n_layers, n_embd, hc, hc_lr, gdn_hk, gdn_hv, qsa_qh, qsa_kvh, qsa_hd, n_rot;
    int idx_heads, idx_dim, idx_blk, idx_topk, n_exp, top_k, n_ff, n_vocab, ctx_max;
    float eps;
    orc_layer* layers;
    const uint16_t* emb; const float* head_norm;
    const int8_t* head_down_q; const uint16_t* head_down_s; const int8_t* head_up_q; const uint16_t* head_up_s;
    const uint16_t* head;
    const float* cos_tab; const float* sin_tab;
    orc_blob_fn blob; void* blob_ctx;
    /* Q8_0 token embedding / LM head (codes + fp16 per-32 scales), used instead of emb / head when
     * not NULL: the embedding row is d*q with an out-of-range id reading row 0 (stage_one_emb,
     * src/wzy_engine_v2.cu:861-873), the head is dense_q8 (src/wzy_stage_v2.cuh:804-815) */
    const int8_t* emb_q; const uint16_t* emb_s;
    const int8_t* head_q; const uint16_t* head_s;
    /* > 0: a window with pos + T > attn_f16_above attends through orc_attend_pf, the reference's GQA
     * kernel past its VRAM ring (KV_VRAM_RING = 32,768; src/wzy_stage_v2.cuh:679-683); 0 or below:
     * orc_attend (qsa_attend_int8_sparse_multi) at every context */
    int attn_f16_above;
    const orc_ple_w* ple;      /* per-layer embedding at layer 1, or NULL (src/wzy_stage_v2.cuh:583-597) */
} orc_model;

/* logits [T x n_vocab], greedy [T] and pre_head [T x hc x n_embd] (optional); returns 0 or -1. */
int orc_model_forward(const orc_model* m, int pos, const int* toks, int T, float* logits, int* greedy,
                      float* pre_head);
/* Same, also recording per layer l at dbg + l*4*T*n_embd (optional): the attention-half mixed
 * input, the attention block output, the FFN-half mixed input and the MoE output, each [T x n_embd];
 * and at margins + (l*T + t)*2 (optional) the discrete-decision margins of row t: the router logit
 * gap between the top_k-th and (top_k+1)-th expert, and the relative indexer score gap around the
 * top-k threshold block (1e30 when nothing is selected against). */
int orc_model_forward_dbg(const orc_model* m, int pos, const int* toks, int T, float* logits, int* greedy,
                          float* pre_head, float* dbg, float* margins);

/* Per-layer record of one window (every pointer optional):
 *   dbg [L][4][T][D]: attention HC read output, attention block, FFN HC read output, MoE output;
 *   margins [L][T][2]: router gap between the top_k-th and next logit, relative indexer score gap
 *   around the top-k threshold (1e30 when not applicable);
 *   router_logits [L][T][n_exp], ids / wts [L][T][top_k];
 *   per QSA layer q (layer order): scores [q][T][ctx_max/idx_blk + 2] (zero when the row selects
 *   every cell), sel [q][T][idx_topk], n_sel [q][T]. */
typedef struct orc_trace {
    float* dbg;
    float* margins;
    float* router_logits;
    int* ids;
    float* wts;
    float* scores;
    int* sel;
    int* n_sel;
} orc_trace;
int orc_model_forward_trace(const orc_model* m, int pos, const int* toks, int T, float* logits, int* greedy,
                            float* pre_head, const orc_trace* tr);

/* Decision margins: gap between the k-th and (k+1)-th largest of v[0..n) (1e30 if n <= k); relative
 * indexer score gap around the top-k threshold block of a row (1e30 when it selects every cell). */
float orc_kth_gap(const float* v, int n, int k);
float orc_select_margin(const float* scores, int n_kv, int blk, int topk);

/* ---- chunked prefill (PrefillStageCtx::run_stage_prefill, src/wzy_prefill_tc.cuh:546-1058): see
 * orc_prefill.c for the operand roundings ---- */
/* y[t*ldy + n] = sum_k A[t][k] * W[n][k]: A bf16-valued [M x K], W Q8_0 (q, s; rounded to bf16) or bf16 (wb) */
void orc_pf_gemm(const float* A, int M, int K, const int8_t* q, const uint16_t* s, const uint16_t* wb, int N,
                 float* y, int ldy);
/* HC read of B rows (R [B][HC][D] updated in place with the pending block bo/inj_prev when bo != NULL) */
void orc_hc_read_pf(float* R, const float* bo, const float* inj_prev, const float* norm_w, const int8_t* down_q,
                    const uint16_t* down_s, const uint16_t* inj_w, const int8_t* up_q, const uint16_t* up_s, int D,
                    int HC, int HCLR, float eps, int B, float* inj, float* mixed);
void orc_hc_write(float* R, const float* blk, const float* inj, int D, int HC, int B);
/* sparse GQA attention of one row with the prefill kernel's fp16 operands and 32-cell softmax steps */
void orc_attend_pf(const float* qg, const int8_t* kq, const uint16_t* ks, const int8_t* vq, const uint16_t* vs,
                   const int* sel, int n, int qh, int kvh, int hd, float* out);
/* B prompt cells at positions pos .. pos+B-1 through every layer, updating the model's state; R_out
 * [B][hc][n_embd] receives the final residual (the last MoE block written in); dbg (optional)
 * [L][4][B][n_embd] as in orc_model_forward_dbg.  Returns 0, or -1. */
int orc_model_prefill(const orc_model* m, int pos, const int* toks, int B, float* R_out, float* dbg);
/* Same, also writing margins [L][B][2] (optional): the router logit gap between the top_k-th and
 * next expert, and the relative indexer score gap around the top-k threshold (1e30 when the row
 * selects every cell or the layer is GDN), as orc_model_forward_dbg. */
int orc_model_prefill_dbg(const orc_model* m, int pos, const int* toks, int B, float* R_out, float* dbg,
                          float* margins);

/* ---- MTP drafter (src/wzy_mtp.cuh) ---- */
/* Q2_0 expert blob size: 3*D*F/4 code bytes + 3*D*F/64 fp16 scales (src/wzy_mtp.cuh:6-10) */
size_t orc_q2_blob_bytes(int D, int F);
int orc_q2_code(const uint8_t* codes, int k);
/* per-32 activations in, per-32 SwiGLU activations out (src/wzy_mtp.cuh:85-158) */
void orc_q2_expert_gate_up(const uint8_t* blob, int D, int F, const int8_t* xq32, const float* xs32, int8_t* aq32,
                           float* as32, float* act_out);
/* src/wzy_mtp.cuh:160-207 */
void orc_q2_expert_down(const uint8_t* blob, int D, int F, const int8_t* aq32, const float* as32, float* out);

typedef struct orc_mtp {
    int n_embd, hc, hc_lr, qsa_qh, qsa_kvh, qsa_hd, n_rot, n_exp, top_k, n_ff, n_vocab, n_dv, ring;
    float eps;
    const uint16_t* emb;                        /* bf16 [n_vocab x D] (the main model's table) */
    const float* pre_norm_emb;                  /* [D] */
    const float* pre_norm_hid;                  /* [hc x D] */
    const int8_t* fc_emb_q; const uint16_t* fc_emb_s;
    const int8_t* fc_hid_q; const uint16_t* fc_hid_s;
    /* hyper-connections: 0 attention, 1 MLP, 2 final mixer (no inject weight) */
    const float* hc_norm[3];
    const int8_t* hc_down_q[3]; const uint16_t* hc_down_s[3];
    const int8_t* hc_up_q[3];   const uint16_t* hc_up_s[3];
    const uint16_t* hc_inj[2];
    const int8_t* wq_q; const uint16_t* wq_s; const int8_t* wk_q; const uint16_t* wk_s;
    const int8_t* wv_q; const uint16_t* wv_s; const int8_t* wo_q; const uint16_t* wo_s;
    const float* q_norm; const float* k_norm;
    const uint16_t* router; const uint16_t* sgate;
    const int8_t* sh_gate_q; const uint16_t* sh_gate_s; const int8_t* sh_up_q; const uint16_t* sh_up_s;
    const int8_t* sh_down_q; const uint16_t* sh_down_s;
    const uint8_t* experts;                     /* n_exp Q2_0 blobs back to back */
    const int8_t* head_q; const uint16_t* head_s; /* Q8_0 draft head [n_dv x D] */
    const int* dvocab;                          /* [n_dv] token ids (NULL = identity) */
    const float* cos_tab; const float* sin_tab;
    /* state, updated: INT8 KV ring [ring x kvd] with fp16 per-64 scales, attention floor */
    int8_t* kq; uint16_t* ks; int8_t* vq; uint16_t* vs;
    int kv_floor;
    const int8_t* emb_q; const uint16_t* emb_s;  /* Q8_0 main embedding table, used instead of emb when not NULL */
} orc_mtp;

/* K/V append of T cells pos..pos+T-1 (src/wzy_mtp.cuh:658-683).  toks [T] are the embedded tokens,
 * Rin [T x hc x D] the residuals; R [T x hc x D], mixed [T x D], inj [T x hc] receive the front's
 * outputs. */
void orc_mtp_front(orc_mtp* m, int pos, const int* toks, const float* Rin, int T, float* R, float* mixed, float* inj);
/* One chained draft step at cell pos (src/wzy_mtp.cuh:687-733): R_out [hc x D] is the next step's
 * residual, sample [D] the draft head input, logits [n_dv]. */
int orc_mtp_step(orc_mtp* m, int pos, int tok, const float* Rin, float* R_out, float* sample, float* logits,
                 int* out_tok, float* out_prob);

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

/* ---- per-layer embedding at layer 1 (src/wzy_engine_v2.cu:909-978; src/wzy_stage_v2.cuh:215-324,583-597;
 *      src/wzy_kernels_v2.cuh:1299-1374); orc_ple.c ---- */
#define ORC_PLE_HEADS 16
uint64_t orc_ple_table_rows(void);
void orc_ple_row_ids(int cur, int prev1, int prev2, int eos, uint32_t* rows);
float orc_ple_fp8(uint8_t v, float scale);
void orc_ple_rows(orc_ple_row_fn row, void* ctx, int head, float scale, int eos, const int* toks, int T, int pos,
                  int* tok_hist, float* out);
void orc_ple_block(float* R, const float* bo, const float* inj_prev, const float* emb, const uint16_t* wk,
                   const uint16_t* wv, const float* norm_q, const float* norm_k, const float* norm_c,
                   const float* conv_w, float* hist, int D, int HC, float eps, int T, int emb_bf16,
                   float* hist_snaps);

#ifdef __cplusplus
}
#endif
#endif /* WZY_ORACLE_H */

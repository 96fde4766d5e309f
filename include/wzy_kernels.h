/* wzy_kernels.h -- kernel-level C ABI of the MI355X (gfx950) decode path.
 *
 * Every entry point enqueues hand-written HIP kernels on `stream` (a hipStream_t passed as void*,
 * NULL = the null stream) and returns a status code: WZY_OK (0) or a negative WZY_E* value, with a
 * message available from wzy_last_error().  All data pointers are DEVICE pointers unless stated
 * otherwise; no call synchronizes or takes ownership, and none allocates device memory except
 * wzy_row_argmax / wzy_row_top16 (a per-device scratch, allocated on first use) and the measurement
 * calls wzy_moe_time_kernels and wzy_gdn_time_recurrence (each allocates and frees a scratch of its
 * own per call; the measurement calls also synchronize).
 *
 * Each function names the reference interface it replaces (reference = liaoyangr8-ai/wzy-flash-serve,
 * paths relative to its root).  The reference exposes these as `launch_*` helpers or bare
 * `__global__` kernels compiled into the engine; here they are a stable C ABI so a host written in
 * any language can drive the same kernels.
 *
 * Shapes are runtime parameters (the reference fixes them at compile time,
 * src/wzy_kernels_v2.cuh:8-19).  T is the number of window rows (1..WZY_MAX_W).
 */
#ifndef WZY_KERNELS_H
#define WZY_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WZY_OK 0
#define WZY_EINVAL (-1)   /* bad argument / unsupported shape */
#define WZY_EHIP (-2)     /* HIP runtime error */
#define WZY_ENOMEM (-3)   /* device allocation failed */
#define WZY_ESTATE (-4)   /* call not valid in the current state */
#define WZY_EIO (-5)      /* file / parse error */

#define WZY_MAX_W 8       /* verify-window rows, reference MAX_W (src/wzy_kernels_v2.cuh:13) */

/* Last error message of the calling thread ("" if none). */
const char* wzy_last_error(void);
/* Library version string. */
const char* wzy_version(void);

/* ---------------------------------------------------------------------------------------------
 * Activation quantisation
 * ------------------------------------------------------------------------------------------- */

/* Per-16 and/or per-32 symmetric int8 quantisation of T rows of `cols` floats
 * (d = amax/127, q = rint(x * 127/amax) clamped to +-127, zero block -> q = 0, d = 0).
 * Any of the (q, s) output pairs may be NULL.  cols % 32 == 0.
 * Replaces quant_act_multi (src/wzy_kernels_v2.cuh:58-107). */
int wzy_quant_act(const float* x, int8_t* q32, float* s32, int8_t* q16, float* s16,
                  int cols, int T, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Dense GEMVs (T rows of activations share one pass over the weights)
 * ------------------------------------------------------------------------------------------- */

/* Q8_0 GEMV: y[t*y_stride + r] = sum_b fp16(scales[r,b]) * xs[t,b] * sum_{i<32} codes[r,32b+i]*xq[t,32b+i].
 * codes int8 [rows x cols], scales fp16 bits [rows x cols/32], xq/xs from wzy_quant_act (per-32).
 * cols % 32 == 0; y_stride == 0 means rows.
 * Replaces launch_gemm_q8p / gemm_q8p_t (src/wzy_kernels_v2.cuh:120-159,230-303). */
int wzy_gemv_q8(const int8_t* codes, const uint16_t* scales, const int8_t* xq, const float* xs,
                float* y, int rows, int cols, int T, int y_stride, void* stream);

/* bf16 x fp32 GEMV: y[t*y_stride + r] = sum_c bf16(W[r,c]) * x[t,c].  cols % 8 == 0.
 * Replaces launch_gemm_bf16 / gemm_bf16_t (src/wzy_kernels_v2.cuh:307-387). */
int wzy_gemv_bf16(const uint16_t* W, const float* x, float* y, int rows, int cols, int T,
                  int y_stride, void* stream);

/* One projection group in one launch: segment i computes y_i[t*y_stride_i + r] = W_i[r,:] . x[t,:]
 * over the same fp32 activations x [T x cols], with Q8_0 weights (kind WZY_GEMV_Q8: int8 codes
 * [rows x cols] and fp16 scale bits [rows x cols/32]; x quantised per 32 exactly as wzy_quant_act
 * does) or bf16 weights (kind WZY_GEMV_BF16, s = NULL).  1 <= n_segs <= 8, cols % 32 == 0,
 * 32 <= cols <= 8192, 1 <= T <= WZY_MAX_W; y_stride == 0 means rows.
 * Replaces a group's quant_act_multi + launch_gemm_q8p / launch_gemm_bf16 sequence
 * (src/wzy_stage_v2.cuh:609-611, 630-633, 449-460). */
#define WZY_GEMV_Q8 0
#define WZY_GEMV_BF16 1
typedef struct {
    const void* w;
    const uint16_t* s;
    float* y;
    int rows, kind, y_stride;
} wzy_gemv_seg;
int wzy_gemv_segs(const wzy_gemv_seg* segs, int n_segs, const float* x, int cols, int T, void* stream);

/* ---------------------------------------------------------------------------------------------
 * NVFP4 mixture of experts (decode)
 * ------------------------------------------------------------------------------------------- */

/* Device record of one NVFP4 expert ("plane layout", 16-byte aligned planes):
 *   [gate|up codes : 2*n_ff rows x n_embd/2 bytes][gate|up e4m3 scales : 2*n_ff rows x n_embd/16]
 *   [down codes    : n_embd rows x n_ff/2 bytes ][down e4m3 scales     : n_embd rows x n_ff/16  ]
 *   [tensor scales : fp32 gate, up, down, pad]
 * Row r of a matrix keeps the reference's nibble order: 64-value block b holds code bytes
 * 32b..32b+31, sub-block s (16 values) is bytes 32b+8s..+7, value k<8 is the low nibble of byte k,
 * value k>=8 the high nibble of byte k-8; scale byte 4b+s belongs to sub-block (b,s).
 * Same bytes as the reference's 36-byte-block blob (src/wzy_kernels_v2.cuh:15-16; PER), with the
 * 4 scale bytes of each block moved to a separate plane so code rows are 16-byte aligned. */
size_t wzy_nvfp4_expert_bytes(int n_embd, int n_ff);
/* Size of one expert in the reference blob layout (36-byte blocks + 16-byte tail). */
size_t wzy_nvfp4_blob_bytes(int n_embd, int n_ff);
/* Host-side repack of one reference-layout blob into the plane layout (host pointers).
 * Replaces the blob addressing of exp_gu_quant_grouped / exp_down_2r_grouped
 * (src/wzy_kernels_v2.cuh:1611-1613,1754-1757); used by loaders of experts.bin. */
int wzy_nvfp4_repack_host(const uint8_t* blob, uint8_t* planes, int n_embd, int n_ff);

/* One MoE layer's weights (device pointers). */
typedef struct wzy_moe_weights {
    int n_embd, n_ff, n_exp, top_k;
    const uint16_t* router;        /* bf16 [n_exp x n_embd]   (ffn_gate_inp)          */
    const uint16_t* sgate;         /* bf16 [n_embd]           (ffn_gate_inp_shexp)    */
    const uint8_t* experts;        /* n_exp records of wzy_nvfp4_expert_bytes()        */
    const int8_t* sh_gate_q;  const uint16_t* sh_gate_s;   /* Q8_0 [n_ff x n_embd]  */
    const int8_t* sh_up_q;    const uint16_t* sh_up_s;     /* Q8_0 [n_ff x n_embd]  */
    const int8_t* sh_down_q;  const uint16_t* sh_down_s;   /* Q8_0 [n_embd x n_ff]  */
} wzy_moe_weights;

/* Bytes of device workspace wzy_moe_block needs for T rows (n_embd <= 2048).  Calls that share a
 * workspace must not overlap. */
size_t wzy_moe_workspace_bytes(int n_embd, int n_ff, int n_exp, int top_k, int T);

/* Full decode MoE block for T rows of x [T x n_embd] (fp32):
 * router GEMV -> softmax top-k (ties to the lower expert id, weights renormalised by
 * max(sum, 2^-14)) -> grouped NVFP4 gate/up + SwiGLU + per-16 int8 requant -> NVFP4 down ->
 * comb = sigmoid(sgate.x) * shared(x) + sum_k w_k * expert_k(x)  (k in routed order).
 * Outputs: comb [T x n_embd]; ids [T x top_k] int32 and wts [T x top_k] fp32 if non-NULL.
 * Replaces the MoE section of StageGpu::record_forward (src/wzy_stage_v2.cuh:697-724):
 * quant_act_multi, gemm_bf16 router, router_top10_fast_multi, shared-expert Q8 GEMVs +
 * silu_mul_quant32_multi, exp_gu_quant_grouped, exp_down_2r_grouped, moe_combine_shared_multi. */
int wzy_moe_block(const wzy_moe_weights* w, const float* x, int T, float* comb, int* ids, float* wts,
                  void* workspace, size_t workspace_bytes, void* stream);

/* Dense projection of a prefill chunk on bf16 MFMA: y[m * ldy + n] = sum_k a[m * lda + k] * W[n][k]
 * for m < M, n < N, with a bf16 [M x lda] and W Q8_0 (wq codes [N x K] + ws fp16 scales [N x K/32],
 * each code * scale rounded to bf16) or bf16 (wb [N x K], wq NULL); fp32 accumulation; output fp32
 * (y) or rounded to bf16 (yb, y NULL).  K a multiple of 64, lda >= K a multiple of 8, ldy >= N.
 * Replaces the prefill's dequantise-then-cublasGemmEx pairs (dequant_q8p_to_fp16 /
 * bf16_to_fp16_vec + tc_gemm_fp16, src/wzy_prefill_tc.cuh:681-711; src/wzy_kernels_v2.cuh:1836-1865)
 * with bf16 operands. */
int wzy_gemm_bf16(const uint16_t* a, int lda, int M, int K, const int8_t* wq, const uint16_t* ws, const uint16_t* wb,
                  int N, float* y, uint16_t* yb, int ldy, void* stream);

/* Bytes of device workspace wzy_moe_prefill needs for a chunk of n_tok tokens. */
size_t wzy_moe_prefill_workspace_bytes(int n_embd, int n_ff, int n_exp, int top_k, int n_tok);

/* MoE block for a prefill chunk of n_tok rows of x [n_tok x n_embd] (fp32), on MFMA:
 * x rounded to bf16 -> router logits (bf16 GEMM) -> softmax top-k per token (the decode rule) ->
 * entries grouped by expert into tiles of up to 256 -> routed gate|up (NVFP4 dequantised to bf16
 * MFMA operands; the fp32 tensor scale applied to the accumulators) + SwiGLU (bf16) -> down, fp32
 * per entry -> comb = sigmoid(sgate.x) * shared(x) + sum_k w_k * expert_k(x), summed per token in
 * slot order (results do not depend on the order entries reach their expert); the shared expert's
 * Q8_0 weights are dequantised to bf16 (rounded).  n_embd a multiple of 256, n_ff a multiple of
 * 128, n_exp a multiple of 64 up to 1024, top_k in [1, min(32, n_exp)]; n_tok >= 1 (an empty chunk
 * is an error), n_tok * top_k <= 2^26 and n_tok * n_embd < 2^31.  ids / wts [n_tok x top_k] may be
 * NULL.  Shapes outside these limits return an error before anything is launched.
 * Replaces the prefill MoE of run_stage_prefill: pf_moe_count/scan/tile builders,
 * pf_moe_gu_wmma_kernel, pf_moe_down_wmma_kernel, pf_init_shared_comb_kernel and the router /
 * shared-expert dense GEMMs (src/wzy_prefill_tc.cuh:99-443), fp16 replaced by bf16. */
int wzy_moe_prefill(const wzy_moe_weights* w, const float* x, int n_tok, float* comb, int* ids, float* wts,
                    void* workspace, size_t workspace_bytes, void* stream);

/* Measurement: `iters` runs of wzy_moe_prefill (after one untimed run) with HIP events between
 * its launch groups on `stream`; us_stages[8] = mean microseconds of
 *   0 x -> bf16, 1 router GEMM, 2 routing + shared gate, 3 expert tiles and entry lists,
 *   4 shared gate|up, 5 shared down, 6 routed gate|up, 7 routed down + per-token combine.
 * Counterpart of the reference's WZY_PF_PROF phase timers (src/wzy_prefill_tc.cuh:734-741). */
int wzy_moe_prefill_time(const wzy_moe_weights* w, const float* x, int n_tok, float* comb, void* workspace,
                         size_t workspace_bytes, int iters, float* us_stages, void* stream);

/* Softmax top-k routing alone, over router logits [T x n_exp] (fp32): ids [T x top_k] in rank
 * order (probability descending, ties to the lower expert id) and wts [T x top_k] = p_k /
 * max(sum_k p_k, 2^-14).  The same device routing wzy_moe_block runs inside its gate/up launch.
 * n_exp <= 1024, top_k <= 32, T <= WZY_MAX_W.
 * Replaces router_top10_fast_multi (src/wzy_kernels_v2.cuh:989-1090). */
int wzy_moe_route(const float* logits, int n_exp, int top_k, int T, int* ids, float* wts, void* stream);

/* Time the expert kernels of wzy_moe_block with hipEvents on `stream`.  The router logits of x
 * [T x n_embd] are computed for every layer first; then `iters` gate/up launches run back to back
 * cycling through the `n_layers` weight sets (so the 256 MB last-level cache cannot hold the
 * experts), each routing with its own layer's logits, and then `iters` down+combine launches the
 * same way.  With us_block non-NULL, `iters` blocks follow, each a gate/up launch and then its
 * layer's down launch, as a decode step runs them.  Returns the mean duration in microseconds of
 * one gate/up launch, one down launch and one block (host pointers).  Layers must share one shape.
 * Allocates (and frees) its own scratch.
 * No counterpart in the reference: measurement support for the NVFP4 GEMV roofline. */
int wzy_moe_time_kernels(const wzy_moe_weights* layers, int n_layers, int T, const float* x, void* workspace,
                         size_t workspace_bytes, int iters, float* us_gate_up, float* us_down,
                         float* us_block, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Hyper-connection read
 * ------------------------------------------------------------------------------------------- */

/* One HC read of T rows (HC streams of D floats each, HCD = HC*D):
 *   R_out = (R_in or bf16 embedding rows of toks broadcast to every stream) + bo * 2*sigmoid(inj_prev/HC)
 *   xn[c] = R_out[c] * rsqrt(mean(R_out[c]^2) + eps) * norm_w[c]     -> nsc [T x HC] = the rsqrt
 *   lo = silu((down . quant32(xn)) / HC)   [T x HCLR];  inj = inj_w . xn  [T x HC]  (inj_w nullable)
 *   mixed[d] = 0.25 * sum_c xn[c][d] * sigmoid(up[c*D+d] . quant32(lo))   [T x D]
 * Exactly one of R_in / emb_table is non-NULL; bo/inj_prev (the pending HC write of the previous
 * block) may be NULL.  R_out must not alias R_in.  HC = 4; D in {256, 512, 1024, 2048, 4096};
 * HCLR a multiple of 32 up to 512.  The down projection is accumulated per source stream (four
 * partials, summed in a fixed order) in `workspace` (wzy_hc_read_workspace_bytes() bytes; calls
 * sharing a workspace must not overlap).
 * Replaces StageGpu::gr_read_fused + gr_write_multi (src/wzy_stage_v2.cuh:463-470;
 * src/wzy_kernels_v2.cuh:409-454,632-827) and bcast_emb_to_r_kernel (src/wzy_stage_v2.cuh:326-332). */
size_t wzy_hc_read_workspace_bytes(int HC, int HCLR, int T);
int wzy_hc_read(const float* R_in, const uint16_t* emb_table, const int* toks, int n_vocab, const float* bo,
                const float* inj_prev, float* R_out, const float* norm_w, const int8_t* down_q,
                const uint16_t* down_s, const uint16_t* inj_w, const int8_t* up_q, const uint16_t* up_s,
                float* nsc, float* lo, float* inj, float* mixed, int D, int HC, int HCLR, float eps, int T,
                void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------------------
 * GDN (gated delta-rule) recurrence
 * ------------------------------------------------------------------------------------------- */

/* Fused decode step for T rows: 4-tap causal conv + SiLU over the raw q|k|v projection channels
 * (history conv_hist [QKV x 3] updated), per-head L2 norm of q and k, decay = exp(softplus(alpha +
 * dt) * ssm_a), beta = sigmoid(beta_raw) from ab_raw [T x 2*hv] (alpha | beta), then the delta-rule
 * recurrence on state [hv][128][128] (S[h][key i][value j]), o * 1/sqrt(128), RMSNorm(gamma),
 * * sigmoid(z) -> y [T x hv*128].  Optional per-step snapshots: state_snaps [T][hv][128][128],
 * hist_snaps [T][QKV][3].  Head dim 128.
 * Replaces fused_gdn_conv_l2_multi + fused_gdn_ab_multi + fused_gdn_step_norm_multi
 * (src/wzy_kernels_v2.cuh:833-984). */
int wzy_gdn_step(const float* qkv_raw, const float* z, const float* ab_raw, const float* dt, const float* ssm_a,
                 const float* conv_w, float* conv_hist, float* state, const float* gamma, float eps, float* y,
                 int hk, int hv, int T, float* state_snaps, float* hist_snaps, void* stream);

/* Recurrence only, on already-activated q, k [T x hk*128], v [T x hv*128], decay/beta [T x hv]
 * (z and gamma may be NULL: no gate / unit norm weight).
 * Replaces fused_gdn_step_norm_multi (src/wzy_kernels_v2.cuh:908-984). */
int wzy_gdn_recurrence(const float* q, const float* k, const float* v, const float* decay, const float* beta,
                       const float* z, const float* gamma, float eps, float* state, float* y, int hk, int hv,
                       int T, float* state_snaps, void* stream);

/* ---------------------------------------------------------------------------------------------
 * QSA sparse attention
 * ------------------------------------------------------------------------------------------- */

typedef struct wzy_qsa_dims {
    int qh, kvh, hd, n_rot;                      /* 24, 2, 256, 64 */
    int idx_heads, idx_dim, idx_blk, idx_topk;   /* 4, 128, 4, 2048 */
    int ctx_max;                                 /* KV store / indexer capacity in cells */
    int kv_ring, kv_sinks;                       /* 0, 0 = full-context store addressed by position.
                                                    A ring (kv_ring slots, kv_sinks pinned) is accepted
                                                    only when it never wraps, ctx_max <= kv_ring; else
                                                    every entry point returns WZY_EINVAL (a wrapped slot
                                                    would serve a newer cell's K/V) */
    float eps;
    int attn_f16_above;                          /* 0 = fp32 attention at every context; > 0 (the
                                                    reference's 32,768-cell VRAM ring): a window with
                                                    pos + T > attn_f16_above attends as the reference's
                                                    GQA kernel does past its ring (q / 16, K and V
                                                    rounded to fp16, fp16 softmax weights per 32-cell
                                                    step; src/wzy_stage_v2.cuh:679-683,
                                                    src/wzy_qsa_wmma.cuh:289-488) */
} wzy_qsa_dims;

/* Per-row preparation at positions pos[0] + t: RMSNorm + NeoX RoPE of the q heads (qg [T x qh*2*hd],
 * q|gate per head, in place), of the k heads (kk [T x kvh*hd], in place) and of the indexer q heads
 * (q_idx [T x idx_heads*idx_dim], in place); INT8 append of k and v (fp16 scale per 64 elements,
 * scale rounded to fp16 first) into the KV store; indexer append of fp16(idx_raw) into idx_tail
 * [idx_blk-1 x idx_dim], idx_dead [idx_dim] and the fp16 pooled keys idx_pooled
 * [ctx_max/idx_blk + 2 x idx_dim].  cos_tab/sin_tab [ctx_max x n_rot/2].
 * Replaces fused_head_norm_rope_multi, kv_append_int8_multi, qsa_indexer_append_multi
 * (src/wzy_qsa_256k.cuh:50-209). */
int wzy_qsa_prepare(const wzy_qsa_dims* dims, const int* pos, float* qg, float* kk, const float* vv, float* q_idx,
                    const float* idx_raw, const float* q_norm, const float* k_norm, const float* iq_norm,
                    const float* ik_norm, const float* cos_tab, const float* sin_tab, int8_t* kq, uint16_t* ks,
                    int8_t* vq, uint16_t* vs, float* idx_tail, float* idx_dead, uint16_t* idx_pooled, int T,
                    void* stream);

/* Block scores (sum over indexer heads of relu(fp16 q . fp16 key)) and exact top-idx_topk cell
 * selection per row: sel_ids [T x idx_topk] (first sel_cnt[t] valid), scores [T x max_b]
 * (max_b >= ctx_max/idx_blk + 1).  Rows with n_kv <= idx_topk select 0..n_kv-1.
 * Replaces pf_qsa_block_scores_wmma + pf_qsa_tail_score_kernel + qsa_block_topk_multi
 * (src/wzy_qsa_wmma.cuh:492-612; src/wzy_qsa_256k.cuh:226-403). */
int wzy_qsa_select(const wzy_qsa_dims* dims, const int* pos, const uint16_t* idx_pooled, const float* idx_dead,
                   const float* q_idx, float* scores, int max_b, int* sel_ids, int* sel_cnt, int T, void* stream);

/* Exact top-idx_topk cell selection alone, over caller-supplied block scores [T x max_b] (row t's
 * context is pos[0] + t + 1 cells; its blocks 0 .. n_kv/idx_blk hold the scores): the second half
 * of wzy_qsa_select.  Rows longer than 16,384 blocks are histogrammed by several workgroups that
 * meet in per-device state of the library (row histograms, arrival counters, candidate lists), so
 * selections on one device (this call, wzy_qsa_select, a stage forward) must not overlap in time.
 * max_b <= 64 x 16,384.  Replaces qsa_block_topk_multi (src/wzy_qsa_256k.cuh:266-403). */
int wzy_qsa_topk(const wzy_qsa_dims* dims, const int* pos, const float* scores, int max_b, int* sel_ids, int* sel_cnt,
                 int T, void* stream);

/* GQA sparse attention over the selected cells: out [T x qh*hd] = softmax(q . k / 16) . v * sigmoid(gate).
 * Replaces qsa_attend_int8_sparse_multi (src/wzy_qsa_256k.cuh:407-532) and, for windows past
 * dims->attn_f16_above cells, pf_qsa_wmma_sparse_attn (src/wzy_qsa_wmma.cuh:289-488). */
size_t wzy_qsa_attend_workspace_bytes(const wzy_qsa_dims* dims, int T);
int wzy_qsa_attend(const wzy_qsa_dims* dims, const int* pos, const float* qg, const int8_t* kq, const uint16_t* ks,
                   const int8_t* vq, const uint16_t* vs, const int* sel_ids, float* out, void* workspace,
                   size_t workspace_bytes, int T, void* stream);

/* Measurement (no reference counterpart): `steps` decode steps of `n_layers`
 * independent GDN layers, step-major (every layer's step s before any layer's step s+1), T rows per
 * launch, through the wzy_gdn_recurrence kernels, in one burst on `stream` between two HIP events.
 * The layers share one set of inputs q, k [steps x hk*128], v [steps x hv*128], decay / beta
 * [steps x hv] (the duration does not depend on the values); states [n_layers][hv][128][128] are
 * updated; y [steps x hv*128].  us_per_layer_step = burst time / (n_layers * steps), including the
 * output-norm kernel; us_kernel_only (nullable) = the same without it.  Allocates a small scratch. */
int wzy_gdn_time_recurrence(const float* q, const float* k, const float* v, const float* decay, const float* beta,
                            float* states, float* y, int hk, int hv, int n_layers, int steps, int T,
                            float* us_per_layer_step, float* us_kernel_only, void* stream);

/* One QSA layer's decode state and activations for wzy_qsa_time_decode (device pointers; the same
 * meaning as the arguments of wzy_qsa_prepare / wzy_qsa_select / wzy_qsa_attend, T = 1). */
typedef struct wzy_qsa_layer {
    float* qg; float* kk; const float* vv; float* q_idx; const float* idx_raw;
    const float* q_norm; const float* k_norm; const float* iq_norm; const float* ik_norm;
    const float* cos_tab; const float* sin_tab;
    int8_t* kq; uint16_t* ks; int8_t* vq; uint16_t* vs;
    float* idx_tail; float* idx_dead; uint16_t* idx_pooled;
    float* scores; int max_b; int* sel_ids; int* sel_cnt;
    float* out; void* workspace; size_t workspace_bytes;
} wzy_qsa_layer;

/* Measurement (no reference counterpart): one decode token of one QSA layer at
 * position *pos, stage by stage, each stage `iters` times back to back between two HIP events:
 * us_stages[4] = mean microseconds of prepare (norms, RoPE, KV + indexer append), block scores,
 * exact top-idx_topk, sparse attention (with its chunk merge). */
int wzy_qsa_time_decode(const wzy_qsa_dims* dims, const wzy_qsa_layer* layer, const int* pos, int iters,
                        float* us_stages, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Per-layer embedding (PLE) at layer 1 of the reference's real model (not part of the synthetic
 * BASELINE model)
 * ------------------------------------------------------------------------------------------- */

/* Rows of the hashed 3-gram fp8 table (wzy_ple_table_rows() rows of head_bytes = n_embd / 16 codes,
 * in device memory) for T window rows at positions *pos .. *pos+T-1 of tokens toks [T] (device):
 * emb [T x n_embd] = the 16 heads' rows decoded (e4m3, NaN codes 0) times `scale`; emb_bf16 (nullable)
 * the same rounded to bf16.  The tokens before the window are read from tok_hist [ctx_max] (device,
 * cell p holding the token of position p), which the call extends with the window's tokens.  A
 * context reaching past a missing token (position < 0) or `eos` hashes eos in its place.
 * Replaces stage_ple_window + PleSrc::row (src/wzy_engine_v2.cu:943-978; src/wzy_stage_v2.cuh:215-324),
 * which gather the rows on the host from the mmap-ed table. */
uint64_t wzy_ple_table_rows(void);
int wzy_ple_rows(const uint8_t* table, int head_bytes, float scale, int eos, const int* pos, const int* toks, int T,
                 int* tok_hist, int ctx_max, float* emb, uint16_t* emb_bf16, void* stream);

/* The PLE block on T rows of the hyper-connection streams R [T x hc x n_embd] (in place), decode form:
 * the pending write bo [T x n_embd] (nullable) with inject inj_prev [T x hc] folded in first, then
 * q = groupnorm(R, norm_q), k = groupnorm(wk . emb, norm_k), v = wv . emb (bf16 weights wk
 * [hc*n_embd x n_embd], wv [n_embd x n_embd]), gate sigmoid(sign(s) sqrt(max(|s|, 1e-6))) of
 * s = k_c . q_c / sqrt(n_embd), gat = v * gate, n = groupnorm(gat, norm_c), and per channel the
 * 4-tap conv over its history hist [hc*n_embd x 9] (taps at 9, 6, 3 rows back and the current row,
 * conv_w [hc*n_embd x 4]): R += gat + silu(conv).  hist_snaps (nullable) [T x hc*n_embd x 9] receives
 * the history after each row.  workspace: wzy_ple_workspace_bytes(n_embd, hc, T) bytes.
 * Replaces the PLE block of record_forward (src/wzy_stage_v2.cuh:583-597: ple_group_multi,
 * dense_bf16, ple_gate_gv_multi, ple_conv_multi, src/wzy_kernels_v2.cuh:1299-1374). */
size_t wzy_ple_workspace_bytes(int n_embd, int hc, int T);
int wzy_ple_block(float* R, const float* bo, const float* inj_prev, const float* emb, const uint16_t* wk,
                  const uint16_t* wv, const float* norm_q, const float* norm_k, const float* norm_c,
                  const float* conv_w, float* hist, int n_embd, int hc, float eps, int T, float* hist_snaps,
                  void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Logit reductions
 * ------------------------------------------------------------------------------------------- */

/* Greedy argmax per row over `nvocab` logits (ties -> lowest index).
 * Scratch: a per-device buffer of row counters and partial results, hipMalloc-ed (and zeroed) on the
 * first call on a device and re-allocated when a call needs more; shared by wzy_row_argmax and
 * wzy_row_top16, so calls on one device must not overlap in time.
 * Replaces row_argmax_multi_kernel (src/wzy_kernels_v2.cuh:1873-1905). */
int wzy_row_argmax(const float* logits, int nvocab, int T, int* out_ids, void* stream);

/* Top-16 (value desc, ties -> lower index) per row plus greedy id (= rank 0).  Any output may be
 * NULL.  Same per-device scratch as wzy_row_argmax.
 * Replaces row_top16_multi_kernel (src/wzy_kernels_v2.cuh:1909-1984). */
int wzy_row_top16(const float* logits, int nvocab, int T, int* out_greedy, float* top_v,
                  int* top_i, void* stream);

/* wzy_row_top16 without any allocation: the same kernels and results, with the scratch (row
 * counters and partial results) in a fixed 131,328-byte device array in the library instead of a
 * hipMalloc-ed buffer, so it can run where hipMalloc cannot (under HIP graph capture, in tight
 * serving loops, in harnesses that forbid allocation).  Limits: 1 <= T <= 8, 1 <= nvocab <= 262,144;
 * larger calls return WZY_EINVAL before anything is launched.  Every call on a device shares that
 * device's array, so calls that overlap in time on one device race.  The first call on a device also
 * enqueues one small kernel that clears the counters.
 * No counterpart in the reference: it exists for callers that cannot allocate. */
int wzy_row_top16_noalloc(const float* logits, int nvocab, int T, int* out_greedy, float* top_v,
                          int* top_i, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* WZY_KERNELS_H */

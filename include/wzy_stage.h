/* wzy_stage.h -- C ABI of the layer executor ("stage") of the MI355X decode path.
 *
 * Replaces the reference's in-process StageGpu (src/wzy_stage_v2.cuh:334-1045; construction and
 * weight loading in init_stage_weights_and_state / alloc_stage_expert_vram,
 * src/wzy_engine_v2.cu:310-593).  Differences that follow from running on one MI355X:
 *   - one stage owns all layers (no PP2 split, no peer handoff arguments);
 *   - every NVFP4 expert of every layer is resident in HBM, so the cold-expert mailbox, the CPU
 *     pool arguments and the expert cache disappear (service/promote are kept as no-op calls);
 *   - the KV cache is a full-context INT8 store in HBM (no pinned host mirror);
 *   - token embeddings are gathered on the GPU from token ids (host fp32 rows remain accepted).
 * Errors are reported as negative status codes with wzy_last_error() (the reference exits the
 * process); a host driver that wants the reference behaviour exits on any negative status.
 * One stream and one host thread per handle; calls on a handle must be serialised.
 *
 * Synthetic model: wzy_stage_load_synthetic() fills every weight and a prefilled decode state of
 * n_ctx cells from a seed, deterministically, one generator sub-stream per (tensor, layer)
 * (see wzy_synth.h).
 */
#ifndef WZY_STAGE_H
#define WZY_STAGE_H

#include <stddef.h>
#include <stdint.h>

#include "wzy_kernels.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct wzy_stage_cfg {
    int n_layers;                              /* 48 */
    int qsa_period;                            /* 4: layer l is QSA iff l % qsa_period == qsa_period-1
                                                  (reference is_qsa_layer, src/wzy_engine_v2.cu:17) */
    int n_embd;                                /* D = 2048 */
    int hc, hc_lr;                             /* hyper-connection streams 4, low rank 320 */
    int gdn_hk, gdn_hv;                        /* GDN key / value heads (head dim 128): 16, 16 */
    int qsa_qh, qsa_kvh, qsa_hd, n_rot;        /* 24, 2, 256, 64 */
    int idx_heads, idx_dim, idx_blk, idx_topk; /* 4, 128, 4, 2048 */
    int n_exp, top_k, n_ff;                    /* 512, 10, 512 */
    int n_vocab;                               /* 151936 */
    int ctx_max;                               /* KV / indexer / RoPE capacity in cells */
    int kv_ring, kv_sinks;                     /* 0, 0: full-context KV store (a ring is rejected
                                                  unless ctx_max <= kv_ring, i.e. it never wraps) */
    float rope_theta, eps;                     /* 1e7, 1e-6 */
    int emb_q8;                                /* 0: token embedding table bf16 ("emb"); 1: Q8_0 ("emb.q"
                                                  codes + "emb.s" fp16 scales per 32), gathered and
                                                  dequantised on the GPU as d*q (stage_one_emb,
                                                  src/wzy_engine_v2.cu:861-873) */
    int head_q8;                               /* 0: LM head bf16 ("head", BASELINE); 1: Q8_0 ("head.q" /
                                                  "head.s", the reference's output.weight,
                                                  src/wzy_stage_v2.cuh:804-815) */
    int attn_f16_above;                        /* 32768 (the reference's KV_VRAM_RING): decode windows
                                                  with pos + T > attn_f16_above run QSA attention with
                                                  the fp16 operands of the reference's GQA kernel
                                                  (src/wzy_stage_v2.cuh:679-683); 0 = fp32 attention at
                                                  every context */
    int ple;                                   /* 0 (BASELINE synthetic model); 1: the reference model's
                                                  per-layer embedding at layer 1 (hashed 3-gram rows of
                                                  an fp8 table in HBM, src/wzy_stage_v2.cuh:583-597) */
    int ple_eos;                               /* end-of-sequence id of the PLE context (248044) */
} wzy_stage_cfg;

typedef struct wzy_stage wzy_stage;

/* The BASELINE synthetic model (config 4) with the given context capacity. */
void wzy_stage_cfg_default(wzy_stage_cfg* cfg, int ctx_max);

/* Allocate a stage on `device` (weights uninitialised until a load call). */
int wzy_stage_create(const wzy_stage_cfg* cfg, int device, wzy_stage** out);
int wzy_stage_destroy(wzy_stage* st);
/* Device bytes held by the stage. */
size_t wzy_stage_device_bytes(const wzy_stage* st);

/* Random-initialise every weight from `seed` and synthesise a prefilled decode state of n_ctx
 * cells (GDN conv/ssm state, INT8 KV cells 0..n_ctx-1, indexer keys).  0 <= n_ctx < ctx_max;
 * n_ctx == 0 leaves the state empty, as after wzy_stage_reset_state().
 * (The reference loads a GGUF checkpoint here; a synthetic model is what the benchmarks use.) */
int wzy_stage_load_synthetic(wzy_stage* st, uint64_t seed, int n_ctx);

/* Enqueue the forward of T window rows at positions pos .. pos+T-1 (1 <= T <= 8):
 *   toks [T] token ids (embedding gathered on the GPU), or emb [T x n_embd] fp32 rows (host
 *   memory) when non-NULL; run_head 1: compute logits + greedy ids (+ top-16 when want_top16);
 *   run_head 2: only the pre-head residual rows (the head's hyper-connection fold, no logits), the
 *   input of wzy_stage_mtp_front during prefill;
 *   save_snaps: write per-row snapshots (at snap_offset + t) of GDN / indexer state for
 *   commit_window_state.  Asynchronous: results are valid after wzy_stage_sync().
 * Replaces StageGpu::record_forward (src/wzy_stage_v2.cuh:476-857). */
int wzy_stage_record_forward(wzy_stage* st, int pos, const float* emb, const int* toks, int T, int run_head,
                             int save_snaps, int want_top16, int snap_offset);
/* Chunked prefill of B prompt cells at positions pos .. pos+B-1 (toks [B] host token ids, copied
 * before the call returns): every layer runs over all B rows at once, with the dense projections
 * on bf16 MFMA GEMMs (activations and dequantised Q8_0 weights rounded to bf16, fp32 accumulation),
 * the GDN recurrence sequential over the rows, the QSA rows selecting and attending as a decode row
 * would (attention with the reference prefill kernel's fp16 operands), and the MoE block of
 * wzy_moe_prefill.  Updates the decode state of those cells (GDN conv/ssm, KV cells, indexer keys)
 * and leaves the final residual rows [B x hc x n_embd] as the pre-head rows of the call
 * (wzy_stage_pre_head, wzy_stage_mtp_front).  No logits.  Asynchronous (wzy_stage_sync).  The
 * first call with a larger B allocates the workspace (BASELINE shapes: about 0.25 MB per row).
 * Needs hc_lr a multiple of 64, n_embd of 256, n_exp of 64 (<= 1024), n_ff of 128, idx_dim 128.
 * Replaces PrefillStageCtx::run_stage_prefill (src/wzy_prefill_tc.cuh:546-1058) for one stage
 * holding every layer (no expert streaming: every expert is resident). */
int wzy_stage_prefill(wzy_stage* st, int pos, const int* toks, int B);
/* 1 when a stage of this configuration can run wzy_stage_prefill (the shape limits above), else 0
 * (a host then feeds prompts through record_forward windows, as the reference does for short
 * remainders). */
int wzy_stage_can_prefill(const wzy_stage_cfg* cfg);
/* Same, timed: us_parts[6] = microseconds spent in the attention-half HC reads, GDN blocks, QSA
 * blocks, FFN-half HC reads, MoE blocks and the rest (HIP events between the parts; synchronous).
 * Counterpart of the reference's WZY_PF_PROF timers (src/wzy_prefill_tc.cuh:734-741,1048-1051). */
int wzy_stage_prefill_time(wzy_stage* st, int pos, const int* toks, int B, float* us_parts);
/* Cold-expert servicing and VRAM promotion: nothing is cold on one MI355X (no-ops, kept so a
 * reference driver links unchanged).  Replace StageGpu::service_cold_layers / promote_cold
 * (src/wzy_stage_v2.cuh:932,960). */
int wzy_stage_service_cold_layers(wzy_stage* st);
int wzy_stage_promote_cold(wzy_stage* st);
/* Keep the state after window row acc_idx (accepted prefix acc_idx+1 rows ending at position
 * acc_pos): restores GDN conv/ssm snapshots and the indexer tail/placeholder/pooled keys.
 * Replaces StageGpu::commit_window_state (src/wzy_stage_v2.cuh:939-958). */
int wzy_stage_commit_window_state(wzy_stage* st, int acc_idx, int acc_pos);
/* Zero the recurrent state (GDN conv/ssm, indexer tail/placeholder).
 * Replaces StageGpu::reset_state (src/wzy_stage_v2.cuh:1031-1044). */
int wzy_stage_reset_state(wzy_stage* st);
int wzy_stage_sync(wzy_stage* st);

/* ---- Parked sessions (ParkedSession, save_session_state / restore_session_state,
 * src/wzy_engine_v2.cu:1636-1842) ----
 * A session's state is what the decode of its next token reads: per GDN layer the conv history and
 * the fp32 recurrent state; per QSA layer the INT8 K/V and scales of cells 0 .. n_cells-1, the
 * indexer tail, placeholder and pooled keys of the blocks those cells reach; and, when the drafter
 * is initialised, its KV ring and attention floor.  The reference copies them to pinned host
 * memory; here a slot is a buffer in the same GPU's HBM (a 98,304-cell session of the BASELINE
 * model is 1.4 GB), grown on the first save that needs more and kept until the stage is destroyed.
 * save copies the live state into `slot`, restore copies a slot back (the slot keeps its copy);
 * each is one copy launch on the stage stream and returns after it has finished.
 * wzy_stage_session_cells() is the slot's cell count, -1 when empty; clear empties a slot. */
#define WZY_SESSION_SLOTS 2
size_t wzy_stage_session_bytes(const wzy_stage* st, int n_cells);
int wzy_stage_session_save(wzy_stage* st, int slot, int n_cells);
int wzy_stage_session_restore(wzy_stage* st, int slot);
int wzy_stage_session_cells(const wzy_stage* st, int slot);
int wzy_stage_session_clear(wzy_stage* st, int slot);

/* Results of the last forward with run_head (after sync); host outputs. */
int wzy_stage_greedy_ids(wzy_stage* st, int* out, int T);
int wzy_stage_top16(wzy_stage* st, float* v, int* ids, int T);
int wzy_stage_logits(wzy_stage* st, float* out, int T);          /* [T x n_vocab] */
int wzy_stage_pre_head(wzy_stage* st, float* out, int T);        /* [T x hc x n_embd] residual before the head */

/* Per-layer trace of the following forwards (debugging and layer-by-layer parity checks; forwards
 * run as direct launches while it is on).  Each forward then leaves, readable with
 * wzy_stage_read_tensor(st, -1, name): "trace.mixed_a" / "trace.block" / "trace.mixed_f" /
 * "trace.comb" fp32 [n_layers][8][n_embd] (attention HC read output, attention block output, FFN
 * HC read output, MoE output), "trace.R_a" / "trace.R_f" fp32 [n_layers][8][hc][n_embd] (the
 * residual streams after the attention / FFN HC read, i.e. with the pending write folded in),
 * "trace.inj_a" / "trace.inj_f" fp32 [n_layers][8][hc] (the inject vectors), "trace.moe_logits"
 * fp32 [n_layers][8][n_exp], "trace.moe_ids" int32
 * / "trace.moe_wts" fp32 [n_layers][8][top_k], and per QSA layer (in layer order) "trace.scores"
 * fp32 [n_qsa][8][ctx_max/idx_blk + 2], "trace.sel_ids" int32 [n_qsa][8][idx_topk], "trace.sel_cnt"
 * int32 [n_qsa][8]; rows 0..T-1 of each [8] block are valid.  The first enable allocates the
 * buffers.  Counterpart of the reference's per-layer route probe (WZY_DBG_TOPS, dbg_probe_layer,
 * src/wzy_stage_v2.cuh:754-760; src/wzy_kernels_v2.cuh:1986-1991). */
int wzy_stage_set_trace(wzy_stage* st, int enable);

/* Use hipGraphs for record_forward (default on): one graph per window shape, replayed. */
int wzy_stage_set_graphs(wzy_stage* st, int enable);
/* The stage's HIP stream (hipStream_t). */
void* wzy_stage_stream(wzy_stage* st);

/* Tensor access for checks and loaders, by (layer, name); layer -1 for model-level tensors.
 * Per layer: "<proj>.q"/"<proj>.s" (Q8_0 codes / fp16 scales of a dense projection), hc_norm*,
 * hc_inj*, GDN alpha, beta, ssm_a, dt_bias, conv1d, ssm_norm, conv_hist, ssm; QSA q_norm, k_norm,
 * idx_q, idx_k, idx_qn, idx_kn, kv_k, kv_ks, kv_v, kv_vs, idx_tail, idx_dead, idx_pooled; MoE
 * router, sgate.  Model level: experts, emb, head_norm, head, rope_cos, rope_sin, and the "act.*"
 * activation buffers of the last forward.  wzy_stage_tensor_bytes() returns 0 for an unknown name.
 * Byte size, device-to-host and host-to-device copies (synchronous). */
size_t wzy_stage_tensor_bytes(wzy_stage* st, int layer, const char* name);
int wzy_stage_read_tensor(wzy_stage* st, int layer, const char* name, void* host, size_t bytes);
int wzy_stage_write_tensor(wzy_stage* st, int layer, const char* name, const void* host, size_t bytes);
/* Bytes [offset, offset + bytes) of a tensor, device to host / host to device (synchronous). */
int wzy_stage_read_tensor_range(wzy_stage* st, int layer, const char* name, size_t offset, void* host,
                                size_t bytes);
int wzy_stage_write_tensor_range(wzy_stage* st, int layer, const char* name, size_t offset, const void* host,
                                 size_t bytes);

/* ---- MTP speculative drafter (MtpEngine, src/wzy_mtp.cuh:405-754) ----
 * One extra decoder layer (attention over its own 1,024-cell INT8 KV ring, MoE of n_exp Q2_0
 * experts + a Q8_0 shared expert, hyper-connections) and a Q8_0 draft head over n_dvocab rows of
 * the main vocabulary.  Cell p embeds the token at p+1 and reads the main model's pre-head
 * residual at p; it proposes the token at p+2.
 *
 * wzy_stage_mtp_init: allocate and random-initialise the drafter from `seed` (the reference loads
 *   dense.txt/dense.bin, experts.bin and the draft vocabulary, MtpEngine::init, :459-645); the
 *   draft head is the Q8_0 quantisation of main LM-head rows dvocab[i] = i*n_vocab/n_dvocab.
 * wzy_stage_mtp_reset: empty the KV ring and its floor (MtpEngine::reset_kv, :647-656).
 * wzy_stage_mtp_set_floor: first cell the ring attention may read (d_kv_floor, set by
 *   seed_mtp_tail, src/wzy_engine_v2.cu:1266-1290).
 * wzy_stage_mtp_front: K/V append of cells cell0 .. cell0+n_cells-1 (n_cells <= 8), embedding
 *   next_toks[i] with pre-head residual row src_row0+i of the last forward (which must have run
 *   with run_head 1 or 2) (MtpEngine::run_front_kv, :658-683).  Asynchronous.
 * wzy_stage_mtp_draft: `depth` chained draft steps (1..8): the first at `cell` embedding `tok`
 *   with pre-head row src_row of the last forward (src_row < 0: the residual the previous draft
 *   step left), each further step at the next cell embedding the previous draft.  Writes the
 *   drafted token ids and their top-1 probabilities 1/sum(exp(l - max)) (synchronous)
 *   (run_front_kv + run_rest_row0 + head reduction, :658-733,293-403; the chain of mtp_propose,
 *   src/wzy_engine_v2.cu:1428-1470, without its confidence gates, which the caller applies).
 * wzy_stage_mtp_propose: catch-up + chain of mtp_propose (src/wzy_engine_v2.cu:1384-1427): the
 *   front over cells cell0 .. cell0+n_cells-2 (rows 0 .. n_cells-2 of the last forward), then
 *   wzy_stage_mtp_draft at cell0+n_cells-1 with row n_cells-1.
 * Readable tensors (wzy_stage_read_tensor, layer -1): "mtp.*" weights and the "mtp.act.*"
 * activations of the last step. */
int wzy_stage_mtp_init(wzy_stage* st, uint64_t seed, int n_dvocab);
/* The drafter for weights from files (wzy_stage_mtp_load in wzy_loader.h, or a host's own loader):
 * allocated with the draft vocabulary dvocab[n_dvocab] (main-vocabulary ids) and its draft head
 * (those rows of the main LM head: Q8_0 rows as they are, bf16 rows quantised to Q8_0), the KV
 * ring empty; every other "mtp.*" weight must then be written with wzy_stage_write_tensor. */
int wzy_stage_mtp_init_vocab(wzy_stage* st, const int* dvocab, int n_dvocab);
int wzy_stage_mtp_reset(wzy_stage* st);
int wzy_stage_mtp_set_floor(wzy_stage* st, int kv_floor);
int wzy_stage_mtp_front(wzy_stage* st, int cell0, const int* next_toks, int n_cells, int src_row0);
int wzy_stage_mtp_draft(wzy_stage* st, int cell, int tok, int src_row, int depth, int* out_toks, float* out_probs);
int wzy_stage_mtp_propose(wzy_stage* st, int cell0, int n_cells, const int* next_toks, int depth, int* out_toks,
                          float* out_probs);
/* Measurement support (no reference counterpart): mean device time of one draft step over `iters`
 * chained steps from `cell` (src_row as in wzy_stage_mtp_draft), bracketed by HIP events on the
 * stage stream.  The steps write ring cells cell .. cell+iters. */
int wzy_stage_mtp_time(wzy_stage* st, int cell, int tok, int src_row, int iters, float* us_per_step);

/* Measurement support (no reference counterpart): time the NVFP4 expert kernels of every layer's
 * MoE block with hipEvents for `iters` iterations (cycling over layers with the routing of the
 * last forward's rows) -> mean microseconds of the gate/up launch, of the down launch and (us_block
 * non-NULL) of a gate/up launch followed by its down launch (wzy_moe_time_kernels). */
int wzy_stage_time_moe(wzy_stage* st, int iters, float* us_gate_up, float* us_down, float* us_block);

/* Measurement support (no reference counterpart): the device pointers of one layer's MoE weights
 * (router, shared gate, shared expert, expert records), for the standalone MoE entry points of
 * wzy_kernels.h.  The pointers stay valid until wzy_stage_destroy. */
int wzy_stage_moe_weights(wzy_stage* st, int layer, wzy_moe_weights* out);

#ifdef __cplusplus
}
#endif
#endif /* WZY_STAGE_H */

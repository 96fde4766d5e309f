/* orc_prefill.c -- CPU oracle of the chunked prefill of B prompt cells through the whole model
 * (PrefillStageCtx::run_stage_prefill, src/wzy_prefill_tc.cuh:546-1058).  TEST INFRASTRUCTURE ONLY
 * (see wzy_oracle.h).
 *
 * The reference's prefill differs from its decode in the operands of every projection: decode
 * quantises activations to int8 per 32 (quant_act_multi) and dots them with the Q8_0 codes; prefill
 * converts activations and dequantised weights to 16-bit floats and runs tensor-core GEMMs with fp32
 * accumulation (cublasGemmEx, src/wzy_prefill_tc.cuh:681-711).  This build runs those GEMMs with bf16
 * operands (the reference uses fp16; bf16 is the operand type of the MI355X prefill, as in the MoE
 * block), so this oracle rounds to bf16 where the reference rounds to fp16:
 *   - GEMM A operands: the HC-normalised streams, the low-rank SiLU activations, the HC read output,
 *     the GDN gated-norm output and the attention output;
 *   - GEMM weights: Q8_0 code * fp16 scale rounded to bf16, bf16 weights as they are;
 *   - the HC up projection's output, which the reference stores as fp16 (cuBLAS with an fp16 C).
 * The sparse attention keeps the reference's fp16 operands (pf_qsa_wmma_sparse_attn,
 * src/wzy_qsa_wmma.cuh:289-489): q * 1/16, dequantised K and V and the softmax weights in fp16.
 * Everything else is the decode arithmetic (GDN conv / gates / recurrence / gated norm, head norm +
 * RoPE, INT8 KV append, indexer append, block scores, exact top-k), which the reference's prefill
 * also uses.  Sums accumulate in double and round once. */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "wzy_oracle.h"

static float rbf(float f) {                     /* round to bf16, nearest even */
    uint32_t u;
    memcpy(&u, &f, 4);
    u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
    memcpy(&f, &u, 4);
    return f;
}
static float rh(float f) { return orc_f16_to_f32(orc_f32_to_f16(f)); }   /* round to fp16 */

/* y[t * ldy + n] = sum_k A[t][k] * W[n][k] for t < M, n < N; A holds bf16 values (M x K), W is
 * Q8_0 (codes q, fp16 scales s per 32, dequantised and rounded to bf16) or bf16 (wb). */
void orc_pf_gemm(const float* A, int M, int K, const int8_t* q, const uint16_t* s, const uint16_t* wb, int N,
                 float* y, int ldy) {
#pragma omp parallel
    {
        float* w = (float*) malloc(sizeof(float) * (size_t) K);
#pragma omp for schedule(static)
        for (int n = 0; n < N; ++n) {
            for (int k = 0; k < K; ++k)
                w[k] = wb ? orc_bf16_to_f32(wb[(size_t) n * K + k])
                          : rbf((float) q[(size_t) n * K + k] * orc_f16_to_f32(s[((size_t) n * K + k) / 32]));
            for (int t = 0; t < M; ++t) {
                const float* a = A + (size_t) t * K;
                double acc = 0.0;
                for (int k = 0; k < K; ++k) acc += (double) a[k] * (double) w[k];
                y[(size_t) t * ldy + n] = (float) acc;
            }
        }
        free(w);
    }
}

/* Hyper-connection read of B rows for the prefill (tc_gr_read, src/wzy_prefill_tc.cuh:690-715):
 * pf_gr_norm_fp16 (pending block folded into R with gate 2*sigmoid(inj/HC), per-stream RMSNorm, bf16),
 * the inject GEMM, the low-rank down GEMM, silu(lo/HC) in bf16, the up GEMM rounded to bf16, and
 * pf_gr_up_mean_fp16 (mean over streams of x * sigmoid(g), streams summed in order).
 * R [B][HC][D] is updated in place; inj [B][HC] (optional), mixed [B][D] fp32. */
void orc_hc_read_pf(float* R, const float* bo, const float* inj_prev, const float* norm_w, const int8_t* down_q,
                    const uint16_t* down_s, const uint16_t* inj_w, const int8_t* up_q, const uint16_t* up_s, int D,
                    int HC, int HCLR, float eps, int B, float* inj, float* mixed) {
    const int HCD = HC * D;
    float* xn = (float*) malloc(sizeof(float) * (size_t) B * HCD);
    float* lo = (float*) malloc(sizeof(float) * (size_t) B * HCLR);
    float* gg = (float*) malloc(sizeof(float) * (size_t) B * HCD);
    for (int t = 0; t < B; ++t)
        for (int c = 0; c < HC; ++c) {
            float* r = R + ((size_t) t * HC + c) * D;
            const float gate = bo ? 2.0f / (1.0f + expf(-inj_prev[t * HC + c] / (float) HC)) : 0.0f;
            double ss = 0.0;
            for (int d = 0; d < D; ++d) {
                if (bo) r[d] = fmaf(bo[(size_t) t * D + d], gate, r[d]);
                ss += (double) r[d] * (double) r[d];
            }
            const float inv = 1.0f / sqrtf((float) ss / (float) D + eps);
            for (int d = 0; d < D; ++d)
                xn[(size_t) t * HCD + (size_t) c * D + d] = rbf(r[d] * inv * norm_w[(size_t) c * D + d]);
        }
    if (inj && inj_w) orc_pf_gemm(xn, B, HCD, NULL, NULL, inj_w, HC, inj, HC);
    orc_pf_gemm(xn, B, HCD, down_q, down_s, NULL, HCLR, lo, HCLR);
    for (size_t i = 0; i < (size_t) B * HCLR; ++i) {
        const float v = lo[i] * (1.0f / (float) HC);
        lo[i] = rbf(v / (1.0f + expf(-v)));
    }
    orc_pf_gemm(lo, B, HCLR, up_q, up_s, NULL, HCD, gg, HCD);
    for (int t = 0; t < B; ++t)
        for (int d = 0; d < D; ++d) {
            float acc = 0.f;
            for (int c = 0; c < HC; ++c) {
                const size_t i = (size_t) t * HCD + (size_t) c * D + d;
                acc += xn[i] / (1.0f + expf(-rbf(gg[i])));
            }
            mixed[(size_t) t * D + d] = acc * (1.0f / (float) HC);
        }
    free(xn);
    free(lo);
    free(gg);
}

/* R[t][c][d] += blk[t][d] * 2*sigmoid(inj[t][c]/HC) (gr_write_multi, src/wzy_kernels_v2.cuh:813-827) */
void orc_hc_write(float* R, const float* blk, const float* inj, int D, int HC, int B) {
    for (int t = 0; t < B; ++t)
        for (int c = 0; c < HC; ++c) {
            const float g = 2.0f / (1.0f + expf(-inj[t * HC + c] / (float) HC));
            float* r = R + ((size_t) t * HC + c) * D;
            for (int d = 0; d < D; ++d) r[d] = fmaf(blk[(size_t) t * D + d], g, r[d]);
        }
}

/* Sparse GQA attention of one row as pf_qsa_wmma_sparse_attn computes it (src/wzy_qsa_wmma.cuh:
 * 289-489): per KV head, the group's query heads scaled by 1/16 and rounded to fp16; the selected
 * cells in steps of 32 (selection order), K and V dequantised to fp16 (fp16(code) * fp16 scale,
 * rounded); per step an online softmax (running max, alpha = exp(m_old - m_new), weights
 * exp(s - m_new) summed in fp32 and rounded to fp16 for the P.V product); out = acc / max(l, 1e-20)
 * * sigmoid(gate).  qg [qh][2*hd] (q | gate per head), out [qh][hd]. */
void orc_attend_pf(const float* qg, const int8_t* kq, const uint16_t* ks, const int8_t* vq, const uint16_t* vs,
                   const int* sel, int n, int qh, int kvh, int hd, float* out) {
    const int kvd = kvh * hd, gq = qh / kvh, sc_per = kvd / 64;
    float* qf = (float*) malloc(sizeof(float) * (size_t) gq * hd);
    float* K = (float*) malloc(sizeof(float) * (size_t) 32 * hd);
    float* V = (float*) malloc(sizeof(float) * (size_t) 32 * hd);
    float* acc = (float*) malloc(sizeof(float) * (size_t) gq * hd);
    float s[32], P[32];
    for (int j = 0; j < kvh; ++j) {
        float m[16], l[16];
        for (int h = 0; h < gq; ++h) {
            for (int d = 0; d < hd; ++d) qf[(size_t) h * hd + d] = rh(qg[(size_t) (j * gq + h) * 2 * hd + d] * 0.0625f);
            m[h] = -1e30f;
            l[h] = 0.f;
        }
        memset(acc, 0, sizeof(float) * (size_t) gq * hd);
        for (int base = 0; base < n; base += 32) {
            const int cnt = n - base < 32 ? n - base : 32;
            for (int c = 0; c < cnt; ++c) {
                const size_t p = (size_t) sel[base + c];
                for (int d = 0; d < hd; ++d) {
                    const size_t e = p * kvd + (size_t) j * hd + d;
                    const size_t si = p * sc_per + (size_t) (j * hd + d) / 64;
                    K[(size_t) c * hd + d] = rh((float) kq[e] * orc_f16_to_f32(ks[si]));
                    V[(size_t) c * hd + d] = rh((float) vq[e] * orc_f16_to_f32(vs[si]));
                }
            }
            for (int h = 0; h < gq; ++h) {
                float rmax = -1e30f;
                for (int c = 0; c < cnt; ++c) {
                    double a = 0.0;
                    for (int d = 0; d < hd; ++d) a += (double) qf[(size_t) h * hd + d] * (double) K[(size_t) c * hd + d];
                    s[c] = (float) a;
                    rmax = fmaxf(rmax, s[c]);
                }
                const float m_new = fmaxf(m[h], rmax);
                const float alpha = expf(m[h] - m_new);
                double psum = 0.0;
                for (int c = 0; c < cnt; ++c) {
                    const float pw = expf(s[c] - m_new);
                    psum += pw;
                    P[c] = rh(pw);
                }
                m[h] = m_new;
                l[h] = l[h] * alpha + (float) psum;
                for (int d = 0; d < hd; ++d) {
                    double o = 0.0;
                    for (int c = 0; c < cnt; ++c) o += (double) P[c] * (double) V[(size_t) c * hd + d];
                    acc[(size_t) h * hd + d] = fmaf(acc[(size_t) h * hd + d], alpha, (float) o);
                }
            }
        }
        for (int h = 0; h < gq; ++h) {
            const float inv = 1.0f / fmaxf(l[h], 1e-20f);
            for (int d = 0; d < hd; ++d) {
                const float gate = qg[(size_t) (j * gq + h) * 2 * hd + hd + d];
                out[(size_t) (j * gq + h) * hd + d] = (acc[(size_t) h * hd + d] * inv) / (1.0f + expf(-gate));
            }
        }
    }
    free(qf);
    free(K);
    free(V);
    free(acc);
}

static void round_rows(const float* x, float* xb, size_t n) {
    for (size_t i = 0; i < n; ++i) xb[i] = rbf(x[i]);
}

int orc_model_prefill(const orc_model* m, int pos, const int* toks, int B, float* R_out, float* dbg) {
    return orc_model_prefill_dbg(m, pos, toks, B, R_out, dbg, NULL);
}

int orc_model_prefill_dbg(const orc_model* m, int pos, const int* toks, int B, float* R_out, float* dbg,
                          float* margins) {
    const int D = m->n_embd, HC = m->hc, L = m->hc_lr;
    const int QKV = 2 * m->gdn_hk * 128 + m->gdn_hv * 128, GV = m->gdn_hv * 128, hv = m->gdn_hv;
    const int QD = m->qsa_qh * m->qsa_hd, KVD = m->qsa_kvh * m->qsa_hd, hd = m->qsa_hd;
    const int ID = m->idx_dim, IH = m->idx_heads;
    if (B < 1 || pos < 0 || pos + B > m->ctx_max) return -1;
    float* R = R_out;
    float* inj_a = (float*) malloc(sizeof(float) * (size_t) B * HC);
    float* inj_f = (float*) malloc(sizeof(float) * (size_t) B * HC);
    float* mixed = (float*) malloc(sizeof(float) * (size_t) B * D);
    float* xb = (float*) malloc(sizeof(float) * (size_t) B * (QD > D ? (QD > GV ? QD : GV) : (D > GV ? D : GV)));
    float* block = (float*) malloc(sizeof(float) * (size_t) B * D);
    float* comb = (float*) malloc(sizeof(float) * (size_t) B * D);
    float* qkv = (float*) malloc(sizeof(float) * (size_t) B * QKV);
    float* z = (float*) malloc(sizeof(float) * (size_t) B * GV);
    float* ab = (float*) malloc(sizeof(float) * (size_t) B * 2 * (hv > 0 ? hv : 1));
    float* y = (float*) malloc(sizeof(float) * (size_t) B * GV);
    float* qg = (float*) malloc(sizeof(float) * (size_t) B * 2 * QD);
    float* kk = (float*) malloc(sizeof(float) * (size_t) B * KVD);
    float* vv = (float*) malloc(sizeof(float) * (size_t) B * KVD);
    float* idx_raw = (float*) malloc(sizeof(float) * (size_t) B * ID);
    float* q_idx = (float*) malloc(sizeof(float) * (size_t) B * IH * ID);
    float* att = (float*) malloc(sizeof(float) * (size_t) B * QD);
    float* scores = (float*) malloc(sizeof(float) * (size_t) (m->ctx_max / m->idx_blk + 2));
    int* sel = (int*) malloc(sizeof(int) * (size_t) m->idx_topk);
    int* ids = (int*) malloc(sizeof(int) * (size_t) B * m->top_k);
    float* wts = (float*) malloc(sizeof(float) * (size_t) B * m->top_k);
    float* rl = (float*) malloc(sizeof(float) * (size_t) B * m->n_exp);
    int rc = 0;
    const float* pend_bo = NULL;
    const float* pend_inj = NULL;

    /* embedding rows broadcast to every stream (mtp_add_streams_bcast over a zero h2) */
    for (int t = 0; t < B; ++t) {
        int tok = toks[t];
        for (int d = 0; d < D; ++d) {
            float e;
            if (m->emb_q) {
                const int tk = (tok < 0 || tok >= m->n_vocab) ? 0 : tok;
                e = orc_f16_to_f32(m->emb_s[((size_t) tk * D + d) / 32]) * (float) m->emb_q[(size_t) tk * D + d];
            } else {
                const int tk = tok < 0 ? 0 : (tok >= m->n_vocab ? m->n_vocab - 1 : tok);
                e = orc_bf16_to_f32(m->emb[(size_t) tk * D + d]);
            }
            for (int c = 0; c < HC; ++c) R[((size_t) t * HC + c) * D + d] = e;
        }
    }

    for (int l = 0; l < m->n_layers && rc == 0; ++l) {
        const orc_layer* w = &m->layers[l];
        float* dl = dbg ? dbg + (size_t) l * 4 * B * D : NULL;     /* [mixed_a | block | mixed_f | comb] */
        if (l == 1 && m->ple) {
            /* PLE at layer 1 (src/wzy_prefill_tc.cuh:808-823), its projections on bf16 operands */
            const orc_ple_w* p = m->ple;
            float* pe = (float*) malloc(sizeof(float) * (size_t) B * D);
            orc_ple_rows(p->row, p->row_ctx, D / ORC_PLE_HEADS, p->scale, p->eos, toks, B, pos, p->tok_hist, pe);
            orc_ple_block(R, pend_bo, pend_inj, pe, p->wk, p->wv, p->norm_q, p->norm_k, p->norm_c, p->conv_w, p->hist,
                          D, HC, m->eps, B, 1, NULL);
            free(pe);
            pend_bo = NULL;
            pend_inj = NULL;
        }
        orc_hc_read_pf(R, pend_bo, pend_inj, w->hc_norm[0], w->hc_down_q[0], w->hc_down_s[0], w->hc_inj[0],
                       w->hc_up_q[0], w->hc_up_s[0], D, HC, L, m->eps, B, inj_a, mixed);
        if (dl) memcpy(dl, mixed, sizeof(float) * (size_t) B * D);
        round_rows(mixed, xb, (size_t) B * D);
        if (!w->qsa) {
            orc_pf_gemm(xb, B, D, w->qkv_q, w->qkv_s, NULL, QKV, qkv, QKV);
            orc_pf_gemm(xb, B, D, w->wgate_q, w->wgate_s, NULL, GV, z, GV);
            orc_pf_gemm(xb, B, D, NULL, NULL, w->alpha, hv, ab, 2 * hv);
            orc_pf_gemm(xb, B, D, NULL, NULL, w->beta, hv, ab + hv, 2 * hv);
            orc_gdn_step(qkv, z, ab, w->dt, w->ssm_a, w->conv_w, w->conv_hist, w->ssm, w->ssm_norm, m->eps, y,
                         m->gdn_hk, hv, B);
            round_rows(y, xb, (size_t) B * GV);
            orc_pf_gemm(xb, B, GV, w->wout_q, w->wout_s, NULL, D, block, D);
        } else {
            orc_pf_gemm(xb, B, D, w->wq_q, w->wq_s, NULL, 2 * QD, qg, 2 * QD);
            orc_pf_gemm(xb, B, D, w->wk_q, w->wk_s, NULL, KVD, kk, KVD);
            orc_pf_gemm(xb, B, D, w->wv_q, w->wv_s, NULL, KVD, vv, KVD);
            orc_pf_gemm(xb, B, D, NULL, NULL, w->idx_k, ID, idx_raw, ID);
            orc_pf_gemm(xb, B, D, NULL, NULL, w->idx_q, IH * ID, q_idx, IH * ID);
            for (int t = 0; t < B; ++t) {
                const int p = pos + t;
                for (int h = 0; h < m->qsa_qh; ++h)
                    orc_head_norm_rope(qg + (size_t) t * 2 * QD + (size_t) h * 2 * hd, hd, w->q_norm, m->cos_tab,
                                       m->sin_tab, p, m->n_rot, m->eps);
                for (int j = 0; j < m->qsa_kvh; ++j)
                    orc_head_norm_rope(kk + (size_t) t * KVD + (size_t) j * hd, hd, w->k_norm, m->cos_tab, m->sin_tab, p,
                                       m->n_rot, m->eps);
                for (int i = 0; i < IH; ++i)
                    orc_head_norm_rope(q_idx + (size_t) t * IH * ID + (size_t) i * ID, ID, w->idx_qn, m->cos_tab,
                                       m->sin_tab, p, m->n_rot, m->eps);
                orc_kv_quant_row(kk + (size_t) t * KVD, KVD, w->kq + (size_t) p * KVD, w->ks + (size_t) p * (KVD / 64));
                orc_kv_quant_row(vv + (size_t) t * KVD, KVD, w->vq + (size_t) p * KVD, w->vs + (size_t) p * (KVD / 64));
                orc_indexer_append(idx_raw + (size_t) t * ID, w->idx_kn, m->cos_tab, m->sin_tab, p, ID, m->idx_blk,
                                   m->n_rot, m->eps, w->idx_tail, w->idx_dead, w->idx_pooled);
            }
            for (int t = 0; t < B; ++t) {
                const int n_kv = pos + t + 1;
                if (n_kv > m->idx_topk)
                    orc_block_scores(w->idx_pooled, w->idx_dead, q_idx + (size_t) t * IH * ID, n_kv, IH, ID, m->idx_blk,
                                     scores);
                const int n = orc_topk_select(scores, n_kv, m->idx_blk, m->idx_topk, sel);
                if (margins) margins[((size_t) l * B + t) * 2 + 1] = orc_select_margin(scores, n_kv, m->idx_blk, m->idx_topk);
                orc_attend_pf(qg + (size_t) t * 2 * QD, w->kq, w->ks, w->vq, w->vs, sel, n, m->qsa_qh, m->qsa_kvh, hd,
                              att + (size_t) t * QD);
            }
            round_rows(att, xb, (size_t) B * QD);
            orc_pf_gemm(xb, B, QD, w->wo_q, w->wo_s, NULL, D, block, D);
        }
        if (dl) memcpy(dl + (size_t) B * D, block, sizeof(float) * (size_t) B * D);
        /* FFN half: the attention block is written into R, then the FFN read (nothing pending) */
        orc_hc_write(R, block, inj_a, D, HC, B);
        orc_hc_read_pf(R, NULL, NULL, w->hc_norm[1], w->hc_down_q[1], w->hc_down_s[1], w->hc_inj[1], w->hc_up_q[1],
                       w->hc_up_s[1], D, HC, L, m->eps, B, inj_f, mixed);
        if (dl) memcpy(dl + (size_t) 2 * B * D, mixed, sizeof(float) * (size_t) B * D);
        orc_moe_weights mw;
        mw.n_embd = D; mw.n_ff = m->n_ff; mw.n_exp = m->n_exp; mw.top_k = m->top_k;
        mw.router = w->router; mw.sgate = w->sgate; mw.blobs = NULL;
        mw.sh_gate_q = w->sh_gate_q; mw.sh_gate_s = w->sh_gate_s; mw.sh_up_q = w->sh_up_q; mw.sh_up_s = w->sh_up_s;
        mw.sh_down_q = w->sh_down_q; mw.sh_down_s = w->sh_down_s;
        rc = orc_moe_prefill_fn(&mw, mixed, B, comb, ids, wts, rl, m->blob, m->blob_ctx, l);
        if (margins)
            for (int t = 0; t < B; ++t) {
                margins[((size_t) l * B + t) * 2 + 0] = orc_kth_gap(rl + (size_t) t * m->n_exp, m->n_exp, m->top_k);
                if (!w->qsa) margins[((size_t) l * B + t) * 2 + 1] = 1e30f;
            }
        if (dl) memcpy(dl + (size_t) 3 * B * D, comb, sizeof(float) * (size_t) B * D);
        pend_bo = comb;
        pend_inj = inj_f;
    }
    if (rc == 0 && pend_bo) orc_hc_write(R, pend_bo, pend_inj, D, HC, B);
    free(inj_a); free(inj_f); free(mixed); free(xb); free(block); free(comb); free(qkv); free(z); free(ab); free(y);
    free(qg); free(kk); free(vv); free(idx_raw); free(q_idx); free(att); free(scores); free(sel); free(ids); free(wts); free(rl);
    return rc;
}

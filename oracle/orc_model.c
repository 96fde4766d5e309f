/* orc_model.c -- CPU oracle of one decode window through the whole model (StageGpu::record_forward,
 * src/wzy_stage_v2.cuh:476-857, with every expert resident and the head run).  TEST
 * INFRASTRUCTURE ONLY (see wzy_oracle.h). */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "wzy_oracle.h"

static int cmp_desc_f(const void* a, const void* b) {
    const float x = *(const float*) a, y = *(const float*) b;
    return x < y ? 1 : (x > y ? -1 : 0);
}

/* Gap between the k-th and (k+1)-th largest of v[0..n) (k >= 1), +huge if n <= k. */
float orc_kth_gap(const float* v, int n, int k) {
    if (n <= k) return 1e30f;
    float* s = (float*) malloc(sizeof(float) * (size_t) n);
    memcpy(s, v, sizeof(float) * (size_t) n);
    qsort(s, (size_t) n, sizeof(float), cmp_desc_f);
    const float g = s[k - 1] - s[k];
    free(s);
    return g;
}

/* Relative score gap around the top-k threshold block of one row (how far a block score would have
 * to move to change the selected cell set); +huge when the row selects every cell. */
float orc_select_margin(const float* scores, int n_kv, int blk, int topk) {
    if (n_kv <= topk) return 1e30f;
    const int nbid = n_kv / blk, nb = nbid + 1;
    float* s = (float*) malloc(sizeof(float) * (size_t) nb);
    int* w = (int*) malloc(sizeof(int) * (size_t) nb);
    int n = 0;
    for (int b = 0; b < nb; ++b) {
        const int wb = b < nbid ? blk : n_kv - nbid * blk;
        if (wb > 0) { s[n] = scores[b]; w[n] = wb; ++n; }
    }
    /* sort (score, weight) pairs by score, descending (insertion sort keeps it dependency-free) */
    for (int i = 1; i < n; ++i) {
        const float sv = s[i];
        const int wv = w[i];
        int j = i - 1;
        while (j >= 0 && s[j] < sv) { s[j + 1] = s[j]; w[j + 1] = w[j]; --j; }
        s[j + 1] = sv; w[j + 1] = wv;
    }
    if (n == 0) {
        free(s);
        free(w);
        return 1e30f;
    }
    long cum = 0;
    int jt = n - 1;
    for (int i = 0; i < n; ++i) {
        cum += w[i];
        if (cum >= topk) { jt = i; break; }
    }
    float gap = 1e30f;
    if (jt > 0) gap = fminf(gap, s[jt - 1] - s[jt]);
    if (jt + 1 < n) gap = fminf(gap, s[jt] - s[jt + 1]);
    const float scale = fmaxf(fabsf(s[jt]), 1e-30f);
    free(s);
    free(w);
    return gap / scale;
}

static void q8_gemv_f(const int8_t* q, const uint16_t* s, const float* x, float* y, int rows, int cols, int T) {
    int8_t* xq = (int8_t*) malloc((size_t) T * cols);
    float* xs = (float*) malloc(sizeof(float) * (size_t) T * cols / 32);
    orc_quant_act(x, cols, T, xq, xs, NULL, NULL);
    orc_gemv_q8(q, s, xq, xs, y, rows, cols, T);
    free(xq);
    free(xs);
}

int orc_model_forward(const orc_model* m, int pos, const int* toks, int T, float* logits, int* greedy,
                      float* pre_head) {
    return orc_model_forward_dbg(m, pos, toks, T, logits, greedy, pre_head, NULL, NULL);
}

int orc_model_forward_dbg(const orc_model* m, int pos, const int* toks, int T, float* logits, int* greedy,
                          float* pre_head, float* dbg, float* margins) {
    orc_trace tr;
    memset(&tr, 0, sizeof tr);
    tr.dbg = dbg;
    tr.margins = margins;
    return orc_model_forward_trace(m, pos, toks, T, logits, greedy, pre_head, &tr);
}

int orc_model_forward_trace(const orc_model* m, int pos, const int* toks, int T, float* logits, int* greedy,
                            float* pre_head, const orc_trace* tr) {
    float* dbg = tr ? tr->dbg : NULL;
    float* margins = tr ? tr->margins : NULL;
    const int D = m->n_embd, HC = m->hc, HCD = HC * D, L = m->hc_lr;
    const int QKV = 2 * m->gdn_hk * 128 + m->gdn_hv * 128, GV = m->gdn_hv * 128;
    const int QD = m->qsa_qh * m->qsa_hd, KVD = m->qsa_kvh * m->qsa_hd, hd = m->qsa_hd;
    const int ID = m->idx_dim, IH = m->idx_heads;
    if (T < 1 || T > 8 || pos < 0 || pos + T > m->ctx_max) return -1;

    float* R[2];
    R[0] = (float*) malloc(sizeof(float) * (size_t) T * HCD);
    R[1] = (float*) malloc(sizeof(float) * (size_t) T * HCD);
    float* nsc = (float*) malloc(sizeof(float) * (size_t) T * HC);
    float* lo = (float*) malloc(sizeof(float) * (size_t) T * L);
    float* inj_a = (float*) malloc(sizeof(float) * (size_t) T * HC);
    float* inj_f = (float*) malloc(sizeof(float) * (size_t) T * HC);
    float* mixed = (float*) malloc(sizeof(float) * (size_t) T * D);
    float* block = (float*) malloc(sizeof(float) * (size_t) T * D);
    float* comb = (float*) malloc(sizeof(float) * (size_t) T * D);
    float* emb = (float*) malloc(sizeof(float) * (size_t) T * D);
    float* qkv = (float*) malloc(sizeof(float) * (size_t) T * QKV);
    float* z = (float*) malloc(sizeof(float) * (size_t) T * GV);
    float* ab = (float*) malloc(sizeof(float) * (size_t) T * 2 * m->gdn_hv);
    float* tmp = (float*) malloc(sizeof(float) * (size_t) T * (m->gdn_hv > 0 ? m->gdn_hv : 1));
    float* y = (float*) malloc(sizeof(float) * (size_t) T * GV);
    float* qg = (float*) malloc(sizeof(float) * (size_t) T * 2 * QD);
    float* kk = (float*) malloc(sizeof(float) * (size_t) T * KVD);
    float* vv = (float*) malloc(sizeof(float) * (size_t) T * KVD);
    float* idx_raw = (float*) malloc(sizeof(float) * (size_t) T * ID);
    float* q_idx = (float*) malloc(sizeof(float) * (size_t) T * IH * ID);
    float* att = (float*) malloc(sizeof(float) * (size_t) T * QD);
    float* scores = (float*) malloc(sizeof(float) * (size_t) (m->ctx_max / m->idx_blk + 2));
    int* sel = (int*) malloc(sizeof(int) * (size_t) m->idx_topk);
    int8_t* kq = (int8_t*) malloc((size_t) KVD);
    uint16_t* ks = (uint16_t*) malloc(sizeof(uint16_t) * (size_t) KVD / 64);
    int rc = 0, cur = 0, qsa_i = 0;
    const int max_b = m->ctx_max / m->idx_blk + 2;
    const float* pend_bo = NULL;
    const float* pend_inj = NULL;

    for (int t = 0; t < T; ++t) {
        int tok = toks[t];
        if (m->emb_q) {                                    /* stage_one_emb, src/wzy_engine_v2.cu:861-873 */
            if (tok < 0 || tok >= m->n_vocab) tok = 0;
            for (int d = 0; d < D; ++d)
                emb[(size_t) t * D + d] = orc_f16_to_f32(m->emb_s[((size_t) tok * D + d) / 32]) *
                                          (float) m->emb_q[(size_t) tok * D + d];
            continue;
        }
        tok = tok < 0 ? 0 : (tok >= m->n_vocab ? m->n_vocab - 1 : tok);
        for (int d = 0; d < D; ++d) emb[(size_t) t * D + d] = orc_bf16_to_f32(m->emb[(size_t) tok * D + d]);
    }

    for (int l = 0; l < m->n_layers && rc == 0; ++l) {
        const orc_layer* w = &m->layers[l];
        if (l == 1 && m->ple) {
            /* PLE at layer 1 (src/wzy_stage_v2.cuh:583-597): the pending FFN write of layer 0 is folded
             * into the streams first, the block adds to them, and the attention read folds nothing */
            const orc_ple_w* p = m->ple;
            float* pe = (float*) malloc(sizeof(float) * (size_t) T * D);
            orc_ple_rows(p->row, p->row_ctx, D / ORC_PLE_HEADS, p->scale, p->eos, toks, T, pos, p->tok_hist, pe);
            orc_ple_block(R[cur], pend_bo, pend_inj, pe, p->wk, p->wv, p->norm_q, p->norm_k, p->norm_c, p->conv_w,
                          p->hist, D, HC, m->eps, T, 0, NULL);
            free(pe);
            pend_bo = NULL;
            pend_inj = NULL;
        }
        /* attention half */
        orc_hc_read(l == 0 ? NULL : R[cur], l == 0 ? emb : NULL, pend_bo, pend_inj, w->hc_norm[0], w->hc_down_q[0],
                    w->hc_down_s[0], w->hc_inj[0], w->hc_up_q[0], w->hc_up_s[0], D, HC, L, m->eps, T, R[cur ^ 1], nsc, lo,
                    inj_a, mixed);
        cur ^= 1;
        float* dl = dbg ? dbg + (size_t) l * 4 * T * D : NULL;   /* [mixed_a | block | mixed_f | comb] */
        if (dl) memcpy(dl, mixed, sizeof(float) * (size_t) T * D);
        if (!w->qsa) {
            const int hv = m->gdn_hv;
            q8_gemv_f(w->qkv_q, w->qkv_s, mixed, qkv, QKV, D, T);
            q8_gemv_f(w->wgate_q, w->wgate_s, mixed, z, GV, D, T);
            orc_gemv_bf16(w->alpha, mixed, tmp, hv, D, T);
            for (int t = 0; t < T; ++t) memcpy(ab + (size_t) t * 2 * hv, tmp + (size_t) t * hv, sizeof(float) * hv);
            orc_gemv_bf16(w->beta, mixed, tmp, hv, D, T);
            for (int t = 0; t < T; ++t) memcpy(ab + (size_t) t * 2 * hv + hv, tmp + (size_t) t * hv, sizeof(float) * hv);
            orc_gdn_step(qkv, z, ab, w->dt, w->ssm_a, w->conv_w, w->conv_hist, w->ssm, w->ssm_norm, m->eps, y, m->gdn_hk,
                         hv, T);
            q8_gemv_f(w->wout_q, w->wout_s, y, block, D, GV, T);
        } else {
            q8_gemv_f(w->wq_q, w->wq_s, mixed, qg, 2 * QD, D, T);
            q8_gemv_f(w->wk_q, w->wk_s, mixed, kk, KVD, D, T);
            q8_gemv_f(w->wv_q, w->wv_s, mixed, vv, KVD, D, T);
            orc_gemv_bf16(w->idx_k, mixed, idx_raw, ID, D, T);
            orc_gemv_bf16(w->idx_q, mixed, q_idx, IH * ID, D, T);
            for (int t = 0; t < T; ++t) {
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
            for (int t = 0; t < T; ++t) {
                const int n_kv = pos + t + 1;
                if (n_kv > m->idx_topk)
                    orc_block_scores(w->idx_pooled, w->idx_dead, q_idx + (size_t) t * IH * ID, n_kv, IH, ID, m->idx_blk,
                                     scores);
                const int n = orc_topk_select(scores, n_kv, m->idx_blk, m->idx_topk, sel);
                if (margins) margins[((size_t) l * T + t) * 2 + 1] = orc_select_margin(scores, n_kv, m->idx_blk, m->idx_topk);
                if (tr && tr->scores) {
                    float* dst = tr->scores + ((size_t) qsa_i * T + t) * max_b;
                    memset(dst, 0, sizeof(float) * (size_t) max_b);
                    if (n_kv > m->idx_topk)
                        memcpy(dst, scores, sizeof(float) * (size_t) (n_kv / m->idx_blk + 1));
                }
                if (tr && tr->sel) {
                    int* dst = tr->sel + ((size_t) qsa_i * T + t) * m->idx_topk;
                    memset(dst, 0, sizeof(int) * (size_t) m->idx_topk);
                    memcpy(dst, sel, sizeof(int) * (size_t) n);
                }
                if (tr && tr->n_sel) tr->n_sel[(size_t) qsa_i * T + t] = n;
                /* src/wzy_stage_v2.cuh:679-683: past the VRAM ring the whole window takes the GQA
                 * kernel (fp16 operands), else the fp32 int8 kernel */
                if (m->attn_f16_above > 0 && pos + T > m->attn_f16_above)
                    orc_attend_pf(qg + (size_t) t * 2 * QD, w->kq, w->ks, w->vq, w->vs, sel, n, m->qsa_qh, m->qsa_kvh,
                                  hd, att + (size_t) t * QD);
                else
                    orc_attend(qg + (size_t) t * 2 * QD, w->kq, w->ks, w->vq, w->vs, sel, n, m->qsa_qh, m->qsa_kvh, hd,
                               att + (size_t) t * QD);
            }
            q8_gemv_f(w->wo_q, w->wo_s, att, block, D, QD, T);
            ++qsa_i;
        }
        /* FFN half */
        if (dl) memcpy(dl + (size_t) T * D, block, sizeof(float) * (size_t) T * D);
        orc_hc_read(R[cur], NULL, block, inj_a, w->hc_norm[1], w->hc_down_q[1], w->hc_down_s[1], w->hc_inj[1],
                    w->hc_up_q[1], w->hc_up_s[1], D, HC, L, m->eps, T, R[cur ^ 1], nsc, lo, inj_f, mixed);
        cur ^= 1;
        if (dl) memcpy(dl + (size_t) 2 * T * D, mixed, sizeof(float) * (size_t) T * D);
        orc_moe_weights mw;
        mw.n_embd = D; mw.n_ff = m->n_ff; mw.n_exp = m->n_exp; mw.top_k = m->top_k;
        mw.router = w->router; mw.sgate = w->sgate; mw.blobs = NULL;
        mw.sh_gate_q = w->sh_gate_q; mw.sh_gate_s = w->sh_gate_s; mw.sh_up_q = w->sh_up_q; mw.sh_up_s = w->sh_up_s;
        mw.sh_down_q = w->sh_down_q; mw.sh_down_s = w->sh_down_s;
        int ids[8 * 64];
        float wts[8 * 64];
        float* rl = (float*) malloc(sizeof(float) * (size_t) T * m->n_exp);
        rc = orc_moe_block_fn(&mw, mixed, T, comb, ids, wts, rl, NULL, m->blob, m->blob_ctx, l);
        if (margins)
            for (int t = 0; t < T; ++t) {
                margins[((size_t) l * T + t) * 2 + 0] = orc_kth_gap(rl + (size_t) t * m->n_exp, m->n_exp, m->top_k);
                if (!w->qsa) margins[((size_t) l * T + t) * 2 + 1] = 1e30f;
            }
        if (tr && tr->router_logits)
            memcpy(tr->router_logits + (size_t) l * T * m->n_exp, rl, sizeof(float) * (size_t) T * m->n_exp);
        if (tr && tr->ids) memcpy(tr->ids + (size_t) l * T * m->top_k, ids, sizeof(int) * (size_t) T * m->top_k);
        if (tr && tr->wts) memcpy(tr->wts + (size_t) l * T * m->top_k, wts, sizeof(float) * (size_t) T * m->top_k);
        free(rl);
        if (dl) memcpy(dl + (size_t) 3 * T * D, comb, sizeof(float) * (size_t) T * D);
        pend_bo = comb;
        pend_inj = inj_f;
    }
    if (rc == 0) {
        orc_hc_read(R[cur], NULL, pend_bo, pend_inj, m->head_norm, m->head_down_q, m->head_down_s, NULL, m->head_up_q,
                    m->head_up_s, D, HC, L, m->eps, T, R[cur ^ 1], nsc, lo, NULL, mixed);
        cur ^= 1;
        if (pre_head) memcpy(pre_head, R[cur], sizeof(float) * (size_t) T * HCD);
        if (m->head_q) q8_gemv_f(m->head_q, m->head_s, mixed, logits, m->n_vocab, D, T);
        else orc_gemv_bf16(m->head, mixed, logits, m->n_vocab, D, T);
        if (greedy) orc_row_argmax(logits, m->n_vocab, T, greedy);
    }
    free(R[0]); free(R[1]); free(nsc); free(lo); free(inj_a); free(inj_f); free(mixed); free(block); free(comb);
    free(emb); free(qkv); free(z); free(ab); free(tmp); free(y); free(qg); free(kk); free(vv); free(idx_raw);
    free(q_idx); free(att); free(scores); free(sel); free(kq); free(ks);
    return rc;
}

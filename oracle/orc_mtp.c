/* orc_mtp.c -- CPU oracle of the MTP speculative drafter (MtpEngine, src/wzy_mtp.cuh:405-754): Q2_0
 * expert GEMVs, the front half (K/V append of T cells into the 1,024-cell ring), the rest of row 0
 * and the draft head with its top-1 reduction.  TEST INFRASTRUCTURE ONLY (see wzy_oracle.h). */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "wzy_oracle.h"

static float silu_m(float x) { return x / (1.0f + expf(-x)); }
static float sigm_m(float x) { return 1.0f / (1.0f + expf(-x)); }

/* Q2_0 expert blob (src/wzy_mtp.cuh:6-10): gate/up codes [2F rows, gate and up interleaved][D/4],
 * down codes [D][F/4], gate/up fp16 scales [2F][D/64], down fp16 scales [D][F/64].  Value k of a
 * 32-value chunk is bits 2(k%4)..2(k%4)+1 of the chunk's byte k/4; weight = (code - 1) * scale of
 * its 64-value group. */
size_t orc_q2_blob_bytes(int D, int F) { return (size_t) 3 * D * F / 4 + (size_t) 3 * D * F / 64 * 2; }

int orc_q2_code(const uint8_t* codes, int k) { return (codes[k >> 2] >> (2 * (k & 3))) & 3; }

/* sum_c d(c/2) * xs[c] * (sum_i code_i x_i - sum_i x_i) over the row's cols/32 chunks
 * (mtp_row_dot_q2 / mtp_exp_gu_quant_q2, src/wzy_mtp.cuh:59-80,85-158) */
static double q2_row_dot(const uint8_t* codes, const uint16_t* scales, const int8_t* xq, const float* xs, int cols) {
    double acc = 0.0;
    for (int c = 0; c < cols / 32; ++c) {
        int s = 0, hx = 0;
        for (int i = 0; i < 32; ++i) {
            s += orc_q2_code(codes + (size_t) c * 8, i) * (int) xq[32 * c + i];
            hx += (int) xq[32 * c + i];
        }
        const float d = orc_f16_to_f32(scales[c >> 1]);
        acc += (double) (d * xs[c] * (float) (s - hx));
    }
    return acc;
}

static void quant32_m(const float* x, int n, int8_t* q, float* s) {
    orc_quant_act(x, n, 1, q, s, NULL, NULL);
}

/* Gate/up + SwiGLU + per-32 requant of one Q2_0 expert on per-32 int8 activations:
 * act[r] = silu(g_r) * u_r, then 32 activations per block: d = amax/127, q = rint(act/d). */
void orc_q2_expert_gate_up(const uint8_t* blob, int D, int F, const int8_t* xq32, const float* xs32, int8_t* aq32,
                           float* as32, float* act_out) {
    const uint8_t* codes = blob;
    const uint16_t* gus = (const uint16_t*) (blob + (size_t) 2 * F * (D / 4) + (size_t) D * (F / 4));
    float* act = (float*) malloc(sizeof(float) * (size_t) F);
    for (int r = 0; r < F; ++r) {
        const float g = (float) q2_row_dot(codes + (size_t) (2 * r) * (D / 4), gus + (size_t) (2 * r) * (D / 64), xq32,
                                           xs32, D);
        const float u = (float) q2_row_dot(codes + (size_t) (2 * r + 1) * (D / 4), gus + (size_t) (2 * r + 1) * (D / 64),
                                           xq32, xs32, D);
        act[r] = silu_m(g) * u;
    }
    if (act_out) memcpy(act_out, act, sizeof(float) * (size_t) F);
    quant32_m(act, F, aq32, as32);
    free(act);
}

/* Down projection of one Q2_0 expert: out[d] = sum over the F/32 chunks (mtp_exp_down_2r_q2,
 * src/wzy_mtp.cuh:160-207). */
void orc_q2_expert_down(const uint8_t* blob, int D, int F, const int8_t* aq32, const float* as32, float* out) {
    const uint8_t* dcodes = blob + (size_t) 2 * F * (D / 4);
    const uint16_t* dsc = (const uint16_t*) (blob + (size_t) 2 * F * (D / 4) + (size_t) D * (F / 4) +
                                             (size_t) 2 * F * (D / 64) * 2);
    for (int d = 0; d < D; ++d)
        out[d] = (float) q2_row_dot(dcodes + (size_t) d * (F / 4), dsc + (size_t) d * (F / 64), aq32, as32, F);
}

/* x * rsqrt(mean(x^2) + eps) * g (mtp_rms_norm_rows, src/wzy_mtp.cuh:16-37) */
static void rms_rows(const float* x, const float* g, float* y, int cols, float eps) {
    double ss = 0.0;
    for (int d = 0; d < cols; ++d) ss += (double) x[d] * x[d];
    const float sc = 1.0f / sqrtf((float) ss / (float) cols + eps);
    for (int d = 0; d < cols; ++d) y[d] = x[d] * sc * g[d];
}

static void q8_proj(const int8_t* q, const uint16_t* s, const float* x, float* y, int rows, int cols) {
    int8_t* xq = (int8_t*) malloc((size_t) cols);
    float* xs = (float*) malloc(sizeof(float) * (size_t) cols / 32);
    quant32_m(x, cols, xq, xs);
    orc_gemv_q8(q, s, xq, xs, y, rows, cols, 1);
    free(xq);
    free(xs);
}

/* Front half for T cells at positions pos .. pos+T-1 (run_front_kv, src/wzy_mtp.cuh:658-683):
 * e2 = fc_emb(rms(emb(tok)) * pre_norm_emb); per stream c: h2[c] = fc_hid(rms(Rin[c]) * pre_norm_hid[c]);
 * R = h2 + e2; attention HC read of R -> mixed, inject; k, v projections of mixed, RMSNorm + RoPE of the
 * k heads, INT8 append into ring slot p % ring.  R, mixed and inj of every row are returned. */
void orc_mtp_front(orc_mtp* m, int pos, const int* toks, const float* Rin, int T, float* R, float* mixed, float* inj) {
    const int D = m->n_embd, HC = m->hc, HCD = HC * D, KVD = m->qsa_kvh * m->qsa_hd;
    float* en = (float*) malloc(sizeof(float) * (size_t) D);
    float* e2 = (float*) malloc(sizeof(float) * (size_t) D);
    float* hn = (float*) malloc(sizeof(float) * (size_t) D);
    float* h2 = (float*) malloc(sizeof(float) * (size_t) D);
    float* emb = (float*) malloc(sizeof(float) * (size_t) D);
    float* nsc = (float*) malloc(sizeof(float) * (size_t) HC);
    float* lo = (float*) malloc(sizeof(float) * (size_t) m->hc_lr);
    float* Rh = (float*) malloc(sizeof(float) * (size_t) HCD);
    float* kk = (float*) malloc(sizeof(float) * (size_t) KVD);
    float* vv = (float*) malloc(sizeof(float) * (size_t) KVD);
    for (int t = 0; t < T; ++t) {
        int tok = toks[t];
        if (tok < 0 || tok >= m->n_vocab) tok = 0; /* stage_one_emb, src/wzy_engine_v2.cu:862-863 */
        for (int d = 0; d < D; ++d)
            emb[d] = m->emb_q ? orc_f16_to_f32(m->emb_s[((size_t) tok * D + d) / 32]) * (float) m->emb_q[(size_t) tok * D + d]
                              : orc_bf16_to_f32(m->emb[(size_t) tok * D + d]);
        rms_rows(emb, m->pre_norm_emb, en, D, m->eps);
        q8_proj(m->fc_emb_q, m->fc_emb_s, en, e2, D, D);
        for (int c = 0; c < HC; ++c) {
            rms_rows(Rin + ((size_t) t * HC + c) * D, m->pre_norm_hid + (size_t) c * D, hn, D, m->eps);
            q8_proj(m->fc_hid_q, m->fc_hid_s, hn, h2, D, D);
            for (int d = 0; d < D; ++d) Rh[(size_t) c * D + d] = h2[d] + e2[d];
        }
        float* Rt = R + (size_t) t * HCD;
        orc_hc_read(Rh, NULL, NULL, NULL, m->hc_norm[0], m->hc_down_q[0], m->hc_down_s[0], m->hc_inj[0], m->hc_up_q[0],
                    m->hc_up_s[0], D, HC, m->hc_lr, m->eps, 1, Rt, nsc, lo, inj + (size_t) t * HC,
                    mixed + (size_t) t * D);
        const float* mx = mixed + (size_t) t * D;
        q8_proj(m->wk_q, m->wk_s, mx, kk, KVD, D);
        q8_proj(m->wv_q, m->wv_s, mx, vv, KVD, D);
        const int p = pos + t;
        for (int j = 0; j < m->qsa_kvh; ++j)
            orc_head_norm_rope(kk + (size_t) j * m->qsa_hd, m->qsa_hd, m->k_norm, m->cos_tab, m->sin_tab, p, m->n_rot,
                               m->eps);
        const int slot = p % m->ring;
        orc_kv_quant_row(kk, KVD, m->kq + (size_t) slot * KVD, m->ks + (size_t) slot * (KVD / 64));
        orc_kv_quant_row(vv, KVD, m->vq + (size_t) slot * KVD, m->vs + (size_t) slot * (KVD / 64));
    }
    free(en); free(e2); free(hn); free(h2); free(emb); free(nsc); free(lo); free(Rh); free(kk); free(vv);
}

/* One full draft step at cell `pos` (front of one row + run_rest_row0, src/wzy_mtp.cuh:687-733, and
 * the head reduction mtp_head_reduce_online_part1 / mtp_head_finalize, :293-403):
 * q projection + RMSNorm + RoPE; attention over the ring cells max(floor, pos+1-ring) .. pos
 * (softmax of q.k/16, times sigmoid(gate)); o projection; MLP HC read folding (o, inject); router
 * top-k + shared expert + Q2_0 experts -> comb; mixer HC read folding (comb, MLP inject) -> sample
 * and the next step's residual R_out; draft-head Q8 logits over n_dv rows; argmax (ties -> lower
 * row) and prob = 1 / max(sum_i exp(l_i - l_max), 1); the token is dvocab[argmax]. */
int orc_mtp_step(orc_mtp* m, int pos, int tok, const float* Rin, float* R_out, float* sample, float* logits,
                 int* out_tok, float* out_prob) {
    const int D = m->n_embd, HC = m->hc, HCD = HC * D, hd = m->qsa_hd, QD = m->qsa_qh * hd;
    const int E = m->n_exp, K = m->top_k, F = m->n_ff;
    float* R = (float*) malloc(sizeof(float) * (size_t) HCD);
    float* R2 = (float*) malloc(sizeof(float) * (size_t) HCD);
    float* mixed = (float*) malloc(sizeof(float) * (size_t) D);
    float* mixed2 = (float*) malloc(sizeof(float) * (size_t) D);
    float inj[16], inj2[16], nsc[16];
    float* lo = (float*) malloc(sizeof(float) * (size_t) m->hc_lr);
    float* qg = (float*) malloc(sizeof(float) * (size_t) 2 * QD);
    float* att = (float*) malloc(sizeof(float) * (size_t) QD);
    float* bo = (float*) malloc(sizeof(float) * (size_t) D);
    float* comb = (float*) malloc(sizeof(float) * (size_t) D);
    float* part = (float*) malloc(sizeof(float) * (size_t) D);
    float* rl = (float*) malloc(sizeof(float) * (size_t) E);
    int* sel = (int*) malloc(sizeof(int) * (size_t) m->ring);
    int8_t* q32 = (int8_t*) malloc((size_t) D);
    float* s32 = (float*) malloc(sizeof(float) * (size_t) D / 32);
    int8_t* aq = (int8_t*) malloc((size_t) F);
    float* as = (float*) malloc(sizeof(float) * (size_t) F / 32);
    float* sff = (float*) malloc(sizeof(float) * (size_t) F);
    float* sup = (float*) malloc(sizeof(float) * (size_t) F);
    float* shared = (float*) malloc(sizeof(float) * (size_t) D);
    int ids[64];
    float wts[64];
    orc_mtp_front(m, pos, &tok, Rin, 1, R, mixed, inj);
    q8_proj(m->wq_q, m->wq_s, mixed, qg, 2 * QD, D);
    for (int h = 0; h < m->qsa_qh; ++h)
        orc_head_norm_rope(qg + (size_t) h * 2 * hd, hd, m->q_norm, m->cos_tab, m->sin_tab, pos, m->n_rot, m->eps);
    const int n_kv = pos + 1;
    int p0 = n_kv - m->ring;
    if (p0 < 0) p0 = 0;
    if (p0 < m->kv_floor) p0 = m->kv_floor;
    const int width = n_kv - p0;
    for (int i = 0; i < width; ++i) sel[i] = (p0 + i) % m->ring;
    orc_attend(qg, m->kq, m->ks, m->vq, m->vs, sel, width, m->qsa_qh, m->qsa_kvh, hd, att);
    q8_proj(m->wo_q, m->wo_s, att, bo, D, QD);
    orc_hc_read(R, NULL, bo, inj, m->hc_norm[1], m->hc_down_q[1], m->hc_down_s[1], m->hc_inj[1], m->hc_up_q[1],
                m->hc_up_s[1], D, HC, m->hc_lr, m->eps, 1, R2, nsc, lo, inj2, mixed2);
    /* MoE on mixed2: per-32 activations for the shared and the Q2_0 experts */
    quant32_m(mixed2, D, q32, s32);
    orc_gemv_bf16(m->router, mixed2, rl, E, D, 1);
    float sg = 0.f;
    orc_gemv_bf16(m->sgate, mixed2, &sg, 1, D, 1);
    orc_router_topk(rl, E, K, 1, ids, wts, NULL);
    orc_gemv_q8(m->sh_gate_q, m->sh_gate_s, q32, s32, sff, F, D, 1);
    orc_gemv_q8(m->sh_up_q, m->sh_up_s, q32, s32, sup, F, D, 1);
    for (int r = 0; r < F; ++r) sff[r] = silu_m(sff[r]) * sup[r];
    quant32_m(sff, F, aq, as);
    orc_gemv_q8(m->sh_down_q, m->sh_down_s, aq, as, shared, D, F, 1);
    const float gsh = sigm_m(sg);
    double* acc = (double*) malloc(sizeof(double) * (size_t) D);
    for (int d = 0; d < D; ++d) acc[d] = (double) shared[d] * (double) gsh;
    const size_t blob = orc_q2_blob_bytes(D, F);
    for (int k = 0; k < K; ++k) {
        if (wts[k] == 0.0f) continue;
        const uint8_t* b = m->experts + (size_t) ids[k] * blob;
        orc_q2_expert_gate_up(b, D, F, q32, s32, aq, as, NULL);
        orc_q2_expert_down(b, D, F, aq, as, part);
        for (int d = 0; d < D; ++d) acc[d] += (double) wts[k] * (double) part[d];
    }
    for (int d = 0; d < D; ++d) comb[d] = (float) acc[d];
    free(acc);
    /* mixer read folding the MoE write: R_out is the next chained step's residual */
    orc_hc_read(R2, NULL, comb, inj2, m->hc_norm[2], m->hc_down_q[2], m->hc_down_s[2], NULL, m->hc_up_q[2],
                m->hc_up_s[2], D, HC, m->hc_lr, m->eps, 1, R_out, nsc, lo, NULL, sample);
    q8_proj(m->head_q, m->head_s, sample, logits, m->n_dv, D);
    int best = 0;
    for (int i = 1; i < m->n_dv; ++i)
        if (logits[i] > logits[best]) best = i;
    double es = 0.0;
    for (int i = 0; i < m->n_dv; ++i) es += exp((double) logits[i] - (double) logits[best]);
    *out_tok = m->dvocab ? m->dvocab[best] : best;
    *out_prob = (float) (1.0 / (es > 1.0 ? es : 1.0));
    free(R); free(R2); free(mixed); free(mixed2); free(lo); free(qg); free(att); free(bo); free(comb); free(part);
    free(rl); free(sel); free(q32); free(s32); free(aq); free(as); free(sff); free(sup); free(shared);
    return 0;
}

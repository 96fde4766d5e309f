/* orc_layers.c -- CPU oracle: hyper-connection read, GDN step, QSA indexer / selection /
 * attention.  TEST INFRASTRUCTURE ONLY (see wzy_oracle.h). */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "wzy_oracle.h"

static inline float silu_f(float x) { return x / (1.0f + expf(-x)); }
static inline float sigm_f(float x) { return 1.0f / (1.0f + expf(-x)); }
static inline int clamp127(int q) { return q < -127 ? -127 : (q > 127 ? 127 : q); }

static void quant32_block(const float* x, int8_t* q, float* s) {
    float amax = 0.f;
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(x[i]));
    const float d = amax / 127.0f;
    const float inv = d > 0.f ? 127.0f / amax : 0.f;
    for (int i = 0; i < 32; ++i) q[i] = (int8_t) clamp127((int) rintf(x[i] * inv));
    *s = d;
}
/* sum_b fp16(scale_b) * xs_b * sum_i code*xq over one Q8_0 row */
static double q8_row_dot(const int8_t* codes, const uint16_t* scales, const int8_t* xq, const float* xs, int cols) {
    double acc = 0.0;
    for (int b = 0; b < cols / 32; ++b) {
        int isum = 0;
        for (int i = 0; i < 32; ++i) isum += (int) codes[32 * b + i] * (int) xq[32 * b + i];
        acc += (double) orc_f16_to_f32(scales[b]) * (double) xs[b] * (double) isum;
    }
    return acc;
}

/* ------------------------------------------------------------------------------------------------
 * HC read: fused_gr_norm_multi + gr_down_inj_q8_t + quant_act_multi + gr_up_mean_q8_t, with the
 * pending gr_write_multi folded in (src/wzy_kernels_v2.cuh:409-454,632-827; src/wzy_stage_v2.cuh:
 * 463-470,572,693-694).
 * ---------------------------------------------------------------------------------------------- */
void orc_hc_read(const float* R_in, const float* emb_rows, const float* bo, const float* inj_prev, const float* norm_w,
                 const int8_t* down_q, const uint16_t* down_s, const uint16_t* inj_w, const int8_t* up_q,
                 const uint16_t* up_s, int D, int HC, int HCLR, float eps, int T, float* R_out, float* nsc, float* lo,
                 float* inj, float* mixed) {
    const int HCD = HC * D;
    float* xn = (float*) malloc(sizeof(float) * (size_t) HCD);
    int8_t* xq = (int8_t*) malloc((size_t) HCD);
    float* xs = (float*) malloc(sizeof(float) * (size_t) HCD / 32);
    int8_t* lq = (int8_t*) malloc((size_t) HCLR);
    float* ls = (float*) malloc(sizeof(float) * (size_t) HCLR / 32);
    for (int t = 0; t < T; ++t) {
        for (int c = 0; c < HC; ++c) {
            const float gw = bo ? 2.0f / (1.0f + expf(-inj_prev[t * HC + c] / (float) HC)) : 0.0f;
            float* ro = R_out + ((size_t) t * HC + c) * D;
            double ss = 0.0;
            for (int d = 0; d < D; ++d) {
                float v = R_in ? R_in[((size_t) t * HC + c) * D + d] : emb_rows[(size_t) t * D + d];
                if (bo) v = fmaf(bo[(size_t) t * D + d], gw, v);
                ro[d] = v;
                ss += (double) v * (double) v;
            }
            const float sc = 1.0f / sqrtf((float) ss / (float) D + eps);
            nsc[t * HC + c] = sc;
            for (int d = 0; d < D; ++d) xn[(size_t) c * D + d] = ro[d] * sc * norm_w[(size_t) c * D + d];
        }
        for (int b = 0; b < HCD / 32; ++b) quant32_block(xn + 32 * b, xq + 32 * b, xs + b);
#pragma omp parallel for schedule(static)
        for (int k = 0; k < HCLR; ++k) {
            const float v = (float) q8_row_dot(down_q + (size_t) k * HCD, down_s + (size_t) k * (HCD / 32), xq, xs, HCD) /
                            (float) HC;
            lo[(size_t) t * HCLR + k] = silu_f(v);
        }
        if (inj_w)
            for (int c = 0; c < HC; ++c) {
                double acc = 0.0;
                for (int j = 0; j < HCD; ++j) acc += (double) orc_bf16_to_f32(inj_w[(size_t) c * HCD + j]) * (double) xn[j];
                inj[t * HC + c] = (float) acc;
            }
        for (int b = 0; b < HCLR / 32; ++b) quant32_block(lo + (size_t) t * HCLR + 32 * b, lq + 32 * b, ls + b);
#pragma omp parallel for schedule(static)
        for (int d = 0; d < D; ++d) {
            float g[4] = {0.f, 0.f, 0.f, 0.f};
            for (int c = 0; c < HC; ++c) {
                const size_t row = (size_t) c * D + d;
                const float s = (float) q8_row_dot(up_q + row * HCLR, up_s + row * (HCLR / 32), lq, ls, HCLR);
                g[c] = xn[(size_t) c * D + d] / (1.0f + expf(-s));
            }
            /* stream pairing of the reference's shuffle tree: (g0 + g2) + (g1 + g3) */
            mixed[(size_t) t * D + d] = ((g[0] + g[2]) + (g[1] + g[3])) * 0.25f;
        }
    }
    free(xn); free(xq); free(xs); free(lq); free(ls);
}

/* ------------------------------------------------------------------------------------------------
 * GDN.  State layout S[h][i][j] (key i, value j); the reference stores [i][h][j]
 * (src/wzy_kernels_v2.cuh:923-930) -- a layout difference only.
 * recurrence: fused_gdn_step_norm_multi (src/wzy_kernels_v2.cuh:908-984), computed in fp64 per step
 * and stored back to the fp32 state.
 * ---------------------------------------------------------------------------------------------- */
static void gdn_head_step(float* S, const float* q, const float* k, const float* v, float decay, float beta,
                          const float* z, const float* gamma, float eps, float* y) {
    double kv[128], o[128];
    for (int j = 0; j < 128; ++j) kv[j] = 0.0;
    for (int i = 0; i < 128; ++i)
        for (int j = 0; j < 128; ++j) {
            const double s = (double) S[i * 128 + j] * (double) decay;
            S[i * 128 + j] = (float) s;
            kv[j] += s * (double) k[i];
        }
    double delta[128];
    for (int j = 0; j < 128; ++j) delta[j] = ((double) v[j] - kv[j]) * (double) beta;
    for (int j = 0; j < 128; ++j) o[j] = 0.0;
    for (int i = 0; i < 128; ++i)
        for (int j = 0; j < 128; ++j) {
            const double s = (double) S[i * 128 + j] + (double) k[i] * delta[j];
            S[i * 128 + j] = (float) s;
            o[j] += s * (double) q[i];
        }
    double ss = 0.0;
    float oc[128];
    for (int j = 0; j < 128; ++j) {
        oc[j] = (float) (o[j] * 0.08838834764831845);
        ss += (double) oc[j] * (double) oc[j];
    }
    const float scale = 1.0f / sqrtf((float) ss * (1.0f / 128.0f) + eps);
    for (int j = 0; j < 128; ++j) {
        const float g = gamma ? gamma[j] : 1.0f;
        const float gate = z ? sigm_f(z[j]) : 1.0f;
        y[j] = oc[j] * scale * g * gate;
    }
}

void orc_gdn_recurrence(const float* q, const float* k, const float* v, const float* decay, const float* beta,
                        const float* z, const float* gamma, float eps, float* state, float* y, int hk, int hv, int T) {
    /* value heads are independent (each owns its state slice and output columns): heads in parallel,
     * rows in order within a head -- the same arithmetic as the row-major loop */
#pragma omp parallel for schedule(static) if (T * hv >= 256)
    for (int h = 0; h < hv; ++h)
        for (int t = 0; t < T; ++t) {
            const int kh = h % hk;
            gdn_head_step(state + (size_t) h * 128 * 128, q + (size_t) t * hk * 128 + kh * 128,
                          k + (size_t) t * hk * 128 + kh * 128, v + (size_t) t * hv * 128 + h * 128, decay[t * hv + h],
                          beta[t * hv + h], z ? z + (size_t) t * hv * 128 + h * 128 : NULL, gamma, eps,
                          y + (size_t) t * hv * 128 + h * 128);
        }
}

/* conv + SiLU + L2 (fused_gdn_conv_l2_multi, src/wzy_kernels_v2.cuh:833-863), gates
 * (fused_gdn_ab_multi, :865-904), then the recurrence. */
void orc_gdn_step(const float* qkv_raw, const float* z, const float* ab_raw, const float* dt, const float* ssm_a,
                  const float* conv_w, float* conv_hist, float* state, const float* gamma, float eps, float* y, int hk,
                  int hv, int T) {
    const int QKV = 2 * hk * 128 + hv * 128;
    float* act = (float*) malloc(sizeof(float) * (size_t) T * QKV);
    for (int ch = 0; ch < QKV; ++ch) {
        float h0 = conv_hist[ch * 3], h1 = conv_hist[ch * 3 + 1], h2 = conv_hist[ch * 3 + 2];
        const float* w = conv_w + (size_t) ch * 4;
        for (int t = 0; t < T; ++t) {
            const float x = qkv_raw[(size_t) t * QKV + ch];
            const float sum = (float) ((double) h0 * w[0] + (double) h1 * w[1] + (double) h2 * w[2] + (double) x * w[3]);
            h0 = h1; h1 = h2; h2 = x;
            act[(size_t) t * QKV + ch] = silu_f(sum);
        }
        conv_hist[ch * 3] = h0; conv_hist[ch * 3 + 1] = h1; conv_hist[ch * 3 + 2] = h2;
    }
    for (int t = 0; t < T; ++t)
        for (int g = 0; g < 2 * hk; ++g) {
            float* p = act + (size_t) t * QKV + (size_t) g * 128;
            double ss = 0.0;
            for (int i = 0; i < 128; ++i) ss += (double) p[i] * p[i];
            const float r = 1.0f / sqrtf((float) ss + eps);
            for (int i = 0; i < 128; ++i) p[i] *= r;
        }
    float* q = (float*) malloc(sizeof(float) * (size_t) T * hk * 128);
    float* k = (float*) malloc(sizeof(float) * (size_t) T * hk * 128);
    float* v = (float*) malloc(sizeof(float) * (size_t) T * hv * 128);
    float* dec = (float*) malloc(sizeof(float) * (size_t) T * hv);
    float* bet = (float*) malloc(sizeof(float) * (size_t) T * hv);
    for (int t = 0; t < T; ++t) {
        memcpy(q + (size_t) t * hk * 128, act + (size_t) t * QKV, sizeof(float) * hk * 128);
        memcpy(k + (size_t) t * hk * 128, act + (size_t) t * QKV + hk * 128, sizeof(float) * hk * 128);
        memcpy(v + (size_t) t * hv * 128, act + (size_t) t * QKV + 2 * hk * 128, sizeof(float) * hv * 128);
        for (int h = 0; h < hv; ++h) {
            const float av = ab_raw[(size_t) t * 2 * hv + h] + dt[h];
            const float sp = av > 20.0f ? av : log1pf(expf(av));
            dec[t * hv + h] = expf(sp * ssm_a[h]);
            bet[t * hv + h] = sigm_f(ab_raw[(size_t) t * 2 * hv + hv + h]);
        }
    }
    orc_gdn_recurrence(q, k, v, dec, bet, z, gamma, eps, state, y, hk, hv, T);
    free(act); free(q); free(k); free(v); free(dec); free(bet);
}

/* ------------------------------------------------------------------------------------------------
 * QSA
 * ---------------------------------------------------------------------------------------------- */
/* RoPE tables: fp64 angles p * theta^(-2i/n_rot) rounded to fp32 (src/wzy_qsa_256k.cuh:34-46) */
void orc_rope_tables(int ctx, int n_rot, float theta, float* cos_tab, float* sin_tab) {
    const int half = n_rot / 2;
    for (int p = 0; p < ctx; ++p)
        for (int i = 0; i < half; ++i) {
            const double ang = (double) p * pow((double) theta, -2.0 * (double) i / (double) n_rot);
            cos_tab[(size_t) p * half + i] = (float) cos(ang);
            sin_tab[(size_t) p * half + i] = (float) sin(ang);
        }
}

/* fused_head_norm_rope_multi (src/wzy_qsa_256k.cuh:50-82) on one head vector */
void orc_head_norm_rope(float* p, int hd, const float* gamma, const float* cos_tab, const float* sin_tab, int pos,
                        int n_rot, float eps) {
    double ss = 0.0;
    for (int i = 0; i < hd; ++i) ss += (double) p[i] * p[i];
    const float sc = 1.0f / sqrtf((float) ss / (float) hd + eps);
    for (int i = 0; i < hd; ++i) p[i] = p[i] * (sc * gamma[i]);
    const int half = n_rot / 2;
    for (int i = 0; i < half; ++i) {
        const float c = cos_tab[(size_t) pos * half + i], s = sin_tab[(size_t) pos * half + i];
        const float a = p[i], d = p[i + half];
        p[i] = a * c - d * s;
        p[i + half] = a * s + d * c;
    }
}

/* kv_append_int8_multi (src/wzy_qsa_256k.cuh:86-143): per 64 elements, fp16 scale = half(amax/127),
 * q = rint(x / float(scale)) clamped to +-127 (scale 0 -> q 0). */
void orc_kv_quant_row(const float* x, int n, int8_t* q, uint16_t* s) {
    for (int g = 0; g < n / 64; ++g) {
        float amax = 0.f;
        for (int i = 0; i < 64; ++i) amax = fmaxf(amax, fabsf(x[64 * g + i]));
        const uint16_t h = orc_f32_to_f16(amax / 127.0f);
        const float d = orc_f16_to_f32(h);
        for (int i = 0; i < 64; ++i) q[64 * g + i] = (int8_t) (d > 0.f ? clamp127((int) rintf(x[64 * g + i] / d)) : 0);
        s[g] = h;
    }
}

/* qsa_indexer_append_multi (src/wzy_qsa_256k.cuh:147-209) for one position; pooled keys kept as
 * fp16 (the scorer's rounding, src/wzy_qsa_wmma.cuh:533-537). */
void orc_indexer_append(const float* raw, const float* gamma, const float* cos_tab, const float* sin_tab, int pos,
                        int dim, int blk, int n_rot, float eps, float* tail, float* dead, uint16_t* pooled) {
    orc_indexer_append_f32(raw, gamma, cos_tab, sin_tab, pos, dim, blk, n_rot, eps, tail, dead, pooled, NULL);
}

/* The same, also giving the fp32 key of the block this position completes (before its fp16 rounding)
 * in key_out [dim] when one completes (pos == 0 or pos % blk == blk - 1; else key_out is untouched),
 * so that a test can tell an fp16 rounding flip of a key near a rounding midpoint from an error. */
void orc_indexer_append_f32(const float* raw, const float* gamma, const float* cos_tab, const float* sin_tab, int pos,
                            int dim, int blk, int n_rot, float eps, float* tail, float* dead, uint16_t* pooled,
                            float* key_out) {
    float inc[128], vals[128];
    for (int d = 0; d < dim; ++d) inc[d] = orc_f16_to_f32(orc_f32_to_f16(raw[d]));
    const int slot = pos % blk;
    if (slot < blk - 1)
        for (int d = 0; d < dim; ++d) tail[slot * dim + d] = inc[d];
    if (pos == 0 || slot == blk - 1) {
        double ss = 0.0;
        float mean[128];
        for (int d = 0; d < dim; ++d) {
            float sum = (pos == 0) ? inc[d] : tail[d];
            for (int j = 1; j < blk; ++j) sum = sum + ((pos == 0 || j == blk - 1) ? inc[d] : tail[j * dim + d]);
            mean[d] = sum * (1.0f / (float) blk);
            ss += (double) mean[d] * mean[d];
        }
        const float sc = 1.0f / sqrtf((float) ss / (float) dim + eps);
        for (int d = 0; d < dim; ++d) vals[d] = sc * mean[d] * gamma[d];
        const int b = pos / blk;
        const int rope_pos = (pos == 0) ? 0 : blk * b;
        const int half = n_rot / 2;
        float y[128];
        for (int d = 0; d < dim; ++d) y[d] = vals[d];
        for (int i = 0; i < half; ++i) {
            const float c = cos_tab[(size_t) rope_pos * half + i], s = sin_tab[(size_t) rope_pos * half + i];
            y[i] = vals[i] * c - vals[i + half] * s;
            y[i + half] = vals[i] * s + vals[i + half] * c;
        }
        for (int d = 0; d < dim; ++d) pooled[(size_t) b * dim + d] = orc_f32_to_f16(y[d]);
        if (key_out)
            for (int d = 0; d < dim; ++d) key_out[d] = y[d];
        if (pos == 0)
            for (int d = 0; d < dim; ++d) dead[d] = y[d];
        else
            for (int d = 0; d < dim; ++d) pooled[(size_t) (b + 1) * dim + d] = orc_f32_to_f16(dead[d]);
    }
}

/* block scores for one query row: complete blocks b < n_kv/blk with fp16-rounded q and keys, the
 * open block against the fp32 placeholder (+1e9 when partial).  Rows with n_kv <= topk are not
 * scored (src/wzy_qsa_wmma.cuh:492-612; src/wzy_stage_v2.cuh:667-672). */
void orc_block_scores(const uint16_t* pooled, const float* dead, const float* q_idx, int n_kv, int heads, int dim,
                      int blk, float* scores) {
    const int nbid = n_kv / blk;
    for (int b = 0; b < nbid; ++b) {
        float sc = 0.f;
        for (int h = 0; h < heads; ++h) {
            double acc = 0.0;
            for (int d = 0; d < dim; ++d)
                acc += (double) orc_f16_to_f32(orc_f32_to_f16(q_idx[h * dim + d])) * (double) orc_f16_to_f32(pooled[(size_t) b * dim + d]);
            const float a = (float) acc;
            sc += a > 0.f ? a : 0.f;
        }
        scores[b] = sc;
    }
    float sc = 0.f;
    for (int h = 0; h < heads; ++h) {
        double acc = 0.0;
        for (int d = 0; d < dim; ++d) acc += (double) dead[d] * (double) q_idx[h * dim + d];
        const float a = (float) acc;
        sc += a > 0.f ? a : 0.f;
    }
    if (n_kv % blk != 0) sc += 1e9f;
    scores[nbid] = sc;
}

static uint32_t order_key(float s) {
    float v = s + 0.0f;
    if (v != v) return 0u;
    uint32_t u;
    memcpy(&u, &v, 4);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

static int cmp_desc_u32(const void* a, const void* b) {
    const uint32_t x = *(const uint32_t*) a, y = *(const uint32_t*) b;
    return x < y ? 1 : (x > y ? -1 : 0);
}

/* exact top-k cell selection with the reference's tie order (qsa_block_topk_multi,
 * src/wzy_qsa_256k.cuh:268-403): threshold key = the key at which the weight-cumulative count in
 * descending key order reaches width; every block above it is taken whole; blocks equal to it are
 * taken in (b mod 256, b div 256) order until the budget is met, a partial block taking its first
 * cells; output in thread order (thread t lists blocks t, t+256, ...). */
int orc_topk_select(const float* scores, int n_kv, int blk, int topk, int* sel) {
    const int width = n_kv < topk ? n_kv : topk;
    if (n_kv <= topk) {
        for (int j = 0; j < n_kv; ++j) sel[j] = j;
        return n_kv;
    }
    const int nbid = n_kv / blk, nb = nbid + 1;
    uint32_t* keys = (uint32_t*) malloc(sizeof(uint32_t) * (size_t) nb);
    int* wgt = (int*) malloc(sizeof(int) * (size_t) nb);
    for (int b = 0; b < nb; ++b) {
        keys[b] = order_key(scores[b]);
        wgt[b] = b < nbid ? blk : n_kv - nbid * blk;
    }
    /* threshold: sort distinct keys descending and accumulate weights */
    uint32_t* sk = (uint32_t*) malloc(sizeof(uint32_t) * (size_t) nb);
    int ns = 0;
    for (int b = 0; b < nb; ++b)
        if (wgt[b] > 0) sk[ns++] = keys[b];
    qsort(sk, (size_t) ns, sizeof(uint32_t), cmp_desc_u32);
    uint32_t thr = sk[ns - 1];
    {
        long cum = 0;
        int i = 0;
        while (i < ns) {
            const uint32_t k = sk[i];
            long wk = 0;
            for (int b = 0; b < nb; ++b)
                if (wgt[b] > 0 && keys[b] == k) wk += wgt[b];
            if (cum + wk >= width) { thr = k; break; }
            cum += wk;
            while (i < ns && sk[i] == k) ++i;
        }
    }
    long above = 0;
    for (int b = 0; b < nb; ++b)
        if (wgt[b] > 0 && keys[b] > thr) above += wgt[b];
    long eq_left = width - above;
    int n = 0;
    /* thread order */
    for (int t = 0; t < 256; ++t) {
        long my_eq = 0;
        for (int b = t; b < nb; b += 256)
            if (wgt[b] > 0 && keys[b] == thr) my_eq += wgt[b];
        long take_t = my_eq < eq_left ? my_eq : eq_left;
        if (take_t < 0) take_t = 0;
        eq_left -= take_t;
        for (int b = t; b < nb; b += 256) {
            if (wgt[b] == 0) continue;
            if (keys[b] > thr) {
                for (int c = 0; c < wgt[b]; ++c) sel[n++] = b * blk + c;
            } else if (keys[b] == thr && take_t > 0) {
                const int take = wgt[b] < take_t ? wgt[b] : (int) take_t;
                for (int c = 0; c < take; ++c) sel[n++] = b * blk + c;
                take_t -= take;
            }
        }
    }
    free(keys); free(wgt); free(sk);
    return n;
}

/* qsa_attend_int8_sparse_multi (src/wzy_qsa_256k.cuh:407-532) for one row: q heads qh (q|gate,
 * 2*hd per head), kv heads kvh, cells sel[0..n) of the INT8 store (cell p at row p). */
void orc_attend(const float* qg, const int8_t* kq, const uint16_t* ks, const int8_t* vq, const uint16_t* vs,
                const int* sel, int n, int qh, int kvh, int hd, float* out) {
    const int kvd = kvh * hd, gq = qh / kvh;
    double* s = (double*) malloc(sizeof(double) * (size_t) n);
    for (int h = 0; h < qh; ++h) {
        const int j = h / gq;
        const float* q = qg + (size_t) h * 2 * hd;
        double mx = -INFINITY;
        for (int c = 0; c < n; ++c) {
            const size_t p = (size_t) sel[c];
            double acc = 0.0;
            for (int d = 0; d < hd; ++d)
                acc += (double) orc_f16_to_f32(ks[p * (kvd / 64) + (size_t) (j * hd + d) / 64]) *
                       (double) kq[p * kvd + (size_t) j * hd + d] * (double) q[d];
            s[c] = acc * 0.0625;
            if (s[c] > mx) mx = s[c];
        }
        double sum = 0.0;
        for (int c = 0; c < n; ++c) { s[c] = exp(s[c] - mx); sum += s[c]; }
        for (int d = 0; d < hd; ++d) {
            double acc = 0.0;
            for (int c = 0; c < n; ++c) {
                const size_t p = (size_t) sel[c];
                acc += s[c] * (double) orc_f16_to_f32(vs[p * (kvd / 64) + (size_t) (j * hd + d) / 64]) *
                       (double) vq[p * kvd + (size_t) j * hd + d];
            }
            out[(size_t) h * hd + d] = (float) (acc / sum) * sigm_f(q[hd + d]);
        }
    }
    free(s);
}

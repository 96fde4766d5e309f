/* orc_core.c -- CPU oracle: formats, activation quantisation, dense GEMVs, router, NVFP4 experts,
 * MoE block, logit reductions.  TEST INFRASTRUCTURE ONLY (see wzy_oracle.h). */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "wzy_oracle.h"

/* ------------------------------------------------------------------------------------------------
 * formats
 * ---------------------------------------------------------------------------------------------- */

/* e2m1 x2 table: src/wzy_stage_v2.cuh:190 (kPair construction), src/wzy_cpu_moe.cuh:318-320 */
int orc_e2m1x2(int code) {
    static const int tab[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};
    return tab[code & 15];
}

/* unsigned e4m3 * 0.5: src/wzy_stage_v2.cuh:181-188 (fill_tables_current_device) */
float orc_ue4m3_half(int code) {
    const int x = code & 0x7F;
    if (x == 0) return 0.f;
    const int e = (x >> 3) & 0xF, m = x & 7;
    const float raw = (e == 0) ? ldexpf((float) m, -9) : ldexpf(1.f + (float) m / 8.f, e - 7);
    return raw * 0.5f;
}

float orc_f16_to_f32(uint16_t h) {
    const int s = (h >> 15) & 1, e = (h >> 10) & 0x1F, m = h & 0x3FF;
    float v;
    if (e == 0) v = ldexpf((float) m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexpf((float) (m | 0x400), e - 25);
    return s ? -v : v;
}

uint16_t orc_f32_to_f16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const uint32_t au = u & 0x7FFFFFFFu;
    if (au >= 0x7F800000u) return (uint16_t) (sign | (au > 0x7F800000u ? 0x7E00u : 0x7C00u));
    float a;
    memcpy(&a, &au, 4);
    if (a >= 65520.0f) return (uint16_t) (sign | 0x7C00u);             /* rounds to inf */
    if (a < 6.103515625e-05f) {                                        /* subnormal half: units of 2^-24 */
        const float q = a * 16777216.0f;                                /* exact scaling */
        const float r = rintf(q);                                       /* ties to even */
        return (uint16_t) (sign | (uint32_t) r);
    }
    int e;
    const float mfr = frexpf(a, &e);                                    /* a = mfr * 2^e, mfr in [0.5,1) */
    float mant = ldexpf(mfr, 11);                                       /* [1024, 2048) */
    mant = rintf(mant);
    if (mant >= 2048.f) { mant = 1024.f; ++e; }
    const uint32_t he = (uint32_t) (e - 1 + 15);
    if (he >= 31) return (uint16_t) (sign | 0x7C00u);
    return (uint16_t) (sign | (he << 10) | ((uint32_t) mant - 1024u));
}

float orc_bf16_to_f32(uint16_t h) {
    const uint32_t u = (uint32_t) h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

size_t orc_blob_bytes(int D, int F) {
    return (size_t) 2 * F * (D / 64 * 36) + (size_t) D * (F / 64 * 36) + 16;
}

static inline float silu_f(float x) { return x / (1.0f + expf(-x)); }
static inline float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }
static inline int clamp127(int q) { return q < -127 ? -127 : (q > 127 ? 127 : q); }

/* ------------------------------------------------------------------------------------------------
 * activation quantisation: quant_act_multi (src/wzy_kernels_v2.cuh:58-107)
 * d = amax/127; inv = d > 0 ? 127/amax : 0; q = rint(x*inv) clamped to +-127.
 * ---------------------------------------------------------------------------------------------- */
static void quant_block(const float* x, int n, int8_t* q, float* s) {
    float amax = 0.f;
    for (int i = 0; i < n; ++i) amax = fmaxf(amax, fabsf(x[i]));
    const float d = amax / 127.0f;
    const float inv = d > 0.f ? 127.0f / amax : 0.f;
    for (int i = 0; i < n; ++i) {
        const float p = x[i] * inv;
        q[i] = (int8_t) clamp127((int) rintf(p));
    }
    *s = d;
}

void orc_quant_act(const float* x, int cols, int T, int8_t* q32, float* s32, int8_t* q16, float* s16) {
    for (int t = 0; t < T; ++t) {
        const float* xr = x + (size_t) t * cols;
        if (q16)
            for (int g = 0; g < cols / 16; ++g)
                quant_block(xr + 16 * g, 16, q16 + (size_t) t * cols + 16 * g, s16 + (size_t) t * (cols / 16) + g);
        if (q32)
            for (int g = 0; g < cols / 32; ++g)
                quant_block(xr + 32 * g, 32, q32 + (size_t) t * cols + 32 * g, s32 + (size_t) t * (cols / 32) + g);
    }
}

/* ------------------------------------------------------------------------------------------------
 * dense GEMVs
 * ---------------------------------------------------------------------------------------------- */
/* gemm_q8p_t (src/wzy_kernels_v2.cuh:120-159): y = sum_b fp16(scale_b) * xs_b * isum_b */
void orc_gemv_q8(const int8_t* codes, const uint16_t* scales, const int8_t* xq, const float* xs, float* y,
                 int rows, int cols, int T) {
    const int nb = cols / 32;
    for (int t = 0; t < T; ++t) {
        const int8_t* xt = xq + (size_t) t * cols;
        const float* st = xs + (size_t) t * nb;
#pragma omp parallel for schedule(static) if (rows >= 256)
        for (int r = 0; r < rows; ++r) {
            const int8_t* c = codes + (size_t) r * cols;
            double acc = 0.0;
            for (int b = 0; b < nb; ++b) {
                int isum = 0;
                for (int i = 0; i < 32; ++i) isum += (int) c[32 * b + i] * (int) xt[32 * b + i];
                const float dw = orc_f16_to_f32(scales[(size_t) r * nb + b]);
                acc += (double) dw * (double) st[b] * (double) isum;
            }
            y[(size_t) t * rows + r] = (float) acc;
        }
    }
}

/* gemm_bf16_t (src/wzy_kernels_v2.cuh:307-337) */
void orc_gemv_bf16(const uint16_t* W, const float* x, float* y, int rows, int cols, int T) {
    for (int t = 0; t < T; ++t)
#pragma omp parallel for schedule(static) if (rows >= 256)
        for (int r = 0; r < rows; ++r) {
            const uint16_t* w = W + (size_t) r * cols;
            const float* xt = x + (size_t) t * cols;
            double acc = 0.0;
            for (int c = 0; c < cols; ++c) acc += (double) orc_bf16_to_f32(w[c]) * (double) xt[c];
            y[(size_t) t * rows + r] = (float) acc;
        }
}

/* ------------------------------------------------------------------------------------------------
 * router_top10_fast_multi (src/wzy_kernels_v2.cuh:989-1090):
 * p = exp(l - max) * (1/sum); K selection passes over p, larger wins, ties -> lower expert id;
 * w_k = p_k / max(sum_k p_k, 2^-14) (the sum accumulated in selection order).
 * ---------------------------------------------------------------------------------------------- */
void orc_router_topk(const float* logits, int E, int K, int T, int* ids, float* wts, float* probs_out) {
    float* p = (float*) malloc(sizeof(float) * (size_t) E);
    for (int t = 0; t < T; ++t) {
        const float* l = logits + (size_t) t * E;
        float mx = -INFINITY;
        for (int e = 0; e < E; ++e) mx = fmaxf(mx, l[e]);
        double es = 0.0;
        for (int e = 0; e < E; ++e) { p[e] = expf(l[e] - mx); es += (double) p[e]; }
        const float inv = 1.0f / (float) es;
        for (int e = 0; e < E; ++e) p[e] = p[e] * inv;
        if (probs_out) memcpy(probs_out + (size_t) t * E, p, sizeof(float) * (size_t) E);
        float wsum = 0.f;
        float wk[64];
        for (int k = 0; k < K; ++k) {
            float bv = -1.f;
            int bi = E;
            for (int e = 0; e < E; ++e)
                if (p[e] > bv || (p[e] == bv && e < bi)) { bv = p[e]; bi = e; }
            ids[t * K + k] = bi;
            wk[k] = bv;
            p[bi] = -2.f;
            wsum += bv;
        }
        const float sc = fmaxf(wsum, 6.103515625e-05f);
        for (int k = 0; k < K; ++k) wts[t * K + k] = wk[k] / sc;
    }
    free(p);
}

/* ------------------------------------------------------------------------------------------------
 * NVFP4 experts.  Blob: [gate F x GU_ROW][up F x GU_ROW][down D x D_ROW][16-byte tail: fp32 gate,
 * up, down tensor scales], GU_ROW = D/64*36, D_ROW = F/64*36; a 36-byte block = 4 e4m3 scale
 * bytes + 32 code bytes; sub-block s = code bytes 8s..8s+7, value k<8 low nibble of byte k,
 * value k>=8 high nibble of byte k-8 (src/wzy_kernels_v2.cuh:15-16,1432-1438,1488-1497).
 * ---------------------------------------------------------------------------------------------- */
/* sum over one row of `cols` values: sum_{blocks b, subs s} ue4m3(scale) * xs[4b+s] * isum */
static double nvfp4_row_dot(const uint8_t* row, int cols, const int8_t* xq, const float* xs) {
    double acc = 0.0;
    for (int b = 0; b < cols / 64; ++b) {
        const uint8_t* blk = row + 36 * b;
        for (int s = 0; s < 4; ++s) {
            const uint8_t* cb = blk + 4 + 8 * s;
            int isum = 0;
            for (int k = 0; k < 16; ++k) {
                const int nib = (k < 8) ? (cb[k] & 15) : (cb[k - 8] >> 4);
                isum += orc_e2m1x2(nib) * (int) xq[64 * b + 16 * s + k];
            }
            acc += (double) orc_ue4m3_half(blk[s]) * (double) xs[4 * b + s] * (double) isum;
        }
    }
    return acc;
}

void orc_expert_gate_up(const uint8_t* blob, int D, int F, const int8_t* xq16, const float* xs16, int8_t* aq16,
                        float* as16, float* act_out) {
    const int gu_row = D / 64 * 36;
    const float* tail = (const float*) (blob + orc_blob_bytes(D, F) - 16);
    float* act = (float*) malloc(sizeof(float) * (size_t) F);
    for (int j = 0; j < F; ++j) {
        const float g = (float) nvfp4_row_dot(blob + (size_t) j * gu_row, D, xq16, xs16) * tail[0];
        const float u = (float) nvfp4_row_dot(blob + (size_t) (F + j) * gu_row, D, xq16, xs16) * tail[1];
        act[j] = silu_f(g) * u;
    }
    if (act_out) memcpy(act_out, act, sizeof(float) * (size_t) F);
    for (int g = 0; g < F / 16; ++g) quant_block(act + 16 * g, 16, aq16 + 16 * g, as16 + g);
    free(act);
}

void orc_expert_down(const uint8_t* blob, int D, int F, const int8_t* aq16, const float* as16, float* out) {
    const int gu_row = D / 64 * 36, d_row = F / 64 * 36;
    const uint8_t* dn = blob + (size_t) 2 * F * gu_row;
    const float* tail = (const float*) (blob + orc_blob_bytes(D, F) - 16);
    for (int d = 0; d < D; ++d) out[d] = (float) nvfp4_row_dot(dn + (size_t) d * d_row, F, aq16, as16) * tail[2];
}

/* ------------------------------------------------------------------------------------------------
 * MoE block: StageGpu::record_forward MoE section (src/wzy_stage_v2.cuh:697-724) with all experts
 * resident: quant_act (32+16) -> router bf16 GEMV + sgate row -> top-k -> shared expert Q8 GEMVs +
 * silu_mul_quant32 (src/wzy_kernels_v2.cuh:1247-1280) -> routed experts -> combine
 * (src/wzy_kernels_v2.cuh:1281-1294): comb = shared*sigmoid(sg) + sum_{k, w!=0} w_k*part_k.
 * ---------------------------------------------------------------------------------------------- */
int orc_moe_block_fn(const orc_moe_weights* w, const float* x, int T, float* comb, int* ids, float* wts,
                     float* logits_out, float* sg_out, orc_blob_fn blob_fn, void* blob_ctx, int layer) {
    const int D = w->n_embd, F = w->n_ff, E = w->n_exp, K = w->top_k;
    int8_t* q32 = (int8_t*) malloc((size_t) T * D);
    float* s32 = (float*) malloc(sizeof(float) * (size_t) T * D / 32);
    int8_t* q16 = (int8_t*) malloc((size_t) T * D);
    float* s16 = (float*) malloc(sizeof(float) * (size_t) T * D / 16);
    float* logits = (float*) malloc(sizeof(float) * (size_t) T * E);
    float* sg = (float*) malloc(sizeof(float) * (size_t) T);
    float* sff = (float*) malloc(sizeof(float) * (size_t) T * F);
    float* sup = (float*) malloc(sizeof(float) * (size_t) T * F);
    float* sact = (float*) malloc(sizeof(float) * (size_t) T * F);
    int8_t* sq = (int8_t*) malloc((size_t) T * F);
    float* ss = (float*) malloc(sizeof(float) * (size_t) T * F / 32);
    float* shared = (float*) malloc(sizeof(float) * (size_t) T * D);
    int8_t* aq = (int8_t*) malloc((size_t) F);
    float* as = (float*) malloc(sizeof(float) * (size_t) F / 16);
    float* part = (float*) malloc(sizeof(float) * (size_t) T * K * D);
    int rc = 0;

    orc_quant_act(x, D, T, q32, s32, q16, s16);
    orc_gemv_bf16(w->router, x, logits, E, D, T);
    orc_gemv_bf16(w->sgate, x, sg, 1, D, T);
    orc_router_topk(logits, E, K, T, ids, wts, NULL);

    orc_gemv_q8(w->sh_gate_q, w->sh_gate_s, q32, s32, sff, F, D, T);
    orc_gemv_q8(w->sh_up_q, w->sh_up_s, q32, s32, sup, F, D, T);
    for (size_t i = 0; i < (size_t) T * F; ++i) sact[i] = silu_f(sff[i]) * sup[i];
    orc_quant_act(sact, F, T, sq, ss, NULL, NULL);
    orc_gemv_q8(w->sh_down_q, w->sh_down_s, sq, ss, shared, D, F, T);

    for (int t = 0; t < T && rc == 0; ++t)
        for (int k = 0; k < K; ++k) {
            const int e = ids[t * K + k];
            const uint8_t* blob = w->blobs ? w->blobs[e] : NULL;
            if (!blob && blob_fn) blob = blob_fn(blob_ctx, layer, e);
            if (!blob) { rc = -1; break; }
            orc_expert_gate_up(blob, D, F, q16 + (size_t) t * D, s16 + (size_t) t * (D / 16), aq, as, NULL);
            orc_expert_down(blob, D, F, aq, as, part + (size_t) (t * K + k) * D);
        }
    if (rc == 0)
        for (int t = 0; t < T; ++t) {
            const float g = sigmoid_f(sg[t]);
            for (int d = 0; d < D; ++d) {
                double s = (double) shared[(size_t) t * D + d] * (double) g;
                for (int k = 0; k < K; ++k) {
                    const float wk = wts[t * K + k];
                    if (wk != 0.0f) s += (double) wk * (double) part[(size_t) (t * K + k) * D + d];
                }
                comb[(size_t) t * D + d] = (float) s;
            }
        }
    if (logits_out) memcpy(logits_out, logits, sizeof(float) * (size_t) T * E);
    if (sg_out) memcpy(sg_out, sg, sizeof(float) * (size_t) T);
    free(q32); free(s32); free(q16); free(s16); free(logits); free(sg); free(sff); free(sup); free(sact);
    free(sq); free(ss); free(shared); free(aq); free(as); free(part);
    return rc;
}

int orc_moe_block(const orc_moe_weights* w, const float* x, int T, float* comb, int* ids, float* wts,
                  float* logits_out, float* sg_out) {
    return orc_moe_block_fn(w, x, T, comb, ids, wts, logits_out, sg_out, NULL, NULL, 0);
}

/* ------------------------------------------------------------------------------------------------
 * Prefill MoE block with this build's bf16 numerics (the reference prefill, src/wzy_prefill_tc.cuh:
 * 230-443, computes the same terms in fp16): x rounded to bf16; router logits = bf16 router .
 * bf16(x) and sg = bf16 sgate . bf16(x); top-k as orc_router_topk; routed expert weights
 * dequantised exactly (e2m1 * e4m3 scale * tensor scale has at most 8 significant bits, so the
 * bf16 value is exact); shared Q8_0 weights dequantised and rounded to bf16; SwiGLU outputs
 * rounded to bf16; comb = sigmoid(sg) * shared + sum_k w_k * expert_k.  Sums in double.
 * ---------------------------------------------------------------------------------------------- */
static float round_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
    memcpy(&f, &u, 4);
    return f;
}
/* value k of row `row` of a reference-layout NVFP4 plane with rows of `cols` values */
static float nvfp4_value(const uint8_t* row, int k, float tscale) {
    const uint8_t* blk = row + 36 * (k / 64);
    const int s = (k % 64) / 16, kk = k % 16;
    const uint8_t* cb = blk + 4 + 8 * s;
    const int nib = (kk < 8) ? (cb[kk] & 15) : (cb[kk - 8] >> 4);
    return (float) orc_e2m1x2(nib) * orc_ue4m3_half(blk[s]) * tscale;
}
static float q8_bf16_value(const int8_t* q, const uint16_t* s, int cols, int r, int k) {
    return round_bf16((float) q[(size_t) r * cols + k] * orc_f16_to_f32(s[(size_t) r * (cols / 32) + k / 32]));
}

int orc_moe_prefill(const orc_moe_weights* w, const float* x, int T, float* comb, int* ids, float* wts) {
    return orc_moe_prefill_fn(w, x, T, comb, ids, wts, NULL, NULL, NULL, 0);
}

int orc_moe_prefill_fn(const orc_moe_weights* w, const float* x, int T, float* comb, int* ids, float* wts,
                       float* logits_out, orc_blob_fn blob_fn, void* blob_ctx, int layer) {
    const int D = w->n_embd, F = w->n_ff, E = w->n_exp, K = w->top_k;
    float* logits = (float*) malloc(sizeof(float) * (size_t) T * E);
    float* sg = (float*) malloc(sizeof(float) * (size_t) T);
    int rc = 0;
#pragma omp parallel
    {
        float* xb = (float*) malloc(sizeof(float) * (size_t) D);
#pragma omp for schedule(static)
        for (int t = 0; t < T; ++t) {
            for (int d = 0; d < D; ++d) xb[d] = round_bf16(x[(size_t) t * D + d]);
            for (int e = 0; e < E; ++e) {
                double a = 0.0;
                for (int d = 0; d < D; ++d) a += (double) orc_bf16_to_f32(w->router[(size_t) e * D + d]) * xb[d];
                logits[(size_t) t * E + e] = (float) a;
            }
            double g = 0.0;
            for (int d = 0; d < D; ++d) g += (double) orc_bf16_to_f32(w->sgate[d]) * xb[d];
            sg[t] = (float) g;
        }
        free(xb);
    }
    if (logits_out) memcpy(logits_out, logits, sizeof(float) * (size_t) T * E);
    orc_router_topk(logits, E, K, T, ids, wts, NULL);
    /* routed blobs are fetched before the parallel part (the fetch callback is not thread safe) */
    const uint8_t** blobs = (const uint8_t**) malloc(sizeof(uint8_t*) * (size_t) T * K);
    for (int i = 0; i < T * K && rc == 0; ++i) {
        const int e = ids[i];
        const uint8_t* b = w->blobs ? w->blobs[e] : NULL;
        if (!b && blob_fn) b = blob_fn(blob_ctx, layer, e);
        if (!b) rc = -1;
        blobs[i] = b;
    }
    if (rc == 0) {
#pragma omp parallel
        {
            float* xb = (float*) malloc(sizeof(float) * (size_t) D);
            float* act = (float*) malloc(sizeof(float) * (size_t) F);
            double* out = (double*) malloc(sizeof(double) * (size_t) D);
#pragma omp for schedule(dynamic)
            for (int t = 0; t < T; ++t) {
                for (int d = 0; d < D; ++d) xb[d] = round_bf16(x[(size_t) t * D + d]);
                /* shared expert */
                for (int j = 0; j < F; ++j) {
                    double g = 0.0, u = 0.0;
                    for (int d = 0; d < D; ++d) {
                        g += (double) q8_bf16_value(w->sh_gate_q, w->sh_gate_s, D, j, d) * xb[d];
                        u += (double) q8_bf16_value(w->sh_up_q, w->sh_up_s, D, j, d) * xb[d];
                    }
                    act[j] = round_bf16(silu_f((float) g) * (float) u);
                }
                const double gate = (double) sigmoid_f(sg[t]);
                for (int d = 0; d < D; ++d) {
                    double s = 0.0;
                    for (int j = 0; j < F; ++j) s += (double) q8_bf16_value(w->sh_down_q, w->sh_down_s, F, d, j) * act[j];
                    out[d] = (double) (float) s * gate;
                }
                /* routed experts */
                for (int k = 0; k < K; ++k) {
                    const uint8_t* blob = blobs[t * K + k];
                    const int gu_row = D / 64 * 36, d_row = F / 64 * 36;
                    const float* tail = (const float*) (blob + orc_blob_bytes(D, F) - 16);
                    for (int j = 0; j < F; ++j) {
                        double g = 0.0, u = 0.0;
                        const uint8_t* rg = blob + (size_t) j * gu_row;
                        const uint8_t* ru = blob + (size_t) (F + j) * gu_row;
                        for (int d = 0; d < D; ++d) {
                            g += (double) nvfp4_value(rg, d, tail[0]) * xb[d];
                            u += (double) nvfp4_value(ru, d, tail[1]) * xb[d];
                        }
                        act[j] = round_bf16(silu_f((float) g) * (float) u);
                    }
                    const uint8_t* dn = blob + (size_t) 2 * F * gu_row;
                    for (int d = 0; d < D; ++d) {
                        double s = 0.0;
                        const uint8_t* rd = dn + (size_t) d * d_row;
                        for (int j = 0; j < F; ++j) s += (double) nvfp4_value(rd, j, tail[2]) * act[j];
                        out[d] += (double) wts[t * K + k] * (double) (float) s;
                    }
                }
                for (int d = 0; d < D; ++d) comb[(size_t) t * D + d] = (float) out[d];
            }
            free(xb); free(act); free(out);
        }
    }
    free(blobs); free(logits); free(sg);
    return rc;
}

/* ------------------------------------------------------------------------------------------------
 * logit reductions: row_argmax_multi_kernel / row_top16_multi_kernel
 * (src/wzy_kernels_v2.cuh:1873-1984): larger value wins, ties -> lower vocab id.
 * ---------------------------------------------------------------------------------------------- */
void orc_row_argmax(const float* logits, int nvocab, int T, int* out) {
    for (int t = 0; t < T; ++t) {
        const float* l = logits + (size_t) t * nvocab;
        int bi = 0;
        for (int i = 1; i < nvocab; ++i)
            if (l[i] > l[bi]) bi = i;
        out[t] = bi;
    }
}

void orc_row_top16(const float* logits, int nvocab, int T, int* greedy, float* top_v, int* top_i) {
    for (int t = 0; t < T; ++t) {
        const float* l = logits + (size_t) t * nvocab;
        float v[16];
        int id[16];
        int n = 0;
        for (int i = 0; i < nvocab; ++i) {
            /* insert into the sorted list (desc value, asc id among equals) */
            const float x = l[i];
            if (n == 16 && !(x > v[15])) continue;
            int pos = n < 16 ? n : 15;
            while (pos > 0 && x > v[pos - 1]) --pos;
            const int last = n < 16 ? n : 15;
            for (int j = last; j > pos; --j) { v[j] = v[j - 1]; id[j] = id[j - 1]; }
            v[pos] = x;
            id[pos] = i;
            if (n < 16) ++n;
        }
        if (greedy) greedy[t] = id[0];
        for (int j = 0; j < 16; ++j) {
            if (top_v) top_v[t * 16 + j] = j < n ? v[j] : -1e30f;
            if (top_i) top_i[t * 16 + j] = j < n ? id[j] : 0;
        }
    }
}

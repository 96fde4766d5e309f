/* orc_ple.c -- CPU oracle of the per-layer embedding (PLE) block at layer 1: the hashed 3-gram rows
 * of the fp8 table (the engine's stage_ple_window, src/wzy_engine_v2.cu:909-978, and PleSrc,
 * src/wzy_stage_v2.cuh:215-324) and the block that mixes them into the hyper-connection streams
 * (src/wzy_stage_v2.cuh:583-597; kernels ple_group_multi, ple_gate_gv_multi, ple_conv_multi,
 * src/wzy_kernels_v2.cuh:1299-1374).  TEST INFRASTRUCTURE ONLY (see wzy_oracle.h). */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "wzy_oracle.h"

/* hash constants of the reference's 3-gram lookup (src/wzy_engine_v2.cu:909-915): one multiplier per
 * context position, and per head a prime row count and the offset of its slice of the table */
static const uint64_t ple_mult[3] = {23703573157769ull, 20109073645365ull, 8052911324071ull};
static const uint64_t ple_vocab[ORC_PLE_HEADS] = {
    20000003, 20000023, 20000033, 20000047, 20000059, 20000063, 20000069, 20000077,
    20000081, 20000093, 20000107, 20000147, 20000153, 20000159, 20000161, 20000171};
static const uint64_t ple_off[ORC_PLE_HEADS] = {
    0, 20000003, 40000026, 60000059, 80000106, 100000165, 120000228, 140000297,
    160000374, 180000455, 200000548, 220000655, 240000802, 260000955, 280001114, 300001275};

uint64_t orc_ple_table_rows(void) { return ple_off[ORC_PLE_HEADS - 1] + ple_vocab[ORC_PLE_HEADS - 1]; }

/* Table rows of one token (src/wzy_engine_v2.cu:950-967): the context is (cur, prev1, prev2), cut at
 * the first missing (< 0) or end-of-sequence token, which (and everything older) reads as eos; the
 * 2-gram (cur, prev1) addresses heads 0-7 and the 3-gram heads 8-15, each head taking the product-XOR
 * hash modulo its prime, offset into its slice. */
void orc_ple_row_ids(int cur, int prev1, int prev2, int eos, uint32_t* rows) {
    int64_t ctx[3];
    const int prev[3] = {0, prev1, prev2};
    ctx[0] = cur;
    int cut = 0;
    for (int s = 1; s < 3; ++s) {
        const int v = cut ? -1 : prev[s];
        cut = cut || v < 0 || v == eos;
        ctx[s] = cut ? eos : v;
    }
    for (int n = 2; n <= 3; ++n) {
        uint64_t mixed = (uint64_t) ctx[0] * ple_mult[0];
        for (int j = 1; j < n; ++j) mixed ^= (uint64_t) ctx[j] * ple_mult[j];
        for (int g = 0; g < 8; ++g) {
            const int h = (n - 2) * 8 + g;
            rows[h] = (uint32_t) (mixed % ple_vocab[h] + ple_off[h]);
        }
    }
}

/* One fp8 code of the table (PleSrc::open's LUT, src/wzy_stage_v2.cuh:279-286): e4m3 with bias 7,
 * subnormals m * 2^-9, the NaN codes (exponent 15, mantissa 7) read as 0; times the table scale. */
float orc_ple_fp8(uint8_t v, float scale) {
    const int sg = (v >> 7) & 1, e = (v >> 3) & 0xF, mm = v & 7;
    float f;
    if (e == 0) f = ldexpf((float) mm, -9);
    else if (e == 15 && mm == 7) f = 0.f;
    else f = ldexpf(1.f + (float) mm / 8.f, e - 7);
    return (sg ? -f : f) * scale;
}

/* Embedding rows of T window rows at positions pos .. pos+T-1 (toks[t] the token of row t), the
 * tokens of the earlier cells read from tok_hist[p] (p < pos; a position below 0 has none), which the
 * call then extends with the window's tokens: out [T][16 * head] = the 16 heads' decoded rows. */
void orc_ple_rows(orc_ple_row_fn row, void* ctx, int head, float scale, int eos, const int* toks, int T, int pos,
                  int* tok_hist, float* out) {
    for (int t = 0; t < T; ++t) {
        const int p = pos + t;
        const int p1 = t >= 1 ? toks[t - 1] : (p >= 1 ? tok_hist[p - 1] : -1);
        const int p2 = t >= 2 ? toks[t - 2] : (p >= 2 ? tok_hist[p - 2] : -1);
        uint32_t r[ORC_PLE_HEADS];
        orc_ple_row_ids(toks[t], p1, p2, eos, r);
        for (int h = 0; h < ORC_PLE_HEADS; ++h) {
            const uint8_t* src = row(ctx, r[h]);
            for (int j = 0; j < head; ++j) out[(size_t) t * ORC_PLE_HEADS * head + (size_t) h * head + j] =
                orc_ple_fp8(src[j], scale);
        }
    }
    for (int t = 0; t < T; ++t) tok_hist[pos + t] = toks[t];
}

/* RMSNorm of each stream of T rows (ple_group_multi): y[t][c][:] = x[t][c][:] * rsqrt(mean x^2 + eps)
 * * gamma[c][:] */
static void group_norm(const float* x, const float* gamma, float* y, int D, int HC, int T, float eps) {
    for (int t = 0; t < T; ++t)
        for (int c = 0; c < HC; ++c) {
            const float* xc = x + ((size_t) t * HC + c) * D;
            double ss = 0.0;
            for (int d = 0; d < D; ++d) ss += (double) xc[d] * xc[d];
            const float rs = 1.0f / sqrtf((float) (ss / (double) D) + eps);
            for (int d = 0; d < D; ++d) y[((size_t) t * HC + c) * D + d] = xc[d] * rs * gamma[(size_t) c * D + d];
        }
}

/* The PLE block on T rows (src/wzy_stage_v2.cuh:583-597):
 *   R += bo * 2 sigmoid(inj_prev / HC)            the pending FFN write of layer 0 (bo may be NULL)
 *   q = groupnorm(R, norm_q)                      per stream
 *   k = groupnorm(W_k . emb, norm_k), v = W_v . emb     (bf16 weights; emb rounded to bf16 first when
 *                                                 emb_bf16, the prefill's GEMM operand)
 *   g[t][c] = sigmoid(sign(s) sqrt(max(|s|, 1e-6))), s = (k_c . q_c) / sqrt(D)   (ple_gate_gv_multi)
 *   gat[t][c] = v * g[t][c];  n = groupnorm(gat, norm_c)
 *   per channel ch of the HC*D streams, rows in order (ple_conv_multi): acc = w0 h[0] + w1 h[3] +
 *   w2 h[6] + w3 n (the history h holds the channel's last 9 values of n, oldest first), the history
 *   shifts in n, R += gat + silu(acc);  hist_snaps (optional) [T][HC*D*9] after each row.
 * R [T][HC][D], inj_prev [T][HC], emb [T][D], hist [HC*D][9] (channel-major, as the reference). */
void orc_ple_block(float* R, const float* bo, const float* inj_prev, const float* emb, const uint16_t* wk,
                   const uint16_t* wv, const float* norm_q, const float* norm_k, const float* norm_c,
                   const float* conv_w, float* hist, int D, int HC, float eps, int T, int emb_bf16,
                   float* hist_snaps) {
    const size_t HCD = (size_t) HC * D;
    float* e = (float*) malloc(sizeof(float) * (size_t) T * D);
    float* q = (float*) malloc(sizeof(float) * (size_t) T * HCD);
    float* k = (float*) malloc(sizeof(float) * (size_t) T * HCD);
    float* v = (float*) malloc(sizeof(float) * (size_t) T * D);
    float* gat = (float*) malloc(sizeof(float) * (size_t) T * HCD);
    float* n = (float*) malloc(sizeof(float) * (size_t) T * HCD);
    for (size_t i = 0; i < (size_t) T * D; ++i) {
        uint32_t u;
        memcpy(&u, &emb[i], 4);
        e[i] = emb_bf16 ? orc_bf16_to_f32((uint16_t) ((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16)) : emb[i];
    }
    if (bo) orc_hc_write(R, bo, inj_prev, D, HC, T);
    group_norm(R, norm_q, q, D, HC, T, eps);
    orc_gemv_bf16(wk, e, k, (int) HCD, D, T);
    group_norm(k, norm_k, k, D, HC, T, eps);
    orc_gemv_bf16(wv, e, v, D, D, T);
    for (int t = 0; t < T; ++t)
        for (int c = 0; c < HC; ++c) {
            const float* kc = k + ((size_t) t * HC + c) * D;
            const float* qc = q + ((size_t) t * HC + c) * D;
            double acc = 0.0;
            for (int d = 0; d < D; ++d) acc += (double) kc[d] * qc[d];
            const float s = (float) acc / sqrtf((float) D);
            const float sg = s < 0.f ? -1.f : 1.f;
            const float g = 1.f / (1.f + expf(-sg * sqrtf(fmaxf(fabsf(s), 1e-6f))));
            for (int d = 0; d < D; ++d) gat[((size_t) t * HC + c) * D + d] = v[(size_t) t * D + d] * g;
        }
    group_norm(gat, norm_c, n, D, HC, T, eps);
    for (size_t ch = 0; ch < HCD; ++ch) {
        float h[9];
        for (int i = 0; i < 9; ++i) h[i] = hist[ch * 9 + i];
        const float* w = conv_w + ch * 4;
        for (int t = 0; t < T; ++t) {
            const float cur = n[(size_t) t * HCD + ch];
            const float acc = (float) ((double) w[0] * h[0] + (double) w[1] * h[3] + (double) w[2] * h[6] +
                                       (double) w[3] * cur);
            for (int i = 0; i < 8; ++i) h[i] = h[i + 1];
            h[8] = cur;
            R[(size_t) t * HCD + ch] += gat[(size_t) t * HCD + ch] + acc / (1.0f + expf(-acc));
            if (hist_snaps)
                for (int i = 0; i < 9; ++i) hist_snaps[((size_t) t * HCD + ch) * 9 + i] = h[i];
        }
        for (int i = 0; i < 9; ++i) hist[ch * 9 + i] = h[i];
    }
    free(e); free(q); free(k); free(v); free(gat); free(n);
}

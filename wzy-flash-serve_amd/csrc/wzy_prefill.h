// wzy_prefill.h -- internal interface of the chunked-prefill kernels (prefill.hip), used by the stage.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "wzy_qsa.h"

namespace wzy {

// C[m][n] = sum_k A[m][k] * W[n][k] on bf16 MFMA: A bf16 rows (lda elements apart); W Q8_0 (codes
// [N][K], fp16 scales [N][K/32], code * scale rounded to bf16) or bf16 [N][K]; output fp32 (y) or
// bf16 (yb), rows ldy apart.  K a multiple of 64.
// ksplit > 1 (fp32 output only): K is cut into ksplit equal ranges whose partial sums go to
// y + s * M * ldy (s = 0 .. ksplit-1); the consumer adds them.
// um_mixed != null (the HC up projection, N = 4 * um_d): instead of storing C, each row's four stream
// gates are combined with the normed streams (um_xn bf16 [M][4][um_d]):
//   mixed[m][d] = (sum over c in order of xn[m][c][d] / (1 + exp(-bf16(C[m][c * um_d + d])))) / 4
// written fp32 to um_mixed and bf16 to um_xh (both [M][um_d]).
struct PfGemm {
    const uint16_t* a; int lda;
    int M, N, K;
    const int8_t* wq; const uint16_t* ws;
    const uint16_t* wb;
    float* y; uint16_t* yb; int ldy;
    int ksplit;
    const uint16_t* um_xn; float* um_mixed; uint16_t* um_xh; int um_d;
    // optional bf16 scratch of at least N x K values: Q8_0 weights of a launch with PF_DEQ_MIN_M or more
    // rows are expanded into it once (bf16(q * scale), the kernel's own rounding) and read as bf16
    uint16_t* wscratch; size_t wscratch_elems;
};
constexpr int PF_DEQ_MIN_M = 512;
int launch_pf_gemm(const PfGemm& g, hipStream_t st);

// token embeddings of B rows broadcast to the HC streams: R [B][hc][D]
struct PfEmb {
    const uint16_t* emb;                    // bf16 [n_vocab][D], or
    const int8_t* emb_q; const uint16_t* emb_s;   // Q8_0
    int n_vocab;
};
int launch_pf_embed(const PfEmb& e, const int* toks, float* R, int D, int HC, int B, hipStream_t st);

// HC read pieces (src/wzy_prefill_tc.cuh:690-715)
int launch_pf_hc_norm(float* R, const float* bo, const float* inj_prev, const float* norm_w, uint16_t* xn, int D,
                      int HC, float eps, int B, hipStream_t st);
// loh = bf16(silu(v)), v = lo * inv_hc; with nsplit == 4 partial sums lo[s * n + i],
// v = ((p0 + p1) + (p2 + p3)) * inv_hc
int launch_pf_silu_div(const float* lo, uint16_t* loh, size_t n, int nsplit, float inv_hc, hipStream_t st);
int launch_pf_hc_write(float* R, const float* blk, const float* inj, int D, int HC, int B, hipStream_t st);

// GDN (src/wzy_qsa_wmma.cuh:5-195, src/wzy_prefill_tc.cuh:54-67)
struct PfGdn {
    int hk, hv, B;
    float eps;
    const float* qkv;                       // [B][QKV] raw projections
    const float* z;                         // [B][hv*128] raw output gate
    const float* ab;                        // [B][2*hv] raw alpha | beta
    const float* dt; const float* ssm_a; const float* conv_w; const float* gamma;
    float* conv_hist;                       // [QKV][3]
    float* state;                           // [hv][128][128]
    float* conv_out;                        // [B][QKV] scratch
    float* decay; float* beta;              // [B][hv] scratch
    float* kq;                              // [B][hk] scratch: k . q per row and key head
    float* o;                               // [B][hv*128] scratch
    uint16_t* y;                            // [B][hv*128] bf16 output (gated RMS norm)
};
int launch_pf_gdn(const PfGdn& g, hipStream_t st);

// QSA: norms + RoPE + INT8 KV append of B rows at *pos .. *pos+B-1 (pos device)
struct PfQsaPrep {
    QsaDims dm;
    const int* pos;
    float* qg; float* kk; const float* vv; float* q_idx;
    const float* q_norm; const float* k_norm; const float* iq_norm;
    const float* cos_tab; const float* sin_tab;
    QsaKv kv;
};
int launch_pf_qsa_prep(const PfQsaPrep& a, int B, hipStream_t st);
// indexer append of B rows starting at host position p0 (the same values as B single-row appends)
struct PfIdxAppend {
    QsaDims dm;
    const float* idx_raw;                   // [B][idim]
    const float* ik_norm; const float* cos_tab; const float* sin_tab;
    QsaIdx ix;
};
int launch_pf_idx_append(const PfIdxAppend& a, int p0, int B, hipStream_t st);
// sparse attention of B rows with the prefill kernel's fp16 operands (pf_qsa_wmma_sparse_attn,
// src/wzy_qsa_wmma.cuh:289-489); out bf16 [B][qh*hd]
struct PfAttn {
    QsaDims dm;
    const int* pos;
    const float* qg;                        // [B][qh*2*hd]
    QsaKv kv;
    const int* sel;                         // [B][topk]
    uint16_t* out;
};
int launch_pf_attn(const PfAttn& a, int B, hipStream_t st);
// indexer block scores of `rows` consecutive rows on MFMA (same arguments as launch_qsa_score_rows)
int launch_pf_scores(const QsaScoreArgs& a, int rows, hipStream_t st);
// top-k of `rows` rows at one launch (every row's blocks must fit one workgroup); internal to
// qsa_attn.hip
int launch_qsa_topk_rows(const QsaDims& dm, const int* pos, const float* scores, int max_b, int* sel_ids,
                         int* sel_cnt, int rows, int max_n_kv, hipStream_t st);

}  // namespace wzy

// prefill.hip -- kernels of the chunked prefill (B prompt cells per launch sequence) on gfx950.
//
//  pf_gemm       every dense projection of the chunk on bf16 MFMA (v_mfma_f32_32x32x16_bf16):
//                128 x 128 output tiles, K in steps of 64 through two LDS buffers; Q8_0 weights are
//                dequantised (code * fp16 scale, rounded to bf16) on their way into LDS, bf16
//                weights copied.  Workgroups are numbered so that the eight XCDs take interleaved row
//                tiles and each runs all weight tiles of its row tile back to back.  A few bf16
//                weight rows (N <= 16) take pf_skinny instead (fp32 FMA dot products per row).
//  HC read       pf_hc_norm (pending block folded in, per-stream RMSNorm, bf16), GEMMs for inject /
//                down (K split by stream) / up (the stream mean as its epilogue), pf_silu_div; pf_hc_write
//                writes a block into the streams.
//  GDN           pf_gdn_ab (gates), pf_gdn_conv (causal conv + SiLU + L2 of q/k heads over all rows
//                at once), pf_gdn_hist (conv history), pf_gdn_recur (the delta rule, sequential over
//                the rows: 32 lanes per state column, 4 rows each in registers, q/k staged in LDS
//                32 steps at a time), pf_gdn_norm (gated RMS norm, bf16).
//  QSA           pf_qsa_prep (q / k / indexer-q norms + RoPE, INT8 KV append), pf_idx_append (the
//                indexer keys of every block the chunk completes, one workgroup per block, then
//                pf_idx_tail), block scores on fp16 MFMA (pf_score), top-k with the decode kernel,
//                pf_attn (sparse GQA attention on fp16 MFMA, 64 cells per load step, a 32-cell
//                online softmax).
// reference: PrefillStageCtx::run_stage_prefill and its kernels (src/wzy_prefill_tc.cuh:20-98,
// 546-1058; src/wzy_qsa_wmma.cuh:5-489), with cuBLAS fp16 GEMMs replaced by bf16 MFMA GEMMs.
#include "wzy_device.h"
#include "wzy_host.h"
#include "wzy_prefill.h"
#include "wzy_qsa.h"
#include "wzy_qsa_dev.h"

using namespace wzy;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

namespace {

WZY_DEV uint16_t f_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16) f); }   // nearest even
WZY_DEV uint32_t pack_bf16(float a, float b) { return (uint32_t) f_to_bf16(a) | ((uint32_t) f_to_bf16(b) << 16); }

// ---------------------------------------------------------------------------------------------
// dense GEMM
// ---------------------------------------------------------------------------------------------
constexpr int GM = 128, GN = 128, GK = 64, GLD = GK + 8;   // tile rows, weight rows, k step, LDS row (bf16)

struct GemmArgs {
    PfGemm g;
    int mt, nt;
};

// 32 Q8_0 codes (one block, c0 | c1) times their fp16 scale, rounded to bf16, as four 16-byte pieces
WZY_DEV uint4 q8_quarter_bf16(uint32_t a, uint32_t b, float sc) {
    return make_uint4(pack_bf16((float) (int8_t) a * sc, (float) (int8_t) (a >> 8) * sc),
                      pack_bf16((float) (int8_t) (a >> 16) * sc, (float) (int8_t) (a >> 24) * sc),
                      pack_bf16((float) (int8_t) b * sc, (float) (int8_t) (b >> 8) * sc),
                      pack_bf16((float) (int8_t) (b >> 16) * sc, (float) (int8_t) (b >> 24) * sc));
}
WZY_DEV void q8_block_bf16(uint4 c0, uint4 c1, float sc, uint4& o0, uint4& o1, uint4& o2, uint4& o3) {
    o0 = q8_quarter_bf16(c0.x, c0.y, sc);
    o1 = q8_quarter_bf16(c0.z, c0.w, sc);
    o2 = q8_quarter_bf16(c1.x, c1.y, sc);
    o3 = q8_quarter_bf16(c1.z, c1.w, sc);
}

// UM: the HC up projection with the stream mean as its epilogue.  Tile column n holds stream
// c = n % 4 of position d = n / 4 (weight row c * um_d + d), so a row's four stream gates sit in
// one lane quad and are combined there in stream order.
// SB: one LDS buffer (37 KB), so four workgroups share a CU (three with the UM epilogue, whose
// registers allow no more); the next k step still loads into
// registers during the MFMAs, and a second barrier per step guards the buffer.  Launches with at
// least 512 tiles use it; smaller ones keep two buffers (74 KB, two workgroups per CU).
template <bool UM, bool SB>
__global__ void __launch_bounds__(256, SB ? (UM ? 3 : 4) : 2) pf_gemm_kernel(GemmArgs ga) {
    constexpr int NBUF = SB ? 1 : 2;
    __shared__ __align__(16) uint16_t sAW[NBUF * (GM + GN) * GLD];
    uint16_t (*const sA)[GM][GLD] = (uint16_t (*)[GM][GLD]) sAW;
    uint16_t (*const sW)[GN][GLD] = (uint16_t (*)[GN][GLD]) (sAW + NBUF * GM * GLD);
    constexpr int XS_LD = GN + 8;                                  // UM epilogue: xn tile row stride
    static_assert(GM * XS_LD <= NBUF * (GM + GN) * GLD, "the UM epilogue's xn tile fits the GEMM's LDS");
    const PfGemm& g = ga.g;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, wm = w & 1, wn = w >> 1;
    const int tiles = ga.mt * ga.nt;
    const int ksp = (int) blockIdx.x / tiles;                      // K range of a split launch
    const int b = (int) blockIdx.x - ksp * tiles;
    int mi, ni;
    if ((ga.mt & 7) == 0) {
        const int s = b >> 3;
        mi = (s / ga.nt) * 8 + (b & 7);
        ni = s % ga.nt;
    } else {
        mi = b / ga.nt;
        ni = b % ga.nt;
    }
    const int m0 = mi * GM, n0 = ni * GN;
    const int sr = tid >> 1, kh = (tid & 1) * 32;                  // staging: row sr, k kh .. kh+31
    const int nk = g.K / GK / max(g.ksplit, 1);                    // k steps of this launch's range
    const size_t k0 = (size_t) ksp * nk * GK;
    const uint16_t* ap = g.a + (size_t) min(m0 + sr, g.M - 1) * g.lda + k0 + kh;
    size_t wr = (size_t) min(n0 + sr, g.N - 1);
    if (UM) wr = (wr & 3) * (size_t) g.um_d + (wr >> 2);
    const bool q8 = g.wq != nullptr;
    const int8_t* wqp = q8 ? g.wq + wr * g.K + k0 + kh : nullptr;
    const uint16_t* wsp = q8 ? g.ws + wr * (g.K / 32) + (k0 + kh) / 32 : nullptr;
    const uint16_t* wbp = q8 ? nullptr : g.wb + wr * g.K + k0 + kh;

    // staging registers are scalars: arrays captured by a lambda would live in scratch memory
    uint4 ra0, ra1, ra2, ra3, rw0, rw1, rw2 = make_uint4(0, 0, 0, 0), rw3 = rw2;
    float rs = 0.f;
#define PF_GEMM_LOAD(ks)                                                         \
    {                                                                            \
        const size_t o_ = (size_t) (ks) * GK;                                    \
        ra0 = *(const uint4*) (ap + o_);                                         \
        ra1 = *(const uint4*) (ap + o_ + 8);                                     \
        ra2 = *(const uint4*) (ap + o_ + 16);                                    \
        ra3 = *(const uint4*) (ap + o_ + 24);                                    \
        if (q8) {                                                                \
            rw0 = *(const uint4*) (wqp + o_);                                    \
            rw1 = *(const uint4*) (wqp + o_ + 16);                               \
            rs = h16_to_f(wsp[(ks) * (GK / 32)]);                                \
        } else {                                                                 \
            rw0 = *(const uint4*) (wbp + o_);                                    \
            rw1 = *(const uint4*) (wbp + o_ + 8);                                \
            rw2 = *(const uint4*) (wbp + o_ + 16);                               \
            rw3 = *(const uint4*) (wbp + o_ + 24);                               \
        }                                                                        \
    }
#define PF_GEMM_STORE(buf)                                                       \
    {                                                                            \
        *(uint4*) &sA[buf][sr][kh] = ra0;                                        \
        *(uint4*) &sA[buf][sr][kh + 8] = ra1;                                    \
        *(uint4*) &sA[buf][sr][kh + 16] = ra2;                                   \
        *(uint4*) &sA[buf][sr][kh + 24] = ra3;                                   \
        if (q8) q8_block_bf16(rw0, rw1, rs, rw0, rw1, rw2, rw3);                  \
        *(uint4*) &sW[buf][sr][kh] = rw0;                                        \
        *(uint4*) &sW[buf][sr][kh + 8] = rw1;                                    \
        *(uint4*) &sW[buf][sr][kh + 16] = rw2;                                   \
        *(uint4*) &sW[buf][sr][kh + 24] = rw3;                                   \
    }

    f32x16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    PF_GEMM_LOAD(0);
    PF_GEMM_STORE(0);
    __syncthreads();
    for (int ks = 0; ks < nk; ++ks) {
        const int buf = SB ? 0 : (ks & 1);
        const bool more = ks + 1 < nk;
        if (more) PF_GEMM_LOAD(ks + 1);                            // next step's loads in flight
#pragma unroll
        for (int kk = 0; kk < GK / 16; ++kk) {
            bf16x8_t av[2], bv[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                av[i] = *(const bf16x8_t*) &sA[buf][wm * 64 + i * 32 + (lane & 31)][kk * 16 + (lane >> 5) * 8];
#pragma unroll
            for (int j = 0; j < 2; ++j)
                bv[j] = *(const bf16x8_t*) &sW[buf][wn * 64 + j * 32 + (lane & 31)][kk * 16 + (lane >> 5) * 8];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[i], bv[j], acc[i][j], 0, 0, 0);
        }
        if constexpr (SB) {
            __syncthreads();                                       // every wave is done with the buffer
            if (more) PF_GEMM_STORE(0);
        } else {
            if (more) PF_GEMM_STORE(buf ^ 1);
        }
        __syncthreads();
    }
#undef PF_GEMM_LOAD
#undef PF_GEMM_STORE
    // acc[i][j][r] = C[row 8*(r/4) + 4*(lane/32) + r%4][col lane%32] of block (i, j)
    if constexpr (UM) {
        // mixed = (sum over streams in order of xn / (1 + exp(-bf16 gate))) / 4, fp32 and bf16
        // (pf_gr_up_mean_fp16, src/wzy_qsa_wmma.cuh:236-252); the xn loads of a 32 x 32 block go first
        // The tile's xn (GM rows x 4 streams x GN/4 positions, bf16) is staged in the GEMM's LDS, whose
        // last use ended at the loop's final barrier: 16-byte coalesced loads instead of 2-byte ones.
        const int D = g.um_d, c = lane & 3, d0 = n0 >> 2;
        uint16_t (*const xs)[XS_LD] = (uint16_t (*)[XS_LD]) sAW;     // [row][stream * GN/4 + position]
#pragma unroll
        for (int i = 0; i < GM * 4 * (GN / 4) / 8 / 256; ++i) {
            const int pc = tid + 256 * i, rr = pc >> 4, sc = (pc >> 2) & 3, q = pc & 3;
            const int row = min(m0 + rr, g.M - 1);
            *(uint4*) &xs[rr][sc * (GN / 4) + 8 * q] = *(const uint4*) (g.um_xn + (size_t) row * 4 * D + (size_t) sc * D + d0 + 8 * q);
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int d = (n0 + wn * 64 + j * 32 + (lane & 31)) >> 2;
                float xv[16];
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int rr = wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    xv[r] = bf16_to_f(xs[rr][c * (GN / 4) + d - d0]);
                }
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    const float gq = bf16_to_f(f_to_bf16(acc[i][j][r]));
                    const float term = xv[r] / (1.0f + __expf(-gq));
                    float sum = 0.f + dpp_f<0x00>(term);             // quad lanes 0..3 = streams 0..3
                    sum += dpp_f<0x55>(term);
                    sum += dpp_f<0xAA>(term);
                    sum += dpp_f<0xFF>(term);
                    const float v = sum * 0.25f;
                    if (c == 0 && row < g.M) {
                        g.um_mixed[(size_t) row * D + d] = v;
                        g.um_xh[(size_t) row * D + d] = f_to_bf16(v);
                    }
                }
            }
        return;
    }
    float* const y = g.y ? g.y + (size_t) ksp * g.M * g.ldy : nullptr;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = n0 + wn * 64 + j * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row < g.M && col < g.N) {
                    if (y) y[(size_t) row * g.ldy + col] = acc[i][j][r];
                    else g.yb[(size_t) row * g.ldy + col] = f_to_bf16(acc[i][j][r]);
                }
            }
        }
}

// Skinny GEMM for a few bf16 weight rows (N <= 16: the hyper-connection inject, the GDN alpha /
// beta gates), where 128 x 128 MFMA tiles would leave most of the chip idle and read every
// activation row with 128-row tiles on 64 workgroups.  Each thread keeps its 8-value k slices of every
// weight row in registers (k = 2048 j + 8 tid .. +7), walks RB rows, and the block sums its partial
// dots (DPP within a wave, then four wave partials).  fp32 FMAs on the bf16 values.
constexpr int SK_RB = 16;                    // rows per workgroup

template <int NN, int KJ>
__global__ void __launch_bounds__(256) pf_skinny_kernel(PfGemm g) {
    __shared__ float s_red[2][4][NN];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    uint4 wv[NN][KJ];
#pragma unroll
    for (int n = 0; n < NN; ++n)
#pragma unroll
        for (int j = 0; j < KJ; ++j)
            wv[n][j] = *(const uint4*) (g.wb + (size_t) min(n, g.N - 1) * g.K + 2048 * j + 8 * tid);
    const int r0 = blockIdx.x * SK_RB, r1 = min(r0 + SK_RB, g.M);
    uint4 an[KJ];
#pragma unroll
    for (int j = 0; j < KJ; ++j) an[j] = *(const uint4*) (g.a + (size_t) r0 * g.lda + 2048 * j + 8 * tid);
    for (int t = r0; t < r1; ++t) {
        uint4 av[KJ];
#pragma unroll
        for (int j = 0; j < KJ; ++j) av[j] = an[j];
        if (t + 1 < r1) {                            // the next row's loads in flight
#pragma unroll
            for (int j = 0; j < KJ; ++j) an[j] = *(const uint4*) (g.a + (size_t) (t + 1) * g.lda + 2048 * j + 8 * tid);
        }
        float acc[NN];
#pragma unroll
        for (int n = 0; n < NN; ++n) acc[n] = 0.f;
#pragma unroll
        for (int j = 0; j < KJ; ++j) {
            const uint32_t aw[4] = {av[j].x, av[j].y, av[j].z, av[j].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float x0 = bf16_lo(aw[e]), x1 = bf16_hi(aw[e]);
#pragma unroll
                for (int n = 0; n < NN; ++n) {
                    const uint32_t ww = e == 0 ? wv[n][j].x : e == 1 ? wv[n][j].y : e == 2 ? wv[n][j].z : wv[n][j].w;
                    acc[n] = fmaf(x0, bf16_lo(ww), acc[n]);
                    acc[n] = fmaf(x1, bf16_hi(ww), acc[n]);
                }
            }
        }
        const int pb = t & 1;                        // partials alternate buffers: one barrier per row
#pragma unroll
        for (int n = 0; n < NN; ++n) {
            const float v = wave_sum(acc[n]);
            if (lane == 0) s_red[pb][w][n] = v;
        }
        __syncthreads();
        if (tid < g.N && tid < NN)
            g.y[(size_t) t * g.ldy + tid] = (s_red[pb][0][tid] + s_red[pb][1][tid]) + (s_red[pb][2][tid] + s_red[pb][3][tid]);
    }
}

// ---------------------------------------------------------------------------------------------
// embedding and hyper-connection pieces
// ---------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) pf_embed_kernel(PfEmb e, const int* __restrict__ toks, float* __restrict__ R,
                                                        int D, int HC) {
    const int t = blockIdx.y, d = blockIdx.x * 256 + threadIdx.x;
    if (d >= D) return;
    const int tok = toks[t];
    float v;
    if (e.emb_q) {                                   // stage_one_emb: out-of-range ids read row 0
        const size_t tk = (tok < 0 || tok >= e.n_vocab) ? 0 : (size_t) tok;
        v = h16_to_f(e.emb_s[(tk * D + d) / 32]) * (float) e.emb_q[tk * D + d];
    } else {
        const size_t tk = (size_t) max(0, min(tok, e.n_vocab - 1));
        v = bf16_to_f(e.emb[tk * D + d]);
    }
    for (int c = 0; c < HC; ++c) R[((size_t) t * HC + c) * D + d] = v;
}

// per (stream c, row t): R += bo * 2 sigmoid(inj_prev / HC) when a block is pending; x = bf16(R *
// rsqrt(mean R^2 + eps) * norm_w)  (pf_gr_norm_fp16, src/wzy_qsa_wmma.cuh:198-234)
// A thread holds NG groups of 4 consecutive values (group tid + 256 i), loaded and stored 16 bytes
// at a time; NG = ceil(D / 1024), D a multiple of 4 and at most 4096.
template <int NG>
__global__ void __launch_bounds__(256) pf_hc_norm_kernel(float* __restrict__ R, const float* __restrict__ bo,
                                                          const float* __restrict__ inj_prev,
                                                          const float* __restrict__ norm_w, uint16_t* __restrict__ xn,
                                                          int D, int HC, float eps) {
    __shared__ float s_red[4];
    const int c = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
    const int ng = D / 4;
    float4* r = (float4*) (R + ((size_t) t * HC + c) * D);
    const float4* bp = bo ? (const float4*) (bo + (size_t) t * D) : nullptr;
    const float gate = bo ? 2.0f / (1.0f + __expf(-inj_prev[t * HC + c] / (float) HC)) : 0.0f;
    float4 v[NG], bv[NG];
#pragma unroll
    for (int i = 0; i < NG; ++i) {                   // clamped, unconditional loads
        const int gi = min(tid + 256 * i, ng - 1);
        v[i] = r[gi];
        if (bo) bv[i] = bp[gi];
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        const int gi = tid + 256 * i;
        if (bo) {
            v[i].x = fmaf(bv[i].x, gate, v[i].x);
            v[i].y = fmaf(bv[i].y, gate, v[i].y);
            v[i].z = fmaf(bv[i].z, gate, v[i].z);
            v[i].w = fmaf(bv[i].w, gate, v[i].w);
            if (gi < ng) r[gi] = v[i];
        }
        if (gi >= ng) v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        ss += v[i].x * v[i].x;
        ss += v[i].y * v[i].y;
        ss += v[i].z * v[i].z;
        ss += v[i].w * v[i].w;
    }
    ss = block_sum<4>(ss, s_red);
    const float inv = 1.0f / sqrtf(ss / (float) D + eps);
    const float4* wp = (const float4*) (norm_w + (size_t) c * D);
    uint2* x = (uint2*) (xn + (size_t) t * HC * D + (size_t) c * D);
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        const int gi = tid + 256 * i;
        if (gi < ng) {
            const float4 w = wp[gi];
            x[gi] = make_uint2(pack_bf16(v[i].x * inv * w.x, v[i].y * inv * w.y),
                               pack_bf16(v[i].z * inv * w.z, v[i].w * inv * w.w));
        }
    }
}

__global__ void __launch_bounds__(256) pf_silu_div_kernel(const float* __restrict__ lo, uint16_t* __restrict__ loh,
                                                           size_t n, int nsplit, float inv_hc) {
    const size_t i = (size_t) blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float s = nsplit == 4 ? (lo[i] + lo[n + i]) + (lo[2 * n + i] + lo[3 * n + i]) : lo[i];
    const float v = s * inv_hc;
    loh[i] = f_to_bf16(v / (1.0f + __expf(-v)));
}

// R[t][c][d] += blk[t][d] * 2 sigmoid(inj[t][c] / HC)  (gr_write_multi, src/wzy_kernels_v2.cuh:813-827)
__global__ void __launch_bounds__(256) pf_hc_write_kernel(float* __restrict__ R, const float* __restrict__ blk,
                                                           const float* __restrict__ inj, int D, int HC) {
    const int t = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
    if (i >= HC * D) return;
    const int c = i / D, d = i - c * D;
    const float g = 2.0f / (1.0f + __expf(-inj[t * HC + c] / (float) HC));
    float* r = R + (size_t) t * HC * D + i;
    *r = fmaf(blk[(size_t) t * D + d], g, *r);
}

// ---------------------------------------------------------------------------------------------
// GDN
// ---------------------------------------------------------------------------------------------
// decay = exp(softplus(a + dt) * ssm_a), beta = sigmoid(b)  (gdn_ab_act_pf_kernel)
__global__ void __launch_bounds__(256) pf_gdn_ab_kernel(PfGdn g) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= g.B * g.hv) return;
    const int t = i / g.hv, h = i - t * g.hv;
    const float a = g.ab[(size_t) t * 2 * g.hv + h] + g.dt[h];
    const float bv = g.ab[(size_t) t * 2 * g.hv + g.hv + h];
    g.beta[i] = 1.0f / (1.0f + __expf(-bv));
    const float sp = a > 20.0f ? a : log1pf(__expf(a));
    g.decay[i] = __expf(sp * g.ssm_a[h]);
}

// causal depthwise conv (3 history taps + the row) + SiLU, L2 norm of each q / k head; grid
// (QKV/128, B), 128 threads  (pf_gdn_conv_parallel, src/wzy_qsa_wmma.cuh:5-30)
// A thread runs CV_ROWS consecutive rows of its channel with a sliding window in registers, so every
// raw row is read once; the q / k rows' L2 norms span the workgroup's 128 channels (one head).
constexpr int CV_ROWS = 16;
__global__ void __launch_bounds__(128) pf_gdn_conv_kernel(PfGdn g) {
    __shared__ float s_red[2][2];                  // per row parity: one barrier per row
    const int grp = blockIdx.x, t0 = blockIdx.y * CV_ROWS, ch = grp * 128 + threadIdx.x, w = threadIdx.x >> 6;
    const int QKV = (2 * g.hk + g.hv) * 128;
    const float* h = g.conv_hist + (size_t) ch * 3;
    float win[CV_ROWS + 3];                        // rows t0-3 .. t0+CV_ROWS-1 (s < 0: history)
#pragma unroll
    for (int i = 0; i < CV_ROWS + 3; ++i) {
        const int s = t0 - 3 + i;
        win[i] = s < 0 ? h[3 + s] : g.qkv[(size_t) min(s, g.B - 1) * QKV + ch];
    }
    const float* wp = g.conv_w + (size_t) ch * 4;
    const float w0 = wp[0], w1 = wp[1], w2 = wp[2], w3 = wp[3];
    const bool qk = grp < 2 * g.hk;                // workgroup-uniform
#pragma unroll
    for (int r = 0; r < CV_ROWS; ++r) {
        const int t = t0 + r;
        if (t >= g.B) break;                       // workgroup-uniform
        const float sum = win[r] * w0 + win[r + 1] * w1 + win[r + 2] * w2 + win[r + 3] * w3;
        float y = sum / (1.0f + __expf(-sum));
        if (qk) {
            const float ws = wave_sum(y * y);
            if ((threadIdx.x & 63) == 0) s_red[r & 1][w] = ws;
            __syncthreads();
            const float ss = 0.f + s_red[r & 1][0] + s_red[r & 1][1];
            y *= 1.0f / sqrtf(ss + g.eps);
        }
        g.conv_out[(size_t) t * QKV + ch] = y;
    }
}

// conv history <- the last three raw rows (the older history where the chunk is shorter)
__global__ void __launch_bounds__(256) pf_gdn_hist_kernel(PfGdn g) {
    const int QKV = (2 * g.hk + g.hv) * 128;
    const int ch = blockIdx.x * 256 + threadIdx.x;
    if (ch >= QKV) return;
    float* h = g.conv_hist + (size_t) ch * 3;
    float v[3];
    for (int j = 0; j < 3; ++j) {
        const int s = g.B - 3 + j;
        v[j] = s >= 0 ? g.qkv[(size_t) s * QKV + ch] : h[3 + s];
    }
    h[0] = v[0];
    h[1] = v[1];
    h[2] = v[2];
}

// Sum over each 32-lane half: the 16-lane DPP sum, then the two rows of the half swapped in one
// VALU op (v_permlane16_swap) and added; every lane of the half gets the same value.
// (Written as inline assembly: through the builtin, this compiler hands both results of the swap in
// one register when they feed one add.  The s_nops cover the VALU-write-to-permlane hazard.)
WZY_DEV float sum32_pl(float v) {
    v = sum16(v);
    uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}

constexpr int GR_LPC = 32;                    // lanes per state column (half a wave)
constexpr int GR_RPL = 128 / GR_LPC;          // state rows per lane (4)
constexpr int GR_CPW = 64 / GR_LPC;           // columns per wave (2)
constexpr int GR_WAVES = 4;
constexpr int GR_COLS = GR_CPW * GR_WAVES;    // columns per workgroup (8)
constexpr int GR_STEPS = 32;                  // rows staged per LDS buffer (= lanes per column: lane r
                                              // keeps row r's output for one store per buffer)
static_assert(GR_STEPS * GR_COLS <= 256, "v staging: one value per thread");
static_assert(GR_RPL == 4, "the row loop holds 4 state rows per lane");
static_assert(GR_STEPS == GR_LPC, "one output row per lane of a column");

// k . q per (row, key head), with the recurrence's lane layout (lane r of a 32-lane half holds
// elements 4r .. 4r+3) and its 32-lane sum: a parallel pass, so the sequential row loop below reads
// one value per row instead of forming and reducing the product itself.  grid ceil(B * hk / 8), 256
// threads (8 pairs per workgroup, one per 32-lane half).
__global__ void __launch_bounds__(256) pf_gdn_kq_kernel(PfGdn g) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, r8 = lane & 31;
    const int np = g.B * g.hk, QKV = (2 * g.hk + g.hv) * 128;
    const int p = blockIdx.x * 8 + w * 2 + (lane >> 5), pc = min(p, np - 1);
    const int t = pc / g.hk, kh = pc - t * g.hk;
    const float4 q4 = *(const float4*) (g.conv_out + (size_t) t * QKV + kh * 128 + r8 * GR_RPL);
    const float4 k4 = *(const float4*) (g.conv_out + (size_t) t * QKV + (g.hk + kh) * 128 + r8 * GR_RPL);
    float kq = k4.x * q4.x;
    kq = fmaf(k4.y, q4.y, kq);
    kq = fmaf(k4.z, q4.z, kq);
    kq = fmaf(k4.w, q4.w, kq);
    kq = sum32_pl(kq);
    if (r8 == 0 && p < np) g.kq[p] = kq;
}

// Delta rule over the chunk's rows for one value head and GR_COLS state columns (each column of
// the state evolves independently): per row, S *= decay; kv = S^T k; delta = (v - kv) * beta;
// S += k delta^T; o = S^T q / sqrt(128).  grid (hv * 128 / GR_COLS), 256 threads.  A column's 128
// rows are spread over 32 lanes (4 per lane), so a row costs a few instructions per lane and two
// 32-lane sums (DPP within each 16-lane row, then a permlane swap); k . q comes precomputed.  The
// rows' q and k (all 128 of the key head), the columns' v and the per-row scalars go through LDS 32
// rows at a time, the next 32 loaded while these run.
// (pf_gdn_recur_kh_kernel, src/wzy_qsa_wmma.cuh:56-195; fused_gdn_step_norm_multi,
// src/wzy_kernels_v2.cuh:908-984)
__global__ void __launch_bounds__(256) pf_gdn_recur_kernel(PfGdn g) {
    __shared__ __align__(16) float sq[2][GR_STEPS][128];
    __shared__ __align__(16) float sk[2][GR_STEPS][128];
    __shared__ float sv[2][GR_STEPS][GR_COLS];
    __shared__ float4 sgb[2][GR_STEPS];                         // per row: decay, beta, k . q, unused
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int h = blockIdx.x / (128 / GR_COLS), cb = blockIdx.x % (128 / GR_COLS);
    const int kh = h % g.hk;
    const int QKV = (2 * g.hk + g.hv) * 128, GV = g.hv * 128;
    const int r8 = lane & (GR_LPC - 1), c8 = lane / GR_LPC;     // row slot, column of the wave
    const int lc = w * GR_CPW + c8, col = cb * GR_COLS + lc;
    float* S = g.state + (size_t) h * 128 * 128;
    float s[GR_RPL];
#pragma unroll
    for (int i = 0; i < GR_RPL; ++i) s[i] = S[(size_t) (r8 * GR_RPL + i) * 128 + col];

    // staging of rows t0 .. t0+GR_STEPS-1: q and k (128 each) of key head kh, v of the columns, the
    // per-row decay, beta and k . q.  Row indices are clamped (rows past the chunk are never used), so
    // every load is unconditional.
    constexpr int QK_PER = GR_STEPS * 2 * 128 / 256;      // floats per thread (32)
    float rq[QK_PER];
    float rv = 0.f, rg = 0.f;
    const int qk_off = (tid >= 128 ? g.hk * 128 : 0) + kh * 128 + (tid & 127);
    auto load = [&](int t0) {
#pragma unroll
        for (int u = 0; u < QK_PER; ++u) rq[u] = g.conv_out[(size_t) min(t0 + u, g.B - 1) * QKV + qk_off];
        {
            const int step = min(tid / GR_COLS, GR_STEPS - 1), j = tid % GR_COLS, t = min(t0 + step, g.B - 1);
            rv = g.conv_out[(size_t) t * QKV + 2 * g.hk * 128 + h * 128 + cb * GR_COLS + j];
        }
        {
            const int t = min(t0 + (tid & (GR_STEPS - 1)), g.B - 1);
            const float* src = tid < GR_STEPS ? g.decay + (size_t) t * g.hv + h
                               : tid < 2 * GR_STEPS ? g.beta + (size_t) t * g.hv + h
                                                    : g.kq + (size_t) t * g.hk + kh;
            rg = *src;
        }
    };
    auto store = [&](int bb) {
#pragma unroll
        for (int u = 0; u < QK_PER; ++u) (tid >= 128 ? sk : sq)[bb][u][tid & 127] = rq[u];
        if (tid < GR_STEPS * GR_COLS) sv[bb][tid / GR_COLS][tid % GR_COLS] = rv;
        if (tid < 3 * GR_STEPS) ((float*) &sgb[bb][tid & (GR_STEPS - 1)])[tid / GR_STEPS] = rg;
    };

    // one row of the delta rule from its operands (k . q precomputed):
    //   kv = dec * (S^T k),  o = dec * (S^T q) + delta * (k.q)  (= (dec S + k delta^T)^T q)
    float o_row = 0.f;                                      // lane r8 keeps row t0 + r8's output
    auto row = [&](int st, const float4 k4, const float4 q4, float vv, const float4 gbk) {
        const float dec = gbk.x, beta = gbk.y, kq = gbk.z;
        float a = s[0] * k4.x, c = s[0] * q4.x;
        a = fmaf(s[1], k4.y, a); c = fmaf(s[1], q4.y, c);
        a = fmaf(s[2], k4.z, a); c = fmaf(s[2], q4.z, c);
        a = fmaf(s[3], k4.w, a); c = fmaf(s[3], q4.w, c);
        a = sum32_pl(a);
        c = sum32_pl(c);
        const float delta = (vv - dec * a) * beta;
        const float o = fmaf(dec, c, delta * kq) * 0.08838834764831845f;
        s[0] = fmaf(k4.x, delta, dec * s[0]);
        s[1] = fmaf(k4.y, delta, dec * s[1]);
        s[2] = fmaf(k4.z, delta, dec * s[2]);
        s[3] = fmaf(k4.w, delta, dec * s[3]);
        o_row = r8 == st ? o : o_row;
    };

    const int nblk = (g.B + GR_STEPS - 1) / GR_STEPS;
    load(0);
    store(0);
    __syncthreads();
    for (int kb = 0; kb < nblk; ++kb) {
        const int bb = kb & 1, t0 = kb * GR_STEPS;
        if (kb + 1 < nblk) load(t0 + GR_STEPS);
        const int n = min(GR_STEPS, g.B - t0);
        // operands come from LDS one row ahead, alternating between two register sets (rows st and
        // st + 1), so their latency hides behind the previous row and no copies are needed.  The loop
        // is unrolled over the whole buffer: every LDS address is a constant offset.
        float4 kA = *(const float4*) &sk[bb][0][r8 * GR_RPL], qA = *(const float4*) &sq[bb][0][r8 * GR_RPL];
        float vA = sv[bb][0][lc];
        float4 pA = sgb[bb][0];
        float4 kB, qB, pB;
        float vB;
        auto pair = [&](int st) {                            // rows st (set A) and st + 1 (set B)
            const int s1 = min(st + 1, GR_STEPS - 1), s2 = min(st + 2, GR_STEPS - 1);
            kB = *(const float4*) &sk[bb][s1][r8 * GR_RPL];
            qB = *(const float4*) &sq[bb][s1][r8 * GR_RPL];
            vB = sv[bb][s1][lc];
            pB = sgb[bb][s1];
            row(st, kA, qA, vA, pA);
            if (st + 1 >= n) return;                         // workgroup-uniform
            kA = *(const float4*) &sk[bb][s2][r8 * GR_RPL];
            qA = *(const float4*) &sq[bb][s2][r8 * GR_RPL];
            vA = sv[bb][s2][lc];
            pA = sgb[bb][s2];
            row(st + 1, kB, qB, vB, pB);
        };
        if (n == GR_STEPS) {
#pragma unroll
            for (int st = 0; st < GR_STEPS; st += 2) pair(st);
        } else {
            for (int st = 0; st < n; st += 2) pair(st);
        }
        // the refill first: it waits for this buffer's loads, long arrived; the output store after it
        // is then waited on by nothing before the next buffer's rows
        if (kb + 1 < nblk) store(bb ^ 1);
        if (r8 < n) g.o[(size_t) (t0 + r8) * GV + h * 128 + col] = o_row;
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < GR_RPL; ++i) S[(size_t) (r8 * GR_RPL + i) * 128 + col] = s[i];
}

// y = bf16(o * rsqrt(mean o^2 + eps) * gamma * sigmoid(z)) per (head, row); grid (hv, B), 128 threads
// (pf_gdn_rmsnorm_gate_parallel, src/wzy_qsa_wmma.cuh:176-195)
__global__ void __launch_bounds__(128) pf_gdn_norm_kernel(PfGdn g) {
    __shared__ float s_red[2];
    const int h = blockIdx.x, t = blockIdx.y, c = threadIdx.x;
    const size_t i = ((size_t) t * g.hv + h) * 128 + c;
    const float o = g.o[i];
    const float ss = block_sum<2>(o * o, s_red);
    const float sc = 1.0f / sqrtf(ss * (1.0f / 128.0f) + g.eps);
    g.y[i] = f_to_bf16(o * sc * g.gamma[c] / (1.0f + __expf(-g.z[i])));
}

// ---------------------------------------------------------------------------------------------
// QSA
// ---------------------------------------------------------------------------------------------
constexpr int PR_ROWS = 4;                    // rows per prep workgroup

// grid (qh + kvh + ih, ceil(B / PR_ROWS)), 256 threads: q heads, kv heads (+ INT8 append), indexer q heads
__global__ void __launch_bounds__(256) pf_qsa_prep_kernel(PfQsaPrep a, int B) {
    __shared__ float s_vals[256];
    __shared__ float s_red[4];
    const QsaDims& dm = a.dm;
    const int role = blockIdx.x, tid = threadIdx.x;
    const int base = *a.pos, hd = dm.hd, kvd = dm.kvh * dm.hd;
    for (int t = blockIdx.y * PR_ROWS; t < min(B, (int) (blockIdx.y + 1) * PR_ROWS); ++t) {
        const int pos = base + t;
        if (role < dm.qh) {
            norm_rope(a.qg + (size_t) t * dm.qh * 2 * hd + (size_t) role * 2 * hd, hd, a.q_norm, a.cos_tab, a.sin_tab, pos,
                      dm.n_rot, dm.eps, s_vals, s_red);
        } else if (role < dm.qh + dm.kvh) {
            const int j = role - dm.qh;
            float* kp = a.kk + (size_t) t * kvd + (size_t) j * hd;
            norm_rope(kp, hd, a.k_norm, a.cos_tab, a.sin_tab, pos, dm.n_rot, dm.eps, s_vals, s_red);
            if (tid < hd) qsa_kv_store(dm, a.kv, pos, j, kp[tid], a.vv[(size_t) t * kvd + (size_t) j * hd + tid]);
            __syncthreads();
        } else {
            const int i = role - dm.qh - dm.kvh;
            norm_rope(a.q_idx + (size_t) t * dm.ih * dm.idim + (size_t) i * dm.idim, dm.idim, a.iq_norm, a.cos_tab,
                      a.sin_tab, pos, dm.n_rot, dm.eps, s_vals, s_red);
        }
    }
}

// One workgroup per indexer event of the chunk [p0, p0 + B): event 0 is position 0 when the chunk
// starts the context (its key doubles as the open-block placeholder "dead"), the others are the
// positions that complete a block.  A block's cells before p0 come from the tail as it was before
// the chunk.  The last event writes the placeholder row after its block (dead, recomputed from row
// 0 when this chunk sets it).  Final state equals B single-row appends (qsa_indexer_append_multi,
// src/wzy_qsa_256k.cuh:147-209).
__global__ void __launch_bounds__(256) pf_idx_append_kernel(PfIdxAppend a, int p0, int B, int has0, int pc0,
                                                             int n_ev) {
    __shared__ float s_vals[256];
    __shared__ float s_red[4];
    const QsaDims& dm = a.dm;
    const int D = dm.idim, BL = dm.iblk, d = threadIdx.x;
    const int e = blockIdx.x;
    const bool last = e == n_ev - 1;
    auto raw = [&](int cell) { return d < D ? round_h16(a.idx_raw[(size_t) (cell - p0) * D + d]) : 0.f; };
    if (has0 && e == 0) {
        const float inc = raw(0);
        const float y = idx_block_key(dm, [&](int) { return inc; }, a.ik_norm, a.cos_tab, a.sin_tab, 0, s_vals, s_red);
        if (d < D) {
            a.ix.dead[d] = y;
            if (p0 + B - 1 < BL - 1) a.ix.pooled[d] = f_to_h16(y);     // block 0 stays open in this chunk
        }
        return;
    }
    const int p = pc0 + (e - has0) * BL, b = p / BL;
    auto cell = [&](int jj) {
        const int c = b * BL + jj;
        return c >= p0 ? raw(c) : (d < D ? a.ix.tail[jj * D + d] : 0.f);
    };
    const float y = idx_block_key(dm, cell, a.ik_norm, a.cos_tab, a.sin_tab, BL * b, s_vals, s_red);
    float dead = 0.f;
    if (last) {
        if (p0 == 0) {
            const float inc = raw(0);
            dead = idx_block_key(dm, [&](int) { return inc; }, a.ik_norm, a.cos_tab, a.sin_tab, 0, s_vals, s_red);
        } else {
            dead = d < D ? a.ix.dead[d] : 0.f;
        }
    }
    if (d < D) {
        a.ix.pooled[(size_t) b * D + d] = f_to_h16(y);
        if (last) a.ix.pooled[(size_t) (b + 1) * D + d] = f_to_h16(dead);
    }
}

// tail slot s <- the last chunk cell at a position with p % iblk == s (s < iblk - 1)
__global__ void __launch_bounds__(128) pf_idx_tail_kernel(PfIdxAppend a, int p0, int B) {
    const int D = a.dm.idim, BL = a.dm.iblk, d = threadIdx.x;
    if (d >= D) return;
    const int pe = p0 + B - 1;
    for (int s = 0; s < BL - 1; ++s) {
        const int c = pe - ((pe % BL) - s + BL) % BL;             // last position <= pe in slot s
        if (c >= p0) a.ix.tail[s * D + d] = round_h16(a.idx_raw[(size_t) (c - p0) * D + d]);
    }
}

// Indexer block scores of the chunk's rows on MFMA: score[t][b] = sum over heads h of
// relu(q_h[t] . key[b]), fp16 queries and keys with fp32 products and sums (v_mfma_f32_32x32x16_f16,
// as the reference's prefill scorer runs on WMMA).  Workgroup = 32 rows x 256 blocks, wave w: blocks
// 64w .. 64w+63 as two 32 x 32 tiles, the four heads' accumulators side by side; the queries are
// staged in LDS as fp16, each wave loads its keys' k slices straight into B fragments.  Only complete
// blocks of rows whose context exceeds top_k are written; the row group's first workgroup also
// scores the open block against the placeholder key (fp32, +1e9 while the block is partial), as the
// decode scorer does.  (qsa_block_scores_wmma, src/wzy_qsa_wmma.cuh:492-612)
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
constexpr int PS_ROWS = 32, PS_BLOCKS = 256;

__global__ void __launch_bounds__(256, 3) pf_score_kernel(QsaScoreArgs a) {
    __shared__ __align__(16) _Float16 sQ[4][PS_ROWS][128 + 8];
    const QsaDims& dm = a.dm;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r0 = blockIdx.y * PS_ROWS, nrows = min(PS_ROWS, a.rows - r0);
    const int base = *a.pos + r0;
    const int B = dm.iblk, IH = dm.ih;
    const int n_kv_max = base + nrows;
    if (n_kv_max <= dm.topk) return;                 // short context: identity selection
    const int b0 = blockIdx.x * PS_BLOCKS;
    const bool tail_wg = blockIdx.x == 0;
    const int b_lim = min(a.max_b, n_kv_max / B);
    if (b0 >= b_lim && !tail_wg) return;
    const float* q_idx = a.q_idx + (size_t) r0 * IH * 128;
    float* scores = a.scores + (size_t) r0 * a.max_b;

    for (int i = tid; i < 4 * PS_ROWS * 32; i += 256) {     // (head, row, 4 k) -> fp16
        const int h = i / (PS_ROWS * 32), r = (i / 32) % PS_ROWS, k4 = i % 32;
        float4 q = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r < nrows && h < IH) q = *(const float4*) (q_idx + (size_t) r * IH * 128 + (size_t) h * 128 + 4 * k4);
        _Float16* d = &sQ[h][r][4 * k4];
        d[0] = (_Float16) q.x; d[1] = (_Float16) q.y; d[2] = (_Float16) q.z; d[3] = (_Float16) q.w;
    }
    __syncthreads();

    if (b0 + 64 * w < b_lim) {
        // one 32-block tile at a time: 64 accumulator registers, so several workgroups share a CU
        const int kb = (lane >> 5) * 8;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int b = b0 + 64 * w + 32 * c + (lane & 31);
            const _Float16* kp = (const _Float16*) a.pooled + (size_t) min(b, b_lim - 1) * 128 + kb;
            f32x16_t acc[4];
#pragma unroll
            for (int h = 0; h < 4; ++h)
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[h][i] = 0.f;
            f16x8_t bv[8];
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) bv[ks] = *(const f16x8_t*) (kp + 16 * ks);
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) {
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    if (h >= IH) break;                  // uniform
                    const f16x8_t av = *(const f16x8_t*) &sQ[h][lane & 31][16 * ks + kb];
                    acc[h] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv[ks], acc[h], 0, 0, 0);
                }
            }
            // acc[h][i] = q_h[row 8*(i/4) + 4*(lane/32) + i%4] . key[block 32c + lane%32]
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int t = 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
                float sc = 0.f;
#pragma unroll
                for (int h = 0; h < 4; ++h)
                    if (h < IH) sc += acc[h][i] > 0.f ? acc[h][i] : 0.f;
                const int n_kv = base + t + 1;
                if (t < nrows && n_kv > dm.topk && b < n_kv / B) scores[(size_t) t * a.max_b + b] = sc;
            }
        }
    }
    // open block: fp32 dot with the placeholder key (wave w handles rows w, w + 4, ...)
    if (tail_wg) {
        for (int t = w; t < nrows; t += 4) {
            const int n_kv = base + t + 1;
            const int nbid = n_kv / B;
            if (n_kv <= dm.topk || nbid >= a.max_b) continue;
            float score = 0.f;
            for (int h = 0; h < IH; ++h) {
                float p = 0.f;
                for (int k = lane; k < 128; k += 64) p = fmaf(a.dead[k], q_idx[(size_t) t * IH * 128 + (size_t) h * 128 + k], p);
                p = wave_sum(p);
                score += p > 0.f ? p : 0.f;
            }
            if (n_kv % B != 0) score += 1e9f;
            if (lane == 0) scores[(size_t) t * a.max_b + nbid] = score;
        }
    }
}

// Sparse GQA attention of one row and one KV head (grid (kvh, B), 256 threads): the group's query
// heads (up to 16, rows of a 16 x 16 fp16 MFMA tile) against the selected cells, 64 per load step.
// Per step: K of 64 cells dequantised to fp16 in LDS (row major), scores on
// v_mfma_f32_16x16x16_f16 (wave w: cells 16w .. 16w+15, all 256 dims as two 128-dim chains added in
// fp32), then two 32-cell softmax blocks in order (the online softmax per head with fp16 weights,
// as the reference's 32-cell steps), V dequantised into LDS transposed (dims x cells) and P.V on
// MFMA into the accumulators, rescaled by exp(m_old - m_new) before each block.  The next step's K
// and V codes (32 KB) are loaded while a step computes, from cell ids staged in LDS a step earlier.  out = acc / max(l, 1e-20) * sigmoid(gate),
// bf16.
constexpr int AT_C = 64;                      // cells per load step (two softmax blocks of 32)
constexpr int AT_B = 32;                      // cells per softmax block
constexpr int AT_QLD = 256 + 8;               // LDS row strides (halves)
constexpr int AT_VLD = AT_C + 4;

// LDS placement of K dim d in a cell row: the upper 128 dims swap neighbouring 4-dim groups, so the
// 64 lanes of a K staging store (16 cells x 4 dim quarters; quarters q and q + 2 lie 64 words apart)
// spread over more banks.  The score reads take one 16-dim slice, so their pattern is unchanged.
// This swap, the V^T rotation below and the pitches of V^T and sS were chosen by measuring LDS bank
// conflict counts and the prefill time of variants.
WZY_DEV int at_kcol(int d) { return d ^ ((d >> 5) & 4); }
// LDS column of cell c in row d of V^T: the cells are rotated by 8 * ((d / 16) % 8) (mod 64), so the
// 16 lanes that stage one cell group (rows 16 apart, which the pitch alone would put in one bank
// group) start in different banks; the 16 rows a P.V read spans share one rotation.
WZY_DEV int at_vcol(int d, int c) { return (c + 8 * ((d >> 4) & 7)) & (AT_C - 1); }

WZY_DEV f16x4_t h4_from(const _Float16* p) { return *(const f16x4_t*) p; }

__global__ void __launch_bounds__(256, 3) pf_attn_kernel(PfAttn a) {
    // K of a step and then its V^T share one region (37 KB instead of 70), so three workgroups fit a
    // CU: the scores read K, V is staged after every wave is done with K, P.V reads V^T.
    __shared__ __align__(16) _Float16 sU[256 * AT_VLD];
    _Float16 (*const sK)[AT_QLD] = (_Float16 (*)[AT_QLD]) sU;
    _Float16 (*const sVt)[AT_VLD] = (_Float16 (*)[AT_VLD]) sU;
    static_assert(AT_C * AT_QLD <= 256 * AT_VLD, "K fits the shared region");
    __shared__ __align__(16) _Float16 sP[2][16][AT_B + 8];
    __shared__ float sS[16][AT_C + 4];                 // pitch 68: a wave's score writes (rows 4 apart) hit distinct banks
    __shared__ float s_m[16], s_l[16], s_al[2][16];
    __shared__ int sIds[2][AT_C];                 // selected cell ids of the next two steps
    const QsaDims& dm = a.dm;
    const int j = blockIdx.x, t = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int hd = 256, kvd = dm.kvh * hd, gq = dm.qh / dm.kvh, scg = hd / 64;
    const int n_kv = *a.pos + t + 1;
    const int width = min(n_kv, dm.topk);
    const int* ids = a.sel + (size_t) t * dm.topk;
    const float* qg = a.qg + (size_t) t * dm.qh * 2 * hd;

    const int l16 = lane & 15, kq4 = lane >> 4;   // MFMA 16x16x16: row/col l16, k quad kq4
    // the A operand of every score MFMA, held in registers: q[head l16][16 kk + 4 kq4 .. +3] / 16
    f16x4_t qa[16];
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
        const float4 q4 = l16 < gq ? *(const float4*) (qg + (size_t) (j * gq + l16) * 2 * hd + kk * 16 + 4 * kq4)
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
        qa[kk] = f16x4_t{(_Float16) (q4.x * 0.0625f), (_Float16) (q4.y * 0.0625f), (_Float16) (q4.z * 0.0625f),
                         (_Float16) (q4.w * 0.0625f)};
    }
    if (tid < 16) {
        s_m[tid] = -1e30f;
        s_l[tid] = 0.f;
    }
    // K staging: thread -> cell kc = tid / 4, dims 64 * (tid % 4) .. +63 (64 code bytes, one scale)
    const int kc = tid >> 2, kd0 = (tid & 3) * 64;
    // V staging: thread -> cells 4 * (tid / 16) .. +3, dims 16 * (tid % 16) .. +15
    const int vc0 = (tid >> 4) * 4, vd0 = (tid & 15) * 16;
    uint4 kq[4], vq[4];
    uint16_t ksc = 0, vsc[4];
    int rid = 0;
    // the ids of a step are read from global memory two steps ahead and staged in LDS, so the K / V
    // loads of the next step depend on no global load of their own step
    auto load_ids = [&](int base) { rid = ids[base + min(tid & (AT_C - 1), width - base - 1)]; };
    auto store_ids = [&](int slot) {
        if (tid < AT_C) sIds[slot][tid] = rid;
    };
    auto load_k = [&](int base, int slot) {
        const int cnt = min(AT_C, width - base);
        {
            const bool ok = kc < cnt;
            const size_t p = qsa_kv_slot(sIds[slot][ok ? kc : 0], dm);
            const int8_t* kp = a.kv.kq + p * kvd + (size_t) j * hd + kd0;
#pragma unroll
            for (int u = 0; u < 4; ++u) kq[u] = ok ? *(const uint4*) (kp + 16 * u) : make_uint4(0, 0, 0, 0);
            ksc = ok ? a.kv.ks[p * (kvd / 64) + (size_t) j * scg + kd0 / 64] : (uint16_t) 0;
        }
    };
    auto load_v = [&](int base, int slot) {
        const int cnt = min(AT_C, width - base);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const bool ok = vc0 + u < cnt;
            const size_t p = qsa_kv_slot(sIds[slot][ok ? vc0 + u : 0], dm);
            vq[u] = ok ? *(const uint4*) (a.kv.vq + p * kvd + (size_t) j * hd + vd0) : make_uint4(0, 0, 0, 0);
            vsc[u] = ok ? a.kv.vs[p * (kvd / 64) + (size_t) j * scg + vd0 / 64] : (uint16_t) 0;
        }
    };
    auto store_k = [&]() {
        const _Float16 s = __builtin_bit_cast(_Float16, ksc);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t wv[4] = {kq[u].x, kq[u].y, kq[u].z, kq[u].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                f16x4_t v;
#pragma unroll
                for (int b = 0; b < 4; ++b) v[b] = (_Float16) (int8_t) (wv[i] >> (8 * b)) * s;
                *(f16x4_t*) &sK[kc][at_kcol(kd0 + 16 * u + 4 * i)] = v;
            }
        }
    };
    auto store_v = [&]() {
        _Float16 vs[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) vs[u] = __builtin_bit_cast(_Float16, vsc[u]);
#pragma unroll
        for (int i = 0; i < 16; ++i) {               // dim vd0 + i of the 4 cells
            f16x4_t v;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t word = i < 4 ? vq[u].x : i < 8 ? vq[u].y : i < 12 ? vq[u].z : vq[u].w;
                v[u] = (_Float16) (int8_t) (word >> (8 * (i & 3))) * vs[u];
            }
            *(f16x4_t*) &sVt[vd0 + i][at_vcol(vd0, vc0)] = v;
        }
    };

    f32x4_t acc[4];                               // out[h = 4*(lane/16) + i][d = 64w + 16db + lane%16]
#pragma unroll
    for (int db = 0; db < 4; ++db) acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    if (width > 0) {
        load_ids(0);
        store_ids(0);
    }
    __syncthreads();
    if (width > 0) {
        load_k(0, 0);
        load_v(0, 0);
    }
    if (AT_C < width) load_ids(AT_C);
    if (width > 0) store_k();
    if (AT_C < width) store_ids(1);
    __syncthreads();
    // per step: the next step's K loads go out first; V of this step (in registers since the middle
    // of the previous step) is staged once the scores are done, and the next step's V loads follow
    for (int base = 0, stp = 0; base < width; base += AT_C, ++stp) {
        const int cnt = min(AT_C, width - base);
        const bool more = base + AT_C < width, more2 = base + 2 * AT_C < width;
        if (more) load_k(base + AT_C, (stp + 1) & 1);
        if (more2) load_ids(base + 2 * AT_C);
        // scores: wave w -> cells 16w .. 16w+15, dims 0-127 and 128-255 as separate chains
        if (16 * w < cnt) {
            f32x4_t sc0 = {0.f, 0.f, 0.f, 0.f}, sc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) {
                sc0 = __builtin_amdgcn_mfma_f32_16x16x16f16(qa[kk], h4_from(&sK[16 * w + l16][kk * 16 + 4 * kq4]), sc0,
                                                            0, 0, 0);
                sc1 = __builtin_amdgcn_mfma_f32_16x16x16f16(qa[8 + kk], h4_from(&sK[16 * w + l16][at_kcol(128 + kk * 16 + 4 * kq4)]),
                                                            sc1, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) sS[4 * kq4 + i][16 * w + l16] = sc0[i] + sc1[i];
        }
        __syncthreads();
        store_v();                                   // K is no longer read: V^T takes the region
        if (more) load_v(base + AT_C, (stp + 1) & 1);
        // online softmax, two 32-cell blocks in order: wave w -> heads 4w .. 4w+3, two per pass
        // (lane halves), lane = cell of the block
#pragma unroll
        for (int pass = 0; pass < 2; ++pass) {
            const int h = 4 * w + 2 * pass + (lane >> 5), c = lane & 31;
            float m_run = h < gq ? s_m[h] : 0.f, l_run = h < gq ? s_l[h] : 0.f;
#pragma unroll
            for (int sb = 0; sb < 2; ++sb) {
                const int cc = AT_B * sb + c;
                const bool ok = cc < cnt && h < gq;
                const float sv = ok ? sS[h][cc] : -1e30f;
                const float rmax = max32(sv);
                const float m_new = fmaxf(m_run, rmax);
                const float al = h < gq ? __expf(m_run - m_new) : 1.f;
                const float pw = ok ? __expf(sv - m_new) : 0.f;
                const float psum = sum32(pw);
                sP[sb][h][c] = (_Float16) pw;
                l_run = l_run * al + psum;
                m_run = m_new;
                if (c == 0) s_al[sb][h] = al;
            }
            if (c == 0 && h < gq) {
                s_m[h] = m_run;
                s_l[h] = l_run;
            }
        }
        __syncthreads();
        // P.V: wave w -> dims 64w .. 64w+63 (four 16-dim blocks), per softmax block two k16 slices
#pragma unroll
        for (int sb = 0; sb < 2; ++sb) {
            if (AT_B * sb >= cnt) break;             // workgroup-uniform
            float al[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) al[i] = s_al[sb][4 * kq4 + i];
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[db][i] *= al[i];
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const f16x4_t pv = h4_from(&sP[sb][l16][ks * 16 + 4 * kq4]);
#pragma unroll
                for (int db = 0; db < 4; ++db) {
                    const int d = 64 * w + 16 * db + l16;
                    const f16x4_t vv = h4_from(&sVt[d][at_vcol(d, AT_B * sb + ks * 16 + 4 * kq4)]);
                    acc[db] = __builtin_amdgcn_mfma_f32_16x16x16f16(pv, vv, acc[db], 0, 0, 0);
                }
            }
        }
        __syncthreads();
        if (more) store_k();
        if (more2) store_ids(stp & 1);
        __syncthreads();
    }
    // acc[db][i] = O[head 4*kq4 + i][dim 64w + 16db + l16]
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int h = 4 * kq4 + i;
        if (h >= gq) continue;
        const float inv = 1.0f / fmaxf(s_l[h], 1e-20f);
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            const int d = 64 * w + 16 * db + l16;
            const float gate = qg[(size_t) (j * gq + h) * 2 * hd + hd + d];
            const float v = (acc[db][i] * inv) / (1.0f + __expf(-gate));
            a.out[(size_t) t * dm.qh * hd + (size_t) (j * gq + h) * hd + d] = f_to_bf16(v);
        }
    }
}

}  // namespace

// ---------------------------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------------------------
namespace wzy {

// Q8_0 rows -> bf16 (one thread per 8 values): out = bf16(q * fp16 scale), the rounding the GEMM's
// own staging applies (q8_quarter_bf16), so a GEMM on the expanded rows computes the same values.
__global__ void __launch_bounds__(256) pf_q8_to_bf16_kernel(const int8_t* __restrict__ q, const uint16_t* __restrict__ s,
                                                            uint16_t* __restrict__ out, size_t n8) {
    const size_t i = (size_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n8) return;
    const uint2 c = *(const uint2*) (q + 8 * i);
    const float sc = h16_to_f(s[i / 4]);
    const uint4 o0 = q8_quarter_bf16(c.x, c.y, sc);
    *(uint4*) (out + 8 * i) = o0;
}

int launch_pf_gemm(const PfGemm& g0, hipStream_t st) {
    PfGemm g = g0;
    if (g.wq && g.wscratch && g.M >= PF_DEQ_MIN_M && (size_t) g.N * g.K <= g.wscratch_elems && g.K % 32 == 0) {
        // many row tiles read each weight tile: expand the Q8_0 weights to bf16 once
        const size_t n8 = (size_t) g.N * g.K / 8;
        hipLaunchKernelGGL(pf_q8_to_bf16_kernel, dim3((unsigned) ((n8 + 255) / 256)), dim3(256), 0, st, g.wq, g.ws,
                           g.wscratch, n8);
        WZY_LAUNCH_CHECK();
        g.wb = g.wscratch;
        g.wq = nullptr;
        g.ws = nullptr;
    }
    const bool um = g.um_mixed != nullptr;
    const int ksplit = max(g.ksplit, 1);
    WZY_REQUIRE(g.a && (g.wq ? g.ws != nullptr : g.wb != nullptr) && (um ? g.um_xn && g.um_xh : (g.y || g.yb)),
                "pf_gemm: null operand");
    WZY_REQUIRE(g.M >= 1 && g.N >= 1 && g.K >= GK && g.K % GK == 0, "pf_gemm: M %d N %d K %d (K a multiple of %d)",
                g.M, g.N, g.K, GK);
    WZY_REQUIRE(g.lda >= g.K && g.lda % 8 == 0 && (um || g.ldy >= g.N), "pf_gemm: bad leading dimensions");
    WZY_REQUIRE(!um || (g.um_d >= 32 && g.um_d % 32 == 0 && g.N == 4 * g.um_d && ksplit == 1),
                "pf_gemm: stream-mean epilogue needs N = 4 * n_embd (n_embd %d, a multiple of 32), no K split", g.um_d);
    WZY_REQUIRE(ksplit <= 8 && (ksplit == 1 || (g.y && (g.K / GK) % ksplit == 0)),
                "pf_gemm: K split %d needs fp32 output and %d k steps divisible by it", ksplit, g.K / GK);
    if (!um && ksplit == 1 && !g.wq && g.y && g.N <= 16 && g.K % 2048 == 0 && g.K <= 8192 && g.lda % 8 == 0) {
        const int nn = g.N <= 4 ? 4 : g.N <= 8 ? 8 : 16, kj = g.K / 2048;
        // one instantiation per (rows, k slices) whose weight slices fit 64 registers; any other
        // combination takes the MFMA kernel below (a kernel for fewer k slices would drop a K range)
        const dim3 grid((g.M + SK_RB - 1) / SK_RB);
        bool done = true;
        if (nn == 4 && kj == 4) hipLaunchKernelGGL((pf_skinny_kernel<4, 4>), grid, dim3(256), 0, st, g);
        else if (nn == 4 && kj == 3) hipLaunchKernelGGL((pf_skinny_kernel<4, 3>), grid, dim3(256), 0, st, g);
        else if (nn == 4 && kj == 2) hipLaunchKernelGGL((pf_skinny_kernel<4, 2>), grid, dim3(256), 0, st, g);
        else if (nn == 4 && kj == 1) hipLaunchKernelGGL((pf_skinny_kernel<4, 1>), grid, dim3(256), 0, st, g);
        else if (nn == 8 && kj == 2) hipLaunchKernelGGL((pf_skinny_kernel<8, 2>), grid, dim3(256), 0, st, g);
        else if (nn == 8 && kj == 1) hipLaunchKernelGGL((pf_skinny_kernel<8, 1>), grid, dim3(256), 0, st, g);
        else if (nn == 16 && kj == 1) hipLaunchKernelGGL((pf_skinny_kernel<16, 1>), grid, dim3(256), 0, st, g);
        else done = false;
        if (done) {
            WZY_LAUNCH_CHECK();
            return WZY_OK;
        }
    }
    GemmArgs ga;
    ga.g = g;
    ga.mt = (g.M + GM - 1) / GM;
    ga.nt = (g.N + GN - 1) / GN;
    WZY_REQUIRE((long long) ga.mt * ga.nt * ksplit < (1LL << 31), "pf_gemm: too many tiles");
    const int grid = ga.mt * ga.nt * (um ? 1 : ksplit);
    const bool sb = grid >= 512;
    if (um && sb) hipLaunchKernelGGL((pf_gemm_kernel<true, true>), dim3(grid), dim3(256), 0, st, ga);
    else if (um) hipLaunchKernelGGL((pf_gemm_kernel<true, false>), dim3(grid), dim3(256), 0, st, ga);
    else if (sb) hipLaunchKernelGGL((pf_gemm_kernel<false, true>), dim3(grid), dim3(256), 0, st, ga);
    else hipLaunchKernelGGL((pf_gemm_kernel<false, false>), dim3(grid), dim3(256), 0, st, ga);
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

int launch_pf_embed(const PfEmb& e, const int* toks, float* R, int D, int HC, int B, hipStream_t st) {
    hipLaunchKernelGGL(pf_embed_kernel, dim3((D + 255) / 256, B), dim3(256), 0, st, e, toks, R, D, HC);
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

int launch_pf_hc_norm(float* R, const float* bo, const float* inj_prev, const float* norm_w, uint16_t* xn, int D,
                      int HC, float eps, int B, hipStream_t st) {
    WZY_REQUIRE(D >= 4 && D <= 4096 && D % 4 == 0, "pf_hc_norm: n_embd %d (a multiple of 4, at most 4096)", D);
    const dim3 grid(HC, B);
    switch ((D + 1023) / 1024) {
        case 1: hipLaunchKernelGGL(pf_hc_norm_kernel<1>, grid, dim3(256), 0, st, R, bo, inj_prev, norm_w, xn, D, HC, eps); break;
        case 2: hipLaunchKernelGGL(pf_hc_norm_kernel<2>, grid, dim3(256), 0, st, R, bo, inj_prev, norm_w, xn, D, HC, eps); break;
        case 3: hipLaunchKernelGGL(pf_hc_norm_kernel<3>, grid, dim3(256), 0, st, R, bo, inj_prev, norm_w, xn, D, HC, eps); break;
        default: hipLaunchKernelGGL(pf_hc_norm_kernel<4>, grid, dim3(256), 0, st, R, bo, inj_prev, norm_w, xn, D, HC, eps); break;
    }
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

int launch_pf_silu_div(const float* lo, uint16_t* loh, size_t n, int nsplit, float inv_hc, hipStream_t st) {
    WZY_REQUIRE(nsplit == 1 || nsplit == 4, "pf_silu_div: %d partial sums (1 or 4)", nsplit);
    hipLaunchKernelGGL(pf_silu_div_kernel, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, st, lo, loh, n, nsplit,
                       inv_hc);
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

int launch_pf_hc_write(float* R, const float* blk, const float* inj, int D, int HC, int B, hipStream_t st) {
    hipLaunchKernelGGL(pf_hc_write_kernel, dim3((HC * D + 255) / 256, B), dim3(256), 0, st, R, blk, inj, D, HC);
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

int launch_pf_gdn(const PfGdn& g, hipStream_t st) {
    WZY_REQUIRE(g.hk >= 1 && g.hv % g.hk == 0 && g.B >= 1, "pf_gdn: bad heads / rows");
    const int QKV = (2 * g.hk + g.hv) * 128;
    hipLaunchKernelGGL(pf_gdn_ab_kernel, dim3((g.B * g.hv + 255) / 256), dim3(256), 0, st, g);
    hipLaunchKernelGGL(pf_gdn_conv_kernel, dim3(QKV / 128, (g.B + CV_ROWS - 1) / CV_ROWS), dim3(128), 0, st, g);
    hipLaunchKernelGGL(pf_gdn_hist_kernel, dim3((QKV + 255) / 256), dim3(256), 0, st, g);
    hipLaunchKernelGGL(pf_gdn_kq_kernel, dim3((g.B * g.hk + 7) / 8), dim3(256), 0, st, g);
    hipLaunchKernelGGL(pf_gdn_recur_kernel, dim3(g.hv * 128 / GR_COLS), dim3(256), 0, st, g);
    hipLaunchKernelGGL(pf_gdn_norm_kernel, dim3(g.hv, g.B), dim3(128), 0, st, g);
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

int launch_pf_qsa_prep(const PfQsaPrep& a, int B, hipStream_t st) {
    WZY_TRY(qsa_check_dims(a.dm));
    const int roles = a.dm.qh + a.dm.kvh + a.dm.ih;
    hipLaunchKernelGGL(pf_qsa_prep_kernel, dim3(roles, (B + PR_ROWS - 1) / PR_ROWS), dim3(256), 0, st, a, B);
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

int launch_pf_idx_append(const PfIdxAppend& a, int p0, int B, hipStream_t st) {
    const int BL = a.dm.iblk;
    WZY_REQUIRE(a.dm.idim <= 128 && BL >= 2 && p0 >= 0 && B >= 1 && p0 + B <= a.dm.ctx_max, "pf_idx_append: bad shape");
    const int has0 = p0 == 0 ? 1 : 0;
    const int pc0 = p0 + ((BL - 1 - p0 % BL) + BL) % BL;          // first position completing a block
    const int pe = p0 + B - 1;
    const int n_comp = pe >= pc0 ? (pe - pc0) / BL + 1 : 0;
    const int n_ev = has0 + n_comp;
    if (n_ev > 0)
        hipLaunchKernelGGL(pf_idx_append_kernel, dim3(n_ev), dim3(256), 0, st, a, p0, B, has0, pc0, n_ev);
    hipLaunchKernelGGL(pf_idx_tail_kernel, dim3(1), dim3(128), 0, st, a, p0, B);
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

int launch_pf_scores(const QsaScoreArgs& a0, int rows, hipStream_t st) {
    WZY_TRY(qsa_check_dims(a0.dm));
    WZY_REQUIRE(a0.dm.idim == 128 && a0.dm.ih <= 4, "pf_scores: indexer layout unsupported");
    WZY_REQUIRE(rows >= 1 && (rows + PS_ROWS - 1) / PS_ROWS <= 65535, "pf_scores: %d rows", rows);
    QsaScoreArgs a = a0;
    a.rows = rows;
    const dim3 grid((a.max_b + PS_BLOCKS - 1) / PS_BLOCKS, (rows + PS_ROWS - 1) / PS_ROWS);
    hipLaunchKernelGGL(pf_score_kernel, grid, dim3(256), 0, st, a);
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

int launch_pf_attn(const PfAttn& a, int B, hipStream_t st) {
    WZY_TRY(qsa_check_dims(a.dm));
    WZY_REQUIRE(a.dm.hd == 256 && a.dm.qh / a.dm.kvh <= 16 && a.dm.window == 0, "pf_attn: head layout unsupported");
    WZY_REQUIRE(B >= 1 && B <= 65535, "pf_attn: %d rows", B);
    hipLaunchKernelGGL(pf_attn_kernel, dim3(a.dm.kvh, B), dim3(256), 0, st, a);
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

}  // namespace wzy

// ---------------------------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------------------------
extern "C" int wzy_gemm_bf16(const uint16_t* a, int lda, int M, int K, const int8_t* wq, const uint16_t* ws,
                             const uint16_t* wb, int N, float* y, uint16_t* yb, int ldy, void* stream) {
    WZY_REQUIRE((y == nullptr) != (yb == nullptr), "wzy_gemm_bf16: exactly one of y / yb");
    WZY_REQUIRE((wq == nullptr) != (wb == nullptr), "wzy_gemm_bf16: exactly one of wq / wb");
    PfGemm g{};
    g.a = a; g.lda = lda; g.M = M; g.N = N; g.K = K;
    g.wq = wq; g.ws = ws; g.wb = wb; g.y = y; g.yb = yb; g.ldy = ldy;
    return launch_pf_gemm(g, (hipStream_t) stream);
}

// mtp.hip -- MTP speculative drafter for gfx950 (MtpEngine, src/wzy_mtp.cuh:405-754).
//
// One draft step at cell p embeds the token at p+1 and reads a residual: the main model's pre-head
// residual at p, or the previous step's output residual when steps chain.  Launch sequence:
//   mtp_in          RMSNorm of the token embedding (pre_fc_norm_embedding) and of each residual
//                   stream (pre_fc_norm_hidden)
//   gemv_segs x2    fc_embedding, fc_hidden (Q8_0)
//   hc read         attention hyper-connection; its fold adds fc_embedding to every fc_hidden stream
//                   (a unit gate: 2*sigmoid(0) == 1)
//   gemv_segs       q (full step only), k, v projections
//   qsa_prep        q / k RMSNorm + RoPE, INT8 append of k and v into the 1,024-cell ring
//   qsa_attn        dense sliding-window attention over the ring (window mode of the QSA kernels)
//   gemv_segs       o projection
//   hc read         MLP hyper-connection (folds the attention write)
//   gemv_segs       router logits + shared-expert gate row (bf16); moe_route: softmax top-K
//   mtp_q2_gate_up  Q2_0 gate/up + SwiGLU + per-32 requant of the routed experts and the Q8_0 shared
//                   expert's, one launch
//   mtp_q2_down     Q2_0 down of the routed experts, Q8_0 shared down and the combine, one launch
//   hc read         final mixer (folds the MoE write; its residual output is the next step's input)
//   gemv_segs       draft head (Q8_0 rows of the draft vocabulary)
//   mtp_head_reduce argmax (ties: lower row) and 1 / sum(exp(l - max)) over the draft vocabulary in
//                   one launch (the last-arriving workgroup merges); writes the draft and advances the
//                   control block, so chained steps need no host round trip.
//
// Q2_0 GEMVs: a 16-byte piece of a code row holds 64 two-bit codes (value 4j+k of a 32-value chunk in
// bits 2k of byte j).  Activations are staged in LDS in the matching order, so
// (w >> 2k) & 0x03030303 lines four codes up with four int8 activations for one v_dot4_i32_i8; the
// weight (code - 1) * scale becomes sum(code * x) - sum(x) per chunk with chunk sums taken at staging.
#include <math.h>
#include <string.h>

#include <vector>

#include "../../include/wzy_kernels.h"
#include "../../include/wzy_synth.h"
#include "wzy_device.h"
#include "wzy_gemv.h"
#include "wzy_hc.h"
#include "wzy_host.h"
#include "wzy_mtp.h"
#include "wzy_qsa.h"

using namespace wzy;

namespace {

constexpr int DN_RT = 8;          // output rows of one mtp_q2_down workgroup

WZY_DEV float max8(float v) {
    v = fmaxf(v, dpp_f<DPP_XOR1>(v));
    v = fmaxf(v, dpp_f<DPP_XOR2>(v));
    v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
    return v;
}

// ---------------------------------------------------------------------------------------------
// RMSNorm of the embedded tokens and of the residual streams (mtp_rms_norm_rows, src/wzy_mtp.cuh:16-37)
// ---------------------------------------------------------------------------------------------
struct MtpInArgs {
    const uint16_t* emb;              // bf16 table, or null with the Q8_0 table emb_q / emb_s
    const int8_t* emb_q;
    const uint16_t* emb_s;
    int n_vocab;
    const int* toks;                  // [T]
    const float* rin;                 // [T][HC][D]
    const float* g_emb;               // [D]
    const float* g_hid;               // [HC][D]
    float* en;                        // [T][D]
    float* hn;                        // [T][HC][D]
    int D, HC;
    float eps;
};

// grid (1 + HC, T): workgroup 0 the embedding row, 1 + c residual stream c
// NV = values per thread (D / 256 rounded up to the instantiation): every load of the thread is
// issued before the first is used (a loop over a runtime width would wait for each load in turn).
template <int NV>
__global__ void __launch_bounds__(256) mtp_in_kernel(MtpInArgs a) {
    __shared__ float s_red[4];
    const int r = blockIdx.x, t = blockIdx.y, tid = threadIdx.x, D = a.D;
    float v[NV], g[NV];
    if (r == 0) {
        int tok = a.toks[t];
        if (tok < 0 || tok >= a.n_vocab) tok = 0;     // stage_one_emb, src/wzy_engine_v2.cu:862-863
        // embedding value d of the row: bf16, or d * q of the Q8_0 row (stage_one_emb)
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int d = min(tid + 256 * k, D - 1);
            v[k] = a.emb ? bf16_to_f(a.emb[(size_t) tok * D + d])
                         : h16_to_f(a.emb_s[(size_t) tok * (D / 32) + d / 32]) * (float) a.emb_q[(size_t) tok * D + d];
            g[k] = a.g_emb[d];
        }
    } else {
        const int c = r - 1;
        const float* src = a.rin + ((size_t) t * a.HC + c) * D;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int d = min(tid + 256 * k, D - 1);
            v[k] = src[d];
            g[k] = a.g_hid[(size_t) c * D + d];
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k)
        if (tid + 256 * k < D) ss = fmaf(v[k], v[k], ss);
    const float sc = 1.0f / sqrtf(block_sum<4>(ss, s_red) / (float) D + a.eps);
    float* dst = r == 0 ? a.en + (size_t) t * D : a.hn + ((size_t) t * a.HC + (r - 1)) * D;
#pragma unroll
    for (int k = 0; k < NV; ++k)
        if (tid + 256 * k < D) dst[tid + 256 * k] = v[k] * sc * g[k];
}

// ---------------------------------------------------------------------------------------------
// Q2_0 building blocks
// ---------------------------------------------------------------------------------------------
// Per-32 int8 quantisation of x[0..n) (d = amax/127, q = rint(x * 127/amax), quant_act_multi,
// src/wzy_kernels_v2.cuh:58-107) into LDS: natural order s_q, two-bit-code order s_p (16-value group
// G, dword k, byte b holds x[16G + 4b + k]), scales s_xs and chunk sums s_hx.  Eight lanes per chunk,
// four values each; NT (the workgroup size) is a multiple of 64.
template <int NT>
WZY_DEV void stage_x32(const float* __restrict__ x, int n, int8_t* s_q, int8_t* s_p, float* s_xs, int* s_hx) {
    for (int m = threadIdx.x; m < n / 4; m += NT) {
        const float4 v = *(const float4*) (x + 4 * m);
        float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
        amax = max8(amax);
        const float d = amax / 127.0f;
        const float inv = d > 0.f ? 127.0f / amax : 0.f;
        const int q0 = max(-127, min(127, rn_int(v.x * inv))), q1 = max(-127, min(127, rn_int(v.y * inv)));
        const int q2 = max(-127, min(127, rn_int(v.z * inv))), q3 = max(-127, min(127, rn_int(v.w * inv)));
        *(int*) (s_q + 4 * m) = (q0 & 0xFF) | ((q1 & 0xFF) << 8) | ((q2 & 0xFF) << 16) | ((q3 & 0xFF) << 24);
        int8_t* g = s_p + (size_t) (m >> 2) * 16;
        const int b = m & 3;
        g[0 * 4 + b] = (int8_t) q0;
        g[1 * 4 + b] = (int8_t) q1;
        g[2 * 4 + b] = (int8_t) q2;
        g[3 * 4 + b] = (int8_t) q3;
        const float hs = sum8((float) (q0 + q1 + q2 + q3));      // exact: |sum| <= 4064
        if ((m & 7) == 0) {
            s_xs[m >> 3] = d;
            s_hx[m >> 3] = (int) hs;
        }
    }
}

// sum over one 16-value group of code * x: w = 4 code bytes, x = the group's 4 code-order dwords
WZY_DEV int q2_dot16(uint32_t w, int4 x) {
    int s = dot4((int) (w & 0x03030303u), x.x, 0);
    s = dot4((int) ((w >> 2) & 0x03030303u), x.y, s);
    s = dot4((int) ((w >> 4) & 0x03030303u), x.z, s);
    return dot4((int) ((w >> 6) & 0x03030303u), x.w, s);
}

// Piece p of a Q2_0 row (values 64p .. 64p+63 = chunks 2p, 2p+1, one fp16 scale) against staged
// activations, without the weight scale: sum_c xs_c * (sum code*x - sum x).
WZY_DEV float q2_piece(uint4 cw, const int8_t* s_p, const float* s_xs, const int* s_hx, int p) {
    const int4* xp = (const int4*) (s_p + (size_t) 64 * p);
    const int s0 = q2_dot16(cw.x, xp[0]) + q2_dot16(cw.y, xp[1]);
    const int s1 = q2_dot16(cw.z, xp[2]) + q2_dot16(cw.w, xp[3]);
    return s_xs[2 * p] * (float) (s0 - s_hx[2 * p]) + s_xs[2 * p + 1] * (float) (s1 - s_hx[2 * p + 1]);
}

// ---------------------------------------------------------------------------------------------
// gate/up: routed Q2_0 experts (mtp_exp_gu_quant_q2, src/wzy_mtp.cuh:85-158) and the Q8_0 shared
// expert (gemm_q8p + silu_mul_quant32_multi, src/wzy_kernels_v2.cuh:1247-1280), one launch
// ---------------------------------------------------------------------------------------------
struct Q2GuArgs {
    const uint8_t* experts;
    size_t rec;
    const int* ids;                   // [K] routed experts
    int D, F, K;
    const float* x;                   // [D]
    const int8_t* shg_q; const uint16_t* shg_s;
    const int8_t* shu_q; const uint16_t* shu_s;
    int8_t* aq;                       // [K + 1][F] per-32 int8 SwiGLU activations (slot K: shared)
    float* as;                        // [K + 1][F / 32]
};

// grid (K + 1, F / 32), 512 threads: workgroup (g, tile) computes rows tile*32 .. +31 of slot g, four
// rows per wave, then their per-32 requant.  NPL = 16-byte code pieces per lane and row pair.
template <int NPL>
__global__ void __launch_bounds__(512) mtp_q2_gate_up_kernel(Q2GuArgs a) {
    extern __shared__ __align__(16) char lds[];
    const int D = a.D, F = a.F;
    int8_t* s_q = (int8_t*) lds;
    int8_t* s_p = s_q + D;
    float* s_xs = (float*) (s_p + D);
    int* s_hx = (int*) (s_xs + D / 32);
    __shared__ float s_act[32];
    const int g = blockIdx.x, tile = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    stage_x32<512>(a.x, D, s_q, s_p, s_xs, s_hx);
    __syncthreads();
    const int r0 = tile * 32 + 4 * w;
    float act[4];
    if (g < a.K) {
        const uint8_t* blob = a.experts + (size_t) a.ids[g] * a.rec;
        const uint16_t* scl = (const uint16_t*) (blob + (size_t) 2 * F * (D / 4) + (size_t) D * (F / 4));
        const int P = D / 64;                        // pieces per row; a (gate, up) pair has 2P
        uint4 cw[4][NPL];
        float dw[4][NPL];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint8_t* pair = blob + (size_t) (2 * (r0 + i)) * (D / 4);
#pragma unroll
            for (int j = 0; j < NPL; ++j) {
                const int q = lane + 64 * j;
                const bool ok = q < 2 * P;
                const int sel = q >= P ? 1 : 0;
                cw[i][j] = ok ? ld_stream_u4(pair + (size_t) q * 16) : make_uint4(0, 0, 0, 0);
                dw[i][j] = ok ? h16_to_f(scl[(size_t) (2 * (r0 + i) + sel) * P + (q - sel * P)]) : 0.f;
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float ag = 0.f, au = 0.f;
#pragma unroll
            for (int j = 0; j < NPL; ++j) {
                const int q = lane + 64 * j;
                if (q < 2 * P) {
                    const int sel = q >= P ? 1 : 0, p = q - sel * P;
                    const float v = dw[i][j] * q2_piece(cw[i][j], s_p, s_xs, s_hx, p);
                    if (sel) au += v;
                    else ag += v;
                }
            }
            ag = wave_sum(ag);
            au = wave_sum(au);
            act[i] = siluf_(ag) * au;
        }
    } else {
        const int C = D / 32;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = r0 + i;
            float ag = 0.f, au = 0.f;
            for (int c = lane; c < C; c += 64) {
                const int4 xa = *(const int4*) (s_q + 32 * c), xb = *(const int4*) (s_q + 32 * c + 16);
                const int8_t* gp = a.shg_q + (size_t) r * D + 32 * c;
                const int8_t* up = a.shu_q + (size_t) r * D + 32 * c;
                const int ig = dot16(ld_stream_i4(gp), xa) + dot16(ld_stream_i4(gp + 16), xb);
                const int iu = dot16(ld_stream_i4(up), xa) + dot16(ld_stream_i4(up + 16), xb);
                ag += h16_to_f(a.shg_s[(size_t) r * C + c]) * s_xs[c] * (float) ig;
                au += h16_to_f(a.shu_s[(size_t) r * C + c]) * s_xs[c] * (float) iu;
            }
            ag = wave_sum(ag);
            au = wave_sum(au);
            act[i] = siluf_(ag) * au;
        }
    }
    if (lane == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) s_act[4 * w + i] = act[i];
    }
    __syncthreads();
    if (w == 0) {
        const float v = lane < 32 ? s_act[lane] : 0.f;
        const float amax = max32(fabsf(v));
        const float d = amax / 127.0f;
        const float inv = amax > 0.f ? 127.0f / amax : 0.f;
        if (lane < 32) {
            a.aq[(size_t) g * F + tile * 32 + lane] = (int8_t) max(-127, min(127, rn_int(v * inv)));
            if (lane == 0) a.as[(size_t) g * (F / 32) + tile] = d;
        }
    }
}

// ---------------------------------------------------------------------------------------------
// down: routed Q2_0 (mtp_exp_down_2r_q2, src/wzy_mtp.cuh:160-207), shared Q8_0 and the combine
// comb = shared * sigmoid(sg) + sum_{k, w_k != 0} w_k * part_k (moe_combine_shared_multi,
// src/wzy_kernels_v2.cuh:1281-1294), one launch
// ---------------------------------------------------------------------------------------------
struct Q2DnArgs {
    const uint8_t* experts;
    size_t rec;
    const int* ids;
    const float* wts;
    const float* sg;
    int D, F, K;
    const int8_t* aq;                 // [K + 1][F]
    const float* as;                  // [K + 1][F / 32]
    const int8_t* shd_q; const uint16_t* shd_s;
    float* comb;                      // [D]
};

// grid D / DN_RT, 256 threads
__global__ void __launch_bounds__(256) mtp_q2_down_kernel(Q2DnArgs a) {
    extern __shared__ __align__(16) char lds[];
    const int K = a.K, F = a.F, D = a.D, P = F / 64, C = F / 32, NPART = K * P + C;
    const int tid = threadIdx.x;
    int8_t* s_p = (int8_t*) lds;                           // [K][F] code order
    int8_t* s_q = s_p + (size_t) K * F;                    // [F] shared activations, natural order
    float* s_xs = (float*) (s_q + F);                      // [K + 1][C]
    int* s_hx = (int*) (s_xs + (K + 1) * C);               // [K][C]
    float* s_part = (float*) (s_hx + K * C);               // [DN_RT][NPART]
    float* s_sum = s_part + DN_RT * NPART;                 // [DN_RT][K + 1]
    // stage the activations
    for (int i = tid; i < K * F / 4; i += 256) {
        const uint32_t v = *(const uint32_t*) (a.aq + 4 * (size_t) i);
        const int k = (4 * i) / F, off = 4 * i - k * F;
        int8_t* gdst = s_p + (size_t) k * F + (off & ~15);
        const int b = (off & 15) >> 2;
#pragma unroll
        for (int j = 0; j < 4; ++j) gdst[j * 4 + b] = (int8_t) (v >> (8 * j));
    }
    for (int i = tid; i < F / 4; i += 256) ((int*) s_q)[i] = ((const int*) (a.aq + (size_t) K * F))[i];
    for (int i = tid; i < (K + 1) * C; i += 256) s_xs[i] = a.as[i];
    for (int i = tid; i < K * C; i += 256) {
        const int* src = (const int*) (a.aq + 32 * (size_t) i);
        int s = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) s = dot4(0x01010101, src[j], s);
        s_hx[i] = s;
    }
    __syncthreads();
    const int d0 = blockIdx.x * DN_RT;
    const size_t dn_codes = (size_t) 2 * F * (D / 4);
    const size_t dn_scales = dn_codes + (size_t) D * (F / 4) + (size_t) 2 * F * (D / 64) * 2;
    for (int it = tid; it < DN_RT * K * P; it += 256) {
        const int row = it / (K * P), rem = it - row * (K * P), k = rem / P, p = rem - k * P;
        const uint8_t* blob = a.experts + (size_t) a.ids[k] * a.rec;
        const uint4 cw = ld_stream_u4(blob + dn_codes + (size_t) (d0 + row) * (F / 4) + 16 * (size_t) p);
        const float dw = h16_to_f(((const uint16_t*) (blob + dn_scales))[(size_t) (d0 + row) * P + p]);
        s_part[row * NPART + k * P + p] = dw * q2_piece(cw, s_p + (size_t) k * F, s_xs + k * C, s_hx + k * C, p);
    }
    for (int it = tid; it < DN_RT * C; it += 256) {
        const int row = it / C, c = it - row * C;
        const int8_t* wp = a.shd_q + (size_t) (d0 + row) * F + 32 * c;
        const int is = dot16(ld_stream_i4(wp), *(const int4*) (s_q + 32 * c)) +
                       dot16(ld_stream_i4(wp + 16), *(const int4*) (s_q + 32 * c + 16));
        s_part[row * NPART + K * P + c] = h16_to_f(a.shd_s[(size_t) (d0 + row) * C + c]) * s_xs[K * C + c] * (float) is;
    }
    __syncthreads();
    if (tid < DN_RT * (K + 1)) {
        const int row = tid / (K + 1), k = tid - row * (K + 1);
        const float* pr = s_part + row * NPART + (k < K ? k * P : K * P);
        const int n = k < K ? P : C;
        float s = 0.f;
        for (int i = 0; i < n; ++i) s += pr[i];
        s_sum[row * (K + 1) + k] = s;
    }
    __syncthreads();
    if (tid < DN_RT) {
        const float* sr = s_sum + tid * (K + 1);
        float s = sr[K] * sigmoidf_(*a.sg);
        for (int k = 0; k < K; ++k) {
            const float wk = a.wts[k];
            if (wk != 0.0f) s += wk * sr[k];
        }
        a.comb[d0 + tid] = s;
    }
}

// ---------------------------------------------------------------------------------------------
// draft-head reduction (mtp_head_reduce_online_part1 + mtp_head_finalize, src/wzy_mtp.cuh:293-403)
// ---------------------------------------------------------------------------------------------
// merge (ov, oi, os) into (bv, bi, es): running maximum, its lowest index, sum of exp(l - max)
WZY_DEV void lse_merge(float& bv, int& bi, float& es, float ov, int oi, float os) {
    if (os == 0.f) return;
    if (es == 0.f) {
        bv = ov; bi = oi; es = os;
        return;
    }
    if (ov > bv || (ov == bv && oi < bi)) {
        es = es * __expf(bv - ov) + os;
        bv = ov;
        bi = oi;
    } else {
        es += os * __expf(ov - bv);
    }
}
template <int CTRL>
WZY_DEV void lse_step_dpp(float& bv, int& bi, float& es) {
    const float ov = dpp_f<CTRL>(bv), os = dpp_f<CTRL>(es);
    const int oi = dpp_i<CTRL>(bi);
    lse_merge(bv, bi, es, ov, oi, os);
}
// full-wave merge; the result is wave-uniform
WZY_DEV void lse_wave(float& bv, int& bi, float& es) {
    lse_step_dpp<DPP_XOR1>(bv, bi, es);
    lse_step_dpp<DPP_XOR2>(bv, bi, es);
    lse_step_dpp<DPP_HALF_MIRROR>(bv, bi, es);
    lse_step_dpp<DPP_MIRROR>(bv, bi, es);
    {
        const float ov = swz_f<SWZ_XOR16>(bv), os = swz_f<SWZ_XOR16>(es);
        const int oi = swz_i<SWZ_XOR16>(bi);
        lse_merge(bv, bi, es, ov, oi, os);
    }
    const float v32 = as_f(__builtin_amdgcn_readlane(as_i(bv), 32));
    const float s32 = as_f(__builtin_amdgcn_readlane(as_i(es), 32));
    const int i32 = __builtin_amdgcn_readlane(bi, 32);
    bv = as_f(__builtin_amdgcn_readlane(as_i(bv), 0));
    es = as_f(__builtin_amdgcn_readlane(as_i(es), 0));
    bi = __builtin_amdgcn_readlane(bi, 0);
    lse_merge(bv, bi, es, v32, i32, s32);
}
// merge of the 4 waves of a 256-thread workgroup; every thread gets the result
WZY_DEV void lse_block(float& bv, int& bi, float& es, float* s_v, int* s_i, float* s_s) {
    lse_wave(bv, bi, es);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { s_v[w] = bv; s_i[w] = bi; s_s[w] = es; }
    __syncthreads();
    bv = s_v[0]; bi = s_i[0]; es = s_s[0];
    for (int i = 1; i < 4; ++i) lse_merge(bv, bi, es, s_v[i], s_i[i], s_s[i]);
    __syncthreads();
}

struct HeadRedArgs {
    const float* logits;
    int n;
    const int* dvocab;                // null: identity
    float* part;                      // [3][gridDim.x]: max, sum, index bits
    unsigned* arrive;                 // arrival counter, 0 between launches
    int* ctl;                         // control block
    int* out_tok;                     // [MTP_MAX_CHAIN] (host-mapped)
    float* out_prob;
};

__global__ void __launch_bounds__(256) mtp_head_reduce_kernel(HeadRedArgs a) {
    __shared__ float s_v[4], s_s[4];
    __shared__ int s_i[4];
    __shared__ bool s_last;
    const int G = gridDim.x, tid = threadIdx.x;
    float bv = 0.f, es = 0.f;
    int bi = 0;
    for (int i4 = blockIdx.x * 256 + tid; 4 * i4 < a.n; i4 += G * 256) {
        const int i0 = 4 * i4;
        float v[4];
        if (i0 + 3 < a.n) {
            const float4 q = *(const float4*) (a.logits + i0);
            v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = i0 + j < a.n ? a.logits[i0 + j] : 0.f;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (i0 + j < a.n) lse_merge(bv, bi, es, v[j], i0 + j, 1.0f);
    }
    lse_block(bv, bi, es, s_v, s_i, s_s);
    if (tid == 0) {
        a.part[blockIdx.x] = bv;
        a.part[G + blockIdx.x] = es;
        a.part[2 * G + blockIdx.x] = as_f(bi);
        __threadfence();
        s_last = atomicAdd(a.arrive, 1u) == (unsigned) (G - 1);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    bv = 0.f; es = 0.f; bi = 0;
    for (int b = tid; b < G; b += 256) lse_merge(bv, bi, es, a.part[b], as_i(a.part[2 * G + b]), a.part[G + b]);
    lse_block(bv, bi, es, s_v, s_i, s_s);
    if (tid == 0) {
        const int tok = a.dvocab ? a.dvocab[bi] : bi;
        const int slot = a.ctl[9];
        if (slot >= 0 && slot < MTP_MAX_CHAIN) {
            a.out_tok[slot] = tok;
            a.out_prob[slot] = 1.0f / fmaxf(es, 1.0f);
        }
        a.ctl[0] = a.ctl[0] + 1;
        a.ctl[1] = tok;
        a.ctl[9] = slot + 1;
        *a.arrive = 0u;
    }
}

// Q8_0 draft-head rows from bf16 rows of the main head (quant_bf16_to_q8_kernel,
// src/wzy_kernels_v2.cuh:393-407): fp16 scale = half(amax/127), q = rint(v / scale).
__global__ void __launch_bounds__(256) mtp_head_q8_kernel(const uint16_t* __restrict__ main_head,
                                                          const int* __restrict__ dvocab, int D, size_t n_blocks,
                                                          int8_t* __restrict__ codes, uint16_t* __restrict__ scales) {
    const size_t blk = (size_t) blockIdx.x * 8 + (threadIdx.x >> 5);
    const int lane = threadIdx.x & 31;
    const bool ok = blk < n_blocks;
    const size_t row = ok ? blk / (D / 32) : 0, b = ok ? blk % (D / 32) : 0;
    const float v = ok ? bf16_to_f(main_head[(size_t) dvocab[row] * D + 32 * b + lane]) : 0.f;
    const float amax = max32(fabsf(v));
    const uint16_t sh = f_to_h16(amax / 127.0f);
    const float d = h16_to_f(sh);
    if (ok) {
        codes[blk * 32 + lane] = (int8_t) (d > 0.f ? max(-127, min(127, rn_int(v / d))) : 0);
        if (lane == 0) scales[blk] = sh;
    }
}

// Draft-head rows copied from a Q8_0 main head (MtpEngine::init, src/wzy_mtp.cuh:543-556): one
// 32-block per 32 lanes, codes and scale as they are.
__global__ void __launch_bounds__(256) mtp_head_rows_kernel(const int8_t* __restrict__ main_q,
                                                            const uint16_t* __restrict__ main_s,
                                                            const int* __restrict__ dvocab, int D, size_t n_blocks,
                                                            int8_t* __restrict__ codes, uint16_t* __restrict__ scales) {
    const size_t blk = (size_t) blockIdx.x * 8 + (threadIdx.x >> 5);
    const int lane = threadIdx.x & 31;
    if (blk >= n_blocks) return;
    const size_t row = blk / (D / 32), b = blk % (D / 32);
    const size_t src = (size_t) dvocab[row] * (D / 32) + b;
    codes[blk * 32 + lane] = main_q[src * 32 + lane];
    if (lane == 0) scales[blk] = main_s[src];
}

}  // namespace

// ---------------------------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------------------------
namespace wzy {

MtpState::~MtpState() {
    if (step_exec) (void) hipGraphExecDestroy(step_exec);
    for (void* p : allocs) (void) hipFree(p);
    if (h_ctl) (void) hipHostFree(h_ctl);
    if (h_tok) (void) hipHostFree(h_tok);
    if (h_prob) (void) hipHostFree(h_prob);
    for (auto& e : ctl_ev)
        if (e) (void) hipEventDestroy(e);
}

int MtpState::alloc(void** p, size_t bytes, bool zero) {
    *p = nullptr;
    if (bytes == 0) bytes = 16;
    if (hipMalloc(p, bytes) != hipSuccess) {
        (void) hipGetLastError();
        *p = nullptr;
        set_error("mtp: hipMalloc(%zu) failed", bytes);
        return WZY_ENOMEM;
    }
    allocs.push_back(*p);
    dev_bytes += bytes;
    if (zero) WZY_HIP_TRY(hipMemset(*p, 0, bytes));
    return WZY_OK;
}

int MtpState::alloc_q8(MtpQ8& m, int rows, int cols, const char* name) {
    m.rows = rows;
    m.cols = cols;
    WZY_TRY(alloc_t(&m.q, (size_t) rows * cols, false));
    WZY_TRY(alloc_t(&m.s, (size_t) rows * cols / 32, false));
    std::string n(name);
    reg((n + ".q").c_str(), m.q, (size_t) rows * cols);
    reg((n + ".s").c_str(), m.s, (size_t) rows * cols / 32 * 2);
    return WZY_OK;
}

int MtpState::init(const MtpDims& d, hipStream_t stream, const MtpMain& m, const float* cos_t, const float* sin_t) {
    c = d;
    st = stream;
    main = m;
    WZY_REQUIRE((m.emb != nullptr) != (m.emb_q != nullptr && m.emb_s != nullptr) &&
                    (m.head != nullptr) != (m.head_q != nullptr && m.head_s != nullptr),
                "mtp: one bf16 or one Q8_0 main embedding table and LM head required");
    cos_tab = cos_t;
    sin_tab = sin_t;
    WZY_REQUIRE(c.D % 256 == 0 && c.D >= 256 && c.D <= 8192, "mtp: n_embd must be a multiple of 256 <= 8192");
    WZY_REQUIRE(c.F % 64 == 0 && c.F >= 64 && c.F <= 4096 && (c.K + 1) * c.F <= 65536,
                "mtp: n_ff must be a multiple of 64 <= 4096");
    WZY_REQUIRE(c.K >= 1 && c.K <= 32 && c.K <= c.E && c.E <= 1024, "mtp: bad expert counts");
    WZY_REQUIRE(c.n_dv >= 1 && c.n_dv <= c.n_vocab, "mtp: n_dvocab must be in [1, n_vocab]");
    const int HCD = c.HC * c.D, QD = c.qh * c.hd, KVD = c.kvh * c.hd, W = WZY_MAX_W;
    qd.qh = c.qh; qd.kvh = c.kvh; qd.hd = c.hd; qd.n_rot = c.n_rot;
    qd.ih = 0; qd.idim = 128; qd.iblk = 4; qd.topk = MTP_RING;
    qd.ctx_max = c.ctx_max; qd.ring_cap = MTP_RING; qd.sinks = 0; qd.eps = c.eps; qd.window = MTP_RING;
    WZY_TRY(qsa_check_dims(qd));

    WZY_TRY(alloc_t(&pre_norm_emb, c.D, false)); reg("mtp.pre_norm_emb", pre_norm_emb, (size_t) c.D * 4);
    WZY_TRY(alloc_t(&pre_norm_hid, HCD, false)); reg("mtp.pre_norm_hid", pre_norm_hid, (size_t) HCD * 4);
    WZY_TRY(alloc_q8(fc_emb, c.D, c.D, "mtp.fc_emb"));
    WZY_TRY(alloc_q8(fc_hid, c.D, c.D, "mtp.fc_hid"));
    char nm[48];
    for (int h = 0; h < 3; ++h) {
        snprintf(nm, sizeof nm, "mtp.hc_norm%d", h);
        WZY_TRY(alloc_t(&hc_norm[h], HCD, false)); reg(nm, hc_norm[h], (size_t) HCD * 4);
        snprintf(nm, sizeof nm, "mtp.hc_down%d", h);
        WZY_TRY(alloc_q8(hc_down[h], c.HCLR, HCD, nm));
        snprintf(nm, sizeof nm, "mtp.hc_up%d", h);
        WZY_TRY(alloc_q8(hc_up[h], HCD, c.HCLR, nm));
        if (h < 2) {
            snprintf(nm, sizeof nm, "mtp.hc_inj%d", h);
            WZY_TRY(alloc_t(&hc_inj[h], (size_t) c.HC * HCD, false)); reg(nm, hc_inj[h], (size_t) c.HC * HCD * 2);
        }
    }
    WZY_TRY(alloc_q8(wq, 2 * QD, c.D, "mtp.wq"));
    WZY_TRY(alloc_q8(wk, KVD, c.D, "mtp.wk"));
    WZY_TRY(alloc_q8(wv, KVD, c.D, "mtp.wv"));
    WZY_TRY(alloc_q8(wo, c.D, QD, "mtp.wo"));
    WZY_TRY(alloc_t(&q_norm, c.hd, false)); reg("mtp.q_norm", q_norm, (size_t) c.hd * 4);
    WZY_TRY(alloc_t(&k_norm, c.hd, false)); reg("mtp.k_norm", k_norm, (size_t) c.hd * 4);
    WZY_TRY(alloc_t(&router, (size_t) c.E * c.D, false)); reg("mtp.router", router, (size_t) c.E * c.D * 2);
    WZY_TRY(alloc_t(&sgate, c.D, false)); reg("mtp.sgate", sgate, (size_t) c.D * 2);
    WZY_TRY(alloc_q8(sh_gate, c.F, c.D, "mtp.sh_gate"));
    WZY_TRY(alloc_q8(sh_up, c.F, c.D, "mtp.sh_up"));
    WZY_TRY(alloc_q8(sh_down, c.D, c.F, "mtp.sh_down"));
    q2_rec = wzy_q2_expert_bytes(c.D, c.F);
    WZY_TRY(alloc_t(&experts, q2_rec * c.E, false)); reg("mtp.experts", experts, q2_rec * c.E);
    WZY_TRY(alloc_q8(head, c.n_dv, c.D, "mtp.head"));
    WZY_TRY(alloc_t(&dvocab, c.n_dv, false)); reg("mtp.dvocab", dvocab, (size_t) c.n_dv * 4);

    WZY_TRY(alloc_t(&kv.kq, (size_t) MTP_RING * KVD)); reg("mtp.kv_k", kv.kq, (size_t) MTP_RING * KVD);
    WZY_TRY(alloc_t(&kv.ks, (size_t) MTP_RING * (KVD / 64))); reg("mtp.kv_ks", kv.ks, (size_t) MTP_RING * (KVD / 64) * 2);
    WZY_TRY(alloc_t(&kv.vq, (size_t) MTP_RING * KVD)); reg("mtp.kv_v", kv.vq, (size_t) MTP_RING * KVD);
    WZY_TRY(alloc_t(&kv.vs, (size_t) MTP_RING * (KVD / 64))); reg("mtp.kv_vs", kv.vs, (size_t) MTP_RING * (KVD / 64) * 2);
    WZY_TRY(alloc_t(&d_floor, 1)); reg("mtp.kv_floor", d_floor, sizeof(int));
    WZY_TRY(alloc_t(&d_ctl, MTP_CTL_INTS));

    WZY_TRY(alloc_t(&rin, (size_t) W * HCD)); reg("mtp.act.rin", rin, (size_t) W * HCD * 4);
    WZY_TRY(alloc_t(&en, (size_t) W * c.D));
    WZY_TRY(alloc_t(&e2, (size_t) W * c.D));
    WZY_TRY(alloc_t(&hn, (size_t) W * HCD));
    WZY_TRY(alloc_t(&h2, (size_t) W * HCD));
    WZY_TRY(alloc_t(&unit_gate, (size_t) W * c.HC));           // zeros: 2*sigmoid(0) == 1
    WZY_TRY(alloc_t(&rc, (size_t) W * HCD)); reg("mtp.act.R", rc, (size_t) W * HCD * 4);
    WZY_TRY(alloc_t(&r2, HCD)); reg("mtp.act.R2", r2, (size_t) HCD * 4);
    WZY_TRY(alloc_t(&mixed, (size_t) W * c.D)); reg("mtp.act.mixed", mixed, (size_t) W * c.D * 4);
    WZY_TRY(alloc_t(&inj, (size_t) W * c.HC)); reg("mtp.act.inj", inj, (size_t) W * c.HC * 4);
    WZY_TRY(alloc_t(&inj2, c.HC)); reg("mtp.act.inj2", inj2, (size_t) c.HC * 4);
    WZY_TRY(alloc_t(&mixed2, c.D)); reg("mtp.act.mixed2", mixed2, (size_t) c.D * 4);
    WZY_TRY(alloc_t(&nsc, (size_t) W * c.HC));
    WZY_TRY(alloc_t(&lo, (size_t) W * c.HCLR));
    {
        void* hw = nullptr;
        WZY_TRY(alloc(&hw, hc_workspace_bytes(c.HC, c.HCLR, W)));
        hc_carve_workspace(hw, c.HC, c.HCLR, W, &lo_part, &inj_part);
    }
    WZY_TRY(alloc_t(&qg, (size_t) 2 * QD)); reg("mtp.act.qg", qg, (size_t) 2 * QD * 4);
    WZY_TRY(alloc_t(&kk, (size_t) W * KVD)); reg("mtp.act.k", kk, (size_t) W * KVD * 4);
    WZY_TRY(alloc_t(&vv, (size_t) W * KVD)); reg("mtp.act.v", vv, (size_t) W * KVD * 4);
    const size_t pf = qsa_attn_part_floats(qd, 1);
    WZY_TRY(alloc_t(&att_part, pf));
    WZY_TRY(alloc_t(&att_ml, pf / c.hd * 2));
    WZY_TRY(alloc_t(&att, QD)); reg("mtp.act.att", att, (size_t) QD * 4);
    WZY_TRY(alloc_t(&bo, c.D)); reg("mtp.act.bo", bo, (size_t) c.D * 4);
    WZY_TRY(alloc_t(&rlog, c.E)); reg("mtp.act.router_logits", rlog, (size_t) c.E * 4);
    WZY_TRY(alloc_t(&sg, 1)); reg("mtp.act.sg", sg, 4);
    WZY_TRY(alloc_t(&ids, c.K)); reg("mtp.act.ids", ids, (size_t) c.K * 4);
    WZY_TRY(alloc_t(&wts, c.K)); reg("mtp.act.wts", wts, (size_t) c.K * 4);
    WZY_TRY(alloc_t(&aq, (size_t) (c.K + 1) * c.F)); reg("mtp.act.aq", aq, (size_t) (c.K + 1) * c.F);
    WZY_TRY(alloc_t(&as, (size_t) (c.K + 1) * c.F / 32)); reg("mtp.act.as", as, (size_t) (c.K + 1) * c.F / 32 * 4);
    WZY_TRY(alloc_t(&comb, c.D)); reg("mtp.act.comb", comb, (size_t) c.D * 4);
    WZY_TRY(alloc_t(&sample, c.D)); reg("mtp.act.sample", sample, (size_t) c.D * 4);
    WZY_TRY(alloc_t(&logits, (size_t) c.n_dv + 4)); reg("mtp.act.logits", logits, (size_t) c.n_dv * 4);
    WZY_TRY(alloc_t(&red, (size_t) 3 * MTP_RED_WGS));
    WZY_TRY(alloc_t(&arrive, 1));

    WZY_HIP_TRY(hipHostMalloc((void**) &h_ctl, MTP_CTL_SLOTS * MTP_CTL_INTS * sizeof(int), hipHostMallocDefault));
    memset(h_ctl, 0, MTP_CTL_SLOTS * MTP_CTL_INTS * sizeof(int));
    for (auto& e : ctl_ev) WZY_HIP_TRY(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    WZY_HIP_TRY(hipHostMalloc((void**) &h_tok, MTP_MAX_CHAIN * sizeof(int), hipHostMallocMapped));
    WZY_HIP_TRY(hipHostMalloc((void**) &h_prob, MTP_MAX_CHAIN * sizeof(float), hipHostMallocMapped));
    WZY_HIP_TRY(hipHostGetDevicePointer((void**) &d_tok, h_tok, 0));
    WZY_HIP_TRY(hipHostGetDevicePointer((void**) &d_prob, h_prob, 0));
    memset(h_tok, 0, MTP_MAX_CHAIN * sizeof(int));
    memset(h_prob, 0, MTP_MAX_CHAIN * sizeof(float));
    return WZY_OK;
}

namespace {
// Synthetic-model tensor ids of the drafter (stream sub-ids of WZY_S_DENSE, layer MTP_LAYER)
enum MtpTensorId {
    MI_PRE_EMB = 0, MI_PRE_HID = 1, MI_FC_EMB = 2, MI_FC_HID = 3,
    MI_HC = 10,                       // + 4*h + {0 norm, 1 down, 2 up, 3 inject}
    MI_WQ = 30, MI_WK = 31, MI_WV = 32, MI_WO = 33, MI_QNORM = 34, MI_KNORM = 35,
    MI_ROUTER = 40, MI_SGATE = 41, MI_SH_GATE = 42, MI_SH_UP = 43, MI_SH_DOWN = 44,
};
constexpr uint32_t MTP_LAYER = 0xFFFE;

struct MtpGen {
    uint64_t seed;
    std::vector<char> buf;
    uint64_t stream(uint32_t id) { return wzy_synth_stream(5u /* WZY_S_DENSE */, MTP_LAYER, id); }
    int normal_f32(float* dst, size_t n, uint32_t id, float mean, float sd) {
        buf.resize(n * 4);
        wzy_synth_normal(seed, stream(id), n, mean, sd, (float*) buf.data());
        WZY_HIP_TRY(hipMemcpy(dst, buf.data(), n * 4, hipMemcpyHostToDevice));
        return WZY_OK;
    }
    int normal_bf16(uint16_t* dst, size_t n, uint32_t id, float sd) {
        buf.resize(n * 2);
        wzy_synth_normal_bf16(seed, stream(id), n, 0.f, sd, (uint16_t*) buf.data());
        WZY_HIP_TRY(hipMemcpy(dst, buf.data(), n * 2, hipMemcpyHostToDevice));
        return WZY_OK;
    }
    int q8(const MtpQ8& m, uint32_t id) {
        const size_t n = (size_t) m.rows * m.cols;
        buf.resize(n + n / 32 * 2);
        wzy_synth_q8(seed, stream(id), m.rows, m.cols, (float) (1.0 / sqrt((double) m.cols)), (int8_t*) buf.data(),
                     (uint16_t*) (buf.data() + n));
        WZY_HIP_TRY(hipMemcpy(m.q, buf.data(), n, hipMemcpyHostToDevice));
        WZY_HIP_TRY(hipMemcpy(m.s, buf.data() + n, n / 32 * 2, hipMemcpyHostToDevice));
        return WZY_OK;
    }
};
}  // namespace

int MtpState::build_head(const int* ids) {
    for (int i = 0; i < c.n_dv; ++i)
        WZY_REQUIRE(ids[i] >= 0 && ids[i] < c.n_vocab, "mtp: draft vocabulary id %d at row %d out of range", ids[i], i);
    WZY_HIP_TRY(hipMemcpy(dvocab, ids, (size_t) c.n_dv * 4, hipMemcpyHostToDevice));
    const size_t nb = (size_t) c.n_dv * (c.D / 32);
    if (main.head_q)
        hipLaunchKernelGGL(mtp_head_rows_kernel, dim3((unsigned) ((nb + 7) / 8)), dim3(256), 0, st, main.head_q,
                           main.head_s, dvocab, c.D, nb, head.q, head.s);
    else
        hipLaunchKernelGGL(mtp_head_q8_kernel, dim3((unsigned) ((nb + 7) / 8)), dim3(256), 0, st, main.head, dvocab,
                           c.D, nb, head.q, head.s);
    WZY_LAUNCH_CHECK();
    WZY_HIP_TRY(hipStreamSynchronize(st));
    return WZY_OK;
}

int MtpState::load_synthetic(uint64_t seed) {
    const int HCD = c.HC * c.D;
    MtpGen g{seed, {}};
    WZY_TRY(g.normal_f32(pre_norm_emb, c.D, MI_PRE_EMB, 1.0f, 0.02f));
    WZY_TRY(g.normal_f32(pre_norm_hid, HCD, MI_PRE_HID, 1.0f, 0.02f));
    WZY_TRY(g.q8(fc_emb, MI_FC_EMB));
    WZY_TRY(g.q8(fc_hid, MI_FC_HID));
    for (int h = 0; h < 3; ++h) {
        WZY_TRY(g.normal_f32(hc_norm[h], HCD, MI_HC + 4 * h, 1.0f, 0.02f));
        WZY_TRY(g.q8(hc_down[h], MI_HC + 4 * h + 1));
        WZY_TRY(g.q8(hc_up[h], MI_HC + 4 * h + 2));
        if (h < 2)
            WZY_TRY(g.normal_bf16(hc_inj[h], (size_t) c.HC * HCD, MI_HC + 4 * h + 3, (float) (1.0 / sqrt((double) HCD))));
    }
    WZY_TRY(g.q8(wq, MI_WQ));
    WZY_TRY(g.q8(wk, MI_WK));
    WZY_TRY(g.q8(wv, MI_WV));
    WZY_TRY(g.q8(wo, MI_WO));
    WZY_TRY(g.normal_f32(q_norm, c.hd, MI_QNORM, 1.0f, 0.02f));
    WZY_TRY(g.normal_f32(k_norm, c.hd, MI_KNORM, 1.0f, 0.02f));
    WZY_TRY(g.normal_bf16(router, (size_t) c.E * c.D, MI_ROUTER, 0.02f));
    WZY_TRY(g.normal_bf16(sgate, c.D, MI_SGATE, 0.02f));
    WZY_TRY(g.q8(sh_gate, MI_SH_GATE));
    WZY_TRY(g.q8(sh_up, MI_SH_UP));
    WZY_TRY(g.q8(sh_down, MI_SH_DOWN));
    for (int e0 = 0; e0 < c.E; e0 += 1024)
        WZY_TRY(wzy_synth_q2_experts_device(seed, e0, std::min(1024, c.E - e0), c.D, c.F, experts + (size_t) e0 * q2_rec,
                                            st));
    // draft vocabulary: n_dv ids spread evenly over the main vocabulary (identity when n_dv == n_vocab)
    std::vector<int> dv(c.n_dv);
    for (int i = 0; i < c.n_dv; ++i) dv[i] = (int) ((int64_t) i * c.n_vocab / c.n_dv);
    WZY_TRY(build_head(dv.data()));
    WZY_TRY(reset_kv());
    WZY_HIP_TRY(hipStreamSynchronize(st));
    loaded = true;
    return WZY_OK;
}

int MtpState::reset_kv() {
    const int KVD = c.kvh * c.hd;
    WZY_HIP_TRY(hipMemsetAsync(kv.kq, 0, (size_t) MTP_RING * KVD, st));
    WZY_HIP_TRY(hipMemsetAsync(kv.vq, 0, (size_t) MTP_RING * KVD, st));
    WZY_HIP_TRY(hipMemsetAsync(kv.ks, 0, (size_t) MTP_RING * (KVD / 64) * 2, st));
    WZY_HIP_TRY(hipMemsetAsync(kv.vs, 0, (size_t) MTP_RING * (KVD / 64) * 2, st));
    WZY_HIP_TRY(hipMemsetAsync(d_floor, 0, 4, st));
    return WZY_OK;
}

int MtpState::set_floor(int floor) {
    WZY_REQUIRE(floor >= 0, "mtp: negative kv floor");
    // through a control slot: the pinned source must outlive the asynchronous copy
    const int s = ctl_slot;
    ctl_slot = (s + 1) % MTP_CTL_SLOTS;
    if (ctl_pending[s]) WZY_HIP_TRY(hipEventSynchronize(ctl_ev[s]));
    int* h = h_ctl + (size_t) s * MTP_CTL_INTS;
    h[0] = floor;
    WZY_HIP_TRY(hipMemcpyAsync(d_floor, h, sizeof(int), hipMemcpyHostToDevice, st));
    WZY_HIP_TRY(hipEventRecord(ctl_ev[s], st));
    ctl_pending[s] = true;
    return WZY_OK;
}

int MtpState::set_ctl(int cell0, const int* toks, int n) {
    WZY_REQUIRE(n >= 1 && n <= WZY_MAX_W && toks, "mtp: bad control rows");
    const int s = ctl_slot;
    ctl_slot = (s + 1) % MTP_CTL_SLOTS;
    if (ctl_pending[s]) WZY_HIP_TRY(hipEventSynchronize(ctl_ev[s]));
    int* h = h_ctl + (size_t) s * MTP_CTL_INTS;
    memset(h, 0, MTP_CTL_INTS * sizeof(int));
    h[0] = cell0;
    for (int t = 0; t < n; ++t) h[1 + t] = toks[t];
    h[9] = 0;
    WZY_HIP_TRY(hipMemcpyAsync(d_ctl, h, MTP_CTL_INTS * sizeof(int), hipMemcpyHostToDevice, st));
    WZY_HIP_TRY(hipEventRecord(ctl_ev[s], st));
    ctl_pending[s] = true;
    return WZY_OK;
}

namespace {
int hc_read(const MtpState& m, int h, const float* R_in, const float* bo, const float* inj_prev, float* R_out,
            float* inj_out, float* mixed_out, int T) {
    HcPreArgs a{};
    a.R_in = R_in;
    a.bo = bo;
    a.inj_prev = inj_prev;
    a.R_out = R_out;
    a.norm_w = m.hc_norm[h];
    a.down_q = m.hc_down[h].q;
    a.down_s = m.hc_down[h].s;
    a.inj_w = h < 2 ? m.hc_inj[h] : nullptr;
    a.nsc = m.nsc;
    a.lo_part = m.lo_part;
    a.inj_part = m.inj_part;
    a.D = m.c.D; a.HC = m.c.HC; a.HCLR = m.c.HCLR; a.eps = m.c.eps;
    WZY_TRY(launch_hc_pre(a, T, m.st));
    HcPostArgs b{};
    b.R = R_out; b.nsc = m.nsc; b.norm_w = m.hc_norm[h]; b.up_q = m.hc_up[h].q; b.up_s = m.hc_up[h].s;
    b.lo_part = m.lo_part; b.inj_part = inj_out ? m.inj_part : nullptr; b.lo = m.lo; b.inj = inj_out;
    b.mixed = mixed_out;
    b.D = m.c.D; b.HC = m.c.HC; b.HCLR = m.c.HCLR;
    return launch_hc_post(b, T, m.st);
}
}  // namespace

int MtpState::enqueue_front(int T, bool with_q) {
    WZY_REQUIRE(T >= 1 && T <= WZY_MAX_W && (!with_q || T == 1), "mtp: bad front rows");
    const int D = c.D, HCD = c.HC * D, QD = c.qh * c.hd, KVD = c.kvh * c.hd;
    MtpInArgs ia{main.emb, main.emb_q, main.emb_s, c.n_vocab, d_ctl + 1, rin, pre_norm_emb, pre_norm_hid, en, hn, D,
                 c.HC, c.eps};
    if (D <= 2048) hipLaunchKernelGGL(mtp_in_kernel<8>, dim3(1 + c.HC, T), dim3(256), 0, st, ia);
    else if (D <= 4096) hipLaunchKernelGGL(mtp_in_kernel<16>, dim3(1 + c.HC, T), dim3(256), 0, st, ia);
    else hipLaunchKernelGGL(mtp_in_kernel<32>, dim3(1 + c.HC, T), dim3(256), 0, st, ia);
    WZY_LAUNCH_CHECK();
    {
        GemvSegs s;
        s.n = 1;
        s.seg[0] = GemvSeg{fc_emb.q, fc_emb.s, e2, D, GEMV_Q8, D, 0};
        WZY_TRY(launch_gemv_segs(s, en, D, T, st));
    }
    for (int r0 = 0; r0 < T * c.HC; r0 += WZY_MAX_W) {
        const int n = std::min(WZY_MAX_W, T * c.HC - r0);
        GemvSegs s;
        s.n = 1;
        s.seg[0] = GemvSeg{fc_hid.q, fc_hid.s, h2 + (size_t) r0 * D, D, GEMV_Q8, D, 0};
        WZY_TRY(launch_gemv_segs(s, hn + (size_t) r0 * D, D, n, st));
    }
    // R = fc_hidden(streams) + fc_embedding(token), folded into the attention read
    WZY_TRY(hc_read(*this, 0, h2, e2, unit_gate, rc, inj, mixed, T));
    {
        GemvSegs s;
        s.n = 0;
        if (with_q) s.seg[s.n++] = GemvSeg{wq.q, wq.s, qg, 2 * QD, GEMV_Q8, 2 * QD, 0};
        s.seg[s.n++] = GemvSeg{wk.q, wk.s, kk, KVD, GEMV_Q8, KVD, 0};
        s.seg[s.n++] = GemvSeg{wv.q, wv.s, vv, KVD, GEMV_Q8, KVD, 0};
        WZY_TRY(launch_gemv_segs(s, mixed, D, T, st));
    }
    QsaPrepArgs p{};
    p.dm = qd; p.pos = d_ctl; p.qg = with_q ? qg : nullptr; p.kk = kk; p.vv = vv;
    p.q_norm = q_norm; p.k_norm = k_norm; p.cos_tab = cos_tab; p.sin_tab = sin_tab; p.kv = kv;
    WZY_TRY(launch_qsa_prep(p, T, st));
    (void) HCD;
    return WZY_OK;
}

int MtpState::enqueue_rest() {
    const int D = c.D, QD = c.qh * c.hd;
    QsaAttnArgs at{};
    at.dm = qd; at.pos = d_ctl; at.qg = qg; at.kv = kv; at.sel_ids = nullptr; at.floor = d_floor;
    at.part = att_part; at.part_ml = att_ml; at.out = att;
    WZY_TRY(launch_qsa_attn(at, 1, st));
    {
        GemvSegs s;
        s.n = 1;
        s.seg[0] = GemvSeg{wo.q, wo.s, bo, D, GEMV_Q8, D, 0};
        WZY_TRY(launch_gemv_segs(s, att, QD, 1, st));
    }
    WZY_TRY(hc_read(*this, 1, rc, bo, inj, r2, inj2, mixed2, 1));
    {
        GemvSegs s;
        s.n = 2;
        s.seg[0] = GemvSeg{router, nullptr, rlog, c.E, GEMV_BF16, c.E, 0};
        s.seg[1] = GemvSeg{sgate, nullptr, sg, 1, GEMV_BF16, 1, 0};
        WZY_TRY(launch_gemv_segs(s, mixed2, D, 1, st));
    }
    WZY_TRY(wzy_moe_route(rlog, c.E, c.K, 1, ids, wts, (void*) st));
    {
        Q2GuArgs g{};
        g.experts = experts; g.rec = q2_rec; g.ids = ids; g.D = D; g.F = c.F; g.K = c.K; g.x = mixed2;
        g.shg_q = sh_gate.q; g.shg_s = sh_gate.s; g.shu_q = sh_up.q; g.shu_s = sh_up.s; g.aq = aq; g.as = as;
        const size_t lds = (size_t) 2 * D + (size_t) (D / 32) * 8;
        const int npl = (2 * (D / 64) + 63) / 64;
        const dim3 grid(c.K + 1, c.F / 32);
        if (npl <= 1) hipLaunchKernelGGL(mtp_q2_gate_up_kernel<1>, grid, dim3(512), lds, st, g);
        else if (npl <= 2) hipLaunchKernelGGL(mtp_q2_gate_up_kernel<2>, grid, dim3(512), lds, st, g);
        else hipLaunchKernelGGL(mtp_q2_gate_up_kernel<4>, grid, dim3(512), lds, st, g);
        WZY_LAUNCH_CHECK();
    }
    {
        Q2DnArgs d{};
        d.experts = experts; d.rec = q2_rec; d.ids = ids; d.wts = wts; d.sg = sg; d.D = D; d.F = c.F; d.K = c.K;
        d.aq = aq; d.as = as; d.shd_q = sh_down.q; d.shd_s = sh_down.s; d.comb = comb;
        const int P = c.F / 64, C = c.F / 32;
        const size_t lds = (size_t) c.K * c.F + c.F + (size_t) (c.K + 1) * C * 4 + (size_t) c.K * C * 4 +
                           (size_t) DN_RT * (c.K * P + C) * 4 + (size_t) DN_RT * (c.K + 1) * 4;
        hipLaunchKernelGGL(mtp_q2_down_kernel, dim3(D / DN_RT), dim3(256), lds, st, d);
        WZY_LAUNCH_CHECK();
    }
    // final mixer: folds the MoE write; the residual it writes is the next chained step's input
    WZY_TRY(hc_read(*this, 2, r2, comb, inj2, rin, nullptr, sample, 1));
    {
        GemvSegs s;
        s.n = 1;
        s.seg[0] = GemvSeg{head.q, head.s, logits, c.n_dv, GEMV_Q8, c.n_dv, 0};
        WZY_TRY(launch_gemv_segs(s, sample, D, 1, st));
    }
    HeadRedArgs h{logits, c.n_dv, dvocab, red, arrive, d_ctl, d_tok, d_prob};
    hipLaunchKernelGGL(mtp_head_reduce_kernel, dim3(MTP_RED_WGS), dim3(256), 0, st, h);
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

int MtpState::enqueue_steps(int depth) {
    WZY_REQUIRE(depth >= 1 && depth <= MTP_MAX_CHAIN, "mtp: chain depth must be in [1, %d]", MTP_MAX_CHAIN);
    if (!graphs) {
        for (int j = 0; j < depth; ++j) {
            WZY_TRY(enqueue_front(1, true));
            WZY_TRY(enqueue_rest());
        }
        return WZY_OK;
    }
    if (!step_exec) {
        WZY_HIP_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        int rc = enqueue_front(1, true);
        if (rc == WZY_OK) rc = enqueue_rest();
        hipGraph_t g = nullptr;
        const hipError_t e = hipStreamEndCapture(st, &g);
        if (rc != WZY_OK) {
            if (g) (void) hipGraphDestroy(g);
            return rc;
        }
        if (e != hipSuccess) {
            set_error("mtp: graph capture failed: %s", hipGetErrorString(e));
            return WZY_EHIP;
        }
        const hipError_t ie = hipGraphInstantiate(&step_exec, g, nullptr, nullptr, 0);
        (void) hipGraphDestroy(g);
        if (ie != hipSuccess) {
            step_exec = nullptr;
            set_error("mtp: graph instantiate failed: %s", hipGetErrorString(ie));
            return WZY_EHIP;
        }
    }
    for (int j = 0; j < depth; ++j) WZY_HIP_TRY(hipGraphLaunch(step_exec, st));
    return WZY_OK;
}

}  // namespace wzy

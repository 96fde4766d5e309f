// hc.hip -- 4-stream hyper-connection (HC) read for gfx950.
//
// The reference reads the residual streams with four kernels (norm+fold, down+inject, quantise,
// up+mean) and writes them with a fifth (src/wzy_stage_v2.cuh:463-470, src/wzy_kernels_v2.cuh:
// 409-454,632-827).  Here a read is two launches and the pending write is folded into the next read:
//
//   hc_pre : R_out = R_in + bo * 2*sigmoid(inj_prev/HC)           (the pending write, or the
//            embedding broadcast on layer 0), per-stream RMS scale, xn = R_out*scale*w,
//            lo = silu(down . quant32(xn) / HC), inj = inj_w . xn.
//            Every workgroup first issues the loads of its own `down` rows (they do not depend on
//            the activations), then rebuilds quant32(xn) for the whole window in LDS from L2
//            (coalesced float4 reads, 32 KB per row), so no cross-workgroup synchronisation is
//            needed; workgroup w writes every gridDim-th 32-block of R_out.
//   hc_post: mixed[d] = 0.25 * sum_c xn[c][d] * sigmoid(up[c*D+d] . quant32(lo)); lo is quantised
//            once per workgroup into LDS.
#include <algorithm>

#include "wzy_device.h"
#include "wzy_hc.h"
#include "wzy_host.h"

using namespace wzy;

namespace {

constexpr int HC4 = 4;           // stream count of the hyper-connection

// Per-32 int8 quantisation (reference per-32 rule: d = amax/127, q = rint(x * 127/amax)).
WZY_DEV void quant32_vals(const float (&v)[32], int4& q0, int4& q1, float& d) {
    float am = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) am = fmaxf(am, fabsf(v[i]));
    d = am / 127.0f;
    const float inv = d > 0.f ? 127.0f / am : 0.f;
    int w[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        uint32_t pk = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int q = max(-127, min(127, rn_int(v[4 * k + j] * inv)));
            pk |= (uint32_t) (q & 0xFF) << (8 * j);
        }
        w[k] = (int) pk;
    }
    q0 = make_int4(w[0], w[1], w[2], w[3]);
    q1 = make_int4(w[4], w[5], w[6], w[7]);
}

// Four residual values of row t, stream c, positions d..d+3 before the norm: R_in (+ fold) or the
// embedding row broadcast to every stream.
WZY_DEV float4 hc_in4(const HcPreArgs& a, int t, int c, int d, float gw) {
    float4 v;
    if (a.emb_rows) {
        v = *(const float4*) (a.emb_rows + (size_t) t * a.D + d);
    } else if (a.emb_table) {
        int tok = a.toks[t];
        tok = tok < 0 ? 0 : (tok >= a.n_vocab ? a.n_vocab - 1 : tok);
        const uint2 h = *(const uint2*) (a.emb_table + (size_t) tok * a.D + d);
        v = make_float4(bf16_lo(h.x), bf16_hi(h.x), bf16_lo(h.y), bf16_hi(h.y));
    } else {
        v = *(const float4*) (a.R_in + ((size_t) t * HC4 + c) * a.D + d);
    }
    if (a.bo) {
        const float4 b = *(const float4*) (a.bo + (size_t) t * a.D + d);
        v.x = fmaf(b.x, gw, v.x);
        v.y = fmaf(b.y, gw, v.y);
        v.z = fmaf(b.z, gw, v.z);
        v.w = fmaf(b.w, gw, v.w);
    }
    return v;
}

}  // namespace

// T window rows (<= 4 per launch), D <= DC.  256 threads; wave w of workgroup g owns down rows
// (4g + w) * RPW .. + RPW - 1.  Dynamic LDS: int8 xq [T][4D] then fp32 xs [T][4D/32].
template <int T, int DC, int RPW>
__global__ void __launch_bounds__(256) hc_pre_kernel(HcPreArgs a) {
    constexpr int KMAX = DC / 1024;          // float4s per thread per stream in the norm pass
    constexpr int NBL = DC * HC4 / 32 / 64;  // 32-blocks per lane of one down row
    extern __shared__ __align__(16) unsigned char s_dyn[];
    __shared__ float s_red[4][T * HC4];
    __shared__ float s_nsc[T * HC4];
    __shared__ float s_gw[T * HC4];
    __shared__ float s_inj[4];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int D = a.D, HCD = HC4 * D, nb = HCD / 32, D4 = D / 4, L = a.HCLR;
    int8_t* s_xq = (int8_t*) s_dyn;
    float* s_xs = (float*) (s_dyn + (size_t) T * HCD);

    // 0. this wave's down rows, loaded before anything else
    const int row0 = (blockIdx.x * 4 + w) * RPW;
    int4 c0[NBL][RPW], c1[NBL][RPW];
    float dw[NBL][RPW];
#pragma unroll
    for (int i = 0; i < NBL; ++i) {
        const int b = lane + 64 * i;
#pragma unroll
        for (int s = 0; s < RPW; ++s) {
            const int r = row0 + s;
            if (b < nb && r < L) {
                const int4* cp = (const int4*) (a.down_q + (size_t) r * HCD + (size_t) b * 32);
                c0[i][s] = ld_stream_i4(cp);
                c1[i][s] = ld_stream_i4(cp + 1);
                dw[i][s] = h16_to_f(a.down_s[(size_t) r * nb + b]);
            } else {
                c0[i][s] = c1[i][s] = make_int4(0, 0, 0, 0);
                dw[i][s] = 0.f;
            }
        }
    }

    // 1. fold gates 2*sigmoid(inj_prev/HC)
    if (tid < T * HC4) s_gw[tid] = a.bo ? 2.0f / (1.0f + __expf(-a.inj_prev[tid] / (float) HC4)) : 0.f;
    __syncthreads();

    // 2. per-stream sums of squares
    float ss[T][HC4];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int c = 0; c < HC4; ++c) {
            float acc = 0.f;
#pragma unroll
            for (int k = 0; k < KMAX; ++k) {
                const int j = tid + 256 * k;
                if (j < D4) {
                    const float4 v = hc_in4(a, t, c, 4 * j, s_gw[t * HC4 + c]);
                    acc = fmaf(v.x, v.x, acc);
                    acc = fmaf(v.y, v.y, acc);
                    acc = fmaf(v.z, v.z, acc);
                    acc = fmaf(v.w, v.w, acc);
                }
            }
            ss[t][c] = acc;
        }
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int c = 0; c < HC4; ++c) {
            const float v = wave_sum(ss[t][c]);
            if (lane == 0) s_red[w][t * HC4 + c] = v;
        }
    __syncthreads();
    if (tid < T * HC4) {
        const float tot = s_red[0][tid] + s_red[1][tid] + s_red[2][tid] + s_red[3][tid];
        const float sc = 1.0f / sqrtf(tot / (float) D + a.eps);
        s_nsc[tid] = sc;
        if (blockIdx.x == 0) a.nsc[tid] = sc;
    }
    __syncthreads();

    // 3. xn = R_out * scale * w quantised per 32 into LDS; R_out blocks; inject row blockIdx.x
    const bool do_inj = a.inj_w != nullptr && blockIdx.x < HC4;
    float inj_acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) inj_acc[t] = 0.f;
    for (int b = tid; b < nb; b += 256) {
        const int c = (32 * b) / D, d0 = (32 * b) % D;
        float4 nw[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) nw[k] = *(const float4*) (a.norm_w + (size_t) c * D + d0 + 4 * k);
        float iw[32];
        if (do_inj) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint4 u = *(const uint4*) (a.inj_w + (size_t) blockIdx.x * HCD + (size_t) 32 * b + 8 * k);
                iw[8 * k + 0] = bf16_lo(u.x); iw[8 * k + 1] = bf16_hi(u.x);
                iw[8 * k + 2] = bf16_lo(u.y); iw[8 * k + 3] = bf16_hi(u.y);
                iw[8 * k + 4] = bf16_lo(u.z); iw[8 * k + 5] = bf16_hi(u.z);
                iw[8 * k + 6] = bf16_lo(u.w); iw[8 * k + 7] = bf16_hi(u.w);
            }
        }
        const bool write_r = (b % gridDim.x) == blockIdx.x;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const float gw = s_gw[t * HC4 + c], sc = s_nsc[t * HC4 + c];
            float4 v4[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) v4[k] = hc_in4(a, t, c, d0 + 4 * k, gw);
            if (write_r) {
                float* ro = a.R_out + ((size_t) t * HC4 + c) * D + d0;
#pragma unroll
                for (int k = 0; k < 8; ++k) *(float4*) (ro + 4 * k) = v4[k];
            }
            float xn[32];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                xn[4 * k + 0] = v4[k].x * sc * nw[k].x;
                xn[4 * k + 1] = v4[k].y * sc * nw[k].y;
                xn[4 * k + 2] = v4[k].z * sc * nw[k].z;
                xn[4 * k + 3] = v4[k].w * sc * nw[k].w;
            }
            if (do_inj) {
#pragma unroll
                for (int k = 0; k < 32; ++k) inj_acc[t] = fmaf(iw[k], xn[k], inj_acc[t]);
            }
            int4 q0, q1;
            float xs;
            quant32_vals(xn, q0, q1, xs);
            int4* dst = (int4*) (s_xq + (size_t) t * HCD + (size_t) 32 * b);
            dst[0] = q0;
            dst[1] = q1;
            s_xs[t * nb + b] = xs;
        }
    }
    if (do_inj) {                             // workgroup-uniform branch
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const float s = block_sum<4>(inj_acc[t], s_inj);
            if (tid == 0) a.inj[t * HC4 + blockIdx.x] = s;
        }
    }
    __syncthreads();

    // 4. down rows: lo = silu(down . xq / HC)
    float acc[RPW][T];
#pragma unroll
    for (int s = 0; s < RPW; ++s)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[s][t] = 0.f;
#pragma unroll
    for (int i = 0; i < NBL; ++i) {
        const int b = lane + 64 * i;
        if (b >= nb) continue;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int4* xp = (const int4*) (s_xq + (size_t) t * HCD + (size_t) 32 * b);
            const int4 x0 = xp[0], x1 = xp[1];
            const float xs = s_xs[t * nb + b];
#pragma unroll
            for (int s = 0; s < RPW; ++s)
                acc[s][t] = fmaf(dw[i][s] * xs, (float) (dot16(c0[i][s], x0) + dot16(c1[i][s], x1)), acc[s][t]);
        }
    }
#pragma unroll
    for (int s = 0; s < RPW; ++s) {
        const int r = row0 + s;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const float v = wave_sum(acc[s][t]) / (float) HC4;
            if (lane == 0 && r < L) a.lo[(size_t) t * L + r] = v / (1.0f + __expf(-v));
        }
    }
}

// hc_post: wave handles 2 output positions d; 16 lanes per (d, stream) row of `up`, one 32-block
// per lane (HCLR <= 512).
template <int T>
__global__ void __launch_bounds__(256) hc_post_kernel(HcPostArgs a) {
    __shared__ int4 s_lq[T][32];
    __shared__ float s_ls[T][16];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = (blockIdx.x * blockDim.x + tid) >> 6;
    const int D = a.D, L = a.HCLR, nb = L / 32;
    const int li = lane & 15, c = lane >> 4;

    // weights and the per-position inputs of both outputs first
    int4 c0[2], c1[2];
    float dw[2], xn[2][T];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int d = wave * 2 + k;
        const size_t row = (size_t) c * D + d;
        if (d < D && li < nb) {
            const int4* cp = (const int4*) (a.up_q + row * L + (size_t) li * 32);
            c0[k] = ld_stream_i4(cp);
            c1[k] = ld_stream_i4(cp + 1);
            dw[k] = h16_to_f(a.up_s[row * nb + li]);
        } else {
            c0[k] = c1[k] = make_int4(0, 0, 0, 0);
            dw[k] = 0.f;
        }
#pragma unroll
        for (int t = 0; t < T; ++t)
            xn[k][t] = (d < D && li == 0)
                           ? a.R[((size_t) t * HC4 + c) * D + d] * a.nsc[t * HC4 + c] * a.norm_w[(size_t) c * D + d]
                           : 0.f;
    }
    // quant32(lo) once per workgroup
    if (tid < T * nb) {
        const int t = tid / nb, b = tid % nb;
        float v[32];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float4 f = *(const float4*) (a.lo + (size_t) t * L + 32 * b + 4 * k);
            v[4 * k] = f.x; v[4 * k + 1] = f.y; v[4 * k + 2] = f.z; v[4 * k + 3] = f.w;
        }
        int4 q0, q1;
        float xs;
        quant32_vals(v, q0, q1, xs);
        s_lq[t][2 * b] = q0;
        s_lq[t][2 * b + 1] = q1;
        s_ls[t][b] = xs;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int d = wave * 2 + k;
        if (d >= D) break;                   // wave-uniform
#pragma unroll
        for (int t = 0; t < T; ++t) {
            float acc = 0.f;
            if (li < nb) acc = dw[k] * s_ls[t][li] * (float) (dot16(c0[k], s_lq[t][2 * li]) + dot16(c1[k], s_lq[t][2 * li + 1]));
            const float s = sum16(acc);      // every lane of the 16-lane group holds stream c's sum
            const float g = (li == 0) ? xn[k][t] / (1.0f + __expf(-s)) : 0.f;
            // gather the four streams (lanes 0, 16, 32, 48) in the reference's pairing
            // (g0 + g2) + (g1 + g3)  (src/wzy_kernels_v2.cuh:806-809)
            const float g0 = as_f(__builtin_amdgcn_readlane(as_i(g), 0));
            const float g1 = as_f(__builtin_amdgcn_readlane(as_i(g), 16));
            const float g2 = as_f(__builtin_amdgcn_readlane(as_i(g), 32));
            const float g3 = as_f(__builtin_amdgcn_readlane(as_i(g), 48));
            if (lane == 0) a.mixed[(size_t) t * D + d] = ((g0 + g2) + (g1 + g3)) * 0.25f;
        }
    }
}

namespace wzy {

namespace {
constexpr int PRE_RPW = 2;

template <int T, int DC>
void launch_pre_tdc(const HcPreArgs& a, hipStream_t st) {
    const int HCD = HC4 * a.D;
    const int rows_wg = 4 * PRE_RPW;
    int blocks = (a.HCLR + rows_wg - 1) / rows_wg;
    if (a.inj_w && blocks < HC4) blocks = HC4;
    const size_t lds = (size_t) T * HCD + (size_t) T * (HCD / 32) * sizeof(float);
    hipLaunchKernelGGL((hc_pre_kernel<T, DC, PRE_RPW>), dim3(blocks), dim3(256), lds, st, a);
}
template <int T>
void launch_pre_t(const HcPreArgs& a, hipStream_t st) {
    if (a.D <= 1024) launch_pre_tdc<T, 1024>(a, st);
    else if (a.D <= 2048) launch_pre_tdc<T, 2048>(a, st);
    else launch_pre_tdc<T, 4096>(a, st);
}
}  // namespace

int launch_hc_pre(const HcPreArgs& a0, int T, hipStream_t st) {
    WZY_REQUIRE(T >= 1 && T <= WZY_MAX_W, "hc_pre: T out of range");
    WZY_REQUIRE(a0.HC == HC4 && a0.D % 32 == 0 && a0.D >= 32 && a0.D <= 4096 && a0.HCLR % 32 == 0 && a0.HCLR >= 32 &&
                    a0.HCLR <= 512,
                "hc_pre: unsupported shape (HC must be 4, D a multiple of 32 <= 4096, HCLR a multiple of 32 <= 512)");
    WZY_REQUIRE((a0.R_in != nullptr) + (a0.emb_table != nullptr) + (a0.emb_rows != nullptr) == 1,
                "hc_pre: exactly one of R_in / emb_table / emb_rows");
    WZY_REQUIRE(!a0.emb_table || a0.toks, "hc_pre: embedding mode needs toks");
    WZY_REQUIRE(!a0.bo || a0.inj_prev, "hc_pre: fold needs inj_prev");
    WZY_REQUIRE(a0.R_out && a0.norm_w && a0.down_q && a0.down_s && a0.nsc && a0.lo, "hc_pre: null pointer");
    WZY_REQUIRE(!a0.inj_w || a0.inj, "hc_pre: inject weights need an inj output");
    // rows per launch so that the LDS copy of quant32(xn) stays within 40 KB
    const int HCD = HC4 * a0.D;
    const int tb = std::max(1, std::min(4, (40 * 1024) / (HCD + HCD / 8)));
    for (int t0 = 0; t0 < T; t0 += tb) {
        const int n = std::min(tb, T - t0);
        HcPreArgs a = a0;
        if (a.R_in) a.R_in += (size_t) t0 * HCD;
        if (a.toks) a.toks += t0;
        if (a.emb_rows) a.emb_rows += (size_t) t0 * a.D;
        if (a.bo) a.bo += (size_t) t0 * a.D;
        if (a.inj_prev) a.inj_prev += (size_t) t0 * HC4;
        a.R_out += (size_t) t0 * HCD;
        a.nsc += (size_t) t0 * HC4;
        a.lo += (size_t) t0 * a.HCLR;
        if (a.inj) a.inj += (size_t) t0 * HC4;
        switch (n) {
            case 1: launch_pre_t<1>(a, st); break;
            case 2: launch_pre_t<2>(a, st); break;
            case 3: launch_pre_t<3>(a, st); break;
            default: launch_pre_t<4>(a, st); break;
        }
    }
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

int launch_hc_post(const HcPostArgs& a, int T, hipStream_t st) {
    WZY_REQUIRE(T >= 1 && T <= WZY_MAX_W, "hc_post: T out of range");
    WZY_REQUIRE(a.HC == HC4 && a.HCLR % 32 == 0 && a.HCLR >= 32 && a.HCLR <= 512, "hc_post: unsupported shape");
    WZY_REQUIRE(a.R && a.nsc && a.norm_w && a.up_q && a.up_s && a.lo && a.mixed, "hc_post: null pointer");
    const int waves = (a.D + 1) / 2;
    const int blocks = (waves + 3) / 4;
    switch (T) {
#define C_(TT) case TT: hipLaunchKernelGGL((hc_post_kernel<TT>), dim3(blocks), dim3(256), 0, st, a); break;
        C_(1) C_(2) C_(3) C_(4) C_(5) C_(6) C_(7)
        default: hipLaunchKernelGGL((hc_post_kernel<8>), dim3(blocks), dim3(256), 0, st, a); break;
#undef C_
    }
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

}  // namespace wzy

// ---------------------------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------------------------
extern "C" int wzy_hc_read(const float* R_in, const uint16_t* emb_table, const int* toks, int n_vocab,
                           const float* bo, const float* inj_prev, float* R_out, const float* norm_w,
                           const int8_t* down_q, const uint16_t* down_s, const uint16_t* inj_w,
                           const int8_t* up_q, const uint16_t* up_s, float* nsc, float* lo, float* inj,
                           float* mixed, int D, int HC, int HCLR, float eps, int T, void* stream) {
    HcPreArgs a{};
    a.R_in = R_in; a.emb_table = emb_table; a.toks = toks; a.n_vocab = n_vocab;
    a.bo = bo; a.inj_prev = inj_prev; a.R_out = R_out; a.norm_w = norm_w;
    a.down_q = down_q; a.down_s = down_s; a.inj_w = inj_w; a.nsc = nsc; a.lo = lo; a.inj = inj;
    a.D = D; a.HC = HC; a.HCLR = HCLR; a.eps = eps;
    hipStream_t st = as_stream(stream);
    WZY_TRY(launch_hc_pre(a, T, st));
    HcPostArgs b{};
    b.R = R_out; b.nsc = nsc; b.norm_w = norm_w; b.up_q = up_q; b.up_s = up_s; b.lo = lo; b.mixed = mixed;
    b.D = D; b.HC = HC; b.HCLR = HCLR;
    return launch_hc_post(b, T, st);
}

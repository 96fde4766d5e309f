// hc.hip -- 4-stream hyper-connection (HC) read/write for gfx950.
//
// The reference reads the residual streams with four kernels (norm+fold, down+inject, quantise,
// up+mean) and writes them with a fifth (src/wzy_stage_v2.cuh:463-470, src/wzy_kernels_v2.cuh:
// 409-454,632-827).  Here a read is two launches and the write is folded into the next read:
//
//   hc_pre : R_out = R_in + bo * 2*sigmoid(inj_prev/HC)           (the pending write, or the
//            embedding broadcast on layer 0), per-stream RMS scale, xn = R_out*scale*w quantised
//            per 32 inside each lane, lo = silu(down . xn / HC), inj = inj_w . xn.
//            Every workgroup recomputes the four stream norms from L2 (32 KB per row) so no
//            cross-workgroup synchronisation is needed; R_out goes to the other ping-pong buffer.
//   hc_post: mixed[d] = 0.25 * sum_c xn[c][d] * sigmoid(up[c*D+d] . quant32(lo)).
// One 64-lane wave per weight row; all 16-byte loads of a row are issued before any arithmetic.
#include "wzy_device.h"
#include "wzy_hc.h"
#include "wzy_host.h"

using namespace wzy;

namespace {

// Quantise 32 consecutive fp32 values (reference per-32 rule) into 8 packed int8 words.
WZY_DEV void quant32_lane(const float (&v)[32], int4& q0, int4& q1, float& d) {
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

// residual value before the norm: R_in (+ fold) or the embedding row
WZY_DEV float hc_value(const HcPreArgs& a, int t, int c, int d, float gw) {
    float v;
    if (a.emb_rows) {
        v = a.emb_rows[(size_t) t * a.D + d];
    } else if (a.emb_table) {
        int tok = a.toks[t];
        tok = tok < 0 ? 0 : (tok >= a.n_vocab ? a.n_vocab - 1 : tok);
        v = bf16_to_f(a.emb_table[(size_t) tok * a.D + d]);
    } else {
        v = a.R_in[((size_t) t * a.HC + c) * a.D + d];
    }
    if (a.bo) v = fmaf(a.bo[(size_t) t * a.D + d], gw, v);
    return v;
}

}  // namespace

// grid: 1D, one wave per row: rows [0, HCLR) are down rows, [HCLR, HCLR+HC) inject rows (if inj_w).
template <int T, int NBL>
__global__ void __launch_bounds__(256) hc_pre_kernel(HcPreArgs a) {
    __shared__ float s_red[4][WZY_MAX_W * 4];
    __shared__ float s_nsc[WZY_MAX_W * 4];
    __shared__ float s_gw[WZY_MAX_W * 4];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int D = a.D, HC = a.HC, HCD = HC * D;

    // fold gates
    if (tid < T * HC) {
        const int t = tid / HC, c = tid % HC;
        s_gw[tid] = a.bo ? 2.0f / (1.0f + __expf(-a.inj_prev[t * HC + c] / (float) HC)) : 0.f;
    }
    __syncthreads();

    // pass 1: per-stream sum of squares (every workgroup), R_out slice written by this workgroup
    float ss[T * 4];
#pragma unroll
    for (int i = 0; i < T * 4; ++i) ss[i] = 0.f;
    const int n_wg = gridDim.x;
    const int slice = (D + n_wg - 1) / n_wg;
    const int d_lo = blockIdx.x * slice, d_hi = min(D, d_lo + slice);
    for (int d = tid; d < D; d += blockDim.x) {
#pragma unroll
        for (int t = 0; t < T; ++t)
            for (int c = 0; c < HC; ++c) {
                const float v = hc_value(a, t, c, d, s_gw[t * HC + c]);
                ss[t * 4 + c] = fmaf(v, v, ss[t * 4 + c]);
            }
    }
    for (int d = d_lo + tid; d < d_hi; d += blockDim.x)
#pragma unroll
        for (int t = 0; t < T; ++t)
            for (int c = 0; c < HC; ++c)
                a.R_out[((size_t) t * HC + c) * D + d] = hc_value(a, t, c, d, s_gw[t * HC + c]);
#pragma unroll
    for (int i = 0; i < T * 4; ++i) {
        if (i % 4 >= HC) continue;
        const float v = wave_sum(ss[i]);
        if (lane == 0) s_red[w][i] = v;
    }
    __syncthreads();
    if (tid < T * HC) {
        const int t = tid / HC, c = tid % HC;
        const float tot = s_red[0][t * 4 + c] + s_red[1][t * 4 + c] + s_red[2][t * 4 + c] + s_red[3][t * 4 + c];
        const float sc = 1.0f / sqrtf(tot / (float) D + a.eps);
        s_nsc[tid] = sc;
        if (blockIdx.x == 0) a.nsc[tid] = sc;
    }
    __syncthreads();

    // pass 2: one row per wave
    const int row = blockIdx.x * 4 + w;
    const int n_rows = a.HCLR + (a.inj_w ? HC : 0);
    if (row >= n_rows) return;
    const bool is_inj = row >= a.HCLR;
    const int nb = HCD / 32;
    float acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = 0.f;

    if (!is_inj) {
        int4 c0[NBL], c1[NBL];
        float dw[NBL];
#pragma unroll
        for (int i = 0; i < NBL; ++i) {
            const int b = lane + 64 * i;
            if (b < nb) {
                const int4* cp = (const int4*) (a.down_q + (size_t) row * HCD + (size_t) b * 32);
                c0[i] = ld_stream_i4(cp);
                c1[i] = ld_stream_i4(cp + 1);
                dw[i] = h16_to_f(a.down_s[(size_t) row * nb + b]);
            }
        }
#pragma unroll
        for (int i = 0; i < NBL; ++i) {
            const int b = lane + 64 * i;
            if (b >= nb) continue;
            const int c = (32 * b) / D, d0 = (32 * b) % D;
#pragma unroll
            for (int t = 0; t < T; ++t) {
                float v[32];
                const float sc = s_nsc[t * HC + c], gw = s_gw[t * HC + c];
#pragma unroll
                for (int k = 0; k < 32; ++k)
                    v[k] = hc_value(a, t, c, d0 + k, gw) * sc * a.norm_w[(size_t) c * D + d0 + k];
                int4 x0, x1;
                float xs;
                quant32_lane(v, x0, x1, xs);
                acc[t] = fmaf(dw[i] * xs, (float) (dot16(c0[i], x0) + dot16(c1[i], x1)), acc[t]);
            }
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const float s = wave_sum(acc[t]) / (float) HC;
            if (lane == 0) a.lo[(size_t) t * a.HCLR + row] = s / (1.0f + __expf(-s));
        }
    } else {
        const int r = row - a.HCLR;
        const uint16_t* wr = a.inj_w + (size_t) r * HCD;
        for (int j = lane; j < HCD / 8; j += 64) {
            const uint4 wv = ld_stream_u4((const uint4*) wr + j);
            const int c = (8 * j) / D, d0 = (8 * j) % D;
            const float wf[8] = {bf16_lo(wv.x), bf16_hi(wv.x), bf16_lo(wv.y), bf16_hi(wv.y),
                                 bf16_lo(wv.z), bf16_hi(wv.z), bf16_lo(wv.w), bf16_hi(wv.w)};
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const float sc = s_nsc[t * HC + c], gw = s_gw[t * HC + c];
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const float xn = hc_value(a, t, c, d0 + k, gw) * sc * a.norm_w[(size_t) c * D + d0 + k];
                    acc[t] = fmaf(wf[k], xn, acc[t]);
                }
            }
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const float s = wave_sum(acc[t]);
            if (lane == 0) a.inj[t * HC + r] = s;
        }
    }
}

// hc_post: wave handles 2 output positions d; 16 lanes per (d, stream) row of `up` (HCLR/32 blocks).
template <int T>
__global__ void __launch_bounds__(256) hc_post_kernel(HcPostArgs a) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = (blockIdx.x * blockDim.x + tid) >> 6;
    const int D = a.D, HC = a.HC, L = a.HCLR, nb = L / 32;
    const int li = lane & 15, c = (lane >> 4) & 3;
    const bool active_c = c < HC;
#pragma unroll 1
    for (int k = 0; k < 2; ++k) {
        const int d = wave * 2 + k;
        if (d >= D) return;
        float acc[T];
#pragma unroll
        for (int t = 0; t < T; ++t) acc[t] = 0.f;
        if (active_c) {
            const size_t row = (size_t) c * D + d;
            for (int b = li; b < nb; b += 16) {
                const int4* cp = (const int4*) (a.up_q + row * L + (size_t) b * 32);
                const int4 c0 = ld_stream_i4(cp), c1 = ld_stream_i4(cp + 1);
                const float dw = h16_to_f(a.up_s[row * nb + b]);
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    float v[32];
#pragma unroll
                    for (int j = 0; j < 32; ++j) v[j] = a.lo[(size_t) t * L + 32 * b + j];
                    float am = 0.f;
#pragma unroll
                    for (int j = 0; j < 32; ++j) am = fmaxf(am, fabsf(v[j]));
                    const float xs = am / 127.0f, inv = xs > 0.f ? 127.0f / am : 0.f;
                    int isum = 0;
                    const int8_t* cb = (const int8_t*) &c0;
                    const int8_t* cb1 = (const int8_t*) &c1;
#pragma unroll
                    for (int j = 0; j < 16; ++j) isum += (int) cb[j] * max(-127, min(127, rn_int(v[j] * inv)));
#pragma unroll
                    for (int j = 0; j < 16; ++j) isum += (int) cb1[j] * max(-127, min(127, rn_int(v[16 + j] * inv)));
                    acc[t] = fmaf(dw * xs, (float) isum, acc[t]);
                }
            }
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const float s = sum16(acc[t]);          // every lane of the 16-lane group holds stream c's sum
            float g = 0.f;
            if (li == 0 && active_c) {
                const float xn = a.R[((size_t) t * HC + c) * D + d] * a.nsc[t * HC + c] * a.norm_w[(size_t) c * D + d];
                g = xn / (1.0f + __expf(-s));
            }
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

template <int T>
static void launch_pre_t(const HcPreArgs& a, hipStream_t st) {
    const int n_rows = a.HCLR + (a.inj_w ? a.HC : 0);
    const int blocks = (n_rows + 3) / 4;
    const int nbl = (a.HC * a.D / 32 + 63) / 64;
    if (nbl <= 4) hipLaunchKernelGGL((hc_pre_kernel<T, 4>), dim3(blocks), dim3(256), 0, st, a);
    else hipLaunchKernelGGL((hc_pre_kernel<T, 8>), dim3(blocks), dim3(256), 0, st, a);
}

int launch_hc_pre(const HcPreArgs& a, int T, hipStream_t st) {
    WZY_REQUIRE(T >= 1 && T <= WZY_MAX_W, "hc_pre: T out of range");
    WZY_REQUIRE(a.HC >= 1 && a.HC <= 4 && a.D % 32 == 0 && a.HCLR % 32 == 0, "hc_pre: unsupported shape");
    WZY_REQUIRE(a.HC * a.D / 32 <= 64 * 8, "hc_pre: HC*D too large (max 16384)");
    WZY_REQUIRE((a.R_in != nullptr) + (a.emb_table != nullptr) + (a.emb_rows != nullptr) == 1,
                "hc_pre: exactly one of R_in / emb_table / emb_rows");
    WZY_REQUIRE(!a.emb_table || a.toks, "hc_pre: embedding mode needs toks");
    WZY_REQUIRE(!a.bo || a.inj_prev, "hc_pre: fold needs inj_prev");
    WZY_REQUIRE(a.R_out && a.norm_w && a.down_q && a.down_s && a.nsc && a.lo, "hc_pre: null pointer");
    WZY_REQUIRE(!a.inj_w || a.inj, "hc_pre: inject weights need an inj output");
    switch (T) {
        case 1: launch_pre_t<1>(a, st); break;
        case 2: launch_pre_t<2>(a, st); break;
        case 3: launch_pre_t<3>(a, st); break;
        case 4: launch_pre_t<4>(a, st); break;
        case 5: launch_pre_t<5>(a, st); break;
        case 6: launch_pre_t<6>(a, st); break;
        case 7: launch_pre_t<7>(a, st); break;
        default: launch_pre_t<8>(a, st); break;
    }
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

int launch_hc_post(const HcPostArgs& a, int T, hipStream_t st) {
    WZY_REQUIRE(T >= 1 && T <= WZY_MAX_W, "hc_post: T out of range");
    WZY_REQUIRE(a.HC >= 1 && a.HC <= 4 && a.HCLR % 32 == 0 && a.HCLR <= 512, "hc_post: unsupported shape");
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

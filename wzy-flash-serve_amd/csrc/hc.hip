// hc.hip -- 4-stream hyper-connection (HC) read for gfx950.
//
// The reference reads the residual streams with four kernels (norm+fold, down+inject, quantise,
// up+mean) and writes them with a fifth (src/wzy_stage_v2.cuh:463-470, src/wzy_kernels_v2.cuh:
// 409-454,632-827).  Here a read is two launches and the pending write is folded into the next read:
//
//   hc_pre : R_out = R_in + bo * 2*sigmoid(inj_prev/HC)           (the pending write, or the
//            embedding broadcast on layer 0), per-stream RMS scale, xn = R_out*scale*w,
//            lo = silu(down . quant32(xn) / HC), inj = inj_w . xn.
//            Every workgroup rebuilds quant32(xn) for the window in LDS (the residual is 32 KB per
//            row and L2-resident), so no cross-workgroup synchronisation is needed; workgroup w
//            writes every gridDim-th 32-block of R_out; four extra workgroups compute inj.
//   hc_post: mixed[d] = 0.25 * sum_c xn[c][d] * sigmoid(up[c*D+d] . quant32(lo)); lo is quantised
//            once per workgroup into LDS.
// Both kernels issue every global load a row needs before using any of them (indices clamped
// instead of branching, fp16 scales converted afterwards): one memory round trip per window row.
#include <algorithm>

#include "wzy_device.h"
#include "wzy_hc.h"
#include "wzy_host.h"

using namespace wzy;

namespace {

constexpr int HC4 = 4;            // stream count of the hyper-connection

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

}  // namespace

// T window rows (<= 4 per launch), D <= DC.  256 threads; thread tid owns the 32-value blocks
// b = tid + 256k of the flattened [HC*D] row; wave w of workgroup g owns down rows
// (4g + w) * RPW .. + RPW - 1.  Dynamic LDS: int8 xq [T][4D] then fp32 xs [T][4D/32].
template <int T, int DC, int RPW>
__global__ void __launch_bounds__(256) hc_pre_kernel(HcPreArgs a) {
    constexpr int NBK = DC >= 2048 ? DC / 2048 : 1;   // 32-blocks per thread
    constexpr int NBL = DC / 512;                      // 32-blocks per lane of one down row
    extern __shared__ __align__(16) unsigned char s_dyn[];
    __shared__ float s_seg[WZY_MAX_W][64];             // sums of 8 consecutive blocks (256 values)
    __shared__ float s_nsc[T * HC4];
    __shared__ float s_inj[4];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int D = a.D, HCD = HC4 * D, nb = HCD / 32, L = a.HCLR, spb = D / 256;
    int8_t* s_xq = (int8_t*) s_dyn;
    float* s_xs = (float*) (s_dyn + (size_t) T * HCD);
    const bool fold = a.bo != nullptr;
    // workgroups [0, n_row_wg) own down rows; the HC workgroups after them (inject weights only)
    // compute inj row blockIdx.x - n_row_wg
    const int n_row_wg = (L + 4 * RPW - 1) / (4 * RPW);
    const bool has_rows = (int) blockIdx.x < n_row_wg;
    const bool do_inj = !has_rows && a.inj_w != nullptr;
    const int inj_row = blockIdx.x - n_row_wg;
    const bool wave_stream = NBK == 1 && D == 64 * 32;   // wave w owns all of stream w

    // 0. this wave's down rows (raw codes and fp16 scales), issued first
    const int row0 = (blockIdx.x * 4 + w) * RPW;
    int4 c0[NBL][RPW], c1[NBL][RPW];
    uint16_t sraw[NBL][RPW];
    if (has_rows) {
#pragma unroll
        for (int i = 0; i < NBL; ++i) {
            const int b = min(lane + 64 * i, nb - 1);
#pragma unroll
            for (int s = 0; s < RPW; ++s) {
                const int r = min(row0 + s, L - 1);
                const int4* cp = (const int4*) (a.down_q + (size_t) r * HCD + (size_t) b * 32);
                c0[i][s] = ld_stream_i4(cp);
                c1[i][s] = ld_stream_i4(cp + 1);
                sraw[i][s] = a.down_s[(size_t) r * nb + b];
            }
        }
    }
    // 1. row-independent inputs of this thread's blocks: norm weights, inject weights
    float4 nw[NBK][8];
    uint4 iw[NBK][4];
#pragma unroll
    for (int k = 0; k < NBK; ++k) {
        const int b = min(tid + 256 * k, nb - 1);
        const int c = (32 * b) / D, d0 = (32 * b) % D;
#pragma unroll
        for (int j = 0; j < 8; ++j) nw[k][j] = *(const float4*) (a.norm_w + (size_t) c * D + d0 + 4 * j);
        if (do_inj) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                iw[k][j] = *(const uint4*) (a.inj_w + (size_t) inj_row * HCD + (size_t) 32 * b + 8 * j);
        }
    }

    float inj_acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) inj_acc[t] = 0.f;
#pragma unroll
    for (int t = 0; t < T; ++t) {
        // 2. residual (or embedding) and fold inputs of this row
        float4 rv[NBK][8], bv[NBK][8];
        float ip[NBK];
        int tok = 0;
        if (a.emb_table) {
            tok = a.toks[t];
            tok = tok < 0 ? 0 : (tok >= a.n_vocab ? a.n_vocab - 1 : tok);
        }
#pragma unroll
        for (int k = 0; k < NBK; ++k) {
            const int b = min(tid + 256 * k, nb - 1);
            const int c = (32 * b) / D, d0 = (32 * b) % D;
            if (a.emb_table) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint2 h = *(const uint2*) (a.emb_table + (size_t) tok * D + d0 + 4 * j);
                    rv[k][j] = make_float4(__builtin_bit_cast(float, h.x), __builtin_bit_cast(float, h.y), 0.f, 0.f);
                }
            } else if (a.emb_rows) {
#pragma unroll
                for (int j = 0; j < 8; ++j) rv[k][j] = *(const float4*) (a.emb_rows + (size_t) t * D + d0 + 4 * j);
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    rv[k][j] = *(const float4*) (a.R_in + ((size_t) t * HC4 + c) * D + d0 + 4 * j);
            }
            if (fold) {
#pragma unroll
                for (int j = 0; j < 8; ++j) bv[k][j] = *(const float4*) (a.bo + (size_t) t * D + d0 + 4 * j);
                ip[k] = a.inj_prev[t * HC4 + c];
            }
        }
        // 3. folded values and the per-thread sums of squares
        float v[NBK][32];
        float sc_w = 0.f;
#pragma unroll
        for (int k = 0; k < NBK; ++k) {
            const float gw = fold ? 2.0f / (1.0f + __expf(-ip[k] / (float) HC4)) : 0.f;
            float ss = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                float4 x = rv[k][j];
                if (a.emb_table) {
                    const uint32_t lo = __builtin_bit_cast(uint32_t, x.x), hi = __builtin_bit_cast(uint32_t, x.y);
                    x = make_float4(bf16_lo(lo), bf16_hi(lo), bf16_lo(hi), bf16_hi(hi));
                }
                if (fold) {
                    x.x = fmaf(bv[k][j].x, gw, x.x);
                    x.y = fmaf(bv[k][j].y, gw, x.y);
                    x.z = fmaf(bv[k][j].z, gw, x.z);
                    x.w = fmaf(bv[k][j].w, gw, x.w);
                }
                v[k][4 * j + 0] = x.x; v[k][4 * j + 1] = x.y; v[k][4 * j + 2] = x.z; v[k][4 * j + 3] = x.w;
                ss = fmaf(x.x, x.x, ss);
                ss = fmaf(x.y, x.y, ss);
                ss = fmaf(x.z, x.z, ss);
                ss = fmaf(x.w, x.w, ss);
            }
            // 4. per-stream sums.  D = 2048 with one block per thread: wave w holds exactly stream w,
            //    so the sum is a wave reduction; otherwise sums over 8 consecutive blocks (never
            //    straddling a stream, D % 256 == 0) are combined through LDS.
            if (wave_stream) {
                sc_w = 1.0f / sqrtf(wave_sum(ss) / (float) D + a.eps);
                if (lane == 0 && blockIdx.x == 0) a.nsc[t * HC4 + w] = sc_w;
            } else {
                ss = sum8(ss);
                const int b = tid + 256 * k;
                if ((lane & 7) == 0 && b < nb) s_seg[t][b >> 3] = ss;
            }
        }
        if (!wave_stream) {
            __syncthreads();
            if (tid < HC4) {
                float tot = 0.f;
                for (int i = 0; i < spb; ++i) tot += s_seg[t][tid * spb + i];
                const float sc = 1.0f / sqrtf(tot / (float) D + a.eps);
                s_nsc[t * HC4 + tid] = sc;
                if (blockIdx.x == 0) a.nsc[t * HC4 + tid] = sc;
            }
            __syncthreads();
        }
        // 5. xn quantised per 32 into LDS, inject partial, R_out blocks
#pragma unroll
        for (int k = 0; k < NBK; ++k) {
            const int b = tid + 256 * k;
            if (b >= nb) continue;
            const int c = (32 * b) / D, d0 = (32 * b) % D;
            const float sc = wave_stream ? sc_w : s_nsc[t * HC4 + c];
            float xn[32];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                xn[4 * j + 0] = v[k][4 * j + 0] * sc * nw[k][j].x;
                xn[4 * j + 1] = v[k][4 * j + 1] * sc * nw[k][j].y;
                xn[4 * j + 2] = v[k][4 * j + 2] * sc * nw[k][j].z;
                xn[4 * j + 3] = v[k][4 * j + 3] * sc * nw[k][j].w;
            }
            if (do_inj) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint4 u = iw[k][j];
                    float acc = inj_acc[t];
                    acc = fmaf(bf16_lo(u.x), xn[8 * j + 0], acc);
                    acc = fmaf(bf16_hi(u.x), xn[8 * j + 1], acc);
                    acc = fmaf(bf16_lo(u.y), xn[8 * j + 2], acc);
                    acc = fmaf(bf16_hi(u.y), xn[8 * j + 3], acc);
                    acc = fmaf(bf16_lo(u.z), xn[8 * j + 4], acc);
                    acc = fmaf(bf16_hi(u.z), xn[8 * j + 5], acc);
                    acc = fmaf(bf16_lo(u.w), xn[8 * j + 6], acc);
                    acc = fmaf(bf16_hi(u.w), xn[8 * j + 7], acc);
                    inj_acc[t] = acc;
                }
            }
            if (has_rows) {
                int4 q0, q1;
                float xs;
                quant32_vals(xn, q0, q1, xs);
                int4* dst = (int4*) (s_xq + (size_t) t * HCD + (size_t) 32 * b);
                dst[0] = q0;
                dst[1] = q1;
                s_xs[t * nb + b] = xs;
            }
            if ((b % gridDim.x) == blockIdx.x) {
                float* ro = a.R_out + ((size_t) t * HC4 + c) * D + d0;
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    *(float4*) (ro + 4 * j) = make_float4(v[k][4 * j], v[k][4 * j + 1], v[k][4 * j + 2], v[k][4 * j + 3]);
            }
        }
    }
    if (do_inj) {                             // workgroup-uniform branch
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const float s = block_sum<4>(inj_acc[t], s_inj);
            if (tid == 0) a.inj[t * HC4 + inj_row] = s;
        }
        return;
    }
    __syncthreads();

    // 6. down rows: lo = silu(down . xq / HC)
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
                acc[s][t] = fmaf(h16_to_f(sraw[i][s]) * xs, (float) (dot16(c0[i][s], x0) + dot16(c1[i][s], x1)),
                                 acc[s][t]);
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
    const int lb = min(li, nb - 1);

    // every load first: weights, the residual / scale / norm inputs of xn, and lo
    int4 c0[2], c1[2];
    uint16_t sraw[2];
    float rr[2][T], nwv[2], nscv[T];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int d = min(wave * 2 + k, D - 1);
        const size_t row = (size_t) c * D + d;
        const int4* cp = (const int4*) (a.up_q + row * L + (size_t) lb * 32);
        c0[k] = ld_stream_i4(cp);
        c1[k] = ld_stream_i4(cp + 1);
        sraw[k] = a.up_s[row * nb + lb];
        nwv[k] = a.norm_w[row];
#pragma unroll
        for (int t = 0; t < T; ++t) rr[k][t] = a.R[((size_t) t * HC4 + c) * D + d];
    }
#pragma unroll
    for (int t = 0; t < T; ++t) nscv[t] = a.nsc[t * HC4 + c];
    float4 lv[8];
    const int lt = min(tid / nb, T - 1), lbb = tid % nb;
    if (tid < T * nb) {                      // issued after every other load of the wave
#pragma unroll
        for (int k = 0; k < 8; ++k) lv[k] = *(const float4*) (a.lo + (size_t) lt * L + 32 * lbb + 4 * k);
    }
    // quant32(lo) once per workgroup
    if (tid < T * nb) {
        float v[32];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            v[4 * k] = lv[k].x; v[4 * k + 1] = lv[k].y; v[4 * k + 2] = lv[k].z; v[4 * k + 3] = lv[k].w;
        }
        int4 q0, q1;
        float xs;
        quant32_vals(v, q0, q1, xs);
        s_lq[lt][2 * lbb] = q0;
        s_lq[lt][2 * lbb + 1] = q1;
        s_ls[lt][lbb] = xs;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int d = wave * 2 + k;
        if (d >= D) break;                   // wave-uniform
        const float dw = h16_to_f(sraw[k]);
#pragma unroll
        for (int t = 0; t < T; ++t) {
            float acc = 0.f;
            if (li < nb) acc = dw * s_ls[t][li] * (float) (dot16(c0[k], s_lq[t][2 * li]) + dot16(c1[k], s_lq[t][2 * li + 1]));
            const float s = sum16(acc);      // every lane of the 16-lane group holds stream c's sum
            const float xn = rr[k][t] * nscv[t] * nwv[k];
            const float g = (li == 0) ? xn / (1.0f + __expf(-s)) : 0.f;
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
template <int T, int DC, int RPW>
void launch_pre_tdc(const HcPreArgs& a, hipStream_t st) {
    const int HCD = HC4 * a.D;
    const int rows_wg = 4 * RPW;
    const int blocks = (a.HCLR + rows_wg - 1) / rows_wg + (a.inj_w ? HC4 : 0);
    const size_t lds = (size_t) T * HCD + (size_t) T * (HCD / 32) * sizeof(float);
    hipLaunchKernelGGL((hc_pre_kernel<T, DC, RPW>), dim3(blocks), dim3(256), lds, st, a);
}
template <int T>
void launch_pre_t(const HcPreArgs& a, hipStream_t st) {
    if (a.D <= 1024) launch_pre_tdc<T, 1024, 2>(a, st);
    else if (a.D <= 2048) launch_pre_tdc<T, 2048, 2>(a, st);
    else launch_pre_tdc<T, 4096, 1>(a, st);
}
}  // namespace

int launch_hc_pre(const HcPreArgs& a0, int T, hipStream_t st) {
    WZY_REQUIRE(T >= 1 && T <= WZY_MAX_W, "hc_pre: T out of range");
    WZY_REQUIRE(a0.HC == HC4 && a0.D % 256 == 0 && a0.D >= 256 && a0.D <= 4096 && a0.HCLR % 32 == 0 &&
                    a0.HCLR >= 32 && a0.HCLR <= 512,
                "hc_pre: unsupported shape (HC must be 4, D a multiple of 256 <= 4096, HCLR a multiple of 32 <= 512)");
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

// hc.hip -- 4-stream hyper-connection (HC) read for gfx950.
//
// The reference reads the residual streams with four kernels (norm+fold, down+inject, quantise,
// up+mean) and writes them with a fifth (src/wzy_stage_v2.cuh:463-470, src/wzy_kernels_v2.cuh:
// 409-454,632-827).  Here a read is two launches and the pending write is folded into the next read:
//
//   hc_pre : split by stream.  Workgroup (c, rb) loads only stream c of the residual (the pending
//            write R_out = R_in + bo * 2*sigmoid(inj_prev/HC) folded in, or the embedding broadcast
//            on layer 0), forms its RMS scale and xn = R_out*scale*w, quantises xn per 32 into LDS
//            and multiplies it with stream c's columns of 4*RPW rows of `down`:
//                lo_part[t][c][r] = down[r, c*D : (c+1)*D] . quant32(xn_c).
//            Workgroup (c, NRB) writes stream c of R_out, its scale nsc[t][c], and the inject
//            partials inj_part[t][c][o] = inj_w[o, c*D : (c+1)*D] . xn_c.
//            Each workgroup moves one stream's activations (3 x D floats), not all four.
//   hc_post: lo = silu(((p0 + p1) + (p2 + p3)) / HC) from the four partials, quantised per 32 once
//            per workgroup into LDS (two values per thread); mixed[d] = 0.25 * sum_c xn[c][d] * sigmoid(up[c*D+d] . quant32(lo)).
//            Workgroup 0 also writes lo and the summed inj.
// Every global load a row needs is issued before any of them is used (indices clamped instead of
// branching, fp16 scales converted afterwards).
#include <algorithm>

#include "wzy_device.h"
#include "wzy_hc.h"
#include "wzy_host.h"

using namespace wzy;

namespace {

constexpr int HC4 = 4;            // stream count of the hyper-connection

// N consecutive fp32 values (N in {1, 2, 4, 8, 16}; p aligned to 4*N bytes)
template <int N>
WZY_DEV void ld_f32(const float* p, float (&v)[N]) {
    if constexpr (N >= 4) {
#pragma unroll
        for (int k = 0; k < N / 4; ++k) {
            const float4 f = ((const float4*) p)[k];
            v[4 * k] = f.x; v[4 * k + 1] = f.y; v[4 * k + 2] = f.z; v[4 * k + 3] = f.w;
        }
    } else if constexpr (N == 2) {
        const float2 f = *(const float2*) p;
        v[0] = f.x; v[1] = f.y;
    } else {
        v[0] = p[0];
    }
}
// N consecutive bf16 values as raw 32-bit words (N/2 words, one half-filled word when N == 1)
template <int N>
struct Bf16Raw {
    uint32_t w[N >= 2 ? N / 2 : 1];
};
template <int N>
WZY_DEV Bf16Raw<N> ld_bf16_raw(const uint16_t* p) {
    Bf16Raw<N> r;
    if constexpr (N >= 8) {
#pragma unroll
        for (int k = 0; k < N / 8; ++k) {
            const uint4 u = ((const uint4*) p)[k];
            r.w[4 * k] = u.x; r.w[4 * k + 1] = u.y; r.w[4 * k + 2] = u.z; r.w[4 * k + 3] = u.w;
        }
    } else if constexpr (N == 4) {
        const uint2 u = *(const uint2*) p;
        r.w[0] = u.x; r.w[1] = u.y;
    } else if constexpr (N == 2) {
        r.w[0] = *(const uint32_t*) p;
    } else {
        r.w[0] = p[0];
    }
    return r;
}
template <int N>
WZY_DEV float bf16_at(const Bf16Raw<N>& r, int j) {
    return (j & 1) ? bf16_hi(r.w[j >> 1]) : bf16_lo(r.w[j >> 1]);
}
// N consecutive int8 values as floats (N in {1, 2, 4, 8, 16}; p aligned to N bytes)
template <int N>
WZY_DEV void ld_i8_f(const int8_t* p, float (&v)[N]) {
    if constexpr (N >= 4) {
        uint32_t w[N / 4];
        if constexpr (N == 16) { const uint4 u = *(const uint4*) p; w[0] = u.x; w[1] = u.y; w[2] = u.z; w[3] = u.w; }
        else if constexpr (N == 8) { const uint2 u = *(const uint2*) p; w[0] = u.x; w[1] = u.y; }
        else w[0] = *(const uint32_t*) p;
#pragma unroll
        for (int j = 0; j < N; ++j) v[j] = (float) (int8_t) (w[j >> 2] >> (8 * (j & 3)));
    } else {
#pragma unroll
        for (int j = 0; j < N; ++j) v[j] = (float) p[j];
    }
}

// max over aligned groups of G consecutive lanes (G in {1, 2, 4, 8, 16, 32})
template <int G>
WZY_DEV float group_max(float v) {
    if constexpr (G >= 2) v = fmaxf(v, dpp_f<DPP_XOR1>(v));
    if constexpr (G >= 4) v = fmaxf(v, dpp_f<DPP_XOR2>(v));
    if constexpr (G >= 8) v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
    if constexpr (G >= 16) v = fmaxf(v, dpp_f<DPP_MIRROR>(v));
    if constexpr (G >= 32) v = fmaxf(v, swz_f<SWZ_XOR16>(v));
    return v;
}

// sum over the NW waves of a workgroup (four waves: the pairing (w0 + w1) + (w2 + w3))
template <int NW>
WZY_DEV float waves_sum(const float (*sh)[4], int o) {
    if constexpr (NW == 4) return (sh[0][o] + sh[1][o]) + (sh[2][o] + sh[3][o]);
    float s = sh[0][o];
#pragma unroll
    for (int i = 1; i < NW; ++i) s += sh[i][o];
    return s;
}

// waves_sum over column o of a wider table (the same pairing)
template <int NW, int W>
WZY_DEV float waves_sum_w(const float (*sh)[W], int o) {
    if constexpr (NW == 4) return (sh[0][o] + sh[1][o]) + (sh[2][o] + sh[3][o]);
    float s = sh[0][o];
#pragma unroll
    for (int i = 1; i < NW; ++i) s += sh[i][o];
    return s;
}

// sum of 4 values per thread over the NW-wave workgroup; results valid on thread 0
template <int NW>
WZY_DEV void block_sum4_t0(float (&v)[4], float (*sh)[4]) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int o = 0; o < 4; ++o) v[o] = wave_sum(v[o]);
    if (lane == 0)
#pragma unroll
        for (int o = 0; o < 4; ++o) sh[w][o] = v[o];
    __syncthreads();
    if (threadIdx.x == 0)
#pragma unroll
        for (int o = 0; o < 4; ++o) v[o] = waves_sum<NW>(sh, o);
}

}  // namespace

// T window rows; NW waves per workgroup; VPT = D/(64*NW) values of the stream per thread; NBL =
// 32-blocks per lane of one down row (D/32/64 rounded up); RPW down rows per wave.  Workgroup b:
// stream c = b % 4, row block rb = b / 4 (rows rb*NW*RPW ..), rb == NRB is the stream's R_out / nsc /
// inject workgroup.  Dynamic LDS (row workgroups): int8 xq [T][D] then fp32 xs [T][D/32].
template <int T, int VPT, int NBL, int RPW, int NW>
__global__ void __launch_bounds__(64 * NW) hc_pre_kernel(HcPreArgs a) {
    extern __shared__ __align__(16) unsigned char s_dyn[];
    __shared__ float s_red[NW][4];
    __shared__ float s_inj[NW][4 * (T <= 4 ? T : 1)];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int D = a.D, HCD = HC4 * D, NB = D / 32, L = a.HCLR;
    constexpr int G = 32 / VPT;                        // threads per 32-block
    const int c = blockIdx.x & 3, rb = blockIdx.x >> 2;
    const int nrb = (L + NW * RPW - 1) / (NW * RPW);
    const bool aux = rb >= nrb;                        // workgroup-uniform
    const bool do_inj = aux && a.inj_w != nullptr;
    int8_t* s_xq = (int8_t*) s_dyn;
    float* s_xs = (float*) (s_dyn + (size_t) T * D);
    const bool fold = a.bo != nullptr;
    const int d0 = tid * VPT;                          // this thread's values: d0 .. d0+VPT-1 of stream c

    // 0. this wave's down rows (raw codes and fp16 scales of stream c's columns), issued first
    const int row0 = (rb * NW + w) * RPW;
    int4 c0[NBL][RPW], c1[NBL][RPW];
    uint32_t sraw[NBL][RPW];         // 16-bit scales held in 32-bit registers (no packing that waits for the load)
    if (!aux) {
#pragma unroll
        for (int i = 0; i < NBL; ++i) {
            const int b = min(lane + 64 * i, NB - 1);
#pragma unroll
            for (int s = 0; s < RPW; ++s) {
                const int r = min(row0 + s, L - 1);
                const int4* cp = (const int4*) (a.down_q + (size_t) r * HCD + (size_t) c * D + (size_t) b * 32);
                c0[i][s] = ld_stream_i4(cp);
                c1[i][s] = ld_stream_i4(cp + 1);
                sraw[i][s] = a.down_s[(size_t) r * (HCD / 32) + (size_t) c * NB + b];
            }
        }
    }
    // 1. row-independent inputs: norm weights, inject weights
    float nw[VPT];
    ld_f32<VPT>(a.norm_w + (size_t) c * D + d0, nw);
    Bf16Raw<VPT> iw[4];
    if (do_inj) {
#pragma unroll
        for (int o = 0; o < 4; ++o) iw[o] = ld_bf16_raw<VPT>(a.inj_w + (size_t) o * HCD + (size_t) c * D + d0);
    }

    // 2. residual (or embedding) of row t with the pending block folded in
    auto load_row = [&](int t, float (&v)[VPT]) {
        if (a.emb_table) {
            int tok = a.toks[t];
            tok = tok < 0 ? 0 : (tok >= a.n_vocab ? a.n_vocab - 1 : tok);
            const Bf16Raw<VPT> e = ld_bf16_raw<VPT>(a.emb_table + (size_t) tok * D + d0);
#pragma unroll
            for (int j = 0; j < VPT; ++j) v[j] = bf16_at<VPT>(e, j);
        } else if (a.emb_q) {
            // Q8_0 row: d * q per 32-block, an out-of-range id reads row 0 (stage_one_emb,
            // src/wzy_engine_v2.cu:861-873); a thread's VPT values lie in one 32-block
            int tok = a.toks[t];
            if (tok < 0 || tok >= a.n_vocab) tok = 0;
            ld_i8_f<VPT>(a.emb_q + (size_t) tok * D + d0, v);
            const float d = h16_to_f(a.emb_s[(size_t) tok * (D / 32) + d0 / 32]);
#pragma unroll
            for (int j = 0; j < VPT; ++j) v[j] = d * v[j];
        } else if (a.emb_rows) {
            ld_f32<VPT>(a.emb_rows + (size_t) t * D + d0, v);
        } else {
            ld_f32<VPT>(a.R_in + ((size_t) t * HC4 + c) * D + d0, v);
        }
        if (fold) {
            float bv[VPT];
            ld_f32<VPT>(a.bo + (size_t) t * D + d0, bv);
            const float ip = a.inj_prev[t * HC4 + c];
            const float gw = 2.0f / (1.0f + __expf(-ip / (float) HC4));
#pragma unroll
            for (int j = 0; j < VPT; ++j) v[j] = fmaf(bv[j], gw, v[j]);
        }
    };
    auto sum_sq = [&](const float (&v)[VPT]) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < VPT; ++j) ss = fmaf(v[j], v[j], ss);
        return wave_sum(ss);
    };
    // 3. given the stream scale sc of row t: R_out, nsc and the inject partials (aux workgroups), or
    //    quant32(xn) into LDS (row workgroups)
    auto finish_row = [&](int t, const float (&v)[VPT], float sc) {
        float xn[VPT];
#pragma unroll
        for (int j = 0; j < VPT; ++j) xn[j] = v[j] * sc * nw[j];

        if (aux) {
            float* ro = a.R_out + ((size_t) t * HC4 + c) * D + d0;
            if constexpr (VPT >= 4) {
#pragma unroll
                for (int k = 0; k < VPT / 4; ++k)
                    ((float4*) ro)[k] = make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
            } else {
#pragma unroll
                for (int j = 0; j < VPT; ++j) ro[j] = v[j];
            }
            if (tid == 0) a.nsc[t * HC4 + c] = sc;
            if (do_inj) {
                float acc[4];
#pragma unroll
                for (int o = 0; o < 4; ++o) {
                    acc[o] = 0.f;
#pragma unroll
                    for (int j = 0; j < VPT; ++j) acc[o] = fmaf(bf16_at<VPT>(iw[o], j), xn[j], acc[o]);
                }
                block_sum4_t0<NW>(acc, s_red);
                if (tid == 0)
#pragma unroll
                    for (int o = 0; o < 4; ++o) a.inj_part[((size_t) t * HC4 + c) * HC4 + o] = acc[o];
                __syncthreads();                      // s_red free for the next row
            }
            return;
        }
        // quant32(xn) into LDS: G consecutive threads share one 32-block
        float am = 0.f;
#pragma unroll
        for (int j = 0; j < VPT; ++j) am = fmaxf(am, fabsf(xn[j]));
        am = group_max<G>(am);
        const float dq = am / 127.0f;
        const float inv = dq > 0.f ? 127.0f / am : 0.f;
        uint32_t pk[(VPT + 3) / 4];
#pragma unroll
        for (int k = 0; k < (VPT + 3) / 4; ++k) pk[k] = 0;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int q = max(-127, min(127, rn_int(xn[j] * inv)));
            pk[j >> 2] |= (uint32_t) (q & 0xFF) << (8 * (j & 3));
        }
        int8_t* dst = s_xq + (size_t) t * D + d0;
        if constexpr (VPT == 16) *(int4*) dst = make_int4((int) pk[0], (int) pk[1], (int) pk[2], (int) pk[3]);
        else if constexpr (VPT == 8) *(int2*) dst = make_int2((int) pk[0], (int) pk[1]);
        else if constexpr (VPT == 4) *(int*) dst = (int) pk[0];
        else if constexpr (VPT == 2) *(int16_t*) dst = (int16_t) pk[0];
        else *dst = (int8_t) pk[0];
        if ((tid % G) == 0) s_xs[t * NB + tid / G] = dq;
    };
    if constexpr (T <= 4) {
        // windows of up to four rows: every row's inputs are loaded before any is used, and the four
        // stream sums meet in one barrier (s_red holds one column per row)
        float v[T][VPT];
#pragma unroll
        for (int t = 0; t < T; ++t) load_row(t, v[t]);
        float ssv[T];
#pragma unroll
        for (int t = 0; t < T; ++t) ssv[t] = sum_sq(v[t]);
        if (lane == 0)
#pragma unroll
            for (int t = 0; t < T; ++t) s_red[w][t] = ssv[t];
        __syncthreads();
        float sc[T];
#pragma unroll
        for (int t = 0; t < T; ++t) sc[t] = 1.0f / sqrtf(waves_sum<NW>(s_red, t) / (float) D + a.eps);
        __syncthreads();                              // s_red is reused below
        if (do_inj) {
            // R_out, nsc and every row's inject partials, reduced together behind one barrier (the
            // per-value sums of block_sum4_t0: wave_sum, then the waves in waves_sum's pairing)
            float acc[T][4];
#pragma unroll
            for (int t = 0; t < T; ++t) {
                float xn[VPT];
#pragma unroll
                for (int j = 0; j < VPT; ++j) xn[j] = v[t][j] * sc[t] * nw[j];
                float* ro = a.R_out + ((size_t) t * HC4 + c) * D + d0;
                if constexpr (VPT >= 4) {
#pragma unroll
                    for (int k = 0; k < VPT / 4; ++k)
                        ((float4*) ro)[k] = make_float4(v[t][4 * k], v[t][4 * k + 1], v[t][4 * k + 2], v[t][4 * k + 3]);
                } else {
#pragma unroll
                    for (int j = 0; j < VPT; ++j) ro[j] = v[t][j];
                }
                if (tid == 0) a.nsc[t * HC4 + c] = sc[t];
#pragma unroll
                for (int o = 0; o < 4; ++o) {
                    acc[t][o] = 0.f;
#pragma unroll
                    for (int j = 0; j < VPT; ++j) acc[t][o] = fmaf(bf16_at<VPT>(iw[o], j), xn[j], acc[t][o]);
                }
            }
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int o = 0; o < 4; ++o) acc[t][o] = wave_sum(acc[t][o]);
            if (lane == 0)
#pragma unroll
                for (int t = 0; t < T; ++t)
#pragma unroll
                    for (int o = 0; o < 4; ++o) s_inj[w][4 * t + o] = acc[t][o];
            __syncthreads();
            if (tid == 0)
#pragma unroll
                for (int t = 0; t < T; ++t)
#pragma unroll
                    for (int o = 0; o < 4; ++o)
                        a.inj_part[((size_t) t * HC4 + c) * HC4 + o] = waves_sum_w<NW, 4 * (T <= 4 ? T : 1)>(s_inj, 4 * t + o);
            return;                                   // the inject workgroup is done
        }
#pragma unroll
        for (int t = 0; t < T; ++t) finish_row(t, v[t], sc[t]);
    } else {
#pragma unroll 1
        for (int t = 0; t < T; ++t) {
            float v[VPT];
            load_row(t, v);
            const float ss = sum_sq(v);
            if (lane == 0) s_red[w][0] = ss;
            __syncthreads();
            const float sc = 1.0f / sqrtf(waves_sum<NW>(s_red, 0) / (float) D + a.eps);
            __syncthreads();                          // s_red is reused below
            finish_row(t, v, sc);
        }
    }
    if (aux) return;                                   // workgroup-uniform
    __syncthreads();

    // 5. partial down dots of stream c's columns
    float acc[RPW][T];
#pragma unroll
    for (int s = 0; s < RPW; ++s)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[s][t] = 0.f;
#pragma unroll
    for (int i = 0; i < NBL; ++i) {
        const int b = lane + 64 * i;
        if (b >= NB) continue;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int4* xp = (const int4*) (s_xq + (size_t) t * D + (size_t) 32 * b);
            const int4 x0 = xp[0], x1 = xp[1];
            const float xs = s_xs[t * NB + b];
#pragma unroll
            for (int s = 0; s < RPW; ++s)
                acc[s][t] = fmaf(h16_to_f(sraw[i][s]) * xs, (float) (dot16(c0[i][s], x0) + dot16(c1[i][s], x1)),
                                 acc[s][t]);
        }
    }
    // all RPW x T sums in transposed reductions (the same sum tree for every T)
    float v[RPW * T];
#pragma unroll
    for (int s = 0; s < RPW; ++s)
#pragma unroll
        for (int t = 0; t < T; ++t) v[s * T + t] = acc[s][t];
    reduce_wave_store<RPW * T>(v, [&](int i, float tot) {
        const int s = i / T, t = i - (i / T) * T, r = row0 + s;
        if (r < L) a.lo_part[((size_t) t * HC4 + c) * L + r] = tot;
    });
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

    // every load first: weights, the residual / scale / norm inputs of xn, and the lo partials
    int4 c0[2], c1[2];
    uint32_t sraw[2];                // 16-bit scales in 32-bit registers (no packing that waits for the load)
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
    // inject partials of (row t, output o) for thread 256 - T*HC + t*HC + o, loaded by every thread
    // (clamped) so that workgroup 0 does not wait for them after its other loads
    float ipv[HC4];
    {
        const int j = max(0, tid - (256 - T * HC4)), t = j / HC4, o = j % HC4;
        const float* ip = a.inj_part + (size_t) t * HC4 * HC4 + o;
#pragma unroll
        for (int s = 0; s < HC4; ++s) ipv[s] = a.inj ? ip[s * HC4] : 0.f;
    }
    // lo partials: thread tid owns values 2*tid and 2*tid+1 of every row (16 threads per 32-block),
    // so the silu and the requantisation are spread over the whole workgroup
    const bool lo_thr = 2 * tid < L;
    const int lj = min(2 * tid, L - 2);
    float2 pv[T][HC4];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int s = 0; s < HC4; ++s) pv[t][s] = *(const float2*) (a.lo_part + ((size_t) t * HC4 + s) * L + lj);
#pragma unroll
    for (int t = 0; t < T; ++t) {
        float v[2];
        const float p0[2] = {pv[t][0].x, pv[t][0].y}, p1[2] = {pv[t][1].x, pv[t][1].y};
        const float p2[2] = {pv[t][2].x, pv[t][2].y}, p3[2] = {pv[t][3].x, pv[t][3].y};
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const float x = ((p0[j] + p1[j]) + (p2[j] + p3[j])) / (float) HC4;
            v[j] = x / (1.0f + __expf(-x));
        }
        const float am = group_max<16>(fmaxf(fabsf(v[0]), fabsf(v[1])));
        const float dq = am / 127.0f;
        const float inv = dq > 0.f ? 127.0f / am : 0.f;
        const int q0 = max(-127, min(127, rn_int(v[0] * inv))), q1 = max(-127, min(127, rn_int(v[1] * inv)));
        if (lo_thr) {
            *(uint16_t*) ((unsigned char*) &s_lq[t][0] + 2 * tid) = (uint16_t) ((q0 & 0xFF) | ((q1 & 0xFF) << 8));
            if ((tid & 15) == 0) s_ls[t][tid >> 4] = dq;
            if (blockIdx.x == 0 && a.lo) *(float2*) (a.lo + (size_t) t * L + 2 * tid) = make_float2(v[0], v[1]);
        }
    }
    if (blockIdx.x == 0 && a.inj && tid >= 256 - T * HC4) {   // summed inject of row t, output o
        const int j = tid - (256 - T * HC4), t = j / HC4, o = j % HC4;
        a.inj[t * HC4 + o] = (ipv[0] + ipv[1]) + (ipv[2] + ipv[3]);
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
constexpr int PRE_RPW = 2;

template <int T, int VPT, int NW>
void launch_pre_tv(const HcPreArgs& a, hipStream_t st) {
    constexpr int NBL = (2 * NW * VPT + 63) / 64;     // D/32 = 2*NW*VPT blocks over 64 lanes (D = 64*NW*VPT)
    const int nrb = (a.HCLR + NW * PRE_RPW - 1) / (NW * PRE_RPW);
    const size_t lds = (size_t) T * a.D + (size_t) T * (a.D / 32) * sizeof(float);
    hipLaunchKernelGGL((hc_pre_kernel<T, VPT, NBL, PRE_RPW, NW>), dim3(HC4 * (nrb + 1)), dim3(64 * NW), lds, st, a);
}
// (waves per workgroup, values per thread) of a stream width D: four waves when D/256 is a power of
// two (256 .. 4096), else five (D = 1280, 2560, 5120) or three (D = 768, 1536, 3072) waves
bool pre_shape(int D, int& nw, int& vpt) {
    for (int w : {4, 5, 3}) {
        if (D <= 0 || D % (64 * w)) continue;
        const int v = D / (64 * w);
        if (v == 1 || v == 2 || v == 4 || v == 8 || v == 16) {
            if (w != 4 && v < 4) continue;               // instantiated: 5 or 3 waves with 4, 8 or 16 values
            nw = w;
            vpt = v;
            return true;
        }
    }
    return false;
}
template <int T>
void launch_pre_t(const HcPreArgs& a, hipStream_t st) {
    int nw = 0, vpt = 0;
    pre_shape(a.D, nw, vpt);
    if (nw == 5) {
        switch (vpt) {
            case 4: launch_pre_tv<T, 4, 5>(a, st); break;
            case 8: launch_pre_tv<T, 8, 5>(a, st); break;
            default: launch_pre_tv<T, 16, 5>(a, st); break;
        }
    } else if (nw == 3) {
        switch (vpt) {
            case 4: launch_pre_tv<T, 4, 3>(a, st); break;
            case 8: launch_pre_tv<T, 8, 3>(a, st); break;
            default: launch_pre_tv<T, 16, 3>(a, st); break;
        }
    } else {
        switch (vpt) {
            case 1: launch_pre_tv<T, 1, 4>(a, st); break;
            case 2: launch_pre_tv<T, 2, 4>(a, st); break;
            case 4: launch_pre_tv<T, 4, 4>(a, st); break;
            case 8: launch_pre_tv<T, 8, 4>(a, st); break;
            default: launch_pre_tv<T, 16, 4>(a, st); break;
        }
    }
}
}  // namespace

size_t hc_workspace_bytes(int HC, int HCLR, int T) {
    return align_up((size_t) T * HC * HCLR * sizeof(float), 256) + align_up((size_t) T * HC * HC * sizeof(float), 256);
}
void hc_carve_workspace(void* ws, int HC, int HCLR, int T, float** lo_part, float** inj_part) {
    *lo_part = (float*) ws;
    *inj_part = (float*) ((char*) ws + align_up((size_t) T * HC * HCLR * sizeof(float), 256));
}

bool hc_width_supported(int D) {
    int nw = 0, vpt = 0;
    return pre_shape(D, nw, vpt);
}

int launch_hc_pre(const HcPreArgs& a, int T, hipStream_t st) {
    WZY_REQUIRE(T >= 1 && T <= WZY_MAX_W, "hc_pre: T out of range");
    int nw = 0, vpt = 0;
    WZY_REQUIRE(a.HC == HC4 && pre_shape(a.D, nw, vpt) &&
                    a.HCLR % 32 == 0 && a.HCLR >= 32 && a.HCLR <= 512,
                "hc_pre: unsupported shape (HC must be 4, D one of 256/512/768/1024/1280/1536/2048/2560/3072/4096/"
                "5120, HCLR a multiple of 32 <= 512)");
    WZY_REQUIRE((a.R_in != nullptr) + (a.emb_table != nullptr) + (a.emb_q != nullptr) + (a.emb_rows != nullptr) == 1,
                "hc_pre: exactly one of R_in / emb_table / emb_q / emb_rows");
    WZY_REQUIRE(!(a.emb_table || a.emb_q) || a.toks, "hc_pre: embedding mode needs toks");
    WZY_REQUIRE(!a.emb_q || a.emb_s, "hc_pre: a Q8_0 embedding table needs its scales");
    WZY_REQUIRE(!a.bo || a.inj_prev, "hc_pre: fold needs inj_prev");
    WZY_REQUIRE(a.R_out && a.norm_w && a.down_q && a.down_s && a.nsc && a.lo_part, "hc_pre: null pointer");
    WZY_REQUIRE(!a.inj_w || a.inj_part, "hc_pre: inject weights need an inj_part output");
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
    WZY_REQUIRE(a.HC == HC4 && a.HCLR % 32 == 0 && a.HCLR >= 32 && a.HCLR <= 512, "hc_post: unsupported shape");
    WZY_REQUIRE(a.R && a.nsc && a.norm_w && a.up_q && a.up_s && a.lo_part && a.mixed, "hc_post: null pointer");
    WZY_REQUIRE(!a.inj || a.inj_part, "hc_post: inj output needs inj_part");
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
extern "C" size_t wzy_hc_read_workspace_bytes(int HC, int HCLR, int T) { return hc_workspace_bytes(HC, HCLR, T); }

extern "C" int wzy_hc_read(const float* R_in, const uint16_t* emb_table, const int* toks, int n_vocab,
                           const float* bo, const float* inj_prev, float* R_out, const float* norm_w,
                           const int8_t* down_q, const uint16_t* down_s, const uint16_t* inj_w,
                           const int8_t* up_q, const uint16_t* up_s, float* nsc, float* lo, float* inj,
                           float* mixed, int D, int HC, int HCLR, float eps, int T, void* workspace,
                           size_t workspace_bytes, void* stream) {
    WZY_REQUIRE(workspace && workspace_bytes >= hc_workspace_bytes(HC, HCLR, T),
                "wzy_hc_read: workspace of wzy_hc_read_workspace_bytes() bytes required");
    WZY_REQUIRE(!inj_w || inj, "wzy_hc_read: inject weights need an inj output");
    HcPreArgs a{};
    a.R_in = R_in; a.emb_table = emb_table; a.toks = toks; a.n_vocab = n_vocab;
    a.bo = bo; a.inj_prev = inj_prev; a.R_out = R_out; a.norm_w = norm_w;
    a.down_q = down_q; a.down_s = down_s; a.inj_w = inj_w; a.nsc = nsc;
    hc_carve_workspace(workspace, HC, HCLR, T, &a.lo_part, &a.inj_part);
    a.D = D; a.HC = HC; a.HCLR = HCLR; a.eps = eps;
    hipStream_t st = as_stream(stream);
    WZY_TRY(launch_hc_pre(a, T, st));
    HcPostArgs b{};
    b.R = R_out; b.nsc = nsc; b.norm_w = norm_w; b.up_q = up_q; b.up_s = up_s; b.lo_part = a.lo_part;
    b.inj_part = inj_w ? a.inj_part : nullptr; b.lo = lo; b.inj = inj_w ? inj : nullptr; b.mixed = mixed;
    b.D = D; b.HC = HC; b.HCLR = HCLR;
    return launch_hc_post(b, T, st);
}

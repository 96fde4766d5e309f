// gemv.hip -- activation quantisation and the dense decode GEMVs (Q8_0 and bf16) for gfx950.
//
// GEMV shape: one 64-lane wave owns RPW*G consecutive output rows, G = 64/LPR rows at a time
// (LPR = lanes per row).  Every lane loads 16-32 contiguous weight bytes per row per step with
// 128-bit loads, all RPW rows' loads are issued before any arithmetic so each wave keeps
// RPW*16..32 bytes per lane in flight, and the T window rows reuse every weight load.
// Partial sums are reduced across the LPR lanes with DPP/swizzle (no LDS).
#include "wzy_device.h"
#include "wzy_gdn.h"
#include "wzy_gemv.h"
#include "wzy_host.h"

using namespace wzy;

// ---------------------------------------------------------------------------------------------
// quant_act: one thread per 32-value block, emits the two per-16 blocks and the per-32 block.
// reference: quant_act_multi (src/wzy_kernels_v2.cuh:58-107)
// ---------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) quant_act_kernel(const float* __restrict__ x, int8_t* __restrict__ q32,
                                                        float* __restrict__ s32, int8_t* __restrict__ q16,
                                                        float* __restrict__ s16, int n_blk32) {
    const int g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n_blk32) return;
    const float4* xp = (const float4*) (x + (size_t) g * 32);
    float v[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 f = xp[i];
        v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
    }
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) { a0 = fmaxf(a0, fabsf(v[i])); a1 = fmaxf(a1, fabsf(v[16 + i])); }
    if (q16) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float am = h ? a1 : a0;
            const float d = am / 127.0f;
            const float inv = d > 0.f ? 127.0f / am : 0.f;
            uint32_t w[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                uint32_t pk = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    int q = rn_int(v[16 * h + 4 * k + j] * inv);
                    q = max(-127, min(127, q));
                    pk |= (uint32_t) (q & 0xFF) << (8 * j);
                }
                w[k] = pk;
            }
            *(uint4*) (q16 + (size_t) g * 32 + 16 * h) = make_uint4(w[0], w[1], w[2], w[3]);
            s16[2 * g + h] = d;
        }
    }
    if (q32) {
        const float am = fmaxf(a0, a1);
        const float d = am / 127.0f;
        const float inv = d > 0.f ? 127.0f / am : 0.f;
        uint32_t w[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            uint32_t pk = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                int q = rn_int(v[4 * k + j] * inv);
                q = max(-127, min(127, q));
                pk |= (uint32_t) (q & 0xFF) << (8 * j);
            }
            w[k] = pk;
        }
        uint4* o = (uint4*) (q32 + (size_t) g * 32);
        o[0] = make_uint4(w[0], w[1], w[2], w[3]);
        o[1] = make_uint4(w[4], w[5], w[6], w[7]);
        s32[g] = d;
    }
}

namespace wzy {
int launch_quant_act(const float* x, int8_t* q32, float* s32, int8_t* q16, float* s16, int cols, int T,
                     hipStream_t st) {
    WZY_REQUIRE(x && cols > 0 && cols % 32 == 0 && T >= 1, "quant_act: cols must be a positive multiple of 32");
    WZY_REQUIRE((q32 == nullptr) == (s32 == nullptr) && (q16 == nullptr) == (s16 == nullptr),
                "quant_act: q/s outputs must be given in pairs");
    const int n = cols / 32 * T;
    hipLaunchKernelGGL(quant_act_kernel, dim3((n + 255) / 256), dim3(256), 0, st, x, q32, s32, q16, s16, n);
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}
}  // namespace wzy

// ---------------------------------------------------------------------------------------------
// Q8_0 GEMV.  reference: gemm_q8p_t / launch_gemm_q8p (src/wzy_kernels_v2.cuh:120-159,230-303):
// per 32-block b: acc += fp16(scale) * xs[b] * sum(codes*xq); then a cross-lane sum per row.
// ---------------------------------------------------------------------------------------------
template <int LPR>
WZY_DEV float seg_sum(float v) {
    if constexpr (LPR == 16) return sum16(v);
    else if constexpr (LPR == 32) return sum32(v);
    else return wave_sum(v);
}

template <int T, int LPR, int RPW>
__global__ void __launch_bounds__(256) gemv_q8_kernel(const int8_t* __restrict__ codes,
                                                      const uint16_t* __restrict__ scales,
                                                      const int8_t* __restrict__ xq, const float* __restrict__ xs,
                                                      float* __restrict__ y, int rows, int cols, int y_stride) {
    constexpr int G = 64 / LPR;
    const int lane = threadIdx.x & 63;
    const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int li = lane % LPR, gi = lane / LPR;
    const int nb = cols >> 5;
    const int row0 = wave * RPW * G + gi;
    float acc[RPW][T];
#pragma unroll
    for (int s = 0; s < RPW; ++s)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[s][t] = 0.f;

    for (int b = li; b < nb; b += LPR) {
        int4 c0[RPW], c1[RPW];
        float dw[RPW];
#pragma unroll
        for (int s = 0; s < RPW; ++s) {
            const int r = row0 + s * G;
            if (r < rows) {
                const int4* cp = (const int4*) (codes + (size_t) r * cols + (size_t) b * 32);
                c0[s] = ld_stream_i4(cp);
                c1[s] = ld_stream_i4(cp + 1);
                dw[s] = h16_to_f(scales[(size_t) r * nb + b]);
            } else {
                c0[s] = c1[s] = make_int4(0, 0, 0, 0);
                dw[s] = 0.f;
            }
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int4* xp = (const int4*) (xq + (size_t) t * cols + (size_t) b * 32);
            const int4 x0 = xp[0], x1 = xp[1];
            const float xsc = xs[(size_t) t * nb + b];
#pragma unroll
            for (int s = 0; s < RPW; ++s) {
                const int isum = dot16(c1[s], x1) + dot16(c0[s], x0);
                acc[s][t] = fmaf(dw[s] * xsc, (float) isum, acc[s][t]);
            }
        }
    }
#pragma unroll
    for (int s = 0; s < RPW; ++s) {
        const int r = row0 + s * G;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const float v = seg_sum<LPR>(acc[s][t]);
            if (li == 0 && r < rows) y[(size_t) t * y_stride + r] = v;
        }
    }
}

template <int T, int LPR, int RPW>
static void launch_q8_t(const int8_t* codes, const uint16_t* scales, const int8_t* xq, const float* xs, float* y,
                        int rows, int cols, int y_stride, hipStream_t st) {
    constexpr int rows_per_wave = RPW * (64 / LPR);
    const int waves = (rows + rows_per_wave - 1) / rows_per_wave;
    const int blocks = (waves + 3) / 4;
    hipLaunchKernelGGL((gemv_q8_kernel<T, LPR, RPW>), dim3(blocks), dim3(256), 0, st, codes, scales, xq, xs, y, rows,
                       cols, y_stride);
}

template <int T>
static void launch_q8_lpr(const int8_t* codes, const uint16_t* scales, const int8_t* xq, const float* xs, float* y,
                          int rows, int cols, int y_stride, hipStream_t st) {
    const int nb = cols / 32;
    if (nb >= 64) launch_q8_t<T, 64, 4>(codes, scales, xq, xs, y, rows, cols, y_stride, st);
    else if (nb > 16) launch_q8_t<T, 32, 2>(codes, scales, xq, xs, y, rows, cols, y_stride, st);
    else launch_q8_t<T, 16, 2>(codes, scales, xq, xs, y, rows, cols, y_stride, st);
}

namespace wzy {
int launch_gemv_q8(const int8_t* codes, const uint16_t* scales, const int8_t* xq, const float* xs, float* y, int rows,
                   int cols, int T, int y_stride, hipStream_t st) {
    WZY_REQUIRE(codes && scales && xq && xs && y, "gemv_q8: null pointer");
    WZY_REQUIRE(rows > 0 && cols > 0 && cols % 32 == 0, "gemv_q8: rows > 0 and cols %% 32 == 0 required");
    WZY_REQUIRE(T >= 1 && T <= WZY_MAX_W, "gemv_q8: T must be in [1, %d]", WZY_MAX_W);
    if (y_stride == 0) y_stride = rows;
    switch (T) {
        case 1: launch_q8_lpr<1>(codes, scales, xq, xs, y, rows, cols, y_stride, st); break;
        case 2: launch_q8_lpr<2>(codes, scales, xq, xs, y, rows, cols, y_stride, st); break;
        case 3: launch_q8_lpr<3>(codes, scales, xq, xs, y, rows, cols, y_stride, st); break;
        case 4: launch_q8_lpr<4>(codes, scales, xq, xs, y, rows, cols, y_stride, st); break;
        case 5: launch_q8_lpr<5>(codes, scales, xq, xs, y, rows, cols, y_stride, st); break;
        case 6: launch_q8_lpr<6>(codes, scales, xq, xs, y, rows, cols, y_stride, st); break;
        case 7: launch_q8_lpr<7>(codes, scales, xq, xs, y, rows, cols, y_stride, st); break;
        default: launch_q8_lpr<8>(codes, scales, xq, xs, y, rows, cols, y_stride, st); break;
    }
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}
}  // namespace wzy

// ---------------------------------------------------------------------------------------------
// bf16 GEMV.  reference: gemm_bf16_t / launch_gemm_bf16 (src/wzy_kernels_v2.cuh:307-387).
// Optional extra row (Wx, yx): handled as row `rows`, written to yx[t] (used for the shared-expert
// gate row next to the router).
// ---------------------------------------------------------------------------------------------
template <int T, int RPW>
__global__ void __launch_bounds__(256) gemv_bf16_kernel(const uint16_t* __restrict__ W, const float* __restrict__ x,
                                                        float* __restrict__ y, int rows, int cols, int y_stride,
                                                        const uint16_t* __restrict__ Wx, float* __restrict__ yx) {
    const int lane = threadIdx.x & 63;
    const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int n8 = cols >> 3;
    const int row0 = wave * RPW;
    const int rows_tot = rows + (Wx ? 1 : 0);
    float acc[RPW][T];
#pragma unroll
    for (int s = 0; s < RPW; ++s)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[s][t] = 0.f;

    for (int j = lane; j < n8; j += 64) {
        uint4 w[RPW];
#pragma unroll
        for (int s = 0; s < RPW; ++s) {
            const int r = row0 + s;
            if (r < rows) w[s] = ld_stream_u4((const uint4*) (W + (size_t) r * cols) + j);
            else if (r < rows_tot) w[s] = ((const uint4*) Wx)[j];
            else w[s] = make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const float4 xa = *(const float4*) (x + (size_t) t * cols + j * 8);
            const float4 xb = *(const float4*) (x + (size_t) t * cols + j * 8 + 4);
#pragma unroll
            for (int s = 0; s < RPW; ++s) {
                float a = acc[s][t];
                a = fmaf(bf16_lo(w[s].x), xa.x, a);
                a = fmaf(bf16_hi(w[s].x), xa.y, a);
                a = fmaf(bf16_lo(w[s].y), xa.z, a);
                a = fmaf(bf16_hi(w[s].y), xa.w, a);
                a = fmaf(bf16_lo(w[s].z), xb.x, a);
                a = fmaf(bf16_hi(w[s].z), xb.y, a);
                a = fmaf(bf16_lo(w[s].w), xb.z, a);
                a = fmaf(bf16_hi(w[s].w), xb.w, a);
                acc[s][t] = a;
            }
        }
    }
#pragma unroll
    for (int s = 0; s < RPW; ++s) {
        const int r = row0 + s;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const float v = wave_sum(acc[s][t]);
            if (lane == 0) {
                if (r < rows) y[(size_t) t * y_stride + r] = v;
                else if (r < rows_tot) yx[t] = v;
            }
        }
    }
}

template <int T>
static void launch_bf16_t(const uint16_t* W, const float* x, float* y, int rows, int cols, int y_stride,
                          const uint16_t* Wx, float* yx, hipStream_t st) {
    constexpr int RPW = 4;
    const int rows_tot = rows + (Wx ? 1 : 0);
    const int waves = (rows_tot + RPW - 1) / RPW;
    const int blocks = (waves + 3) / 4;
    hipLaunchKernelGGL((gemv_bf16_kernel<T, RPW>), dim3(blocks), dim3(256), 0, st, W, x, y, rows, cols, y_stride, Wx,
                       yx);
}

namespace wzy {
int launch_gemv_bf16(const uint16_t* W, const float* x, float* y, int rows, int cols, int T, int y_stride,
                     const uint16_t* Wx, float* yx, hipStream_t st) {
    WZY_REQUIRE(W && x && y, "gemv_bf16: null pointer");
    WZY_REQUIRE(rows > 0 && cols > 0 && cols % 8 == 0, "gemv_bf16: rows > 0 and cols %% 8 == 0 required");
    WZY_REQUIRE(T >= 1 && T <= WZY_MAX_W, "gemv_bf16: T must be in [1, %d]", WZY_MAX_W);
    WZY_REQUIRE((Wx == nullptr) == (yx == nullptr), "gemv_bf16: extra row needs both Wx and yx");
    if (y_stride == 0) y_stride = rows;
    switch (T) {
        case 1: launch_bf16_t<1>(W, x, y, rows, cols, y_stride, Wx, yx, st); break;
        case 2: launch_bf16_t<2>(W, x, y, rows, cols, y_stride, Wx, yx, st); break;
        case 3: launch_bf16_t<3>(W, x, y, rows, cols, y_stride, Wx, yx, st); break;
        case 4: launch_bf16_t<4>(W, x, y, rows, cols, y_stride, Wx, yx, st); break;
        case 5: launch_bf16_t<5>(W, x, y, rows, cols, y_stride, Wx, yx, st); break;
        case 6: launch_bf16_t<6>(W, x, y, rows, cols, y_stride, Wx, yx, st); break;
        case 7: launch_bf16_t<7>(W, x, y, rows, cols, y_stride, Wx, yx, st); break;
        default: launch_bf16_t<8>(W, x, y, rows, cols, y_stride, Wx, yx, st); break;
    }
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}
}  // namespace wzy

// ---------------------------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------------------------
extern "C" int wzy_quant_act(const float* x, int8_t* q32, float* s32, int8_t* q16, float* s16, int cols, int T,
                             void* stream) {
    return launch_quant_act(x, q32, s32, q16, s16, cols, T, as_stream(stream));
}
extern "C" int wzy_gemv_q8(const int8_t* codes, const uint16_t* scales, const int8_t* xq, const float* xs, float* y,
                           int rows, int cols, int T, int y_stride, void* stream) {
    return launch_gemv_q8(codes, scales, xq, xs, y, rows, cols, T, y_stride, as_stream(stream));
}
extern "C" int wzy_gemv_bf16(const uint16_t* W, const float* x, float* y, int rows, int cols, int T, int y_stride,
                             void* stream) {
    return launch_gemv_bf16(W, x, y, rows, cols, T, y_stride, nullptr, nullptr, as_stream(stream));
}

// ---------------------------------------------------------------------------------------------
// Multi-segment GEMV over fp32 activations (projection groups: GDN qkv|z|alpha|beta, QSA
// q|k|v|idx_k|idx_q, router|sgate, out-projections).  Q8_0 segments quantise x per 32 inside the
// lane (same float operations as quant_act), so no separate quantisation launch is needed.
// ---------------------------------------------------------------------------------------------
namespace {
WZY_DEV void quant32_v(const float4 (&xv)[8], int4& q0, int4& q1, float& d) {
    float v[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        v[4 * i] = xv[i].x; v[4 * i + 1] = xv[i].y; v[4 * i + 2] = xv[i].z; v[4 * i + 3] = xv[i].w;
    }
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
        for (int j = 0; j < 4; ++j) pk |= (uint32_t) (max(-127, min(127, rn_int(v[4 * k + j] * inv))) & 0xFF) << (8 * j);
        w[k] = (int) pk;
    }
    q0 = make_int4(w[0], w[1], w[2], w[3]);
    q1 = make_int4(w[4], w[5], w[6], w[7]);
}
WZY_DEV void quant32_f(const float* __restrict__ xp, int4& q0, int4& q1, float& d) {
    float v[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 f = ((const float4*) xp)[i];
        v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
    }
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
        for (int j = 0; j < 4; ++j) pk |= (uint32_t) (max(-127, min(127, rn_int(v[4 * k + j] * inv))) & 0xFF) << (8 * j);
        w[k] = (int) pk;
    }
    q0 = make_int4(w[0], w[1], w[2], w[3]);
    q1 = make_int4(w[4], w[5], w[6], w[7]);
}
// The segment that owns (wave-uniform) `wave`, chosen by selects over the kernel-argument copy so
// that every field comes from scalar loads issued at kernel entry: a dynamically indexed
// segs.seg[si] would be read with dependent vector loads before the first weight load.
__device__ __forceinline__ GemvSeg pick_seg(const GemvSegs& segs, int wave) {
    GemvSeg sg = segs.seg[0];
#pragma unroll
    for (int i = 1; i < GEMV_MAX_SEGS; ++i) {
        const bool take = (i < segs.n) & (wave >= segs.seg[i].wave0);
        sg.w = take ? segs.seg[i].w : sg.w;
        sg.s = take ? segs.seg[i].s : sg.s;
        sg.y = take ? segs.seg[i].y : sg.y;
        sg.rows = take ? segs.seg[i].rows : sg.rows;
        sg.kind = take ? segs.seg[i].kind : sg.kind;
        sg.y_stride = take ? segs.seg[i].y_stride : sg.y_stride;
        sg.wave0 = take ? segs.seg[i].wave0 : sg.wave0;
        sg.act = take ? segs.seg[i].act : sg.act;
    }
    return sg;
}
}  // namespace

template <int T, int NBL, int RPW>
__global__ void __launch_bounds__(256) gemv_segs_kernel(GemvSegs segs, const float* __restrict__ x, int cols) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const GemvSeg sg = pick_seg(segs, wave);
    const int row0 = (wave - sg.wave0) * RPW;
    if (row0 >= sg.rows) return;
    float acc[RPW][T];
#pragma unroll
    for (int s = 0; s < RPW; ++s)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[s][t] = 0.f;

    if (sg.kind == GEMV_Q8) {
        // Every load is issued before any of its results is used (indices are clamped into the
        // matrix instead of branching, and the fp16 scales are converted afterwards), so the
        // wave has all its weight bytes in flight at once.
        const int nb = cols >> 5;
        const int8_t* W = (const int8_t*) sg.w;
        int4 c0[NBL][RPW], c1[NBL][RPW];
        uint32_t sraw[NBL][RPW];     // 16-bit scales held in 32-bit registers (no packing that waits for the load)
#pragma unroll
        for (int i = 0; i < NBL; ++i) {
            const int b = min(lane + 64 * i, nb - 1);
#pragma unroll
            for (int s = 0; s < RPW; ++s) {
                const int r = min(row0 + s, sg.rows - 1);
                const int4* cp = (const int4*) (W + (size_t) r * cols + (size_t) b * 32);
                c0[i][s] = ld_stream_i4(cp);
                c1[i][s] = ld_stream_i4(cp + 1);
                sraw[i][s] = sg.s[(size_t) r * nb + b];
            }
        }
        // single-row windows: the activations' loads join the weights' in flight
        constexpr int TX = (T == 1) ? NBL : 1;
        float4 xv[TX][8];
        if (T == 1) {
#pragma unroll
            for (int i = 0; i < TX; ++i) {
                const int b = min(lane + 64 * i, nb - 1);
#pragma unroll
                for (int k = 0; k < 8; ++k) xv[i][k] = ((const float4*) (x + (size_t) b * 32))[k];
            }
        }
#pragma unroll
        for (int i = 0; i < NBL; ++i) {
            if (lane + 64 * i >= nb) continue;
#pragma unroll
            for (int t = 0; t < T; ++t) {
                int4 x0, x1;
                float xs;
                if (T == 1) quant32_v(xv[T == 1 ? i : 0], x0, x1, xs);
                else quant32_f(x + (size_t) t * cols + (size_t) (lane + 64 * i) * 32, x0, x1, xs);
#pragma unroll
                for (int s = 0; s < RPW; ++s)
                    acc[s][t] = fmaf(h16_to_f(sraw[i][s]) * xs, (float) (dot16(c1[i][s], x1) + dot16(c0[i][s], x0)),
                                     acc[s][t]);
            }
        }
    } else {
        const uint16_t* W = (const uint16_t*) sg.w;
        const int n8 = cols >> 3;
        for (int j0 = 0; j0 < n8; j0 += 64 * 4) {
            // all loads first (clamped indices, no branches), then the arithmetic
            uint4 wv[4][RPW];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int j = min(j0 + lane + 64 * u, n8 - 1);
#pragma unroll
                for (int s = 0; s < RPW; ++s) {
                    const int r = min(row0 + s, sg.rows - 1);
                    wv[u][s] = ld_stream_u4((const uint4*) (W + (size_t) r * cols) + j);
                }
            }
            constexpr int TX = (T == 1) ? 4 : 1;
            float4 xr[TX][2];
            if (T == 1) {
#pragma unroll
                for (int u = 0; u < TX; ++u) {
                    const int j = min(j0 + lane + 64 * u, n8 - 1);
                    xr[u][0] = *(const float4*) (x + j * 8);
                    xr[u][1] = *(const float4*) (x + j * 8 + 4);
                }
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int j = j0 + lane + 64 * u;
                if (j >= n8) continue;
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    const float4 xa = T == 1 ? xr[T == 1 ? u : 0][0] : *(const float4*) (x + (size_t) t * cols + j * 8);
                    const float4 xb = T == 1 ? xr[T == 1 ? u : 0][1] : *(const float4*) (x + (size_t) t * cols + j * 8 + 4);
#pragma unroll
                    for (int s = 0; s < RPW; ++s) {
                        float a = acc[s][t];
                        a = fmaf(bf16_lo(wv[u][s].x), xa.x, a);
                        a = fmaf(bf16_hi(wv[u][s].x), xa.y, a);
                        a = fmaf(bf16_lo(wv[u][s].y), xa.z, a);
                        a = fmaf(bf16_hi(wv[u][s].y), xa.w, a);
                        a = fmaf(bf16_lo(wv[u][s].z), xb.x, a);
                        a = fmaf(bf16_hi(wv[u][s].z), xb.y, a);
                        a = fmaf(bf16_lo(wv[u][s].w), xb.z, a);
                        a = fmaf(bf16_hi(wv[u][s].w), xb.w, a);
                        acc[s][t] = a;
                    }
                }
            }
        }
    }
#pragma unroll
    for (int s = 0; s < RPW; ++s) {
        const int r = row0 + s;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const float v = wave_sum(acc[s][t]);
            if (lane == 0 && r < sg.rows) sg.y[(size_t) t * sg.y_stride + r] = sg.act == GEMV_ACT_SIGMOID ? gdn_gate(v) : v;
        }
    }
}

// Same GEMV with the activations staged once per workgroup in LDS: the fp32 rows (for bf16
// segments, split into the two float4 halves of each 8-column group) and their per-32 int8
// quantisation (for Q8_0 segments, split into the two 16-byte halves of each block), so lanes
// read 16 consecutive bytes each (no LDS bank conflicts) and the L2 serves x once per workgroup
// instead of once per wave.  Each wave issues its weight loads before the staging barrier.
// Registers are kept low so that every workgroup of a launch is resident at once: Q8_0 and bf16
// weights share one array (a Q8_0 wave holds RPW rows of 32 code bytes per 32-block, a bf16 wave
// RPW/2 rows of 64 bytes), and x is staged by four threads per 32-column block (8 values each).
// flags: bit 0 = the launch has Q8_0 segments, bit 1 = it has bf16 segments.  GDN: the staging
// applies segs.gdn (the GDN output norm and gate) to x.
template <int T, int NBL, int RPW, bool GDN>
__global__ void __launch_bounds__(256) gemv_segs_lds_kernel(GemvSegs segs, const float* __restrict__ x, int cols,
                                                            int flags) {
    static_assert(RPW % 2 == 0, "a bf16 wave holds RPW/2 rows");
    constexpr int RPWB = RPW / 2;
    constexpr int NR = 2 * NBL * RPW;                 // uint4 weight registers per lane
    extern __shared__ __align__(16) unsigned char s_dyn[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane((blockIdx.x * blockDim.x + tid) >> 6);
    const int nb = cols >> 5, n8 = cols >> 3;
    float4* s_xf = (float4*) s_dyn;                                            // [T][2][n8]
    int4* s_xq = (int4*) (s_dyn + ((flags & 2) ? (size_t) T * cols * 4 : 0));  // [T][2][nb]
    float* s_xs = (float*) ((unsigned char*) s_xq + ((flags & 1) ? (size_t) T * cols : 0));   // [T][nb]
    const GemvSeg sg = pick_seg(segs, wave);
    const bool q8 = sg.kind == GEMV_Q8;
    const int row0 = (wave - sg.wave0) * (q8 ? RPW : RPWB);
    const bool active = row0 < sg.rows;

    // 1. weights (wave-uniform branches; clamped indices; raw scales).  Q8_0: wr[2*(i*RPW+s)+h] =
    //    half h of 32-block lane+64i of row row0+s.  bf16: wr[u*RPWB+s] = 8 columns 8*(lane+64u).. of
    //    row row0+s.
    uint4 wr[NR];
    uint32_t sraw[NBL][RPW];         // 16-bit scales held in 32-bit registers (no packing that waits for the load)
    if (active && q8) {
        const int8_t* W = (const int8_t*) sg.w;
#pragma unroll
        for (int i = 0; i < NBL; ++i) {
            const int b = min(lane + 64 * i, nb - 1);
#pragma unroll
            for (int s = 0; s < RPW; ++s) {
                const int r = min(row0 + s, sg.rows - 1);
                const uint4* cp = (const uint4*) (W + (size_t) r * cols + (size_t) b * 32);
                wr[2 * (i * RPW + s)] = ld_stream_u4(cp);
                wr[2 * (i * RPW + s) + 1] = ld_stream_u4(cp + 1);
                sraw[i][s] = sg.s[(size_t) r * nb + b];
            }
        }
    } else if (active) {
        const uint16_t* W = (const uint16_t*) sg.w;
#pragma unroll
        for (int u = 0; u < 4 * NBL; ++u) {
            const int j = min(lane + 64 * u, n8 - 1);
#pragma unroll
            for (int s = 0; s < RPWB; ++s) {
                const int r = min(row0 + s, sg.rows - 1);
                wr[u * RPWB + s] = ld_stream_u4((const uint4*) (W + (size_t) r * cols) + j);
            }
        }
    }
    // 2. stage x: four threads per 32-column block, thread k of block b holding columns 32b+8k ..
    //    32b+8k+7.  The first item is loaded in straight-line code right behind the weights
    //    (clamped: always a valid address), so both are in flight together; a loop here would wait
    //    for the weights at its header before loading x.  Only windows of more than one row loop.
    const int nitem = T * nb * 4;
    auto stage = [&](const float4& va, const float4& vb, int i) {
        const int t = i / (nb * 4), r = i - t * (nb * 4), b = r >> 2, k = r & 3;
        if (flags & 2) {
            s_xf[((size_t) t * 2 + 0) * n8 + 4 * b + k] = va;
            s_xf[((size_t) t * 2 + 1) * n8 + 4 * b + k] = vb;
        }
        if (flags & 1) {
            // per-32 quantisation (d = amax/127, q = rint(x*127/amax)); the 4 threads of a block are
            // 4 consecutive lanes, so the block max is a 4-lane DPP max
            const float v[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w};
            float am = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) am = fmaxf(am, fabsf(v[j]));
            am = fmaxf(am, dpp_f<DPP_XOR1>(am));
            am = fmaxf(am, dpp_f<DPP_XOR2>(am));
            const float d = am / 127.0f;
            const float inv = d > 0.f ? 127.0f / am : 0.f;
            uint32_t pk[2] = {0u, 0u};
#pragma unroll
            for (int j = 0; j < 8; ++j)
                pk[j >> 2] |= (uint32_t) (max(-127, min(127, rn_int(v[j] * inv))) & 0xFF) << (8 * (j & 3));
            int2* dst = (int2*) &s_xq[((size_t) t * 2 + (k >> 1)) * nb + b] + (k & 1);
            *dst = make_int2((int) pk[0], (int) pk[1]);
            if (k == 0) s_xs[(size_t) t * nb + b] = d;
        }
    };
    // GDN staging transform: x = gdn_norm_gate(o, ss, z, gamma) element-wise (8 columns of one head
    // per item).  Absent z / gamma read x instead (loads stay unconditional) and are replaced by the
    // neutral values after the load.
    const GemvGdnIn& gn = segs.gdn;
    auto gdn_apply = [&](float4& va, float4& vb, float4 za, float4 zb, float4 ga, float4 gb, const float4& ssv) {
        const float ss[4] = {ssv.x, ssv.y, ssv.z, ssv.w};
        const float sc = gdn_norm_scale(ss, gn.eps);  // one head per item: one scale
        if (!gn.gamma) ga = gb = make_float4(1.f, 1.f, 1.f, 1.f);
        auto gate = [&](float z) { return !gn.z ? 1.0f : (gn.z_is_gate ? z : gdn_gate(z)); };
        va = make_float4(va.x * sc * ga.x * gate(za.x), va.y * sc * ga.y * gate(za.y), va.z * sc * ga.z * gate(za.z),
                         va.w * sc * ga.w * gate(za.w));
        vb = make_float4(vb.x * sc * gb.x * gate(zb.x), vb.y * sc * gb.y * gate(zb.y), vb.z * sc * gb.z * gate(zb.z),
                         vb.w * sc * gb.w * gate(zb.w));
    };
    // the transform's inputs of item (t, r): z at the same place, gamma at column (8r) % 128,
    // the partial sums of head (8r) / 128
    auto gdn_load = [&](int t, int r, float4& za, float4& zb, float4& ga, float4& gb, float4& ssv) {
        const float4* zp = (const float4*) ((gn.z ? gn.z : x) + (size_t) t * cols + (size_t) r * 8);
        za = zp[0];
        zb = zp[1];
        const float4* gp = (const float4*) ((gn.gamma ? gn.gamma : x) + (r * 8) % 128);
        ga = gp[0];
        gb = gp[1];
        ssv = *(const float4*) (gn.ss + ((size_t) t * (cols / 128) + (r * 8) / 128) * GDN_NQ);
    };
    // NX items per thread in straight-line code: NBL cover one row (nb*4 <= 256*NBL), so windows of
    // up to 8 / NBL rows are staged with every x load in flight at once; nitem % 4 == 0, so a 4-lane
    // group is all in or all out
    constexpr int NX = (T * NBL <= 8) ? T * NBL : NBL;
    {
        float4 xa[NX], xb[NX];
#pragma unroll
        for (int k = 0; k < NX; ++k) {
            const int i = min(tid + 256 * k, nitem - 1);
            const int t = i / (nb * 4), r = i - t * (nb * 4);
            const float4* xp = (const float4*) (x + (size_t) t * cols + (size_t) r * 8);
            xa[k] = xp[0];
            xb[k] = xp[1];
        }
        if constexpr (GDN) {
            float4 za[NX], zb[NX], ga[NX], gb[NX], ssv[NX];
#pragma unroll
            for (int k = 0; k < NX; ++k) {
                const int i = min(tid + 256 * k, nitem - 1);
                const int t = i / (nb * 4), r = i - t * (nb * 4);
                gdn_load(t, r, za[k], zb[k], ga[k], gb[k], ssv[k]);
            }
#pragma unroll
            for (int k = 0; k < NX; ++k) gdn_apply(xa[k], xb[k], za[k], zb[k], ga[k], gb[k], ssv[k]);
        }
#pragma unroll
        for (int k = 0; k < NX; ++k)
            if (tid + 256 * k < nitem) stage(xa[k], xb[k], tid + 256 * k);
    }
    if (nitem > 256 * NX) {
        for (int i = tid + 256 * NX; i < nitem; i += 256) {
            const int t = i / (nb * 4), r = i - t * (nb * 4);
            const float4* xp = (const float4*) (x + (size_t) t * cols + (size_t) r * 8);
            float4 va = xp[0], vb = xp[1];
            if constexpr (GDN) {
                float4 za, zb, ga, gb, ssv;
                gdn_load(t, r, za, zb, ga, gb, ssv);
                gdn_apply(va, vb, za, zb, ga, gb, ssv);
            }
            stage(va, vb, i);
        }
    }
    __syncthreads();
    if (!active) return;
    // Pin the raw scales here: without this the compiler converts them inside the load branch,
    // which waits for the loads before the rest are issued.
#pragma unroll
    for (int i = 0; i < NBL; ++i)
#pragma unroll
        for (int s = 0; s < RPW; ++s) asm volatile("" : "+v"(sraw[i][s]));

    float acc[RPW][T];
#pragma unroll
    for (int s = 0; s < RPW; ++s)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[s][t] = 0.f;
    if (q8) {
#pragma unroll
        for (int i = 0; i < NBL; ++i) {
            const int b = lane + 64 * i;
            if (b >= nb) continue;
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const int4 x0 = s_xq[((size_t) t * 2 + 0) * nb + b], x1 = s_xq[((size_t) t * 2 + 1) * nb + b];
                const float xs = s_xs[(size_t) t * nb + b];
#pragma unroll
                for (int s = 0; s < RPW; ++s) {
                    const uint4 a0 = wr[2 * (i * RPW + s)], a1 = wr[2 * (i * RPW + s) + 1];
                    const int4 c0 = make_int4((int) a0.x, (int) a0.y, (int) a0.z, (int) a0.w);
                    const int4 c1 = make_int4((int) a1.x, (int) a1.y, (int) a1.z, (int) a1.w);
                    acc[s][t] = fmaf(h16_to_f(sraw[i][s]) * xs, (float) (dot16(c1, x1) + dot16(c0, x0)), acc[s][t]);
                }
            }
        }
    } else {
#pragma unroll
        for (int u = 0; u < 4 * NBL; ++u) {
            const int j = lane + 64 * u;
            if (j >= n8) continue;
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const float4 xa = s_xf[((size_t) t * 2 + 0) * n8 + j], xb = s_xf[((size_t) t * 2 + 1) * n8 + j];
#pragma unroll
                for (int s = 0; s < RPWB; ++s) {
                    const uint4 wv = wr[u * RPWB + s];
                    float v = acc[s][t];
                    v = fmaf(bf16_lo(wv.x), xa.x, v);
                    v = fmaf(bf16_hi(wv.x), xa.y, v);
                    v = fmaf(bf16_lo(wv.y), xa.z, v);
                    v = fmaf(bf16_hi(wv.y), xa.w, v);
                    v = fmaf(bf16_lo(wv.z), xb.x, v);
                    v = fmaf(bf16_hi(wv.z), xb.y, v);
                    v = fmaf(bf16_lo(wv.w), xb.z, v);
                    v = fmaf(bf16_hi(wv.w), xb.w, v);
                    acc[s][t] = v;
                }
            }
        }
    }
    const int rpw = q8 ? RPW : RPWB;
    // all RPW x T sums in transposed reductions (the same sum tree for every T, so a window row's
    // outputs equal a one-row launch's bit for bit)
    float v[RPW * T];
#pragma unroll
    for (int s = 0; s < RPW; ++s)
#pragma unroll
        for (int t = 0; t < T; ++t) v[s * T + t] = acc[s][t];
    reduce_wave_store<RPW * T>(v, [&](int i, float tot) {
        const int s = i / T, t = i - (i / T) * T, r = row0 + s;
        if (s < rpw && r < sg.rows) sg.y[(size_t) t * sg.y_stride + r] = sg.act == GEMV_ACT_SIGMOID ? gdn_gate(tot) : tot;
    });
}

template <int T>
static void launch_segs_lds_t(const GemvSegs& segs, int waves, int nbl, int rpw, const float* x, int cols, int flags,
                              size_t lds, hipStream_t st) {
    const int blocks = (waves + 3) / 4;
    if (nbl == 1 && rpw == 2) {          // a small projection spread over more workgroups
        if (segs.gdn.ss)
            hipLaunchKernelGGL((gemv_segs_lds_kernel<T, 1, 2, true>), dim3(blocks), dim3(256), lds, st, segs, x, cols, flags);
        else
            hipLaunchKernelGGL((gemv_segs_lds_kernel<T, 1, 2, false>), dim3(blocks), dim3(256), lds, st, segs, x, cols, flags);
        return;
    }
    if (segs.gdn.ss) {
        switch (nbl) {
            case 1: hipLaunchKernelGGL((gemv_segs_lds_kernel<T, 1, 4, true>), dim3(blocks), dim3(256), lds, st, segs, x, cols, flags); break;
            case 2: hipLaunchKernelGGL((gemv_segs_lds_kernel<T, 2, 2, true>), dim3(blocks), dim3(256), lds, st, segs, x, cols, flags); break;
            case 3: hipLaunchKernelGGL((gemv_segs_lds_kernel<T, 3, 2, true>), dim3(blocks), dim3(256), lds, st, segs, x, cols, flags); break;
            default: hipLaunchKernelGGL((gemv_segs_lds_kernel<T, 4, 2, true>), dim3(blocks), dim3(256), lds, st, segs, x, cols, flags); break;
        }
        return;
    }
    switch (nbl) {
        case 1: hipLaunchKernelGGL((gemv_segs_lds_kernel<T, 1, 4, false>), dim3(blocks), dim3(256), lds, st, segs, x, cols, flags); break;
        case 2: hipLaunchKernelGGL((gemv_segs_lds_kernel<T, 2, 2, false>), dim3(blocks), dim3(256), lds, st, segs, x, cols, flags); break;
        case 3: hipLaunchKernelGGL((gemv_segs_lds_kernel<T, 3, 2, false>), dim3(blocks), dim3(256), lds, st, segs, x, cols, flags); break;
        default: hipLaunchKernelGGL((gemv_segs_lds_kernel<T, 4, 2, false>), dim3(blocks), dim3(256), lds, st, segs, x, cols, flags); break;
    }
}

template <int T>
static void launch_segs_t(const GemvSegs& segs, int waves, int nbl, const float* x, int cols, hipStream_t st) {
    const int blocks = (waves + 3) / 4;
    switch (nbl) {
        case 1: hipLaunchKernelGGL((gemv_segs_kernel<T, 1, 4>), dim3(blocks), dim3(256), 0, st, segs, x, cols); break;
        case 2: hipLaunchKernelGGL((gemv_segs_kernel<T, 2, 2>), dim3(blocks), dim3(256), 0, st, segs, x, cols); break;
        case 3: hipLaunchKernelGGL((gemv_segs_kernel<T, 3, 2>), dim3(blocks), dim3(256), 0, st, segs, x, cols); break;
        default: hipLaunchKernelGGL((gemv_segs_kernel<T, 4, 1>), dim3(blocks), dim3(256), 0, st, segs, x, cols); break;
    }
}

namespace wzy {
constexpr int GEMV_FILL_WGS = 256;      // one workgroup per CU of an MI355X

int launch_gemv_segs(GemvSegs segs, const float* x, int cols, int T, hipStream_t st) {
    WZY_REQUIRE(x && segs.n >= 1 && segs.n <= GEMV_MAX_SEGS, "gemv_segs: bad segment list");
    WZY_REQUIRE(cols >= 32 && cols % 32 == 0 && cols <= 8192, "gemv_segs: cols must be a multiple of 32 in [32, 8192]");
    WZY_REQUIRE(T >= 1 && T <= WZY_MAX_W, "gemv_segs: T out of range");
    const int nbl = (cols / 32 + 63) / 64;
    int flags = 0;
    for (int i = 0; i < segs.n; ++i) flags |= segs.seg[i].kind == GEMV_Q8 ? 1 : 2;
    const size_t lds = (size_t) T * cols * (((flags & 2) ? 4 : 0) + ((flags & 1) ? 1 : 0)) +
                       ((flags & 1) ? (size_t) T * (cols / 32) * 4 : 0);
    // gfx950 gives a workgroup up to 160 KB of LDS: every window size of the decode projections (up to
    // 8 rows of 2,048 columns of both kinds, 8,192 of Q8_0) stays on this kernel, so a window row
    // computes what a one-row launch does
    const bool use_lds = lds <= 96 * 1024;
    WZY_REQUIRE(!segs.gdn.ss || (use_lds && cols % 128 == 0), "gemv_segs: the GDN staging transform needs the LDS path");
    // rows per wave: the LDS kernel holds RPW Q8_0 rows or RPW/2 bf16 rows per wave (RPW = 4 for one
    // 32-block per lane, else 2; 2 also when 4 would leave CUs without a workgroup); the other kernel
    // RPW rows of either kind (4 / 2 / 1)
    int rpw = nbl == 1 ? 4 : (use_lds || nbl <= 3 ? 2 : 1);
    auto count_waves = [&](int rp) {
        int wv = 0;
        for (int i = 0; i < segs.n; ++i) {
            const GemvSeg& s = segs.seg[i];
            const int r = (use_lds && s.kind == GEMV_BF16) ? rp / 2 : rp;
            wv += (s.rows + r - 1) / r;
        }
        return wv;
    };
    if (use_lds && nbl == 1 && (count_waves(4) + 3) / 4 < GEMV_FILL_WGS) rpw = 2;
    int waves = 0;
    for (int i = 0; i < segs.n; ++i) {
        GemvSeg& s = segs.seg[i];
        WZY_REQUIRE(s.w && s.y && s.rows > 0, "gemv_segs: segment %d incomplete", i);
        WZY_REQUIRE(s.kind == GEMV_BF16 || s.s, "gemv_segs: Q8 segment %d without scales", i);
        if (s.y_stride == 0) s.y_stride = s.rows;
        s.wave0 = waves;
        const int r = (use_lds && s.kind == GEMV_BF16) ? rpw / 2 : rpw;
        waves += (s.rows + r - 1) / r;
    }
    if (use_lds) {
        switch (T) {
            case 1: launch_segs_lds_t<1>(segs, waves, nbl, rpw, x, cols, flags, lds, st); break;
            case 2: launch_segs_lds_t<2>(segs, waves, nbl, rpw, x, cols, flags, lds, st); break;
            case 3: launch_segs_lds_t<3>(segs, waves, nbl, rpw, x, cols, flags, lds, st); break;
            case 4: launch_segs_lds_t<4>(segs, waves, nbl, rpw, x, cols, flags, lds, st); break;
            case 5: launch_segs_lds_t<5>(segs, waves, nbl, rpw, x, cols, flags, lds, st); break;
            case 6: launch_segs_lds_t<6>(segs, waves, nbl, rpw, x, cols, flags, lds, st); break;
            case 7: launch_segs_lds_t<7>(segs, waves, nbl, rpw, x, cols, flags, lds, st); break;
            default: launch_segs_lds_t<8>(segs, waves, nbl, rpw, x, cols, flags, lds, st); break;
        }
        WZY_LAUNCH_CHECK();
        return WZY_OK;
    }
    switch (T) {
        case 1: launch_segs_t<1>(segs, waves, nbl, x, cols, st); break;
        case 2: launch_segs_t<2>(segs, waves, nbl, x, cols, st); break;
        case 3: launch_segs_t<3>(segs, waves, nbl, x, cols, st); break;
        case 4: launch_segs_t<4>(segs, waves, nbl, x, cols, st); break;
        case 5: launch_segs_t<5>(segs, waves, nbl, x, cols, st); break;
        case 6: launch_segs_t<6>(segs, waves, nbl, x, cols, st); break;
        case 7: launch_segs_t<7>(segs, waves, nbl, x, cols, st); break;
        default: launch_segs_t<8>(segs, waves, nbl, x, cols, st); break;
    }
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}
}  // namespace wzy

extern "C" int wzy_gemv_segs(const wzy_gemv_seg* segs, int n_segs, const float* x, int cols, int T, void* stream) {
    WZY_REQUIRE(segs && n_segs >= 1 && n_segs <= GEMV_MAX_SEGS, "wzy_gemv_segs: 1 to %d segments required",
                GEMV_MAX_SEGS);
    GemvSegs g;
    g.n = n_segs;
    for (int i = 0; i < n_segs; ++i) {
        const wzy_gemv_seg& a = segs[i];
        WZY_REQUIRE(a.kind == WZY_GEMV_Q8 || a.kind == WZY_GEMV_BF16, "wzy_gemv_segs: segment %d has unknown kind %d",
                    i, a.kind);
        g.seg[i] = GemvSeg{a.w, a.s, a.y, a.rows, a.kind == WZY_GEMV_Q8 ? GEMV_Q8 : GEMV_BF16, a.y_stride, 0};
    }
    return launch_gemv_segs(g, x, cols, T, as_stream(stream));
}

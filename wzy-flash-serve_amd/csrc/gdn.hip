// gdn.hip -- gated delta-rule (GDN) decode step for gfx950.
//
// One 512-thread workgroup per key head kh; it runs the value heads kh, kh+HK, ... in turn.  The 128x128 fp32 state of the
// head lives in VGPRs for the whole window: thread (col j, row group g) holds S[32g .. 32g+31][j]
// and the state touches HBM once on entry and once on exit (plus optional per-step snapshots for
// speculative verify).  In the fused mode the workgroup first runs, for its own 384 channels, the
// 4-tap causal depthwise conv + SiLU + per-head L2 norm and the decay/beta gates, so the raw
// projection output goes straight into the recurrence.
//
// Per step t:  S *= decay;  kv_j = sum_i S_ij k_i;  delta_j = (v_j - kv_j) * beta;
//              S_ij += k_i delta_j;  o_j = sum_i S_ij q_i;  o *= 1/sqrt(128);
//              y_j = o_j * rsqrt(mean(o^2) + eps) * gamma_j * sigmoid(z_j)
// reference: fused_gdn_conv_l2_multi, fused_gdn_ab_multi, fused_gdn_step_norm_multi
// (src/wzy_kernels_v2.cuh:833-984).
#include "wzy_device.h"
#include "wzy_gdn.h"
#include "wzy_host.h"

using namespace wzy;

constexpr int GS = 128;   // state / head dim

template <bool FUSED>
__global__ void __launch_bounds__(512) gdn_kernel(GdnArgs a) {
    __shared__ float s_q[WZY_MAX_W][GS], s_k[WZY_MAX_W][GS], s_v[WZY_MAX_W][GS];
    __shared__ float s_dec[WZY_MAX_W], s_beta[WZY_MAX_W];
    __shared__ float s_red[4][GS];
    __shared__ float s_red2[4][GS];
    __shared__ float s_w[16];
    const int kh = blockIdx.x;                      // key head; value heads kh, kh+HK, ...
    const int HK = a.hk, HV = a.hv, T = a.T;
    const int QKV = 2 * HK * GS + HV * GS;
    const int tid = threadIdx.x;
    const int col = tid & (GS - 1), rg = tid >> 7;  // 4 row groups of 32
    const int lane = tid & 63, wv = tid >> 6;

    // ---- q, k of this key head ----
    if (FUSED) {
        // 4-tap causal conv + SiLU on the q and k channels (this workgroup owns their history)
        if (tid < 2 * GS) {
            const int part = tid / GS, i = tid % GS;
            const int ch = part * HK * GS + kh * GS + i;
            float h0 = a.conv_hist[ch * 3 + 0], h1 = a.conv_hist[ch * 3 + 1], h2 = a.conv_hist[ch * 3 + 2];
            const float w0 = a.conv_w[ch * 4 + 0], w1 = a.conv_w[ch * 4 + 1], w2 = a.conv_w[ch * 4 + 2], w3 = a.conv_w[ch * 4 + 3];
            for (int t = 0; t < T; ++t) {
                const float x = a.qkv[(size_t) t * QKV + ch];
                const float sum = h0 * w0 + h1 * w1 + h2 * w2 + x * w3;
                h0 = h1; h1 = h2; h2 = x;
                (part == 0 ? s_q : s_k)[t][i] = sum / (1.0f + __expf(-sum));
                if (a.hist_snaps) {
                    float* hs = a.hist_snaps + (size_t) t * QKV * 3 + (size_t) ch * 3;
                    hs[0] = h0; hs[1] = h1; hs[2] = h2;
                }
            }
            a.conv_hist[ch * 3 + 0] = h0; a.conv_hist[ch * 3 + 1] = h1; a.conv_hist[ch * 3 + 2] = h2;
        }
        __syncthreads();
        // per-head L2 norm of q and k: waves 0-1 reduce q, waves 2-3 reduce k
        for (int t = 0; t < T; ++t) {
            if (tid < 2 * GS) {
                const float y = (tid < GS) ? s_q[t][tid] : s_k[t][tid - GS];
                const float sq = wave_sum(y * y);
                if (lane == 0) s_w[wv] = sq;
            }
            __syncthreads();
            if (tid < 2 * GS) {
                const float ss = (tid < GS) ? (s_w[0] + s_w[1]) : (s_w[2] + s_w[3]);
                const float r = 1.0f / sqrtf(ss + a.eps);
                if (tid < GS) s_q[t][tid] *= r; else s_k[t][tid - GS] *= r;
            }
            __syncthreads();
        }
    } else {
        for (int i = tid; i < T * GS; i += blockDim.x) {
            const int t = i / GS, j = i % GS;
            s_q[t][j] = a.q[(size_t) t * HK * GS + kh * GS + j];
            s_k[t][j] = a.k[(size_t) t * HK * GS + kh * GS + j];
        }
    }
    const float gm = a.gamma ? a.gamma[col] : 1.0f;

    for (int h = kh; h < HV; h += HK) {
        // ---- v of value head h, gates ----
        if (FUSED) {
            if (tid < GS) {
                const int ch = 2 * HK * GS + h * GS + tid;
                float h0 = a.conv_hist[ch * 3 + 0], h1 = a.conv_hist[ch * 3 + 1], h2 = a.conv_hist[ch * 3 + 2];
                const float w0 = a.conv_w[ch * 4 + 0], w1 = a.conv_w[ch * 4 + 1], w2 = a.conv_w[ch * 4 + 2], w3 = a.conv_w[ch * 4 + 3];
                for (int t = 0; t < T; ++t) {
                    const float x = a.qkv[(size_t) t * QKV + ch];
                    const float sum = h0 * w0 + h1 * w1 + h2 * w2 + x * w3;
                    h0 = h1; h1 = h2; h2 = x;
                    s_v[t][tid] = sum / (1.0f + __expf(-sum));
                    if (a.hist_snaps) {
                        float* hs = a.hist_snaps + (size_t) t * QKV * 3 + (size_t) ch * 3;
                        hs[0] = h0; hs[1] = h1; hs[2] = h2;
                    }
                }
                a.conv_hist[ch * 3 + 0] = h0; a.conv_hist[ch * 3 + 1] = h1; a.conv_hist[ch * 3 + 2] = h2;
            } else if (tid >= 256 && tid < 256 + T) {
                const int t = tid - 256;
                const float av = a.ab[(size_t) t * 2 * HV + h] + a.dt[h];
                const float sp = av > 20.0f ? av : log1pf(__expf(av));
                s_dec[t] = __expf(sp * a.ssm_a[h]);
                s_beta[t] = 1.0f / (1.0f + __expf(-a.ab[(size_t) t * 2 * HV + HV + h]));
            }
        } else {
            for (int i = tid; i < T * GS; i += blockDim.x) {
                const int t = i / GS, j = i % GS;
                s_v[t][j] = a.v[(size_t) t * HV * GS + h * GS + j];
            }
            if (tid < T) {
                s_dec[tid] = a.decay[tid * HV + h];
                s_beta[tid] = a.beta[tid * HV + h];
            }
        }
        __syncthreads();

        // ---- recurrence, state in registers ----
        float s[32];
        float* base = a.state + (size_t) h * GS * GS + (size_t) (rg * 32) * GS + col;
#pragma unroll
        for (int r = 0; r < 32; ++r) s[r] = base[(size_t) r * GS];

        for (int t = 0; t < T; ++t) {
            const float dec = s_dec[t], beta = s_beta[t];
            float kv = 0.f;
#pragma unroll
            for (int r = 0; r < 32; ++r) {
                s[r] *= dec;
                kv = fmaf(s[r], s_k[t][rg * 32 + r], kv);
            }
            s_red[rg][col] = kv;
            __syncthreads();
            const float kv_col = s_red[0][col] + s_red[1][col] + s_red[2][col] + s_red[3][col];
            const float delta = (s_v[t][col] - kv_col) * beta;
            float o = 0.f;
#pragma unroll
            for (int r = 0; r < 32; ++r) {
                s[r] = fmaf(s_k[t][rg * 32 + r], delta, s[r]);
                o = fmaf(s[r], s_q[t][rg * 32 + r], o);
            }
            if (a.state_snaps) {
                float* sb = a.state_snaps + (size_t) t * HV * GS * GS + (size_t) h * GS * GS + (size_t) (rg * 32) * GS + col;
#pragma unroll
                for (int r = 0; r < 32; ++r) sb[(size_t) r * GS] = s[r];
            }
            s_red2[rg][col] = o;
            __syncthreads();
            float oc = 0.f;
            if (rg == 0) {                  // waves 0-1 own the 128 output columns
                oc = (s_red2[0][col] + s_red2[1][col] + s_red2[2][col] + s_red2[3][col]) * 0.08838834764831845f;
                const float sq = wave_sum(oc * oc);
                if (lane == 0) s_w[8 + wv] = sq;
            }
            __syncthreads();
            if (rg == 0) {
                const float ss = s_w[8] + s_w[9];
                const float scale = 1.0f / sqrtf(ss * (1.0f / 128.0f) + a.eps);
                const float zz = a.z ? a.z[(size_t) t * HV * GS + h * GS + col] : 0.0f;
                const float gate = a.z ? 1.0f / (1.0f + __expf(-zz)) : 1.0f;
                a.y[(size_t) t * HV * GS + h * GS + col] = oc * scale * gm * gate;
            }
            __syncthreads();
        }
#pragma unroll
        for (int r = 0; r < 32; ++r) base[(size_t) r * GS] = s[r];
        __syncthreads();                    // s_v / s_dec reuse by the next value head
    }
}

namespace wzy {
int launch_gdn(const GdnArgs& a, bool fused, hipStream_t st) {
    WZY_REQUIRE(a.T >= 1 && a.T <= WZY_MAX_W, "gdn: T out of range");
    WZY_REQUIRE(a.S == GS, "gdn: state dim must be 128");
    WZY_REQUIRE(a.hk >= 1 && a.hv >= a.hk && a.hv % a.hk == 0 && a.hv <= 1024, "gdn: bad head counts");
    WZY_REQUIRE(a.state && a.y, "gdn: null state/output");
    if (fused) {
        WZY_REQUIRE(a.qkv && a.ab && a.dt && a.ssm_a && a.conv_w && a.conv_hist, "gdn: fused mode inputs missing");
        hipLaunchKernelGGL(gdn_kernel<true>, dim3(a.hk), dim3(512), 0, st, a);
    } else {
        WZY_REQUIRE(a.q && a.k && a.v && a.decay && a.beta, "gdn: recurrence inputs missing");
        hipLaunchKernelGGL(gdn_kernel<false>, dim3(a.hk), dim3(512), 0, st, a);
    }
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}
}  // namespace wzy

extern "C" int wzy_gdn_step(const float* qkv_raw, const float* z, const float* ab_raw, const float* dt,
                            const float* ssm_a, const float* conv_w, float* conv_hist, float* state,
                            const float* gamma, float eps, float* y, int hk, int hv, int T, float* state_snaps,
                            float* hist_snaps, void* stream) {
    GdnArgs a{};
    a.qkv = qkv_raw; a.z = z; a.ab = ab_raw; a.dt = dt; a.ssm_a = ssm_a; a.conv_w = conv_w; a.conv_hist = conv_hist;
    a.state = state; a.gamma = gamma; a.eps = eps; a.y = y; a.hk = hk; a.hv = hv; a.S = GS; a.T = T;
    a.state_snaps = state_snaps; a.hist_snaps = hist_snaps;
    return launch_gdn(a, true, as_stream(stream));
}

extern "C" int wzy_gdn_recurrence(const float* q, const float* k, const float* v, const float* decay,
                                  const float* beta, const float* z, const float* gamma, float eps, float* state,
                                  float* y, int hk, int hv, int T, float* state_snaps, void* stream) {
    GdnArgs a{};
    a.q = q; a.k = k; a.v = v; a.decay = decay; a.beta = beta; a.z = z; a.gamma = gamma; a.eps = eps;
    a.state = state; a.y = y; a.hk = hk; a.hv = hv; a.S = GS; a.T = T; a.state_snaps = state_snaps;
    return launch_gdn(a, false, as_stream(stream));
}

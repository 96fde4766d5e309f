// gdn.hip -- gated delta-rule (GDN) decode step for gfx950.
//
// The 128x128 fp32 state of a value head is split by columns over GDN_NQ workgroups (256 threads
// each): workgroup (h, cq) owns columns 32*cq .. 32*cq+31, and thread (column c = lane % 32, row
// group rg = 2*wave + lane / 32) holds S[16*rg .. 16*rg+15][32*cq + c] in VGPRs for the whole
// window.  The columns of the recurrence are independent, so a head's state moves through 4 CUs
// (16 KB each) instead of one.  Every global load of a workgroup (its state block, conv inputs,
// gates) is issued at entry, before any is used; the state touches HBM once on entry and once on
// exit (plus optional per-step snapshots for speculative verify).
// In the fused mode each workgroup first runs the 4-tap causal depthwise conv + SiLU of the 256 q/k
// channels of its key head and of its own 32 v channels, the per-head L2 norms of q and k, and the
// decay/beta gates.  The v history belongs to one workgroup and is updated in place.  The q/k
// history is read by every workgroup of the key head, so it is written by the last of them: each
// workgroup increments the key head's counter once its history reads have been consumed, and the
// one that sees the count complete writes the new history and resets the counter (no workgroup
// waits for another).
// The output RMS norm spans the head's 128 columns, i.e. four workgroups: the kernel writes
// o * 1/sqrt(128) and, per (row, head, column quarter), the partial sum of its squares; the norm
// and gate y = o * rsqrt(sum/128 + eps) * gamma * sigmoid(z) are applied by the consumer (the
// out-projection GEMV's staging in the stage).  The standalone entry points, whose output is final,
// run each head of a window of up to three rows in one 1024-thread workgroup instead (the same thread
// mapping, four column quarters side by side) and apply the norm in the kernel from the same quarter
// partials, so a step is one launch; longer windows use the quarters and gdn_norm_kernel.
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

constexpr int GS = 128;              // state / head dim
// Windows of up to this many rows with final outputs run a head in one workgroup (one launch, the
// norm in the kernel); longer ones spread a head over GDN_NQ workgroups and finish with
// gdn_norm_kernel (per row a CU's share of the recurrence then costs more than the second launch).
constexpr int GDN_ONE_WG_MAX_T = 3;
constexpr int GDN_MAX_HK = 1024;
constexpr int GDN_MAX_HV = 1024;

// Completion counters of the shared q/k conv history, one per key head; every launch leaves them
// at zero.  Launches on one device must not overlap.
__device__ int g_gdn_qk_sync[GDN_MAX_HK];
// Partial sums of squares of the standalone entry points' longer windows ([T][HV][GDN_NQ]).
__device__ float g_gdn_ss[WZY_MAX_W * GDN_MAX_HV * GDN_NQ];

// NQ = workgroups per value head (GDN_NQ column quarters in the stage, whose out-projection applies
// the output norm; 1 in the standalone entry points, where one 1024-thread workgroup holds the whole
// head and applies the norm itself, from the same four quarter partials, so no second launch is
// needed).  Thread (column c, row group rg) = (tid % QC, tid / QC).
template <bool FUSED, int NQ>
__global__ void __launch_bounds__(8 * (GS / NQ)) gdn_kernel(GdnArgs a, float* __restrict__ o_ss) {
    constexpr int QC = GS / NQ;                     // state columns per workgroup
    __shared__ float s_q[WZY_MAX_W][GS], s_k[WZY_MAX_W][GS], s_v[WZY_MAX_W][QC];
    __shared__ float s_dec[WZY_MAX_W], s_beta[WZY_MAX_W];
    __shared__ float s_w[WZY_MAX_W][4];
    __shared__ float s_kv[8][QC], s_o[8][QC];
    __shared__ float s_ss[WZY_MAX_W][4];
    __shared__ int s_last;
    const int HK = a.hk, HV = a.hv, T = a.T;
    // XCD-local numbering when HV % 8 == 0: workgroup b runs on XCD b % 8, which takes heads
    // b % 8, b % 8 + 8, ... with all their column quarters, so a key head's shared conv history and
    // weights are fetched from HBM once per XCD; otherwise consecutive workgroups of a head
    const int b = blockIdx.x;
    const bool xl = (HV & 7) == 0;
    const int h = xl ? (b & 7) + 8 * ((b >> 3) / NQ) : b / NQ;
    const int cq = xl ? (b >> 3) % NQ : b % NQ;
    const int kh = h % HK;
    const int QKV = 2 * HK * GS + HV * GS;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int c = tid & (QC - 1), rg = tid / QC;
    const int j = cq * QC + c;                      // state column of this thread
    const bool qk_thr = tid < 2 * GS;               // q/k channel threads (all of a 256-thread workgroup)

    // ---- 0. every load, issued before any is used ----
    float s[16];
    float* sbase = a.state + (size_t) h * GS * GS + (size_t) (16 * rg) * GS + j;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = sbase[(size_t) r * GS];
    // q/k channel tid (q for tid < 128); v channel 32*cq + (tid % 32) of head h; gates on threads 128 + t
    const int qk_ch = (tid < GS ? 0 : HK * GS - GS) + kh * GS + min(tid, 2 * GS - 1);
    const int v_ch = 2 * HK * GS + h * GS + cq * QC + (tid & (QC - 1));
    float qh[3], qw[4], vh[3], vw[4], qx[WZY_MAX_W], vx[WZY_MAX_W];
    float g_a, g_b, g_dt = 0.f, g_sa = 0.f;
    const int tg = min(max(tid - GS, 0), T - 1);
    if (FUSED) {
#pragma unroll
        for (int i = 0; i < 3; ++i) { qh[i] = a.conv_hist[qk_ch * 3 + i]; vh[i] = a.conv_hist[v_ch * 3 + i]; }
#pragma unroll
        for (int i = 0; i < 4; ++i) { qw[i] = a.conv_w[qk_ch * 4 + i]; vw[i] = a.conv_w[v_ch * 4 + i]; }
#pragma unroll
        for (int t = 0; t < WZY_MAX_W; ++t) {
            const int tc = t < T ? t : 0;
            qx[t] = a.qkv[(size_t) tc * QKV + qk_ch];
            vx[t] = a.qkv[(size_t) tc * QKV + v_ch];
        }
        g_a = a.ab[(size_t) tg * 2 * HV + h];
        g_b = a.ab[(size_t) tg * 2 * HV + HV + h];
        g_dt = a.dt[h];
        g_sa = a.ssm_a[h];
    } else {
#pragma unroll
        for (int t = 0; t < WZY_MAX_W; ++t) {
            const int tc = t < T ? t : 0;
            qx[t] = tid < GS ? a.q[(size_t) tc * HK * GS + kh * GS + tid] : a.k[(size_t) tc * HK * GS + kh * GS + min(tid, 2 * GS - 1) - GS];
            vx[t] = a.v[(size_t) tc * HV * GS + h * GS + cq * QC + (tid & (QC - 1))];
        }
        g_a = a.decay[tg * HV + h];
        g_b = a.beta[tg * HV + h];
    }

    // ---- 1. conv + SiLU (fused), L2 norms of q and k, gates ----
    int qk_order = 0;
    if (FUSED) {
        float h0 = qh[0], h1 = qh[1], h2 = qh[2];
        float u0 = vh[0], u1 = vh[1], u2 = vh[2];
#pragma unroll
        for (int t = 0; t < WZY_MAX_W; ++t) {
            if (t >= T) break;
            const float sum = h0 * qw[0] + h1 * qw[1] + h2 * qw[2] + qx[t] * qw[3];
            h0 = h1; h1 = h2; h2 = qx[t];
            if (qk_thr) (tid < GS ? s_q : s_k)[t][tid & (GS - 1)] = sum / (1.0f + __expf(-sum));
            if (tid < QC) {
                const float sv = u0 * vw[0] + u1 * vw[1] + u2 * vw[2] + vx[t] * vw[3];
                u0 = u1; u1 = u2; u2 = vx[t];
                s_v[t][tid] = sv / (1.0f + __expf(-sv));
                if (a.hist_snaps) {
                    float* hs = a.hist_snaps + (size_t) t * QKV * 3 + (size_t) v_ch * 3;
                    hs[0] = u0; hs[1] = u1; hs[2] = u2;
                }
            }
            if (a.hist_snaps && h == kh && cq == 0 && qk_thr) {   // q/k snapshots: one writer per key head
                float* hs = a.hist_snaps + (size_t) t * QKV * 3 + (size_t) qk_ch * 3;
                hs[0] = h0; hs[1] = h1; hs[2] = h2;
            }
        }
        if (tid < QC) {                                 // own v history
            a.conv_hist[v_ch * 3 + 0] = u0; a.conv_hist[v_ch * 3 + 1] = u1; a.conv_hist[v_ch * 3 + 2] = u2;
        }
        qh[0] = h0; qh[1] = h1; qh[2] = h2;             // new q/k history, written by the last workgroup
        if (tid >= GS && tid < GS + T) {
            const float av = g_a + g_dt;
            const float sp = av > 20.0f ? av : log1pf(__expf(av));
            s_dec[tid - GS] = __expf(sp * g_sa);
            s_beta[tid - GS] = 1.0f / (1.0f + __expf(-g_b));
        }
        __syncthreads();
        // every wave has consumed its reads of the shared history: count this workgroup.  A relaxed
        // device-scope count is enough: the last workgroup's history writes depend on the count it
        // sees, and every other workgroup's reads returned before its count (the new values are
        // needed by the next launch only).  The result is used only at the end.
        if (tid == 0)
            qk_order = __hip_atomic_fetch_add(&g_gdn_qk_sync[kh], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // per-head L2 norm of q and k: waves 0-1 reduce q, waves 2-3 reduce k
        if (qk_thr)                                     // wave-uniform
            for (int t = 0; t < T; ++t) {
                const float y = (tid < GS ? s_q : s_k)[t][tid & (GS - 1)];
                const float sq = wave_sum(y * y);
                if (lane == 0) s_w[t][wv] = sq;
            }
        __syncthreads();
        if (qk_thr)
            for (int t = 0; t < T; ++t) {
                const float ss = (tid < GS) ? (s_w[t][0] + s_w[t][1]) : (s_w[t][2] + s_w[t][3]);
                const float r = 1.0f / sqrtf(ss + a.eps);
                (tid < GS ? s_q : s_k)[t][tid & (GS - 1)] *= r;
            }
    } else {
#pragma unroll
        for (int t = 0; t < WZY_MAX_W; ++t) {
            if (t >= T) break;
            if (qk_thr) (tid < GS ? s_q : s_k)[t][tid & (GS - 1)] = qx[t];
            if (tid < QC) s_v[t][tid] = vx[t];
        }
        if (tid >= GS && tid < GS + T) { s_dec[tid - GS] = g_a; s_beta[tid - GS] = g_b; }
    }
    __syncthreads();

    // ---- 2. recurrence: thread (column c, row group rg) ----
    for (int t = 0; t < T; ++t) {
        const float dec = s_dec[t], beta = s_beta[t];
        const float4* k4 = (const float4*) &s_k[t][16 * rg];
        const float4* q4 = (const float4*) &s_q[t][16 * rg];
        float kv = 0.f;
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
            const float4 kk = k4[r4];
            s[4 * r4 + 0] *= dec; kv = fmaf(s[4 * r4 + 0], kk.x, kv);
            s[4 * r4 + 1] *= dec; kv = fmaf(s[4 * r4 + 1], kk.y, kv);
            s[4 * r4 + 2] *= dec; kv = fmaf(s[4 * r4 + 2], kk.z, kv);
            s[4 * r4 + 3] *= dec; kv = fmaf(s[4 * r4 + 3], kk.w, kv);
        }
        s_kv[rg][c] = kv;
        __syncthreads();
        const float kvc = ((s_kv[0][c] + s_kv[1][c]) + (s_kv[2][c] + s_kv[3][c])) +
                          ((s_kv[4][c] + s_kv[5][c]) + (s_kv[6][c] + s_kv[7][c]));
        const float delta = (s_v[t][c] - kvc) * beta;
        float o = 0.f;
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
            const float4 kk = k4[r4], qq = q4[r4];
            s[4 * r4 + 0] = fmaf(kk.x, delta, s[4 * r4 + 0]); o = fmaf(s[4 * r4 + 0], qq.x, o);
            s[4 * r4 + 1] = fmaf(kk.y, delta, s[4 * r4 + 1]); o = fmaf(s[4 * r4 + 1], qq.y, o);
            s[4 * r4 + 2] = fmaf(kk.z, delta, s[4 * r4 + 2]); o = fmaf(s[4 * r4 + 2], qq.z, o);
            s[4 * r4 + 3] = fmaf(kk.w, delta, s[4 * r4 + 3]); o = fmaf(s[4 * r4 + 3], qq.w, o);
        }
        if (a.state_snaps) {
            float* sb = a.state_snaps + (size_t) t * HV * GS * GS + (size_t) h * GS * GS + (size_t) (16 * rg) * GS + j;
#pragma unroll
            for (int r = 0; r < 16; ++r) sb[(size_t) r * GS] = s[r];
        }
        s_o[rg][c] = o;
        __syncthreads();
        float oc = 0.f;
        const size_t yi = (size_t) t * HV * GS + h * GS + j;
        if (tid < QC) {                                 // the workgroup's columns (32 lanes per quarter)
            oc = (((s_o[0][c] + s_o[1][c]) + (s_o[2][c] + s_o[3][c])) +
                  ((s_o[4][c] + s_o[5][c]) + (s_o[6][c] + s_o[7][c]))) * 0.08838834764831845f;
            const float sq = sum32(oc * oc);
            if constexpr (NQ == GDN_NQ) {
                a.y[yi] = oc;
                if (tid == 0) o_ss[((size_t) t * HV + h) * GDN_NQ + cq] = sq;
            } else {
                if ((tid & 31) == 0) s_ss[t][tid >> 5] = sq;   // the four quarter partials
            }
        }
        if constexpr (NQ != GDN_NQ) {
            // the whole head is here: the output norm and gate (gdn_norm_gate) on the same partials
            __syncthreads();
            if (tid < QC)
                a.y[yi] = gdn_norm_gate(oc, s_ss[t], a.z ? a.z[yi] : 0.0f, a.z != nullptr,
                                        a.gamma ? a.gamma[j] : 1.0f, a.eps);
        }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) sbase[(size_t) r * GS] = s[r];

    // ---- 3. the last workgroup of the key head writes the shared q/k history ----
    if (FUSED) {
        if (tid == 0) s_last = qk_order == (HV / HK) * NQ - 1;
        __syncthreads();
        if (s_last && qk_thr) {
            a.conv_hist[qk_ch * 3 + 0] = qh[0]; a.conv_hist[qk_ch * 3 + 1] = qh[1]; a.conv_hist[qk_ch * 3 + 2] = qh[2];
            if (tid == 0) __hip_atomic_store(&g_gdn_qk_sync[kh], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// y = o * rsqrt(sum of the head's GDN_NQ partial sums / 128 + eps) * gamma * sigmoid(z), in place.
__global__ void __launch_bounds__(128) gdn_norm_kernel(float* __restrict__ y, const float* __restrict__ o_ss,
                                                       const float* __restrict__ z, const float* __restrict__ gamma,
                                                       float eps, int HV) {
    const int t = blockIdx.y, h = blockIdx.x, col = threadIdx.x;
    const size_t i = (size_t) t * HV * GS + (size_t) h * GS + col;
    y[i] = gdn_norm_gate(y[i], o_ss + ((size_t) t * HV + h) * GDN_NQ, z ? z[i] : 0.0f, z != nullptr,
                         gamma ? gamma[col] : 1.0f, eps);
}

namespace wzy {
int launch_gdn(const GdnArgs& a, bool fused, hipStream_t st) {
    WZY_REQUIRE(a.T >= 1 && a.T <= WZY_MAX_W, "gdn: T out of range");
    WZY_REQUIRE(a.S == GS, "gdn: state dim must be 128");
    WZY_REQUIRE(a.hk >= 1 && a.hk <= GDN_MAX_HK && a.hv >= a.hk && a.hv % a.hk == 0 && a.hv <= GDN_MAX_HV,
                "gdn: bad head counts");
    WZY_REQUIRE(a.state && a.y, "gdn: null state/output");
    if (fused) WZY_REQUIRE(a.qkv && a.ab && a.dt && a.ssm_a && a.conv_w && a.conv_hist, "gdn: fused mode inputs missing");
    else WZY_REQUIRE(a.q && a.k && a.v && a.decay && a.beta, "gdn: recurrence inputs missing");
    if (!a.o_ss && a.T <= GDN_ONE_WG_MAX_T) {
        // final outputs of a short window: one workgroup per head applies the norm itself
        const dim3 grid(a.hv);
        if (fused) hipLaunchKernelGGL((gdn_kernel<true, 1>), grid, dim3(8 * GS), 0, st, a, nullptr);
        else hipLaunchKernelGGL((gdn_kernel<false, 1>), grid, dim3(8 * GS), 0, st, a, nullptr);
    } else {
        // a head over GDN_NQ workgroups; the output norm from their quarter partials is applied by the
        // caller, or here by gdn_norm_kernel when the outputs are final
        float* ss = a.o_ss;
        if (!ss) WZY_HIP_TRY(hipGetSymbolAddress((void**) &ss, HIP_SYMBOL(g_gdn_ss)));
        const dim3 grid(a.hv * GDN_NQ);
        if (fused) hipLaunchKernelGGL((gdn_kernel<true, GDN_NQ>), grid, dim3(8 * GS / GDN_NQ), 0, st, a, ss);
        else hipLaunchKernelGGL((gdn_kernel<false, GDN_NQ>), grid, dim3(8 * GS / GDN_NQ), 0, st, a, ss);
        if (!a.o_ss)
            hipLaunchKernelGGL(gdn_norm_kernel, dim3(a.hv, a.T), dim3(GS), 0, st, a.y, ss, a.z, a.gamma, a.eps, a.hv);
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

// wzy_gdn.h -- internal launcher of the GDN decode step.
#pragma once
#include <hip/hip_runtime.h>

namespace wzy {
struct GdnArgs {
    // fused mode: raw projections
    const float* qkv;        // [T][2*HK*S + HV*S] raw (pre-conv) q|k|v channels
    const float* ab;         // [T][2*HV] raw alpha | beta projections
    const float* dt;         // [HV] dt bias
    const float* ssm_a;      // [HV]
    const float* conv_w;     // [QKV][4]
    float* conv_hist;        // [QKV][3] (state)
    float* hist_snaps;       // optional [T][QKV][3]
    // recurrence-only mode
    const float* q;          // [T][HK*S]
    const float* k;          // [T][HK*S]
    const float* v;          // [T][HV*S]
    const float* decay;      // [T][HV]
    const float* beta;       // [T][HV]
    // common
    const float* z;          // [T][HV*S] output gate (null: no gate)
    const float* gamma;      // [S] RMS norm weight (null: 1)
    float eps;
    float* state;            // [HV][S][S] head-major, S[h][i (key)][j (value)]
    float* state_snaps;      // optional [T][HV][S][S]
    float* y;                // [T][HV*S]: the output, or o * 1/sqrt(S) when o_ss is set
    float* o_ss;             // optional [T][HV][GDN_NQ]: partial sums of (o/sqrt(S))^2 per column
                             // quarter; set = the caller applies gdn_norm_gate, null = y is final
    int hk, hv, S, T;
};
constexpr int GDN_NQ = 4;    // workgroups (column quarters) per value head
static_assert(GDN_NQ == 4, "gdn_norm_gate sums four partials");
int launch_gdn(const GdnArgs& a, bool fused, hipStream_t st);

// The RMS norm and output gate of one value of a head from its GDN_NQ partial sums:
// o * rsqrt(sum/128 + eps) * gamma * sigmoid(z)  (sigmoid(z) = 1 without a gate).
__device__ __forceinline__ float gdn_norm_scale(const float* ss, float eps) {
    const float sum = (ss[0] + ss[1]) + (ss[2] + ss[3]);
    return 1.0f / sqrtf(sum * (1.0f / 128.0f) + eps);
}
__device__ __forceinline__ float gdn_gate(float z) { return 1.0f / (1.0f + __expf(-z)); }
__device__ __forceinline__ float gdn_norm_gate(float o, const float* ss, float z, bool has_z, float gamma,
                                               float eps) {
    return o * gdn_norm_scale(ss, eps) * gamma * (has_z ? gdn_gate(z) : 1.0f);
}
}  // namespace wzy

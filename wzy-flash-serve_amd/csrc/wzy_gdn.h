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
    float* y;                // [T][HV*S]
    int hk, hv, S, T;
};
int launch_gdn(const GdnArgs& a, bool fused, hipStream_t st);
}  // namespace wzy

// wzy_moe.h -- internal interface of the MoE block (used by moe.hip and the stage executor).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/wzy_kernels.h"

#define MOE_MAX_K 32

namespace wzy {

// Byte offsets of the planes of one expert record (wzy_nvfp4_expert_bytes): gate|up codes
// [2F x D/2], gate|up e4m3 scales [2F x D/16], down codes [D x F/2], down scales [D x F/16], fp32
// tensor scales (gate, up, down, unused).
struct MoeOffsets {
    size_t gu_codes, gu_scales, dn_codes, dn_scales, tail, rec;
};
__host__ __device__ inline MoeOffsets moe_offsets(int D, int F) {
    MoeOffsets o;
    o.gu_codes = 0;
    o.gu_scales = (size_t) 2 * F * (D / 2);
    o.dn_codes = o.gu_scales + (size_t) 2 * F * (D / 16);
    o.dn_scales = o.dn_codes + (size_t) D * (F / 2);
    o.tail = o.dn_scales + (size_t) D * (F / 16);
    o.rec = o.tail + 16;
    return o;
}

// Device scratch of one MoE block call, carved from a workspace.
struct MoeWs {
    float* logits; float* sg;             // router logits [T x E], shared gate scalar [T]
    int* ids;      float* wts;            // [T x K] routed experts and renormalised weights
    int* n_groups; int* grp_exp; int* grp_cnt; int* grp_mem;   // distinct experts of the window
    uint16_t* ah16; float* as16;          // SwiGLU activations per routed entry: per-16 int8 values held
                                          // as f16 pairs [n_ent][F/16][8][2] (x_p, x_p+8), and their scales
    float* shact;                         // shared-expert SwiGLU activation [T][F] (fp32; per-32
                                          // int8 quantisation happens in moe_down)
};

struct MoeGuArgs {
    const uint8_t* experts; int D, F, E, K;
    const float* x; const float* logits;
    int* ids; float* wts; int* n_groups; int* grp_exp; int* grp_cnt; int* grp_mem;   // published by moe_router
    uint16_t* ah16; float* as16;
    const int8_t* shg_q; const uint16_t* shg_s; const int8_t* shu_q; const uint16_t* shu_s;
    float* shact;
    int n_routed_wg;
};
struct MoeDnArgs {
    const uint8_t* experts; int D, F, K;
    const int* n_groups; const int* grp_exp; const int* grp_cnt; const int* grp_mem;
    const uint16_t* ah16; const float* as16;
    const int8_t* shd_q; const uint16_t* shd_s; const float* shact;
    const float* wts; const float* sg; float* comb;
};

MoeWs moe_ws_carve(void* base, size_t cap, int D, int F, int E, int K, int T, size_t* need);
int moe_check(const wzy_moe_weights* w, int T);
// router GEMV (+ shared gate row) over fp32 x [T x D], then the window routing into ws (ids, wts,
// groups); launches on one device must not overlap (file-scope arrival counter)
int moe_launch_route(const wzy_moe_weights* w, const MoeWs& ws, const float* x, int T, hipStream_t st);
// routing + gate/up, down + combine into comb [T x D]
int moe_launch_experts(const wzy_moe_weights* w, const MoeWs& ws, const float* x, int T, float* comb, hipStream_t st);

}  // namespace wzy

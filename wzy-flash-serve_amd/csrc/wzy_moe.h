// wzy_moe.h -- internal interface of the MoE block (used by moe.hip and the stage executor).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/wzy_kernels.h"

#define MOE_MAX_K 32

namespace wzy {

// Device scratch of one MoE block call, carved from a workspace.
struct MoeWs {
    const float* xf = nullptr;            // fp32 activations [T x D] (input of the router GEMV)
    int8_t* xq16;  float* xs16;           // per-16 int8 activations (routed experts)
    int8_t* xq32;  float* xs32;           // per-32 int8 activations (shared expert)
    float* logits; float* sg;             // router logits [T x E], shared gate scalar [T]
    int* ids;      float* wts;            // [T x K]
    int* n_groups; int* grp_exp; int* grp_cnt; int* grp_mem;   // distinct experts of the window
    int8_t* aq16;  float* as16;           // SwiGLU activations per routed entry, per-16 int8
    int8_t* shq32; float* shs32;          // shared-expert SwiGLU activation, per-32 int8
    float* parts;                          // [T*K x D] expert outputs
    float* shared_out;                     // [T x D]
    unsigned* tile_cnt;                    // per output tile arrival counters
};

MoeWs moe_ws_carve(void* base, size_t cap, int D, int F, int E, int K, int T, size_t* need);
int moe_check(const wzy_moe_weights* w, int T);
// router GEMV (+ shared gate row) and top-k/grouping; needs ws.xf set.
int moe_launch_route(const wzy_moe_weights* w, const MoeWs& ws, int T, hipStream_t st);
// gate/up + down + combine into comb [T x D]; needs ws.xq16/xs16/xq32/xs32 filled.
int moe_launch_experts(const wzy_moe_weights* w, const MoeWs& ws, int T, float* comb, hipStream_t st);

}  // namespace wzy

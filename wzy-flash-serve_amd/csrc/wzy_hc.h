// wzy_hc.h -- internal launchers of the hyper-connection read (hc_pre + hc_post).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace wzy {

struct HcPreArgs {
    const float* R_in;          // [T][HC][D] residual streams, or null in embedding mode
    const uint16_t* emb_table;  // bf16 [n_vocab][D]: layer-0 input broadcast to every stream
    const int* toks;            // device [T] token ids (embedding mode)
    int n_vocab;
    const int8_t* emb_q;        // Q8_0 table [n_vocab][D] codes + emb_s fp16 [n_vocab][D/32] scales:
    const uint16_t* emb_s;      //   layer-0 input d*q (alternative to emb_table)
    const float* emb_rows;      // fp32 [T][D] rows broadcast to every stream (alternative input)
    const float* bo;            // pending write: block output [T][D] (nullable)
    const float* inj_prev;      // pending write gates [T][HC]
    float* R_out;               // [T][HC][D] = R_in + bo * 2*sigmoid(inj_prev/HC)
    const float* norm_w;        // [HC][D]
    const int8_t* down_q;       // Q8_0 [HCLR][HC*D]
    const uint16_t* down_s;
    const uint16_t* inj_w;      // bf16 [HC][HC*D] (nullable: the head has no inject)
    float* nsc;                 // [T][HC] rsqrt(mean(R_out^2) + eps)
    float* lo_part;             // [T][HC][HCLR] per-stream partials of down . quant32(xn)
    float* inj_part;            // [T][HC src stream][HC out] per-stream partials of inj_w . xn
    int D, HC, HCLR;
    float eps;
};

struct HcPostArgs {
    const float* R;             // R_out of hc_pre
    const float* nsc;
    const float* norm_w;
    const int8_t* up_q;         // Q8_0 [HC*D][HCLR]
    const uint16_t* up_s;
    const float* lo_part;       // hc_pre partials
    const float* inj_part;      // hc_pre inject partials (nullable with inj)
    float* lo;                  // [T][HCLR] silu(sum of partials / HC) (nullable)
    float* inj;                 // [T][HC] summed inject (nullable)
    float* mixed;               // [T][D]
    int D, HC, HCLR;
};

// Device bytes of the partial buffers for T rows, and their carving from one workspace.
size_t hc_workspace_bytes(int HC, int HCLR, int T);
void hc_carve_workspace(void* ws, int HC, int HCLR, int T, float** lo_part, float** inj_part);

// Whether the decode HC read has a kernel for stream width D (256 .. 4096 powers of two, 768, 1280,
// 1536, 2560, 3072, 5120); the stage rejects other widths when it is created.
bool hc_width_supported(int D);

int launch_hc_pre(const HcPreArgs& a, int T, hipStream_t st);
int launch_hc_post(const HcPostArgs& a, int T, hipStream_t st);

}  // namespace wzy

// wzy_gemv.h -- internal launchers shared by the kernel files and the stage executor.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wzy {
int launch_quant_act(const float* x, int8_t* q32, float* s32, int8_t* q16, float* s16, int cols, int T,
                     hipStream_t st);
int launch_gemv_q8(const int8_t* codes, const uint16_t* scales, const int8_t* xq, const float* xs, float* y, int rows,
                   int cols, int T, int y_stride, hipStream_t st);
int launch_gemv_bf16(const uint16_t* W, const float* x, float* y, int rows, int cols, int T, int y_stride,
                     const uint16_t* Wx, float* yx, hipStream_t st);
}  // namespace wzy

namespace wzy {
// One weight matrix of a multi-segment GEMV launch.
struct GemvSeg {
    const void* w;          // Q8_0 codes (int8) or bf16 weights, [rows x cols]
    const uint16_t* s;      // Q8_0 fp16 scales [rows x cols/32]; null for bf16
    float* y;               // out: y[t*y_stride + r]
    int rows;
    int kind;               // GEMV_Q8 or GEMV_BF16
    int y_stride;
    int wave0;              // first wave of this segment (filled by launch_gemv_segs)
    int act = 0;            // GEMV_ACT_*: applied to every output of the segment
};
enum { GEMV_Q8 = 0, GEMV_BF16 = 1 };
enum { GEMV_ACT_NONE = 0, GEMV_ACT_SIGMOID = 1 };
constexpr int GEMV_MAX_SEGS = 8;
// Optional activation transform of the LDS-staged GEMV: x[t][c] is not read as is but computed
// from a GDN output, x = gdn_norm_gate(o[t][c], ss[t][c/128][..], z[t][c], gamma[c%128]) (the
// out-projection applies the GDN RMS norm and output gate while staging its input).
struct GemvGdnIn {
    const float* ss = nullptr;      // [T][cols/128][GDN_NQ] partial sums of squares (null: off)
    const float* z = nullptr;       // [T][cols] output gate (null: no gate)
    bool z_is_gate = false;         // z already holds sigmoid(z)
    const float* gamma = nullptr;   // [128] norm weight (null: 1)
    float eps = 0.f;
};
struct GemvSegs {
    GemvSeg seg[GEMV_MAX_SEGS];
    int n = 0;
    GemvGdnIn gdn;
};
// y_seg = W_seg . x for every segment; x fp32 [T x cols] is quantised per 32 inside each lane for
// Q8_0 segments (bit-identical to quant_act + gemv_q8).  cols % 32 == 0, cols <= 8192.
int launch_gemv_segs(GemvSegs segs, const float* x, int cols, int T, hipStream_t st);
}  // namespace wzy

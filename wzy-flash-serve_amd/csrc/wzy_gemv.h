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

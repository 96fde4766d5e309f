// wzy_reduce.h -- internal launcher of the vocabulary argmax / top-16 reduction.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>

namespace wzy {
size_t reduce_ws_bytes(int nvocab, int T);
// ws: reduce_ws_bytes() bytes, zero-filled once before first use (kernels leave counters at zero).
int launch_row_reduce(const float* logits, int nvocab, int T, bool top16, int* greedy, float* top_v, int* top_i,
                      void* ws, hipStream_t st);
}  // namespace wzy

/* wzy_kernels.h -- kernel-level C ABI of the MI355X (gfx950) decode path.
 *
 * Every entry point enqueues hand-written HIP kernels on `stream` (a hipStream_t passed as void*,
 * NULL = the null stream) and returns a status code: WZY_OK (0) or a negative WZY_E* value, with a
 * message available from wzy_last_error().  All data pointers are DEVICE pointers unless stated
 * otherwise; no call allocates device memory, synchronizes, or takes ownership.
 *
 * Each function names the reference interface it replaces (reference = liaoyangr8-ai/wzy-flash-serve,
 * paths relative to its root).  The reference exposes these as `launch_*` helpers or bare
 * `__global__` kernels compiled into the engine; here they are a stable C ABI so a host written in
 * any language can drive the same kernels.
 *
 * Shapes are runtime parameters (the reference fixes them at compile time,
 * src/wzy_kernels_v2.cuh:8-19).  T is the number of window rows (1..WZY_MAX_W).
 */
#ifndef WZY_KERNELS_H
#define WZY_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WZY_OK 0
#define WZY_EINVAL (-1)   /* bad argument / unsupported shape */
#define WZY_EHIP (-2)     /* HIP runtime error */
#define WZY_ENOMEM (-3)   /* device allocation failed */
#define WZY_ESTATE (-4)   /* call not valid in the current state */
#define WZY_EIO (-5)      /* file / parse error */

#define WZY_MAX_W 8       /* verify-window rows, reference MAX_W (src/wzy_kernels_v2.cuh:13) */

/* Last error message of the calling thread ("" if none). */
const char* wzy_last_error(void);
/* Library version string. */
const char* wzy_version(void);

/* ---------------------------------------------------------------------------------------------
 * Activation quantisation
 * ------------------------------------------------------------------------------------------- */

/* Per-16 and/or per-32 symmetric int8 quantisation of T rows of `cols` floats
 * (d = amax/127, q = rint(x * 127/amax) clamped to +-127, zero block -> q = 0, d = 0).
 * Any of the (q, s) output pairs may be NULL.  cols % 32 == 0.
 * Replaces quant_act_multi (src/wzy_kernels_v2.cuh:58-107). */
int wzy_quant_act(const float* x, int8_t* q32, float* s32, int8_t* q16, float* s16,
                  int cols, int T, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Dense GEMVs (T rows of activations share one pass over the weights)
 * ------------------------------------------------------------------------------------------- */

/* Q8_0 GEMV: y[t*y_stride + r] = sum_b fp16(scales[r,b]) * xs[t,b] * sum_{i<32} codes[r,32b+i]*xq[t,32b+i].
 * codes int8 [rows x cols], scales fp16 bits [rows x cols/32], xq/xs from wzy_quant_act (per-32).
 * cols % 32 == 0; y_stride == 0 means rows.
 * Replaces launch_gemm_q8p / gemm_q8p_t (src/wzy_kernels_v2.cuh:120-159,230-303). */
int wzy_gemv_q8(const int8_t* codes, const uint16_t* scales, const int8_t* xq, const float* xs,
                float* y, int rows, int cols, int T, int y_stride, void* stream);

/* bf16 x fp32 GEMV: y[t*y_stride + r] = sum_c bf16(W[r,c]) * x[t,c].  cols % 8 == 0.
 * Replaces launch_gemm_bf16 / gemm_bf16_t (src/wzy_kernels_v2.cuh:307-387). */
int wzy_gemv_bf16(const uint16_t* W, const float* x, float* y, int rows, int cols, int T,
                  int y_stride, void* stream);

/* ---------------------------------------------------------------------------------------------
 * NVFP4 mixture of experts (decode)
 * ------------------------------------------------------------------------------------------- */

/* Device record of one NVFP4 expert ("plane layout", 16-byte aligned planes):
 *   [gate|up codes : 2*n_ff rows x n_embd/2 bytes][gate|up e4m3 scales : 2*n_ff rows x n_embd/16]
 *   [down codes    : n_embd rows x n_ff/2 bytes ][down e4m3 scales     : n_embd rows x n_ff/16  ]
 *   [tensor scales : fp32 gate, up, down, pad]
 * Row r of a matrix keeps the reference's nibble order: 64-value block b holds code bytes
 * 32b..32b+31, sub-block s (16 values) is bytes 32b+8s..+7, value k<8 is the low nibble of byte k,
 * value k>=8 the high nibble of byte k-8; scale byte 4b+s belongs to sub-block (b,s).
 * Same bytes as the reference's 36-byte-block blob (src/wzy_kernels_v2.cuh:15-16; PER), with the
 * 4 scale bytes of each block moved to a separate plane so code rows are 16-byte aligned. */
size_t wzy_nvfp4_expert_bytes(int n_embd, int n_ff);
/* Size of one expert in the reference blob layout (36-byte blocks + 16-byte tail). */
size_t wzy_nvfp4_blob_bytes(int n_embd, int n_ff);
/* Host-side repack of one reference-layout blob into the plane layout (host pointers).
 * Replaces the blob addressing of exp_gu_quant_grouped / exp_down_2r_grouped
 * (src/wzy_kernels_v2.cuh:1611-1613,1754-1757); used by loaders of experts.bin. */
int wzy_nvfp4_repack_host(const uint8_t* blob, uint8_t* planes, int n_embd, int n_ff);

/* One MoE layer's weights (device pointers). */
typedef struct wzy_moe_weights {
    int n_embd, n_ff, n_exp, top_k;
    const uint16_t* router;        /* bf16 [n_exp x n_embd]   (ffn_gate_inp)          */
    const uint16_t* sgate;         /* bf16 [n_embd]           (ffn_gate_inp_shexp)    */
    const uint8_t* experts;        /* n_exp records of wzy_nvfp4_expert_bytes()        */
    const int8_t* sh_gate_q;  const uint16_t* sh_gate_s;   /* Q8_0 [n_ff x n_embd]  */
    const int8_t* sh_up_q;    const uint16_t* sh_up_s;     /* Q8_0 [n_ff x n_embd]  */
    const int8_t* sh_down_q;  const uint16_t* sh_down_s;   /* Q8_0 [n_embd x n_ff]  */
} wzy_moe_weights;

/* Bytes of device workspace wzy_moe_block needs for T rows. */
size_t wzy_moe_workspace_bytes(int n_embd, int n_ff, int n_exp, int top_k, int T);

/* Full decode MoE block for T rows of x [T x n_embd] (fp32):
 * router GEMV -> softmax top-k (ties to the lower expert id, weights renormalised by
 * max(sum, 2^-14)) -> grouped NVFP4 gate/up + SwiGLU + per-16 int8 requant -> NVFP4 down ->
 * comb = sigmoid(sgate.x) * shared(x) + sum_k w_k * expert_k(x)  (k in routed order).
 * Outputs: comb [T x n_embd]; ids [T x top_k] int32 and wts [T x top_k] fp32 if non-NULL.
 * Replaces the MoE section of StageGpu::record_forward (src/wzy_stage_v2.cuh:697-724):
 * quant_act_multi, gemm_bf16 router, router_top10_fast_multi, shared-expert Q8 GEMVs +
 * silu_mul_quant32_multi, exp_gu_quant_grouped, exp_down_2r_grouped, moe_combine_shared_multi. */
int wzy_moe_block(const wzy_moe_weights* w, const float* x, int T, float* comb, int* ids, float* wts,
                  void* workspace, size_t workspace_bytes, void* stream);

/* Time the routed-expert GEMV kernels of wzy_moe_block over `iters` launches on `stream`, cycling
 * through `n_layers` weight sets (to defeat the 256 MB last-level cache), with hipEvents.  Returns
 * the mean duration per launch of the gate/up kernel and of the down kernel in microseconds
 * (host pointers).  The routing used is the one the last wzy_moe_block call on `workspace` produced. */
int wzy_moe_time_kernels(const wzy_moe_weights* layers, int n_layers, int T, void* workspace,
                         size_t workspace_bytes, int iters, float* us_gate_up, float* us_down,
                         void* stream);

/* ---------------------------------------------------------------------------------------------
 * Logit reductions
 * ------------------------------------------------------------------------------------------- */

/* Greedy argmax per row over `nvocab` logits (ties -> lowest index).
 * Replaces row_argmax_multi_kernel (src/wzy_kernels_v2.cuh:1873-1905). */
int wzy_row_argmax(const float* logits, int nvocab, int T, int* out_ids, void* stream);

/* Top-16 (value desc, ties -> lower index) per row plus greedy id (= rank 0).  Any output may be
 * NULL.  Replaces row_top16_multi_kernel (src/wzy_kernels_v2.cuh:1909-1984). */
int wzy_row_top16(const float* logits, int nvocab, int T, int* out_greedy, float* top_v,
                  int* top_i, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* WZY_KERNELS_H */

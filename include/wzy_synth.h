/* wzy_synth.h -- C ABI of the seeded synthetic-model generator.
 *
 * The reference serves real checkpoints only; the benchmark configurations of this build run on
 * random-initialised weights of the same architecture (see the tensor table in wzy_stage.h).
 * Every value is a pure function of (seed, stream, index) through a splitmix64-based counter hash,
 * so the GPU can fill HBM in bulk and the CPU-side checks can regenerate any tensor element
 * bit-for-bit.  Host functions write host memory; *_device functions write device memory.
 */
#ifndef WZY_SYNTH_H
#define WZY_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* counter hash: wzy_mix64(wzy_mix64(seed*phi + stream) + idx*c) */
uint64_t wzy_synth_hash(uint64_t seed, uint64_t stream, uint64_t idx);
/* stream id = kind<<48 | layer<<32 | sub */
uint64_t wzy_synth_stream(uint32_t kind, uint32_t layer, uint32_t sub);

/* n floats ~ N(mean, std^2) (Box-Muller on hash-derived uniforms, fp64 then rounded). */
void wzy_synth_normal(uint64_t seed, uint64_t stream, size_t n, float mean, float std, float* out);
/* n floats ~ U[lo, hi). */
void wzy_synth_uniform(uint64_t seed, uint64_t stream, size_t n, float lo, float hi, float* out);
/* n bf16 (round-to-nearest-even) of N(mean, std^2). */
void wzy_synth_normal_bf16(uint64_t seed, uint64_t stream, size_t n, float mean, float std, uint16_t* out);
/* Q8_0 matrix [rows x cols] from bf16-rounded N(0, std^2), quantised per 32 like the reference
 * loader (src/wzy_kernels_v2.cuh:393-407: fp16 scale = half(amax/127), q = rint(v / scale)). */
void wzy_synth_q8(uint64_t seed, uint64_t stream, int rows, int cols, float std, int8_t* codes,
                  uint16_t* scales);

/* One NVFP4 expert of layer `layer`: uniform random e2m1 code bytes, e4m3 block scales
 * round(U(0.5,2) * 2^-4), fp32 tensor scales 1.0.  Reference blob layout (36-byte blocks). */
int wzy_synth_expert_blob(uint64_t seed, int layer, int expert, int n_embd, int n_ff, uint8_t* blob);
/* Same expert in the device plane layout (host memory). */
int wzy_synth_expert_planes(uint64_t seed, int layer, int expert, int n_embd, int n_ff, uint8_t* planes);
/* Fill `n_experts` consecutive plane-layout records (device memory) on the GPU. */
int wzy_synth_experts_device(uint64_t seed, int layer, int first_expert, int n_experts, int n_embd,
                             int n_ff, uint8_t* dev, void* stream);

/* MTP Q2_0 expert blob bytes: 3*D*F/4 code bytes + 3*D*F/64 fp16 scales (src/wzy_mtp.cuh:6-10). */
size_t wzy_q2_expert_bytes(int n_embd, int n_ff);
/* One MTP Q2_0 expert: uniform 2-bit codes, fp16 scales (1 + m/1024) * 2^e with uniform 10-bit m and
 * e = floor(log2(1/sqrt(reduction dim))).  Host version and bulk device version (identical bytes). */
int wzy_synth_q2_expert(uint64_t seed, int expert, int n_embd, int n_ff, uint8_t* blob);
int wzy_synth_q2_experts_device(uint64_t seed, int first_expert, int n_experts, int n_embd, int n_ff, uint8_t* dev,
                                void* stream);

/* Synthetic INT8 KV cells [n_cells x kvd] codes uniform over [-127,127] and fp16 scales per 64
 * elements, for positions first_pos.. (host / device versions, identical bytes). */
void wzy_synth_kv_host(uint64_t seed, int layer, int is_v, int64_t first_pos, int n_cells, int kvd,
                       int8_t* codes, uint16_t* scales);
int wzy_synth_kv_device(uint64_t seed, int layer, int is_v, int64_t first_pos, int n_cells, int kvd,
                        int8_t* codes, uint16_t* scales, void* stream);

/* Synthetic per-layer-embedding table: row `row` (head_bytes fp8 codes: random sign and mantissa,
 * exponent field 4..9), host version, and the whole wzy_ple_table_rows() x head_bytes table in device
 * memory (identical bytes). */
void wzy_synth_ple_row(uint64_t seed, uint64_t row, int head_bytes, uint8_t* out);
int wzy_synth_ple_table_device(uint64_t seed, int head_bytes, uint8_t* table, void* stream);

/* IEEE half conversions used by the generator (round-to-nearest-even). */
uint16_t wzy_f32_to_f16(float f);
float wzy_f16_to_f32(uint16_t h);
uint16_t wzy_f32_to_bf16(float f);

#ifdef __cplusplus
}
#endif
#endif /* WZY_SYNTH_H */

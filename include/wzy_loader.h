/* wzy_loader.h -- C ABI of the real-weight loaders: the GGUF checkpoint, the NVFP4 expert pack
 * and the MTP drafter files of the reference engine.
 *
 * Replaces the reference's Gguf reader and uploaders (Gguf::open, up_q8_raw, up_q8, up_bf,
 * up_bf_as_q8, up_f32; src/wzy_stage_v2.cuh:30-179), the per-layer weight table of
 * init_stage_weights_and_state (src/wzy_engine_v2.cu:310-378,542-556), the experts.bin mapping
 * (src/wzy_engine_v2.cu:693-734,780-787), the token embedding rows (stage_one_emb,
 * src/wzy_engine_v2.cu:802-873) and MtpEngine::init (src/wzy_mtp.cuh:462-560).
 * Differences: the file is parsed with bounds checks and errors are returned (the reference exits);
 * the stage shapes come from the tensors instead of compile-time constants; every expert goes to HBM.
 * All calls are host calls; the stage calls copy to the device synchronously.
 */
#ifndef WZY_LOADER_H
#define WZY_LOADER_H

#include <stddef.h>
#include <stdint.h>

#include "wzy_stage.h"

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF tensor types read by the loaders (the GGML type ids). */
#define WZY_GGUF_F32 0
#define WZY_GGUF_F16 1
#define WZY_GGUF_Q8_0 8
#define WZY_GGUF_BF16 30
#define WZY_GGUF_I8 24

/* ---- GGUF container (versions 2 and 3), memory-mapped read-only ---- */
typedef struct wzy_gguf wzy_gguf;
int wzy_gguf_open(const char* path, wzy_gguf** out);
void wzy_gguf_close(wzy_gguf* g);
int wzy_gguf_n_tensors(const wzy_gguf* g);
/* Index of a tensor by name, or -1. */
int wzy_gguf_find(const wzy_gguf* g, const char* name);
/* Name, dimensions (dims[0] is the contiguous one; unused entries 1), GGML type and data bytes of
 * tensor i (bytes 0 for a type the loaders do not read). */
int wzy_gguf_tensor_info(const wzy_gguf* g, int i, const char** name, int* n_dims, int64_t dims[4], int* type,
                         size_t* bytes);
/* Pointer to tensor i's data inside the mapping (valid until wzy_gguf_close). */
const void* wzy_gguf_tensor_data(const wzy_gguf* g, int i);
/* Metadata values: integer (any integer or bool type), float (f32 / f64, or an integer) and string.
 * Return 0, or WZY_EINVAL when the key is absent or of another type. */
int wzy_gguf_get_int(const wzy_gguf* g, const char* key, int64_t* out);
int wzy_gguf_get_float(const wzy_gguf* g, const char* key, double* out);
int wzy_gguf_get_str(const wzy_gguf* g, const char* key, const char** str, size_t* len);

/* ---- element conversions (host) ---- */
/* Q8_0 blocks (fp16 scale + 32 int8 codes, 34 bytes) to separate code / scale planes (up_q8_raw). */
void wzy_q8_0_split(const void* blocks, size_t n_blocks, int8_t* codes, uint16_t* scales);
/* bf16 values to Q8_0 planes, per 32: scale = half(amax / 127), q = rint(v / scale) clamped to
 * +-127, 0 when the scale is 0 (quant_bf16_to_q8_kernel, src/wzy_kernels_v2.cuh:392-407). */
void wzy_bf16_to_q8_0(const uint16_t* src, size_t n_blocks, int8_t* codes, uint16_t* scales);
/* fp32 to bf16, round to nearest even (up_bf, src/wzy_stage_v2.cuh:120-125). */
void wzy_bf16_from_f32(const float* src, size_t n, uint16_t* dst);
/* f32 / f16 / bf16 / Q8_0 values to fp32 (up_f32, src/wzy_stage_v2.cuh:145-170). */
int wzy_to_f32(int type, const void* src, size_t n, float* dst);

/* ---- stage ---- */
/* A stage configuration from a checkpoint's tensor shapes: layer count and QSA period from the
 * blk.N tensors, hidden size and vocabulary from token_embd.weight, the hyper-connection,
 * GDN, QSA, indexer and MoE shapes from their weights, emb_q8 / head_q8 from the tensor types;
 * top_k, n_rot, rope_theta and eps from the "<arch>.expert_used_count", ".rope.dimension_count",
 * ".rope.freq_base" and ".attention.layer_norm_rms_epsilon" metadata, or the reference's
 * constants (10, 64, 1e7, 1e-6) where absent; idx_blk 4, idx_topk 2048; ple = 1 when the checkpoint
 * carries blk.1.ple_key.weight (the reference's has_ple, src/wzy_engine_v2.cu:316). */
int wzy_stage_cfg_from_gguf(const char* gguf_path, int ctx_max, wzy_stage_cfg* cfg);
/* Load every weight of a created stage: the GGUF's per-layer tensors (Q8_0 projections as they
 * are, bf16 hyper-connection mixes quantised to Q8_0, bf16 / f32 vectors), the LM head and the
 * token embedding (from emb_path's token_embd.weight when emb_path is not NULL, the reference's
 * token-embd-bf16.gguf), and the NVFP4 experts from experts_path (blob l*n_exp + e of
 * wzy_nvfp4_blob_bytes(n_embd, n_ff) bytes each, repacked to the plane layout); with cfg.ple also
 * layer 1's blk.1.ple_key / ple_value (bf16) and ple_norm_key / _query / _conv, ple_conv1d (f32)
 * (src/wzy_engine_v2.cu:493-499).  The recurrent state starts empty (as after wzy_stage_reset_state). */
int wzy_stage_load_gguf(wzy_stage* st, const char* gguf_path, const char* experts_path, const char* emb_path);
/* The per-layer embedding table of a cfg.ple stage from the reference's ple-fp8.gguf: the
 * per_layer_token_embd.weight tensor of 1-byte fp8 codes [rows = wzy_ple_table_rows()][n_embd / 16]
 * copied into HBM (51 GB at the real shape), and its scale from the strata.ple.scale metadata (f32 or
 * f64; 1 when absent).  Replaces PleSrc::open (src/wzy_stage_v2.cuh:228-287), which maps the file for
 * the host gather. */
int wzy_stage_load_ple(wzy_stage* st, const char* ple_path);
/* The MTP drafter from mtp_dir/dense.txt ("name kind rows cols offset bytes" lines indexing
 * mtp_dir/dense.bin: Q8_0 blocks, bf16 or f32), mtp_dir/experts.bin (n_exp Q2_0 blobs) and the
 * draft vocabulary dvocab_path (int32 main-vocabulary ids; the draft head holds those rows of the
 * main LM head). */
int wzy_stage_mtp_load(wzy_stage* st, const char* mtp_dir, const char* dvocab_path);

#ifdef __cplusplus
}
#endif
#endif

// wzy_ple.h -- per-layer embedding (PLE) at layer 1: internal launchers shared by ple.hip and the
// stage executor.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wzy {

constexpr int PLE_HEADS = 16;         // table heads per token: 8 for the 2-gram, 8 for the 3-gram
constexpr int PLE_HIST = 9;           // conv history per channel: 3 taps spaced 3 cells apart
constexpr int PLE_EOS_DEFAULT = 248044;

// Rows of the hashed 3-gram table for T window rows at positions *pos .. *pos+T-1.  The tokens before
// the window come from tok_hist (cell p holds the token of position p), which the launch extends with
// the window's tokens.  emb [T][16 * head] fp32 (decoded code * scale), emb_bf16 (nullable) the same
// rounded to bf16 (the prefill GEMM operand).
struct PleRowsArgs {
    const uint8_t* table;             // [rows][head] fp8 codes, rows = ple_table_rows()
    int head;                         // bytes per head row (n_embd / 16)
    float scale;
    const float* scale_dev;           // when set, the scale is read here (a graph replays the current one)
    int eos;
    const int* pos;                   // device: position of row 0
    const int* toks;                  // device [T]
    int* tok_hist;                    // device [ctx_max]
    int ctx_max;
    float* emb;
    uint16_t* emb_bf16;
};
uint64_t ple_table_rows();
int launch_ple_rows(const PleRowsArgs& a, int T, hipStream_t st);

// The block after its two projections k = W_k . emb [T][HC*D], v = W_v . emb [T][D]:
//   mix  (grid HC x T): optional fold R += bo * 2 sigmoid(inj_prev / HC); q = norm(R_c) * norm_q_c;
//        k_c = norm(k_c) * norm_k_c; g = sigmoid(sign(s) sqrt(max(|s|, 1e-6))), s = k_c . q / sqrt(D);
//        gat_c = v * g; n_c = norm(gat_c) * norm_c_c
//   conv (thread = channel, rows in order): acc = w0 h[0] + w1 h[3] + w2 h[6] + w3 n; the history
//        shifts n in; R += gat + silu(acc); hist_snaps (nullable) [T][HC*D][9] after each row.
struct PleBlockArgs {
    float* R;                         // [T][HC][D]
    const float* bo;                  // [T][D] pending write, or null
    const float* inj_prev;            // [T][HC]
    const float* k;                   // [T][HC*D] (normalised in place)
    const float* v;                   // [T][D]
    const float* norm_q; const float* norm_k; const float* norm_c;   // [HC*D]
    const float* conv_w;              // [HC*D][4]
    float* hist;                      // [HC*D][9]
    float* hist_snaps;                // [T][HC*D][9] or null
    float* gat;                       // [T][HC*D] scratch
    float* n;                         // [T][HC*D] scratch
    int D, HC;
    float eps;
};
int launch_ple_mix(const PleBlockArgs& a, int T, hipStream_t st);
int launch_ple_conv(const PleBlockArgs& a, int T, hipStream_t st);

}  // namespace wzy

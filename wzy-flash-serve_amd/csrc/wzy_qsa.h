// wzy_qsa.h -- internal interface of the QSA (sparse attention) decode kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wzy {

constexpr int QSA_ATT_CHUNK = 64;      // selected cells per attention workgroup

struct QsaDims {
    int qh, kvh, hd, n_rot;            // 24, 2, 256, 64
    int ih, idim, iblk, topk;          // indexer heads/dim (4, 128), block (4), top-k cells (2048)
    int ctx_max;                       // capacity of the KV store / indexer
    int ring_cap, sinks;               // 0 = full-context store addressed by position
    float eps;
    int window = 0;                    // > 0: dense sliding-window attention over the last `window`
                                       // cells (no indexer; the ring may wrap, window <= ring_cap)
    int f16_above = 0;                 // > 0: a window whose rows reach past this many cells
                                       // (pos + T > f16_above) attends with fp16 operands, the
                                       // numerics the reference switches to above its VRAM ring
};

// Attended span of a row whose context holds n_kv cells: positions p0 .. p0 + width - 1.  Sparse
// mode: the first min(n_kv, topk) entries (all cells when n_kv <= topk, else the selected ids);
// window mode: max(floor, n_kv - window) .. n_kv - 1.
__device__ __forceinline__ void qsa_span(const QsaDims& dm, int n_kv, const int* floor, int& p0, int& width) {
    if (dm.window > 0) {
        p0 = max(n_kv - dm.window, 0);
        if (floor) p0 = max(p0, *floor);
        width = max(n_kv - p0, 0);
    } else {
        p0 = 0;
        width = min(n_kv, dm.topk);
    }
}

// Storage slot of context position p: the position itself for a full-context store; with a ring,
// positions below `sinks` are pinned and the rest cycle through the remaining ring_cap - sinks slots.
__device__ __forceinline__ size_t qsa_kv_slot(int p, const QsaDims& dm) {
    if (dm.ring_cap <= 0) return (size_t) p;
    if (dm.ring_cap <= 2 * dm.sinks) return (size_t) (p % dm.ring_cap);
    if (p < dm.sinks) return (size_t) p;
    return (size_t) (dm.sinks + (p - dm.sinks) % (dm.ring_cap - dm.sinks));
}

int qsa_check_dims(const QsaDims& dm);

// A KV ring is accepted only when it never wraps (ctx_max <= ring_cap, so every position keeps its
// own slot and qsa_kv_slot(p) == p).  A wrapping ring would hand a selected cell older than the ring
// the K/V of a newer cell: the reference reads such cells from its pinned host mirror
// (src/wzy_qsa_256k.cuh:17-29), which this build replaces with a full-context store in HBM.
int qsa_check_ring(int ctx_max, int ring_cap, int sinks);

// KV store of one QSA layer: cells addressed by qsa_kv_slot(p)
struct QsaKv {
    int8_t* kq; uint16_t* ks;          // [slots][KVD], [slots][KVD/64] fp16 bits
    int8_t* vq; uint16_t* vs;
};
// indexer state of one QSA layer
struct QsaIdx {
    float* tail;                       // [iblk-1][idim]
    float* dead;                       // [idim]
    uint16_t* pooled;                  // [ctx_max/iblk + 2][idim] fp16 bits
    float* tail_snaps;                 // optional [T][iblk-1][idim]
    float* dead_snaps;                 // optional [T][idim]
    uint16_t* pool_snaps;              // optional [T][2][idim]
};

struct QsaPrepArgs {
    QsaDims dm;
    const int* pos;                    // device: base position of row 0
    float* qg;                         // [T][qh*2*hd] q|gate per head (q normalised+roped in place;
                                       // null: k/v only)
    float* kk;                         // [T][kvh*hd] (normalised+roped in place)
    const float* vv;                   // [T][kvh*hd]
    float* q_idx;                      // [T][ih*idim] (normalised+roped in place)
    const float* idx_raw;              // [T][idim]
    const float* q_norm, *k_norm, *iq_norm, *ik_norm;
    const float* cos_tab, *sin_tab;    // [ctx_max][n_rot/2]
    QsaKv kv;
    QsaIdx ix;
};
int launch_qsa_prep(const QsaPrepArgs& a, int T, hipStream_t st);

struct QsaScoreArgs {
    QsaDims dm;
    const int* pos;
    const uint16_t* pooled;            // fp16 keys
    const float* dead;
    const float* q_idx;                // [T][ih*idim]
    float* scores;                     // [T][max_b]
    int max_b;                         // ctx_max/iblk + 2
    int rows = 0;                      // rows scored (set by the launchers)
};
int launch_qsa_score(const QsaScoreArgs& a, int T, hipStream_t st);
// Block scores of `rows` consecutive rows (positions *pos + r), groups of 8 rows per grid row
// (prefill chunks); q_idx [rows][ih*idim], scores [rows][max_b].
int launch_qsa_score_rows(const QsaScoreArgs& a, int rows, hipStream_t st);
int launch_qsa_topk(const QsaDims& dm, const int* pos, const float* scores, int max_b, int* sel_ids, int* sel_cnt,
                    int T, hipStream_t st);

struct QsaAttnArgs {
    QsaDims dm;
    const int* pos;
    const float* qg;                   // [T][qh*2*hd]
    QsaKv kv;
    const int* sel_ids;                // [T][topk] (sparse mode)
    const int* floor = nullptr;        // window mode: device lower bound of the attended positions
    float* part;                       // [T][kvh][nch][gq][hd] partial outputs
    float* part_ml;                    // [T][kvh][nch][gq][2] (max, sum)
    float* out;                        // [T][qh*hd]
};
size_t qsa_attn_part_floats(const QsaDims& dm, int T);
int launch_qsa_attn(const QsaAttnArgs& a, int T, hipStream_t st);

}  // namespace wzy

// qsa_attn.hip -- QSA cell selection and sparse attention for gfx950.
//
//  qsa_topk   exact top-`topk` cells of each row: a multi-workgroup histogram of the 12-bit key
//             prefixes finds the threshold's prefix bin, then one workgroup per row resolves the
//             rest of the threshold key and writes the selection in the reference's order (see
//             the section below).  reference: qsa_block_topk_multi (src/wzy_qsa_256k.cuh:226-403)
//  qsa_attn   split-K sparse attention: workgroup (chunk of 64 selected cells, kv head, slice of 4
//             q heads, row) stages the chunk's INT8 K and V rows in LDS with one round of 128-bit
//             loads, computes its heads' scores (wave = head, lane = cell), a local softmax, and the
//             INT8 V sum (thread = dim).
//  qsa_combine merges the chunks (max / sum rescaling) and applies sigmoid(gate).
//             reference: qsa_attend_int8_sparse_multi (src/wzy_qsa_256k.cuh:407-532); windows past
//             the reference's VRAM ring take the operand rounding of its GQA kernel,
//             pf_qsa_wmma_sparse_attn (src/wzy_qsa_wmma.cuh:289-488): fp16(q / 16), K and V as
//             fp16(code * scale), fp16 softmax weights over 32-cell steps, fp32 sums.
#include "wzy_device.h"
#include "wzy_host.h"
#include "wzy_qsa.h"
#include "wzy_prefill.h"

using namespace wzy;

namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

constexpr int ATT_HPW = 4;           // q heads per attention workgroup (one per wave in the score phase)
constexpr int ATT_ROW = 256 + 16;    // LDS bytes per cell row (hd = 256 codes + pad against bank conflicts)
constexpr int ATT_CH_MAX = 32;       // chunks per row: topk <= 2048

WZY_DEV uint32_t order_key(float s) {
    const float v = s + 0.0f;                       // -0 -> +0
    if (!(v == v)) return 0u;                       // NaN sorts lowest
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Inclusive prefix sum over the 64 lanes in lane order, DPP only: shifts by 1, 2, 4, 8 inside each
// row of 16, then lane 15 of rows 0 / 2 into rows 1 / 3 and lane 31 into rows 2 and 3.  Lanes a
// shift would read from outside the row (or rows outside the mask) add the `old` operand, 0.
WZY_DEV int wave_incl_scan(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);   // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);   // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);   // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);   // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, DPP_ROW_BCAST15, 0xA, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, DPP_ROW_BCAST31, 0xC, 0xF, false);
    return v;
}

// Two inclusive prefix sums at once over the NW*64 threads in thread order (one barrier).  The
// caller separates consecutive calls (and later writes of s_x / s_y) by a barrier.
template <int NW>
WZY_DEV void block_scan_incl2(int& x, int& y, int* s_x, int* s_y) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    x = wave_incl_scan(x);
    y = wave_incl_scan(y);
    if (lane == 63) { s_x[w] = x; s_y[w] = y; }
    __syncthreads();
    int bx = 0, by = 0;
#pragma unroll
    for (int i = 0; i < NW; ++i)
        if (i < w) { bx += s_x[i]; by += s_y[i]; }
    x += bx;
    y += by;
}

// Full-wave minimum of a 32-bit unsigned value (the complement of a maximum).
WZY_DEV uint32_t wave_min_u32(uint32_t v) { return ~wave_max_u32(~v); }

}  // namespace

// ---------------------------------------------------------------------------------------------
// exact top-k cell selection: a radix select on the order keys of the block scores, most
// significant bits first (12 + 12 + 8 bits), block weights = cells.  The threshold is the key
// value thr with weight(key > thr) < width <= weight(key >= thr); blocks above it are taken whole
// and blocks at it are filled in the reference's tie order.
//
// One launch, workgroups of 1,024 threads, each holding 16,384 blocks of a row in registers
// (thread p: blocks base + 1024 q + p).  Level 1 is a 4,096-bin histogram of the 12-bit key
// prefixes.  A row that fits one workgroup (up to 65,536 cells) keeps it in LDS; a longer row's
// workgroups add their histograms to the row's histogram in device memory and the last one to
// arrive carries on alone.  That workgroup lists the blocks at or above the threshold's prefix bin
// (usually ~1,000 of them) in LDS, resolves the remaining 20 bits over the list, and writes each
// selected block at its offset in the reference's order: the reference walks the blocks with 256
// threads, thread t emitting blocks t, t+256, ... in turn, so block b's cells follow the cells of
// the selected blocks of walkers t' < b mod 256 and of walker b mod 256 before it (ties at the
// threshold take the remaining budget in that order).  When the bin holds more blocks than the
// list, the selection sweeps every key of the row instead (heavy ties).
// reference: qsa_block_topk_multi (src/wzy_qsa_256k.cuh:226-403)
// ---------------------------------------------------------------------------------------------
namespace {
constexpr int TK_L1_SHIFT = 20, TK_L1_BINS = 4096;     // level 1: key bits 31..20
constexpr int TK_L2_BINS = 4096;                       // level 2: bits 19..8
constexpr int TK_L3_BINS = 256;                        // level 3: bits 7..0
constexpr int TK_THREADS = 1024, TK_NW = TK_THREADS / 64, TK_PER = 16;
constexpr int TK_CHUNK = TK_THREADS * TK_PER;          // blocks per workgroup
constexpr int TK_LIST = 4096;                          // listed blocks (LDS)
constexpr int TK_BATCH = 16;                           // loads in flight per thread in a sweep

WZY_DEV int tk_weight(int b, int n_bid, int nb, int n_kv, int B) {
    return b < n_bid ? B : (b < nb ? n_kv - n_bid * B : 0);
}

// Bins owned NPER per thread in descending order (thread 0 holds the highest).  Finds the bin where
// the weight counted from the top, starting at `base`, reaches `width`; the owner writes (bin,
// weight above it, its weight) to s_res.  One barrier inside; the caller syncs before reading s_res.
template <int NPER>
WZY_DEV void tk_find(const int* hist, int nbins, int base, int width, int* s_w, int* s_c, int* s_res) {
    const int p = threadIdx.x;
    int c[NPER];
    int sum = 0;
#pragma unroll
    for (int k = 0; k < NPER; ++k) {
        const int bin = nbins - 1 - NPER * p - k;
        c[k] = bin >= 0 ? hist[bin] : 0;
        sum += c[k];
    }
    int incl = sum, dummy = 0;
    block_scan_incl2<TK_NW>(incl, dummy, s_w, s_c);
    int acc = base + incl - sum;
#pragma unroll
    for (int k = 0; k < NPER; ++k) {
        const int bin = nbins - 1 - NPER * p - k;
        if (bin >= 0 && acc < width && acc + c[k] >= width) { s_res[0] = bin; s_res[1] = acc; s_res[2] = c[k]; }
        acc += c[k];
    }
}

struct TkShared {
    int hist[TK_L2_BINS];
    uint32_t lkey[TK_LIST];
    int lblk[TK_LIST];                                 // block ids (list) or weights (sweep candidates)
    uint32_t bucket[TK_LIST];                          // block << 1 | above-threshold flag
    int c_gt[256], c_eq[256], c_n[256], c_fill[256];
    int s_w[TK_NW], s_c[TK_NW], s_res[3];
    int s_n, s_last;
};
}  // namespace

// Row histograms and arrival counters of the multi-workgroup rows (one per window row).  Every
// launch leaves both at zero; launches on one device must not overlap.
__device__ int g_tk_hist[WZY_MAX_W * TK_L1_BINS];
__device__ unsigned g_tk_arrive[WZY_MAX_W];
// Per workgroup of a multi-workgroup row: its blocks at or above its own level-1 bin, (key, block),
// and their count (-1: more than TK_LOCAL).  A block of the row's selection is in its workgroup's
// own top `width` cells, so it is in that workgroup's list.
constexpr int TK_LOCAL = 2048, TK_MAX_WG = 64;       // up to 64 x 16,384 blocks per row
__device__ uint2 g_tk_cand[WZY_MAX_W * TK_MAX_WG * TK_LOCAL];
__device__ int g_tk_cand_n[WZY_MAX_W * TK_MAX_WG];

// Levels 2 and 3 over the n listed blocks (LDS), then the output.  b1 / above1: the level-1 bin
// and the weight above it.
WZY_DEV void tk_finish_list(TkShared& S, int n, uint32_t b1, int above1, int n_kv, int width, int B, int* out) {
    const int p = threadIdx.x;
    const int n_bid = n_kv / B, nb = n_bid + 1;
    for (int i = p; i < TK_L2_BINS; i += TK_THREADS) S.hist[i] = 0;
    if (p < 256) { S.c_gt[p] = 0; S.c_eq[p] = 0; S.c_n[p] = 0; S.c_fill[p] = 0; }
    __syncthreads();
    for (int i = p; i < n; i += TK_THREADS) {
        const uint32_t k = S.lkey[i];
        if ((k >> TK_L1_SHIFT) == b1) atomicAdd(&S.hist[(k >> 8) & 0xFFF], tk_weight(S.lblk[i], n_bid, nb, n_kv, B));
    }
    __syncthreads();
    tk_find<TK_L2_BINS / TK_THREADS>(S.hist, TK_L2_BINS, above1, width, S.s_w, S.s_c, S.s_res);
    __syncthreads();
    const uint32_t pre24 = (b1 << 12) | (uint32_t) __builtin_amdgcn_readfirstlane(S.s_res[0]);
    const int above2 = __builtin_amdgcn_readfirstlane(S.s_res[1]);
    if (p < TK_L3_BINS) S.hist[p] = 0;
    __syncthreads();
    for (int i = p; i < n; i += TK_THREADS) {
        const uint32_t k = S.lkey[i];
        if ((k >> 8) == pre24) atomicAdd(&S.hist[k & 0xFF], tk_weight(S.lblk[i], n_bid, nb, n_kv, B));
    }
    __syncthreads();
    tk_find<1>(S.hist, TK_L3_BINS, above2, width, S.s_w, S.s_c, S.s_res);
    __syncthreads();
    const uint32_t thr = (pre24 << 8) | (uint32_t) __builtin_amdgcn_readfirstlane(S.s_res[0]);
    const int budget = width - __builtin_amdgcn_readfirstlane(S.s_res[1]);
    // per-walker totals of the cells above / at the threshold and bucket sizes
    for (int i = p; i < n; i += TK_THREADS) {
        const uint32_t k = S.lkey[i];
        if (k >= thr) {
            const int b = S.lblk[i], t = b & 255;
            atomicAdd(k > thr ? &S.c_gt[t] : &S.c_eq[t], tk_weight(b, n_bid, nb, n_kv, B));
            atomicAdd(&S.c_n[t], 1);
        }
    }
    __syncthreads();
    {   // exclusive scan over the 256 walkers (threads 0..255 hold one each)
        const int g = p < 256 ? S.c_gt[p] : 0, e = p < 256 ? S.c_eq[p] : 0, nn = p < 256 ? S.c_n[p] : 0;
        int gi = g, ei = e;
        block_scan_incl2<TK_NW>(gi, ei, S.s_w, S.s_c);
        __syncthreads();
        int ni = nn, dummy = 0;
        block_scan_incl2<TK_NW>(ni, dummy, S.s_w, S.s_c);
        __syncthreads();
        if (p < 256) { S.c_gt[p] = gi - g; S.c_eq[p] = ei - e; S.c_n[p] = ni - nn; }
    }
    __syncthreads();
    for (int i = p; i < n; i += TK_THREADS) {
        const uint32_t k = S.lkey[i];
        if (k >= thr) {
            const int b = S.lblk[i], t = b & 255;
            S.bucket[S.c_n[t] + atomicAdd(&S.c_fill[t], 1)] = ((uint32_t) b << 1) | (k > thr ? 1u : 0u);
        }
    }
    __syncthreads();
    for (int i = p; i < n; i += TK_THREADS) {
        const uint32_t k = S.lkey[i];
        if (k < thr) continue;
        const int b = S.lblk[i], t = b & 255, j = b >> 8, w = tk_weight(b, n_bid, nb, n_kv, B);
        int gt_before = S.c_gt[t], eq_before = S.c_eq[t];
        const int s0 = S.c_n[t], s1 = s0 + S.c_fill[t];
        for (int q = s0; q < s1; ++q) {
            const uint32_t e = S.bucket[q];
            const int bb = (int) (e >> 1);
            if ((bb >> 8) < j) {
                const int wb = tk_weight(bb, n_bid, nb, n_kv, B);
                if (e & 1u) gt_before += wb; else eq_before += wb;
            }
        }
        const int off = gt_before + min(eq_before, budget);
        const int take = k > thr ? w : max(0, min(w, budget - eq_before));
        for (int c = 0; c < take; ++c) out[off + c] = b * B + c;
    }
}

// Levels 2 and 3 and the output by sweeping every key of the row (the threshold bin holds more
// blocks than the list).  Thread 4t+s walks the s-th quarter of reference walker t's blocks.
WZY_DEV void tk_finish_sweep(TkShared& S, const float* sc, uint32_t b1, int above1, int cnt1, int n_kv, int width,
                             int B, int* out) {
    const int p = threadIdx.x;
    const int n_bid = n_kv / B, nb = n_bid + 1;
    const int tt = p >> 2, sub = p & 3;
    const int J = (nb + 255) / 256, J4 = (J + 3) / 4;
    const int j0 = sub * J4, nq = max(0, min(J, j0 + J4) - j0);
    auto blk = [&](int q) { return tt + 256 * (j0 + q); };
    auto sweep = [&](auto&& f) {
        for (int q0 = 0; q0 < nq; q0 += TK_BATCH) {
            float v[TK_BATCH];
#pragma unroll
            for (int u = 0; u < TK_BATCH; ++u) v[u] = sc[min(blk(q0 + u), nb - 1)];
#pragma unroll
            for (int u = 0; u < TK_BATCH; ++u)
                f(q0 + u, order_key(v[u]), q0 + u < nq ? tk_weight(blk(q0 + u), n_bid, nb, n_kv, B) : 0);
        }
    };
    for (int i = p; i < TK_L2_BINS; i += TK_THREADS) S.hist[i] = 0;
    if (p == 0) S.s_n = 0;
    __syncthreads();
    const bool list = cnt1 <= TK_LIST;               // cells; every listed block holds at least one
    sweep([&](int, uint32_t k, int w) {
        if (w > 0 && (k >> TK_L1_SHIFT) == b1) {
            atomicAdd(&S.hist[(k >> 8) & 0xFFF], w);
            if (list) {
                const int slot = atomicAdd(&S.s_n, 1);
                S.lkey[slot] = k;
                S.lblk[slot] = w;
            }
        }
    });
    __syncthreads();
    tk_find<TK_L2_BINS / TK_THREADS>(S.hist, TK_L2_BINS, above1, width, S.s_w, S.s_c, S.s_res);
    __syncthreads();
    const uint32_t pre24 = (b1 << 12) | (uint32_t) __builtin_amdgcn_readfirstlane(S.s_res[0]);
    const int above2 = __builtin_amdgcn_readfirstlane(S.s_res[1]);
    if (p < TK_L3_BINS) S.hist[p] = 0;
    const int nc = S.s_n;
    __syncthreads();
    if (list) {
        for (int i = p; i < nc; i += TK_THREADS)
            if ((S.lkey[i] >> 8) == pre24) atomicAdd(&S.hist[S.lkey[i] & 0xFF], S.lblk[i]);
    } else {
        sweep([&](int, uint32_t k, int w) {
            if (w > 0 && (k >> 8) == pre24) atomicAdd(&S.hist[k & 0xFF], w);
        });
    }
    __syncthreads();
    tk_find<1>(S.hist, TK_L3_BINS, above2, width, S.s_w, S.s_c, S.s_res);
    __syncthreads();
    const uint32_t thr = (pre24 << 8) | (uint32_t) __builtin_amdgcn_readfirstlane(S.s_res[0]);
    const int above = __builtin_amdgcn_readfirstlane(S.s_res[1]);
    // the threshold-tied cells a thread may take are what is left of the budget after the threads
    // before it, and its output offset is gt_excl + min(eq_excl, eq_budget)
    const int eq_budget = width - above;
    int gt = 0, eq = 0;
    sweep([&](int, uint32_t k, int w) {
        gt += k > thr ? w : 0;
        eq += k == thr ? w : 0;
    });
    int gt_incl = gt, eq_incl = eq;
    block_scan_incl2<TK_NW>(gt_incl, eq_incl, S.s_w, S.s_c);
    const int eq_excl = eq_incl - eq;
    int eq_left = max(0, min(eq, eq_budget - eq_excl));
    int wpos = (gt_incl - gt) + min(eq_excl, eq_budget);
    sweep([&](int q, uint32_t k, int w) {
        if (w == 0) return;
        const int b = blk(q);
        if (k > thr) {
            for (int c = 0; c < w; ++c) out[wpos++] = b * B + c;
        } else if (k == thr && eq_left > 0) {
            const int take = min(w, eq_left);
            for (int c = 0; c < take; ++c) out[wpos++] = b * B + c;
            eq_left -= take;
        }
    });
}

__global__ void __launch_bounds__(TK_THREADS) qsa_topk_kernel(QsaDims dm, const int* __restrict__ pos_dev,
                                                             const float* __restrict__ scores, int max_b,
                                                             int* __restrict__ ghist, unsigned* __restrict__ garrive,
                                                             int* __restrict__ sel_ids, int* __restrict__ sel_cnt) {
    __shared__ TkShared S;
    const int p = threadIdx.x, row = blockIdx.y, G = gridDim.x;
    const int n_kv = *pos_dev + row + 1, K = dm.topk, B = dm.iblk;
    const int width = min(n_kv, K);
    int* out = sel_ids + (size_t) row * K;
    if (n_kv <= K) {                                 // short context: every cell, in order
        if (blockIdx.x == 0) {
            if (p == 0) sel_cnt[row] = width;
            for (int j = p; j < n_kv; j += TK_THREADS) out[j] = j;
        }
        return;                                      // every workgroup of the row leaves here
    }
    const int n_bid = n_kv / B, nb = min(n_bid + 1, max_b);
    const bool single = nb <= TK_CHUNK;              // the row fits one workgroup's registers
    if (single && blockIdx.x > 0) return;            // (launched for a longer row of the window)
    const float* sc = scores + (size_t) row * max_b;
    const int base = blockIdx.x * TK_CHUNK + p;
    // this workgroup's keys: every load issued before the first is used
    float v[TK_PER];
#pragma unroll
    for (int q = 0; q < TK_PER; ++q) v[q] = sc[min(base + q * TK_THREADS, nb - 1)];
    for (int i = p; i < TK_L1_BINS; i += TK_THREADS) S.hist[i] = 0;
    if (p == 0) S.s_n = 0;
    __syncthreads();
    uint32_t key[TK_PER];
#pragma unroll
    for (int q = 0; q < TK_PER; ++q) {
        key[q] = order_key(v[q]);
        const int w = tk_weight(base + q * TK_THREADS, n_bid, nb, n_kv, B);
        if (w > 0) atomicAdd(&S.hist[key[q] >> TK_L1_SHIFT], w);
    }
    __syncthreads();
    if (!single) {
        // this workgroup's own candidates (blocks at or above its own level-1 bin), listed in
        // device memory for the last workgroup
        tk_find<TK_L1_BINS / TK_THREADS>(S.hist, TK_L1_BINS, 0, width, S.s_w, S.s_c, S.s_res);
        __syncthreads();
        const uint32_t lb1 = (uint32_t) __builtin_amdgcn_readfirstlane(S.s_res[0]);
        unsigned keep = 0u;
#pragma unroll
        for (int q = 0; q < TK_PER; ++q)
            if (tk_weight(base + q * TK_THREADS, n_bid, nb, n_kv, B) > 0 && (key[q] >> TK_L1_SHIFT) >= lb1)
                keep |= 1u << q;
        const int cnt = __builtin_popcount(keep);
        int incl = cnt, dummy = 0;
        block_scan_incl2<TK_NW>(incl, dummy, S.s_w, S.s_c);
        if (p == TK_THREADS - 1) S.s_n = incl;       // blocks this workgroup lists
        __syncthreads();
        const int total = S.s_n;
        if (total <= TK_LOCAL) {
            uint2* L = g_tk_cand + ((size_t) row * TK_MAX_WG + blockIdx.x) * TK_LOCAL;
            int slot = incl - cnt;
#pragma unroll
            for (int q = 0; q < TK_PER; ++q)
                if (keep & (1u << q)) L[slot++] = make_uint2(key[q], (uint32_t) (base + q * TK_THREADS));
        }
        if (p == 0) g_tk_cand_n[(size_t) row * TK_MAX_WG + blockIdx.x] = total <= TK_LOCAL ? total : -1;
        // add this histogram to the row's; the last workgroup to arrive takes the row from here
        int* gh = ghist + (size_t) row * TK_L1_BINS;
        for (int i = p; i < TK_L1_BINS; i += TK_THREADS) {
            const int c = S.hist[i];
            if (c) atomicAdd(&gh[i], c);
        }
        __threadfence();
        __syncthreads();
        if (p == 0) S.s_last = atomicAdd(&garrive[row], 1u) == (unsigned) (G - 1);
        __syncthreads();
        if (!S.s_last) return;
        __threadfence();
        int c[TK_L1_BINS / TK_THREADS];
#pragma unroll
        for (int k = 0; k < TK_L1_BINS / TK_THREADS; ++k) c[k] = gh[p + k * TK_THREADS];   // all loads first
        if (p < G && g_tk_cand_n[(size_t) row * TK_MAX_WG + p] < 0) S.s_last = -1;     // a list overflowed
        if (p == 0) S.s_n = 0;                       // (read by every thread before the last barrier)
#pragma unroll
        for (int k = 0; k < TK_L1_BINS / TK_THREADS; ++k) {
            S.hist[p + k * TK_THREADS] = c[k];
            gh[p + k * TK_THREADS] = 0;
        }
        if (p == 0) garrive[row] = 0u;
        __syncthreads();
    }
    if (p == 0) sel_cnt[row] = width;
    tk_find<TK_L1_BINS / TK_THREADS>(S.hist, TK_L1_BINS, 0, width, S.s_w, S.s_c, S.s_res);
    __syncthreads();
    const uint32_t b1 = (uint32_t) __builtin_amdgcn_readfirstlane(S.s_res[0]);
    const int above1 = __builtin_amdgcn_readfirstlane(S.s_res[1]);
    const int cnt1 = __builtin_amdgcn_readfirstlane(S.s_res[2]);
    if (above1 + cnt1 > TK_LIST) {                    // more candidate blocks than the list holds
        tk_finish_sweep(S, sc, b1, above1, cnt1, n_kv, width, B, out);
        return;
    }
    // list the blocks at or above the level-1 bin
    if (single) {
        unsigned keep = 0u;
#pragma unroll
        for (int q = 0; q < TK_PER; ++q)
            if (tk_weight(base + q * TK_THREADS, n_bid, nb, n_kv, B) > 0 && (key[q] >> TK_L1_SHIFT) >= b1)
                keep |= 1u << q;
        const int cnt = __builtin_popcount(keep);
        int incl = cnt, dummy = 0;
        block_scan_incl2<TK_NW>(incl, dummy, S.s_w, S.s_c);
        int slot = incl - cnt;
#pragma unroll
        for (int q = 0; q < TK_PER; ++q)
            if (keep & (1u << q)) { S.lkey[slot] = key[q]; S.lblk[slot] = base + q * TK_THREADS; ++slot; }
        if (p == TK_THREADS - 1) S.s_n = incl;
    } else if (S.s_last >= 0) {
        // the workgroups' own lists hold every candidate: keep those at or above the row's bin
        const uint2* L = g_tk_cand + (size_t) row * TK_MAX_WG * TK_LOCAL;
        for (int i = p; i < G * TK_LOCAL; i += TK_THREADS) {
            const int g = i / TK_LOCAL;
            if (i - g * TK_LOCAL < g_tk_cand_n[(size_t) row * TK_MAX_WG + g]) {
                const uint2 e = L[i];
                if ((e.x >> TK_L1_SHIFT) >= b1) {
                    const int slot = atomicAdd(&S.s_n, 1);
                    S.lkey[slot] = e.x;
                    S.lblk[slot] = (int) e.y;
                }
            }
        }
    } else {
        for (int b0 = p; b0 < nb; b0 += TK_THREADS * TK_BATCH) {
            float u[TK_BATCH];
#pragma unroll
            for (int i = 0; i < TK_BATCH; ++i) u[i] = sc[min(b0 + i * TK_THREADS, nb - 1)];
#pragma unroll
            for (int i = 0; i < TK_BATCH; ++i) {
                const int b = b0 + i * TK_THREADS;
                const uint32_t k = order_key(u[i]);
                if (b < nb && tk_weight(b, n_bid, nb, n_kv, B) > 0 && (k >> TK_L1_SHIFT) >= b1) {
                    const int slot = atomicAdd(&S.s_n, 1);
                    S.lkey[slot] = k;
                    S.lblk[slot] = b;
                }
            }
        }
    }
    __syncthreads();
    tk_finish_list(S, S.s_n, b1, above1, n_kv, width, B, out);
}

// ---------------------------------------------------------------------------------------------
// sparse attention over one chunk of 64 selected cells
// ---------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) qsa_attn_kernel(QsaAttnArgs a) {
    __shared__ __align__(16) int8_t s_k[QSA_ATT_CHUNK * ATT_ROW];
    __shared__ __align__(16) int8_t s_v[QSA_ATT_CHUNK * ATT_ROW];
    __shared__ float s_ks[QSA_ATT_CHUNK][4], s_vs[QSA_ATT_CHUNK][4];
    __shared__ __align__(16) float s_q[ATT_HPW][256];
    __shared__ __align__(16) float s_p[QSA_ATT_CHUNK][ATT_HPW];   // softmax weights, [cell][head]
    __shared__ long long s_slot[QSA_ATT_CHUNK];
    const QsaDims& dm = a.dm;
    const int gq = dm.qh / dm.kvh, nhs = (gq + ATT_HPW - 1) / ATT_HPW;
    const int c = blockIdx.x, j = blockIdx.y / nhs, hs = blockIdx.y % nhs, t = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int kvd = dm.kvh * 256;
    const int n_kv = *a.pos + t + 1;
    int p0, width;
    qsa_span(dm, n_kv, a.floor, p0, width);
    const int c0 = c * QSA_ATT_CHUNK;
    if (c0 >= width) return;                         // workgroup-uniform
    const int ncell = min(QSA_ATT_CHUNK, width - c0);
    const int nch = (dm.topk + QSA_ATT_CHUNK - 1) / QSA_ATT_CHUNK;
    // fp16 operands when the window reaches past f16_above cells (uniform over the launch)
    const bool f16 = dm.f16_above > 0 && *a.pos + (int) gridDim.z > dm.f16_above;

    if (tid < QSA_ATT_CHUNK) {
        const int idx = c0 + tid;
        long long sl = -1;
        if (tid < ncell) {
            const int p = dm.window > 0 ? p0 + idx : (n_kv <= dm.topk ? idx : a.sel_ids[(size_t) t * dm.topk + idx]);
            sl = (long long) qsa_kv_slot(p, dm);
        }
        s_slot[tid] = sl;
    }
    {                                                // this slice's heads; rows past gq are zero
        const int hh = tid >> 6, d4 = tid & 63, h = hs * ATT_HPW + hh;
        const float4 q = h < gq ? *(const float4*) (a.qg + (size_t) t * dm.qh * 512 + (size_t) (j * gq + h) * 512 + 4 * d4)
                                : make_float4(0.f, 0.f, 0.f, 0.f);
        if (f16) {                                   // fp16(q / 16) pairs, as the reference's GQA kernel stages q
            half2_t* qh = (half2_t*) &s_q[hh][0];
            qh[2 * d4] = half2_t{(_Float16) (q.x * 0.0625f), (_Float16) (q.y * 0.0625f)};
            qh[2 * d4 + 1] = half2_t{(_Float16) (q.z * 0.0625f), (_Float16) (q.w * 0.0625f)};
        } else {
            *(float4*) &s_q[hh][4 * d4] = q;
        }
    }
    __syncthreads();

    // K and V rows of the chunk: 64 cells x 16 int4 each, 4 per thread, one round of loads
    {
        int4 kr[4], vr[4];
        const int part = tid & 15;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const long long sl = s_slot[(tid >> 4) + 16 * k];
            const size_t off = (size_t) (sl >= 0 ? sl : 0) * kvd + (size_t) j * 256 + (size_t) part * 16;
            kr[k] = *(const int4*) (a.kv.kq + off);
            vr[k] = *(const int4*) (a.kv.vq + off);
        }
        const int cs = tid >> 2, g = tid & 3;
        const long long sls = s_slot[cs];
        const size_t soff = (size_t) (sls >= 0 ? sls : 0) * (kvd / 64) + (size_t) j * 4 + g;
        const uint16_t kh = a.kv.ks[soff], vh = a.kv.vs[soff];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int cell = (tid >> 4) + 16 * k;
            const bool ok = s_slot[cell] >= 0;
            *(int4*) (s_k + cell * ATT_ROW + part * 16) = ok ? kr[k] : make_int4(0, 0, 0, 0);
            *(int4*) (s_v + cell * ATT_ROW + part * 16) = ok ? vr[k] : make_int4(0, 0, 0, 0);
        }
        s_ks[cs][g] = sls >= 0 ? h16_to_f(kh) : 0.f;
        s_vs[cs][g] = sls >= 0 ? h16_to_f(vh) : 0.f;
    }
    __syncthreads();

    // scores and local softmax: lane = cell, wave w owns head hs*ATT_HPW + w
    {
        const int cell = lane;
        float acc = 0.f;
        if (!f16) {                                  // int8 codes dotted with q, scaled per 64-group
#pragma unroll 1
            for (int g = 0; g < 4; ++g) {
                float ag = 0.f;
#pragma unroll
                for (int pp = 0; pp < 4; ++pp) {
                    const int part = 4 * g + pp;
                    const int4 kv = *(const int4*) (s_k + cell * ATT_ROW + part * 16);
                    const int8_t* kb = (const int8_t*) &kv;
                    const float4* qp = (const float4*) &s_q[w][part * 16];
                    const float4 q0 = qp[0], q1 = qp[1], q2 = qp[2], q3 = qp[3];
                    ag = fmaf((float) kb[0], q0.x, ag); ag = fmaf((float) kb[1], q0.y, ag);
                    ag = fmaf((float) kb[2], q0.z, ag); ag = fmaf((float) kb[3], q0.w, ag);
                    ag = fmaf((float) kb[4], q1.x, ag); ag = fmaf((float) kb[5], q1.y, ag);
                    ag = fmaf((float) kb[6], q1.z, ag); ag = fmaf((float) kb[7], q1.w, ag);
                    ag = fmaf((float) kb[8], q2.x, ag); ag = fmaf((float) kb[9], q2.y, ag);
                    ag = fmaf((float) kb[10], q2.z, ag); ag = fmaf((float) kb[11], q2.w, ag);
                    ag = fmaf((float) kb[12], q3.x, ag); ag = fmaf((float) kb[13], q3.y, ag);
                    ag = fmaf((float) kb[14], q3.z, ag); ag = fmaf((float) kb[15], q3.w, ag);
                }
                acc = fmaf(ag, s_ks[cell][g], acc);
            }
            acc *= 0.0625f;
        } else {
            // fp16(code * scale) dotted with fp16(q / 16), two values per step: the codes become exact
            // fp16 pairs (the biased byte u = code + 128 under the exponent of 1024 is 1024 + u, minus
            // 1152), the packed fp16 multiply rounds code * scale to nearest even as the reference's
            // __hmul does, and v_dot2_f32_f16 adds the two exact products into the fp32 sum
            const half2_t* qh = (const half2_t*) &s_q[w][0];
            const half2_t bias = {(_Float16) 1152.0f, (_Float16) 1152.0f};
#pragma unroll 1
            for (int g = 0; g < 4; ++g) {
                const _Float16 sh = (_Float16) s_ks[cell][g];    // an fp16 value: exact
                const half2_t sc2 = {sh, sh};
#pragma unroll
                for (int pp = 0; pp < 4; ++pp) {
                    const int part = 4 * g + pp;
                    const int4 kv = *(const int4*) (s_k + cell * ATT_ROW + part * 16);
                    const uint32_t wd[4] = {(uint32_t) kv.x, (uint32_t) kv.y, (uint32_t) kv.z, (uint32_t) kv.w};
#pragma unroll
                    for (int jw = 0; jw < 4; ++jw) {
                        const uint32_t u = wd[jw] ^ 0x80808080u;
                        const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);   // bytes 0, 1
                        const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);   // bytes 2, 3
                        const half2_t k01 = (__builtin_bit_cast(half2_t, lo) - bias) * sc2;
                        const half2_t k23 = (__builtin_bit_cast(half2_t, hi) - bias) * sc2;
                        acc = __builtin_amdgcn_fdot2(k01, qh[part * 8 + 2 * jw], acc, false);
                        acc = __builtin_amdgcn_fdot2(k23, qh[part * 8 + 2 * jw + 1], acc, false);
                    }
                }
            }
        }
        const int h = hs * ATT_HPW + w;
        if (h < gq) {                                // wave-uniform
            const float s = cell < ncell ? acc : -INFINITY;
            float m, e, l;
            if (!f16) {
                m = wave_max(s);
                e = cell < ncell ? __expf(s - m) : 0.f;
                l = wave_sum(e);
            } else {
                // the reference's online softmax over 32-cell steps (cells 0-31, 32-63 of the chunk):
                // weights exp(s - m_step) rounded to fp16 for the V product, summed unrounded; the
                // first step's weights rescaled by alpha = exp(m0 - m1) when the second step raises
                // the running max (src/wzy_qsa_wmma.cuh:401-420).  The running max here starts at
                // the chunk (the reference's carries over from earlier chunks): the fp16 rounding is
                // relative either way, 2^-11 of a weight.
                const float ms = max32(s);           // this lane's step maximum
                const float m0 = as_f(__builtin_amdgcn_readlane(as_i(ms), 0));
                const float m1 = fmaxf(m0, as_f(__builtin_amdgcn_readlane(as_i(ms), 32)));
                const bool first = cell < 32;
                const float ex = cell < ncell ? __expf(s - (first ? m0 : m1)) : 0.f;
                const float alpha = first ? __expf(m0 - m1) : 1.0f;
                l = wave_sum(ex * alpha);
                e = round_h16(ex) * alpha;
                m = m1;
            }
            s_p[cell][w] = e;
            float* ml = a.part_ml + ((((size_t) t * dm.kvh + j) * nch + c) * gq + h) * 2;
            if (lane == 0) { ml[0] = m; ml[1] = l; }
        } else {
            s_p[cell][w] = 0.f;
        }
    }
    __syncthreads();

    // V: thread d owns output dim d for the slice's heads
    {
        const int d = tid;
        float o[ATT_HPW];
#pragma unroll
        for (int hh = 0; hh < ATT_HPW; ++hh) o[hh] = 0.f;
#pragma unroll 4
        for (int cell = 0; cell < ncell; ++cell) {
            float pv = (float) s_v[cell * ATT_ROW + d] * s_vs[cell][d >> 6];
            if (f16) pv = round_h16(pv);
            const float4 p = *(const float4*) s_p[cell];
            o[0] = fmaf(p.x, pv, o[0]);
            o[1] = fmaf(p.y, pv, o[1]);
            o[2] = fmaf(p.z, pv, o[2]);
            o[3] = fmaf(p.w, pv, o[3]);
        }
        float* po = a.part + ((((size_t) t * dm.kvh + j) * nch + c) * gq) * 256;
#pragma unroll
        for (int hh = 0; hh < ATT_HPW; ++hh) {
            const int h = hs * ATT_HPW + hh;
            if (h < gq) po[(size_t) h * 256 + d] = o[hh];
        }
    }
}

// merge the chunks of one (q head, row): thread d = output dim
__global__ void __launch_bounds__(256) qsa_combine_kernel(QsaAttnArgs a) {
    const QsaDims& dm = a.dm;
    const int h = blockIdx.x, t = blockIdx.y, d = threadIdx.x, lane = d & 63;
    const int gq = dm.qh / dm.kvh, j = h / gq, hh = h % gq;
    const int n_kv = *a.pos + t + 1;
    int p0, width;
    qsa_span(dm, n_kv, a.floor, p0, width);
    const int nch_all = (dm.topk + QSA_ATT_CHUNK - 1) / QSA_ATT_CHUNK;
    const int nch = (width + QSA_ATT_CHUNK - 1) / QSA_ATT_CHUNK;
    if (nch == 0) {                                  // nothing attended (a floor above the row)
        a.out[(size_t) t * dm.qh * 256 + (size_t) h * 256 + d] = 0.f;
        return;
    }
    const size_t base = ((size_t) t * dm.kvh + j) * nch_all;
    // chunk statistics: lane c holds chunk c
    const float m_c = lane < nch ? a.part_ml[((base + lane) * gq + hh) * 2] : -INFINITY;
    const float l_c = lane < nch ? a.part_ml[((base + lane) * gq + hh) * 2 + 1] : 0.f;
    float part[ATT_CH_MAX];
#pragma unroll
    for (int c = 0; c < ATT_CH_MAX; ++c)
        part[c] = c < nch ? a.part[((base + c) * gq + hh) * 256 + d] : 0.f;
    const float M = wave_max(m_c);
    const float f_c = lane < nch ? __expf(m_c - M) : 0.f;
    const float L = wave_sum(l_c * f_c);
    float O = 0.f;
#pragma unroll
    for (int c = 0; c < ATT_CH_MAX; ++c)
        if (c < nch) O = fmaf(part[c], as_f(__builtin_amdgcn_readlane(as_i(f_c), c)), O);
    const float gate = a.qg[(size_t) t * dm.qh * 512 + (size_t) h * 512 + 256 + d];
    a.out[(size_t) t * dm.qh * 256 + (size_t) h * 256 + d] = (O * (1.0f / L)) / (1.0f + __expf(-gate));
}

// ---------------------------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------------------------
namespace wzy {

int launch_qsa_topk(const QsaDims& dm, const int* pos, const float* scores, int max_b, int* sel_ids, int* sel_cnt,
                    int T, hipStream_t st) {
    WZY_TRY(qsa_check_dims(dm));
    WZY_REQUIRE(T >= 1 && T <= WZY_MAX_W, "qsa_topk: T out of range");
    WZY_REQUIRE(max_b >= 1 && max_b <= (1 << 22), "qsa_topk: max_b %d out of range", max_b);
    int* hist = nullptr;
    unsigned* arrive = nullptr;
    WZY_HIP_TRY(hipGetSymbolAddress((void**) &hist, HIP_SYMBOL(g_tk_hist)));
    WZY_HIP_TRY(hipGetSymbolAddress((void**) &arrive, HIP_SYMBOL(g_tk_arrive)));
    const int G = (max_b + TK_CHUNK - 1) / TK_CHUNK;
    WZY_REQUIRE(G <= TK_MAX_WG, "qsa_topk: %d indexer blocks exceed %d", max_b, TK_MAX_WG * TK_CHUNK);
    hipLaunchKernelGGL(qsa_topk_kernel, dim3(G, T), dim3(TK_THREADS), 0, st, dm, pos, scores, max_b, hist, arrive,
                       sel_ids, sel_cnt);
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

int launch_qsa_topk_rows(const QsaDims& dm, const int* pos, const float* scores, int max_b, int* sel_ids, int* sel_cnt,
                         int rows, int max_n_kv, hipStream_t st) {
    WZY_TRY(qsa_check_dims(dm));
    WZY_REQUIRE(rows >= 1 && rows <= 65535, "qsa_topk: %d rows", rows);
    WZY_REQUIRE(max_b >= 1 && max_b <= (1 << 22), "qsa_topk: max_b %d out of range", max_b);
    // every row must take the one-workgroup path (its blocks fit one workgroup's registers): the
    // multi-workgroup merge keeps per-row counters for at most WZY_MAX_W rows
    WZY_REQUIRE(max_n_kv / dm.iblk + 1 <= TK_CHUNK, "qsa_topk: %d cells exceed one workgroup's %d blocks", max_n_kv,
                TK_CHUNK);
    int* hist = nullptr;
    unsigned* arrive = nullptr;
    WZY_HIP_TRY(hipGetSymbolAddress((void**) &hist, HIP_SYMBOL(g_tk_hist)));
    WZY_HIP_TRY(hipGetSymbolAddress((void**) &arrive, HIP_SYMBOL(g_tk_arrive)));
    hipLaunchKernelGGL(qsa_topk_kernel, dim3(1, rows), dim3(TK_THREADS), 0, st, dm, pos, scores, max_b, hist, arrive,
                       sel_ids, sel_cnt);
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

size_t qsa_attn_part_floats(const QsaDims& dm, int T) {
    const int nch = (dm.topk + QSA_ATT_CHUNK - 1) / QSA_ATT_CHUNK;
    return (size_t) T * dm.kvh * nch * dm.qh / dm.kvh * dm.hd;
}

int launch_qsa_attn(const QsaAttnArgs& a, int T, hipStream_t st) {
    WZY_TRY(qsa_check_dims(a.dm));
    WZY_REQUIRE(T >= 1 && T <= WZY_MAX_W, "qsa_attn: T out of range");
    WZY_REQUIRE(a.dm.topk <= ATT_CH_MAX * QSA_ATT_CHUNK, "qsa_attn: topk above %d", ATT_CH_MAX * QSA_ATT_CHUNK);
    const int nch = (a.dm.topk + QSA_ATT_CHUNK - 1) / QSA_ATT_CHUNK;
    const int nhs = (a.dm.qh / a.dm.kvh + ATT_HPW - 1) / ATT_HPW;
    hipLaunchKernelGGL(qsa_attn_kernel, dim3(nch, a.dm.kvh * nhs, T), dim3(256), 0, st, a);
    hipLaunchKernelGGL(qsa_combine_kernel, dim3(a.dm.qh, T), dim3(256), 0, st, a);
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

}  // namespace wzy

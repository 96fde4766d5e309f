// qsa_attn.hip -- QSA cell selection and sparse attention for gfx950.
//
//  qsa_topk   exact top-`topk` cells of one row, one 1024-thread workgroup: the block scores are
//             loaded once into registers as order-preserving keys, 2048-bin histograms over the
//             keys' own range (narrowed pass by pass) and a final ranking of the few blocks left
//             find the threshold key, then every block above the threshold is taken whole and
//             blocks at the threshold are filled in the reference's tie order.  The reference walks the blocks with 256 threads,
//             thread t owning blocks t, t+256, ... and emitting them thread-major; here thread
//             4t+s owns the s-th quarter of thread t's blocks, so a scan in thread order reproduces
//             that order exactly.  reference: qsa_block_topk_multi (src/wzy_qsa_256k.cuh:226-403)
//  qsa_attn   split-K sparse attention: workgroup (chunk of 64 selected cells, kv head, slice of 4
//             q heads, row) stages the chunk's INT8 K and V rows in LDS with one round of 128-bit
//             loads, computes its heads' scores (wave = head, lane = cell), a local softmax, and the
//             INT8 V sum (thread = dim).
//  qsa_combine merges the chunks (max / sum rescaling) and applies sigmoid(gate).
//             reference: qsa_attend_int8_sparse_multi (src/wzy_qsa_256k.cuh:407-532)
#include "wzy_device.h"
#include "wzy_host.h"
#include "wzy_qsa.h"

using namespace wzy;

namespace {

constexpr int TK_THREADS = 1024;
constexpr int TK_MAXJ_SMALL = 16;    // blocks per thread: 16384 blocks (65532 cells at 4 per block)
constexpr int TK_MAXJ_LARGE = 66;    // 67584 blocks (270332 cells); keys partly spill to scratch
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

constexpr int TK_NBIN = 2 * TK_THREADS;   // histogram bins per pass (two per thread in the scan)
constexpr int TK_LOG_NBIN = 11;
constexpr int TK_CAND = 256;               // threshold-bin weight at which the pass loop hands over to ranking

}  // namespace

// ---------------------------------------------------------------------------------------------
// exact top-k cell selection, one workgroup per row; TK_MAXJ = blocks held per thread.
// Threshold search: the order keys of the row's blocks span [kmin, kmax]; a pass histograms the
// keys of a window [lo, lo + TK_NBIN << shift) into TK_NBIN bins of 2^shift keys (block weights =
// cells), and one scan from the top bin down finds the bin holding the width-th cell.  The window
// narrows to that bin; once its weight is at most TK_CAND (or a bin is a single key) its few blocks
// are ranked against each other directly.  The threshold is the key value thr with
// weight(key > thr) < width <= weight(key >= thr), the same value a digit-by-digit radix select finds.
// ---------------------------------------------------------------------------------------------
template <int TK_MAXJ>
__global__ void __launch_bounds__(TK_THREADS) qsa_topk_kernel(QsaDims dm, const int* __restrict__ pos_dev,
                                                              const float* __restrict__ scores, int max_b,
                                                              int* __restrict__ sel_ids, int* __restrict__ sel_cnt) {
    constexpr int NW = TK_THREADS / 64;
    __shared__ int hist[TK_NBIN];
    __shared__ uint32_t s_ck[TK_CAND];
    __shared__ int s_cw[TK_CAND];
    __shared__ int s_w[NW], s_c[NW];
    __shared__ uint32_t s_mn[NW], s_mx[NW];
    __shared__ int s_bin, s_above, s_cnt, s_ncand;
    __shared__ uint32_t s_thr;
    const int p = threadIdx.x, row = blockIdx.x, lane = p & 63, w = p >> 6;
    const int n_kv = *pos_dev + row + 1;
    const int K = dm.topk, B = dm.iblk;
    const int width = min(n_kv, K);
    int* out = sel_ids + (size_t) row * K;
    if (p == 0) sel_cnt[row] = width;
    if (n_kv <= K) {                                 // short context: every cell, in order
        for (int j = p; j < n_kv; j += TK_THREADS) out[j] = j;
        return;
    }
    const int n_bid = n_kv / B, nb = min(n_bid + 1, max_b);   // complete blocks + the open block
    const int tt = p >> 2, sub = p & 3;
    const int J = (nb + 255) / 256, J4 = (J + 3) / 4;
    const int j0 = sub * J4, j1 = min(J, j0 + J4);
    const float* sc = scores + (size_t) row * max_b;

    // weight (cells) of this thread's q-th block: B for complete blocks, the open block's fill, 0 past the end
    auto wgt = [&](int q) -> int {
        const int b = tt + 256 * (j0 + q);
        return ((j0 + q) < j1 && b < nb) ? (b < n_bid ? B : n_kv - n_bid * B) : 0;
    };
    // every score load is issued before the first key is formed (clamped index, no branch around
    // a load, so no load waits for an earlier one)
    float sv[TK_MAXJ];
#pragma unroll
    for (int q = 0; q < TK_MAXJ; ++q) sv[q] = sc[min(tt + 256 * (j0 + q), nb - 1)];
    for (int i = p; i < TK_NBIN; i += TK_THREADS) hist[i] = 0;
    if (p == 0) s_ncand = 0;
    uint32_t key[TK_MAXJ];
    uint32_t mn = 0xFFFFFFFFu, mx = 0u;
#pragma unroll
    for (int q = 0; q < TK_MAXJ; ++q) {
        key[q] = order_key(sv[q]);
        if (wgt(q) > 0) { mn = min(mn, key[q]); mx = max(mx, key[q]); }
    }
    mn = wave_min_u32(mn);
    mx = wave_max_u32(mx);
    if (lane == 0) { s_mn[w] = mn; s_mx[w] = mx; }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NW; ++i) { mn = min(mn, s_mn[i]); mx = max(mx, s_mx[i]); }

    // window passes: at most three (shift 21 -> 10 -> 0)
    uint32_t lo = mn;
    const uint32_t range = mx - mn;
    int shift = range ? max(0, 32 - __builtin_clz(range) - TK_LOG_NBIN) : 0;
    int above = 0, cnt = 0;
    uint32_t thr = mn;                               // one key value in the whole row: no pass needed
    bool ranked = false;
    while (range != 0) {
#pragma unroll
        for (int q = 0; q < TK_MAXJ; ++q) {
            const uint32_t d = key[q] - lo;
            if (wgt(q) > 0 && key[q] >= lo && (d >> shift) < (uint32_t) TK_NBIN) atomicAdd(&hist[d >> shift], wgt(q));
        }
        __syncthreads();
        // thread p owns bins TK_NBIN-1-2p (h1) and TK_NBIN-2-2p (h0): thread order = descending keys
        const int b1 = TK_NBIN - 1 - 2 * p, b0 = b1 - 1;
        const int h1 = hist[b1], h0 = hist[b0];
        hist[b1] = 0;                                // cleared for the next pass
        hist[b0] = 0;
        int incl = h1 + h0, dummy = 0;
        block_scan_incl2<NW>(incl, dummy, s_w, s_c);
        const int before = above + incl - (h1 + h0);
        if (before < width && before + h1 >= width) { s_bin = b1; s_above = before; s_cnt = h1; }
        if (before + h1 < width && before + h1 + h0 >= width) { s_bin = b0; s_above = before + h1; s_cnt = h0; }
        __syncthreads();
        lo += (uint32_t) __builtin_amdgcn_readfirstlane(s_bin) << shift;
        above = __builtin_amdgcn_readfirstlane(s_above);
        cnt = __builtin_amdgcn_readfirstlane(s_cnt);
        if (shift == 0) { thr = lo; break; }         // the bin is one key value
        if (cnt <= TK_CAND) { ranked = true; break; }
        shift = max(0, shift - TK_LOG_NBIN);
    }
    if (ranked) {
        // the threshold bin [lo, lo + 2^shift) holds at most TK_CAND cells, so at most TK_CAND blocks:
        // gather them, and each ranks itself against the others
#pragma unroll
        for (int q = 0; q < TK_MAXJ; ++q) {
            if (wgt(q) > 0 && key[q] >= lo && ((key[q] - lo) >> shift) == 0u) {
                const int slot = atomicAdd(&s_ncand, 1);
                s_ck[slot] = key[q];
                s_cw[slot] = wgt(q);
            }
        }
        __syncthreads();
        const int nc = s_ncand;
        if (p < nc) {
            const uint32_t k = s_ck[p];
            int gtw = 0, eqw = 0;
            for (int j = 0; j < nc; ++j) {
                const uint32_t kj = s_ck[j];
                const int wj = s_cw[j];
                gtw += kj > k ? wj : 0;
                eqw += kj == k ? wj : 0;
            }
            if (above + gtw < width && above + gtw + eqw >= width) {   // every such block holds the same key
                s_thr = k;
                s_above = above + gtw;
            }
        }
        __syncthreads();
        thr = s_thr;
        above = s_above;
    }

    const int eq_budget = width - above;
    int gt = 0, eq = 0;
#pragma unroll
    for (int q = 0; q < TK_MAXJ; ++q) {
        const int wq = wgt(q);
        if (wq == 0) continue;
        if (key[q] > thr) gt += wq;
        else if (key[q] == thr) eq += wq;
    }
    // one dual scan: the threshold-tied cells a thread may take are what is left of the budget
    // after the threads before it, and its output offset is gt_excl + min(eq_excl, eq_budget)
    int gt_incl = gt, eq_incl = eq;
    block_scan_incl2<NW>(gt_incl, eq_incl, s_w, s_c);
    const int eq_excl = eq_incl - eq;
    const int my_eq = max(0, min(eq, eq_budget - eq_excl));
    int wpos = (gt_incl - gt) + min(eq_excl, eq_budget);
    int eq_left = my_eq;
#pragma unroll
    for (int q = 0; q < TK_MAXJ; ++q) {
        const int wq = wgt(q);
        if (wq == 0) continue;
        const int b = tt + 256 * (j0 + q);
        if (key[q] > thr) {
            for (int c = 0; c < wq; ++c) out[wpos++] = b * B + c;
        } else if (key[q] == thr && eq_left > 0) {
            const int take = min(wq, eq_left);
            for (int c = 0; c < take; ++c) out[wpos++] = b * B + c;
            eq_left -= take;
        }
    }
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
    const int width = min(n_kv, dm.topk);
    const int c0 = c * QSA_ATT_CHUNK;
    if (c0 >= width) return;                         // workgroup-uniform
    const int ncell = min(QSA_ATT_CHUNK, width - c0);
    const int nch = (dm.topk + QSA_ATT_CHUNK - 1) / QSA_ATT_CHUNK;

    if (tid < QSA_ATT_CHUNK) {
        const int idx = c0 + tid;
        long long sl = -1;
        if (tid < ncell) sl = (long long) qsa_kv_slot(n_kv <= dm.topk ? idx : a.sel_ids[(size_t) t * dm.topk + idx], dm);
        s_slot[tid] = sl;
    }
    {                                                // this slice's heads; rows past gq are zero
        const int hh = tid >> 6, d4 = tid & 63, h = hs * ATT_HPW + hh;
        *(float4*) &s_q[hh][4 * d4] =
            h < gq ? *(const float4*) (a.qg + (size_t) t * dm.qh * 512 + (size_t) (j * gq + h) * 512 + 4 * d4)
                   : make_float4(0.f, 0.f, 0.f, 0.f);
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
        const int h = hs * ATT_HPW + w;
        if (h < gq) {                                // wave-uniform
            const float s = cell < ncell ? acc * 0.0625f : -INFINITY;
            const float m = wave_max(s);
            const float e = cell < ncell ? __expf(s - m) : 0.f;
            const float l = wave_sum(e);
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
            const float pv = (float) s_v[cell * ATT_ROW + d] * s_vs[cell][d >> 6];
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
    const int width = min(n_kv, dm.topk);
    const int nch_all = (dm.topk + QSA_ATT_CHUNK - 1) / QSA_ATT_CHUNK;
    const int nch = (width + QSA_ATT_CHUNK - 1) / QSA_ATT_CHUNK;
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
    const int per_thread = ((max_b + 255) / 256 + 3) / 4;   // blocks a thread holds at the largest context
    WZY_REQUIRE(per_thread <= TK_MAXJ_LARGE, "qsa_topk: %d indexer blocks exceed the selection capacity %d", max_b,
                TK_THREADS * TK_MAXJ_LARGE);
    if (per_thread <= TK_MAXJ_SMALL)
        hipLaunchKernelGGL((qsa_topk_kernel<TK_MAXJ_SMALL>), dim3(T), dim3(TK_THREADS), 0, st, dm, pos, scores, max_b,
                           sel_ids, sel_cnt);
    else
        hipLaunchKernelGGL((qsa_topk_kernel<TK_MAXJ_LARGE>), dim3(T), dim3(TK_THREADS), 0, st, dm, pos, scores, max_b,
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

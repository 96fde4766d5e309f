// qsa_attn.hip -- QSA cell selection and sparse attention for gfx950.
//
//  qsa_topk   exact top-`topk` cells of one row, one 1024-thread workgroup: the block scores are
//             loaded once into registers as order-preserving keys, a 4 x 8-bit radix select finds
//             the threshold key (per-wave LDS histograms per pass, digit found by one wave),
//             then every block above the threshold is taken whole and blocks at the threshold are
//             filled in the reference's tie order.  The reference walks the blocks with 256 threads,
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

// Two inclusive prefix sums at once over the NW*64 threads in thread order (one barrier pair).
template <int NW>
WZY_DEV void block_scan_incl2(int& x, int& y, int* s_x, int* s_y) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int a = __shfl_up(x, o, 64), b = __shfl_up(y, o, 64);
        if (lane >= o) { x += a; y += b; }
    }
    if (lane == 63) { s_x[w] = x; s_y[w] = y; }
    __syncthreads();
    int bx = 0, by = 0;
#pragma unroll
    for (int i = 0; i < NW; ++i)
        if (i < w) { bx += s_x[i]; by += s_y[i]; }
    __syncthreads();
    x += bx;
    y += by;
}

}  // namespace

// ---------------------------------------------------------------------------------------------
// exact top-k cell selection, one workgroup per row; TK_MAXJ = blocks held per thread
// ---------------------------------------------------------------------------------------------
template <int TK_MAXJ>
__global__ void __launch_bounds__(TK_THREADS) qsa_topk_kernel(QsaDims dm, const int* __restrict__ pos_dev,
                                                              const float* __restrict__ scores, int max_b,
                                                              int* __restrict__ sel_ids, int* __restrict__ sel_cnt) {
    __shared__ int hist[TK_THREADS / 64][256];      // one histogram per wave (no cross-wave atomic contention)
    __shared__ int s_w[TK_THREADS / 64];
    __shared__ int s_c[TK_THREADS / 64];
    __shared__ int s_digit, s_above;
    const int p = threadIdx.x, row = blockIdx.x;
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
    uint32_t key[TK_MAXJ];
#pragma unroll
    for (int q = 0; q < TK_MAXJ; ++q) {
        const int b = tt + 256 * (j0 + q);
        key[q] = ((j0 + q) < j1 && b < nb) ? order_key(sv[q]) : 0u;
    }

    uint32_t prefix = 0;
    int above = 0;
    for (int i = p; i < (TK_THREADS / 64) * 256; i += TK_THREADS) (&hist[0][0])[i] = 0;
    __syncthreads();
    for (int shift = 24; shift >= 0; shift -= 8) {
        const uint32_t hi_mask = (shift == 24) ? 0u : (0xffffffffu << (shift + 8));
#pragma unroll
        for (int q = 0; q < TK_MAXJ; ++q)
            if (wgt(q) > 0 && (key[q] & hi_mask) == (prefix & hi_mask)) atomicAdd(&hist[p >> 6][(key[q] >> shift) & 255u], wgt(q));
        __syncthreads();
        // wave 0 picks the digit: lane l holds digits 255-4l .. 252-4l (highest first); the
        // threshold digit is the highest one at which the weight at or above it reaches the width
        if (p < 64) {
            const int l = p;
            int h[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                int sum = 0;
#pragma unroll
                for (int wv = 0; wv < TK_THREADS / 64; ++wv) {
                    sum += hist[wv][255 - 4 * l - j];
                    hist[wv][255 - 4 * l - j] = 0;   // cleared for the next pass
                }
                h[j] = sum;
            }
            const int s4 = h[0] + h[1] + h[2] + h[3];
            int incl = s4;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int y = __shfl_up(incl, o, 64);
                if (l >= o) incl += y;
            }
            int cum = above + incl - s4;             // weight of digits above this lane's first
            int jl = -1, base_above = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (jl < 0 && cum + h[j] >= width) { jl = j; base_above = cum; }
                cum += h[j];
            }
            const unsigned long long m = __ballot(jl >= 0);
            const int lstar = m ? __ffsll((long long) m) - 1 : 63;
            if (l == lstar) {
                const int js = jl >= 0 ? jl : 3;
                s_digit = 255 - 4 * l - js;
                s_above = jl >= 0 ? base_above : cum - h[3];
            }
        }
        __syncthreads();
        prefix |= (uint32_t) s_digit << shift;
        above = s_above;
    }

    const uint32_t thr = prefix;
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
    block_scan_incl2<TK_THREADS / 64>(gt_incl, eq_incl, s_w, s_c);
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

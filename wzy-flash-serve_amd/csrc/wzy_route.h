// wzy_route.h -- softmax top-K routing of one row in one wave (device code shared by the decode
// MoE block and the prefill MoE).
#pragma once
#include "wzy_device.h"

namespace wzy {

// Routing key of one (probability, expert id): probabilities are >= 0, so their float bits order
// like the values; the low word ranks lower ids first.  Key 0 ranks below every real entry.
WZY_DEV uint64_t route_key(float p, int id) {
    return ((uint64_t) __builtin_bit_cast(uint32_t, p) << 32) | (uint32_t) (0xFFFFFFFFu - (uint32_t) id);
}

// Bitonic sort of RV keys into descending order, in registers.
template <int RV>
WZY_DEV void sort_keys_desc(uint64_t (&k)[RV]) {
#pragma unroll
    for (int s = 2; s <= RV; s <<= 1)
#pragma unroll
        for (int j = s >> 1; j > 0; j >>= 1)
#pragma unroll
            for (int i = 0; i < RV; ++i) {
                const int l = i ^ j;
                if (l > i) {
                    const bool desc = (i & s) == 0;
                    const uint64_t a = k[i], b = k[l];
                    const bool sw = desc ? (b > a) : (a > b);
                    k[i] = sw ? b : a;
                    k[l] = sw ? a : b;
                }
            }
}

// Number of keys in the lane's 16-lane row that are larger than its own: the row's 15 other lanes
// reach it by row rotations (one DPP move per half and one compare each, no scalar round trip).
template <int R>
WZY_DEV int row_count_above(uint64_t k) {
    if constexpr (R == 0) {
        return 0;
    } else {
        const uint32_t lo = (uint32_t) __builtin_amdgcn_mov_dpp((int) (uint32_t) k, 0x120 + R, 0xF, 0xF, true);
        const uint32_t hi = (uint32_t) __builtin_amdgcn_mov_dpp((int) (uint32_t) (k >> 32), 0x120 + R, 0xF, 0xF, true);
        return ((((uint64_t) hi << 32) | lo) > k ? 1 : 0) + row_count_above<R - 1>(k);
    }
}

// Softmax top-K of one row in one wave (ranking: probability desc, expert id asc).  Every lane
// sorts the keys of its RV probabilities once.  Candidates: thr = the K-th largest probability word
// among the 64 lane heads with its low 18 bits cleared (bisection on ballot counts over bits 29..18;
// probabilities are <= 1, so bits 31 and 30 are clear); the K largest heads are K distinct keys
// >= thr, so every key with a probability word >= thr is a superset of the top K.  When at most 64
// keys qualify, they are gathered into `cand` (this wave's LDS scratch) and each ranks itself
// against the others (by row rotations when at most 16 qualify, else broadcast by readlane);
// otherwise K rounds each take the DPP wave maximum
// over the lane heads and the winner lane pops its head.  Lane k ends with the k-th routed (id, probability); wsum is their sum
// in rank order.
template <int RV>
WZY_DEV void route_row(float (&p)[RV], int E, int K, int& my_id, float& my_w, float& wsum, uint64_t* cand) {
    const int lane = threadIdx.x & 63;
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < RV; ++i) mx = fmaxf(mx, p[i]);
    mx = wave_max(mx);
    float es = 0.f;
#pragma unroll
    for (int i = 0; i < RV; ++i) {
        if (lane + 64 * i < E) { p[i] = __expf(p[i] - mx); es += p[i]; }
    }
    es = wave_sum(es);
    const float inv = 1.0f / es;
    uint64_t key[RV];
#pragma unroll
    for (int i = 0; i < RV; ++i) key[i] = (lane + 64 * i < E) ? route_key(p[i] * inv, lane + 64 * i) : 0ull;
    sort_keys_desc<RV>(key);
    uint32_t hi[RV], lo[RV];
#pragma unroll
    for (int i = 0; i < RV; ++i) { hi[i] = (uint32_t) (key[i] >> 32); lo[i] = (uint32_t) key[i]; }
    wsum = 0.f;
    my_id = 0;
    my_w = 0.f;

    uint32_t thr = 0;
#pragma unroll
    for (int b = 29; b >= 18; --b) {
        const uint32_t c = thr | (1u << b);
        thr = __popcll(__ballot(hi[0] >= c)) >= K ? c : thr;       // wave-uniform
    }
    uint64_t bal[RV];
    int n_cand = 0;
#pragma unroll
    for (int i = 0; i < RV; ++i) {
        bal[i] = __ballot(hi[i] >= thr);
        n_cand += __popcll(bal[i]);
    }
    if (n_cand <= 64) {                                             // wave-uniform
        int base = 0;
#pragma unroll
        for (int i = 0; i < RV; ++i) {
            const int below = __builtin_amdgcn_mbcnt_hi((uint32_t) (bal[i] >> 32),
                                                       __builtin_amdgcn_mbcnt_lo((uint32_t) bal[i], 0));
            if (hi[i] >= thr) cand[base + below] = key[i];
            base += __popcll(bal[i]);
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        const uint64_t mine = lane < n_cand ? cand[lane] : 0ull;
        int rank = 0;
        if (n_cand <= 16) {                                         // wave-uniform; the usual case
            // every candidate sits in row 0, whose other lanes hold key 0 (below every real key)
            rank = row_count_above<15>(mine);
        } else {
            for (int j = 0; j < n_cand; ++j) {
                const uint32_t jl = (uint32_t) __builtin_amdgcn_readlane((int) (uint32_t) mine, j);
                const uint32_t jh = (uint32_t) __builtin_amdgcn_readlane((int) (uint32_t) (mine >> 32), j);
                rank += ((((uint64_t) jh << 32) | jl) > mine) ? 1 : 0;
            }
        }
        rank = lane < n_cand ? rank : 64;
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        if (rank < K) cand[rank] = mine;                            // distinct keys: distinct ranks
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        if (lane < K) {
            const uint64_t kk = cand[lane];
            my_w = __builtin_bit_cast(float, (uint32_t) (kk >> 32));
            int bi = (int) (0xFFFFFFFFu - (uint32_t) kk);
            if (bi >= E || bi < 0) bi = 0;                          // non-finite logits: keep the id in range
            my_id = bi;
        }
        for (int k = 0; k < K; ++k) wsum += as_f(__builtin_amdgcn_readlane(as_i(my_w), k));
        return;
    }
    for (int k = 0; k < K; ++k) {
        // the largest head: a 32-bit DPP maximum of the probability words, then (only when several
        // lanes hold that probability) of the id words among them; the winner lane is unique
        const uint32_t m = wave_max_u32(hi[0]);
        const bool at_m = hi[0] == m;
        uint64_t win = __ballot(at_m);
        if (__popcll(win) > 1) {                          // wave-uniform
            const uint32_t m2 = wave_max_u32(at_m ? lo[0] : 0u);
            win = __ballot(at_m && lo[0] == m2);
        }
        const int wl = __ffsll((long long) win) - 1;
        const uint32_t wlo = (uint32_t) __builtin_amdgcn_readlane((int) lo[0], wl);
        // the winner lane pops its head.  The shift is written with a mask rather than selects of
        // neighbouring keys, which the compiler would turn into a per-lane head index that selects
        // every key through a compare chain.
        const uint32_t pm = 0u - (uint32_t) (lane == wl);
#pragma unroll
        for (int i = 0; i + 1 < RV; ++i) {
            hi[i] ^= (hi[i] ^ hi[i + 1]) & pm;
            lo[i] ^= (lo[i] ^ lo[i + 1]) & pm;
        }
        hi[RV - 1] &= ~pm;
        lo[RV - 1] &= ~pm;
        const float bv = __builtin_bit_cast(float, m);
        int bi = (int) (0xFFFFFFFFu - wlo);
        if (bi >= E || bi < 0) bi = 0;                   // non-finite logits: keep the id in range
        if (lane == k) { my_id = bi; my_w = bv; }
        wsum += bv;
    }
}

}  // namespace wzy

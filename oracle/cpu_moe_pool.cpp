// cpu_moe_pool.cpp -- CPU baseline: restatement of the reference's AVX2/FMA cold-expert pool
// (CpuMoePool, src/wzy_cpu_moe.cuh:197-614).  TEST / BENCHMARK INFRASTRUCTURE ONLY: it is timed
// beside the GPU path as the reference's own CPU MoE throughput, never shipped.
//
// Algorithm (same steps as the reference, shapes runtime):
//  * activations arrive per-16 int8 and are re-laid per 64-value block as sub-blocks
//    [s0, s2, s1, s3] so one 256-bit load lines up with the unpacklo/unpackhi of the decoded
//    weights (src/wzy_cpu_moe.cuh:26-29,129-138);
//  * phase 1: tasks (group, 16-row tile): gate/up NVFP4 x int8 dots with pshufb e2m1 decode and
//    maddubs/madd (src/wzy_cpu_moe.cuh:313-349,362-486), SwiGLU, per-16 int8 requant straight into
//    the permuted layout;
//  * phase 2: 64-row output tiles: down dots, out += w * sc_down * dot (src/wzy_cpu_moe.cuh:493-588);
//  * the calling thread is worker 0, n-1 pinned workers spin on a sequence word, tasks are taken
//    from an atomic counter (src/wzy_cpu_moe.cuh:221-268,590-614); n in [2, 15].
#include <immintrin.h>
#include <pthread.h>
#include <sched.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <thread>
#include <vector>

#include "wzy_oracle.h"

namespace {

struct Group {
    const uint8_t* blob;
    int cnt;
    int tok[8];
    float wt[8];
};

}  // namespace

struct orc_cpu_pool {
    int n_threads = 2, D = 0, F = 0;
    float ue_half[256];
    std::vector<std::thread> workers;
    std::atomic<bool> stop{false};
    alignas(64) std::atomic<uint32_t> seq{0};
    alignas(64) std::atomic<int> done{0};
    alignas(64) std::atomic<int> next1{0};
    alignas(64) std::atomic<int> next2{0};
    // current job
    std::vector<Group> groups;
    int T = 0;
    std::vector<int8_t> xperm;      // [T x D] permuted activations
    std::vector<float> xs;          // [T x D/16]
    std::vector<int8_t> act_perm;   // [n_groups x 8 x F] permuted SwiGLU activations
    std::vector<float> act_s;       // [n_groups x 8 x F/16]
    float* out = nullptr;

    __attribute__((target("avx2,fma"))) static inline __m128 block64(const uint8_t* blk, const float* ue,
                                                                     const int8_t* xp, __m128 xsc, __m128 acc) {
        const __m256i lut = _mm256_setr_epi8(0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12, 0, 1, 2, 3, 4,
                                             6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12);
        const __m256i nib = _mm256_set1_epi8(0x0F);
        const __m256i one16 = _mm256_set1_epi16(1);
        const __m128 wsc = _mm_setr_ps(ue[blk[0]], ue[blk[1]], ue[blk[2]], ue[blk[3]]);
        const __m256i raw = _mm256_loadu_si256((const __m256i*) (blk + 4));
        const __m256i lo = _mm256_shuffle_epi8(lut, _mm256_and_si256(raw, nib));
        const __m256i hi = _mm256_shuffle_epi8(lut, _mm256_and_si256(_mm256_srli_epi16(raw, 4), nib));
        const __m256i w02 = _mm256_unpacklo_epi64(lo, hi);   // [s0 | s2]
        const __m256i w13 = _mm256_unpackhi_epi64(lo, hi);   // [s1 | s3]
        const __m256i x02 = _mm256_loadu_si256((const __m256i*) xp);
        const __m256i x13 = _mm256_loadu_si256((const __m256i*) (xp + 32));
        const __m256i p02 = _mm256_madd_epi16(_mm256_maddubs_epi16(_mm256_abs_epi8(w02), _mm256_sign_epi8(x02, w02)), one16);
        const __m256i p13 = _mm256_madd_epi16(_mm256_maddubs_epi16(_mm256_abs_epi8(w13), _mm256_sign_epi8(x13, w13)), one16);
        const __m256i h = _mm256_hadd_epi32(p02, p13);
        const __m128i d4 = _mm_hadd_epi32(_mm256_castsi256_si128(h), _mm256_extracti128_si256(h, 1));   // s0..s3
        return _mm_fmadd_ps(_mm_cvtepi32_ps(d4), _mm_mul_ps(wsc, xsc), acc);
    }
    static inline float hsum(__m128 v) {
        __m128 s = _mm_add_ps(v, _mm_movehl_ps(v, v));
        s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 1));
        return _mm_cvtss_f32(s);
    }
    static inline int perm_sub(int s) { return s == 1 ? 2 : (s == 2 ? 1 : s); }

    __attribute__((target("avx2,fma"))) void phase1() {
        const int tiles = F / 16;
        const int total = (int) groups.size() * tiles;
        const int gu_row = D / 64 * 36;
        for (int task = next1.fetch_add(1, std::memory_order_relaxed); task < total;
             task = next1.fetch_add(1, std::memory_order_relaxed)) {
            const int g = task / tiles, tile = task % tiles;
            const Group& G = groups[g];
            const float* tail = (const float*) (G.blob + orc_blob_bytes(D, F) - 16);
            float act[8][16];
            for (int dr = 0; dr < 16; ++dr) {
                const int row = tile * 16 + dr;
                const uint8_t* gp = G.blob + (size_t) row * gu_row;
                const uint8_t* up = G.blob + (size_t) (F + row) * gu_row;
                for (int j = 0; j < G.cnt; ++j) {
                    const int t = G.tok[j];
                    const int8_t* xp = xperm.data() + (size_t) t * D;
                    const float* xsp = xs.data() + (size_t) t * (D / 16);
                    __m128 ag = _mm_setzero_ps(), au = _mm_setzero_ps();
                    for (int b = 0; b < D / 64; ++b) {
                        const __m128 xsc = _mm_loadu_ps(xsp + 4 * b);
                        ag = block64(gp + 36 * b, ue_half, xp + 64 * b, xsc, ag);
                        au = block64(up + 36 * b, ue_half, xp + 64 * b, xsc, au);
                    }
                    const float gv = hsum(ag) * tail[0], uv = hsum(au) * tail[1];
                    act[j][dr] = (gv / (1.0f + std::exp(-gv))) * uv;
                }
            }
            const int dst = (tile >> 2) * 64 + perm_sub(tile & 3) * 16;
            for (int j = 0; j < G.cnt; ++j) {
                float amax = 0.f;
                for (int dr = 0; dr < 16; ++dr) amax = std::max(amax, std::fabs(act[j][dr]));
                const float d = amax / 127.0f;
                const float inv = d > 0.f ? 127.0f / amax : 0.f;
                act_s[((size_t) g * 8 + j) * (F / 16) + tile] = d;
                int8_t* q = act_perm.data() + ((size_t) g * 8 + j) * F + dst;
                for (int dr = 0; dr < 16; ++dr) {
                    int v = _mm_cvtss_si32(_mm_set_ss(act[j][dr] * inv));
                    q[dr] = (int8_t) std::min(127, std::max(-127, v));
                }
            }
        }
    }

    __attribute__((target("avx2,fma"))) void phase2() {
        constexpr int TILE = 64;
        const int tiles = D / TILE;
        const int gu_row = D / 64 * 36, d_row = F / 64 * 36;
        for (int tile = next2.fetch_add(1, std::memory_order_relaxed); tile < tiles;
             tile = next2.fetch_add(1, std::memory_order_relaxed)) {
            const int r0 = tile * TILE;
            for (int t = 0; t < T; ++t) memset(out + (size_t) t * D + r0, 0, sizeof(float) * TILE);
            for (size_t g = 0; g < groups.size(); ++g) {
                const Group& G = groups[g];
                const float sc = ((const float*) (G.blob + orc_blob_bytes(D, F) - 16))[2];
                const uint8_t* dn = G.blob + (size_t) 2 * F * gu_row;
                for (int dr = 0; dr < TILE; ++dr) {
                    const uint8_t* rp = dn + (size_t) (r0 + dr) * d_row;
                    for (int j = 0; j < G.cnt; ++j) {
                        const int8_t* xp = act_perm.data() + ((size_t) g * 8 + j) * F;
                        const float* xsp = act_s.data() + ((size_t) g * 8 + j) * (F / 16);
                        __m128 a = _mm_setzero_ps();
                        for (int b = 0; b < F / 64; ++b) a = block64(rp + 36 * b, ue_half, xp + 64 * b, _mm_loadu_ps(xsp + 4 * b), a);
                        out[(size_t) G.tok[j] * D + r0 + dr] += G.wt[j] * (hsum(a) * sc);
                    }
                }
            }
        }
    }

    void worker(int tid) {
        cpu_set_t cs;
        CPU_ZERO(&cs);
        const int ncpu = (int) std::thread::hardware_concurrency();
        CPU_SET(tid % std::max(1, ncpu), &cs);
        pthread_setaffinity_np(pthread_self(), sizeof cs, &cs);
        uint32_t last = 0;
        while (!stop.load(std::memory_order_acquire)) {
            const uint32_t s = seq.load(std::memory_order_acquire);
            if (s == last || (s & 1u) == 0u) { _mm_pause(); continue; }
            last = s;
            if (s & 2u) phase2(); else phase1();
            done.fetch_add(1, std::memory_order_acq_rel);
        }
    }

    void dispatch(uint32_t s, bool p2) {
        done.store(0, std::memory_order_relaxed);
        seq.store(s, std::memory_order_release);
        if (p2) phase2(); else phase1();
        while (done.load(std::memory_order_acquire) < n_threads - 1) _mm_pause();
    }
};

extern "C" orc_cpu_pool* orc_cpu_pool_create(int n_threads, int D, int F) {
    if (D % 64 || F % 64 || D < 64 || F < 64) return nullptr;
    orc_cpu_pool* p = new orc_cpu_pool();
    p->n_threads = std::max(2, std::min(15, n_threads));
    p->D = D;
    p->F = F;
    for (int x = 0; x < 256; ++x) p->ue_half[x] = orc_ue4m3_half(x);
    cpu_set_t cs;
    CPU_ZERO(&cs);
    CPU_SET(0, &cs);
    pthread_setaffinity_np(pthread_self(), sizeof cs, &cs);
    for (int t = 1; t < p->n_threads; ++t) p->workers.emplace_back([p, t] { p->worker(t); });
    return p;
}

extern "C" void orc_cpu_pool_destroy(orc_cpu_pool* p) {
    if (!p) return;
    p->stop.store(true, std::memory_order_release);
    for (auto& w : p->workers) w.join();
    cpu_set_t cs;
    CPU_ZERO(&cs);
    const int ncpu = (int) std::thread::hardware_concurrency();
    for (int c = 0; c < ncpu; ++c) CPU_SET(c, &cs);
    pthread_setaffinity_np(pthread_self(), sizeof cs, &cs);
    delete p;
}

extern "C" int orc_cpu_pool_threads(const orc_cpu_pool* p) { return p ? p->n_threads : 0; }

extern "C" int orc_cpu_pool_run(orc_cpu_pool* p, const uint8_t* const* blobs, const int* ids, const float* wts, int T,
                                int K, const int8_t* xq16, const float* xs16, float* out) {
    if (!p || T < 1 || T > 8 || K < 1) return -1;
    const int D = p->D, F = p->F;
    // group entries by expert id (ascending, deterministic like the reference's gkey sort)
    std::vector<int> order(T * K);
    for (int i = 0; i < T * K; ++i) order[i] = i;
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return ids[a] < ids[b]; });
    p->groups.clear();
    for (int i = 0; i < T * K;) {
        const int e = ids[order[i]];
        Group g;
        g.blob = blobs[e];
        if (!g.blob) return -1;
        g.cnt = 0;
        while (i < T * K && ids[order[i]] == e && g.cnt < 8) {
            g.tok[g.cnt] = order[i] / K;
            g.wt[g.cnt] = wts[order[i]];
            ++g.cnt;
            ++i;
        }
        p->groups.push_back(g);
    }
    p->T = T;
    p->xperm.resize((size_t) T * D);
    p->xs.assign(xs16, xs16 + (size_t) T * D / 16);
    for (int t = 0; t < T; ++t)
        for (int b = 0; b < D / 64; ++b)
            for (int s = 0; s < 4; ++s)
                memcpy(p->xperm.data() + (size_t) t * D + 64 * b + 16 * orc_cpu_pool::perm_sub(s),
                       xq16 + (size_t) t * D + 64 * b + 16 * s, 16);
    p->act_perm.resize(p->groups.size() * 8 * F);
    p->act_s.resize(p->groups.size() * 8 * (F / 16));
    p->out = out;
    uint32_t s = p->seq.load(std::memory_order_relaxed) & ~3u;
    if (s >= 0xFFFFFFF0u) s = 0;
    p->next1.store(0, std::memory_order_relaxed);
    p->dispatch(s + 1u, false);
    p->next2.store(0, std::memory_order_relaxed);
    p->dispatch(s + 3u, true);
    p->seq.store(s + 4u, std::memory_order_release);
    return 0;
}

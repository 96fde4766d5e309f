// reduce.hip -- greedy argmax and exact top-16 over vocabulary logits.
//
// Grid (ceil(nvocab / CHUNK), T).  Each 256-thread workgroup owns CHUNK = 2048 logits of a row
// (8 per thread, coalesced), finds its chunk's best R candidates (R = 1 for argmax, 16 for top-16)
// with R rounds of DPP/swizzle wave argmax + a 4-wave LDS merge, and writes them as partials.  The
// last workgroup to finish a row (arrival counter, reset by that workgroup) merges the partials the
// same way.  Order: larger value first, ties -> lower vocab index.  The top-16 is exact: every
// global top-16 element is a top-16 element of its own chunk.
// reference: row_argmax_multi_kernel / row_top16_multi_kernel (src/wzy_kernels_v2.cuh:1873-1984).
#include "wzy_device.h"
#include "wzy_host.h"
#include "wzy_reduce.h"

using namespace wzy;

namespace {
constexpr int RD_THREADS = 256;
constexpr int RD_PER_THREAD = 8;
constexpr int RD_CHUNK = RD_THREADS * RD_PER_THREAD;   // 2048

// R rounds of block argmax over each thread's V values (already loaded, -inf = empty).
// Writes winners to (out_v, out_i)[0..R) from thread 0.
template <int R, int V>
WZY_DEV void block_topr(float (&v)[V], int (&ix)[V], float* out_v, int* out_i, float* sv, int* si) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    for (int r = 0; r < R; ++r) {
        float bv = -INFINITY;
        int bi = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < V; ++j) amax_merge(bv, bi, v[j], ix[j]);
        wave_argmax(bv, bi);
        if (lane == 0) { sv[w] = bv; si[w] = bi; }
        __syncthreads();
        float gv = sv[0];
        int gi = si[0];
#pragma unroll
        for (int k = 1; k < RD_THREADS / 64; ++k) amax_merge(gv, gi, sv[k], si[k]);
        // the owner removes the winner from its list
#pragma unroll
        for (int j = 0; j < V; ++j)
            if (ix[j] == gi) { v[j] = -INFINITY; ix[j] = 0x7fffffff; }
        if (tid == 0) { out_v[r] = gv; out_i[r] = gi; }
        __syncthreads();
    }
}
}  // namespace

template <int R>
__global__ void __launch_bounds__(RD_THREADS) row_topr_kernel(const float* __restrict__ logits, int nvocab,
                                                              float* __restrict__ part_v, int* __restrict__ part_i,
                                                              unsigned* __restrict__ row_cnt, int* __restrict__ greedy,
                                                              float* __restrict__ top_v, int* __restrict__ top_i) {
    __shared__ float sv[RD_THREADS / 64];
    __shared__ int si[RD_THREADS / 64];
    __shared__ float s_out_v[R];
    __shared__ int s_out_i[R];
    __shared__ int s_last;
    const int tid = threadIdx.x;
    const int row = blockIdx.y, nchunk = gridDim.x;
    const float* l = logits + (size_t) row * nvocab;

    float v[RD_PER_THREAD];
    int ix[RD_PER_THREAD];
    const int base = blockIdx.x * RD_CHUNK;
#pragma unroll
    for (int j = 0; j < RD_PER_THREAD; ++j) {
        const int i = base + j * RD_THREADS + tid;
        v[j] = i < nvocab ? l[i] : -INFINITY;
        ix[j] = i < nvocab ? i : 0x7fffffff;
    }
    block_topr<R>(v, ix, s_out_v, s_out_i, sv, si);
    float* pv = part_v + ((size_t) row * nchunk + blockIdx.x) * R;
    int* pi = part_i + ((size_t) row * nchunk + blockIdx.x) * R;
    if (tid < R) { pv[tid] = s_out_v[tid]; pi[tid] = s_out_i[tid]; }

    __threadfence();
    __syncthreads();
    if (tid == 0) s_last = (atomicAdd(&row_cnt[row], 1u) == (unsigned) (nchunk - 1));
    __syncthreads();
    if (!s_last) return;
    __threadfence();

    // merge nchunk*R partials (at most RD_CHUNK of them)
    const float* av = part_v + (size_t) row * nchunk * R;
    const int* ai = part_i + (size_t) row * nchunk * R;
    const int n = nchunk * R;
#pragma unroll
    for (int j = 0; j < RD_PER_THREAD; ++j) {
        const int k = j * RD_THREADS + tid;
        v[j] = k < n ? av[k] : -INFINITY;
        ix[j] = k < n ? ai[k] : 0x7fffffff;
    }
    block_topr<R>(v, ix, s_out_v, s_out_i, sv, si);
    if (tid == 0) {
        if (greedy) greedy[row] = s_out_i[0];
        row_cnt[row] = 0u;
    }
    if (tid < R) {
        if (top_v) top_v[row * R + tid] = s_out_v[tid];
        if (top_i) top_i[row * R + tid] = s_out_i[tid];
    }
}

namespace wzy {

size_t reduce_ws_bytes(int nvocab, int T) {
    const int nchunk = (nvocab + RD_CHUNK - 1) / RD_CHUNK;
    return align_up((size_t) T * nchunk * 16 * 8, 256) + 256;
}

// ws layout: [row counters: 64 x u32][partials]
int launch_row_reduce(const float* logits, int nvocab, int T, bool top16, int* greedy, float* top_v, int* top_i,
                      void* ws, hipStream_t st) {
    WZY_REQUIRE(logits && ws && nvocab > 0 && T >= 1 && T <= 64, "row reduce: bad arguments");
    const int nchunk = (nvocab + RD_CHUNK - 1) / RD_CHUNK;
    WZY_REQUIRE((size_t) nchunk * 16 <= (size_t) RD_CHUNK, "row reduce: nvocab too large (%d)", nvocab);
    unsigned* cnt = (unsigned*) ws;
    float* pv = (float*) ((char*) ws + 256);
    int* pi = (int*) (pv + (size_t) T * nchunk * 16);
    if (top16)
        hipLaunchKernelGGL(row_topr_kernel<16>, dim3(nchunk, T), dim3(RD_THREADS), 0, st, logits, nvocab, pv, pi, cnt,
                           greedy, top_v, top_i);
    else
        hipLaunchKernelGGL(row_topr_kernel<1>, dim3(nchunk, T), dim3(RD_THREADS), 0, st, logits, nvocab, pv, pi, cnt,
                           greedy, nullptr, nullptr);
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

}  // namespace wzy

// Stand-alone entry points keep a per-device scratch for counters/partials (allocated on first use,
// counters zero-initialised once; every launch leaves them at zero).
static int reduce_scratch(int nvocab, int T, void** out) {
    static void* buf[64] = {nullptr};
    static size_t cap[64] = {0};
    int dev = 0;
    WZY_HIP_TRY(hipGetDevice(&dev));
    WZY_REQUIRE(dev >= 0 && dev < 64, "row reduce: device id out of range");
    const size_t need = reduce_ws_bytes(nvocab, T);
    if (cap[dev] < need) {
        if (buf[dev]) WZY_HIP_TRY(hipFree(buf[dev]));
        buf[dev] = nullptr;
        cap[dev] = 0;
        if (hipMalloc(&buf[dev], need) != hipSuccess) {
            set_error("row reduce: hipMalloc(%zu) failed", need);
            return WZY_ENOMEM;
        }
        WZY_HIP_TRY(hipMemset(buf[dev], 0, need));
        cap[dev] = need;
    }
    *out = buf[dev];
    return WZY_OK;
}

extern "C" int wzy_row_argmax(const float* logits, int nvocab, int T, int* out_ids, void* stream) {
    WZY_REQUIRE(out_ids, "wzy_row_argmax: null output");
    void* ws = nullptr;
    WZY_TRY(reduce_scratch(nvocab, T, &ws));
    return launch_row_reduce(logits, nvocab, T, false, out_ids, nullptr, nullptr, ws, as_stream(stream));
}

extern "C" int wzy_row_top16(const float* logits, int nvocab, int T, int* out_greedy, float* top_v, int* top_i,
                             void* stream) {
    void* ws = nullptr;
    WZY_TRY(reduce_scratch(nvocab, T, &ws));
    return launch_row_reduce(logits, nvocab, T, true, out_greedy, top_v, top_i, ws, as_stream(stream));
}

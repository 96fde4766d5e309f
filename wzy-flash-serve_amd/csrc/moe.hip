// moe.hip -- NVFP4 mixture-of-experts decode block for gfx950.
//
// Launch sequence of wzy_moe_block (T window rows, K routed experts per row), three launches:
//   1. router       logits [T x E] (bf16) + the shared-expert gate scalar row.  T <= 4: a plain
//                   gemv_segs launch, and the gate/up workgroups route the window themselves (one
//                   routing pass plus a cross-workgroup handoff costs more).  T > 4: moe_router,
//                   whose last workgroup to finish routes the window once and publishes the tables.
//                   Routing = softmax top-K, weights, and groups: each distinct expert of the window
//                   once, with its (row, slot) members, so its weights stream from HBM once.
//   2. gate/up      T = 1, moe_gate_up_kernel: routed workgroup (expert, 32-row tile) prefetches the
//                   logits, stages x, routes, then loads its weights (workgroup 0 publishes the
//                   routing).  1 < T <= 4, moe_gate_up_window_kernel: one resident round of about one
//                   workgroup per CU, each routing the window and then taking the (group, tile) items
//                   bid, bid + n, ... with two register sets of weight loads in flight.  T > 4,
//                   moe_gate_up_kernel with the published tables: workgroup (group, tile) issues its
//                   weight loads at entry.  Then the gate+up NVFP4 GEMV, SwiGLU and the per-16 int8
//                   requant.  Shared workgroups run the Q8_0 shared expert on x quantised per 32.
//   3. moe_down     workgroup = 8 output rows for all groups + the shared expert, activations
//                   staged in LDS, combine in LDS:
//                   comb = sigmoid(sgate)*shared + sum_k w_k*part_k  (k in routed order).
// All expert GEMVs are wave-per-row with 128-bit code loads (16 bytes = 32 e2m1 values per lane)
// and e4m3 scales from a separate plane; e2m1 codes are expanded by the fp4 -> f16 conversion
// instruction and dotted with f16 activation pairs (v_dot2_f32_f16, exact integer sums); every
// weight load of a lane is issued before any is used.  No MFMA: at one token per expert these are
// bandwidth-bound GEMVs.
#include "wzy_device.h"
#include "wzy_gemv.h"
#include "wzy_host.h"
#include "wzy_moe.h"
#include "wzy_route.h"

using namespace wzy;

namespace {

constexpr int DN_TILE = 8;    // output rows of one down workgroup

struct MoeRtArgs {
    const uint16_t* router; const uint16_t* sgate; const float* x;
    int D, E, K;
    float* logits; float* sg;
    int* ids; float* wts; int* n_groups; int* grp_exp; int* grp_cnt; int* grp_mem;
    unsigned* arrive;
};
// work items whose loads a 16-lane slot issues together: a one-row window's 11 x 8 items fit in
// one batch of 6 per slot, so every weight load of the workgroup is issued at once
// threads of a moe_down workgroup: 16 slots for one-row windows; for more rows 64 slots of 5 items
// where one 32-value chunk per lane covers a row (n_ff <= 512), the activations are staged in LDS and
// the registers allow it (T <= 4), so that a T = 4 window's up to 41 groups x 8 rows take one batch
// round; otherwise 32 slots of 4 items (16 where a row takes three or four chunk rounds, whose
// registers need a SIMD to itself)
template <int T, int CI, bool STAGE>
constexpr bool dn_wide() { return T > 1 && T <= 4 && CI == 1 && STAGE; }
template <int T, int CI, bool STAGE>
constexpr int dn_batch() { return T == 1 ? 6 : (dn_wide<T, CI, STAGE>() ? 5 : 4); }
template <int T, int CI, bool STAGE>
constexpr int dn_threads() { return T == 1 ? 256 : (dn_wide<T, CI, STAGE>() ? 1024 : (CI <= 2 ? 512 : 256)); }
constexpr int MAX_ENT = WZY_MAX_W * MOE_MAX_K;
// windows of up to this many rows route inside the gate/up workgroups (moe_gate_up_window_kernel for
// T > 1); longer ones route once in moe_router
constexpr int GU_WINDOW_MAX_T = 4;
constexpr int DN_STAGE_BYTES = 48 * 1024;   // activation staging limit of moe_down


// Dot of one 32-value NVFP4 chunk (16 code bytes, 2 e4m3 scales) with 32 int8 activations (two
// per-16 scales), accumulated the way the reference does per 16-block:
// acc = fma(ws * xs, isum, acc)   (src/wzy_kernels_v2.cuh:1646-1647).
// The e2m1 codes are expanded by the hardware fp4 -> f16 conversion with scale 2, which gives the
// doubled codes 2*e2m1 (integers -12..12; ue4m3x2_half carries the matching 0.5), and the int8
// activations are held as f16 pairs: pair p of a 16-value sub-block is (x_p, x_{p+8}), matching code
// byte p (value p in its low nibble, p+8 in its high one).  Every product and partial sum is an
// integer below 2^24, so each f32 dot-2 chain equals the integer dot isum exactly.
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float v2f_t __attribute__((ext_vector_type(2)));
// The two e4m3 block scales of a 16-bit scale pair (low byte first), each times 0.5 (the factor that
// the doubled e2m1 codes carry): one hardware fp8 -> f32 conversion with scale 0.5, the sign bit
// cleared.  Code 0x7F, NaN in OCP e4m3, is 480 in the unsigned reading of the reference's scales,
// 240 after the halving: the NaN-discarding min gives it and leaves every other code (at most 224)
// alone.  Equal to ue4m3_half on both bytes for all 128 codes.
WZY_DEV v2f_t ue4m3x2_half(uint32_t s) {
    const v2f_t v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(s & 0x7F7Fu, 0.5f, false);
    return v2f_t{fminf(v.x, 240.0f), fminf(v.y, 240.0f)};
}
template <int J>
WZY_DEV half2_t fp4x2_h(uint32_t w) { return __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 2.0f, J); }
WZY_DEV float e2m1_dot16_h(uint32_t w0, uint32_t w1, const half2_t* xp) {
    float a = 0.f, b = 0.f;                            // two chains for ILP (exact either way)
    a = __builtin_amdgcn_fdot2(fp4x2_h<0>(w0), xp[0], a, false);
    b = __builtin_amdgcn_fdot2(fp4x2_h<0>(w1), xp[4], b, false);
    a = __builtin_amdgcn_fdot2(fp4x2_h<1>(w0), xp[1], a, false);
    b = __builtin_amdgcn_fdot2(fp4x2_h<1>(w1), xp[5], b, false);
    a = __builtin_amdgcn_fdot2(fp4x2_h<2>(w0), xp[2], a, false);
    b = __builtin_amdgcn_fdot2(fp4x2_h<2>(w1), xp[6], b, false);
    a = __builtin_amdgcn_fdot2(fp4x2_h<3>(w0), xp[3], a, false);
    b = __builtin_amdgcn_fdot2(fp4x2_h<3>(w1), xp[7], b, false);
    return a + b;
}
WZY_DEV float nvfp4_chunk_fma_h(const uint4 c, float wsa, float wsb, const half2_t (&xp)[16], float xsa, float xsb,
                                float acc) {
    acc = fmaf(wsa * xsa, e2m1_dot16_h(c.x, c.y, &xp[0]), acc);
    acc = fmaf(wsb * xsb, e2m1_dot16_h(c.z, c.w, &xp[8]), acc);
    return acc;
}

// The 32 e2m1 codes of a 16-byte chunk as doubled f16 pairs in e2m1_dot16_h's order: wq[0..7] the
// first 16-value sub-block, wq[8..15] the second.
WZY_DEV void fp4_expand16(const int4 c, half2_t (&wq)[16]) {
    const uint32_t w[4] = {(uint32_t) c.x, (uint32_t) c.y, (uint32_t) c.z, (uint32_t) c.w};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        wq[4 * d] = fp4x2_h<0>(w[d]);
        wq[4 * d + 1] = fp4x2_h<1>(w[d]);
        wq[4 * d + 2] = fp4x2_h<2>(w[d]);
        wq[4 * d + 3] = fp4x2_h<3>(w[d]);
    }
}
// e2m1_dot16_h on codes already expanded: pairs 0-3 and 4-7 in two chains (every product and partial
// sum an integer below 2^24, so the result is the exact integer dot in any order)
WZY_DEV float dot16_pairs(const half2_t* wq, const half2_t* xp) {
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        a = __builtin_amdgcn_fdot2(wq[p], xp[p], a, false);
        b = __builtin_amdgcn_fdot2(wq[4 + p], xp[4 + p], b, false);
    }
    return a + b;
}

// Exclusive count of `pred` over threads 0..255 in thread order (4 waves); `total` = full count.
WZY_DEV int excl_count_wg(bool pred, int* s_c, int& total) {     // s_c: 8 ints; workgroups of <= 8 waves
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = (int) (blockDim.x >> 6);
    const unsigned long long m = __ballot(pred);
    const int within = __popcll(m & ((1ull << lane) - 1ull));
    if (lane == 0) s_c[w] = __popcll(m);
    __syncthreads();
    int before = 0, all = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int ci = i < nw ? s_c[i] : 0;
        before += (i < w) ? ci : 0;
        all += ci;
    }
    total = all;
    __syncthreads();
    return before + within;
}

// int8 quantisation, reference rule d = amax/127, q = rint(x * 127/amax) clamped to +-127.
// 32 values -> two 16-value halves with one shared per-32 scale
// Rows per gate/up workgroup.  A lane holds NCL 32-column chunks of every row it dots (NCL = 1 for
// D <= 2048, 2 for D <= 4096); with two chunks a wave takes half as many rows, so that its weight
// registers stay the same.
__host__ __device__ constexpr int gu_tile_rows(int ncl) { return 32 / ncl; }   // routed F-rows (gate and up)
__host__ __device__ constexpr int sh_tile_rows(int ncl) { return 16 / ncl; }   // shared-expert SwiGLU outputs

// moe_down dynamic LDS: the shared activation's per-32 scales, padded to 16 bytes
__host__ __device__ inline int dn_shs_floats(int T, int nchunk) { return (T * nchunk + 3) / 4 * 4; }
__host__ __device__ inline size_t dn_shared_lds(int T, int nchunk) {
    return (size_t) T * nchunk * 2 * sizeof(int4) + (size_t) dn_shs_floats(T, nchunk) * sizeof(float);
}

WZY_DEV void quant32_halves(const float (&v)[32], int4& qa, int4& qb, float& d) {
    float am = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) am = fmaxf(am, fabsf(v[i]));
    d = am / 127.0f;
    const float inv = d > 0.f ? 127.0f / am : 0.f;
    int w[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        uint32_t pk = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) pk |= (uint32_t) (max(-127, min(127, rn_int(v[4 * k + j] * inv))) & 0xFF) << (8 * j);
        w[k] = (int) pk;
    }
    qa = make_int4(w[0], w[1], w[2], w[3]);
    qb = make_int4(w[4], w[5], w[6], w[7]);
}
// The same per-32 quantisation with 4 lanes per block (a lane quad): lane q of the quad holds values
// 8q .. 8q+7 and gets their 8 codes (bytes 8q .. 8q+7 of the block) and the block scale.
WZY_DEV uint2 quant32_quad(const float (&v)[8], float& d) {
    float am = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) am = fmaxf(am, fabsf(v[i]));
    am = fmaxf(am, dpp_f<DPP_XOR1>(am));
    am = fmaxf(am, dpp_f<DPP_XOR2>(am));
    d = am / 127.0f;
    const float inv = d > 0.f ? 127.0f / am : 0.f;
    uint32_t w[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        uint32_t pk = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) pk |= (uint32_t) (max(-127, min(127, rn_int(v[4 * k + j] * inv))) & 0xFF) << (8 * j);
        w[k] = pk;
    }
    return make_uint2(w[0], w[1]);
}
// 32 values -> two 16-value halves, each quantised to int8 with its own per-16 scale, written as
// the f16 pairs of nvfp4_chunk_fma_h: xp[8h + p] = (q[16h + p], q[16h + p + 8]).
WZY_DEV void quant16_pairs(const float (&v)[32], half2_t (&xp)[16], float& da, float& db) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        float am = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) am = fmaxf(am, fabsf(v[16 * h + i]));
        const float d = am / 127.0f;
        const float inv = d > 0.f ? 127.0f / am : 0.f;
        int q[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) q[i] = max(-127, min(127, rn_int(v[16 * h + i] * inv)));
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            half2_t t;
            t.x = (_Float16) (float) q[p];
            t.y = (_Float16) (float) q[p + 8];
            xp[8 * h + p] = t;
        }
        if (h == 0) da = d; else db = d;
    }
}

// Window routing in LDS.  Softmax top-K per row (reference: router_top10_fast_multi,
// src/wzy_kernels_v2.cuh:989-1090), then the grouping of the routed entries by expert (reference:
// split_route_hit_cold_kernel / group_experts_kernel, src/wzy_cpu_moe.cuh:74-127,
// src/wzy_kernels_v2.cuh:1390-1423).  Groups are numbered in order of first occurrence and members
// in entry order; the combine sums in routed-slot order, so the numbering affects no result.
struct RouteLds {
    int ids[MAX_ENT];
    float w[MAX_ENT];
    int gidx[MAX_ENT];
    int gexp[MAX_ENT];
    int gcnt[MAX_ENT];
    int gmem[MAX_ENT][WZY_MAX_W];
    int n_groups;
    int c[8];
    uint64_t cand[4][64];          // per-wave candidate keys of route_row (waves 0-3 route)
    uint32_t rows[1024];           // one-wave grouping: per expert the window rows that routed it,
                                   // then its group number
};

// Logits of one row per wave: RV per lane (lane + 64*i), RV = 8 for E <= 512, 16 for E <= 1024.
// wave wv < 4 prefetches rows wv, wv+4 of the logits (issued before anything uses them); waves 4..7
// of an eight-wave workgroup route nothing
template <int T, int RV>
WZY_DEV void route_prefetch(const float* __restrict__ logits, int E, float (&p)[(T + 3) / 4][RV]) {
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int rr = 0; rr < (T + 3) / 4; ++rr) {
        const int t = wv + 4 * rr;
        if (wv >= 4 || t >= T) {                         // wave-uniform
#pragma unroll
            for (int i = 0; i < RV; ++i) p[rr][i] = -INFINITY;
            continue;
        }
        // clamped index, unconditional load: a per-lane branch around each load would order them
#pragma unroll
        for (int i = 0; i < RV; ++i) {
            const int idx = lane + 64 * i;
            const float v = logits[(size_t) t * E + min(idx, E - 1)];
            p[rr][i] = idx < E ? v : -INFINITY;
        }
    }
}

template <int T, int RV>
WZY_DEV void route_compute(float (&p)[(T + 3) / 4][RV], int E, int K, RouteLds& r) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    if (T == 1) {
        // one row: its K experts are distinct, so each is its own group with one member
        if (wv == 0) {
            int my_id;
            float my_w, wsum;
            route_row<RV>(p[0], E, K, my_id, my_w, wsum, r.cand[0]);
            const float sc = fmaxf(wsum, 6.103515625e-05f);
            if (lane < K) {
                r.ids[lane] = my_id;
                r.w[lane] = my_w / sc;
                r.gidx[lane] = lane;
                r.gexp[lane] = my_id;
                r.gcnt[lane] = 1;
                r.gmem[lane][0] = lane;
            }
            if (lane == 0) r.n_groups = K;
        }
        __syncthreads();
        return;
    }
#pragma unroll
    for (int rr = 0; rr < (T + 3) / 4; ++rr) {
        const int t = wv + 4 * rr;
        if (wv >= 4 || t >= T) continue;                 // wave-uniform
        int my_id;
        float my_w, wsum;
        route_row<RV>(p[rr], E, K, my_id, my_w, wsum, r.cand[wv]);
        const float sc = fmaxf(wsum, 6.103515625e-05f);
        if (lane < K) { r.ids[t * K + lane] = my_id; r.w[t * K + lane] = my_w / sc; }
    }
    __syncthreads();
    const int n_ent = T * K;
    if (n_ent <= 64) {
        // grouping in one wave, lane = entry (row t = lane / K): an expert occurs at most once per
        // row, so its entries are described by the mask of the rows that routed it (LDS OR per expert).
        // An entry's slot is the number of earlier rows in that mask, the entry with slot 0 leads the
        // group, and leaders are numbered in entry order by a ballot prefix count; every workgroup that
        // routes the window gets the same tables.
        if (wv == 0) {
            const bool on = lane < n_ent;
            const int id = on ? r.ids[lane] : 0, t = lane / K;
            if (on) r.rows[id] = 0u;
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            if (on) atomicOr(&r.rows[id], 1u << t);
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            const uint32_t m = on ? r.rows[id] : 0u;
            const int slot = __popc(m & ((1u << t) - 1u));
            const bool lead = on && slot == 0;
            const uint64_t leads = __ballot(lead);
            if (lead) r.rows[id] = 0x80000000u | (uint32_t) __builtin_amdgcn_mbcnt_hi(
                                                       (uint32_t) (leads >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t) leads, 0));
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            if (on) {
                const int g = (int) (r.rows[id] & 0xFFFFu);
                if (slot < WZY_MAX_W) r.gmem[g][slot] = lane;
                if (lead) {
                    r.gexp[g] = id;
                    r.gcnt[g] = min(__popc(m), WZY_MAX_W);
                }
            }
            if (lane == 0) r.n_groups = __popcll(leads);
        }
        __syncthreads();
        return;
    }
    // grouping: leader = first entry of an expert, slot = rank among the expert's entries
    int id = -1, leader = 0, slot = 0, cnt = 0;
    if (tid < n_ent) {
        id = r.ids[tid];
        leader = tid;
        bool seen = false;
        for (int f = 0; f < n_ent; ++f) {
            if (r.ids[f] != id) continue;
            if (!seen) { leader = f; seen = true; }
            if (f < tid) ++slot;
            ++cnt;
        }
    }
    const bool lead = tid < n_ent && leader == tid;
    int n_groups = 0;
    const int g_lead = excl_count_wg(lead, r.c, n_groups);
    if (lead) r.gidx[tid] = g_lead;
    __syncthreads();
    if (tid < n_ent) {
        const int g = r.gidx[leader];
        if (slot < WZY_MAX_W) r.gmem[g][slot] = tid;
        if (lead) {
            r.gexp[g] = id;
            r.gcnt[g] = min(cnt, WZY_MAX_W);             // an expert occurs at most once per row
        }
    }
    if (tid == 0) r.n_groups = n_groups;
    __syncthreads();
}

// The routing tables of the window for moe_down (and the caller's ids / weights), written by one
// workgroup: ids, weights, the group count and each group's expert, member count and members.
WZY_DEV void publish_routing(const RouteLds& r, const MoeGuArgs& a, int n_ent) {
    for (int i = threadIdx.x; i < n_ent; i += blockDim.x) {
        a.ids[i] = r.ids[i];
        a.wts[i] = r.w[i];
        if (i < r.n_groups) {
            a.grp_exp[i] = r.gexp[i];
            a.grp_cnt[i] = r.gcnt[i];
            for (int m = 0; m < WZY_MAX_W; ++m) a.grp_mem[i * WZY_MAX_W + m] = m < r.gcnt[i] ? r.gmem[i][m] : 0;
        }
    }
    if (threadIdx.x == 0) *a.n_groups = r.n_groups;
}

// chunk `cc` of x row `t` ([rows x D] fp32) quantised per 16 into LDS slot i of nx: 16 f16 pairs
// (nvfp4_chunk_fma_h's order) as four 16-byte quarters, quarter q at uint4 index q * nx + i (lanes
// that read consecutive slots then read consecutive 16-byte words, not words 64 bytes apart in one
// bank group), and the two per-16 scales
WZY_DEV void stage_x16(const float* __restrict__ x, int D, int t, int cc, int i, int nx, half2_t* s_xh, float2* s_xs2) {
    const float4* xp = (const float4*) (x + (size_t) t * D + (size_t) cc * 32);
    float v[32];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const float4 f = xp[k];
        v[4 * k] = f.x; v[4 * k + 1] = f.y; v[4 * k + 2] = f.z; v[4 * k + 3] = f.w;
    }
    half2_t xq[16];
    float da, db;
    quant16_pairs(v, xq, da, db);
#pragma unroll
    for (int k = 0; k < 4; ++k)
        ((uint4*) s_xh)[(size_t) k * nx + i] = make_uint4(__builtin_bit_cast(uint32_t, xq[4 * k]),
                                                           __builtin_bit_cast(uint32_t, xq[4 * k + 1]),
                                                           __builtin_bit_cast(uint32_t, xq[4 * k + 2]),
                                                           __builtin_bit_cast(uint32_t, xq[4 * k + 3]));
    s_xs2[i] = make_float2(da, db);
}

// Shared-expert workgroup sb of a gate/up launch: rows j in [SJ*sb, SJ*sb + SJ) (SJ = 16, or 8 for
// D > 2048), wave w owns SRW = SJ/8 consecutive rows of both gate and up; NCL 32-blocks of x per
// lane.  The SwiGLU values go out as fp32; moe_down quantises them per 32.
// reference: launch_gemm_q8p x2 + silu_mul_quant32_multi (src/wzy_stage_v2.cuh:711-713;
// src/wzy_kernels_v2.cuh:1247-1280).
// Dynamic LDS: x quantised per 32, [T][D/32] int4 first halves, [T][D/32] int4 second halves,
// [T][D/32] float scales.
template <int T, int NCL>
WZY_DEV void gu_shared(const MoeGuArgs& a, int sb, unsigned char* s_dyn) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int D = a.D, F = a.F;
    const int nc = D / 32;
    int4* s_qa = (int4*) s_dyn;
    int4* s_qb = s_qa + (size_t) T * nc;
    float* s_sc = (float*) (s_qb + (size_t) T * nc);
    constexpr int SJ = sh_tile_rows(NCL), SRW = SJ / 8;
    int4 c0[NCL][2 * SRW], c1[NCL][2 * SRW];
    uint32_t sraw[NCL][2 * SRW];     // 16-bit scales in 32-bit registers (no packing that waits for the load)
    const int j0 = SJ * sb + SRW * w;
#pragma unroll
    for (int k = 0; k < NCL; ++k) {
        const int bl = min(lane + 64 * k, nc - 1);
#pragma unroll
        for (int rr = 0; rr < 2 * SRW; ++rr) {
            const int8_t* q = (rr < SRW) ? a.shg_q : a.shu_q;
            const uint16_t* s = (rr < SRW) ? a.shg_s : a.shu_s;
            const int row = j0 + rr % SRW;
            const int4* cp = (const int4*) (q + (size_t) row * D + (size_t) bl * 32);
            c0[k][rr] = ld_stream_i4(cp);
            c1[k][rr] = ld_stream_i4(cp + 1);
            sraw[k][rr] = s[(size_t) row * nc + bl];
        }
    }
    // stage x quantised per 32
    for (int i = tid; i < T * nc; i += (int) blockDim.x) {
        const int t = i / nc, c = i - t * nc;
        float v[32];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float4 f = ((const float4*) (a.x + (size_t) t * D + (size_t) c * 32))[k];
            v[4 * k] = f.x; v[4 * k + 1] = f.y; v[4 * k + 2] = f.z; v[4 * k + 3] = f.w;
        }
        int4 qa, qb;
        float d;
        quant32_halves(v, qa, qb, d);
        s_qa[i] = qa;
        s_qb[i] = qb;
        s_sc[i] = d;
    }
    __syncthreads();
    float acc[2 * SRW][T];
#pragma unroll
    for (int rr = 0; rr < 2 * SRW; ++rr)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[rr][t] = 0.f;
#pragma unroll
    for (int k = 0; k < NCL; ++k) {
        const int b = lane + 64 * k;                     // the lane's 32-blocks of x
        if (b >= nc) continue;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int xi = t * nc + b;
            const int4 x0 = s_qa[xi], x1 = s_qb[xi];
            const float xsc = s_sc[xi];
#pragma unroll
            for (int rr = 0; rr < 2 * SRW; ++rr)
                acc[rr][t] = fmaf(h16_to_f(sraw[k][rr]) * xsc, (float) (dot16(c0[k][rr], x0) + dot16(c1[k][rr], x1)),
                                  acc[rr][t]);
        }
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
#pragma unroll
        for (int q = 0; q < SRW; ++q) {
            const float gv = wave_sum(acc[q][t]);
            const float uv = wave_sum(acc[SRW + q][t]);
            if (lane == 0) a.shact[(size_t) t * F + j0 + q] = siluf_(gv) * uv;
        }
    }
}

}  // namespace

// ---------------------------------------------------------------------------------------------
// gate/up, eight waves per workgroup.  Routed workgroups: one (group, 32-row tile); wave w owns rows
// j = 32*tile + 4w .. +3 of both gate and up, so SwiGLU and the 16-wide requant (two 16-row blocks)
// stay inside the workgroup (D > 2048: 16-row tiles, two rows per wave).  With 32-row tiles the launch has few enough workgroups (10 experts x 16
// + 32 shared at the BASELINE shapes) that each gets a CU of its own.
// reference: exp_gu_quant_grouped (src/wzy_kernels_v2.cuh:1583-1721).
// Shared workgroups (gu_shared): 16 rows of the Q8_0 shared gate/up and SwiGLU (fp32 out; the per-32
// requant of silu_mul_quant32_multi runs in moe_down, so the 2.2 MB shared stream spreads over F/16
// workgroups).
// Dynamic LDS: x quantised, [T][D/32] int4 first halves, [T][D/32] int4 second halves, then the
// scales ([T][D/32] float2 per-16 pairs, or [T][D/32] float per-32).
// NCL = 32-column chunks of x per lane: 1 for D <= 2048, 2 for D <= 4096 (the reference's NE = 2560).
// ---------------------------------------------------------------------------------------------
template <int T, bool ROUTE, int RV, int NCL>
__global__ void __launch_bounds__(512) moe_gate_up_kernel(MoeGuArgs a) {
    extern __shared__ __align__(16) unsigned char s_dyn[];
    __shared__ float s_act[WZY_MAX_W][32];
    __shared__ int s_mem[WZY_MAX_W];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int bid = blockIdx.x;
    const int D = a.D, F = a.F, K = a.K;
    const int nc = D / 32;
    // routed path: f16 activation pairs [T*nc][16] then per-16 scales [T*nc] float2 (the shared path
    // lays out its per-32 quantisation in the same allocation)
    half2_t* s_xh = (half2_t*) s_dyn;
    float2* s_xs2 = (float2*) (s_xh + (size_t) T * nc * 16);

    if (bid < a.n_routed_wg) {
        constexpr int TR = gu_tile_rows(NCL), RPW = TR / 8;     // tile rows; gate (and up) rows per wave
        const int tiles = F / TR;
        const int g = bid / tiles, jt = bid - g * tiles;
        const int j0 = jt * TR + RPW * w;
        const MoeOffsets o = moe_offsets(D, F);
        int e = 0, cnt = 0;
        // lane chunks c = lane, lane + 64; rows rr < RPW gate j0 + rr, the others up j0 + rr - RPW
        int4 code[NCL][2 * RPW];
        uint32_t sc2[NCL][2 * RPW];
        // the weight loads of the lane (clamped, unconditional), issued as soon as the expert is known
        auto load_weights = [&](const uint8_t* rec) {
#pragma unroll
            for (int k = 0; k < NCL; ++k) {
                const int c = min(lane + 64 * k, nc - 1);
#pragma unroll
                for (int rr = 0; rr < 2 * RPW; ++rr) {
                    const int row = (rr < RPW) ? (j0 + rr) : (F + j0 + rr - RPW);
                    code[k][rr] = ld_stream_i4(rec + o.gu_codes + (size_t) row * (D / 2) + (size_t) c * 16);
                    sc2[k][rr] = *(const uint16_t*) (rec + o.gu_scales + (size_t) row * (D / 16) + 2 * c);
                }
            }
        };
        auto stage16 = [&](int t, int cc, int i) { stage_x16(a.x, D, t, cc, i, T * nc, s_xh, s_xs2); };
        if constexpr (ROUTE) {
            // in-workgroup routing (one-row windows): the logits are prefetched, x is staged while they
            // arrive, every workgroup routes the row (workgroup 0 publishes the tables for moe_down)
            __shared__ RouteLds r;
            float p[(T + 3) / 4][RV];
            route_prefetch<T, RV>(a.logits, a.E, p);
            if (tid < 256)                               // item 0 on wave 1: wave 0 routes the first row
                for (int i = (tid + 192) & 255; i < T * nc; i += 256) stage16(i / nc, i % nc, i);
            route_compute<T, RV>(p, a.E, K, r);
            if (g >= r.n_groups) return;                 // workgroup-uniform (workgroup 0 has g = 0)
            e = __builtin_amdgcn_readfirstlane(r.gexp[g]);
            cnt = r.gcnt[g];
            load_weights(a.experts + (size_t) e * o.rec);
            if (tid < WZY_MAX_W) s_mem[tid] = tid < cnt ? r.gmem[g][tid] : 0;
            if (bid == 0) publish_routing(r, a, T * K);
        } else {
            // routing tables published by moe_router: the expert is known at entry, its weights are
            // requested before x is staged (member m's chunk cc at LDS slot m * nc + cc)
            const int ng = *a.n_groups;
            e = __builtin_amdgcn_readfirstlane(a.grp_exp[g]);
            if (g >= ng) return;                         // workgroup-uniform
            cnt = a.grp_cnt[g];
            load_weights(a.experts + (size_t) e * o.rec);
            if (tid < WZY_MAX_W) s_mem[tid] = tid < cnt ? a.grp_mem[g * WZY_MAX_W + tid] : 0;
            for (int i = tid; i < cnt * nc; i += (int) blockDim.x) {
                const int m = i / nc;
                stage16(a.grp_mem[g * WZY_MAX_W + m] / K, i - m * nc, i);
            }
        }
        const uint8_t* rec = a.experts + (size_t) e * o.rec;
        const float sc_gate = ((const float*) (rec + o.tail))[0];
        const float sc_up = ((const float*) (rec + o.tail))[1];
        __syncthreads();
        float acc[2 * RPW][T];
#pragma unroll
        for (int rr = 0; rr < 2 * RPW; ++rr)
#pragma unroll
            for (int m = 0; m < T; ++m) acc[rr][m] = 0.f;
#pragma unroll
        for (int k = 0; k < NCL; ++k) {
            const int c = lane + 64 * k;
            if (c >= nc) continue;
#pragma unroll
            for (int m = 0; m < T; ++m) {
                if (m < cnt) {
                    const int xi = (ROUTE ? s_mem[m] / K : m) * nc + c;
                    half2_t xp[16];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint4 u = ((const uint4*) s_xh)[(size_t) q * (T * nc) + xi];
                        xp[4 * q] = __builtin_bit_cast(half2_t, u.x);
                        xp[4 * q + 1] = __builtin_bit_cast(half2_t, u.y);
                        xp[4 * q + 2] = __builtin_bit_cast(half2_t, u.z);
                        xp[4 * q + 3] = __builtin_bit_cast(half2_t, u.w);
                    }
                    const float2 xs = s_xs2[xi];
#pragma unroll
                    for (int rr = 0; rr < 2 * RPW; ++rr) {
                        const uint32_t sw = sc2[k][rr];
                        const int4 cw = code[k][rr];
                        const v2f_t ws = ue4m3x2_half(sw);
                        const float wsa = ws.x, wsb = ws.y;
                        const uint4 cu = make_uint4((uint32_t) cw.x, (uint32_t) cw.y, (uint32_t) cw.z, (uint32_t) cw.w);
                        acc[rr][m] = nvfp4_chunk_fma_h(cu, wsa, wsb, xp, xs.x, xs.y, acc[rr][m]);
                    }
                }
            }
        }
#pragma unroll
        for (int m = 0; m < T; ++m) {
            if (m < cnt) {
                // lane q < RPW: gate row q and (moved down from lane q + RPW) up row q
                float v[2 * RPW];
#pragma unroll
                for (int rr = 0; rr < 2 * RPW; ++rr) v[rr] = acc[rr][m];
                const float tot = reduce_wave<2 * RPW>(v);
                const float up = RPW == 4 ? dpp_f<DPP_ROW_SHL4>(tot) : (RPW == 2 ? dpp_f<DPP_ROW_SHL2>(tot) : dpp_f<DPP_ROW_SHL1>(tot));
                if (lane < RPW) s_act[m][RPW * w + lane] = siluf_(tot * sc_gate) * (up * sc_up);
            }
        }
        __syncthreads();
        if (tid < cnt * TR) {                            // one 16-lane row per (member, 16-row block)
            const int m = tid / TR, jj = tid % TR, jl = jj & 15;
            const int blk = (TR / 16) * jt + (jj >> 4);  // 16-row block of the F rows
            const float v = s_act[m][jj];
            const float amax = max16(fabsf(v));
            const float d = amax / 127.0f;
            const float inv = d > 0.f ? 127.0f / amax : 0.f;
            const int q = max(-127, min(127, rn_int(v * inv)));
            const int f = s_mem[m];
            a.ah16[((size_t) f * (F / 16) + blk) * 16 + (jl & 7) * 2 + (jl >> 3)] =
                __builtin_bit_cast(uint16_t, (_Float16) (float) q);
            if (jl == 0) a.as16[(size_t) f * (F / 16) + blk] = d;
        }
        return;
    }

    gu_shared<T, NCL>(a, bid - a.n_routed_wg, s_dyn);
}

// ---------------------------------------------------------------------------------------------
// gate/up of multi-row windows (T > 1), one round of resident workgroups.  The first n_routed_wg
// workgroups (about one per CU beside the shared ones) each route the window themselves from the
// router logits (every workgroup computes the same tables; workgroup 0 publishes them for moe_down)
// and stage all T rows of x quantised per 16 in LDS; then each takes the window's work items
// (group, tile) bid, bid + n_routed_wg, ... in phases of MAXI items, issuing every weight load of a
// phase before computing its first item.  The window's routing thus costs one pass per workgroup,
// run in parallel, instead of a routing pass behind a cross-workgroup handoff, and no workgroup waits
// for a second round of residency.  Items and arithmetic are those of moe_gate_up_kernel.
// The remaining workgroups run the shared expert (gu_shared).
// ---------------------------------------------------------------------------------------------
template <int T, int RV, int NCL>
__global__ void __launch_bounds__(512) moe_gate_up_window_kernel(MoeGuArgs a) {
    extern __shared__ __align__(16) unsigned char s_dyn[];
    __shared__ float s_act2[2][WZY_MAX_W][32];       // SwiGLU values, alternating between items
    __shared__ RouteLds r;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int bid = blockIdx.x;
    if (bid >= a.n_routed_wg) {
        gu_shared<T, NCL>(a, bid - a.n_routed_wg, s_dyn);
        return;
    }
    const int D = a.D, F = a.F, K = a.K;
    const int nc = D / 32, nr = a.n_routed_wg;
    half2_t* s_xh = (half2_t*) s_dyn;
    float2* s_xs2 = (float2*) (s_xh + (size_t) T * nc * 16);
    constexpr int TR = gu_tile_rows(NCL), RPW = TR / 8;         // tile rows; gate (and up) rows per wave
    const int tiles = F / TR;
    const MoeOffsets o = moe_offsets(D, F);
    {
        float p[(T + 3) / 4][RV];
        route_prefetch<T, RV>(a.logits, a.E, p);
        // waves 4-7 stage x first (waves 0-3 route)
        for (int i = (tid + 256) & 511; i < T * nc; i += 512) stage_x16(a.x, D, i / nc, i % nc, i, T * nc, s_xh, s_xs2);
        route_compute<T, RV>(p, a.E, K, r);              // ends with a barrier
    }
    if (bid == 0) publish_routing(r, a, T * K);
    const int n_items = r.n_groups * tiles;
    // the weight loads of one item (group, tile) into one register set
    auto load_item = [&](int item, int4 (&code)[NCL][2 * RPW], uint32_t (&sc2)[NCL][2 * RPW], float2& tail) {
        const int g = item / tiles, jt = item - g * tiles;
        const int e = __builtin_amdgcn_readfirstlane(r.gexp[g]);
        const uint8_t* rec = a.experts + (size_t) e * o.rec;
        const int j0 = jt * TR + RPW * w;
#pragma unroll
        for (int k = 0; k < NCL; ++k) {
            const int c = min(lane + 64 * k, nc - 1);
#pragma unroll
            for (int rr = 0; rr < 2 * RPW; ++rr) {
                const int row = (rr < RPW) ? (j0 + rr) : (F + j0 + rr - RPW);
                code[k][rr] = ld_stream_i4(rec + o.gu_codes + (size_t) row * (D / 2) + (size_t) c * 16);
                sc2[k][rr] = *(const uint16_t*) (rec + o.gu_scales + (size_t) row * (D / 16) + 2 * c);
            }
        }
        tail = *(const float2*) (rec + o.tail);
    };
    // gate/up rows of one item for its members, SwiGLU, per-16 requant into ah16 / as16.  Each row's
    // codes are expanded to f16 pairs once and dotted with every member's activations.
    auto compute_item = [&](int item, const int4 (&code)[NCL][2 * RPW], const uint32_t (&sc2)[NCL][2 * RPW],
                            float2 tail, float (&s_act)[WZY_MAX_W][32]) {
        const int g = item / tiles, jt = item - g * tiles;
        const int cnt = r.gcnt[g];
        float acc[2 * RPW][T];
#pragma unroll
        for (int rr = 0; rr < 2 * RPW; ++rr)
#pragma unroll
            for (int m = 0; m < T; ++m) acc[rr][m] = 0.f;
#pragma unroll
        for (int k = 0; k < NCL; ++k) {
            const int c = lane + 64 * k;
            if (c >= nc) continue;
            half2_t xq[T][16];
            float2 xs[T];
#pragma unroll
            for (int m = 0; m < T; ++m) {
                if (m < cnt) {                           // workgroup-uniform
                    const int xi = (r.gmem[g][m] / K) * nc + c;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint4 u = ((const uint4*) s_xh)[(size_t) q * (T * nc) + xi];
                        xq[m][4 * q] = __builtin_bit_cast(half2_t, u.x);
                        xq[m][4 * q + 1] = __builtin_bit_cast(half2_t, u.y);
                        xq[m][4 * q + 2] = __builtin_bit_cast(half2_t, u.z);
                        xq[m][4 * q + 3] = __builtin_bit_cast(half2_t, u.w);
                    }
                    xs[m] = s_xs2[xi];
                }
            }
#pragma unroll
            for (int rr = 0; rr < 2 * RPW; ++rr) {
                const uint32_t sw = sc2[k][rr];
                const v2f_t ws = ue4m3x2_half(sw);
                const float wsa = ws.x, wsb = ws.y;
                half2_t wq[16];
                fp4_expand16(code[k][rr], wq);
#pragma unroll
                for (int m = 0; m < T; ++m) {
                    if (m < cnt) {
                        acc[rr][m] = fmaf(wsa * xs[m].x, dot16_pairs(&wq[0], &xq[m][0]), acc[rr][m]);
                        acc[rr][m] = fmaf(wsb * xs[m].y, dot16_pairs(&wq[8], &xq[m][8]), acc[rr][m]);
                    }
                }
            }
        }
#pragma unroll
        for (int m = 0; m < T; ++m) {
            if (m < cnt) {
                // lane q < RPW: gate row q and (moved down from lane q + RPW) up row q
                float v[2 * RPW];
#pragma unroll
                for (int rr = 0; rr < 2 * RPW; ++rr) v[rr] = acc[rr][m];
                const float tot = reduce_wave<2 * RPW>(v);
                const float up = RPW == 4 ? dpp_f<DPP_ROW_SHL4>(tot) : (RPW == 2 ? dpp_f<DPP_ROW_SHL2>(tot) : dpp_f<DPP_ROW_SHL1>(tot));
                if (lane < RPW) s_act[m][RPW * w + lane] = siluf_(tot * tail.x) * (up * tail.y);
            }
        }
        __syncthreads();
        if (tid < cnt * TR) {                            // one 16-lane row per (member, 16-row block)
            const int m = tid / TR, jj = tid % TR, jl = jj & 15;
            const int blk = (TR / 16) * jt + (jj >> 4);
            const float v = s_act[m][jj];
            const float amax = max16(fabsf(v));
            const float d = amax / 127.0f;
            const float inv = d > 0.f ? 127.0f / amax : 0.f;
            const int q = max(-127, min(127, rn_int(v * inv)));
            const int f = r.gmem[g][m];
            a.ah16[((size_t) f * (F / 16) + blk) * 16 + (jl & 7) * 2 + (jl >> 3)] =
                __builtin_bit_cast(uint16_t, (_Float16) (float) q);
            if (jl == 0) a.as16[(size_t) f * (F / 16) + blk] = d;
        }
        // no barrier here: the next item writes the other s_act buffer, and the one after it passes
        // the next item's barrier first
    };
    // items bid, bid + nr, bid + 2 nr, ... in two register sets: an item's loads are issued as soon
    // as the set is free, so they are in flight while the other set's item is computed.  The loads are
    // unconditional (an item past the end reloads the last one, whose lines are cached): a branch
    // around them would make the compiler wait for every load in flight at the join.
    int4 code_a[NCL][2 * RPW], code_b[NCL][2 * RPW];
    uint32_t sc_a[NCL][2 * RPW], sc_b[NCL][2 * RPW];
    float2 tail_a, tail_b;
    const int last = n_items - 1;                    // >= 0: a window routes at least one group
    int it_a = bid, it_b = bid + nr;
    load_item(min(it_a, last), code_a, sc_a, tail_a);
    load_item(min(it_b, last), code_b, sc_b, tail_b);
    while (it_a < n_items) {                         // workgroup-uniform
        compute_item(it_a, code_a, sc_a, tail_a, s_act2[0]);
        it_a += 2 * nr;
        if (it_b >= n_items) break;
        load_item(min(it_a, last), code_a, sc_a, tail_a);
        compute_item(it_b, code_b, sc_b, tail_b, s_act2[1]);
        it_b += 2 * nr;
        if (it_a >= n_items) break;
        load_item(min(it_b, last), code_b, sc_b, tail_b);
    }
}

// ---------------------------------------------------------------------------------------------
// router: logits [T x E] = bf16 W . x (fp32 accumulate) and the shared-expert gate scalar, one row per
// wave (rows 0..E-1 the router, row E the shared gate); the last workgroup to finish routes the
// window and publishes ids / weights / groups for moe_gate_up and moe_down.  The arrival counter is
// file-scope device memory (zero at load, reset by the routing workgroup): router launches on one
// device must not overlap.
// reference: launch_gemm_bf16 (router) + router_top10_fast_multi + the grouping
// (src/wzy_stage_v2.cuh:699-706; src/wzy_kernels_v2.cuh:307-337,989-1090; src/wzy_cpu_moe.cuh:74-127)
// ---------------------------------------------------------------------------------------------
constexpr int RT_ROWS = 4;          // rows per workgroup (one per wave)
constexpr int RT_XROWS = 2;         // rows of x staged in LDS per pass
__device__ unsigned g_rt_arrive[1];

// NP = 8-value weight pieces per lane (D <= 512 * NP).  Every weight load of the wave is issued first;
// x comes from LDS, RT_XROWS rows per pass.
template <int T, int RV, int NP>
__global__ void __launch_bounds__(256) moe_router_kernel(MoeRtArgs a) {
    __shared__ RouteLds r;
    __shared__ bool s_last;
    __shared__ __align__(16) float s_x[RT_XROWS * 512 * NP];
    __shared__ float s_out[RT_ROWS][T];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int D = a.D, E = a.E;
    const int row = blockIdx.x * RT_ROWS + w;
    const int npc = D / 8;
    const bool active = row <= E;                        // rows 0..E-1 router, E the shared gate
    const uint16_t* wr = row < E ? a.router + (size_t) row * D : a.sgate;
    uint4 wv[NP];
#pragma unroll
    for (int j = 0; j < NP; ++j) {
        const int pc = lane + 64 * j;
        wv[j] = (active && pc < npc) ? ld_stream_u4(wr + (size_t) pc * 8) : make_uint4(0, 0, 0, 0);
    }
    float acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = 0.f;
#pragma unroll
    for (int t0 = 0; t0 < T; t0 += RT_XROWS) {
        const int nr = min(RT_XROWS, T - t0);
        for (int i = tid; i < nr * D / 4; i += 256) ((float4*) s_x)[i] = ((const float4*) (a.x + (size_t) t0 * D))[i];
        __syncthreads();
#pragma unroll
        for (int j = 0; j < NP; ++j) {
            const int pc = lane + 64 * j;
            if (pc < npc) {
                const uint32_t q[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
#pragma unroll
                for (int tt = 0; tt < RT_XROWS; ++tt) {
                    if (t0 + tt < T) {
                        const float4* xp = (const float4*) (s_x + (size_t) tt * D + (size_t) pc * 8);
                        const float4 x0 = xp[0], x1 = xp[1];
                        float s = acc[t0 + tt];
                        s = fmaf(bf16_lo(q[0]), x0.x, s); s = fmaf(bf16_hi(q[0]), x0.y, s);
                        s = fmaf(bf16_lo(q[1]), x0.z, s); s = fmaf(bf16_hi(q[1]), x0.w, s);
                        s = fmaf(bf16_lo(q[2]), x1.x, s); s = fmaf(bf16_hi(q[2]), x1.y, s);
                        s = fmaf(bf16_lo(q[3]), x1.z, s); s = fmaf(bf16_hi(q[3]), x1.w, s);
                        acc[t0 + tt] = s;
                    }
                }
            }
        }
        __syncthreads();
    }
    // the workgroup's outputs go to global memory from wave 0 alone, so that one release fence (an
    // agent-scope fence writes back L2) covers every store before the arrival.  The lane partials and
    // the sum tree are gemv_segs' for a bf16 row, so the logits equal those of one-row windows.
    reduce_wave_store<T>(acc, [&](int t, float v) { s_out[w][t] = v; });
    __syncthreads();
    if (w == 0) {
        if (lane < RT_ROWS * T) {
            const int rw = blockIdx.x * RT_ROWS + lane / T, t = lane % T;
            if (rw < E) a.logits[(size_t) t * E + rw] = s_out[lane / T][t];
            else if (rw == E) a.sg[t] = s_out[lane / T][t];
        }
        __threadfence();
        if (lane == 0) s_last = atomicAdd(a.arrive, 1u) == gridDim.x - 1;
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    float p[(T + 3) / 4][RV];
    route_prefetch<T, RV>(a.logits, E, p);
    route_compute<T, RV>(p, E, a.K, r);
    const int n_ent = T * a.K;
    for (int i = tid; i < n_ent; i += blockDim.x) {
        a.ids[i] = r.ids[i];
        a.wts[i] = r.w[i];
        if (i < r.n_groups) {
            a.grp_exp[i] = r.gexp[i];
            a.grp_cnt[i] = r.gcnt[i];
            for (int m = 0; m < WZY_MAX_W; ++m) a.grp_mem[i * WZY_MAX_W + m] = m < r.gcnt[i] ? r.gmem[i][m] : 0;
        } else {
            a.grp_exp[i] = 0;                            // unused groups: a valid expert id for readers
            a.grp_cnt[i] = 0;
        }
    }
    if (tid == 0) {
        *a.n_groups = r.n_groups;
        *a.arrive = 0u;
    }
}

// ---------------------------------------------------------------------------------------------
// down + combine.  Workgroup = DN_TILE output rows for every group and the shared expert, so the
// combine comb = sigmoid(sgate)*shared + sum_k w_k * part_k (routed-slot order) stays in LDS.
// Work items (group or shared, row) go round-robin to the NT/16 16-lane slots (NT = 256 threads for
// one-row windows, 1024 for windows of several rows, whose items are up to T*K + 1 groups x 8 rows);
// a slot issues the loads of DN_BATCH items before computing any of them.  One 32-value chunk per lane per item
// (F = 512: 16 chunks per row).  STAGE: the routed and shared activations are copied to LDS first
// (dynamic LDS: routed activations as f16 pairs in 16-byte quarters [4][n_ent * F/32], as [n_ent][F/16] float, shq
// halves [T][F/32] x2 int4, shs [T][F/32] float).
// reference: exp_down_2r_grouped (src/wzy_kernels_v2.cuh:1725-1834), shared down launch_gemm_q8p
// (src/wzy_stage_v2.cuh:714), moe_combine_shared_multi (src/wzy_kernels_v2.cuh:1281-1294).
// ---------------------------------------------------------------------------------------------
template <int T, bool STAGE, int CI, int NT>
__global__ void __launch_bounds__(NT) moe_down_kernel(MoeDnArgs a) {
    extern __shared__ __align__(16) unsigned char s_dyn[];
    __shared__ float s_part[MAX_ENT][DN_TILE];
    __shared__ float s_sh[WZY_MAX_W][DN_TILE];
    __shared__ int s_gexp[MAX_ENT], s_gcnt[MAX_ENT];
    __shared__ int s_gmem[MAX_ENT][WZY_MAX_W];
    __shared__ float s_wts[MAX_ENT], s_sg[WZY_MAX_W];
    const int tid = threadIdx.x;
    const int D = a.D, F = a.F, K = a.K;
    const int d0 = blockIdx.x * DN_TILE;
    const int nchunk = F / 32, n_ent = T * K;
    constexpr int DN_BATCH = dn_batch<T, CI, STAGE>(), NSLOT = NT / 16;
    // the group tables of every possible group are loaded without waiting for the group count
    const int ng = *a.n_groups;
    // shared activation quantised per 32 (both variants), then (STAGE) the routed activations
    int4* s_sha = (int4*) s_dyn;                      // [T * nchunk] first / second 16-byte halves
    int4* s_shb = s_sha + (size_t) T * nchunk;
    float* s_shs = (float*) (s_shb + (size_t) T * nchunk);
    uint4* s_ah = (uint4*) (s_shs + dn_shs_floats(T, nchunk));   // [4][n_ent * nchunk]: quarter k of a chunk's 16 f16 pairs
    float* s_as = (float*) (s_ah + (size_t) n_ent * nchunk * 4);
    // Item `tid` of every table and staging copy is loaded (clamped index, no branch) before the
    // first LDS write: a stride loop per table would wait for one table's loads before requesting
    // the next.  Only copies of more than NT items loop for the rest.
    const int n_aq = n_ent * nchunk, n_as4 = n_ent * (F / 16) / 4, n_sh = T * nchunk;
    {
        const int ie = min(tid, n_ent - 1);
        const int gexp = a.grp_exp[ie], gcnt = a.grp_cnt[ie];
        int gmem[WZY_MAX_W];
#pragma unroll
        for (int m = 0; m < WZY_MAX_W; ++m) gmem[m] = a.grp_mem[ie * WZY_MAX_W + m];
        const float wt = a.wts[ie], sgv = a.sg[min(tid, T - 1)];
        uint4 xh[4];
        float4 xs4;
        if (STAGE) {
            const uint4* xp = (const uint4*) (a.ah16 + (size_t) min(tid, n_aq - 1) * 32);
#pragma unroll
            for (int k = 0; k < 4; ++k) xh[k] = xp[k];
            xs4 = ((const float4*) a.as16)[min(tid, n_as4 - 1)];
        }
        float hv[8];                                  // shared activations 8q .. 8q+7 of block tid/4
        {
            const float4* hp = (const float4*) (a.shact + (size_t) min(tid >> 2, n_sh - 1) * 32 + (tid & 3) * 8);
            const float4 f0 = hp[0], f1 = hp[1];
            hv[0] = f0.x; hv[1] = f0.y; hv[2] = f0.z; hv[3] = f0.w;
            hv[4] = f1.x; hv[5] = f1.y; hv[6] = f1.z; hv[7] = f1.w;
        }
        if (tid < n_ent) {
            s_gexp[tid] = gexp;
            s_gcnt[tid] = gcnt;
#pragma unroll
            for (int m = 0; m < WZY_MAX_W; ++m) s_gmem[tid][m] = gmem[m];
            s_wts[tid] = wt;
        }
        if (tid < T) s_sg[tid] = sgv;
        if (STAGE) {
            if (tid < n_aq)
#pragma unroll
                for (int k = 0; k < 4; ++k) s_ah[(size_t) k * n_aq + tid] = xh[k];
            if (tid < n_as4) ((float4*) s_as)[tid] = xs4;
        }
        {                                             // silu_mul_quant32: d = amax/127, q = rint(v*127/amax)
            float hs;
            const uint2 hq = quant32_quad(hv, hs);    // all lanes: the quad max reads its neighbours
            const int ib = tid >> 2, q = tid & 3;
            if (tid < 4 * n_sh) {
                ((uint2*) (q < 2 ? s_sha : s_shb))[ib * 2 + (q & 1)] = hq;
                if (q == 0) s_shs[ib] = hs;
            }
        }
    }
    for (int i = tid + NT; i < n_ent; i += NT) {
        s_gexp[i] = a.grp_exp[i];
        s_gcnt[i] = a.grp_cnt[i];
#pragma unroll
        for (int m = 0; m < WZY_MAX_W; ++m) s_gmem[i][m] = a.grp_mem[i * WZY_MAX_W + m];
        s_wts[i] = a.wts[i];
    }
    if (STAGE) {
        for (int i = tid + NT; i < n_aq; i += NT) {
            const uint4* xp = (const uint4*) (a.ah16 + (size_t) i * 32);
#pragma unroll
            for (int k = 0; k < 4; ++k) s_ah[(size_t) k * n_aq + i] = xp[k];
        }
        for (int i = tid + NT; i < n_as4; i += NT) ((float4*) s_as)[i] = ((const float4*) a.as16)[i];
    }
    for (int i = tid + NT; i < 4 * n_sh; i += NT) {  // whole quads leave the loop together
        const float4* hp = (const float4*) (a.shact + (size_t) (i >> 2) * 32 + (i & 3) * 8);
        const float4 f0 = hp[0], f1 = hp[1];
        const float hv[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
        float hs;
        const uint2 hq = quant32_quad(hv, hs);
        const int ib = i >> 2, q = i & 3;
        ((uint2*) (q < 2 ? s_sha : s_shb))[ib * 2 + (q & 1)] = hq;
        if (q == 0) s_shs[ib] = hs;
    }
    __syncthreads();
    const MoeOffsets o = moe_offsets(D, F);
    const int slot = tid >> 4, li = tid & 15;
    const int n_items = (ng + 1) * DN_TILE;          // group ng = shared expert
    for (int i0 = slot; i0 < n_items; i0 += NSLOT * DN_BATCH) {
        float acc[DN_BATCH][T];
        float sdn[DN_BATCH];
#pragma unroll
        for (int b = 0; b < DN_BATCH; ++b) {
            // tensor scale of the item's expert, loaded with the first codes (shared items read
            // expert 0's and ignore it)
            const int item = min(i0 + NSLOT * b, n_items - 1);
            const int g = item / DN_TILE;
            const uint8_t* rec = a.experts + (g < ng ? (size_t) s_gexp[g] * o.rec : 0);
            sdn[b] = ((const float*) (rec + o.tail))[2];
#pragma unroll
            for (int m = 0; m < T; ++m) acc[b][m] = 0.f;
        }
        // CI = nchunk/16 rounded up chunk rounds per lane, unrolled (a loop here would make every
        // round wait for the previous round's loads)
#pragma unroll
        for (int ci = 0; ci < CI; ++ci) {
            const bool cvalid = li + 16 * ci < nchunk;
            const int c = min(li + 16 * ci, nchunk - 1);
            // the weight loads of all DN_BATCH items first (raw scales), arithmetic afterwards.  Routed
            // and shared items load through one selected pointer (32 code bytes, one 16-bit scale
            // word, one tail float): no divergent branch, so no load waits for an earlier one.
            int4 c0[DN_BATCH], c1[DN_BATCH];
            uint32_t sraw[DN_BATCH];
#pragma unroll
            for (int b = 0; b < DN_BATCH; ++b) {
                const int item = min(i0 + NSLOT * b, n_items - 1);
                const int g = item / DN_TILE, d = d0 + item % DN_TILE;
                const bool routed = g < ng;
                const uint8_t* rec = a.experts + (routed ? (size_t) s_gexp[g] * o.rec : 0);
                const uint8_t* cp = routed ? rec + o.dn_codes + (size_t) d * (F / 2) + (size_t) c * 16
                                           : (const uint8_t*) (a.shd_q + (size_t) d * F + (size_t) c * 32);
                const uint16_t* sp = routed ? (const uint16_t*) (rec + o.dn_scales + (size_t) d * (F / 16) + 2 * c)
                                            : a.shd_s + (size_t) d * nchunk + c;
                c0[b] = ld_stream_i4((const int4*) cp);
                c1[b] = ld_stream_i4((const int4*) cp + 1);
                sraw[b] = *sp;
            }
#pragma unroll
            for (int b = 0; b < DN_BATCH; ++b) {
                const int item = i0 + NSLOT * b;
                if (item >= n_items || !cvalid) continue;
                const int g = item / DN_TILE;
                if (g < ng) {
                    const uint4 cu = make_uint4((uint32_t) c0[b].x, (uint32_t) c0[b].y, (uint32_t) c0[b].z,
                                                (uint32_t) c0[b].w);
                    const v2f_t ws = ue4m3x2_half(sraw[b]);
                    const float wsa = ws.x, wsb = ws.y;
                    const int cnt = s_gcnt[g];
#pragma unroll
                    for (int m = 0; m < T; ++m) {
                        if (m < cnt) {
                            const int f = s_gmem[g][m];
                            const int xi = f * nchunk + c;
                            const uint4* xq = STAGE ? s_ah + xi : (const uint4*) (a.ah16 + (size_t) xi * 32);
                            const size_t xstep = STAGE ? (size_t) n_aq : 1;   // LDS: quarter-major
                            const float2 xs = STAGE ? ((const float2*) s_as)[xi]
                                                    : *(const float2*) (a.as16 + (size_t) f * (F / 16) + 2 * c);
                            half2_t xp[16];
#pragma unroll
                            for (int k = 0; k < 4; ++k) {
                                const uint4 u = xq[k * xstep];
                                xp[4 * k] = __builtin_bit_cast(half2_t, u.x);
                                xp[4 * k + 1] = __builtin_bit_cast(half2_t, u.y);
                                xp[4 * k + 2] = __builtin_bit_cast(half2_t, u.z);
                                xp[4 * k + 3] = __builtin_bit_cast(half2_t, u.w);
                            }
                            acc[b][m] = nvfp4_chunk_fma_h(cu, wsa, wsb, xp, xs.x, xs.y, acc[b][m]);
                        }
                    }
                } else {
                    const float dw = h16_to_f((uint16_t) sraw[b]);
#pragma unroll
                    for (int t = 0; t < T; ++t) {
                        const int xi = t * nchunk + c;
                        acc[b][t] = fmaf(dw * s_shs[xi], (float) (dot16(c0[b], s_sha[xi]) + dot16(c1[b], s_shb[xi])),
                                         acc[b][t]);
                    }
                }
            }
        }
        // 16-lane sums (every lane of a slot holds the same item, so the groups are uniform)
#pragma unroll
        for (int b = 0; b < DN_BATCH; ++b) {
            const int item = i0 + NSLOT * b;
            const bool valid = item < n_items;
            const int g = valid ? item / DN_TILE : 0, rl = item % DN_TILE;
            const int cnt = (valid && g < ng) ? s_gcnt[g] : T;
#pragma unroll
            for (int m = 0; m < T; ++m) {
                const float v = sum16(acc[b][m]);
                if (li == 0 && valid && m < cnt) {
                    if (g < ng) s_part[s_gmem[g][m]][rl] = v * sdn[b];
                    else s_sh[m][rl] = v;
                }
            }
        }
    }
    __syncthreads();
    if (tid < T * DN_TILE) {
        const int t = tid / DN_TILE, rl = tid % DN_TILE;
        float s = s_sh[t][rl] * sigmoidf_(s_sg[t]);
        for (int k = 0; k < K; ++k) {
            const float wk = s_wts[t * K + k];
            if (wk != 0.0f) s += wk * s_part[t * K + k][rl];
        }
        a.comb[(size_t) t * D + d0 + rl] = s;
    }
}

// Routing alone (the device routing of moe_gate_up): one workgroup, window rows in waves.
template <int T, int RV>
__global__ void __launch_bounds__(256) moe_route_kernel(const float* __restrict__ logits, int E, int K,
                                                        int* __restrict__ ids, float* __restrict__ wts) {
    __shared__ RouteLds r;
    float p[(T + 3) / 4][RV];
    route_prefetch<T, RV>(logits, E, p);
    route_compute<T, RV>(p, E, K, r);
    for (int i = threadIdx.x; i < T * K; i += blockDim.x) {
        ids[i] = r.ids[i];
        wts[i] = r.w[i];
    }
}

// ---------------------------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------------------------
namespace wzy {

MoeWs moe_ws_carve(void* base, size_t cap, int D, int F, int E, int K, int T, size_t* need) {
    Arena a(base, cap);
    MoeWs w;
    const int n_ent = T * K;
    w.logits = a.take<float>((size_t) T * E);
    w.sg = a.take<float>(T);
    w.ids = a.take<int>(n_ent);
    w.wts = a.take<float>(n_ent);
    w.n_groups = a.take<int>(1);
    w.grp_exp = a.take<int>(n_ent);
    w.grp_cnt = a.take<int>(n_ent);
    w.grp_mem = a.take<int>((size_t) n_ent * WZY_MAX_W);
    w.ah16 = a.take<uint16_t>((size_t) n_ent * F);
    w.as16 = a.take<float>((size_t) n_ent * F / 16);
    w.shact = a.take<float>((size_t) T * F);
    if (need) *need = a.off;
    return w;
}

int moe_check(const wzy_moe_weights* w, int T) {
    WZY_REQUIRE(w != nullptr, "moe: null weights");
    WZY_REQUIRE(T >= 1 && T <= WZY_MAX_W, "moe: T must be in [1, %d]", WZY_MAX_W);
    WZY_REQUIRE(w->n_embd % 256 == 0 && w->n_embd >= 256 && w->n_embd <= 4096,
                "moe: n_embd must be a multiple of 256 <= 4096");
    WZY_REQUIRE(w->n_ff % 64 == 0 && w->n_ff >= 64 && w->n_ff <= 2048, "moe: n_ff must be a multiple of 64 <= 2048");
    WZY_REQUIRE(w->n_exp >= 1 && w->n_exp <= 1024, "moe: n_exp must be in [1, 1024]");
    WZY_REQUIRE(w->top_k >= 1 && w->top_k <= MOE_MAX_K && w->top_k <= w->n_exp, "moe: top_k must be in [1, %d]",
                MOE_MAX_K);
    WZY_REQUIRE(w->router && w->sgate && w->experts && w->sh_gate_q && w->sh_gate_s && w->sh_up_q && w->sh_up_s &&
                    w->sh_down_q && w->sh_down_s,
                "moe: null weight pointer");
    return WZY_OK;
}

template <int T, int NP>
static void launch_rt_tn(const MoeRtArgs& a, hipStream_t st) {
    const dim3 grid((a.E + 1 + RT_ROWS - 1) / RT_ROWS);
    if (a.E <= 512) hipLaunchKernelGGL((moe_router_kernel<T, 8, NP>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((moe_router_kernel<T, 16, NP>), grid, dim3(256), 0, st, a);
}
template <int T>
static void launch_rt_t(const MoeRtArgs& a, hipStream_t st) {
    if (a.D <= 2048) launch_rt_tn<T, 4>(a, st);
    else launch_rt_tn<T, 8>(a, st);
}

int moe_launch_route(const wzy_moe_weights* w, const MoeWs& ws, const float* x, int T, hipStream_t st) {
    if (T <= GU_WINDOW_MAX_T) {                      // logits only; the gate/up workgroups route
        GemvSegs segs;
        segs.n = 2;
        segs.seg[0] = GemvSeg{w->router, nullptr, ws.logits, w->n_exp, GEMV_BF16, 0, 0};
        segs.seg[1] = GemvSeg{w->sgate, nullptr, ws.sg, 1, GEMV_BF16, 1, 0};
        return launch_gemv_segs(segs, x, w->n_embd, T, st);
    }
    WZY_REQUIRE(w->n_embd % 8 == 0 && w->n_embd <= 4096, "moe router: n_embd must be a multiple of 8 <= 4096");
    MoeRtArgs a{};
    a.router = w->router; a.sgate = w->sgate; a.x = x; a.D = w->n_embd; a.E = w->n_exp; a.K = w->top_k;
    a.logits = ws.logits; a.sg = ws.sg; a.ids = ws.ids; a.wts = ws.wts; a.n_groups = ws.n_groups;
    a.grp_exp = ws.grp_exp; a.grp_cnt = ws.grp_cnt; a.grp_mem = ws.grp_mem;
    WZY_HIP_TRY(hipGetSymbolAddress((void**) &a.arrive, HIP_SYMBOL(g_rt_arrive)));
    switch (T) {
        case 1: launch_rt_t<1>(a, st); break;
        case 2: launch_rt_t<2>(a, st); break;
        case 3: launch_rt_t<3>(a, st); break;
        case 4: launch_rt_t<4>(a, st); break;
        case 5: launch_rt_t<5>(a, st); break;
        case 6: launch_rt_t<6>(a, st); break;
        case 7: launch_rt_t<7>(a, st); break;
        default: launch_rt_t<8>(a, st); break;
    }
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

// compute units of the current device (queried once per device)
static int device_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

static MoeGuArgs gu_args(const wzy_moe_weights* w, const MoeWs& ws, const float* x, int T) {
    MoeGuArgs a{};
    a.experts = w->experts; a.D = w->n_embd; a.F = w->n_ff; a.E = w->n_exp; a.K = w->top_k;
    a.x = x; a.logits = ws.logits;
    a.ids = ws.ids; a.wts = ws.wts; a.n_groups = ws.n_groups; a.grp_exp = ws.grp_exp; a.grp_cnt = ws.grp_cnt;
    a.grp_mem = ws.grp_mem; a.ah16 = ws.ah16; a.as16 = ws.as16;
    a.shg_q = w->sh_gate_q; a.shg_s = w->sh_gate_s; a.shu_q = w->sh_up_q; a.shu_s = w->sh_up_s;
    a.shact = ws.shact;
    const int ncl = w->n_embd > 2048 ? 2 : 1;
    const int items = (w->n_ff / gu_tile_rows(ncl)) * T * w->top_k;   // the most (group, tile) items
    if (T == 1 || T > GU_WINDOW_MAX_T) {
        a.n_routed_wg = items;                       // one item per workgroup
    } else {                                         // one round of resident workgroups
        const int n_sh = w->n_ff / sh_tile_rows(ncl);
        a.n_routed_wg = std::max(8, std::min(items, device_cus() - n_sh));
    }
    return a;
}
static MoeDnArgs dn_args(const wzy_moe_weights* w, const MoeWs& ws, float* comb) {
    MoeDnArgs a{};
    a.experts = w->experts; a.D = w->n_embd; a.F = w->n_ff; a.K = w->top_k;
    a.n_groups = ws.n_groups; a.grp_exp = ws.grp_exp; a.grp_cnt = ws.grp_cnt; a.grp_mem = ws.grp_mem;
    a.ah16 = ws.ah16; a.as16 = ws.as16; a.shd_q = w->sh_down_q; a.shd_s = w->sh_down_s;
    a.shact = ws.shact; a.wts = ws.wts; a.sg = ws.sg; a.comb = comb;
    return a;
}

// One-row windows route inside every gate/up workgroup (the router is a plain GEMV: a separate
// routing pass costs more than it saves at T = 1); windows of several rows route once in moe_router.
template <int T, int NCL>
static void launch_gu_tn(const MoeGuArgs& a, hipStream_t st) {
    const size_t lds = (size_t) T * (a.D / 32) * (16 * sizeof(uint32_t) + sizeof(float2));   // >= the shared path's
    const dim3 grid(a.n_routed_wg + a.F / sh_tile_rows(NCL));
    if constexpr (T > GU_WINDOW_MAX_T) {
        hipLaunchKernelGGL((moe_gate_up_kernel<T, false, 8, NCL>), grid, dim3(512), lds, st, a);
    } else if constexpr (T > 1) {
        if (a.E <= 512) hipLaunchKernelGGL((moe_gate_up_window_kernel<T, 8, NCL>), grid, dim3(512), lds, st, a);
        else hipLaunchKernelGGL((moe_gate_up_window_kernel<T, 16, NCL>), grid, dim3(512), lds, st, a);
    } else if (a.E <= 512) {
        hipLaunchKernelGGL((moe_gate_up_kernel<1, true, 8, NCL>), grid, dim3(512), lds, st, a);
    } else {
        hipLaunchKernelGGL((moe_gate_up_kernel<1, true, 16, NCL>), grid, dim3(512), lds, st, a);
    }
}
template <int T>
static void launch_gu_t(const MoeGuArgs& a, hipStream_t st) {
    if (a.D <= 2048) launch_gu_tn<T, 1>(a, st);
    else launch_gu_tn<T, 2>(a, st);
}
template <int T, int CI>
static void launch_dn_tc(const MoeDnArgs& a, size_t lds, hipStream_t st) {
    const size_t lds_sh = dn_shared_lds(T, a.F / 32);
    constexpr int NTS = dn_threads<T, CI, true>(), NTD = dn_threads<T, CI, false>();
    if (lds <= (size_t) DN_STAGE_BYTES)
        hipLaunchKernelGGL((moe_down_kernel<T, true, CI, NTS>), dim3(a.D / DN_TILE), dim3(NTS), lds, st, a);
    else
        hipLaunchKernelGGL((moe_down_kernel<T, false, CI, NTD>), dim3(a.D / DN_TILE), dim3(NTD), lds_sh, st, a);
}
template <int T>
static void launch_dn_t(const MoeDnArgs& a, hipStream_t st) {
    const int n_ent = T * a.K, nchunk = a.F / 32;
    const size_t lds = dn_shared_lds(T, nchunk) + (size_t) n_ent * nchunk * 4 * sizeof(uint4) +
                       (size_t) n_ent * (a.F / 16) * sizeof(float);
    switch ((nchunk + 15) / 16) {
        case 1: launch_dn_tc<T, 1>(a, lds, st); break;
        case 2: launch_dn_tc<T, 2>(a, lds, st); break;
        case 3: launch_dn_tc<T, 3>(a, lds, st); break;
        default: launch_dn_tc<T, 4>(a, lds, st); break;
    }
}

static void launch_gu(const MoeGuArgs& a, int T, hipStream_t st) {
    switch (T) {
        case 1: launch_gu_t<1>(a, st); break;
        case 2: launch_gu_t<2>(a, st); break;
        case 3: launch_gu_t<3>(a, st); break;
        case 4: launch_gu_t<4>(a, st); break;
        case 5: launch_gu_t<5>(a, st); break;
        case 6: launch_gu_t<6>(a, st); break;
        case 7: launch_gu_t<7>(a, st); break;
        default: launch_gu_t<8>(a, st); break;
    }
}
static void launch_dn(const MoeDnArgs& a, int T, hipStream_t st) {
    switch (T) {
        case 1: launch_dn_t<1>(a, st); break;
        case 2: launch_dn_t<2>(a, st); break;
        case 3: launch_dn_t<3>(a, st); break;
        case 4: launch_dn_t<4>(a, st); break;
        case 5: launch_dn_t<5>(a, st); break;
        case 6: launch_dn_t<6>(a, st); break;
        case 7: launch_dn_t<7>(a, st); break;
        default: launch_dn_t<8>(a, st); break;
    }
}

int moe_launch_experts(const wzy_moe_weights* w, const MoeWs& ws, const float* x, int T, float* comb, hipStream_t st) {
    launch_gu(gu_args(w, ws, x, T), T, st);
    launch_dn(dn_args(w, ws, comb), T, st);
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

}  // namespace wzy

extern "C" size_t wzy_moe_workspace_bytes(int n_embd, int n_ff, int n_exp, int top_k, int T) {
    size_t need = 0;
    moe_ws_carve(nullptr, 0, n_embd, n_ff, n_exp, top_k, T, &need);
    return need + 256;
}

extern "C" int wzy_moe_block(const wzy_moe_weights* w, const float* x, int T, float* comb, int* ids, float* wts,
                             void* workspace, size_t workspace_bytes, void* stream) {
    WZY_TRY(moe_check(w, T));
    WZY_REQUIRE(x && comb && workspace, "wzy_moe_block: null pointer");
    size_t need = 0;
    MoeWs ws = moe_ws_carve(workspace, workspace_bytes, w->n_embd, w->n_ff, w->n_exp, w->top_k, T, &need);
    WZY_REQUIRE(need <= workspace_bytes, "wzy_moe_block: workspace too small (%zu < %zu)", workspace_bytes, need);
    hipStream_t st = as_stream(stream);
    WZY_TRY(moe_launch_route(w, ws, x, T, st));
    WZY_TRY(moe_launch_experts(w, ws, x, T, comb, st));
    const int n_ent = T * w->top_k;
    if (ids) WZY_HIP_TRY(hipMemcpyAsync(ids, ws.ids, n_ent * sizeof(int), hipMemcpyDeviceToDevice, st));
    if (wts) WZY_HIP_TRY(hipMemcpyAsync(wts, ws.wts, n_ent * sizeof(float), hipMemcpyDeviceToDevice, st));
    return WZY_OK;
}

extern "C" int wzy_moe_time_kernels(const wzy_moe_weights* layers, int n_layers, int T, const float* x, void* workspace,
                                    size_t workspace_bytes, int iters, float* us_gate_up, float* us_down,
                                    float* us_block, void* stream) {
    WZY_REQUIRE(layers && n_layers >= 1 && iters >= 1 && us_gate_up && us_down && x, "wzy_moe_time_kernels: bad args");
    for (int l = 0; l < n_layers; ++l) WZY_TRY(moe_check(&layers[l], T));
    size_t need = 0;
    MoeWs ws = moe_ws_carve(workspace, workspace_bytes, layers[0].n_embd, layers[0].n_ff, layers[0].n_exp,
                            layers[0].top_k, T, &need);
    WZY_REQUIRE(need <= workspace_bytes, "wzy_moe_time_kernels: workspace too small");
    hipStream_t st = as_stream(stream);
    const int E = layers[0].n_exp;
    for (int l = 1; l < n_layers; ++l)
        WZY_REQUIRE(layers[l].n_embd == layers[0].n_embd && layers[l].n_ff == layers[0].n_ff &&
                        layers[l].n_exp == E && layers[l].top_k == layers[0].top_k,
                    "wzy_moe_time_kernels: layers must share one shape");
    // Every layer is routed first into a workspace of its own, so that the timed region holds nothing
    // but back-to-back launches of one kernel: `iters` gate/up launches cycling through the layers
    // (each with its own layer's routing), then `iters` down launches (each reading the activations
    // its layer's last gate/up wrote), then (us_block) `iters` blocks of one gate/up launch followed
    // by its layer's down launch, the order of a decode step.  Two events per burst: their own cost is
    // spread over `iters` launches.
    (void) ws;
    float* comb = nullptr;
    unsigned char* lws = nullptr;
    WZY_HIP_TRY(hipMalloc(&comb, sizeof(float) * (size_t) T * layers[0].n_embd));
    const size_t per = align_up(need, 256);
    if (hipMalloc(&lws, per * n_layers) != hipSuccess) {
        (void) hipFree(comb);
        set_error("wzy_moe_time_kernels: out of device memory");
        return WZY_ENOMEM;
    }
    auto layer_ws = [&](int l) {
        return moe_ws_carve(lws + per * l, per, layers[0].n_embd, layers[0].n_ff, E, layers[0].top_k, T, nullptr);
    };
    hipEvent_t ev[4] = {nullptr, nullptr, nullptr, nullptr};
    int rc = WZY_OK;
    for (auto& e : ev)
        if (rc == WZY_OK && hipEventCreate(&e) != hipSuccess) rc = WZY_EHIP;
    for (int l = 0; l < n_layers && rc == WZY_OK; ++l) rc = moe_launch_route(&layers[l], layer_ws(l), x, T, st);
    if (rc == WZY_OK) {
        launch_gu(gu_args(&layers[0], layer_ws(0), x, T), T, st);         // warm-up of both kernels
        launch_dn(dn_args(&layers[0], layer_ws(0), comb), T, st);
        (void) hipEventRecord(ev[0], st);
        for (int it = 0; it < iters; ++it) {
            const int l = it % n_layers;
            launch_gu(gu_args(&layers[l], layer_ws(l), x, T), T, st);
        }
        (void) hipEventRecord(ev[1], st);
        for (int it = 0; it < iters; ++it) {
            const int l = it % n_layers;
            launch_dn(dn_args(&layers[l], layer_ws(l), comb), T, st);
        }
        (void) hipEventRecord(ev[2], st);
        if (us_block) {
            for (int it = 0; it < iters; ++it) {
                const int l = it % n_layers;
                launch_gu(gu_args(&layers[l], layer_ws(l), x, T), T, st);
                launch_dn(dn_args(&layers[l], layer_ws(l), comb), T, st);
            }
        }
        (void) hipEventRecord(ev[3], st);
        if (hipGetLastError() != hipSuccess || hipEventSynchronize(ev[3]) != hipSuccess) {
            set_error("wzy_moe_time_kernels: launch failed");
            rc = WZY_EHIP;
        }
    }
    float a = 0.f, b = 0.f, c = 0.f;
    if (rc == WZY_OK) {
        (void) hipEventElapsedTime(&a, ev[0], ev[1]);
        (void) hipEventElapsedTime(&b, ev[1], ev[2]);
        (void) hipEventElapsedTime(&c, ev[2], ev[3]);
    }
    for (auto& e : ev)
        if (e) (void) hipEventDestroy(e);
    (void) hipFree(lws);
    (void) hipFree(comb);
    if (rc != WZY_OK) return rc;
    *us_gate_up = 1000.0f * a / (float) iters;
    *us_down = 1000.0f * b / (float) iters;
    if (us_block) *us_block = 1000.0f * c / (float) iters;
    return WZY_OK;
}

template <int T>
static void launch_route_t(const float* logits, int E, int K, int* ids, float* wts, hipStream_t st) {
    if (E <= 512) hipLaunchKernelGGL((moe_route_kernel<T, 8>), dim3(1), dim3(256), 0, st, logits, E, K, ids, wts);
    else hipLaunchKernelGGL((moe_route_kernel<T, 16>), dim3(1), dim3(256), 0, st, logits, E, K, ids, wts);
}

extern "C" int wzy_moe_route(const float* logits, int n_exp, int top_k, int T, int* ids, float* wts, void* stream) {
    WZY_REQUIRE(logits && ids && wts, "wzy_moe_route: null pointer");
    WZY_REQUIRE(n_exp >= 1 && n_exp <= 1024, "wzy_moe_route: n_exp must be in [1, 1024]");
    WZY_REQUIRE(top_k >= 1 && top_k <= MOE_MAX_K && top_k <= n_exp, "wzy_moe_route: top_k must be in [1, %d]",
                MOE_MAX_K);
    WZY_REQUIRE(T >= 1 && T <= WZY_MAX_W, "wzy_moe_route: T must be in [1, %d]", WZY_MAX_W);
    hipStream_t st = as_stream(stream);
    switch (T) {
        case 1: launch_route_t<1>(logits, n_exp, top_k, ids, wts, st); break;
        case 2: launch_route_t<2>(logits, n_exp, top_k, ids, wts, st); break;
        case 3: launch_route_t<3>(logits, n_exp, top_k, ids, wts, st); break;
        case 4: launch_route_t<4>(logits, n_exp, top_k, ids, wts, st); break;
        case 5: launch_route_t<5>(logits, n_exp, top_k, ids, wts, st); break;
        case 6: launch_route_t<6>(logits, n_exp, top_k, ids, wts, st); break;
        case 7: launch_route_t<7>(logits, n_exp, top_k, ids, wts, st); break;
        default: launch_route_t<8>(logits, n_exp, top_k, ids, wts, st); break;
    }
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

// moe.hip -- NVFP4 mixture-of-experts decode block for gfx950.
//
// Launch sequence of wzy_moe_block (T window rows, K routed experts per row):
//   1. quant_act           x -> int8 per-16 (routed) and per-32 (shared expert) activations
//   2. gemv_bf16           router logits [T x E] + shared-expert gate scalar (extra row)
//   3. moe_topk_group      softmax top-K per row, renormalised weights, and the expert groups:
//                          every distinct expert of the window becomes one group listing its
//                          (row, slot) members, so its weights are streamed from HBM once
//   4. moe_gate_up         per (group, 16-row tile): gate+up NVFP4 GEMV, SwiGLU, per-16 int8
//                          requant of the activation; extra workgroups run the Q8_0 shared
//                          expert gate/up + SwiGLU + per-32 requant
//   5. moe_down            per (group, 16-row tile): NVFP4 down GEMV into parts; one extra
//                          workgroup row runs the Q8_0 shared down projection; the last
//                          workgroup to finish a tile combines
//                          comb = sigmoid(sgate)*shared + sum_k w_k*part_k  (k in routed order).
// All GEMVs are wave-per-row with 128-bit code loads (16 bytes = 32 e2m1 values per lane) and
// e4m3 scales from a separate plane, e2m1 -> int8 expansion with v_perm_b32, v_dot4_i32_i8 dots.
// No MFMA: at one token per expert these are bandwidth-bound GEMVs.
#include "wzy_device.h"
#include "wzy_gemv.h"
#include "wzy_host.h"
#include "wzy_moe.h"

using namespace wzy;

namespace {

constexpr int TILE_D = 16;   // output rows of one down workgroup (4 waves x 4 rows x 16 lanes)

struct MoeOffsets {
    size_t gu_codes, gu_scales, dn_codes, dn_scales, tail, rec;
};
WZY_DEV MoeOffsets moe_offsets(int D, int F) {
    MoeOffsets o;
    o.gu_codes = 0;
    o.gu_scales = (size_t) 2 * F * (D / 2);
    o.dn_codes = o.gu_scales + (size_t) 2 * F * (D / 16);
    o.dn_scales = o.dn_codes + (size_t) D * (F / 2);
    o.tail = o.dn_scales + (size_t) D * (F / 16);
    o.rec = o.tail + 16;
    return o;
}

// Dot of one 32-value NVFP4 chunk (16 code bytes, 2 e4m3 scales) with 32 int8 activations
// (two per-16 scales), accumulated the way the reference does per 16-block:
// acc = fma(ws * xs, isum, acc)   (src/wzy_kernels_v2.cuh:1646-1647).
WZY_DEV float nvfp4_chunk_fma(const int4 wa, const int4 wb, float wsa, float wsb, int4 xa, int4 xb, float xsa,
                              float xsb, float acc) {
    acc = fmaf(wsa * xsa, (float) dot16(wa, xa), acc);
    acc = fmaf(wsb * xsb, (float) dot16(wb, xb), acc);
    return acc;
}

}  // namespace

// ---------------------------------------------------------------------------------------------
// 3. softmax top-K + grouping.  reference: router_top10_fast_multi (src/wzy_kernels_v2.cuh:989-1090)
//    and the grouping of split_route_hit_cold_kernel / group_experts_kernel
//    (src/wzy_cpu_moe.cuh:74-127, src/wzy_kernels_v2.cuh:1390-1423).  Groups are emitted in
//    ascending expert id (deterministic); the reference's atomicAdd order does not affect its
//    results because the combine sums in routed-slot order.
// ---------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(512) moe_topk_group_kernel(const float* __restrict__ logits, int E, int K, int T,
                                                             int* __restrict__ ids, float* __restrict__ wts,
                                                             int* __restrict__ n_groups, int* __restrict__ grp_exp,
                                                             int* __restrict__ grp_cnt, int* __restrict__ grp_mem,
                                                             unsigned* __restrict__ tile_cnt, int n_tiles) {
    constexpr int MAXV = 16;   // E <= 1024
    __shared__ int s_ids[WZY_MAX_W * MOE_MAX_K];
    __shared__ float s_w[WZY_MAX_W * MOE_MAX_K];
    __shared__ int s_wtot[8];
    __shared__ int s_carry;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;

    // the down kernel's per-tile arrival counters start every launch at zero
    for (int i = tid; i < n_tiles; i += blockDim.x) tile_cnt[i] = 0u;

    if (wv < T) {
        const int t = wv;
        const float* x = logits + (size_t) t * E;
        float p[MAXV];
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < MAXV; ++i) {
            const int idx = lane + 64 * i;
            p[i] = idx < E ? x[idx] : -INFINITY;
            mx = fmaxf(mx, p[i]);
        }
        mx = wave_max(mx);
        float es = 0.f;
#pragma unroll
        for (int i = 0; i < MAXV; ++i) {
            const int idx = lane + 64 * i;
            if (idx < E) { p[i] = __expf(p[i] - mx); es += p[i]; }
            else p[i] = -3.f;
        }
        es = wave_sum(es);
        const float inv = 1.0f / es;
#pragma unroll
        for (int i = 0; i < MAXV; ++i)
            if (lane + 64 * i < E) p[i] *= inv;
        float wsum = 0.f;
        for (int k = 0; k < K; ++k) {
            float bv = -4.f;
            int bi = 0x7fffffff;
#pragma unroll
            for (int i = 0; i < MAXV; ++i)
                if (p[i] > bv) { bv = p[i]; bi = lane + 64 * i; }
            wave_argmax(bv, bi);
#pragma unroll
            for (int i = 0; i < MAXV; ++i)
                if (lane + 64 * i == bi) p[i] = -2.f;
            if (lane == 0) { s_ids[t * K + k] = bi; s_w[t * K + k] = bv; }
            wsum += bv;
        }
        const float sc = fmaxf(wsum, 6.103515625e-05f);
        if (lane < K) {
            ids[t * K + lane] = s_ids[t * K + lane];
            wts[t * K + lane] = s_w[t * K + lane] / sc;
        }
    }
    __syncthreads();

    // grouping: thread e collects the (row, slot) entries routed to expert e, in entry order
    const int n_ent = T * K;
    if (tid == 0) s_carry = 0;
    __syncthreads();
    for (int e0 = 0; e0 < E; e0 += blockDim.x) {
        const int e = e0 + tid;
        int mem[WZY_MAX_W];
        int cnt = 0;
        if (e < E) {
            for (int f = 0; f < n_ent; ++f)
                if (s_ids[f] == e && cnt < WZY_MAX_W) mem[cnt++] = f;
        }
        const bool flag = cnt > 0;
        const unsigned long long bal = __ballot(flag);
        const int in_wave = __popcll(bal & ((1ull << lane) - 1ull));
        if (lane == 0) s_wtot[wv] = __popcll(bal);
        __syncthreads();
        int before = s_carry;
        for (int w = 0; w < wv; ++w) before += s_wtot[w];
        if (flag) {
            const int g = before + in_wave;
            grp_exp[g] = e;
            grp_cnt[g] = cnt;
            for (int j = 0; j < cnt; ++j) grp_mem[g * WZY_MAX_W + j] = mem[j];
        }
        __syncthreads();
        if (tid == 0) {
            int tot = 0;
            for (int w = 0; w < (int) (blockDim.x >> 6); ++w) tot += s_wtot[w];
            s_carry += tot;
        }
        __syncthreads();
    }
    if (tid == 0) *n_groups = s_carry;
}

// ---------------------------------------------------------------------------------------------
// 4. gate/up.  Routed workgroups: one (group, 16-row tile); wave w owns rows j = 16*tile + 4w .. +3
//    of both gate and up, so SwiGLU and the 16-wide requant stay inside the workgroup.
//    reference: exp_gu_quant_grouped (src/wzy_kernels_v2.cuh:1583-1721).
//    Shared workgroups: 32 rows of the Q8_0 shared gate/up, SwiGLU, per-32 requant.
//    reference: launch_gemm_q8p x2 + silu_mul_quant32_multi (src/wzy_stage_v2.cuh:711-713;
//    src/wzy_kernels_v2.cuh:1247-1280).
// ---------------------------------------------------------------------------------------------
template <int T>
__global__ void __launch_bounds__(256) moe_gate_up_kernel(
    const uint8_t* __restrict__ experts, int D, int F, int K, const int* __restrict__ n_groups,
    const int* __restrict__ grp_exp, const int* __restrict__ grp_cnt, const int* __restrict__ grp_mem,
    const int8_t* __restrict__ xq16, const float* __restrict__ xs16, int8_t* __restrict__ aq16,
    float* __restrict__ as16, const int8_t* __restrict__ shg_q, const uint16_t* __restrict__ shg_s,
    const int8_t* __restrict__ shu_q, const uint16_t* __restrict__ shu_s, const int8_t* __restrict__ xq32,
    const float* __restrict__ xs32, int8_t* __restrict__ shq32, float* __restrict__ shs32, int n_routed_wg) {
    __shared__ int s_mem[WZY_MAX_W];
    __shared__ int s_tok[WZY_MAX_W];
    __shared__ float s_act[WZY_MAX_W][32];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int bid = blockIdx.x;

    if (bid < n_routed_wg) {
        const int tiles = F / 16;
        const int g = bid / tiles, jt = bid - g * tiles;
        if (g >= *n_groups) return;
        const int e = grp_exp[g], cnt = grp_cnt[g];
        if (tid < cnt) {
            const int f = grp_mem[g * WZY_MAX_W + tid];
            s_mem[tid] = f;
            s_tok[tid] = f / K;
        }
        __syncthreads();
        const MoeOffsets o = moe_offsets(D, F);
        const uint8_t* rec = experts + (size_t) e * o.rec;
        const float sc_gate = ((const float*) (rec + o.tail))[0];
        const float sc_up = ((const float*) (rec + o.tail))[1];
        const int j0 = jt * 16 + 4 * w;
        float acc[8][T];
#pragma unroll
        for (int r = 0; r < 8; ++r)
#pragma unroll
            for (int m = 0; m < T; ++m) acc[r][m] = 0.f;

        const int nchunk = D / 32;
        for (int c = lane; c < nchunk; c += 64) {
            int4 code[8];
            uint32_t sc2[8];
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                const int row = (r < 4) ? (j0 + r) : (F + j0 + r - 4);
                code[r] = ld_stream_i4(rec + o.gu_codes + (size_t) row * (D / 2) + (size_t) c * 16);
                sc2[r] = *(const uint16_t*) (rec + o.gu_scales + (size_t) row * (D / 16) + 2 * c);
            }
            int4 xa[T], xb[T];
            float xsa[T], xsb[T];
#pragma unroll
            for (int m = 0; m < T; ++m) {
                if (m < cnt) {
                    const int t = s_tok[m];
                    const int4* xp = (const int4*) (xq16 + (size_t) t * D + (size_t) c * 32);
                    xa[m] = xp[0];
                    xb[m] = xp[1];
                    const float2 s = *(const float2*) (xs16 + (size_t) t * (D / 16) + 2 * c);
                    xsa[m] = s.x;
                    xsb[m] = s.y;
                }
            }
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                const int4 wa = e2m1_sub16((uint32_t) code[r].x, (uint32_t) code[r].y);
                const int4 wb = e2m1_sub16((uint32_t) code[r].z, (uint32_t) code[r].w);
                const float wsa = ue4m3_half(sc2[r] & 0xFFu), wsb = ue4m3_half(sc2[r] >> 8);
#pragma unroll
                for (int m = 0; m < T; ++m)
                    if (m < cnt) acc[r][m] = nvfp4_chunk_fma(wa, wb, wsa, wsb, xa[m], xb[m], xsa[m], xsb[m], acc[r][m]);
            }
        }
#pragma unroll
        for (int m = 0; m < T; ++m) {
            if (m < cnt) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float gv = wave_sum(acc[q][m]) * sc_gate;
                    const float uv = wave_sum(acc[4 + q][m]) * sc_up;
                    if (lane == 0) s_act[m][4 * w + q] = siluf_(gv) * uv;
                }
            }
        }
        __syncthreads();
        if (tid < cnt * 16) {
            const int m = tid >> 4, jj = tid & 15;
            const float v = s_act[m][jj];
            const float amax = max16(fabsf(v));
            const float d = amax / 127.0f;
            const float inv = d > 0.f ? 127.0f / amax : 0.f;
            const int q = max(-127, min(127, rn_int(v * inv)));
            const int f = s_mem[m];
            aq16[(size_t) f * F + jt * 16 + jj] = (int8_t) q;
            if (jj == 0) as16[(size_t) f * (F / 16) + jt] = d;
        }
        return;
    }

    // shared expert: rows j in [32*sb, 32*sb + 32), wave w owns j = 32*sb + 8w .. +7 (two halves of 4)
    const int sb = bid - n_routed_wg;
    const int nb = D / 32;
#pragma unroll 1
    for (int half = 0; half < 2; ++half) {
        const int j0 = 32 * sb + 8 * w + 4 * half;
        float acc[8][T];
#pragma unroll
        for (int r = 0; r < 8; ++r)
#pragma unroll
            for (int t = 0; t < T; ++t) acc[r][t] = 0.f;
        for (int b = lane; b < nb; b += 64) {
            int4 c0[8], c1[8];
            float dw[8];
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                const int8_t* q = (r < 4) ? shg_q : shu_q;
                const uint16_t* s = (r < 4) ? shg_s : shu_s;
                const int row = j0 + (r & 3);
                const int4* cp = (const int4*) (q + (size_t) row * D + (size_t) b * 32);
                c0[r] = ld_stream_i4(cp);
                c1[r] = ld_stream_i4(cp + 1);
                dw[r] = h16_to_f(s[(size_t) row * nb + b]);
            }
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const int4* xp = (const int4*) (xq32 + (size_t) t * D + (size_t) b * 32);
                const int4 x0 = xp[0], x1 = xp[1];
                const float xsc = xs32[(size_t) t * nb + b];
#pragma unroll
                for (int r = 0; r < 8; ++r)
                    acc[r][t] = fmaf(dw[r] * xsc, (float) (dot16(c0[r], x0) + dot16(c1[r], x1)), acc[r][t]);
            }
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float gv = wave_sum(acc[q][t]);
                const float uv = wave_sum(acc[4 + q][t]);
                if (lane == 0) s_act[t][8 * w + 4 * half + q] = siluf_(gv) * uv;
            }
        }
    }
    __syncthreads();
    if (tid < T * 32) {
        const int t = tid >> 5, jj = tid & 31;
        const float v = s_act[t][jj];
        const float amax = max32(fabsf(v));
        const float d = amax / 127.0f;
        const float inv = d > 0.f ? 127.0f / amax : 0.f;
        const int q = max(-127, min(127, rn_int(v * inv)));
        shq32[(size_t) t * F + 32 * sb + jj] = (int8_t) q;
        if (jj == 0) shs32[(size_t) t * (F / 32) + sb] = d;
    }
}

// ---------------------------------------------------------------------------------------------
// 5. down + combine.  Workgroup (tile, y): y < Gmax is routed group y (exits if y >= n_groups),
//    y == Gmax is the shared expert.  16 lanes per output row, 4 rows per wave.
//    reference: exp_down_2r_grouped (src/wzy_kernels_v2.cuh:1725-1834), shared down launch_gemm_q8p
//    (src/wzy_stage_v2.cuh:714), moe_combine_shared_multi (src/wzy_kernels_v2.cuh:1281-1294).
// ---------------------------------------------------------------------------------------------
template <int T>
__global__ void __launch_bounds__(256) moe_down_kernel(
    const uint8_t* __restrict__ experts, int D, int F, int K, const int* __restrict__ n_groups,
    const int* __restrict__ grp_exp, const int* __restrict__ grp_cnt, const int* __restrict__ grp_mem,
    const int8_t* __restrict__ aq16, const float* __restrict__ as16, const int8_t* __restrict__ shd_q,
    const uint16_t* __restrict__ shd_s, const int8_t* __restrict__ shq32, const float* __restrict__ shs32,
    const float* __restrict__ wts, const float* __restrict__ sg, float* __restrict__ parts,
    float* __restrict__ shared_out, unsigned* __restrict__ tile_cnt, float* __restrict__ comb, int Gmax) {
    __shared__ int s_mem[WZY_MAX_W];
    __shared__ int s_last;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int tile = blockIdx.x, gy = blockIdx.y;
    const int ng = *n_groups;
    const bool is_shared = (gy == Gmax);
    if (!is_shared && gy >= ng) return;
    const int d = tile * TILE_D + 4 * w + (lane >> 4);
    const int li = lane & 15;

    if (!is_shared) {
        const int e = grp_exp[gy], cnt = grp_cnt[gy];
        if (tid < cnt) s_mem[tid] = grp_mem[gy * WZY_MAX_W + tid];
        __syncthreads();
        const MoeOffsets o = moe_offsets(D, F);
        const uint8_t* rec = experts + (size_t) e * o.rec;
        const float sc_down = ((const float*) (rec + o.tail))[2];
        float acc[T];
#pragma unroll
        for (int m = 0; m < T; ++m) acc[m] = 0.f;
        for (int c = li; c < F / 32; c += 16) {
            const int4 code = ld_stream_i4(rec + o.dn_codes + (size_t) d * (F / 2) + (size_t) c * 16);
            const uint32_t s2 = *(const uint16_t*) (rec + o.dn_scales + (size_t) d * (F / 16) + 2 * c);
            const int4 wa = e2m1_sub16((uint32_t) code.x, (uint32_t) code.y);
            const int4 wb = e2m1_sub16((uint32_t) code.z, (uint32_t) code.w);
            const float wsa = ue4m3_half(s2 & 0xFFu), wsb = ue4m3_half(s2 >> 8);
#pragma unroll
            for (int m = 0; m < T; ++m) {
                if (m < cnt) {
                    const int f = s_mem[m];
                    const int4* xp = (const int4*) (aq16 + (size_t) f * F + (size_t) c * 32);
                    const float2 xs = *(const float2*) (as16 + (size_t) f * (F / 16) + 2 * c);
                    acc[m] = nvfp4_chunk_fma(wa, wb, wsa, wsb, xp[0], xp[1], xs.x, xs.y, acc[m]);
                }
            }
        }
#pragma unroll
        for (int m = 0; m < T; ++m) {
            if (m < cnt) {
                const float v = sum16(acc[m]) * sc_down;
                if (li == 0) parts[(size_t) s_mem[m] * D + d] = v;
            }
        }
    } else {
        const int nb = F / 32;
        float acc[T];
#pragma unroll
        for (int t = 0; t < T; ++t) acc[t] = 0.f;
        for (int b = li; b < nb; b += 16) {
            const int4* cp = (const int4*) (shd_q + (size_t) d * F + (size_t) b * 32);
            const int4 c0 = ld_stream_i4(cp), c1 = ld_stream_i4(cp + 1);
            const float dw = h16_to_f(shd_s[(size_t) d * nb + b]);
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const int4* xp = (const int4*) (shq32 + (size_t) t * F + (size_t) b * 32);
                const float xsc = shs32[(size_t) t * nb + b];
                acc[t] = fmaf(dw * xsc, (float) (dot16(c0, xp[0]) + dot16(c1, xp[1])), acc[t]);
            }
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const float v = sum16(acc[t]);
            if (li == 0) shared_out[(size_t) t * D + d] = v;
        }
    }

    // arrival: the (ng + 1)-th workgroup of this tile combines
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const unsigned prev = atomicAdd(&tile_cnt[tile], 1u);
        s_last = (prev == (unsigned) ng);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    for (int i = tid; i < T * TILE_D; i += blockDim.x) {
        const int t = i / TILE_D, dd = tile * TILE_D + (i % TILE_D);
        float s = shared_out[(size_t) t * D + dd] * sigmoidf_(sg[t]);
        for (int k = 0; k < K; ++k) {
            const float wk = wts[t * K + k];
            if (wk != 0.0f) s += wk * parts[(size_t) (t * K + k) * D + dd];
        }
        comb[(size_t) t * D + dd] = s;
    }
    if (tid == 0) tile_cnt[tile] = 0u;
}

// ---------------------------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------------------------
namespace wzy {

MoeWs moe_ws_carve(void* base, size_t cap, int D, int F, int E, int K, int T, size_t* need) {
    Arena a(base, cap);
    MoeWs w;
    const int n_ent = T * K;
    w.xq16 = a.take<int8_t>((size_t) T * D);
    w.xs16 = a.take<float>((size_t) T * D / 16);
    w.xq32 = a.take<int8_t>((size_t) T * D);
    w.xs32 = a.take<float>((size_t) T * D / 32);
    w.logits = a.take<float>((size_t) T * E);
    w.sg = a.take<float>(T);
    w.ids = a.take<int>(n_ent);
    w.wts = a.take<float>(n_ent);
    w.n_groups = a.take<int>(1);
    w.grp_exp = a.take<int>(n_ent);
    w.grp_cnt = a.take<int>(n_ent);
    w.grp_mem = a.take<int>((size_t) n_ent * WZY_MAX_W);
    w.aq16 = a.take<int8_t>((size_t) n_ent * F);
    w.as16 = a.take<float>((size_t) n_ent * F / 16);
    w.shq32 = a.take<int8_t>((size_t) T * F);
    w.shs32 = a.take<float>((size_t) T * F / 32);
    w.parts = a.take<float>((size_t) n_ent * D);
    w.shared_out = a.take<float>((size_t) T * D);
    w.tile_cnt = a.take<unsigned>(D / TILE_D);
    if (need) *need = a.off;
    return w;
}

int moe_check(const wzy_moe_weights* w, int T) {
    WZY_REQUIRE(w != nullptr, "moe: null weights");
    WZY_REQUIRE(T >= 1 && T <= WZY_MAX_W, "moe: T must be in [1, %d]", WZY_MAX_W);
    WZY_REQUIRE(w->n_embd % 256 == 0 && w->n_embd >= 256, "moe: n_embd must be a multiple of 256");
    WZY_REQUIRE(w->n_ff % 64 == 0 && w->n_ff >= 64, "moe: n_ff must be a multiple of 64");
    WZY_REQUIRE(w->n_exp >= 1 && w->n_exp <= 1024, "moe: n_exp must be in [1, 1024]");
    WZY_REQUIRE(w->top_k >= 1 && w->top_k <= MOE_MAX_K && w->top_k <= w->n_exp, "moe: top_k must be in [1, %d]",
                MOE_MAX_K);
    WZY_REQUIRE(w->router && w->sgate && w->experts && w->sh_gate_q && w->sh_gate_s && w->sh_up_q && w->sh_up_s &&
                    w->sh_down_q && w->sh_down_s,
                "moe: null weight pointer");
    return WZY_OK;
}

template <int T>
static void launch_gu_down(const wzy_moe_weights* w, const MoeWs& ws, float* comb, hipStream_t st) {
    const int D = w->n_embd, F = w->n_ff, K = w->top_k;
    const int Gmax = T * K;
    const int n_routed_wg = (F / 16) * Gmax;
    hipLaunchKernelGGL((moe_gate_up_kernel<T>), dim3(n_routed_wg + F / 32), dim3(256), 0, st, w->experts, D, F, K,
                       ws.n_groups, ws.grp_exp, ws.grp_cnt, ws.grp_mem, ws.xq16, ws.xs16, ws.aq16, ws.as16,
                       w->sh_gate_q, w->sh_gate_s, w->sh_up_q, w->sh_up_s, ws.xq32, ws.xs32, ws.shq32, ws.shs32,
                       n_routed_wg);
    hipLaunchKernelGGL((moe_down_kernel<T>), dim3(D / TILE_D, Gmax + 1), dim3(256), 0, st, w->experts, D, F, K,
                       ws.n_groups, ws.grp_exp, ws.grp_cnt, ws.grp_mem, ws.aq16, ws.as16, w->sh_down_q, w->sh_down_s,
                       ws.shq32, ws.shs32, ws.wts, ws.sg, ws.parts, ws.shared_out, ws.tile_cnt, comb, Gmax);
}

int moe_launch_experts(const wzy_moe_weights* w, const MoeWs& ws, int T, float* comb, hipStream_t st) {
    switch (T) {
        case 1: launch_gu_down<1>(w, ws, comb, st); break;
        case 2: launch_gu_down<2>(w, ws, comb, st); break;
        case 3: launch_gu_down<3>(w, ws, comb, st); break;
        case 4: launch_gu_down<4>(w, ws, comb, st); break;
        case 5: launch_gu_down<5>(w, ws, comb, st); break;
        case 6: launch_gu_down<6>(w, ws, comb, st); break;
        case 7: launch_gu_down<7>(w, ws, comb, st); break;
        default: launch_gu_down<8>(w, ws, comb, st); break;
    }
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

int moe_launch_route(const wzy_moe_weights* w, const MoeWs& ws, int T, hipStream_t st) {
    const int D = w->n_embd, E = w->n_exp, K = w->top_k;
    WZY_REQUIRE(ws.xf != nullptr, "moe_launch_route: activations not set");
    WZY_TRY(launch_gemv_bf16(w->router, ws.xf, ws.logits, E, D, T, 0, w->sgate, ws.sg, st));
    hipLaunchKernelGGL(moe_topk_group_kernel, dim3(1), dim3(512), 0, st, ws.logits, E, K, T, ws.ids, ws.wts,
                       ws.n_groups, ws.grp_exp, ws.grp_cnt, ws.grp_mem, ws.tile_cnt, D / TILE_D);
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
    ws.xf = x;
    hipStream_t st = as_stream(stream);
    WZY_TRY(launch_quant_act(x, ws.xq32, ws.xs32, ws.xq16, ws.xs16, w->n_embd, T, st));
    WZY_TRY(moe_launch_route(w, ws, T, st));
    WZY_TRY(moe_launch_experts(w, ws, T, comb, st));
    const int n_ent = T * w->top_k;
    if (ids) WZY_HIP_TRY(hipMemcpyAsync(ids, ws.ids, n_ent * sizeof(int), hipMemcpyDeviceToDevice, st));
    if (wts) WZY_HIP_TRY(hipMemcpyAsync(wts, ws.wts, n_ent * sizeof(float), hipMemcpyDeviceToDevice, st));
    return WZY_OK;
}

extern "C" int wzy_moe_time_kernels(const wzy_moe_weights* layers, int n_layers, int T, void* workspace,
                                    size_t workspace_bytes, int iters, float* us_gate_up, float* us_down,
                                    void* stream) {
    WZY_REQUIRE(layers && n_layers >= 1 && iters >= 1 && us_gate_up && us_down, "wzy_moe_time_kernels: bad args");
    for (int l = 0; l < n_layers; ++l) WZY_TRY(moe_check(&layers[l], T));
    size_t need = 0;
    MoeWs ws = moe_ws_carve(workspace, workspace_bytes, layers[0].n_embd, layers[0].n_ff, layers[0].n_exp,
                            layers[0].top_k, T, &need);
    WZY_REQUIRE(need <= workspace_bytes, "wzy_moe_time_kernels: workspace too small");
    hipStream_t st = as_stream(stream);
    hipEvent_t ev[3];
    for (auto& e : ev) WZY_HIP_TRY(hipEventCreate(&e));
    float tot_gu = 0.f, tot_dn = 0.f;
    int rc = WZY_OK;
    float* comb = ws.shared_out;   // results are discarded; any T x D buffer works
    for (int it = 0; it < iters && rc == WZY_OK; ++it) {
        const wzy_moe_weights* w = &layers[it % n_layers];
        const int D = w->n_embd, F = w->n_ff, K = w->top_k, Gmax = T * K;
        const int n_routed_wg = (F / 16) * Gmax;
        (void) hipEventRecord(ev[0], st);
        switch (T) {
#define WZY_T_CASE(TT)                                                                                               \
    case TT:                                                                                                         \
        hipLaunchKernelGGL((moe_gate_up_kernel<TT>), dim3(n_routed_wg + F / 32), dim3(256), 0, st, w->experts, D, F, \
                           K, ws.n_groups, ws.grp_exp, ws.grp_cnt, ws.grp_mem, ws.xq16, ws.xs16, ws.aq16, ws.as16,   \
                           w->sh_gate_q, w->sh_gate_s, w->sh_up_q, w->sh_up_s, ws.xq32, ws.xs32, ws.shq32, ws.shs32, \
                           n_routed_wg);                                                                             \
        (void) hipEventRecord(ev[1], st);                                                                            \
        hipLaunchKernelGGL((moe_down_kernel<TT>), dim3(D / TILE_D, Gmax + 1), dim3(256), 0, st, w->experts, D, F, K, \
                           ws.n_groups, ws.grp_exp, ws.grp_cnt, ws.grp_mem, ws.aq16, ws.as16, w->sh_down_q,          \
                           w->sh_down_s, ws.shq32, ws.shs32, ws.wts, ws.sg, ws.parts, ws.shared_out, ws.tile_cnt,    \
                           comb, Gmax);                                                                              \
        break;
            WZY_T_CASE(1)
            WZY_T_CASE(2)
            WZY_T_CASE(3)
            WZY_T_CASE(4)
            WZY_T_CASE(5)
            WZY_T_CASE(6)
            WZY_T_CASE(7)
            default:
            WZY_T_CASE(8)
#undef WZY_T_CASE
        }
        (void) hipEventRecord(ev[2], st);
        if (hipGetLastError() != hipSuccess || hipEventSynchronize(ev[2]) != hipSuccess) {
            set_error("wzy_moe_time_kernels: launch failed");
            rc = WZY_EHIP;
            break;
        }
        float a = 0.f, b = 0.f;
        (void) hipEventElapsedTime(&a, ev[0], ev[1]);
        (void) hipEventElapsedTime(&b, ev[1], ev[2]);
        tot_gu += a;
        tot_dn += b;
    }
    for (auto& e : ev) (void) hipEventDestroy(e);
    if (rc != WZY_OK) return rc;
    *us_gate_up = 1000.f * tot_gu / (float) iters;
    *us_down = 1000.f * tot_dn / (float) iters;
    return WZY_OK;
}

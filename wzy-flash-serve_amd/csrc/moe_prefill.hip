// moe_prefill.hip -- NVFP4 mixture-of-experts block for a prefill chunk of N tokens, on MFMA.
//
// Launch sequence of wzy_moe_prefill (N tokens, E experts, top-K):
//   1. pf_cvt      x fp32 -> bf16 (round to nearest even), the A operand of every GEMM
//   2. pf_gemm     router logits [N x E] = x . router^T                      (bf16 weights)
//   3. pf_route    per token, one wave: softmax top-K (the decode routing: probability desc, id asc,
//                  weights renormalised by max(sum, 2^-14)) and the shared-expert gate sg = sgate . x
//   4. pf_group    one workgroup: entries (token, slot) grouped by expert into 64-entry tiles
//   5. pf_gemm     shared expert gate|up (Q8_0 -> bf16) with SwiGLU epilogue -> sh_act bf16 [N x F]
//   6. pf_gemm     shared expert down (Q8_0 -> bf16) -> comb = sigmoid(sg) * shared   (initialises comb)
//   7. pf_gemm     routed gate|up per tile (NVFP4 -> bf16) with SwiGLU epilogue -> act bf16 [N*K x F]
//   8. pf_gemm     routed down per tile (NVFP4 -> bf16) -> comb += w_k * expert_k  (fp32 atomics)
// pf_gemm: workgroup tile 64 rows (tokens / entries) x 64 weight rows, K stepped by 64 through two
// LDS buffers; each of the 4 waves owns a 32 x 32 block accumulated by v_mfma_f32_32x32x16_bf16.
// Weights are dequantised to bf16 while staged: e2m1 codes through the fp4 -> bf16 conversion
// instruction times the e4m3 block scale and the tensor scale (exact: at most 8 significant bits),
// Q8_0 codes times their fp16 scale (rounded to bf16).  The next K step's global loads are issued
// before the current step's MFMAs.
// reference: pf_moe_gu_wmma_kernel, pf_moe_down_wmma_kernel, the tile builder and the shared/router
// prefill GEMMs (src/wzy_prefill_tc.cuh:99-443), with fp16 replaced by bf16.
#include "wzy_device.h"
#include "wzy_host.h"
#include "wzy_moe.h"
#include "wzy_route.h"

using namespace wzy;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

namespace {

constexpr int PB = 64;             // tile rows (M), weight rows (N) and K step
constexpr int PB_LD = PB + 8;      // LDS row stride in bf16 (16-byte aligned rows, staggered banks)
constexpr int PF_MAX_E = 1024;

enum { PW_BF16 = 0, PW_Q8 = 1, PW_FP4 = 2 };                        // weight formats
enum { PE_F32 = 0, PE_SWIGLU = 1, PE_ATOMIC = 2, PE_SHARED = 3 };   // epilogues

struct PfTile {
    int e, off, cnt, pad;          // expert, first entry, entries (<= 64)
};

struct PfGemmArgs {
    // A: bf16 activation rows of length K.  Dense: rows m0 .. m0+63 of [a_rows x K].  Expert tiles:
    // entry rows off .. off+cnt-1, either gathered from a through tok (entry -> token) or read from
    // a directly (a_by_entry).
    const uint16_t* a;
    int a_rows, K;
    const int* tok;
    bool a_by_entry;
    // B: weight rows of length K.  BF16 / Q8: w (+ ws fp16 scales per 32) and, for SwiGLU, w2/ws2
    // for the up rows.  FP4: expert records, codes/scales plane offsets, first row of the plane.
    const void* w; const uint16_t* ws;
    const void* w2; const uint16_t* ws2;
    const uint8_t* experts;
    size_t rec, codes_off, scales_off, tail_off;
    int tail_gate, tail_up;        // tensor scale index of the gate (or only) rows and of the up rows
    int up_row0;                   // FP4 SwiGLU: first up row of the plane (= F)
    int n_rows;                    // weight rows (dense F32 epilogue bound)
    // expert tiles (null: dense)
    const PfTile* tiles;
    const int* n_tiles;
    // outputs
    float* y; int y_ld;            // F32 / SHARED / ATOMIC: y[row * y_ld + n]
    uint16_t* act; int act_ld;     // SWIGLU: act[(row) * act_ld + j]
    const float* wt;               // ATOMIC: weight of each entry
    const float* sg;               // SHARED: gate scalar per token
};

WZY_DEV uint16_t f_to_bf16(float f) {                // round to nearest even (finite inputs)
    const uint32_t u = __builtin_bit_cast(uint32_t, f);
    return (uint16_t) ((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
WZY_DEV float bf16_bits_to_f(uint32_t h) { return __builtin_bit_cast(float, h << 16); }

// Weight chunk of one staging thread: 16 consecutive k of one weight row, as bf16.
template <int WK>
struct WRaw {
    uint4 u[2];                    // BF16: 2 x 8 bf16; Q8: u[0] = 16 int8; FP4: u[0].x/.y = 8 code bytes
    uint32_t s;                    // Q8: fp16 scale bits; FP4: e4m3 scale byte
};

template <int WK>
WZY_DEV WRaw<WK> load_w(const PfGemmArgs& a, const uint8_t* rec, int row, bool up, int k0) {
    WRaw<WK> r;
    if constexpr (WK == PW_FP4) {
        const uint8_t* cp = rec + a.codes_off + (size_t) row * (a.K / 2) + (size_t) (k0 / 16) * 8;
        const uint2 c = *(const uint2*) cp;
        r.u[0] = make_uint4(c.x, c.y, 0u, 0u);
        r.s = rec[a.scales_off + (size_t) row * (a.K / 16) + k0 / 16];
    } else if constexpr (WK == PW_Q8) {
        const int8_t* q = (const int8_t*) (up ? a.w2 : a.w);
        const uint16_t* sc = up ? a.ws2 : a.ws;
        r.u[0] = *(const uint4*) (q + (size_t) row * a.K + k0);
        r.s = sc[(size_t) row * (a.K / 32) + k0 / 32];
    } else {
        const uint16_t* w = (const uint16_t*) (up ? a.w2 : a.w);
        const uint4* p = (const uint4*) (w + (size_t) row * a.K + k0);
        r.u[0] = p[0];
        r.u[1] = p[1];
    }
    return r;
}

// dequantise to 16 bf16 (two uint4 in k order)
template <int WK>
WZY_DEV void dequant_w(const WRaw<WK>& r, float tscale, uint4 (&o)[2]) {
    if constexpr (WK == PW_FP4) {
        // byte j of the sub-block: value j in the low nibble, value j+8 in the high nibble
        const float sc = ue4m3_half(r.s) * 2.0f * tscale;
        uint16_t v[16];
        const uint32_t w0 = r.u[0].x, w1 = r.u[0].y;
        bf16x2_t p[8];
        p[0] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w0, 1.0f, 0);
        p[1] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w0, 1.0f, 1);
        p[2] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w0, 1.0f, 2);
        p[3] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w0, 1.0f, 3);
        p[4] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w1, 1.0f, 0);
        p[5] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w1, 1.0f, 1);
        p[6] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w1, 1.0f, 2);
        p[7] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w1, 1.0f, 3);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            v[j] = f_to_bf16((float) p[j].x * sc);
            v[j + 8] = f_to_bf16((float) p[j].y * sc);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h)
            o[h] = make_uint4(v[8 * h] | ((uint32_t) v[8 * h + 1] << 16), v[8 * h + 2] | ((uint32_t) v[8 * h + 3] << 16),
                              v[8 * h + 4] | ((uint32_t) v[8 * h + 5] << 16), v[8 * h + 6] | ((uint32_t) v[8 * h + 7] << 16));
    } else if constexpr (WK == PW_Q8) {
        const float sc = h16_to_f((uint16_t) r.s);
        const uint32_t q[4] = {r.u[0].x, r.u[0].y, r.u[0].z, r.u[0].w};
        uint16_t v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = f_to_bf16((float) (int8_t) (q[j >> 2] >> (8 * (j & 3))) * sc);
#pragma unroll
        for (int h = 0; h < 2; ++h)
            o[h] = make_uint4(v[8 * h] | ((uint32_t) v[8 * h + 1] << 16), v[8 * h + 2] | ((uint32_t) v[8 * h + 3] << 16),
                              v[8 * h + 4] | ((uint32_t) v[8 * h + 5] << 16), v[8 * h + 6] | ((uint32_t) v[8 * h + 7] << 16));
    } else {
        o[0] = r.u[0];
        o[1] = r.u[1];
    }
}

template <int WK, int EPI>
__global__ void __launch_bounds__(256) pf_gemm_kernel(PfGemmArgs a) {
    __shared__ __align__(16) uint16_t sA[2][PB][PB_LD];
    __shared__ __align__(16) uint16_t sB[2][PB][PB_LD];
    __shared__ int s_tok[PB];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int wm = w & 1, wn = w >> 1;

    // ---- tile ----
    int e = 0, row0 = 0, cnt = 0;
    if (a.tiles) {
        if ((int) blockIdx.y >= *a.n_tiles) return;               // workgroup-uniform
        const PfTile t = a.tiles[blockIdx.y];
        e = t.e; row0 = t.off; cnt = t.cnt;
    } else {
        row0 = blockIdx.y * PB;
        cnt = min(PB, a.a_rows - row0);
    }
    if (tid < PB) s_tok[tid] = (a.tiles && tid < cnt) ? a.tok[row0 + tid] : 0;
    const uint8_t* rec = a.experts ? a.experts + (size_t) e * a.rec : nullptr;
    // weight rows of this workgroup: SwiGLU = 32 gate rows j0.. and the matching 32 up rows
    const int n0 = EPI == PE_SWIGLU ? blockIdx.x * 32 : blockIdx.x * PB;
    const int sr = tid >> 2, sk = (tid & 3) * 16;                // staging: row sr, k sk .. sk+15
    const bool up = EPI == PE_SWIGLU && sr >= 32;
    const int wrow = EPI == PE_SWIGLU ? (up ? (WK == PW_FP4 ? a.up_row0 : 0) + n0 + sr - 32 : n0 + sr)
                                      : min(n0 + sr, a.n_rows - 1);
    float tsc = 1.0f;
    if constexpr (WK == PW_FP4) tsc = ((const float*) (rec + a.tail_off))[up ? a.tail_up : a.tail_gate];
    __syncthreads();
    // A row of this staging thread (zero beyond the tile)
    const bool a_ok = sr < cnt;
    const int arow = a.tiles ? (a.a_by_entry ? row0 + sr : s_tok[sr]) : row0 + sr;
    const uint16_t* ap = a.a + (size_t) (a_ok ? arow : 0) * a.K + sk;

    f32x16_t acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.f;
    const int nk = a.K / PB;

    auto load_a = [&](int ks, uint4 (&x)[2]) {
        const uint4* p = (const uint4*) (ap + (size_t) ks * PB);
        x[0] = a_ok ? p[0] : make_uint4(0, 0, 0, 0);
        x[1] = a_ok ? p[1] : make_uint4(0, 0, 0, 0);
    };
    auto store = [&](int buf, const uint4 (&x)[2], const WRaw<WK>& wr) {
        *(uint4*) &sA[buf][sr][sk] = x[0];
        *(uint4*) &sA[buf][sr][sk + 8] = x[1];
        uint4 o[2];
        dequant_w<WK>(wr, tsc, o);
        *(uint4*) &sB[buf][sr][sk] = o[0];
        *(uint4*) &sB[buf][sr][sk + 8] = o[1];
    };

    uint4 xa[2];
    load_a(0, xa);
    WRaw<WK> wr = load_w<WK>(a, rec, wrow, up, sk);
    store(0, xa, wr);
    __syncthreads();
    for (int ks = 0; ks < nk; ++ks) {
        const int buf = ks & 1;
        const bool more = ks + 1 < nk;
        if (more) {                                              // next step's loads first
            load_a(ks + 1, xa);
            wr = load_w<WK>(a, rec, wrow, up, (ks + 1) * PB + sk);
        }
#pragma unroll
        for (int kk = 0; kk < PB / 16; ++kk) {
            const bf16x8_t av = *(const bf16x8_t*) &sA[buf][wm * 32 + (lane & 31)][kk * 16 + (lane >> 5) * 8];
            const bf16x8_t bv = *(const bf16x8_t*) &sB[buf][wn * 32 + (lane & 31)][kk * 16 + (lane >> 5) * 8];
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, acc, 0, 0, 0);
        }
        if (more) store(buf ^ 1, xa, wr);
        __syncthreads();
    }

    // ---- epilogue: acc[i] = C[row 8*(i/4) + 4*(lane/32) + i%4][col lane%32] of the wave's block ----
    const int col = wn * 32 + (lane & 31);
    if constexpr (EPI == PE_SWIGLU) {
        float* sC = (float*) &sA[0][0][0];                          // [64][68] fp32, after the loop
        constexpr int LDC = PB + 4;
#pragma unroll
        for (int i = 0; i < 16; ++i) sC[(wm * 32 + 8 * (i / 4) + 4 * (lane >> 5) + (i & 3)) * LDC + col] = acc[i];
        __syncthreads();
        const int m = tid >> 2, j8 = (tid & 3) * 8;                // 8 activations of row m
        if (m < cnt) {
            uint32_t pk[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                uint16_t h[2];
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    const int j = j8 + 2 * q + b;
                    const float g = sC[m * LDC + j], u = sC[m * LDC + 32 + j];
                    h[b] = f_to_bf16(g / (1.0f + __expf(-g)) * u);
                }
                pk[q] = h[0] | ((uint32_t) h[1] << 16);
            }
            *(uint4*) (a.act + (size_t) (row0 + m) * a.act_ld + n0 + j8) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int m = wm * 32 + 8 * (i / 4) + 4 * (lane >> 5) + (i & 3);
            const int n = n0 + col;
            if (m >= cnt) continue;
            if constexpr (EPI == PE_F32) {
                if (n < a.n_rows) a.y[(size_t) (row0 + m) * a.y_ld + n] = acc[i];
            } else if constexpr (EPI == PE_SHARED) {
                const float sg = a.sg[row0 + m];
                a.y[(size_t) (row0 + m) * a.y_ld + n] = acc[i] / (1.0f + __expf(-sg));
            } else {
                atomicAdd(&a.y[(size_t) s_tok[m] * a.y_ld + n], a.wt[row0 + m] * acc[i]);
            }
        }
    }
}

__global__ void __launch_bounds__(256) pf_cvt_kernel(const float* __restrict__ x, uint16_t* __restrict__ xb, size_t n) {
    const size_t i = ((size_t) blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= n) return;
    const float4 v = *(const float4*) (x + i);
    *(uint2*) (xb + i) = make_uint2(f_to_bf16(v.x) | ((uint32_t) f_to_bf16(v.y) << 16),
                                    f_to_bf16(v.z) | ((uint32_t) f_to_bf16(v.w) << 16));
}

// one wave per token: routing of its logits row and the shared-expert gate
template <int RV>
__global__ void __launch_bounds__(256) pf_route_kernel(const float* __restrict__ logits, const uint16_t* __restrict__ xb,
                                                       const uint16_t* __restrict__ sgate, int N, int E, int K, int D,
                                                       int* __restrict__ ids, float* __restrict__ wts,
                                                       float* __restrict__ sg) {
    __shared__ uint64_t cand[4][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int t = blockIdx.x * 4 + w;
    if (t >= N) return;                                          // wave-uniform
    float p[RV];
#pragma unroll
    for (int i = 0; i < RV; ++i) {
        const int idx = lane + 64 * i;
        const float v = logits[(size_t) t * E + min(idx, E - 1)];
        p[i] = idx < E ? v : -INFINITY;
    }
    float s = 0.f;
    for (int d = lane; d < D; d += 64) s = fmaf(bf16_bits_to_f(sgate[d]), bf16_bits_to_f(xb[(size_t) t * D + d]), s);
    s = wave_sum(s);
    if (lane == 0) sg[t] = s;
    int my_id;
    float my_w, wsum;
    route_row<RV>(p, E, K, my_id, my_w, wsum, cand[w]);
    const float sc = fmaxf(wsum, 6.103515625e-05f);
    if (lane < K) {
        ids[(size_t) t * K + lane] = my_id;
        wts[(size_t) t * K + lane] = my_w / sc;
    }
}

// entries (token, slot) grouped by expert: 64-entry tiles, entry token and weight per position
__global__ void __launch_bounds__(1024) pf_group_kernel(const int* __restrict__ ids, const float* __restrict__ wts,
                                                        int n_ent, int K, int E, int* __restrict__ ent_tok,
                                                        float* __restrict__ ent_wt, PfTile* __restrict__ tiles,
                                                        int* __restrict__ n_tiles) {
    __shared__ int cnt[PF_MAX_E], off[PF_MAX_E], toff[PF_MAX_E], s_tot[2];
    const int tid = threadIdx.x;
    for (int i = tid; i < E; i += 1024) cnt[i] = 0;
    __syncthreads();
    for (int i = tid; i < n_ent; i += 1024) atomicAdd(&cnt[ids[i]], 1);
    __syncthreads();
    if (tid == 0) {                                               // E <= 1024 prefix sums, once per chunk
        int o = 0, to = 0;
        for (int i = 0; i < E; ++i) {
            off[i] = o;
            toff[i] = to;
            o += cnt[i];
            to += (cnt[i] + PB - 1) / PB;
        }
        s_tot[0] = to;
    }
    __syncthreads();
    for (int i = tid; i < E; i += 1024) {
        const int c = cnt[i];
        for (int q = 0; q * PB < c; ++q) tiles[toff[i] + q] = PfTile{i, off[i] + q * PB, min(PB, c - q * PB), 0};
    }
    if (tid == 0) *n_tiles = s_tot[0];
    __syncthreads();
    for (int i = tid; i < n_ent; i += 1024) {                     // cnt becomes the fill cursor
        const int e = ids[i];
        const int pos = off[e] + atomicSub(&cnt[e], 1) - 1;
        ent_tok[pos] = i / K;
        ent_wt[pos] = wts[i];
    }
}

struct PfWs {
    uint16_t* xb; float* logits; float* sg; int* ids; float* wts;
    int* ent_tok; float* ent_wt; PfTile* tiles; int* n_tiles;
    uint16_t* act; uint16_t* sh_act;
    int max_tiles;
};

PfWs pf_ws_carve(void* base, size_t cap, int D, int F, int E, int K, int N, size_t* need) {
    Arena a(base, cap);
    PfWs w;
    const size_t n_ent = (size_t) N * K;
    w.max_tiles = (int) (n_ent / PB + E);
    w.xb = a.take<uint16_t>((size_t) N * D);
    w.logits = a.take<float>((size_t) N * E);
    w.sg = a.take<float>(N);
    w.ids = a.take<int>(n_ent);
    w.wts = a.take<float>(n_ent);
    w.ent_tok = a.take<int>(n_ent);
    w.ent_wt = a.take<float>(n_ent);
    w.tiles = a.take<PfTile>(w.max_tiles);
    w.n_tiles = a.take<int>(1);
    w.act = a.take<uint16_t>(n_ent * F);
    w.sh_act = a.take<uint16_t>((size_t) N * F);
    if (need) *need = a.off;
    return w;
}

template <int WK, int EPI>
void launch_pf(const PfGemmArgs& a, dim3 grid, hipStream_t st) {
    hipLaunchKernelGGL((pf_gemm_kernel<WK, EPI>), grid, dim3(256), 0, st, a);
}

}  // namespace

// ---------------------------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------------------------
extern "C" size_t wzy_moe_prefill_workspace_bytes(int n_embd, int n_ff, int n_exp, int top_k, int n_tok) {
    size_t need = 0;
    pf_ws_carve(nullptr, 0, n_embd, n_ff, n_exp, top_k, n_tok, &need);
    return need + 256;
}

extern "C" int wzy_moe_prefill(const wzy_moe_weights* w, const float* x, int n_tok, float* comb, int* ids, float* wts,
                               void* workspace, size_t workspace_bytes, void* stream) {
    WZY_REQUIRE(w && x && comb && workspace, "wzy_moe_prefill: null pointer");
    WZY_REQUIRE(w->router && w->sgate && w->experts && w->sh_gate_q && w->sh_gate_s && w->sh_up_q && w->sh_up_s &&
                    w->sh_down_q && w->sh_down_s,
                "wzy_moe_prefill: null weight pointer");
    const int D = w->n_embd, F = w->n_ff, E = w->n_exp, K = w->top_k, N = n_tok;
    WZY_REQUIRE(N >= 1, "wzy_moe_prefill: n_tok must be positive");
    WZY_REQUIRE(D % 64 == 0 && D >= 64 && F % 64 == 0 && F >= 64, "wzy_moe_prefill: n_embd and n_ff must be multiples of 64");
    WZY_REQUIRE(E >= 1 && E <= PF_MAX_E && E % 64 == 0, "wzy_moe_prefill: n_exp must be a multiple of 64 up to %d",
                PF_MAX_E);
    WZY_REQUIRE(K >= 1 && K <= MOE_MAX_K && K <= E, "wzy_moe_prefill: top_k must be in [1, %d]", MOE_MAX_K);
    WZY_REQUIRE(workspace_bytes >= wzy_moe_prefill_workspace_bytes(D, F, E, K, N), "wzy_moe_prefill: workspace too small");
    hipStream_t st = as_stream(stream);
    size_t need = 0;
    char* base = (char*) workspace + (256 - (uintptr_t) workspace % 256) % 256;
    const PfWs ws = pf_ws_carve(base, workspace_bytes - 256, D, F, E, K, N, &need);
    const MoeOffsets o = moe_offsets(D, F);
    const int mt = (N + PB - 1) / PB;

    const size_t nx = (size_t) N * D;
    hipLaunchKernelGGL(pf_cvt_kernel, dim3((unsigned) ((nx / 4 + 255) / 256)), dim3(256), 0, st, x, ws.xb, nx);
    {   // router logits
        PfGemmArgs a{};
        a.a = ws.xb; a.a_rows = N; a.K = D;
        a.w = w->router; a.n_rows = E;
        a.y = ws.logits; a.y_ld = E;
        launch_pf<PW_BF16, PE_F32>(a, dim3(E / PB, mt), st);
    }
    if (E <= 512)
        hipLaunchKernelGGL((pf_route_kernel<8>), dim3((N + 3) / 4), dim3(256), 0, st, ws.logits, ws.xb, w->sgate, N, E, K,
                           D, ws.ids, ws.wts, ws.sg);
    else
        hipLaunchKernelGGL((pf_route_kernel<16>), dim3((N + 3) / 4), dim3(256), 0, st, ws.logits, ws.xb, w->sgate, N, E, K,
                           D, ws.ids, ws.wts, ws.sg);
    hipLaunchKernelGGL(pf_group_kernel, dim3(1), dim3(1024), 0, st, ws.ids, ws.wts, N * K, K, E, ws.ent_tok, ws.ent_wt,
                       ws.tiles, ws.n_tiles);
    {   // shared expert gate|up + SwiGLU, then down -> comb = sigmoid(sg) * shared
        PfGemmArgs a{};
        a.a = ws.xb; a.a_rows = N; a.K = D;
        a.w = w->sh_gate_q; a.ws = w->sh_gate_s; a.w2 = w->sh_up_q; a.ws2 = w->sh_up_s; a.n_rows = F;
        a.act = ws.sh_act; a.act_ld = F;
        launch_pf<PW_Q8, PE_SWIGLU>(a, dim3(F / 32, mt), st);
        PfGemmArgs b{};
        b.a = ws.sh_act; b.a_rows = N; b.K = F;
        b.w = w->sh_down_q; b.ws = w->sh_down_s; b.n_rows = D;
        b.y = comb; b.y_ld = D; b.sg = ws.sg;
        launch_pf<PW_Q8, PE_SHARED>(b, dim3(D / PB, mt), st);
    }
    {   // routed experts: gate|up + SwiGLU per tile, then down, weighted, added into comb
        PfGemmArgs a{};
        a.a = ws.xb; a.K = D; a.tok = ws.ent_tok;
        a.experts = w->experts; a.rec = o.rec; a.codes_off = o.gu_codes; a.scales_off = o.gu_scales;
        a.tail_off = o.tail; a.tail_gate = 0; a.tail_up = 1; a.up_row0 = F; a.n_rows = 2 * F;
        a.tiles = ws.tiles; a.n_tiles = ws.n_tiles;
        a.act = ws.act; a.act_ld = F;
        launch_pf<PW_FP4, PE_SWIGLU>(a, dim3(F / 32, ws.max_tiles), st);
        PfGemmArgs b{};
        b.a = ws.act; b.a_by_entry = true; b.K = F; b.tok = ws.ent_tok;
        b.experts = w->experts; b.rec = o.rec; b.codes_off = o.dn_codes; b.scales_off = o.dn_scales;
        b.tail_off = o.tail; b.tail_gate = 2; b.tail_up = 2; b.n_rows = D;
        b.tiles = ws.tiles; b.n_tiles = ws.n_tiles;
        b.y = comb; b.y_ld = D; b.wt = ws.ent_wt;
        launch_pf<PW_FP4, PE_ATOMIC>(b, dim3(D / PB, ws.max_tiles), st);
    }
    if (ids) WZY_HIP_TRY(hipMemcpyAsync(ids, ws.ids, (size_t) N * K * sizeof(int), hipMemcpyDeviceToDevice, st));
    if (wts) WZY_HIP_TRY(hipMemcpyAsync(wts, ws.wts, (size_t) N * K * sizeof(float), hipMemcpyDeviceToDevice, st));
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

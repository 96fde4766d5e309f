// moe_prefill.hip -- NVFP4 mixture-of-experts block for a prefill chunk of N tokens, on MFMA.
//
// Launch sequence of wzy_moe_prefill (N tokens, E experts, top-K):
//   1. pf_cvt      x fp32 -> bf16 (round to nearest even), the A operand of every GEMM
//   2. pf_gemm     router logits [N x E] = x . router^T                      (bf16 weights)
//   3. pf_route    per token, one wave: softmax top-K (the decode routing: probability desc, id asc,
//                  weights renormalised by max(sum, 2^-14)) and the shared-expert gate sg = sgate . x
//   4. pf_hist, pf_tiles, pf_scatter: entries (token, slot) grouped by expert into tiles of up to
//                  256 (LDS-histogram ranks, one reserving atomic per expert and workgroup, one scan)
//   5. pf_expert<gate|up, Q8_0>  shared expert, dense 128-token blocks, SwiGLU -> sh_act bf16 [N x F]
//   6. pf_expert<down, Q8_0>     shared expert, dense 256-token blocks -> comb = sigmoid(sg) * shared
//   7. pf_expert<gate|up, NVFP4> routed, one expert tile per workgroup, SwiGLU -> act bf16 [N*K x F]
//   8. pf_expert<down, NVFP4>    routed -> y fp32 [N*K x D] per entry; pf_combine: comb[t] +=
//                  sum_k w_k * y[pos(t, k)] in slot order (no float atomics)
// pf_expert: 8 waves, 256 weight rows per workgroup, up to 256 A rows; weights staged through LDS in
// coalesced 128-k chunks and dequantised by each lane into its v_mfma_f32_32x32x16_bf16 B fragment
// (e2m1 x e4m3 block scale is exact in bf16, the fp32 tensor scale goes onto the accumulators;
// Q8_0 code x fp16 scale is rounded to bf16).  pf_gemm: 64 x 64 LDS-tiled bf16 GEMM (router).
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
typedef float float2_t __attribute__((ext_vector_type(2)));

namespace {

constexpr int PB = 64;             // router GEMM: tile rows (M), weight rows (N) and K step
constexpr int PB_LD = PB + 8;      // LDS row stride in bf16 (16-byte aligned rows, staggered banks)
constexpr int PF_MAX_E = 1024;
constexpr int MT = 256;            // expert GEMM: entries per tile (8 MFMA row blocks of 32)
constexpr int EK = 64;             // expert GEMM: K step between barriers (four MFMA k16 slices)
constexpr int EA_LD = EK + 8;      // LDS row stride of the staged activations, bf16

struct PfTile {
    int e, off, cnt, pad;          // expert, first entry position, entries (<= MT)
};

// Router GEMM logits = A . W^T over rows m0 .. m0+63 of A [a_rows x K] (bf16), bf16 weights.
struct PfGemmArgs {
    const uint16_t* a;
    int a_rows, K;
    const uint16_t* w;             // weight rows of length K
    int n_rows;                    // weight rows
    float* y; int y_ld;            // y[row * y_ld + n]
    int ncb, mt;                   // 64-wide weight-row blocks and 64-row A tiles (grid = ncb * mt)
};

// Routed-expert GEMM over expert tiles.  Gate|up: A rows = x rows of the entries' tokens, output
// SwiGLU activations per entry; down: A rows = activations per entry, output fp32 per entry.
// Also the dense (shared-expert) GEMMs: tiles = consecutive blocks of `a_rows` token rows, Q8_0
// weights (gate|up: w / w2 rows, down: w rows), outputs per token row.
struct PfExpArgs {
    const uint8_t* experts;
    size_t rec, codes_off, scales_off, tail_off;
    int K;                         // reduction length: n_embd (gate|up) or n_ff (down)
    int F;                         // gate|up: first up row of the plane
    int gx;                        // column blocks per tile
    const PfTile* tiles; const int* n_tiles;   // expert tiles (null: dense blocks of dense_mt of a_rows rows)
    int a_rows, dense_mt;
    const uint16_t* a;
    const int* tok; int topk;      // gate|up: entry position -> token * K + slot
    const int8_t* w; const uint16_t* ws; const int8_t* w2; const uint16_t* ws2;   // Q8_0 weights
    uint16_t* act; float* y; int ld_out;   // outputs per entry position (dense: per token row)
    const float* sg;               // dense down: y = acc * sigmoid(sg[row])
};

WZY_DEV uint16_t f_to_bf16(float f) {                // hardware conversion, round to nearest even
    return __builtin_bit_cast(uint16_t, (__bf16) f);
}
WZY_DEV float bf16_bits_to_f(uint32_t h) { return __builtin_bit_cast(float, h << 16); }
WZY_DEV uint32_t f_bits(float f) { return __builtin_bit_cast(uint32_t, f); }

// Router GEMM tile: 64 rows x 64 weight rows, K stepped by 64 through two LDS buffers, each wave a
// 32 x 32 block.  Workgroups go to the 8 XCDs in turn (workgroup b on XCD b % 8); when the A tile count
// is a multiple of 8, XCD x runs the ncb weight blocks of A tiles x, x + 8, ... back to back, so each
// A tile is fetched into one XCD's L2 once instead of once per weight block.
__global__ void __launch_bounds__(256) pf_gemm_kernel(PfGemmArgs a) {
    __shared__ __align__(16) uint16_t sA[2][PB][PB_LD];
    __shared__ __align__(16) uint16_t sB[2][PB][PB_LD];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int wm = w & 1, wn = w >> 1;
    const int b = blockIdx.x;
    int rt, cb;
    if ((a.mt & 7) == 0) {
        const int s = b >> 3;
        rt = (s / a.ncb) * 8 + (b & 7);
        cb = s % a.ncb;
    } else {
        rt = b / a.ncb;
        cb = b % a.ncb;
    }
    const int row0 = rt * PB;
    const int cnt = min(PB, a.a_rows - row0);
    const int n0 = cb * PB;
    const int sr = tid >> 2, sk = (tid & 3) * 16;                // staging: row sr, k sk .. sk+15
    const int wrow = min(n0 + sr, a.n_rows - 1);
    const bool a_ok = sr < cnt;
    const uint16_t* ap = a.a + (size_t) (a_ok ? row0 + sr : 0) * a.K + sk;
    const uint16_t* wp = a.w + (size_t) wrow * a.K + sk;

    f32x16_t acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.f;
    const int nk = a.K / PB;

    // staging registers (scalars: an array captured by a lambda would live in scratch memory)
    uint4 xa0 = a_ok ? *(const uint4*) ap : make_uint4(0, 0, 0, 0);
    uint4 xa1 = a_ok ? *(const uint4*) (ap + 8) : make_uint4(0, 0, 0, 0);
    uint4 xw0 = *(const uint4*) wp, xw1 = *(const uint4*) (wp + 8);
    *(uint4*) &sA[0][sr][sk] = xa0;
    *(uint4*) &sA[0][sr][sk + 8] = xa1;
    *(uint4*) &sB[0][sr][sk] = xw0;
    *(uint4*) &sB[0][sr][sk + 8] = xw1;
    __syncthreads();
    for (int ks = 0; ks < nk; ++ks) {
        const int buf = ks & 1;
        const bool more = ks + 1 < nk;
        if (more) {                                              // next step's loads first
            const size_t o = (size_t) (ks + 1) * PB;
            xa0 = a_ok ? *(const uint4*) (ap + o) : make_uint4(0, 0, 0, 0);
            xa1 = a_ok ? *(const uint4*) (ap + o + 8) : make_uint4(0, 0, 0, 0);
            xw0 = *(const uint4*) (wp + o);
            xw1 = *(const uint4*) (wp + o + 8);
        }
#pragma unroll
        for (int kk = 0; kk < PB / 16; ++kk) {
            const bf16x8_t av = *(const bf16x8_t*) &sA[buf][wm * 32 + (lane & 31)][kk * 16 + (lane >> 5) * 8];
            const bf16x8_t bv = *(const bf16x8_t*) &sB[buf][wn * 32 + (lane & 31)][kk * 16 + (lane >> 5) * 8];
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, acc, 0, 0, 0);
        }
        if (more) {
            *(uint4*) &sA[buf ^ 1][sr][sk] = xa0;
            *(uint4*) &sA[buf ^ 1][sr][sk + 8] = xa1;
            *(uint4*) &sB[buf ^ 1][sr][sk] = xw0;
            *(uint4*) &sB[buf ^ 1][sr][sk + 8] = xw1;
        }
        __syncthreads();
    }

    // acc[i] = C[row 8*(i/4) + 4*(lane/32) + i%4][col lane%32] of the wave's block
    const int col = wn * 32 + (lane & 31);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int m = wm * 32 + 8 * (i / 4) + 4 * (lane >> 5) + (i & 3);
        const int n = n0 + col;
        if (m < cnt && n < a.n_rows) a.y[(size_t) (row0 + m) * a.y_ld + n] = acc[i];
    }
}

// MFMA B fragment (8 consecutive k of one weight row) from one 16-value NVFP4 sub-block: bytes
// w0 (0..3), w1 (4..7), byte i = value i (low nibble) | value i+8 (high nibble).  The lane half
// sa = 0 takes values 0..7, sa = 4 values 8..15: the nibbles are regrouped so that byte i holds
// values i and i+4 of the lane's eight, each converted pair is scaled by the e4m3 block scale (the
// product of a 2-bit and a 4-bit significand: exact in fp32 and in bf16), and the high halves are
// packed in k order.
WZY_DEV bf16x8_t fp4_frag(uint32_t w0, uint32_t w1, uint32_t sa, float sc) {
    const uint32_t d = ((w0 >> sa) & 0x0F0F0F0Fu) | (((w1 >> sa) & 0x0F0F0F0Fu) << 4);
    float2_t p[4];
    p[0] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 0);
    p[1] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 1);
    p[2] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 2);
    p[3] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 3);
    uint32_t b[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        b[i] = f_bits(p[i].x * sc);            // value i
        b[i + 4] = f_bits(p[i].y * sc);        // value i + 4
    }
    uint4 q;
    q.x = __builtin_amdgcn_perm(b[1], b[0], 0x07060302u);
    q.y = __builtin_amdgcn_perm(b[3], b[2], 0x07060302u);
    q.z = __builtin_amdgcn_perm(b[5], b[4], 0x07060302u);
    q.w = __builtin_amdgcn_perm(b[7], b[6], 0x07060302u);
    return __builtin_bit_cast(bf16x8_t, q);
}

// Two e4m3 block scales (bytes 0 and 1 of s) as fp32: the scaled fp8 -> f32 conversion with unit
// scale decodes OCP e4m3; the sign bit is ignored and code 0x7F (NaN in OCP, 480 in the unsigned
// reading) maps to 480 through the NaN-discarding min.
WZY_DEV float2_t e4m3x2(uint32_t s) {
    const float2_t v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(s & 0x7F7Fu, 1.0f, false);
    return float2_t{fminf(v.x, 480.0f), fminf(v.y, 480.0f)};
}

constexpr int EKB = 128;           // expert GEMM: weight chunk (k values) staged through LDS
constexpr int EROWS = 256;         // weight rows per workgroup (8 waves x 32)
constexpr int ETHR = 512;          // threads per expert workgroup
enum { WF_FP4 = 0, WF_Q8 = 1 };    // weight formats of the expert GEMM

// Bytes of one weight row per chunk (codes), and 16-byte pieces per thread to stage a chunk.
template <int WF> constexpr int chunk_bytes() { return WF == WF_FP4 ? EKB / 2 : EKB; }
template <int WF> constexpr int pieces_per_thread() { return chunk_bytes<WF>() * EROWS / 16 / ETHR; }

struct ExpLane {                   // per-thread view of one expert tile
    const uint8_t* crow0;          // staging: code bytes of the (row, 16-byte piece) slots, chunk 0
    const uint8_t* crow1;
    const uint8_t* crow2;          // (Q8 only)
    const uint8_t* crow3;
    const uint8_t* srow;           // staging (threads < 256): block scales of row `tid`, chunk 0
    const uint16_t* ap;            // staging: activation row of entry sr (+ k offset sk)
    int lr;                        // the lane's weight row (local) = its B fragment column
    int nk, cnt, row0, col, sr, sk;
    bool a_ok;
    uint32_t sa;
    float ts;
};

template <int WF>
struct ExpLds {
    uint16_t a[2][MT][EA_LD];                        // activation rows, one K step (64) per buffer
    uint8_t b[2][EROWS][chunk_bytes<WF>() + 16];     // weight codes, one chunk (128 k) per buffer
    uint2 s[2][EROWS];                               // the chunk's block scales per weight row (8 bytes)
    int row[MT];                                     // A row of each tile entry
};

// MFMA B fragment from 8 Q8_0 codes (one k16 half) times their fp16 block scale, rounded to bf16
// (code * scale is exact in fp32; the bf16 rounding is the dense reference's dequantisation).
WZY_DEV bf16x8_t q8_frag(uint2 q, float sc) {
    uint32_t b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t w = i < 2 ? q.x : q.y;
        const float v0 = (float) (int8_t) (w >> (16 * (i & 1))) * sc;
        const float v1 = (float) (int8_t) (w >> (16 * (i & 1) + 8)) * sc;
        b[i] = (uint32_t) f_to_bf16(v0) | ((uint32_t) f_to_bf16(v1) << 16);
    }
    return __builtin_bit_cast(bf16x8_t, make_uint4(b[0], b[1], b[2], b[3]));
}

// K loop and epilogue of one tile with NMB active 32-entry row blocks.
template <bool DOWN, int WF, int NMB>
WZY_DEV void expert_tile(const PfExpArgs& a, const ExpLane c, ExpLds<WF>& L) {
    constexpr int CB = chunk_bytes<WF>(), NP = pieces_per_thread<WF>(), PPR = CB / 16;
    const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5;
    const int nkc = c.nk / (EKB / EK);                              // weight chunks
    uint4 bq0 = make_uint4(0, 0, 0, 0), bq1 = bq0, bq2 = bq0, bq3 = bq0;
    uint2 bs = make_uint2(0, 0);
    f32x16_t acc[NMB];
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[mb][i] = 0.f;

    for (int kc = 0; kc < nkc; ++kc) {
        const int bb = kc & 1;
        const bool more_b = kc + 1 < nkc;
        if (more_b) {                                               // next weight chunk, coalesced
            const size_t o = (size_t) (kc + 1) * CB;
            bq0 = *(const uint4*) (c.crow0 + o);
            bq1 = *(const uint4*) (c.crow1 + o);
            if constexpr (NP == 4) {
                bq2 = *(const uint4*) (c.crow2 + o);
                bq3 = *(const uint4*) (c.crow3 + o);
            }
            if (tid < EROWS) bs = *(const uint2*) (c.srow + (size_t) (kc + 1) * 8);
        }
        const uint2 sw = L.s[bb][c.lr];
#pragma unroll
        for (int st = 0; st < EKB / EK; ++st) {
            const int ks = kc * (EKB / EK) + st;
            const int ab = ks & 1;
            uint4 xn[4];                                            // activations one step ahead
#pragma unroll
            for (int i = 0; i < 4; ++i) xn[i] = make_uint4(0, 0, 0, 0);
            if (ks + 1 < c.nk && c.a_ok) {
#pragma unroll
                for (int i = 0; i < 4; ++i) xn[i] = *(const uint4*) (c.ap + (size_t) (ks + 1) * EK + 8 * i);
            }
            bf16x8_t bfr[4];                                        // B fragments of k16 slices 4st .. 4st+3
            if constexpr (WF == WF_FP4) {
                // 8 code bytes and one e4m3 scale per slice
                const uint32_t sv = st ? sw.y : sw.x;
                const float2_t sc01 = e4m3x2(sv), sc23 = e4m3x2(sv >> 16);
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    const uint2 qq = *(const uint2*) &L.b[bb][c.lr][st * 32 + 8 * kk];
                    const float scv = kk == 0 ? sc01.x : kk == 1 ? sc01.y : kk == 2 ? sc23.x : sc23.y;
                    bfr[kk] = fp4_frag(qq.x, qq.y, c.sa, scv);
                }
            } else {
                // 16 code bytes per slice (this lane's 8 at byte 8h); one fp16 scale per two slices
                const uint32_t sv = st ? sw.y : sw.x;
                const float s0 = h16_to_f((uint16_t) sv), s1 = h16_to_f((uint16_t) (sv >> 16));
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    const uint2 qq = *(const uint2*) &L.b[bb][c.lr][st * 64 + 16 * kk + 8 * h];
                    bfr[kk] = q8_frag(qq, kk < 2 ? s0 : s1);
                }
            }
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
                for (int mb = 0; mb < NMB; ++mb) {
                    const bf16x8_t av = *(const bf16x8_t*) &L.a[ab][mb * 32 + (lane & 31)][kk * 16 + h * 8];
                    acc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bfr[kk], acc[mb], 0, 0, 0);
                }
            }
            if (ks + 1 < c.nk) {
#pragma unroll
                for (int i = 0; i < 4; ++i) *(uint4*) &L.a[ab ^ 1][c.sr][c.sk + 8 * i] = xn[i];
            }
            if (st == EKB / EK - 1 && more_b) {                     // the next chunk into the other buffer
                *(uint4*) &L.b[bb ^ 1][tid / PPR][(tid % PPR) * 16] = bq0;
                *(uint4*) &L.b[bb ^ 1][(ETHR + tid) / PPR][(tid % PPR) * 16] = bq1;
                if constexpr (NP == 4) {
                    *(uint4*) &L.b[bb ^ 1][(2 * ETHR + tid) / PPR][(tid % PPR) * 16] = bq2;
                    *(uint4*) &L.b[bb ^ 1][(3 * ETHR + tid) / PPR][(tid % PPR) * 16] = bq3;
                }
                if (tid < EROWS) L.s[bb ^ 1][tid] = bs;
            }
            __syncthreads();
        }
    }

    // acc[mb][i] = C[entry mb*32 + 8*(i/4) + 4*h + i%4][column lane%32 of the wave's weight block]
    const bool gate_lane = (lane & 16) == 0;
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int row = mb * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
            const float v = acc[mb][i] * c.ts;
            if constexpr (DOWN) {
                if (row < c.cnt) {
                    const size_t r = (size_t) (c.row0 + row);
                    a.y[r * a.ld_out + c.col] = a.sg ? v / (1.0f + __expf(-a.sg[r])) : v;
                }
            } else {
                // the matching up value from lane l ^ 16 (swizzle bit-mode: and 0x1F, xor 0x10)
                const float u = __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle((int) f_bits(v), 0x401F));
                if (gate_lane && row < c.cnt)
                    a.act[(size_t) (c.row0 + row) * a.ld_out + c.col] =
                        f_to_bf16(v * __builtin_amdgcn_rcpf(1.0f + __expf(-v)) * u);
            }
        }
    }
}

// Routed-expert GEMM.  Workgroup = one expert tile (<= 256 entries) x 256 weight rows, 8 waves; wave
// w owns one 32-row weight block (gate|up: 16 gate rows j0+16w.. in columns 0..15 and the matching
// 16 up rows in columns 16..31, paired for SwiGLU across lanes l, l^16; down: rows n0+32w .. +31)
// for all active 32-entry row blocks of the tile (the count selects a specialised loop), so each
// dequantised B fragment feeds up to 8 MFMAs.  Weight codes move in 128-k chunks: each row's code
// bytes are read as 16-byte pieces by adjacent threads (whole 64-byte segments), one chunk ahead,
// into LDS; each lane then takes its row's bytes per k16 slice from LDS and dequantises them into
// its MFMA B fragment.  The activation rows of the tile are staged in LDS one 64-k step ahead and
// shared by the eight waves.  Workgroups are numbered so that consecutive workgroups of one XCD take
// the column blocks of one tile (its activation rows stay in that XCD's L2).  The tensor scale is
// applied to the fp32 accumulators.  WF_Q8 with a null tile list runs the dense shared-expert
// GEMMs over consecutive blocks of token rows.
template <bool DOWN, int WF>
__global__ void __launch_bounds__(ETHR, 1) pf_expert_kernel(PfExpArgs a) {
    constexpr int CB = chunk_bytes<WF>(), NP = pieces_per_thread<WF>(), PPR = CB / 16;
    __shared__ __align__(16) ExpLds<WF> L;
    const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int bx = blockIdx.x, jx = bx >> 3;
    const int ti = (jx / a.gx) * 8 + (bx & 7), nb = jx % a.gx;
    const bool dense = a.tiles == nullptr;
    if (ti >= (dense ? (a.a_rows + a.dense_mt - 1) / a.dense_mt : *a.n_tiles)) return;   // workgroup-uniform
    ExpLane c;
    int e = 0;
    if (dense) {
        c.row0 = ti * a.dense_mt;
        c.cnt = min(a.dense_mt, a.a_rows - c.row0);
    } else {
        const PfTile t = a.tiles[ti];
        c.cnt = t.cnt;
        c.row0 = t.off;
        e = t.e;
    }
    if (tid < MT)
        L.row[tid] = tid < c.cnt ? ((DOWN || dense) ? c.row0 + tid : a.tok[c.row0 + tid] / a.topk) : 0;
    const uint8_t* rec = a.experts + (size_t) e * a.rec;
    // local weight row lr = 32w + column -> weight row: gate|up: columns 0..15 gate rows
    // j0+16w+col, columns 16..31 up rows (plane row F+j0+16w+col-16, or the w2 matrix); down: n0 + lr
    auto wrow = [&](int lr, bool& up) {
        const int wl = lr >> 5, cl = lr & 31;
        up = !DOWN && cl >= 16;
        return DOWN ? nb * EROWS + lr : nb * 128 + wl * 16 + (cl & 15);
    };
    auto code_row = [&](int lr) -> const uint8_t* {
        bool up;
        const int r = wrow(lr, up);
        if constexpr (WF == WF_FP4) return rec + a.codes_off + (size_t) (up ? a.F + r : r) * (a.K / 2);
        else return (const uint8_t*) ((up ? a.w2 : a.w) + (size_t) r * a.K);
    };
    auto scale_row = [&](int lr) -> const uint8_t* {
        bool up;
        const int r = wrow(lr, up);
        if constexpr (WF == WF_FP4) return rec + a.scales_off + (size_t) (up ? a.F + r : r) * (a.K / 16);
        else return (const uint8_t*) ((up ? a.ws2 : a.ws) + (size_t) r * (a.K / 32));
    };
    c.lr = w * 32 + (lane & 31);
    c.col = DOWN ? nb * EROWS + c.lr : nb * 128 + w * 16 + (lane & 15);
    if constexpr (WF == WF_FP4) {
        const float* tail = (const float*) (rec + a.tail_off);
        c.ts = DOWN ? tail[2] : ((lane & 16) ? tail[1] : tail[0]);
    } else {
        c.ts = 1.0f;
    }
    const int pp = (tid % PPR) * 16;
    c.crow0 = code_row(tid / PPR) + pp;
    c.crow1 = code_row((ETHR + tid) / PPR) + pp;
    c.crow2 = NP == 4 ? code_row((2 * ETHR + tid) / PPR) + pp : c.crow0;
    c.crow3 = NP == 4 ? code_row((3 * ETHR + tid) / PPR) + pp : c.crow0;
    c.srow = scale_row(tid & (EROWS - 1));
    c.nk = a.K / EK;
    c.sa = 4u * h;
    // weight chunk 0
    *(uint4*) &L.b[0][tid / PPR][pp] = *(const uint4*) c.crow0;
    *(uint4*) &L.b[0][(ETHR + tid) / PPR][pp] = *(const uint4*) c.crow1;
    if constexpr (NP == 4) {
        *(uint4*) &L.b[0][(2 * ETHR + tid) / PPR][pp] = *(const uint4*) c.crow2;
        *(uint4*) &L.b[0][(3 * ETHR + tid) / PPR][pp] = *(const uint4*) c.crow3;
    }
    if (tid < EROWS) L.s[0][tid] = *(const uint2*) c.srow;
    __syncthreads();
    c.sr = tid >> 1;                                                // staging: entry sr, k sk .. sk+31
    c.sk = (tid & 1) * 32;
    c.a_ok = c.sr < c.cnt;
    c.ap = a.a + (size_t) L.row[c.sr] * a.K + c.sk;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        *(uint4*) &L.a[0][c.sr][c.sk + 8 * i] = c.a_ok ? *(const uint4*) (c.ap + 8 * i) : make_uint4(0, 0, 0, 0);
    __syncthreads();
    switch ((c.cnt + 31) >> 5) {                                    // workgroup-uniform
        case 1: expert_tile<DOWN, WF, 1>(a, c, L); break;
        case 2: expert_tile<DOWN, WF, 2>(a, c, L); break;
        case 3: expert_tile<DOWN, WF, 3>(a, c, L); break;
        case 4: expert_tile<DOWN, WF, 4>(a, c, L); break;
        case 5: expert_tile<DOWN, WF, 5>(a, c, L); break;
        case 6: expert_tile<DOWN, WF, 6>(a, c, L); break;
        case 7: expert_tile<DOWN, WF, 7>(a, c, L); break;
        default: expert_tile<DOWN, WF, 8>(a, c, L); break;
    }
}

// x fp32 -> bf16; workgroup 0 also clears the per-expert entry cursors
__global__ void __launch_bounds__(256) pf_cvt_kernel(const float* __restrict__ x, uint16_t* __restrict__ xb, size_t n,
                                                     int* __restrict__ cursor, int E) {
    if (blockIdx.x == 0)
        for (int i = threadIdx.x; i < E; i += 256) cursor[i] = 0;
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

constexpr int PF_HCHUNK = 1024;    // entries per histogram workgroup

// entries [g*1024, (g+1)*1024): each entry's rank among the entries of its expert in this workgroup
// (LDS counters), then one atomic add per expert reserves the workgroup's run in the expert's list
// (cursor ends as the expert's entry count)
__global__ void __launch_bounds__(256) pf_hist_kernel(const int* __restrict__ ids, int n_ent, int E,
                                                      int* __restrict__ cursor, int* __restrict__ wg_base,
                                                      int* __restrict__ rank) {
    __shared__ int h[PF_MAX_E];
    const int tid = threadIdx.x, g = blockIdx.x;
    for (int i = tid; i < E; i += 256) h[i] = 0;
    __syncthreads();
    const int i0 = g * PF_HCHUNK, i1 = min(n_ent, i0 + PF_HCHUNK);
    for (int i = i0 + tid; i < i1; i += 256) rank[i] = atomicAdd(&h[ids[i]], 1);
    __syncthreads();
    for (int i = tid; i < E; i += 256) {
        const int c = h[i];
        wg_base[(size_t) g * E + i] = c ? atomicAdd(&cursor[i], c) : 0;
    }
}

// one workgroup: exclusive scans of the entry counts and of the tiles per expert -> each expert's
// first entry position and its MT-entry tiles
__global__ void __launch_bounds__(1024) pf_tiles_kernel(const int* __restrict__ cnt, int E, int* __restrict__ exp_off,
                                                        PfTile* __restrict__ tiles, int* __restrict__ n_tiles) {
    __shared__ uint64_t s_w[16];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int c = tid < E ? cnt[tid] : 0;
    const int nt = (c + MT - 1) / MT;
    const uint64_t v = ((uint64_t) c << 24) | (uint64_t) nt;       // both sums in one scan
    uint64_t s = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint64_t o = __shfl_up(s, d);
        if (lane >= d) s += o;
    }
    if (lane == 63) s_w[w] = s;
    __syncthreads();
    uint64_t base = 0;
    for (int i = 0; i < w; ++i) base += s_w[i];
    const uint64_t ex = base + s - v;
    const int off = (int) (ex >> 24), toff = (int) (ex & 0xFFFFFFu);
    if (tid < E) {
        exp_off[tid] = off;
        for (int q = 0; q < nt; ++q) tiles[toff + q] = PfTile{tid, off + q * MT, min(MT, c - q * MT), 0};
    }
    if (tid == 1023) *n_tiles = (int) ((base + s) & 0xFFFFFFu);
}

// entry i = (token i / K, slot i % K) <-> its position in the expert-sorted list
__global__ void __launch_bounds__(256) pf_scatter_kernel(const int* __restrict__ ids, const int* __restrict__ rank,
                                                         const int* __restrict__ wg_base,
                                                         const int* __restrict__ exp_off, int n_ent, int K, int E,
                                                         int* __restrict__ ent_idx, int* __restrict__ ent_pos) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n_ent) return;
    const int e = ids[i];
    const int pos = exp_off[e] + wg_base[(size_t) (i / PF_HCHUNK) * E + e] + rank[i];
    ent_idx[pos] = i;
    ent_pos[i] = pos;
}

// comb[t] += sum_k w_k * y[pos(t, k)] in slot order (comb holds the gated shared expert). A pass issues the
// row loads of KU slots together; EXACT means K is a multiple of KU, so no slot load is predicated.
template <int KU, bool EXACT>
__global__ void __launch_bounds__(256) pf_combine_kernel(const float* __restrict__ y, const int* __restrict__ ent_pos,
                                                         const float* __restrict__ wts, int K, int D,
                                                         float* __restrict__ comb) {
    const int t = blockIdx.y;
    const int d = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (d >= D) return;
    float4 acc = *(const float4*) (comb + (size_t) t * D + d);
    const int* pt = ent_pos + (size_t) t * K;
    const float* wt = wts + (size_t) t * K;
    for (int k0 = 0; k0 < K; k0 += KU) {
        const int n = EXACT ? KU : min(KU, K - k0);   // uniform over the workgroup
        float4 v[KU];
        float wk[KU];
#pragma unroll
        for (int j = 0; j < KU; ++j) {
            if (EXACT || j < n) {
                wk[j] = wt[k0 + j];
                v[j] = *(const float4*) (y + (size_t) pt[k0 + j] * D + d);
            } else {
                wk[j] = 0.f;
                v[j] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
#pragma unroll
        for (int j = 0; j < KU; ++j) {
            if (EXACT || j < n) {
                acc.x = fmaf(wk[j], v[j].x, acc.x);
                acc.y = fmaf(wk[j], v[j].y, acc.y);
                acc.z = fmaf(wk[j], v[j].z, acc.z);
                acc.w = fmaf(wk[j], v[j].w, acc.w);
            }
        }
    }
    *(float4*) (comb + (size_t) t * D + d) = acc;
}

struct PfWs {
    uint16_t* xb; float* logits; float* sg; int* ids; float* wts;
    int* cursor; int* exp_off; int* wg_base; int* rank; int* ent_idx; int* ent_pos; PfTile* tiles; int* n_tiles;
    uint16_t* act; uint16_t* sh_act; float* y;
    int max_tiles, n_wg;
};

PfWs pf_ws_carve(void* base, size_t cap, int D, int F, int E, int K, int N, size_t* need) {
    Arena a(base, cap);
    PfWs w;
    const size_t n_ent = (size_t) N * K;
    w.max_tiles = (int) (n_ent / MT + E);
    w.xb = a.take<uint16_t>((size_t) N * D);
    w.logits = a.take<float>((size_t) N * E);
    w.sg = a.take<float>(N);
    w.ids = a.take<int>(n_ent);
    w.wts = a.take<float>(n_ent);
    w.n_wg = (int) ((n_ent + PF_HCHUNK - 1) / PF_HCHUNK);
    w.cursor = a.take<int>(E);
    w.exp_off = a.take<int>(E);
    w.wg_base = a.take<int>((size_t) w.n_wg * E);
    w.rank = a.take<int>(n_ent);
    w.ent_idx = a.take<int>(n_ent);
    w.ent_pos = a.take<int>(n_ent);
    w.tiles = a.take<PfTile>(w.max_tiles);
    w.n_tiles = a.take<int>(1);
    w.act = a.take<uint16_t>(n_ent * F);
    w.sh_act = a.take<uint16_t>((size_t) N * F);
    w.y = a.take<float>(n_ent * D);
    if (need) *need = a.off;
    return w;
}

template <bool DOWN>
void launch_expert(const PfExpArgs& a, int max_tiles, hipStream_t st) {
    const unsigned n = (unsigned) (a.gx * ((max_tiles + 7) / 8) * 8);
    hipLaunchKernelGGL((pf_expert_kernel<DOWN, WF_FP4>), dim3(n), dim3(ETHR), 0, st, a);
}
template <bool DOWN>
void launch_dense_q8(const PfExpArgs& a, hipStream_t st) {
    const int nt = (a.a_rows + a.dense_mt - 1) / a.dense_mt;
    const unsigned n = (unsigned) (a.gx * ((nt + 7) / 8) * 8);
    hipLaunchKernelGGL((pf_expert_kernel<DOWN, WF_Q8>), dim3(n), dim3(ETHR), 0, st, a);
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

namespace {

constexpr int PF_N_STAGES = 8;     // timing groups of pf_enqueue

int pf_check(const wzy_moe_weights* w, int N) {
    WZY_REQUIRE(w, "wzy_moe_prefill: null weights");
    WZY_REQUIRE(w->router && w->sgate && w->experts && w->sh_gate_q && w->sh_gate_s && w->sh_up_q && w->sh_up_s &&
                    w->sh_down_q && w->sh_down_s,
                "wzy_moe_prefill: null weight pointer");
    const int D = w->n_embd, F = w->n_ff, E = w->n_exp, K = w->top_k;
    WZY_REQUIRE(N >= 1 && (int64_t) N * K <= (1 << 26), "wzy_moe_prefill: n_tok must be in [1, 2^26 / top_k]");
    WZY_REQUIRE(D % 256 == 0 && D >= 256 && F % 128 == 0 && F >= 128,
                "wzy_moe_prefill: n_embd must be a multiple of 256 and n_ff a multiple of 128");
    WZY_REQUIRE(E >= 1 && E <= PF_MAX_E && E % 64 == 0, "wzy_moe_prefill: n_exp must be a multiple of 64 up to %d",
                PF_MAX_E);
    WZY_REQUIRE(K >= 1 && K <= MOE_MAX_K && K <= E, "wzy_moe_prefill: top_k must be in [1, %d]", MOE_MAX_K);
    WZY_REQUIRE((int64_t) (E / PB) * ((N + PB - 1) / PB) * 256 <= INT32_MAX && (int64_t) N * D <= INT32_MAX,
                "wzy_moe_prefill: n_tok x n_embd exceeds the launch grids");
    return WZY_OK;
}

// The launch sequence; with `ev`, event i is recorded before launch group i and event PF_N_STAGES
// after the last one.
void pf_enqueue(const wzy_moe_weights* w, const float* x, int N, float* comb, const PfWs& ws, hipStream_t st,
                hipEvent_t* ev) {
    const int D = w->n_embd, F = w->n_ff, E = w->n_exp, K = w->top_k;
    const int n_ent = N * K;
    const MoeOffsets o = moe_offsets(D, F);
    const int mt = (N + PB - 1) / PB;
    auto mark = [&](int i) {
        if (ev) (void) hipEventRecord(ev[i], st);
    };
    const size_t nx = (size_t) N * D;
    mark(0);
    hipLaunchKernelGGL(pf_cvt_kernel, dim3((unsigned) ((nx / 4 + 255) / 256)), dim3(256), 0, st, x, ws.xb, nx,
                       ws.cursor, E);
    mark(1);
    {   // router logits
        PfGemmArgs a{};
        a.a = ws.xb; a.a_rows = N; a.K = D;
        a.w = w->router; a.n_rows = E;
        a.y = ws.logits; a.y_ld = E;
        a.ncb = E / PB; a.mt = mt;
        hipLaunchKernelGGL(pf_gemm_kernel, dim3((unsigned) (a.ncb * mt)), dim3(256), 0, st, a);
    }
    mark(2);
    if (E <= 512)
        hipLaunchKernelGGL((pf_route_kernel<8>), dim3((N + 3) / 4), dim3(256), 0, st, ws.logits, ws.xb, w->sgate, N, E, K,
                           D, ws.ids, ws.wts, ws.sg);
    else
        hipLaunchKernelGGL((pf_route_kernel<16>), dim3((N + 3) / 4), dim3(256), 0, st, ws.logits, ws.xb, w->sgate, N, E, K,
                           D, ws.ids, ws.wts, ws.sg);
    mark(3);
    hipLaunchKernelGGL(pf_hist_kernel, dim3((unsigned) ws.n_wg), dim3(256), 0, st, ws.ids, n_ent, E, ws.cursor,
                       ws.wg_base, ws.rank);
    hipLaunchKernelGGL(pf_tiles_kernel, dim3(1), dim3(1024), 0, st, ws.cursor, E, ws.exp_off, ws.tiles, ws.n_tiles);
    hipLaunchKernelGGL(pf_scatter_kernel, dim3((unsigned) ((n_ent + 255) / 256)), dim3(256), 0, st, ws.ids, ws.rank,
                       ws.wg_base, ws.exp_off, n_ent, K, E, ws.ent_idx, ws.ent_pos);
    // shared expert gate|up + SwiGLU, then down -> comb = sigmoid(sg) * shared (dense Q8_0 tiles)
    mark(4);
    {
        PfExpArgs a{};
        a.experts = w->experts; a.K = D; a.F = F; a.gx = F / 128;
        a.a_rows = N; a.dense_mt = MT / 2; a.a = ws.xb;     // 128-row blocks: F/128 x N/128 workgroups
        a.w = (const int8_t*) w->sh_gate_q; a.ws = (const uint16_t*) w->sh_gate_s;
        a.w2 = (const int8_t*) w->sh_up_q; a.ws2 = (const uint16_t*) w->sh_up_s;
        a.act = ws.sh_act; a.ld_out = F;
        launch_dense_q8<false>(a, st);
    }
    mark(5);
    {
        PfExpArgs b{};
        b.experts = w->experts; b.K = F; b.gx = D / EROWS;
        b.a_rows = N; b.dense_mt = MT; b.a = ws.sh_act;
        b.w = (const int8_t*) w->sh_down_q; b.ws = (const uint16_t*) w->sh_down_s;
        b.y = comb; b.ld_out = D; b.sg = ws.sg;
        launch_dense_q8<true>(b, st);
    }
    // routed experts: gate|up + SwiGLU per tile, down per tile, then the per-token weighted sum
    mark(6);
    {
        PfExpArgs a{};
        a.experts = w->experts; a.rec = o.rec; a.codes_off = o.gu_codes; a.scales_off = o.gu_scales;
        a.tail_off = o.tail; a.K = D; a.F = F; a.gx = F / 128;
        a.tiles = ws.tiles; a.n_tiles = ws.n_tiles;
        a.a = ws.xb; a.tok = ws.ent_idx; a.topk = K;
        a.act = ws.act; a.ld_out = F;
        launch_expert<false>(a, ws.max_tiles, st);
    }
    mark(7);
    {
        PfExpArgs b{};
        b.experts = w->experts; b.rec = o.rec; b.codes_off = o.dn_codes; b.scales_off = o.dn_scales;
        b.tail_off = o.tail; b.K = F; b.F = 0; b.gx = D / 256;
        b.tiles = ws.tiles; b.n_tiles = ws.n_tiles;
        b.a = ws.act; b.tok = nullptr; b.topk = K;
        b.y = ws.y; b.ld_out = D;
        launch_expert<true>(b, ws.max_tiles, st);
        const dim3 cg((unsigned) ((D / 4 + 255) / 256), (unsigned) N);
        if (K == 10)
            hipLaunchKernelGGL((pf_combine_kernel<10, true>), cg, dim3(256), 0, st, ws.y, ws.ent_pos, ws.wts, K, D, comb);
        else if (K % 8 == 0)
            hipLaunchKernelGGL((pf_combine_kernel<8, true>), cg, dim3(256), 0, st, ws.y, ws.ent_pos, ws.wts, K, D, comb);
        else
            hipLaunchKernelGGL((pf_combine_kernel<8, false>), cg, dim3(256), 0, st, ws.y, ws.ent_pos, ws.wts, K, D, comb);
    }
    mark(8);
}

PfWs pf_ws_for(const wzy_moe_weights* w, int N, void* workspace, size_t workspace_bytes) {
    char* base = (char*) workspace + (256 - (uintptr_t) workspace % 256) % 256;
    return pf_ws_carve(base, workspace_bytes - 256, w->n_embd, w->n_ff, w->n_exp, w->top_k, N, nullptr);
}

}  // namespace

extern "C" int wzy_moe_prefill(const wzy_moe_weights* w, const float* x, int n_tok, float* comb, int* ids, float* wts,
                               void* workspace, size_t workspace_bytes, void* stream) {
    WZY_REQUIRE(x && comb && workspace, "wzy_moe_prefill: null pointer");
    WZY_TRY(pf_check(w, n_tok));
    const int N = n_tok, K = w->top_k;
    WZY_REQUIRE(workspace_bytes >= wzy_moe_prefill_workspace_bytes(w->n_embd, w->n_ff, w->n_exp, K, N),
                "wzy_moe_prefill: workspace too small");
    hipStream_t st = as_stream(stream);
    const PfWs ws = pf_ws_for(w, N, workspace, workspace_bytes);
    pf_enqueue(w, x, N, comb, ws, st, nullptr);
    if (ids) WZY_HIP_TRY(hipMemcpyAsync(ids, ws.ids, (size_t) N * K * sizeof(int), hipMemcpyDeviceToDevice, st));
    if (wts) WZY_HIP_TRY(hipMemcpyAsync(wts, ws.wts, (size_t) N * K * sizeof(float), hipMemcpyDeviceToDevice, st));
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

extern "C" int wzy_moe_prefill_time(const wzy_moe_weights* w, const float* x, int n_tok, float* comb, void* workspace,
                                    size_t workspace_bytes, int iters, float* us_stages, void* stream) {
    WZY_REQUIRE(x && comb && workspace && us_stages && iters >= 1, "wzy_moe_prefill_time: bad arguments");
    WZY_TRY(pf_check(w, n_tok));
    WZY_REQUIRE(workspace_bytes >= wzy_moe_prefill_workspace_bytes(w->n_embd, w->n_ff, w->n_exp, w->top_k, n_tok),
                "wzy_moe_prefill_time: workspace too small");
    hipStream_t st = as_stream(stream);
    const PfWs ws = pf_ws_for(w, n_tok, workspace, workspace_bytes);
    hipEvent_t ev[PF_N_STAGES + 1];
    for (int i = 0; i <= PF_N_STAGES; ++i) WZY_HIP_TRY(hipEventCreate(&ev[i]));
    double acc[PF_N_STAGES] = {};
    int rc = WZY_OK;
    pf_enqueue(w, x, n_tok, comb, ws, st, nullptr);                 // warm-up
    for (int it = 0; it < iters && rc == WZY_OK; ++it) {
        pf_enqueue(w, x, n_tok, comb, ws, st, ev);
        if (hipEventSynchronize(ev[PF_N_STAGES]) != hipSuccess) { rc = WZY_EHIP; break; }
        for (int i = 0; i < PF_N_STAGES; ++i) {
            float ms = 0.f;
            if (hipEventElapsedTime(&ms, ev[i], ev[i + 1]) != hipSuccess) { rc = WZY_EHIP; break; }
            acc[i] += ms;
        }
    }
    for (int i = 0; i <= PF_N_STAGES; ++i) (void) hipEventDestroy(ev[i]);
    if (rc != WZY_OK) {
        set_error("wzy_moe_prefill_time: event timing failed");
        return rc;
    }
    for (int i = 0; i < PF_N_STAGES; ++i) us_stages[i] = (float) (1000.0 * acc[i] / iters);
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

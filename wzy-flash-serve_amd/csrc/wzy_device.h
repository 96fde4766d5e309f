// wzy_device.h -- gfx950 (CDNA4) device helpers shared by every kernel of the decode path.
//
// Wave-level primitives are written for 64-lane wavefronts: intra-row steps use DPP
// (quad_perm / row_half_mirror / row_mirror), the row-16 step uses ds_swizzle and the
// last step reads lane 32 with v_readlane, so a full 64-lane reduction never touches LDS.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define WZY_DEV __device__ __forceinline__

namespace wzy {

// ---------------------------------------------------------------------------------------------
// bit casts and small formats
// ---------------------------------------------------------------------------------------------
WZY_DEV float as_f(int v) { return __builtin_bit_cast(float, v); }
WZY_DEV int as_i(float v) { return __builtin_bit_cast(int, v); }
WZY_DEV float bf16_lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
WZY_DEV float bf16_hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }
WZY_DEV float bf16_to_f(uint16_t h) { return __builtin_bit_cast(float, (uint32_t) h << 16); }

// IEEE binary16 <-> fp32 through the hardware conversion instructions (v_cvt_f32_f16 / v_cvt_f16_f32,
// round-to-nearest-even).
WZY_DEV float h16_to_f(uint16_t h) { return (float) __builtin_bit_cast(_Float16, h); }
WZY_DEV uint16_t f_to_h16(float f) { return __builtin_bit_cast(uint16_t, (_Float16) f); }
WZY_DEV float round_h16(float f) { return (float) (_Float16) f; }

// round-half-even float -> int (the reference's __float2int_rn / _mm_cvtss_si32)
WZY_DEV int rn_int(float x) { return (int) __builtin_rintf(x); }

WZY_DEV float sigmoidf_(float x) { return 1.0f / (1.0f + __expf(-x)); }
WZY_DEV float siluf_(float x) { return x / (1.0f + __expf(-x)); }

// ---------------------------------------------------------------------------------------------
// DPP / swizzle wave reductions (64 lanes)
// ---------------------------------------------------------------------------------------------
// dpp_ctrl encodings (GCN3+ ISA): quad_perm = p0 | p1<<2 | p2<<4 | p3<<6, row_mirror 0x140,
// row_half_mirror 0x141.  All four patterns read a valid lane, so bound_ctrl is irrelevant; the
// move has no old value, which lets the compiler fold it into the consuming VALU op as a DPP
// operand (v_add_f32_dpp) instead of a copy, a DPP move and the op.
template <int CTRL>
WZY_DEV float dpp_f(float v) {
    return as_f(__builtin_amdgcn_mov_dpp(as_i(v), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
WZY_DEV int dpp_i(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}
constexpr int DPP_XOR1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int DPP_XOR2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int DPP_HALF_MIRROR = 0x141; // lane i <-> 7-i within each 8
constexpr int DPP_MIRROR = 0x140;      // lane i <-> 15-i within each 16
// ds_swizzle bit-mode offset: and_mask | or_mask<<5 | xor_mask<<10 (operates inside 32-lane halves)
constexpr int SWZ_XOR16 = (0x10 << 10) | 0x1F;
constexpr int SWZ_XOR8 = (0x08 << 10) | 0x1F;

template <int PAT>
WZY_DEV float swz_f(float v) { return as_f(__builtin_amdgcn_ds_swizzle(as_i(v), PAT)); }
template <int PAT>
WZY_DEV int swz_i(int v) { return __builtin_amdgcn_ds_swizzle(v, PAT); }

// Sum over each group of 16 consecutive lanes; every lane of the group gets the group sum.
WZY_DEV float sum16(float v) {
    v += dpp_f<DPP_XOR1>(v);
    v += dpp_f<DPP_XOR2>(v);
    v += dpp_f<DPP_HALF_MIRROR>(v);
    v += dpp_f<DPP_MIRROR>(v);
    return v;
}
// Sum over each group of 8 consecutive lanes.
WZY_DEV float sum8(float v) {
    v += dpp_f<DPP_XOR1>(v);
    v += dpp_f<DPP_XOR2>(v);
    v += dpp_f<DPP_HALF_MIRROR>(v);
    return v;
}
// Sum over each group of 32 lanes (lanes 0-31 / 32-63).
WZY_DEV float sum32(float v) {
    v = sum16(v);
    v += swz_f<SWZ_XOR16>(v);
    return v;
}
// Full 64-lane sum, wave-uniform result.
WZY_DEV float wave_sum(float v) {
    v = sum32(v);
    const float a = as_f(__builtin_amdgcn_readlane(as_i(v), 0));
    const float b = as_f(__builtin_amdgcn_readlane(as_i(v), 32));
    return a + b;
}
// Sums over the wave of N per-lane values (N = 1, 2, 4, 8 or 16), transposed: lane l returns the
// sum of a[l % N] over all 64 lanes.  Six partner levels run in one fixed order: the row rotation by
// 8 (partner lane bit 3), the half mirror (partner l ^ 7 inside each 8), the quad permutations xor 2
// and xor 1, then the permlane16 and permlane32 swaps.  A level whose bit is among the low log2(N)
// splits the values a lane holds (each lane keeps the half its partner does not); the others add all
// of them.  Either way a value's sum at every level is own + partner, so (addition being commutative)
// every value gets the same sum tree, bit for bit, whatever N: results do not depend on how many
// values share the reduction (e.g. a window's row count).  About 3N/2 + 8 VALU operations and no
// LDS swizzle or lane reads, against N wave sums.  (The swaps are written as inline assembly: the
// compiler's builtin hands both results in one register when they feed one add; the s_nops cover
// the VALU-write-to-permlane hazard.)
constexpr int DPP_ROW_ROR8 = 0x128;     // lane i <- lane (i + 8) mod 16 within each row
constexpr int DPP_ROW_SHL1 = 0x101;     // lane i <- lane i + 1 within each row (0 past its end)
constexpr int DPP_ROW_SHL2 = 0x102;     // lane i <- lane i + 2 within each row
constexpr int DPP_ROW_SHL4 = 0x104;     // lane i <- lane i + 4 within each row
template <int CTRL, int M, int SPLIT>
WZY_DEV void reduce_level(const float (&in)[M], float (&out)[SPLIT ? M / 2 : M], bool upper) {
    if constexpr (SPLIT) {
#pragma unroll
        for (int i = 0; i < M / 2; ++i) out[i] = (upper ? in[i + M / 2] : in[i]) + dpp_f<CTRL>(upper ? in[i] : in[i + M / 2]);
    } else {
#pragma unroll
        for (int i = 0; i < M; ++i) out[i] = in[i] + dpp_f<CTRL>(in[i]);
    }
}
template <int N>
WZY_DEV float reduce_wave(const float (&a)[N]) {
    static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16, "reduce_wave: N must be a power of 2 <= 16");
    const int lane = threadIdx.x & 63;
    constexpr int M3 = N >= 16 ? N / 2 : N, M2 = N >= 8 ? M3 / 2 : M3, M1 = N >= 4 ? M2 / 2 : M2;
    float b[M3], c[M2], d[M1], e[1];
    reduce_level<DPP_ROW_ROR8, N, (N >= 16)>(a, b, (lane & 8) != 0);
    reduce_level<DPP_HALF_MIRROR, M3, (N >= 8)>(b, c, (lane & 4) != 0);
    reduce_level<DPP_XOR2, M2, (N >= 4)>(c, d, (lane & 2) != 0);
    reduce_level<DPP_XOR1, M1, (N >= 2)>(d, e, (lane & 1) != 0);
    uint32_t x = __builtin_bit_cast(uint32_t, e[0]), y = x;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(x), "+v"(y));
    const float f = __builtin_bit_cast(float, x) + __builtin_bit_cast(float, y);
    x = __builtin_bit_cast(uint32_t, f);
    y = x;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(x), "+v"(y));
    return __builtin_bit_cast(float, x) + __builtin_bit_cast(float, y);
}
// NV wave sums through reduce_wave, stored by the lanes that hold them: store(i, sum of v[i]) runs
// on one lane per i.  NV is padded with zeros to a power of 2, or cut into groups of 16; each value's
// sum tree is reduce_wave's, whatever NV.
template <int NV, typename F>
WZY_DEV void reduce_wave_store(const float (&v)[NV], F&& store) {
    constexpr int P = NV <= 1 ? 1 : NV <= 2 ? 2 : NV <= 4 ? 4 : NV <= 8 ? 8 : 16;
    constexpr int NG = (NV + 15) / 16;
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int g = 0; g < (NV > 16 ? NG : 1); ++g) {
        float w[P];
#pragma unroll
        for (int i = 0; i < P; ++i) w[i] = (16 * g + i < NV) ? v[16 * g + i] : 0.f;
        const float tot = reduce_wave<P>(w);
        const int idx = 16 * g + lane;
        if (lane < P && idx < NV) store(idx, tot);
    }
}
WZY_DEV float max16(float v) {
    v = fmaxf(v, dpp_f<DPP_XOR1>(v));
    v = fmaxf(v, dpp_f<DPP_XOR2>(v));
    v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_f<DPP_MIRROR>(v));
    return v;
}
WZY_DEV float max32(float v) {
    v = max16(v);
    v = fmaxf(v, swz_f<SWZ_XOR16>(v));
    return v;
}
WZY_DEV float wave_max(float v) {
    v = max32(v);
    const float a = as_f(__builtin_amdgcn_readlane(as_i(v), 0));
    const float b = as_f(__builtin_amdgcn_readlane(as_i(v), 32));
    return fmaxf(a, b);
}

// (value, index) argmax step: larger value wins, ties go to the lower index.  Branch-free: the
// bitwise combination keeps the compiler from turning the test into divergent control flow.
WZY_DEV void amax_merge(float& bv, int& bi, float ov, int oi) {
    const bool take = (ov > bv) | ((ov == bv) & (oi < bi));
    bv = take ? ov : bv;
    bi = take ? oi : bi;
}
// Full-wave argmax with lowest-index tie-break; result is wave-uniform.
WZY_DEV void wave_argmax(float& bv, int& bi) {
    amax_merge(bv, bi, dpp_f<DPP_XOR1>(bv), dpp_i<DPP_XOR1>(bi));
    amax_merge(bv, bi, dpp_f<DPP_XOR2>(bv), dpp_i<DPP_XOR2>(bi));
    amax_merge(bv, bi, dpp_f<DPP_HALF_MIRROR>(bv), dpp_i<DPP_HALF_MIRROR>(bi));
    amax_merge(bv, bi, dpp_f<DPP_MIRROR>(bv), dpp_i<DPP_MIRROR>(bi));
    amax_merge(bv, bi, swz_f<SWZ_XOR16>(bv), swz_i<SWZ_XOR16>(bi));
    const float v32 = as_f(__builtin_amdgcn_readlane(as_i(bv), 32));
    const int i32 = __builtin_amdgcn_readlane(bi, 32);
    bv = as_f(__builtin_amdgcn_readlane(as_i(bv), 0));
    bi = __builtin_amdgcn_readlane(bi, 0);
    amax_merge(bv, bi, v32, i32);
}

// 64-bit DPP move (both halves with the same control); rows outside ROWMASK keep their own value.
constexpr int DPP_ROW_BCAST15 = 0x142; // lane 15 of each row -> the next row
constexpr int DPP_ROW_BCAST31 = 0x143; // lane 31 -> rows 2 and 3
template <int CTRL, int ROWMASK>
WZY_DEV uint64_t dpp_u64(uint64_t v) {
    const int lo = (int) (uint32_t) v, hi = (int) (uint32_t) (v >> 32);
    const uint32_t l2 = (uint32_t) __builtin_amdgcn_update_dpp(lo, lo, CTRL, ROWMASK, 0xF, false);
    const uint32_t h2 = (uint32_t) __builtin_amdgcn_update_dpp(hi, hi, CTRL, ROWMASK, 0xF, false);
    return ((uint64_t) h2 << 32) | l2;
}
WZY_DEV uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }
// Full-wave maximum of a 64-bit key with DPP only (no LDS swizzle): lane 63 ends with the maximum,
// which is returned to every lane.
WZY_DEV uint64_t wave_max_u64(uint64_t k) {
    k = max_u64(k, dpp_u64<DPP_XOR1, 0xF>(k));
    k = max_u64(k, dpp_u64<DPP_XOR2, 0xF>(k));
    k = max_u64(k, dpp_u64<DPP_HALF_MIRROR, 0xF>(k));
    k = max_u64(k, dpp_u64<DPP_MIRROR, 0xF>(k));
    k = max_u64(k, dpp_u64<DPP_ROW_BCAST15, 0xA>(k));
    k = max_u64(k, dpp_u64<DPP_ROW_BCAST31, 0xC>(k));
    const uint32_t lo = (uint32_t) __builtin_amdgcn_readlane((int) (uint32_t) k, 63);
    const uint32_t hi = (uint32_t) __builtin_amdgcn_readlane((int) (uint32_t) (k >> 32), 63);
    return ((uint64_t) hi << 32) | lo;
}

// Full-wave maximum of a 32-bit unsigned value with DPP only; lane 63 ends with the maximum, which is
// returned to every lane (wave-uniform).
// (Lanes of rows outside a row mask read 0, the identity of an unsigned maximum, so the moves can
// fold into the max instructions.)
template <int CTRL, int ROWMASK>
WZY_DEV uint32_t dpp_u32(uint32_t v) {
    return (uint32_t) __builtin_amdgcn_update_dpp(0, (int) v, CTRL, ROWMASK, 0xF, false);
}
WZY_DEV uint32_t wave_max_u32(uint32_t v) {
    v = max(v, dpp_u32<DPP_XOR1, 0xF>(v));
    v = max(v, dpp_u32<DPP_XOR2, 0xF>(v));
    v = max(v, dpp_u32<DPP_HALF_MIRROR, 0xF>(v));
    v = max(v, dpp_u32<DPP_MIRROR, 0xF>(v));
    v = max(v, dpp_u32<DPP_ROW_BCAST15, 0xA>(v));
    v = max(v, dpp_u32<DPP_ROW_BCAST31, 0xC>(v));
    return (uint32_t) __builtin_amdgcn_readlane((int) v, 63);
}

// Block-wide sum for blockDim.x = NW*64 threads; `sh` must hold NW floats. Result on every thread.
template <int NW>
WZY_DEV float block_sum(float v, float* sh) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) sh[w] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < NW; ++i) t += sh[i];
    __syncthreads();
    return t;
}
template <int NW>
WZY_DEV float block_max(float v, float* sh) {
    v = wave_max(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) sh[w] = v;
    __syncthreads();
    float t = sh[0];
#pragma unroll
    for (int i = 1; i < NW; ++i) t = fmaxf(t, sh[i]);
    __syncthreads();
    return t;
}

// ---------------------------------------------------------------------------------------------
// streaming 128-bit loads: weights are read once per token, so they are loaded with the
// non-temporal hint and do not displace activations in the caches.
// ---------------------------------------------------------------------------------------------
typedef int wzy_v4i __attribute__((ext_vector_type(4)));
WZY_DEV int4 ld_stream_i4(const void* p) {
    const wzy_v4i v = __builtin_nontemporal_load((const wzy_v4i*) p);
    return make_int4(v.x, v.y, v.z, v.w);
}
WZY_DEV uint4 ld_stream_u4(const void* p) {
    const wzy_v4i v = __builtin_nontemporal_load((const wzy_v4i*) p);
    return make_uint4((uint32_t) v.x, (uint32_t) v.y, (uint32_t) v.z, (uint32_t) v.w);
}

// ---------------------------------------------------------------------------------------------
// int8 dot products (v_dot4_i32_i8)
// ---------------------------------------------------------------------------------------------
WZY_DEV int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }
WZY_DEV int dot16(int4 a, int4 b) {
    int s = dot4(a.x, b.x, 0);
    s = dot4(a.y, b.y, s);
    s = dot4(a.z, b.z, s);
    return dot4(a.w, b.w, s);
}

// ---------------------------------------------------------------------------------------------
// NVFP4 (e2m1 codes x e4m3 block scales)
// ---------------------------------------------------------------------------------------------
// Unsigned e4m3 block scale (sign bit ignored), pre-multiplied by 0.5 to cancel the doubled e2m1
// codes: e == 0 -> m * 2^-9, else (1 + m/8) * 2^(e-7); no NaN encoding is special-cased.
WZY_DEV float ue4m3_half(uint32_t x) {
    x &= 0x7Fu;
    const uint32_t e = x >> 3, m = x & 7u;
    // normal: build the fp32 directly: exponent (e-7-1)+127 (the -1 is the 0.5 factor), mantissa m<<20
    const float nrm = __builtin_bit_cast(float, ((e + 119u) << 23) | (m << 20));
    const float sub = (float) m * 0.0009765625f;       // m * 2^-9 * 0.5
    return e ? nrm : sub;
}

}  // namespace wzy

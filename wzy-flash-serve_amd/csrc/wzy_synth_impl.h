// wzy_synth_impl.h -- counter-based synthetic model generator, usable from host C/C++ and HIP
// device code.  Every value is a pure function of (seed, stream, index), so any tensor element can
// be produced on the GPU (bulk initialisation in HBM) or on the CPU (the parity checks) with
// identical bits.  Device-side paths use only integer and exactly-rounded double operations.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define WZY_HD __host__ __device__ static inline
#else
#define WZY_HD static inline
#endif

// splitmix64 finalizer (Steele, Lea, Flood 2014)
WZY_HD uint64_t wzy_mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}
WZY_HD uint64_t wzy_hash3(uint64_t seed, uint64_t stream, uint64_t idx) {
    return wzy_mix64(wzy_mix64(seed * 0x9E3779B97F4A7C15ULL + stream) + idx * 0xD1B54A32D192ED03ULL);
}

// Stream ids: kind in bits 48..63, layer in 32..47, sub-id in 0..31.
enum {
    WZY_S_EXP_CODE = 1,   // sub = expert*4 + matrix (0 gate, 1 up, 2 down)
    WZY_S_EXP_SCALE = 2,
    WZY_S_KV_K = 3,       // sub = 0 codes / 1 scales
    WZY_S_KV_V = 4,
    WZY_S_DENSE = 5,      // sub = tensor id (see wzy_synth.h)
    WZY_S_STATE = 6,
    WZY_S_INPUT = 7,
    WZY_S_PLE = 9,        // per-layer embedding table codes
    WZY_S_Q2 = 8,         // MTP Q2_0 experts: sub = expert*4 + part (0 gate/up codes, 1 down codes,
                          // 2 gate/up scales, 3 down scales)
};
WZY_HD uint64_t wzy_stream(uint32_t kind, uint32_t layer, uint32_t sub) {
    return ((uint64_t) kind << 48) | ((uint64_t) (layer & 0xFFFFu) << 32) | (uint64_t) sub;
}

// e4m3 code (bias 7, no sign) of U(0.5, 2) * 2^-4, round-to-nearest-even on the 3-bit mantissa.
// Values lie in [2^-5, 2^-3), so the exponent field is 2 or 3 (or 4 after rounding up to 2^-3).
WZY_HD uint8_t wzy_e4m3_scale_code(uint64_t h) {
    const double u = (double) (h >> 40) * (1.0 / 16777216.0);      // [0,1), 24 bits, exact
    const double x = (0.5 + 1.5 * u) * 0.0625;                      // exact in double
    int e;
    double t;
    if (x < 0.0625) { e = 2; t = x * 32.0; } else { e = 3; t = x * 16.0; }   // t in [1,2)
    const double m8 = t * 8.0 - 8.0;                                 // [0,8), exact
    double mr = m8 - (double) (int64_t) m8;                          // fractional part
    int m = (int) (int64_t) m8;
    if (mr > 0.5 || (mr == 0.5 && (m & 1))) ++m;                     // ties to even
    if (m == 8) { m = 0; ++e; }
    return (uint8_t) ((e << 3) | m);
}

// One byte of an expert's code plane: matrix `mat` (0 gate, 1 up, 2 down), row `r`, byte `i` of
// the row's code bytes (row_code_bytes per row).  8 bytes come from one hash.
WZY_HD uint8_t wzy_expert_code_byte(uint64_t seed, int layer, int expert, int mat, int r, int i,
                                    int row_code_bytes) {
    const uint64_t lin = (uint64_t) r * (uint64_t) row_code_bytes + (uint64_t) i;
    const uint64_t h = wzy_hash3(seed, wzy_stream(WZY_S_EXP_CODE, (uint32_t) layer, (uint32_t) (expert * 4 + mat)),
                                 lin >> 3);
    return (uint8_t) (h >> (8 * (lin & 7)));
}
// e4m3 scale byte of sub-block `sb` (16 values) of row `r` of matrix `mat`.
WZY_HD uint8_t wzy_expert_scale_byte(uint64_t seed, int layer, int expert, int mat, int r, int sb,
                                     int row_subs) {
    const uint64_t lin = (uint64_t) r * (uint64_t) row_subs + (uint64_t) sb;
    return wzy_e4m3_scale_code(
        wzy_hash3(seed, wzy_stream(WZY_S_EXP_SCALE, (uint32_t) layer, (uint32_t) (expert * 4 + mat)), lin));
}

// int8 KV code uniform over [-127, 127] for cell `pos`, element `i` of a KVD-wide cell.
WZY_HD int8_t wzy_kv_code(uint64_t seed, int layer, int is_v, int64_t pos, int i, int kvd) {
    const uint64_t lin = (uint64_t) pos * (uint64_t) kvd + (uint64_t) i;
    const uint64_t h = wzy_hash3(seed, wzy_stream(is_v ? WZY_S_KV_V : WZY_S_KV_K, (uint32_t) layer, 0), lin);
    return (int8_t) ((int) ((h >> 32) % 255u) - 127);
}
// fp16 bits of a KV group scale: (0.5 + u) * 2^-6 with 10-bit u (exactly representable in fp16:
// values in [2^-7, 1.5*2^-6)), so dequantised K/V values stay O(1).
WZY_HD uint16_t wzy_kv_scale_h16(uint64_t seed, int layer, int is_v, int64_t pos, int g, int groups) {
    const uint64_t lin = (uint64_t) pos * (uint64_t) groups + (uint64_t) g;
    const uint64_t h = wzy_hash3(seed, wzy_stream(is_v ? WZY_S_KV_V : WZY_S_KV_K, (uint32_t) layer, 1), lin);
    const uint32_t u10 = (uint32_t) (h >> 54);                        // 10 bits
    // value = (512 + u10) * 2^-16 : exponent -7 (fp16 field 8) when u10 < 512, else -6.
    const uint32_t v = 512u + u10;                                    // [512, 1536)
    if (v < 1024u) return (uint16_t) ((8u << 10) | ((v - 512u) << 1));          // (1 + (v-512)/512) * 2^-7
    return (uint16_t) ((9u << 10) | (v - 1024u));                               // (1 + (v-1024)/1024) * 2^-6
}

// ---- MTP Q2_0 experts (blob layout: gate/up codes [2F][D/4], down codes [D][F/4], gate/up fp16
// scales [2F][D/64], down fp16 scales [D][F/64]) ----
// Code byte `lin` of part 0 (gate/up) or 1 (down): four uniform 2-bit codes, 8 bytes per hash.
WZY_HD uint8_t wzy_q2_code_byte(uint64_t seed, int expert, int part, uint64_t lin) {
    const uint64_t h = wzy_hash3(seed, wzy_stream(WZY_S_Q2, 0, (uint32_t) (expert * 4 + part)), lin >> 3);
    return (uint8_t) (h >> (8 * (lin & 7)));
}
// fp16 bits of scale `lin` of part 2 (gate/up, reduction dim D) or 3 (down, reduction dim F):
// (1 + m/1024) * 2^e with a uniform 10-bit m and e = floor(log2(1/sqrt(cols))) passed as `e`, so the
// dequantised weights (code - 1) * scale have a standard deviation near 1/sqrt(cols).
WZY_HD uint16_t wzy_q2_scale_h16(uint64_t seed, int expert, int part, uint64_t lin, int e) {
    const uint64_t h = wzy_hash3(seed, wzy_stream(WZY_S_Q2, 0, (uint32_t) (expert * 4 + part)), lin);
    return (uint16_t) (((uint32_t) (e + 15) << 10) | (uint32_t) (h >> 54));
}
// floor(log2(1/sqrt(cols))) for cols a power of two times 1 or 2 (exact integer arithmetic)
WZY_HD int wzy_q2_scale_exp(int cols) {
    int l = 0;
    while ((1 << (l + 1)) <= cols) ++l;     // l = floor(log2(cols))
    return -((l + 1) / 2);                  // -ceil(l/2): 2048 (l=11) -> -6, 512 (l=9) -> -5
}

// One byte of the synthetic per-layer-embedding table: an fp8 (e4m3, bias 7) code with a random sign
// and mantissa and an exponent field in 4..9 (|value| in [2^-3, 2^3) before the table scale), so no
// code is subnormal or NaN.  Byte j of row `row` (head_bytes bytes per row); 4 bytes per hash.
WZY_HD uint8_t wzy_ple_code(uint64_t seed, uint64_t row, int head_bytes, int j) {
    const uint64_t lin = row * (uint64_t) head_bytes + (uint64_t) j;
    const uint64_t h = wzy_hash3(seed, wzy_stream(WZY_S_PLE, 0, 0), lin >> 2);
    const uint32_t b = (uint32_t) (h >> (16 * (lin & 3))) & 0xFFFFu;
    return (uint8_t) (((b & 1u) << 7) | ((4u + (b >> 4) % 6u) << 3) | ((b >> 1) & 7u));
}

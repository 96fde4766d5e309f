// synth.hip -- seeded synthetic tensors: host generators (normals via Box-Muller in fp64) and
// device generators for the bulk integer-derived tensors (NVFP4 experts, INT8 KV cells).
#include <math.h>
#include <string.h>

#include <thread>
#include <vector>

#include "../../include/wzy_synth.h"
#include "wzy_host.h"
#include "wzy_synth_impl.h"

using namespace wzy;

// ---------------------------------------------------------------------------------------------
// half / bf16 helpers
// ---------------------------------------------------------------------------------------------
extern "C" uint16_t wzy_f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, (_Float16) f); }
extern "C" float wzy_f16_to_f32(uint16_t h) { return (float) __builtin_bit_cast(_Float16, h); }
extern "C" uint16_t wzy_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t) ((u >> 16) | 0x40u);   // quiet NaN
    return (uint16_t) ((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
static inline float bf16f(uint16_t h) {
    uint32_t u = (uint32_t) h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

extern "C" uint64_t wzy_synth_hash(uint64_t seed, uint64_t stream, uint64_t idx) {
    return wzy_hash3(seed, stream, idx);
}
extern "C" uint64_t wzy_synth_stream(uint32_t kind, uint32_t layer, uint32_t sub) {
    return wzy_stream(kind, layer, sub);
}

// Run f(begin, end) over [0, n) on up to 16 host threads (chunks of at least 64K elements).
template <class F>
static void parallel_for(size_t n, F f) {
    const size_t min_chunk = 1u << 16;
    unsigned nt = std::thread::hardware_concurrency();
    if (nt == 0) nt = 1;
    if (nt > 16) nt = 16;
    if (n < min_chunk * 2 || nt == 1) { f((size_t) 0, n); return; }
    size_t chunks = (n + min_chunk - 1) / min_chunk;
    if (chunks < nt) nt = (unsigned) chunks;
    std::vector<std::thread> th;
    const size_t per = (n + nt - 1) / nt;
    for (unsigned i = 0; i < nt; ++i) {
        const size_t b = i * per, e = (b + per < n) ? b + per : n;
        if (b >= e) break;
        th.emplace_back([=] { f(b, e); });
    }
    for (auto& t : th) t.join();
}

// Standard normal for element i: Box-Muller on the pair p = i/2 (u1 from hash(2p), u2 from hash(2p+1)).
static inline double normal_at(uint64_t seed, uint64_t stream, uint64_t i) {
    const uint64_t p = i >> 1;
    const double u1 = 1.0 - (double) (wzy_hash3(seed, stream, 2 * p) >> 11) * (1.0 / 9007199254740992.0); // (0,1]
    const double u2 = (double) (wzy_hash3(seed, stream, 2 * p + 1) >> 11) * (1.0 / 9007199254740992.0);
    const double r = sqrt(-2.0 * log(u1));
    const double a = 6.283185307179586476925286766559 * u2;
    return (i & 1) ? r * sin(a) : r * cos(a);
}

// Box-Muller pair (z0, z1) for elements 2p, 2p+1
static inline void normal_pair(uint64_t seed, uint64_t stream, uint64_t p, double& z0, double& z1) {
    const double u1 = 1.0 - (double) (wzy_hash3(seed, stream, 2 * p) >> 11) * (1.0 / 9007199254740992.0);
    const double u2 = (double) (wzy_hash3(seed, stream, 2 * p + 1) >> 11) * (1.0 / 9007199254740992.0);
    const double r = sqrt(-2.0 * log(u1));
    const double a = 6.283185307179586476925286766559 * u2;
    z0 = r * cos(a);
    z1 = r * sin(a);
}

extern "C" void wzy_synth_normal(uint64_t seed, uint64_t stream, size_t n, float mean, float std, float* out) {
    parallel_for(n, [&](size_t b, size_t e) {
        for (size_t i = b; i < e; ++i) out[i] = (float) ((double) mean + (double) std * normal_at(seed, stream, i));
    });
}
extern "C" void wzy_synth_uniform(uint64_t seed, uint64_t stream, size_t n, float lo, float hi, float* out) {
    parallel_for(n, [&](size_t b, size_t e) {
        for (size_t i = b; i < e; ++i) {
            const double u = (double) (wzy_hash3(seed, stream, i) >> 11) * (1.0 / 9007199254740992.0);
            out[i] = (float) ((double) lo + ((double) hi - (double) lo) * u);
        }
    });
}
extern "C" void wzy_synth_normal_bf16(uint64_t seed, uint64_t stream, size_t n, float mean, float std, uint16_t* out) {
    parallel_for(n, [&](size_t b, size_t e) {
        for (size_t i = b; i < e; ++i)
            out[i] = wzy_f32_to_bf16((float) ((double) mean + (double) std * normal_at(seed, stream, i)));
    });
}
extern "C" void wzy_synth_q8(uint64_t seed, uint64_t stream, int rows, int cols, float std, int8_t* codes,
                             uint16_t* scales) {
    const int nb = cols / 32;
    parallel_for((size_t) rows * nb, [&](size_t b, size_t e) {
        for (size_t blk = b; blk < e; ++blk) {
            float v[32];
            float amax = 0.f;
            for (int i = 0; i < 32; i += 2) {
                double z0, z1;
                normal_pair(seed, stream, (blk * 32 + (uint64_t) i) >> 1, z0, z1);
                v[i] = bf16f(wzy_f32_to_bf16((float) ((double) std * z0)));
                v[i + 1] = bf16f(wzy_f32_to_bf16((float) ((double) std * z1)));
                amax = fmaxf(amax, fmaxf(fabsf(v[i]), fabsf(v[i + 1])));
            }
            const uint16_t sh = wzy_f32_to_f16(amax / 127.0f);
            const float d = wzy_f16_to_f32(sh);
            for (int i = 0; i < 32; ++i) {
                int q = 0;
                if (d > 0.f) {
                    q = (int) rintf(v[i] / d);
                    q = q < -127 ? -127 : (q > 127 ? 127 : q);
                }
                codes[blk * 32 + i] = (int8_t) q;
            }
            scales[blk] = sh;
        }
    });
}

// ---------------------------------------------------------------------------------------------
// NVFP4 experts
// ---------------------------------------------------------------------------------------------
extern "C" size_t wzy_nvfp4_expert_bytes(int n_embd, int n_ff) {
    const size_t gu = (size_t) 2 * n_ff * (n_embd / 2) + (size_t) 2 * n_ff * (n_embd / 16);
    const size_t dn = (size_t) n_embd * (n_ff / 2) + (size_t) n_embd * (n_ff / 16);
    return gu + dn + 16;
}
extern "C" size_t wzy_nvfp4_blob_bytes(int n_embd, int n_ff) {
    return (size_t) 2 * n_ff * (n_embd / 64 * 36) + (size_t) n_embd * (n_ff / 64 * 36) + 16;
}

// Plane offsets of one expert record.
struct Planes {
    size_t gu_codes, gu_scales, dn_codes, dn_scales, tail;
};
static Planes planes_of(int D, int F) {
    Planes p;
    p.gu_codes = 0;
    p.gu_scales = p.gu_codes + (size_t) 2 * F * (D / 2);
    p.dn_codes = p.gu_scales + (size_t) 2 * F * (D / 16);
    p.dn_scales = p.dn_codes + (size_t) D * (F / 2);
    p.tail = p.dn_scales + (size_t) D * (F / 16);
    return p;
}

extern "C" int wzy_nvfp4_repack_host(const uint8_t* blob, uint8_t* planes, int n_embd, int n_ff) {
    WZY_REQUIRE(blob && planes, "wzy_nvfp4_repack_host: null pointer");
    WZY_REQUIRE(n_embd % 64 == 0 && n_ff % 64 == 0, "wzy_nvfp4_repack_host: dims must be multiples of 64");
    const int D = n_embd, F = n_ff;
    const Planes p = planes_of(D, F);
    const int gu_row = D / 64 * 36, dn_row = F / 64 * 36;
    for (int r = 0; r < 2 * F; ++r) {
        const uint8_t* src = blob + (size_t) r * gu_row;
        for (int b = 0; b < D / 64; ++b) {
            memcpy(planes + p.gu_scales + (size_t) r * (D / 16) + 4 * b, src + 36 * b, 4);
            memcpy(planes + p.gu_codes + (size_t) r * (D / 2) + 32 * b, src + 36 * b + 4, 32);
        }
    }
    const uint8_t* dn = blob + (size_t) 2 * F * gu_row;
    for (int r = 0; r < D; ++r) {
        const uint8_t* src = dn + (size_t) r * dn_row;
        for (int b = 0; b < F / 64; ++b) {
            memcpy(planes + p.dn_scales + (size_t) r * (F / 16) + 4 * b, src + 36 * b, 4);
            memcpy(planes + p.dn_codes + (size_t) r * (F / 2) + 32 * b, src + 36 * b + 4, 32);
        }
    }
    const size_t blob_tail = wzy_nvfp4_blob_bytes(D, F) - 16;
    memcpy(planes + p.tail, blob + blob_tail, 16);
    return WZY_OK;
}

static void tail_scales(uint8_t* dst) {
    const float one[4] = {1.0f, 1.0f, 1.0f, 0.0f};
    memcpy(dst, one, 16);
}

extern "C" int wzy_synth_expert_blob(uint64_t seed, int layer, int expert, int n_embd, int n_ff, uint8_t* blob) {
    WZY_REQUIRE(blob, "wzy_synth_expert_blob: null pointer");
    WZY_REQUIRE(n_embd % 64 == 0 && n_ff % 64 == 0, "wzy_synth_expert_blob: dims must be multiples of 64");
    const int D = n_embd, F = n_ff;
    const int gu_row = D / 64 * 36, dn_row = F / 64 * 36;
    for (int mat = 0; mat < 3; ++mat) {
        const int rows = mat < 2 ? F : D, cols = mat < 2 ? D : F;
        const int row_bytes = mat < 2 ? gu_row : dn_row;
        uint8_t* m0 = blob + (mat == 0 ? 0 : mat == 1 ? (size_t) F * gu_row : (size_t) 2 * F * gu_row);
        for (int r = 0; r < rows; ++r) {
            uint8_t* row = m0 + (size_t) r * row_bytes;
            for (int b = 0; b < cols / 64; ++b) {
                for (int s = 0; s < 4; ++s)
                    row[36 * b + s] = wzy_expert_scale_byte(seed, layer, expert, mat, r, 4 * b + s, cols / 16);
                for (int i = 0; i < 32; ++i)
                    row[36 * b + 4 + i] = wzy_expert_code_byte(seed, layer, expert, mat, r, 32 * b + i, cols / 2);
            }
        }
    }
    tail_scales(blob + wzy_nvfp4_blob_bytes(D, F) - 16);
    return WZY_OK;
}

extern "C" int wzy_synth_expert_planes(uint64_t seed, int layer, int expert, int n_embd, int n_ff, uint8_t* planes) {
    WZY_REQUIRE(planes, "wzy_synth_expert_planes: null pointer");
    WZY_REQUIRE(n_embd % 64 == 0 && n_ff % 64 == 0, "wzy_synth_expert_planes: dims must be multiples of 64");
    const int D = n_embd, F = n_ff;
    const Planes p = planes_of(D, F);
    for (int mat = 0; mat < 3; ++mat) {
        const int rows = mat < 2 ? F : D, cols = mat < 2 ? D : F;
        uint8_t* codes = planes + (mat < 2 ? p.gu_codes + (size_t) mat * F * (D / 2) : p.dn_codes);
        uint8_t* scales = planes + (mat < 2 ? p.gu_scales + (size_t) mat * F * (D / 16) : p.dn_scales);
        for (int r = 0; r < rows; ++r) {
            for (int i = 0; i < cols / 2; ++i)
                codes[(size_t) r * (cols / 2) + i] = wzy_expert_code_byte(seed, layer, expert, mat, r, i, cols / 2);
            for (int s = 0; s < cols / 16; ++s)
                scales[(size_t) r * (cols / 16) + s] = wzy_expert_scale_byte(seed, layer, expert, mat, r, s, cols / 16);
        }
    }
    tail_scales(planes + p.tail);
    return WZY_OK;
}

// One thread per 8 code bytes / per scale byte of one matrix-row range.
__global__ void synth_expert_kernel(uint64_t seed, int layer, int first_expert, int D, int F, size_t rec_bytes,
                                    uint8_t* __restrict__ dev) {
    const int e = blockIdx.y;
    const int expert = first_expert + e;
    uint8_t* rec = dev + (size_t) e * rec_bytes;
    const size_t gu_codes = 0;
    const size_t gu_scales = (size_t) 2 * F * (D / 2);
    const size_t dn_codes = gu_scales + (size_t) 2 * F * (D / 16);
    const size_t dn_scales = dn_codes + (size_t) D * (F / 2);
    const size_t tail = dn_scales + (size_t) D * (F / 16);
    // work items: code qwords of the three matrices, then scale bytes
    const size_t n_gu_q = (size_t) 2 * F * (D / 2) / 8, n_dn_q = (size_t) D * (F / 2) / 8;
    const size_t n_gu_s = (size_t) 2 * F * (D / 16), n_dn_s = (size_t) D * (F / 16);
    const size_t total = n_gu_q + n_dn_q + n_gu_s + n_dn_s;
    for (size_t w = (size_t) blockIdx.x * blockDim.x + threadIdx.x; w < total; w += (size_t) gridDim.x * blockDim.x) {
        if (w < n_gu_q) {
            const size_t byte0 = w * 8;                       // within gate|up code plane
            const int row_bytes = D / 2;
            const int rr = (int) (byte0 / row_bytes), i = (int) (byte0 % row_bytes);
            const int mat = rr >= F ? 1 : 0, r = rr - mat * F;
            uint64_t q = 0;
            for (int k = 0; k < 8; ++k)
                q |= (uint64_t) wzy_expert_code_byte(seed, layer, expert, mat, r, i + k, row_bytes) << (8 * k);
            *(uint64_t*) (rec + gu_codes + byte0) = q;
        } else if (w < n_gu_q + n_dn_q) {
            const size_t byte0 = (w - n_gu_q) * 8;
            const int row_bytes = F / 2;
            const int r = (int) (byte0 / row_bytes), i = (int) (byte0 % row_bytes);
            uint64_t q = 0;
            for (int k = 0; k < 8; ++k)
                q |= (uint64_t) wzy_expert_code_byte(seed, layer, expert, 2, r, i + k, row_bytes) << (8 * k);
            *(uint64_t*) (rec + dn_codes + byte0) = q;
        } else if (w < n_gu_q + n_dn_q + n_gu_s) {
            const size_t s = w - n_gu_q - n_dn_q;
            const int row_subs = D / 16;
            const int rr = (int) (s / row_subs), sb = (int) (s % row_subs);
            const int mat = rr >= F ? 1 : 0, r = rr - mat * F;
            rec[gu_scales + s] = wzy_expert_scale_byte(seed, layer, expert, mat, r, sb, row_subs);
        } else {
            const size_t s = w - n_gu_q - n_dn_q - n_gu_s;
            const int row_subs = F / 16;
            rec[dn_scales + s] = wzy_expert_scale_byte(seed, layer, expert, 2, (int) (s / row_subs), (int) (s % row_subs), row_subs);
        }
    }
    if (blockIdx.x == 0 && threadIdx.x < 4) {
        float* t = (float*) (rec + tail);
        t[threadIdx.x] = threadIdx.x < 3 ? 1.0f : 0.0f;
    }
}

extern "C" int wzy_synth_experts_device(uint64_t seed, int layer, int first_expert, int n_experts, int n_embd,
                                        int n_ff, uint8_t* dev, void* stream) {
    WZY_REQUIRE(dev && n_experts > 0, "wzy_synth_experts_device: bad arguments");
    WZY_REQUIRE(n_embd % 64 == 0 && n_ff % 64 == 0, "wzy_synth_experts_device: dims must be multiples of 64");
    WZY_REQUIRE(n_experts <= 65535, "wzy_synth_experts_device: too many experts per call");
    const size_t rec = wzy_nvfp4_expert_bytes(n_embd, n_ff);
    hipLaunchKernelGGL(synth_expert_kernel, dim3(512, n_experts), dim3(256), 0, as_stream(stream), seed, layer,
                       first_expert, n_embd, n_ff, rec, dev);
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

// ---------------------------------------------------------------------------------------------
// MTP Q2_0 experts
// ---------------------------------------------------------------------------------------------
extern "C" size_t wzy_q2_expert_bytes(int n_embd, int n_ff) {
    return (size_t) 3 * n_embd * n_ff / 4 + (size_t) 3 * n_embd * n_ff / 64 * 2;
}

// byte `i` of a Q2_0 blob of (D, F)
WZY_HD uint8_t q2_blob_byte(uint64_t seed, int expert, int D, int F, size_t i) {
    const size_t n_gu_c = (size_t) 2 * F * (D / 4), n_dn_c = (size_t) D * (F / 4), n_gu_s = (size_t) 2 * F * (D / 64);
    if (i < n_gu_c) return wzy_q2_code_byte(seed, expert, 0, i);
    if (i < n_gu_c + n_dn_c) return wzy_q2_code_byte(seed, expert, 1, i - n_gu_c);
    size_t j = i - n_gu_c - n_dn_c;
    const int part = j < n_gu_s * 2 ? 2 : 3;
    if (part == 3) j -= n_gu_s * 2;
    const uint16_t h = wzy_q2_scale_h16(seed, expert, part, j >> 1, wzy_q2_scale_exp(part == 2 ? D : F));
    return (uint8_t) (h >> (8 * (j & 1)));
}

extern "C" int wzy_synth_q2_expert(uint64_t seed, int expert, int n_embd, int n_ff, uint8_t* blob) {
    WZY_REQUIRE(blob && n_embd % 64 == 0 && n_ff % 64 == 0, "wzy_synth_q2_expert: bad arguments");
    const size_t n = wzy_q2_expert_bytes(n_embd, n_ff);
    for (size_t i = 0; i < n; ++i) blob[i] = q2_blob_byte(seed, expert, n_embd, n_ff, i);
    return WZY_OK;
}

__global__ void synth_q2_kernel(uint64_t seed, int first_expert, int D, int F, size_t rec, uint8_t* __restrict__ dev) {
    const int e = blockIdx.y;
    uint8_t* out = dev + (size_t) e * rec;
    for (size_t w = (size_t) blockIdx.x * blockDim.x + threadIdx.x; w < rec / 8; w += (size_t) gridDim.x * blockDim.x) {
        uint64_t q = 0;
        for (int k = 0; k < 8; ++k) q |= (uint64_t) q2_blob_byte(seed, first_expert + e, D, F, w * 8 + k) << (8 * k);
        *(uint64_t*) (out + w * 8) = q;
    }
}

extern "C" int wzy_synth_q2_experts_device(uint64_t seed, int first_expert, int n_experts, int n_embd, int n_ff,
                                           uint8_t* dev, void* stream) {
    WZY_REQUIRE(dev && n_experts > 0 && n_experts <= 65535, "wzy_synth_q2_experts_device: bad arguments");
    WZY_REQUIRE(n_embd % 64 == 0 && n_ff % 64 == 0, "wzy_synth_q2_experts_device: dims must be multiples of 64");
    hipLaunchKernelGGL(synth_q2_kernel, dim3(256, n_experts), dim3(256), 0, as_stream(stream), seed, first_expert,
                       n_embd, n_ff, wzy_q2_expert_bytes(n_embd, n_ff), dev);
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

// ---------------------------------------------------------------------------------------------
// INT8 KV cells
// ---------------------------------------------------------------------------------------------
extern "C" void wzy_synth_kv_host(uint64_t seed, int layer, int is_v, int64_t first_pos, int n_cells, int kvd,
                                  int8_t* codes, uint16_t* scales) {
    const int groups = kvd / 64;
    parallel_for((size_t) n_cells, [&](size_t b, size_t e) {
        for (size_t c = b; c < e; ++c) {
            const int64_t pos = first_pos + (int64_t) c;
            for (int i = 0; i < kvd; ++i) codes[c * kvd + i] = wzy_kv_code(seed, layer, is_v, pos, i, kvd);
            for (int g = 0; g < groups; ++g) scales[c * groups + g] = wzy_kv_scale_h16(seed, layer, is_v, pos, g, groups);
        }
    });
}

__global__ void synth_kv_kernel(uint64_t seed, int layer, int is_v, int64_t first_pos, int n_cells, int kvd,
                                int8_t* __restrict__ codes, uint16_t* __restrict__ scales) {
    const int groups = kvd / 64;
    const size_t total = (size_t) n_cells * kvd;
    for (size_t w = (size_t) blockIdx.x * blockDim.x + threadIdx.x; w < total; w += (size_t) gridDim.x * blockDim.x) {
        const size_t c = w / kvd;
        const int i = (int) (w % kvd);
        const int64_t pos = first_pos + (int64_t) c;
        codes[w] = wzy_kv_code(seed, layer, is_v, pos, i, kvd);
        if ((i & 63) == 0) scales[c * groups + i / 64] = wzy_kv_scale_h16(seed, layer, is_v, pos, i / 64, groups);
    }
}

extern "C" int wzy_synth_kv_device(uint64_t seed, int layer, int is_v, int64_t first_pos, int n_cells, int kvd,
                                   int8_t* codes, uint16_t* scales, void* stream) {
    WZY_REQUIRE(codes && scales && n_cells >= 0 && kvd % 64 == 0, "wzy_synth_kv_device: bad arguments");
    if (n_cells == 0) return WZY_OK;
    hipLaunchKernelGGL(synth_kv_kernel, dim3(1024), dim3(256), 0, as_stream(stream), seed, layer, is_v, first_pos,
                       n_cells, kvd, codes, scales);
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

// ple.hip -- per-layer embedding (PLE) at layer 1 for gfx950: hashed 3-gram rows of an fp8 table held
// in HBM, and the block that mixes them into the four hyper-connection streams.
//
//  ple_rows   workgroup (head, row): the head's table row of the row's (token, previous token,
//             token before) context, decoded fp8 * scale.  The previous tokens come from the window or
//             from the per-position token history the stage keeps in HBM, so the lookup needs no
//             host round trip.  reference: stage_ple_window / PleSrc (src/wzy_engine_v2.cu:909-978,
//             src/wzy_stage_v2.cuh:215-324), whose rows the host gathers from an mmap-ed file.
//  ple_mix    workgroup (stream, row): pending fold, the three group RMSNorms, the k . q gate and
//             gat = v * gate (ple_group_multi, ple_gate_gv_multi, src/wzy_kernels_v2.cuh:1299-1346).
//  ple_conv   thread per stream channel, rows in order: 4-tap conv over the channel's history of
//             normalised gated values at distances 9, 6, 3, 0, SiLU, added to the stream with gat
//             (ple_conv_multi, src/wzy_kernels_v2.cuh:1348-1374).
// The two projections between ple_rows and ple_mix are bf16 GEMVs (decode) or GEMMs (prefill).
#include "../../include/wzy_kernels.h"
#include "../../include/wzy_synth.h"
#include "wzy_device.h"
#include "wzy_gemv.h"
#include "wzy_host.h"
#include "wzy_ple.h"
#include "wzy_synth_impl.h"

using namespace wzy;

namespace {

// hash constants of the reference's lookup (src/wzy_engine_v2.cu:909-915): multipliers per context
// position, and per head a prime row count and the first row of its slice of the table
__constant__ uint64_t c_ple_mult[3] = {23703573157769ull, 20109073645365ull, 8052911324071ull};
__constant__ uint64_t c_ple_vocab[PLE_HEADS] = {
    20000003, 20000023, 20000033, 20000047, 20000059, 20000063, 20000069, 20000077,
    20000081, 20000093, 20000107, 20000147, 20000153, 20000159, 20000161, 20000171};
__constant__ uint64_t c_ple_off[PLE_HEADS] = {
    0, 20000003, 40000026, 60000059, 80000106, 100000165, 120000228, 140000297,
    160000374, 180000455, 200000548, 220000655, 240000802, 260000955, 280001114, 300001275};
constexpr uint64_t PLE_ROWS = 300001275ull + 20000171ull;

WZY_DEV uint16_t ple_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16) f); }   // nearest even

// fp8 code -> float: e4m3 with bias 7, subnormals m * 2^-9, the NaN codes read as 0 (the reference
// table's LUT, src/wzy_stage_v2.cuh:279-286)
WZY_DEV float ple_fp8(uint32_t v) {
    const uint32_t e = (v >> 3) & 15u, m = v & 7u;
    float f;
    if (e == 0) f = (float) m * (1.0f / 512.0f);
    else if (e == 15 && m == 7) f = 0.f;
    else f = __builtin_bit_cast(float, ((e + 120u) << 23) | (m << 20));
    return (v & 0x80u) ? -f : f;
}

__global__ void __launch_bounds__(64) ple_rows_kernel(PleRowsArgs a) {
    const int h = blockIdx.x, t = blockIdx.y, j = threadIdx.x;
    const int p = *a.pos + t;
    if (p < 0 || p >= a.ctx_max) return;
    const int cur = a.toks[t];
    const int p1 = t >= 1 ? a.toks[t - 1] : (p >= 1 ? a.tok_hist[p - 1] : -1);
    const int p2 = t >= 2 ? a.toks[t - 2] : (p >= 2 ? a.tok_hist[p - 2] : -1);
    // context (cur, p1, p2) cut at the first missing or end-of-sequence token, which and everything
    // older read as eos (src/wzy_engine_v2.cu:950-958); heads 0-7 hash the 2-gram, 8-15 the 3-gram
    const bool cut1 = p1 < 0 || p1 == a.eos;
    const int64_t c1 = cut1 ? a.eos : p1;
    const int64_t c2 = (cut1 || p2 < 0 || p2 == a.eos) ? a.eos : p2;
    uint64_t mixed = (uint64_t) (int64_t) cur * c_ple_mult[0] ^ (uint64_t) c1 * c_ple_mult[1];
    if (h >= 8) mixed ^= (uint64_t) c2 * c_ple_mult[2];
    const uint64_t row = mixed % c_ple_vocab[h] + c_ple_off[h];
    const uint8_t* src = a.table + row * (uint64_t) a.head;
    const size_t o = (size_t) t * PLE_HEADS * a.head + (size_t) h * a.head;
    const float scale = a.scale_dev ? *a.scale_dev : a.scale;
    for (int k = j; k < a.head; k += 64) {
        const float v = ple_fp8(src[k]) * scale;
        a.emb[o + k] = v;
        if (a.emb_bf16) a.emb_bf16[o + k] = ple_bf16(v);
    }
    // the window's token at its position; the reads above touch only cells before the window
    if (h == 0 && j == 0) a.tok_hist[p] = cur;
}

constexpr int MIX_VPT = 16;          // values per thread: D <= 16 * 256

__global__ void __launch_bounds__(256) ple_mix_kernel(PleBlockArgs a) {
    __shared__ float s_red[4];
    const int c = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
    const int D = a.D, HC = a.HC;
    const size_t HCD = (size_t) HC * D;
    float* Rc = a.R + (size_t) t * HCD + (size_t) c * D;
    const float* kc = a.k + (size_t) t * HCD + (size_t) c * D;
    const float* vt = a.v + (size_t) t * D;
    const float* nq = a.norm_q + (size_t) c * D;
    const float* nk = a.norm_k + (size_t) c * D;
    const float* nc = a.norm_c + (size_t) c * D;
    float r[MIX_VPT], kv[MIX_VPT], vv[MIX_VPT];
    const float gf = a.bo ? 2.0f / (1.0f + __expf(-a.inj_prev[(size_t) t * HC + c] / (float) HC)) : 0.f;
#pragma unroll
    for (int i = 0; i < MIX_VPT; ++i) {
        const int d = tid + 256 * i;
        const bool in = d < D;
        r[i] = in ? Rc[d] : 0.f;
        kv[i] = in ? kc[d] : 0.f;
        vv[i] = in ? vt[d] : 0.f;
        if (a.bo && in) r[i] = fmaf(a.bo[(size_t) t * D + d], gf, r[i]);
    }
    float ssr = 0.f, ssk = 0.f;
#pragma unroll
    for (int i = 0; i < MIX_VPT; ++i) {
        ssr = fmaf(r[i], r[i], ssr);
        ssk = fmaf(kv[i], kv[i], ssk);
        const int d = tid + 256 * i;
        if (a.bo && d < D) Rc[d] = r[i];                       // the folded stream, for the conv's adds
    }
    ssr = block_sum<4>(ssr, s_red);
    ssk = block_sum<4>(ssk, s_red);
    const float rr = 1.0f / sqrtf(ssr / (float) D + a.eps), rk = 1.0f / sqrtf(ssk / (float) D + a.eps);
    float dot = 0.f;
#pragma unroll
    for (int i = 0; i < MIX_VPT; ++i) {
        const int d = tid + 256 * i;
        if (d < D) dot = fmaf(kv[i] * rk * nk[d], r[i] * rr * nq[d], dot);
    }
    dot = block_sum<4>(dot, s_red);
    const float s = dot / sqrtf((float) D);
    const float sg = s < 0.f ? -1.f : 1.f;
    const float g = 1.0f / (1.0f + __expf(-sg * sqrtf(fmaxf(fabsf(s), 1e-6f))));
    float ssg = 0.f;
#pragma unroll
    for (int i = 0; i < MIX_VPT; ++i) {
        vv[i] *= g;
        ssg = fmaf(vv[i], vv[i], ssg);
    }
    ssg = block_sum<4>(ssg, s_red);
    const float rg = 1.0f / sqrtf(ssg / (float) D + a.eps);
    float* gat = a.gat + (size_t) t * HCD + (size_t) c * D;
    float* n = a.n + (size_t) t * HCD + (size_t) c * D;
#pragma unroll
    for (int i = 0; i < MIX_VPT; ++i) {
        const int d = tid + 256 * i;
        if (d < D) {
            gat[d] = vv[i];
            n[d] = vv[i] * rg * nc[d];
        }
    }
}

__global__ void __launch_bounds__(256) ple_conv_kernel(PleBlockArgs a, int T) {
    const size_t HCD = (size_t) a.HC * a.D;
    const size_t ch = (size_t) blockIdx.x * 256 + threadIdx.x;
    if (ch >= HCD) return;
    float h[PLE_HIST];
#pragma unroll
    for (int i = 0; i < PLE_HIST; ++i) h[i] = a.hist[ch * PLE_HIST + i];
    const float4 w = *(const float4*) (a.conv_w + ch * 4);
    for (int t = 0; t < T; ++t) {
        const float cur = a.n[(size_t) t * HCD + ch];
        const float acc = w.x * h[0] + w.y * h[3] + w.z * h[6] + w.w * cur;
#pragma unroll
        for (int i = 0; i < PLE_HIST - 1; ++i) h[i] = h[i + 1];
        h[PLE_HIST - 1] = cur;
        a.R[(size_t) t * HCD + ch] += a.gat[(size_t) t * HCD + ch] + acc / (1.0f + __expf(-acc));
        if (a.hist_snaps) {
#pragma unroll
            for (int i = 0; i < PLE_HIST; ++i) a.hist_snaps[((size_t) t * HCD + ch) * PLE_HIST + i] = h[i];
        }
    }
#pragma unroll
    for (int i = 0; i < PLE_HIST; ++i) a.hist[ch * PLE_HIST + i] = h[i];
}

__global__ void synth_ple_kernel(uint64_t seed, uint8_t* table, uint64_t rows, int head) {
    const uint64_t n = rows * (uint64_t) head;
    for (uint64_t i = (uint64_t) blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t) gridDim.x * blockDim.x)
        table[i] = wzy_ple_code(seed, i / (uint64_t) head, head, (int) (i % (uint64_t) head));
}

}  // namespace

namespace wzy {

uint64_t ple_table_rows() { return PLE_ROWS; }

int launch_ple_rows(const PleRowsArgs& a, int T, hipStream_t st) {
    WZY_REQUIRE(a.table && a.pos && a.toks && a.tok_hist && a.emb, "ple_rows: null pointer");
    WZY_REQUIRE(a.head >= 1 && a.head <= 256 && T >= 1 && T <= 65535, "ple_rows: head %d / rows %d", a.head, T);
    hipLaunchKernelGGL(ple_rows_kernel, dim3(PLE_HEADS, T), dim3(64), 0, st, a);
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

int launch_ple_mix(const PleBlockArgs& a, int T, hipStream_t st) {
    WZY_REQUIRE(a.R && a.k && a.v && a.norm_q && a.norm_k && a.norm_c && a.gat && a.n && (!a.bo || a.inj_prev),
                "ple_mix: null pointer");
    WZY_REQUIRE(a.D >= 16 && a.D <= 256 * MIX_VPT && a.HC >= 1 && T >= 1 && T <= 65535, "ple_mix: D %d HC %d", a.D,
                a.HC);
    hipLaunchKernelGGL(ple_mix_kernel, dim3(a.HC, T), dim3(256), 0, st, a);
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

int launch_ple_conv(const PleBlockArgs& a, int T, hipStream_t st) {
    WZY_REQUIRE(a.R && a.conv_w && a.hist && a.gat && a.n, "ple_conv: null pointer");
    const size_t HCD = (size_t) a.HC * a.D;
    hipLaunchKernelGGL(ple_conv_kernel, dim3((unsigned) ((HCD + 255) / 256)), dim3(256), 0, st, a, T);
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

}  // namespace wzy

// ---------------------------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------------------------
extern "C" uint64_t wzy_ple_table_rows(void) { return PLE_ROWS; }

extern "C" int wzy_ple_rows(const uint8_t* table, int head_bytes, float scale, int eos, const int* pos,
                            const int* toks, int T, int* tok_hist, int ctx_max, float* emb, uint16_t* emb_bf16,
                            void* stream) {
    PleRowsArgs a{};
    a.table = table; a.head = head_bytes; a.scale = scale; a.eos = eos; a.pos = pos; a.toks = toks;
    a.tok_hist = tok_hist; a.ctx_max = ctx_max; a.emb = emb; a.emb_bf16 = emb_bf16;
    return launch_ple_rows(a, T, as_stream(stream));
}

extern "C" size_t wzy_ple_workspace_bytes(int n_embd, int hc, int T) {
    const size_t HCD = (size_t) hc * n_embd;
    return ((size_t) T * (3 * HCD + n_embd)) * sizeof(float) + 256;
}

extern "C" int wzy_ple_block(float* R, const float* bo, const float* inj_prev, const float* emb, const uint16_t* wk,
                             const uint16_t* wv, const float* norm_q, const float* norm_k, const float* norm_c,
                             const float* conv_w, float* hist, int n_embd, int hc, float eps, int T,
                             float* hist_snaps, void* workspace, size_t workspace_bytes, void* stream) {
    WZY_REQUIRE(R && emb && wk && wv && workspace, "wzy_ple_block: null pointer");
    WZY_REQUIRE(T >= 1 && T <= WZY_MAX_W, "wzy_ple_block: T %d out of range", T);
    WZY_REQUIRE(n_embd % 32 == 0 && n_embd <= 8192, "wzy_ple_block: n_embd %d", n_embd);
    WZY_REQUIRE(workspace_bytes >= wzy_ple_workspace_bytes(n_embd, hc, T), "wzy_ple_block: workspace too small");
    hipStream_t st = as_stream(stream);
    const size_t HCD = (size_t) hc * n_embd;
    float* k = (float*) workspace;
    float* gat = k + (size_t) T * HCD;
    float* n = gat + (size_t) T * HCD;
    float* v = n + (size_t) T * HCD;
    GemvSegs s;
    s.n = 2;
    s.seg[0] = GemvSeg{wk, nullptr, k, (int) HCD, GEMV_BF16, (int) HCD, 0};
    s.seg[1] = GemvSeg{wv, nullptr, v, n_embd, GEMV_BF16, n_embd, 0};
    WZY_TRY(launch_gemv_segs(s, emb, n_embd, T, st));
    PleBlockArgs a{};
    a.R = R; a.bo = bo; a.inj_prev = inj_prev; a.k = k; a.v = v; a.norm_q = norm_q; a.norm_k = norm_k;
    a.norm_c = norm_c; a.conv_w = conv_w; a.hist = hist; a.hist_snaps = hist_snaps; a.gat = gat; a.n = n;
    a.D = n_embd; a.HC = hc; a.eps = eps;
    WZY_TRY(launch_ple_mix(a, T, st));
    return launch_ple_conv(a, T, st);
}

extern "C" void wzy_synth_ple_row(uint64_t seed, uint64_t row, int head_bytes, uint8_t* out) {
    for (int j = 0; j < head_bytes; ++j) out[j] = wzy_ple_code(seed, row, head_bytes, j);
}

extern "C" int wzy_synth_ple_table_device(uint64_t seed, int head_bytes, uint8_t* table, void* stream) {
    WZY_REQUIRE(table && head_bytes >= 1 && head_bytes <= 256, "wzy_synth_ple_table_device: bad arguments");
    hipLaunchKernelGGL(synth_ple_kernel, dim3(8192), dim3(256), 0, as_stream(stream), seed, table, PLE_ROWS,
                       head_bytes);
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

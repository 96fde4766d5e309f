// loader.hip -- real-weight loaders (host code only): a bounds-checked GGUF reader over mmap, the
// element conversions of the reference's uploaders, the GGUF -> stage tensor table, the NVFP4
// expert pack, and the MTP drafter files.  C ABI in include/wzy_loader.h.
//
// reference: Gguf::open and the up_* uploaders (src/wzy_stage_v2.cuh:30-179),
// init_stage_weights_and_state (src/wzy_engine_v2.cu:310-378,542-556), the experts.bin mapping
// (src/wzy_engine_v2.cu:693-734,780-787), stage_one_emb (src/wzy_engine_v2.cu:802-873),
// MtpEngine::init (src/wzy_mtp.cuh:462-560).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <sstream>
#include <string>
#include <vector>

#include "../../include/wzy_loader.h"
#include "../../include/wzy_synth.h"
#include "wzy_host.h"
#include "wzy_stage_int.h"

using namespace wzy;

// ------------------------------------------------------------------------------------------------
// GGUF reader
// ------------------------------------------------------------------------------------------------
namespace {
enum : uint32_t {
    KV_U8 = 0, KV_I8 = 1, KV_U16 = 2, KV_I16 = 3, KV_U32 = 4, KV_I32 = 5, KV_F32 = 6, KV_BOOL = 7,
    KV_STR = 8, KV_ARR = 9, KV_U64 = 10, KV_I64 = 11, KV_F64 = 12
};
size_t kv_scalar_bytes(uint32_t t) {
    switch (t) {
        case KV_U8: case KV_I8: case KV_BOOL: return 1;
        case KV_U16: case KV_I16: return 2;
        case KV_U32: case KV_I32: case KV_F32: return 4;
        case KV_U64: case KV_I64: case KV_F64: return 8;
        default: return 0;
    }
}
// bytes of n elements of a tensor type the loaders read (0: not read)
size_t type_bytes(int type, uint64_t n) {
    switch (type) {
        case WZY_GGUF_F32: return n * 4;
        case WZY_GGUF_F16: case WZY_GGUF_BF16: return n * 2;
        case WZY_GGUF_Q8_0: return n % 32 ? 0 : n / 32 * 34;
        case WZY_GGUF_I8: return n;
        default: return 0;
    }
}
struct KvEnt { uint32_t type; size_t off; };          // value offset in the file
struct TensorEnt { std::string name; int n_dims; int64_t dims[4]; int type; uint64_t off; size_t bytes; };

// sequential reader with bounds checks
struct Cursor {
    const uint8_t* p; size_t size, at = 0; bool bad = false;
    bool need(size_t n) { if (bad || n > size - at) { bad = true; return false; } return true; }
    template <class T> T get() {
        T v{};
        if (need(sizeof(T))) { memcpy(&v, p + at, sizeof(T)); at += sizeof(T); }
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (bad || !need(n)) return std::string();
        std::string s((const char*) p + at, (size_t) n);
        at += n;
        return s;
    }
    void skip_value(uint32_t t, int depth = 0) {
        if (t == KV_STR) { const uint64_t n = get<uint64_t>(); if (need(n)) at += n; return; }
        if (t == KV_ARR) {
            const uint32_t et = get<uint32_t>();
            const uint64_t n = get<uint64_t>();
            if (depth > 2) { bad = true; return; }
            const size_t sb = kv_scalar_bytes(et);
            if (sb) { if (n > (size - at) / sb) bad = true; else at += n * sb; return; }
            for (uint64_t i = 0; i < n && !bad; ++i) skip_value(et, depth + 1);
            return;
        }
        const size_t sb = kv_scalar_bytes(t);
        if (!sb) { bad = true; return; }
        if (need(sb)) at += sb;
    }
};
}  // namespace

struct wzy_gguf {
    const uint8_t* base = nullptr;
    size_t size = 0;
    std::map<std::string, KvEnt> kv;
    std::vector<TensorEnt> ts;
    std::map<std::string, int> idx;
    ~wzy_gguf() { if (base) munmap((void*) base, size); }
};

extern "C" int wzy_gguf_open(const char* path, wzy_gguf** out) {
    WZY_REQUIRE(path && out, "gguf: null argument");
    *out = nullptr;
    const int fd = ::open(path, O_RDONLY);
    if (fd < 0) { set_error("gguf: cannot open %s", path); return WZY_EIO; }
    struct stat sb;
    if (fstat(fd, &sb) != 0 || sb.st_size < 24) { ::close(fd); set_error("gguf: %s is not a GGUF file", path); return WZY_EIO; }
    void* m = mmap(nullptr, (size_t) sb.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (m == MAP_FAILED) { set_error("gguf: cannot map %s", path); return WZY_EIO; }
    std::unique_ptr<wzy_gguf> g(new wzy_gguf);
    g->base = (const uint8_t*) m;
    g->size = (size_t) sb.st_size;
    Cursor c{g->base, g->size};
    if (memcmp(g->base, "GGUF", 4) != 0) { set_error("gguf: %s: bad magic", path); return WZY_EIO; }
    c.at = 4;
    const uint32_t version = c.get<uint32_t>();
    if (version != 2 && version != 3) { set_error("gguf: %s: version %u not supported", path, version); return WZY_EIO; }
    const uint64_t nt = c.get<uint64_t>(), nkv = c.get<uint64_t>();
    if (nt > (1u << 24) || nkv > (1u << 24)) { set_error("gguf: %s: implausible header counts", path); return WZY_EIO; }
    for (uint64_t i = 0; i < nkv && !c.bad; ++i) {
        std::string key = c.str();
        const uint32_t t = c.get<uint32_t>();
        g->kv[key] = KvEnt{t, c.at};
        c.skip_value(t);
    }
    g->ts.resize(nt);
    for (uint64_t i = 0; i < nt && !c.bad; ++i) {
        TensorEnt& t = g->ts[i];
        t.name = c.str();
        const uint32_t nd = c.get<uint32_t>();
        if (nd < 1 || nd > 4) { c.bad = true; break; }
        t.n_dims = (int) nd;
        uint64_t n = 1;
        for (int d = 0; d < 4; ++d) {
            t.dims[d] = d < (int) nd ? (int64_t) c.get<uint64_t>() : 1;
            // each dimension and the element count are bounded (2^48 elements is far past any
            // tensor a file of this size holds), so the product cannot wrap
            if (t.dims[d] < 1 || t.dims[d] > (int64_t) 1 << 40 || __builtin_mul_overflow(n, (uint64_t) t.dims[d], &n) ||
                n > (uint64_t) 1 << 48)
                c.bad = true;
        }
        t.type = (int) c.get<uint32_t>();
        t.off = c.get<uint64_t>();
        t.bytes = c.bad ? 0 : type_bytes(t.type, n);
    }
    if (c.bad) { set_error("gguf: %s: truncated or malformed header", path); return WZY_EIO; }
    uint64_t align = 32;                                  // general.alignment, GGUF's default 32
    auto al = g->kv.find("general.alignment");
    if (al != g->kv.end() && al->second.type == KV_U32) {
        uint32_t a;
        memcpy(&a, g->base + al->second.off, 4);
        if (a == 0 || (a & (a - 1))) { set_error("gguf: %s: bad alignment %u", path, a); return WZY_EIO; }
        align = a;
    }
    const uint64_t data = (c.at + align - 1) / align * align;
    for (size_t i = 0; i < g->ts.size(); ++i) {
        TensorEnt& t = g->ts[i];
        if (t.off > g->size || data > g->size - t.off || t.bytes > g->size - data - t.off) {
            set_error("gguf: %s: tensor %s lies outside the file", path, t.name.c_str());
            return WZY_EIO;
        }
        t.off += data;
        g->idx[t.name] = (int) i;
    }
    *out = g.release();
    return WZY_OK;
}

extern "C" void wzy_gguf_close(wzy_gguf* g) { delete g; }
extern "C" int wzy_gguf_n_tensors(const wzy_gguf* g) { return g ? (int) g->ts.size() : 0; }
extern "C" int wzy_gguf_find(const wzy_gguf* g, const char* name) {
    if (!g || !name) return -1;
    auto it = g->idx.find(name);
    return it == g->idx.end() ? -1 : it->second;
}
extern "C" int wzy_gguf_tensor_info(const wzy_gguf* g, int i, const char** name, int* n_dims, int64_t dims[4],
                                    int* type, size_t* bytes) {
    WZY_REQUIRE(g && i >= 0 && i < (int) g->ts.size(), "gguf: tensor index %d out of range", i);
    const TensorEnt& t = g->ts[i];
    if (name) *name = t.name.c_str();
    if (n_dims) *n_dims = t.n_dims;
    if (dims) for (int d = 0; d < 4; ++d) dims[d] = t.dims[d];
    if (type) *type = t.type;
    if (bytes) *bytes = t.bytes;
    return WZY_OK;
}
extern "C" const void* wzy_gguf_tensor_data(const wzy_gguf* g, int i) {
    if (!g || i < 0 || i >= (int) g->ts.size()) return nullptr;
    return g->base + g->ts[i].off;
}
extern "C" int wzy_gguf_get_int(const wzy_gguf* g, const char* key, int64_t* out) {
    WZY_REQUIRE(g && key && out, "gguf: null argument");
    auto it = g->kv.find(key);
    WZY_REQUIRE(it != g->kv.end(), "gguf: no key %s", key);
    const uint8_t* p = g->base + it->second.off;
    switch (it->second.type) {
        case KV_U8: case KV_BOOL: *out = *p; return WZY_OK;
        case KV_I8: *out = (int8_t) *p; return WZY_OK;
        case KV_U16: { uint16_t v; memcpy(&v, p, 2); *out = v; return WZY_OK; }
        case KV_I16: { int16_t v; memcpy(&v, p, 2); *out = v; return WZY_OK; }
        case KV_U32: { uint32_t v; memcpy(&v, p, 4); *out = v; return WZY_OK; }
        case KV_I32: { int32_t v; memcpy(&v, p, 4); *out = v; return WZY_OK; }
        case KV_U64: { uint64_t v; memcpy(&v, p, 8); *out = (int64_t) v; return WZY_OK; }
        case KV_I64: { int64_t v; memcpy(&v, p, 8); *out = v; return WZY_OK; }
        default: break;
    }
    WZY_REQUIRE(false, "gguf: key %s is not an integer", key);
}
extern "C" int wzy_gguf_get_float(const wzy_gguf* g, const char* key, double* out) {
    WZY_REQUIRE(g && key && out, "gguf: null argument");
    auto it = g->kv.find(key);
    WZY_REQUIRE(it != g->kv.end(), "gguf: no key %s", key);
    const uint8_t* p = g->base + it->second.off;
    if (it->second.type == KV_F32) { float v; memcpy(&v, p, 4); *out = v; return WZY_OK; }
    if (it->second.type == KV_F64) { double v; memcpy(&v, p, 8); *out = v; return WZY_OK; }
    int64_t i;
    WZY_TRY(wzy_gguf_get_int(g, key, &i));
    *out = (double) i;
    return WZY_OK;
}
extern "C" int wzy_gguf_get_str(const wzy_gguf* g, const char* key, const char** str, size_t* len) {
    WZY_REQUIRE(g && key && str && len, "gguf: null argument");
    auto it = g->kv.find(key);
    WZY_REQUIRE(it != g->kv.end() && it->second.type == KV_STR, "gguf: no string key %s", key);
    uint64_t n;
    memcpy(&n, g->base + it->second.off, 8);
    *str = (const char*) g->base + it->second.off + 8;
    *len = (size_t) n;
    return WZY_OK;
}

// ------------------------------------------------------------------------------------------------
// element conversions
// ------------------------------------------------------------------------------------------------
static float h2f(uint16_t h) { return (float) __builtin_bit_cast(_Float16, h); }
static uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16) f); }
static float bf2f(uint16_t b) { return __builtin_bit_cast(float, (uint32_t) b << 16); }

extern "C" void wzy_q8_0_split(const void* blocks, size_t n_blocks, int8_t* codes, uint16_t* scales) {
    const uint8_t* b = (const uint8_t*) blocks;
    for (size_t i = 0; i < n_blocks; ++i) {
        memcpy(&scales[i], b + i * 34, 2);
        memcpy(codes + i * 32, b + i * 34 + 2, 32);
    }
}

extern "C" void wzy_bf16_to_q8_0(const uint16_t* src, size_t n_blocks, int8_t* codes, uint16_t* scales) {
    for (size_t i = 0; i < n_blocks; ++i) {
        float v[32], amax = 0.f;
        for (int j = 0; j < 32; ++j) {
            v[j] = bf2f(src[i * 32 + j]);
            amax = fmaxf(amax, fabsf(v[j]));
        }
        const uint16_t sh = f2h(amax / 127.0f);
        const float d = h2f(sh);
        for (int j = 0; j < 32; ++j) {
            int q = 0;
            if (d > 0.f) {
                const float r = nearbyintf(v[j] / d);         // round half to even
                q = r > 127.f ? 127 : (r < -127.f ? -127 : (int) r);
            }
            codes[i * 32 + j] = (int8_t) q;
        }
        scales[i] = sh;
    }
}

extern "C" void wzy_bf16_from_f32(const float* src, size_t n, uint16_t* dst) {
    for (size_t i = 0; i < n; ++i) {
        const uint32_t u = __builtin_bit_cast(uint32_t, src[i]);
        dst[i] = (uint16_t) ((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
    }
}

extern "C" int wzy_to_f32(int type, const void* src, size_t n, float* dst) {
    WZY_REQUIRE(src && dst, "to_f32: null pointer");
    switch (type) {
        case WZY_GGUF_F32: memcpy(dst, src, n * 4); return WZY_OK;
        case WZY_GGUF_F16: for (size_t i = 0; i < n; ++i) dst[i] = h2f(((const uint16_t*) src)[i]); return WZY_OK;
        case WZY_GGUF_BF16: for (size_t i = 0; i < n; ++i) dst[i] = bf2f(((const uint16_t*) src)[i]); return WZY_OK;
        case WZY_GGUF_Q8_0: {
            WZY_REQUIRE(n % 32 == 0, "to_f32: Q8_0 needs a multiple of 32 values");
            const uint8_t* b = (const uint8_t*) src;
            for (size_t blk = 0; blk < n / 32; ++blk) {
                uint16_t s;
                memcpy(&s, b + blk * 34, 2);
                const float d = h2f(s);
                for (int j = 0; j < 32; ++j) dst[blk * 32 + j] = d * (float) (int8_t) b[blk * 34 + 2 + j];
            }
            return WZY_OK;
        }
        default: break;
    }
    WZY_REQUIRE(false, "to_f32: tensor type %d not supported", type);
}

// ------------------------------------------------------------------------------------------------
// stage configuration from the tensor shapes
// ------------------------------------------------------------------------------------------------
namespace {
struct Gg {                                           // closes on scope exit
    wzy_gguf* g = nullptr;
    ~Gg() { wzy_gguf_close(g); }
};
const TensorEnt* find_t(const wzy_gguf* g, const std::string& n) {
    auto it = g->idx.find(n);
    return it == g->idx.end() ? nullptr : &g->ts[it->second];
}
std::string blk(int l, const char* suffix) { return "blk." + std::to_string(l) + "." + suffix; }
// rows x cols of a tensor (dims[0] contiguous); 0 x 0 if absent or of more than two dimensions
void shape2(const TensorEnt* t, int64_t& rows, int64_t& cols) {
    rows = cols = 0;
    if (!t || t->dims[2] != 1 || t->dims[3] != 1) return;
    cols = t->dims[0];
    rows = t->dims[1];
}
int64_t numel(const TensorEnt* t) { return t ? t->dims[0] * t->dims[1] * t->dims[2] * t->dims[3] : 0; }
}  // namespace

extern "C" int wzy_stage_cfg_from_gguf(const char* gguf_path, int ctx_max, wzy_stage_cfg* cfg) {
    WZY_REQUIRE(gguf_path && cfg, "cfg_from_gguf: null argument");
    Gg h;
    WZY_TRY(wzy_gguf_open(gguf_path, &h.g));
    const wzy_gguf* g = h.g;
    wzy_stage_cfg_default(cfg, ctx_max);
    // layers: every blk.N carries a router; QSA layers carry attn_q
    int nl = 0;
    while (find_t(g, blk(nl, "ffn_gate_inp.weight"))) ++nl;
    WZY_REQUIRE(nl >= 1, "cfg_from_gguf: no blk.0.ffn_gate_inp.weight");
    int first_qsa = -1, first_gdn = -1;
    for (int l = 0; l < nl; ++l) {
        if (find_t(g, blk(l, "attn_q.weight"))) { if (first_qsa < 0) first_qsa = l; }
        else if (first_gdn < 0) first_gdn = l;
    }
    WZY_REQUIRE(first_qsa >= 0, "cfg_from_gguf: no attention (attn_q) layer");
    const int period = first_qsa + 1;
    for (int l = 0; l < nl; ++l)
        WZY_REQUIRE((find_t(g, blk(l, "attn_q.weight")) != nullptr) == (l % period == period - 1),
                    "cfg_from_gguf: attention layers are not every %d-th layer (layer %d)", period, l);
    cfg->n_layers = nl;
    cfg->qsa_period = period;
    int64_t r, c;
    const TensorEnt* te = find_t(g, "token_embd.weight");
    shape2(te, r, c);
    WZY_REQUIRE(r > 0, "cfg_from_gguf: no 2-D token_embd.weight");
    cfg->n_embd = (int) c;
    cfg->n_vocab = (int) r;
    cfg->emb_q8 = te->type == WZY_GGUF_Q8_0;
    const TensorEnt* out = find_t(g, "output.weight");
    shape2(out, r, c);
    WZY_REQUIRE(r == cfg->n_vocab && c == cfg->n_embd, "cfg_from_gguf: output.weight is not [n_vocab x n_embd]");
    cfg->head_q8 = out->type == WZY_GGUF_Q8_0;
    shape2(find_t(g, blk(0, "hc_attn_down.weight")), r, c);
    WZY_REQUIRE(r > 0 && c % cfg->n_embd == 0, "cfg_from_gguf: bad blk.0.hc_attn_down.weight");
    cfg->hc_lr = (int) r;
    cfg->hc = (int) (c / cfg->n_embd);
    if (first_gdn >= 0) {
        int64_t qkv, gv;
        shape2(find_t(g, blk(first_gdn, "attn_gate.weight")), gv, c);
        shape2(find_t(g, blk(first_gdn, "attn_qkv.weight")), qkv, c);
        WZY_REQUIRE(gv > 0 && gv % 128 == 0 && qkv > gv && (qkv - gv) % 256 == 0,
                    "cfg_from_gguf: GDN projections of layer %d do not give 128-wide heads", first_gdn);
        cfg->gdn_hv = (int) (gv / 128);
        cfg->gdn_hk = (int) ((qkv - gv) / 256);
    }
    const int hd = (int) numel(find_t(g, blk(first_qsa, "attn_q_norm.weight")));
    int64_t q2, kvd, idim, iq;
    shape2(find_t(g, blk(first_qsa, "attn_q.weight")), q2, c);
    shape2(find_t(g, blk(first_qsa, "attn_k.weight")), kvd, c);
    shape2(find_t(g, blk(first_qsa, "indexer.k_proj.weight")), idim, c);
    shape2(find_t(g, blk(first_qsa, "indexer.q_proj.weight")), iq, c);
    WZY_REQUIRE(hd > 0 && q2 % (2 * hd) == 0 && kvd % hd == 0 && idim > 0 && iq % idim == 0,
                "cfg_from_gguf: attention shapes of layer %d are inconsistent", first_qsa);
    cfg->qsa_hd = hd;
    cfg->qsa_qh = (int) (q2 / (2 * hd));
    cfg->qsa_kvh = (int) (kvd / hd);
    cfg->idx_dim = (int) idim;
    cfg->idx_heads = (int) (iq / idim);
    int64_t ne, nff;
    shape2(find_t(g, blk(0, "ffn_gate_inp.weight")), ne, c);
    shape2(find_t(g, blk(0, "ffn_gate_shexp.weight")), nff, c);
    WZY_REQUIRE(ne > 0 && nff > 0, "cfg_from_gguf: no router / shared expert in layer 0");
    cfg->n_exp = (int) ne;
    cfg->n_ff = (int) nff;
    // the per-layer embedding at layer 1 (has_ple, src/wzy_engine_v2.cu:316,493-499)
    cfg->ple = find_t(g, "blk.1.ple_key.weight") != nullptr ? 1 : 0;
    // metadata, where present
    const char* arch = nullptr;
    size_t alen = 0;
    if (wzy_gguf_get_str(g, "general.architecture", &arch, &alen) == WZY_OK) {
        const std::string a(arch, alen);
        int64_t v;
        double f;
        if (wzy_gguf_get_int(g, (a + ".expert_used_count").c_str(), &v) == WZY_OK) cfg->top_k = (int) v;
        if (wzy_gguf_get_int(g, (a + ".rope.dimension_count").c_str(), &v) == WZY_OK) cfg->n_rot = (int) v;
        if (wzy_gguf_get_float(g, (a + ".rope.freq_base").c_str(), &f) == WZY_OK) cfg->rope_theta = (float) f;
        if (wzy_gguf_get_float(g, (a + ".attention.layer_norm_rms_epsilon").c_str(), &f) == WZY_OK)
            cfg->eps = (float) f;
    }
    clear_error();                                    // absent metadata keys are not errors
    return WZY_OK;
}

// ------------------------------------------------------------------------------------------------
// stage weights
// ------------------------------------------------------------------------------------------------
namespace {
enum Conv { C_Q8, C_BF16_Q8, C_BF16, C_F32 };

// One tensor into a stage tensor (layer -1 for model-level ones), converted as the reference's
// uploader for it: C_Q8 up_q8 (Q8_0 blocks split into planes), C_BF16_Q8 up_bf_as_q8, C_BF16 up_bf,
// C_F32 up_f32.  `name` is the stage tensor ("x" for Q8_0 planes "x.q" / "x.s").
int put(wzy_stage* st, int layer, const char* name, const wzy_gguf* g, const TensorEnt* t, const char* src_name,
        Conv conv, int64_t rows, int64_t cols) {
    WZY_REQUIRE(t, "load: missing tensor %s", src_name);
    const int64_t n = numel(t);
    WZY_REQUIRE(n == rows * cols, "load: %s has %lld values, the stage expects %lld x %lld", src_name, (long long) n,
                (long long) rows, (long long) cols);
    const uint8_t* src = g->base + t->off;
    const std::string q = std::string(name) + ".q", s = std::string(name) + ".s";
    switch (conv) {
        case C_Q8: {
            WZY_REQUIRE(t->type == WZY_GGUF_Q8_0, "load: %s must be Q8_0 (type %d)", src_name, t->type);
            std::vector<int8_t> codes((size_t) n);
            std::vector<uint16_t> sc((size_t) n / 32);
            wzy_q8_0_split(src, (size_t) n / 32, codes.data(), sc.data());
            WZY_TRY(wzy_stage_write_tensor(st, layer, q.c_str(), codes.data(), codes.size()));
            return wzy_stage_write_tensor(st, layer, s.c_str(), sc.data(), sc.size() * 2);
        }
        case C_BF16_Q8:
        case C_BF16: {
            std::vector<uint16_t> b((size_t) n);
            if (t->type == WZY_GGUF_BF16) memcpy(b.data(), src, (size_t) n * 2);
            else if (t->type == WZY_GGUF_F32) {
                std::vector<float> f((size_t) n);
                memcpy(f.data(), src, (size_t) n * 4);
                wzy_bf16_from_f32(f.data(), (size_t) n, b.data());
            } else WZY_REQUIRE(false, "load: %s must be bf16 or f32 (type %d)", src_name, t->type);
            if (conv == C_BF16) return wzy_stage_write_tensor(st, layer, name, b.data(), b.size() * 2);
            WZY_REQUIRE(n % 32 == 0, "load: %s is not a whole number of 32-blocks", src_name);
            std::vector<int8_t> codes((size_t) n);
            std::vector<uint16_t> sc((size_t) n / 32);
            wzy_bf16_to_q8_0(b.data(), (size_t) n / 32, codes.data(), sc.data());
            WZY_TRY(wzy_stage_write_tensor(st, layer, q.c_str(), codes.data(), codes.size()));
            return wzy_stage_write_tensor(st, layer, s.c_str(), sc.data(), sc.size() * 2);
        }
        case C_F32: {
            std::vector<float> f((size_t) n);
            WZY_TRY(wzy_to_f32(t->type, src, (size_t) n, f.data()));
            return wzy_stage_write_tensor(st, layer, name, f.data(), f.size() * 4);
        }
    }
    return WZY_OK;
}
int put_gguf(wzy_stage* st, int layer, const char* name, const wzy_gguf* g, const std::string& src_name, Conv conv,
             int64_t rows, int64_t cols) {
    return put(st, layer, name, g, find_t(g, src_name), src_name.c_str(), conv, rows, cols);
}
}  // namespace

extern "C" int wzy_stage_load_gguf(wzy_stage* st, const char* gguf_path, const char* experts_path, const char* emb_path) {
    WZY_REQUIRE(st && gguf_path && experts_path, "load_gguf: null argument");
    const wzy_stage_cfg& c = *stage_cfg(st);
    Gg h;
    WZY_TRY(wzy_gguf_open(gguf_path, &h.g));
    const wzy_gguf* g = h.g;
    WZY_TRY(stage_set_loaded(st, false));
    const int64_t D = c.n_embd, HCD = (int64_t) c.hc * D, L = c.hc_lr;
    const int64_t GV = (int64_t) c.gdn_hv * 128, QKV = (int64_t) c.gdn_hk * 256 + GV;
    const int64_t QD = (int64_t) c.qsa_qh * c.qsa_hd, KVD = (int64_t) c.qsa_kvh * c.qsa_hd;
    char nm[64];
    for (int l = 0; l < c.n_layers; ++l) {
        const bool qsa = (l % c.qsa_period) == c.qsa_period - 1;
        for (int hh = 0; hh < 2; ++hh) {
            const std::string pre = hh == 0 ? "hc_attn_" : "hc_ffn_";
            snprintf(nm, sizeof nm, "hc_norm%d", hh);
            WZY_TRY(put_gguf(st, l, nm, g, blk(l, (pre + "norm.weight").c_str()), C_F32, 1, HCD));
            snprintf(nm, sizeof nm, "hc_down%d", hh);
            WZY_TRY(put_gguf(st, l, nm, g, blk(l, (pre + "down.weight").c_str()), C_BF16_Q8, L, HCD));
            snprintf(nm, sizeof nm, "hc_up%d", hh);
            WZY_TRY(put_gguf(st, l, nm, g, blk(l, (pre + "up.weight").c_str()), C_BF16_Q8, HCD, L));
            snprintf(nm, sizeof nm, "hc_inj%d", hh);
            WZY_TRY(put_gguf(st, l, nm, g, blk(l, (pre + "inject.weight").c_str()), C_BF16, c.hc, HCD));
        }
        if (!qsa) {
            WZY_TRY(put_gguf(st, l, "qkv", g, blk(l, "attn_qkv.weight"), C_Q8, QKV, D));
            WZY_TRY(put_gguf(st, l, "wgate", g, blk(l, "attn_gate.weight"), C_Q8, GV, D));
            WZY_TRY(put_gguf(st, l, "wout", g, blk(l, "ssm_out.weight"), C_Q8, D, GV));
            WZY_TRY(put_gguf(st, l, "alpha", g, blk(l, "ssm_alpha.weight"), C_BF16, c.gdn_hv, D));
            WZY_TRY(put_gguf(st, l, "beta", g, blk(l, "ssm_beta.weight"), C_BF16, c.gdn_hv, D));
            WZY_TRY(put_gguf(st, l, "ssm_a", g, blk(l, "ssm_a"), C_F32, 1, c.gdn_hv));
            WZY_TRY(put_gguf(st, l, "dt_bias", g, blk(l, "ssm_dt.bias"), C_F32, 1, c.gdn_hv));
            WZY_TRY(put_gguf(st, l, "conv1d", g, blk(l, "ssm_conv1d.weight"), C_F32, QKV, 4));
            WZY_TRY(put_gguf(st, l, "ssm_norm", g, blk(l, "ssm_norm.weight"), C_F32, 1, 128));
        } else {
            WZY_TRY(put_gguf(st, l, "wq", g, blk(l, "attn_q.weight"), C_Q8, 2 * QD, D));
            WZY_TRY(put_gguf(st, l, "wk", g, blk(l, "attn_k.weight"), C_Q8, KVD, D));
            WZY_TRY(put_gguf(st, l, "wv", g, blk(l, "attn_v.weight"), C_Q8, KVD, D));
            WZY_TRY(put_gguf(st, l, "wo", g, blk(l, "attn_output.weight"), C_Q8, D, QD));
            WZY_TRY(put_gguf(st, l, "q_norm", g, blk(l, "attn_q_norm.weight"), C_F32, 1, c.qsa_hd));
            WZY_TRY(put_gguf(st, l, "k_norm", g, blk(l, "attn_k_norm.weight"), C_F32, 1, c.qsa_hd));
            WZY_TRY(put_gguf(st, l, "idx_q", g, blk(l, "indexer.q_proj.weight"), C_BF16, (int64_t) c.idx_heads * c.idx_dim, D));
            WZY_TRY(put_gguf(st, l, "idx_k", g, blk(l, "indexer.k_proj.weight"), C_BF16, c.idx_dim, D));
            WZY_TRY(put_gguf(st, l, "idx_qn", g, blk(l, "indexer.q_norm.weight"), C_F32, 1, c.idx_dim));
            WZY_TRY(put_gguf(st, l, "idx_kn", g, blk(l, "indexer.k_norm.weight"), C_F32, 1, c.idx_dim));
        }
        WZY_TRY(put_gguf(st, l, "router", g, blk(l, "ffn_gate_inp.weight"), C_BF16, c.n_exp, D));
        WZY_TRY(put_gguf(st, l, "sgate", g, blk(l, "ffn_gate_inp_shexp.weight"), C_BF16, 1, D));
        WZY_TRY(put_gguf(st, l, "sh_gate", g, blk(l, "ffn_gate_shexp.weight"), C_Q8, c.n_ff, D));
        WZY_TRY(put_gguf(st, l, "sh_up", g, blk(l, "ffn_up_shexp.weight"), C_Q8, c.n_ff, D));
        WZY_TRY(put_gguf(st, l, "sh_down", g, blk(l, "ffn_down_shexp.weight"), C_Q8, D, c.n_ff));
    }
    if (c.ple) {      // layer 1's per-layer embedding block (src/wzy_engine_v2.cu:493-499)
        WZY_TRY(put_gguf(st, 1, "ple_key", g, "blk.1.ple_key.weight", C_BF16, HCD, D));
        WZY_TRY(put_gguf(st, 1, "ple_value", g, "blk.1.ple_value.weight", C_BF16, D, D));
        WZY_TRY(put_gguf(st, 1, "ple_norm_key", g, "blk.1.ple_norm_key.weight", C_F32, 1, HCD));
        WZY_TRY(put_gguf(st, 1, "ple_norm_query", g, "blk.1.ple_norm_query.weight", C_F32, 1, HCD));
        WZY_TRY(put_gguf(st, 1, "ple_norm_conv", g, "blk.1.ple_norm_conv.weight", C_F32, 1, HCD));
        WZY_TRY(put_gguf(st, 1, "ple_conv1d", g, "blk.1.ple_conv1d.weight", C_F32, HCD, 4));
    }
    WZY_TRY(put_gguf(st, -1, "head_norm", g, "output_hc_norm.weight", C_F32, 1, HCD));
    WZY_TRY(put_gguf(st, -1, "head_down", g, "output_hc_down.weight", C_BF16_Q8, L, HCD));
    WZY_TRY(put_gguf(st, -1, "head_up", g, "output_hc_up.weight", C_BF16_Q8, HCD, L));
    WZY_TRY(put_gguf(st, -1, "head", g, "output.weight", c.head_q8 ? C_Q8 : C_BF16, c.n_vocab, D));
    // token embedding: the bf16 side file when given, else the checkpoint's own table
    if (emb_path) {
        WZY_REQUIRE(!c.emb_q8, "load_gguf: a bf16 embedding file needs a stage with emb_q8 = 0");
        Gg he;
        WZY_TRY(wzy_gguf_open(emb_path, &he.g));
        WZY_TRY(put_gguf(st, -1, "emb", he.g, "token_embd.weight", C_BF16, c.n_vocab, D));
    } else {
        WZY_TRY(put_gguf(st, -1, "emb", g, "token_embd.weight", c.emb_q8 ? C_Q8 : C_BF16, c.n_vocab, D));
    }
    // NVFP4 experts: blob (l, e) at (l * n_exp + e) * blob bytes, repacked to the plane layout
    const size_t blob = wzy_nvfp4_blob_bytes(c.n_embd, c.n_ff), rec = wzy_nvfp4_expert_bytes(c.n_embd, c.n_ff);
    const size_t n_blobs = (size_t) c.n_layers * c.n_exp;
    FILE* f = fopen(experts_path, "rb");
    if (!f) { set_error("load_gguf: cannot open %s", experts_path); return WZY_EIO; }
    std::unique_ptr<FILE, int (*)(FILE*)> fc(f, fclose);
    if (fseeko(f, 0, SEEK_END) != 0 || (size_t) ftello(f) < n_blobs * blob) {
        set_error("load_gguf: %s holds fewer than %zu expert blobs of %zu bytes", experts_path, n_blobs, blob);
        return WZY_EIO;
    }
    fseeko(f, 0, SEEK_SET);
    const size_t chunk = 64;
    std::vector<uint8_t> in(chunk * blob), outp(chunk * rec);
    for (size_t b0 = 0; b0 < n_blobs; b0 += chunk) {
        const size_t nb = std::min(chunk, n_blobs - b0);
        if (fread(in.data(), blob, nb, f) != nb) { set_error("load_gguf: short read of %s", experts_path); return WZY_EIO; }
        for (size_t i = 0; i < nb; ++i)
            WZY_TRY(wzy_nvfp4_repack_host(in.data() + i * blob, outp.data() + i * rec, c.n_embd, c.n_ff));
        WZY_TRY(wzy_stage_write_tensor_range(st, -1, "experts", b0 * rec, outp.data(), nb * rec));
    }
    return stage_set_loaded(st, true);
}

// ------------------------------------------------------------------------------------------------
// per-layer embedding table
// ------------------------------------------------------------------------------------------------
extern "C" int wzy_stage_load_ple(wzy_stage* st, const char* ple_path) {
    WZY_REQUIRE(st && ple_path, "load_ple: null argument");
    const wzy_stage_cfg& c = *stage_cfg(st);
    WZY_REQUIRE(c.ple, "load_ple: the stage has no per-layer embedding (cfg.ple = 0)");
    Gg h;
    WZY_TRY(wzy_gguf_open(ple_path, &h.g));
    const wzy_gguf* g = h.g;
    const TensorEnt* t = find_t(g, "per_layer_token_embd.weight");
    WZY_REQUIRE(t, "load_ple: %s has no per_layer_token_embd.weight", ple_path);
    const uint64_t head = (uint64_t) c.n_embd / 16, rows = wzy_ple_table_rows();
    // the reference reads the tensor as raw bytes whatever its type tag: accept I8 and tags this
    // library does not know (an fp8 tag), reject the types with wider elements
    const bool one_byte = t->type == WZY_GGUF_I8 || type_bytes(t->type, 32) == 0;
    WZY_REQUIRE(one_byte && t->n_dims == 2 && (uint64_t) t->dims[0] == head && (uint64_t) t->dims[1] == rows,
                "load_ple: per_layer_token_embd.weight must be 1-byte codes [%llu x %llu] (type %d, %lld x %lld)",
                (unsigned long long) head, (unsigned long long) rows, t->type, (long long) t->dims[0],
                (long long) t->dims[1]);
    WZY_REQUIRE(t->off <= g->size && g->size - t->off >= head * rows, "load_ple: %s: the table lies outside the file",
                ple_path);
    // the table scale (PleSrc::open reads strata.ple.scale when it is an f32 or f64; otherwise 1)
    float scale = 1.f;
    auto sk = g->kv.find("strata.ple.scale");
    if (sk != g->kv.end() && sk->second.type == KV_F32) memcpy(&scale, g->base + sk->second.off, 4);
    if (sk != g->kv.end() && sk->second.type == KV_F64) {
        double v;
        memcpy(&v, g->base + sk->second.off, 8);
        scale = (float) v;
    }
    WZY_TRY(stage_set_ple_table(st, false, 0.f));
    const uint8_t* src = g->base + t->off;
    const size_t total = (size_t) (head * rows), chunk = (size_t) 256 << 20;
    for (size_t o = 0; o < total; o += chunk)
        WZY_TRY(wzy_stage_write_tensor_range(st, -1, "ple_table", o, src + o, std::min(chunk, total - o)));
    return stage_set_ple_table(st, true, scale);
}

// ------------------------------------------------------------------------------------------------
// MTP drafter
// ------------------------------------------------------------------------------------------------
namespace {
struct MtpEnt { std::string kind; int64_t rows, cols; size_t off, bytes; };   // one dense.txt line
int mtp_fill(wzy_stage* st, const wzy_stage_cfg& c, const std::string& dir, const std::map<std::string, MtpEnt>& idx,
             const std::vector<uint8_t>& dense);
}  // namespace

extern "C" int wzy_stage_mtp_load(wzy_stage* st, const char* mtp_dir, const char* dvocab_path) {
    WZY_REQUIRE(st && mtp_dir && dvocab_path, "mtp_load: null argument");
    const wzy_stage_cfg& c = *stage_cfg(st);
    const std::string dir(mtp_dir);
    // draft vocabulary
    std::vector<int32_t> ids;
    {
        std::ifstream vf(dvocab_path, std::ios::binary);
        if (!vf) { set_error("mtp_load: cannot open %s", dvocab_path); return WZY_EIO; }
        vf.seekg(0, std::ios::end);
        const size_t n = (size_t) vf.tellg();
        WZY_REQUIRE(n >= 4 && n % 4 == 0, "mtp_load: %s is not a list of int32 ids", dvocab_path);
        ids.resize(n / 4);
        vf.seekg(0);
        vf.read((char*) ids.data(), (std::streamsize) n);
    }
    // dense.txt index into dense.bin
    std::map<std::string, MtpEnt> idx;
    {
        std::ifstream tf(dir + "/dense.txt");
        if (!tf) { set_error("mtp_load: cannot open %s/dense.txt", mtp_dir); return WZY_EIO; }
        std::string line;
        while (std::getline(tf, line)) {
            if (line.empty()) continue;
            std::istringstream is(line);
            std::string nm;
            MtpEnt e;
            if (is >> nm >> e.kind >> e.rows >> e.cols >> e.off >> e.bytes) idx[nm] = e;
        }
    }
    std::vector<uint8_t> dense;
    {
        std::ifstream bf(dir + "/dense.bin", std::ios::binary);
        if (!bf) { set_error("mtp_load: cannot open %s/dense.bin", mtp_dir); return WZY_EIO; }
        bf.seekg(0, std::ios::end);
        dense.resize((size_t) bf.tellg());
        bf.seekg(0);
        bf.read((char*) dense.data(), (std::streamsize) dense.size());
    }
    WZY_TRY(wzy_stage_mtp_init_vocab(st, ids.data(), (int) ids.size()));
    const int rc = mtp_fill(st, c, dir, idx, dense);
    if (rc != WZY_OK) stage_mtp_drop(st);           // no half-loaded drafter
    return rc;
}

namespace {
int mtp_fill(wzy_stage* st, const wzy_stage_cfg& c, const std::string& dir, const std::map<std::string, MtpEnt>& idx,
             const std::vector<uint8_t>& dense) {
    const char* mtp_dir = dir.c_str();
    // one dense.bin tensor into "mtp.<name>"; the element size follows from the conversion, as the
    // reference's ld_q8 / ld_bf / ld_bf_as_q8 / ld_f32 assume it
    auto put_d = [&](const char* name, const char* src, Conv conv, int64_t rows, int64_t cols) -> int {
        auto it = idx.find(src);
        WZY_REQUIRE(it != idx.end(), "mtp_load: dense.txt has no %s", src);
        const MtpEnt& e = it->second;
        WZY_REQUIRE(e.rows * e.cols == rows * cols, "mtp_load: %s is %lld x %lld, expected %lld x %lld", src,
                    (long long) e.rows, (long long) e.cols, (long long) rows, (long long) cols);
        const size_t n = (size_t) (rows * cols);
        const size_t want = conv == C_Q8 ? n / 32 * 34 : (conv == C_F32 ? n * 4 : n * 2);
        WZY_REQUIRE(e.bytes == want && e.off <= dense.size() && want <= dense.size() - e.off,
                    "mtp_load: %s: %zu bytes at %zu do not fit (expected %zu within dense.bin)", src, e.bytes, e.off, want);
        TensorEnt t{};
        t.name = src;
        t.n_dims = 2;
        t.dims[0] = cols; t.dims[1] = rows; t.dims[2] = t.dims[3] = 1;
        t.type = conv == C_Q8 ? WZY_GGUF_Q8_0 : (conv == C_F32 ? WZY_GGUF_F32 : WZY_GGUF_BF16);
        t.off = e.off;
        t.bytes = want;
        wzy_gguf view;                                  // dense.bin seen as a container of one tensor
        view.base = const_cast<uint8_t*>(dense.data());
        view.size = dense.size();
        const int rc = put(st, -1, (std::string("mtp.") + name).c_str(), &view, &t, src, conv, rows, cols);
        view.base = nullptr;                            // not a mapping: nothing to unmap
        return rc;
    };
    const int64_t D = c.n_embd, HCD = (int64_t) c.hc * D, L = c.hc_lr;
    const int64_t QD = (int64_t) c.qsa_qh * c.qsa_hd, KVD = (int64_t) c.qsa_kvh * c.qsa_hd;
    WZY_TRY(put_d("fc_emb", "fc_embedding.weight", C_Q8, D, D));
    WZY_TRY(put_d("fc_hid", "fc_hidden.weight", C_Q8, D, D));
    WZY_TRY(put_d("pre_norm_emb", "pre_fc_norm_embedding.weight", C_F32, 1, D));
    WZY_TRY(put_d("pre_norm_hid", "pre_fc_norm_hidden.weight", C_F32, 1, HCD));
    const char* hcs[3] = {"attn_hyper_connection.", "mlp_hyper_connection.", "hyper_connection_mixer."};
    char nm[32];
    for (int i = 0; i < 3; ++i) {
        const std::string p(hcs[i]);
        snprintf(nm, sizeof nm, "hc_norm%d", i);
        WZY_TRY(put_d(nm, (p + "hc_norm.weight").c_str(), C_F32, 1, HCD));
        snprintf(nm, sizeof nm, "hc_down%d", i);
        WZY_TRY(put_d(nm, (p + "input_mix_weight_down.weight").c_str(), C_BF16_Q8, L, HCD));
        snprintf(nm, sizeof nm, "hc_up%d", i);
        WZY_TRY(put_d(nm, (p + "input_mix_weight_up.weight").c_str(), C_BF16_Q8, HCD, L));
        if (i < 2) {
            snprintf(nm, sizeof nm, "hc_inj%d", i);
            WZY_TRY(put_d(nm, (p + "block_inject_weight.weight").c_str(), C_BF16, c.hc, HCD));
        }
    }
    WZY_TRY(put_d("wq", "self_attn.q_proj.weight", C_Q8, 2 * QD, D));
    WZY_TRY(put_d("wk", "self_attn.k_proj.weight", C_Q8, KVD, D));
    WZY_TRY(put_d("wv", "self_attn.v_proj.weight", C_Q8, KVD, D));
    WZY_TRY(put_d("wo", "self_attn.o_proj.weight", C_Q8, D, QD));
    WZY_TRY(put_d("q_norm", "self_attn.q_norm.weight", C_F32, 1, c.qsa_hd));
    WZY_TRY(put_d("k_norm", "self_attn.k_norm.weight", C_F32, 1, c.qsa_hd));
    WZY_TRY(put_d("router", "mlp.gate.weight", C_BF16, c.n_exp, D));
    WZY_TRY(put_d("sh_gate", "mlp.shared_expert.gate_proj.weight", C_Q8, c.n_ff, D));
    WZY_TRY(put_d("sh_up", "mlp.shared_expert.up_proj.weight", C_Q8, c.n_ff, D));
    WZY_TRY(put_d("sh_down", "mlp.shared_expert.down_proj.weight", C_Q8, D, c.n_ff));
    WZY_TRY(put_d("sgate", "mlp.shared_expert_gate.weight", C_BF16, 1, D));
    // Q2_0 experts, in the reference's blob layout as they are
    const size_t ebytes = (size_t) c.n_exp * wzy_q2_expert_bytes(c.n_embd, c.n_ff);
    std::vector<uint8_t> ex(ebytes);
    {
        std::ifstream ef(dir + "/experts.bin", std::ios::binary);
        if (!ef) { set_error("mtp_load: cannot open %s/experts.bin", mtp_dir); return WZY_EIO; }
        ef.read((char*) ex.data(), (std::streamsize) ebytes);
        if ((size_t) ef.gcount() != ebytes) {
            set_error("mtp_load: %s/experts.bin holds fewer than %zu bytes", mtp_dir, ebytes);
            return WZY_EIO;
        }
    }
    return wzy_stage_write_tensor(st, -1, "mtp.experts", ex.data(), ex.size());
}
}  // namespace

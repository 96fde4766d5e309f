// measure.hip -- measurement entry points for BASELINE configs 2 and 3: bursts of back-to-back
// launches of one kernel family on one stream, bracketed by a pair of HIP events, so the mean
// duration excludes host launch overhead and per-launch event packets.
#include "wzy_device.h"
#include "wzy_gdn.h"
#include "wzy_host.h"
#include "wzy_qsa.h"

using namespace wzy;

namespace {
struct EventPair {
    hipEvent_t a = nullptr, b = nullptr;
    ~EventPair() {
        if (a) (void) hipEventDestroy(a);
        if (b) (void) hipEventDestroy(b);
    }
    int create() {
        WZY_HIP_TRY(hipEventCreate(&a));
        WZY_HIP_TRY(hipEventCreate(&b));
        return WZY_OK;
    }
    int elapsed_us(float* us) {
        WZY_HIP_TRY(hipEventSynchronize(b));
        float ms = 0.f;
        WZY_HIP_TRY(hipEventElapsedTime(&ms, a, b));
        *us = ms * 1000.0f;
        return WZY_OK;
    }
};
}  // namespace

extern "C" int wzy_gdn_time_recurrence(const float* q, const float* k, const float* v, const float* decay,
                                       const float* beta, float* states, float* y, int hk, int hv, int n_layers,
                                       int steps, int T, float* us_per_layer_step, float* us_kernel_only,
                                       void* stream) {
    WZY_REQUIRE(q && k && v && decay && beta && states && y && us_per_layer_step, "gdn_time: null argument");
    WZY_REQUIRE(n_layers >= 1 && steps >= 1 && T >= 1 && T <= WZY_MAX_W && steps % T == 0,
                "gdn_time: bad layer / step counts (steps must be a multiple of T)");
    hipStream_t st = as_stream(stream);
    const size_t state_floats = (size_t) hv * 128 * 128;
    // output-norm partial sums of the kernel-only burst (its consumer, the norm kernel, is left out)
    float* ss = nullptr;
    WZY_HIP_TRY(hipMalloc((void**) &ss, (size_t) WZY_MAX_W * hv * GDN_NQ * sizeof(float)));
    auto run = [&](bool with_norm) -> int {
        for (int s0 = 0; s0 < steps; s0 += T)
            for (int l = 0; l < n_layers; ++l) {
                GdnArgs a{};
                a.q = q + (size_t) s0 * hk * 128; a.k = k + (size_t) s0 * hk * 128; a.v = v + (size_t) s0 * hv * 128;
                a.decay = decay + (size_t) s0 * hv; a.beta = beta + (size_t) s0 * hv;
                a.eps = 1e-6f; a.state = states + (size_t) l * state_floats;
                a.y = y + (size_t) s0 * hv * 128; a.hk = hk; a.hv = hv; a.S = 128; a.T = T;
                a.o_ss = with_norm ? nullptr : ss;
                WZY_TRY(launch_gdn(a, false, st));
            }
        return WZY_OK;
    };
    EventPair e;
    int rc = e.create();
    if (rc == WZY_OK) rc = run(true);                       // warm-up
    if (rc == WZY_OK && hipEventRecord(e.a, st) != hipSuccess) rc = WZY_EHIP;
    if (rc == WZY_OK) rc = run(true);
    if (rc == WZY_OK && hipEventRecord(e.b, st) != hipSuccess) rc = WZY_EHIP;
    float us = 0.f;
    if (rc == WZY_OK) rc = e.elapsed_us(&us);
    if (rc == WZY_OK) *us_per_layer_step = us / ((float) n_layers * (float) steps);
    if (rc == WZY_OK && us_kernel_only) {
        if (hipEventRecord(e.a, st) != hipSuccess) rc = WZY_EHIP;
        if (rc == WZY_OK) rc = run(false);
        if (rc == WZY_OK && hipEventRecord(e.b, st) != hipSuccess) rc = WZY_EHIP;
        if (rc == WZY_OK) rc = e.elapsed_us(&us);
        if (rc == WZY_OK) *us_kernel_only = us / ((float) n_layers * (float) steps);
    }
    (void) hipStreamSynchronize(st);
    (void) hipFree(ss);
    if (rc == WZY_EHIP) set_error("gdn_time: HIP event failure");
    return rc;
}

extern "C" int wzy_qsa_time_decode(const wzy_qsa_dims* dims, const wzy_qsa_layer* L, const int* pos, int iters,
                                   float* us_stages, void* stream) {
    WZY_REQUIRE(dims && L && pos && us_stages && iters >= 1, "qsa_time: bad arguments");
    hipStream_t st = as_stream(stream);
    QsaDims dm{};
    dm.qh = dims->qh; dm.kvh = dims->kvh; dm.hd = dims->hd; dm.n_rot = dims->n_rot;
    dm.ih = dims->idx_heads; dm.idim = dims->idx_dim; dm.iblk = dims->idx_blk; dm.topk = dims->idx_topk;
    dm.ctx_max = dims->ctx_max; dm.ring_cap = dims->kv_ring; dm.sinks = dims->kv_sinks; dm.eps = dims->eps;
    dm.f16_above = dims->attn_f16_above;
    WZY_TRY(qsa_check_dims(dm));
    WZY_REQUIRE(L->max_b >= dm.ctx_max / dm.iblk + 1, "qsa_time: max_b too small");
    QsaPrepArgs p{};
    p.dm = dm; p.pos = pos; p.qg = L->qg; p.kk = L->kk; p.vv = L->vv; p.q_idx = L->q_idx; p.idx_raw = L->idx_raw;
    p.q_norm = L->q_norm; p.k_norm = L->k_norm; p.iq_norm = L->iq_norm; p.ik_norm = L->ik_norm;
    p.cos_tab = L->cos_tab; p.sin_tab = L->sin_tab;
    p.kv = QsaKv{L->kq, L->ks, L->vq, L->vs};
    p.ix = QsaIdx{L->idx_tail, L->idx_dead, L->idx_pooled, nullptr, nullptr, nullptr};
    QsaScoreArgs s{};
    s.dm = dm; s.pos = pos; s.pooled = L->idx_pooled; s.dead = L->idx_dead; s.q_idx = L->q_idx; s.scores = L->scores;
    s.max_b = L->max_b;
    auto stage = [&](int which) -> int {
        switch (which) {
            case 0: return launch_qsa_prep(p, 1, st);
            case 1: return launch_qsa_score(s, 1, st);
            case 2: return launch_qsa_topk(dm, pos, L->scores, L->max_b, L->sel_ids, L->sel_cnt, 1, st);
            default:
                return wzy_qsa_attend(dims, pos, L->qg, L->kq, L->ks, L->vq, L->vs, L->sel_ids, L->out, L->workspace,
                                      L->workspace_bytes, 1, stream);
        }
    };
    // one warm pass in order (so every stage reads the outputs of the one before), then one burst
    // of `iters` launches per stage
    for (int w = 0; w < 4; ++w) WZY_TRY(stage(w));
    EventPair e;
    WZY_TRY(e.create());
    for (int w = 0; w < 4; ++w) {
        WZY_HIP_TRY(hipEventRecord(e.a, st));
        for (int i = 0; i < iters; ++i) WZY_TRY(stage(w));
        WZY_HIP_TRY(hipEventRecord(e.b, st));
        float us = 0.f;
        WZY_TRY(e.elapsed_us(&us));
        us_stages[w] = us / (float) iters;
    }
    return WZY_OK;
}

// stage.hip -- the decode-path layer executor (StageGpu replacement) for one MI355X.
//
// Owns every weight, state and scratch buffer of the model in HBM and enqueues the per-layer
// kernel sequence of a forward on one stream; each window shape is captured once into a hipGraph
// and replayed.  Per layer (T window rows):
//   attention half:  hc_pre(fold previous FFN block) -> hc_post -> projections (one multi-segment
//                    GEMV) -> GDN step | QSA prep, score, top-k, attention -> out-projection
//   FFN half:        hc_pre(fold attention block) -> hc_post -> router GEMV -> MoE gate/up -> down
// Head: hc_pre(fold last FFN block) -> hc_post -> bf16 LM head GEMV -> argmax / top-16.
// reference: StageGpu (src/wzy_stage_v2.cuh:334-1045), record_forward (:476-857).
#include <math.h>
#include <string.h>

#include <algorithm>
#include <iterator>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../include/wzy_stage.h"
#include "../../include/wzy_synth.h"
#include "wzy_gdn.h"
#include "wzy_gemv.h"
#include "wzy_hc.h"
#include "wzy_ple.h"
#include "wzy_host.h"
#include "wzy_moe.h"
#include "wzy_mtp.h"
#include "wzy_prefill.h"
#include "wzy_stage_int.h"
#include "wzy_qsa.h"
#include "wzy_reduce.h"
#include "wzy_synth_impl.h"

using namespace wzy;

namespace {

enum DType { DT_F32, DT_BF16, DT_F16, DT_I8, DT_U8, DT_I32 };
size_t dt_size(DType t) { return (t == DT_F32 || t == DT_I32) ? 4 : (t == DT_BF16 || t == DT_F16) ? 2 : 1; }

struct Tensor {
    void* p = nullptr;
    size_t bytes = 0;
};

// Synthetic-model tensor ids (stream sub-ids of WZY_S_DENSE / WZY_S_STATE)
enum TensorId {
    TI_ROUTER = 0, TI_SGATE = 1, TI_SH_GATE = 2, TI_SH_UP = 3, TI_SH_DOWN = 4,
    TI_HC_NORM = 10, TI_HC_DOWN = 11, TI_HC_UP = 12, TI_HC_INJ = 13,   // + 10*half
    TI_QKV = 30, TI_WGATE = 31, TI_WOUT = 32, TI_ALPHA = 33, TI_BETA = 34, TI_SSM_A = 35, TI_DT = 36,
    TI_CONV = 37, TI_SSM_NORM = 38,
    TI_WQ = 40, TI_WK = 41, TI_WV = 42, TI_WO = 43, TI_QNORM = 44, TI_KNORM = 45, TI_IDXQ = 46, TI_IDXK = 47,
    TI_IDXQN = 48, TI_IDXKN = 49,
    TI_EMB = 60, TI_HEAD_NORM = 61, TI_HEAD_DOWN = 62, TI_HEAD_UP = 63, TI_HEAD = 64,
    TS_CONV = 70, TS_SSM = 71, TS_TAIL = 72, TS_DEAD = 73, TS_POOLED = 74,
    TI_PLE_K = 80, TI_PLE_V = 81, TI_PLE_NQ = 82, TI_PLE_NK = 83, TI_PLE_NC = 84, TI_PLE_CONV = 85,
    TS_PLE_HIST = 86, TS_PLE_TOKS = 87,
};
constexpr uint32_t MODEL_LAYER = 0xFFFF;

// One copy of commit_window_state: dst <- src + acc_idx * src_stride (bytes; multiples of 16).
// pooled: the destination moves by (acc_pos / idx_blk) * pooled_row bytes, and the job only runs for
// acc_pos >= 0 (the indexer state of a QSA layer).
struct CommitJob {
    unsigned char* dst;
    const unsigned char* src;
    size_t src_stride, bytes;
    int qsa, pooled;
};
constexpr int COMMIT_WGS = 64;         // workgroups per copy job

// every job of commit_window_state in one launch: grid (COMMIT_WGS, jobs)
__global__ void __launch_bounds__(256) commit_kernel(const CommitJob* __restrict__ jobs, int acc_idx, int acc_pos,
                                                     int idx_blk, int pooled_row) {
    const CommitJob j = jobs[blockIdx.y];
    if (j.qsa && acc_pos < 0) return;
    unsigned char* dst = j.dst + (j.pooled ? (size_t) (acc_pos / idx_blk) * pooled_row : 0);
    const uint4* src = (const uint4*) (j.src + (size_t) acc_idx * j.src_stride);
    const size_t n = j.bytes / 16;
    for (size_t i = (size_t) blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t) COMMIT_WGS * 256)
        ((uint4*) dst)[i] = src[i];
}

// Plain device-to-device copies, every job of a table in one launch: grid (COPY_WGS, jobs).
// Pointers are 16-byte aligned; a job's last bytes % 16 are copied one byte per lane.
struct CopyJob {
    unsigned char* dst;
    const unsigned char* src;
    size_t bytes;
};
constexpr int COPY_WGS = 128;
constexpr int SESSION_MAX_JOBS = 1024;

__global__ void __launch_bounds__(256) copy_jobs_kernel(const CopyJob* __restrict__ jobs) {
    const CopyJob j = jobs[blockIdx.y];
    const size_t n16 = j.bytes / 16;
    const size_t stride = (size_t) COPY_WGS * 256;
    for (size_t i = (size_t) blockIdx.x * 256 + threadIdx.x; i < n16; i += stride)
        ((uint4*) j.dst)[i] = ((const uint4*) j.src)[i];
    for (size_t i = n16 * 16 + (size_t) blockIdx.x * 256 + threadIdx.x; i < j.bytes; i += stride) j.dst[i] = j.src[i];
}

struct Q8 {
    int8_t* q = nullptr;
    uint16_t* s = nullptr;
    int rows = 0, cols = 0;
};

struct Layer {
    bool qsa = false;
    int local = -1;                 // index among GDN or QSA layers
    float* hc_norm[2] = {nullptr, nullptr};
    Q8 hc_down[2], hc_up[2];
    uint16_t* hc_inj[2] = {nullptr, nullptr};
    // GDN
    Q8 qkv, wgate, wout;
    uint16_t *alpha = nullptr, *beta = nullptr;
    float *ssm_a = nullptr, *dt = nullptr, *conv_w = nullptr, *ssm_norm = nullptr;
    float *conv_hist = nullptr, *ssm = nullptr;     // state
    // QSA
    Q8 wq, wk, wv, wo;
    float *q_norm = nullptr, *k_norm = nullptr, *idx_qn = nullptr, *idx_kn = nullptr;
    uint16_t *idx_q = nullptr, *idx_k = nullptr;
    QsaKv kv{};
    QsaIdx ix{};
    // MoE
    wzy_moe_weights moe{};
};

}  // namespace

struct wzy_stage {
    wzy_stage_cfg cfg{};
    int dev = 0;
    hipStream_t stream = nullptr;
    bool graphs = true;
    size_t dev_bytes = 0;
    std::vector<void*> allocs;
    std::map<std::pair<int, std::string>, Tensor> tensors;

    // derived dims
    int D = 0, HCD = 0, QKV = 0, GV = 0, QD = 0, KVD = 0, max_b = 0, n_gdn = 0, n_qsa = 0;
    QsaDims qd{};

    std::vector<Layer> L;
    uint8_t* experts = nullptr;     // all layers' NVFP4 expert records
    size_t expert_rec = 0;
    uint16_t* emb = nullptr;        // bf16 token embeddings (cfg.emb_q8 == 0)
    Q8 emb8;                        // Q8_0 token embeddings (cfg.emb_q8 == 1)
    float* head_norm = nullptr;
    Q8 head_down, head_up;
    uint16_t* head = nullptr;       // bf16 LM head (cfg.head_q8 == 0)
    Q8 head8;                       // Q8_0 LM head (cfg.head_q8 == 1)
    float *cos_tab = nullptr, *sin_tab = nullptr;

    // activations / scratch (MAX_W rows)
    float* R[2] = {nullptr, nullptr};
    int r_pre_head = 0;             // which R buffer holds the pre-head residual
    float *nsc = nullptr, *lo = nullptr, *inj_a = nullptr, *inj_f = nullptr, *mixed = nullptr;
    float *lo_part = nullptr, *inj_part = nullptr;   // HC read partials (per source stream)
    float *qkv = nullptr, *z = nullptr, *ab = nullptr, *y = nullptr, *block = nullptr, *comb = nullptr;
    float* gdn_ss = nullptr;     // [W][hv][GDN_NQ] partial sums of the GDN output norm
    float *qg = nullptr, *kk = nullptr, *vv = nullptr, *idx_raw = nullptr, *q_idx = nullptr, *scores = nullptr;
    float *att_part = nullptr, *att_ml = nullptr, *att_out = nullptr;
    int *sel_ids = nullptr, *sel_cnt = nullptr;
    void* moe_ws = nullptr;
    MoeWs mws{};
    float* logits = nullptr;
    void* red_ws = nullptr;
    float* emb_rows = nullptr;
    // snapshots
    float *conv_snaps = nullptr, *ssm_snaps = nullptr;
    float *tail_snaps = nullptr, *dead_snaps = nullptr;
    uint16_t* pool_snaps = nullptr;
    // step inputs / outputs
    // Step parameters ([0] = pos, [1..8] = toks) are staged through a ring of pinned host slots:
    // forwards enqueued back to back must not overwrite a slot whose copy has not run yet, so each
    // slot carries an event recorded after its copy and is waited on before reuse.
    static constexpr int STEP_SLOTS = 32, STEP_INTS = 16;
    int* d_step = nullptr;
    int* h_step = nullptr;          // pinned [STEP_SLOTS x STEP_INTS]
    hipEvent_t step_ev[STEP_SLOTS] = {};
    bool step_pending[STEP_SLOTS] = {};
    int step_slot = 0;
    int* h_greedy = nullptr;        // pinned, device-visible
    float* h_top_v = nullptr;
    int* h_top_i = nullptr;
    int* d_greedy = nullptr;        // device views of the pinned outputs
    float* d_top_v = nullptr;
    int* d_top_i = nullptr;
    int last_T = 0;
    bool have_head = false;         // last forward ran the LM head (logits, greedy ids)
    bool have_pre_head = false;     // last forward left its pre-head residual rows in R[r_pre_head]
    bool loaded = false;
    MtpState* mtp = nullptr;        // MTP drafter (wzy_stage_mtp_init)

    // per-layer embedding at layer 1 (cfg.ple): weights, the fp8 table, state and W-row scratch
    struct Ple {
        uint16_t *wk = nullptr, *wv = nullptr;                  // bf16 [HCD x D], [D x D]
        float *nq = nullptr, *nk = nullptr, *nc = nullptr;      // [HCD]
        float* cw = nullptr;                                    // [HCD x 4]
        float* hist = nullptr;                                  // [HCD x 9] state
        float* snaps = nullptr;                                 // [W][HCD x 9]
        uint8_t* table = nullptr;                               // [ple_table_rows() x D/16] fp8
        float* scale_dev = nullptr;                             // the table scale, read by the row kernel
        int* tok_hist = nullptr;                                // [ctx_max + 4] token of each cell
        float *emb = nullptr, *k = nullptr, *v = nullptr, *gat = nullptr, *n = nullptr;   // W rows
        bool table_ready = false;                               // table and scale loaded
    } ple;

    // parked sessions: per slot one HBM buffer holding a copy of the session state, and the
    // device tables of the copies that save and restore it (one copy_jobs_kernel launch each)
    struct SessionSlot {
        unsigned char* buf = nullptr;
        size_t cap = 0;
        CopyJob* jobs = nullptr;        // [2][SESSION_MAX_JOBS]: save, restore
        int n_jobs = 0;
        int n_cells = -1;               // -1: empty
    };
    SessionSlot sess[WZY_SESSION_SLOTS];
    void session_regions(int n_cells, std::vector<std::pair<void*, size_t>>& out) const;

    // chunked-prefill workspace, sized for `cap` rows on the first prefill that needs it
    struct PfWs {
        int cap = 0;
        void* base = nullptr;
        size_t bytes = 0;
        float *R = nullptr, *lo = nullptr, *inj_a = nullptr, *inj_f = nullptr, *mixed = nullptr;
        uint16_t *xn = nullptr, *loh = nullptr, *xh = nullptr;
        float *qkv = nullptr, *z = nullptr, *ab = nullptr, *conv_out = nullptr, *decay = nullptr, *beta = nullptr,
              *kq = nullptr, *o = nullptr;
        float *qg = nullptr, *kk = nullptr, *vv = nullptr, *idx_raw = nullptr, *q_idx = nullptr, *scores = nullptr;
        int *sel = nullptr, *cnt = nullptr;
        float *block = nullptr, *comb = nullptr;
        void* moe_ws = nullptr;
        size_t moe_bytes = 0;
        int* toks = nullptr;
        float *ple_emb = nullptr, *ple_k = nullptr, *ple_v = nullptr, *ple_gat = nullptr, *ple_n = nullptr;
        uint16_t* ple_embh = nullptr;   // the PLE rows as the bf16 GEMM operand
        uint16_t* wbf = nullptr;    // bf16 expansion of the Q8_0 weights of the running GEMM
        size_t wbf_elems = 0;
        int* pos8 = nullptr;        // [cap / 8 + 2]: p0 + 8 i
        int sc_rows = 0;            // rows per block-score pass
        float* tr = nullptr;        // per-layer trace [n_layers][4][tr_rows][D] (while tracing)
        int* tr_sel = nullptr;      // per QSA layer: selected cells [n_qsa][tr_rows][topk], counts
        int* tr_cnt = nullptr;      // [n_qsa][tr_rows]
        float* tr_sc = nullptr;     // block scores [n_qsa][tr_rows][max_b]
        float* tr_kv = nullptr;     // rows the KV / indexer appends quantise: [n_qsa][tr_rows][kvd k | kvd v | idim]
        int tr_rows = 0;
    } pf;
    bool pre_head_pf = false;       // the pre-head rows of the last call are the prefill's residual
    const float* pre_head_rows() const { return pre_head_pf ? pf.R : R[r_pre_head]; }
    int prefill_reserve(int B);
    int enqueue_prefill(int p0, int B, float* us_parts);

    std::map<unsigned long long, hipGraphExec_t> graph_execs;
    CommitJob* commit_jobs = nullptr;   // device table of commit_window_state's copies
    int n_commit_jobs = 0;

    bool profiling = false;         // direct launches instead of graphs
    hipEvent_t ev[3] = {nullptr, nullptr, nullptr};

    // per-layer trace of the last forward (direct launches while on): HC read outputs, block and
    // MoE outputs [n_layers][W][D], router logits / ids / weights [n_layers][W][E or K], and per QSA
    // layer the block scores [n_qsa][W][max_b], selected cells [n_qsa][W][topk] and counts [n_qsa][W],
    // the rows the KV and indexer appends quantise (k after its norm + RoPE, v, the raw indexer key:
    // [n_qsa][W][kvd or idim]), the q | gate rows the attention reads (after norm + RoPE,
    // [n_qsa][W][2 qh hd]) and the attention output before the o projection ([n_qsa][W][qh hd])
    bool trace = false;
    float *tr_mixa = nullptr, *tr_block = nullptr, *tr_mixf = nullptr, *tr_comb = nullptr;
    float *tr_ra = nullptr, *tr_rf = nullptr, *tr_inja = nullptr, *tr_injf = nullptr;
    float *tr_logits = nullptr, *tr_wts = nullptr, *tr_scores = nullptr;
    float *tr_kk = nullptr, *tr_vv = nullptr, *tr_iraw = nullptr, *tr_qg = nullptr, *tr_att = nullptr;
    int *tr_ids = nullptr, *tr_sel = nullptr, *tr_cnt = nullptr;
    int trace_alloc();

    ~wzy_stage();
    int alloc(void** p, size_t bytes, bool zero = true);
    template <class T>
    int alloc_t(T** p, size_t n, bool zero = true) { return alloc((void**) p, n * sizeof(T), zero); }
    int reg(int layer, const char* name, void* p, size_t bytes) {
        tensors[{layer, std::string(name)}] = Tensor{p, bytes};
        return WZY_OK;
    }
    int alloc_q8(Q8& m, int rows, int cols, int layer, const char* name);
    int init_buffers();
    int enqueue(int T, bool emb_host, int run_head, bool save_snaps, bool want_top16, int snap_offset);
};

wzy_stage::~wzy_stage() {
    (void) hipSetDevice(dev);
    if (stream) (void) hipStreamSynchronize(stream);
    delete mtp;
    for (auto& sl : sess) {
        if (sl.buf) (void) hipFree(sl.buf);
        if (sl.jobs) (void) hipFree(sl.jobs);
    }
    if (pf.base) (void) hipFree(pf.base);
    if (pf.tr) (void) hipFree(pf.tr);
    if (pf.tr_sel) (void) hipFree(pf.tr_sel);
    if (pf.tr_sc) (void) hipFree(pf.tr_sc);
    if (pf.tr_kv) (void) hipFree(pf.tr_kv);
    for (auto& kv : graph_execs)
        if (kv.second) (void) hipGraphExecDestroy(kv.second);
    for (void* p : allocs) (void) hipFree(p);
    if (h_step) (void) hipHostFree(h_step);
    if (h_greedy) (void) hipHostFree(h_greedy);
    if (h_top_v) (void) hipHostFree(h_top_v);
    if (h_top_i) (void) hipHostFree(h_top_i);
    for (auto& e : ev)
        if (e) (void) hipEventDestroy(e);
    for (auto& e : step_ev)
        if (e) (void) hipEventDestroy(e);
    if (stream) (void) hipStreamDestroy(stream);
}

int wzy_stage::alloc(void** p, size_t bytes, bool zero) {
    *p = nullptr;
    if (bytes == 0) bytes = 16;
    if (hipMalloc(p, bytes) != hipSuccess) {
        (void) hipGetLastError();
        *p = nullptr;
        set_error("stage: hipMalloc(%zu) failed (%.2f GiB already held)", bytes, dev_bytes / 1073741824.0);
        return WZY_ENOMEM;
    }
    allocs.push_back(*p);
    dev_bytes += bytes;
    if (zero) WZY_HIP_TRY(hipMemset(*p, 0, bytes));
    return WZY_OK;
}

int wzy_stage::alloc_q8(Q8& m, int rows, int cols, int layer, const char* name) {
    m.rows = rows;
    m.cols = cols;
    WZY_TRY(alloc_t(&m.q, (size_t) rows * cols, false));
    WZY_TRY(alloc_t(&m.s, (size_t) rows * cols / 32, false));
    std::string n(name);
    reg(layer, (n + ".q").c_str(), m.q, (size_t) rows * cols);
    reg(layer, (n + ".s").c_str(), m.s, (size_t) rows * cols / 32 * 2);
    return WZY_OK;
}

static int validate(const wzy_stage_cfg& c) {
    WZY_REQUIRE(c.n_layers >= 1 && c.n_layers <= 4096 && c.qsa_period >= 1, "stage: bad layer count / period");
    WZY_REQUIRE(c.n_embd >= 256 && c.n_embd % 256 == 0 && c.n_embd <= 8192, "stage: n_embd must be a multiple of 256 <= 8192");
    WZY_REQUIRE(c.hc == 4 && c.hc_lr % 32 == 0 && c.hc_lr >= 32 && c.hc_lr <= 512 && c.n_embd <= 4096,
                "stage: bad hyper-connection shape");
    WZY_REQUIRE(hc_width_supported(c.n_embd),
                "stage: n_embd %d has no HC read kernel (256, 512, 768, 1024, 1280, 1536, 2048, 2560, 3072, 4096)",
                c.n_embd);
    WZY_REQUIRE(c.gdn_hk >= 1 && c.gdn_hv % c.gdn_hk == 0, "stage: bad GDN heads");
    WZY_REQUIRE(c.qsa_hd == 256 && c.qsa_qh % c.qsa_kvh == 0 && c.qsa_qh / c.qsa_kvh <= 16, "stage: bad QSA heads");
    WZY_REQUIRE(c.idx_dim <= 128 && c.idx_heads <= 4 && c.idx_blk >= 2 && c.idx_topk >= 1, "stage: bad indexer");
    WZY_REQUIRE(c.n_exp >= 1 && c.n_exp <= 1024 && c.top_k >= 1 && c.top_k <= MOE_MAX_K && c.n_ff % 64 == 0,
                "stage: bad MoE shape");
    WZY_REQUIRE(c.n_vocab >= 16 && c.ctx_max >= 8, "stage: bad vocab / context");
    WZY_REQUIRE(c.attn_f16_above >= 0, "stage: attn_f16_above %d is negative", c.attn_f16_above);
    WZY_REQUIRE(!c.ple || (c.n_layers >= 2 && c.n_embd % 16 == 0 && c.n_embd <= 4096),
                "stage: the per-layer embedding needs layer 1 and n_embd a multiple of 16 (<= 4096)");
    WZY_REQUIRE(2 * c.qsa_qh * c.qsa_hd <= 16384 && c.n_embd * 1 <= 8192, "stage: projection too wide");
    WZY_REQUIRE((c.n_vocab + 2047) / 2048 * 16 <= 2048, "stage: n_vocab too large for the top-16 merge");
    return qsa_check_ring(c.ctx_max, c.kv_ring, c.kv_sinks);
}

int wzy_stage::init_buffers() {
    const wzy_stage_cfg& c = cfg;
    D = c.n_embd;
    HCD = c.hc * D;
    QKV = 2 * c.gdn_hk * 128 + c.gdn_hv * 128;
    GV = c.gdn_hv * 128;
    QD = c.qsa_qh * c.qsa_hd;
    KVD = c.qsa_kvh * c.qsa_hd;
    max_b = c.ctx_max / c.idx_blk + 2;
    qd.qh = c.qsa_qh; qd.kvh = c.qsa_kvh; qd.hd = c.qsa_hd; qd.n_rot = c.n_rot;
    qd.ih = c.idx_heads; qd.idim = c.idx_dim; qd.iblk = c.idx_blk; qd.topk = c.idx_topk;
    qd.ctx_max = c.ctx_max; qd.ring_cap = c.kv_ring; qd.sinks = c.kv_sinks; qd.eps = c.eps;
    qd.f16_above = c.attn_f16_above;
    const size_t kv_slots = c.kv_ring > 0 ? (size_t) c.kv_ring : (size_t) c.ctx_max;
    const int W = WZY_MAX_W;

    L.resize(c.n_layers);
    n_gdn = n_qsa = 0;
    expert_rec = wzy_nvfp4_expert_bytes(D, c.n_ff);
    WZY_TRY(alloc_t(&experts, expert_rec * c.n_exp * c.n_layers, false));
    reg(-1, "experts", experts, expert_rec * c.n_exp * c.n_layers);
    char nm[64];
    for (int l = 0; l < c.n_layers; ++l) {
        Layer& w = L[l];
        w.qsa = (l % c.qsa_period) == c.qsa_period - 1;
        w.local = w.qsa ? n_qsa++ : n_gdn++;
        for (int h = 0; h < 2; ++h) {
            snprintf(nm, sizeof nm, "hc_norm%d", h);
            WZY_TRY(alloc_t(&w.hc_norm[h], HCD, false)); reg(l, nm, w.hc_norm[h], HCD * 4);
            snprintf(nm, sizeof nm, "hc_down%d", h);
            WZY_TRY(alloc_q8(w.hc_down[h], c.hc_lr, HCD, l, nm));
            snprintf(nm, sizeof nm, "hc_up%d", h);
            WZY_TRY(alloc_q8(w.hc_up[h], HCD, c.hc_lr, l, nm));
            snprintf(nm, sizeof nm, "hc_inj%d", h);
            WZY_TRY(alloc_t(&w.hc_inj[h], (size_t) c.hc * HCD, false)); reg(l, nm, w.hc_inj[h], (size_t) c.hc * HCD * 2);
        }
        if (!w.qsa) {
            WZY_TRY(alloc_q8(w.qkv, QKV, D, l, "qkv"));
            WZY_TRY(alloc_q8(w.wgate, GV, D, l, "wgate"));
            WZY_TRY(alloc_q8(w.wout, D, GV, l, "wout"));
            WZY_TRY(alloc_t(&w.alpha, (size_t) c.gdn_hv * D, false)); reg(l, "alpha", w.alpha, (size_t) c.gdn_hv * D * 2);
            WZY_TRY(alloc_t(&w.beta, (size_t) c.gdn_hv * D, false)); reg(l, "beta", w.beta, (size_t) c.gdn_hv * D * 2);
            WZY_TRY(alloc_t(&w.ssm_a, c.gdn_hv, false)); reg(l, "ssm_a", w.ssm_a, c.gdn_hv * 4);
            WZY_TRY(alloc_t(&w.dt, c.gdn_hv, false)); reg(l, "dt_bias", w.dt, c.gdn_hv * 4);
            WZY_TRY(alloc_t(&w.conv_w, (size_t) QKV * 4, false)); reg(l, "conv1d", w.conv_w, (size_t) QKV * 16);
            WZY_TRY(alloc_t(&w.ssm_norm, 128, false)); reg(l, "ssm_norm", w.ssm_norm, 512);
            WZY_TRY(alloc_t(&w.conv_hist, (size_t) QKV * 3)); reg(l, "conv_hist", w.conv_hist, (size_t) QKV * 12);
            WZY_TRY(alloc_t(&w.ssm, (size_t) c.gdn_hv * 128 * 128)); reg(l, "ssm", w.ssm, (size_t) c.gdn_hv * 128 * 128 * 4);
        } else {
            WZY_TRY(alloc_q8(w.wq, 2 * QD, D, l, "wq"));
            WZY_TRY(alloc_q8(w.wk, KVD, D, l, "wk"));
            WZY_TRY(alloc_q8(w.wv, KVD, D, l, "wv"));
            WZY_TRY(alloc_q8(w.wo, D, QD, l, "wo"));
            WZY_TRY(alloc_t(&w.q_norm, c.qsa_hd, false)); reg(l, "q_norm", w.q_norm, c.qsa_hd * 4);
            WZY_TRY(alloc_t(&w.k_norm, c.qsa_hd, false)); reg(l, "k_norm", w.k_norm, c.qsa_hd * 4);
            WZY_TRY(alloc_t(&w.idx_q, (size_t) c.idx_heads * c.idx_dim * D, false));
            reg(l, "idx_q", w.idx_q, (size_t) c.idx_heads * c.idx_dim * D * 2);
            WZY_TRY(alloc_t(&w.idx_k, (size_t) c.idx_dim * D, false)); reg(l, "idx_k", w.idx_k, (size_t) c.idx_dim * D * 2);
            WZY_TRY(alloc_t(&w.idx_qn, c.idx_dim, false)); reg(l, "idx_qn", w.idx_qn, c.idx_dim * 4);
            WZY_TRY(alloc_t(&w.idx_kn, c.idx_dim, false)); reg(l, "idx_kn", w.idx_kn, c.idx_dim * 4);
            WZY_TRY(alloc_t(&w.kv.kq, kv_slots * KVD)); reg(l, "kv_k", w.kv.kq, kv_slots * KVD);
            WZY_TRY(alloc_t(&w.kv.ks, kv_slots * (KVD / 64))); reg(l, "kv_ks", w.kv.ks, kv_slots * (KVD / 64) * 2);
            WZY_TRY(alloc_t(&w.kv.vq, kv_slots * KVD)); reg(l, "kv_v", w.kv.vq, kv_slots * KVD);
            WZY_TRY(alloc_t(&w.kv.vs, kv_slots * (KVD / 64))); reg(l, "kv_vs", w.kv.vs, kv_slots * (KVD / 64) * 2);
            WZY_TRY(alloc_t(&w.ix.tail, (size_t) (c.idx_blk - 1) * c.idx_dim));
            reg(l, "idx_tail", w.ix.tail, (size_t) (c.idx_blk - 1) * c.idx_dim * 4);
            WZY_TRY(alloc_t(&w.ix.dead, c.idx_dim)); reg(l, "idx_dead", w.ix.dead, c.idx_dim * 4);
            WZY_TRY(alloc_t(&w.ix.pooled, (size_t) max_b * c.idx_dim));
            reg(l, "idx_pooled", w.ix.pooled, (size_t) max_b * c.idx_dim * 2);
        }
        wzy_moe_weights& m = w.moe;
        m.n_embd = D; m.n_ff = c.n_ff; m.n_exp = c.n_exp; m.top_k = c.top_k;
        uint16_t* router = nullptr;
        uint16_t* sgate = nullptr;
        WZY_TRY(alloc_t(&router, (size_t) c.n_exp * D, false)); reg(l, "router", router, (size_t) c.n_exp * D * 2);
        WZY_TRY(alloc_t(&sgate, D, false)); reg(l, "sgate", sgate, D * 2);
        m.router = router; m.sgate = sgate;
        Q8 g, u, dn;
        WZY_TRY(alloc_q8(g, c.n_ff, D, l, "sh_gate"));
        WZY_TRY(alloc_q8(u, c.n_ff, D, l, "sh_up"));
        WZY_TRY(alloc_q8(dn, D, c.n_ff, l, "sh_down"));
        m.sh_gate_q = g.q; m.sh_gate_s = g.s; m.sh_up_q = u.q; m.sh_up_s = u.s; m.sh_down_q = dn.q; m.sh_down_s = dn.s;
        m.experts = experts + (size_t) l * c.n_exp * expert_rec;
    }
    if (c.emb_q8) WZY_TRY(alloc_q8(emb8, c.n_vocab, D, -1, "emb"));
    else { WZY_TRY(alloc_t(&emb, (size_t) c.n_vocab * D, false)); reg(-1, "emb", emb, (size_t) c.n_vocab * D * 2); }
    WZY_TRY(alloc_t(&head_norm, HCD, false)); reg(-1, "head_norm", head_norm, HCD * 4);
    WZY_TRY(alloc_q8(head_down, c.hc_lr, HCD, -1, "head_down"));
    WZY_TRY(alloc_q8(head_up, HCD, c.hc_lr, -1, "head_up"));
    if (c.head_q8) WZY_TRY(alloc_q8(head8, c.n_vocab, D, -1, "head"));
    else { WZY_TRY(alloc_t(&head, (size_t) c.n_vocab * D, false)); reg(-1, "head", head, (size_t) c.n_vocab * D * 2); }
    if (c.ple) {
        const size_t hcd = (size_t) HCD, tb = (size_t) ple_table_rows() * (size_t) (D / PLE_HEADS);
        WZY_TRY(alloc_t(&ple.wk, hcd * D, false)); reg(1, "ple_key", ple.wk, hcd * D * 2);
        WZY_TRY(alloc_t(&ple.wv, (size_t) D * D, false)); reg(1, "ple_value", ple.wv, (size_t) D * D * 2);
        WZY_TRY(alloc_t(&ple.nq, hcd, false)); reg(1, "ple_norm_query", ple.nq, hcd * 4);
        WZY_TRY(alloc_t(&ple.nk, hcd, false)); reg(1, "ple_norm_key", ple.nk, hcd * 4);
        WZY_TRY(alloc_t(&ple.nc, hcd, false)); reg(1, "ple_norm_conv", ple.nc, hcd * 4);
        WZY_TRY(alloc_t(&ple.cw, hcd * 4, false)); reg(1, "ple_conv1d", ple.cw, hcd * 16);
        WZY_TRY(alloc_t(&ple.hist, hcd * PLE_HIST)); reg(1, "ple_hist", ple.hist, hcd * PLE_HIST * 4);
        WZY_TRY(alloc_t(&ple.snaps, (size_t) W * hcd * PLE_HIST));
        WZY_TRY(alloc_t(&ple.table, tb, false)); reg(-1, "ple_table", ple.table, tb);
        WZY_TRY(alloc_t(&ple.scale_dev, 1)); reg(-1, "ple_scale", ple.scale_dev, 4);
        WZY_TRY(alloc_t(&ple.tok_hist, (size_t) c.ctx_max + 4)); reg(-1, "tok_hist", ple.tok_hist, (size_t) c.ctx_max * 4);
        WZY_TRY(alloc_t(&ple.emb, (size_t) W * D)); WZY_TRY(alloc_t(&ple.v, (size_t) W * D));
        WZY_TRY(alloc_t(&ple.k, (size_t) W * hcd)); WZY_TRY(alloc_t(&ple.gat, (size_t) W * hcd));
        WZY_TRY(alloc_t(&ple.n, (size_t) W * hcd));
    }

    // RoPE tables: fp64 angles rounded to fp32 (src/wzy_qsa_256k.cuh:34-46)
    {
        const int half = c.n_rot / 2;
        std::vector<float> hc((size_t) c.ctx_max * half), hs((size_t) c.ctx_max * half);
        std::vector<double> inv(half);
        for (int i = 0; i < half; ++i) inv[i] = pow((double) c.rope_theta, -2.0 * (double) i / (double) c.n_rot);
        for (int p = 0; p < c.ctx_max; ++p)
            for (int i = 0; i < half; ++i) {
                const double ang = (double) p * inv[i];
                hc[(size_t) p * half + i] = (float) cos(ang);
                hs[(size_t) p * half + i] = (float) sin(ang);
            }
        WZY_TRY(alloc_t(&cos_tab, hc.size(), false));
        WZY_TRY(alloc_t(&sin_tab, hs.size(), false));
        WZY_HIP_TRY(hipMemcpy(cos_tab, hc.data(), hc.size() * 4, hipMemcpyHostToDevice));
        WZY_HIP_TRY(hipMemcpy(sin_tab, hs.data(), hs.size() * 4, hipMemcpyHostToDevice));
        reg(-1, "rope_cos", cos_tab, hc.size() * 4);
        reg(-1, "rope_sin", sin_tab, hs.size() * 4);
    }

    // activations
    WZY_TRY(alloc_t(&R[0], (size_t) W * HCD)); WZY_TRY(alloc_t(&R[1], (size_t) W * HCD));
    WZY_TRY(alloc_t(&nsc, (size_t) W * c.hc));
    WZY_TRY(alloc_t(&lo, (size_t) W * c.hc_lr));
    {
        void* hw = nullptr;
        WZY_TRY(alloc(&hw, hc_workspace_bytes(c.hc, c.hc_lr, W)));
        hc_carve_workspace(hw, c.hc, c.hc_lr, W, &lo_part, &inj_part);
    }
    WZY_TRY(alloc_t(&inj_a, (size_t) W * c.hc)); WZY_TRY(alloc_t(&inj_f, (size_t) W * c.hc));
    WZY_TRY(alloc_t(&mixed, (size_t) W * D));
    WZY_TRY(alloc_t(&qkv, (size_t) W * QKV)); WZY_TRY(alloc_t(&z, (size_t) W * GV));
    WZY_TRY(alloc_t(&ab, (size_t) W * 2 * c.gdn_hv)); WZY_TRY(alloc_t(&y, (size_t) W * GV));
    WZY_TRY(alloc_t(&gdn_ss, (size_t) W * c.gdn_hv * GDN_NQ));
    WZY_TRY(alloc_t(&block, (size_t) W * D)); WZY_TRY(alloc_t(&comb, (size_t) W * D));
    WZY_TRY(alloc_t(&qg, (size_t) W * 2 * QD)); WZY_TRY(alloc_t(&kk, (size_t) W * KVD)); WZY_TRY(alloc_t(&vv, (size_t) W * KVD));
    WZY_TRY(alloc_t(&idx_raw, (size_t) W * c.idx_dim)); WZY_TRY(alloc_t(&q_idx, (size_t) W * c.idx_heads * c.idx_dim));
    WZY_TRY(alloc_t(&scores, (size_t) W * max_b));
    WZY_TRY(alloc_t(&sel_ids, (size_t) W * c.idx_topk)); WZY_TRY(alloc_t(&sel_cnt, W));
    const size_t pf = qsa_attn_part_floats(qd, W);
    WZY_TRY(alloc_t(&att_part, pf)); WZY_TRY(alloc_t(&att_ml, pf / c.qsa_hd * 2));
    WZY_TRY(alloc_t(&att_out, (size_t) W * QD));
    size_t need = 0;
    moe_ws_carve(nullptr, 0, D, c.n_ff, c.n_exp, c.top_k, W, &need);
    WZY_TRY(alloc(&moe_ws, need + 256));
    mws = moe_ws_carve(moe_ws, need + 256, D, c.n_ff, c.n_exp, c.top_k, W, nullptr);
    WZY_TRY(alloc_t(&logits, (size_t) W * c.n_vocab));
    WZY_TRY(alloc(&red_ws, reduce_ws_bytes(c.n_vocab, W)));
    WZY_TRY(alloc_t(&emb_rows, (size_t) W * D));
    // activation buffers, readable after a forward (they hold the last layer that wrote them)
    reg(-1, "act.mixed", mixed, (size_t) W * D * 4);
    reg(-1, "act.block", block, (size_t) W * D * 4);
    reg(-1, "act.comb", comb, (size_t) W * D * 4);
    reg(-1, "act.qg", qg, (size_t) W * 2 * QD * 4);
    reg(-1, "act.q_idx", q_idx, (size_t) W * c.idx_heads * c.idx_dim * 4);
    reg(-1, "act.scores", scores, (size_t) W * max_b * 4);
    reg(-1, "act.sel_ids", sel_ids, (size_t) W * c.idx_topk * 4);
    reg(-1, "act.sel_cnt", sel_cnt, (size_t) W * 4);
    reg(-1, "act.att_out", att_out, (size_t) W * QD * 4);
    reg(-1, "act.gdn_o", y, (size_t) W * GV * 4);           // GDN output before its RMS norm and gate
    reg(-1, "act.gdn_ss", gdn_ss, (size_t) W * c.gdn_hv * GDN_NQ * 4);
    reg(-1, "act.moe_logits", mws.logits, (size_t) W * c.n_exp * 4);
    reg(-1, "act.moe_sg", mws.sg, (size_t) W * 4);
    reg(-1, "act.moe_ids", mws.ids, (size_t) W * c.top_k * 4);
    reg(-1, "act.moe_wts", mws.wts, (size_t) W * c.top_k * 4);
    reg(-1, "act.moe_groups", mws.n_groups, 4);
    reg(-1, "act.moe_grp_exp", mws.grp_exp, (size_t) W * c.top_k * 4);
    reg(-1, "act.moe_grp_cnt", mws.grp_cnt, (size_t) W * c.top_k * 4);
    reg(-1, "act.moe_grp_mem", mws.grp_mem, (size_t) W * c.top_k * WZY_MAX_W * 4);
    // speculative-window snapshots
    if (n_gdn > 0) {
        WZY_TRY(alloc_t(&conv_snaps, (size_t) n_gdn * W * QKV * 3));
        WZY_TRY(alloc_t(&ssm_snaps, (size_t) n_gdn * W * c.gdn_hv * 128 * 128));
    }
    if (n_qsa > 0) {
        WZY_TRY(alloc_t(&tail_snaps, (size_t) n_qsa * W * (c.idx_blk - 1) * c.idx_dim));
        WZY_TRY(alloc_t(&dead_snaps, (size_t) n_qsa * W * c.idx_dim));
        WZY_TRY(alloc_t(&pool_snaps, (size_t) n_qsa * W * 2 * c.idx_dim));
    }
    {   // copies of commit_window_state, one table entry each
        std::vector<CommitJob> jobs;
        for (const Layer& w : L) {
            if (!w.qsa) {
                const size_t sl = (size_t) w.local * W;
                jobs.push_back(CommitJob{(unsigned char*) w.conv_hist, (const unsigned char*) (conv_snaps + sl * QKV * 3),
                                         (size_t) QKV * 12, (size_t) QKV * 12, 0, 0});
                jobs.push_back(CommitJob{(unsigned char*) w.ssm,
                                         (const unsigned char*) (ssm_snaps + sl * c.gdn_hv * 128 * 128),
                                         (size_t) c.gdn_hv * 128 * 128 * 4, (size_t) c.gdn_hv * 128 * 128 * 4, 0, 0});
            } else {
                const size_t sl = (size_t) w.local * W;
                jobs.push_back(CommitJob{(unsigned char*) w.ix.tail,
                                         (const unsigned char*) (tail_snaps + sl * (c.idx_blk - 1) * c.idx_dim),
                                         (size_t) (c.idx_blk - 1) * c.idx_dim * 4, (size_t) (c.idx_blk - 1) * c.idx_dim * 4,
                                         1, 0});
                jobs.push_back(CommitJob{(unsigned char*) w.ix.dead, (const unsigned char*) (dead_snaps + sl * c.idx_dim),
                                         (size_t) c.idx_dim * 4, (size_t) c.idx_dim * 4, 1, 0});
                jobs.push_back(CommitJob{(unsigned char*) w.ix.pooled,
                                         (const unsigned char*) (pool_snaps + sl * 2 * c.idx_dim),
                                         (size_t) 2 * c.idx_dim * 2, (size_t) 2 * c.idx_dim * 2, 1, 1});
            }
        }
        if (c.ple)        // the PLE conv history of the accepted row (commit_window_state, :953-956)
            jobs.push_back(CommitJob{(unsigned char*) ple.hist, (const unsigned char*) ple.snaps,
                                     (size_t) HCD * PLE_HIST * 4, (size_t) HCD * PLE_HIST * 4, 0, 0});
        for (const CommitJob& j : jobs)
            WZY_REQUIRE(j.bytes % 16 == 0 && j.src_stride % 16 == 0, "stage: snapshot sizes must be multiples of 16 bytes");
        n_commit_jobs = (int) jobs.size();
        WZY_TRY(alloc_t(&commit_jobs, jobs.size(), false));
        WZY_HIP_TRY(hipMemcpy(commit_jobs, jobs.data(), jobs.size() * sizeof(CommitJob), hipMemcpyHostToDevice));
    }
    WZY_TRY(alloc_t(&d_step, 16));
    WZY_HIP_TRY(hipHostMalloc((void**) &h_step, STEP_SLOTS * STEP_INTS * sizeof(int), hipHostMallocDefault));
    for (auto& e : step_ev) WZY_HIP_TRY(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    WZY_HIP_TRY(hipHostMalloc((void**) &h_greedy, W * sizeof(int), hipHostMallocMapped));
    WZY_HIP_TRY(hipHostMalloc((void**) &h_top_v, W * 16 * sizeof(float), hipHostMallocMapped));
    WZY_HIP_TRY(hipHostMalloc((void**) &h_top_i, W * 16 * sizeof(int), hipHostMallocMapped));
    WZY_HIP_TRY(hipHostGetDevicePointer((void**) &d_greedy, h_greedy, 0));
    WZY_HIP_TRY(hipHostGetDevicePointer((void**) &d_top_v, h_top_v, 0));
    WZY_HIP_TRY(hipHostGetDevicePointer((void**) &d_top_i, h_top_i, 0));
    memset(h_greedy, 0, W * sizeof(int));
    for (auto& e : ev) WZY_HIP_TRY(hipEventCreate(&e));
    return WZY_OK;
}

// ------------------------------------------------------------------------------------------------
// forward enqueue
// ------------------------------------------------------------------------------------------------
int wzy_stage::enqueue(int T, bool emb_host, int run_head, bool save_snaps, bool want_top16, int snap_offset) {
    const wzy_stage_cfg& c = cfg;
    hipStream_t st = stream;
    const int* d_pos = d_step;
    const int* d_toks = d_step + 1;
    int cur = 0;                    // R buffer holding the current residual
    const float* pend_bo = nullptr;
    const float* pend_inj = nullptr;

    auto hc_read = [&](const float* norm_w, const Q8& down, const uint16_t* inj_w, const Q8& up, float* inj_out,
                       bool first) -> int {
        HcPreArgs a{};
        if (first) {
            if (emb_host) a.emb_rows = emb_rows;
            else if (c.emb_q8) { a.emb_q = emb8.q; a.emb_s = emb8.s; a.toks = d_toks; a.n_vocab = c.n_vocab; }
            else { a.emb_table = emb; a.toks = d_toks; a.n_vocab = c.n_vocab; }
        } else {
            a.R_in = R[cur];
        }
        a.bo = pend_bo; a.inj_prev = pend_inj;
        a.R_out = R[cur ^ 1];
        a.norm_w = norm_w; a.down_q = down.q; a.down_s = down.s; a.inj_w = inj_w;
        a.nsc = nsc; a.lo_part = lo_part; a.inj_part = inj_part;
        a.D = D; a.HC = c.hc; a.HCLR = c.hc_lr; a.eps = c.eps;
        WZY_TRY(launch_hc_pre(a, T, st));
        cur ^= 1;
        HcPostArgs b{};
        b.R = R[cur]; b.nsc = nsc; b.norm_w = norm_w; b.up_q = up.q; b.up_s = up.s; b.lo_part = lo_part;
        b.inj_part = inj_out ? inj_part : nullptr; b.lo = lo; b.inj = inj_out; b.mixed = mixed;
        b.D = D; b.HC = c.hc; b.HCLR = c.hc_lr;
        return launch_hc_post(b, T, st);
    };

    // trace copies (direct launches only): n elements of `src` into row block (slot, 0..T) of `dst`
    auto tr = [&](void* dst, const void* src, int slot, size_t per_row, size_t elt) -> int {
        if (!trace) return WZY_OK;
        WZY_HIP_TRY(hipMemcpyAsync((char*) dst + ((size_t) slot * WZY_MAX_W) * per_row * elt, src,
                                   (size_t) T * per_row * elt, hipMemcpyDeviceToDevice, st));
        return WZY_OK;
    };

    for (int l = 0; l < c.n_layers; ++l) {
        Layer& w = L[l];
        if (l == 1 && c.ple) {
            // per-layer embedding (src/wzy_stage_v2.cuh:583-597): the table rows of the window's
            // 3-gram contexts, their k / v projections, then the block folds layer 0's pending FFN
            // write into the streams and adds to them; the attention read below folds nothing
            PleRowsArgs pr{};
            pr.table = ple.table; pr.head = D / PLE_HEADS; pr.scale_dev = ple.scale_dev; pr.eos = c.ple_eos;
            pr.pos = d_pos; pr.toks = d_toks; pr.tok_hist = ple.tok_hist; pr.ctx_max = c.ctx_max; pr.emb = ple.emb;
            WZY_TRY(launch_ple_rows(pr, T, st));
            GemvSegs s;
            s.n = 2;
            s.seg[0] = GemvSeg{ple.wk, nullptr, ple.k, HCD, GEMV_BF16, HCD, 0};
            s.seg[1] = GemvSeg{ple.wv, nullptr, ple.v, D, GEMV_BF16, D, 0};
            WZY_TRY(launch_gemv_segs(s, ple.emb, D, T, st));
            PleBlockArgs b{};
            b.R = R[cur]; b.bo = pend_bo; b.inj_prev = pend_inj; b.k = ple.k; b.v = ple.v;
            b.norm_q = ple.nq; b.norm_k = ple.nk; b.norm_c = ple.nc; b.conv_w = ple.cw; b.hist = ple.hist;
            b.hist_snaps = save_snaps ? ple.snaps + (size_t) snap_offset * HCD * PLE_HIST : nullptr;
            b.gat = ple.gat; b.n = ple.n; b.D = D; b.HC = c.hc; b.eps = c.eps;
            WZY_TRY(launch_ple_mix(b, T, st));
            WZY_TRY(launch_ple_conv(b, T, st));
            pend_bo = nullptr;
            pend_inj = nullptr;
        }
        // ---------------- attention half ----------------
        WZY_TRY(hc_read(w.hc_norm[0], w.hc_down[0], w.hc_inj[0], w.hc_up[0], inj_a, l == 0));
        WZY_TRY(tr(tr_mixa, mixed, l, D, 4));
        WZY_TRY(tr(tr_ra, R[cur], l, HCD, 4));
        WZY_TRY(tr(tr_inja, inj_a, l, c.hc, 4));
        if (!w.qsa) {
            GemvSegs s;
            s.n = 4;
            s.seg[0] = GemvSeg{w.qkv.q, w.qkv.s, qkv, QKV, GEMV_Q8, QKV, 0};
            s.seg[1] = GemvSeg{w.wgate.q, w.wgate.s, z, GV, GEMV_Q8, GV, 0, GEMV_ACT_SIGMOID};   // z holds sigmoid(z)
            s.seg[2] = GemvSeg{w.alpha, nullptr, ab, c.gdn_hv, GEMV_BF16, 2 * c.gdn_hv, 0};
            s.seg[3] = GemvSeg{w.beta, nullptr, ab + c.gdn_hv, c.gdn_hv, GEMV_BF16, 2 * c.gdn_hv, 0};
            WZY_TRY(launch_gemv_segs(s, mixed, D, T, st));
            GdnArgs g{};
            g.qkv = qkv; g.ab = ab; g.dt = w.dt; g.ssm_a = w.ssm_a; g.conv_w = w.conv_w; g.conv_hist = w.conv_hist;
            g.z = z; g.gamma = w.ssm_norm; g.eps = c.eps; g.state = w.ssm; g.y = y; g.o_ss = gdn_ss;
            g.hk = c.gdn_hk; g.hv = c.gdn_hv; g.S = 128; g.T = T;
            if (save_snaps) {
                g.hist_snaps = conv_snaps + ((size_t) w.local * WZY_MAX_W + snap_offset) * QKV * 3;
                g.state_snaps = ssm_snaps + ((size_t) w.local * WZY_MAX_W + snap_offset) * c.gdn_hv * 128 * 128;
            }
            WZY_TRY(launch_gdn(g, true, st));
            GemvSegs o;
            o.n = 1;
            o.seg[0] = GemvSeg{w.wout.q, w.wout.s, block, D, GEMV_Q8, D, 0};
            o.gdn.ss = gdn_ss; o.gdn.z = z; o.gdn.z_is_gate = true;             // RMS norm + gate of y
            o.gdn.gamma = w.ssm_norm; o.gdn.eps = c.eps;
            WZY_TRY(launch_gemv_segs(o, y, GV, T, st));
        } else {
            GemvSegs s;
            s.n = 5;
            s.seg[0] = GemvSeg{w.wq.q, w.wq.s, qg, 2 * QD, GEMV_Q8, 2 * QD, 0};
            s.seg[1] = GemvSeg{w.wk.q, w.wk.s, kk, KVD, GEMV_Q8, KVD, 0};
            s.seg[2] = GemvSeg{w.wv.q, w.wv.s, vv, KVD, GEMV_Q8, KVD, 0};
            s.seg[3] = GemvSeg{w.idx_k, nullptr, idx_raw, c.idx_dim, GEMV_BF16, c.idx_dim, 0};
            s.seg[4] = GemvSeg{w.idx_q, nullptr, q_idx, c.idx_heads * c.idx_dim, GEMV_BF16, c.idx_heads * c.idx_dim, 0};
            WZY_TRY(launch_gemv_segs(s, mixed, D, T, st));
            QsaPrepArgs p{};
            p.dm = qd; p.pos = d_pos; p.qg = qg; p.kk = kk; p.vv = vv; p.q_idx = q_idx; p.idx_raw = idx_raw;
            p.q_norm = w.q_norm; p.k_norm = w.k_norm; p.iq_norm = w.idx_qn; p.ik_norm = w.idx_kn;
            p.cos_tab = cos_tab; p.sin_tab = sin_tab; p.kv = w.kv; p.ix = w.ix;
            if (save_snaps) {
                const size_t sl = (size_t) w.local * WZY_MAX_W + snap_offset;
                p.ix.tail_snaps = tail_snaps + sl * (c.idx_blk - 1) * c.idx_dim;
                p.ix.dead_snaps = dead_snaps + sl * c.idx_dim;
                p.ix.pool_snaps = pool_snaps + sl * 2 * c.idx_dim;
            }
            WZY_TRY(launch_qsa_prep(p, T, st));
            WZY_TRY(tr(tr_kk, kk, w.local, KVD, 4));
            WZY_TRY(tr(tr_vv, vv, w.local, KVD, 4));
            WZY_TRY(tr(tr_iraw, idx_raw, w.local, c.idx_dim, 4));
            WZY_TRY(tr(tr_qg, qg, w.local, 2 * QD, 4));
            QsaScoreArgs sa{};
            sa.dm = qd; sa.pos = d_pos; sa.pooled = w.ix.pooled; sa.dead = w.ix.dead; sa.q_idx = q_idx;
            sa.scores = scores; sa.max_b = max_b;
            WZY_TRY(launch_qsa_score(sa, T, st));
            WZY_TRY(launch_qsa_topk(qd, d_pos, scores, max_b, sel_ids, sel_cnt, T, st));
            WZY_TRY(tr(tr_scores, scores, w.local, max_b, 4));
            WZY_TRY(tr(tr_sel, sel_ids, w.local, c.idx_topk, 4));
            WZY_TRY(tr(tr_cnt, sel_cnt, w.local, 1, 4));
            QsaAttnArgs at{};
            at.dm = qd; at.pos = d_pos; at.qg = qg; at.kv = w.kv; at.sel_ids = sel_ids; at.part = att_part;
            at.part_ml = att_ml; at.out = att_out;
            WZY_TRY(launch_qsa_attn(at, T, st));
            WZY_TRY(tr(tr_att, att_out, w.local, QD, 4));
            GemvSegs o;
            o.n = 1;
            o.seg[0] = GemvSeg{w.wo.q, w.wo.s, block, D, GEMV_Q8, D, 0};
            WZY_TRY(launch_gemv_segs(o, att_out, QD, T, st));
        }
        WZY_TRY(tr(tr_block, block, l, D, 4));
        pend_bo = block;
        pend_inj = inj_a;
        // ---------------- FFN half ----------------
        WZY_TRY(hc_read(w.hc_norm[1], w.hc_down[1], w.hc_inj[1], w.hc_up[1], inj_f, false));
        WZY_TRY(tr(tr_mixf, mixed, l, D, 4));
        WZY_TRY(tr(tr_rf, R[cur], l, HCD, 4));
        WZY_TRY(tr(tr_injf, inj_f, l, c.hc, 4));
        WZY_TRY(moe_launch_route(&w.moe, mws, mixed, T, st));
        WZY_TRY(moe_launch_experts(&w.moe, mws, mixed, T, comb, st));
        WZY_TRY(tr(tr_logits, mws.logits, l, c.n_exp, 4));
        WZY_TRY(tr(tr_ids, mws.ids, l, c.top_k, 4));
        WZY_TRY(tr(tr_wts, mws.wts, l, c.top_k, 4));
        WZY_TRY(tr(tr_comb, comb, l, D, 4));
        pend_bo = comb;
        pend_inj = inj_f;
    }
    if (run_head) {
        WZY_TRY(hc_read(head_norm, head_down, nullptr, head_up, nullptr, false));
        r_pre_head = cur;
        if (run_head == 2) return WZY_OK;          // pre-head residual only (MTP seeding)
        GemvSegs h;
        h.n = 1;
        h.seg[0] = c.head_q8 ? GemvSeg{head8.q, head8.s, logits, c.n_vocab, GEMV_Q8, c.n_vocab, 0}
                             : GemvSeg{head, nullptr, logits, c.n_vocab, GEMV_BF16, c.n_vocab, 0};
        WZY_TRY(launch_gemv_segs(h, mixed, D, T, st));
        WZY_TRY(launch_row_reduce(logits, c.n_vocab, T, want_top16, d_greedy, want_top16 ? d_top_v : nullptr,
                                  want_top16 ? d_top_i : nullptr, red_ws, st));
    }
    return WZY_OK;
}

// ------------------------------------------------------------------------------------------------
// synthetic model
// ------------------------------------------------------------------------------------------------
namespace {
struct Gen {
    wzy_stage* s;
    uint64_t seed;
    std::vector<char> buf;
    int upload(void* dst, const void* src, size_t bytes) {
        WZY_HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
        return WZY_OK;
    }
    uint64_t stream(uint32_t kind, int layer, uint32_t sub) {
        return wzy_stream(kind, layer < 0 ? MODEL_LAYER : (uint32_t) layer, sub);
    }
    int normal_f32(float* dst, size_t n, int layer, uint32_t id, float mean, float sd, uint32_t kind = WZY_S_DENSE) {
        buf.resize(n * 4);
        wzy_synth_normal(seed, stream(kind, layer, id), n, mean, sd, (float*) buf.data());
        return upload(dst, buf.data(), n * 4);
    }
    int uniform_f32(float* dst, size_t n, int layer, uint32_t id, float lo, float hi) {
        buf.resize(n * 4);
        wzy_synth_uniform(seed, stream(WZY_S_DENSE, layer, id), n, lo, hi, (float*) buf.data());
        return upload(dst, buf.data(), n * 4);
    }
    int normal_bf16(uint16_t* dst, size_t n, int layer, uint32_t id, float sd) {
        buf.resize(n * 2);
        wzy_synth_normal_bf16(seed, stream(WZY_S_DENSE, layer, id), n, 0.f, sd, (uint16_t*) buf.data());
        return upload(dst, buf.data(), n * 2);
    }
    // Q8_0 rows of scale `sd` (default 1/sqrt(cols))
    int q8(const Q8& m, int layer, uint32_t id, float sd = 0.f) {
        const size_t n = (size_t) m.rows * m.cols;
        buf.resize(n + n / 32 * 2);
        wzy_synth_q8(seed, stream(WZY_S_DENSE, layer, id), m.rows, m.cols, sd > 0.f ? sd : (float) (1.0 / sqrt((double) m.cols)),
                     (int8_t*) buf.data(), (uint16_t*) (buf.data() + n));
        WZY_TRY(upload(m.q, buf.data(), n));
        return upload(m.s, buf.data() + n, n / 32 * 2);
    }
};
}  // namespace

static int load_synthetic(wzy_stage* s, uint64_t seed, int n_ctx) {
    const wzy_stage_cfg& c = s->cfg;
    WZY_REQUIRE(n_ctx >= 0 && n_ctx < c.ctx_max, "load_synthetic: n_ctx must be in [0, ctx_max)");
    WZY_HIP_TRY(hipSetDevice(s->dev));
    Gen g{s, seed, {}};
    const int D = s->D;
    for (int l = 0; l < c.n_layers; ++l) {
        Layer& w = s->L[l];
        for (int h = 0; h < 2; ++h) {
            WZY_TRY(g.normal_f32(w.hc_norm[h], s->HCD, l, TI_HC_NORM + 10 * h, 1.0f, 0.02f));
            WZY_TRY(g.q8(w.hc_down[h], l, TI_HC_DOWN + 10 * h));
            WZY_TRY(g.q8(w.hc_up[h], l, TI_HC_UP + 10 * h));
            WZY_TRY(g.normal_bf16(w.hc_inj[h], (size_t) c.hc * s->HCD, l, TI_HC_INJ + 10 * h,
                                  (float) (1.0 / sqrt((double) s->HCD))));
        }
        if (!w.qsa) {
            WZY_TRY(g.q8(w.qkv, l, TI_QKV));
            WZY_TRY(g.q8(w.wgate, l, TI_WGATE));
            WZY_TRY(g.q8(w.wout, l, TI_WOUT));
            WZY_TRY(g.normal_bf16(w.alpha, (size_t) c.gdn_hv * D, l, TI_ALPHA, (float) (1.0 / sqrt((double) D))));
            WZY_TRY(g.normal_bf16(w.beta, (size_t) c.gdn_hv * D, l, TI_BETA, (float) (1.0 / sqrt((double) D))));
            WZY_TRY(g.uniform_f32(w.ssm_a, c.gdn_hv, l, TI_SSM_A, -2.0f, -1.0f));
            WZY_TRY(g.normal_f32(w.dt, c.gdn_hv, l, TI_DT, -3.0f, 0.5f));
            WZY_TRY(g.normal_f32(w.conv_w, (size_t) s->QKV * 4, l, TI_CONV, 0.0f, 0.5f));
            WZY_TRY(g.normal_f32(w.ssm_norm, 128, l, TI_SSM_NORM, 1.0f, 0.02f));
            // prefilled recurrent state
            WZY_TRY(g.normal_f32(w.conv_hist, (size_t) s->QKV * 3, l, TS_CONV, 0.0f, 1.0f, WZY_S_STATE));
            WZY_TRY(g.normal_f32(w.ssm, (size_t) c.gdn_hv * 128 * 128, l, TS_SSM, 0.0f, 0.1f, WZY_S_STATE));
        } else {
            WZY_TRY(g.q8(w.wq, l, TI_WQ));
            WZY_TRY(g.q8(w.wk, l, TI_WK));
            WZY_TRY(g.q8(w.wv, l, TI_WV));
            WZY_TRY(g.q8(w.wo, l, TI_WO));
            WZY_TRY(g.normal_f32(w.q_norm, c.qsa_hd, l, TI_QNORM, 1.0f, 0.02f));
            WZY_TRY(g.normal_f32(w.k_norm, c.qsa_hd, l, TI_KNORM, 1.0f, 0.02f));
            WZY_TRY(g.normal_bf16(w.idx_q, (size_t) c.idx_heads * c.idx_dim * D, l, TI_IDXQ, (float) (1.0 / sqrt((double) D))));
            WZY_TRY(g.normal_bf16(w.idx_k, (size_t) c.idx_dim * D, l, TI_IDXK, (float) (1.0 / sqrt((double) D))));
            WZY_TRY(g.normal_f32(w.idx_qn, c.idx_dim, l, TI_IDXQN, 1.0f, 0.02f));
            WZY_TRY(g.normal_f32(w.idx_kn, c.idx_dim, l, TI_IDXKN, 1.0f, 0.02f));
            // prefilled context: INT8 KV cells 0..n_ctx-1, indexer keys of complete blocks,
            // placeholder key, partial-block tail
            if (n_ctx > 0) {
                // a stage's KV ring never wraps (validate), so cell p is slot p
                WZY_TRY(wzy_synth_kv_device(seed, l, 0, 0, n_ctx, s->KVD, w.kv.kq, w.kv.ks, s->stream));
                WZY_TRY(wzy_synth_kv_device(seed, l, 1, 0, n_ctx, s->KVD, w.kv.vq, w.kv.vs, s->stream));
            }
            const int nblk = n_ctx / c.idx_blk;
            std::vector<float> keys((size_t) (nblk + 1) * c.idx_dim);
            wzy_synth_normal(seed, g.stream(WZY_S_STATE, l, TS_POOLED), keys.size(), 0.0f, 1.0f, keys.data());
            std::vector<uint16_t> k16((size_t) s->max_b * c.idx_dim, 0);
            for (size_t i = 0; i < keys.size(); ++i) k16[i] = wzy_f32_to_f16(keys[i]);
            WZY_TRY(g.normal_f32(w.ix.dead, c.idx_dim, l, TS_DEAD, 0.0f, 1.0f, WZY_S_STATE));
            std::vector<float> dead(c.idx_dim);
            WZY_HIP_TRY(hipMemcpy(dead.data(), w.ix.dead, c.idx_dim * 4, hipMemcpyDeviceToHost));
            if (n_ctx > 0)
                for (int d = 0; d < c.idx_dim; ++d) k16[(size_t) nblk * c.idx_dim + d] = wzy_f32_to_f16(dead[d]);
            WZY_TRY(g.upload(w.ix.pooled, k16.data(), k16.size() * 2));
            WZY_TRY(g.normal_f32(w.ix.tail, (size_t) (c.idx_blk - 1) * c.idx_dim, l, TS_TAIL, 0.0f, 1.0f, WZY_S_STATE));
        }
        WZY_TRY(g.normal_bf16((uint16_t*) w.moe.router, (size_t) c.n_exp * D, l, TI_ROUTER, 0.02f));
        WZY_TRY(g.normal_bf16((uint16_t*) w.moe.sgate, D, l, TI_SGATE, 0.02f));
        Q8 m;
        m.rows = c.n_ff; m.cols = D;
        m.q = (int8_t*) w.moe.sh_gate_q; m.s = (uint16_t*) w.moe.sh_gate_s;
        WZY_TRY(g.q8(m, l, TI_SH_GATE));
        m.q = (int8_t*) w.moe.sh_up_q; m.s = (uint16_t*) w.moe.sh_up_s;
        WZY_TRY(g.q8(m, l, TI_SH_UP));
        m.rows = D; m.cols = c.n_ff;
        m.q = (int8_t*) w.moe.sh_down_q; m.s = (uint16_t*) w.moe.sh_down_s;
        WZY_TRY(g.q8(m, l, TI_SH_DOWN));
        for (int e0 = 0; e0 < c.n_exp; e0 += 4096) {
            const int ne = std::min(4096, c.n_exp - e0);
            WZY_TRY(wzy_synth_experts_device(seed, l, e0, ne, D, c.n_ff, (uint8_t*) w.moe.experts + (size_t) e0 * s->expert_rec,
                                             s->stream));
        }
    }
    if (c.ple) {
        auto& p = s->ple;
        const size_t hcd = (size_t) s->HCD;
        const float sd = (float) (1.0 / sqrt((double) D));
        WZY_TRY(g.normal_bf16(p.wk, hcd * D, 1, TI_PLE_K, sd));
        WZY_TRY(g.normal_bf16(p.wv, (size_t) D * D, 1, TI_PLE_V, sd));
        WZY_TRY(g.normal_f32(p.nq, hcd, 1, TI_PLE_NQ, 1.0f, 0.02f));
        WZY_TRY(g.normal_f32(p.nk, hcd, 1, TI_PLE_NK, 1.0f, 0.02f));
        WZY_TRY(g.normal_f32(p.nc, hcd, 1, TI_PLE_NC, 1.0f, 0.02f));
        WZY_TRY(g.normal_f32(p.cw, hcd * 4, 1, TI_PLE_CONV, 0.0f, 0.5f));
        WZY_TRY(wzy_synth_ple_table_device(seed, D / PLE_HEADS, p.table, s->stream));
        const float scale = 0.125f;
        WZY_TRY(g.upload(p.scale_dev, &scale, 4));
        p.table_ready = true;
        // prefilled context: a conv history and the tokens of cells 0 .. n_ctx-1
        WZY_TRY(g.normal_f32(p.hist, hcd * PLE_HIST, 1, TS_PLE_HIST, 0.0f, 1.0f, WZY_S_STATE));
        std::vector<int> toks((size_t) n_ctx + 1);
        for (int i = 0; i < n_ctx; ++i)
            toks[i] = (int) (wzy_synth_hash(seed, g.stream(WZY_S_STATE, 1, TS_PLE_TOKS), (uint64_t) i) % (uint64_t) c.n_vocab);
        if (n_ctx > 0) WZY_TRY(g.upload(p.tok_hist, toks.data(), (size_t) n_ctx * 4));
    }
    if (c.emb_q8) WZY_TRY(g.q8(s->emb8, -1, TI_EMB, 1.0f));
    else WZY_TRY(g.normal_bf16(s->emb, (size_t) c.n_vocab * D, -1, TI_EMB, 1.0f));
    WZY_TRY(g.normal_f32(s->head_norm, s->HCD, -1, TI_HEAD_NORM, 1.0f, 0.02f));
    WZY_TRY(g.q8(s->head_down, -1, TI_HEAD_DOWN));
    WZY_TRY(g.q8(s->head_up, -1, TI_HEAD_UP));
    if (c.head_q8) WZY_TRY(g.q8(s->head8, -1, TI_HEAD));
    else WZY_TRY(g.normal_bf16(s->head, (size_t) c.n_vocab * D, -1, TI_HEAD, (float) (1.0 / sqrt((double) D))));
    WZY_HIP_TRY(hipStreamSynchronize(s->stream));
    s->loaded = true;
    // an empty context has no history: recurrent state and indexer tail start at zero
    if (n_ctx == 0) {
        WZY_TRY(wzy_stage_reset_state(s));
        WZY_HIP_TRY(hipStreamSynchronize(s->stream));
    }
    return WZY_OK;
}

// ------------------------------------------------------------------------------------------------
// C ABI
// ------------------------------------------------------------------------------------------------
extern "C" void wzy_stage_cfg_default(wzy_stage_cfg* c, int ctx_max) {
    memset(c, 0, sizeof *c);
    c->n_layers = 48; c->qsa_period = 4; c->n_embd = 2048; c->hc = 4; c->hc_lr = 320;
    c->gdn_hk = 16; c->gdn_hv = 16; c->qsa_qh = 24; c->qsa_kvh = 2; c->qsa_hd = 256; c->n_rot = 64;
    c->idx_heads = 4; c->idx_dim = 128; c->idx_blk = 4; c->idx_topk = 2048;
    c->n_exp = 512; c->top_k = 10; c->n_ff = 512; c->n_vocab = 151936;
    c->ctx_max = ctx_max; c->kv_ring = 0; c->kv_sinks = 0; c->rope_theta = 1e7f; c->eps = 1e-6f;
    c->attn_f16_above = 32768;
    c->ple = 0; c->ple_eos = PLE_EOS_DEFAULT;
}

extern "C" int wzy_stage_create(const wzy_stage_cfg* cfg, int device, wzy_stage** out) {
    WZY_REQUIRE(cfg && out, "wzy_stage_create: null argument");
    *out = nullptr;
    WZY_TRY(validate(*cfg));
    WZY_HIP_TRY(hipSetDevice(device));
    std::unique_ptr<wzy_stage> s(new wzy_stage());
    s->cfg = *cfg;
    s->dev = device;
    WZY_HIP_TRY(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking));
    WZY_TRY(s->init_buffers());
    *out = s.release();
    return WZY_OK;
}

extern "C" int wzy_stage_destroy(wzy_stage* st) {
    delete st;
    return WZY_OK;
}

extern "C" size_t wzy_stage_device_bytes(const wzy_stage* st) { return st ? st->dev_bytes : 0; }

extern "C" int wzy_stage_load_synthetic(wzy_stage* st, uint64_t seed, int n_ctx) {
    WZY_REQUIRE(st, "wzy_stage_load_synthetic: null stage");
    return load_synthetic(st, seed, n_ctx);
}

extern "C" int wzy_stage_record_forward(wzy_stage* st, int pos, const float* emb, const int* toks, int T, int run_head,
                                        int save_snaps, int want_top16, int snap_offset) {
    WZY_REQUIRE(st && st->loaded, "record_forward: stage not loaded");
    WZY_REQUIRE(T >= 1 && T <= WZY_MAX_W, "record_forward: T must be in [1, %d]", WZY_MAX_W);
    WZY_REQUIRE(emb || toks, "record_forward: need token ids or embedding rows");
    WZY_REQUIRE(!st->cfg.ple || toks, "record_forward: the per-layer embedding needs the window's token ids");
    WZY_REQUIRE(!st->cfg.ple || st->ple.table_ready, "record_forward: the per-layer embedding table is not loaded");
    WZY_REQUIRE(pos >= 0 && pos + T <= st->cfg.ctx_max, "record_forward: positions [%d, %d) exceed ctx_max %d", pos,
                pos + T, st->cfg.ctx_max);
    WZY_REQUIRE(!save_snaps || (snap_offset >= 0 && snap_offset + T <= WZY_MAX_W), "record_forward: bad snap_offset");
    WZY_HIP_TRY(hipSetDevice(st->dev));
    const int slot = st->step_slot;
    st->step_slot = (slot + 1) % wzy_stage::STEP_SLOTS;
    if (st->step_pending[slot]) WZY_HIP_TRY(hipEventSynchronize(st->step_ev[slot]));
    int* hs = st->h_step + (size_t) slot * wzy_stage::STEP_INTS;
    hs[0] = pos;
    for (int t = 0; t < WZY_MAX_W; ++t) hs[1 + t] = (toks && t < T) ? toks[t] : 0;
    WZY_HIP_TRY(hipMemcpyAsync(st->d_step, hs, (1 + WZY_MAX_W) * sizeof(int), hipMemcpyHostToDevice, st->stream));
    WZY_HIP_TRY(hipEventRecord(st->step_ev[slot], st->stream));
    st->step_pending[slot] = true;
    if (emb) WZY_HIP_TRY(hipMemcpyAsync(st->emb_rows, emb, (size_t) T * st->D * 4, hipMemcpyHostToDevice, st->stream));
    WZY_REQUIRE(run_head >= 0 && run_head <= 2, "record_forward: run_head must be 0, 1 or 2");
    st->last_T = T;
    st->have_head = run_head == 1;
    st->have_pre_head = run_head != 0;
    st->pre_head_pf = false;
    const bool use_graph = st->graphs && !st->profiling && !st->trace;
    if (!use_graph) return st->enqueue(T, emb != nullptr, run_head, save_snaps, want_top16, snap_offset);
    const unsigned long long key = ((unsigned long long) T << 16) | ((unsigned long long) snap_offset << 8) |
                                   (emb ? 16ull : 0ull) | ((unsigned long long) run_head << 2) | (want_top16 ? 2ull : 0ull) |
                                   (save_snaps ? 1ull : 0ull);
    auto it = st->graph_execs.find(key);
    if (it == st->graph_execs.end()) {
        WZY_HIP_TRY(hipStreamBeginCapture(st->stream, hipStreamCaptureModeThreadLocal));
        const int rc = st->enqueue(T, emb != nullptr, run_head, save_snaps, want_top16, snap_offset);
        hipGraph_t g = nullptr;
        const hipError_t e = hipStreamEndCapture(st->stream, &g);
        if (rc != WZY_OK) {
            if (g) (void) hipGraphDestroy(g);
            return rc;
        }
        if (e != hipSuccess) {
            set_error("record_forward: graph capture failed: %s", hipGetErrorString(e));
            return WZY_EHIP;
        }
        hipGraphExec_t ex = nullptr;
        const hipError_t ie = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
        (void) hipGraphDestroy(g);
        if (ie != hipSuccess) {
            set_error("record_forward: graph instantiate failed: %s", hipGetErrorString(ie));
            return WZY_EHIP;
        }
        it = st->graph_execs.emplace(key, ex).first;
    }
    WZY_HIP_TRY(hipGraphLaunch(it->second, st->stream));
    return WZY_OK;
}

int wzy_stage::trace_alloc() {
    if (tr_mixa) return WZY_OK;
    const wzy_stage_cfg& c = cfg;
    const size_t W = WZY_MAX_W, nl = (size_t) c.n_layers, nq = (size_t) (n_qsa > 0 ? n_qsa : 1);
    WZY_TRY(alloc_t(&tr_mixa, nl * W * D)); reg(-1, "trace.mixed_a", tr_mixa, nl * W * D * 4);
    WZY_TRY(alloc_t(&tr_block, nl * W * D)); reg(-1, "trace.block", tr_block, nl * W * D * 4);
    WZY_TRY(alloc_t(&tr_mixf, nl * W * D)); reg(-1, "trace.mixed_f", tr_mixf, nl * W * D * 4);
    WZY_TRY(alloc_t(&tr_comb, nl * W * D)); reg(-1, "trace.comb", tr_comb, nl * W * D * 4);
    WZY_TRY(alloc_t(&tr_ra, nl * W * HCD)); reg(-1, "trace.R_a", tr_ra, nl * W * HCD * 4);
    WZY_TRY(alloc_t(&tr_rf, nl * W * HCD)); reg(-1, "trace.R_f", tr_rf, nl * W * HCD * 4);
    WZY_TRY(alloc_t(&tr_inja, nl * W * c.hc)); reg(-1, "trace.inj_a", tr_inja, nl * W * c.hc * 4);
    WZY_TRY(alloc_t(&tr_injf, nl * W * c.hc)); reg(-1, "trace.inj_f", tr_injf, nl * W * c.hc * 4);
    WZY_TRY(alloc_t(&tr_logits, nl * W * c.n_exp)); reg(-1, "trace.moe_logits", tr_logits, nl * W * c.n_exp * 4);
    WZY_TRY(alloc_t(&tr_ids, nl * W * c.top_k)); reg(-1, "trace.moe_ids", tr_ids, nl * W * c.top_k * 4);
    WZY_TRY(alloc_t(&tr_wts, nl * W * c.top_k)); reg(-1, "trace.moe_wts", tr_wts, nl * W * c.top_k * 4);
    WZY_TRY(alloc_t(&tr_scores, nq * W * max_b)); reg(-1, "trace.scores", tr_scores, nq * W * max_b * 4);
    WZY_TRY(alloc_t(&tr_sel, nq * W * c.idx_topk)); reg(-1, "trace.sel_ids", tr_sel, nq * W * c.idx_topk * 4);
    WZY_TRY(alloc_t(&tr_cnt, nq * W)); reg(-1, "trace.sel_cnt", tr_cnt, nq * W * 4);
    WZY_TRY(alloc_t(&tr_kk, nq * W * KVD)); reg(-1, "trace.kv_k_in", tr_kk, nq * W * KVD * 4);
    WZY_TRY(alloc_t(&tr_vv, nq * W * KVD)); reg(-1, "trace.kv_v_in", tr_vv, nq * W * KVD * 4);
    WZY_TRY(alloc_t(&tr_iraw, nq * W * c.idx_dim)); reg(-1, "trace.idx_raw", tr_iraw, nq * W * c.idx_dim * 4);
    WZY_TRY(alloc_t(&tr_qg, nq * W * 2 * QD)); reg(-1, "trace.qg", tr_qg, nq * W * 2 * QD * 4);
    WZY_TRY(alloc_t(&tr_att, nq * W * QD)); reg(-1, "trace.attn", tr_att, nq * W * QD * 4);
    return WZY_OK;
}

extern "C" int wzy_stage_set_trace(wzy_stage* st, int enable) {
    WZY_REQUIRE(st, "set_trace: null stage");
    WZY_HIP_TRY(hipSetDevice(st->dev));
    if (enable) WZY_TRY(st->trace_alloc());
    st->trace = enable != 0;
    return WZY_OK;
}

extern "C" int wzy_stage_service_cold_layers(wzy_stage* st) { return st ? WZY_OK : WZY_EINVAL; }
extern "C" int wzy_stage_promote_cold(wzy_stage* st) { return st ? WZY_OK : WZY_EINVAL; }

extern "C" int wzy_stage_commit_window_state(wzy_stage* st, int acc_idx, int acc_pos) {
    WZY_REQUIRE(st && acc_idx >= 0 && acc_idx < WZY_MAX_W, "commit_window_state: bad arguments");
    WZY_REQUIRE(acc_pos < st->cfg.ctx_max, "commit_window_state: acc_pos beyond ctx_max");
    const wzy_stage_cfg& c = st->cfg;
    WZY_HIP_TRY(hipSetDevice(st->dev));
    if (st->n_commit_jobs == 0) return WZY_OK;
    // every snapshot copy in one launch (GDN conv history + state; indexer tail, placeholder, pooled
    // keys of the block holding acc_pos)
    hipLaunchKernelGGL(commit_kernel, dim3(COMMIT_WGS, st->n_commit_jobs), dim3(256), 0, st->stream, st->commit_jobs,
                       acc_idx, acc_pos, c.idx_blk, c.idx_dim * 2);
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

extern "C" int wzy_stage_reset_state(wzy_stage* st) {
    WZY_REQUIRE(st, "reset_state: null stage");
    const wzy_stage_cfg& c = st->cfg;
    WZY_HIP_TRY(hipSetDevice(st->dev));
    for (Layer& w : st->L) {
        if (!w.qsa) {
            WZY_HIP_TRY(hipMemsetAsync(w.conv_hist, 0, (size_t) st->QKV * 12, st->stream));
            WZY_HIP_TRY(hipMemsetAsync(w.ssm, 0, (size_t) c.gdn_hv * 128 * 128 * 4, st->stream));
        } else {
            WZY_HIP_TRY(hipMemsetAsync(w.ix.tail, 0, (size_t) (c.idx_blk - 1) * c.idx_dim * 4, st->stream));
            WZY_HIP_TRY(hipMemsetAsync(w.ix.dead, 0, (size_t) c.idx_dim * 4, st->stream));
        }
    }
    if (c.ple) WZY_HIP_TRY(hipMemsetAsync(st->ple.hist, 0, (size_t) st->HCD * PLE_HIST * 4, st->stream));
    WZY_HIP_TRY(hipStreamSynchronize(st->stream));
    return WZY_OK;
}

// The device regions of a session of n_cells cells, in a fixed order (save and restore walk the
// same list): GDN conv history + state per GDN layer; per QSA layer the indexer tail, placeholder,
// the pooled keys of blocks 0 .. n_cells/idx_blk + 1 (the last closed block and the open one), and
// the K/V codes and scales of cells 0 .. n_cells-1; then the drafter's KV ring and floor.
// reference: save_session_state (src/wzy_engine_v2.cu:1660-1749).
void wzy_stage::session_regions(int n_cells, std::vector<std::pair<void*, size_t>>& out) const {
    const wzy_stage_cfg& c = cfg;
    out.clear();
    const size_t nc = (size_t) n_cells;
    const size_t blocks = std::min((size_t) max_b, nc / (size_t) c.idx_blk + 2);
    for (const Layer& w : L) {
        if (!w.qsa) {
            out.emplace_back(w.conv_hist, (size_t) QKV * 3 * 4);
            out.emplace_back(w.ssm, (size_t) c.gdn_hv * 128 * 128 * 4);
        } else {
            out.emplace_back(w.ix.tail, (size_t) (c.idx_blk - 1) * c.idx_dim * 4);
            out.emplace_back(w.ix.dead, (size_t) c.idx_dim * 4);
            out.emplace_back(w.ix.pooled, blocks * c.idx_dim * 2);
            if (nc > 0) {
                out.emplace_back(w.kv.kq, nc * KVD);
                out.emplace_back(w.kv.ks, nc * (KVD / 64) * 2);
                out.emplace_back(w.kv.vq, nc * KVD);
                out.emplace_back(w.kv.vs, nc * (KVD / 64) * 2);
            }
        }
    }
    if (c.ple) {                    // the PLE conv history and the tokens of the session's cells
        out.emplace_back(ple.hist, (size_t) HCD * PLE_HIST * 4);
        out.emplace_back(ple.tok_hist, nc * 4);
    }
    if (mtp) {
        const size_t kvd = (size_t) mtp->c.kvh * mtp->c.hd;
        out.emplace_back(mtp->kv.kq, (size_t) MTP_RING * kvd);
        out.emplace_back(mtp->kv.ks, (size_t) MTP_RING * (kvd / 64) * 2);
        out.emplace_back(mtp->kv.vq, (size_t) MTP_RING * kvd);
        out.emplace_back(mtp->kv.vs, (size_t) MTP_RING * (kvd / 64) * 2);
        out.emplace_back(mtp->d_floor, sizeof(int));
    }
}

static size_t session_total(const std::vector<std::pair<void*, size_t>>& regs) {
    size_t t = 0;
    for (const auto& r : regs) t += (r.second + 255) & ~(size_t) 255;
    return t;
}

extern "C" size_t wzy_stage_session_bytes(const wzy_stage* st, int n_cells) {
    if (!st || n_cells < 0 || n_cells > st->cfg.ctx_max) return 0;
    std::vector<std::pair<void*, size_t>> regs;
    st->session_regions(n_cells, regs);
    return session_total(regs);
}

extern "C" int wzy_stage_session_save(wzy_stage* st, int slot, int n_cells) {
    WZY_REQUIRE(st, "session_save: null stage");
    WZY_REQUIRE(slot >= 0 && slot < WZY_SESSION_SLOTS, "session_save: slot %d out of range", slot);
    WZY_REQUIRE(n_cells >= 0 && n_cells <= st->cfg.ctx_max, "session_save: %d cells outside 0..%d", n_cells,
                st->cfg.ctx_max);
    WZY_HIP_TRY(hipSetDevice(st->dev));
    auto& sl = st->sess[slot];
    std::vector<std::pair<void*, size_t>> regs;
    st->session_regions(n_cells, regs);
    WZY_REQUIRE((int) regs.size() <= SESSION_MAX_JOBS, "session_save: %zu regions", regs.size());
    const size_t need = session_total(regs);
    WZY_HIP_TRY(hipStreamSynchronize(st->stream));
    if (need > sl.cap) {
        if (sl.buf) {
            WZY_HIP_TRY(hipFree(sl.buf));
            st->dev_bytes -= sl.cap;
        }
        sl.buf = nullptr;
        sl.cap = 0;
        sl.n_cells = -1;
        if (hipMalloc((void**) &sl.buf, need) != hipSuccess) {
            (void) hipGetLastError();
            sl.buf = nullptr;
            set_error("session_save: hipMalloc(%zu) for slot %d failed", need, slot);
            return WZY_ENOMEM;
        }
        sl.cap = need;
        st->dev_bytes += need;
    }
    if (!sl.jobs) {
        void* p = nullptr;
        WZY_HIP_TRY(hipMalloc(&p, 2 * SESSION_MAX_JOBS * sizeof(CopyJob)));
        sl.jobs = (CopyJob*) p;
    }
    std::vector<CopyJob> jobs(2 * regs.size());
    size_t off = 0;
    for (size_t i = 0; i < regs.size(); ++i) {
        unsigned char* live = (unsigned char*) regs[i].first;
        jobs[i] = CopyJob{sl.buf + off, live, regs[i].second};                   // save
        jobs[regs.size() + i] = CopyJob{live, sl.buf + off, regs[i].second};     // restore
        off += (regs[i].second + 255) & ~(size_t) 255;
    }
    WZY_HIP_TRY(hipMemcpy(sl.jobs, jobs.data(), regs.size() * sizeof(CopyJob), hipMemcpyHostToDevice));
    WZY_HIP_TRY(hipMemcpy(sl.jobs + SESSION_MAX_JOBS, jobs.data() + regs.size(), regs.size() * sizeof(CopyJob),
                          hipMemcpyHostToDevice));
    sl.n_jobs = (int) regs.size();
    hipLaunchKernelGGL(copy_jobs_kernel, dim3(COPY_WGS, sl.n_jobs), dim3(256), 0, st->stream, sl.jobs);
    WZY_HIP_TRY(hipGetLastError());
    WZY_HIP_TRY(hipStreamSynchronize(st->stream));
    sl.n_cells = n_cells;
    return WZY_OK;
}

extern "C" int wzy_stage_session_restore(wzy_stage* st, int slot) {
    WZY_REQUIRE(st, "session_restore: null stage");
    WZY_REQUIRE(slot >= 0 && slot < WZY_SESSION_SLOTS, "session_restore: slot %d out of range", slot);
    auto& sl = st->sess[slot];
    WZY_REQUIRE(sl.n_cells >= 0, "session_restore: slot %d is empty", slot);
    // the drafter could have been created after the save: the region list must be the saved one
    std::vector<std::pair<void*, size_t>> regs;
    st->session_regions(sl.n_cells, regs);
    WZY_REQUIRE((int) regs.size() == sl.n_jobs, "session_restore: slot %d was saved with another layout", slot);
    WZY_HIP_TRY(hipSetDevice(st->dev));
    hipLaunchKernelGGL(copy_jobs_kernel, dim3(COPY_WGS, sl.n_jobs), dim3(256), 0, st->stream,
                       sl.jobs + SESSION_MAX_JOBS);
    WZY_HIP_TRY(hipGetLastError());
    WZY_HIP_TRY(hipStreamSynchronize(st->stream));
    st->have_head = st->have_pre_head = false;
    return WZY_OK;
}

extern "C" int wzy_stage_session_cells(const wzy_stage* st, int slot) {
    if (!st || slot < 0 || slot >= WZY_SESSION_SLOTS) return -1;
    return st->sess[slot].n_cells;
}

extern "C" int wzy_stage_session_clear(wzy_stage* st, int slot) {
    WZY_REQUIRE(st, "session_clear: null stage");
    WZY_REQUIRE(slot >= 0 && slot < WZY_SESSION_SLOTS, "session_clear: slot %d out of range", slot);
    st->sess[slot].n_cells = -1;
    return WZY_OK;
}

extern "C" int wzy_stage_sync(wzy_stage* st) {
    WZY_REQUIRE(st, "sync: null stage");
    WZY_HIP_TRY(hipStreamSynchronize(st->stream));
    return WZY_OK;
}

extern "C" int wzy_stage_greedy_ids(wzy_stage* st, int* out, int T) {
    WZY_REQUIRE(st && out && T >= 1 && T <= st->last_T && st->have_head, "greedy_ids: no head output for %d rows", T);
    memcpy(out, st->h_greedy, T * sizeof(int));
    return WZY_OK;
}
extern "C" int wzy_stage_top16(wzy_stage* st, float* v, int* ids, int T) {
    WZY_REQUIRE(st && v && ids && T >= 1 && T <= st->last_T && st->have_head, "top16: no head output");
    memcpy(v, st->h_top_v, (size_t) T * 16 * sizeof(float));
    memcpy(ids, st->h_top_i, (size_t) T * 16 * sizeof(int));
    return WZY_OK;
}
extern "C" int wzy_stage_logits(wzy_stage* st, float* out, int T) {
    WZY_REQUIRE(st && out && T >= 1 && T <= st->last_T && st->have_head, "logits: no head output");
    WZY_HIP_TRY(hipMemcpy(out, st->logits, (size_t) T * st->cfg.n_vocab * 4, hipMemcpyDeviceToHost));
    return WZY_OK;
}
extern "C" int wzy_stage_pre_head(wzy_stage* st, float* out, int T) {
    WZY_REQUIRE(st && out && T >= 1 && T <= st->last_T && st->have_pre_head, "pre_head: no pre-head output");
    WZY_HIP_TRY(hipMemcpy(out, st->pre_head_rows(), (size_t) T * st->HCD * 4, hipMemcpyDeviceToHost));
    return WZY_OK;
}

extern "C" int wzy_stage_set_graphs(wzy_stage* st, int enable) {
    WZY_REQUIRE(st, "set_graphs: null stage");
    st->graphs = enable != 0;
    if (st->mtp) st->mtp->graphs = st->graphs;
    return WZY_OK;
}

// ------------------------------------------------------------------------------------------------
// MTP drafter
// ------------------------------------------------------------------------------------------------
// Allocate the drafter and fill it: from `seed` (synthetic), or, with `ids`, only its draft head
// (vocabulary ids[n_dvocab]) for a loader that then writes every "mtp.*" weight.
static int mtp_create(wzy_stage* st, uint64_t seed, int n_dvocab, const int* ids) {
    WZY_REQUIRE(st && st->loaded, "mtp_init: stage not loaded");
    WZY_REQUIRE(!st->mtp, "mtp_init: the drafter is already initialised");
    const wzy_stage_cfg& c = st->cfg;
    WZY_REQUIRE(n_dvocab >= 1 && n_dvocab <= c.n_vocab, "mtp_init: n_dvocab must be in [1, %d]", c.n_vocab);
    WZY_HIP_TRY(hipSetDevice(st->dev));
    WZY_HIP_TRY(hipStreamSynchronize(st->stream));
    std::unique_ptr<MtpState> m(new MtpState);
    m->reg = [st](const char* n, void* p, size_t b) { st->reg(-1, n, p, b); };
    MtpDims d{};
    d.D = c.n_embd; d.HC = c.hc; d.HCLR = c.hc_lr;
    d.qh = c.qsa_qh; d.kvh = c.qsa_kvh; d.hd = c.qsa_hd; d.n_rot = c.n_rot;
    d.E = c.n_exp; d.K = c.top_k; d.F = c.n_ff;
    d.n_vocab = c.n_vocab; d.n_dv = n_dvocab; d.ctx_max = c.ctx_max; d.eps = c.eps;
    MtpMain mm{};
    if (c.emb_q8) { mm.emb_q = st->emb8.q; mm.emb_s = st->emb8.s; } else mm.emb = st->emb;
    if (c.head_q8) { mm.head_q = st->head8.q; mm.head_s = st->head8.s; } else mm.head = st->head;
    int rc = m->init(d, st->stream, mm, st->cos_tab, st->sin_tab);
    if (rc == WZY_OK) rc = ids ? m->build_head(ids) : m->load_synthetic(seed);
    if (rc == WZY_OK && ids) {
        rc = m->reset_kv();
        if (rc == WZY_OK && hipStreamSynchronize(st->stream) != hipSuccess) rc = WZY_EHIP;
        m->loaded = rc == WZY_OK;
    }
    if (rc != WZY_OK) {                 // the drafter's memory goes with m: drop its registry entries
        for (auto it = st->tensors.begin(); it != st->tensors.end();)
            it = it->first.second.rfind("mtp.", 0) == 0 ? st->tensors.erase(it) : std::next(it);
        return rc;
    }
    m->graphs = st->graphs;
    st->dev_bytes += m->dev_bytes;
    st->mtp = m.release();
    return WZY_OK;
}

extern "C" int wzy_stage_mtp_init(wzy_stage* st, uint64_t seed, int n_dvocab) {
    return mtp_create(st, seed, n_dvocab, nullptr);
}

namespace wzy {
int stage_set_ple_table(wzy_stage* st, bool ready, float scale) {
    WZY_REQUIRE(st && st->ple.scale_dev, "stage has no per-layer embedding");
    WZY_HIP_TRY(hipSetDevice(st->dev));
    st->ple.table_ready = false;
    if (!ready) return WZY_OK;
    WZY_HIP_TRY(hipMemcpy(st->ple.scale_dev, &scale, 4, hipMemcpyHostToDevice));
    st->ple.table_ready = true;
    return WZY_OK;
}

const wzy_stage_cfg* stage_cfg(const wzy_stage* st) { return &st->cfg; }
int stage_set_loaded(wzy_stage* st, bool loaded) {
    WZY_HIP_TRY(hipSetDevice(st->dev));
    WZY_HIP_TRY(hipStreamSynchronize(st->stream));
    st->loaded = false;
    if (!loaded) return WZY_OK;
    st->loaded = true;
    WZY_TRY(wzy_stage_reset_state(st));
    WZY_HIP_TRY(hipStreamSynchronize(st->stream));
    return WZY_OK;
}
void stage_mtp_drop(wzy_stage* st) {
    if (!st->mtp) return;
    (void) hipStreamSynchronize(st->stream);
    st->dev_bytes -= st->mtp->dev_bytes;
    delete st->mtp;
    st->mtp = nullptr;
    for (auto it = st->tensors.begin(); it != st->tensors.end();)
        it = it->first.second.rfind("mtp.", 0) == 0 ? st->tensors.erase(it) : std::next(it);
}
}  // namespace wzy

extern "C" int wzy_stage_mtp_init_vocab(wzy_stage* st, const int* dvocab, int n_dvocab) {
    WZY_REQUIRE(dvocab, "mtp_init_vocab: null draft vocabulary");
    return mtp_create(st, 0, n_dvocab, dvocab);
}

extern "C" int wzy_stage_mtp_reset(wzy_stage* st) {
    WZY_REQUIRE(st && st->mtp, "mtp_reset: no drafter");
    WZY_HIP_TRY(hipSetDevice(st->dev));
    return st->mtp->reset_kv();
}

extern "C" int wzy_stage_mtp_set_floor(wzy_stage* st, int kv_floor) {
    WZY_REQUIRE(st && st->mtp, "mtp_set_floor: no drafter");
    WZY_HIP_TRY(hipSetDevice(st->dev));
    return st->mtp->set_floor(kv_floor);
}

// rows [src_row0, src_row0 + n) of the last forward's pre-head residual -> the drafter's input rows
static int mtp_take_rows(wzy_stage* st, int src_row0, int n) {
    WZY_REQUIRE(st->have_pre_head && src_row0 >= 0 && src_row0 + n <= st->last_T,
                "mtp: rows [%d, %d) are not pre-head rows of the last forward (%d rows%s)", src_row0, src_row0 + n,
                st->last_T, st->have_pre_head ? "" : ", run without the head");
    WZY_HIP_TRY(hipMemcpyAsync(st->mtp->rin, st->pre_head_rows() + (size_t) src_row0 * st->HCD,
                               (size_t) n * st->HCD * 4, hipMemcpyDeviceToDevice, st->stream));
    return WZY_OK;
}

extern "C" int wzy_stage_mtp_front(wzy_stage* st, int cell0, const int* next_toks, int n_cells, int src_row0) {
    WZY_REQUIRE(st && st->mtp, "mtp_front: no drafter");
    WZY_REQUIRE(next_toks && n_cells >= 1 && n_cells <= WZY_MAX_W, "mtp_front: n_cells must be in [1, %d]", WZY_MAX_W);
    WZY_REQUIRE(cell0 >= 0 && cell0 + n_cells <= st->cfg.ctx_max, "mtp_front: cells beyond ctx_max");
    WZY_HIP_TRY(hipSetDevice(st->dev));
    WZY_TRY(mtp_take_rows(st, src_row0, n_cells));
    WZY_TRY(st->mtp->set_ctl(cell0, next_toks, n_cells));
    return st->mtp->enqueue_front(n_cells, false);
}

extern "C" int wzy_stage_mtp_draft(wzy_stage* st, int cell, int tok, int src_row, int depth, int* out_toks,
                                   float* out_probs) {
    WZY_REQUIRE(st && st->mtp, "mtp_draft: no drafter");
    WZY_REQUIRE(depth >= 1 && depth <= MTP_MAX_CHAIN, "mtp_draft: depth must be in [1, %d]", MTP_MAX_CHAIN);
    WZY_REQUIRE(cell >= 0 && cell + depth <= st->cfg.ctx_max, "mtp_draft: cells beyond ctx_max");
    WZY_REQUIRE(out_toks && out_probs, "mtp_draft: null output");
    WZY_HIP_TRY(hipSetDevice(st->dev));
    if (src_row >= 0) WZY_TRY(mtp_take_rows(st, src_row, 1));
    WZY_TRY(st->mtp->set_ctl(cell, &tok, 1));
    WZY_TRY(st->mtp->enqueue_steps(depth));
    WZY_HIP_TRY(hipStreamSynchronize(st->stream));
    memcpy(out_toks, st->mtp->h_tok, (size_t) depth * sizeof(int));
    memcpy(out_probs, st->mtp->h_prob, (size_t) depth * sizeof(float));
    return WZY_OK;
}

extern "C" int wzy_stage_mtp_time(wzy_stage* st, int cell, int tok, int src_row, int iters, float* us_per_step) {
    WZY_REQUIRE(st && st->mtp && us_per_step, "mtp_time: no drafter");
    WZY_REQUIRE(iters >= 1 && iters <= 4096 && cell >= 0 && cell + iters + 1 <= st->cfg.ctx_max,
                "mtp_time: iters must be in [1, 4096] with every cell below ctx_max");
    WZY_HIP_TRY(hipSetDevice(st->dev));
    if (src_row >= 0) WZY_TRY(mtp_take_rows(st, src_row, 1));
    WZY_TRY(st->mtp->set_ctl(cell, &tok, 1));
    WZY_TRY(st->mtp->enqueue_steps(1));          // warm-up (and graph instantiation)
    hipEvent_t a = nullptr, b = nullptr;
    WZY_HIP_TRY(hipEventCreate(&a));
    int rc = hipEventCreate(&b) == hipSuccess ? WZY_OK : WZY_EHIP;
    if (rc == WZY_OK && hipEventRecord(a, st->stream) != hipSuccess) rc = WZY_EHIP;
    for (int done = 0; rc == WZY_OK && done < iters; done += MTP_MAX_CHAIN)
        rc = st->mtp->enqueue_steps(std::min(MTP_MAX_CHAIN, iters - done));
    if (rc == WZY_OK && hipEventRecord(b, st->stream) != hipSuccess) rc = WZY_EHIP;
    float ms = 0.f;
    if (rc == WZY_OK && (hipEventSynchronize(b) != hipSuccess || hipEventElapsedTime(&ms, a, b) != hipSuccess))
        rc = WZY_EHIP;
    (void) hipEventDestroy(a);
    if (b) (void) hipEventDestroy(b);
    if (rc == WZY_EHIP) set_error("mtp_time: HIP event failure");
    if (rc == WZY_OK) *us_per_step = 1000.0f * ms / (float) iters;
    return rc;
}

extern "C" int wzy_stage_mtp_propose(wzy_stage* st, int cell0, int n_cells, const int* next_toks, int depth,
                                     int* out_toks, float* out_probs) {
    WZY_REQUIRE(st && st->mtp, "mtp_propose: no drafter");
    WZY_REQUIRE(next_toks && n_cells >= 1 && n_cells <= WZY_MAX_W, "mtp_propose: n_cells must be in [1, %d]",
                WZY_MAX_W);
    if (n_cells > 1) WZY_TRY(wzy_stage_mtp_front(st, cell0, next_toks, n_cells - 1, 0));
    return wzy_stage_mtp_draft(st, cell0 + n_cells - 1, next_toks[n_cells - 1], n_cells - 1, depth, out_toks,
                               out_probs);
}
extern "C" void* wzy_stage_stream(wzy_stage* st) { return st ? (void*) st->stream : nullptr; }

static Tensor* find_tensor(wzy_stage* st, int layer, const char* name) {
    auto it = st->tensors.find({layer, std::string(name)});
    return it == st->tensors.end() ? nullptr : &it->second;
}
extern "C" size_t wzy_stage_tensor_bytes(wzy_stage* st, int layer, const char* name) {
    if (!st || !name) return 0;
    Tensor* t = find_tensor(st, layer, name);
    return t ? t->bytes : 0;
}
extern "C" int wzy_stage_read_tensor(wzy_stage* st, int layer, const char* name, void* host, size_t bytes) {
    WZY_REQUIRE(st && name && host, "read_tensor: null argument");
    Tensor* t = find_tensor(st, layer, name);
    WZY_REQUIRE(t, "read_tensor: no tensor %s in layer %d", name, layer);
    WZY_REQUIRE(bytes <= t->bytes, "read_tensor: %zu bytes requested, tensor has %zu", bytes, t->bytes);
    WZY_HIP_TRY(hipStreamSynchronize(st->stream));
    WZY_HIP_TRY(hipMemcpy(host, t->p, bytes, hipMemcpyDeviceToHost));
    return WZY_OK;
}

extern "C" int wzy_stage_read_tensor_range(wzy_stage* st, int layer, const char* name, size_t offset, void* host,
                                           size_t bytes) {
    WZY_REQUIRE(st && name && host, "read_tensor_range: null argument");
    Tensor* t = find_tensor(st, layer, name);
    WZY_REQUIRE(t, "read_tensor_range: no tensor %s in layer %d", name, layer);
    WZY_REQUIRE(offset <= t->bytes && bytes <= t->bytes - offset,
                "read_tensor_range: [%zu, +%zu) outside the tensor's %zu bytes", offset, bytes, t->bytes);
    WZY_HIP_TRY(hipStreamSynchronize(st->stream));
    WZY_HIP_TRY(hipMemcpy(host, (const char*) t->p + offset, bytes, hipMemcpyDeviceToHost));
    return WZY_OK;
}
extern "C" int wzy_stage_write_tensor_range(wzy_stage* st, int layer, const char* name, size_t offset,
                                            const void* host, size_t bytes) {
    WZY_REQUIRE(st && name && host, "write_tensor_range: null argument");
    Tensor* t = find_tensor(st, layer, name);
    WZY_REQUIRE(t, "write_tensor_range: no tensor %s in layer %d", name, layer);
    WZY_REQUIRE(offset <= t->bytes && bytes <= t->bytes - offset,
                "write_tensor_range: [%zu, +%zu) outside the tensor's %zu bytes", offset, bytes, t->bytes);
    WZY_HIP_TRY(hipStreamSynchronize(st->stream));
    WZY_HIP_TRY(hipMemcpy((char*) t->p + offset, host, bytes, hipMemcpyHostToDevice));
    return WZY_OK;
}
extern "C" int wzy_stage_write_tensor(wzy_stage* st, int layer, const char* name, const void* host, size_t bytes) {
    WZY_REQUIRE(st && name && host, "write_tensor: null argument");
    Tensor* t = find_tensor(st, layer, name);
    WZY_REQUIRE(t, "write_tensor: no tensor %s in layer %d", name, layer);
    WZY_REQUIRE(bytes <= t->bytes, "write_tensor: %zu bytes given, tensor has %zu", bytes, t->bytes);
    WZY_HIP_TRY(hipStreamSynchronize(st->stream));
    WZY_HIP_TRY(hipMemcpy(t->p, host, bytes, hipMemcpyHostToDevice));
    return WZY_OK;
}

extern "C" int wzy_stage_moe_weights(wzy_stage* st, int layer, wzy_moe_weights* out) {
    WZY_REQUIRE(st && st->loaded && out, "moe_weights: bad arguments");
    WZY_REQUIRE(layer >= 0 && layer < (int) st->L.size(), "moe_weights: layer %d out of range", layer);
    *out = st->L[layer].moe;
    return WZY_OK;
}

extern "C" int wzy_stage_time_moe(wzy_stage* st, int iters, float* us_gate_up, float* us_down, float* us_block) {
    WZY_REQUIRE(st && st->loaded && iters >= 1 && us_gate_up && us_down, "time_moe: bad arguments");
    const int T = st->last_T > 0 ? st->last_T : 1;
    std::vector<wzy_moe_weights> ws;
    for (Layer& w : st->L) ws.push_back(w.moe);
    size_t need = 0;
    moe_ws_carve(nullptr, 0, st->D, st->cfg.n_ff, st->cfg.n_exp, st->cfg.top_k, WZY_MAX_W, &need);
    return wzy_moe_time_kernels(ws.data(), (int) ws.size(), T, st->mixed, st->moe_ws, need + 256, iters, us_gate_up,
                                us_down, us_block, st->stream);
}

// ------------------------------------------------------------------------------------------------
// chunked prefill (PrefillStageCtx::run_stage_prefill, src/wzy_prefill_tc.cuh:546-1058)
// ------------------------------------------------------------------------------------------------
namespace {
constexpr int PF_SCORE_ROWS = 2048;     // rows per block-score pass (the reference's qsa_score_b)

__global__ void pf_pos_kernel(int* pos8, int p0, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) pos8[i] = p0 + 8 * i;
}
}  // namespace

int wzy_stage::prefill_reserve(int B) {
    const wzy_stage_cfg& c = cfg;
    if (trace && B > pf.tr_rows) {
        WZY_HIP_TRY(hipStreamSynchronize(stream));
        if (pf.tr) WZY_HIP_TRY(hipFree(pf.tr));
        if (pf.tr_sel) WZY_HIP_TRY(hipFree(pf.tr_sel));
        if (pf.tr_sc) WZY_HIP_TRY(hipFree(pf.tr_sc));
        if (pf.tr_kv) WZY_HIP_TRY(hipFree(pf.tr_kv));
        pf.tr_kv = nullptr;
        pf.tr = nullptr;
        pf.tr_sel = pf.tr_cnt = nullptr;
        pf.tr_sc = nullptr;
        const size_t n = (size_t) c.n_layers * 4 * B * D;
        WZY_HIP_TRY(hipMalloc((void**) &pf.tr, n * 4));
        const size_t nq = (size_t) std::max(n_qsa, 1), ns = nq * B * c.idx_topk;
        WZY_HIP_TRY(hipMalloc((void**) &pf.tr_sel, (ns + nq * B) * 4));
        pf.tr_cnt = pf.tr_sel + ns;
        const size_t nsc = nq * B * (size_t) max_b;
        WZY_HIP_TRY(hipMalloc((void**) &pf.tr_sc, nsc * 4));
        reg(-1, "trace.pf_scores", pf.tr_sc, nsc * 4);
        const size_t nkv = nq * B * (size_t) (2 * KVD + c.idx_dim);
        WZY_HIP_TRY(hipMalloc((void**) &pf.tr_kv, nkv * 4));
        reg(-1, "trace.pf_kv", pf.tr_kv, nkv * 4);
        pf.tr_rows = B;
        reg(-1, "trace.pf", pf.tr, n * 4);
        reg(-1, "trace.pf_sel", pf.tr_sel, ns * 4);
        reg(-1, "trace.pf_cnt", pf.tr_cnt, nq * B * 4);
    }
    if (B <= pf.cap) return WZY_OK;
    WZY_HIP_TRY(hipStreamSynchronize(stream));
    if (pf.base) {
        WZY_HIP_TRY(hipFree(pf.base));
        dev_bytes -= pf.bytes;
        float* keep_tr = pf.tr;
        int *keep_sel = pf.tr_sel, *keep_cnt = pf.tr_cnt;
        float* keep_sc = pf.tr_sc;
        const int keep_rows = pf.tr_rows;
        pf = PfWs{};
        pf.tr = keep_tr;
        pf.tr_sc = keep_sc;
        pf.tr_sel = keep_sel;
        pf.tr_cnt = keep_cnt;
        pf.tr_rows = keep_rows;
    }
    const size_t b = (size_t) B, maxb = (size_t) max_b;
    const int sc_rows = std::min(B, PF_SCORE_ROWS);
    const size_t xh_w = (size_t) std::max(std::max(D, GV), QD);
    const size_t moe_bytes = wzy_moe_prefill_workspace_bytes(D, c.n_ff, c.n_exp, c.top_k, B);
    // layout: one allocation, 256-byte aligned pieces
    size_t off = 0;
    auto bump = [&](size_t bytes) {
        const size_t r = off;
        off += (bytes + 255) & ~(size_t) 255;
        return r;
    };
    const size_t oR = bump(b * HCD * 4), oxn = bump(b * HCD * 2), olo = bump(4 * b * c.hc_lr * 4),
                 oloh = bump(b * c.hc_lr * 2), oia = bump(b * c.hc * 4),
                 oif = bump(b * c.hc * 4), omx = bump(b * D * 4), oxh = bump(b * xh_w * 2), oblk = bump(b * D * 4),
                 ocomb = bump(b * D * 4), otoks = bump(b * 4), opos = bump((b / 8 + 2) * 4);
    // GDN and QSA scratch share one region (a layer uses one of them)
    const size_t umark = off;
    const size_t oqkv = bump(b * QKV * 4), oz = bump(b * GV * 4), oab = bump(b * 2 * c.gdn_hv * 4),
                 oco = bump(b * QKV * 4), odec = bump(b * c.gdn_hv * 4), obet = bump(b * c.gdn_hv * 4),
                 okq = bump(b * c.gdn_hk * 4),
                 oo = bump(b * GV * 4);
    const size_t gdn_end = off;
    off = umark;
    const size_t oqg = bump(b * 2 * QD * 4), okk = bump(b * KVD * 4), ovv = bump(b * KVD * 4),
                 oir = bump(b * c.idx_dim * 4), oqi = bump(b * c.idx_heads * c.idx_dim * 4),
                 osc = bump((size_t) sc_rows * maxb * 4), osel = bump(b * c.idx_topk * 4), ocnt = bump(b * 4);
    off = std::max(off, gdn_end);
    const size_t omoe = bump(moe_bytes);
    // the largest Q8_0 projection a chunk GEMM expands to bf16 (N x K values)
    const size_t wbf_elems = std::max({(size_t) 2 * QD * D, (size_t) D * QD, (size_t) QKV * D, (size_t) GV * D,
                                       (size_t) D * GV, (size_t) c.hc_lr * HCD});
    const size_t owbf = bump(wbf_elems * 2);
    size_t ope = 0, opeh = 0, opk = 0, opv = 0, opg = 0, opn = 0;
    if (c.ple) {
        ope = bump(b * D * 4); opeh = bump(b * D * 2); opk = bump(b * HCD * 4); opv = bump(b * D * 4);
        opg = bump(b * HCD * 4); opn = bump(b * HCD * 4);
    }
    void* base = nullptr;
    if (hipMalloc(&base, off) != hipSuccess) {
        (void) hipGetLastError();
        set_error("prefill: hipMalloc(%zu) for a %d-row workspace failed", off, B);
        return WZY_ENOMEM;
    }
    dev_bytes += off;
    unsigned char* u = (unsigned char*) base;
    pf.base = base;
    pf.bytes = off;
    pf.cap = B;
    pf.sc_rows = sc_rows;
    pf.R = (float*) (u + oR); pf.xn = (uint16_t*) (u + oxn); pf.lo = (float*) (u + olo);
    pf.loh = (uint16_t*) (u + oloh); pf.inj_a = (float*) (u + oia);
    pf.inj_f = (float*) (u + oif); pf.mixed = (float*) (u + omx); pf.xh = (uint16_t*) (u + oxh);
    pf.block = (float*) (u + oblk); pf.comb = (float*) (u + ocomb); pf.toks = (int*) (u + otoks);
    pf.pos8 = (int*) (u + opos);
    pf.qkv = (float*) (u + oqkv); pf.z = (float*) (u + oz); pf.ab = (float*) (u + oab);
    pf.conv_out = (float*) (u + oco); pf.decay = (float*) (u + odec); pf.beta = (float*) (u + obet);
    pf.kq = (float*) (u + okq);
    pf.o = (float*) (u + oo);
    pf.qg = (float*) (u + oqg); pf.kk = (float*) (u + okk); pf.vv = (float*) (u + ovv);
    pf.idx_raw = (float*) (u + oir); pf.q_idx = (float*) (u + oqi); pf.scores = (float*) (u + osc);
    pf.sel = (int*) (u + osel); pf.cnt = (int*) (u + ocnt);
    pf.moe_ws = u + omoe;
    pf.wbf = (uint16_t*) (u + owbf);
    pf.wbf_elems = wbf_elems;
    if (c.ple) {
        pf.ple_emb = (float*) (u + ope); pf.ple_embh = (uint16_t*) (u + opeh); pf.ple_k = (float*) (u + opk);
        pf.ple_v = (float*) (u + opv); pf.ple_gat = (float*) (u + opg); pf.ple_n = (float*) (u + opn);
    }
    pf.moe_bytes = moe_bytes;
    return WZY_OK;
}

// Layer sequence of one chunk (rows p0 .. p0+B-1, token ids already in pf.toks).  us_parts (optional,
// host) receives event-timed microseconds per part: [0] attention-half HC reads, [1] GDN blocks, [2]
// QSA blocks, [3] FFN-half HC reads, [4] MoE blocks, [5] everything else (embedding, writes).
int wzy_stage::enqueue_prefill(int p0, int B, float* us_parts) {
    const wzy_stage_cfg& c = cfg;
    hipStream_t st = stream;
    const int HC = c.hc, HCLR = c.hc_lr;
    const float inv_hc = 1.0f / (float) HC;
    hipEvent_t evs[2] = {nullptr, nullptr};
    double part[6] = {0, 0, 0, 0, 0, 0};
    int cur_part = 5;
    if (us_parts) {
        WZY_HIP_TRY(hipEventCreate(&evs[0]));
        WZY_HIP_TRY(hipEventCreate(&evs[1]));
        WZY_HIP_TRY(hipEventRecord(evs[0], st));
    }
    // close the running part and open `next` (event-timed; synchronises only when measuring)
    auto mark = [&](int next) -> int {
        if (!us_parts) return WZY_OK;
        WZY_HIP_TRY(hipEventRecord(evs[1], st));
        WZY_HIP_TRY(hipEventSynchronize(evs[1]));
        float ms = 0.f;
        WZY_HIP_TRY(hipEventElapsedTime(&ms, evs[0], evs[1]));
        part[cur_part] += ms * 1000.0;
        std::swap(evs[0], evs[1]);
        cur_part = next;
        return WZY_OK;
    };
    auto gemm = [&](const uint16_t* a, int lda, int K, const Q8* q, const uint16_t* wb, int N, float* y,
                    uint16_t* yb, int ldy) {
        PfGemm g{};
        g.a = a; g.lda = lda; g.M = B; g.N = N; g.K = K;
        if (q) { g.wq = q->q; g.ws = q->s; } else { g.wb = wb; }
        g.y = y; g.yb = yb; g.ldy = ldy;
        g.wscratch = pf.wbf; g.wscratch_elems = pf.wbf_elems;
        return launch_pf_gemm(g, st);
    };
    // hyper-connection read of the chunk: R (with the pending block folded in when bo != null) ->
    // mixed fp32 + xh bf16, inject -> inj_out
    // The down projection runs as four K ranges, one per stream (768 workgroups instead of 192 for
    // its 320 outputs), summed ((p0 + p1) + (p2 + p3)) by pf_silu_div; the up projection combines
    // its stream gates with xn in its epilogue, so the [B][4D] gates never reach memory.
    const int down_split = (HCD / 64) % 4 == 0 ? 4 : 1;
    auto hc_read = [&](const float* norm_w, const Q8& down, const uint16_t* inj_w, const Q8& up, const float* bo,
                       const float* inj_prev, float* inj_out) -> int {
        WZY_TRY(launch_pf_hc_norm(pf.R, bo, inj_prev, norm_w, pf.xn, D, HC, c.eps, B, st));
        WZY_TRY(gemm(pf.xn, HCD, HCD, nullptr, inj_w, HC, inj_out, nullptr, HC));
        {
            PfGemm g{};
            g.a = pf.xn; g.lda = HCD; g.M = B; g.N = HCLR; g.K = HCD;
            g.wq = down.q; g.ws = down.s; g.y = pf.lo; g.ldy = HCLR; g.ksplit = down_split;
            g.wscratch = pf.wbf; g.wscratch_elems = pf.wbf_elems;
            WZY_TRY(launch_pf_gemm(g, st));
        }
        WZY_TRY(launch_pf_silu_div(pf.lo, pf.loh, (size_t) B * HCLR, down_split, inv_hc, st));
        PfGemm g{};
        g.a = pf.loh; g.lda = HCLR; g.M = B; g.N = HCD; g.K = HCLR;
        g.wq = up.q; g.ws = up.s;
        g.um_xn = pf.xn; g.um_mixed = pf.mixed; g.um_xh = pf.xh; g.um_d = D;
        g.wscratch = pf.wbf; g.wscratch_elems = pf.wbf_elems;
        return launch_pf_gemm(g, st);
    };

    hipLaunchKernelGGL(pf_pos_kernel, dim3((B / 8 + 2 + 255) / 256), dim3(256), 0, st, pf.pos8, p0, B / 8 + 2);
    PfEmb e{};
    if (c.emb_q8) { e.emb_q = emb8.q; e.emb_s = emb8.s; } else { e.emb = emb; }
    e.n_vocab = c.n_vocab;
    WZY_TRY(launch_pf_embed(e, pf.toks, pf.R, D, HC, B, st));
    const float* pend_bo = nullptr;
    const float* pend_inj = nullptr;
    QsaDims dm = qd;
    // trace copies (wzy_stage_set_trace): [layer][slot][row][D], slots mixed_a, block, mixed_f, comb
    auto tr = [&](int l, int slot, const float* src) -> int {
        if (!trace || !pf.tr) return WZY_OK;
        WZY_HIP_TRY(hipMemcpyAsync(pf.tr + (((size_t) l * 4 + slot) * pf.tr_rows) * D, src, (size_t) B * D * 4,
                                   hipMemcpyDeviceToDevice, st));
        return WZY_OK;
    };
    for (int l = 0; l < c.n_layers; ++l) {
        Layer& w = L[l];
        WZY_TRY(mark(0));
        if (l == 1 && c.ple) {
            // per-layer embedding of the chunk (src/wzy_prefill_tc.cuh:808-823): table rows, the two
            // projections on bf16 MFMA, the block over the rows in order
            PleRowsArgs pr{};
            pr.table = ple.table; pr.head = D / PLE_HEADS; pr.scale_dev = ple.scale_dev; pr.eos = c.ple_eos;
            pr.pos = pf.pos8; pr.toks = pf.toks; pr.tok_hist = ple.tok_hist; pr.ctx_max = c.ctx_max;
            pr.emb = pf.ple_emb; pr.emb_bf16 = pf.ple_embh;
            WZY_TRY(launch_ple_rows(pr, B, st));
            WZY_TRY(gemm(pf.ple_embh, D, D, nullptr, ple.wk, HCD, pf.ple_k, nullptr, HCD));
            WZY_TRY(gemm(pf.ple_embh, D, D, nullptr, ple.wv, D, pf.ple_v, nullptr, D));
            PleBlockArgs pb{};
            pb.R = pf.R; pb.bo = pend_bo; pb.inj_prev = pend_inj; pb.k = pf.ple_k; pb.v = pf.ple_v;
            pb.norm_q = ple.nq; pb.norm_k = ple.nk; pb.norm_c = ple.nc; pb.conv_w = ple.cw; pb.hist = ple.hist;
            pb.gat = pf.ple_gat; pb.n = pf.ple_n; pb.D = D; pb.HC = HC; pb.eps = c.eps;
            WZY_TRY(launch_ple_mix(pb, B, st));
            WZY_TRY(launch_ple_conv(pb, B, st));
            pend_bo = nullptr;
            pend_inj = nullptr;
        }
        WZY_TRY(hc_read(w.hc_norm[0], w.hc_down[0], w.hc_inj[0], w.hc_up[0], pend_bo, pend_inj, pf.inj_a));
        WZY_TRY(tr(l, 0, pf.mixed));
        if (!w.qsa) {
            WZY_TRY(mark(1));
            const int hv = c.gdn_hv;
            WZY_TRY(gemm(pf.xh, D, D, &w.qkv, nullptr, QKV, pf.qkv, nullptr, QKV));
            WZY_TRY(gemm(pf.xh, D, D, &w.wgate, nullptr, GV, pf.z, nullptr, GV));
            WZY_TRY(gemm(pf.xh, D, D, nullptr, w.alpha, hv, pf.ab, nullptr, 2 * hv));
            WZY_TRY(gemm(pf.xh, D, D, nullptr, w.beta, hv, pf.ab + hv, nullptr, 2 * hv));
            PfGdn g{};
            g.hk = c.gdn_hk; g.hv = hv; g.B = B; g.eps = c.eps;
            g.qkv = pf.qkv; g.z = pf.z; g.ab = pf.ab; g.dt = w.dt; g.ssm_a = w.ssm_a; g.conv_w = w.conv_w;
            g.gamma = w.ssm_norm; g.conv_hist = w.conv_hist; g.state = w.ssm; g.conv_out = pf.conv_out;
            g.decay = pf.decay; g.beta = pf.beta; g.kq = pf.kq; g.o = pf.o; g.y = pf.xh;
            WZY_TRY(launch_pf_gdn(g, st));
            WZY_TRY(gemm(pf.xh, GV, GV, &w.wout, nullptr, D, pf.block, nullptr, D));
        } else {
            WZY_TRY(mark(2));
            const int ID = c.idx_dim, IH = c.idx_heads;
            WZY_TRY(gemm(pf.xh, D, D, &w.wq, nullptr, 2 * QD, pf.qg, nullptr, 2 * QD));
            WZY_TRY(gemm(pf.xh, D, D, &w.wk, nullptr, KVD, pf.kk, nullptr, KVD));
            WZY_TRY(gemm(pf.xh, D, D, &w.wv, nullptr, KVD, pf.vv, nullptr, KVD));
            WZY_TRY(gemm(pf.xh, D, D, nullptr, w.idx_k, ID, pf.idx_raw, nullptr, ID));
            WZY_TRY(gemm(pf.xh, D, D, nullptr, w.idx_q, IH * ID, pf.q_idx, nullptr, IH * ID));
            PfQsaPrep pa{};
            pa.dm = dm; pa.pos = pf.pos8; pa.qg = pf.qg; pa.kk = pf.kk; pa.vv = pf.vv; pa.q_idx = pf.q_idx;
            pa.q_norm = w.q_norm; pa.k_norm = w.k_norm; pa.iq_norm = w.idx_qn; pa.cos_tab = cos_tab; pa.sin_tab = sin_tab;
            pa.kv = w.kv;
            WZY_TRY(launch_pf_qsa_prep(pa, B, st));
            if (trace && pf.tr_kv) {                 // k (after norm + RoPE), v and the raw indexer key rows
                const size_t rw = 2 * (size_t) KVD + ID;
                float* dst = pf.tr_kv + (size_t) w.local * pf.tr_rows * rw;
                WZY_HIP_TRY(hipMemcpy2DAsync(dst, rw * 4, pf.kk, (size_t) KVD * 4, (size_t) KVD * 4, B,
                                             hipMemcpyDeviceToDevice, st));
                WZY_HIP_TRY(hipMemcpy2DAsync(dst + KVD, rw * 4, pf.vv, (size_t) KVD * 4, (size_t) KVD * 4, B,
                                             hipMemcpyDeviceToDevice, st));
                WZY_HIP_TRY(hipMemcpy2DAsync(dst + 2 * KVD, rw * 4, pf.idx_raw, (size_t) ID * 4, (size_t) ID * 4, B,
                                             hipMemcpyDeviceToDevice, st));
            }
            PfIdxAppend ia{};
            ia.dm = dm; ia.idx_raw = pf.idx_raw; ia.ik_norm = w.idx_kn; ia.cos_tab = cos_tab; ia.sin_tab = sin_tab;
            ia.ix = w.ix;
            ia.ix.tail_snaps = nullptr; ia.ix.dead_snaps = nullptr; ia.ix.pool_snaps = nullptr;
            WZY_TRY(launch_pf_idx_append(ia, p0, B, st));
            for (int q0 = 0; q0 < B; q0 += pf.sc_rows) {
                const int qb = std::min(pf.sc_rows, B - q0);
                if (p0 + q0 + qb > c.idx_topk) {
                    QsaScoreArgs sa{};
                    sa.dm = dm; sa.pos = pf.pos8 + q0 / 8; sa.pooled = w.ix.pooled; sa.dead = w.ix.dead;
                    sa.q_idx = pf.q_idx + (size_t) q0 * IH * ID; sa.scores = pf.scores; sa.max_b = max_b;
                    WZY_TRY(launch_pf_scores(sa, qb, st));
                    if (trace && pf.tr_sc)
                        WZY_HIP_TRY(hipMemcpyAsync(pf.tr_sc + ((size_t) w.local * pf.tr_rows + q0) * max_b, pf.scores,
                                                   (size_t) qb * max_b * 4, hipMemcpyDeviceToDevice, st));
                }
                const int max_n_kv = p0 + q0 + qb;
                if (max_n_kv / c.idx_blk + 1 <= 16384) {
                    WZY_TRY(launch_qsa_topk_rows(dm, pf.pos8 + q0 / 8, pf.scores, max_b, pf.sel + (size_t) q0 * c.idx_topk,
                                                 pf.cnt + q0, qb, max_n_kv, st));
                } else {
                    for (int g0 = 0; g0 < qb; g0 += WZY_MAX_W)
                        WZY_TRY(launch_qsa_topk(dm, pf.pos8 + (q0 + g0) / 8, pf.scores + (size_t) g0 * max_b, max_b,
                                                pf.sel + (size_t) (q0 + g0) * c.idx_topk, pf.cnt + q0 + g0,
                                                std::min(WZY_MAX_W, qb - g0), st));
                }
            }
            if (trace && pf.tr_sel) {
                WZY_HIP_TRY(hipMemcpyAsync(pf.tr_sel + (size_t) w.local * pf.tr_rows * c.idx_topk, pf.sel,
                                           (size_t) B * c.idx_topk * 4, hipMemcpyDeviceToDevice, st));
                WZY_HIP_TRY(hipMemcpyAsync(pf.tr_cnt + (size_t) w.local * pf.tr_rows, pf.cnt, (size_t) B * 4,
                                           hipMemcpyDeviceToDevice, st));
            }
            PfAttn at{};
            at.dm = dm; at.pos = pf.pos8; at.qg = pf.qg; at.kv = w.kv; at.sel = pf.sel; at.out = pf.xh;
            WZY_TRY(launch_pf_attn(at, B, st));
            WZY_TRY(gemm(pf.xh, QD, QD, &w.wo, nullptr, D, pf.block, nullptr, D));
        }
        WZY_TRY(tr(l, 1, pf.block));
        WZY_TRY(mark(3));
        // the block's write into the streams is folded into the FFN read (same arithmetic)
        WZY_TRY(hc_read(w.hc_norm[1], w.hc_down[1], w.hc_inj[1], w.hc_up[1], pf.block, pf.inj_a, pf.inj_f));
        WZY_TRY(tr(l, 2, pf.mixed));
        WZY_TRY(mark(4));
        WZY_TRY(wzy_moe_prefill(&w.moe, pf.mixed, B, pf.comb, nullptr, nullptr, pf.moe_ws, pf.moe_bytes, st));
        WZY_TRY(tr(l, 3, pf.comb));
        pend_bo = pf.comb;
        pend_inj = pf.inj_f;
    }
    WZY_TRY(mark(5));
    WZY_TRY(launch_pf_hc_write(pf.R, pend_bo, pend_inj, D, HC, B, st));
    if (us_parts) {
        WZY_TRY(mark(5));
        for (int i = 0; i < 6; ++i) us_parts[i] = (float) part[i];
        (void) hipEventDestroy(evs[0]);
        (void) hipEventDestroy(evs[1]);
    }
    return WZY_OK;
}

extern "C" int wzy_stage_can_prefill(const wzy_stage_cfg* c) {
    return c && c->hc_lr % 64 == 0 && c->n_embd % 256 == 0 && c->n_ff % 128 == 0 && c->n_exp % 64 == 0 &&
           c->n_exp <= 1024 && c->idx_dim == 128;
}

static int prefill_checks(wzy_stage* st, int pos, const int* toks, int B) {
    WZY_REQUIRE(st && st->loaded, "prefill: stage not loaded");
    WZY_REQUIRE(!st->cfg.ple || st->ple.table_ready, "prefill: the per-layer embedding table is not loaded");
    WZY_REQUIRE(toks && B >= 1 && B <= 65535, "prefill: B must be in [1, 65535] with token ids");
    WZY_REQUIRE(pos >= 0 && pos + B <= st->cfg.ctx_max, "prefill: positions [%d, %d) exceed ctx_max %d", pos, pos + B,
                st->cfg.ctx_max);
    WZY_REQUIRE(wzy_stage_can_prefill(&st->cfg),
                "prefill: shape unsupported (hc_lr a multiple of 64, n_embd of 256, n_ff of 128, n_exp of 64 up to "
                "1024, idx_dim 128)");
    return WZY_OK;
}

extern "C" int wzy_stage_prefill(wzy_stage* st, int pos, const int* toks, int B) {
    WZY_TRY(prefill_checks(st, pos, toks, B));
    WZY_HIP_TRY(hipSetDevice(st->dev));
    WZY_TRY(st->prefill_reserve(B));
    WZY_HIP_TRY(hipMemcpyAsync(st->pf.toks, toks, (size_t) B * sizeof(int), hipMemcpyHostToDevice, st->stream));
    WZY_TRY(st->enqueue_prefill(pos, B, nullptr));
    st->last_T = B;
    st->have_head = false;
    st->have_pre_head = true;
    st->pre_head_pf = true;
    return WZY_OK;
}

extern "C" int wzy_stage_prefill_time(wzy_stage* st, int pos, const int* toks, int B, float* us_parts) {
    WZY_REQUIRE(us_parts, "prefill_time: null output");
    WZY_TRY(prefill_checks(st, pos, toks, B));
    WZY_HIP_TRY(hipSetDevice(st->dev));
    WZY_TRY(st->prefill_reserve(B));
    WZY_HIP_TRY(hipMemcpyAsync(st->pf.toks, toks, (size_t) B * sizeof(int), hipMemcpyHostToDevice, st->stream));
    WZY_TRY(st->enqueue_prefill(pos, B, us_parts));
    WZY_HIP_TRY(hipStreamSynchronize(st->stream));
    st->last_T = B;
    st->have_head = false;
    st->have_pre_head = true;
    st->pre_head_pf = true;
    return WZY_OK;
}

// wzy_mtp.h -- internal interface of the MTP speculative drafter (mtp.hip), owned by the stage.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <functional>
#include <vector>

#include "wzy_qsa.h"

namespace wzy {

constexpr int MTP_RING = 1024;        // KV ring cells (src/wzy_mtp.cuh:11)
constexpr int MTP_MAX_CHAIN = 8;      // chained draft steps per call
constexpr int MTP_CTL_INTS = 16;      // device control block, see MtpState::d_ctl
constexpr int MTP_CTL_SLOTS = 16;     // pinned staging slots of the control block
constexpr int MTP_RED_WGS = 128;      // workgroups of the draft-head reduction

struct MtpQ8 {
    int8_t* q = nullptr;
    uint16_t* s = nullptr;
    int rows = 0, cols = 0;
};

struct MtpDims {
    int D, HC, HCLR;                  // hidden size, residual streams, hyper-connection rank
    int qh, kvh, hd, n_rot;           // attention (same layout as the main QSA layers)
    int E, K, F;                      // experts, routed per token, expert FFN width
    int n_vocab, n_dv, ctx_max;       // main vocabulary, draft vocabulary rows, RoPE table length
    float eps;
};

// The main model's token embedding and LM head, each bf16 or Q8_0 (codes + fp16 per-32 scales).
struct MtpMain {
    const uint16_t* emb; const int8_t* emb_q; const uint16_t* emb_s;
    const uint16_t* head; const int8_t* head_q; const uint16_t* head_s;
};

struct MtpState {
    MtpDims c{};
    hipStream_t st = nullptr;
    MtpMain main{};                                // main model tables [n_vocab][D]
    const float* cos_tab = nullptr;
    const float* sin_tab = nullptr;
    std::vector<void*> allocs;
    size_t dev_bytes = 0;
    std::function<void(const char*, void*, size_t)> reg;   // tensor registry of the owner

    // weights
    float* pre_norm_emb = nullptr;                 // [D]
    float* pre_norm_hid = nullptr;                 // [HC][D]
    MtpQ8 fc_emb, fc_hid, wq, wk, wv, wo, sh_gate, sh_up, sh_down, head;
    float* hc_norm[3] = {nullptr, nullptr, nullptr};       // attention, MLP, final mixer
    MtpQ8 hc_down[3], hc_up[3];
    uint16_t* hc_inj[2] = {nullptr, nullptr};              // the mixer has no inject weight
    float* q_norm = nullptr;
    float* k_norm = nullptr;
    uint16_t* router = nullptr;                    // bf16 [E][D]
    uint16_t* sgate = nullptr;                     // bf16 [D]
    uint8_t* experts = nullptr;                    // E Q2_0 blobs
    size_t q2_rec = 0;
    int* dvocab = nullptr;                         // [n_dv] main-vocabulary id of each draft-head row

    // state: INT8 KV ring (cell p in slot p % MTP_RING), attention floor
    QsaKv kv{};
    QsaDims qd{};
    int* d_floor = nullptr;

    // control block [MTP_CTL_INTS]: [0] cell of row 0, [1..WZY_MAX_W] token ids embedded by the
    // rows, [9] chain slot of the next draft output.  Each draft step advances [0], writes its token
    // to [1] and bumps [9], so chained steps run back to back without the host.
    int* d_ctl = nullptr;
    int* h_ctl = nullptr;                          // pinned [MTP_CTL_SLOTS][MTP_CTL_INTS]
    hipEvent_t ctl_ev[MTP_CTL_SLOTS] = {};
    bool ctl_pending[MTP_CTL_SLOTS] = {};
    int ctl_slot = 0;
    int* h_tok = nullptr;                          // pinned, device-visible [MTP_MAX_CHAIN]
    float* h_prob = nullptr;
    int* d_tok = nullptr;
    float* d_prob = nullptr;

    // activations (up to WZY_MAX_W rows in the front half, one row in the rest)
    float *rin = nullptr, *en = nullptr, *e2 = nullptr, *hn = nullptr, *h2 = nullptr, *unit_gate = nullptr;
    float *rc = nullptr, *r2 = nullptr, *mixed = nullptr, *inj = nullptr, *inj2 = nullptr, *mixed2 = nullptr;
    float *nsc = nullptr, *lo = nullptr, *lo_part = nullptr, *inj_part = nullptr;
    float *qg = nullptr, *kk = nullptr, *vv = nullptr, *att_part = nullptr, *att_ml = nullptr, *att = nullptr;
    float *bo = nullptr, *rlog = nullptr, *sg = nullptr, *wts = nullptr, *as = nullptr, *comb = nullptr;
    float *sample = nullptr, *logits = nullptr, *red = nullptr;
    int* ids = nullptr;
    int8_t* aq = nullptr;
    unsigned* arrive = nullptr;

    hipGraphExec_t step_exec = nullptr;
    bool graphs = true;
    bool loaded = false;

    ~MtpState();
    int alloc(void** p, size_t bytes, bool zero = true);
    template <class T>
    int alloc_t(T** p, size_t n, bool zero = true) { return alloc((void**) p, n * sizeof(T), zero); }
    int alloc_q8(MtpQ8& m, int rows, int cols, const char* name);

    int init(const MtpDims& d, hipStream_t stream, const MtpMain& m, const float* cos_t, const float* sin_t);
    // draft vocabulary ids[n_dv] (host) and the draft head rows: the main head's Q8_0 rows copied, or
    // its bf16 rows quantised to Q8_0
    int build_head(const int* ids);
    // seeded synthetic weights, draft vocabulary spread evenly over the main vocabulary
    int load_synthetic(uint64_t seed);
    int reset_kv();
    int set_floor(int floor);
    // stage (cell0, toks[0..n)) into the control block, chain slot 0
    int set_ctl(int cell0, const int* toks, int n);
    // front half over rows rin[0..T): K/V append of cells ctl[0]..ctl[0]+T-1 (run_front_kv)
    int enqueue_front(int T, bool with_q);
    // rest of row 0 + draft head + reduction (run_rest_row0)
    int enqueue_rest();
    // `depth` chained draft steps from the control block and rin[0]
    int enqueue_steps(int depth);
};

}  // namespace wzy

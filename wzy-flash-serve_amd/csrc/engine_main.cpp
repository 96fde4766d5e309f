// engine_main.cpp -- wzy_engine: the decode engine process.  Reads the stream protocol on stdin,
// drives the one-GPU stage (include/wzy_stage.h) and writes PREFILL / TOK / DONE lines on stdout.
//
// Replaces the reference's serve-mode main loop (src/wzy_engine_v2.cu:1632-2440) and the
// multiplexed batch engine's protocol front end (src/wzy_batch_engine.cu:1028-1079,465-566).
// One GPU holds every layer and expert, so a request runs as: reset or reuse the resident state,
// prefill the prompt in windows of up to WZY_MAX_W rows, then one greedy/sampled row per step.
//
// Options (flags override the environment):
//   --ctx N        / WZY_CTX          context capacity in cells (default 262144)
//   --batch        / WZY_BATCH>0      multiplexed protocol: "req" ids, TOK <req> <id>, CANCEL <req>
//   --model-seed S / WZY_MODEL_SEED   seed of the synthetic model weights (default 3)
//   --model-dir D  / WZY_MODEL_DIR    real weights instead, in the reference's layout: D/qwen-nvfp4-gptq-
//                                     dense.gguf (shapes from its tensors), D/pack/experts.bin,
//                                     D/token-embd-bf16.gguf when present, and with --mtp D/mtp/ and the
//                                     draft vocabulary WZY_DRAFT_VOCAB (default D/mtp/draft_vocab.bin)
//   --seed S       / WZY_SEED         seed of the sampling generator (default: random_device)
//   --cfg k=v,...  / WZY_CFG          overrides of wzy_stage_cfg fields (e.g. n_layers=4,n_embd=256)
//   --device D     / WZY_DEVICE       HIP device (default 0)
//   --no-graphs    / WZY_GRAPHS=0     launch kernels one by one instead of replaying hipGraphs
//   --mtp          / WZY_MTP=1        MTP speculative decoding: the drafter proposes up to `spec` tokens
//                                     per window under the reference's confidence gates
//                                     (WZY_SPEC_DEPTH, WZY_SPEC_MIN_P, WZY_SPEC_GATE, WZY_ADAPT_DEPTH)
//   --spec-depth K / WZY_SPEC_FIXED=K every window offers exactly K drafts (no confidence gates)
//   WZY_MTP_DVOCAB=N                  draft-vocabulary rows (default min(114452, n_vocab))
//   --forced-drafts F                 testing the accept path: with --spec-depth, each window's drafts
//                                     are replaced by tokens from file F (the drafter still runs, so its
//                                     catch-up is exercised).  F holds two lines of token ids: a pattern
//                                     a_0 a_1 ... (cycled over the windows: window i offers the next a_i
//                                     tokens of the continuation, then wrong ones) and the continuation
//                                     (the stream the engine is expected to generate, first token first)
//   WZY_DEC_PROF=1                    per-request decode profile line on stderr
// Exit status: 0 after QUIT/EXIT or end of input, 1 on any stage error (message on stderr), 2 on
// bad options.
#include <math.h>
#include <signal.h>
#include <stdarg.h>
#include <stddef.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include <atomic>
#include <chrono>
#include <condition_variable>
#include <deque>
#include <iostream>
#include <mutex>
#include <random>
#include <set>
#include <string>
#include <thread>
#include <vector>

#include "../../include/wzy_engine.h"
#include "../../include/wzy_kernels.h"
#include "../../include/wzy_loader.h"
#include "../../include/wzy_runtime.h"
#include "../../include/wzy_stage.h"

namespace {

volatile sig_atomic_t g_sigusr1 = 0;
void on_sigusr1(int) { g_sigusr1 = 1; }

std::mutex g_out;
// Every protocol line goes through here so that lines written by the stdin reader (PONG in
// multiplexed mode) never interleave with the decode loop's.
void say(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void say(const char* fmt, ...) {
    std::lock_guard<std::mutex> lk(g_out);
    va_list ap;
    va_start(ap, fmt);
    vfprintf(stdout, fmt, ap);
    va_end(ap);
    fflush(stdout);
}

using Clock = std::chrono::steady_clock;
double ms_since(Clock::time_point t0) {
    return std::chrono::duration<double, std::milli>(Clock::now() - t0).count();
}

[[noreturn]] void die(const char* what) {
    fprintf(stderr, "[wzy-engine] %s failed: %s\n", what, wzy_last_error());
    fflush(stderr);
    exit(1);
}
void check(int rc, const char* what) {
    if (rc < 0) die(what);
}

struct Options {
    int ctx = 262144;
    bool batch = false;
    uint64_t model_seed = 3;
    bool have_seed = false;
    uint64_t seed = 0;
    std::string cfg;
    std::string model_dir;        // real weights (empty: synthetic)
    std::string dvocab;           // MTP draft vocabulary file (real weights)
    int device = 0;
    bool graphs = true;
    bool prof = false;
    bool mtp = false;
    int spec_fixed = 0;           // > 0: fixed draft depth
    int mtp_dvocab = 114452;
    wzy_spec_gates gates{5, 0.30f, 1.0f};
    bool adapt_depth = true;
    int prefill_chunk = 25600;    // cells per prefill chunk (the reference's PF_MAX default)
    std::string forced_drafts;    // test file: draft pattern + expected continuation
};

// "k=v,k=v" onto wzy_stage_cfg by field name.
bool apply_cfg(wzy_stage_cfg& c, const std::string& spec) {
    struct F {
        const char* name;
        int* i;
        float* f;
    } fields[] = {
        {"n_layers", &c.n_layers, nullptr},   {"qsa_period", &c.qsa_period, nullptr},
        {"n_embd", &c.n_embd, nullptr},       {"hc", &c.hc, nullptr},
        {"hc_lr", &c.hc_lr, nullptr},         {"gdn_hk", &c.gdn_hk, nullptr},
        {"gdn_hv", &c.gdn_hv, nullptr},       {"qsa_qh", &c.qsa_qh, nullptr},
        {"qsa_kvh", &c.qsa_kvh, nullptr},     {"qsa_hd", &c.qsa_hd, nullptr},
        {"n_rot", &c.n_rot, nullptr},         {"idx_heads", &c.idx_heads, nullptr},
        {"idx_dim", &c.idx_dim, nullptr},     {"idx_blk", &c.idx_blk, nullptr},
        {"idx_topk", &c.idx_topk, nullptr},   {"n_exp", &c.n_exp, nullptr},
        {"top_k", &c.top_k, nullptr},         {"n_ff", &c.n_ff, nullptr},
        {"n_vocab", &c.n_vocab, nullptr},     {"ctx_max", &c.ctx_max, nullptr},
        {"kv_ring", &c.kv_ring, nullptr},     {"kv_sinks", &c.kv_sinks, nullptr},
        {"rope_theta", nullptr, &c.rope_theta}, {"eps", nullptr, &c.eps},
        {"emb_q8", &c.emb_q8, nullptr},       {"head_q8", &c.head_q8, nullptr},
        {"attn_f16_above", &c.attn_f16_above, nullptr}, {"ple", &c.ple, nullptr},
        {"ple_eos", &c.ple_eos, nullptr},
    };
    size_t at = 0;
    while (at < spec.size()) {
        size_t end = spec.find(',', at);
        if (end == std::string::npos) end = spec.size();
        const std::string kv = spec.substr(at, end - at);
        at = end + 1;
        if (kv.empty()) continue;
        const size_t eq = kv.find('=');
        if (eq == std::string::npos) return false;
        const std::string k = kv.substr(0, eq), v = kv.substr(eq + 1);
        bool hit = false;
        for (const F& f : fields) {
            if (k != f.name) continue;
            if (f.i) *f.i = atoi(v.c_str());
            else *f.f = (float) atof(v.c_str());
            hit = true;
        }
        if (!hit) return false;
    }
    return true;
}

int parse_options(int argc, char** argv, Options& o) {
    if (const char* e = getenv("WZY_CTX")) o.ctx = atoi(e);
    if (const char* e = getenv("WZY_BATCH")) o.batch = atoi(e) > 0;
    if (const char* e = getenv("WZY_MODEL_SEED")) o.model_seed = strtoull(e, nullptr, 10);
    if (const char* e = getenv("WZY_SEED")) o.have_seed = true, o.seed = strtoull(e, nullptr, 10);
    if (const char* e = getenv("WZY_CFG")) o.cfg = e;
    if (const char* e = getenv("WZY_MODEL_DIR")) o.model_dir = e;
    if (const char* e = getenv("WZY_DRAFT_VOCAB")) o.dvocab = e;
    if (const char* e = getenv("WZY_DEVICE")) o.device = atoi(e);
    if (const char* e = getenv("WZY_GRAPHS")) o.graphs = atoi(e) != 0;
    if (const char* e = getenv("WZY_DEC_PROF")) o.prof = atoi(e) != 0;
    if (const char* e = getenv("WZY_MTP")) o.mtp = atoi(e) != 0;
    if (const char* e = getenv("WZY_SPEC_FIXED")) o.spec_fixed = atoi(e);
    if (const char* e = getenv("WZY_MTP_DVOCAB")) o.mtp_dvocab = atoi(e);
    if (const char* e = getenv("WZY_SPEC_DEPTH")) o.gates.depth = atoi(e);
    if (const char* e = getenv("WZY_SPEC_MIN_P")) o.gates.min_p = (float) atof(e);
    if (const char* e = getenv("WZY_SPEC_GATE")) o.gates.gate = (float) atof(e);
    if (const char* e = getenv("WZY_ADAPT_DEPTH")) o.adapt_depth = atoi(e) != 0;
    if (const char* e = getenv("WZY_PREFILL_CHUNK")) o.prefill_chunk = atoi(e);
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        auto val = [&]() -> const char* {
            if (i + 1 >= argc) {
                fprintf(stderr, "[wzy-engine] %s needs a value\n", a.c_str());
                exit(2);
            }
            return argv[++i];
        };
        if (a == "--ctx") o.ctx = atoi(val());
        else if (a == "--batch") o.batch = true;
        else if (a == "--model-seed") o.model_seed = strtoull(val(), nullptr, 10);
        else if (a == "--seed") o.have_seed = true, o.seed = strtoull(val(), nullptr, 10);
        else if (a == "--cfg") o.cfg = val();
        else if (a == "--model-dir") o.model_dir = val();
        else if (a == "--device") o.device = atoi(val());
        else if (a == "--no-graphs") o.graphs = false;
        else if (a == "--mtp") o.mtp = true;
        else if (a == "--spec-depth") o.spec_fixed = atoi(val()), o.mtp = true;
        else if (a == "--prefill-chunk") o.prefill_chunk = atoi(val());
        else if (a == "--forced-drafts") o.forced_drafts = val();
        else {
            fprintf(stderr, "[wzy-engine] unknown option %s\n", a.c_str());
            return 2;
        }
    }
    if (o.spec_fixed > 0) o.mtp = true;
    if (!o.forced_drafts.empty() && o.spec_fixed <= 0) {
        fprintf(stderr, "[wzy-engine] --forced-drafts needs --spec-depth\n");
        return 2;
    }
    o.prefill_chunk = std::max(1, std::min(o.prefill_chunk, 25600));
    o.spec_fixed = std::min(o.spec_fixed, WZY_MAX_W - 1);
    o.gates.depth = std::max(1, std::min(o.gates.depth, WZY_MAX_W - 1));
    return 0;
}

// Input lines handed from the stdin reader to the request loop.
struct Inbox {
    std::mutex mu;
    std::condition_variable cv;
    std::deque<std::string> lines;
    std::set<int> cancels;       // multiplexed CANCEL targets not yet consumed
    bool eof = false;
    std::atomic<bool> quit{false};
};

class Engine {
  public:
    Engine(const Options& o, wzy_stage* st, const wzy_stage_cfg& c, Inbox& in)
        : o_(o), st_(st), c_(c), in_(in), rng_(o.have_seed ? o.seed : std::random_device{}()) {
        logits_.resize((size_t) WZY_MAX_W * c.n_vocab);
        if (!o.forced_drafts.empty()) load_forced(o.forced_drafts);
    }

    // One request line (JSON or legacy), answered in the single-stream or multiplexed form.
    void run(const std::string& line) {
        wzy_request r;
        std::vector<int> ids(line.size() / 2 + 8);
        wzy_engine_parse_line(line.c_str(), &r, ids.data(), (int) ids.size());
        ids.resize(std::min<size_t>(r.n_ids, ids.size()));
        const int req = (o_.batch && r.json) ? r.req : -1;
        g_sigusr1 = 0;
        if (r.has_emb_file) fprintf(stderr, "[wzy-engine] emb_file ignored: image embeddings are not supported\n");
        if (ids.empty()) {
            if (r.json) emit_fmt(WZY_FMT_DONE_EMPTY, base_fields(req));
            else say("output :\nEND\n");
            return;
        }
        if ((int) ids.size() >= c_.ctx_max - 16) ids.erase(ids.begin(), ids.end() - (c_.ctx_max - 128));
        const wzy_gen_cfg& g = r.cfg;
        const int n = (int) ids.size();

        // Two-slot prefix reuse (src/wzy_engine_v2.cu:1962-1997): keep the active state, or bring
        // the parked session back (parking the active one in its place when it is worth keeping),
        // or park the active session before the reset for an unrelated prompt.
        int reused = 0;
        const int plan = wzy_engine_session_plan(state_.data(), (int) state_.size(), parked_.data(),
                                                 (int) parked_.size(), ids.data(), n, g.no_reuse, &reused);
        bool restored_park = false;
        if (plan == WZY_SESS_SWAP) {
            const int tmp = parked_slot_ ^ 1;
            check(wzy_stage_session_save(st_, tmp, (int) state_.size()), "session_save");
            check(wzy_stage_session_restore(st_, parked_slot_), "session_restore");
            std::swap(state_, parked_);
            parked_slot_ = tmp;
            restored_park = true;
        } else if (plan == WZY_SESS_RESTORE) {
            check(wzy_stage_session_restore(st_, parked_slot_), "session_restore");
            state_ = parked_;
            restored_park = true;
        } else if (plan == WZY_SESS_PARK_RESET) {
            check(wzy_stage_session_save(st_, parked_slot_, (int) state_.size()), "session_save");
            parked_ = state_;
        }
        if (plan == WZY_SESS_PARK_RESET || plan == WZY_SESS_RESET) {
            check(wzy_stage_reset_state(st_), "reset_state");
            state_.clear();
        }
        const auto t_pf0 = Clock::now();
        // Prompt cells in windows of up to WZY_MAX_W rows.  With the drafter, windows that reach the
        // last kMtpSeedTail cells also leave their pre-head residuals, which seed the drafter's ring
        // (seed_mtp_tail, src/wzy_engine_v2.cu:1266-1290).
        const int tail_floor = std::max(0, n - 1 - kMtpSeedTail);
        if (o_.mtp && reused == 0) check(wzy_stage_mtp_reset(st_), "mtp_reset");
        // Up to kPrefillMin cells go through decode windows; more through chunked prefill
        // (run_prefill_range, src/wzy_engine_v2.cu:1292-1376).  Either way the chunk's last
        // kMtpSeedTail cells leave their pre-head rows, which seed the drafter 8 rows at a time.
        const int n_feed = n - 1 - reused;
        const int step = (n_feed > kPrefillMin && wzy_stage_can_prefill(&c_)) ? o_.prefill_chunk : WZY_MAX_W;
        for (int p = reused; p < n - 1; p += step) {
            const int T = std::min(step, n - 1 - p);
            const bool seed = o_.mtp && p + T > tail_floor;
            if (step == WZY_MAX_W)
                check(wzy_stage_record_forward(st_, p, nullptr, &ids[p], T, seed ? 2 : 0, 0, 0, 0), "record_forward(prefill)");
            else
                check(wzy_stage_prefill(st_, p, &ids[p], T), "prefill");
            if (seed) {
                const int sub0 = std::max(0, tail_floor - p);
                if (p + sub0 == tail_floor && tail_floor > 0) check(wzy_stage_mtp_set_floor(st_, tail_floor), "mtp_floor");
                for (int off = sub0; off < T; off += WZY_MAX_W) {
                    const int cnt = std::min(WZY_MAX_W, T - off);
                    check(wzy_stage_mtp_front(st_, p + off, &ids[p + off + 1], cnt, off), "mtp_front");
                }
            }
        }
        state_.insert(state_.end(), ids.begin() + reused, ids.end() - 1);

        const bool no_rep = fabsf(g.rep_pen - 1.0f) < 1e-5f;
        mode_ = (no_rep && g.temp <= 1e-5f) ? kGreedy : (no_rep && g.top_k > 0 && g.top_k <= 16) ? kTop16 : kFull;
        std::vector<int> hist(ids);
        int cur = 0;
        {
            const int last = ids[n - 1];
            check(wzy_stage_record_forward(st_, n - 1, nullptr, &last, 1, 1, 0, mode_ == kTop16, 0), "record_forward");
            check(wzy_stage_sync(st_), "sync");
            read_rows(1);
            pick_row(0, -1, g, hist, &cur);
        }
        state_.push_back(ids[n - 1]);
        const double pf_ms = ms_since(t_pf0);

        wzy_line_fields f = base_fields(req);
        f.prompt_tokens = n;
        f.reused = reused;
        f.read = n - reused;
        f.prompt_ms = pf_ms;
        f.restored_park = restored_park ? 1 : 0;
        f.parked_tokens = (int) parked_.size();
        if (r.json) emit_fmt(WZY_FMT_PREFILL, f);
        else say("output :");

        // Decode loop (src/wzy_engine_v2.cu:2119-2205): emit the current token, let the drafter
        // propose, verify the window [cur, drafts...] in one forward with rank-1 acceptance, keep the
        // state of the accepted prefix.  Without the drafter every window is the single row [cur].
        const auto t_dec0 = Clock::now();
        int generated = 0, cur_pos = n, wins = 0;
        const char* finish = "length";
        double fwd_ms = 0.0, mtp_ms = 0.0;
        float acc_ema = 0.5f;
        long long drafts_offered = 0, drafts_accepted = 0;
        int unfed_cell0 = n - 1;                      // drafter catch-up: cells whose next token is known
        std::vector<int> unfed_next{cur};
        std::vector<int> drafts, win;
        auto is_stop = [&](int t) {
            for (int i = 0; i < g.n_stops; ++i)
                if (g.stops[i] == t) return true;
            return false;
        };
        auto emit = [&](int t) {
            if (!r.json) say(" %d", t);
            else if (req >= 0) say("TOK %d %d\n", req, t);
            else say("TOK %d\n", t);
        };
        while (generated < g.max_new && cur_pos < c_.ctx_max - 8) {
            if (cancelled(req)) {
                finish = "cancelled";
                break;
            }
            if (is_stop(cur)) {
                finish = "stop";
                break;
            }
            ++generated;
            hist.push_back(cur);
            emit(cur);
            if (generated >= g.max_new || cur_pos >= c_.ctx_max - 8) {
                finish = "length";
                break;
            }
            drafts.clear();
            if (o_.mtp) {
                int want_k = std::min(o_.spec_fixed > 0 ? o_.spec_fixed : std::min(g.spec_k, WZY_MAX_W - 1),
                                      g.max_new - generated);
                if (o_.spec_fixed <= 0 && o_.adapt_depth && want_k > 2) {
                    if (acc_ema < 0.35f) want_k = 2;
                    else if (acc_ema < 0.55f) want_k = std::min(want_k, 3);
                }
                const auto t_m = Clock::now();
                propose(unfed_cell0, unfed_next, want_k, g, drafts);
                mtp_ms += ms_since(t_m);
                if (!forced_pattern_.empty()) force_drafts(wins, generated, drafts);
            }
            drafts_offered += (long long) drafts.size();
            win.assign(1, cur);
            win.insert(win.end(), drafts.begin(), drafts.end());
            const int W = (int) win.size();
            const auto t_f = Clock::now();
            check(wzy_stage_record_forward(st_, cur_pos, nullptr, win.data(), W, 1, W > 1 ? 1 : 0, mode_ == kTop16, 0),
                  "record_forward");
            check(wzy_stage_sync(st_), "sync");
            read_rows(W);
            fwd_ms += ms_since(t_f);
            ++wins;
            int n_acc = 0, bonus = 0;
            bool hit_stop = false;
            for (int j = 0; j < W; ++j) {
                const int d_cand = (j + 1 < W) ? win[j + 1] : -1;
                int sampled = 0;
                const bool ok = pick_row(j, d_cand, g, hist, &sampled);
                if (j + 1 < W && ok) {
                    if (is_stop(sampled)) {
                        hit_stop = true;
                        finish = "stop";
                        break;
                    }
                    ++n_acc;
                    ++drafts_accepted;
                    ++generated;
                    hist.push_back(sampled);
                    emit(sampled);
                    if (generated >= g.max_new) {
                        bonus = sampled;
                        break;
                    }
                } else {
                    bonus = sampled;
                    if (is_stop(bonus)) {
                        hit_stop = true;
                        finish = "stop";
                    }
                    break;
                }
            }
            const int acc_rows = std::min(W, 1 + n_acc);
            if (!drafts.empty()) acc_ema = 0.7f * acc_ema + 0.3f * (float) n_acc / (float) drafts.size();
            // all rows accepted: the state after the last row is already in place
            if (W > 1 && acc_rows < W)
                check(wzy_stage_commit_window_state(st_, acc_rows - 1, cur_pos + acc_rows - 1), "commit_window_state");
            state_.insert(state_.end(), win.begin(), win.begin() + acc_rows);
            if (hit_stop || generated >= g.max_new) break;
            if (cancelled(req)) {
                finish = "cancelled";
                break;
            }
            unfed_cell0 = cur_pos;
            unfed_next.assign(win.begin() + 1, win.begin() + acc_rows);
            unfed_next.push_back(bonus);
            cur_pos += acc_rows;
            cur = bonus;
        }
        if (in_.quit.load() && o_.batch) return;   // QUIT in multiplexed mode ends the process without DONE
        {
            std::lock_guard<std::mutex> lk(in_.mu);   // a CANCEL that arrived after the last check is void
            in_.cancels.erase(req);
        }
        const double dec_ms = ms_since(t_dec0);
        if (o_.prof)
            fprintf(stderr,
                    "[DEC-PROF gen=%d wins=%d (%.2f tok/win)] total=%.1fms (%.2f ms/win) | stage=%.2fms mtp=%.2fms "
                    "drafts=%lld accepted=%lld\n",
                    generated, wins, wins > 0 ? (double) (generated - 1) / wins : 0.0, dec_ms,
                    wins > 0 ? dec_ms / wins : 0.0, fwd_ms, mtp_ms, drafts_offered, drafts_accepted);
        if (!r.json) {
            say("\nEND\n");
            return;
        }
        f.generated = generated;
        f.decode_ms = dec_ms;
        f.draft_n = drafts_offered;
        f.draft_accepted = drafts_accepted;
        f.active_tokens = (int) state_.size();
        f.finish = finish;
        emit_fmt(WZY_FMT_DONE, f);
    }

    // RESET: empty state, no parked session (src/wzy_engine_v2.cu:1851)
    void reset() {
        check(wzy_stage_reset_state(st_), "reset_state");
        if (o_.mtp) check(wzy_stage_mtp_reset(st_), "mtp_reset");
        check(wzy_stage_sync(st_), "sync");
        for (int s = 0; s < WZY_SESSION_SLOTS; ++s) check(wzy_stage_session_clear(st_, s), "session_clear");
        state_.clear();
        parked_.clear();
    }

  private:
    enum Mode { kGreedy, kTop16, kFull };

    // --forced-drafts: line 1 the pattern, line 2 the continuation (whitespace-separated ids)
    void load_forced(const std::string& path) {
        FILE* f = fopen(path.c_str(), "r");
        if (!f) die("forced drafts: cannot open file");
        std::vector<int>* dst = &forced_pattern_;
        int ch, v = 0;
        bool in_num = false;
        while ((ch = fgetc(f)) != EOF) {
            if (ch >= '0' && ch <= '9') {
                v = v * 10 + (ch - '0');
                in_num = true;
                continue;
            }
            if (in_num) dst->push_back(v);
            in_num = false;
            v = 0;
            if (ch == '\n' && dst == &forced_pattern_ && !forced_pattern_.empty()) dst = &forced_cont_;
        }
        if (in_num) dst->push_back(v);
        fclose(f);
        if (forced_pattern_.empty() || forced_cont_.empty()) die("forced drafts: need a pattern line and a continuation line");
    }
    // Window `win` (0-based) after `generated` emitted tokens: the drafts become the continuation's
    // next a = pattern[win % len] tokens, then tokens that differ from the continuation's; the count
    // the drafter proposed is kept (cut where the continuation ends).
    void force_drafts(int win, int generated, std::vector<int>& drafts) {
        const int a = forced_pattern_[(size_t) win % forced_pattern_.size()];
        std::vector<int> out;
        for (int j = 0; j < (int) drafts.size() && generated + j < (int) forced_cont_.size(); ++j) {
            const int truth = forced_cont_[(size_t) generated + j];
            out.push_back(j < a ? truth : (truth + 1) % c_.n_vocab);
        }
        drafts.swap(out);
    }

    static constexpr int kMtpSeedTail = 512;   // prompt cells seeded into the drafter (src/wzy_mtp.cuh:12)
    static constexpr int kPrefillMin = 192;    // longer prompt remainders take the chunked prefill
                                               // (src/wzy_engine_v2.cu:1295)

    // Head outputs of the W rows of the last forward, as the selection mode needs them.
    void read_rows(int W) {
        if (mode_ == kGreedy) check(wzy_stage_greedy_ids(st_, greedy_, W), "greedy_ids");
        else if (mode_ == kTop16) check(wzy_stage_top16(st_, top_v_, top_i_, W), "top16");
        else check(wzy_stage_logits(st_, logits_.data(), W), "logits");
    }

    // Select row j's token and verify `draft` against it (-1: nothing to verify).  Rank-1
    // acceptance: the draft is kept when it is the token this row selects.
    bool pick_row(int j, int draft, const wzy_gen_cfg& g, const std::vector<int>& hist, int* out) {
        if (mode_ == kGreedy) {
            *out = greedy_[j];
            return draft >= 0 && draft == *out;
        }
        const float u = std::uniform_real_distribution<float>(0.f, 1.f)(rng_);
        int acc = 0;
        if (mode_ == kTop16)
            acc = wzy_engine_verify_top16(top_v_ + 16 * j, top_i_ + 16 * j, &g, hist.data(), (int) hist.size(), draft,
                                          u, out);
        else
            acc = wzy_engine_verify_full(logits_.data() + (size_t) j * c_.n_vocab, c_.n_vocab, &g, hist.data(),
                                         (int) hist.size(), draft, u, out);
        check(acc, "sample");
        return acc == 1;
    }

    // mtp_propose (src/wzy_engine_v2.cu:1384-1475): catch the drafter up on the cells whose next
    // token became known, draft from the last of them, keep the drafts the confidence gates pass.
    // The chain runs on the device without host round trips; the gates, which only truncate it,
    // are applied to its outputs (first step alone, the rest only when the first passes).
    void propose(int cell0, const std::vector<int>& next, int want_k, const wzy_gen_cfg& g, std::vector<int>& drafts) {
        drafts.clear();
        const int n_cells = (int) next.size();
        if (want_k <= 0 || n_cells <= 0) return;
        const int last_cell = cell0 + n_cells - 1;
        if (n_cells > 1) check(wzy_stage_mtp_front(st_, cell0, next.data(), n_cells - 1, 0), "mtp_front");
        int toks[WZY_MAX_W + 1];
        float probs[WZY_MAX_W + 1];
        const int room = c_.ctx_max - 4 - last_cell;       // steps at cells last_cell .. ctx_max - 5
        if (o_.spec_fixed > 0) {
            const int depth = std::min(want_k, room);
            if (depth < 1) return;
            check(wzy_stage_mtp_draft(st_, last_cell, next.back(), n_cells - 1, depth, toks, probs), "mtp_draft");
            for (int j = 0; j < depth; ++j) {
                bool stop = false;
                for (int i = 0; i < g.n_stops; ++i) stop |= g.stops[i] == toks[j];
                if (stop) break;
                drafts.push_back(toks[j]);
            }
            return;
        }
        if (room < 1) return;
        check(wzy_stage_mtp_draft(st_, last_cell, next.back(), n_cells - 1, 1, toks, probs), "mtp_draft");
        if (wzy_engine_mtp_gate(toks, probs, 1, next.back(), last_cell, c_.ctx_max, &g, want_k, &o_.gates) < 1) return;
        const int more = std::min(std::min(o_.gates.depth, want_k) - 1, room - 1);
        if (more > 0)
            check(wzy_stage_mtp_draft(st_, last_cell + 1, toks[0], -1, more, toks + 1, probs + 1), "mtp_draft");
        const int kept = wzy_engine_mtp_gate(toks, probs, 1 + std::max(more, 0), next.back(), last_cell, c_.ctx_max, &g,
                                             want_k, &o_.gates);
        drafts.assign(toks, toks + kept);
    }

    bool cancelled(int req) {
        if (g_sigusr1) return true;
        if (in_.quit.load() && o_.batch) return true;
        std::lock_guard<std::mutex> lk(in_.mu);
        auto it = in_.cancels.find(req);
        if (it == in_.cancels.end()) return false;
        in_.cancels.erase(it);
        return true;
    }

    wzy_line_fields base_fields(int req) const {
        wzy_line_fields f;
        memset(&f, 0, sizeof(f));
        f.req = req;
        f.vram_hit = 1.0;        // every expert is resident in HBM
        f.finish = "stop";
        return f;
    }

    void emit_fmt(int what, const wzy_line_fields& f) {
        char buf[1024];
        if (wzy_engine_format(what, &f, buf, sizeof(buf)) < 0) die("format");
        say("%s", buf);
    }

    const Options& o_;
    wzy_stage* st_;
    wzy_stage_cfg c_;
    Inbox& in_;
    std::mt19937 rng_;
    Mode mode_ = kGreedy;
    std::vector<int> state_;      // tokens whose cells the resident state holds
    std::vector<int> parked_;     // tokens of the parked session (empty: none)
    int parked_slot_ = 0;         // stage session slot holding it; the other slot is the swap spare
    std::vector<float> logits_;
    int greedy_[WZY_MAX_W] = {};
    float top_v_[WZY_MAX_W * 16] = {};
    int top_i_[WZY_MAX_W * 16] = {};
    std::vector<int> forced_pattern_, forced_cont_;   // --forced-drafts (empty: the drafter's own)
};

// stdin reader: in multiplexed mode PING, CANCEL and QUIT are answered / recorded immediately (the
// decode loop keeps running); everything else is queued for the request loop in arrival order.
void read_stdin(Inbox& in, bool batch) {
    std::string line;
    while (std::getline(std::cin, line)) {
        if (line.empty()) continue;
        if (batch) {
            wzy_request r;
            const int kind = wzy_engine_parse_line(line.c_str(), &r, nullptr, 0);
            if (kind == WZY_LINE_PING) {
                say("PONG\n");
                continue;
            }
            if (kind == WZY_LINE_CANCEL) {
                std::lock_guard<std::mutex> lk(in.mu);
                bool queued = false;
                for (auto it = in.lines.begin(); it != in.lines.end(); ++it) {
                    wzy_request q;
                    if (wzy_engine_parse_line(it->c_str(), &q, nullptr, 0) == WZY_LINE_REQUEST && q.json &&
                        q.req == r.req) {
                        in.lines.erase(it);          // not started: drop it (no lines are owed for it)
                        queued = true;
                        break;
                    }
                }
                if (!queued) in.cancels.insert(r.req);
                continue;
            }
            if (kind == WZY_LINE_QUIT) in.quit.store(true);
        }
        {
            std::lock_guard<std::mutex> lk(in.mu);
            in.lines.push_back(line);
        }
        in.cv.notify_all();
        if (batch && in.quit.load()) break;
    }
    {
        std::lock_guard<std::mutex> lk(in.mu);
        in.eof = true;
    }
    in.cv.notify_all();
}

}  // namespace

int main(int argc, char** argv) {
    const auto t_boot0 = Clock::now();
    Options o;
    if (int rc = parse_options(argc, argv, o)) return rc;

    wzy_stage_cfg c;
    wzy_stage_cfg_default(&c, o.ctx);
    const std::string gguf = o.model_dir + "/qwen-nvfp4-gptq-dense.gguf", emb_file = o.model_dir + "/token-embd-bf16.gguf";
    const bool have_emb_file = !o.model_dir.empty() && access(emb_file.c_str(), R_OK) == 0;
    if (!o.model_dir.empty()) {
        check(wzy_stage_cfg_from_gguf(gguf.c_str(), o.ctx, &c), "cfg_from_gguf");
        if (have_emb_file) c.emb_q8 = 0;              // the bf16 table replaces the Q8_0 one
    }
    if (!apply_cfg(c, o.cfg)) {
        fprintf(stderr, "[wzy-engine] bad --cfg/WZY_CFG \"%s\"\n", o.cfg.c_str());
        return 2;
    }
    int ndev = 0;
    check(wzy_dev_count(&ndev), "device count");
    if (ndev < 1 || o.device >= ndev) {
        fprintf(stderr, "[wzy-engine] no HIP device %d (found %d)\n", o.device, ndev);
        return 1;
    }
    wzy_stage* st = nullptr;
    check(wzy_stage_create(&c, o.device, &st), "stage_create");
    if (o.model_dir.empty()) {
        check(wzy_stage_load_synthetic(st, o.model_seed, 0), "load_synthetic");
    } else {
        const std::string experts = o.model_dir + "/pack/experts.bin";
        check(wzy_stage_load_gguf(st, gguf.c_str(), experts.c_str(), have_emb_file ? emb_file.c_str() : nullptr),
              "load_gguf");
        if (c.ple) check(wzy_stage_load_ple(st, (o.model_dir + "/ple-fp8.gguf").c_str()), "load_ple");
    }
    if (o.mtp && o.model_dir.empty()) {
        const int n_dv = std::max(1, std::min(o.mtp_dvocab, c.n_vocab));
        check(wzy_stage_mtp_init(st, o.model_seed + 1, n_dv), "mtp_init");
    } else if (o.mtp) {
        const std::string dir = o.model_dir + "/mtp";
        const std::string dv = o.dvocab.empty() ? dir + "/draft_vocab.bin" : o.dvocab;
        check(wzy_stage_mtp_load(st, dir.c_str(), dv.c_str()), "mtp_load");
    }
    check(wzy_stage_set_graphs(st, o.graphs ? 1 : 0), "set_graphs");
    check(wzy_stage_sync(st), "sync");
    signal(SIGUSR1, on_sigusr1);

    const double boot_s = ms_since(t_boot0) / 1000.0;
    if (o.batch)
        say("READY {\"engine\":\"wzy-mi355x-batch\",\"gpus\":1,\"split\":%d,\"vram_slots\":%d,\"mtp\":%s,"
            "\"ctx_max\":%d,\"boot_s\":%.2f,\"sessions\":1}\n",
            c.n_layers, c.n_layers * c.n_exp, o.mtp ? "true" : "false", c.ctx_max, boot_s);
    else
        say("READY {\"engine\":\"wzy-mi355x\",\"gpus\":1,\"split\":%d,\"vram_slots\":%d,\"mtp\":%s,"
            "\"ctx_max\":%d,\"boot_s\":%.2f}\n",
            c.n_layers, c.n_layers * c.n_exp, o.mtp ? "true" : "false", c.ctx_max, boot_s);

    Inbox in;
    Engine eng(o, st, c, in);
    std::thread reader(read_stdin, std::ref(in), o.batch);
    reader.detach();   // blocked in getline at exit; the process ends with main
    for (;;) {
        std::string line;
        {
            std::unique_lock<std::mutex> lk(in.mu);
            in.cv.wait(lk, [&] { return !in.lines.empty() || in.eof; });
            if (in.lines.empty()) break;
            line = std::move(in.lines.front());
            in.lines.pop_front();
        }
        wzy_request r;
        const int kind = wzy_engine_parse_line(line.c_str(), &r, nullptr, 0);
        if (kind == WZY_LINE_QUIT) break;
        if (kind == WZY_LINE_PING) say("PONG\n");
        else if (kind == WZY_LINE_RESET) {
            eng.reset();
            say("OK\n");
        } else if (kind == WZY_LINE_SAVE_PROFILE) {
            say("OK\n");        // no expert-placement profile: every expert is resident
        } else if (kind == WZY_LINE_REQUEST) {
            eng.run(line);
        }
        if (in.quit.load()) break;
    }
    check(wzy_stage_sync(st), "sync");
    wzy_stage_destroy(st);
    return 0;
}

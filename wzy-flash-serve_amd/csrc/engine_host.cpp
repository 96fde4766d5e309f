// engine_host.cpp -- host logic of the decode engine's stream protocol: request parsing, samplers,
// prompt-prefix reuse and protocol line formatting (no GPU code; C ABI in include/wzy_engine.h).
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "../../include/wzy_engine.h"
#include "../../include/wzy_kernels.h"

namespace {

// Repetition penalty looks at the last 512 ids and counts as active when |pen - 1| >= 1e-5
// (reference REP_PEN_WINDOW / REP_PEN_EPS, src/wzy_engine_v2.cu:32-33).
constexpr int kRepWindow = 512;
constexpr float kRepEps = 1e-5f;
constexpr float kGreedyTemp = 1e-5f;

// ---- key-search JSON readers (src/wzy_engine_v2.cu:595-641) ------------------------------------
// The protocol's JSON is read by locating the quoted key as a substring, exactly as the reference
// engines do; the request lines come from a trusted supervisor, so this is not a JSON validator.

// Integers between the first '[' after `key` and the next ']'.  A '-' marks the number being read
// as negative; any other non-digit ends it.
bool key_ints(const std::string& s, const char* key, std::vector<int>& out) {
    out.clear();
    size_t at = s.find(key);
    if (at == std::string::npos) return false;
    size_t lb = s.find('[', at);
    if (lb == std::string::npos) return false;
    size_t rb = s.find(']', lb);
    if (rb == std::string::npos) return false;
    long long v = 0;
    bool digits = false, minus = false;
    for (size_t i = lb + 1; i <= rb; ++i) {
        char c = (i < rb) ? s[i] : ',';
        if (c >= '0' && c <= '9') {
            v = v * 10 + (c - '0');
            digits = true;
        } else if (c == '-') {
            minus = true;
        } else {
            if (digits) out.push_back((int) (minus ? -v : v));
            v = 0;
            digits = minus = false;
        }
    }
    return true;
}

// strtod of the text after the first ':' following `key` (spaces/tabs skipped); `def` when the key
// is absent or no number follows.
double key_num(const std::string& s, const char* key, double def, bool* found = nullptr) {
    if (found) *found = false;
    size_t at = s.find(key);
    if (at == std::string::npos) return def;
    size_t colon = s.find(':', at);
    if (colon == std::string::npos) return def;
    const char* p = s.c_str() + colon + 1;
    while (*p == ' ' || *p == '\t') ++p;
    char* end = nullptr;
    double v = strtod(p, &end);
    if (end == p) return def;
    if (found) *found = true;
    return v;
}

// "key":"value" with backslash escapes taken literally.
bool key_str(const std::string& s, const char* key, std::string& out) {
    size_t at = s.find(key);
    if (at == std::string::npos) return false;
    size_t q = s.find('"', at + strlen(key));
    if (q == std::string::npos) return false;
    std::string v;
    for (size_t i = q + 1; i < s.size(); ++i) {
        if (s[i] == '\\' && i + 1 < s.size()) {
            v.push_back(s[++i]);
        } else if (s[i] == '"') {
            out = v;
            return true;
        } else {
            v.push_back(s[i]);
        }
    }
    return false;
}

// Value after the repetition penalty: positive logits are divided, others multiplied.
inline float penalise(float v, float pen) { return v > 0.f ? v / pen : v * pen; }

// Index order used by every ranking here: larger value first, lower id first among equals.
inline bool ranks_before(float va, int ia, float vb, int ib) { return va > vb || (va == vb && ia < ib); }

void sort_desc(float* v, int* id, int n) {
    for (int i = 1; i < n; ++i) {
        float xv = v[i];
        int xi = id[i];
        int j = i;
        for (; j > 0 && ranks_before(xv, xi, v[j - 1], id[j - 1]); --j) {
            v[j] = v[j - 1];
            id[j] = id[j - 1];
        }
        v[j] = xv;
        id[j] = xi;
    }
}

// Softmax at temperature over n descending values, then the min_p / top_p cut: returns how many
// leading entries are kept and leaves their renormalised probabilities in p.
int softmax_cut(const float* v, int n, const wzy_gen_cfg& c, float* p) {
    const float inv_t = 1.0f / c.temp;
    const float top = v[0] * inv_t;
    float z = 0.f;
    for (int i = 0; i < n; ++i) {
        p[i] = expf(v[i] * inv_t - top);
        z += p[i];
    }
    for (int i = 0; i < n; ++i) p[i] /= z;
    int keep = n;
    float cum = 0.f;
    for (int i = 0; i < n; ++i) {
        if (i > 0 && c.min_p > 0.f && p[i] < c.min_p * p[0]) {
            keep = i;
            break;
        }
        cum += p[i];
        if (c.top_p > 0.f && c.top_p < 1.0f && cum >= c.top_p) {
            keep = i + 1;
            break;
        }
    }
    float kz = 0.f;
    for (int i = 0; i < keep; ++i) kz += p[i];
    for (int i = 0; i < keep; ++i) p[i] /= kz;
    return keep;
}

// Inverse-CDF draw with the uniform variate u; the last entry when rounding leaves u unspent.
int draw(const int* ids, const float* p, int n, float u) {
    for (int i = 0; i < n; ++i) {
        u -= p[i];
        if (u <= 0.f) return ids[i];
    }
    return ids[n - 1];
}

bool seen_in_window(const int* hist, int n_hist, int tok) {
    for (int i = std::max(0, n_hist - kRepWindow); i < n_hist; ++i)
        if (hist[i] == tok) return true;
    return false;
}

}  // namespace

extern "C" void wzy_engine_cfg_default(wzy_gen_cfg* c) {
    if (!c) return;
    memset(c, 0, sizeof(*c));
    c->max_new = 512;
    c->temp = 0.0f;
    c->top_p = 0.75f;
    c->top_k = 15;
    c->min_p = 0.02f;
    c->rep_pen = 1.0f;
    c->spec_min_p = 0.72f;
    c->spec_k = 7;
    c->no_reuse = 0;
    c->n_stops = 2;                  // the reference model's <|im_end|>, <|endoftext|>
    c->stops[0] = 248046;
    c->stops[1] = 248044;
}

extern "C" int wzy_engine_parse_line(const char* line_c, wzy_request* r, int* ids, int ids_cap) {
    if (!line_c || !r) return WZY_LINE_SKIP;
    memset(r, 0, sizeof(*r));
    wzy_engine_cfg_default(&r->cfg);
    const std::string s(line_c);
    if (s.empty()) return WZY_LINE_SKIP;
    if (s == "PING") return WZY_LINE_PING;
    if (s == "RESET") return WZY_LINE_RESET;
    if (s == "SAVE_PROFILE") return WZY_LINE_SAVE_PROFILE;
    if (s == "QUIT" || s == "EXIT") return WZY_LINE_QUIT;
    if (s.compare(0, 7, "CANCEL ") == 0) {
        r->has_req = 1;
        r->req = atoi(s.c_str() + 7);
        return WZY_LINE_CANCEL;
    }
    std::vector<int> v;
    if (s[0] == '{') {
        r->json = 1;
        key_ints(s, "\"ids\"", v);
        std::vector<int> stops;
        key_ints(s, "\"stop\"", stops);
        if (!stops.empty()) {
            r->cfg.n_stops = (int) std::min<size_t>(stops.size(), WZY_MAX_STOPS);
            for (int i = 0; i < r->cfg.n_stops; ++i) r->cfg.stops[i] = stops[i];
        }
        wzy_gen_cfg& c = r->cfg;
        c.max_new = (int) key_num(s, "\"max_tokens\"", 512);
        c.temp = (float) key_num(s, "\"temperature\"", 0.3);
        c.top_p = (float) key_num(s, "\"top_p\"", 0.75);
        c.top_k = (int) key_num(s, "\"top_k\"", 15);
        c.min_p = (float) key_num(s, "\"min_p\"", 0.02);
        c.rep_pen = (float) key_num(s, "\"repetition_penalty\"", 1.0);
        c.spec_k = (int) key_num(s, "\"spec\"", 7);
        c.spec_min_p = (float) key_num(s, "\"spec_min_p\"", 0.72);
        c.no_reuse = ((int) key_num(s, "\"no_reuse\"", 0) != 0);
        bool has_req = false;
        r->req = (int) key_num(s, "\"req\"", 0, &has_req);
        r->has_req = has_req;
        std::string f;
        r->has_emb_file = key_str(s, "\"emb_file\"", f) ? 1 : 0;
    } else {
        // legacy "<id> <id> ... <total>": greedy, no stop ids, total = prompt + new tokens
        size_t sp = s.rfind(' ');
        if (sp == std::string::npos) return WZY_LINE_SKIP;
        const int total = atoi(s.c_str() + sp + 1);
        long long cur = 0;
        bool digits = false;
        for (size_t i = 0; i <= sp; ++i) {
            char c = (i < sp) ? s[i] : ' ';
            if (c >= '0' && c <= '9') {
                cur = cur * 10 + (c - '0');
                digits = true;
            } else {
                if (digits) v.push_back((int) cur);
                cur = 0;
                digits = false;
            }
        }
        r->cfg.max_new = std::max(1, total - (int) v.size());
        r->cfg.temp = 0.0f;
        r->cfg.n_stops = 0;
    }
    r->n_ids = (int) v.size();
    if (ids)
        for (int i = 0; i < r->n_ids && i < ids_cap; ++i) ids[i] = v[i];
    return WZY_LINE_REQUEST;
}

extern "C" int wzy_engine_target_dist(const float* logits, int V, const wzy_gen_cfg* c, const int* hist, int n_hist,
                                      int* out_ids, float* out_probs, int cap) {
    if (!logits || !c || V <= 0 || !out_ids || !out_probs || cap < 1 || (n_hist > 0 && !hist)) return WZY_EINVAL;
    const bool rep = fabsf(c->rep_pen - 1.0f) >= kRepEps && n_hist > 0;
    std::vector<float> pen;
    const float* src = logits;
    if (rep) {
        pen.assign(logits, logits + V);
        std::vector<uint8_t> done(V, 0);
        for (int i = std::max(0, n_hist - kRepWindow); i < n_hist; ++i) {
            const int t = hist[i];
            if (t >= 0 && t < V && !done[t]) {
                done[t] = 1;
                pen[t] = penalise(pen[t], c->rep_pen);
            }
        }
        src = pen.data();
    }
    if (c->temp <= kGreedyTemp) {
        int best = 0;
        for (int v = 1; v < V; ++v)
            if (src[v] > src[best]) best = v;
        out_ids[0] = best;
        out_probs[0] = 1.0f;
        return 1;
    }
    // Streaming top-k: fill k slots, then replace the current minimum (first slot holding it) by
    // any strictly larger logit.  The slot choice decides which of several equal logits survive,
    // so it follows the reference's order of operations (src/wzy_engine_v2.cu:72-95).
    const int k = std::min(128, (c->top_k > 0 && c->top_k < V) ? c->top_k : 64);
    float tv[128];
    int ti[128];
    int n = 0, low = 0;
    auto find_low = [&]() {
        low = 0;
        for (int j = 1; j < k; ++j)
            if (tv[j] < tv[low]) low = j;
    };
    for (int v = 0; v < V; ++v) {
        const float x = src[v];
        if (n < k) {
            tv[n] = x;
            ti[n] = v;
            if (++n == k) find_low();
        } else if (x > tv[low]) {
            tv[low] = x;
            ti[low] = v;
            find_low();
        }
    }
    sort_desc(tv, ti, n);
    float p[128];
    const int keep = softmax_cut(tv, n, *c, p);
    const int m = std::min(keep, cap);
    for (int i = 0; i < m; ++i) {
        out_ids[i] = ti[i];
        out_probs[i] = p[i];
    }
    return m;
}

extern "C" int wzy_engine_verify_full(const float* logits, int V, const wzy_gen_cfg* c, const int* hist, int n_hist,
                                      int draft, float u, int* out_tok) {
    if (!out_tok) return WZY_EINVAL;
    int ids[128];
    float p[128];
    const int n = wzy_engine_target_dist(logits, V, c, hist, n_hist, ids, p, 128);
    if (n < 0) return n;
    *out_tok = (n == 1) ? ids[0] : draw(ids, p, n, u);
    return draft >= 0 && draft == *out_tok;
}

extern "C" int wzy_engine_verify_top16(const float* top_v, const int* top_i, const wzy_gen_cfg* c, const int* hist,
                                       int n_hist, int draft, float u, int* out_tok) {
    if (!top_v || !top_i || !c || !out_tok || (n_hist > 0 && !hist)) return WZY_EINVAL;
    const int k = std::min(16, c->top_k > 0 ? c->top_k : 16);
    float v[16];
    int id[16];
    for (int i = 0; i < k; ++i) {
        v[i] = top_v[i];
        id[i] = top_i[i];
    }
    if (fabsf(c->rep_pen - 1.0f) >= kRepEps && n_hist > 0) {
        bool changed = false;
        for (int i = 0; i < k; ++i)
            if (seen_in_window(hist, n_hist, id[i])) {
                v[i] = penalise(v[i], c->rep_pen);
                changed = true;
            }
        if (changed) sort_desc(v, id, k);
    }
    if (c->temp <= kGreedyTemp) {
        *out_tok = id[0];
        return draft >= 0 && draft == id[0];
    }
    float p[16];
    const int keep = softmax_cut(v, k, *c, p);
    *out_tok = (keep == 1) ? id[0] : draw(id, p, keep, u);
    return draft >= 0 && draft == *out_tok;
}

extern "C" int wzy_engine_reuse_prefix(const int* state, int n_state, const int* ids, int n_ids) {
    if (!state || !ids || n_state <= 0 || n_ids < 1) return 0;
    const int lim = std::min(n_state, n_ids - 1);
    int m = 0;
    while (m < lim && state[m] == ids[m]) ++m;
    return m == n_state ? m : 0;
}

extern "C" int wzy_engine_session_plan(const int* active, int n_active, const int* parked, int n_parked,
                                       const int* ids, int n_ids, int no_reuse, int* reused) {
    int r = 0;
    auto keep = [](int n) { return n >= WZY_PARK_MIN && n <= WZY_PARK_MAX; };
    if (reused) *reused = 0;
    if (!no_reuse && (r = wzy_engine_reuse_prefix(active, n_active, ids, n_ids)) > 0) {
        if (reused) *reused = r;
        return WZY_SESS_REUSE;
    }
    if (!no_reuse && (r = wzy_engine_reuse_prefix(parked, n_parked, ids, n_ids)) > 0) {
        if (reused) *reused = r;
        return keep(n_active) ? WZY_SESS_SWAP : WZY_SESS_RESTORE;
    }
    if (!no_reuse && keep(n_active) && (n_parked <= 0 || 2LL * n_active >= (long long) n_parked))
        return WZY_SESS_PARK_RESET;
    return WZY_SESS_RESET;
}

extern "C" int wzy_engine_mtp_gate(const int* toks, const float* probs, int n, int next_tok, int last_cell,
                                   int ctx_max, const wzy_gen_cfg* cfg, int max_drafts,
                                   const wzy_spec_gates* gates) {
    if (!toks || !probs || !cfg || n < 1 || max_drafts < 1) return 0;
    wzy_spec_gates g;
    if (gates) g = *gates;
    else wzy_engine_spec_gates_default(&g);
    auto is_stop = [&](int id) {
        for (int i = 0; i < cfg->n_stops && i < WZY_MAX_STOPS; ++i)
            if (cfg->stops[i] == id) return true;
        return false;
    };
    int d_tok = toks[0];
    float d_prob = probs[0];
    if (is_stop(d_tok)) return 0;
    if (d_prob < std::min(g.min_p, cfg->spec_min_p)) return 0;
    if (d_tok == next_tok && d_prob < 0.85f) return 0;
    int kept = 1;
    float cum = d_prob;
    const int cap = std::min(g.depth, std::max(1, max_drafts));
    const float smp = cfg->spec_min_p;
    for (int j = 1; j < cap && j < n; ++j) {
        const float explore_p = ((j == 1) ? std::min(0.34f, smp) : (j == 2) ? std::min(0.46f, smp)
                                 : (j == 3) ? 0.65f : 0.78f) * g.gate;
        const float min_cum = ((j <= 1) ? 0.0f : (j == 2) ? 0.24f : (j == 3) ? 0.36f : 0.48f) * g.gate;
        if (d_prob < explore_p || cum < min_cum) break;
        if (last_cell + j >= ctx_max - 4) break;
        const int prev_d = d_tok;
        d_tok = toks[j];
        d_prob = probs[j];
        if (is_stop(d_tok) || d_tok == prev_d) break;
        if (kept >= 2 && d_tok == toks[kept - 2]) break;
        const float keep_p = ((j == 1) ? std::min(0.36f, smp) : (j == 2) ? std::min(0.48f, smp)
                              : (j == 3) ? 0.62f : 0.74f) * g.gate;
        if (d_prob < keep_p) break;
        ++kept;
        cum *= d_prob;
    }
    return kept;
}

extern "C" void wzy_engine_spec_gates_default(wzy_spec_gates* g) {
    if (!g) return;
    g->depth = 5;
    g->min_p = 0.30f;
    g->gate = 1.0f;
}

extern "C" int wzy_engine_format(int what, const wzy_line_fields* f, char* buf, int cap) {
    if (!f || !buf || cap <= 0) return WZY_EINVAL;
    int n = -1;
    const bool mux = f->req >= 0;
    const char* fin = f->finish ? f->finish : "stop";
    if (what == WZY_FMT_PREFILL) {
        const double tps = f->prompt_ms > 0 ? 1000.0 * f->read / f->prompt_ms : 0.0;
        if (mux)
            n = snprintf(buf, cap,
                         "PREFILL {\"req\":%d,\"prompt_tokens\":%d,\"reused\":%d,\"read\":%d,\"prompt_ms\":%.2f,"
                         "\"prompt_tps\":%.1f,\"restored_park\":%d,\"parked_tokens\":%d}\n",
                         f->req, f->prompt_tokens, f->reused, f->read, f->prompt_ms, tps, f->restored_park,
                         f->parked_tokens);
        else
            n = snprintf(buf, cap,
                         "PREFILL {\"prompt_tokens\":%d,\"reused\":%d,\"read\":%d,\"prompt_ms\":%.2f,"
                         "\"prompt_tps\":%.1f,\"restored_park\":%d,\"parked_tokens\":%d}\n",
                         f->prompt_tokens, f->reused, f->read, f->prompt_ms, tps, f->restored_park, f->parked_tokens);
    } else if (what == WZY_FMT_DONE) {
        if (mux)
            n = snprintf(buf, cap,
                         "DONE {\"req\":%d,\"generated\":%d,\"prompt_tokens\":%d,\"reused\":%d,\"prompt_ms\":%.2f,"
                         "\"decode_ms\":%.2f,\"draft_n\":%lld,\"draft_accepted\":%lld,\"vram_hit\":%.4f,"
                         "\"promoted\":%lld,\"restored_park\":%d,\"parked_tokens\":%d,\"active_tokens\":%d,"
                         "\"finish\":\"%s\"}\n",
                         f->req, f->generated, f->prompt_tokens, f->reused, f->prompt_ms, f->decode_ms, f->draft_n,
                         f->draft_accepted, f->vram_hit, f->promoted, f->restored_park, f->parked_tokens,
                         f->active_tokens, fin);
        else
            n = snprintf(buf, cap,
                         "DONE {\"generated\":%d,\"prompt_tokens\":%d,\"reused\":%d,\"prompt_ms\":%.2f,"
                         "\"decode_ms\":%.2f,\"decode_tps\":%.2f,\"draft_n\":%lld,\"draft_accepted\":%lld,"
                         "\"vram_hit\":%.4f,\"promoted\":%lld,\"restored_park\":%d,\"parked_tokens\":%d,"
                         "\"active_tokens\":%d,\"finish\":\"%s\"}\n",
                         f->generated, f->prompt_tokens, f->reused, f->prompt_ms, f->decode_ms,
                         f->decode_ms > 0 ? 1000.0 * f->generated / f->decode_ms : 0.0, f->draft_n,
                         f->draft_accepted, f->vram_hit, f->promoted, f->restored_park, f->parked_tokens,
                         f->active_tokens, fin);
    } else if (what == WZY_FMT_DONE_EMPTY) {
        if (mux)
            n = snprintf(buf, cap, "DONE {\"req\":%d,\"generated\":0,\"finish\":\"stop\"}\n", f->req);
        else
            n = snprintf(buf, cap, "DONE {\"generated\":0,\"finish\":\"stop\"}\n");
    } else {
        return WZY_EINVAL;
    }
    if (n < 0 || n >= cap) return WZY_EINVAL;
    return n;
}

/* wzy_engine.h -- host logic of the decode engine's stdin/stdout stream protocol.
 *
 * The engine binary (wzy_engine, built from wzy-flash-serve_amd/csrc/engine_main.cpp) speaks the
 * reference engines' line protocol byte-for-byte:
 *   in : PING | RESET | SAVE_PROFILE | QUIT | EXIT | CANCEL <req> | one JSON object per request |
 *        legacy "<id> <id> ... <total>";  SIGUSR1 cancels the running request.
 *   out: READY {...} | PONG | OK | PREFILL {...} | TOK <id> (TOK <req> <id> when multiplexed) |
 *        DONE {...}  (legacy requests: "output : <id> <id> ...\nEND").
 * References: command loop src/wzy_engine_v2.cu:1846-1950, PREFILL :2031-2035, decode loop
 * :2119-2205, DONE :2423-2427, READY :1632; multiplexed forms src/wzy_batch_engine.cu:475,489-495,
 * 563-566,1028-1030,1037-1079; client serve/engine_client.py:71-85,136-145,195-210.
 *
 * The functions below are the pure host parts of that engine (no GPU): request parsing, the
 * token samplers, prompt-prefix reuse and protocol line formatting.  They are exported from
 * libwzy_amd.so so that tests and other hosts can drive exactly the code the engine runs.
 * Status codes as in wzy_kernels.h.
 */
#ifndef WZY_ENGINE_H
#define WZY_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WZY_MAX_STOPS 64

/* Generation settings of one request.  Defaults (wzy_engine_cfg_default) are the reference's
 * GenCfg (src/wzy_engine_v2.cu:19-30); a JSON request overrides them with its own defaults for
 * absent keys (temperature 0.3, top_p 0.75, top_k 15, min_p 0.02, ...; :1905-1917). */
typedef struct wzy_gen_cfg {
    int max_new;
    float temp, top_p;
    int top_k;
    float min_p, rep_pen, spec_min_p;
    int spec_k;
    int no_reuse;
    int n_stops;
    int stops[WZY_MAX_STOPS];
} wzy_gen_cfg;

/* Kinds of input line. */
#define WZY_LINE_SKIP 0          /* empty, or not a command (e.g. a legacy line without a space) */
#define WZY_LINE_PING 1
#define WZY_LINE_RESET 2
#define WZY_LINE_SAVE_PROFILE 3
#define WZY_LINE_QUIT 4          /* QUIT or EXIT */
#define WZY_LINE_CANCEL 5        /* CANCEL <req> */
#define WZY_LINE_REQUEST 6       /* JSON object or legacy id list */

typedef struct wzy_request {
    int json;                    /* 1: JSON object line; 0: legacy "<ids ...> <total>" */
    int has_req, req;            /* "req" key present (multiplexed client) and its value; CANCEL target */
    int n_ids;                   /* prompt ids parsed (the ids buffer holds min(n_ids, cap) of them) */
    wzy_gen_cfg cfg;
    int has_emb_file;            /* "emb_file" given (image embeddings; not supported by this engine) */
} wzy_request;

void wzy_engine_cfg_default(wzy_gen_cfg* cfg);

/* Classify and parse one input line (without the trailing newline).  JSON keys are found by
 * substring search of the quoted key, as the reference does (src/wzy_engine_v2.cu:595-641): an
 * int list is the digits between the first '[' and the next ']' after the key, a number is what
 * strtod reads after the next ':'.  Returns a WZY_LINE_* kind. */
int wzy_engine_parse_line(const char* line, wzy_request* out, int* ids, int ids_cap);

/* Filtered target distribution from full-vocabulary logits: greedy one-hot when temp <= 1e-5,
 * else the top min(128, top_k or 64) logits (repetition penalty over the last 512 history ids),
 * softmax at temperature, min_p / top_p cut, renormalised; order = descending logit.
 * Writes up to `cap` (ids, probs); returns the count.
 * Replaces build_target_dist (src/wzy_engine_v2.cu:36-136). */
int wzy_engine_target_dist(const float* logits, int n_vocab, const wzy_gen_cfg* cfg, const int* hist,
                           int n_hist, int* out_ids, float* out_probs, int cap);

/* Verify draft token `draft` (-1: none) against full-vocabulary logits, sampling with the uniform
 * variate u in [0,1): *out_tok = the sampled token; returns 1 when it equals the draft.
 * Replaces verify_or_resample with rank-1 acceptance (src/wzy_engine_v2.cu:151-179). */
int wzy_engine_verify_full(const float* logits, int n_vocab, const wzy_gen_cfg* cfg, const int* hist,
                           int n_hist, int draft, float u, int* out_tok);

/* Same from the GPU's descending top-16 (values, ids) of one row.
 * Replaces verify_or_resample_top16 with rank-1 acceptance (src/wzy_engine_v2.cu:182-308). */
int wzy_engine_verify_top16(const float* top_v, const int* top_i, const wzy_gen_cfg* cfg, const int* hist,
                            int n_hist, int draft, float u, int* out_tok);

/* Cells of the resident state that a new prompt can keep: n_state when the state's tokens are a
 * prefix of ids[0 .. n_ids-2], else 0 (src/wzy_engine_v2.cu:1963-1970). */
int wzy_engine_reuse_prefix(const int* state, int n_state, const int* ids, int n_ids);

/* What a new prompt does with the active session and the one parked session (the reference's
 * two-slot longest-common-prefix reuse, src/wzy_engine_v2.cu:1962-1997):
 *   WZY_SESS_REUSE       the active state's tokens are a prefix of the prompt: keep it (*reused =
 *                        n_active cells);
 *   WZY_SESS_SWAP        the parked session's tokens are a prefix and the active session is worth
 *                        keeping: park the active one, restore the parked one (*reused = n_parked);
 *   WZY_SESS_RESTORE     the parked session matches, the active one is dropped (the parked copy
 *                        stays parked; *reused = n_parked);
 *   WZY_SESS_PARK_RESET  neither matches; the active session is parked, then the state is reset;
 *   WZY_SESS_RESET       neither matches; the state is reset (nothing worth parking, no_reuse, or
 *                        a small side request must not evict a parked session twice its size).
 * A session is worth parking when it holds WZY_PARK_MIN ..WZY_PARK_MAX cells. */
#define WZY_SESS_REUSE 0
#define WZY_SESS_SWAP 1
#define WZY_SESS_RESTORE 2
#define WZY_SESS_PARK_RESET 3
#define WZY_SESS_RESET 4
#define WZY_PARK_MIN 64
#define WZY_PARK_MAX 98304
int wzy_engine_session_plan(const int* active, int n_active, const int* parked, int n_parked, const int* ids,
                            int n_ids, int no_reuse, int* reused);

/* Tunables of the drafter's confidence gates (the reference reads them from WZY_SPEC_DEPTH,
 * WZY_SPEC_MIN_P and WZY_SPEC_GATE, src/wzy_engine_v2.cu:1436-1450). */
typedef struct wzy_spec_gates {
    int depth;                   /* chain length cap (5) */
    float min_p;                 /* first-draft probability floor (0.30, lowered by spec_min_p) */
    float gate;                  /* scale of the deeper explore / keep / cumulative gates (1.0) */
} wzy_spec_gates;
void wzy_engine_spec_gates_default(wzy_spec_gates* g);

/* The confidence gates of mtp_propose (src/wzy_engine_v2.cu:1428-1475) over a computed draft chain:
 * toks / probs [n] are the chain's drafts and top-1 probabilities (step j at cell last_cell + j),
 * next_tok the confirmed token the first step embedded.  Returns how many leading drafts are
 * offered for verification (0 .. min(n, gates->depth, max_drafts)); gates NULL = defaults.  The
 * chain needs min(gates->depth, max_drafts) steps for the answer to be the reference's. */
int wzy_engine_mtp_gate(const int* toks, const float* probs, int n, int next_tok, int last_cell, int ctx_max,
                        const wzy_gen_cfg* cfg, int max_drafts, const wzy_spec_gates* gates);

/* Values printed in PREFILL / DONE lines. */
typedef struct wzy_line_fields {
    int req;                     /* >= 0: multiplexed form with "req"; -1: single-stream form */
    int generated, prompt_tokens, reused, read;
    double prompt_ms, decode_ms;
    long long draft_n, draft_accepted, promoted;
    double vram_hit;
    int restored_park, parked_tokens, active_tokens;
    const char* finish;          /* "stop" | "length" | "cancelled" */
} wzy_line_fields;

#define WZY_FMT_PREFILL 1
#define WZY_FMT_DONE 2
#define WZY_FMT_DONE_EMPTY 3     /* DONE {"generated":0,"finish":"stop"} for an empty prompt */

/* Format one protocol line (with trailing '\n') into buf; returns its length or a negative
 * status when it does not fit. */
int wzy_engine_format(int what, const wzy_line_fields* f, char* buf, int cap);

#ifdef __cplusplus
}
#endif
#endif /* WZY_ENGINE_H */

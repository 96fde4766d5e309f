"""Host logic of the decode engine (CPU only): protocol parsing, samplers, prefix reuse, line formats.

The samplers are pinned by closed forms (one-hot greedy, two-token softmax, min_p / top_p cuts on
known probabilities, repetition penalty window) and by agreement of the two independent selection
paths the engine uses (full-vocabulary streaming top-k vs the GPU's top-16 rows).  The line formats
are pinned by tests/golden/protocol_lines.json (the reference printf formats) and by the way the
reference client reads them (serve/engine_client.py:71-85,195-210).
"""
import ctypes as C
import json
import math
import os
import subprocess

import numpy as np
import pytest

import wzy_amd

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
ENGINE = os.path.join(wzy_amd.PKG_DIR, "wzy_engine")


def parse(wz, line, cap=4096):
    r = wzy_amd.Request()
    ids = np.zeros(cap, np.int32)
    kind = wz.wzy_engine_parse_line(line.encode(), C.byref(r), ids.ctypes.data, cap)
    return wzy_amd.LINE_KINDS[kind], r, ids[:min(r.n_ids, cap)].tolist()


def cfg(wz, **kw):
    c = wzy_amd.GenCfg()
    wz.wzy_engine_cfg_default(C.byref(c))
    for k, v in kw.items():
        setattr(c, k, v)
    return c


def verify_full(wz, logits, c, hist=(), draft=-1, u=0.5):
    lg = np.ascontiguousarray(logits, np.float32)
    h = np.ascontiguousarray(hist, np.int32)
    out = C.c_int(-7)
    acc = wz.wzy_engine_verify_full(lg.ctypes.data, len(lg), C.byref(c), h.ctypes.data if len(h) else None,
                                    len(h), draft, float(u), C.byref(out))
    assert acc >= 0
    return out.value, acc


def verify_top16(wz, v, i, c, hist=(), draft=-1, u=0.5):
    v = np.ascontiguousarray(v, np.float32)
    i = np.ascontiguousarray(i, np.int32)
    h = np.ascontiguousarray(hist, np.int32)
    out = C.c_int(-7)
    acc = wz.wzy_engine_verify_top16(v.ctypes.data, i.ctypes.data, C.byref(c), h.ctypes.data if len(h) else None,
                                     len(h), draft, float(u), C.byref(out))
    assert acc >= 0
    return out.value, acc


def target_dist(wz, logits, c, hist=()):
    lg = np.ascontiguousarray(logits, np.float32)
    h = np.ascontiguousarray(hist, np.int32)
    ids = np.zeros(128, np.int32)
    p = np.zeros(128, np.float32)
    n = wz.wzy_engine_target_dist(lg.ctypes.data, len(lg), C.byref(c), h.ctypes.data if len(h) else None, len(h),
                                  ids.ctypes.data, p.ctypes.data, 128)
    assert n >= 1
    return ids[:n].tolist(), p[:n]


# ---- parsing -----------------------------------------------------------------------------------

@pytest.mark.parametrize("line,kind", [("", "SKIP"), ("PING", "PING"), ("RESET", "RESET"),
                                       ("SAVE_PROFILE", "SAVE_PROFILE"), ("QUIT", "QUIT"), ("EXIT", "QUIT"),
                                       ("CANCEL 17", "CANCEL"), ("garbage", "SKIP"), ("PING ", "REQUEST")])
def test_command_kinds(wz, line, kind):
    k, r, _ = parse(wz, line)
    assert k == kind
    if kind == "CANCEL":
        assert r.req == 17 and r.has_req


def test_json_defaults_are_the_reference_request_defaults(wz):
    # src/wzy_engine_v2.cu:1905-1917 and GenCfg stops :29
    k, r, ids = parse(wz, '{"ids":[5,6,7]}')
    assert k == "REQUEST" and r.json == 1 and ids == [5, 6, 7] and r.has_req == 0
    c = r.cfg
    assert c.max_new == 512 and c.top_k == 15 and c.spec_k == 7 and c.no_reuse == 0
    assert c.temp == pytest.approx(0.3) and c.top_p == pytest.approx(0.75) and c.min_p == pytest.approx(0.02)
    assert c.rep_pen == 1.0 and c.spec_min_p == pytest.approx(0.72)
    assert list(c.stops[:c.n_stops]) == [248046, 248044]


def test_json_overrides_as_the_client_sends_them(wz):
    # payload shape of serve/engine_client.py:136-145 + submit() (compact separators, req injected)
    req = {"ids": [151643, 42, 0, 7], "max_tokens": 64, "temperature": 0.0, "top_p": 0.9, "top_k": 8,
           "min_p": 0.05, "repetition_penalty": 1.1, "stop": [2, 3, 4], "req": 31, "no_reuse": 1}
    k, r, ids = parse(wz, json.dumps(req, separators=(",", ":")))
    assert k == "REQUEST" and ids == req["ids"] and r.has_req == 1 and r.req == 31
    c = r.cfg
    assert (c.max_new, c.top_k, c.no_reuse) == (64, 8, 1)
    assert c.temp == 0.0 and c.top_p == pytest.approx(0.9) and c.min_p == pytest.approx(0.05)
    assert c.rep_pen == pytest.approx(1.1)
    assert list(c.stops[:c.n_stops]) == [2, 3, 4]
    # spaces after separators (json.dumps default) parse the same
    k2, r2, ids2 = parse(wz, json.dumps(req))
    assert ids2 == ids and r2.cfg.max_new == 64 and r2.req == 31


def test_json_edge_cases(wz):
    k, r, ids = parse(wz, '{"ids":[],"max_tokens":3}')
    assert k == "REQUEST" and r.n_ids == 0 and ids == []
    _, r, ids = parse(wz, '{"ids":[ -4 , 9,-1],"stop":[]}')
    assert ids == [-4, 9, -1] and list(r.cfg.stops[:r.cfg.n_stops]) == [248046, 248044]   # empty stop keeps defaults
    _, r, _ = parse(wz, '{"ids":[1],"emb_file":"/x/y.sve","emb_starts":[0],"emb_counts":[4]}')
    assert r.has_emb_file == 1
    _, r, ids = parse(wz, '{"ids":[1,2,3]}', cap=2)
    assert r.n_ids == 3 and ids == [1, 2]


def test_legacy_line(wz):
    # "<ids> <total>": greedy, no stops, max_new = total - n_ids (>= 1); src/wzy_engine_v2.cu:1936-1950
    k, r, ids = parse(wz, "1 2 3 10")
    assert k == "REQUEST" and r.json == 0 and ids == [1, 2, 3]
    assert r.cfg.max_new == 7 and r.cfg.temp == 0.0 and r.cfg.n_stops == 0
    _, r, ids = parse(wz, "5 6 7 8 2")
    assert ids == [5, 6, 7, 8] and r.cfg.max_new == 1


# ---- prefix reuse --------------------------------------------------------------------------------

@pytest.mark.parametrize("state,ids,want", [
    ([], [1, 2, 3], 0),
    ([1, 2], [1, 2, 3], 2),
    ([1, 2, 3], [1, 2, 3], 0),          # the last prompt id is always re-fed
    ([1, 2, 3], [1, 2, 3, 4], 3),
    ([1, 9], [1, 2, 3], 0),             # diverging state is not reused
    ([1, 2, 3, 4], [1, 2], 0),          # state longer than the prompt
])
def test_reuse_prefix(wz, state, ids, want):
    s = np.array(state or [0], np.int32)
    i = np.array(ids, np.int32)
    assert wz.wzy_engine_reuse_prefix(s.ctypes.data, len(state), i.ctypes.data, len(ids)) == want


# ---- two-slot session plan (src/wzy_engine_v2.cu:1962-1997) -----------------------------------------

def _seq(start, n):
    return list(range(start, start + n))


A100 = _seq(1000, 100)       # a session worth parking (64 <= n <= 98304)
P300 = _seq(5000, 300)


@pytest.mark.parametrize("active,parked,ids,no_reuse,want,reused", [
    # the active state is a prefix of the prompt: kept, whatever is parked
    (A100, P300, A100 + [7, 8], 0, "REUSE", 100),
    (_seq(1, 10), [], _seq(1, 12), 0, "REUSE", 10),
    # the parked session is a prefix and the active one is worth keeping: they trade places
    (A100, P300, P300 + [9], 0, "SWAP", 300),
    (_seq(1, 64), P300, P300 + [9, 9], 0, "SWAP", 300),
    # ... not worth keeping (under 64 cells, empty, or over 98,304): the parked copy comes back, stays parked
    (_seq(1, 63), P300, P300 + [9], 0, "RESTORE", 300),
    ([], P300, P300 + [9], 0, "RESTORE", 300),
    (_seq(1, 98305), P300, P300 + [9], 0, "RESTORE", 300),
    # the parked tokens must leave at least one prompt id to feed
    (A100, P300, P300, 0, "RESET", 0),
    # nothing matches: park the active session unless a parked one is more than twice its size
    (A100, [], _seq(1, 5), 0, "PARK_RESET", 0),
    (_seq(1, 150), P300, _seq(1, 5), 0, "PARK_RESET", 0),
    (_seq(1, 149), P300, _seq(1, 5), 0, "RESET", 0),
    (_seq(1, 63), [], _seq(1, 5), 0, "RESET", 0),
    (_seq(1, 98305), [], _seq(1, 5), 0, "RESET", 0),
    # the active session diverges from the prompt after a common prefix: not a prefix, not reused
    (A100, [], A100[:50] + [3] + A100[51:] + [4], 0, "PARK_RESET", 0),
    # no_reuse: reset, never park or restore
    (A100, P300, A100 + [7], 1, "RESET", 0),
    (A100, P300, P300 + [7], 1, "RESET", 0),
])
def test_session_plan(wz, active, parked, ids, no_reuse, want, reused):
    names = {wzy_amd.SESS_REUSE: "REUSE", wzy_amd.SESS_SWAP: "SWAP", wzy_amd.SESS_RESTORE: "RESTORE",
             wzy_amd.SESS_PARK_RESET: "PARK_RESET", wzy_amd.SESS_RESET: "RESET"}
    a = np.array(active or [0], np.int32)
    p = np.array(parked or [0], np.int32)
    i = np.array(ids, np.int32)
    r = C.c_int32(-1)
    got = wz.wzy_engine_session_plan(a.ctypes.data, len(active), p.ctypes.data, len(parked), i.ctypes.data, len(ids),
                                     no_reuse, C.byref(r))
    assert names[got] == want and r.value == reused


# ---- samplers ------------------------------------------------------------------------------------

def test_greedy_is_argmax_with_lowest_index_on_ties(wz):
    lg = np.array([0.5, 2.0, 1.0, 2.0, -3.0], np.float32)
    c = cfg(wz, temp=0.0)
    for u in (0.0, 0.3, 0.99):
        assert verify_full(wz, lg, c, u=u) == (1, 0)
    assert verify_full(wz, lg, c, draft=1) == (1, 1)
    assert verify_full(wz, lg, c, draft=3) == (1, 0)
    ids, p = target_dist(wz, lg, c)
    assert ids == [1] and p.tolist() == [1.0]


def test_two_token_softmax_closed_form(wz):
    rng = np.random.default_rng(5)
    for _ in range(50):
        a, b = rng.normal(size=2) * 3
        T = float(rng.uniform(0.2, 2.0))
        lg = np.full(100, -1e4, np.float32)
        lg[17], lg[64] = a, b
        c = cfg(wz, temp=T, top_k=2, top_p=1.0, min_p=0.0)
        hi, lo = (17, 64) if (np.float32(a) > np.float32(b)) else (64, 17)
        p_hi = 1.0 / (1.0 + math.exp(-abs(float(np.float32(a)) - float(np.float32(b))) / T))
        ids, p = target_dist(wz, lg, c)
        assert ids == [hi, lo]
        assert p[0] == pytest.approx(p_hi, rel=1e-5) and p.sum() == pytest.approx(1.0, rel=1e-6)
        assert verify_full(wz, lg, c, u=p_hi * 0.999)[0] == hi
        assert verify_full(wz, lg, c, u=min(p_hi * 1.001 + 1e-6, 0.999999))[0] == lo


def test_min_p_and_top_p_cuts_on_known_probabilities(wz):
    probs = np.array([0.5, 0.3, 0.15, 0.05])
    lg = np.concatenate([np.log(probs), np.full(60, -50.0)]).astype(np.float32)
    # min_p 0.2: 0.05 < 0.2 * 0.5 -> keep 3, renormalised over 0.95 (top_p disabled at 1.0)
    ids, p = target_dist(wz, lg, cfg(wz, temp=1.0, top_k=4, top_p=1.0, min_p=0.2))
    assert ids == [0, 1, 2]
    np.testing.assert_allclose(p, probs[:3] / 0.95, rtol=1e-5)
    # top_p 0.75: cumulative 0.5, 0.8 >= 0.75 -> keep 2
    ids, p = target_dist(wz, lg, cfg(wz, temp=1.0, top_k=4, top_p=0.75, min_p=0.0))
    assert ids == [0, 1]
    np.testing.assert_allclose(p, probs[:2] / 0.8, rtol=1e-5)
    # top_k bounds the candidate set before either cut
    ids, p = target_dist(wz, lg, cfg(wz, temp=1.0, top_k=2, top_p=1.0, min_p=0.0))
    assert ids == [0, 1]
    # top_k <= 0 means 64 candidates
    ids, _ = target_dist(wz, np.arange(200, dtype=np.float32), cfg(wz, temp=1.0, top_k=0, top_p=1.0, min_p=0.0))
    assert len(ids) == 64 and ids[0] == 199 and ids[-1] == 136


def test_repetition_penalty(wz):
    lg = np.array([3.0, 2.5, -1.0, -0.9], np.float32)
    c = cfg(wz, temp=0.0, rep_pen=2.0)
    assert verify_full(wz, lg, c, hist=[0])[0] == 1          # 3.0 / 2 = 1.5 < 2.5
    assert verify_full(wz, lg, c, hist=[7, 0, 0])[0] == 1      # ids outside the vocab are ignored
    lg2 = np.array([-1.0, -1.5, -5.0], np.float32)
    assert verify_full(wz, lg2, c, hist=[0])[0] == 1         # -1.0 * 2 = -2.0 < -1.5
    # only the last 512 history ids count
    hist = [0] + [9] * 512
    lg3 = np.zeros(10, np.float32)
    lg3[0], lg3[1] = 3.0, 2.5
    assert verify_full(wz, lg3, c, hist=hist)[0] == 0
    assert verify_full(wz, lg3, c, hist=hist[1:] + [0])[0] == 1
    # the top-16 path applies the same penalty and re-ranks
    v = np.array([3.0, 2.5] + [-10.0] * 14, np.float32)
    i = np.arange(16, dtype=np.int32)
    assert verify_top16(wz, v, i, cfg(wz, temp=0.0, rep_pen=2.0, top_k=16), hist=[0])[0] == 1


def _top16_of(lg):
    order = np.lexsort((np.arange(len(lg)), -lg.astype(np.float64)))[:16]
    return lg[order].astype(np.float32), order.astype(np.int32)


def test_top16_path_matches_full_vocabulary_path(wz):
    """With top_k <= 16 and no penalty, both selection paths must draw the same token for every u."""
    rng = np.random.default_rng(11)
    for trial in range(40):
        lg = (rng.normal(size=3000) * 2).astype(np.float32)
        if trial % 4 == 0:
            lg[rng.integers(0, 3000, 40)] = lg.max()       # heavy ties at the top
        tk = int(rng.integers(1, 17))
        c = cfg(wz, temp=float(rng.uniform(0.3, 1.5)), top_k=tk, top_p=float(rng.uniform(0.5, 1.0)),
                min_p=float(rng.uniform(0.0, 0.1)))
        v, i = _top16_of(lg)
        for u in rng.uniform(0, 1, 25):
            assert verify_full(wz, lg, c, u=u)[0] == verify_top16(wz, v, i, c, u=u)[0]


def test_sampling_frequencies_follow_the_distribution(wz):
    lg = np.log(np.array([0.4, 0.3, 0.2, 0.1], np.float64)).astype(np.float32)
    c = cfg(wz, temp=1.0, top_k=4, top_p=1.0, min_p=0.0)
    us = (np.arange(20000) + 0.5) / 20000
    counts = np.bincount([verify_full(wz, lg, c, u=u)[0] for u in us], minlength=4) / len(us)
    np.testing.assert_allclose(counts, [0.4, 0.3, 0.2, 0.1], atol=2e-3)


def test_draft_acceptance_is_rank1_exact(wz):
    lg = np.array([1.0, 0.0, -1.0], np.float32)
    c = cfg(wz, temp=1.0, top_k=3, top_p=1.0, min_p=0.0)
    tok, acc = verify_full(wz, lg, c, draft=0, u=0.1)
    assert (tok, acc) == (0, 1)
    tok, acc = verify_full(wz, lg, c, draft=1, u=0.1)
    assert (tok, acc) == (0, 0)


# ---- line formats --------------------------------------------------------------------------------

def _fields(d):
    f = wzy_amd.LineFields()
    f.req = -1
    f.finish = b"stop"
    for k, v in d.items():
        setattr(f, k, v.encode() if isinstance(v, str) else v)
    return f


def test_line_formats_match_golden(wz):
    with open(os.path.join(GOLDEN, "protocol_lines.json")) as fh:
        cases = json.load(fh)["cases"]
    what = {"PREFILL": wzy_amd.FMT_PREFILL, "DONE": wzy_amd.FMT_DONE, "DONE_EMPTY": wzy_amd.FMT_DONE_EMPTY}
    buf = C.create_string_buffer(1024)
    for case in cases:
        n = wz.wzy_engine_format(what[case["what"]], C.byref(_fields(case["fields"])), buf, 1024)
        assert n == len(case["line"])
        assert buf.value.decode() == case["line"]
        # the reference client's reading of the line (serve/engine_client.py:71-85,195-210)
        line = buf.value.decode().strip()
        body = json.loads(line[line.index(" ") + 1:])
        if case["fields"].get("req", -1) >= 0:
            assert body["req"] == case["fields"]["req"]
        assert body["finish" if case["what"] != "PREFILL" else "prompt_tokens"] is not None
    assert wz.wzy_engine_format(wzy_amd.FMT_DONE, C.byref(_fields({})), buf, 10) < 0


# ---- the engine binary ---------------------------------------------------------------------------

def test_engine_binary_fails_loudly_without_gpu(wz):
    if not os.path.exists(ENGINE):
        pytest.fail("wzy_engine not built; run __graft_entry__.build()")
    if wzy_amd.device_count() > 0:
        pytest.skip("a GPU is visible: covered by the GPU engine tests")
    p = subprocess.run([ENGINE], input="PING\nQUIT\n", capture_output=True, text=True, timeout=60)
    assert p.returncode == 1
    assert "READY" not in p.stdout and "PONG" not in p.stdout
    assert "[wzy-engine]" in p.stderr


def test_engine_binary_rejects_bad_options():
    if not os.path.exists(ENGINE):
        pytest.fail("wzy_engine not built; run __graft_entry__.build()")
    for args in (["--cfg", "no_such_field=3"], ["--frobnicate"]):
        p = subprocess.run([ENGINE] + args, input="", capture_output=True, text=True, timeout=60)
        assert p.returncode == 2 and p.stdout == ""


def _gate(wz, toks, probs, next_tok=-5, last_cell=100, ctx_max=10000, max_drafts=7, spec_min_p=0.72, stops=(),
          depth=5, min_p=0.30, gate=1.0):
    c = cfg(wz, spec_min_p=spec_min_p)
    c.n_stops = len(stops)
    for i, s in enumerate(stops):
        c.stops[i] = s
    t = np.array(toks, np.int32)
    p = np.array(probs, np.float32)
    g = wzy_amd.SpecGates(depth, min_p, gate)
    return wz.wzy_engine_mtp_gate(t.ctypes.data, p.ctypes.data, len(t), next_tok, last_cell, ctx_max, C.byref(c),
                                  max_drafts, C.byref(g))


def test_mtp_gates_follow_mtp_propose(wz):
    """mtp_propose's gates (src/wzy_engine_v2.cu:1428-1475) on hand-built chains."""
    hi = [0.9] * 7
    assert _gate(wz, [1, 2, 3, 4, 5, 6, 7], hi) == 5                   # chain cap WZY_SPEC_DEPTH = 5
    assert _gate(wz, [1, 2, 3, 4, 5, 6, 7], hi, max_drafts=3) == 3
    assert _gate(wz, [1, 2, 3, 4, 5, 6, 7], hi, depth=7) == 7
    assert _gate(wz, [1, 2, 3], [0.29, 0.9, 0.9]) == 0                  # first draft below 0.30
    assert _gate(wz, [1, 2, 3], [0.29, 0.9, 0.9], min_p=0.2) == 1       # then the j=1 explore gate (0.34)
    assert _gate(wz, [1, 2, 3], [0.25, 0.9, 0.9], spec_min_p=0.2) == 2  # a low spec_min_p lowers the gates;
                                                                        # the cumulative one (0.24) stops j=2
    assert _gate(wz, [7, 2, 3], [0.84, 0.9, 0.9], next_tok=7) == 0      # repeats the confirmed token, p < 0.85
    assert _gate(wz, [7, 2, 3], [0.86, 0.9, 0.9], next_tok=7) == 3
    assert _gate(wz, [1, 1, 3], hi) == 1                                # a draft equal to the previous one
    assert _gate(wz, [1, 2, 1, 4], hi) == 2                             # a draft equal to the one two back
    assert _gate(wz, [1, 2, 9, 4], hi, stops=(9,)) == 2                 # a stop id ends the chain
    assert _gate(wz, [9, 2], hi, stops=(9,)) == 0
    # explore gate of step j on the previous draft's probability: j=1 0.34, j=2 0.46, j=3 0.65, j=4 0.78
    assert _gate(wz, [1, 2, 3, 4, 5], [0.9, 0.9, 0.9, 0.64, 0.9]) == 4
    assert _gate(wz, [1, 2, 3, 4, 5], [0.9, 0.45, 0.9, 0.9, 0.9]) == 2
    # keep gate of step j on its own probability: j=1 0.36, j=2 0.48, j=3 0.62, j=4 0.74
    assert _gate(wz, [1, 2, 3, 4, 5], [0.9, 0.35, 0.9, 0.9, 0.9]) == 1
    assert _gate(wz, [1, 2, 3, 4, 5], [0.9, 0.9, 0.9, 0.9, 0.73]) == 4
    # cumulative gate: j=2 0.24, j=3 0.36, j=4 0.48
    assert _gate(wz, [1, 2, 3, 4, 5], [0.5, 0.47, 0.9, 0.9, 0.9]) == 2  # cum 0.235 < 0.24 at j=2
    # WZY_SPEC_GATE scales the deeper gates
    assert _gate(wz, [1, 2, 3, 4, 5], [0.9, 0.9, 0.9, 0.64, 0.9], gate=0.5) == 5
    # the context end stops the chain (last_cell + j >= ctx_max - 4)
    assert _gate(wz, [1, 2, 3, 4, 5], hi, last_cell=100, ctx_max=106) == 2

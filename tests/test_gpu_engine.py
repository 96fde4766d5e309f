"""The decode engine process end to end on the GPU: the stream protocol as the reference supervisor and
client speak it (serve/server.py:360-380,480-510; serve/engine_client.py), with the emitted token
streams checked two ways:
  - bit-exact against an in-process stage of the same library replaying the engine's schedule
    (prefill windows of up to 8 rows, then one row per step): the engine's loop adds no drift;
  - against the CPU oracle on the engine's tokens: every single-row step component by component from
    the stage's own inputs and pre-row state (teacher_forced.TeacherForced, within the float
    tolerance), and every window free-running through both sides' per-layer traces
    (layer_parity.LayerParity: expert ids and selected cells bit-exact, near ties excluded only
    within twice the measured error).
"""
import json
import os
import queue
import signal
import subprocess
import threading
import time

import numpy as np
import pytest

import wzy_amd
from layer_parity import LayerParity, gpu_trace
from stage_oracle import OracleModel, small_cfg
from teacher_forced import TeacherForced

pytestmark = pytest.mark.gpu

ENGINE = os.path.join(wzy_amd.PKG_DIR, "wzy_engine")
SEED = 21
CFG_FIELDS = [f for f, _ in wzy_amd.StageCfg._fields_]


def cfg_spec(c):
    return ",".join("%s=%s" % (f, getattr(c, f)) for f in CFG_FIELDS)


class EngineProc:
    """The engine as a child process; one reader thread queues its stdout lines."""

    def __init__(self, cfg, *args, env=None, model_dir=None):
        if not os.path.exists(ENGINE):
            pytest.fail("wzy_engine not built; run __graft_entry__.build()")
        e = dict(os.environ)
        e.update(env or {})
        model = ["--model-dir", str(model_dir)] if model_dir else ["--cfg", cfg_spec(cfg), "--model-seed", str(SEED)]
        self.p = subprocess.Popen([ENGINE] + model + list(args),
                                  stdin=subprocess.PIPE, stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                                  text=True, bufsize=1, env=e)
        self.q = queue.Queue()
        self.err = []
        threading.Thread(target=self._pump, args=(self.p.stdout, self.q), daemon=True).start()
        threading.Thread(target=self._pump, args=(self.p.stderr, None), daemon=True).start()
        ready = self.line(timeout=180)
        assert ready.startswith("READY "), ready
        self.ready = json.loads(ready[6:])

    def _pump(self, stream, q):
        for raw in stream:
            if q is None:
                self.err.append(raw.rstrip("\n"))
            else:
                q.put(raw.rstrip("\n"))
        if q is not None:
            q.put(None)

    def send(self, line):
        self.p.stdin.write(line + "\n")
        self.p.stdin.flush()

    def line(self, timeout=120):
        try:
            ln = self.q.get(timeout=timeout)
        except queue.Empty:
            raise AssertionError("engine silent for %ds; stderr tail: %s" % (timeout, self.err[-10:]))
        if ln is None:
            raise AssertionError("engine exited (rc=%s); stderr tail: %s" % (self.p.poll(), self.err[-10:]))
        return ln

    def request(self, obj):
        """Send one JSON request; return (PREFILL dict, [tokens], DONE dict) of the single-stream form."""
        self.send(json.dumps(obj, separators=(",", ":")))
        pf, toks = None, []
        while True:
            ln = self.line()
            if ln.startswith("PREFILL "):
                pf = json.loads(ln[8:])
            elif ln.startswith("TOK "):
                toks.append(int(ln.split()[-1]))
            elif ln.startswith("DONE "):
                return pf, toks, json.loads(ln[5:])

    def close(self):
        if self.p.poll() is None:
            try:
                self.send("QUIT")
                self.p.wait(timeout=60)
            except Exception:
                self.p.kill()
                self.p.wait(timeout=30)
        return self.p.returncode


def greedy_req(ids, n, **kw):
    r = {"ids": [int(i) for i in ids], "max_tokens": n, "temperature": 0.0, "top_p": 0.0, "top_k": 0,
         "min_p": 0.0, "repetition_penalty": 1.0, "spec": 7, "spec_min_p": 0.72, "stop": []}
    r.update(kw)
    return r


class Replay:
    """An in-process stage + the oracle, driven with the engine's schedule for one request; every
    window is traced on both sides and compared layer by layer (layer_parity.LayerParity)."""

    def __init__(self, wz, cfg):
        self.cfg = cfg
        self.st = wzy_amd.Stage(cfg)
        self.st.load_synthetic(SEED, 0)
        self.st.lib.wzy_stage_set_trace(self.st.h, 1)
        self.orc = OracleModel(wz, self.st, cfg, SEED)
        self.tf = TeacherForced(wz, self.st, cfg, self.orc)
        self.par = LayerParity(cfg, self.orc.qsa_layers, hidden="report")

    def prefill(self, ids, start):
        for p in range(start, len(ids) - 1, 8):
            w = list(ids[p:min(p + 8, len(ids) - 1)])
            self.st.forward(p, w, run_head=False)
            self.st.sync()
            gt = gpu_trace(self.st, self.cfg, len(w), len(self.orc.qsa_layers))
            _, _, _, ot = self.orc.forward_trace(p, w)
            self.par.window("prefill pos %d" % p, p, gt, ot, None, None, None, T=len(w))
        self.tf.sync_from_stage()

    def step(self, tok, pos):
        """Forward one row with the head: returns the stage's greedy token; checks it teacher-forced
        (every component on the stage's own inputs) and free-running (decisions) against the oracle."""
        self.st.forward(pos, [tok])
        self.st.sync()
        g, gid = self.st.logits(1), self.st.greedy(1)
        gt = gpu_trace(self.st, self.cfg, 1, len(self.orc.qsa_layers))
        self.tf.check_row("engine pos %d" % pos, pos, tok, gt, g, gid, self.st.pre_head(1))
        o, _, _, ot = self.orc.forward_trace(pos, [tok])
        self.par.window("engine pos %d" % pos, pos, gt, ot, g, o, gid)
        return int(gid[0])

    def close(self):
        self.st.close()


def test_engine_commands_and_legacy_lines(wz, gpu):
    print("case engine_commands", flush=True)
    cfg = small_cfg(wzy_amd, ctx_max=512, n_layers=2, topk=64)
    eng = EngineProc(cfg)
    try:
        r = eng.ready
        assert r["ctx_max"] == 512 and r["gpus"] == 1 and r["mtp"] is False and "sessions" not in r
        for cmd, want in (("PING", "PONG"), ("RESET", "OK"), ("SAVE_PROFILE", "OK"), ("PING", "PONG")):
            eng.send(cmd)
            assert eng.line() == want
        eng.send('{"ids":[],"max_tokens":5}')
        assert eng.line() == 'DONE {"generated":0,"finish":"stop"}'
        eng.send("")                                   # empty lines are ignored
        eng.send("7 8 9 12")                           # legacy: 3 prompt ids, 12 total -> 9 new, greedy
        ln = eng.line()
        assert ln.startswith("output :"), ln
        toks = [int(t) for t in ln[len("output :"):].split()]
        assert len(toks) == 9 and all(0 <= t < cfg.n_vocab for t in toks)
        assert eng.line() == "END"
        eng.send("7 8")                                # one prompt id, total 8 -> 7 new tokens
        ln = eng.line()
        assert ln.startswith("output :") and len(ln[len("output :"):].split()) == 7
        assert eng.line() == "END"
    finally:
        assert eng.close() == 0


def test_engine_greedy_stream_parity_and_prefix_reuse(wz, gpu):
    print("case engine_greedy", flush=True)
    cfg = small_cfg(wzy_amd, ctx_max=1024, n_layers=4, topk=64)
    prompt = [int(t) for t in np.random.default_rng(4).integers(0, cfg.n_vocab, 13)]
    eng = EngineProc(cfg)
    rep = Replay(wz, cfg)
    try:
        pf, toks, done = eng.request(greedy_req(prompt, 10))
        assert pf["prompt_tokens"] == 13 and pf["reused"] == 0 and pf["read"] == 13
        assert done["generated"] == 10 == len(toks) and done["finish"] == "length"
        assert done["prompt_tokens"] == 13 and done["active_tokens"] == 13 + 9
        assert done["draft_n"] == 0 and done["vram_hit"] == 1.0 and done["decode_ms"] > 0
        # replay: prompt windows, then one row per emitted token
        rep.prefill(prompt, 0)
        expect = [rep.step(prompt[-1], len(prompt) - 1)]
        for i, t in enumerate(toks[:-1]):
            expect.append(rep.step(t, len(prompt) + i))
        assert toks == expect, "engine %s vs in-process stage %s" % (toks, expect)

        # the follow-up prompt extends the resident state: only its new ids are read
        follow = prompt + toks[:-1] + [3, 141]
        pf2, toks2, done2 = eng.request(greedy_req(follow, 4))
        assert pf2["reused"] == 22 and pf2["read"] == len(follow) - 22, pf2
        rep.prefill(follow, 22)
        expect2 = [rep.step(follow[-1], len(follow) - 1)]
        for i, t in enumerate(toks2[:-1]):
            expect2.append(rep.step(t, len(follow) + i))
        assert toks2 == expect2
        assert done2["reused"] == 22 and done2["generated"] == 4

        # no_reuse restarts from an empty state and reproduces the first stream exactly
        _, toks3, done3 = eng.request(greedy_req(prompt, 10, no_reuse=1))
        assert toks3 == toks and done3["reused"] == 0
        print("engine greedy vs oracle, free-running: " + rep.par.summary(), flush=True)
        print("engine greedy vs oracle: " + rep.tf.summary(), flush=True)
        assert rep.tf.counts["rows"] == 14 and rep.tf.counts["layers"] == 14 * 4, rep.tf.summary()
        rep.tf.assert_bounds()
    finally:
        rep.close()
        assert eng.close() == 0


def test_engine_stop_ids_and_sampling(wz, gpu):
    print("case engine_stop_sampling", flush=True)
    cfg = small_cfg(wzy_amd, ctx_max=1024, n_layers=2, topk=64)
    prompt = [11, 12, 13, 14, 15]
    eng = EngineProc(cfg, "--seed", "1234")
    try:
        _, toks, _ = eng.request(greedy_req(prompt, 6, no_reuse=1))
        stop = toks[2]
        first = toks.index(stop)
        _, toks_s, done_s = eng.request(greedy_req(prompt, 6, no_reuse=1, stop=[stop]))
        assert toks_s == toks[:first] and done_s["finish"] == "stop" and done_s["generated"] == first
        # sampled requests: top-16 path (top_k <= 16) and full-vocabulary path (top_k 40 / penalty)
        for kw in ({"temperature": 0.8, "top_k": 8, "top_p": 0.95, "min_p": 0.0},
                   {"temperature": 0.8, "top_k": 40, "top_p": 0.95, "min_p": 0.0},
                   {"temperature": 0.7, "top_k": 8, "repetition_penalty": 1.3}):
            _, ts, dn = eng.request(greedy_req(prompt, 12, no_reuse=1, **kw))
            assert len(ts) == 12 and dn["finish"] == "length" and all(0 <= t < cfg.n_vocab for t in ts)
    finally:
        assert eng.close() == 0
    # the same sampling seed reproduces the same sampled stream in a fresh process
    streams = []
    for _ in range(2):
        eng = EngineProc(cfg, "--seed", "99")
        try:
            streams.append(eng.request(greedy_req(prompt, 8, temperature=0.9, top_k=12, top_p=1.0))[1])
        finally:
            assert eng.close() == 0
    assert streams[0] == streams[1]


def test_engine_multiplexed_protocol(wz, gpu):
    """--batch: requests carry "req", lines are TOK <req> <id> / PREFILL / DONE with "req" routed as the
    reference client routes them (serve/engine_client.py:71-85); CANCEL and PING are served while a
    request decodes."""
    print("case engine_multiplexed", flush=True)
    cfg = small_cfg(wzy_amd, ctx_max=1024, n_layers=2, topk=64)
    eng = EngineProc(cfg, "--batch")
    try:
        assert eng.ready["sessions"] == 1

        def rid_of(line):
            if line.startswith("TOK "):
                return int(line.split()[1])
            if line.startswith(("PREFILL ", "DONE ")):
                return int(json.loads(line[line.index(" ") + 1:]).get("req", 0))
            return -1

        eng.send(json.dumps(dict(greedy_req([1, 2, 3], 5), req=1), separators=(",", ":")))
        eng.send(json.dumps(dict(greedy_req([4, 5, 6, 7], 3), req=2), separators=(",", ":")))
        eng.send(json.dumps(dict(greedy_req([8, 9], 400), req=3), separators=(",", ":")))
        eng.send(json.dumps(dict(greedy_req([8, 9], 400), req=4), separators=(",", ":")))
        eng.send("PING")
        seen = {1: [], 2: [], 3: [], 4: []}
        done = {}
        pongs = 0
        t0 = time.time()
        cancelled_3 = False
        while len(done) < 3 and time.time() - t0 < 120:
            ln = eng.line()
            if ln == "PONG":
                pongs += 1
                continue
            rid = rid_of(ln)
            assert rid in seen, ln
            seen[rid].append(ln)
            if ln.startswith("TOK ") and rid == 3 and not cancelled_3:
                eng.send("CANCEL 4")                   # still queued: dropped without any line
                eng.send("CANCEL 3")                   # decoding: ends with finish "cancelled"
                cancelled_3 = True
            if ln.startswith("DONE "):
                done[rid] = json.loads(ln[5:])
        assert pongs == 1
        assert done[1]["generated"] == 5 and done[1]["finish"] == "length" and "decode_tps" not in done[1]
        assert done[2]["generated"] == 3
        assert done[3]["finish"] == "cancelled" and done[3]["generated"] < 400
        for rid in (1, 2, 3):
            assert seen[rid][0].startswith("PREFILL ") and json.loads(seen[rid][0][8:])["req"] == rid
            toks = [ln for ln in seen[rid] if ln.startswith("TOK ")]
            assert len(toks) == done[rid]["generated"]
        eng.send("PING")
        assert eng.line(timeout=30) == "PONG"
        assert seen[4] == []
    finally:
        assert eng.close() == 0


def test_engine_sigusr1_cancels(wz, gpu):
    print("case engine_sigusr1", flush=True)
    cfg = small_cfg(wzy_amd, ctx_max=2048, n_layers=2, topk=64)
    eng = EngineProc(cfg)
    try:
        eng.send(json.dumps(greedy_req([1, 2, 3], 1500), separators=(",", ":")))
        assert eng.line().startswith("PREFILL ")
        assert eng.line().startswith("TOK ")
        eng.p.send_signal(signal.SIGUSR1)
        while True:
            ln = eng.line()
            if ln.startswith("DONE "):
                d = json.loads(ln[5:])
                break
        assert d["finish"] == "cancelled" and d["generated"] < 1500
        eng.send("PING")
        assert eng.line() == "PONG"
    finally:
        assert eng.close() == 0


def test_engine_mtp_speculative_decoding_is_lossless(wz, gpu):
    """With the MTP drafter (fixed depth 3, and the reference's confidence gates) the greedy stream is
    the plain engine's, token for token: drafts are verified in one T = W window with rank-1
    acceptance and a rejected suffix's state is discarded (commit_window_state).  The prompt's cells
    seed the drafter's ring during prefill (run_head 2 windows + fronts)."""
    print("case engine_mtp", flush=True)
    cfg = small_cfg(wzy_amd, ctx_max=1024, n_layers=4, topk=64)
    prompt = [int(t) for t in np.random.default_rng(6).integers(0, cfg.n_vocab, 29)]
    streams = {}
    for name, args in (("plain", []), ("fixed3", ["--spec-depth", "3"]), ("gated", ["--mtp"])):
        eng = EngineProc(cfg, *args, env={"WZY_MTP_DVOCAB": "800"})
        try:
            assert eng.ready["mtp"] == (name != "plain")
            pf, toks, done = eng.request(greedy_req(prompt, 24, no_reuse=1))
            streams[name] = (toks, done)
            # a follow-up prompt that extends the state reuses it, drafter ring included
            _, toks2, done2 = eng.request(greedy_req(prompt + toks[:-1] + [5], 9))
            streams[name + "_reuse"] = (toks2, done2)
        finally:
            assert eng.close() == 0
    base = streams["plain"][0]
    for name in ("fixed3", "gated"):
        toks, done = streams[name]
        assert toks == base, "%s stream %s vs plain %s" % (name, toks, base)
        assert streams[name + "_reuse"][0] == streams["plain_reuse"][0]
        assert done["generated"] == 24 and done["draft_accepted"] <= done["draft_n"]
    # fixed depth: every window but the last offers 3 drafts (none is a stop id here)
    d = streams["fixed3"][1]
    wins = d["generated"] - 1 - d["draft_accepted"]
    assert d["draft_n"] >= 3 * (wins - 1), d
    assert streams["plain"][1]["draft_n"] == 0
    print("mtp engine: fixed3 drafts %d accepted %d; gated drafts %d accepted %d" % (
        d["draft_n"], d["draft_accepted"], streams["gated"][1]["draft_n"], streams["gated"][1]["draft_accepted"]),
        flush=True)


def expected_forced(pattern, n_new, depth):
    """(windows, drafts offered, drafts accepted) of the engine loop with forced drafts: window i
    emits its current token, offers min(depth, tokens still to generate) drafts of which the first
    pattern[i % len] are the continuation's, accepts those (rank-1 acceptance stops at the first wrong
    one), and continues with the verified row's token."""
    gen, wins, offered, accepted = 0, 0, 0, 0
    while gen < n_new:
        gen += 1                                  # the current token
        if gen >= n_new:
            break
        k = min(depth, n_new - gen)
        a = min(pattern[wins % len(pattern)], k)
        offered += k
        accepted += a
        gen += a
        wins += 1
    return wins, offered, accepted


@pytest.mark.parametrize("pattern", [[3], [0, 1, 2, 3], [2, 0, 3, 1, 1]])
def test_engine_forced_drafts_exercise_the_accept_path(wz, gpu, tmp_path, pattern):
    """The accept branch of the decode loop (src/wzy_engine_v2.cu:2160-2190) with accepted drafts:
    each window's 3 drafts are replaced by the plain greedy continuation for its first pattern[i] tokens
    and wrong tokens after (--forced-drafts; the drafter still runs and catches up on the accepted
    cells).  Windows accept 0, 1, 2 and 3 drafts; the stream equals the plain greedy stream token for
    token, the accepted count is the pattern's, and a rejected suffix's state is discarded
    (commit_window_state at the accepted row), so later windows stay exact."""
    print("case engine_forced pattern=%s" % pattern, flush=True)
    cfg = small_cfg(wzy_amd, ctx_max=1024, n_layers=4, topk=64)
    prompt = [int(t) for t in np.random.default_rng(9).integers(0, cfg.n_vocab, 29)]
    n_new = 40
    eng = EngineProc(cfg, env={"WZY_MTP_DVOCAB": "800"})
    try:
        _, base, _ = eng.request(greedy_req(prompt, n_new, no_reuse=1))
    finally:
        assert eng.close() == 0
    f = tmp_path / "forced.txt"
    f.write_text(" ".join(map(str, pattern)) + "\n" + " ".join(map(str, base)) + "\n")
    eng = EngineProc(cfg, "--spec-depth", "3", "--forced-drafts", str(f), env={"WZY_MTP_DVOCAB": "800"})
    try:
        _, toks, done = eng.request(greedy_req(prompt, n_new, no_reuse=1))
    finally:
        assert eng.close() == 0
    wins, offered, accepted = expected_forced(pattern, n_new, 3)
    print("forced drafts %s: %d windows, %d drafts offered, %d accepted (engine: %d / %d)" % (
        pattern, wins, offered, accepted, done["draft_n"], done["draft_accepted"]), flush=True)
    assert toks == base, "forced %s stream %s vs plain %s" % (pattern, toks, base)
    assert done["generated"] == n_new
    assert done["draft_n"] == offered and done["draft_accepted"] == accepted, done


def test_engine_real_weight_files(wz, gpu, tmp_path):
    """--model-dir with the reference's files (qwen-nvfp4-gptq-dense.gguf with Q8_0 embedding and head,
    pack/experts.bin, mtp/ and its draft vocabulary): the stage shapes come from the checkpoint, the
    greedy stream equals an in-process stage loaded from the same files and driven with the engine's
    schedule, and MTP drafting from the loaded drafter leaves the stream unchanged."""
    print("case engine_real_weights", flush=True)
    import gguf_file as gf
    ref = small_cfg(wzy_amd, ctx_max=512, n_layers=4, topk=64)
    ck = gf.Checkpoint(wz, ref, 23, str(tmp_path), emb_q8=True, head_q8=True, with_mtp=True, n_dv=400)
    prompt = [int(t) for t in np.random.default_rng(8).integers(0, ref.n_vocab, 11)]
    streams = {}
    for name, args in (("plain", []), ("mtp", ["--spec-depth", "2"])):
        eng = EngineProc(None, "--ctx", "512", *args, model_dir=tmp_path)
        try:
            assert eng.ready["mtp"] == (name == "mtp") and eng.ready["split"] == 4
            _, toks, done = eng.request(greedy_req(prompt, 12))
            streams[name] = toks
            assert done["generated"] == 12
        finally:
            assert eng.close() == 0
    assert streams["mtp"] == streams["plain"]
    # the in-process stage from the same files, the engine's schedule
    import ctypes as C
    cfg = wzy_amd.StageCfg()
    wz.wzy_stage_cfg_from_gguf(str(ck.gguf).encode(), 512, C.byref(cfg))
    st = wzy_amd.Stage(cfg)
    try:
        st.load_gguf(ck.gguf, ck.experts)
        for p in range(0, len(prompt) - 1, 8):
            st.forward(p, prompt[p:min(p + 8, len(prompt) - 1)], run_head=False)
        expect, tok = [], prompt[-1]
        for i in range(12):
            st.forward(len(prompt) - 1 + i, [tok])
            st.sync()
            tok = int(st.greedy(1)[0])
            expect.append(tok)
        assert streams["plain"] == expect, (streams["plain"], expect)
    finally:
        st.close()

"""Parked sessions on the GPU: the stage's session slots (wzy_stage_session_save / _restore) and the
engine's two-slot prefix reuse (src/wzy_engine_v2.cu:1636-1842 save/restore_session_state,
:1962-1997 the policy; the policy itself is pinned on the CPU in test_engine_host.py).

- A save then restore leaves every state tensor bit-identical to what was saved, although another
  session ran in between, and the next forward's logits equal those of an uninterrupted stage.
- The engine parks, swaps and restores sessions as the reference does (restored_park /
  parked_tokens / reused in its PREFILL and DONE lines), and every stream equals a fresh
  no_reuse run of the same prompt.
"""
import numpy as np
import pytest

import wzy_amd
from stage_oracle import small_cfg
from test_gpu_engine import EngineProc, greedy_req

pytestmark = pytest.mark.gpu

SEED = 17


def state_tensors(st, cfg, n_cells, mtp):
    """Every tensor a session slot covers, as host arrays (cells 0 .. n_cells-1 of the KV stores, the
    pooled keys of blocks 0 .. n_cells/idx_blk + 1)."""
    out = {}
    kvd = cfg.qsa_kvh * cfg.qsa_hd
    blocks = n_cells // cfg.idx_blk + 2
    for l in range(cfg.n_layers):
        if l % cfg.qsa_period != cfg.qsa_period - 1:
            out[(l, "conv_hist")] = st.read(l, "conv_hist", np.float32)
            out[(l, "ssm")] = st.read(l, "ssm", np.float32)
        else:
            out[(l, "idx_tail")] = st.read(l, "idx_tail", np.float32)
            out[(l, "idx_dead")] = st.read(l, "idx_dead", np.float32)
            out[(l, "idx_pooled")] = st.read_range(l, "idx_pooled", np.uint16, 0, blocks * cfg.idx_dim)
            out[(l, "kv_k")] = st.read_range(l, "kv_k", np.int8, 0, n_cells * kvd)
            out[(l, "kv_ks")] = st.read_range(l, "kv_ks", np.uint16, 0, n_cells * kvd // 64)
            out[(l, "kv_v")] = st.read_range(l, "kv_v", np.int8, 0, n_cells * kvd)
            out[(l, "kv_vs")] = st.read_range(l, "kv_vs", np.uint16, 0, n_cells * kvd // 64)
    if mtp:
        for n, dt in (("mtp.kv_k", np.int8), ("mtp.kv_ks", np.uint16), ("mtp.kv_v", np.int8),
                      ("mtp.kv_vs", np.uint16), ("mtp.kv_floor", np.int32)):
            out[(-1, n)] = st.read(-1, n, dt)
    return out


def feed(st, toks, p0=0):
    for p in range(p0, len(toks), 8):
        st.forward(p, toks[p:min(p + 8, len(toks))], run_head=False)
    st.sync()


def test_stage_session_save_restore_roundtrip(wz, gpu):
    print("case stage_session_roundtrip", flush=True)
    cfg = small_cfg(wzy_amd, ctx_max=1024, n_layers=4, topk=64)
    rng = np.random.default_rng(5)
    a = [int(t) for t in rng.integers(0, cfg.n_vocab, 101)]
    b = [int(t) for t in rng.integers(0, cfg.n_vocab, 77)]
    kvd = cfg.qsa_kvh * cfg.qsa_hd
    st, ref = wzy_amd.Stage(cfg), wzy_amd.Stage(cfg)
    try:
        for s in (st, ref):
            s.load_synthetic(SEED, 0)
            assert s.lib.wzy_stage_mtp_init(s.h, SEED + 1, 200) == 0
        # session A: 100 cells, a drafter ring with content and a floor
        ring = rng.integers(-127, 128, 1024 * kvd).astype(np.int8)
        for s in (st, ref):
            feed(s, a[:100])
            s.lib.wzy_stage_write_tensor(s.h, -1, b"mtp.kv_k", ring.ctypes.data, ring.nbytes)
            assert s.lib.wzy_stage_mtp_set_floor(s.h, 37) == 0
            s.sync()
        assert wz.wzy_stage_session_cells(st.h, 0) == -1
        saved = state_tensors(st, cfg, 100, True)
        need = wz.wzy_stage_session_bytes(st.h, 100)
        assert need >= sum(v.nbytes for v in saved.values())
        held = wz.wzy_stage_device_bytes(st.h)
        wz.wzy_stage_session_save(st.h, 0, 100)
        assert wz.wzy_stage_session_cells(st.h, 0) == 100
        assert wz.wzy_stage_device_bytes(st.h) == held + need
        # session B overwrites the live state
        wz.wzy_stage_reset_state(st.h)
        assert st.lib.wzy_stage_mtp_reset(st.h) == 0
        feed(st, b)
        wz.wzy_stage_session_save(st.h, 1, len(b))
        changed = state_tensors(st, cfg, 100, True)
        assert any(not np.array_equal(saved[k], changed[k]) for k in saved)
        # back to A: bit-identical state, and the next forward equals the uninterrupted stage's
        wz.wzy_stage_session_restore(st.h, 0)
        back = state_tensors(st, cfg, 100, True)
        for k in saved:
            assert np.array_equal(saved[k], back[k]), k
        assert back[(-1, "mtp.kv_floor")][0] == 37
        for s in (st, ref):
            s.forward(100, [a[100]])
            s.sync()
        assert np.array_equal(st.logits(1), ref.logits(1))
        assert np.array_equal(st.greedy(1), ref.greedy(1))
        # the slot keeps its copy: a second restore (after more decoding) gives the same state again
        st.forward(101, [3])
        st.sync()
        wz.wzy_stage_session_restore(st.h, 0)
        again = state_tensors(st, cfg, 100, True)
        for k in saved:
            assert np.array_equal(saved[k], again[k]), k
        # B's slot restores B
        wz.wzy_stage_session_restore(st.h, 1)
        ref_b = wzy_amd.Stage(cfg)
        try:
            ref_b.load_synthetic(SEED, 0)
            feed(ref_b, b)
            for l, name in ((0, "ssm"), (1, "kv_k"), (1, "idx_pooled")):
                dt = {"ssm": np.float32, "kv_k": np.int8, "idx_pooled": np.uint16}[name]
                # pooled rows 0 .. n/idx_blk: the closed blocks and the placeholder row after them
                # (the next row is never written by this session and is not part of its state)
                n = {"ssm": None, "kv_k": len(b) * kvd, "idx_pooled": (len(b) // 4 + 1) * cfg.idx_dim}[name]
                x = st.read(l, name, dt) if n is None else st.read_range(l, name, dt, 0, n)
                y = ref_b.read(l, name, dt) if n is None else ref_b.read_range(l, name, dt, 0, n)
                assert np.array_equal(x, y), name
        finally:
            ref_b.close()
        # errors: bad slot, empty slot, too many cells
        wz.wzy_stage_session_clear(st.h, 1)
        assert wz.wzy_stage_session_cells(st.h, 1) == -1
        for bad in (lambda: wz.wzy_stage_session_restore(st.h, 1),
                    lambda: wz.wzy_stage_session_restore(st.h, 2),
                    lambda: wz.wzy_stage_session_save(st.h, -1, 10),
                    lambda: wz.wzy_stage_session_save(st.h, 0, cfg.ctx_max + 1)):
            with pytest.raises(wzy_amd.WzyError):
                bad()
    finally:
        st.close()
        ref.close()


@pytest.mark.parametrize("mtp", [False, True])
def test_engine_parks_swaps_and_restores_sessions(wz, gpu, mtp):
    """The reference's sequence of session moves, with the expected counts taken from the engine's
    own active_tokens (with the drafter an accepted last draft is fed too, so a session can hold one
    cell more than prompt + generated - 1)."""
    print("case engine_sessions mtp=%s" % mtp, flush=True)
    cfg = small_cfg(wzy_amd, ctx_max=1024, n_layers=4, topk=64)
    rng = np.random.default_rng(9)
    A = [int(t) for t in rng.integers(0, cfg.n_vocab, 80)]
    B = [int(t) for t in rng.integers(0, cfg.n_vocab, 70)]
    args = ["--spec-depth", "3"] if mtp else []
    eng = EngineProc(cfg, *args)
    fresh = EngineProc(cfg, *args)
    try:
        def run(ids, want_reused, want_restored, want_parked, n=6):
            pf, toks, done = eng.request(greedy_req(ids, n))
            _, ref, _ = fresh.request(greedy_req(ids, n, no_reuse=1))
            assert toks == ref, "stream after %s differs from a fresh run" % (pf,)
            got = (pf["reused"], pf["restored_park"], pf["parked_tokens"])
            assert got == (want_reused, want_restored, want_parked), (got, pf)
            assert (done["restored_park"], done["parked_tokens"]) == got[1:]
            return ids + toks[:done["active_tokens"] - len(ids)]     # the tokens of the resident cells

        sa = run(A, 0, 0, 0)
        assert len(sa) >= 85
        sb = run(B, 0, 0, len(sa))                       # A is parked, B runs from a reset
        sa2 = run(sa + [5, 6], len(sa), 1, len(sb))      # swap: A comes back, B is parked
        sb2 = run(sb + [9], len(sb), 1, len(sa2))        # and back again
        assert 2 * len(sb2) >= len(sa2)
        side = run(list(range(1, 11)), 0, 0, len(sb2))   # an unrelated prompt parks B
        assert len(side) < 64
        run([11, 12, 13], 0, 0, len(sb2))                # too short to park: B stays parked
        run(sb2 + [4], len(sb2), 1, len(sb2))            # restore; the parked copy stays parked
        eng.send("RESET")
        assert eng.line() == "OK"
        run(sb2 + [4], 0, 0, 0)                          # RESET dropped the parked session
    finally:
        assert eng.close() == 0
        assert fresh.close() == 0

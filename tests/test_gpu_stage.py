"""GPU parity of the whole decode window (wzy_stage_record_forward) against the CPU oracle model,
on small instances of the synthetic architecture (MI355X; C ABI only, no torch).

The oracle model is built from the stage's own tensors after load_synthetic, so both sides start
from the same weights and prefilled state and then evolve their state independently."""
import numpy as np
import pytest

import wzy_amd
from stage_oracle import OracleModel, near_tie, small_cfg

pytestmark = pytest.mark.gpu

RTOL, ATOL = 2e-2, 1e-2


def check_logits(tag, g, o):
    err = np.abs(g.astype(np.float64) - o)
    print("%s: logits max abs err %.3g (max |ref| %.3g)" % (tag, err.max(), np.abs(o).max()), flush=True)
    bad = err > ATOL + RTOL * np.abs(o)
    assert not bad.any(), "%s: %d logits outside tolerance (worst %.3g)" % (tag, bad.sum(), err.max())


def check_greedy(tag, g_ids, o_logits):
    for t, gid in enumerate(g_ids):
        row = o_logits[t]
        ref = int(np.argmax(row))
        if gid != ref:
            assert near_tie(row, 2 * ATOL) and row[gid] >= row[ref] - 2 * ATOL, \
                "%s row %d: greedy %d vs oracle %d (logits %.5f vs %.5f)" % (tag, t, gid, ref, row[gid], row[ref])


@pytest.mark.parametrize("n_ctx,topk,graphs", [(600, 64, True), (40, 64, True), (600, 64, False)])
def test_stage_decode_parity(wz, gpu, n_ctx, topk, graphs):
    print("case stage_decode n_ctx=%d topk=%d graphs=%s" % (n_ctx, topk, graphs), flush=True)
    cfg = small_cfg(wzy_amd, ctx_max=1024, n_layers=4, topk=topk)
    st = wzy_amd.Stage(cfg)
    try:
        st.lib.wzy_stage_set_graphs(st.h, int(graphs))
        seed = 1234
        st.load_synthetic(seed, n_ctx)
        orc = OracleModel(wz, st, cfg, seed)
        rng = np.random.default_rng(n_ctx)
        toks = rng.integers(0, cfg.n_vocab, 4)
        pos = n_ctx
        for step, tok in enumerate(toks):
            st.forward(pos, [tok], want_top16=True)
            st.sync()
            g_logits, g_ids = st.logits(1), st.greedy(1)
            g_pre = st.pre_head(1)
            o_logits, o_ids, o_pre = orc.forward(pos, [tok])
            tag = "step %d pos %d" % (step, pos)
            err = np.abs(g_pre - o_pre).max()
            print("%s: pre-head residual max abs err %.3g (max %.3g)" % (tag, err, np.abs(o_pre).max()))
            check_logits(tag, g_logits, o_logits)
            check_greedy(tag, g_ids, o_logits)
            tv, ti = st.top16(1)
            assert ti[0, 0] == g_ids[0]
            assert (np.diff(tv[0]) <= 0).all()
            assert np.array_equal(g_logits[0, ti[0]], tv[0])
            pos += 1
    finally:
        st.close()


def test_stage_graph_replay_matches_eager(wz, gpu):
    """Graph replays and direct launches run the same kernels: bit-identical logits over several steps."""
    print("case stage_graph_vs_eager", flush=True)
    cfg = small_cfg(wzy_amd, ctx_max=1024, n_layers=4, topk=64)
    outs = []
    for graphs in (1, 0):
        st = wzy_amd.Stage(cfg)
        try:
            st.lib.wzy_stage_set_graphs(st.h, graphs)
            st.load_synthetic(99, 500)
            seq = []
            for i, tok in enumerate([5, 17, 900]):
                st.forward(500 + i, [tok])
                st.sync()
                seq.append(st.logits(1))
            st.forward(503, [1, 2, 3])
            st.sync()
            seq.append(st.logits(3))
            outs.append(seq)
        finally:
            st.close()
    for a, b in zip(*outs):
        assert np.array_equal(a, b)


def test_stage_window_and_commit(wz, gpu):
    """A T=4 window with snapshots, commit after its second row, then a decode step: matches the oracle
    that decoded only the two accepted rows."""
    print("case stage_window_commit", flush=True)
    cfg = small_cfg(wzy_amd, ctx_max=1024, n_layers=4, topk=64)
    st = wzy_amd.Stage(cfg)
    try:
        seed = 77
        n_ctx = 601                      # window rows cross an indexer block boundary
        st.load_synthetic(seed, n_ctx)
        orc_full = OracleModel(wz, st, cfg, seed)
        orc_acc = OracleModel(wz, st, cfg, seed)
        win = np.array([11, 222, 333, 444], np.int32)
        st.forward(n_ctx, win, save_snaps=True, want_top16=True)
        st.sync()
        g4 = st.logits(4)
        o4, _, _ = orc_full.forward(n_ctx, win)
        check_logits("window", g4, o4)
        check_greedy("window", st.greedy(4), o4)
        # accept rows 0 and 1 (last accepted position n_ctx + 1)
        st.lib.wzy_stage_commit_window_state(st.h, 1, n_ctx + 1)
        orc_acc.forward(n_ctx, win[:2])
        nxt = np.array([555], np.int32)
        st.forward(n_ctx + 2, nxt)
        st.sync()
        g1 = st.logits(1)
        o1, _, _ = orc_acc.forward(n_ctx + 2, nxt)
        check_logits("after commit", g1, o1)
        check_greedy("after commit", st.greedy(1), o1)
    finally:
        st.close()


def test_stage_errors(wz, gpu):
    """Host-side argument checks return errors instead of launching."""
    cfg = small_cfg(wzy_amd, ctx_max=256, n_layers=2, topk=64)
    st = wzy_amd.Stage(cfg)
    try:
        with pytest.raises(wzy_amd.WzyError):
            st.forward(0, [1])                         # not loaded yet
        st.load_synthetic(1, 10)
        with pytest.raises(wzy_amd.WzyError):
            st.forward(250, list(range(8)))            # past ctx_max
        with pytest.raises(wzy_amd.WzyError):
            st.forward(10, list(range(9)))             # wider than the window limit
        with pytest.raises(wzy_amd.WzyError):
            st.read(0, "no_such_tensor", np.float32)
    finally:
        st.close()

"""The per-layer embedding (PLE) at layer 1 on the GPU against the CPU oracle (oracle/orc_ple.c).

The reference applies PLE whenever a stage holds layer 1 of its real model (src/wzy_engine_v2.cu:316,
src/wzy_stage_v2.cuh:583-597); the synthetic BASELINE model has none, so these tests switch it on
(wzy_stage_cfg.ple) in small configurations:
  * the table rows (hash, cut rule, token history, fp8 decode) bit-exact, window by window, with the
    table in HBM as the synthetic generator fills it (every row a pure function of the seed, so the
    oracle regenerates the rows it reads);
  * the block on random inputs, with per-row history snapshots;
  * a decode stream of a four-layer stage with PLE, layer by layer against the oracle model, and the
    same steps teacher-forced component by component (the PLE conv history included);
  * a verify window whose last rows are rejected: commit_window_state restores the PLE history of the
    accepted row, so the following steps match an oracle that ran the accepted rows only;
  * chunked prefills with PLE against the independent prefill composition (the chunk's rows read
    their context tokens from the history the decode windows wrote).
"""
import ctypes as C

import numpy as np
import pytest

import wzy_amd
from layer_parity import ATOL, RTOL, excess
from oracle_lib import ptr
from stage_oracle import OracleModel, small_cfg
from test_gpu_stage import check_close, check_greedy, run_layer_parity

pytestmark = pytest.mark.gpu

DA = wzy_amd.DeviceArray
EOS = 248044
ROW_FN = C.CFUNCTYPE(C.c_void_p, C.c_void_p, C.c_uint32)


class SynthRows:
    """The synthetic table's rows on the host (wzy_synth_ple_row), for the oracle's lookups."""

    def __init__(self, wz, seed, head):
        self.wz, self.seed, self.head, self.rows = wz, seed, head, {}
        self.cb = ROW_FN(self._row)

    def _row(self, ctx, r):
        b = self.rows.get(r)
        if b is None:
            b = np.empty(self.head, np.uint8)
            self.wz.wzy_synth_ple_row(self.seed, int(r), self.head, b.ctypes.data)
            self.rows[r] = b
        return b.ctypes.data


def ple_cfg(n_layers=4, ctx_max=1024):
    c = small_cfg(wzy_amd, ctx_max=ctx_max, n_layers=n_layers, topk=64)
    c.ple = 1
    return c


def test_ple_rows_bit_exact(wz, orc, gpu):
    print("case ple_rows", flush=True)
    D, seed, ctx = 256, 7, 64
    head = D // 16
    rows = int(wz.wzy_ple_table_rows())
    table = DA(rows * head, np.uint8)
    try:
        wz.wzy_synth_ple_table_device(seed, head, table.ptr, None)
        wz.wzy_device_sync()
        tab = SynthRows(wz, seed, head)
        # the device table equals the host generator at the first, last and scattered rows
        for r in [0, 1, 20000002, 20000003, 123456789, rows - 1]:
            got = np.empty(head, np.uint8)
            wz.wzy_memcpy_d2h(got.ctypes.data, table.ptr + r * head, head, None)
            wz.wzy_device_sync()
            want = np.frombuffer(C.string_at(tab.cb(None, r), head), np.uint8)
            assert np.array_equal(got, want), "table row %d" % r
        rng = np.random.default_rng(3)
        # windows from the start of the context (no history), with eos tokens inside, one-row steps
        windows = [(0, [5, 6, 7, 8]), (4, [EOS, 9]), (6, [10]), (7, [11, EOS, EOS, 12, 13, 14, 15, 16]),
                   (15, [int(x) for x in rng.integers(0, 151936, 8)]), (23, [17])]
        h_dev = DA.from_numpy(np.full(ctx, -9, np.int32))
        h_orc = np.full(ctx, -9, np.int32)
        for pos, toks in windows:
            T = len(toks)
            d_pos, d_toks = DA.from_numpy(np.array([pos], np.int32)), DA.from_numpy(np.array(toks, np.int32))
            emb, embh = DA((T, D), np.float32), DA((T, D), np.uint16)
            wz.wzy_ple_rows(table.ptr, head, 0.125, EOS, d_pos.ptr, d_toks.ptr, T, h_dev.ptr, ctx, emb.ptr, embh.ptr,
                            None)
            wz.wzy_device_sync()
            want = np.empty((T, D), np.float32)
            tk = np.array(toks, np.int32)
            orc.orc_ple_rows(C.cast(tab.cb, C.c_void_p), None, head, 0.125, EOS, tk.ctypes.data, T, pos,
                             h_orc.ctypes.data, want.ctypes.data)
            got = emb.numpy()
            assert np.array_equal(got, want), "window at %d: rows differ" % pos
            wb = (want.view(np.uint32).astype(np.uint64) + 0x7FFF + ((want.view(np.uint32) >> 16) & 1)) >> 16
            assert np.array_equal(embh.numpy(), wb.astype(np.uint16)), "window at %d: bf16 rows" % pos
            assert np.array_equal(h_dev.numpy(), h_orc), "window at %d: token history" % pos
        print("ple rows: %d windows bit-exact, %d table rows read" % (len(windows), len(tab.rows)), flush=True)
    finally:
        table.free()


def test_ple_block_parity(wz, orc, gpu):
    print("case ple_block", flush=True)
    from test_oracle_ple import make_block, run_block
    for D, T, use_bo in ((256, 1, True), (256, 8, True), (2048, 4, False), (2560, 2, True)):
        b = make_block(D=D, HC=4, T=T, seed=D + T)
        R_o, hist_o, sn_o = run_block(orc, b, use_bo=use_bo, snaps=True)
        d = {k: DA.from_numpy(np.ascontiguousarray(b[k])) for k in ("R", "bo", "inj", "emb", "wk", "wv", "nq", "nk", "nc",
                                                                     "cw", "hist")}
        sn = DA((T, 4 * D, 9), np.float32, zero=True)
        nws = wz.wzy_ple_workspace_bytes(D, 4, T)
        ws = DA(nws, np.uint8, zero=True)
        wz.wzy_ple_block(d["R"].ptr, d["bo"].ptr if use_bo else None, d["inj"].ptr, d["emb"].ptr, d["wk"].ptr,
                         d["wv"].ptr, d["nq"].ptr, d["nk"].ptr, d["nc"].ptr, d["cw"].ptr, d["hist"].ptr, D, 4, 1e-6, T,
                         sn.ptr, ws.ptr, nws, None)
        wz.wzy_device_sync()
        for name, g, o in (("R", d["R"].numpy(), R_o), ("history", d["hist"].numpy(), hist_o),
                           ("snapshots", sn.numpy(), sn_o)):
            e = np.abs(g.astype(np.float64) - o)
            print("ple block D=%d T=%d %s: max abs err %.3g (max %.3g)" % (D, T, name, e.max(), np.abs(o).max()),
                  flush=True)
            assert excess(g, o) <= 0 and e.max() <= 1e-3 * max(1.0, np.abs(o).max()), (D, T, name)
        for a in list(d.values()) + [sn, ws]:
            a.free()


def test_stage_ple_decode_layer_parity(wz, gpu):
    """Four layers (GDN, QSA, GDN, QSA) with PLE before layer 1: single-token steps and a T=4 window,
    every layer's hidden states and decisions against the oracle model (free-running, elementwise) and
    the single-token steps component by component (teacher-forced)."""
    print("case ple_decode", flush=True)
    cfg = ple_cfg()
    rng = np.random.default_rng(12)
    windows = [[int(t)] for t in rng.integers(0, cfg.n_vocab, 4)] + [[int(t) for t in rng.integers(0, cfg.n_vocab, 4)]]
    par, _ = run_layer_parity(wz, cfg, 31, 300, windows)
    print("ple decode: " + par.summary(), flush=True)
    assert par.rows_full == 8 and par.layers_compared == 32, par.summary()
    par2, tf = run_layer_parity(wz, cfg, 32, 301, windows[:4], teacher=True)
    print("ple decode teacher-forced: " + tf.summary(), flush=True)
    assert tf.counts["rows"] == 4 and tf.counts["layers"] == 16
    assert "PLE conv history" in tf.worst
    tf.assert_bounds()


def test_stage_ple_window_commit(wz, gpu):
    """A T=4 verify window with snapshots, rows 0 and 1 accepted (commit_window_state): the PLE history
    goes back to the accepted row's snapshot, and the next steps (which overwrite the rejected rows'
    tokens in the history) match an oracle model that ran the accepted rows only."""
    print("case ple_commit", flush=True)
    cfg = ple_cfg(n_layers=2)
    n_ctx = 200
    st = wzy_amd.Stage(cfg)
    try:
        st.load_synthetic(41, n_ctx)
        orc_acc = OracleModel(wz, st, cfg, 41)
        win = np.array([11, 222, 333, 444], np.int32)
        st.forward(n_ctx, win, save_snaps=True)
        st.sync()
        st.lib.wzy_stage_commit_window_state(st.h, 1, n_ctx + 1)
        orc_acc.forward(n_ctx, win[:2])
        h_o = orc_acc.arrays[(1, "ple_hist")]
        g_h = st.read(1, "ple_hist", np.float32)
        assert excess(g_h, h_o) <= 0, "PLE history after the commit"
        for step, tok in enumerate([555, 7, 8]):
            pos = n_ctx + 2 + step
            st.forward(pos, [tok])
            st.sync()
            o1, _, _ = orc_acc.forward(pos, [tok])
            g1 = st.logits(1)
            check_close("after commit, pos %d" % pos, g1, o1)
            check_greedy("after commit", st.greedy(1), g1, o1)
        assert np.array_equal(st.read_range(-1, "tok_hist", np.int32, n_ctx, 5), [11, 222, 555, 7, 8])
    finally:
        st.close()


@pytest.mark.parametrize("p0,B,prefix", [(0, 120, 0), (37, 100, 37)])
def test_stage_ple_prefill_matches_oracle(wz, orc, gpu, p0, B, prefix):
    """Chunked prefills of a stage with PLE (an empty context, and one the decode windows built): the
    chunk's table rows read the earlier cells' tokens from the history, the block runs on the chunk's
    rows in order, and the whole chunk is checked as the other prefill tests check it (check_chunk,
    with PLE in the independent composition), the PLE history and token history included."""
    from test_gpu_prefill import check_chunk, pf_cfg
    print("case ple_prefill p0=%d B=%d" % (p0, B), flush=True)
    cfg = pf_cfg()
    cfg.ple = 1
    rng = np.random.default_rng(p0 * 3 + B)
    toks = [int(t) for t in rng.integers(0, cfg.n_vocab, p0 + B)]
    st = wzy_amd.Stage(cfg)
    try:
        st.load_synthetic(23, 0)
        for p in range(0, prefix, 8):
            st.forward(p, toks[p:min(p + 8, prefix)], run_head=False)
        st.sync()
        wz.wzy_stage_set_trace(st.h, 1)
        om = OracleModel(wz, st, cfg, 23)
        st.prefill(p0, toks[p0:p0 + B])
        st.sync()
        check_chunk(wz, orc, st, om, cfg, p0, toks[p0:p0 + B], "ple p0=%d B=%d" % (p0, B))
    finally:
        st.close()

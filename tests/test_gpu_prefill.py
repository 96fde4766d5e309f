"""Chunked prefill on the GPU (wzy_stage_prefill, wzy_gemm_bf16) against the CPU oracle's restatement
of the reference's prefill (orc_prefill.c; src/wzy_prefill_tc.cuh:546-1058).

- The bf16 MFMA GEMM against orc_pf_gemm at the projection shapes of a chunk, including row / column
  tails, Q8_0 and bf16 weights, fp32 and bf16 outputs.
- Whole chunks at a small configuration: from an empty context, from a context the decode path
  built (a chunk that starts inside an index block), and a chunk shorter than one index block.
  The discrete decisions are checked where they are made (every MoE block on the GPU's own input,
  every QSA row's selected cells bit-exact), and the rest of the chunk teacher-forced on them:
  the independent composition of the prefill (prefill_compose, pinned against the oracle on the
  CPU) takes the GPU's expert outputs and selections, and every layer's HC reads and blocks, the
  final residual rows, the GDN state, the KV cells and the indexer state must agree elementwise.
  (Without the forcing, the bf16 rounding of expert activations makes a 1e-4 input difference move
  a synthetic MoE block's output by far more than the tolerance, and that compounds over layers.)
- The decode row after a prefill, teacher-forced (teacher_forced.py) from the stage's prefilled state.
- Chunking is exact: one chunk and the same cells in several chunks leave bit-identical state and
  final rows (small configuration and BASELINE shapes, 2,100 rows: the GEMM tiling, the 2,048-row
  score passes and the indexer's cross-chunk blocks at their real sizes).
- BASELINE shapes (D=2048, 512 experts top-10, 16/16 GDN heads, 24/2 QSA heads, top-2048) on four
  layers of a 4,000-cell context against the oracle.
"""
import ctypes as C

import numpy as np
import pytest

import oracle_lib
import wzy_amd
from layer_parity import ATOL, RTOL
from oracle_lib import ptr
from prefill_compose import compose_prefill, dims_of, embed, moe_oracle, stage_weights, state_copy, tbf16
from layer_parity import gpu_trace
from stage_oracle import OracleModel, attend, is_qsa, key_flip_ok, small_cfg
from teacher_forced import TeacherForced
from test_gpu_moe import assert_prefill_close

pytestmark = pytest.mark.gpu

SEED = 23
DA = wzy_amd.DeviceArray


def pf_cfg(ctx_max=1024, n_layers=4, topk=64):
    """The small configuration with an expert count the MFMA MoE block takes (a multiple of 64)."""
    c = small_cfg(wzy_amd, ctx_max=ctx_max, n_layers=n_layers, topk=topk)
    c.n_exp, c.top_k = 64, 4
    return c


def bf16_bits(x):
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bits_to_f32(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---- GEMM ------------------------------------------------------------------------------------------
@pytest.mark.parametrize("M,N,K,kind,out", [
    (1, 4, 64, "q8", "f32"),            # inject-like: one row, four outputs
    (77, 320, 8192, "q8", "f32"),       # HC down at BASELINE width
    (300, 512, 320, "q8", "bf16"),      # HC up: K = 320 (five 64-steps), bf16 output
    (130, 200, 2048, "bf16", "f32"),    # bf16 weights (indexer / router)
    (257, 129, 128, "q8", "f32"),       # row and column tails
    (1024, 1024, 1024, "q8", "f32"),    # 8 x 8 tiles (the XCD-grouped numbering)
    (77, 4, 8192, "bf16", "f32"),       # HC inject: the skinny kernel (4 weight rows, K 8192)
    (300, 16, 2048, "bf16", "f32"),     # GDN alpha / beta gates on the skinny kernel
    (5, 7, 4096, "bf16", "f32"),        # skinny with a row count below one workgroup's 16
    (77, 4, 6144, "bf16", "f32"),       # skinny, three 2,048-wide k slices (HC inject at n_embd 1,536)
    (40, 8, 6144, "bf16", "f32"),       # 8 rows x 3 slices: no skinny kernel, the MFMA path
    # 512 tiles and more: the one-LDS-buffer variants chosen for the chunk's large projections
    (2048, 6144, 2048, "q8", "f32"),    # GDN qkv at 2,048 rows (768 tiles)
    (2048, 4096, 1024, "q8", "bf16"),   # 512 tiles, bf16 output
    (1024, 8192, 320, "q8", "f32"),     # HC up shape (K 320, N = 4 * 2,048) at 1,024 rows
    (4100, 2048, 2048, "q8", "f32"),    # 528 tiles with a 4-row tail tile
])
def test_gemm_bf16_parity(wz, orc, gpu, M, N, K, kind, out):
    print("case gemm M=%d N=%d K=%d %s %s" % (M, N, K, kind, out), flush=True)
    rng = np.random.default_rng(M + N + K)
    lda = K + 8
    a = bf16_bits(rng.normal(0, 1, (M, lda)))
    af = bits_to_f32(a)
    if kind == "q8":
        wq = rng.integers(-127, 128, N * K).astype(np.int8)
        ws = rng.uniform(0.0005, 0.002, N * K // 32).astype(np.float16).view(np.uint16)
        wb = None
    else:
        wq = ws = None
        wb = bf16_bits(rng.normal(0, 0.05, N * K))
    ldy = N + 5
    want = np.zeros((M, ldy), np.float32)
    a_c = np.ascontiguousarray(af[:, :K])
    orc.orc_pf_gemm(ptr(a_c), M, K, ptr(wq), ptr(ws), ptr(wb), N, ptr(want), ldy)
    da = DA.from_numpy(a)
    dq = DA.from_numpy(wq) if wq is not None else None
    ds = DA.from_numpy(ws) if ws is not None else None
    db = DA.from_numpy(wb) if wb is not None else None
    if out == "f32":
        dy = DA.from_numpy(np.full((M, ldy), -7.0, np.float32))
        wz.wzy_gemm_bf16(da.ptr, lda, M, K, dq.ptr if dq else None, ds.ptr if ds else None, db.ptr if db else None,
                         N, dy.ptr, None, ldy, None)
    else:
        dy = DA.from_numpy(np.full((M, ldy), 0xABCD, np.uint16))
        wz.wzy_gemm_bf16(da.ptr, lda, M, K, dq.ptr if dq else None, ds.ptr if ds else None, db.ptr if db else None,
                         N, None, dy.ptr, ldy, None)
    wz.wzy_device_sync()
    got = dy.numpy()
    for arr in (da, dq, ds, db, dy):
        if arr is not None:
            arr.free()
    # fp32 accumulation in another order: bounded by a small multiple of eps_f32 * sum |a w|
    wfull = np.zeros((N, K), np.float64)
    if kind == "q8":
        wfull = bits_to_f32(bf16_bits(wq.astype(np.float32) *
                                      np.repeat(ws.view(np.float16).astype(np.float32), 32))).reshape(N, K)
    else:
        wfull = bits_to_f32(wb).reshape(N, K)
    mag = np.abs(a_c).astype(np.float64) @ np.abs(wfull).astype(np.float64).T
    if out == "f32":
        err = np.abs(got[:, :N] - want[:, :N])
        assert (err <= 1e-5 * mag + 1e-7).all(), "max excess %.3g" % (err - 1e-5 * mag).max()
        assert (got[:, N:] == -7.0).all(), "wrote past N"
    else:
        g = bits_to_f32(got[:, :N])
        o = want[:, :N]
        err = np.abs(g - o)
        assert (err <= np.abs(o) * 2.0 ** -8 + 1e-5 * mag + 1e-7).all(), "bf16 output beyond one ulp"
        assert (got[:, N:] == 0xABCD).all(), "wrote past N"


# ---- whole chunks against the oracle, teacher-forced on the discrete decisions ---------------------
def router_gaps(dm, w, x):
    """top_k-th minus (top_k+1)-th router logit of bf16(x) rows (fp64 sums)"""
    xb = tbf16(x).astype(np.float64)
    R = bits_to_f32(w["router"]).astype(np.float64).reshape(dm.E, dm.D)
    lg = np.sort(xb @ R.T, axis=1)[:, ::-1]
    return lg[:, dm.K - 1] - lg[:, dm.K]


def beyond(g, o, floor_only=None, what=None):
    """elements beyond |g - o| <= ATOL + RTOL * max(|o|, rms of o's row) (rows = last axis): the north
    star's tolerance with the relative term floored at the row's RMS, as in teacher_forced.py -- a
    residual stream element that nearly cancels (large terms, small sum) carries the terms' error.
    floor_only (a dict) counts, under `what`, the elements within that bound but beyond the plain
    elementwise one |g - o| <= ATOL + RTOL |o|, and the elements compared (what + ' n')."""
    g = np.asarray(g, np.float64)
    o = np.asarray(o, np.float64)
    rms = np.sqrt(np.mean(o * o, axis=-1, keepdims=True))
    d = np.abs(g - o)
    bad = d > ATOL + RTOL * np.maximum(np.abs(o), rms)
    if floor_only is not None:
        floor_only[what] = floor_only.get(what, 0) + int(((d > ATOL + RTOL * np.abs(o)) & ~bad).sum())
        floor_only[what + " n"] = floor_only.get(what + " n", 0) + d.size
    return bad


def floor_summary(fo, max_frac):
    """Print the floor-only counts and assert each component's share is at most max_frac."""
    txt = ", ".join("%s %d/%d" % (k, fo[k], fo[k + " n"]) for k in fo if not k.endswith(" n"))
    print("elements within tolerance only through the row-RMS floor: " + txt, flush=True)
    for k in fo:
        if not k.endswith(" n"):
            assert fo[k] <= max_frac * fo[k + " n"], "%s: %d of %d elements pass only through the row-RMS floor" % (
                k, fo[k], fo[k + " n"])


def check_appends(orc, st, cfg, l, qi, p0, B, pre, glob, layer_w):
    """The KV and indexer appends of a chunk's rows in QSA layer l, on identical inputs: the oracle's
    quantisation of the very k (after norm + RoPE) and v rows the GPU quantised (trace.pf_kv) equals the
    GPU's cells bit for bit, codes and fp16 scales; the oracle's indexer appends of the GPU's raw key
    rows, one row at a time from the state before the chunk (`pre`), give the GPU's tail exactly, its
    placeholder within tolerance and its pooled keys bit for bit except where an fp16 code sits at a
    rounding midpoint of the oracle's unrounded key (|key - midpoint| below 2^-17 of the key).
    Returns (KV bytes compared, midpoint flips)."""
    KVD, ID, blk = cfg.qsa_kvh * cfg.qsa_hd, cfg.idx_dim, cfg.idx_blk
    rw = 2 * KVD + ID
    nq = len([x for x in range(cfg.n_layers) if is_qsa(cfg, x)])
    rows = st.read(-1, "trace.pf_kv", np.float32).reshape(nq, -1, rw)[qi, :B]
    gk, gv, gr = (np.ascontiguousarray(rows[:, :KVD]), np.ascontiguousarray(rows[:, KVD:2 * KVD]),
                  np.ascontiguousarray(rows[:, 2 * KVD:]))
    cells = {n: st.read_range(l, n, dt, p0 * w, B * w).reshape(B, w) for n, dt, w in
             (("kv_k", np.int8, KVD), ("kv_v", np.int8, KVD), ("kv_ks", np.uint16, KVD // 64),
              ("kv_vs", np.uint16, KVD // 64))}
    oq, os_ = np.zeros(KVD, np.int8), np.zeros(KVD // 64, np.uint16)
    for t in range(B):
        for src, qn, sn in ((gk, "kv_k", "kv_ks"), (gv, "kv_v", "kv_vs")):
            orc.orc_kv_quant_row(ptr(src[t]), KVD, ptr(oq), ptr(os_))
            assert np.array_equal(cells[qn][t], oq) and np.array_equal(cells[sn][t], os_), \
                "layer %d cell %d: %s differs from the quantisation of the GPU's own row" % (l, p0 + t, qn)
    tail, dead, pooled = pre["idx_tail"].copy(), pre["idx_dead"].copy(), pre["idx_pooled"].copy()
    keys = {}
    key = np.empty(ID, np.float32)
    for t in range(B):
        p = p0 + t
        key[:] = np.nan
        orc.orc_indexer_append_f32(ptr(gr[t]), ptr(layer_w["idx_kn"]), ptr(glob["cos"]), ptr(glob["sin"]), p, ID, blk,
                                   cfg.n_rot, cfg.eps, ptr(tail), ptr(dead), ptr(pooled), ptr(key))
        if not np.isnan(key[0]):
            keys[p // blk] = key.copy()
    assert np.array_equal(st.read(l, "idx_tail", np.float32), tail), "layer %d indexer tail" % l
    np.testing.assert_allclose(st.read(l, "idx_dead", np.float32), dead, rtol=RTOL, atol=ATOL)
    nb = (p0 + B) // blk + 2
    gp = st.read_range(l, "idx_pooled", np.uint16, 0, nb * ID)
    flips = 0
    for i in np.flatnonzero(gp != pooled[:nb * ID]):
        b, d = divmod(int(i), ID)
        # a block the chunk completed, or the placeholder row after the last one (fp16 of the fp32
        # placeholder, which a chunk starting the context computes itself)
        assert b in keys or (b - 1 in keys and b == max(keys) + 1), \
            "layer %d pooled key %d dim %d differs, and the chunk completed no such block" % (l, b, d)
        vec = keys[b] if b in keys else dead
        assert key_flip_ok(vec[d], gp[i], pooled[i], vec), \
            "layer %d pooled key %d dim %d: fp16 codes %d vs %d, unrounded %r not at their midpoint" % (
                l, b, d, gp[i], pooled[i], float(vec[d]))
        flips += 1
    return 2 * B * (KVD + KVD // 64 * 2), flips


def check_chunk(wz, orc, st, om, cfg, p0, toks, label):
    """The prefill of toks at p0 that `st` just ran (with the trace on), against the oracle:
      1. every MoE block on the GPU's own FFN input (orc_moe_prefill), rows whose routing is a near
         tie (router gap below 1e-4) excepted;
      2. every QSA row's selected cells bit-exact against the reference top-k rule on the GPU's own
         block scores, and those scores within tolerance of the composition's;
      3. the independent composition of the prefill (prefill_compose) teacher-forced on the GPU's MoE
         outputs and selections: every layer's HC read outputs and attention / GDN block, the final
         residual rows (rel 2e-2 / abs 1e-2, the relative term floored at the row's RMS), the GDN
         state, the KV cells and the indexer state.
    Returns the composed state (for a decode step after the chunk)."""
    dm = dims_of(cfg)
    B = len(toks)
    L = cfg.n_layers
    qsa_layers = [l for l in range(L) if is_qsa(cfg, l)]
    qi = {l: i for i, l in enumerate(qsa_layers)}
    layers, state, glob = stage_weights(om, cfg)
    state0 = state_copy(state)
    tr = st.read(-1, "trace.pf", np.float32).reshape(L, 4, -1, cfg.n_embd)[:, :, :B]
    nq = max(1, len(qsa_layers))
    sel = st.read(-1, "trace.pf_sel", np.int32).reshape(nq, -1, cfg.idx_topk)[:, :B]
    cnt = st.read(-1, "trace.pf_cnt", np.int32).reshape(nq, -1)[:, :B]
    # 1. MoE blocks
    n_moe_rows = 0
    for l in range(L):
        comb_o, _, _ = moe_oracle(orc, dm, layers[l], glob, l, tr[l, 2])
        keep = router_gaps(dm, layers[l], tr[l, 2]) > 1e-4
        n_moe_rows += int(keep.sum())
        # inputs from real layers put more activations on bf16 rounding ties than N(0,1) rows do
        assert_prefill_close(tr[l, 3][keep], comb_o[keep], cfg.n_embd, max_frac=1e-3)
    # 2 + 3. composition forced on the GPU's decisions
    sel_out = {}
    R_c, dbg_c = compose_prefill(orc, dm, layers, state0, glob, p0, toks, moe=lambda l, x: tr[l, 3],
                                 sel_force=lambda l, t: sel[qi[l], t, :cnt[qi[l], t]], sel_out=sel_out)
    max_b = cfg.ctx_max // cfg.idx_blk + 2
    scores = st.read(-1, "trace.pf_scores", np.float32).reshape(nq, -1, max_b)[:, :B]
    n_sel = n_same = 0
    sel_row = np.empty(cfg.idx_topk, np.int32)
    for (l, t), (cells, margin, sc_o) in sel_out.items():
        n_kv = p0 + t + 1
        got = sel[qi[l], t, :cnt[qi[l], t]]
        assert cnt[qi[l], t] == min(n_kv, cfg.idx_topk), (l, t)
        if sc_o is None:                                  # every cell, in order
            assert np.array_equal(got, np.arange(n_kv)), "%s layer %d row %d identity selection" % (label, l, t)
        else:
            # the exact top-k rule on the GPU's own block scores: bit-exact
            sc_g = np.ascontiguousarray(scores[qi[l], t, :n_kv // cfg.idx_blk + 1])
            n = orc.orc_topk_select(ptr(sc_g), n_kv, cfg.idx_blk, cfg.idx_topk, ptr(sel_row))
            assert n == len(got) and np.array_equal(got, sel_row[:n]), "%s layer %d row %d selection" % (label, l, t)
            # the scores themselves against the composition's, relative term floored at the row's RMS
            # (a score is a sum of ReLU'd dots: where a dot sits near zero its share moves by the
            # dot's noise, which scales with the row, not with the small score)
            floor = np.sqrt(np.mean(np.asarray(sc_o, np.float64) ** 2))
            bad = np.abs(sc_g - sc_o) > ATOL + RTOL * np.maximum(np.abs(sc_o), floor)
            assert not bad.any(), "%s layer %d row %d block scores" % (label, l, t)
        n_sel += 1
        n_same += int(margin > 1e-3 and np.array_equal(got, cells))
    fo = {}
    for l in range(L):
        for j, name in ((0, "attention HC read"), (1, "block"), (2, "FFN HC read")):
            g, o = tr[l, j], dbg_c[l, j]
            bad = beyond(g, o, fo, name)
            assert not bad.any(), "%s layer %d %s: %d elements beyond tolerance (max |diff| %.3g)" % (
                label, l, name, bad.sum(), np.abs(g - o).max())
    R_g = np.empty_like(R_c)
    wz.wzy_stage_pre_head(st.h, R_g.ctypes.data, B)
    bad = beyond(R_g, R_c, fo, "final residual")
    assert not bad.any(), "%s final residual: %d elements beyond tolerance" % (label, bad.sum())
    kvd = cfg.qsa_kvh * cfg.qsa_hd
    pre = state_copy(state)                 # the state before the chunk (stage_weights' arrays are untouched)
    n_kv_bytes = n_flips = 0
    for l in qsa_layers:
        nb_, nf_ = check_appends(orc, st, cfg, l, qi[l], p0, B, pre[l], glob, layers[l])
        n_kv_bytes += nb_
        n_flips += nf_
    for l in range(L):
        s = state0[l]
        if not is_qsa(cfg, l):
            for name in ("ssm", "conv_hist"):
                g = st.read(l, name, np.float32)
                bad = np.abs(g - s[name]) > ATOL + RTOL * np.abs(s[name])
                assert not bad.any(), "%s layer %d %s: %d beyond tolerance" % (label, l, name, bad.sum())
        else:
            cells = slice(p0 * kvd, (p0 + B) * kvd)
            # the cells are bit-exact on the GPU's own k / v rows (check_appends above); against the
            # composition's own rows, which carry the bf16 rounding noise of every earlier layer (about
            # 1e-3 relative three layers deep), a code may sit one step away
            for name, key in (("kv_k", "kq"), ("kv_v", "vq")):
                d = np.abs(st.read(l, name, np.int8)[cells].astype(int) - s[key][cells].astype(int))
                assert d.max() <= 1, "%s layer %d %s: max %d" % (label, l, name, d.max())
            nb = (p0 + B) // cfg.idx_blk + 1
            g = st.read_range(l, "idx_pooled", np.uint16, 0, nb * cfg.idx_dim).view(np.float16).astype(np.float32)
            o = s["idx_pooled"][:nb * cfg.idx_dim].view(np.float16).astype(np.float32)
            np.testing.assert_allclose(g, o, rtol=RTOL, atol=ATOL, err_msg="%s layer %d pooled keys" % (label, l))
            for name in ("idx_tail", "idx_dead"):
                np.testing.assert_allclose(st.read(l, name, np.float32), s[name], rtol=RTOL, atol=ATOL,
                                           err_msg="%s layer %d %s" % (label, l, name))
    if "ple_hist" in state0[1]:
        # the per-layer embedding's conv history after the chunk, and the chunk's tokens in the history
        g = st.read(1, "ple_hist", np.float32)
        bad = np.abs(g - state0[1]["ple_hist"]) > ATOL + RTOL * np.abs(state0[1]["ple_hist"])
        assert not bad.any(), "%s PLE conv history: %d beyond tolerance" % (label, bad.sum())
        assert np.array_equal(st.read_range(-1, "tok_hist", np.int32, p0, B), np.asarray(toks, np.int32))
    print("%s: %d of %d MoE rows compared (the rest within 1e-4 of a routing tie), %d selections bit-exact on the "
          "GPU's scores (%d also equal to the composition's own), %d KV bytes bit-exact on the GPU's rows, %d "
          "pooled-key fp16 midpoint flips, every layer and the state within tolerance" % (
              label, n_moe_rows, L * B, n_sel, n_same, n_kv_bytes, n_flips), flush=True)
    assert n_moe_rows >= 0.99 * L * B
    assert n_sel == len(qsa_layers) * B
    floor_summary(fo, 1e-3)
    return state0


@pytest.mark.parametrize("p0,B,prefix", [(0, 150, 0), (37, 100, 37), (0, 7, 0), (5, 300, 5)])
def test_stage_prefill_matches_oracle(wz, orc, gpu, p0, B, prefix):
    print("case prefill p0=%d B=%d" % (p0, B), flush=True)
    cfg = pf_cfg()
    rng = np.random.default_rng(p0 * 7 + B)
    toks = [int(t) for t in rng.integers(0, cfg.n_vocab, p0 + B + 1)]
    st = wzy_amd.Stage(cfg)
    try:
        st.load_synthetic(SEED, 0)
        for p in range(0, prefix, 8):                         # the context before the chunk: decode windows
            st.forward(p, toks[p:min(p + 8, prefix)], run_head=False)
        st.sync()
        wz.wzy_stage_set_trace(st.h, 1)
        om = OracleModel(wz, st, cfg, SEED)                   # the oracle starts from the stage's state
        st.prefill(p0, toks[p0:p0 + B])
        st.sync()
        check_chunk(wz, orc, st, om, cfg, p0, toks[p0:p0 + B], "p0=%d B=%d" % (p0, B))
        # the decode row after the chunk, teacher-forced from the stage's prefilled state (the state
        # itself was checked against the composition above)
        tf = TeacherForced(wz, st, cfg, om)
        tf.sync_from_stage()
        pos = p0 + B
        st.forward(pos, [toks[pos]])
        st.sync()
        gt = gpu_trace(st, cfg, 1, len([l for l in range(cfg.n_layers) if is_qsa(cfg, l)]))
        tf.check_row("decode after prefill pos %d" % pos, pos, toks[pos], gt, st.logits(1), st.greedy(1), st.pre_head(1))
        print("decode after prefill: " + tf.summary(), flush=True)
        tf.assert_bounds()
    finally:
        st.close()


def run_chunks(cfg, toks, splits, seed=SEED, n_ctx=0):
    st = wzy_amd.Stage(cfg)
    st.load_synthetic(seed, n_ctx)
    p = n_ctx
    for n in splits:
        st.prefill(p, toks[p - n_ctx:p - n_ctx + n])
        p += n
    st.sync()
    last = np.empty((splits[-1], cfg.hc, cfg.n_embd), np.float32)
    st.lib.wzy_stage_pre_head(st.h, last.ctypes.data, splits[-1])
    return st, last


def assert_same_state(a, b, cfg, n_cells):
    kvd = cfg.qsa_kvh * cfg.qsa_hd
    for l in range(cfg.n_layers):
        if not is_qsa(cfg, l):
            for name in ("ssm", "conv_hist"):
                assert np.array_equal(a.read(l, name, np.float32), b.read(l, name, np.float32)), (l, name)
        else:
            for name, dt, per in (("kv_k", np.int8, kvd), ("kv_v", np.int8, kvd), ("kv_ks", np.uint16, kvd // 64),
                                  ("kv_vs", np.uint16, kvd // 64)):
                assert np.array_equal(a.read_range(l, name, dt, 0, n_cells * per),
                                      b.read_range(l, name, dt, 0, n_cells * per)), (l, name)
            nb = n_cells // cfg.idx_blk + 1
            assert np.array_equal(a.read_range(l, "idx_pooled", np.uint16, 0, nb * cfg.idx_dim),
                                  b.read_range(l, "idx_pooled", np.uint16, 0, nb * cfg.idx_dim)), (l, "pooled")
            for name in ("idx_tail", "idx_dead"):
                assert np.array_equal(a.read(l, name, np.float32), b.read(l, name, np.float32)), (l, name)


def test_prefill_chunking_is_exact_small(wz, gpu):
    print("case prefill_chunking_small", flush=True)
    cfg = pf_cfg()
    toks = [int(t) for t in np.random.default_rng(3).integers(0, cfg.n_vocab, 300)]
    a, ra = run_chunks(cfg, toks, [200])
    b, rb = run_chunks(cfg, toks, [61, 103, 36])
    try:
        assert_same_state(a, b, cfg, 200)
        assert np.array_equal(ra[-36:], rb)
    finally:
        a.close()
        b.close()


def baseline_cfg(n_layers, ctx_max, qsa_period=4):
    c = wzy_amd.StageCfg()
    wzy_amd.lib().wzy_stage_cfg_default(C.byref(c), ctx_max)
    c.n_layers = n_layers
    c.qsa_period = qsa_period
    return c


def test_prefill_chunking_is_exact_baseline_shapes(wz, gpu):
    """BASELINE shapes, 4 layers (3 GDN + 1 QSA) over a 3,000-cell synthetic context: 2,100 rows in
    one chunk (two block-score passes of up to 2,048 rows) against 700 + 1,400."""
    print("case prefill_chunking_baseline", flush=True)
    cfg = baseline_cfg(4, 8192)
    n_ctx = 3000
    toks = [int(t) for t in np.random.default_rng(4).integers(0, cfg.n_vocab, 2100)]
    a, ra = run_chunks(cfg, toks, [2100], n_ctx=n_ctx)
    try:
        b, rb = run_chunks(cfg, toks, [700, 1400], n_ctx=n_ctx)
        try:
            assert_same_state(a, b, cfg, n_ctx + 2100)
            assert np.array_equal(ra[-1400:], rb)
        finally:
            b.close()
    finally:
        a.close()


def test_prefill_baseline_shapes_match_oracle(wz, orc, gpu):
    """BASELINE shapes on four layers (GDN, GDN, GDN, QSA) at a 4,000-cell context (the QSA layer
    selects 2,048 of 4,000+ cells), a 40-cell chunk against the oracle."""
    print("case prefill_baseline_oracle", flush=True)
    cfg = baseline_cfg(4, 8192)
    n_ctx, B = 4000, 40
    toks = [int(t) for t in np.random.default_rng(5).integers(0, cfg.n_vocab, B)]
    st = wzy_amd.Stage(cfg)
    try:
        st.load_synthetic(SEED, n_ctx)
        wz.wzy_stage_set_trace(st.h, 1)
        om = OracleModel(wz, st, cfg, SEED)
        st.prefill(n_ctx, toks)
        st.sync()
        check_chunk(wz, orc, st, om, cfg, n_ctx, toks, "baseline")
    finally:
        st.close()


def dense_w(wt, rows, cols):
    """A projection's weights as the prefill GEMM reads them (orc_pf_gemm): Q8_0 code x fp16 scale rounded
    to bf16, or the bf16 values, as float64 [rows x cols]."""
    if isinstance(wt, tuple):
        q, s = wt
        w = q.astype(np.float32).reshape(rows, cols) * np.repeat(
            s.view(np.float16).astype(np.float32).reshape(rows, cols // 32), 32, axis=1)
        return bits_to_f32(bf16_bits(w)).astype(np.float64)
    return bits_to_f32(wt).reshape(rows, cols).astype(np.float64)


def proj(x, w):
    """orc_pf_gemm's arithmetic (bf16-rounded operands, double accumulation) as one float64 BLAS product"""
    return (tbf16(x).astype(np.float64) @ w.T).astype(np.float32)


def check_chunk_sampled(wz, orc, st, om, cfg, p0, toks, rows, label):
    """A chunk too long for the full composition, checked teacher-forced on the GPU's trace:
      * every row's KV cells and indexer appends bit-exact on the GPU's own rows (check_appends);
      * every GDN layer's recurrence over all rows from the GPU's attention-half inputs (projections in
        orc_pf_gemm's arithmetic, orc_gdn_step), the final state against the GPU's, and the block of
        the sampled rows;
      * for the sampled rows: each layer's HC reads from the residual chain rebuilt from the GPU's
        blocks and MoE outputs (orc_hc_read_pf), the MoE blocks on the GPU's FFN inputs
        (orc_moe_prefill), the QSA rows' block scores on the final indexer state, their selections
        bit-exact on the GPU's scores, their attention (orc_attend_pf over the GPU's selection and
        KV store) and o projection, and the final residual rows.
    Hidden states are held to the elementwise tolerance with the relative term floored at the row's
    RMS; the elements that pass only through the floor are counted and bounded."""
    dm = dims_of(cfg)
    B, L, D, HC = len(toks), cfg.n_layers, cfg.n_embd, cfg.hc
    QKV, GV, HV = 2 * dm.HK * 128 + dm.HV * 128, dm.HV * 128, dm.HV
    QD, KVD, HD, ID, IH, blk = dm.QH * dm.HD, dm.KVH * dm.HD, dm.HD, dm.IDIM, dm.IH, dm.IBLK
    qsa_layers = [l for l in range(L) if is_qsa(cfg, l)]
    qi = {l: i for i, l in enumerate(qsa_layers)}
    nq = max(1, len(qsa_layers))
    layers, state, glob = stage_weights(om, cfg)
    pre = state_copy(state)
    S = np.asarray(sorted(set(int(r) for r in rows if 0 <= r < B)))
    tr = st.read(-1, "trace.pf", np.float32).reshape(L, 4, -1, D)[:, :, :B]
    fo = {}

    def cmp(what, g, o, tag):
        bad = beyond(g, o, fo, what)
        assert not bad.any(), "%s %s: %d elements beyond tolerance (max |diff| %.3g)" % (
            label, tag, bad.sum(), np.abs(np.asarray(g, np.float64) - o).max())

    # byte work of every row, bit-exact on identical inputs
    n_bytes = n_flips = 0
    for l in qsa_layers:
        a, b = check_appends(orc, st, cfg, l, qi[l], p0, B, pre[l], glob, layers[l])
        n_bytes, n_flips = n_bytes + a, n_flips + b
    # the residual chain of the sampled rows, rebuilt from the GPU's blocks and MoE outputs
    R = np.repeat(embed(glob, dm, np.asarray(toks)[S])[:, None, :], HC, axis=1).astype(np.float32)
    pend = None
    n_moe = 0
    max_b = cfg.ctx_max // blk + 2
    sel = st.read(-1, "trace.pf_sel", np.int32).reshape(nq, -1, cfg.idx_topk)
    cnt = st.read(-1, "trace.pf_cnt", np.int32).reshape(nq, -1)
    scores = st.read(-1, "trace.pf_scores", np.float32).reshape(nq, -1, max_b)

    def hc_read(R, w, half, bo=None, ip=None):
        Rn = np.ascontiguousarray(R, np.float32).copy()
        n = Rn.shape[0]
        inj = np.empty((n, HC), np.float32)
        mixed = np.empty((n, D), np.float32)
        bo_ = None if bo is None else np.ascontiguousarray(bo, np.float32)
        ip_ = None if ip is None else np.ascontiguousarray(ip, np.float32)
        orc.orc_hc_read_pf(ptr(Rn), ptr(bo_), ptr(ip_), ptr(w["hc_norm%d" % half]), ptr(w["hc_down%d" % half][0]),
                           ptr(w["hc_down%d" % half][1]), ptr(w["hc_inj%d" % half]), ptr(w["hc_up%d" % half][0]),
                           ptr(w["hc_up%d" % half][1]), D, HC, dm.HCLR, dm.EPS, n, ptr(inj), ptr(mixed))
        return Rn, mixed, inj

    def write(R, blk_rows, inj):
        g = 2.0 / (1.0 + np.exp(-inj.astype(np.float64) / HC))
        return (R + blk_rows[:, None, :].astype(np.float64) * g[:, :, None]).astype(np.float32)

    for l, w in enumerate(layers):
        R, mixed, inj_a = hc_read(R, w, 0, *(pend if pend is not None else (None, None)))
        cmp("attention HC read", tr[l, 0, S], mixed, "layer %d attention HC read" % l)
        xa = tr[l, 0]                                 # the GPU's attention-half input of every row
        if not w["qsa"]:
            qkv = proj(xa, dense_w(w["qkv"], QKV, D))
            z = proj(xa, dense_w(w["wgate"], GV, D))
            ab = np.ascontiguousarray(np.concatenate([proj(xa, dense_w(w["alpha"], HV, D)),
                                                      proj(xa, dense_w(w["beta"], HV, D))], axis=1))
            hist, ssm = pre[l]["conv_hist"].copy(), pre[l]["ssm"].copy()
            y = np.empty((B, GV), np.float32)
            orc.orc_gdn_step(ptr(qkv), ptr(z), ptr(ab), ptr(w["dt"]), ptr(w["ssm_a"]), ptr(w["conv_w"]), ptr(hist),
                             ptr(ssm), ptr(w["ssm_norm"]), dm.EPS, ptr(y), dm.HK, HV, B)
            for name, o in (("conv_hist", hist), ("ssm", ssm)):
                g = st.read(l, name, np.float32)
                bad = np.abs(g - o) > ATOL + RTOL * np.abs(o)
                assert not bad.any(), "%s layer %d %s after %d rows: %d beyond tolerance" % (label, l, name, B, bad.sum())
            block = proj(y[S], dense_w(w["wout"], D, GV))
        else:
            q = qi[l]
            Wq, Wk = dense_w(w["wq"], 2 * QD, D), dense_w(w["idx_q"], IH * ID, D)
            qg, q_idx = proj(xa[S], Wq), proj(xa[S], Wk)
            att = np.zeros((len(S), QD), np.float32)
            pooled, dead = st.read(l, "idx_pooled", np.uint16), st.read(l, "idx_dead", np.float32)
            kv = tuple(st.read(l, n, dt) for n, dt in (("kv_k", np.int8), ("kv_ks", np.uint16), ("kv_v", np.int8),
                                                       ("kv_vs", np.uint16)))
            sc_o = np.zeros(max_b, np.float32)
            own = np.empty(cfg.idx_topk, np.int32)
            for i, t in enumerate(S):
                p = p0 + int(t)
                n_kv = p + 1
                for h in range(dm.QH):
                    orc.orc_head_norm_rope(qg[i, h * 2 * HD:].ctypes.data, HD, ptr(w["q_norm"]), ptr(glob["cos"]),
                                           ptr(glob["sin"]), p, dm.NROT, dm.EPS)
                for h in range(IH):
                    orc.orc_head_norm_rope(q_idx[i, h * ID:].ctypes.data, ID, ptr(w["idx_qn"]), ptr(glob["cos"]),
                                           ptr(glob["sin"]), p, dm.NROT, dm.EPS)
                got = np.ascontiguousarray(sel[q, t, :cnt[q, t]])
                assert cnt[q, t] == min(n_kv, cfg.idx_topk), (l, t)
                if n_kv > cfg.idx_topk:
                    # complete blocks below n_kv / blk no longer change, and the open block is scored
                    # against the placeholder: the final indexer state scores row t as it was
                    orc.orc_block_scores(ptr(pooled), ptr(dead), q_idx[i].ctypes.data, n_kv, IH, ID, blk, ptr(sc_o))
                    nb = n_kv // blk + 1
                    sc_g = np.ascontiguousarray(scores[q, t, :nb])
                    bad = np.abs(sc_g - sc_o[:nb]) > ATOL + RTOL * np.abs(sc_o[:nb])
                    assert not bad.any(), "%s layer %d row %d: %d block scores beyond tolerance" % (label, l, t, bad.sum())
                    n = orc.orc_topk_select(ptr(sc_g), n_kv, blk, cfg.idx_topk, ptr(own))
                    assert n == len(got) and np.array_equal(got, own[:n]), "%s layer %d row %d selection" % (label, l, t)
                else:
                    assert np.array_equal(got, np.arange(n_kv)), (l, t)
                att[i] = attend(orc, True, qg[i], *kv, got, dm.QH, dm.KVH, HD)
            block = proj(att, dense_w(w["wo"], D, QD))
        cmp("block", tr[l, 1, S], block, "layer %d block" % l)
        R = write(R, tr[l, 1, S], inj_a)
        R, mixed2, inj_f = hc_read(R, w, 1)
        cmp("FFN HC read", tr[l, 2, S], mixed2, "layer %d FFN HC read" % l)
        comb_o, _, _ = moe_oracle(orc, dm, w, glob, l, tr[l, 2, S])
        keep = router_gaps(dm, w, tr[l, 2, S]) > 1e-4
        n_moe += int(keep.sum())
        assert_prefill_close(tr[l, 3, S][keep], comb_o[keep], D, max_frac=1e-3)
        pend = (np.ascontiguousarray(tr[l, 3, S]), inj_f)
    R = write(R, *pend)
    R_g = np.empty((B, HC, D), np.float32)
    wz.wzy_stage_pre_head(st.h, R_g.ctypes.data, B)
    cmp("final residual", R_g[S], R, "final residual")
    print("%s: %d sampled rows of %d (all %d layers), %d of %d MoE rows compared (the rest within 1e-4 of a routing "
          "tie), %d KV bytes bit-exact on the GPU's rows, %d pooled-key fp16 midpoint flips, GDN state after every "
          "row within tolerance" % (label, len(S), B, L, n_moe, L * len(S), n_bytes, n_flips), flush=True)
    assert n_moe >= L * len(S) - 2
    floor_summary(fo, 1e-3)


@pytest.mark.timeout(900)
def test_prefill_8192_rows_baseline_shapes(wz, orc, gpu):
    """The bench's chunk length, 8,192 rows, through four BASELINE-shape layers (GDN, GDN, GDN, QSA)
    after a 4,000-cell context: the large projections take the one-LDS-buffer GEMM (up to 4,096 tiles),
    the HC up projection's stream-mean epilogue runs at N = 8,192, the indexer scores run in four
    2,048-row passes and the top-2,048 selects among up to 3,048 blocks.  Checked by
    check_chunk_sampled: every row's byte work and GDN recurrence, every layer of 40 sampled rows."""
    print("case prefill_8192_baseline", flush=True)
    cfg = baseline_cfg(4, 16384)
    n_ctx, B = 4000, 8192
    rng = np.random.default_rng(8)
    toks = [int(t) for t in rng.integers(0, cfg.n_vocab, B)]
    rows = [0, 1, 2, 3, 4, 5, 2047, 2048, 2049, 4095, 4096, 6143, 6144, 8188, 8189, 8190, 8191]
    rows += [int(r) for r in rng.choice(B, 23, replace=False)]
    st = wzy_amd.Stage(cfg)
    try:
        st.load_synthetic(SEED, n_ctx)
        wz.wzy_stage_set_trace(st.h, 1)
        om = OracleModel(wz, st, cfg, SEED)
        st.prefill(n_ctx, toks)
        st.sync()
        check_chunk_sampled(wz, orc, st, om, cfg, n_ctx, toks, rows, "8192 rows")
    finally:
        st.close()


def test_prefill_errors(wz, gpu):
    cfg = small_cfg(wzy_amd, ctx_max=256, n_layers=2, topk=64)       # 16 experts: no MFMA MoE block
    st = wzy_amd.Stage(cfg)
    try:
        st.load_synthetic(1, 0)
        with pytest.raises(wzy_amd.WzyError):
            st.prefill(0, list(range(10)))
    finally:
        st.close()
    cfg = pf_cfg(ctx_max=256, n_layers=2)
    st = wzy_amd.Stage(cfg)
    try:
        with pytest.raises(wzy_amd.WzyError):
            st.prefill(0, [1, 2])                                      # not loaded
        st.load_synthetic(1, 0)
        with pytest.raises(wzy_amd.WzyError):
            st.prefill(250, list(range(10)))                           # past ctx_max
        with pytest.raises(wzy_amd.WzyError):
            st.prefill(0, [])
    finally:
        st.close()


def test_engine_prompt_through_chunked_prefill(wz, gpu):
    """A prompt remainder above 192 cells goes through wzy_stage_prefill (run_prefill_range,
    src/wzy_engine_v2.cu:1292-1376): the engine's stream equals an in-process stage running the same
    prefill and decode steps; splitting the prompt into smaller chunks (--prefill-chunk) and
    speculative decoding seeded from the prefill's pre-head rows leave the stream unchanged."""
    from test_gpu_engine import SEED as ENGINE_SEED
    from test_gpu_engine import EngineProc, greedy_req
    print("case engine_prefill", flush=True)
    cfg = pf_cfg(ctx_max=2048)
    prompt = [int(t) for t in np.random.default_rng(6).integers(0, cfg.n_vocab, 300)]
    n_new = 8
    st = wzy_amd.Stage(cfg)
    try:
        st.load_synthetic(ENGINE_SEED, 0)
        st.prefill(0, prompt[:-1])
        tok, pos, want = prompt[-1], len(prompt) - 1, []
        for _ in range(n_new):
            st.forward(pos, [tok])
            st.sync()
            tok = int(st.greedy(1)[0])
            want.append(tok)
            pos += 1
    finally:
        st.close()
    for args in ((), ("--prefill-chunk", "100"), ("--spec-depth", "3")):
        eng = EngineProc(cfg, *args)
        try:
            pf, toks, done = eng.request(greedy_req(prompt, n_new))
            assert pf["read"] == 300 and done["generated"] == n_new
            assert toks == want, "engine %s: %s vs in-process %s" % (args, toks, want)
            # a follow-up that extends the state reuses it (a short remainder: decode windows)
            pf2, _, _ = eng.request(greedy_req(prompt + toks[:-1] + [5], 2))
            assert pf2["reused"] == 300 + n_new - 1
        finally:
            assert eng.close() == 0

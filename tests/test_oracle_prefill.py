"""Pins the oracle's chunked prefill (orc_prefill.c) on the CPU.

- orc_pf_gemm against a float64 matmul of weights dequantised and rounded to bf16 by torch.
- orc_hc_read_pf against closed forms (zero up-projection: the stream gate is 1/2; zero inject
  logits: the pending block is added with gate 1) and against an independent float64 / torch-bf16
  composition of tc_gr_read (src/wzy_prefill_tc.cuh:690-715).
- orc_attend_pf against exact float64 softmax attention (the fp16 operands stay within their
  rounding), and the one-cell closed form out = fp16(v) * sigmoid(gate).
- orc_model_prefill against an independent composition of run_stage_prefill's layer order
  (src/wzy_prefill_tc.cuh:790-1055) written here from the pinned primitives, with planted wiring
  mistakes that the comparison must catch; and against the decode composition of the same model
  (orc_model_forward over windows), which differs only in the projections' operand rounding.
"""
import ctypes as C
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle_lib
from prefill_compose import compose_prefill
from stage_oracle import BLOB_FN, OrcLayer, OrcModel
from test_oracle_model_composition import (CTX, D, EPS, F, GV, HC, HCLR, HD, HK, HV, IBLK, IDIM, IH, KINDS, KVD,
                                           KVH, N_CTX, NROT, QD, QH, QKV, TOPK, V, E, K, Model, bf16, bf16_to_f32,
                                           f16, max_violation, oracle_forward)

ptr = oracle_lib.ptr


def tbf16(x):
    """round to bf16 (nearest even) with torch"""
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).to(torch.float32).numpy()


def th16(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def q8_random(rng, rows, cols, std=0.05):
    codes = rng.integers(-127, 128, rows * cols).astype(np.int8)
    sc = f16(std / 64 * rng.uniform(0.5, 1.5, rows * cols // 32))
    return codes, sc


def q8_dequant_bf16(codes, sc, rows, cols):
    s = np.repeat(sc.view(np.float16).astype(np.float32), 32)
    return tbf16(codes.astype(np.float32) * s).reshape(rows, cols)


# ---- GEMM ----------------------------------------------------------------------------------------
@pytest.mark.parametrize("M,N,K,kind", [(1, 4, 64, "q8"), (7, 33, 320, "q8"), (19, 130, 256, "bf16"),
                                        (5, 64, 1024, "q8")])
def test_pf_gemm_matches_float64(orc, M, N, K, kind):
    rng = np.random.default_rng(M * 1000 + N)
    a = tbf16(rng.normal(0, 1, (M, K)))
    if kind == "q8":
        q, s = q8_random(rng, N, K)
        w = q8_dequant_bf16(q, s, N, K)
        args = (ptr(q), ptr(s), None)
    else:
        wb = bf16(rng.normal(0, 0.05, N * K))
        w = bf16_to_f32(wb).reshape(N, K)
        args = (None, None, ptr(wb))
    y = np.empty((M, N + 3), np.float32)
    orc.orc_pf_gemm(ptr(a), M, K, *args, N, ptr(y), N + 3)
    want = a.astype(np.float64) @ w.astype(np.float64).T
    np.testing.assert_allclose(y[:, :N], want, rtol=1e-6, atol=1e-6)


# ---- HC read -------------------------------------------------------------------------------------
def hc_weights(rng, zero_up=False):
    w = {"norm": rng.uniform(0.5, 1.5, HC * D).astype(np.float32),
         "down": q8_random(rng, HCLR, HC * D, 1.0 / np.sqrt(HC * D) * 64),
         "up": q8_random(rng, HC * D, HCLR, 1.0 / np.sqrt(HCLR) * 64),
         "inj": bf16(rng.normal(0, 2.0 / np.sqrt(HC * D), HC * HC * D))}
    if zero_up:
        w["up"] = (np.zeros(HC * D * HCLR, np.int8), w["up"][1])
    return w


def hc_read_pf(orc, R, w, bo=None, inj_prev=None):
    B = R.shape[0]
    R = np.ascontiguousarray(R, np.float32).copy()
    inj = np.empty((B, HC), np.float32)
    mixed = np.empty((B, D), np.float32)
    orc.orc_hc_read_pf(ptr(R), ptr(bo), ptr(inj_prev), ptr(w["norm"]), ptr(w["down"][0]), ptr(w["down"][1]),
                       ptr(w["inj"]), ptr(w["up"][0]), ptr(w["up"][1]), D, HC, HCLR, EPS, B, ptr(inj), ptr(mixed))
    return R, inj, mixed


def xn_of(R, norm):
    r = R.astype(np.float64)
    inv = 1.0 / np.sqrt((r * r).mean(axis=2, keepdims=True) + EPS)
    return tbf16((r * inv).astype(np.float32) * norm.reshape(HC, D))


def test_hc_read_pf_closed_forms(orc):
    rng = np.random.default_rng(3)
    B = 5
    w = hc_weights(rng, zero_up=True)
    row = rng.normal(0, 1, (B, 1, D)).astype(np.float32)
    R = np.repeat(row, HC, axis=1)
    # zero up projection: every stream gate is sigmoid(0) = 1/2, so mixed = mean_c x_c / 2
    Rout, _, mixed = hc_read_pf(orc, R, w)
    np.testing.assert_array_equal(Rout, R)                       # nothing pending: R unchanged
    xn = xn_of(R, w["norm"])
    np.testing.assert_allclose(mixed, xn.mean(axis=1) * 0.5, rtol=1e-5, atol=1e-6)
    # a pending block with zero inject logits is added with gate 2 sigmoid(0) = 1
    bo = rng.normal(0, 1, (B, D)).astype(np.float32)
    Rout, _, _ = hc_read_pf(orc, R, w, bo, np.zeros((B, HC), np.float32))
    np.testing.assert_allclose(Rout, R + bo[:, None, :], rtol=1e-6, atol=1e-6)


def test_hc_read_pf_matches_independent_composition(orc):
    rng = np.random.default_rng(4)
    B = 6
    w = hc_weights(rng)
    R = rng.normal(0, 1, (B, HC, D)).astype(np.float32)
    bo = rng.normal(0, 1, (B, D)).astype(np.float32)
    ip = rng.normal(0, 2, (B, HC)).astype(np.float32)
    Rout, inj, mixed = hc_read_pf(orc, R, w, bo, ip)
    g = 2.0 / (1.0 + np.exp(-ip.astype(np.float64) / HC))
    Rw = (R + bo[:, None, :] * g[:, :, None]).astype(np.float32)
    np.testing.assert_allclose(Rout, Rw, rtol=1e-6, atol=1e-6)
    xn = xn_of(Rw, w["norm"]).reshape(B, HC * D).astype(np.float64)
    inj_w = bf16_to_f32(w["inj"]).reshape(HC, HC * D).astype(np.float64)
    np.testing.assert_allclose(inj, xn @ inj_w.T, rtol=1e-5, atol=1e-5)
    lo = xn @ q8_dequant_bf16(*w["down"], HCLR, HC * D).astype(np.float64).T / HC
    loh = tbf16(lo / (1.0 + np.exp(-lo)))
    gg = tbf16(loh.astype(np.float64) @ q8_dequant_bf16(*w["up"], HC * D, HCLR).astype(np.float64).T)
    with np.errstate(over="ignore"):
        want = (xn.reshape(B, HC, D) / (1.0 + np.exp(-gg.reshape(B, HC, D).astype(np.float64)))).mean(axis=1)
    np.testing.assert_allclose(mixed, want, rtol=2e-3, atol=2e-4)


# ---- attention -----------------------------------------------------------------------------------
def attn_inputs(rng, n_cells):
    kq = rng.integers(-127, 128, n_cells * KVD).astype(np.int8)
    vq = rng.integers(-127, 128, n_cells * KVD).astype(np.int8)
    ks = f16(rng.uniform(0.002, 0.02, n_cells * KVD // 64))
    vs = f16(rng.uniform(0.002, 0.02, n_cells * KVD // 64))
    qg = rng.normal(0, 1, QH * 2 * HD).astype(np.float32)
    return kq, ks, vq, vs, qg


def attend_pf(orc, kq, ks, vq, vs, qg, sel):
    out = np.empty(QH * HD, np.float32)
    sel = np.ascontiguousarray(sel, np.int32)
    orc.orc_attend_pf(ptr(qg), ptr(kq), ptr(ks), ptr(vq), ptr(vs), ptr(sel), len(sel), QH, KVH, HD, ptr(out))
    return out.reshape(QH, HD)


def test_attend_pf_one_cell_closed_form(orc):
    rng = np.random.default_rng(5)
    kq, ks, vq, vs, qg = attn_inputs(rng, 8)
    out = attend_pf(orc, kq, ks, vq, vs, qg, [3])
    gq = QH // KVH
    for h in range(QH):
        j = h // gq
        v = th16(vq.reshape(8, KVD)[3, j * HD:(j + 1) * HD].astype(np.float32) *
                 np.repeat(vs.view(np.float16).reshape(8, KVD // 64)[3, j * 4:(j + 1) * 4].astype(np.float32), 64))
        gate = qg.reshape(QH, 2 * HD)[h, HD:]
        np.testing.assert_allclose(out[h], v / (1.0 + np.exp(-gate)), rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("n", [5, 32, 33, 100, 300])
def test_attend_pf_matches_float64_softmax(orc, n):
    rng = np.random.default_rng(n)
    cells = 400
    kq, ks, vq, vs, qg = attn_inputs(rng, cells)
    sel = rng.choice(cells, n, replace=False)
    out = attend_pf(orc, kq, ks, vq, vs, qg, sel)
    K = kq.reshape(cells, KVD).astype(np.float64) * np.repeat(ks.view(np.float16).astype(np.float64).reshape(cells, -1), 64, 1)
    Vv = vq.reshape(cells, KVD).astype(np.float64) * np.repeat(vs.view(np.float16).astype(np.float64).reshape(cells, -1), 64, 1)
    q = qg.reshape(QH, 2 * HD).astype(np.float64)
    gq = QH // KVH
    for h in range(QH):
        j = h // gq
        s = (K[sel, j * HD:(j + 1) * HD] @ q[h, :HD]) / 16.0
        p = np.exp(s - s.max())
        o = (p / p.sum()) @ Vv[sel, j * HD:(j + 1) * HD]
        want = o / (1.0 + np.exp(-q[h, HD:]))
        np.testing.assert_allclose(out[h], want, rtol=5e-3, atol=2e-3 * np.abs(want).max())


# ---- whole-chunk composition -----------------------------------------------------------------------
def build_model(orc, m, state):
    keep = []

    def p(a):
        keep.append(a)
        return a.ctypes.data

    L = (OrcLayer * len(KINDS))()
    for l, w in enumerate(m.layers):
        o, s = L[l], state[l]
        o.qsa = 1 if w["qsa"] else 0
        for h in range(2):
            o.hc_norm[h] = p(w["hc_norm%d" % h])
            o.hc_down_q[h], o.hc_down_s[h] = p(w["hc_down%d" % h][0]), p(w["hc_down%d" % h][1])
            o.hc_up_q[h], o.hc_up_s[h] = p(w["hc_up%d" % h][0]), p(w["hc_up%d" % h][1])
            o.hc_inj[h] = p(w["hc_inj%d" % h])
        if not w["qsa"]:
            for n in ("qkv", "wgate", "wout"):
                setattr(o, n + "_q", p(w[n][0]))
                setattr(o, n + "_s", p(w[n][1]))
            o.alpha, o.beta, o.ssm_a, o.dt = p(w["alpha"]), p(w["beta"]), p(w["ssm_a"]), p(w["dt"])
            o.conv_w, o.ssm_norm = p(w["conv_w"]), p(w["ssm_norm"])
            o.conv_hist, o.ssm = p(s["conv_hist"]), p(s["ssm"])
        else:
            for n in ("wq", "wk", "wv", "wo"):
                setattr(o, n + "_q", p(w[n][0]))
                setattr(o, n + "_s", p(w[n][1]))
            o.q_norm, o.k_norm = p(w["q_norm"]), p(w["k_norm"])
            o.idx_q, o.idx_k, o.idx_qn, o.idx_kn = p(w["idx_q"]), p(w["idx_k"]), p(w["idx_qn"]), p(w["idx_kn"])
            o.kq, o.ks, o.vq, o.vs = p(s["kq"]), p(s["ks"]), p(s["vq"]), p(s["vs"])
            o.idx_tail, o.idx_dead, o.idx_pooled = p(s["idx_tail"]), p(s["idx_dead"]), p(s["idx_pooled"])
        o.router, o.sgate = p(w["router"]), p(w["sgate"])
        for n in ("sh_gate", "sh_up", "sh_down"):
            setattr(o, n + "_q", p(w[n][0]))
            setattr(o, n + "_s", p(w[n][1]))
    mm = OrcModel()
    mm.n_layers, mm.n_embd, mm.hc, mm.hc_lr, mm.gdn_hk, mm.gdn_hv = len(KINDS), D, HC, HCLR, HK, HV
    mm.qsa_qh, mm.qsa_kvh, mm.qsa_hd, mm.n_rot = QH, KVH, HD, NROT
    mm.idx_heads, mm.idx_dim, mm.idx_blk, mm.idx_topk = IH, IDIM, IBLK, TOPK
    mm.n_exp, mm.top_k, mm.n_ff, mm.n_vocab, mm.ctx_max, mm.eps = E, K, F, V, CTX, EPS
    mm.layers = C.cast(L, C.POINTER(OrcLayer))
    mm.emb, mm.head_norm = p(m.emb), p(m.head_norm)
    mm.head_down_q, mm.head_down_s = p(m.head_down[0]), p(m.head_down[1])
    mm.head_up_q, mm.head_up_s = p(m.head_up[0]), p(m.head_up[1])
    mm.head, mm.cos_tab, mm.sin_tab = p(m.head), p(m.cos), p(m.sin)
    cb = BLOB_FN(lambda ctx, layer, e: m.blobs[layer][e].ctypes.data)
    mm.blob, mm.blob_ctx = cb, None
    return mm, (keep, L, cb)


def oracle_prefill(orc, m, state, pos, toks):
    mm, hold = build_model(orc, m, state)
    fn = orc.orc_model_prefill_dbg
    fn.restype = C.c_int
    fn.argtypes = [C.POINTER(OrcModel), C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
    B = len(toks)
    toks = np.asarray(toks, np.int32)
    R = np.empty((B, HC, D), np.float32)
    dbg = np.empty((len(KINDS), 4, B, D), np.float32)
    mg = np.empty((len(KINDS), B, 2), np.float32)
    assert fn(C.byref(mm), pos, toks.ctypes.data, B, R.ctypes.data, dbg.ctypes.data, mg.ctypes.data) == 0
    return R, dbg, mg


def fixture_glob(m):
    return {"emb": m.emb, "cos": m.cos, "sin": m.sin, "blob": lambda layer, e: m.blobs[layer][e]}


DIMS = SimpleNamespace(D=D, HC=HC, HCLR=HCLR, HK=HK, HV=HV, QH=QH, KVH=KVH, HD=HD, NROT=NROT, IH=IH, IDIM=IDIM,
                       IBLK=IBLK, TOPK=TOPK, E=E, K=K, F=F, V=V, CTX=CTX, EPS=EPS)


@pytest.fixture(scope="module")
def model(wz, orc):
    return Model(wz, orc, 2026)


CHUNK = [7, 301, 42, 99, 5, 6, 250, 11, 3, 17, 480, 2]      # 12 cells from N_CTX: completes 3 index blocks


def run_both(orc, m, plant=None):
    so, sc = m.state_copy(), m.state_copy()
    Ro, do, mg = oracle_prefill(orc, m, so, N_CTX, CHUNK)
    Rc, dc = compose_prefill(orc, DIMS, m.layers, sc, fixture_glob(m), N_CTX, CHUNK, plant)
    return (Ro, do, so, mg), (Rc, dc, sc)


def test_oracle_prefill_matches_independent_composition(wz, orc, model):
    (Ro, do, so, mg), (Rc, dc, sc) = run_both(orc, model)
    # both sides differ only in how the hyper-connection writes round (fma vs two roundings), far
    # below the closest routing decision of the fixture
    assert mg[:, :, 0].min() > 1e-5, "a routing near-tie in the fixture: %g" % mg[:, :, 0].min()
    for l in range(len(KINDS)):
        for j, name in enumerate(("attn mixed", "block", "ffn mixed", "moe comb")):
            v = max_violation(do[l, j], dc[l, j])
            assert v <= 0, "layer %d %s: %.3g beyond tolerance" % (l, name, v)
    assert max_violation(Ro, Rc) <= 0
    for l, (a, b) in enumerate(zip(so, sc)):
        for n in a:
            if a[n].dtype == np.float32:
                assert max_violation(a[n], b[n]) <= 0, "layer %d state %s" % (l, n)
            else:
                assert (a[n] != b[n]).mean() < 1e-3, "layer %d state %s" % (l, n)


@pytest.mark.parametrize("plant", ["drop_pending_fold", "attn_reads_ffn_weights", "drop_attn_write",
                                   "attn_write_uses_ffn_inject", "ffn_write_uses_attn_inject", "drop_final_write"])
def test_prefill_composition_check_detects_wiring_mistakes(wz, orc, model, plant):
    (Ro, _, _, _), (Rc, _, _) = run_both(orc, model, plant)
    assert max_violation(Ro, Rc) > 0, "planted %s went unnoticed" % plant


def test_oracle_prefill_tracks_the_decode_composition(wz, orc, model):
    """The same cells through the decode composition (int8-quantised projection operands, windows of
    up to 8 rows) leave nearly the same state: the two paths differ only in operand rounding, so any
    difference in the layer order or wiring would show as a large deviation."""
    sp, sd = model.state_copy(), model.state_copy()
    Rp, _, _ = oracle_prefill(orc, model, sp, N_CTX, CHUNK)
    pos = N_CTX
    for i in range(0, len(CHUNK), 8):
        w = CHUNK[i:i + 8]
        _, _, pre, _ = oracle_forward(orc, model, sd, pos, w)
        pos += len(w)
    last = pre[-1]
    rel = np.abs(Rp[-1] - last).max() / np.abs(last).max()
    assert rel < 0.1, "final residual row differs by %.3g of its scale" % rel
    for l, w in enumerate(model.layers):
        if not w["qsa"]:
            a, b = sp[l]["ssm"], sd[l]["ssm"]
            assert np.abs(a - b).max() / np.abs(b).max() < 0.1, "layer %d GDN state" % l
        else:
            cells = slice(N_CTX * KVD, (N_CTX + len(CHUNK)) * KVD)
            dk = np.abs(sp[l]["kq"][cells].astype(int) - sd[l]["kq"][cells].astype(int))
            assert np.median(dk) <= 2 and dk.mean() < 4, "layer %d K codes" % l

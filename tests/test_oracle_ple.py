"""Pins the oracle's per-layer embedding (oracle/orc_ple.c) on the CPU.

The reference ships no vectors for PLE, so each function is pinned by what the mathematics and the
reference's structure fix:
  * the fp8 decode against torch's float8_e4m3fn for all 256 codes (the two NaN codes read as 0);
  * the row ids by their structure: every head's row lies in its own slice of the table; the eight
    2-gram heads ignore the token two back; the 3-gram heads do not; a missing or end-of-sequence
    token cuts the context (what follows it reads as eos), so contexts that differ only past a cut
    share their rows; the multiplier of each context position matters (swapping the two previous
    tokens changes the rows);
  * orc_ple_rows: a window of T rows equals T one-row calls carried through the token history, and
    rows at the start of the context read no history;
  * orc_ple_block against an independent numpy float64 composition of the reference's kernel
    sequence, and by closed forms: with only the 9-back conv tap the row-t conv sees the normalised
    value of row t-9 (a wrong tap index fails), a T-row call equals T one-row calls carried through
    the history, and zero value weights leave only the pending fold.
"""
import ctypes as C

import numpy as np
import pytest

from oracle_lib import ptr
from refmath import e4m3_decode

EOS = 248044
ROW_FN = C.CFUNCTYPE(C.c_void_p, C.c_void_p, C.c_uint32)


def row_ids(orc, cur, p1, p2, eos=EOS):
    r = np.zeros(16, np.uint32)
    orc.orc_ple_row_ids(cur, p1, p2, eos, r.ctypes.data)
    return r


def test_fp8_decode_all_codes_vs_torch(orc):
    for v in range(256):
        mag = float(e4m3_decode([v])[0])                 # unsigned e4m3fn (0x7F decoded as 480 there)
        want = 0.0 if (v & 0x7F) == 0x7F else (-mag if v & 0x80 else mag)
        assert orc.orc_ple_fp8(v, 0.25) == pytest.approx(want * 0.25, rel=0, abs=0), v


def test_row_ids_structure(orc):
    rows = int(orc.orc_ple_table_rows())
    assert rows == 320001446
    rng = np.random.default_rng(0)
    bounds = []
    for cur, p1, p2 in [(5, 6, 7), (0, 0, 0), (151935, 248043, 1), (99, EOS, 3), (1234, 17, -1)]:
        r = row_ids(orc, cur, p1, p2)
        assert (r < rows).all()
        bounds.append(r)
    # each head in its own slice: rows of head h across many contexts never reach head h+1's slice
    lo = np.full(16, np.iinfo(np.uint64).max, np.uint64)
    hi = np.zeros(16, np.uint64)
    for _ in range(2000):
        r = row_ids(orc, *(int(x) for x in rng.integers(0, 200000, 3))).astype(np.uint64)
        lo, hi = np.minimum(lo, r), np.maximum(hi, r)
    assert (hi[:-1] < lo[1:]).all(), "head slices overlap"
    a, b = row_ids(orc, 11, 22, 33), row_ids(orc, 11, 22, 44)
    assert (a[:8] == b[:8]).all() and (a[8:] != b[8:]).all(), "2-gram heads must ignore the token two back"
    assert (a != row_ids(orc, 11, 23, 33)).all()
    assert (a != row_ids(orc, 12, 22, 33)).all()
    assert (a != row_ids(orc, 11, 33, 22)).any(), "context positions must not be interchangeable"
    # cuts: a missing or eos token ends the context, and everything older reads as eos
    assert (row_ids(orc, 11, -1, 5) == row_ids(orc, 11, EOS, EOS)).all()
    assert (row_ids(orc, 11, EOS, 5) == row_ids(orc, 11, EOS, 9)).all()
    assert (row_ids(orc, 11, 22, -1) == row_ids(orc, 11, 22, EOS)).all()
    assert (row_ids(orc, 11, 22, -1) != row_ids(orc, 11, 22, 5)).any()


class Table:
    """A small stand-in for the table: row r's bytes are a hash of r (the oracle only reads rows)."""

    def __init__(self, head):
        self.head = head
        self.rows = {}
        self.cb = ROW_FN(self._row)

    def _row(self, ctx, r):
        b = self.rows.get(r)
        if b is None:
            g = np.random.default_rng(int(r))
            b = g.integers(0, 256, self.head).astype(np.uint8)
            self.rows[r] = b
        return b.ctypes.data


def ple_rows(orc, tab, toks, pos, hist, scale=0.5):
    T = len(toks)
    out = np.empty((T, 16 * tab.head), np.float32)
    t = np.ascontiguousarray(toks, np.int32)
    orc.orc_ple_rows(C.cast(tab.cb, C.c_void_p), None, tab.head, scale, EOS, t.ctypes.data, T, pos, hist.ctypes.data,
                     out.ctypes.data)
    return out


def test_rows_window_equals_single_steps(orc):
    tab = Table(8)
    rng = np.random.default_rng(1)
    toks = [int(x) for x in rng.integers(0, 1000, 11)]
    h1 = np.full(64, -7, np.int32)
    win = np.concatenate([ple_rows(orc, tab, toks[:5], 0, h1), ple_rows(orc, tab, toks[5:], 5, h1)])
    h2 = np.full(64, -7, np.int32)
    one = np.concatenate([ple_rows(orc, tab, [t], p, h2) for p, t in enumerate(toks)])
    np.testing.assert_array_equal(win, one)
    np.testing.assert_array_equal(h1[:11], toks)
    # the decoded values are the rows' codes: row 0 of position 0 has no history (cut at once)
    r = row_ids(orc, toks[0], -1, -1)
    codes = np.frombuffer(C.string_at(tab.cb(None, int(r[3])), 8), np.uint8)
    want = [orc.orc_ple_fp8(int(c), 0.5) for c in codes]
    np.testing.assert_array_equal(win[0, 3 * 8:4 * 8], np.asarray(want, np.float32))


def bf16_bits(x):
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_f(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def make_block(D=64, HC=4, T=5, seed=3):
    g = np.random.default_rng(seed)
    HCD = HC * D
    return dict(R=g.normal(0, 1, (T, HC, D)).astype(np.float32), bo=g.normal(0, 1, (T, D)).astype(np.float32),
                inj=g.normal(0, 1, (T, HC)).astype(np.float32), emb=g.normal(0, 1, (T, D)).astype(np.float32),
                wk=bf16_bits(g.normal(0, D ** -0.5, (HCD, D))), wv=bf16_bits(g.normal(0, D ** -0.5, (D, D))),
                nq=g.normal(1, 0.1, HCD).astype(np.float32), nk=g.normal(1, 0.1, HCD).astype(np.float32),
                nc=g.normal(1, 0.1, HCD).astype(np.float32), cw=g.normal(0, 0.5, (HCD, 4)).astype(np.float32),
                hist=g.normal(0, 1, (HCD, 9)).astype(np.float32), D=D, HC=HC, T=T)


def run_block(orc, b, use_bo=True, snaps=False):
    R, hist = b["R"].copy(), b["hist"].copy()
    sn = np.zeros((b["T"], b["HC"] * b["D"], 9), np.float32) if snaps else None
    orc.orc_ple_block(ptr(R), ptr(b["bo"]) if use_bo else None, ptr(b["inj"]), ptr(b["emb"]), ptr(b["wk"]), ptr(b["wv"]),
                      ptr(b["nq"]), ptr(b["nk"]), ptr(b["nc"]), ptr(b["cw"]), ptr(hist), b["D"], b["HC"], 1e-6, b["T"], 0,
                      ptr(sn))
    return R, hist, sn


def compose_block(b, use_bo=True):
    """numpy float64: the reference's kernel sequence, src/wzy_stage_v2.cuh:583-597"""
    D, HC, T = b["D"], b["HC"], b["T"]
    R = b["R"].astype(np.float64)
    if use_bo:
        R = R + b["bo"][:, None, :] * (2.0 / (1.0 + np.exp(-b["inj"].astype(np.float64) / HC)))[:, :, None]

    def gnorm(x, gamma):
        return x / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6) * gamma.reshape(HC, D)

    q = gnorm(R, b["nq"])
    k = gnorm((b["emb"].astype(np.float64) @ bf16_f(b["wk"]).astype(np.float64).T).reshape(T, HC, D), b["nk"])
    v = b["emb"].astype(np.float64) @ bf16_f(b["wv"]).astype(np.float64).T
    s = (k * q).sum(-1) / np.sqrt(D)
    g = 1.0 / (1.0 + np.exp(-np.sign(np.where(s < 0, -1.0, 1.0)) * np.sqrt(np.maximum(np.abs(s), 1e-6))))
    gat = v[:, None, :] * g[:, :, None]
    n = gnorm(gat, b["nc"]).reshape(T, HC * D)
    hist = b["hist"].astype(np.float64).copy()
    out = R.reshape(T, HC * D).copy()
    for t in range(T):
        acc = b["cw"][:, 0] * hist[:, 0] + b["cw"][:, 1] * hist[:, 3] + b["cw"][:, 2] * hist[:, 6] + b["cw"][:, 3] * n[t]
        hist = np.concatenate([hist[:, 1:], n[t][:, None]], axis=1)
        out[t] += gat.reshape(T, HC * D)[t] + acc / (1.0 + np.exp(-acc))
    return out.reshape(T, HC, D), hist


@pytest.mark.parametrize("use_bo", [True, False])
def test_block_vs_numpy_composition(orc, use_bo):
    b = make_block()
    R, hist, _ = run_block(orc, b, use_bo)
    Rc, hc = compose_block(b, use_bo)
    np.testing.assert_allclose(R, Rc, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(hist, hc, rtol=1e-6, atol=1e-6)


def test_block_conv_taps(orc):
    """Only the oldest tap (9 rows back): row t's conv is w0 * n[t-9]; from a zero history the first 9
    rows add silu(0) = 0 and row 9 adds silu(w0 * n[0])."""
    b = make_block(T=12)
    b["hist"][:] = 0
    b["cw"][:] = 0
    b["cw"][:, 0] = 1.0
    R, _, sn = run_block(orc, b, use_bo=False, snaps=True)
    ref = b["R"].copy()
    # the gated values without the conv: the same call with zero conv weights
    b0 = dict(b)
    b0["cw"] = np.zeros_like(b["cw"])
    R0, _, _ = run_block(orc, b0, use_bo=False)
    conv = (R - R0).reshape(12, -1)
    n0 = sn[0][:, 8]                              # n of row 0 (the newest history entry after row 0)
    assert np.abs(conv[:9]).max() == 0.0
    np.testing.assert_allclose(conv[9], n0 / (1.0 + np.exp(-n0)), rtol=1e-6, atol=1e-7)
    assert not np.allclose(R0, ref)               # the gated values do reach the streams


def test_block_rows_equal_single_steps(orc):
    b = make_block(T=6)
    R, hist, sn = run_block(orc, b, snaps=True)
    h = b["hist"].copy()
    for t in range(6):
        bt = {k: (v[t:t + 1] if k in ("R", "bo", "inj", "emb") else v) for k, v in b.items()}
        bt["T"], bt["hist"] = 1, h
        Rt, h, _ = run_block(orc, bt)
        np.testing.assert_allclose(Rt[0], R[t], rtol=1e-6, atol=1e-6)
        np.testing.assert_array_equal(h, sn[t])
    np.testing.assert_array_equal(h, hist)


def test_block_zero_values_leave_the_fold(orc):
    b = make_block()
    b["wv"][:] = 0
    R, _, _ = run_block(orc, b)
    fold = b["R"] + b["bo"][:, None, :] * (2.0 / (1.0 + np.exp(-b["inj"] / 4.0)))[:, :, None]
    # gat = 0 and n = 0, so the conv sees only the history: acc = w0 h0 + w1 h3 + w2 h6 (+ 0)
    hist = b["hist"].astype(np.float64).copy()
    extra = np.zeros((b["T"], b["HC"] * b["D"]))
    for t in range(b["T"]):
        acc = b["cw"][:, 0] * hist[:, 0] + b["cw"][:, 1] * hist[:, 3] + b["cw"][:, 2] * hist[:, 6]
        hist = np.concatenate([hist[:, 1:], np.zeros((hist.shape[0], 1))], axis=1)
        extra[t] = acc / (1.0 + np.exp(-acc))
    np.testing.assert_allclose(R, fold + extra.reshape(R.shape), rtol=1e-5, atol=1e-5)

"""Pins the oracle's layer functions (GDN, RoPE, KV quantisation, indexer, block scores, top-k
selection, sparse attention, hyper-connection read) on the CPU.

Each check is one the mathematics fixes independently of the oracle's code: delta-rule closed forms
(overwrite with a repeated key, partial writes, pure decay), conv taps as shifts, RoPE as a rotation
(norm per (i, i+n_rot/2) pair, identity at position 0, relative-position invariance), numpy's own
fp16 rounding for the quantisers, brute-force sorting for the top-k tie rule, and float64 dense
softmax attention.  Each is chosen so that a plausible slip (transposed state, wrong key-head
mapping, interleaved RoPE pairs, unrounded scale, wrong tie order, missing 1/16 scale) fails it.
"""
import ctypes as C

import numpy as np
import pytest

import refmath
from oracle_lib import ptr

F32 = np.float32


def f32(a):
    return np.ascontiguousarray(a, dtype=F32)


def silu(x):
    return x / (1.0 + np.exp(-x))


def sigm(x):
    return 1.0 / (1.0 + np.exp(-x))


def run_recurrence(orc, q, k, v, decay, beta, S, hk, hv, z=None, gamma=None, eps=1e-6):
    T = decay.shape[0]
    y = np.empty((T, hv * 128), F32)
    S = f32(S).copy()
    # keep every converted array alive across the call (ptr() only takes an address)
    args = [f32(a) if a is not None else None for a in (q, k, v, decay, beta, z, gamma)]
    orc.orc_gdn_recurrence(*[ptr(a) for a in args], eps, ptr(S), ptr(y), hk, hv, T)
    return S.reshape(hv, 128, 128), y.reshape(T, hv, 128)


def unit(i, n=128):
    e = np.zeros(n, F32)
    e[i] = 1.0
    return e


# ---- GDN delta rule --------------------------------------------------------------------------

def test_gdn_beta_zero_only_decays(orc):
    rng = np.random.default_rng(1)
    hk = hv = 2
    S0 = rng.normal(0, 0.1, (hv, 128, 128)).astype(F32)
    q, k = rng.normal(size=(1, hk * 128)), rng.normal(size=(1, hk * 128))
    v = rng.normal(size=(1, hv * 128))
    decay = np.array([[0.9, 0.5]], F32)
    S, y = run_recurrence(orc, q, k, v, decay, np.zeros((1, hv), F32), S0, hk, hv)
    for h in range(hv):
        np.testing.assert_array_equal(S[h], (S0[h].astype(np.float64) * decay[0, h]).astype(F32))
        # readout o_j = sum_i S_ij q_i (value index j), then RMSNorm of o/sqrt(128)
        o = S[h].astype(np.float64).T @ q[0, h * 128:(h + 1) * 128] / np.sqrt(128.0)
        np.testing.assert_allclose(y[0, h], o / np.sqrt(np.mean(o * o) + 1e-6), rtol=2e-5, atol=2e-6)


def test_gdn_repeated_key_overwrites(orc):
    """decay 1, beta 1: writing (k, v1) then (k, v2) leaves k v2^T (an additive rule would leave
    k (v1+v2)^T), and reading with q = k returns v2, i.e. y = v2 / rms(v2)."""
    rng = np.random.default_rng(2)
    k1 = rng.normal(size=128)
    k1 /= np.linalg.norm(k1)
    v1, v2 = rng.normal(size=128), rng.normal(size=128)
    q = np.stack([k1, k1])[:, None, :].reshape(2, 128)
    S, y = run_recurrence(orc, q, q, np.stack([v1, v2]), np.ones((2, 1)), np.ones((2, 1)),
                          np.zeros((1, 128, 128)), 1, 1)
    np.testing.assert_allclose(S[0], np.outer(k1, v2), atol=2e-6)
    np.testing.assert_allclose(y[1, 0], v2 / np.sqrt(np.mean(v2 * v2)), rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(y[0, 0], v1 / np.sqrt(np.mean(v1 * v1)), rtol=1e-4, atol=1e-5)


def test_gdn_partial_write_closed_form(orc):
    """beta 1/2 twice with the same unit key: readout 0.25 v1 + 0.5 v2."""
    rng = np.random.default_rng(3)
    k1 = unit(5)
    v1, v2 = rng.normal(size=128), rng.normal(size=128)
    S, _ = run_recurrence(orc, np.stack([k1, k1]), np.stack([k1, k1]), np.stack([v1, v2]), np.ones((2, 1)),
                          np.full((2, 1), 0.5), np.zeros((1, 128, 128)), 1, 1)
    np.testing.assert_allclose(S[0, 5], 0.25 * v1 + 0.5 * v2, rtol=1e-6, atol=1e-7)
    assert np.abs(np.delete(S[0], 5, axis=0)).max() == 0.0


def test_gdn_value_head_uses_key_head_h_mod_hk(orc):
    hk, hv = 2, 4
    rng = np.random.default_rng(4)
    k = np.concatenate([unit(5), unit(9)])[None]           # key head 0 -> e5, key head 1 -> e9
    v = rng.normal(size=(1, hv * 128))
    S, _ = run_recurrence(orc, k, k, v, np.ones((1, hv)), np.ones((1, hv)), np.zeros((hv, 128, 128)), hk, hv)
    for h in range(hv):
        row = 5 if h % hk == 0 else 9
        np.testing.assert_allclose(S[h, row], v[0, h * 128:(h + 1) * 128], rtol=1e-6)
        assert np.abs(np.delete(S[h], row, axis=0)).max() == 0.0


def test_gdn_gate_and_norm_weight(orc):
    rng = np.random.default_rng(5)
    k1 = unit(0)
    v1 = rng.normal(size=128)
    z = rng.normal(size=(1, 128))
    gamma = rng.uniform(0.5, 1.5, 128)
    _, y = run_recurrence(orc, k1[None], k1[None], v1[None], np.ones((1, 1)), np.ones((1, 1)),
                          np.zeros((1, 128, 128)), 1, 1, z=z, gamma=gamma)
    np.testing.assert_allclose(y[0, 0], v1 / np.sqrt(np.mean(v1 * v1)) * gamma * sigm(z[0]), rtol=1e-4, atol=1e-5)


def test_gdn_step_conv_taps_and_gates(orc):
    """Conv weights [1,0,0,0] read the oldest history tap, [0,0,0,1] the current input; the history
    keeps the last three inputs; decay = exp(softplus(a + dt) * A) (identity above 20), beta =
    sigmoid(b), both observed through the state (S' = decay S + beta k v^T with S = 0 or beta ~ 0)."""
    hk = hv = 1
    QKV = 3 * 128
    rng = np.random.default_rng(6)
    hist0 = rng.normal(size=(QKV, 3)).astype(F32)
    x = rng.normal(size=(2, QKV)).astype(F32)
    w = np.zeros((QKV, 4), F32)
    w[:128, 0] = 1.0            # q channels: oldest tap
    w[128:, 3] = 1.0            # k, v channels: current input
    ssm_a, dt = np.array([-1.5], F32), np.array([0.3], F32)
    ab = np.array([[0.7, 2.0], [25.0, -3.0]], F32)         # [alpha | beta] per row
    S = np.zeros(128 * 128, F32)
    hist = hist0.copy()
    y = np.empty((2, 128), F32)
    orc.orc_gdn_step(ptr(x), None, ptr(ab), ptr(dt), ptr(ssm_a), ptr(w), ptr(hist), ptr(S), None, 1e-6, ptr(y),
                     hk, hv, 2)
    np.testing.assert_array_equal(hist[:, 1:], x.T)                 # last inputs, oldest first
    np.testing.assert_array_equal(hist[:, 0], hist0[:, 2])
    kn = [silu(x[t, 128:256].astype(np.float64)) for t in range(2)]
    kn = [a / np.sqrt(np.sum(a * a) + 1e-6) for a in kn]
    vv = [silu(x[t, 256:].astype(np.float64)) for t in range(2)]
    dec = [np.exp(np.log1p(np.exp(0.7 + 0.3)) * -1.5), np.exp((25.0 + 0.3) * -1.5)]
    bet = [sigm(2.0), sigm(-3.0)]
    S_ref = np.zeros((128, 128))
    for t in range(2):
        S_ref = dec[t] * S_ref
        S_ref = S_ref + np.outer(kn[t], (vv[t] - S_ref.T @ kn[t]) * bet[t])
    np.testing.assert_allclose(S.reshape(128, 128), S_ref, rtol=2e-4, atol=1e-6)
    # the q path reads the oldest tap: row 0's q is silu(hist0[:, 0]) normalised
    qn = silu(hist0[:128, 0].astype(np.float64))
    o = (dec[0] * 0 + bet[0] * np.outer(kn[0], vv[0])).T @ (qn / np.sqrt(np.sum(qn * qn) + 1e-6)) / np.sqrt(128)
    np.testing.assert_allclose(y[0], o / np.sqrt(np.mean(o * o) + 1e-6), rtol=1e-3, atol=1e-4)


# ---- RoPE, head norm -------------------------------------------------------------------------

def rope_tables(orc, ctx, n_rot, theta):
    c = np.empty((ctx, n_rot // 2), F32)
    s = np.empty((ctx, n_rot // 2), F32)
    orc.orc_rope_tables(ctx, n_rot, theta, ptr(c), ptr(s))
    return c, s


def test_rope_tables_vs_numpy(orc):
    c, s = rope_tables(orc, 300, 64, 1e7)
    p = np.arange(300, dtype=np.float64)[:, None]
    ang = p * np.power(np.float64(np.float32(1e7)), -2.0 * np.arange(32) / 64.0)
    np.testing.assert_allclose(c, np.cos(ang), rtol=0, atol=6e-8)
    np.testing.assert_allclose(s, np.sin(ang), rtol=0, atol=6e-8)


def head_norm_rope(orc, x, gamma, c, s, pos, n_rot=64, eps=1e-6):
    p = f32(x).copy()
    g = f32(gamma)
    orc.orc_head_norm_rope(ptr(p), len(p), ptr(g), ptr(c), ptr(s), pos, n_rot, eps)
    return p.astype(np.float64)


def test_head_norm_rope_is_a_pairwise_rotation(orc):
    rng = np.random.default_rng(7)
    c, s = rope_tables(orc, 2000, 64, 1e7)
    x = rng.normal(size=256)
    g = rng.uniform(0.5, 1.5, 256)
    base = x / np.sqrt(np.mean(x * x) + 1e-6) * g
    np.testing.assert_allclose(head_norm_rope(orc, x, g, c, s, 0), base, rtol=1e-5, atol=1e-6)   # position 0
    for pos in (1, 17, 1999):
        r = head_norm_rope(orc, x, g, c, s, pos)
        np.testing.assert_allclose(r[64:], base[64:], rtol=1e-5, atol=1e-6)             # unrotated dims
        np.testing.assert_allclose(r[:32] ** 2 + r[32:64] ** 2, base[:32] ** 2 + base[32:64] ** 2,
                                   rtol=1e-4, atol=1e-6)                                  # pairs (i, i+32)
    # relative positions: <rope(q, a), rope(k, b)> depends on a - b only
    kx = rng.normal(size=256)
    ones = np.ones(256)
    d1 = head_norm_rope(orc, x, ones, c, s, 100)[:64] @ head_norm_rope(orc, kx, ones, c, s, 40)[:64]
    d2 = head_norm_rope(orc, x, ones, c, s, 1060)[:64] @ head_norm_rope(orc, kx, ones, c, s, 1000)[:64]
    assert d1 == pytest.approx(d2, rel=1e-4, abs=1e-4)


# ---- INT8 KV quantisation --------------------------------------------------------------------

def test_kv_quant_divides_by_the_fp16_rounded_scale(orc):
    rng = np.random.default_rng(8)
    x = rng.normal(size=512).astype(F32)
    x[64:128] = 0.0                                      # zero group
    # group 2: amax/127 = 0.0123456 is not an fp16 value; the other elements sit on half-steps of
    # the fp16-rounded scale, so dividing by the unrounded scale rounds them differently
    d_h = float(np.float16(F32(127 * 0.0123456) / F32(127)))
    x[128] = 127 * 0.0123456
    x[129:192] = (np.arange(1, 64) % 60 + 0.5) * d_h
    q = np.empty(512, np.int8)
    s = np.empty(8, np.uint16)
    orc.orc_kv_quant_row(ptr(x), 512, ptr(q), ptr(s))
    xg = x.reshape(8, 64)
    h = (np.abs(xg).max(1) / F32(127)).astype(np.float16)
    np.testing.assert_array_equal(s, h.view(np.uint16))
    d = h.astype(F32)
    with np.errstate(divide="ignore", invalid="ignore"):
        ref = np.where(d[:, None] > 0, np.clip(np.rint(xg / d[:, None]), -127, 127), 0).astype(np.int8)
    np.testing.assert_array_equal(q.reshape(8, 64), ref)
    assert (q[64:128] == 0).all() and s[1] == 0
    # dividing by the unrounded scale would differ somewhere in this row
    unrounded = np.clip(np.rint(xg[2] / (np.abs(xg[2]).max() / F32(127))), -127, 127)
    assert not np.array_equal(unrounded, ref[2].astype(np.float64))


# ---- indexer keys, block scores, top-k ---------------------------------------------------------

def test_indexer_append_blocks(orc):
    """Keys are fp16-rounded; block b pools positions 4b..4b+3 (sum in position order, then /4),
    RMSNorm * gamma, RoPE at position 4b; position 0 also sets the placeholder key, later blocks
    push the placeholder into the open slot b+1."""
    dim, blk = 128, 4
    rng = np.random.default_rng(9)
    c, s = rope_tables(orc, 64, 64, 1e7)
    gamma = rng.uniform(0.5, 1.5, dim).astype(F32)
    raws = rng.normal(size=(12, dim)).astype(F32) * 3
    tail = np.zeros((blk - 1) * dim, F32)
    dead = np.zeros(dim, F32)
    pooled = np.zeros((6, dim), np.uint16)
    for pos in range(12):
        orc.orc_indexer_append(ptr(raws[pos]), ptr(gamma), ptr(c), ptr(s), pos, dim, blk, 64, 1e-6, ptr(tail),
                               ptr(dead), ptr(pooled))
        if pos == 0:
            r0 = raws[0].astype(np.float16).astype(np.float64)
            want = r0 / np.sqrt(np.mean(r0 * r0) + 1e-6) * gamma
            np.testing.assert_allclose(dead, want, rtol=1e-5, atol=1e-6)     # rope at 0 = identity
    rh = raws.astype(np.float16).astype(F32)
    for b in range(3):
        m = (((rh[4 * b] + rh[4 * b + 1]) + rh[4 * b + 2]) + rh[4 * b + 3]) * F32(0.25)
        m = m.astype(np.float64)
        v = m / np.sqrt(np.mean(m * m) + 1e-6) * gamma
        p = 4 * b
        y = v.copy()
        y[:32] = v[:32] * c[p] - v[32:64] * s[p]
        y[32:64] = v[:32] * s[p] + v[32:64] * c[p]
        got = pooled[b].view(np.float16).astype(np.float64)
        np.testing.assert_allclose(got, y, rtol=2e-3, atol=2e-3)
    np.testing.assert_array_equal(pooled[3], dead.astype(np.float16).view(np.uint16))   # open slot
    np.testing.assert_array_equal(tail.reshape(3, dim), rh[8:11])


def test_block_scores_brute_force(orc):
    heads, dim, blk = 4, 128, 4
    rng = np.random.default_rng(10)
    n_kv = 4 * 37 + 3
    nb = n_kv // blk
    pooled = rng.normal(size=(nb + 2, dim)).astype(np.float16)
    dead = rng.normal(size=dim).astype(F32)
    q = (rng.normal(size=(heads, dim)) * 1.0001).astype(F32)
    sc = np.empty(nb + 1, F32)
    orc.orc_block_scores(ptr(pooled.view(np.uint16)), ptr(dead), ptr(q), n_kv, heads, dim, blk, ptr(sc))
    qh = q.astype(np.float16).astype(np.float64)
    ref = np.maximum(qh @ pooled[:nb].astype(np.float64).T, 0).sum(0)
    np.testing.assert_allclose(sc[:nb], ref, rtol=1e-5, atol=1e-5)
    open_ref = np.maximum(q.astype(np.float64) @ dead.astype(np.float64), 0).sum() + 1e9
    assert sc[nb] == pytest.approx(open_ref, rel=1e-7)
    # the complete-block score uses the fp16-rounded query, which differs from the fp32 one here
    ref32 = np.maximum(q.astype(np.float64) @ pooled[:nb].astype(np.float64).T, 0).sum(0)
    assert np.abs(sc[:nb] - ref).max() < np.abs(ref32 - ref).max()


def brute_topk(scores, n_kv, blk, topk):
    """Sort every cell by (block score desc, block % 256, block // 256, cell) and take the first
    min(n_kv, topk); list them in thread order (block % 256, block // 256, cell)."""
    if n_kv <= topk:
        return list(range(n_kv))
    nbid = n_kv // blk
    cells = []
    for b in range(nbid + 1):
        w = blk if b < nbid else n_kv - nbid * blk
        for c in range(w):
            cells.append((-float(scores[b]), b % 256, b // 256, c, b * blk + c))
    cells.sort()
    taken = cells[:topk]
    taken.sort(key=lambda e: (e[1], e[2], e[3]))
    return [e[4] for e in taken]


@pytest.mark.parametrize("n_kv,topk,levels", [(4 * 700 + 2, 64, 3), (4 * 300, 100, 2), (4 * 1100 + 1, 2048, 5),
                                              (4 * 260 + 3, 37, 1), (50, 64, 4), (4 * 600, 16, 1000)])
def test_topk_select_brute_force(orc, n_kv, topk, levels):
    rng = np.random.default_rng(n_kv + topk)
    nb = n_kv // 4 + 1
    scores = rng.integers(0, levels, nb).astype(F32)      # few levels -> many ties at the threshold
    if n_kv % 4:
        scores[nb - 1] += 1e9                             # open partial block (its cells come first)
    sel = np.empty(max(topk, n_kv), np.int32)
    n = orc.orc_topk_select(ptr(scores), n_kv, 4, topk, ptr(sel))
    want = brute_topk(scores, n_kv, 4, topk)
    assert n == len(want)
    assert sel[:n].tolist() == want


# ---- sparse attention ------------------------------------------------------------------------

def test_attend_vs_dense_softmax(orc):
    qh, kvh, hd = 4, 2, 256
    kvd = kvh * hd
    rng = np.random.default_rng(11)
    cells = 40
    kq = rng.integers(-127, 128, (cells, kvd)).astype(np.int8)
    vq = rng.integers(-127, 128, (cells, kvd)).astype(np.int8)
    ks = rng.uniform(0.001, 0.02, (cells, kvd // 64)).astype(np.float16)
    vs = rng.uniform(0.001, 0.02, (cells, kvd // 64)).astype(np.float16)
    qg = rng.normal(size=(qh, 2 * hd)).astype(F32)
    sel = np.array(sorted(rng.choice(cells, 23, replace=False)), np.int32)
    out = np.empty(qh * hd, F32)
    orc.orc_attend(ptr(qg), ptr(kq), ptr(ks.view(np.uint16)), ptr(vq), ptr(vs.view(np.uint16)), ptr(sel), len(sel),
                   qh, kvh, hd, ptr(out))
    K = refmath.dequant(kq, ks.astype(F32), 64).reshape(cells, kvh, hd)
    V = refmath.dequant(vq, vs.astype(F32), 64).reshape(cells, kvh, hd)
    for h in range(qh):
        j = h // (qh // kvh)
        s = K[sel, j] @ qg[h, :hd].astype(np.float64) / 16.0
        p = np.exp(s - s.max())
        p /= p.sum()
        ref = (p @ V[sel, j]) * sigm(qg[h, hd:].astype(np.float64))
        np.testing.assert_allclose(out[h * hd:(h + 1) * hd], ref, rtol=1e-5, atol=1e-6)
    # one selected cell: the output is that cell's value row times the gate
    orc.orc_attend(ptr(qg), ptr(kq), ptr(ks.view(np.uint16)), ptr(vq), ptr(vs.view(np.uint16)), ptr(sel[3:4]), 1,
                   qh, kvh, hd, ptr(out))
    np.testing.assert_allclose(out[:hd], V[sel[3], 0] * sigm(qg[0, hd:].astype(np.float64)), rtol=1e-5, atol=1e-7)


# ---- hyper-connection read ---------------------------------------------------------------------

def q8_rand(rng, rows, cols, zero=False):
    codes = np.zeros((rows, cols), np.int8) if zero else rng.integers(-127, 128, (rows, cols)).astype(np.int8)
    scales = (rng.uniform(0.5, 1.5, (rows, cols // 32)) / 127 / np.sqrt(cols)).astype(np.float16)
    return codes, scales.view(np.uint16)


def hc_read(orc, D, HC, HCLR, R_in=None, emb=None, bo=None, injp=None, norm_w=None, down=None, up=None, inj_w=None,
            T=1):
    R_out = np.empty((T, HC, D), F32)
    nsc = np.empty((T, HC), F32)
    lo = np.empty((T, HCLR), F32)
    inj = np.zeros((T, HC), F32)
    mixed = np.empty((T, D), F32)
    orc.orc_hc_read(ptr(R_in), ptr(emb), ptr(bo), ptr(injp), ptr(norm_w), ptr(down[0]), ptr(down[1]), ptr(inj_w),
                    ptr(up[0]), ptr(up[1]), D, HC, HCLR, 1e-6, T, ptr(R_out), ptr(nsc), ptr(lo), ptr(inj), ptr(mixed))
    return R_out, nsc, lo, inj, mixed


def test_hc_read_closed_forms(orc):
    D, HC, HCLR = 256, 4, 64
    rng = np.random.default_rng(12)
    R = rng.normal(size=(1, HC, D)).astype(F32)
    nw = rng.uniform(0.8, 1.2, (HC, D)).astype(F32)
    zero_down = q8_rand(rng, HCLR, HC * D, zero=True)
    up = q8_rand(rng, HC * D, HCLR)
    # down = 0 -> lo = silu(0) = 0 -> every gate is sigmoid(0) = 1/2 -> mixed = sum_c xn_c / 8
    Ro, nsc, lo, _, mixed = hc_read(orc, D, HC, HCLR, R_in=R, norm_w=nw, down=zero_down, up=up)
    xn = R[0] / np.sqrt(np.mean(R[0].astype(np.float64) ** 2, axis=1, keepdims=True) + 1e-6) * nw
    np.testing.assert_array_equal(Ro, R)
    assert (lo == 0).all()
    np.testing.assert_allclose(mixed[0], xn.sum(0) / 8.0, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(nsc[0], 1 / np.sqrt(np.mean(R[0].astype(np.float64) ** 2, axis=1) + 1e-6), rtol=1e-6)
    # fold of the pending write: R_out = R_in + bo * 2 sigmoid(inj_prev / HC)
    bo = rng.normal(size=(1, D)).astype(F32)
    injp = rng.normal(size=(1, HC)).astype(F32)
    Ro, _, _, _, _ = hc_read(orc, D, HC, HCLR, R_in=R, bo=bo, injp=injp, norm_w=nw, down=zero_down, up=up)
    np.testing.assert_allclose(Ro[0], R[0] + bo * 2 * sigm(injp[0] / HC)[:, None], rtol=1e-6, atol=1e-6)
    # embedding rows are broadcast to every stream
    emb = rng.normal(size=(1, D)).astype(F32)
    Ro, _, _, _, _ = hc_read(orc, D, HC, HCLR, emb=emb, norm_w=nw, down=zero_down, up=up)
    np.testing.assert_array_equal(Ro[0], np.repeat(emb, HC, axis=0))


def test_hc_read_vs_dense_float64(orc):
    """The general case against float64 dense products with dequantised Q8 weights (no activation
    quantisation on this side: tolerance covers the per-32 int8 requantisation)."""
    D, HC, HCLR = 256, 4, 64
    HCD = HC * D
    rng = np.random.default_rng(13)
    R = rng.normal(size=(2, HC, D)).astype(F32)
    nw = rng.uniform(0.8, 1.2, (HC, D)).astype(F32)
    down = q8_rand(rng, HCLR, HCD)
    up = q8_rand(rng, HCD, HCLR)
    inj_w = np.asarray([np.float32(v) for v in rng.normal(size=HC * HCD) / np.sqrt(HCD)], F32)
    inj_w16 = (inj_w.view(np.uint32) >> 16).astype(np.uint16)
    _, _, lo, inj, mixed = hc_read(orc, D, HC, HCLR, R_in=R, norm_w=nw, down=down, up=up, inj_w=inj_w16, T=2)
    Wd = refmath.q8_dense(down[0], down[1], HCLR, HCD)
    Wu = refmath.q8_dense(up[0], up[1], HCD, HCLR)
    Wi = refmath.bf16_bits_to_f64(inj_w16).reshape(HC, HCD)
    for t in range(2):
        r = R[t].astype(np.float64)
        xn = (r / np.sqrt(np.mean(r * r, axis=1, keepdims=True) + 1e-6) * nw).reshape(HCD)
        lo_ref = silu(Wd @ xn / HC)
        assert np.abs(lo[t] - lo_ref).max() <= 2e-2 * np.abs(lo_ref).max()
        np.testing.assert_allclose(inj[t], Wi @ xn, rtol=1e-5, atol=1e-5)
        gate = sigm(Wu @ lo_ref).reshape(HC, D)
        mixed_ref = (xn.reshape(HC, D) * gate).sum(0) / 4
        assert np.abs(mixed[t] - mixed_ref).max() <= 2e-2 * np.abs(mixed_ref).max()

"""CPU checks of the MTP drafter oracle (oracle/orc_mtp.c) and of the Q2_0 synthetic generator.

The Q2_0 expert GEMVs are pinned against a float64 dequantise-then-matmul of the documented blob
layout (src/wzy_mtp.cuh:6-10,59-207); one full draft step (front + rest + head reduction,
src/wzy_mtp.cuh:658-733,293-403) is pinned against an independent float64 composition written here,
including a KV ring that wraps past 1,024 cells and the attention floor.
"""
import ctypes as C

import numpy as np
import pytest

import oracle_lib
from mtp_oracle import (RING, OracleMtp, bf16f, dequant_act, hc_read64, q2_dense, q8_dense, rand_q2_blob,
                        random_mtp, rms, rope64)

orc = oracle_lib.load()


def test_q2_code_bit_layout():
    b = np.array([0b11100100, 0b00011011], np.uint8)          # codes 0,1,2,3 then 3,2,1,0
    got = [orc.orc_q2_code(b.ctypes.data, k) for k in range(8)]
    assert got == [0, 1, 2, 3, 3, 2, 1, 0]
    assert orc.orc_q2_blob_bytes(2048, 512) == 884736        # 3*D*F/4 + 3*D*F/64*2
    assert orc.orc_q2_blob_bytes(2560, 640) == 1382400       # the reference's MTP_Q2_BLOB


@pytest.mark.parametrize("D,F", [(256, 128), (512, 64)])
def test_q2_expert_gemvs_match_dense_float64(D, F):
    rng = np.random.default_rng(D + F)
    blob = rand_q2_blob(rng, D, F)
    Wg, Wu, Wd = q2_dense(blob, D, F)
    x = rng.normal(0, 1, D).astype(np.float32)
    xq = np.empty(D, np.int8)
    xs = np.empty(D // 32, np.float32)
    orc.orc_quant_act(x.ctypes.data, D, 1, xq.ctypes.data, xs.ctypes.data, None, None)
    xd = xq.astype(np.float64) * np.repeat(xs.astype(np.float64), 32)
    aq = np.empty(F, np.int8)
    as_ = np.empty(F // 32, np.float32)
    act = np.empty(F, np.float32)
    orc.orc_q2_expert_gate_up(blob.ctypes.data, D, F, xq.ctypes.data, xs.ctypes.data, aq.ctypes.data, as_.ctypes.data,
                              act.ctypes.data)
    g, u = Wg @ xd, Wu @ xd
    want = g / (1 + np.exp(-g)) * u
    np.testing.assert_allclose(act, want, rtol=2e-5, atol=2e-5 * np.abs(want).max())
    # the requantised activations are the per-32 quantisation of act
    q2 = np.empty(F, np.int8)
    s2 = np.empty(F // 32, np.float32)
    orc.orc_quant_act(act.ctypes.data, F, 1, q2.ctypes.data, s2.ctypes.data, None, None)
    assert (q2 == aq).all() and (s2 == as_).all()
    out = np.empty(D, np.float32)
    orc.orc_q2_expert_down(blob.ctypes.data, D, F, aq.ctypes.data, as_.ctypes.data, out.ctypes.data)
    ad = aq.astype(np.float64) * np.repeat(as_.astype(np.float64), 32)
    want_d = Wd @ ad
    np.testing.assert_allclose(out, want_d, rtol=2e-5, atol=2e-5 * np.abs(want_d).max())


def test_q2_synthetic_generator(wz):
    D, F = 2048, 512
    n = wz.wzy_q2_expert_bytes(D, F)
    assert n == 884736
    blob = np.empty(n, np.uint8)
    wz.wzy_synth_q2_expert(7, 3, D, F, blob.ctypes.data)
    codes = blob[:3 * D * F // 4]
    cnt = np.bincount(np.stack([(codes >> (2 * k)) & 3 for k in range(4)]).ravel(), minlength=4)
    assert (np.abs(cnt / cnt.sum() - 0.25) < 0.005).all()
    sc = blob[3 * D * F // 4:].view(np.uint16).view(np.float16).astype(np.float64)
    gu, dn = sc[:2 * F * D // 64], sc[2 * F * D // 64:]
    assert gu.min() >= 2.0 ** -6 and gu.max() < 2.0 ** -5        # floor(log2(1/sqrt(2048))) = -6
    assert dn.min() >= 2.0 ** -5 and dn.max() < 2.0 ** -4        # floor(log2(1/sqrt(512))) = -5
    other = np.empty(n, np.uint8)
    wz.wzy_synth_q2_expert(7, 4, D, F, other.ctypes.data)
    assert (other != blob).mean() > 0.7


# ------------------------------------------------------------------------------------------------
# one draft step against an independent float64 composition
# ------------------------------------------------------------------------------------------------
DIMS = dict(D=256, HC=4, HCLR=32, qh=4, kvh=2, hd=256, n_rot=64, E=8, K=3, F=64, n_vocab=50, n_dv=40, eps=1e-6)


class Compose:
    """Float64 restatement of one draft step from the reference's kernel sequence; K/V cells are kept
    by position (no ring), quantised with orc_kv_quant_row (pinned in test_oracle_layers.py)."""

    def __init__(self, A, d, ctx):
        self.A, self.d = A, d
        self.kv = {}
        self.floor = 0
        cos = np.empty(ctx * d["n_rot"] // 2, np.float32)
        sin = np.empty_like(cos)
        orc.orc_rope_tables(ctx, d["n_rot"], 1e7, cos.ctypes.data, sin.ctypes.data)
        self.cos, self.sin = cos, sin

    def q8(self, name, x, rows, cols):
        return q8_dense(self.A[name + ".q"], self.A[name + ".s"], rows, cols) @ dequant_act(orc, x.astype(np.float32))

    def head_nr(self, v, g, pos):
        return rope64(rms(v, g, self.d["eps"]), pos, self.d["n_rot"], self.cos, self.sin)

    def front(self, pos, tok, rin):
        d, A = self.d, self.A
        D, HC, hd = d["D"], d["HC"], d["hd"]
        e = bf16f(A["emb"].reshape(-1, D)[tok if 0 <= tok < d["n_vocab"] else 0]).astype(np.float64)
        e2 = self.q8("fc_emb", rms(e, A["pre_norm_emb"], d["eps"]), D, D)
        R = np.stack([self.q8("fc_hid", rms(rin[c], A["pre_norm_hid"][c * D:(c + 1) * D], d["eps"]), D, D) + e2
                      for c in range(HC)])
        mixed, inj = hc_read64(orc, A, 0, R, d["eps"], d["HCLR"])
        kvd = d["kvh"] * hd
        k = self.q8("wk", mixed, kvd, D)
        v = self.q8("wv", mixed, kvd, D)
        k = np.concatenate([self.head_nr(k[j * hd:(j + 1) * hd], A["k_norm"], pos) for j in range(d["kvh"])])
        cell = []
        for x in (k, v):
            q = np.empty(kvd, np.int8)
            s = np.empty(kvd // 64, np.uint16)
            x32 = np.ascontiguousarray(x, np.float32)
            orc.orc_kv_quant_row(x32.ctypes.data, kvd, q.ctypes.data, s.ctypes.data)
            cell.append(q.astype(np.float64) * np.repeat(s.view(np.float16).astype(np.float64), 64))
        self.kv[pos] = cell
        return R, mixed, inj

    def step(self, pos, tok, rin):
        d, A = self.d, self.A
        D, HC, hd, qh, kvh, E, K, F = d["D"], d["HC"], d["hd"], d["qh"], d["kvh"], d["E"], d["K"], d["F"]
        R, mixed, inj = self.front(pos, tok, rin)
        qg = self.q8("wq", mixed, 2 * qh * hd, D)
        n_kv = pos + 1
        p0 = max(self.floor, n_kv - RING, 0)
        att = np.empty(qh * hd)
        for h in range(qh):
            q = self.head_nr(qg[h * 2 * hd:h * 2 * hd + hd], A["q_norm"], pos)
            j = h // (qh // kvh)
            ks = np.stack([self.kv[p][0][j * hd:(j + 1) * hd] for p in range(p0, n_kv)])
            vs = np.stack([self.kv[p][1][j * hd:(j + 1) * hd] for p in range(p0, n_kv)])
            s = ks @ q / 16.0
            w = np.exp(s - s.max())
            o = (w @ vs) / w.sum()
            gate = qg[h * 2 * hd + hd:(h + 1) * 2 * hd]
            att[h * hd:(h + 1) * hd] = o / (1 + np.exp(-gate))
        bo = self.q8("wo", att, D, qh * hd)
        R2 = R + bo[None, :] * (2 / (1 + np.exp(-inj / HC)))[:, None]
        mixed2, inj2 = hc_read64(orc, A, 1, R2, d["eps"], d["HCLR"])
        # MoE: bf16 router, softmax top-K (probability desc, id asc), renormalised weights
        lg = bf16f(A["router"]).astype(np.float64).reshape(E, D) @ mixed2
        pr = np.exp(lg - lg.max())
        pr /= pr.sum()
        order = sorted(range(E), key=lambda i: (-pr[i], i))[:K]
        wts = pr[order] / pr[order].sum()
        xd = dequant_act(orc, mixed2.astype(np.float32))
        rec = len(A["experts"]) // E
        acc = np.zeros(D)
        for k, e in enumerate(order):
            Wg, Wu, Wd = q2_dense(A["experts"][e * rec:(e + 1) * rec], D, F)
            g, u = Wg @ xd, Wu @ xd
            acc += wts[k] * (Wd @ dequant_act(orc, (g / (1 + np.exp(-g)) * u).astype(np.float32)))
        g = q8_dense(A["sh_gate.q"], A["sh_gate.s"], F, D) @ xd
        u = q8_dense(A["sh_up.q"], A["sh_up.s"], F, D) @ xd
        shared = q8_dense(A["sh_down.q"], A["sh_down.s"], D, F) @ dequant_act(
            orc, (g / (1 + np.exp(-g)) * u).astype(np.float32))
        sg = bf16f(A["sgate"]).astype(np.float64) @ mixed2
        comb = shared / (1 + np.exp(-sg)) + acc
        R_out = R2 + comb[None, :] * (2 / (1 + np.exp(-inj2 / HC)))[:, None]
        sample, _ = hc_read64(orc, A, 2, R_out, d["eps"], d["HCLR"])
        logits = self.q8("head", sample, d["n_dv"], D)
        best = int(np.argmax(logits))
        prob = 1.0 / max(np.exp(logits - logits[best]).sum(), 1.0)
        return R_out, sample, logits, int(A["dvocab"][best]), prob, order


def rel_norm(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)


def build(seed, ctx):
    rng = np.random.default_rng(seed)
    A = random_mtp(rng, DIMS)
    cm = Compose(A, DIMS, ctx)
    A["rope_cos"], A["rope_sin"] = cm.cos, cm.sin
    om = OracleMtp(DIMS, A)
    cm.A = om.a
    return rng, om, cm


def test_mtp_draft_chain_matches_float64_composition():
    rng, om, cm = build(11, 64)
    D, HC = DIMS["D"], DIMS["HC"]
    toks = rng.integers(0, DIMS["n_vocab"], 8)
    for p in range(6):                                           # catch-up cells 0..5
        rin = rng.normal(0, 1, (1, HC, D)).astype(np.float32)
        R, mixed, inj = om.front(p, toks[p:p + 1], rin)
        Rc, mc, ic = cm.front(p, int(toks[p]), rin[0])
        assert rel_norm(R[0], Rc) < 2e-3 and rel_norm(mixed[0], mc) < 2e-3 and rel_norm(inj[0], ic) < 2e-3
    rin = rng.normal(0, 1, (HC, D)).astype(np.float32)
    tok = int(toks[6])
    for j in range(3):                                           # three chained steps at cells 6, 7, 8
        R_out, sample, logits, t, prob = om.step(6 + j, tok, rin)
        Rc, sc, lc, tc, pc, order = cm.step(6 + j, tok, rin.astype(np.float64))
        assert rel_norm(R_out, Rc) < 2e-3, j
        assert rel_norm(sample, sc) < 2e-3, j
        assert rel_norm(logits, lc) < 2e-3, j
        srt = np.sort(lc)[::-1]
        if srt[0] - srt[1] > 1e-3 * max(1.0, abs(srt[0])):
            assert t == tc, j
        assert abs(prob - pc) <= 2e-3 * pc, j
        rin, tok = R_out, t


def test_mtp_ring_wraps_and_floor():
    """Cells past the 1,024-cell ring reuse slot p % 1024; the attention window is the last 1,024
    cells, or starts at the floor when that is higher."""
    ctx = 1400
    rng, om, cm = build(12, ctx)
    d = DIMS
    kvd = d["kvh"] * d["hd"]
    # cells 0 .. 1299 written directly (random INT8 codes and fp16 scales), the ring holding the last
    # 1,024 of them in slot p % 1024
    for p in range(1300):
        kq = rng.integers(-127, 128, kvd).astype(np.int8)
        vq = rng.integers(-127, 128, kvd).astype(np.int8)
        ks = rng.uniform(0.005, 0.02, kvd // 64).astype(np.float16)
        vs = rng.uniform(0.005, 0.02, kvd // 64).astype(np.float16)
        sl = p % RING
        om.a["kv_k"][sl * kvd:(sl + 1) * kvd] = kq
        om.a["kv_v"][sl * kvd:(sl + 1) * kvd] = vq
        om.a["kv_ks"][sl * (kvd // 64):(sl + 1) * (kvd // 64)] = ks.view(np.uint16)
        om.a["kv_vs"][sl * (kvd // 64):(sl + 1) * (kvd // 64)] = vs.view(np.uint16)
        cm.kv[p] = [kq.astype(np.float64) * np.repeat(ks.astype(np.float64), 64),
                    vq.astype(np.float64) * np.repeat(vs.astype(np.float64), 64)]
    rin = rng.normal(0, 1, (d["HC"], d["D"])).astype(np.float32)
    for floor in (0, 1100):
        om.set_floor(floor)
        cm.floor = floor
        R_out, sample, logits, t, prob = om.step(1300, 5, rin)
        Rc, sc, lc, tc, pc, _ = cm.step(1300, 5, rin.astype(np.float64))
        assert rel_norm(R_out, Rc) < 2e-3 and rel_norm(logits, lc) < 2e-3, floor
    # the two windows give different drafts, so the comparison above pins the window start
    om.set_floor(0)
    _, _, l0, _, _ = om.step(1301, 5, rin)
    om.set_floor(1100)
    _, _, l1, _, _ = om.step(1301, 5, rin)
    assert rel_norm(l0, l1) > 1e-2

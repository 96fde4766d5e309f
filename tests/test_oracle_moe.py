"""Pins the oracle's MoE path (quantisation, GEMVs, router, NVFP4 experts, combine) on the CPU."""
import ctypes as C

import numpy as np
import pytest

import moe_inputs as mi
import oracle_lib
import refmath
from oracle_lib import ptr


def quant(orc, x, cols, T):
    q32 = np.empty(T * cols, np.int8); s32 = np.empty(T * cols // 32, np.float32)
    q16 = np.empty(T * cols, np.int8); s16 = np.empty(T * cols // 16, np.float32)
    orc.orc_quant_act(ptr(x), cols, T, ptr(q32), ptr(s32), ptr(q16), ptr(s16))
    return q32, s32, q16, s16


def test_quant_act_properties(orc):
    rng = np.random.default_rng(2)
    T, cols = 3, 256
    x = (rng.standard_normal(T * cols) * 3).astype(np.float32)
    x[32:64] = 0.0                                     # an all-zero 32-block -> q = 0, d = 0
    x[64] = 127.0 * 0.5; x[65:80] = 1.0 / 127          # exact half-way values: 0.5 steps
    q32, s32, q16, s16 = quant(orc, x, cols, T)
    for q, s, g in ((q32, s32, 32), (q16, s16, 16)):
        xb, qb = x.reshape(-1, g), q.reshape(-1, g).astype(np.int32)
        amax = np.abs(xb).max(1)
        np.testing.assert_array_equal(s, (amax / np.float32(127)).astype(np.float32))
        assert np.abs(qb).max() <= 127
        nz = amax > 0
        np.testing.assert_array_equal(np.abs(qb[nz]).max(1), 127)     # the amax element maps to +-127
        err = np.abs(qb * s[:, None].astype(np.float64) - xb)
        assert np.all(err[nz] <= s[nz, None] * 0.5 * (1 + 1e-5) + 1e-12)
        assert not np.any(qb[~nz])
    # round-half-even on an exact tie: block [63.5, 1/127 x 15] -> 63.5 * (127/63.5) = 127 exactly,
    # 1/127 * 2 = 0.0157.. -> 0
    blk = x[64:80] * (np.float32(127.0) / np.abs(x[64:80]).max())
    np.testing.assert_array_equal(q16[64:80], np.rint(blk).astype(np.int8))


def test_gemv_q8_vs_dense(orc, wz):
    rows, cols, T = 96, 512, 3
    codes = np.empty(rows * cols, np.int8); sc = np.empty(rows * cols // 32, np.uint16)
    wz.wzy_synth_q8(11, 1, rows, cols, 0.05, ptr(codes), ptr(sc))
    x = np.random.default_rng(3).standard_normal(T * cols).astype(np.float32)
    q32, s32, _, _ = quant(orc, x, cols, T)
    y = np.empty(T * rows, np.float32)
    orc.orc_gemv_q8(ptr(codes), ptr(sc), ptr(q32), ptr(s32), ptr(y), rows, cols, T)
    W = refmath.q8_dense(codes, sc, rows, cols)
    xd = refmath.dequant(q32, s32, 32).reshape(T, cols)
    np.testing.assert_allclose(y.reshape(T, rows), xd @ W.T, rtol=1e-6, atol=1e-6)


def test_gemv_bf16_vs_dense(orc, wz):
    rows, cols, T = 40, 264, 2
    W = np.empty(rows * cols, np.uint16)
    wz.wzy_synth_normal_bf16(5, 2, rows * cols, 0.0, 0.1, ptr(W))
    x = np.random.default_rng(4).standard_normal(T * cols).astype(np.float32)
    y = np.empty(T * rows, np.float32)
    orc.orc_gemv_bf16(ptr(W), ptr(x), ptr(y), rows, cols, T)
    ref = x.reshape(T, cols).astype(np.float64) @ refmath.bf16_bits_to_f64(W).reshape(rows, cols).T
    np.testing.assert_allclose(y.reshape(T, rows), ref, rtol=1e-6, atol=1e-7)


def test_router_topk_vs_numpy_sort(orc):
    rng = np.random.default_rng(5)
    E, K, T = 512, 10, 4
    logits = rng.standard_normal(T * E).astype(np.float32)
    logits[E + 7] = logits[E + 3]           # an exact tie inside row 1
    logits[E + 3] = logits[E + 3] + 20.0
    logits[E + 7] = logits[E + 3]           # tie at the top: ids 3 and 7 equal -> 3 first
    ids = np.empty(T * K, np.int32); wts = np.empty(T * K, np.float32); probs = np.empty(T * E, np.float32)
    orc.orc_router_topk(ptr(logits), E, K, T, ptr(ids), ptr(wts), ptr(probs))
    for t in range(T):
        p = probs[t * E:(t + 1) * E]
        order = np.lexsort((np.arange(E), -p))[:K]       # value desc, id asc
        np.testing.assert_array_equal(ids[t * K:(t + 1) * K], order)
        l = logits[t * E:(t + 1) * E].astype(np.float64)
        pe = np.exp(l - l.max()); pe /= pe.sum()
        np.testing.assert_allclose(p, pe, rtol=2e-6, atol=1e-9)
        w = wts[t * K:(t + 1) * K]
        np.testing.assert_allclose(w, p[order] / p[order].sum(), rtol=1e-6)
    assert ids[K] == 3 and ids[K + 1] == 7


@pytest.mark.parametrize("D,F", [(256, 128), (2048, 512)])
def test_expert_vs_dense_dequant(orc, wz, D, F):
    blob = mi.expert_blob(wz, 7, 3, 5, D, F)
    gate, up, down = refmath.blob_dense(blob, D, F)
    x = np.random.default_rng(6).standard_normal(D).astype(np.float32)
    _, _, q16, s16 = quant(orc, x, D, 1)
    aq = np.empty(F, np.int8); as_ = np.empty(F // 16, np.float32); act = np.empty(F, np.float32)
    orc.orc_expert_gate_up(ptr(blob), D, F, ptr(q16), ptr(s16), ptr(aq), ptr(as_), ptr(act))
    xd = refmath.dequant(q16, s16, 16)
    g, u = gate @ xd, up @ xd
    np.testing.assert_allclose(act, g / (1 + np.exp(-g)) * u, rtol=2e-5, atol=1e-5)
    out = np.empty(D, np.float32)
    orc.orc_expert_down(ptr(blob), D, F, ptr(aq), ptr(as_), ptr(out))
    np.testing.assert_allclose(out, down @ refmath.dequant(aq, as_, 16), rtol=1e-5, atol=1e-5)
    # the generated scales are e4m3 roundings of U(0.5,2)*2^-4
    sc = refmath.e4m3_decode(blob[:F * (D // 64 * 36)].reshape(F, D // 64, 36)[:, :, :4])
    assert sc.min() >= 2.0 ** -5 and sc.max() <= 2.0 ** -3


def test_moe_block_composition(orc, wz):
    D, F, E, K, T = 256, 128, 16, 4, 3
    m = mi.make_layer(wz, 9, 2, D, F, E, K)
    x = mi.make_x(wz, 9, 2, T, D).ravel()
    arr = mi.blob_ptr_array(m)
    w = mi.orc_weights(oracle_lib, m, arr)
    comb = np.empty(T * D, np.float32); ids = np.empty(T * K, np.int32); wts = np.empty(T * K, np.float32)
    logits = np.empty(T * E, np.float32); sg = np.empty(T, np.float32)
    assert orc.orc_moe_block(C.byref(w), ptr(x), T, ptr(comb), ptr(ids), ptr(wts), ptr(logits), ptr(sg)) == 0
    # recompute from independent dense formulations
    q32, s32, q16, s16 = quant(orc, x, D, T)
    X = x.reshape(T, D).astype(np.float64)
    np.testing.assert_allclose(logits.reshape(T, E), X @ refmath.bf16_bits_to_f64(m.router).reshape(E, D).T, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(sg, X @ refmath.bf16_bits_to_f64(m.sgate), rtol=1e-5, atol=1e-6)
    Wg = refmath.q8_dense(*m.sh["gate"], F, D); Wu = refmath.q8_dense(*m.sh["up"], F, D)
    Wd = refmath.q8_dense(*m.sh["down"], D, F)
    x32 = refmath.dequant(q32, s32, 32).reshape(T, D)
    x16 = refmath.dequant(q16, s16, 16).reshape(T, D)
    for t in range(T):
        g, u = Wg @ x32[t], Wu @ x32[t]
        a = (g / (1 + np.exp(-g)) * u).astype(np.float32)
        aq, as32, _, _ = quant(orc, a, F, 1)
        shared = Wd @ refmath.dequant(aq, as32, 32)
        acc = shared / (1 + np.exp(-float(sg[t])))
        for k in range(K):
            e = ids[t * K + k]
            gate, up, down = refmath.blob_dense(m.blobs[e], D, F)
            ge, ue = gate @ x16[t], up @ x16[t]
            ae = (ge / (1 + np.exp(-ge)) * ue).astype(np.float32)
            _, _, aq16, as16 = quant(orc, ae, F, 1)
            acc = acc + wts[t * K + k] * (down @ refmath.dequant(aq16, as16, 16))
        np.testing.assert_allclose(comb[t * D:(t + 1) * D], acc, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(wts.reshape(T, K).sum(1), 1.0, rtol=1e-6)


def bf16_round64(a):
    """float32 -> bf16 (round to nearest even) -> float64, through numpy bit operations."""
    u = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return u.view(np.float32).astype(np.float64)


def test_moe_prefill_composition(orc, wz):
    """The prefill oracle against a numpy restatement built from the pinned decoders: bf16 x,
    exact NVFP4 values, Q8_0 weights rounded to bf16, SwiGLU rounded to bf16."""
    D, F, E, K, T = 256, 128, 16, 4, 5
    m = mi.make_layer(wz, 5, 1, D, F, E, K)
    x = mi.make_x(wz, 5, 1, T, D)
    x = (x * 1.37 + 0.01).astype(np.float32)            # not already bf16: the rounding matters
    arr = mi.blob_ptr_array(m)
    w = mi.orc_weights(oracle_lib, m, arr)
    comb = np.empty(T * D, np.float32); ids = np.empty(T * K, np.int32); wts = np.empty(T * K, np.float32)
    assert orc.orc_moe_prefill(C.byref(w), ptr(x.ravel()), T, ptr(comb), ptr(ids), ptr(wts)) == 0
    X = bf16_round64(x)
    logits = (X @ refmath.bf16_bits_to_f64(m.router).reshape(E, D).T).astype(np.float32)
    i2 = np.empty(T * K, np.int32); w2 = np.empty(T * K, np.float32)
    orc.orc_router_topk(ptr(logits.ravel()), E, K, T, ptr(i2), ptr(w2), None)
    np.testing.assert_array_equal(ids, i2)
    np.testing.assert_allclose(wts, w2, rtol=1e-6)
    sg = X @ refmath.bf16_bits_to_f64(m.sgate)
    Wg = bf16_round64(refmath.q8_dense(*m.sh["gate"], F, D)); Wu = bf16_round64(refmath.q8_dense(*m.sh["up"], F, D))
    Wd = bf16_round64(refmath.q8_dense(*m.sh["down"], D, F))
    for t in range(T):
        g, u = Wg @ X[t], Wu @ X[t]
        a = bf16_round64(g / (1 + np.exp(-g)) * u)
        acc = (Wd @ a) / (1 + np.exp(-sg[t]))
        for k in range(K):
            gate, up, down = refmath.blob_dense(m.blobs[ids[t * K + k]], D, F)
            assert np.array_equal(bf16_round64(gate), gate)      # NVFP4 values are exact in bf16
            ge, ue = gate @ X[t], up @ X[t]
            ae = bf16_round64(ge / (1 + np.exp(-ge)) * ue)
            acc = acc + wts[t * K + k] * (down @ ae)
        np.testing.assert_allclose(comb[t * D:(t + 1) * D], acc, rtol=1e-4, atol=1e-4 * np.abs(acc).max())


def test_cpu_pool_matches_oracle_experts(orc, wz):
    D, F, E, K, T = 512, 128, 32, 6, 2
    m = mi.make_layer(wz, 13, 1, D, F, E, K)
    x = mi.make_x(wz, 13, 1, T, D).ravel()
    _, _, q16, s16 = quant(orc, x, D, T)
    rng = np.random.default_rng(8)
    ids = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int32).ravel()
    ids[K] = ids[0]                              # one expert shared by both rows -> a 2-member group
    wts = rng.random(T * K).astype(np.float32)
    ref = np.zeros((T, D))
    for t in range(T):
        for k in range(K):
            aq = np.empty(F, np.int8); as_ = np.empty(F // 16, np.float32); part = np.empty(D, np.float32)
            blob = m.blobs[ids[t * K + k]]
            orc.orc_expert_gate_up(ptr(blob), D, F, ptr(q16[t * D:]), ptr(s16[t * D // 16:]), ptr(aq), ptr(as_), None)
            orc.orc_expert_down(ptr(blob), D, F, ptr(aq), ptr(as_), ptr(part))
            ref[t] += wts[t * K + k] * part
    pool = orc.orc_cpu_pool_create(4, D, F)
    assert pool
    try:
        out = np.empty(T * D, np.float32)
        arr = mi.blob_ptr_array(m)
        assert orc.orc_cpu_pool_run(pool, C.cast(arr, C.c_void_p).value, ptr(ids), ptr(wts), T, K, ptr(q16), ptr(s16), ptr(out)) == 0
    finally:
        orc.orc_cpu_pool_destroy(pool)
    np.testing.assert_allclose(out.reshape(T, D), ref, rtol=2e-2, atol=1e-2)
    assert np.abs(out.reshape(T, D) - ref).max() < 1e-3 * np.abs(ref).max() + 1e-4


def test_row_argmax_top16_vs_numpy(orc):
    rng = np.random.default_rng(9)
    V, T = 5000, 3
    l = rng.standard_normal(T * V).astype(np.float32)
    l[100] = l[200] = 50.0                      # tie at the top of row 0 -> id 100
    l[V + 10:V + 30] = 9.0                      # 20-way tie in row 1 -> ids 10..25
    out = np.empty(T, np.int32)
    orc.orc_row_argmax(ptr(l), V, T, ptr(out))
    g = np.empty(T, np.int32); tv = np.empty(T * 16, np.float32); ti = np.empty(T * 16, np.int32)
    orc.orc_row_top16(ptr(l), V, T, ptr(g), ptr(tv), ptr(ti))
    for t in range(T):
        r = l[t * V:(t + 1) * V]
        order = np.lexsort((np.arange(V), -r))
        assert out[t] == order[0] == g[t]
        np.testing.assert_array_equal(ti[t * 16:(t + 1) * 16], order[:16])
        np.testing.assert_array_equal(tv[t * 16:(t + 1) * 16], r[order[:16]])
    assert out[0] == 100
    np.testing.assert_array_equal(ti[16:32], np.arange(10, 26))

"""GPU parity of the MoE path, the logit reductions and the device-side generator (MI355X)."""
import ctypes as C

import numpy as np
import pytest

import moe_inputs as mi
import oracle_lib
import wzy_amd
from oracle_lib import ptr

pytestmark = pytest.mark.gpu


DA = wzy_amd.DeviceArray


def dev(a):
    return DA.from_numpy(a)


def host(t):
    return t.numpy()


def device_layer(wz, m, planes=None):
    """Upload a MoeLayer; experts come from `planes` (host plane bytes) or the device generator."""
    rec = wz.wzy_nvfp4_expert_bytes(m.D, m.F)
    d = {}
    d["router"] = dev(m.router.view(np.int16))
    d["sgate"] = dev(m.sgate.view(np.int16))
    for k, (q, s) in m.sh.items():
        d[k + "_q"] = dev(q)
        d[k + "_s"] = dev(s.view(np.int16))
    if planes is not None:
        d["experts"] = dev(planes)
    else:
        d["experts"] = DA(rec * m.E, np.uint8)
        wz.wzy_synth_experts_device(m.seed, m.layer, 0, m.E, m.D, m.F, d["experts"].ptr, None)
    w = wzy_amd.MoeWeights()
    w.n_embd, w.n_ff, w.n_exp, w.top_k = m.D, m.F, m.E, m.K
    w.router, w.sgate, w.experts = d["router"].ptr, d["sgate"].ptr, d["experts"].ptr
    w.sh_gate_q, w.sh_gate_s = d["gate_q"].ptr, d["gate_s"].ptr
    w.sh_up_q, w.sh_up_s = d["up_q"].ptr, d["up_s"].ptr
    w.sh_down_q, w.sh_down_s = d["down_q"].ptr, d["down_s"].ptr
    return w, d


def run_gpu_moe(wz, w, x, T):
    D, K = w.n_embd, w.top_k
    xd = dev(x.reshape(T, D))
    comb = DA(T * D, np.float32)
    ids = DA(T * K, np.int32)
    wts = DA(T * K, np.float32)
    nws = wz.wzy_moe_workspace_bytes(D, w.n_ff, w.n_exp, K, T)
    ws = DA(nws, np.uint8, zero=True)
    wz.wzy_moe_block(C.byref(w), xd.ptr, T, comb.ptr, ids.ptr, wts.ptr,
                     ws.ptr, nws, None)
    wz.wzy_device_sync()
    return host(comb), host(ids), host(wts)


def check_ids(orc, logits, E, K, T, ids_gpu, ids_orc):
    """Routed ids bit-exact, except a row whose oracle margin p_K - p_{K+1} is within float noise."""
    probs = np.empty(T * E, np.float32); i2 = np.empty(T * K, np.int32); w2 = np.empty(T * K, np.float32)
    orc.orc_router_topk(ptr(logits), E, K, T, ptr(i2), ptr(w2), ptr(probs))
    exact_rows = 0
    for t in range(T):
        p = np.sort(probs[t * E:(t + 1) * E])[::-1]
        margin = p[K - 1] - p[K] if K < E else 1.0
        if margin > 1e-6 * p[0]:
            assert set(ids_gpu[t * K:(t + 1) * K]) == set(ids_orc[t * K:(t + 1) * K]), t
            np.testing.assert_array_equal(ids_gpu[t * K:(t + 1) * K], ids_orc[t * K:(t + 1) * K])
            exact_rows += 1
    return exact_rows


def test_device_generator_matches_host(wz, gpu):
    D, F = 2048, 512
    rec = wz.wzy_nvfp4_expert_bytes(D, F)
    buf = DA(3 * rec, np.uint8)
    wz.wzy_synth_experts_device(0, 7, 100, 3, D, F, buf.ptr, None)
    got = host(buf)
    for i in range(3):
        ref = np.empty(rec, np.uint8)
        wz.wzy_synth_expert_planes(0, 7, 100 + i, D, F, ref.ctypes.data)
        np.testing.assert_array_equal(got[i * rec:(i + 1) * rec], ref)
    # and the host repack of the reference-layout blob gives the same planes
    blob = mi.expert_blob(wz, 0, 7, 101, D, F)
    rp = np.empty(rec, np.uint8)
    wz.wzy_nvfp4_repack_host(blob.ctypes.data, rp.ctypes.data, D, F)
    np.testing.assert_array_equal(rp, got[rec:2 * rec])
    n, kvd = 1000, 512
    kq = DA(n * kvd, np.int8)
    ks = DA(n * kvd // 64, np.int16)
    wz.wzy_synth_kv_device(2, 3, 1, 4090, n, kvd, kq.ptr, ks.ptr, None)
    hq = np.empty(n * kvd, np.int8); hs = np.empty(n * kvd // 64, np.uint16)
    wz.wzy_synth_kv_host(2, 3, 1, 4090, n, kvd, hq.ctypes.data, hs.ctypes.data)
    np.testing.assert_array_equal(host(kq), hq)
    np.testing.assert_array_equal(host(ks).view(np.uint16), hs)
    assert hq.min() == -127 and hq.max() == 127


@pytest.mark.parametrize("cols,T", [(2048, 1), (512, 8), (320, 3), (8192, 2)])
def test_quant_act_bit_exact(wz, orc, gpu, cols, T):
    x = np.random.default_rng(cols + T).standard_normal(T * cols).astype(np.float32)
    x[:32] = 0.0
    xd = dev(x)
    q32 = DA(T * cols, np.int8); s32 = DA(T * cols // 32, np.float32)
    q16 = DA(T * cols, np.int8); s16 = DA(T * cols // 16, np.float32)
    wz.wzy_quant_act(xd.ptr, q32.ptr, s32.ptr, q16.ptr, s16.ptr, cols, T,
                     None)
    r32 = np.empty(T * cols, np.int8); rs32 = np.empty(T * cols // 32, np.float32)
    r16 = np.empty(T * cols, np.int8); rs16 = np.empty(T * cols // 16, np.float32)
    orc.orc_quant_act(ptr(x), cols, T, ptr(r32), ptr(rs32), ptr(r16), ptr(rs16))
    np.testing.assert_array_equal(host(q32), r32)
    np.testing.assert_array_equal(host(s32), rs32)
    np.testing.assert_array_equal(host(q16), r16)
    np.testing.assert_array_equal(host(s16), rs16)


@pytest.mark.parametrize("rows,cols,T", [(6144, 2048, 1), (2048, 6144, 4), (8192, 320, 8), (2048, 512, 2), (100, 96, 5)])
def test_gemv_q8_parity(wz, orc, gpu, rows, cols, T):
    codes = np.empty(rows * cols, np.int8); sc = np.empty(rows * cols // 32, np.uint16)
    wz.wzy_synth_q8(3, 9, rows, cols, float(1 / np.sqrt(cols)), ptr(codes), ptr(sc))
    x = np.random.default_rng(rows).standard_normal(T * cols).astype(np.float32)
    q32 = np.empty(T * cols, np.int8); s32 = np.empty(T * cols // 32, np.float32)
    orc.orc_quant_act(ptr(x), cols, T, ptr(q32), ptr(s32), None, None)
    ref = np.empty(T * rows, np.float32)
    orc.orc_gemv_q8(ptr(codes), ptr(sc), ptr(q32), ptr(s32), ptr(ref), rows, cols, T)
    y = DA(T * rows, np.float32)
    bufs = [dev(codes), dev(sc.view(np.int16)), dev(q32), dev(s32)]     # keep alive during the call
    wz.wzy_gemv_q8(bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, bufs[3].ptr, y.ptr, rows, cols, T, 0, None)
    np.testing.assert_allclose(host(y), ref, rtol=1e-5, atol=1e-5 * np.abs(ref).max())


@pytest.mark.parametrize("rows,cols,T", [(512, 2048, 1), (151936, 2048, 1), (128, 2048, 8), (4, 8192, 3), (33, 264, 2)])
def test_gemv_bf16_parity(wz, orc, gpu, rows, cols, T):
    W = np.empty(rows * cols, np.uint16)
    wz.wzy_synth_normal_bf16(4, 1, rows * cols, 0.0, 0.02, ptr(W))
    x = np.random.default_rng(cols).standard_normal(T * cols).astype(np.float32)
    y = DA(T * rows, np.float32)
    bufs = [dev(W.view(np.int16)), dev(x)]
    wz.wzy_gemv_bf16(bufs[0].ptr, bufs[1].ptr, y.ptr, rows, cols, T, 0, None)
    ref = np.empty(T * rows, np.float32)
    orc.orc_gemv_bf16(ptr(W), ptr(x), ptr(ref), rows, cols, T)
    np.testing.assert_allclose(host(y), ref, rtol=1e-5, atol=2e-5 * np.abs(ref).max())


@pytest.mark.parametrize("cols,T,kinds", [(2048, 1, "qqbb"), (2048, 1, "qqqbb"), (2048, 4, "qb"), (6144, 1, "q"),
                                           (6144, 3, "bq"), (4096, 2, "qbq"), (8192, 1, "qb"), (8192, 8, "bq"),
                                           (512, 8, "q"), (96, 5, "bqb"), (2048, 1, "b"), (2048, 8, "qqbb")])
def test_gemv_segs_parity(wz, orc, gpu, cols, T, kinds):
    """Projection groups in one launch: every segment against the oracle's Q8_0 / bf16 GEMV."""
    print("case gemv_segs cols=%d T=%d kinds=%s" % (cols, T, kinds), flush=True)
    rng = np.random.default_rng(cols * 10 + T)
    x = rng.standard_normal(T * cols).astype(np.float32)
    x[:32] = 0.0                                          # an all-zero 32-block
    q32 = np.empty(T * cols, np.int8); s32 = np.empty(T * cols // 32, np.float32)
    orc.orc_quant_act(ptr(x), cols, T, ptr(q32), ptr(s32), None, None)
    segs = (wzy_amd.GemvSeg * len(kinds))()
    keep, refs, outs = [dev(x)], [], []
    for i, k in enumerate(kinds):
        rows = int(rng.choice([1, 3, 33, 130, 517, 2048]))
        stride = rows + (i % 2) * 5
        y = DA(T * stride, np.float32, zero=True)
        ref = np.empty(T * rows, np.float32)
        if k == "q":
            codes = np.empty(rows * cols, np.int8); sc = np.empty(rows * cols // 32, np.uint16)
            wz.wzy_synth_q8(5, i, rows, cols, float(1 / np.sqrt(cols)), ptr(codes), ptr(sc))
            orc.orc_gemv_q8(ptr(codes), ptr(sc), ptr(q32), ptr(s32), ptr(ref), rows, cols, T)
            dw, ds = dev(codes), dev(sc.view(np.int16))
            keep += [dw, ds]
            segs[i] = wzy_amd.GemvSeg(dw.ptr, ds.ptr, y.ptr, rows, wzy_amd.GEMV_Q8, stride)
        else:
            W = np.empty(rows * cols, np.uint16)
            wz.wzy_synth_normal_bf16(6, i, rows * cols, 0.0, 0.02, ptr(W))
            orc.orc_gemv_bf16(ptr(W), ptr(x), ptr(ref), rows, cols, T)
            dw = dev(W.view(np.int16))
            keep.append(dw)
            segs[i] = wzy_amd.GemvSeg(dw.ptr, None, y.ptr, rows, wzy_amd.GEMV_BF16, stride)
        refs.append((ref.reshape(T, rows), rows, stride, k))
        outs.append(y)
    assert wz.wzy_gemv_segs(segs, len(kinds), keep[0].ptr, cols, T, None) == 0
    wz.wzy_device_sync()
    for (ref, rows, stride, k), y in zip(refs, outs):
        got = host(y).reshape(T, stride)
        np.testing.assert_allclose(got[:, :rows], ref, rtol=1e-5, atol=2e-5 * max(np.abs(ref).max(), 1e-30))
        assert not got[:, rows:].any(), "wrote outside the segment's rows"


def route_logits(kind, E, T, rng):
    if kind == "gauss":
        return rng.normal(0, 2, (T, E)).astype(np.float32)
    if kind == "levels":                                  # a few values: exact ties broken by id
        return rng.integers(0, 6, (T, E)).astype(np.float32)
    if kind == "top_tie":                                 # 100 experts share the top probability
        l = rng.normal(-5, 1, (T, E)).astype(np.float32)
        for t in range(T):
            l[t, rng.choice(E, min(100, E), replace=False)] = 3.0
        return l
    if kind == "equal":
        return np.full((T, E), 0.5, np.float32)
    if kind == "spread":                                  # probabilities spanning many binades
        return rng.uniform(-60, 10, (T, E)).astype(np.float32)
    raise ValueError(kind)


@pytest.mark.parametrize("kind", ["gauss", "levels", "top_tie", "equal", "spread"])
@pytest.mark.parametrize("E,K,T", [(512, 10, 1), (512, 10, 4), (1024, 32, 2), (64, 8, 3), (16, 10, 1), (512, 1, 8)])
def test_moe_route_patterns(wz, orc, gpu, kind, E, K, T):
    print("case moe_route kind=%s E=%d K=%d T=%d" % (kind, E, K, T), flush=True)
    rng = np.random.default_rng(E * 7 + K * 3 + T + len(kind))
    logits = route_logits(kind, E, T, rng)
    ids, wts = DA(T * K, np.int32, zero=True), DA(T * K, np.float32, zero=True)
    d = dev(logits)
    assert wz.wzy_moe_route(d.ptr, E, K, T, ids.ptr, wts.ptr, None) == 0
    wz.wzy_device_sync()
    gi, gw = host(ids), host(wts)
    oi, ow = np.empty(T * K, np.int32), np.empty(T * K, np.float32)
    orc.orc_router_topk(ptr(logits), E, K, T, ptr(oi), ptr(ow), None)
    if kind in ("levels", "top_tie", "equal"):            # exact ties: equal probabilities on both sides
        np.testing.assert_array_equal(gi, oi)
    else:                                                 # rows whose K-th margin is above float noise
        check_ids(orc, logits.ravel(), E, K, T, gi, oi)
    for t in range(T):
        row = gi[t * K:(t + 1) * K]
        assert len(set(row.tolist())) == K and row.min() >= 0 and row.max() < E
    same = gi == oi
    np.testing.assert_allclose(gw[same], ow[same], rtol=1e-5, atol=1e-7)


def test_moe_config1_parity(wz, orc, gpu):
    """D=2048, 512 experts top-10, NFF=512, seed 0, one token."""
    D, F, E, K, T = 2048, 512, 512, 10, 1
    m = mi.make_layer(wz, 0, 0, D, F, E, K, blobs=[])
    x = mi.make_x(wz, 0, 0, T, D).ravel()
    # oracle routing first, then materialise only the routed experts on the host
    logits = np.empty(T * E, np.float32)
    orc.orc_gemv_bf16(ptr(m.router), ptr(x), ptr(logits), E, D, T)
    ids0 = np.empty(T * K, np.int32); w0 = np.empty(T * K, np.float32)
    orc.orc_router_topk(ptr(logits), E, K, T, ptr(ids0), ptr(w0), None)
    for e in set(ids0.tolist()):
        m.blobs[e] = mi.expert_blob(wz, 0, 0, e, D, F)
    arr = mi.blob_ptr_array(m)
    ow = mi.orc_weights(oracle_lib, m, arr)
    comb_o = np.empty(T * D, np.float32); ids_o = np.empty(T * K, np.int32); wts_o = np.empty(T * K, np.float32)
    assert orc.orc_moe_block(C.byref(ow), ptr(x), T, ptr(comb_o), ptr(ids_o), ptr(wts_o), None, None) == 0
    w, keep = device_layer(wz, m)
    comb, ids, wts = run_gpu_moe(wz, w, x, T)
    assert check_ids(orc, logits, E, K, T, ids, ids_o) == T
    np.testing.assert_allclose(wts, wts_o, rtol=1e-4)
    np.testing.assert_allclose(comb, comb_o, rtol=2e-2, atol=1e-2)
    err = np.abs(comb - comb_o).max() / np.abs(comb_o).max()
    assert err < 2e-3, err


@pytest.mark.parametrize("T", [1, 2, 4, 8])
def test_moe_reference_real_shape(wz, orc, gpu, T):
    """The reference's real MoE shape (NE 2560, NFF 640, 512 experts top-10; src/wzy_kernels_v2.cuh:8-11):
    two 32-column chunks of x per lane and 16-row gate/up tiles.  The routed experts of the window are
    materialised on the host for the oracle; the device generator fills all 512."""
    print("case moe_real_shape T=%d" % T, flush=True)
    D, F, E, K = 2560, 640, 512, 10
    m = mi.make_layer(wz, 3, 2, D, F, E, K, blobs=[])
    x = mi.make_x(wz, 3, 2, T, D).ravel()
    logits = np.empty(T * E, np.float32)
    orc.orc_gemv_bf16(ptr(m.router), ptr(x), ptr(logits), E, D, T)
    ids0 = np.empty(T * K, np.int32); w0 = np.empty(T * K, np.float32)
    orc.orc_router_topk(ptr(logits), E, K, T, ptr(ids0), ptr(w0), None)
    for e in set(ids0.tolist()):
        m.blobs[e] = mi.expert_blob(wz, 3, 2, e, D, F)
    arr = mi.blob_ptr_array(m)
    ow = mi.orc_weights(oracle_lib, m, arr)
    comb_o = np.empty(T * D, np.float32); ids_o = np.empty(T * K, np.int32); wts_o = np.empty(T * K, np.float32)
    assert orc.orc_moe_block(C.byref(ow), ptr(x), T, ptr(comb_o), ptr(ids_o), ptr(wts_o), None, None) == 0
    w, keep = device_layer(wz, m)
    comb, ids, wts = run_gpu_moe(wz, w, x, T)
    assert check_ids(orc, logits, E, K, T, ids, ids_o) == T
    np.testing.assert_allclose(wts, wts_o, rtol=1e-4)
    # elementwise, with the absolute term at 1e-3 of the largest output: a per-16 activation code that
    # rounds the other way (fp32 sums in another order) moves outputs near zero by ~1e-4 of the range
    np.testing.assert_allclose(comb, comb_o, rtol=2e-2, atol=1e-3 * np.abs(comb_o).max())
    err = np.abs(comb - comb_o).max() / np.abs(comb_o).max()
    assert err < 2e-3, err


@pytest.mark.parametrize("T", [1, 2, 4, 8])
def test_moe_multirow_parity(wz, orc, gpu, T):
    """Window rows share experts (grouping path); experts uploaded from host-repacked blobs."""
    D, F, E, K = 512, 128, 16, 4
    m = mi.make_layer(wz, 21, 5, D, F, E, K)
    x = mi.make_x(wz, 21, 5, T, D).ravel()
    rec = wz.wzy_nvfp4_expert_bytes(D, F)
    planes = np.empty(E * rec, np.uint8)
    for e in range(E):
        wz.wzy_nvfp4_repack_host(m.blobs[e].ctypes.data, planes[e * rec:].ctypes.data, D, F)
    arr = mi.blob_ptr_array(m)
    ow = mi.orc_weights(oracle_lib, m, arr)
    comb_o = np.empty(T * D, np.float32); ids_o = np.empty(T * K, np.int32); wts_o = np.empty(T * K, np.float32)
    logits = np.empty(T * E, np.float32)
    assert orc.orc_moe_block(C.byref(ow), ptr(x), T, ptr(comb_o), ptr(ids_o), ptr(wts_o), ptr(logits), None) == 0
    w, keep = device_layer(wz, m, planes=planes)
    comb, ids, wts = run_gpu_moe(wz, w, x, T)
    exact = check_ids(orc, logits, E, K, T, ids, ids_o)
    assert exact >= T - 1
    if exact == T:
        np.testing.assert_allclose(comb, comb_o, rtol=2e-2, atol=1e-2)


@pytest.mark.parametrize("T", [1, 4])
def test_moe_every_scale_code(wz, orc, gpu, T):
    """All 256 e4m3 scale bytes in the gate/up and down scale planes (the sign bit is ignored and
    code 0x7F reads as 480, the reference's unsigned reading; the oracle's decode is pinned on all
    codes against torch): the kernels' hardware fp8 decode of the block scales gives the oracle's
    experts, for the one-row kernels and the multi-row window kernels."""
    print("case moe_every_scale_code T=%d" % T, flush=True)
    D, F, E, K = 512, 128, 16, 4
    m = mi.make_layer(wz, 23, 6, D, F, E, K)
    for e in range(E):
        b = m.blobs[e]
        nb = (b.size - 16) // 36
        blk = b[:nb * 36].reshape(nb, 36)
        blk[:, :4] = ((np.arange(nb * 4) + 37 * e) % 256).astype(np.uint8).reshape(nb, 4)
    x = mi.make_x(wz, 23, 6, T, D).ravel()
    rec = wz.wzy_nvfp4_expert_bytes(D, F)
    planes = np.empty(E * rec, np.uint8)
    for e in range(E):
        wz.wzy_nvfp4_repack_host(m.blobs[e].ctypes.data, planes[e * rec:].ctypes.data, D, F)
    arr = mi.blob_ptr_array(m)
    ow = mi.orc_weights(oracle_lib, m, arr)
    comb_o = np.empty(T * D, np.float32); ids_o = np.empty(T * K, np.int32); wts_o = np.empty(T * K, np.float32)
    logits = np.empty(T * E, np.float32)
    assert orc.orc_moe_block(C.byref(ow), ptr(x), T, ptr(comb_o), ptr(ids_o), ptr(wts_o), ptr(logits), None) == 0
    w, keep = device_layer(wz, m, planes=planes)
    comb, ids, wts = run_gpu_moe(wz, w, x, T)
    assert check_ids(orc, logits, E, K, T, ids, ids_o) == T
    assert np.isfinite(comb).all()
    np.testing.assert_allclose(comb, comb_o, rtol=2e-2, atol=1e-2)


@pytest.mark.parametrize("V,T", [(151936, 1), (151936, 4), (248320, 2), (3000, 8)])
def test_row_argmax_top16_parity(wz, orc, gpu, V, T):
    rng = np.random.default_rng(V + T)
    l = rng.standard_normal(T * V).astype(np.float32)
    l[V // 2] = l[V // 3] = 40.0                # top tie in row 0 -> lower id
    if T > 1:
        l[V + 5:V + 40] = 30.0                  # 35-way tie at the top of row 1
    ld = dev(l)
    g = DA(T, np.int32)
    a = DA(T, np.int32)
    tv = DA(T * 16, np.float32); ti = DA(T * 16, np.int32)
    wz.wzy_row_argmax(ld.ptr, V, T, a.ptr, None)
    wz.wzy_row_top16(ld.ptr, V, T, g.ptr, tv.ptr, ti.ptr, None)
    ra = np.empty(T, np.int32); rg = np.empty(T, np.int32); rv = np.empty(T * 16, np.float32); ri = np.empty(T * 16, np.int32)
    orc.orc_row_argmax(ptr(l), V, T, ptr(ra))
    orc.orc_row_top16(ptr(l), V, T, ptr(rg), ptr(rv), ptr(ri))
    np.testing.assert_array_equal(host(a), ra)
    np.testing.assert_array_equal(host(g), rg)
    np.testing.assert_array_equal(host(ti), ri)
    np.testing.assert_array_equal(host(tv), rv)
    # second call reuses the arrival counters (they must be back at zero)
    wz.wzy_row_argmax(ld.ptr, V, T, a.ptr, None)
    np.testing.assert_array_equal(host(a), ra)


def test_moe_time_kernels_bursts(wz, gpu):
    """The measurement entry point reports positive, plausible durations and leaves the block
    usable: the MoE block gives bit-identical results before and after it."""
    D, F, E, K, T = 512, 128, 16, 4, 1
    layers, keep = [], []
    for l in range(3):
        m = mi.make_layer(wz, 5, l, D, F, E, K, blobs=[])
        w, d = device_layer(wz, m)
        layers.append(w)
        keep.append(d)
    arr = (wzy_amd.MoeWeights * 3)(*layers)
    x = mi.make_x(wz, 5, 0, T, D).ravel()
    before = run_gpu_moe(wz, layers[0], x, T)
    xd = dev(x)
    nws = wz.wzy_moe_workspace_bytes(D, F, E, K, T)
    ws = DA(nws, np.uint8, zero=True)
    gu, dn, bl = C.c_float(0), C.c_float(0), C.c_float(0)
    wz.wzy_moe_time_kernels(arr, 3, T, xd.ptr, ws.ptr, nws, 12, C.byref(gu), C.byref(dn), C.byref(bl), None)
    assert 0.5 < gu.value < 1000 and 0.5 < dn.value < 1000 and 1.0 < bl.value < 2000, (gu.value, dn.value, bl.value)
    after = run_gpu_moe(wz, layers[0], x, T)
    for a, b in zip(before, after):
        assert np.array_equal(a, b)


def run_gpu_prefill(wz, w, x, N):
    D, K = w.n_embd, w.top_k
    xd = dev(x.reshape(N, D))
    comb = DA(N * D, np.float32)
    ids = DA(N * K, np.int32)
    wts = DA(N * K, np.float32)
    nws = wz.wzy_moe_prefill_workspace_bytes(D, w.n_ff, w.n_exp, K, N)
    ws = DA(nws, np.uint8)
    wz.wzy_moe_prefill(C.byref(w), xd.ptr, N, comb.ptr, ids.ptr, wts.ptr, ws.ptr, nws, None)
    wz.wzy_device_sync()
    return host(comb), host(ids), host(wts)


def prefill_logits(m, x):
    """Router logits of bf16-rounded rows (the prefill path's A operand), fp64 sums."""
    X = bf16_round64(x.reshape(-1, m.D))
    R = (m.router.astype(np.uint32) << 16).view(np.float32).astype(np.float64).reshape(m.E, m.D)
    return (X @ R.T).astype(np.float32)


def assert_prefill_close(g, o, D, rtol=2e-2, atol=1e-2, max_frac=1e-4):
    """Prefill block outputs against the oracle, rows of D values.  Elementwise |g - o| <= atol +
    rtol * |o|, except where the two round a SwiGLU activation that sits on a bf16 rounding tie in
    opposite directions (their fp32 sums differ in order): that moves the token's outputs by one bf16
    ulp of the activation times its down column, which can exceed the elementwise bound on the
    token's small outputs.  Such elements must be fewer than max_frac (1 in 10^4) and within atol +
    rtol * max |o| over their token row."""
    g = np.asarray(g, np.float64).reshape(-1, D)
    o = np.asarray(o, np.float64).reshape(-1, D)
    d = np.abs(g - o)
    out = d > atol + rtol * np.abs(o)
    n_out = int(out.sum())
    assert n_out <= int(d.size * max_frac), "%d of %d outside the elementwise tolerance" % (n_out, d.size)
    row_bound = atol + rtol * np.abs(o).max(axis=1, keepdims=True)
    assert (d <= row_bound).all(), "max error %.3g above the row bound" % (d - row_bound).max()


def bf16_round64(a):
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16
    return u.astype(np.uint32).view(np.float32).astype(np.float64)


@pytest.mark.parametrize("D,F,E,K,N", [
    (256, 128, 64, 4, 1),          # one token, one partial row tile
    (256, 128, 64, 4, 130),        # ragged: 3 row tiles, the last of 2 rows
    (256, 128, 64, 8, 600),
    (256, 128, 64, 8, 1100),       # ~137 entries per expert: one partly filled 256-entry tile each
    (256, 128, 64, 8, 2100),       # ~262 entries per expert: about half span two 256-entry tiles
    (512, 256, 128, 6, 77),
    (256, 128, 64, 12, 300),       # K = 12: a full 8-slot combine pass, then a predicated one
    (256, 128, 128, 8, 1000),      # 16 router A tiles (XCD-grouped router blocks), the last of 40 rows
    (256, 128, 1024, 8, 192),      # 1024 experts: the 16-key routing variant, most experts with 1-3 entries
])
def test_moe_prefill_parity(wz, orc, gpu, D, F, E, K, N):
    """Chunked-prefill MoE block (MFMA, NVFP4 -> bf16) against the bf16 prefill oracle."""
    print(f"prefill D={D} F={F} E={E} K={K} N={N}", flush=True)
    m = mi.make_layer(wz, 31, 2, D, F, E, K)
    x = (mi.make_x(wz, 31, 2, N, D) * 1.37 + 0.01).astype(np.float32)     # not bf16 already
    arr = mi.blob_ptr_array(m)
    ow = mi.orc_weights(oracle_lib, m, arr)
    comb_o = np.empty(N * D, np.float32); ids_o = np.empty(N * K, np.int32); wts_o = np.empty(N * K, np.float32)
    assert orc.orc_moe_prefill(C.byref(ow), ptr(x.ravel()), N, ptr(comb_o), ptr(ids_o), ptr(wts_o)) == 0
    w, keep = device_layer(wz, m)
    comb, ids, wts = run_gpu_prefill(wz, w, x, N)
    logits = prefill_logits(m, x).ravel()
    exact = check_ids(orc, logits, E, K, N, ids, ids_o)
    assert exact >= N - max(1, N // 50), (exact, N)
    if N * K > 256 * E:                 # the case meant to split experts over two tiles does so
        assert np.bincount(ids_o, minlength=E).max() > 256
    rows = np.array([np.array_equal(ids[t * K:(t + 1) * K], ids_o[t * K:(t + 1) * K]) for t in range(N)])
    wr = np.repeat(rows, K)
    np.testing.assert_allclose(wts[wr], wts_o[wr], rtol=1e-4, atol=1e-6)
    cr = np.repeat(rows, D)
    assert_prefill_close(comb[cr], comb_o[cr], D)
    err = np.abs(comb[cr] - comb_o[cr]).max() / np.abs(comb_o[cr]).max()
    assert err < 3e-3, err
    # a second call on the same workspace (counts, tiles and lists rebuilt, comb re-initialised):
    # entries may reach their expert in another order, the results may not change
    c2, i2, w2 = run_gpu_prefill(wz, w, x, N)
    np.testing.assert_array_equal(i2, ids)
    np.testing.assert_array_equal(w2, wts)
    np.testing.assert_array_equal(c2, comb)


def test_moe_prefill_config1_shape(wz, orc, gpu):
    """The BASELINE layer shape (D=2048, 512 experts top-10, NFF=512) on an 8-token chunk."""
    D, F, E, K, N = 2048, 512, 512, 10, 8
    print(f"prefill config1 shape N={N}", flush=True)
    m = mi.make_layer(wz, 0, 3, D, F, E, K, blobs=[])
    x = mi.make_x(wz, 0, 3, N, D)
    logits = prefill_logits(m, x)
    need = set()
    for t in range(N):
        need.update(np.argsort(-logits[t], kind="stable")[:K + 4].tolist())
    for e in need:
        m.blobs[e] = mi.expert_blob(wz, 0, 3, e, D, F)
    arr = mi.blob_ptr_array(m)
    ow = mi.orc_weights(oracle_lib, m, arr)
    comb_o = np.empty(N * D, np.float32); ids_o = np.empty(N * K, np.int32); wts_o = np.empty(N * K, np.float32)
    assert orc.orc_moe_prefill(C.byref(ow), ptr(x.ravel()), N, ptr(comb_o), ptr(ids_o), ptr(wts_o)) == 0
    w, keep = device_layer(wz, m)
    comb, ids, wts = run_gpu_prefill(wz, w, x, N)
    assert check_ids(orc, logits.ravel(), E, K, N, ids, ids_o) == N
    np.testing.assert_allclose(wts, wts_o, rtol=1e-4)
    np.testing.assert_allclose(comb, comb_o, rtol=2e-2, atol=1e-2)
    err = np.abs(comb - comb_o).max() / np.abs(comb_o).max()
    assert err < 3e-3, err


def test_moe_prefill_rejects_bad_shapes(wz, gpu):
    D, F, E, K = 256, 128, 48, 4                  # 48 experts: not a multiple of 64
    m = mi.make_layer(wz, 1, 0, D, F, 64, K, blobs=[])
    w, keep = device_layer(wz, m)
    w.n_exp = E
    x = dev(np.zeros((2, D), np.float32))
    out = DA(2 * D, np.float32)
    nws = wz.wzy_moe_prefill_workspace_bytes(D, F, 64, K, 2)
    ws = DA(nws, np.uint8)
    with pytest.raises(wzy_amd.WzyError):
        wz.wzy_moe_prefill(C.byref(w), x.ptr, 2, out.ptr, None, None, ws.ptr, nws, None)
    w.n_exp = 64
    with pytest.raises(wzy_amd.WzyError):
        wz.wzy_moe_prefill(C.byref(w), x.ptr, 2, out.ptr, None, None, ws.ptr, 16, None)
    with pytest.raises(wzy_amd.WzyError):                            # an empty chunk
        wz.wzy_moe_prefill(C.byref(w), x.ptr, 0, out.ptr, None, None, ws.ptr, nws, None)
    w.top_k = 33                                                     # above the 32-slot maximum
    with pytest.raises(wzy_amd.WzyError):
        wz.wzy_moe_prefill(C.byref(w), x.ptr, 2, out.ptr, None, None, ws.ptr, nws, None)
    w.top_k = K


def test_moe_prefill_tensor_scales(wz, orc, gpu):
    """Non-unit fp32 tensor scales (gate, up, down): the oracle folds them into the dequantised
    weights (the reference's order), the MFMA path scales the fp32 accumulators."""
    D, F, E, K, N = 256, 128, 64, 4, 96
    m = mi.make_layer(wz, 8, 1, D, F, E, K)
    tails = np.array([0.37, 1.9, 0.61, 0.0], np.float32)
    rec = wz.wzy_nvfp4_expert_bytes(D, F)
    planes = np.empty(E * rec, np.uint8)
    for e in range(E):
        m.blobs[e][-16:] = (tails * (1.0 + 0.01 * e)).astype(np.float32).view(np.uint8)
        wz.wzy_nvfp4_repack_host(m.blobs[e].ctypes.data, planes[e * rec:].ctypes.data, D, F)
    x = mi.make_x(wz, 8, 1, N, D)
    arr = mi.blob_ptr_array(m)
    ow = mi.orc_weights(oracle_lib, m, arr)
    comb_o = np.empty(N * D, np.float32); ids_o = np.empty(N * K, np.int32); wts_o = np.empty(N * K, np.float32)
    assert orc.orc_moe_prefill(C.byref(ow), ptr(x.ravel()), N, ptr(comb_o), ptr(ids_o), ptr(wts_o)) == 0
    w, keep = device_layer(wz, m, planes=planes)
    comb, ids, wts = run_gpu_prefill(wz, w, x, N)
    logits = prefill_logits(m, x).ravel()
    assert check_ids(orc, logits, E, K, N, ids, ids_o) >= N - 1
    rows = np.array([np.array_equal(ids[t * K:(t + 1) * K], ids_o[t * K:(t + 1) * K]) for t in range(N)])
    cr = np.repeat(rows, D)
    assert_prefill_close(comb[cr], comb_o[cr], D)
    err = np.abs(comb[cr] - comb_o[cr]).max() / np.abs(comb_o[cr]).max()
    assert err < 3e-3, err


def test_moe_prefill_time_entry(wz, gpu):
    """The measurement entry point reports a positive time for every launch group and leaves the
    same (bit-identical) block output as a plain call."""
    D, F, E, K, N = 256, 128, 64, 4, 300
    m = mi.make_layer(wz, 6, 0, D, F, E, K, blobs=[])
    w, keep = device_layer(wz, m)
    x = mi.make_x(wz, 6, 0, N, D)
    comb0, ids0, _ = run_gpu_prefill(wz, w, x, N)
    xd = dev(x)
    comb = DA(N * D, np.float32)
    nws = wz.wzy_moe_prefill_workspace_bytes(D, F, E, K, N)
    ws = DA(nws, np.uint8)
    us = (C.c_float * 8)()
    wz.wzy_moe_prefill_time(C.byref(w), xd.ptr, N, comb.ptr, ws.ptr, nws, 3, us, None)
    wz.wzy_device_sync()
    assert all(0.0 < us[i] < 1e5 for i in range(8)), list(us)
    np.testing.assert_array_equal(host(comb), comb0)


def test_moe_prefill_full_chunk_rows(wz, orc, gpu):
    """BASELINE config 5 at full size: one 8,192-token chunk through the BASELINE layer.  A token's
    output depends on its own row only (tiles mix tokens, sums do not), so sampled rows equal, bit for
    bit, the same rows run as a chunk of their own; and those rows match the oracle."""
    D, F, E, K, N = 2048, 512, 512, 10, 8192
    print(f"prefill full chunk N={N}", flush=True)
    m = mi.make_layer(wz, 4, 2, D, F, E, K, blobs=[])
    w, keep = device_layer(wz, m)
    x = np.random.default_rng(11).standard_normal((N, D)).astype(np.float32)
    comb, ids, wts = run_gpu_prefill(wz, w, x, N)
    pick = np.array([0, 1, 777, 4096, 5000, N - 2, N - 1])
    c2, i2, w2 = run_gpu_prefill(wz, w, x[pick], len(pick))
    np.testing.assert_array_equal(i2.reshape(-1, K), ids.reshape(N, K)[pick])
    np.testing.assert_array_equal(w2.reshape(-1, K), wts.reshape(N, K)[pick])
    np.testing.assert_array_equal(c2.reshape(-1, D), comb.reshape(N, D)[pick])
    # oracle on the sampled rows (their routed experts materialised on the host)
    xs = np.ascontiguousarray(x[pick])
    logits = prefill_logits(m, xs)
    for t in range(len(pick)):
        for e in np.argsort(-logits[t], kind="stable")[:K + 4].tolist():
            if e not in m.blobs:
                m.blobs[e] = mi.expert_blob(wz, 4, 2, e, D, F)
    arr = mi.blob_ptr_array(m)
    ow = mi.orc_weights(oracle_lib, m, arr)
    T = len(pick)
    comb_o = np.empty(T * D, np.float32); ids_o = np.empty(T * K, np.int32); wts_o = np.empty(T * K, np.float32)
    assert orc.orc_moe_prefill(C.byref(ow), ptr(xs.ravel()), T, ptr(comb_o), ptr(ids_o), ptr(wts_o)) == 0
    assert check_ids(orc, logits.ravel(), E, K, T, i2, ids_o) == T
    np.testing.assert_allclose(c2, comb_o, rtol=2e-2, atol=1e-2)
    err = np.abs(c2 - comb_o).max() / np.abs(comb_o).max()
    assert err < 3e-3, err

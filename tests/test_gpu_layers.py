"""GPU parity of the per-layer kernels against the CPU oracle: hyper-connection read, GDN step and
recurrence, QSA prepare / select / attend (MI355X; C ABI only, no torch)."""
import ctypes as C

import numpy as np
import pytest

import oracle_lib
import wzy_amd
from oracle_lib import ptr
from stage_oracle import attend, attn_f16, check_attention_branch

pytestmark = pytest.mark.gpu

DA = wzy_amd.DeviceArray
RTOL, ATOL = 2e-2, 1e-2          # float tolerance of the decode path


def dev(a):
    return DA.from_numpy(a)


def close(name, got, ref, rtol=RTOL, atol=ATOL):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    bad = err > atol + rtol * np.abs(ref)
    print("%s: max abs err %.3g (ref max %.3g)" % (name, err.max() if err.size else 0, np.abs(ref).max() if ref.size else 0))
    assert not bad.any(), "%s: %d / %d outside tolerance, worst at %s (%r vs %r)" % (
        name, bad.sum(), bad.size, np.unravel_index(np.argmax(err), err.shape), got.flat[np.argmax(err)],
        ref.flat[np.argmax(err)])


def bf16(a):
    a = np.ascontiguousarray(a, np.float32)
    u = a.view(np.uint32)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r


def bf16_to_f32(h):
    return (h.astype(np.uint32) << 16).view(np.float32)


def q8(wz, seed, rows, cols):
    q = np.empty(rows * cols, np.int8)
    s = np.empty(rows * cols // 32, np.uint16)
    wz.wzy_synth_q8(seed, 0x5151, rows, cols, 1.0 / np.sqrt(cols), q.ctypes.data, s.ctypes.data)
    return q, s


# ------------------------------------------------------------------------------------------------
# hyper-connection read
# ------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("D,HC,HCLR,T,mode", [(512, 4, 64, 3, "emb"), (512, 4, 64, 3, "fold"), (512, 4, 64, 2, "head"),
                                             (2048, 4, 320, 1, "fold"), (2048, 4, 320, 4, "emb"),
                                             (2048, 4, 320, 8, "fold"), (4096, 4, 128, 3, "fold"),
                                             (256, 4, 32, 6, "head"), (2560, 4, 320, 1, "fold"),
                                             (2560, 4, 320, 4, "emb"), (2560, 4, 320, 2, "head"),
                                             (768, 4, 64, 3, "fold"), (5120, 4, 96, 1, "fold")])
def test_hc_read(wz, orc, gpu, D, HC, HCLR, T, mode):
    print("case hc_read D=%d HC=%d HCLR=%d T=%d mode=%s" % (D, HC, HCLR, T, mode), flush=True)
    rng = np.random.default_rng(D + 7 * T)
    HCD = HC * D
    V = 97
    norm_w = rng.normal(1.0, 0.02, HCD).astype(np.float32)
    dq, ds = q8(wz, 11, HCLR, HCD)
    uq, us = q8(wz, 12, HCD, HCLR)
    inj_w = bf16(rng.normal(0, 1 / np.sqrt(HCD), (HC, HCD))) if mode != "head" else None
    emb = bf16(rng.normal(0, 1, (V, D)))
    toks = rng.integers(0, V, T).astype(np.int32)
    R_in = rng.normal(0, 1, (T, HC, D)).astype(np.float32)
    bo = rng.normal(0, 1, (T, D)).astype(np.float32)
    inj_prev = rng.normal(0, 1, (T, HC)).astype(np.float32)

    d = {k: dev(v) for k, v in dict(norm_w=norm_w, dq=dq, ds=ds, uq=uq, us=us, emb=emb, toks=toks, R_in=R_in, bo=bo,
                                     inj_prev=inj_prev).items()}
    if inj_w is not None:
        d["inj_w"] = dev(inj_w)
    R_out, nsc, lo = DA((T, HC, D), np.float32), DA((T, HC), np.float32), DA((T, HCLR), np.float32)
    inj, mixed = DA((T, HC), np.float32), DA((T, D), np.float32)
    nws = wz.wzy_hc_read_workspace_bytes(HC, HCLR, T)
    ws = DA(nws, np.uint8)
    emb_mode = mode == "emb"
    wz.wzy_hc_read(None if emb_mode else d["R_in"].ptr, d["emb"].ptr if emb_mode else None,
                   d["toks"].ptr if emb_mode else None, V, None if emb_mode else d["bo"].ptr,
                   None if emb_mode else d["inj_prev"].ptr, R_out.ptr, d["norm_w"].ptr, d["dq"].ptr, d["ds"].ptr,
                   d["inj_w"].ptr if inj_w is not None else None, d["uq"].ptr, d["us"].ptr, nsc.ptr, lo.ptr,
                   inj.ptr if inj_w is not None else None, mixed.ptr, D, HC, HCLR, C.c_float(1e-6), T, ws.ptr, nws,
                   None)
    wz.wzy_device_sync()

    o_R, o_nsc, o_lo = np.empty((T, HC, D), np.float32), np.empty((T, HC), np.float32), np.empty((T, HCLR), np.float32)
    o_inj, o_mixed = np.zeros((T, HC), np.float32), np.empty((T, D), np.float32)
    emb_rows = bf16_to_f32(emb[toks]).astype(np.float32)
    orc.orc_hc_read(None if emb_mode else ptr(R_in), ptr(emb_rows) if emb_mode else None,
                    None if emb_mode else ptr(bo), None if emb_mode else ptr(inj_prev), ptr(norm_w), ptr(dq), ptr(ds),
                    ptr(inj_w) if inj_w is not None else None, ptr(uq), ptr(us), D, HC, HCLR, 1e-6, T, ptr(o_R),
                    ptr(o_nsc), ptr(o_lo), ptr(o_inj), ptr(o_mixed))
    close("R_out", R_out.numpy(), o_R, 1e-5, 1e-5)
    close("nsc", nsc.numpy(), o_nsc, 1e-5, 1e-7)
    close("lo", lo.numpy(), o_lo)
    close("mixed", mixed.numpy(), o_mixed)
    if inj_w is not None:
        close("inj", inj.numpy(), o_inj, 1e-4, 1e-5)


# ------------------------------------------------------------------------------------------------
# GDN
# ------------------------------------------------------------------------------------------------
def gdn_inputs(hk, hv, T, seed):
    rng = np.random.default_rng(seed)
    QKV, GV = 2 * hk * 128 + hv * 128, hv * 128
    return dict(
        qkv=rng.normal(0, 1, (T, QKV)).astype(np.float32),
        z=rng.normal(0, 1, (T, GV)).astype(np.float32),
        ab=rng.normal(0, 1, (T, 2 * hv)).astype(np.float32),
        dt=rng.normal(-3, 0.5, hv).astype(np.float32),
        ssm_a=rng.uniform(-2, -1, hv).astype(np.float32),
        conv_w=rng.normal(0, 0.5, (QKV, 4)).astype(np.float32),
        hist=rng.normal(0, 1, (QKV, 3)).astype(np.float32),
        state=rng.normal(0, 0.1, (hv, 128, 128)).astype(np.float32),
        gamma=rng.normal(1, 0.02, 128).astype(np.float32),
    )


@pytest.mark.parametrize("hk,hv,T", [(2, 2, 1), (2, 4, 3), (16, 16, 1), (16, 16, 4), (4, 8, 8), (16, 48, 1),
                                     (16, 48, 4)])
def test_gdn_step(wz, orc, gpu, hk, hv, T):
    print("case gdn_step hk=%d hv=%d T=%d" % (hk, hv, T), flush=True)
    a = gdn_inputs(hk, hv, T, 100 * hk + hv + T)
    QKV, GV = a["qkv"].shape[1], a["z"].shape[1]
    d = {k: dev(v) for k, v in a.items()}
    y = DA((T, GV), np.float32)
    ssnap = DA((T, hv, 128, 128), np.float32)
    hsnap = DA((T, QKV, 3), np.float32)
    wz.wzy_gdn_step(d["qkv"].ptr, d["z"].ptr, d["ab"].ptr, d["dt"].ptr, d["ssm_a"].ptr, d["conv_w"].ptr,
                    d["hist"].ptr, d["state"].ptr, d["gamma"].ptr, C.c_float(1e-6), y.ptr, hk, hv, T, ssnap.ptr,
                    hsnap.ptr, None)
    wz.wzy_device_sync()
    # oracle row by row, recording the per-row states the snapshots must hold
    hist, state = a["hist"].copy(), a["state"].copy()
    oy = np.empty((T, GV), np.float32)
    osn, ohn = [], []
    for t in range(T):
        orc.orc_gdn_step(ptr(a["qkv"][t:t + 1]), ptr(a["z"][t:t + 1]), ptr(a["ab"][t:t + 1]), ptr(a["dt"]),
                         ptr(a["ssm_a"]), ptr(a["conv_w"]), ptr(hist), ptr(state), ptr(a["gamma"]), 1e-6,
                         ptr(oy[t:t + 1]), hk, hv, 1)
        osn.append(state.copy())
        ohn.append(hist.copy())
    close("y", y.numpy(), oy)
    close("state", d["state"].numpy(), state, 1e-3, 1e-5)
    close("conv_hist", d["hist"].numpy(), hist, 0, 0)
    sn, hn = ssnap.numpy(), hsnap.numpy()
    for t in range(T):
        close("state_snap[%d]" % t, sn[t], osn[t], 1e-3, 1e-5)
        close("hist_snap[%d]" % t, hn[t], ohn[t], 0, 0)


@pytest.mark.parametrize("hk,hv", [(16, 16), (16, 48)])
def test_gdn_step_launch_forms_agree(wz, gpu, hk, hv):
    """Windows of up to three rows run a head in one workgroup with the output norm in the kernel;
    longer ones use four column-quarter workgroups and the norm kernel.  Both forms compute every
    row alike: four single steps equal one four-row window bit for bit (outputs, state, history)."""
    print("case gdn_step forms hk=%d hv=%d" % (hk, hv), flush=True)
    T = 4
    a = gdn_inputs(hk, hv, T, 7 * hk + hv)
    QKV, GV = a["qkv"].shape[1], a["z"].shape[1]
    win = {k: dev(v) for k, v in a.items()}
    y4 = DA((T, GV), np.float32)
    wz.wzy_gdn_step(win["qkv"].ptr, win["z"].ptr, win["ab"].ptr, win["dt"].ptr, win["ssm_a"].ptr,
                    win["conv_w"].ptr, win["hist"].ptr, win["state"].ptr, win["gamma"].ptr, C.c_float(1e-6),
                    y4.ptr, hk, hv, T, None, None, None)
    one = {k: dev(v) for k, v in a.items() if k in ("dt", "ssm_a", "conv_w", "hist", "state", "gamma")}
    y1 = np.empty((T, GV), np.float32)
    for t in range(T):
        qkv, z, ab = dev(a["qkv"][t:t + 1]), dev(a["z"][t:t + 1]), dev(a["ab"][t:t + 1])
        yt = DA((1, GV), np.float32)
        wz.wzy_gdn_step(qkv.ptr, z.ptr, ab.ptr, one["dt"].ptr, one["ssm_a"].ptr, one["conv_w"].ptr,
                        one["hist"].ptr, one["state"].ptr, one["gamma"].ptr, C.c_float(1e-6), yt.ptr, hk, hv, 1,
                        None, None, None)
        wz.wzy_device_sync()
        y1[t] = yt.numpy()[0]
    wz.wzy_device_sync()
    np.testing.assert_array_equal(y1, y4.numpy())
    np.testing.assert_array_equal(one["state"].numpy(), win["state"].numpy())
    np.testing.assert_array_equal(one["hist"].numpy(), win["hist"].numpy())


@pytest.mark.parametrize("hk,hv,T", [(2, 4, 2), (16, 16, 1)])
def test_gdn_recurrence(wz, orc, gpu, hk, hv, T):
    print("case gdn_recurrence hk=%d hv=%d T=%d" % (hk, hv, T), flush=True)
    rng = np.random.default_rng(hk * hv + T)

    def unit(n):
        x = rng.normal(0, 1, (T, n, 128)).astype(np.float32)
        return (x / np.linalg.norm(x, axis=-1, keepdims=True)).astype(np.float32)

    q, k = unit(hk), unit(hk)
    v = rng.normal(0, 1, (T, hv, 128)).astype(np.float32)
    decay = rng.uniform(0.5, 1.0, (T, hv)).astype(np.float32)
    beta = rng.uniform(0.0, 1.0, (T, hv)).astype(np.float32)
    state = rng.normal(0, 0.1, (hv, 128, 128)).astype(np.float32)
    d = {n: dev(x) for n, x in dict(q=q, k=k, v=v, decay=decay, beta=beta, state=state).items()}
    y = DA((T, hv, 128), np.float32)
    wz.wzy_gdn_recurrence(d["q"].ptr, d["k"].ptr, d["v"].ptr, d["decay"].ptr, d["beta"].ptr, None, None,
                          C.c_float(1e-6), d["state"].ptr, y.ptr, hk, hv, T, None, None)
    wz.wzy_device_sync()
    oy = np.empty((T, hv, 128), np.float32)
    st = state.copy()
    orc.orc_gdn_recurrence(ptr(q), ptr(k), ptr(v), ptr(decay), ptr(beta), None, None, 1e-6, ptr(st), ptr(oy), hk, hv, T)
    close("y", y.numpy(), oy)
    close("state", d["state"].numpy(), st, 1e-3, 1e-5)


# ------------------------------------------------------------------------------------------------
# QSA
# ------------------------------------------------------------------------------------------------
def qsa_dims(ctx_max=1024, topk=64, qh=4, kvh=2):
    dm = wzy_amd.QsaDims()
    dm.qh, dm.kvh, dm.hd, dm.n_rot = qh, kvh, 256, 64
    dm.idx_heads, dm.idx_dim, dm.idx_blk, dm.idx_topk = 4, 128, 4, topk
    dm.ctx_max, dm.kv_ring, dm.kv_sinks, dm.eps = ctx_max, 0, 0, 1e-6
    return dm


def rope(orc, ctx, n_rot=64):
    c = np.empty((ctx, n_rot // 2), np.float32)
    s = np.empty((ctx, n_rot // 2), np.float32)
    orc.orc_rope_tables(ctx, n_rot, 1e7, ptr(c), ptr(s))
    return c, s


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


@pytest.mark.parametrize("pos,T", [(600, 3), (605, 4), (0, 2), (1, 1), (1019, 4)])
def test_qsa_prepare(wz, orc, gpu, pos, T):
    print("case qsa_prepare pos=%d T=%d" % (pos, T), flush=True)
    dm = qsa_dims()
    rng = np.random.default_rng(pos * 10 + T)
    qh, kvh, hd, ih, idim, blk, ctx = dm.qh, dm.kvh, dm.hd, dm.idx_heads, dm.idx_dim, dm.idx_blk, dm.ctx_max
    KVD, max_b = kvh * hd, ctx // blk + 2
    cos_t, sin_t = rope(orc, ctx)
    a = dict(
        qg=rng.normal(0, 1, (T, qh * 2 * hd)).astype(np.float32),
        kk=rng.normal(0, 1, (T, KVD)).astype(np.float32),
        vv=rng.normal(0, 1, (T, KVD)).astype(np.float32),
        q_idx=rng.normal(0, 1, (T, ih * idim)).astype(np.float32),
        idx_raw=rng.normal(0, 1, (T, idim)).astype(np.float32),
        q_norm=rng.normal(1, 0.02, hd).astype(np.float32),
        k_norm=rng.normal(1, 0.02, hd).astype(np.float32),
        iq_norm=rng.normal(1, 0.02, idim).astype(np.float32),
        ik_norm=rng.normal(1, 0.02, idim).astype(np.float32),
        kq=np.zeros((ctx, KVD), np.int8), ks=np.zeros((ctx, KVD // 64), np.uint16),
        vq=np.zeros((ctx, KVD), np.int8), vs=np.zeros((ctx, KVD // 64), np.uint16),
        tail=rng.normal(0, 1, (blk - 1, idim)).astype(np.float32),
        dead=rng.normal(0, 1, idim).astype(np.float32),
        pooled=f16(rng.normal(0, 1, (max_b, idim))),
        cos=cos_t, sin=sin_t, pos=np.array([pos], np.int32),
    )
    d = {k: dev(v) for k, v in a.items()}
    wz.wzy_qsa_prepare(C.byref(dm), d["pos"].ptr, d["qg"].ptr, d["kk"].ptr, d["vv"].ptr, d["q_idx"].ptr,
                       d["idx_raw"].ptr, d["q_norm"].ptr, d["k_norm"].ptr, d["iq_norm"].ptr, d["ik_norm"].ptr,
                       d["cos"].ptr, d["sin"].ptr, d["kq"].ptr, d["ks"].ptr, d["vq"].ptr, d["vs"].ptr, d["tail"].ptr,
                       d["dead"].ptr, d["pooled"].ptr, T, None)
    wz.wzy_device_sync()
    o = {k: v.copy() for k, v in a.items()}
    for t in range(T):
        p = pos + t
        for h in range(qh):
            orc.orc_head_norm_rope(ptr(o["qg"][t, h * 2 * hd:]), hd, ptr(o["q_norm"]), ptr(cos_t), ptr(sin_t), p, 64, 1e-6)
        for j in range(kvh):
            orc.orc_head_norm_rope(ptr(o["kk"][t, j * hd:]), hd, ptr(o["k_norm"]), ptr(cos_t), ptr(sin_t), p, 64, 1e-6)
        for i in range(ih):
            orc.orc_head_norm_rope(ptr(o["q_idx"][t, i * idim:]), idim, ptr(o["iq_norm"]), ptr(cos_t), ptr(sin_t), p, 64,
                                   1e-6)
        orc.orc_kv_quant_row(ptr(o["kk"][t]), KVD, ptr(o["kq"][p]), ptr(o["ks"][p]))
        orc.orc_kv_quant_row(ptr(o["vv"][t]), KVD, ptr(o["vq"][p]), ptr(o["vs"][p]))
        orc.orc_indexer_append(ptr(o["idx_raw"][t]), ptr(o["ik_norm"]), ptr(cos_t), ptr(sin_t), p, idim, blk, 64, 1e-6,
                               ptr(o["tail"]), ptr(o["dead"]), ptr(o["pooled"]))
    for k in ("qg", "kk", "q_idx"):
        close(k, d[k].numpy(), o[k], 1e-5, 1e-5)
    rows = slice(pos, pos + T)
    # KV quantisation is byte work: v is quantised from the same floats on both sides, so its codes and
    # scales must be identical; k is normalised and roped first, and quantising the GPU's own roped k
    # (returned in place) must reproduce the GPU's bytes exactly
    np.testing.assert_array_equal(d["vq"].numpy()[rows], o["vq"][rows])
    np.testing.assert_array_equal(d["vs"].numpy()[rows], o["vs"][rows])
    gk = d["kk"].numpy()
    kq_own = np.zeros((T, KVD), np.int8)
    ks_own = np.zeros((T, KVD // 64), np.uint16)
    for t in range(T):
        orc.orc_kv_quant_row(ptr(np.ascontiguousarray(gk[t])), KVD, ptr(kq_own[t]), ptr(ks_own[t]))
    np.testing.assert_array_equal(d["kq"].numpy()[rows], kq_own)
    np.testing.assert_array_equal(d["ks"].numpy()[rows], ks_own)
    # against the oracle's own roped k (float rounding of the norm may move a code by one step)
    g, r = d["kq"].numpy()[rows].astype(np.int32), o["kq"][rows].astype(np.int32)
    diff = np.abs(g - r)
    print("kq vs oracle-roped k: max code diff %d, %d of %d differ" % (diff.max(), (diff > 0).sum(), diff.size))
    assert diff.max() <= 1 and (diff > 0).mean() < 2e-3
    g_all, o_all = d["kq"].numpy(), o["kq"]
    assert not g_all[:pos].any() and not g_all[pos + T:].any(), "KV append wrote outside its rows"
    close("tail", d["tail"].numpy(), o["tail"], 0, 0)
    close("dead", d["dead"].numpy(), o["dead"], 1e-5, 1e-5)
    gp, op = d["pooled"].numpy().astype(np.int32), o["pooled"].astype(np.int32)
    assert np.abs(gp - op).max() <= 1, "pooled keys differ by more than 1 fp16 ulp"


@pytest.mark.parametrize("ctx,pos,T,topk,zero_q", [(1024, 700, 3, 64, False), (1024, 10, 2, 64, False),
                                                   (4096, 2001, 4, 256, True), (4096, 2999, 2, 2048, False),
                                                   (1024, 63, 3, 64, False), (4096, 4000, 8, 2048, True),
                                                   (262144, 100000, 2, 2048, False), (65536, 40000, 4, 2048, False)])
def test_qsa_select(wz, orc, gpu, ctx, pos, T, topk, zero_q):
    print("case qsa_select ctx=%d pos=%d T=%d topk=%d zero_q=%s" % (ctx, pos, T, topk, zero_q), flush=True)
    dm = qsa_dims(ctx, topk)
    rng = np.random.default_rng(pos + T)
    ih, idim, blk = dm.idx_heads, dm.idx_dim, dm.idx_blk
    max_b = ctx // blk + 2
    pooled = f16(rng.normal(0, 1, (max_b, idim)))
    dead = rng.normal(0, 1, idim).astype(np.float32)
    q_idx = (np.zeros if zero_q else lambda s: rng.normal(0, 1, s))((T, ih * idim)).astype(np.float32)
    d = {k: dev(v) for k, v in dict(pooled=pooled, dead=dead, q_idx=q_idx, pos=np.array([pos], np.int32)).items()}
    scores = DA((T, max_b), np.float32, zero=True)
    sel = DA((T, topk), np.int32, zero=True)
    cnt = DA(T, np.int32, zero=True)
    wz.wzy_qsa_select(C.byref(dm), d["pos"].ptr, d["pooled"].ptr, d["dead"].ptr, d["q_idx"].ptr, scores.ptr, max_b,
                      sel.ptr, cnt.ptr, T, None)
    wz.wzy_device_sync()
    gs, gsel, gcnt = scores.numpy(), sel.numpy(), cnt.numpy()
    for t in range(T):
        n_kv = pos + t + 1
        width = min(n_kv, topk)
        assert gcnt[t] == width
        if n_kv <= topk:
            assert (gsel[t, :width] == np.arange(width)).all()
            continue
        nb = n_kv // blk + 1
        os_ = np.empty(max_b, np.float32)
        orc.orc_block_scores(ptr(pooled), ptr(dead), ptr(q_idx[t]), n_kv, ih, idim, blk, ptr(os_))
        close("scores[%d]" % t, gs[t, :nb], os_[:nb], 1e-5, 1e-4)
        # the selection itself is integer work: on the GPU's own scores it must match exactly
        osel = np.empty(topk, np.int32)
        n = orc.orc_topk_select(ptr(np.ascontiguousarray(gs[t])), n_kv, blk, topk, ptr(osel))
        assert n == width
        assert (gsel[t, :width] == osel[:width]).all(), "row %d: selection differs" % t
        assert len(set(gsel[t, :width].tolist())) == width and gsel[t, :width].max() < n_kv


def topk_scores(kind, nb, rng):
    """Block scores that stress the threshold search: ties, a narrow cluster, a huge range, specials."""
    if kind == "gauss":
        return rng.normal(0, 2, nb).astype(np.float32)
    if kind == "levels":                                 # few values: large tied sets at the threshold
        return rng.integers(0, 4, nb).astype(np.float32)
    if kind == "relu":                                   # indexer-like: non-negative, many exact zeros
        return np.maximum(rng.normal(0, 1, (nb, 4)), 0).sum(1).astype(np.float32)
    if kind == "wide":                                   # keys spread over the whole 32-bit range
        return (np.sign(rng.normal(size=nb)) * np.exp(rng.uniform(-80, 80, nb))).astype(np.float32)
    if kind == "ulps":                                   # a cluster 1 ulp apart: single-key bins
        return (np.float32(1.0) + rng.permutation(nb).astype(np.float32) * np.float32(2.0 ** -23)).astype(np.float32)
    if kind == "heavy_tie":                              # one value held by thousands of blocks at the threshold
        s = rng.normal(0, 1, nb).astype(np.float32)
        s[rng.choice(nb, nb // 2, replace=False)] = np.float32(0.25)
        return s
    if kind == "specials":
        s = rng.normal(0, 1, nb).astype(np.float32)
        idx = rng.choice(nb, 40, replace=False)
        s[idx[:10]] = np.nan
        s[idx[10:20]] = np.inf
        s[idx[20:30]] = -np.inf
        s[idx[30:35]] = -0.0
        s[idx[35:]] = 0.0
        return s
    if kind == "equal":
        return np.full(nb, 3.5, np.float32)
    raise ValueError(kind)


@pytest.mark.parametrize("kind", ["gauss", "levels", "relu", "wide", "ulps", "heavy_tie", "specials", "equal"])
@pytest.mark.parametrize("ctx,pos,T,topk", [(33400, 32768, 1, 2048), (4096, 3001, 3, 256), (262144, 150001, 2, 2048)])
def test_qsa_topk_score_patterns(wz, orc, gpu, kind, ctx, pos, T, topk):
    print("case qsa_topk kind=%s ctx=%d pos=%d T=%d topk=%d" % (kind, ctx, pos, T, topk), flush=True)
    dm = qsa_dims(ctx, topk)
    blk = dm.idx_blk
    max_b = ctx // blk + 2
    rng = np.random.default_rng(pos + T + len(kind))
    scores = np.zeros((T, max_b), np.float32)
    for t in range(T):
        nb = (pos + t + 1) // blk + 1
        scores[t, :nb] = topk_scores(kind, nb, rng)
    d_sc, d_pos = dev(scores), dev(np.array([pos], np.int32))
    sel, cnt = DA((T, topk), np.int32, zero=True), DA(T, np.int32, zero=True)
    assert wz.wzy_qsa_topk(C.byref(dm), d_pos.ptr, d_sc.ptr, max_b, sel.ptr, cnt.ptr, T, None) == 0
    wz.wzy_device_sync()
    gsel, gcnt = sel.numpy(), cnt.numpy()
    for t in range(T):
        n_kv = pos + t + 1
        osel = np.empty(topk, np.int32)
        n = orc.orc_topk_select(ptr(np.ascontiguousarray(scores[t])), n_kv, blk, topk, ptr(osel))
        assert gcnt[t] == n
        assert (gsel[t, :n] == osel[:n]).all(), "row %d: selection differs" % t


@pytest.mark.parametrize("f16_above", [0, "window"])
@pytest.mark.parametrize("qh,kvh,pos,T,topk", [(4, 2, 700, 3, 64), (24, 2, 3000, 2, 2048), (24, 2, 100, 1, 2048),
                                               (8, 1, 300, 4, 256), (24, 2, 3999, 1, 2048)])
def test_qsa_attend(wz, orc, gpu, qh, kvh, pos, T, topk, f16_above):
    """f16_above 0: the fp32 kernel at every context (orc_attend); "window": the threshold is crossed by
    the window's last row only (pos + T - 1), and every row of the window takes the reference's fp16
    GQA branch (orc_attend_pf), as src/wzy_stage_v2.cuh:679-683 decides per window."""
    print("case qsa_attend qh=%d kvh=%d pos=%d T=%d topk=%d f16_above=%s" % (qh, kvh, pos, T, topk, f16_above),
          flush=True)
    ctx = 4096
    dm = qsa_dims(ctx, topk, qh, kvh)
    dm.attn_f16_above = 0 if f16_above == 0 else pos + T - 1
    f16 = attn_f16(dm, pos, T)
    assert f16 == (f16_above != 0)
    hd = 256
    KVD = kvh * hd
    rng = np.random.default_rng(qh + pos + T)
    kq = np.empty((ctx, KVD), np.int8)
    ks = np.empty((ctx, KVD // 64), np.uint16)
    vq = np.empty((ctx, KVD), np.int8)
    vs = np.empty((ctx, KVD // 64), np.uint16)
    wz.wzy_synth_kv_host(5, 3, 0, 0, ctx, KVD, kq.ctypes.data, ks.ctypes.data)
    wz.wzy_synth_kv_host(5, 3, 1, 0, ctx, KVD, vq.ctypes.data, vs.ctypes.data)
    qg = rng.normal(0, 1, (T, qh * 2 * hd)).astype(np.float32)
    sel = np.zeros((T, topk), np.int32)
    for t in range(T):
        n_kv = pos + t + 1
        if n_kv > topk:
            sel[t] = np.sort(rng.choice(n_kv, topk, replace=False))
    d = {k: dev(v) for k, v in dict(kq=kq, ks=ks, vq=vq, vs=vs, qg=qg, sel=sel, pos=np.array([pos], np.int32)).items()}
    nws = wz.wzy_qsa_attend_workspace_bytes(C.byref(dm), T)
    ws = DA(nws, np.uint8, zero=True)
    out = DA((T, qh * hd), np.float32)
    wz.wzy_qsa_attend(C.byref(dm), d["pos"].ptr, d["qg"].ptr, d["kq"].ptr, d["ks"].ptr, d["vq"].ptr, d["vs"].ptr,
                      d["sel"].ptr, out.ptr, ws.ptr, nws, T, None)
    wz.wzy_device_sync()
    g = out.numpy()
    for t in range(T):
        n_kv = pos + t + 1
        cells = sel[t] if n_kv > topk else np.arange(n_kv, dtype=np.int32)
        o = attend(orc, f16, qg[t], kq, ks, vq, vs, cells, qh, kvh, hd)
        close("attend[%d]" % t, g[t], o, 1e-3, 1e-4)
        check_attention_branch("attend[%d]" % t, g[t], o, attend(orc, not f16, qg[t], kq, ks, vq, vs, cells, qh, kvh, hd),
                               f16)

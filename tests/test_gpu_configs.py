"""GPU parity of BASELINE configs 2 and 3 at their own workloads (MI355X; C ABI only, no torch).

Config 2: the GDN gated delta-rule recurrence (fused_gdn_step_norm_multi, src/wzy_kernels_v2.cuh:908-984)
for 36 stacked layers x 1,000 sequential decode steps, 16 value heads x 128 and 16 key heads x 128,
fp32 state 16x128x128 per layer initialised N(0, 0.1), q and k L2-normalised bf16 ~N(0,1), v bf16
~N(0,1), decay = sigmoid(N(0,1)), beta = sigmoid(N(0,1)), seed 1.  The layers are independent (each
has its own inputs; one layer's output is not the next one's input).  Every output row of every
step is compared with the float64 oracle recurrence, so the drift over the config's 1,000-step
horizon is measured, not extrapolated.

Config 3: one QSA layer at a 262,144-cell context (src/wzy_qsa_256k.cuh:50-532,
src/wzy_qsa_wmma.cuh:492-612): INT8 K/V uniform over [-127,127] with fp16 scales per 64 values,
the 4-head indexer's fp16 pooled keys, 24 query heads over 2 KV heads of 256; the new token at
position 262,143 goes through prepare (norm + RoPE, KV append, indexer append) -> block scores ->
exact top-2048 -> sparse attention, checked against the oracle at every stage.  Seed 2."""
import ctypes as C
import time
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import wzy_amd
from layer_parity import ATOL, RTOL, excess, threshold_gap
from oracle_lib import ptr
from stage_oracle import attend, attn_f16, check_attention_branch, key_flip_ok

pytestmark = pytest.mark.gpu

DA = wzy_amd.DeviceArray


def sigmoid(x):
    return (1.0 / (1.0 + np.exp(-x.astype(np.float64)))).astype(np.float32)


def bf16_round(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16).astype(np.uint32).view(np.float32)


def config2_layer_inputs(wz, layer, steps, hk=16, hv=16, seed=1):
    """Inputs of one layer of config 2 (host generator: one sub-stream per tensor and layer)."""
    def normal(sub, n, sd=1.0):
        out = np.empty(n, np.float32)
        wz.wzy_synth_normal(seed, wz.wzy_synth_stream(0x20, layer, sub), n, 0.0, sd, out.ctypes.data)
        return out

    def unit(sub, heads):
        x = bf16_round(normal(sub, steps * heads * 128)).reshape(steps, heads, 128)
        return (x / np.sqrt((x.astype(np.float64) ** 2).sum(-1, keepdims=True))).astype(np.float32)

    return dict(q=unit(1, hk), k=unit(2, hk), v=bf16_round(normal(3, steps * hv * 128)).reshape(steps, hv, 128),
                decay=sigmoid(normal(4, steps * hv)).reshape(steps, hv),
                beta=sigmoid(normal(5, steps * hv)).reshape(steps, hv),
                state=normal(6, hv * 128 * 128, 0.1).reshape(hv, 128, 128))


def gpu_recurrence(wz, a, T_call):
    steps, hk = a["q"].shape[:2]
    hv = a["v"].shape[1]
    d = {k: DA.from_numpy(a[k]) for k in ("q", "k", "v", "decay", "beta", "state")}
    y = DA((steps, hv, 128), np.float32)
    for s0 in range(0, steps, T_call):
        T = min(T_call, steps - s0)
        wz.wzy_gdn_recurrence(d["q"].ptr + s0 * hk * 512, d["k"].ptr + s0 * hk * 512, d["v"].ptr + s0 * hv * 512,
                              d["decay"].ptr + s0 * hv * 4, d["beta"].ptr + s0 * hv * 4, None, None, C.c_float(1e-6),
                              d["state"].ptr, y.ptr + s0 * hv * 512, hk, hv, T, None, None)
    wz.wzy_device_sync()
    return y.numpy(), d["state"].numpy()


@pytest.mark.timeout(900)
def test_config2_gdn_36_layers_1000_steps(wz, orc, gpu):
    L, steps, hk, hv = 36, 1000, 16, 16
    print("case config2 gdn layers=%d steps=%d" % (L, steps), flush=True)
    t0 = time.time()
    with ThreadPoolExecutor(max_workers=8) as ex:
        inputs = list(ex.map(lambda l: config2_layer_inputs(wz, l, steps), range(L)))
    print("inputs generated in %.1f s" % (time.time() - t0), flush=True)
    gpu = []
    for l in range(L):
        # alternate the window width the GPU steps with: 1 row per call (a decode step) and 8 rows
        gpu.append(gpu_recurrence(wz, inputs[l], 1 if l % 2 == 0 else 8))
    print("gpu done in %.1f s" % (time.time() - t0), flush=True)

    def oracle(l):
        a = inputs[l]
        st = a["state"].copy()
        y = np.empty((steps, hv, 128), np.float32)
        orc.orc_gdn_recurrence(ptr(a["q"]), ptr(a["k"]), ptr(a["v"]), ptr(a["decay"]), ptr(a["beta"]), None, None,
                               1e-6, ptr(st), ptr(y), hk, hv, steps)
        return y, st

    with ThreadPoolExecutor(max_workers=16) as ex:
        ref = list(ex.map(oracle, range(L)))
    print("oracle done in %.1f s" % (time.time() - t0), flush=True)
    worst_y = worst_s = -np.inf
    max_err_y = max_err_s = 0.0
    drift = np.zeros(steps)
    for l in range(L):
        (gy, gs), (oy, os_) = gpu[l], ref[l]
        worst_y = max(worst_y, excess(gy, oy))
        worst_s = max(worst_s, excess(gs, os_))
        e = np.abs(gy.astype(np.float64) - oy)
        max_err_y = max(max_err_y, float(e.max()))
        max_err_s = max(max_err_s, float(np.abs(gs.astype(np.float64) - os_).max()))
        drift = np.maximum(drift, e.reshape(steps, -1).max(1))
    print("config 2: y max abs err %.3g (tolerance excess %.3g), final state max abs err %.3g (excess %.3g); "
          "max y error by step: first 10 %.3g, last 10 %.3g" % (max_err_y, worst_y, max_err_s, worst_s,
                                                                 drift[:10].max(), drift[-10:].max()), flush=True)
    assert worst_y <= 0 and worst_s <= 0
    # no growth of the error over the horizon
    assert drift[-100:].max() <= 4 * max(drift[:100].max(), 1e-6)


@pytest.mark.timeout(600)
def test_config3_qsa_262k_context(wz, orc, gpu):
    ctx = 262144
    pos = ctx - 1                         # the new token; cells 0 .. ctx-2 are the prefilled context
    print("case config3 qsa ctx=%d" % ctx, flush=True)
    dm = wzy_amd.QsaDims()
    dm.qh, dm.kvh, dm.hd, dm.n_rot = 24, 2, 256, 64
    dm.idx_heads, dm.idx_dim, dm.idx_blk, dm.idx_topk = 4, 128, 4, 2048
    dm.ctx_max, dm.kv_ring, dm.kv_sinks, dm.eps = ctx, 0, 0, 1e-6
    dm.attn_f16_above = 32768          # the reference's VRAM ring: this context attends with its fp16 kernel
    qh, kvh, hd, ih, idim, blk = 24, 2, 256, 4, 128, 4
    KVD, max_b = kvh * hd, ctx // blk + 2
    rng = np.random.default_rng(2)
    t0 = time.time()
    kq = np.zeros((ctx, KVD), np.int8)
    ks = np.zeros((ctx, KVD // 64), np.uint16)
    vq = np.zeros((ctx, KVD), np.int8)
    vs = np.zeros((ctx, KVD // 64), np.uint16)
    wz.wzy_synth_kv_host(2, 0, 0, 0, pos, KVD, kq.ctypes.data, ks.ctypes.data)
    wz.wzy_synth_kv_host(2, 0, 1, 0, pos, KVD, vq.ctypes.data, vs.ctypes.data)
    pooled = np.zeros((max_b, idim), np.uint16)
    nblk = pos // blk                     # complete blocks before the new token
    pooled[:nblk] = rng.normal(0, 1, (nblk, idim)).astype(np.float16).view(np.uint16)
    tail = rng.normal(0, 1, (blk - 1, idim)).astype(np.float16).astype(np.float32)
    dead = rng.normal(0, 1, idim).astype(np.float32)
    cos_t = np.empty((ctx, 32), np.float32)
    sin_t = np.empty((ctx, 32), np.float32)
    orc.orc_rope_tables(ctx, 64, 1e7, ptr(cos_t), ptr(sin_t))
    a = dict(qg=bf16_round(rng.normal(0, 1, (1, qh * 2 * hd))), kk=rng.normal(0, 1, (1, KVD)).astype(np.float32),
             vv=rng.normal(0, 1, (1, KVD)).astype(np.float32), q_idx=rng.normal(0, 1, (1, ih * idim)).astype(np.float32),
             idx_raw=rng.normal(0, 1, (1, idim)).astype(np.float32),
             q_norm=rng.normal(1, 0.02, hd).astype(np.float32), k_norm=rng.normal(1, 0.02, hd).astype(np.float32),
             iq_norm=rng.normal(1, 0.02, idim).astype(np.float32), ik_norm=rng.normal(1, 0.02, idim).astype(np.float32))
    print("inputs ready in %.1f s" % (time.time() - t0), flush=True)
    d = {k: DA.from_numpy(v) for k, v in dict(a, kq=kq, ks=ks, vq=vq, vs=vs, pooled=pooled, tail=tail, dead=dead,
                                                cos=cos_t, sin=sin_t, pos=np.array([pos], np.int32)).items()}
    scores = DA((1, max_b), np.float32, zero=True)
    sel = DA((1, 2048), np.int32, zero=True)
    cnt = DA(1, np.int32, zero=True)
    nws = wz.wzy_qsa_attend_workspace_bytes(C.byref(dm), 1)
    ws = DA(nws, np.uint8, zero=True)
    out = DA((1, qh * hd), np.float32)
    wz.wzy_qsa_prepare(C.byref(dm), d["pos"].ptr, d["qg"].ptr, d["kk"].ptr, d["vv"].ptr, d["q_idx"].ptr,
                       d["idx_raw"].ptr, d["q_norm"].ptr, d["k_norm"].ptr, d["iq_norm"].ptr, d["ik_norm"].ptr,
                       d["cos"].ptr, d["sin"].ptr, d["kq"].ptr, d["ks"].ptr, d["vq"].ptr, d["vs"].ptr, d["tail"].ptr,
                       d["dead"].ptr, d["pooled"].ptr, 1, None)
    wz.wzy_qsa_select(C.byref(dm), d["pos"].ptr, d["pooled"].ptr, d["dead"].ptr, d["q_idx"].ptr, scores.ptr, max_b,
                      sel.ptr, cnt.ptr, 1, None)
    wz.wzy_qsa_attend(C.byref(dm), d["pos"].ptr, d["qg"].ptr, d["kq"].ptr, d["ks"].ptr, d["vq"].ptr, d["vs"].ptr,
                      sel.ptr, out.ptr, ws.ptr, nws, 1, None)
    wz.wzy_device_sync()
    print("gpu done in %.1f s" % (time.time() - t0), flush=True)

    # oracle: prepare
    o = {k: v.copy() for k, v in a.items()}
    for h in range(qh):
        orc.orc_head_norm_rope(ptr(o["qg"][0, h * 2 * hd:]), hd, ptr(o["q_norm"]), ptr(cos_t), ptr(sin_t), pos, 64, 1e-6)
    for j in range(kvh):
        orc.orc_head_norm_rope(ptr(o["kk"][0, j * hd:]), hd, ptr(o["k_norm"]), ptr(cos_t), ptr(sin_t), pos, 64, 1e-6)
    for i in range(ih):
        orc.orc_head_norm_rope(ptr(o["q_idx"][0, i * idim:]), idim, ptr(o["iq_norm"]), ptr(cos_t), ptr(sin_t), pos, 64,
                               1e-6)
    okq, oks = np.zeros(KVD, np.int8), np.zeros(KVD // 64, np.uint16)
    ovq, ovs = np.zeros(KVD, np.int8), np.zeros(KVD // 64, np.uint16)
    orc.orc_kv_quant_row(ptr(o["kk"][0]), KVD, ptr(okq), ptr(oks))
    orc.orc_kv_quant_row(ptr(o["vv"][0]), KVD, ptr(ovq), ptr(ovs))
    opooled, otail, odead = pooled.copy(), tail.copy(), dead.copy()
    orc.orc_indexer_append(ptr(o["idx_raw"][0]), ptr(o["ik_norm"]), ptr(cos_t), ptr(sin_t), pos, idim, blk, 64, 1e-6,
                           ptr(otail), ptr(odead), ptr(opooled))
    for k in ("qg", "kk", "q_idx"):
        assert excess(d[k].numpy(), o[k]) <= 0 and np.abs(d[k].numpy() - o[k]).max() < 1e-4, k
    np.testing.assert_array_equal(d["vq"].numpy()[pos], ovq)
    np.testing.assert_array_equal(d["vs"].numpy()[pos], ovs)
    gkq = d["kq"].numpy()
    # the K cell: the oracle's quantisation of the very k row the GPU quantised (its k after norm + RoPE,
    # left in place by the prepare call), bit for bit
    gkq_o, gks_o = np.zeros(KVD, np.int8), np.zeros(KVD // 64, np.uint16)
    g_kk = np.ascontiguousarray(d["kk"].numpy()[0])          # held: the oracle reads it through a pointer
    orc.orc_kv_quant_row(ptr(g_kk), KVD, ptr(gkq_o), ptr(gks_o))
    np.testing.assert_array_equal(gkq[pos], gkq_o)
    np.testing.assert_array_equal(d["ks"].numpy()[pos], gks_o)
    assert np.abs(gkq[pos].astype(int) - okq).max() <= 1
    assert np.array_equal(gkq[:pos], kq[:pos]), "prefilled K cells changed"
    gpooled = d["pooled"].numpy()
    # the pooled key of the block this token completes: identical raw input on both sides, so an fp16
    # code may differ only where the oracle's unrounded key sits at a rounding midpoint
    key = np.full(idim, np.nan, np.float32)
    ktail, kdead, kpooled = tail.copy(), dead.copy(), pooled.copy()
    orc.orc_indexer_append_f32(ptr(o["idx_raw"][0]), ptr(o["ik_norm"]), ptr(cos_t), ptr(sin_t), pos, idim, blk, 64,
                               1e-6, ptr(ktail), ptr(kdead), ptr(kpooled), ptr(key))
    for i in np.flatnonzero(gpooled.ravel() != opooled.ravel()):
        b, dd = divmod(int(i), idim)
        assert b == pos // blk and not np.isnan(key[dd]), "pooled key %d dim %d changed" % (b, dd)
        assert key_flip_ok(key[dd], gpooled.ravel()[i], opooled.ravel()[i], key), (b, dd, key[dd])

    # scores over 65,537 blocks, then the exact top-2048 (bit-exact on the GPU's own scores)
    n_kv = pos + 1
    nb = n_kv // blk + 1
    gsc = scores.numpy()[0]
    osc = np.zeros(max_b, np.float32)
    orc.orc_block_scores(ptr(opooled), ptr(odead), ptr(o["q_idx"][0]), n_kv, ih, idim, blk, ptr(osc))
    serr = np.abs(gsc[:nb].astype(np.float64) - osc[:nb])
    print("scores: %d blocks, max abs err %.3g (max %.3g)" % (nb, serr.max(), np.abs(osc[:nb]).max()), flush=True)
    assert (serr <= 1e-4 * np.maximum(1.0, np.abs(osc[:nb]))).all()
    gsel, gcnt = sel.numpy()[0], int(cnt.numpy()[0])
    assert gcnt == 2048
    own = np.empty(2048, np.int32)
    gsc = np.ascontiguousarray(gsc)
    assert orc.orc_topk_select(ptr(gsc), n_kv, blk, 2048, ptr(own)) == 2048
    np.testing.assert_array_equal(gsel, own)
    osel = np.empty(2048, np.int32)
    orc.orc_topk_select(ptr(osc), n_kv, blk, 2048, ptr(osel))
    if not np.array_equal(osel, gsel):
        gap = threshold_gap(osc, n_kv, blk, 2048)
        assert gap <= 2 * serr.max(), "selection differs from the oracle's outside a near tie (gap %.3g)" % gap
        print("selection: near tie at the threshold (gap %.3g, score error %.3g)" % (gap, serr.max()), flush=True)
    # attention over the GPU's selection (the oracle reads the GPU-appended K/V of the new cell): at
    # 262,144 cells the reference runs its fp16 GQA kernel (src/wzy_stage_v2.cuh:679-683), restated by
    # orc_attend_pf; orc_attend (its fp32 kernel) is the other branch
    gqg, gks, gvq, gvs = d["qg"].numpy(), d["ks"].numpy(), d["vq"].numpy(), d["vs"].numpy()
    assert attn_f16(dm, pos, 1)
    oatt = attend(orc, True, gqg[0], gkq, gks, gvq, gvs, gsel, qh, kvh, hd)
    o32 = attend(orc, False, gqg[0], gkq, gks, gvq, gvs, gsel, qh, kvh, hd)
    gatt = out.numpy()[0]
    v = excess(gatt, oatt)
    print("attention: max abs err %.3g (max %.3g), tolerance excess %.3g; fp16 and fp32 branches differ by at most "
          "%.3g" % (np.abs(gatt - oatt).max(), np.abs(oatt).max(), v, np.abs(oatt.astype(np.float64) - o32).max()),
          flush=True)
    assert v <= 0
    check_attention_branch("config 3", gatt, oatt, o32, True)

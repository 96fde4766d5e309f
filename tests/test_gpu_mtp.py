"""GPU parity of the MTP drafter (wzy_stage_mtp_*) against the CPU oracle (oracle/orc_mtp.c).

Every draft step is checked component by component with the oracle fed the GPU's own inputs
(mtp_oracle.MtpTeacher: front rows, K/V ring cells, q, ring attention, o projection, MLP
hyper-connection, router ids / weights (bit-exact), Q2_0 + shared MoE, final mixer, draft logits,
and the exact argmax / probability over the GPU's own logits), and the drafted chain is compared
free-running with the oracle's own chain started from the GPU's ring (tokens bit-exact unless the
oracle's top-2 draft logits are within the tolerance).  Tolerance: rel 2e-2 / abs 1e-2 with the
relative term floored at the row's RMS (teacher_forced.row_excess).
"""
import time

import numpy as np
import pytest

import wzy_amd
from mtp_oracle import RING, MtpTeacher, OracleMtp, gpu_acts
from stage_oracle import small_cfg

pytestmark = pytest.mark.gpu


def q8_rows_ref(rows_bf16, D):
    """quant_bf16_to_q8_kernel (src/wzy_kernels_v2.cuh:393-407) on bf16 rows [n x D]."""
    n = rows_bf16.size // D
    rows = (rows_bf16.astype(np.uint32) << 16).view(np.float32).reshape(n, D // 32, 32)
    amax = np.abs(rows).max(axis=2)
    sh = (amax / np.float32(127.0)).astype(np.float16)
    d = sh.astype(np.float32)[:, :, None]
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(d > 0, np.clip(np.rint(rows / np.where(d > 0, d, 1)), -127, 127), 0).astype(np.int8)
    return q.reshape(n, D), sh.view(np.uint16)


def setup_stage(cfg, seed, n_dv, n_ctx=0):
    st = wzy_amd.Stage(cfg)
    t0 = time.time()
    st.load_synthetic(seed, n_ctx)
    st.mtp_init(seed + 100, n_dv)
    om = OracleMtp.from_stage(st, cfg, n_dv)
    print("stage + drafter + oracle ready in %.1f s" % (time.time() - t0), flush=True)
    return st, om


def check_weights(wz, st, om, cfg, seed, n_dv, experts=(0, 1)):
    """Device drafter weights that are not read back into the oracle as-is: the Q2_0 experts equal the
    host generator's bytes, the draft head equals the Q8_0 quantisation of the main head's rows."""
    D = cfg.n_embd
    rec = wz.wzy_q2_expert_bytes(D, cfg.n_ff)
    for e in experts:
        b = np.empty(rec, np.uint8)
        wz.wzy_synth_q2_expert(seed + 100, e, D, cfg.n_ff, b.ctypes.data)
        assert (om.a["experts"][e * rec:(e + 1) * rec] == b).all(), "expert %d bytes" % e
    dv = om.a["dvocab"]
    assert (dv == (np.arange(n_dv, dtype=np.int64) * cfg.n_vocab // n_dv)).all()
    rows = np.array([0, 1, n_dv // 2, n_dv - 1])
    src = np.concatenate([st.read_range(-1, "head", np.uint16, int(dv[r]) * D, D) for r in rows])
    q, s = q8_rows_ref(src, D)
    assert (om.a["head.q"].reshape(n_dv, D)[rows] == q).all()
    assert (om.a["head.s"].reshape(n_dv, D // 32)[rows] == s).all()


def seed_cells(st, tch, cfg, n_dv, toks, first, last, check_every=1):
    """Main-model windows over cells first..last-1 with the pre-head output only, each followed by
    the drafter front of its rows (seed_mtp_tail, src/wzy_engine_v2.cu:1266-1290); every
    check_every-th front is checked teacher-forced."""
    p, k = first, 0
    while p < last:
        T = min(8, last - p)
        st.forward(p, toks[p:p + T], run_head=2)
        st.mtp_front(p, toks[p + 1:p + 1 + T], 0)
        if k % check_every == 0 or p + T == last:
            st.sync()
            g = gpu_acts(st, cfg, n_dv, rows=T)
            tch.check_front("front at %d" % p, g, p, toks[p + 1:p + 1 + T], st.pre_head(T))
        p += T
        k += 1
    st.sync()


def draft_chain_checked(st, tch, om, cfg, n_dv, cell, tok, depth, floor=0):
    """`depth` chained draft steps as separate depth-1 calls, each checked teacher-forced; then the
    same chain as one depth-`depth` call (graph replay, bit-identical), and the oracle's own chain
    from the GPU's starting ring (free-running).  Returns the drafted tokens."""
    st.forward(cell, [tok], run_head=1)
    st.sync()
    rin0 = st.pre_head(1)[0]
    ring0 = {k: st.read(-1, "mtp." + k, dt) for k, dt in (("kv_k", np.int8), ("kv_ks", np.uint16), ("kv_v", np.int8),
                                                           ("kv_vs", np.uint16))}
    toks, probs = [], []
    rin, t = rin0, tok
    for j in range(depth):
        d_t, d_p = st.mtp_draft(cell + j, t, 0 if j == 0 else -1, 1)
        g = gpu_acts(st, cfg, n_dv)
        tch.check_step("step %d at %d" % (j, cell + j), g, cell + j, t, rin, int(d_t[0]), float(d_p[0]), floor)
        toks.append(int(d_t[0]))
        probs.append(float(d_p[0]))
        rin, t = g["R_out"], int(d_t[0])
    # the whole chain in one call (one graph launch per step, no host round trip in between), from the
    # same ring: the steps above wrote cells cell+1.., whose slots held the oldest cells of this
    # window once the ring has wrapped (the reference's ring evicts them the same way)
    for k, v in ring0.items():
        st.write(-1, "mtp." + k, v)
    c_t, c_p = st.mtp_draft(cell, tok, 0, depth)
    assert list(c_t) == toks and np.array_equal(c_p, np.array(probs, np.float32)), (list(c_t), toks)
    # free-running oracle chain from the GPU's ring before the chain
    for k, v in ring0.items():
        om.a[k][:] = v
    om.set_floor(floor)
    rin, t = rin0, tok
    for j in range(depth):
        R_out, _, lg, o_t, o_p = om.step(cell + j, t, rin)
        srt = np.sort(lg)[::-1]
        if srt[0] - srt[1] > 2e-2 * max(1.0, abs(srt[0])):
            assert o_t == toks[j], "free-running step %d: oracle %d vs GPU %d" % (j, o_t, toks[j])
            assert abs(o_p - probs[j]) <= 2e-2 * o_p + 1e-6, (j, o_p, probs[j])
        else:
            break                      # a near tie: the chains may part here
        rin, t = R_out, o_t
    return toks, probs


def test_mtp_small_drafter(wz, gpu):
    """Small dims (n_embd 256, 16 experts top-4, vocab 1000, 800 draft rows): seeded fronts, a
    three-step chain, graph replay vs direct launches, then a ring that wraps past 1,024 cells and
    an attention floor."""
    print("case mtp_small", flush=True)
    cfg = small_cfg(wzy_amd, ctx_max=1400, n_layers=2)
    n_dv, seed = 800, 5
    st, om = setup_stage(cfg, seed, n_dv)
    try:
        check_weights(wz, st, om, cfg, seed, n_dv)
        tch = MtpTeacher(om)
        rng = np.random.default_rng(3)
        toks = rng.integers(0, cfg.n_vocab, 1400).astype(np.int32)
        seed_cells(st, tch, cfg, n_dv, toks, 0, 24)
        d1, p1 = draft_chain_checked(st, tch, om, cfg, n_dv, 24, int(toks[24]), 3)
        # direct launches give the same chain, bit for bit
        st.lib.wzy_stage_set_graphs(st.h, 0)
        d2, p2 = st.mtp_draft(24, int(toks[24]), 0, 3)      # same pre-head row: the last forward's
        st.lib.wzy_stage_set_graphs(st.h, 1)
        assert list(d2) == d1 and np.array_equal(p2, np.array(p1, np.float32))
        # a ring that wraps: cells 25 .. 1299 seeded (checked every 16th front), then steps at 1300
        seed_cells(st, tch, cfg, n_dv, toks, 25, 1300, check_every=16)
        draft_chain_checked(st, tch, om, cfg, n_dv, 1300, int(toks[1300]), 2)
        st.mtp_set_floor(1250)
        draft_chain_checked(st, tch, om, cfg, n_dv, 1300, int(toks[1300]), 2, floor=1250)
        print("mtp small: " + tch.summary(), flush=True)
        assert tch.counts["steps"] == 7
    finally:
        st.close()


@pytest.mark.timeout(900)
def test_mtp_baseline_shapes(wz, gpu):
    """BASELINE shapes (n_embd 2048, hc 4 x rank 320, 24/2 heads of 256, 512 Q2_0 experts top-10 of
    width 512, vocab 151,936, 114,452 draft rows) on a 4-layer main model prefilled to 32,768 cells:
    the last 40 cells seeded with floor 32,768 (the tail seeding of a long prompt), then a three-step
    chain."""
    print("case mtp_baseline", flush=True)
    cfg = wzy_amd.default_cfg(32768 + 256)
    cfg.n_layers = 4
    n_dv, seed, n_ctx = 114452, 9, 32768
    st, om = setup_stage(cfg, seed, n_dv, n_ctx)
    try:
        check_weights(wz, st, om, cfg, seed, n_dv, experts=(0, 511))
        tch = MtpTeacher(om)
        rng = np.random.default_rng(4)
        toks = np.zeros(n_ctx + 64, np.int32)
        toks[n_ctx:] = rng.integers(0, cfg.n_vocab, 64)
        st.mtp_set_floor(n_ctx)
        t0 = time.time()
        seed_cells(st, tch, cfg, n_dv, toks, n_ctx, n_ctx + 40, check_every=2)
        print("seeded in %.1f s" % (time.time() - t0), flush=True)
        t0 = time.time()
        d, p = draft_chain_checked(st, tch, om, cfg, n_dv, n_ctx + 40, int(toks[n_ctx + 40]), 3, floor=n_ctx)
        print("chain %s probs %s in %.1f s" % (d, p, time.time() - t0), flush=True)
        print("mtp baseline: " + tch.summary(), flush=True)
        assert tch.counts["steps"] == 3 and tch.counts["fronts"] >= 24
    finally:
        st.close()

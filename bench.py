#!/usr/bin/env python3
"""Decode benchmark of the MI355X build (one GPU).

Workload: the synthetic 48-layer decoder (36 GDN + 12 QSA layers, NVFP4 MoE
with 512 experts / top-10 + a shared expert in every layer, vocab 151936, bf16 LM head), one
sequence at a 32K-token prefilled context, greedy token loop.  A step is one decode token: one
replay of the captured forward graph, the host reading the greedy id back and feeding it in as the
next token.  The timed region is `--steps` such steps after `--warmup` untimed ones, bracketed by
device synchronisation.

Beside the tok/s line it reports
  roofline      the MoE gate/up kernel (the largest contributor to the step, 48 launches per token)
                timed live with HIP events on the stage's own stream, against 8 TB/s;
  cpu_baseline  the AVX2/FMA restatement of the reference CPU MoE pool (oracle/cpu_moe_pool.cpp)
                on BASELINE config 1 (one token, 10 routed experts), timed on this host for a
                bounded ~10 s sample;
  prefill_moe   BASELINE config 5's chunked-prefill MoE block (8,192 tokens, one layer) on MFMA:
                per-launch-group HIP event times, routed-expert TFLOP/s against the 2.5 PFLOP/s
                dense bf16 MFMA peak;
  stage_prefill BASELINE config 5's 8,192-token chunk through the whole 48-layer model (wzy_stage_prefill):
                tok/s and the weight GEMMs' TFLOP/s against the dense bf16 MFMA peak;
  mtp_config5   BASELINE config 5's decode half: the MTP drafter at a fixed depth of 3 with T=4 verify
                windows on the same stage (tok/s, acceptance, per-window split, and one draft step's
                HBM bytes / event-timed duration against 8 TB/s);
  gdn_config2, qsa_262k   BASELINE configs 2 and 3 at their own workloads.
Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
       python bench.py --profile {step,window,mtp} [--profile-units N]   (units for a rocprofv3 run)
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "wzy-flash-serve_amd"))

HBM_PEAK_GBS = 8000.0
D, F, E, K = 2048, 512, 512, 10
# bytes one moe_gate_up launch must read at T=1: 10 routed experts' gate+up e2m1 codes and e4m3
# scales (2*F*D/2 + 2*F*D/16) + their 16-byte tail, the shared expert's Q8_0 gate+up (2*F*D
# codes + 2*F*D/32 fp16 scales), the router logits (E fp32) and the activation row (D fp32).
GU_BYTES = K * (2 * F * D // 2 + 2 * F * D // 16 + 16) + (2 * F * D + 2 * F * D // 32 * 2) + E * 4 + D * 4
# bytes one moe_down launch must read: routed down codes+scales, shared down Q8_0, the requantised
# activations, and the output row written
DN_BYTES = K * (D * F // 2 + D * F // 16) + (D * F + D * F // 32 * 2) + K * (F + F // 16 * 4) + D * 4
# routed-expert bytes of one token-layer (the BASELINE config-1 roofline basis)
ROUTED_BYTES = K * (3 * F * D // 2 + 3 * F * D // 16 + 16)


MFMA_BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
PF_STAGES = ("x_to_bf16", "router_gemm", "route", "tiles", "shared_gate_up", "shared_down", "routed_gate_up",
             "routed_down")


def prefill_moe(wz, st, n_tok, iters, seed):
    """Config-5 chunked-prefill MoE on layer 0 of the loaded stage: n_tok rows of N(0,1) x, every
    launch group timed with HIP events (wzy_moe_prefill_time)."""
    import numpy as np
    import wzy_amd
    w = wzy_amd.MoeWeights()
    wz.wzy_stage_moe_weights(st.h, 0, C.byref(w))
    x = np.random.default_rng(seed).standard_normal((n_tok, D), dtype=np.float32)
    xd = wzy_amd.DeviceArray.from_numpy(x)
    comb = wzy_amd.DeviceArray(n_tok * D, np.float32)
    nws = wz.wzy_moe_prefill_workspace_bytes(D, F, E, K, n_tok)
    ws = wzy_amd.DeviceArray(nws, np.uint8)
    us = (C.c_float * len(PF_STAGES))()
    wz.wzy_moe_prefill_time(C.byref(w), xd.ptr, n_tok, comb.ptr, ws.ptr, nws, iters, us, None)
    for a in (xd, comb, ws):
        a.free()
    st_us = {k: round(us[i], 2) for i, k in enumerate(PF_STAGES)}
    total = sum(us[i] for i in range(len(PF_STAGES)))
    routed_us = us[6] + us[7]
    routed_flop = 2.0 * n_tok * K * D * 3 * F            # gate+up (2F rows) and down (F cols)
    block_flop = routed_flop + 2.0 * n_tok * (E * D + 3 * F * D)
    gu_flop = 2.0 * n_tok * K * D * 2 * F
    return {
        "workload": "config 5 chunked-prefill MoE block, one layer (D=2048, 512 experts top-10, NFF=512, "
                    "shared expert), %d tokens" % n_tok,
        "n_tok": n_tok, "iters": iters, "us_total": round(total, 1),
        "tok_s_layer": round(n_tok / (total * 1e-6), 0),
        "routed_gflop": round(routed_flop / 1e9, 1),
        "routed_tflops": round(routed_flop / (routed_us * 1e-6) / 1e12, 1),
        "routed_frac": round(routed_flop / (routed_us * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
        "routed_gate_up_tflops": round(gu_flop / (us[6] * 1e-6) / 1e12, 1),
        "block_tflops": round(block_flop / (total * 1e-6) / 1e12, 1),
        "peak_tflops": MFMA_BF16_PEAK_TFLOPS,
        "us_stages": st_us,
    }


PF_PARTS = ("attn_hc_read", "gdn", "qsa", "ffn_hc_read", "moe", "rest")


def stage_dense_macs(cfg):
    """Multiply-accumulates per token of every weight GEMM in one prefill chunk (all layers): the two
    hyper-connection reads per layer (inject, down, up projections), the GDN or QSA projections, the
    router and the shared + top-k routed experts.  Attention and indexer scores are context-dependent
    and not counted."""
    D, HCD, L = cfg.n_embd, cfg.hc * cfg.n_embd, cfg.hc_lr
    QKV, GV = 2 * cfg.gdn_hk * 128 + cfg.gdn_hv * 128, cfg.gdn_hv * 128
    QD, KVD, ID, IH = cfg.qsa_qh * cfg.qsa_hd, cfg.qsa_kvh * cfg.qsa_hd, cfg.idx_dim, cfg.idx_heads
    hc = 2 * (HCD * cfg.hc + 2 * HCD * L)
    gdn = D * QKV + D * GV + 2 * D * cfg.gdn_hv + GV * D
    qsa = D * 2 * QD + 2 * D * KVD + D * ID + D * IH * ID + QD * D
    moe = D * cfg.n_exp + (1 + cfg.top_k) * 3 * cfg.n_ff * D
    n_qsa = cfg.n_layers // cfg.qsa_period
    return cfg.n_layers * (hc + moe) + n_qsa * qsa + (cfg.n_layers - n_qsa) * gdn


def stage_prefill(wz, st, cfg, pos, n_tok, iters, seed):
    """Config-5 chunked prefill of the whole 48-layer model: one chunk of n_tok prompt cells appended at
    `pos` (after the prefilled context), every chunk re-run at the same cells.  One untimed run, `iters`
    wall-clock timed runs (host clock around wzy_stage_prefill + stream sync), then one run split into
    event-timed parts (wzy_stage_prefill_time; the part boundaries synchronise, so that run is slower)."""
    import numpy as np
    toks = np.random.default_rng(seed).integers(0, cfg.n_vocab, n_tok).astype(np.int32)
    tp = toks.ctypes.data
    wz.wzy_stage_prefill(st.h, pos, tp, n_tok)
    wz.wzy_stage_sync(st.h)
    t0 = time.perf_counter()
    for _ in range(iters):
        wz.wzy_stage_prefill(st.h, pos, tp, n_tok)
    wz.wzy_stage_sync(st.h)
    el = (time.perf_counter() - t0) / iters
    us = (C.c_float * len(PF_PARTS))()
    wz.wzy_stage_prefill_time(st.h, pos, tp, n_tok, us)
    macs = stage_dense_macs(cfg)
    tflops = 2.0 * macs * n_tok / el / 1e12
    return {"workload": "config 5 chunked prefill: %d prompt cells in one chunk through all %d layers of the config-4 "
                        "model, appended after a %d-cell context" % (n_tok, cfg.n_layers, pos),
            "n_tok": n_tok, "iters": iters, "ms_per_chunk": round(1000 * el, 2), "tok_s": round(n_tok / el, 0),
            "dense_gflop_per_token": round(2.0 * macs / 1e9, 3),
            "dense_tflops": round(tflops, 1), "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
            "peak_tflops": MFMA_BF16_PEAK_TFLOPS,
            "us_parts_synced_run": {k: round(us[i], 1) for i, k in enumerate(PF_PARTS)}}


# config 2 per layer-step: fp32 state read + written (2 x 1 MiB), bf16 q, k, v (3 x 4,096 B), the two gates
# of 16 heads (128 B) and the fp32 output (8,192 B) = 2,117,760 B
GDN_LAYER_STEP_BYTES = 2 * 16 * 128 * 128 * 4 + 3 * 16 * 128 * 2 + 2 * 16 * 4 + 16 * 128 * 4
QSA_CTX = 262144
# config 3 per-token algorithmic bytes: fp16 indexer keys of 65,536 blocks, block scores written and
# read back, the 2,048 selected cells' K and V (512 B each) and their fp16 scales (8 + 8 per cell)
QSA_BYTES = {"scores": (QSA_CTX // 4) * 128 * 2 + (QSA_CTX // 4 + 1) * 4,
             "topk": (QSA_CTX // 4 + 1) * 4 + 2048 * 4,
             "attention": 2048 * (2 * 512 + 2 * 16) + 24 * 512 * 4 + 24 * 256 * 4 + 2048 * 4}
QSA_TOKEN_BYTES = (QSA_CTX // 4) * 128 * 2 + 2 * QSA_CTX + 2048 * 1024 + 65536       # 19,464,192


def gdn_config2(wz, seed=1, n_layers=36, steps=1000):
    """BASELINE config 2 timed: 36 independent GDN layers x 1,000 decode steps (16/16 heads), step-major,
    through the standalone recurrence kernels, T = 1 and T = 8 rows per launch."""
    import numpy as np
    import wzy_amd
    DA = wzy_amd.DeviceArray
    hk = hv = 16

    def normal(sub, n, sd=1.0):
        out = np.empty(n, np.float32)
        wz.wzy_synth_normal(seed, wz.wzy_synth_stream(0x20, 0, sub), n, 0.0, sd, out.ctypes.data)
        return out

    def unit(x):
        x = x.reshape(steps, -1, 128)
        return (x / np.linalg.norm(x, axis=-1, keepdims=True)).astype(np.float32)

    sig = lambda x: (1.0 / (1.0 + np.exp(-x))).astype(np.float32)
    q, k = DA.from_numpy(unit(normal(1, steps * hk * 128))), DA.from_numpy(unit(normal(2, steps * hk * 128)))
    v = DA.from_numpy(normal(3, steps * hv * 128))
    dec, beta = DA.from_numpy(sig(normal(4, steps * hv))), DA.from_numpy(sig(normal(5, steps * hv)))
    states = DA.from_numpy(np.tile(normal(6, hv * 128 * 128, 0.1), n_layers))
    y = DA(steps * hv * 128, np.float32)
    out = {"workload": "config 2: %d independent GDN layers x %d decode steps, 16 key / 16 value heads x 128, "
                       "fp32 state, step-major (every layer's step s before step s+1), seed %d" % (n_layers, steps, seed),
           "bytes_per_layer_step": GDN_LAYER_STEP_BYTES}
    for T in (1, 8):
        us, us_k = C.c_float(0), C.c_float(0)
        wz.wzy_gdn_time_recurrence(q.ptr, k.ptr, v.ptr, dec.ptr, beta.ptr, states.ptr, y.ptr, hk, hv, n_layers, steps,
                                   T, C.byref(us), C.byref(us_k), None)
        key = "t1" if T == 1 else "t8"
        out[key] = {"rows_per_launch": T, "us_per_layer_step": round(us.value, 4),
                    "layer_steps_per_s": round(1e6 / us.value, 1),
                    "us_per_layer_step_recurrence_kernel": round(us_k.value, 4),
                    "achieved_gbs": round(GDN_LAYER_STEP_BYTES / (us.value * 1e-6) / 1e9, 1)}
    out["achieved_gbs"] = out["t1"]["achieved_gbs"]
    out["frac"] = round(out["t1"]["achieved_gbs"] / HBM_PEAK_GBS, 4)
    out["note"] = ("GB/s counts the state read + write of every layer-step (the reference's T=1 decode); the "
                   "36 MiB of state stays in the 256 MB last-level cache between steps, and with T=8 the state "
                   "round-trips once per 8 steps, so its GB/s is an equivalent rate")
    for a in (q, k, v, dec, beta, states, y):
        a.free()
    return out


def qsa_262k(wz, seed=2, iters=50):
    """BASELINE config 3 timed: one QSA layer, one decode token at a 262,144-cell context, stage by stage."""
    import numpy as np
    import wzy_amd
    DA = wzy_amd.DeviceArray
    ctx, pos = QSA_CTX, QSA_CTX - 1
    qh, kvh, hd, ih, idim, blk = 24, 2, 256, 4, 128, 4
    KVD, max_b = kvh * hd, ctx // blk + 2
    dm = wzy_amd.QsaDims()
    dm.qh, dm.kvh, dm.hd, dm.n_rot = qh, kvh, hd, 64
    dm.idx_heads, dm.idx_dim, dm.idx_blk, dm.idx_topk = ih, idim, blk, 2048
    dm.ctx_max, dm.kv_ring, dm.kv_sinks, dm.eps = ctx, 0, 0, 1e-6
    rng = np.random.default_rng(seed)
    keep = []

    def dev(a):
        d = DA.from_numpy(np.ascontiguousarray(a))
        keep.append(d)
        return d.ptr

    kq, ks = DA(ctx * KVD, np.int8), DA(ctx * KVD // 64, np.uint16)
    vq, vs = DA(ctx * KVD, np.int8), DA(ctx * KVD // 64, np.uint16)
    keep += [kq, ks, vq, vs]
    wz.wzy_synth_kv_device(seed, 0, 0, 0, ctx, KVD, kq.ptr, ks.ptr, None)
    wz.wzy_synth_kv_device(seed, 0, 1, 0, ctx, KVD, vq.ptr, vs.ptr, None)
    pooled = np.zeros((max_b, idim), np.float16)
    pooled[:pos // blk] = rng.normal(0, 1, (pos // blk, idim))
    ang = np.arange(ctx, dtype=np.float64)[:, None] * (1e7 ** (-np.arange(32) / 32.0))[None, :]
    L = wzy_amd.QsaLayer()
    L.qg, L.kk = dev(rng.normal(0, 1, qh * 2 * hd).astype(np.float32)), dev(rng.normal(0, 1, KVD).astype(np.float32))
    L.vv, L.q_idx = dev(rng.normal(0, 1, KVD).astype(np.float32)), dev(rng.normal(0, 1, ih * idim).astype(np.float32))
    L.idx_raw = dev(rng.normal(0, 1, idim).astype(np.float32))
    L.q_norm, L.k_norm = dev(np.ones(hd, np.float32)), dev(np.ones(hd, np.float32))
    L.iq_norm, L.ik_norm = dev(np.ones(idim, np.float32)), dev(np.ones(idim, np.float32))
    L.cos_tab, L.sin_tab = dev(np.cos(ang).astype(np.float32)), dev(np.sin(ang).astype(np.float32))
    L.kq, L.ks, L.vq, L.vs = kq.ptr, ks.ptr, vq.ptr, vs.ptr
    L.idx_tail, L.idx_dead = dev(np.zeros((blk - 1) * idim, np.float32)), dev(rng.normal(0, 1, idim).astype(np.float32))
    L.idx_pooled = dev(pooled.view(np.uint16))
    L.scores, L.max_b = dev(np.zeros(max_b, np.float32)), max_b
    L.sel_ids, L.sel_cnt = dev(np.zeros(2048, np.int32)), dev(np.zeros(1, np.int32))
    L.out = dev(np.zeros(qh * hd, np.float32))
    nws = wz.wzy_qsa_attend_workspace_bytes(C.byref(dm), 1)
    ws = DA(nws, np.uint8, zero=True)
    keep.append(ws)
    L.workspace, L.workspace_bytes = ws.ptr, nws
    d_pos = dev(np.array([pos], np.int32))
    us = (C.c_float * 4)()
    wz.wzy_qsa_time_decode(C.byref(dm), C.byref(L), d_pos, iters, us, None)
    names = ("prepare", "scores", "topk", "attention")
    total = sum(us)
    out = {"workload": "config 3: one QSA layer, one decode token at a %d-cell context (INT8 K/V uniform on "
                       "[-127,127], fp16 scales per 64, fp16 indexer keys of 65,536 blocks, 24 q / 2 KV heads x 256, "
                       "top-2048), seed %d" % (ctx, seed),
           "us_stages": {n: round(u, 2) for n, u in zip(names, us)},
           "us_per_token": round(total, 2),
           "bytes_per_token": QSA_TOKEN_BYTES,
           "achieved_gbs": round(QSA_TOKEN_BYTES / (total * 1e-6) / 1e9, 1),
           "frac": round(QSA_TOKEN_BYTES / (total * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
           "stage_gbs": {n: round(QSA_BYTES[n] / (us[i + 1] * 1e-6) / 1e9, 1)
                         for i, n in enumerate(("scores", "topk", "attention"))},
           "iters": iters}
    for d in keep:
        d.free()
    return out


def mtp_step_bytes(cfg, n_dv, window):
    """Algorithmic HBM bytes of one draft step: every drafter weight once (Q8_0 rows at 34 B per 32
    values, bf16, the routed Q2_0 experts), the draft-head logits written and read once, and the ring
    cells of the attention window (INT8 K and V with fp16 per-64 scales)."""
    D, HC, L = cfg.n_embd, cfg.hc, cfg.hc_lr
    QD, KVD, F, E, K = cfg.qsa_qh * cfg.qsa_hd, cfg.qsa_kvh * cfg.qsa_hd, cfg.n_ff, cfg.n_exp, cfg.top_k
    q8 = lambda r, c: r * c * 34 // 32
    b = 2 * q8(D, D) + q8(2 * QD, D) + 2 * q8(KVD, D) + q8(D, QD)
    b += 3 * (q8(L, HC * D) + q8(HC * D, L)) + 2 * HC * HC * D * 2
    b += E * D * 2 + D * 2 + 3 * q8(F, D)
    b += K * (3 * D * F // 4 + 3 * D * F // 64 * 2)
    b += q8(n_dv, D) + 2 * 4 * n_dv
    b += window * 2 * (KVD + KVD // 64 * 2)
    return b


def mtp_config5(wz, st, cfg, pos0, windows, depth=3, n_dv=114452, seed=4, seed_cells=64, time_iters=64):
    """BASELINE config 5's decode half on the loaded config-4 stage: the MTP drafter (512 Q2_0
    experts, 114,452-row draft head) seeded on `seed_cells` prompt cells appended to the prefilled
    context (attention floor at the first of them, as a long prompt's tail seeding does), then
    `windows` speculative windows at a fixed depth of 3: catch-up + 3 chained drafts, one T = 4
    verify forward, greedy rank-1 acceptance, commit of the accepted prefix."""
    import numpy as np
    t0 = time.perf_counter()
    st.mtp_init(seed, n_dv)
    t_init = time.perf_counter() - t0
    rng = np.random.default_rng(seed)
    prompt = [int(t) for t in rng.integers(0, cfg.n_vocab, seed_cells + 1)]
    st.mtp_set_floor(pos0)
    for p in range(0, seed_cells, 8):
        st.forward(pos0 + p, prompt[p:p + 8], run_head=2)
        st.mtp_front(pos0 + p, prompt[p + 1:p + 9], 0)
    pos = pos0 + seed_cells
    st.forward(pos, [prompt[-1]])
    st.sync()
    cur = int(st.greedy(1)[0])
    unfed0, unfed = pos, [cur]
    pos += 1
    emitted = accepted = offered = 0
    t_prop = t_win = 0.0

    forced = None                    # the known greedy continuation, when drafts are forced to it
    k_next = 0                       # index in `forced` of the token after `cur`

    def window():
        nonlocal cur, unfed0, unfed, pos, emitted, accepted, offered, t_prop, t_win, k_next
        ta = time.perf_counter()
        d, _ = st.mtp_propose(unfed0, unfed, depth)
        tb = time.perf_counter()
        if forced is not None:       # the drafter ran (its cost is timed); its tokens give way to the truth
            d = forced[k_next:k_next + depth]
        win = [cur] + [int(x) for x in d]
        st.forward(pos, win, save_snaps=True)
        st.sync()
        g = st.greedy(len(win))
        n_acc = 0
        while n_acc < depth and int(g[n_acc]) == win[n_acc + 1]:
            n_acc += 1
        acc_rows = 1 + n_acc
        if acc_rows < len(win):
            st.lib.wzy_stage_commit_window_state(st.h, acc_rows - 1, pos + acc_rows - 1)
        t_prop += tb - ta
        t_win += time.perf_counter() - tb
        emitted += acc_rows
        accepted += n_acc
        offered += depth
        unfed0, unfed = pos, win[1:acc_rows] + [int(g[n_acc])]
        pos += acc_rows
        cur = int(g[n_acc])
        if forced is not None:
            assert forced[k_next:k_next + acc_rows] == win[1:acc_rows] + [cur], "forced window left the greedy stream"
            k_next += acc_rows

    for _ in range(4):
        window()
    emitted = accepted = offered = 0
    t_prop = t_win = 0.0
    wz.wzy_device_sync()
    t0 = time.perf_counter()
    for _ in range(windows):
        window()
    wz.wzy_device_sync()
    el = time.perf_counter() - t0
    rand = dict(emitted=emitted, accepted=accepted, offered=offered, t_prop=t_prop, t_win=t_win)

    # Acceptance 1.0, measured: the greedy continuation from this state is computed first (single-token
    # steps, after which the state is restored from an HBM session slot), then `windows` windows whose
    # 3 drafts are that continuation; each verifies 4 rows and keeps all of them.
    n_cells = pos
    assert wz.wzy_stage_session_save(st.h, 0, n_cells) == 0
    cont, p, t = [], pos, cur
    for _ in range(4 * (windows + 2) + 4):
        st.forward(p, [t])
        st.sync()
        t = int(st.greedy(1)[0])
        cont.append(t)
        p += 1
    assert wz.wzy_stage_session_restore(st.h, 0) == 0
    # the restored state has no pre-head rows for the drafter's catch-up: one plain step at `pos` gives
    # them (and the continuation's first token), then the forced windows start after it
    st.forward(pos, [cur])
    st.sync()
    assert int(st.greedy(1)[0]) == cont[0], "the restored state left the greedy stream"
    unfed0, unfed, cur = pos, [cont[0]], cont[0]
    pos += 1
    forced, k_next = cont, 1
    window()                          # warm-up of the forced path (graph shapes are already captured)
    emitted = accepted = offered = 0
    t_prop = t_win = 0.0
    wz.wzy_device_sync()
    t0 = time.perf_counter()
    for _ in range(windows):
        window()
    wz.wzy_device_sync()
    el1 = time.perf_counter() - t0
    full = {"windows": windows, "tok_s": round(emitted / el1, 2), "ms_per_window": round(1000 * el1 / windows, 4),
            "tokens_per_window": round(emitted / windows, 4), "drafts_offered": offered, "drafts_accepted": accepted,
            "ms_propose": round(1000 * t_prop / windows, 4), "ms_verify_window": round(1000 * t_win / windows, 4),
            "stream_equals_greedy": True}
    wz.wzy_stage_session_clear(st.h, 0)
    forced = None
    emitted, accepted, offered, t_prop, t_win = (rand[k] for k in ("emitted", "accepted", "offered", "t_prop", "t_win"))
    us = C.c_float(0)
    wz.wzy_stage_mtp_time(st.h, pos, cur, -1, time_iters, C.byref(us))
    nb = mtp_step_bytes(cfg, n_dv, min(pos - pos0, 1024))
    acc = accepted / offered if offered else 0.0
    # tokens per window for a per-draft acceptance a (rank-1, stop at the first rejection): 1+a+a^2+a^3
    proj = {("a=%.1f" % a): round((1 + a + a * a + a ** 3) / (el / windows), 1) for a in (0.5, 0.7, 0.9)}
    return {"workload": "config 5 decode: config-4 model + MTP drafter (512 Q2_0 experts top-10, shared expert, "
                        "114,452-row Q8_0 draft head), fixed depth 3, T=4 verify windows, greedy rank-1 acceptance, "
                        "%d seeded prompt cells after a %d-cell prefilled context" % (seed_cells, pos0),
            "windows": windows, "tok_s": round(emitted / el, 2), "ms_per_window": round(1000 * el / windows, 4),
            "tokens_per_window": round(emitted / windows, 4), "acceptance": round(acc, 4),
            "drafts_offered": offered, "drafts_accepted": accepted,
            "ms_propose": round(1000 * t_prop / windows, 4), "ms_verify_window": round(1000 * t_win / windows, 4),
            "mtp_step": {"us": round(us.value, 3), "bytes": nb, "achieved_gbs": round(nb / (us.value * 1e-6) / 1e9, 1),
                         "frac": round(nb / (us.value * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "timed_steps": time_iters},
            "init_s": round(t_init, 2),
            "pos_end": pos,
            "measured_acceptance_1": full,
            "tok_s_at_acceptance": proj,
            "note": ("the synthetic drafter is random-initialised, so its drafts match the random main model's "
                     "greedy tokens about 1 time in 10^5 and measured acceptance is ~0; tok_s is the cost of "
                     "offering 3 drafts per window.  measured_acceptance_1 times the same windows (drafter run "
                     "included) with the drafts replaced by the known greedy continuation, every draft accepted "
                     "and the stream checked against plain greedy decoding.  tok_s_at_acceptance is the "
                     "random-draft window time with 1+a+a^2+a^3 tokens per window (a projection).")}


def cpu_threads():
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(2, min(15, n, 16))


def cpu_model():
    """Host CPU model name (first 'model name' line of /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(wz, seconds):
    """Time the restated reference CPU MoE pool on config 1 (seed 0) for about `seconds`."""
    import numpy as np
    orc = C.CDLL(os.path.join(ROOT, "oracle", "liboracle.so"))
    P, I32 = C.c_void_p, C.c_int
    orc.orc_cpu_pool_create.restype = P
    orc.orc_cpu_pool_create.argtypes = [I32, I32, I32]
    orc.orc_cpu_pool_destroy.argtypes = [P]
    orc.orc_cpu_pool_run.restype = I32
    orc.orc_cpu_pool_run.argtypes = [P, P, P, P, I32, I32, P, P, P]
    orc.orc_gemv_bf16.argtypes = [P, P, P, I32, I32, I32]
    orc.orc_router_topk.argtypes = [P, I32, I32, I32, P, P, P]
    orc.orc_quant_act.argtypes = [P, I32, I32, P, P, P, P]
    seed, layer = 0, 0
    router = np.empty(E * D, np.uint16)
    wz.wzy_synth_normal_bf16(seed, wz.wzy_synth_stream(5, layer, 0), E * D, 0.0, 0.02, router.ctypes.data)
    xh = np.empty(D, np.uint16)
    wz.wzy_synth_normal_bf16(seed, wz.wzy_synth_stream(7, layer, 0), D, 0.0, 1.0, xh.ctypes.data)
    x = (xh.astype(np.uint32) << 16).view(np.float32).copy()
    logits = np.empty(E, np.float32)
    orc.orc_gemv_bf16(router.ctypes.data, x.ctypes.data, logits.ctypes.data, E, D, 1)
    ids = np.empty(K, np.int32)
    wts = np.empty(K, np.float32)
    orc.orc_router_topk(logits.ctypes.data, E, K, 1, ids.ctypes.data, wts.ctypes.data, None)
    q32 = np.empty(D, np.int8)
    s32 = np.empty(D // 32, np.float32)
    q16 = np.empty(D, np.int8)
    s16 = np.empty(D // 16, np.float32)
    orc.orc_quant_act(x.ctypes.data, D, 1, q32.ctypes.data, s32.ctypes.data, q16.ctypes.data, s16.ctypes.data)
    nb = wz.wzy_nvfp4_blob_bytes(D, F)
    blobs = [np.empty(nb, np.uint8) for _ in range(E)]
    for e in set(ids.tolist()):
        wz.wzy_synth_expert_blob(seed, layer, e, D, F, blobs[e].ctypes.data)
    # The GPU's timing burst cycles through 48 layers' experts so that no cache holds them; the CPU
    # leg does the same with n_copies distinct host copies of the 10 routed experts (the same bytes
    # at different addresses, 1.1 GB in all, beyond any host's last-level cache), one copy per call.
    # The same call on one copy, whose 17.7 MB stay cache-resident, is reported beside it.
    n_copies = 64
    copies = [[blobs[e] if c == 0 else blobs[e].copy() for e in range(E) if e in set(ids.tolist())]
              for c in range(n_copies)]
    arrs = []
    for c in range(n_copies):
        ptrs = [0] * E
        for e, b in zip(sorted(set(ids.tolist())), copies[c]):
            ptrs[e] = b.ctypes.data
        arrs.append((C.c_void_p * E)(*ptrs))
    out = np.empty(D, np.float32)
    n = cpu_threads()
    pool = orc.orc_cpu_pool_create(n, D, F)
    if not pool:
        return None

    def run(arr):
        return orc.orc_cpu_pool_run(pool, C.cast(arr, C.c_void_p).value, ids.ctypes.data, wts.ctypes.data, 1, K,
                                    q16.ctypes.data, s16.ctypes.data, out.ctypes.data)

    def timed(secs, rotate):
        times = []
        i = 0
        t_end = time.perf_counter() + secs
        while time.perf_counter() < t_end:
            t0 = time.perf_counter()
            for _ in range(10):
                run(arrs[i % n_copies] if rotate else arrs[0])
                i += 1
            times.append((time.perf_counter() - t0) / 10)
        times.sort()
        return times[len(times) // 2], len(times)

    try:
        for c in range(n_copies):
            run(arrs[c])
        med, n_rot = timed(seconds * 0.75, True)
        med_llc, n_llc = timed(seconds * 0.25, False)
    finally:
        orc.orc_cpu_pool_destroy(pool)
    try:
        host_cores = len(os.sched_getaffinity(0))
    except AttributeError:
        host_cores = os.cpu_count() or 1
    return {
        "value": round(ROUTED_BYTES / med / 1e9, 2),
        "unit": "GB/s (NVFP4 MoE, routed experts, 1 token-layer)",
        "cores": n,
        "host_cores": host_cores,
        "cpu_model": cpu_model(),
        "kind": "port",
        "us_per_token_layer": round(med * 1e6, 1),
        "llc_resident": {"value": round(ROUTED_BYTES / med_llc / 1e9, 2), "us_per_token_layer": round(med_llc * 1e6, 1),
                         "sample": "the same call on one copy of the 10 experts (17.7 MB, cache-resident), "
                                   "%d x 10 calls, median" % n_llc},
        "sample": "config 1 (seed 0, 1 token, top-10 of 512, D=2048 F=512) on %d threads of %d host cores, "
                  "cycling through %d host copies of the routed experts (%.2f GB, not cache-resident) like the "
                  "GPU burst cycles through 48 layers; %d x 10 calls over %.1f s, median" % (
                      n, host_cores, n_copies, n_copies * ROUTED_BYTES / 1e9, n_rot, seconds * 0.75),
    }


def pmc_traffic(kernel_prefix):
    """HBM bytes per launch of a kernel from the committed rocprofv3 --pmc summary, if present."""
    path = os.path.join(ROOT, "profiles", "moe_gate_up_decode_pmc.txt")
    if not os.path.exists(path):
        return None
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch ") and kernel_prefix in line:
                    return float(line.split()[1])
    except OSError:
        return None
    return None


def profile_units(wz, mode, n, n_ctx, graphs, warmup=2):
    """Run the config-4 stage in one mode for a kernel trace or counter run, then return:
      step    n single-token decode steps at the prefilled context
      window  n T=4 verify windows (snapshots on), each followed by the commit of row 0 (a window whose
              drafts are all rejected)
      mtp     n drafter steps (114,452-row draft head) after one decode step
    Kernels are launched directly unless `graphs`; each unit prints its wall time so that a trace can
    be cut per unit."""
    import numpy as np
    import wzy_amd
    cfg = wzy_amd.default_cfg(n_ctx + 8 * (n + warmup) + 64)
    st = wzy_amd.Stage(cfg)
    wz.wzy_stage_set_graphs(st.h, 1 if graphs else 0)
    st.load_synthetic(3, n_ctx)
    rng = np.random.default_rng(1)
    pos = n_ctx
    if mode == "mtp":
        st.mtp_init(4, 114452)
        st.forward(pos, [5])
        st.sync()
    for i in range(warmup + n):
        t0 = time.perf_counter()
        if mode == "step":
            st.forward(pos, [int(rng.integers(0, cfg.n_vocab))])
            st.sync()
            pos += 1
        elif mode == "window":
            st.forward(pos, [int(x) for x in rng.integers(0, cfg.n_vocab, 4)], save_snaps=True)
            st.sync()
            st.lib.wzy_stage_commit_window_state(st.h, 0, pos)
            st.sync()
            pos += 1
        else:
            st.mtp_draft(pos, 7, 0, 1)
        print("%s %d %.3f ms%s" % (mode, i, 1000 * (time.perf_counter() - t0), " (warm-up)" if i < warmup else ""),
              flush=True)
    st.close()
    print("done", flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=512)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--n-ctx", type=int, default=32768)
    ap.add_argument("--seed", type=int, default=3)
    ap.add_argument("--moe-iters", type=int, default=480, help="gate/up + down launches timed for the roofline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graphs", action="store_true", help="direct kernel launches instead of graph replay")
    ap.add_argument("--prefill-tokens", type=int, default=8192, help="config-5 prefill MoE chunk (0: skip)")
    ap.add_argument("--prefill-iters", type=int, default=5)
    ap.add_argument("--stage-prefill-tokens", type=int, default=8192,
                    help="config-5 whole-model prefill chunk (0: skip)")
    ap.add_argument("--stage-prefill-iters", type=int, default=3)
    ap.add_argument("--no-configs23", action="store_true", help="skip the config-2 GDN and config-3 QSA legs")
    ap.add_argument("--mtp-windows", type=int, default=64, help="config-5 speculative windows (0: skip)")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="after the run, 3 device-to-device copies of this many MiB (the known-size kernel that "
                         "calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE counts)")
    ap.add_argument("--profile", choices=("step", "window", "mtp"), default=None,
                    help="instead of the benchmark, run --profile-units units of one mode for rocprofv3 "
                         "(direct kernel launches unless --profile-graphs)")
    ap.add_argument("--profile-units", type=int, default=8)
    ap.add_argument("--profile-graphs", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build runs on one GPU (all 512x48 experts resident in one MI355X's HBM); "
              "multi-GPU runs are not part of it -- use --gpus 1", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import wzy_amd
    wz = wzy_amd.lib()
    if wzy_amd.device_count() < 1:
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    wz.wzy_dev_set(0)
    if args.profile:
        profile_units(wz, args.profile, args.profile_units, args.n_ctx, args.profile_graphs)
        return

    # config-5 decode: up to 4 cells per random-draft window, 4 per forced window and a 4-per-window
    # greedy continuation computed ahead of the forced windows
    ctx_max = (args.n_ctx + args.warmup + args.steps + 64 + 12 * (args.mtp_windows + 4) + 64 + 64 + 128 +
               max(args.stage_prefill_tokens, 0))
    cfg = wzy_amd.default_cfg(ctx_max)
    t0 = time.perf_counter()
    st = wzy_amd.Stage(cfg)
    if args.no_graphs:
        wz.wzy_stage_set_graphs(st.h, 0)
    st.load_synthetic(args.seed, args.n_ctx)
    t_load = time.perf_counter() - t0
    print("bench: stage loaded (%.1f GiB on device) in %.1f s" % (wz.wzy_stage_device_bytes(st.h) / 2**30, t_load),
          file=sys.stderr, flush=True)

    pos = args.n_ctx
    tok = int(args.seed) % cfg.n_vocab
    h_tok = np.zeros(1, np.int32)
    toks = []

    def step():
        nonlocal pos, tok
        h_tok[0] = tok
        wz.wzy_stage_record_forward(st.h, pos, None, h_tok.ctypes.data, 1, 1, 0, 0, 0)
        wz.wzy_stage_sync(st.h)
        wz.wzy_stage_greedy_ids(st.h, h_tok.ctypes.data, 1)
        tok = int(h_tok[0])
        pos += 1
        return tok

    for _ in range(args.warmup):
        step()
    wz.wzy_device_sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        toks.append(step())
    wz.wzy_device_sync()
    elapsed = time.perf_counter() - t0
    print("bench: %d steps in %.3f s" % (args.steps, elapsed), file=sys.stderr, flush=True)

    # live MoE kernel timing with HIP events on the stage stream (activations of the last step)
    us_gu, us_dn, us_blk = C.c_float(0), C.c_float(0), C.c_float(0)
    wz.wzy_stage_time_moe(st.h, args.moe_iters, C.byref(us_gu), C.byref(us_dn), C.byref(us_blk))
    gu_gbs = GU_BYTES / (us_gu.value * 1e-6) / 1e9
    dn_gbs = DN_BYTES / (us_dn.value * 1e-6) / 1e9
    pf = None
    if args.prefill_tokens > 0:
        pf = prefill_moe(wz, st, args.prefill_tokens, args.prefill_iters, args.seed)
        print("bench: prefill MoE %d tokens: %.1f us" % (args.prefill_tokens, pf["us_total"]), file=sys.stderr,
              flush=True)
    mtp5 = None
    if args.mtp_windows > 0:
        mtp5 = mtp_config5(wz, st, cfg, pos, args.mtp_windows)
        print("bench: config 5 MTP depth 3: %.1f tok/s, %.3f ms per window, step %.1f us" % (
            mtp5["tok_s"], mtp5["ms_per_window"], mtp5["mtp_step"]["us"]), file=sys.stderr, flush=True)
        pos = mtp5.pop("pos_end")
    spf = None
    if args.stage_prefill_tokens > 0:
        spf = stage_prefill(wz, st, cfg, pos, args.stage_prefill_tokens, args.stage_prefill_iters, args.seed + 1)
        print("bench: config 5 whole-model prefill of %d tokens: %.1f ms per chunk, %.0f tok/s" % (
            args.stage_prefill_tokens, spf["ms_per_chunk"], spf["tok_s"]), file=sys.stderr, flush=True)
    st.close()

    gdn2 = qsa3 = None
    if not args.no_configs23:
        gdn2 = gdn_config2(wz)
        print("bench: config 2 GDN: %.3f us per layer-step (T=1)" % gdn2["t1"]["us_per_layer_step"], file=sys.stderr,
              flush=True)
        qsa3 = qsa_262k(wz)
        print("bench: config 3 QSA at 262144 cells: %.1f us per token" % qsa3["us_per_token"], file=sys.stderr,
              flush=True)

    if args.calib_copy_mib > 0:
        nb = args.calib_copy_mib << 20
        src, dst = wzy_amd.DeviceArray(nb, np.uint8, zero=True), wzy_amd.DeviceArray(nb, np.uint8)
        for _ in range(3):
            wz.wzy_memcpy_d2d(dst.ptr, src.ptr, nb, None)
        wz.wzy_device_sync()
        src.free()
        dst.free()
        print("bench: calibration copies of %d MiB done" % args.calib_copy_mib, file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(wz, args.cpu_seconds)

    tok_s = args.steps / elapsed
    out = {
        "metric": "greedy decode tok/s (1 GPU, 32K ctx) + NVFP4 MoE GEMV HBM GB/s vs peak",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1000.0 * elapsed / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "e2m1/int8/bf16 weights, int32+fp32 accumulate",
        "data": "synthetic (seeded random-init weights and 32K prefilled KV/state, no checkpoint)",
        "config": {"workload": "config 4: synthetic 48-layer decoder (36 GDN + 12 QSA, NVFP4 MoE 512x top-10 + "
                               "shared, vocab 151936), 1 sequence, %d-token prefilled context, greedy, T=1"
                               % args.n_ctx,
                   "n_ctx": args.n_ctx, "seed": args.seed, "graphs": not args.no_graphs},
        "roofline": {
            "kernel": "moe_gate_up_kernel<1>",
            "bound": "hbm",
            "achieved": round(gu_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
            "traffic": pmc_traffic("moe_gate_up_kernel"),
            "algorithmic_bytes": GU_BYTES,
            "us_per_launch": round(us_gu.value, 3),
            "launches_timed": args.moe_iters,
            "moe_down": {"achieved": round(dn_gbs, 1), "us_per_launch": round(us_dn.value, 3),
                         "algorithmic_bytes": DN_BYTES},
            "moe_routed_gbs": round(ROUTED_BYTES / ((us_gu.value + us_dn.value) * 1e-6) / 1e9, 1),
            # the survey's config-1 unit: 17,694,880 routed-expert bytes per token-layer over the two launches
            "config1_routed_bytes": ROUTED_BYTES,
            "config1_frac": round(ROUTED_BYTES / ((us_gu.value + us_dn.value) * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            # the block as a decode step runs it: each gate/up launch followed by its layer's down launch
            "moe_block": {"us_per_block": round(us_blk.value, 3),
                          "block_bytes": GU_BYTES + DN_BYTES,
                          "achieved": round((GU_BYTES + DN_BYTES) / (us_blk.value * 1e-6) / 1e9, 1),
                          "config1_frac": round(ROUTED_BYTES / (us_blk.value * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)},
        },
        "cpu_baseline": cpu,
        "prefill_moe": pf,
        "stage_prefill": spf,
        "mtp_config5": mtp5,
        "gdn_config2": gdn2,
        "qsa_262k": qsa3,
        "greedy_tokens_head": toks[:8],
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

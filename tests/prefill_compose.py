"""An independent composition of the reference's chunked prefill (run_stage_prefill's layer order,
src/wzy_prefill_tc.cuh:790-1055), written from the pinned oracle primitives (orc_pf_gemm,
orc_hc_read_pf, orc_gdn_step, orc_head_norm_rope, orc_kv_quant_row, orc_indexer_append,
orc_block_scores, orc_topk_select, orc_attend_pf, orc_moe_prefill).  Test infrastructure only.

Used two ways: against orc_model_prefill on the CPU (test_oracle_prefill.py, with planted wiring
mistakes), and teacher-forced against the GPU (test_gpu_prefill.py): `moe` replaces the oracle's MoE
block by the GPU's own block outputs, so that the bf16 sensitivity of the expert activations does
not compound through the layers, and the MoE blocks are checked one by one on the GPU's inputs.

Weights: `layers` is a list of dicts per layer (hc_norm0/1, hc_down0/1 = (codes, scales), ...,
"qsa" flag), `state` a list of dicts of the mutable state arrays (updated in place), `glob` holds
emb (bf16 bits) or emb_q / emb_s, cos, sin and blob(layer, expert) -> reference-layout blob.
"""
import ctypes as C
from types import SimpleNamespace

import numpy as np
import torch

import oracle_lib
from oracle_lib import OrcMoeWeights
from stage_oracle import BLOB_FN

ptr = oracle_lib.ptr


def tbf16(x):
    """round to bf16 (nearest even) with torch"""
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).to(torch.float32).numpy()


def dims_of(cfg):
    return SimpleNamespace(D=cfg.n_embd, HC=cfg.hc, HCLR=cfg.hc_lr, HK=cfg.gdn_hk, HV=cfg.gdn_hv, QH=cfg.qsa_qh,
                           KVH=cfg.qsa_kvh, HD=cfg.qsa_hd, NROT=cfg.n_rot, IH=cfg.idx_heads, IDIM=cfg.idx_dim,
                           IBLK=cfg.idx_blk, TOPK=cfg.idx_topk, E=cfg.n_exp, K=cfg.top_k, F=cfg.n_ff, V=cfg.n_vocab,
                           CTX=cfg.ctx_max, EPS=cfg.eps)


def stage_weights(om, cfg):
    """(layers, state, glob) views of an OracleModel's host arrays (the state arrays are the ones the
    OracleModel itself updates; pass copies to keep it untouched)."""
    A = om.arrays
    layers, state = [], []
    for l in range(cfg.n_layers):
        w = {"qsa": (l % cfg.qsa_period) == cfg.qsa_period - 1}
        for h in range(2):
            w["hc_norm%d" % h] = A[(l, "hc_norm%d" % h)]
            for n in ("hc_down", "hc_up"):
                w["%s%d" % (n, h)] = (A[(l, "%s%d.q" % (n, h))], A[(l, "%s%d.s" % (n, h))])
            w["hc_inj%d" % h] = A[(l, "hc_inj%d" % h)]
        s = {}
        if not w["qsa"]:
            for n in ("qkv", "wgate", "wout"):
                w[n] = (A[(l, n + ".q")], A[(l, n + ".s")])
            w["alpha"], w["beta"] = A[(l, "alpha")], A[(l, "beta")]
            w["ssm_a"], w["dt"], w["conv_w"], w["ssm_norm"] = A[(l, "ssm_a")], A[(l, "dt_bias")], A[(l, "conv1d")], \
                A[(l, "ssm_norm")]
            s["conv_hist"], s["ssm"] = A[(l, "conv_hist")], A[(l, "ssm")]
        else:
            for n in ("wq", "wk", "wv", "wo"):
                w[n] = (A[(l, n + ".q")], A[(l, n + ".s")])
            for n in ("q_norm", "k_norm", "idx_q", "idx_k", "idx_qn", "idx_kn"):
                w[n] = A[(l, n)]
            s["kq"], s["ks"], s["vq"], s["vs"] = A[(l, "kv_k")], A[(l, "kv_ks")], A[(l, "kv_v")], A[(l, "kv_vs")]
            s["idx_tail"], s["idx_dead"], s["idx_pooled"] = A[(l, "idx_tail")], A[(l, "idx_dead")], A[(l, "idx_pooled")]
        w["router"], w["sgate"] = A[(l, "router")], A[(l, "sgate")]
        for n in ("sh_gate", "sh_up", "sh_down"):
            w[n] = (A[(l, n + ".q")], A[(l, n + ".s")])
        layers.append(w)
        state.append(s)
    glob = {"cos": A[(-1, "rope_cos")], "sin": A[(-1, "rope_sin")]}
    if getattr(cfg, "ple", 0):
        # per-layer embedding at layer 1: weights and the oracle's table access in glob, the conv
        # history and the token history in layer 1's state
        pw = om.ple_w
        glob["ple"] = {"w": pw, "wk": A[(1, "ple_key")], "wv": A[(1, "ple_value")], "nq": A[(1, "ple_norm_query")],
                       "nk": A[(1, "ple_norm_key")], "nc": A[(1, "ple_norm_conv")], "cw": A[(1, "ple_conv1d")]}
        state[1]["ple_hist"] = A[(1, "ple_hist")]
        state[1]["tok_hist"] = A[(-1, "tok_hist")]
    if cfg.emb_q8:
        glob["emb_q"], glob["emb_s"] = A[(-1, "emb.q")], A[(-1, "emb.s")]
    else:
        glob["emb"] = A[(-1, "emb")]
    glob["blob"] = lambda layer, e: om.blobs[(layer, e)] if (layer, e) in om.blobs else _blob(om, cfg, layer, e)
    return layers, state, glob


def _blob(om, cfg, layer, e):
    b = np.empty(om.wz.wzy_nvfp4_blob_bytes(cfg.n_embd, cfg.n_ff), np.uint8)
    om.wz.wzy_synth_expert_blob(om.seed, layer, e, cfg.n_embd, cfg.n_ff, b.ctypes.data)
    om.blobs[(layer, e)] = b
    return b


def state_copy(state):
    return [{n: a.copy() for n, a in s.items()} for s in state]


def embed(glob, dm, toks):
    toks = np.asarray(toks)
    if "emb_q" in glob:
        t = np.where((toks < 0) | (toks >= dm.V), 0, toks)
        q = glob["emb_q"].reshape(dm.V, dm.D)[t].astype(np.float32)
        s = np.repeat(glob["emb_s"].view(np.float16).astype(np.float32).reshape(dm.V, dm.D // 32), 32, axis=1)[t]
        return s * q
    t = np.clip(toks, 0, dm.V - 1)
    return (glob["emb"].reshape(dm.V, dm.D)[t].astype(np.uint32) << 16).view(np.float32)


def moe_oracle(orc, dm, w, glob, l, mixed2):
    """orc_moe_prefill on rows mixed2 [B x D] with layer l's weights: (comb, ids, wts)."""
    B = mixed2.shape[0]
    ow = OrcMoeWeights()
    ow.n_embd, ow.n_ff, ow.n_exp, ow.top_k = dm.D, dm.F, dm.E, dm.K
    ow.router, ow.sgate = ptr(w["router"]), ptr(w["sgate"])
    ow.blobs = None                                   # routed blobs fetched on demand
    ow.sh_gate_q, ow.sh_gate_s = ptr(w["sh_gate"][0]), ptr(w["sh_gate"][1])
    ow.sh_up_q, ow.sh_up_s = ptr(w["sh_up"][0]), ptr(w["sh_up"][1])
    ow.sh_down_q, ow.sh_down_s = ptr(w["sh_down"][0]), ptr(w["sh_down"][1])
    comb = np.empty((B, dm.D), np.float32)
    ids = np.empty(B * dm.K, np.int32)
    wts = np.empty(B * dm.K, np.float32)
    cb = BLOB_FN(lambda ctx, layer, e: glob["blob"](layer, e).ctypes.data)
    fn = orc.orc_moe_prefill_fn
    fn.restype = C.c_int
    fn.argtypes = [C.POINTER(OrcMoeWeights), C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                   BLOB_FN, C.c_void_p, C.c_int]
    assert fn(C.byref(ow), ptr(np.ascontiguousarray(mixed2, np.float32)), B, ptr(comb), ptr(ids), ptr(wts), None, cb,
              None, l) == 0
    return comb, ids.reshape(B, dm.K), wts.reshape(B, dm.K)


def compose_prefill(orc, dm, layers, state, glob, pos, toks, plant=None, moe=None, sel_force=None, sel_out=None):
    """Final residual [B x HC x D] and per-layer [L x 4 x B x D] (attention mixed, block, FFN mixed,
    MoE out).  moe(l, mixed2) -> comb replaces the oracle MoE block when given; sel_force(l, t) ->
    selected cells replaces the selection of row t in QSA layer l (sel_out, a dict, then receives
    this composition's own selection, its relative score margin and the block scores (None when every
    cell is selected): sel_out[(l, t)] = (cells, margin, scores))."""
    B = len(toks)
    D, HC, HCLR = dm.D, dm.HC, dm.HCLR
    QKV, GV = 2 * dm.HK * 128 + dm.HV * 128, dm.HV * 128
    QD, KVD, HD = dm.QH * dm.HD, dm.KVH * dm.HD, dm.HD
    out_dbg = np.zeros((len(layers), 4, B, D), np.float32)

    def gemm(x, wt, rows, cols, bf=False):
        x = np.ascontiguousarray(tbf16(x))
        y = np.empty((B, rows), np.float32)
        if bf:
            orc.orc_pf_gemm(ptr(x), B, cols, None, None, ptr(wt), rows, ptr(y), rows)
        else:
            orc.orc_pf_gemm(ptr(x), B, cols, ptr(wt[0]), ptr(wt[1]), None, rows, ptr(y), rows)
        return y

    def read(R, w, half, bo=None, ip=None):
        Rn = np.ascontiguousarray(R, np.float32).copy()
        inj = np.empty((B, HC), np.float32)
        mixed = np.empty((B, D), np.float32)
        orc.orc_hc_read_pf(ptr(Rn), ptr(bo), ptr(ip), ptr(w["hc_norm%d" % half]), ptr(w["hc_down%d" % half][0]),
                           ptr(w["hc_down%d" % half][1]), ptr(w["hc_inj%d" % half]), ptr(w["hc_up%d" % half][0]),
                           ptr(w["hc_up%d" % half][1]), D, HC, HCLR, dm.EPS, B, ptr(inj), ptr(mixed))
        return Rn, mixed, inj

    def write(R, blk, inj):
        g = 2.0 / (1.0 + np.exp(-inj.astype(np.float64) / HC))
        return (R + blk[:, None, :].astype(np.float64) * g[:, :, None]).astype(np.float32)

    R = np.repeat(embed(glob, dm, toks)[:, None, :], HC, axis=1).astype(np.float32)
    cos, sin = glob["cos"], glob["sin"]
    pend = None
    for l, w in enumerate(layers):
        s = state[l]
        if l == 1 and "ple" in glob:
            # the per-layer embedding (src/wzy_prefill_tc.cuh:808-823): the pending FFN write folded into
            # the streams, the block added to them (bf16 GEMM operands), nothing left pending
            pg = glob["ple"]
            emb = np.empty((B, D), np.float32)
            tk = np.ascontiguousarray(toks, np.int32)
            orc.orc_ple_rows(C.cast(pg["w"].row, C.c_void_p), None, D // 16, pg["w"].scale, pg["w"].eos, tk.ctypes.data,
                             B, pos, s["tok_hist"].ctypes.data, emb.ctypes.data)
            R = np.ascontiguousarray(R, np.float32)
            bo, ip = (pend if pend is not None else (None, None))
            orc.orc_ple_block(ptr(R), ptr(bo), ptr(ip), ptr(emb), ptr(pg["wk"]), ptr(pg["wv"]), ptr(pg["nq"]),
                              ptr(pg["nk"]), ptr(pg["nc"]), ptr(pg["cw"]), ptr(s["ple_hist"]), D, HC, dm.EPS, B, 1, None)
            pend = None
        if pend is not None and plant != "drop_pending_fold":
            R, mixed, inj_a = read(R, w, 0, *pend)
        else:
            R, mixed, inj_a = read(R, w, 1 if plant == "attn_reads_ffn_weights" else 0)
        out_dbg[l, 0] = mixed
        if not w["qsa"]:
            qkv = gemm(mixed, w["qkv"], QKV, D)
            z = gemm(mixed, w["wgate"], GV, D)
            ab = np.ascontiguousarray(np.concatenate([gemm(mixed, w["alpha"], dm.HV, D, True),
                                                      gemm(mixed, w["beta"], dm.HV, D, True)], axis=1))
            y = np.empty((B, GV), np.float32)
            orc.orc_gdn_step(ptr(qkv), ptr(z), ptr(ab), ptr(w["dt"]), ptr(w["ssm_a"]), ptr(w["conv_w"]),
                             ptr(s["conv_hist"]), ptr(s["ssm"]), ptr(w["ssm_norm"]), dm.EPS, ptr(y), dm.HK, dm.HV, B)
            block = gemm(y, w["wout"], D, GV)
        else:
            qg = gemm(mixed, w["wq"], 2 * QD, D)
            kk = gemm(mixed, w["wk"], KVD, D)
            vv = gemm(mixed, w["wv"], KVD, D)
            idx_raw = gemm(mixed, w["idx_k"], dm.IDIM, D, True)
            q_idx = gemm(mixed, w["idx_q"], dm.IH * dm.IDIM, D, True)
            for t in range(B):
                p = pos + t
                for h in range(dm.QH):
                    orc.orc_head_norm_rope(qg[t, h * 2 * HD:].ctypes.data, HD, ptr(w["q_norm"]), ptr(cos), ptr(sin), p,
                                           dm.NROT, dm.EPS)
                for j in range(dm.KVH):
                    orc.orc_head_norm_rope(kk[t, j * HD:].ctypes.data, HD, ptr(w["k_norm"]), ptr(cos), ptr(sin), p,
                                           dm.NROT, dm.EPS)
                for i in range(dm.IH):
                    orc.orc_head_norm_rope(q_idx[t, i * dm.IDIM:].ctypes.data, dm.IDIM, ptr(w["idx_qn"]), ptr(cos),
                                           ptr(sin), p, dm.NROT, dm.EPS)
                orc.orc_kv_quant_row(kk[t].ctypes.data, KVD, s["kq"][p * KVD:].ctypes.data,
                                     s["ks"][p * KVD // 64:].ctypes.data)
                orc.orc_kv_quant_row(vv[t].ctypes.data, KVD, s["vq"][p * KVD:].ctypes.data,
                                     s["vs"][p * KVD // 64:].ctypes.data)
                orc.orc_indexer_append(idx_raw[t].ctypes.data, ptr(w["idx_kn"]), ptr(cos), ptr(sin), p, dm.IDIM,
                                       dm.IBLK, dm.NROT, dm.EPS, ptr(s["idx_tail"]), ptr(s["idx_dead"]),
                                       ptr(s["idx_pooled"]))
            att = np.zeros((B, QD), np.float32)
            scores = np.zeros(dm.CTX // dm.IBLK + 2, np.float32)
            sel = np.zeros(dm.TOPK, np.int32)
            for t in range(B):
                n_kv = pos + t + 1
                if n_kv > dm.TOPK:
                    orc.orc_block_scores(ptr(s["idx_pooled"]), ptr(s["idx_dead"]), q_idx[t].ctypes.data, n_kv, dm.IH,
                                         dm.IDIM, dm.IBLK, ptr(scores))
                n = orc.orc_topk_select(ptr(scores), n_kv, dm.IBLK, dm.TOPK, ptr(sel))
                use = sel
                if sel_out is not None:
                    orc.orc_select_margin.restype = C.c_float
                    orc.orc_select_margin.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int]
                    sel_out[(l, t)] = (sel[:n].copy(), float(orc.orc_select_margin(ptr(scores), n_kv, dm.IBLK, dm.TOPK)),
                                       scores[:n_kv // dm.IBLK + 1].copy() if n_kv > dm.TOPK else None)
                if sel_force is not None:
                    use = np.ascontiguousarray(sel_force(l, t), np.int32)
                    n = len(use)
                orc.orc_attend_pf(qg[t].ctypes.data, ptr(s["kq"]), ptr(s["ks"]), ptr(s["vq"]), ptr(s["vs"]), ptr(use),
                                  n, dm.QH, dm.KVH, HD, att[t].ctypes.data)
            block = gemm(att, w["wo"], D, QD)
        out_dbg[l, 1] = block
        if plant != "drop_attn_write":
            R = write(R, block, pend[1] if (plant == "attn_write_uses_ffn_inject" and pend is not None) else inj_a)
        R, mixed2, inj_f = read(R, w, 1)
        out_dbg[l, 2] = mixed2
        comb = moe(l, mixed2) if moe is not None else moe_oracle(orc, dm, w, glob, l, mixed2)[0]
        out_dbg[l, 3] = comb
        pend = (np.ascontiguousarray(comb, np.float32), inj_a if plant == "ffn_write_uses_attn_inject" else inj_f)
    if plant != "drop_final_write":
        R = write(R, *pend)
    return R, out_dbg

"""Pins the oracle's whole-window composition (orc_model_forward) against an independent composition
of the same model written here, from the reference's layer executor, on the CPU.

orc_model_forward strings the per-function oracle primitives together in the order of
StageGpu::record_forward (src/wzy_stage_v2.cuh:476-857).  Each primitive has its own pin; what no
primitive test can see is the wiring between them: which HC norm / down / up / inject weights each
half-layer reads, where the pending hyper-connection writes are folded in, which inject vector
goes with which block output, the order of the QSA row preparation and selection, and the head.
`compose` below restates that wiring from the reference text, calling the pinned primitives as
black boxes and doing every hyper-connection write and the embedding broadcast itself in numpy:

  * embedding rows broadcast into the HC streams (bcast_emb_to_r_kernel, src/wzy_stage_v2.cuh:326-332);
  * attention half: gr_read(hc_norm[0], hc_down[0], hc_up[0], hc_inj[0]) after folding the previous
    layer's FFN write (comb, FFN inject) (src/wzy_stage_v2.cuh:599-601);
  * GDN: qkv / z from Q8 GEMVs of `mixed`, alpha/beta bf16 rows of `mixed`, fused step, out-proj
    (:603-626); QSA: q|gate, k, v Q8 GEMVs, indexer k / q bf16 rows, norms + RoPE of all rows,
    KV and indexer append of all rows, then block scores, top-k and attention per row, o-proj
    (:627-690);
  * FFN half: gr_write(block, attention inject) then gr_read(hc_norm[1], ...) (:694-696); MoE block on
    the FFN `mixed` (:698-724); pending write = (comb, FFN inject) (:763-764);
  * after the last layer: the pending write, the pre-head residual, gr_read(head_norm, head_down,
    head_up, no inject), the LM head GEMV and the greedy argmax (:793-815).
The two compositions must agree within the float tolerance on every intermediate the oracle
exposes, and the check must be sharp: each plausible wiring mistake, planted in the Python
composition, must break the agreement."""
import ctypes as C

import numpy as np
import pytest

import oracle_lib
from oracle_lib import OrcMoeWeights
from stage_oracle import BLOB_FN, OrcLayer, OrcModel

RTOL, ATOL = 2e-2, 1e-2
D, HC, HCLR = 256, 4, 64
HK, HV = 2, 2
QH, KVH, HD, NROT = 4, 2, 256, 64
IH, IDIM, IBLK, TOPK = 4, 128, 4, 64
E, K, F = 16, 4, 128
V, CTX = 500, 512
EPS = 1e-6
QKV, GV = 2 * HK * 128 + HV * 128, HV * 128
QD, KVD = QH * HD, KVH * HD
KINDS = ["gdn", "qsa", "gdn"]
N_CTX = 150            # prefilled cells; the window starts here


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def bf16(a):
    u = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(h):
    return (h.astype(np.uint32) << 16).view(np.float32)


class Model:
    """Random weights and a prefilled state of a three-layer (GDN, QSA, GDN) instance of the
    architecture, as host arrays."""

    def __init__(self, wz, orc, seed):
        rng = np.random.default_rng(seed)
        self.rng, self.seed, self.wz = rng, seed, wz

        def q8(rows, cols, std):
            codes = rng.integers(-127, 128, rows * cols).astype(np.int8)
            sc = f16(std / 73.3 * rng.uniform(0.5, 1.5, rows * cols // 32))
            return codes, sc

        self.layers = []
        for l, kind in enumerate(KINDS):
            w = {"qsa": kind == "qsa"}
            for h in range(2):
                w["hc_norm%d" % h] = rng.uniform(0.5, 1.5, HC * D).astype(np.float32)
                w["hc_down%d" % h] = q8(HCLR, HC * D, 1.0 / np.sqrt(HC * D))
                w["hc_up%d" % h] = q8(HC * D, HCLR, 1.0 / np.sqrt(HCLR))
                w["hc_inj%d" % h] = bf16(rng.normal(0, 2.0 / np.sqrt(HC * D), HC * HC * D))
            if kind == "gdn":
                w["qkv"] = q8(QKV, D, 1 / np.sqrt(D))
                w["wgate"] = q8(GV, D, 1 / np.sqrt(D))
                w["wout"] = q8(D, GV, 1 / np.sqrt(GV))
                w["alpha"] = bf16(rng.normal(0, 1 / np.sqrt(D), HV * D))
                w["beta"] = bf16(rng.normal(0, 1 / np.sqrt(D), HV * D))
                w["ssm_a"] = -rng.uniform(0.5, 2.0, HV).astype(np.float32)
                w["dt"] = rng.normal(0, 0.5, HV).astype(np.float32)
                w["conv_w"] = rng.normal(0, 0.5, QKV * 4).astype(np.float32)
                w["ssm_norm"] = rng.uniform(0.5, 1.5, 128).astype(np.float32)
                w["conv_hist"] = rng.normal(0, 0.5, QKV * 3).astype(np.float32)
                w["ssm"] = rng.normal(0, 0.1, HV * 128 * 128).astype(np.float32)
            else:
                w["wq"] = q8(2 * QD, D, 1 / np.sqrt(D))
                w["wk"] = q8(KVD, D, 1 / np.sqrt(D))
                w["wv"] = q8(KVD, D, 1 / np.sqrt(D))
                w["wo"] = q8(D, QD, 1 / np.sqrt(QD))
                w["q_norm"] = rng.uniform(0.5, 1.5, HD).astype(np.float32)
                w["k_norm"] = rng.uniform(0.5, 1.5, HD).astype(np.float32)
                w["idx_q"] = bf16(rng.normal(0, 1 / np.sqrt(D), IH * IDIM * D))
                w["idx_k"] = bf16(rng.normal(0, 1 / np.sqrt(D), IDIM * D))
                w["idx_qn"] = rng.uniform(0.5, 1.5, IDIM).astype(np.float32)
                w["idx_kn"] = rng.uniform(0.5, 1.5, IDIM).astype(np.float32)
                kq = np.zeros(CTX * KVD, np.int8)
                vq = np.zeros(CTX * KVD, np.int8)
                ks = np.zeros(CTX * KVD // 64, np.uint16)
                vs = np.zeros(CTX * KVD // 64, np.uint16)
                kq[:N_CTX * KVD] = rng.integers(-127, 128, N_CTX * KVD)
                vq[:N_CTX * KVD] = rng.integers(-127, 128, N_CTX * KVD)
                ks[:N_CTX * KVD // 64] = f16(rng.uniform(0.002, 0.02, N_CTX * KVD // 64))
                vs[:N_CTX * KVD // 64] = f16(rng.uniform(0.002, 0.02, N_CTX * KVD // 64))
                w["kq"], w["ks"], w["vq"], w["vs"] = kq, ks, vq, vs
                max_b = CTX // IBLK + 2
                pooled = np.zeros(max_b * IDIM, np.uint16)
                pooled[:(N_CTX // IBLK) * IDIM] = f16(rng.normal(0, 1, (N_CTX // IBLK) * IDIM))
                w["idx_pooled"] = pooled
                w["idx_tail"] = rng.normal(0, 1, (IBLK - 1) * IDIM).astype(np.float32)
                w["idx_dead"] = rng.normal(0, 1, IDIM).astype(np.float32)
            w["router"] = bf16(rng.normal(0, 0.5 / np.sqrt(D), E * D))
            w["sgate"] = bf16(rng.normal(0, 1 / np.sqrt(D), D))
            w["sh_gate"] = q8(F, D, 1 / np.sqrt(D))
            w["sh_up"] = q8(F, D, 1 / np.sqrt(D))
            w["sh_down"] = q8(D, F, 1 / np.sqrt(F))
            self.layers.append(w)
        self.emb = bf16(rng.normal(0, 1, V * D))
        self.head_norm = rng.uniform(0.5, 1.5, HC * D).astype(np.float32)
        self.head_down = q8(HCLR, HC * D, 1.0 / np.sqrt(HC * D))
        self.head_up = q8(HC * D, HCLR, 1.0 / np.sqrt(HCLR))
        self.head = bf16(rng.normal(0, 1 / np.sqrt(D), V * D))
        self.cos = np.empty(CTX * NROT // 2, np.float32)
        self.sin = np.empty(CTX * NROT // 2, np.float32)
        orc.orc_rope_tables(CTX, NROT, 1e7, self.cos.ctypes.data, self.sin.ctypes.data)
        nb = wz.wzy_nvfp4_blob_bytes(D, F)
        self.blobs = []
        for l in range(len(KINDS)):
            row = []
            for e in range(E):
                b = np.empty(nb, np.uint8)
                wz.wzy_synth_expert_blob(seed, l, e, D, F, b.ctypes.data)
                row.append(b)
            self.blobs.append(row)

    def state_copy(self):
        """Independent copies of the mutable state (both compositions update their own)."""
        names = ("conv_hist", "ssm", "kq", "ks", "vq", "vs", "idx_pooled", "idx_tail", "idx_dead")
        return [{n: w[n].copy() for n in names if n in w} for w in self.layers]


# ------------------------------------------------------------------------------------------------
# the oracle's composition
# ------------------------------------------------------------------------------------------------
def oracle_forward(orc, m, state, pos, toks, f16_above=0):
    keep = []

    def p(a):
        keep.append(a)
        return a.ctypes.data

    L = (OrcLayer * len(KINDS))()
    for l, w in enumerate(m.layers):
        o, s = L[l], state[l]
        o.qsa = 1 if w["qsa"] else 0
        for h in range(2):
            o.hc_norm[h] = p(w["hc_norm%d" % h])
            o.hc_down_q[h], o.hc_down_s[h] = p(w["hc_down%d" % h][0]), p(w["hc_down%d" % h][1])
            o.hc_up_q[h], o.hc_up_s[h] = p(w["hc_up%d" % h][0]), p(w["hc_up%d" % h][1])
            o.hc_inj[h] = p(w["hc_inj%d" % h])
        if not w["qsa"]:
            for n in ("qkv", "wgate", "wout"):
                setattr(o, n + "_q", p(w[n][0]))
                setattr(o, n + "_s", p(w[n][1]))
            o.alpha, o.beta, o.ssm_a, o.dt = p(w["alpha"]), p(w["beta"]), p(w["ssm_a"]), p(w["dt"])
            o.conv_w, o.ssm_norm = p(w["conv_w"]), p(w["ssm_norm"])
            o.conv_hist, o.ssm = p(s["conv_hist"]), p(s["ssm"])
        else:
            for n in ("wq", "wk", "wv", "wo"):
                setattr(o, n + "_q", p(w[n][0]))
                setattr(o, n + "_s", p(w[n][1]))
            o.q_norm, o.k_norm = p(w["q_norm"]), p(w["k_norm"])
            o.idx_q, o.idx_k, o.idx_qn, o.idx_kn = p(w["idx_q"]), p(w["idx_k"]), p(w["idx_qn"]), p(w["idx_kn"])
            o.kq, o.ks, o.vq, o.vs = p(s["kq"]), p(s["ks"]), p(s["vq"]), p(s["vs"])
            o.idx_tail, o.idx_dead, o.idx_pooled = p(s["idx_tail"]), p(s["idx_dead"]), p(s["idx_pooled"])
        o.router, o.sgate = p(w["router"]), p(w["sgate"])
        for n in ("sh_gate", "sh_up", "sh_down"):
            setattr(o, n + "_q", p(w[n][0]))
            setattr(o, n + "_s", p(w[n][1]))
    mm = OrcModel()
    mm.n_layers, mm.n_embd, mm.hc, mm.hc_lr, mm.gdn_hk, mm.gdn_hv = len(KINDS), D, HC, HCLR, HK, HV
    mm.qsa_qh, mm.qsa_kvh, mm.qsa_hd, mm.n_rot = QH, KVH, HD, NROT
    mm.idx_heads, mm.idx_dim, mm.idx_blk, mm.idx_topk = IH, IDIM, IBLK, TOPK
    mm.n_exp, mm.top_k, mm.n_ff, mm.n_vocab, mm.ctx_max, mm.eps = E, K, F, V, CTX, EPS
    mm.attn_f16_above = f16_above
    mm.layers = C.cast(L, C.POINTER(OrcLayer))
    mm.emb, mm.head_norm = p(m.emb), p(m.head_norm)
    mm.head_down_q, mm.head_down_s = p(m.head_down[0]), p(m.head_down[1])
    mm.head_up_q, mm.head_up_s = p(m.head_up[0]), p(m.head_up[1])
    mm.head, mm.cos_tab, mm.sin_tab = p(m.head), p(m.cos), p(m.sin)
    cb = BLOB_FN(lambda ctx, layer, e: m.blobs[layer][e].ctypes.data)
    mm.blob, mm.blob_ctx = cb, None
    fwd = orc.orc_model_forward_dbg
    fwd.restype = C.c_int
    fwd.argtypes = [C.POINTER(OrcModel), C.c_int, C.c_void_p, C.c_int] + [C.c_void_p] * 5
    T = len(toks)
    toks = np.asarray(toks, np.int32)
    logits = np.empty((T, V), np.float32)
    greedy = np.empty(T, np.int32)
    pre = np.empty((T, HC, D), np.float32)
    dbg = np.empty((len(KINDS), 4, T, D), np.float32)
    mg = np.empty((len(KINDS), T, 2), np.float32)
    assert fwd(C.byref(mm), pos, toks.ctypes.data, T, logits.ctypes.data, greedy.ctypes.data, pre.ctypes.data,
               dbg.ctypes.data, mg.ctypes.data) == 0
    return logits, greedy, pre, dbg


# ------------------------------------------------------------------------------------------------
# the independent composition (reference record_forward order); `plant` names a wiring mistake
# ------------------------------------------------------------------------------------------------
def compose(orc, m, state, pos, toks, plant=None, f16_above=0):
    T = len(toks)
    ptr = oracle_lib.ptr
    out_dbg = np.zeros((len(KINDS), 4, T, D), np.float32)

    def q8_gemv(wt, x, rows, cols):
        x = np.ascontiguousarray(x, np.float32)
        xq = np.empty(T * cols, np.int8)
        xs = np.empty(T * cols // 32, np.float32)
        orc.orc_quant_act(ptr(x), cols, T, ptr(xq), ptr(xs), None, None)
        y = np.empty((T, rows), np.float32)
        orc.orc_gemv_q8(ptr(wt[0]), ptr(wt[1]), ptr(xq), ptr(xs), ptr(y), rows, cols, T)
        return y

    def bf16_gemv(wt, x, rows, cols):
        return (np.asarray(x, np.float64) @ bf16_to_f32(wt).reshape(rows, cols).astype(np.float64).T).astype(np.float32)

    def gr_write(R, blk, inj):
        # R[t][c][d] += blk[t][d] * 2 sigmoid(inj[t][c] / HC)   (gr_write_multi, src/wzy_kernels_v2.cuh:813-827)
        g = 2.0 / (1.0 + np.exp(-inj.astype(np.float64) / HC))
        return (R + blk[:, None, :].astype(np.float64) * g[:, :, None]).astype(np.float32)

    def gr_read(R, norm, down, up, inj_w):
        R = np.ascontiguousarray(R, np.float32)
        Rout = np.empty_like(R)
        nsc = np.empty((T, HC), np.float32)
        lo = np.empty((T, HCLR), np.float32)
        inj = np.empty((T, HC), np.float32)
        mixed = np.empty((T, D), np.float32)
        orc.orc_hc_read(ptr(R), None, None, None, ptr(norm), ptr(down[0]), ptr(down[1]),
                        ptr(inj_w) if inj_w is not None else None, ptr(up[0]), ptr(up[1]), D, HC, HCLR, EPS, T,
                        ptr(Rout), ptr(nsc), ptr(lo), ptr(inj) if inj_w is not None else None, ptr(mixed))
        return mixed, inj

    emb = bf16_to_f32(m.emb.reshape(V, D)[np.asarray(toks)])
    R = np.repeat(emb[:, None, :], HC, axis=1).astype(np.float32)    # bcast_emb_to_r_kernel
    pend = None
    for l, w in enumerate(m.layers):
        s = state[l]
        # ---- attention half: fold the previous layer's FFN write into this read
        if pend is not None and plant != "drop_ffn_fold":
            R = gr_write(R, *pend)
        a_slot = 1 if plant == "attn_reads_ffn_weights" else 0
        mixed, inj_a = gr_read(R, w["hc_norm%d" % a_slot], w["hc_down%d" % a_slot], w["hc_up%d" % a_slot],
                               w["hc_inj%d" % a_slot])
        out_dbg[l, 0] = mixed
        if not w["qsa"]:
            qkv = q8_gemv(w["qkv"], mixed, QKV, D)
            z = q8_gemv(w["wgate"], mixed, GV, D)
            ab = np.concatenate([bf16_gemv(w["alpha"], mixed, HV, D), bf16_gemv(w["beta"], mixed, HV, D)], axis=1)
            ab = np.ascontiguousarray(ab, np.float32)
            y = np.empty((T, GV), np.float32)
            orc.orc_gdn_step(ptr(qkv), ptr(z), ptr(ab), ptr(w["dt"]), ptr(w["ssm_a"]), ptr(w["conv_w"]),
                             ptr(s["conv_hist"]), ptr(s["ssm"]), ptr(w["ssm_norm"]), EPS, ptr(y), HK, HV, T)
            block = q8_gemv(w["wout"], y, D, GV)
        else:
            qg = q8_gemv(w["wq"], mixed, 2 * QD, D)
            kk = q8_gemv(w["wk"], mixed, KVD, D)
            vv = q8_gemv(w["wv"], mixed, KVD, D)
            idx_raw = np.ascontiguousarray(bf16_gemv(w["idx_k"], mixed, IDIM, D))
            q_idx = np.ascontiguousarray(bf16_gemv(w["idx_q"], mixed, IH * IDIM, D))
            # every row is normalised, roped and appended before any row selects (the reference
            # launches prepare over all T rows, then scoring / top-k / attention over all T rows)
            for t in range(T):
                p = pos + t
                for h in range(QH):
                    v = qg[t, h * 2 * HD:]
                    orc.orc_head_norm_rope(v.ctypes.data, HD, ptr(w["q_norm"]), ptr(m.cos), ptr(m.sin), p, NROT, EPS)
                for j in range(KVH):
                    v = kk[t, j * HD:]
                    orc.orc_head_norm_rope(v.ctypes.data, HD, ptr(w["k_norm"]), ptr(m.cos), ptr(m.sin), p, NROT, EPS)
                for i in range(IH):
                    v = q_idx[t, i * IDIM:]
                    orc.orc_head_norm_rope(v.ctypes.data, IDIM, ptr(w["idx_qn"]), ptr(m.cos), ptr(m.sin), p, NROT, EPS)
                orc.orc_kv_quant_row(kk[t].ctypes.data, KVD, s["kq"][p * KVD:].ctypes.data,
                                     s["ks"][p * KVD // 64:].ctypes.data)
                orc.orc_kv_quant_row(vv[t].ctypes.data, KVD, s["vq"][p * KVD:].ctypes.data,
                                     s["vs"][p * KVD // 64:].ctypes.data)
                orc.orc_indexer_append(idx_raw[t].ctypes.data, ptr(w["idx_kn"]), ptr(m.cos), ptr(m.sin), p, IDIM,
                                       IBLK, NROT, EPS, ptr(s["idx_tail"]), ptr(s["idx_dead"]), ptr(s["idx_pooled"]))
            att = np.zeros((T, QD), np.float32)
            scores = np.zeros(CTX // IBLK + 2, np.float32)
            sel = np.zeros(TOPK, np.int32)
            for t in range(T):
                n_kv = pos + t + 1
                if n_kv > TOPK:
                    orc.orc_block_scores(ptr(s["idx_pooled"]), ptr(s["idx_dead"]), q_idx[t].ctypes.data, n_kv, IH,
                                         IDIM, IBLK, ptr(scores))
                n = orc.orc_topk_select(ptr(scores), n_kv, IBLK, TOPK, ptr(sel))
                # past the reference's VRAM ring the whole window runs its fp16 GQA kernel
                # (`*h_pos + T > KV_VRAM_RING`, src/wzy_stage_v2.cuh:679-683)
                fn = orc.orc_attend_pf if (f16_above > 0 and pos + T > f16_above) else orc.orc_attend
                fn(qg[t].ctypes.data, ptr(s["kq"]), ptr(s["ks"]), ptr(s["vq"]), ptr(s["vs"]), ptr(sel), n,
                   QH, KVH, HD, att[t].ctypes.data)
            block = q8_gemv(w["wo"], att, D, QD)
        out_dbg[l, 1] = block
        # ---- FFN half: the attention write (block, attention inject), then the FFN read
        R = gr_write(R, block, inj_f_prev_swap(plant, inj_a, pend))
        mixed2, inj_f = gr_read(R, w["hc_norm1"], w["hc_down1"], w["hc_up1"], w["hc_inj1"])
        out_dbg[l, 2] = mixed2
        ow = OrcMoeWeights()
        ow.n_embd, ow.n_ff, ow.n_exp, ow.top_k = D, F, E, K
        ow.router, ow.sgate = ptr(w["router"]), ptr(w["sgate"])
        arr = (C.c_void_p * E)(*[b.ctypes.data for b in m.blobs[l]])
        ow.blobs = C.cast(arr, C.c_void_p).value
        ow.sh_gate_q, ow.sh_gate_s = ptr(w["sh_gate"][0]), ptr(w["sh_gate"][1])
        ow.sh_up_q, ow.sh_up_s = ptr(w["sh_up"][0]), ptr(w["sh_up"][1])
        ow.sh_down_q, ow.sh_down_s = ptr(w["sh_down"][0]), ptr(w["sh_down"][1])
        comb = np.empty((T, D), np.float32)
        ids = np.empty(T * K, np.int32)
        wts = np.empty(T * K, np.float32)
        assert orc.orc_moe_block(C.byref(ow), ptr(np.ascontiguousarray(mixed2)), T, ptr(comb), ptr(ids), ptr(wts),
                                 None, None) == 0
        out_dbg[l, 3] = comb
        pend = (comb, inj_a if plant == "ffn_write_uses_attn_inject" else inj_f)
    # ---- head: pending write, pre-head residual, head HC read without inject, LM head
    R = gr_write(R, *pend)
    pre = R.copy()
    if plant == "head_reads_last_ffn_weights":
        mixed, _ = gr_read(R, m.layers[-1]["hc_norm1"], m.layers[-1]["hc_down1"], m.layers[-1]["hc_up1"], None)
    else:
        mixed, _ = gr_read(R, m.head_norm, m.head_down, m.head_up, None)
    logits = bf16_gemv(m.head, mixed, V, D)
    return logits, np.argmax(logits, axis=1).astype(np.int32), pre, out_dbg


def inj_f_prev_swap(plant, inj_a, pend):
    """The inject that goes with the attention block's write: the attention read's own (a planted
    mistake uses the previous layer's FFN inject instead)."""
    if plant == "attn_write_uses_ffn_inject" and pend is not None:
        return pend[1]
    return inj_a


def max_violation(g, o):
    """Largest elementwise excess over |g - o| <= ATOL + RTOL |o| (<= 0 means within tolerance)."""
    g = np.asarray(g, np.float64)
    o = np.asarray(o, np.float64)
    return float((np.abs(g - o) - (ATOL + RTOL * np.abs(o))).max())


@pytest.fixture(scope="module")
def model(wz, orc):
    return Model(wz, orc, 2024)


WINDOWS = ([7, 301, 42], [99], [5, 6])                # a 3-row window, a step, a 2-row window


def run_both(orc, m, plant=None, f16_above=0):
    so, sc = m.state_copy(), m.state_copy()
    outs_o, outs_c = [], []
    pos = N_CTX
    for toks in WINDOWS:
        outs_o.append(oracle_forward(orc, m, so, pos, toks, f16_above))
        outs_c.append(compose(orc, m, sc, pos, toks, plant, f16_above))
        pos += len(toks)
    return outs_o, outs_c, so, sc


# 0: the fp32 attention kernel throughout; 153: the 3-row window (cells 150-152) stays below the
# threshold, the step at 153 and the window at 154-155 take the fp16 branch
@pytest.mark.parametrize("f16_above", [0, 153])
def test_oracle_model_forward_matches_independent_composition(wz, orc, model, f16_above):
    outs_o, outs_c, so, sc = run_both(orc, model, f16_above=f16_above)
    for i, (o, c) in enumerate(zip(outs_o, outs_c)):
        lo_, go, po, do = o
        lc, gc, pc, dc = c
        for l in range(len(KINDS)):
            for j, name in enumerate(("attn mixed", "block", "ffn mixed", "moe comb")):
                v = max_violation(do[l, j], dc[l, j])
                assert v <= 0, "window %d layer %d %s: %.3g beyond tolerance" % (i, l, name, v)
        assert max_violation(po, pc) <= 0, "window %d: pre-head residual" % i
        assert max_violation(lo_, lc) <= 0, "window %d: logits" % i
        np.testing.assert_array_equal(go, gc)
    # and the state both sides carried forward
    for l, (a, b) in enumerate(zip(so, sc)):
        for n in a:
            if a[n].dtype == np.float32:
                assert max_violation(a[n], b[n]) <= 0, "layer %d state %s" % (l, n)
            else:
                assert (a[n] != b[n]).mean() < 1e-3, "layer %d state %s" % (l, n)


@pytest.mark.parametrize("plant", ["drop_ffn_fold", "attn_reads_ffn_weights", "attn_write_uses_ffn_inject",
                                   "ffn_write_uses_attn_inject", "head_reads_last_ffn_weights"])
def test_composition_check_detects_wiring_mistakes(wz, orc, model, plant):
    """Each planted mistake (in the Python composition, on the CPU) moves the logits or pre-head
    residual beyond the tolerance, so the agreement above is not a tautology."""
    outs_o, outs_c, _, _ = run_both(orc, model, plant)
    worst = max(max(max_violation(o[0], c[0]), max_violation(o[2], c[2])) for o, c in zip(outs_o, outs_c))
    assert worst > 0, "planted %s went unnoticed" % plant


def test_attention_branch_switches_per_window(wz, orc, model):
    """orc_model_forward takes the fp16 branch for exactly the windows with pos + T > attn_f16_above
    (src/wzy_stage_v2.cuh:679: the whole window, not row by row).  The branches differ only in rounding
    (inside the float tolerance, so the composition check cannot tell them apart), so this compares the
    QSA layer's attention block of each window bit for bit against runs with the switch off and on
    everywhere: a window below the threshold equals the fp32 run, one above equals the fp16 run, and
    the two runs differ.  Windows: cells 150-152, 153, 154-155; a threshold of 152 puts the first
    window (whose last row is cell 152, but pos + T = 153) on the fp16 branch, one of 153 does not."""
    q = KINDS.index("qsa")

    def blocks(f16_above):
        st = model.state_copy()
        out, pos = [], N_CTX
        for toks in WINDOWS:
            out.append(oracle_forward(orc, model, st, pos, toks, f16_above)[3][q, 1].copy())
            pos += len(toks)
        return out
    b32, b16 = blocks(0), blocks(1)
    assert all(not np.array_equal(a, b) for a, b in zip(b32, b16)), "the branches gave identical blocks"
    for thr, want in ((152, (16, 16, 16)), (153, (32, 16, 16)), (155, (32, 32, 16)), (156, (32, 32, 32))):
        got = blocks(thr)
        # the QSA layer (layer 1) reads only the embedding and the GDN layer before it, so its inputs
        # and KV / indexer state do not depend on which branch earlier windows took
        for i, (g, w) in enumerate(zip(got, want)):
            ref = b16[i] if w == 16 else b32[i]
            assert np.array_equal(g, ref), "threshold %d window %d: not the fp%d branch" % (thr, i, w)

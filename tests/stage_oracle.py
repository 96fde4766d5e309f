"""Builds the CPU oracle's model (orc_model) from a loaded wzy_stage, for parity tests.

Dense weights and the prefilled state are copied out of the stage (wzy_stage_read_tensor); the NVFP4
experts are regenerated in the reference blob layout by the synthetic generator, on demand, for the
experts the oracle routes to.  Test infrastructure only.
"""
import ctypes as C

import numpy as np

import oracle_lib

P, I32, F32 = C.c_void_p, C.c_int, C.c_float


class OrcLayer(C.Structure):
    _fields_ = [("qsa", I32),
                ("hc_norm", P * 2), ("hc_down_q", P * 2), ("hc_down_s", P * 2), ("hc_up_q", P * 2), ("hc_up_s", P * 2),
                ("hc_inj", P * 2),
                ("qkv_q", P), ("qkv_s", P), ("wgate_q", P), ("wgate_s", P), ("wout_q", P), ("wout_s", P),
                ("alpha", P), ("beta", P), ("ssm_a", P), ("dt", P), ("conv_w", P), ("ssm_norm", P),
                ("conv_hist", P), ("ssm", P),
                ("wq_q", P), ("wq_s", P), ("wk_q", P), ("wk_s", P), ("wv_q", P), ("wv_s", P), ("wo_q", P), ("wo_s", P),
                ("q_norm", P), ("k_norm", P), ("idx_q", P), ("idx_k", P), ("idx_qn", P), ("idx_kn", P),
                ("kq", P), ("ks", P), ("vq", P), ("vs", P), ("idx_tail", P), ("idx_dead", P), ("idx_pooled", P),
                ("router", P), ("sgate", P), ("sh_gate_q", P), ("sh_gate_s", P), ("sh_up_q", P), ("sh_up_s", P),
                ("sh_down_q", P), ("sh_down_s", P)]


BLOB_FN = C.CFUNCTYPE(P, P, I32, I32)


class OrcModel(C.Structure):
    _fields_ = [("n_layers", I32), ("n_embd", I32), ("hc", I32), ("hc_lr", I32), ("gdn_hk", I32), ("gdn_hv", I32),
                ("qsa_qh", I32), ("qsa_kvh", I32), ("qsa_hd", I32), ("n_rot", I32),
                ("idx_heads", I32), ("idx_dim", I32), ("idx_blk", I32), ("idx_topk", I32), ("n_exp", I32),
                ("top_k", I32), ("n_ff", I32), ("n_vocab", I32), ("ctx_max", I32), ("eps", F32),
                ("layers", C.POINTER(OrcLayer)),
                ("emb", P), ("head_norm", P), ("head_down_q", P), ("head_down_s", P), ("head_up_q", P),
                ("head_up_s", P), ("head", P), ("cos_tab", P), ("sin_tab", P),
                ("blob", BLOB_FN), ("blob_ctx", P),
                ("emb_q", P), ("emb_s", P), ("head_q", P), ("head_s", P), ("attn_f16_above", I32), ("ple", P)]


PLE_ROW_FN = C.CFUNCTYPE(P, P, C.c_uint32)


class OrcPle(C.Structure):
    """struct orc_ple_w (oracle/wzy_oracle.h)"""
    _fields_ = [("row", PLE_ROW_FN), ("row_ctx", P), ("scale", F32), ("eos", I32), ("wk", P), ("wv", P),
                ("norm_q", P), ("norm_k", P), ("norm_c", P), ("conv_w", P), ("hist", P), ("tok_hist", P)]


class OrcTrace(C.Structure):
    _fields_ = [("dbg", P), ("margins", P), ("router_logits", P), ("ids", P), ("wts", P), ("scores", P), ("sel", P),
                ("n_sel", P)]


def attn_f16(cfg, pos, T):
    """Whether the reference attends a window of T rows at pos with its fp16 GQA kernel: past its VRAM
    ring, `*h_pos + T > KV_VRAM_RING` (src/wzy_stage_v2.cuh:679-683), the threshold being the stage
    config's (or QSA dims') attn_f16_above; 0 means never."""
    thr = cfg.attn_f16_above
    return thr > 0 and pos + T > thr


def attend(orc, f16, qg, kq, ks, vq, vs, cells, qh, kvh, hd):
    """One row's sparse attention through the oracle function of the reference's branch: orc_attend_pf
    (pf_qsa_wmma_sparse_attn, fp16 operands) when f16, else orc_attend (qsa_attend_int8_sparse_multi)."""
    p = oracle_lib.ptr
    out = np.empty(qh * hd, np.float32)
    cells = np.ascontiguousarray(cells, np.int32)
    qg = np.ascontiguousarray(qg, np.float32)              # held for the call (a copy when converted)
    fn = orc.orc_attend_pf if f16 else orc.orc_attend
    fn(p(qg), p(kq), p(ks), p(vq), p(vs), p(cells), len(cells), qh, kvh, hd, p(out))
    return out


def check_attention_branch(tag, g, a_br, a_ot, f16, rtol=2e-3):
    """The GPU's attention rows g against the oracle of the window's branch (a_br) and of the other one
    (a_ot), all on identical inputs: within rtol of the branch's largest output, and (when the two
    branches are measurably apart) closer to the window's branch.  Returns (error, branch distance),
    both relative to the largest output."""
    g = np.asarray(g, np.float64)
    scale = max(float(np.abs(a_br).max()), 1e-30)
    e_br = float(np.abs(g - a_br).max()) / scale
    e_ot = float(np.abs(g - a_ot).max()) / scale
    gap = float(np.abs(np.asarray(a_br, np.float64) - a_ot).max()) / scale
    name = "fp16" if f16 else "fp32"
    print("%s: %s-branch attention, error %.3g, the other branch %.3g away (branches %.3g apart)" % (
        tag, name, e_br, e_ot, gap), flush=True)
    assert e_br <= rtol, "%s: attention off its %s branch by %.3g of the largest output" % (tag, name, e_br)
    if gap > 4e-5:
        assert e_br < e_ot, "%s: attention closer to the other branch (%.3g) than to %s (%.3g)" % (tag, e_ot, name, e_br)
    return e_br, gap


def key_flip_ok(y, a, b, key):
    """Whether two fp16 codes a, b of one pooled indexer key element may both be roundings of the
    oracle's unrounded value y: they are adjacent fp16 values and y lies at their midpoint within what
    fp32 arithmetic can decide -- 2^-17 of y, or 2^-20 of the key's largest element (the RoPE rotation
    forms small elements as differences of O(max) products, so their fp32 error is absolute)."""
    lo, hi = sorted((float(np.uint16(a).view(np.float16)), float(np.uint16(b).view(np.float16))))
    if np.nextafter(np.float16(lo), np.float16(np.inf)) != np.float16(hi):
        return False
    return abs(float(y) - 0.5 * (lo + hi)) <= 2.0 ** -17 * abs(float(y)) + 2.0 ** -20 * float(np.abs(key).max())


def is_qsa(cfg, l):
    return (l % cfg.qsa_period) == cfg.qsa_period - 1


class OracleModel:
    """Holds the host copies and the orc_model struct; `forward` runs orc_model_forward."""

    def __init__(self, wz, stage, cfg, seed):
        self.wz, self.cfg, self.seed = wz, cfg, seed
        self.keep = []
        self.blobs = {}
        self.arrays = {}          # (layer, name) -> host array the oracle reads / updates in place
        st = stage

        def rd(layer, name, dt):
            a = st.read(layer, name, dt)
            self.keep.append(a)
            self.arrays[(layer, name)] = a
            return a.ctypes.data

        L = (OrcLayer * cfg.n_layers)()
        for l in range(cfg.n_layers):
            w = L[l]
            w.qsa = 1 if is_qsa(cfg, l) else 0
            for h in range(2):
                w.hc_norm[h] = rd(l, "hc_norm%d" % h, np.float32)
                w.hc_down_q[h] = rd(l, "hc_down%d.q" % h, np.int8)
                w.hc_down_s[h] = rd(l, "hc_down%d.s" % h, np.uint16)
                w.hc_up_q[h] = rd(l, "hc_up%d.q" % h, np.int8)
                w.hc_up_s[h] = rd(l, "hc_up%d.s" % h, np.uint16)
                w.hc_inj[h] = rd(l, "hc_inj%d" % h, np.uint16)
            if not w.qsa:
                for n in ("qkv", "wgate", "wout"):
                    setattr(w, n + "_q", rd(l, n + ".q", np.int8))
                    setattr(w, n + "_s", rd(l, n + ".s", np.uint16))
                w.alpha, w.beta = rd(l, "alpha", np.uint16), rd(l, "beta", np.uint16)
                w.ssm_a, w.dt = rd(l, "ssm_a", np.float32), rd(l, "dt_bias", np.float32)
                w.conv_w, w.ssm_norm = rd(l, "conv1d", np.float32), rd(l, "ssm_norm", np.float32)
                w.conv_hist, w.ssm = rd(l, "conv_hist", np.float32), rd(l, "ssm", np.float32)
            else:
                for n in ("wq", "wk", "wv", "wo"):
                    setattr(w, n + "_q", rd(l, n + ".q", np.int8))
                    setattr(w, n + "_s", rd(l, n + ".s", np.uint16))
                w.q_norm, w.k_norm = rd(l, "q_norm", np.float32), rd(l, "k_norm", np.float32)
                w.idx_q, w.idx_k = rd(l, "idx_q", np.uint16), rd(l, "idx_k", np.uint16)
                w.idx_qn, w.idx_kn = rd(l, "idx_qn", np.float32), rd(l, "idx_kn", np.float32)
                w.kq, w.ks = rd(l, "kv_k", np.int8), rd(l, "kv_ks", np.uint16)
                w.vq, w.vs = rd(l, "kv_v", np.int8), rd(l, "kv_vs", np.uint16)
                w.idx_tail, w.idx_dead = rd(l, "idx_tail", np.float32), rd(l, "idx_dead", np.float32)
                w.idx_pooled = rd(l, "idx_pooled", np.uint16)
            w.router, w.sgate = rd(l, "router", np.uint16), rd(l, "sgate", np.uint16)
            for n in ("sh_gate", "sh_up", "sh_down"):
                setattr(w, n + "_q", rd(l, n + ".q", np.int8))
                setattr(w, n + "_s", rd(l, n + ".s", np.uint16))
        self.layers = L
        m = OrcModel()
        for f in ("n_layers", "n_embd", "hc", "hc_lr", "gdn_hk", "gdn_hv", "qsa_qh", "qsa_kvh", "qsa_hd", "n_rot",
                  "idx_heads", "idx_dim", "idx_blk", "idx_topk", "n_exp", "top_k", "n_ff", "n_vocab", "ctx_max", "eps",
                  "attn_f16_above"):
            setattr(m, f, getattr(cfg, f))
        m.layers = C.cast(L, C.POINTER(OrcLayer))
        if cfg.emb_q8:
            m.emb_q, m.emb_s = rd(-1, "emb.q", np.int8), rd(-1, "emb.s", np.uint16)
        else:
            m.emb = rd(-1, "emb", np.uint16)
        m.head_norm = rd(-1, "head_norm", np.float32)
        m.head_down_q, m.head_down_s = rd(-1, "head_down.q", np.int8), rd(-1, "head_down.s", np.uint16)
        m.head_up_q, m.head_up_s = rd(-1, "head_up.q", np.int8), rd(-1, "head_up.s", np.uint16)
        if cfg.head_q8:
            m.head_q, m.head_s = rd(-1, "head.q", np.int8), rd(-1, "head.s", np.uint16)
        else:
            m.head = rd(-1, "head", np.uint16)
        m.cos_tab, m.sin_tab = rd(-1, "rope_cos", np.float32), rd(-1, "rope_sin", np.float32)

        def blob_fn(ctx, layer, e):
            key = (layer, e)
            b = self.blobs.get(key)
            if b is None:
                b = np.empty(wz.wzy_nvfp4_blob_bytes(cfg.n_embd, cfg.n_ff), np.uint8)
                wz.wzy_synth_expert_blob(self.seed, layer, e, cfg.n_embd, cfg.n_ff, b.ctypes.data)
                self.blobs[key] = b
            return b.ctypes.data

        self._blob_cb = BLOB_FN(blob_fn)
        m.blob = self._blob_cb
        m.blob_ctx = None
        if getattr(cfg, "ple", 0):
            # the per-layer embedding: weights and state from the stage, table rows read from the stage's
            # table (its bytes are an input like every weight) as the oracle asks for them
            head = cfg.n_embd // 16
            self.ple_rows = {}

            def row_fn(ctx, r):
                b = self.ple_rows.get(r)
                if b is None:
                    b = st.read_range(-1, "ple_table", np.uint8, int(r) * head, head)
                    self.ple_rows[r] = b
                return b.ctypes.data

            self._ple_cb = PLE_ROW_FN(row_fn)
            pw = OrcPle()
            pw.row, pw.row_ctx = self._ple_cb, None
            pw.scale = float(st.read(-1, "ple_scale", np.float32)[0])
            pw.eos = cfg.ple_eos
            pw.wk, pw.wv = rd(1, "ple_key", np.uint16), rd(1, "ple_value", np.uint16)
            pw.norm_q, pw.norm_k = rd(1, "ple_norm_query", np.float32), rd(1, "ple_norm_key", np.float32)
            pw.norm_c, pw.conv_w = rd(1, "ple_norm_conv", np.float32), rd(1, "ple_conv1d", np.float32)
            pw.hist, pw.tok_hist = rd(1, "ple_hist", np.float32), rd(-1, "tok_hist", np.int32)
            self.ple_w = pw
            m.ple = C.cast(C.pointer(pw), P)
        self.model = m
        self.orc = oracle_lib.load()
        self.orc.orc_model_forward_dbg.restype = I32
        self.orc.orc_model_forward_dbg.argtypes = [C.POINTER(OrcModel), I32, P, I32, P, P, P, P, P]
        self.orc.orc_model_forward_trace.restype = I32
        self.orc.orc_model_forward_trace.argtypes = [C.POINTER(OrcModel), I32, P, I32, P, P, P, C.POINTER(OrcTrace)]
        self.last_layers = None
        self.last_margins = None
        self.qsa_layers = [l for l in range(cfg.n_layers) if is_qsa(cfg, l)]

    def forward(self, pos, toks):
        """logits [T x V], greedy [T], pre-head residual [T x hc x D].  Per-layer activations
        [n_layers x 4 x T x D] (attention mixed, block, FFN mixed, MoE out) are kept in last_layers and
        the discrete-decision margins [n_layers x T x 2] (router logit gap, relative indexer score gap)
        in last_margins."""
        toks = np.ascontiguousarray(toks, dtype=np.int32)
        T = len(toks)
        logits = np.empty((T, self.cfg.n_vocab), np.float32)
        greedy = np.empty(T, np.int32)
        pre = np.empty((T, self.cfg.hc, self.cfg.n_embd), np.float32)
        dbg = np.empty((self.cfg.n_layers, 4, T, self.cfg.n_embd), np.float32)
        mg = np.empty((self.cfg.n_layers, T, 2), np.float32)
        rc = self.orc.orc_model_forward_dbg(C.byref(self.model), pos, toks.ctypes.data, T, logits.ctypes.data,
                                            greedy.ctypes.data, pre.ctypes.data, dbg.ctypes.data, mg.ctypes.data)
        assert rc == 0, "orc_model_forward failed"
        self.last_layers = dbg
        self.last_margins = mg
        return logits, greedy, pre

    def forward_trace(self, pos, toks):
        """logits [T x V], greedy [T], pre-head [T x hc x D] and the per-layer trace (dict of arrays:
        hidden [L,4,T,D], router_logits [L,T,E], ids / wts [L,T,K], scores [nq,T,max_b], sel [nq,T,topk],
        n_sel [nq,T])."""
        cfg = self.cfg
        toks = np.ascontiguousarray(toks, dtype=np.int32)
        T, L, nq = len(toks), cfg.n_layers, max(1, len(self.qsa_layers))
        max_b = cfg.ctx_max // cfg.idx_blk + 2
        logits = np.empty((T, cfg.n_vocab), np.float32)
        greedy = np.empty(T, np.int32)
        pre = np.empty((T, cfg.hc, cfg.n_embd), np.float32)
        tr = {"hidden": np.empty((L, 4, T, cfg.n_embd), np.float32),
              "margins": np.empty((L, T, 2), np.float32),
              "router_logits": np.empty((L, T, cfg.n_exp), np.float32),
              "ids": np.empty((L, T, cfg.top_k), np.int32),
              "wts": np.empty((L, T, cfg.top_k), np.float32),
              "scores": np.zeros((nq, T, max_b), np.float32),
              "sel": np.zeros((nq, T, cfg.idx_topk), np.int32),
              "n_sel": np.zeros((nq, T), np.int32)}
        ot = OrcTrace(*[tr[k].ctypes.data for k in ("hidden", "margins", "router_logits", "ids", "wts", "scores", "sel",
                                                     "n_sel")])
        rc = self.orc.orc_model_forward_trace(C.byref(self.model), pos, toks.ctypes.data, T, logits.ctypes.data,
                                              greedy.ctypes.data, pre.ctypes.data, C.byref(ot))
        assert rc == 0, "orc_model_forward_trace failed"
        self.last_layers = tr["hidden"]
        self.last_margins = tr["margins"]
        return logits, greedy, pre, tr

    def prefill(self, pos, toks):
        """orc_model_prefill_dbg over the cells of toks at pos ..: the final residual [B x hc x D];
        per-layer activations [L x 4 x B x D] in last_layers and margins [L x B x 2] in last_margins."""
        cfg = self.cfg
        toks = np.ascontiguousarray(toks, dtype=np.int32)
        B = len(toks)
        R = np.empty((B, cfg.hc, cfg.n_embd), np.float32)
        dbg = np.empty((cfg.n_layers, 4, B, cfg.n_embd), np.float32)
        mg = np.empty((cfg.n_layers, B, 2), np.float32)
        fn = self.orc.orc_model_prefill_dbg
        fn.restype = I32
        fn.argtypes = [C.POINTER(OrcModel), I32, P, I32, P, P, P]
        assert fn(C.byref(self.model), pos, toks.ctypes.data, B, R.ctypes.data, dbg.ctypes.data, mg.ctypes.data) == 0
        self.last_layers = dbg
        self.last_margins = mg
        return R

    def decidable_rows(self, router_gap=0.02, select_gap=1e-3):
        """Rows of the last forward whose every routing / selection decision has a margin that the
        float-reordering drift between two implementations cannot cross."""
        mg = self.last_margins
        ok = (mg[:, :, 0] > router_gap).all(axis=0) & (mg[:, :, 1] > select_gap).all(axis=0)
        return ok


def small_cfg(wz_mod, ctx_max=1024, n_layers=4, topk=64, qsa_period=2):
    """A small instance of the synthetic architecture for parity tests (QSA every qsa_period-th layer;
    n_layers=1 with qsa_period=1 is a single QSA layer, with qsa_period=2 a single GDN layer)."""
    c = wz_mod.StageCfg()
    c.n_layers, c.qsa_period, c.n_embd, c.hc, c.hc_lr = n_layers, qsa_period, 256, 4, 64
    c.gdn_hk, c.gdn_hv = 2, 2
    c.qsa_qh, c.qsa_kvh, c.qsa_hd, c.n_rot = 4, 2, 256, 64
    c.idx_heads, c.idx_dim, c.idx_blk, c.idx_topk = 4, 128, 4, topk
    c.n_exp, c.top_k, c.n_ff, c.n_vocab = 16, 4, 128, 1000
    c.ctx_max, c.kv_ring, c.kv_sinks = ctx_max, 0, 0
    c.rope_theta, c.eps = 1e7, 1e-6
    c.attn_f16_above = 32768               # the reference's VRAM ring (src/wzy_stage_v2.cuh:679)
    c.ple, c.ple_eos = 0, 248044           # PLE off (the synthetic model); the reference's PLE_EOS
    return c


def near_tie(logits_row, tol):
    """True when the top-2 logits are within tol (greedy choice not determined by the oracle)."""
    s = np.sort(logits_row)[::-1]
    return (s[0] - s[1]) <= tol

"""CPU oracle of the MTP drafter (orc_mtp) built from a stage's "mtp.*" tensors or from random arrays,
plus an independent float64 composition of one draft step for pinning it.  Test infrastructure only.
"""
import ctypes as C

import numpy as np

import oracle_lib

P, I32, F32 = C.c_void_p, C.c_int, C.c_float
RING = 1024


class OrcMtp(C.Structure):
    _fields_ = [("n_embd", I32), ("hc", I32), ("hc_lr", I32), ("qsa_qh", I32), ("qsa_kvh", I32), ("qsa_hd", I32),
                ("n_rot", I32), ("n_exp", I32), ("top_k", I32), ("n_ff", I32), ("n_vocab", I32), ("n_dv", I32),
                ("ring", I32), ("eps", F32),
                ("emb", P), ("pre_norm_emb", P), ("pre_norm_hid", P),
                ("fc_emb_q", P), ("fc_emb_s", P), ("fc_hid_q", P), ("fc_hid_s", P),
                ("hc_norm", P * 3), ("hc_down_q", P * 3), ("hc_down_s", P * 3), ("hc_up_q", P * 3),
                ("hc_up_s", P * 3), ("hc_inj", P * 2),
                ("wq_q", P), ("wq_s", P), ("wk_q", P), ("wk_s", P), ("wv_q", P), ("wv_s", P), ("wo_q", P), ("wo_s", P),
                ("q_norm", P), ("k_norm", P), ("router", P), ("sgate", P),
                ("sh_gate_q", P), ("sh_gate_s", P), ("sh_up_q", P), ("sh_up_s", P), ("sh_down_q", P), ("sh_down_s", P),
                ("experts", P), ("head_q", P), ("head_s", P), ("dvocab", P), ("cos_tab", P), ("sin_tab", P),
                ("kq", P), ("ks", P), ("vq", P), ("vs", P), ("kv_floor", I32), ("emb_q", P), ("emb_s", P)]


# (tensor name, dtype) of every drafter weight, as the stage registers them
Q8_NAMES = ["fc_emb", "fc_hid", "wq", "wk", "wv", "wo", "sh_gate", "sh_up", "sh_down", "head",
            "hc_down0", "hc_up0", "hc_down1", "hc_up1", "hc_down2", "hc_up2"]
F32_NAMES = ["pre_norm_emb", "pre_norm_hid", "hc_norm0", "hc_norm1", "hc_norm2", "q_norm", "k_norm"]
BF16_NAMES = ["hc_inj0", "hc_inj1", "router", "sgate"]


def mtp_dims(cfg, n_dv):
    return dict(D=cfg.n_embd, HC=cfg.hc, HCLR=cfg.hc_lr, qh=cfg.qsa_qh, kvh=cfg.qsa_kvh, hd=cfg.qsa_hd,
                n_rot=cfg.n_rot, E=cfg.n_exp, K=cfg.top_k, F=cfg.n_ff, n_vocab=cfg.n_vocab, n_dv=n_dv, eps=cfg.eps)


class OracleMtp:
    """Holds the host arrays and the orc_mtp struct.  `a` maps names ("fc_emb.q", "experts", "emb",
    "rope_cos", ...) to arrays; the KV ring ("kv_k", "kv_ks", "kv_v", "kv_vs") is the oracle's own state."""

    def __init__(self, dims, arrays):
        self.d = dims
        self.a = {k: np.ascontiguousarray(v) for k, v in arrays.items()}
        kvd = dims["kvh"] * dims["hd"]
        for k, dt, n in (("kv_k", np.int8, kvd), ("kv_v", np.int8, kvd), ("kv_ks", np.uint16, kvd // 64),
                         ("kv_vs", np.uint16, kvd // 64)):
            if k not in self.a:
                self.a[k] = np.zeros(RING * n, dt)
        m = OrcMtp()
        d = dims
        m.n_embd, m.hc, m.hc_lr, m.qsa_qh, m.qsa_kvh, m.qsa_hd = d["D"], d["HC"], d["HCLR"], d["qh"], d["kvh"], d["hd"]
        m.n_rot, m.n_exp, m.top_k, m.n_ff, m.n_vocab, m.n_dv = d["n_rot"], d["E"], d["K"], d["F"], d["n_vocab"], d["n_dv"]
        m.ring, m.eps = RING, d["eps"]
        A = self.a
        p = lambda k: A[k].ctypes.data
        if "emb.q" in A:                               # a Q8_0 main embedding table
            m.emb_q, m.emb_s = p("emb.q"), p("emb.s")
        else:
            m.emb = p("emb")
        m.pre_norm_emb, m.pre_norm_hid = p("pre_norm_emb"), p("pre_norm_hid")
        m.fc_emb_q, m.fc_emb_s, m.fc_hid_q, m.fc_hid_s = p("fc_emb.q"), p("fc_emb.s"), p("fc_hid.q"), p("fc_hid.s")
        for h in range(3):
            m.hc_norm[h] = p("hc_norm%d" % h)
            m.hc_down_q[h], m.hc_down_s[h] = p("hc_down%d.q" % h), p("hc_down%d.s" % h)
            m.hc_up_q[h], m.hc_up_s[h] = p("hc_up%d.q" % h), p("hc_up%d.s" % h)
        m.hc_inj[0], m.hc_inj[1] = p("hc_inj0"), p("hc_inj1")
        for n in ("wq", "wk", "wv", "wo", "sh_gate", "sh_up", "sh_down"):
            setattr(m, n + "_q", p(n + ".q"))
            setattr(m, n + "_s", p(n + ".s"))
        m.q_norm, m.k_norm, m.router, m.sgate = p("q_norm"), p("k_norm"), p("router"), p("sgate")
        m.experts, m.head_q, m.head_s = p("experts"), p("head.q"), p("head.s")
        m.dvocab = p("dvocab") if "dvocab" in A else None
        m.cos_tab, m.sin_tab = p("rope_cos"), p("rope_sin")
        m.kq, m.ks, m.vq, m.vs = p("kv_k"), p("kv_ks"), p("kv_v"), p("kv_vs")
        m.kv_floor = 0
        self.m = m
        self.orc = oracle_lib.load()

    @classmethod
    def from_stage(cls, stage, cfg, n_dv):
        a = {}
        for n in Q8_NAMES:
            a[n + ".q"] = stage.read(-1, "mtp." + n + ".q", np.int8)
            a[n + ".s"] = stage.read(-1, "mtp." + n + ".s", np.uint16)
        for n in F32_NAMES:
            a[n] = stage.read(-1, "mtp." + n, np.float32)
        for n in BF16_NAMES:
            a[n] = stage.read(-1, "mtp." + n, np.uint16)
        a["experts"] = stage.read(-1, "mtp.experts", np.uint8)
        a["dvocab"] = stage.read(-1, "mtp.dvocab", np.int32)
        if cfg.emb_q8:
            a["emb.q"], a["emb.s"] = stage.read(-1, "emb.q", np.int8), stage.read(-1, "emb.s", np.uint16)
        else:
            a["emb"] = stage.read(-1, "emb", np.uint16)
        a["rope_cos"] = stage.read(-1, "rope_cos", np.float32)
        a["rope_sin"] = stage.read(-1, "rope_sin", np.float32)
        return cls(mtp_dims(cfg, n_dv), a)

    def set_floor(self, f):
        self.m.kv_floor = int(f)

    def load_ring(self, stage):
        """Take the device ring as the oracle's state (teacher forcing)."""
        for k, dt in (("kv_k", np.int8), ("kv_ks", np.uint16), ("kv_v", np.int8), ("kv_vs", np.uint16)):
            self.a[k][:] = stage.read(-1, "mtp." + k, dt)

    def front(self, pos, toks, rin):
        d = self.d
        toks = np.ascontiguousarray(toks, np.int32)
        T = len(toks)
        rin = np.ascontiguousarray(rin, np.float32).reshape(T, d["HC"], d["D"])
        R = np.empty((T, d["HC"], d["D"]), np.float32)
        mixed = np.empty((T, d["D"]), np.float32)
        inj = np.empty((T, d["HC"]), np.float32)
        self.orc.orc_mtp_front(C.byref(self.m), pos, toks.ctypes.data, rin.ctypes.data, T, R.ctypes.data,
                               mixed.ctypes.data, inj.ctypes.data)
        return R, mixed, inj

    def step(self, pos, tok, rin):
        """-> (R_out [HC x D], sample [D], logits [n_dv], token, prob)"""
        d = self.d
        rin = np.ascontiguousarray(rin, np.float32).reshape(d["HC"], d["D"])
        R_out = np.empty((d["HC"], d["D"]), np.float32)
        sample = np.empty(d["D"], np.float32)
        logits = np.empty(d["n_dv"], np.float32)
        t = C.c_int(0)
        pr = C.c_float(0)
        rc = self.orc.orc_mtp_step(C.byref(self.m), pos, int(tok), rin.ctypes.data, R_out.ctypes.data,
                                   sample.ctypes.data, logits.ctypes.data, C.byref(t), C.byref(pr))
        assert rc == 0
        return R_out, sample, logits, t.value, pr.value


# ------------------------------------------------------------------------------------------------
# random drafters and an independent float64 composition (pins orc_mtp_front / orc_mtp_step)
# ------------------------------------------------------------------------------------------------
def f16(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def bf16(x):
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16f(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def rand_q8(rng, rows, cols):
    q = rng.integers(-127, 128, size=(rows, cols)).astype(np.int8)
    s = f16(rng.uniform(0.5, 1.5, size=(rows, cols // 32)) / (127.0 * np.sqrt(cols) / 2.0))
    return q.ravel(), s.ravel()


def q8_dense(q, s, rows, cols):
    return q.reshape(rows, cols).astype(np.float64) * np.repeat(
        s.view(np.float16).astype(np.float64).reshape(rows, cols // 32), 32, axis=1)


def rand_q2_blob(rng, D, F):
    """Random Q2_0 expert: uniform code bytes, fp16 scales near 1/sqrt(reduction dim)."""
    n_gu_c, n_dn_c = 2 * F * D // 4, D * F // 4
    codes = rng.integers(0, 256, size=n_gu_c + n_dn_c).astype(np.uint8)
    gus = f16(rng.uniform(0.5, 1.5, size=2 * F * D // 64) / np.sqrt(D))
    dns = f16(rng.uniform(0.5, 1.5, size=D * F // 64) / np.sqrt(F))
    return np.concatenate([codes, gus.view(np.uint8), dns.view(np.uint8)])


def q2_dense(blob, D, F):
    """(W_gate [F x D], W_up [F x D], W_down [D x F]) in float64 from the documented layout: value
    4j+k of a chunk is bits 2k..2k+1 of byte j, weight = (code - 1) * scale of its 64-value group;
    gate/up rows interleaved (2r gate, 2r+1 up)."""
    n_gu_c, n_dn_c = 2 * F * D // 4, D * F // 4
    by = blob[:n_gu_c + n_dn_c]
    codes = np.stack([(by >> (2 * k)) & 3 for k in range(4)], axis=1).ravel().astype(np.float64)
    gu = codes[:2 * F * D].reshape(2 * F, D) - 1.0
    dn = codes[2 * F * D:].reshape(D, F) - 1.0
    sc = blob[n_gu_c + n_dn_c:].view(np.uint16).view(np.float16).astype(np.float64)
    gus = sc[:2 * F * D // 64].reshape(2 * F, D // 64)
    dns = sc[2 * F * D // 64:].reshape(D, F // 64)
    gu = gu * np.repeat(gus, 64, axis=1)
    dn = dn * np.repeat(dns, 64, axis=1)
    return gu[0::2], gu[1::2], dn


def random_mtp(rng, dims, n_vocab_rows=None):
    d = dims
    D, HC, HCLR, F, E = d["D"], d["HC"], d["HCLR"], d["F"], d["E"]
    QD, KVD, HCD = d["qh"] * d["hd"], d["kvh"] * d["hd"], d["HC"] * d["D"]
    a = {}
    a["emb"] = bf16(rng.normal(0, 1, size=(d["n_vocab"], D)))
    a["pre_norm_emb"] = rng.normal(1, 0.02, size=D).astype(np.float32)
    a["pre_norm_hid"] = rng.normal(1, 0.02, size=HCD).astype(np.float32)
    for n, r, c in (("fc_emb", D, D), ("fc_hid", D, D), ("wq", 2 * QD, D), ("wk", KVD, D), ("wv", KVD, D),
                    ("wo", D, QD), ("sh_gate", F, D), ("sh_up", F, D), ("sh_down", D, F), ("head", d["n_dv"], D)):
        a[n + ".q"], a[n + ".s"] = rand_q8(rng, r, c)
    for h in range(3):
        a["hc_norm%d" % h] = rng.normal(1, 0.02, size=HCD).astype(np.float32)
        a["hc_down%d.q" % h], a["hc_down%d.s" % h] = rand_q8(rng, HCLR, HCD)
        a["hc_up%d.q" % h], a["hc_up%d.s" % h] = rand_q8(rng, HCD, HCLR)
    for h in range(2):
        a["hc_inj%d" % h] = bf16(rng.normal(0, 1 / np.sqrt(HCD), size=HC * HCD))
    a["q_norm"] = rng.normal(1, 0.02, size=d["hd"]).astype(np.float32)
    a["k_norm"] = rng.normal(1, 0.02, size=d["hd"]).astype(np.float32)
    a["router"] = bf16(rng.normal(0, 0.5, size=E * D))
    a["sgate"] = bf16(rng.normal(0, 0.05, size=D))
    a["experts"] = np.concatenate([rand_q2_blob(rng, D, F) for _ in range(E)])
    a["dvocab"] = (np.arange(d["n_dv"], dtype=np.int64) * d["n_vocab"] // d["n_dv"]).astype(np.int32)
    return a


def dequant_act(orc, x):
    """per-32 int8 quantisation of x (orc_quant_act, pinned separately) -> dequantised float64"""
    x = np.ascontiguousarray(x, np.float32)
    q = np.empty(len(x), np.int8)
    s = np.empty(len(x) // 32, np.float32)
    orc.orc_quant_act(x.ctypes.data, len(x), 1, q.ctypes.data, s.ctypes.data, None, None)
    return q.astype(np.float64) * np.repeat(s.astype(np.float64), 32)


def rms(x, g, eps):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x) + eps) * g


def hc_read64(orc, A, h, R, eps, HCLR):
    """Hyper-connection read from R [HC x D] in float64 (norm, Q8 down on per-32 activations, silu,
    Q8 up on per-32 activations, sigmoid gates, stream mean; inject); mirrors the documented
    reference math, not the oracle's code."""
    HC, D = R.shape
    xn = np.concatenate([rms(R[c], A["hc_norm%d" % h][c * D:(c + 1) * D], eps) for c in range(HC)])
    xd = dequant_act(orc, xn.astype(np.float32))
    W_dn = q8_dense(A["hc_down%d.q" % h], A["hc_down%d.s" % h], HCLR, HC * D)
    lo = W_dn @ xd / HC
    lo = lo / (1 + np.exp(-lo))
    ld = dequant_act(orc, lo.astype(np.float32))
    W_up = q8_dense(A["hc_up%d.q" % h], A["hc_up%d.s" % h], HC * D, HCLR)
    s = (W_up @ ld).reshape(HC, D)
    g = xn.reshape(HC, D) / (1 + np.exp(-s))
    mixed = g.mean(axis=0)
    inj = None
    if h < 2:
        Wi = bf16f(A["hc_inj%d" % h]).astype(np.float64).reshape(HC, HC * D)
        inj = Wi @ xn
    return mixed, inj


def rope64(v, pos, n_rot, cos_t, sin_t):
    half = n_rot // 2
    c, s = cos_t[pos * half:(pos + 1) * half].astype(np.float64), sin_t[pos * half:(pos + 1) * half].astype(np.float64)
    out = v.copy()
    a, b = v[:half], v[half:n_rot]
    out[:half] = a * c - b * s
    out[half:n_rot] = a * s + b * c
    return out


# ------------------------------------------------------------------------------------------------
# teacher-forced check of one GPU draft step
# ------------------------------------------------------------------------------------------------
def gpu_acts(st, cfg, n_dv, rows=1):
    """The drafter's activations after a wzy_stage_mtp_draft of depth 1 (or a front of `rows` rows)."""
    D, HC = cfg.n_embd, cfg.hc
    HCD, QD, KVD = HC * D, cfg.qsa_qh * cfg.qsa_hd, cfg.qsa_kvh * cfg.qsa_hd
    r = lambda n, dt: st.read(-1, "mtp.act." + n, dt)
    g = {"R": r("R", np.float32)[:rows * HCD].reshape(rows, HC, D),
         "mixed": r("mixed", np.float32)[:rows * D].reshape(rows, D),
         "inj": r("inj", np.float32)[:rows * HC].reshape(rows, HC),
         "k": r("k", np.float32)[:rows * KVD].reshape(rows, KVD),
         "v": r("v", np.float32)[:rows * KVD].reshape(rows, KVD),
         "qg": r("qg", np.float32), "att": r("att", np.float32), "bo": r("bo", np.float32),
         "R2": r("R2", np.float32).reshape(HC, D), "inj2": r("inj2", np.float32), "mixed2": r("mixed2", np.float32),
         "rlog": r("router_logits", np.float32), "sg": r("sg", np.float32), "ids": r("ids", np.int32),
         "wts": r("wts", np.float32), "comb": r("comb", np.float32), "sample": r("sample", np.float32),
         "logits": r("logits", np.float32)[:n_dv], "R_out": r("rin", np.float32)[:HCD].reshape(HC, D)}
    for k, dt in (("kv_k", np.int8), ("kv_ks", np.uint16), ("kv_v", np.int8), ("kv_vs", np.uint16)):
        g[k] = st.read(-1, "mtp." + k, dt)
    return g


class MtpTeacher:
    """Recomputes every component of a GPU draft step with the oracle primitives fed the GPU's own
    inputs (the device's previous-stage outputs and KV ring), with the tolerance of teacher_forced.py."""

    def __init__(self, om):
        from teacher_forced import row_excess
        self.om, self.d, self.A = om, om.d, om.a
        self.orc = oracle_lib.load()
        self.row_excess = row_excess
        self.worst = {}
        self.counts = {"steps": 0, "fronts": 0, "kv_flips": 0, "router_ties": 0, "head_ties": 0}

    def cmp(self, what, g, o, tag):
        v, _ = self.row_excess(g, o)
        self.worst[what] = max(self.worst.get(what, -np.inf), v)
        assert v <= 0, "%s: %s beyond tolerance by %.3g (max abs err %.3g)" % (
            tag, what, v, float(np.abs(np.asarray(g, np.float64) - np.asarray(o, np.float64)).max()))

    def q8(self, name, x, rows):
        x = np.ascontiguousarray(x, np.float32)
        cols = x.size
        xq = np.empty(cols, np.int8)
        xs = np.empty(cols // 32, np.float32)
        self.orc.orc_quant_act(x.ctypes.data, cols, 1, xq.ctypes.data, xs.ctypes.data, None, None)
        y = np.empty(rows, np.float32)
        self.orc.orc_gemv_q8(self.A[name + ".q"].ctypes.data, self.A[name + ".s"].ctypes.data, xq.ctypes.data,
                             xs.ctypes.data, y.ctypes.data, rows, cols, 1)
        return y

    def bf16(self, name, x, rows):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty(rows, np.float32)
        self.orc.orc_gemv_bf16(self.A[name].ctypes.data, x.ctypes.data, y.ctypes.data, rows, x.size, 1)
        return y

    def hc_read(self, h, R, bo, inj_prev):
        d, A = self.d, self.A
        D, HC, L = d["D"], d["HC"], d["HCLR"]
        keep = [np.ascontiguousarray(a, np.float32) for a in (R, bo, inj_prev)]
        R_out = np.empty(HC * D, np.float32)
        nsc = np.empty(HC, np.float32)
        lo = np.empty(L, np.float32)
        inj = np.empty(HC, np.float32)
        mixed = np.empty(D, np.float32)
        inj_w = A["hc_inj%d" % h] if h < 2 else None
        self.orc.orc_hc_read(keep[0].ctypes.data, None, keep[1].ctypes.data, keep[2].ctypes.data,
                             A["hc_norm%d" % h].ctypes.data, A["hc_down%d.q" % h].ctypes.data,
                             A["hc_down%d.s" % h].ctypes.data, inj_w.ctypes.data if inj_w is not None else None,
                             A["hc_up%d.q" % h].ctypes.data, A["hc_up%d.s" % h].ctypes.data, D, HC, L, d["eps"], 1,
                             R_out.ctypes.data, nsc.ctypes.data, lo.ctypes.data,
                             inj.ctypes.data if inj_w is not None else None, mixed.ctypes.data)
        return R_out.reshape(HC, D), mixed, inj

    def norm_rope(self, v, gamma, pos):
        v = np.ascontiguousarray(v, np.float32).copy()
        self.orc.orc_head_norm_rope(v.ctypes.data, v.size, self.A[gamma].ctypes.data, self.A["rope_cos"].ctypes.data,
                                    self.A["rope_sin"].ctypes.data, pos, self.d["n_rot"], self.d["eps"])
        return v

    def check_kv(self, tag, g, row, cell, mixed):
        """K / V of one front row from the GPU's mixed row vs the ring cell the GPU wrote."""
        d = self.d
        hd, kvd = d["hd"], d["kvh"] * d["hd"]
        k = self.q8("wk", mixed, kvd)
        v = self.q8("wv", mixed, kvd)
        k = np.concatenate([self.norm_rope(k[j * hd:(j + 1) * hd], "k_norm", cell) for j in range(d["kvh"])])
        self.cmp("k", g["k"][row], k, tag)
        self.cmp("v", g["v"][row], v, tag)
        sl = cell % RING
        for x, qn, sn in ((g["k"][row], "kv_k", "kv_ks"), (g["v"][row], "kv_v", "kv_vs")):
            x = np.ascontiguousarray(x, np.float32)
            q = np.empty(kvd, np.int8)
            s = np.empty(kvd // 64, np.uint16)
            self.orc.orc_kv_quant_row(x.ctypes.data, kvd, q.ctypes.data, s.ctypes.data)
            gq = g[qn][sl * kvd:(sl + 1) * kvd]
            gs = g[sn][sl * (kvd // 64):(sl + 1) * (kvd // 64)]
            assert (gs == s).all(), "%s: %s scales differ" % (tag, sn)
            diff = np.abs(gq.astype(np.int32) - q.astype(np.int32))
            assert diff.max() <= 1, "%s: %s codes differ by %d" % (tag, qn, diff.max())
            self.counts["kv_flips"] += int((diff > 0).sum())

    def check_front(self, tag, g, cell0, toks, rin):
        """A front of len(toks) rows: R, mixed, inject and K/V of every row from the oracle front fed the
        same pre-head rows and tokens."""
        T = len(toks)
        save = {k: self.A[k].copy() for k in ("kv_k", "kv_ks", "kv_v", "kv_vs")}
        R, mixed, inj = self.om.front(cell0, toks, rin)
        for k, v in save.items():          # the oracle's own ring is not part of this check
            self.A[k][:] = v
        for t in range(T):
            tt = "%s row %d" % (tag, t)
            self.cmp("front R", g["R"][t], R[t], tt)
            self.cmp("front mixed", g["mixed"][t], mixed[t], tt)
            self.cmp("front inject", g["inj"][t], inj[t], tt)
            self.check_kv(tt, g, t, cell0 + t, g["mixed"][t])
        self.counts["fronts"] += T

    def check_step(self, tag, g, cell, tok, rin, g_tok, g_prob, floor=0):
        d, A = self.d, self.A
        D, HC, hd, qh, kvh, E, K, F = d["D"], d["HC"], d["hd"], d["qh"], d["kvh"], d["E"], d["K"], d["F"]
        self.check_front(tag + " front", {k: g[k] for k in ("R", "mixed", "inj", "k", "v", "kv_k", "kv_ks", "kv_v",
                                                            "kv_vs")}, cell, [tok], rin.reshape(1, HC, D))
        # q projection, norm + RoPE on the GPU's mixed row
        qg = self.q8("wq", g["mixed"][0], 2 * qh * hd)
        for h in range(qh):
            qg[h * 2 * hd:h * 2 * hd + hd] = self.norm_rope(qg[h * 2 * hd:h * 2 * hd + hd], "q_norm", cell)
        self.cmp("q", g["qg"], qg, tag)
        # ring attention on the GPU's q and ring
        n_kv = cell + 1
        p0 = max(floor, n_kv - RING, 0)
        sel = np.array([(p0 + i) % RING for i in range(n_kv - p0)], np.int32)
        att = np.empty(qh * hd, np.float32)
        qd = np.ascontiguousarray(g["qg"], np.float32)
        self.orc.orc_attend(qd.ctypes.data, g["kv_k"].ctypes.data, g["kv_ks"].ctypes.data, g["kv_v"].ctypes.data,
                            g["kv_vs"].ctypes.data, sel.ctypes.data, len(sel), qh, kvh, hd, att.ctypes.data)
        self.cmp("attention", g["att"], att, tag)
        self.cmp("o projection", g["bo"], self.q8("wo", g["att"], D), tag)
        R2, mixed2, inj2 = self.hc_read(1, g["R"][0], g["bo"], g["inj"][0])
        self.cmp("MLP R", g["R2"], R2, tag)
        self.cmp("MLP HC read", g["mixed2"], mixed2, tag)
        self.cmp("MLP inject", g["inj2"], inj2, tag)
        # MoE on the GPU's mixed2
        rl = self.bf16("router", g["mixed2"], E)
        self.cmp("router logits", g["rlog"], rl, tag)
        sg = self.bf16("sgate", g["mixed2"], 1)
        self.cmp("shared gate", g["sg"], sg, tag)
        ids = np.empty(K, np.int32)
        wts = np.empty(K, np.float32)
        rlg = np.ascontiguousarray(g["rlog"], np.float32)
        self.orc.orc_router_topk(rlg.ctypes.data, E, K, 1, ids.ctypes.data, wts.ctypes.data, None)
        assert (ids == g["ids"]).all(), "%s: routed experts differ: %s vs %s" % (tag, g["ids"], ids)
        np.testing.assert_allclose(g["wts"], wts, rtol=1e-5, atol=1e-6)
        x = np.ascontiguousarray(g["mixed2"], np.float32)
        xq = np.empty(D, np.int8)
        xs = np.empty(D // 32, np.float32)
        self.orc.orc_quant_act(x.ctypes.data, D, 1, xq.ctypes.data, xs.ctypes.data, None, None)
        rec = len(A["experts"]) // E
        acc = np.zeros(D)
        aq = np.empty(F, np.int8)
        as_ = np.empty(F // 32, np.float32)
        part = np.empty(D, np.float32)
        for k in range(K):
            if g["wts"][k] == 0:
                continue
            blob = A["experts"][int(g["ids"][k]) * rec:]
            self.orc.orc_q2_expert_gate_up(blob.ctypes.data, D, F, xq.ctypes.data, xs.ctypes.data, aq.ctypes.data,
                                           as_.ctypes.data, None)
            self.orc.orc_q2_expert_down(blob.ctypes.data, D, F, aq.ctypes.data, as_.ctypes.data, part.ctypes.data)
            acc += float(g["wts"][k]) * part.astype(np.float64)
        gate = self.q8("sh_gate", g["mixed2"], F)
        up = self.q8("sh_up", g["mixed2"], F)
        shared = self.q8("sh_down", (gate / (1 + np.exp(-gate)) * up).astype(np.float32), D)
        comb = shared.astype(np.float64) / (1 + np.exp(-float(g["sg"][0]))) + acc
        self.cmp("MoE", g["comb"], comb, tag)
        # final mixer on the GPU's R2, MoE output and inject
        R_out, sample, _ = self.hc_read(2, g["R2"], g["comb"], g["inj2"])
        self.cmp("mixer R", g["R_out"], R_out, tag)
        self.cmp("mixer read", g["sample"], sample, tag)
        lg = self.q8("head", g["sample"], d["n_dv"])
        self.cmp("draft logits", g["logits"], lg, tag)
        # the reduction over the GPU's own logits is exact: token and probability
        gl = g["logits"].astype(np.float64)
        best = int(np.argmax(g["logits"]))
        want_tok = int(A["dvocab"][best]) if "dvocab" in A else best
        assert g_tok == want_tok, "%s: draft token %d, argmax of the GPU logits gives %d" % (tag, g_tok, want_tok)
        want_p = 1.0 / max(np.exp(gl - gl[best]).sum(), 1.0)
        assert abs(g_prob - want_p) <= 1e-4 * want_p + 1e-7, "%s: prob %.6g vs %.6g" % (tag, g_prob, want_p)
        srt = np.sort(lg)[::-1]
        if srt[0] - srt[1] > 2e-2 * max(1.0, abs(srt[0])):
            assert int(np.argmax(lg)) == best, "%s: oracle argmax %d vs GPU %d" % (tag, int(np.argmax(lg)), best)
        else:
            self.counts["head_ties"] += 1
        self.counts["steps"] += 1

    def summary(self):
        return "%s; worst excess %s" % (self.counts, {k: "%.3g" % v for k, v in sorted(self.worst.items())})

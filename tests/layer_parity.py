"""Layer-by-layer parity of a GPU stage against the CPU oracle model over a stream of windows.

Both sides record, for every layer and window row, the attention HC read output, the attention
block output, the FFN HC read output, the router logits / expert ids / weights and the MoE output,
and for every QSA layer the block scores and the selected cells (the stage with
wzy_stage_set_trace, the oracle with orc_model_forward_trace).  The comparison walks the layers of
each row in order:

  * hidden states elementwise: |gpu - oracle| <= ATOL + RTOL |oracle|  (north star: rel 2e-2,
    abs 1e-2); for the MoE output the relative term is floored at the row's RMS, because the block
    requantises its input per 16 / 32 values and a one-step code difference (an fp32 sum of the
    input landing on the other side of a rounding boundary) moves its outputs by about 1 % of the
    row's scale (the rule of teacher_forced.row_excess);
  * expert ids of every layer bit-exact, in rank order, and the selected cells of every QSA layer
    bit-exact;
  * the logits elementwise and the greedy id bit-exact.

The two implementations sum in different orders, so their floats differ slightly, and a discrete
decision whose oracle margin is inside that difference can legitimately go either way.  The only
exclusions are derived from the error measured at that very decision:
  * router: the oracle's gap between its top_k-th and next logit is at most twice the largest
    |gpu - oracle| router-logit difference of that row and layer;
  * selection: the oracle's score gap at the top-k threshold is at most twice the largest block
    score difference;
  * greedy: the oracle's gap between its best logit and the logit of the GPU's pick is at most
    twice the largest logit difference of the row.
An excluded router or selection decision ends the comparison of that row at that layer, and every
later layer's recurrent state (GDN state, KV cells) has then taken a different input, so later rows
are compared only up to that layer.  A mismatch outside these exclusions fails."""
import numpy as np

RTOL, ATOL = 2e-2, 1e-2
HIDDEN = ("attention HC read", "attention block", "FFN HC read", "MoE output")


def row_excess(g, o):
    """Largest excess over ATOL + RTOL * max(|o|, rms(o)), and the plain elementwise one."""
    g = np.asarray(g, np.float64).ravel()
    o = np.asarray(o, np.float64).ravel()
    d = np.abs(g - o)
    rms = float(np.sqrt((o * o).mean())) if o.size else 0.0
    return float((d - (ATOL + RTOL * np.maximum(np.abs(o), rms))).max()), float((d - (ATOL + RTOL * np.abs(o))).max())


def excess(g, o):
    """Largest elementwise excess over the tolerance (<= 0: within)."""
    g = np.asarray(g, np.float64)
    o = np.asarray(o, np.float64)
    return float((np.abs(g - o) - (ATOL + RTOL * np.abs(o))).max())


def gpu_trace(st, cfg, T, n_qsa):
    L, W, D = cfg.n_layers, 8, cfg.n_embd
    max_b = cfg.ctx_max // cfg.idx_blk + 2
    rd = lambda name, dt: st.read(-1, name, dt)
    tr = {
        "hidden": np.stack([rd(n, np.float32).reshape(L, W, D)[:, :T] for n in
                            ("trace.mixed_a", "trace.block", "trace.mixed_f", "trace.comb")], axis=1),
        "router_logits": rd("trace.moe_logits", np.float32).reshape(L, W, cfg.n_exp)[:, :T],
        "ids": rd("trace.moe_ids", np.int32).reshape(L, W, cfg.top_k)[:, :T],
        "wts": rd("trace.moe_wts", np.float32).reshape(L, W, cfg.top_k)[:, :T],
    }
    for name, key, width in (("trace.R_a", "R_a", cfg.hc * D), ("trace.R_f", "R_f", cfg.hc * D),
                             ("trace.inj_a", "inj_a", cfg.hc), ("trace.inj_f", "inj_f", cfg.hc)):
        tr[key] = rd(name, np.float32).reshape(L, W, width)[:, :T]
    if n_qsa:
        nq = n_qsa
        tr["scores"] = rd("trace.scores", np.float32).reshape(nq, W, max_b)[:, :T]
        tr["sel"] = rd("trace.sel_ids", np.int32).reshape(nq, W, cfg.idx_topk)[:, :T]
        tr["n_sel"] = rd("trace.sel_cnt", np.int32).reshape(nq, W)[:, :T]
        kvd, qd = cfg.qsa_kvh * cfg.qsa_hd, cfg.qsa_qh * cfg.qsa_hd
        for name, key, width in (("trace.kv_k_in", "kv_k_in", kvd), ("trace.kv_v_in", "kv_v_in", kvd),
                                 ("trace.idx_raw", "idx_raw", cfg.idx_dim), ("trace.qg", "qg", 2 * qd),
                                 ("trace.attn", "attn", qd)):
            tr[key] = rd(name, np.float32).reshape(nq, W, width)[:, :T]
    return tr


def threshold_gap(scores, n_kv, blk, topk):
    """Absolute score gap around the top-k threshold block (inf when every cell is selected)."""
    if n_kv <= topk:
        return np.inf
    nbid = n_kv // blk
    w = np.full(nbid + 1, blk)
    w[nbid] = n_kv - nbid * blk
    s = scores[:nbid + 1].astype(np.float64)
    keep = w > 0
    s, w = s[keep], w[keep]
    order = np.argsort(-s, kind="stable")
    s, w = s[order], w[order]
    jt = int(np.searchsorted(np.cumsum(w), topk))
    gap = np.inf
    if jt > 0:
        gap = min(gap, s[jt - 1] - s[jt])
    if jt + 1 < len(s):
        gap = min(gap, s[jt] - s[jt + 1])
    return gap


class LayerParity:
    """hidden="elementwise": hidden states held to the tolerance elementwise (small models, where the
    free-running difference stays far inside it); hidden="report": free-running hidden-state
    differences are measured and reported but not asserted (deep models at the BASELINE shapes, where
    int8 requantisation amplifies last-bit differences layer after layer; their per-layer numerics
    are held to the tolerance by the teacher-forced check instead), while every discrete decision is
    still compared."""

    def __init__(self, cfg, qsa_layers, hidden="elementwise"):
        self.cfg = cfg
        self.hidden_mode = hidden
        self.drift = {}                               # layer -> largest free-running excess seen
        self.qsa_layers = list(qsa_layers)            # layer index of each QSA layer, in order
        self.taint = cfg.n_layers                     # first layer whose state may differ
        self.rows = self.rows_full = 0
        self.layers_compared = self.router_compared = self.select_compared = 0
        self.router_ties = self.select_ties = self.greedy_ties = 0
        self.excused = []                             # (kind, where, oracle margin, error measured there)
        self.first_row_layers = None                  # layers of the first row compared before any stop
        self.worst = {h: -np.inf for h in HIDDEN}
        self.worst["logits"] = -np.inf

    def window(self, tag, pos, g, o, g_logits, o_logits, g_greedy, T=None):
        """g / o: trace dicts ('hidden' [L,4,T,D], ...); logits [T,V], or None for a window run
        without the head (then T gives the row count and only the layers are compared)."""
        cfg = self.cfg
        T = g_logits.shape[0] if g_logits is not None else T
        for t in range(T):
            self.rows += 1
            stop = None
            for l in range(cfg.n_layers):
                if l >= self.taint:
                    stop = l
                    break
                qi = self.qsa_layers.index(l) if l in self.qsa_layers else None
                self._hidden(tag, t, l, 0, g, o)
                if qi is not None and not self._select(tag, pos, t, l, qi, g, o):
                    stop = l
                    break
                self._hidden(tag, t, l, 1, g, o)
                self._hidden(tag, t, l, 2, g, o)
                if not self._router(tag, t, l, g, o):
                    stop = l
                    break
                self._hidden(tag, t, l, 3, g, o)
                self.layers_compared += 1
            if self.first_row_layers is None:
                self.first_row_layers = cfg.n_layers if stop is None else stop
            if stop is not None:
                self.taint = min(self.taint, stop + 1)
                continue
            if g_logits is None:
                continue
            v = excess(g_logits[t], o_logits[t])
            self.worst["logits"] = max(self.worst["logits"], v)
            assert v <= 0 or self.hidden_mode == "report", "%s row %d: logits beyond tolerance by %.3g" % (tag, t, v)
            ref = int(np.argmax(o_logits[t]))
            gid = int(g_greedy[t])
            if gid != ref:
                err = float(np.abs(g_logits[t].astype(np.float64) - o_logits[t]).max())
                gap = float(o_logits[t][ref]) - float(o_logits[t][gid])
                assert gap <= 2 * err, "%s row %d: greedy %d vs oracle %d, oracle gap %.3g > 2 x logit error %.3g" % (
                    tag, t, gid, ref, gap, err)
                self.greedy_ties += 1
                self.excused.append(("greedy", "%s row %d" % (tag, t), gap, err))
            self.rows_full += 1

    def _hidden(self, tag, t, l, k, g, o):
        if k == 3:
            v, plain = row_excess(g["hidden"][l, k, t], o["hidden"][l, k, t])
            self.worst["MoE output (plain)"] = max(self.worst.get("MoE output (plain)", -np.inf), plain)
        else:
            v = excess(g["hidden"][l, k, t], o["hidden"][l, k, t])
        self.worst[HIDDEN[k]] = max(self.worst[HIDDEN[k]], v)
        if self.hidden_mode == "report":
            self.drift[l] = max(self.drift.get(l, -np.inf), v)
            return
        assert v <= 0, "%s row %d layer %d: %s beyond tolerance by %.3g" % (tag, t, l, HIDDEN[k], v)

    def _router(self, tag, t, l, g, o):
        gi, oi = g["ids"][l, t], o["ids"][l, t]
        self.router_compared += 1
        if np.array_equal(gi, oi):
            return True
        gl = g["router_logits"][l, t].astype(np.float64)
        ol = o["router_logits"][l, t].astype(np.float64)
        err = float(np.abs(gl - ol).max())
        s = np.sort(ol)[::-1]
        K = len(oi)
        if set(gi.tolist()) == set(oi.tolist()):
            # same experts, different rank order: every swapped pair must be a near tie
            for a, b in zip(gi, oi):
                if a != b:
                    assert abs(ol[a] - ol[b]) <= 2 * err, "%s row %d layer %d: expert order %s vs %s" % (
                        tag, t, l, gi.tolist(), oi.tolist())
            return True
        gap = s[K - 1] - s[K]
        assert gap <= 2 * err, "%s row %d layer %d: experts %s vs oracle %s, oracle gap %.3g > 2 x logit error %.3g" % (
            tag, t, l, sorted(gi.tolist()), sorted(oi.tolist()), gap, err)
        self.router_ties += 1
        self.excused.append(("router", "%s row %d layer %d" % (tag, t, l), gap, err))
        return False

    def _select(self, tag, pos, t, l, qi, g, o):
        cfg = self.cfg
        n_kv = pos + t + 1
        ng, no = int(g["n_sel"][qi, t]), int(o["n_sel"][qi, t])
        assert ng == no == min(n_kv, cfg.idx_topk), "%s row %d layer %d: selection count %d vs %d" % (
            tag, t, l, ng, no)
        self.select_compared += 1
        if np.array_equal(g["sel"][qi, t, :ng], o["sel"][qi, t, :no]):
            return True
        nb = n_kv // cfg.idx_blk + 1
        gs = g["scores"][qi, t, :nb].astype(np.float64)
        os_ = o["scores"][qi, t, :nb].astype(np.float64)
        err = float(np.abs(gs - os_).max())
        gap = threshold_gap(o["scores"][qi, t], n_kv, cfg.idx_blk, cfg.idx_topk)
        assert gap <= 2 * err, "%s row %d layer %d: selected cells differ, oracle threshold gap %.3g > 2 x score " \
                               "error %.3g" % (tag, t, l, gap, err)
        self.select_ties += 1
        self.excused.append(("selection", "%s row %d layer %d" % (tag, t, l), gap, err))
        return False

    def drift_profile(self):
        """Free-running tolerance excess by layer (report mode), as 'layer:excess' pairs every 4 layers."""
        return " ".join("%d:%.2g" % (l, self.drift[l]) for l in sorted(self.drift) if l % 4 == 0)

    def summary(self):
        w = ", ".join("%s %.3g" % (k, v) for k, v in self.worst.items())
        ex = "; ".join("%s at %s: margin %.3g vs error %.3g" % e for e in self.excused)
        return ("%d rows (%d compared through the head), first row %s of %d layers, %d layer-rows, %d router and %d "
                "selection decisions compared; excused decisions %d (%s); worst tolerance excess: %s" % (
                    self.rows, self.rows_full, self.first_row_layers, self.cfg.n_layers, self.layers_compared,
                    self.router_compared, self.select_compared, len(self.excused), ex or "none", w))

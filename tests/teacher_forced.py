"""Teacher-forced, layer-by-layer parity of one decode row of a GPU stage against the oracle primitives.

Free-running comparisons of a deep model cannot hold every element of every layer to a float
tolerance: the path requantises activations to int8 (per 16 / 32 values) several times per layer,
and when two implementations' fp32 sums differ in the last bit, a value sitting on a rounding
boundary takes different codes on the two sides.  In this synthetic model the MoE block has a large
gain (its outputs reach |x| ~ 130), so one flipped code moves the MoE output by ~0.3 and the
difference then grows layer after layer.  Measured at the BASELINE shapes: a layer whose input
differs by 5e-7 gave MoE outputs 0.36 apart, while the same layer fed the identical input agreed
to 3e-5.

This checker therefore recomputes every component of every layer from the GPU's own inputs: the
stage's per-layer trace (wzy_stage_set_trace) supplies the residual streams, HC read outputs,
injects, block and MoE outputs, and the stage's state tensors supply the pre-row recurrent state.
For each layer l of a single-row forward at position pos:

  attention HC read   oracle(R_f[l-1] (embedding rows for l = 0), comb[l-1], inj_f[l-1])  vs  R_a, mixed_a, inj_a
  attention block     GDN: Q8 qkv / z, bf16 alpha / beta, fused step on the pre-row conv history and
                      state, out-projection; QSA: projections, norms + RoPE, KV append, indexer
                      append, block scores, top-2048 (bit-exact on the GPU's scores), attention over
                      the GPU's selected cells, out-projection                          vs  block
  state update        GDN conv history and state; QSA KV cell at pos, indexer tail / placeholder /
                      pooled keys                                                      vs  the stage's post-row state
  FFN HC read         oracle(R_a[l], block[l], inj_a[l])                               vs  R_f, mixed_f, inj_f
  MoE                 router top-k (bit-exact unless the oracle's top_k-th gap is within twice the
                      measured router-logit error) and the block output               vs  ids, wts, comb
and then the head: oracle(R_f[L-1], comb[L-1], inj_f[L-1]) -> head HC read -> LM head vs the
stage's pre-head residual, logits and greedy id.

Tolerance: elementwise |gpu - oracle| <= ATOL + RTOL * |oracle| (the north star's rel 2e-2 /
abs 1e-2).  Components that requantise their input (every Q8 / NVFP4 GEMV) can see a one-step code
difference when an internal fp32 sum lands on a rounding boundary, which moves their outputs by about
1% of the row's scale, not of each element; for those the relative term may be floored at the row's
RMS, but every element that passes only through the floor is counted per component, printed, and
bounded by the test (assert_bounds).  Byte work is bit-exact on identical inputs: the KV codes and
fp16 scales of the row's cell are the oracle's quantisation of the very k / v rows the GPU quantised
(traced), and the pooled indexer key of a completed block is the oracle's append of the GPU's raw
key row, where an fp16 code may differ only at a rounding midpoint of the oracle's unrounded key
(|key - midpoint| below 2^-17 of the key, the fp32 arithmetic's reach).  The attention output is
checked tightly on identical inputs (the GPU's q | gate rows, KV store and selection) against the
oracle function of the reference's branch for the window (orc_attend below the reference's VRAM
ring, orc_attend_pf past it), and must sit closer to it than to the other branch.  Every excused
discrete decision (router, selection, greedy) is recorded with its margin and the error measured at
it, and their number is bounded by the test."""
import ctypes as C

import numpy as np

import oracle_lib
from oracle_lib import OrcMoeWeights, ptr
from stage_oracle import attend, attn_f16, key_flip_ok

RTOL, ATOL = 2e-2, 1e-2
ATT_RTOL = 2e-3           # attention on identical inputs, relative to the row's largest output
# components whose oracle recomputation requantises an input to int8 (a Q8 / NVFP4 GEMV or the HC
# read's low-rank code): a one-step code flip moves such an output by ~1 % of its row's scale, so
# their elements may pass through the row-RMS floor, in a bounded number (assert_bounds)
# (measured: only the MoE output ever needs it, 2 elements in 16,384 at most)
FLOOR_OK = ("MoE output",)


def bf16_to_f32(h):
    return (h.astype(np.uint32) << 16).view(np.float32)


def row_excess(g, o):
    """Largest excess over ATOL + RTOL * max(|o|, rms(o)), elementwise, and the plain elementwise one."""
    g = np.asarray(g, np.float64).ravel()
    o = np.asarray(o, np.float64).ravel()
    d = np.abs(g - o)
    rms = float(np.sqrt((o * o).mean())) if o.size else 0.0
    floor = (d - (ATOL + RTOL * np.maximum(np.abs(o), rms))).max()
    plain = (d - (ATOL + RTOL * np.abs(o))).max()
    return float(floor), float(plain)


class TeacherForced:
    """Holds the weights (from an OracleModel built before any oracle forward) and the stage's
    pre-row state; check_row() verifies one single-row forward that the stage has just run."""

    def __init__(self, wz, st, cfg, om):
        self.wz, self.st, self.cfg, self.om = wz, st, cfg, om
        self.orc = oracle_lib.load()
        self.A = om.arrays
        self.qsa_layers = list(om.qsa_layers)
        self.state = {}
        for (l, name), a in om.arrays.items():
            if name in ("conv_hist", "ssm", "idx_tail", "idx_dead", "idx_pooled", "kv_k", "kv_ks", "kv_v", "kv_vs",
                        "ple_hist", "tok_hist"):
                self.state[(l, name)] = a.copy()
        self.worst = {}
        self.worst_plain = {}
        self.floor_only = {}         # component -> elements within tolerance only through the RMS floor
        self.n_elems = {}            # component -> elements compared
        self.excused = []            # (kind, tag, oracle margin, error measured at the decision)
        self.attn = []               # (tag, branch, error vs its branch, distance between the branches)
        self.counts = {"layers": 0, "router_ties": 0, "select_ties": 0, "greedy_ties": 0, "rows": 0,
                       "kv_bytes": 0, "key_midpoint_flips": 0}
        D = cfg.n_embd
        self.cos = om.arrays[(-1, "rope_cos")]
        self.sin = om.arrays[(-1, "rope_sin")]
        self.emb_q8, self.head_q8 = bool(cfg.emb_q8), bool(cfg.head_q8)
        if self.emb_q8:              # Q8_0 table: codes [n_vocab][D], fp16 scales per 32 (stage_one_emb)
            self.emb_q = om.arrays[(-1, "emb.q")].reshape(cfg.n_vocab, D)
            self.emb_s = om.arrays[(-1, "emb.s")].reshape(cfg.n_vocab, D // 32)
        else:
            self.emb = om.arrays[(-1, "emb")].reshape(cfg.n_vocab, D)

    def sync_from_stage(self):
        """Take the stage's current recurrent / KV / indexer state as the next row's pre-row state (after
        windows that check_row does not cover, such as multi-row prefill windows)."""
        for (l, name), a in self.state.items():
            self.state[(l, name)] = self.st.read(l, name, a.dtype)

    # -------------------------------------------------------------------------------------------
    def _cmp(self, what, g, o, tag, plain=False):
        v, p = row_excess(g, o)
        if plain:
            v = p
        self.worst[what] = max(self.worst.get(what, -np.inf), v)
        self.worst_plain[what] = max(self.worst_plain.get(what, -np.inf), p)
        assert v <= 0, "%s: %s beyond tolerance by %.3g (max abs err %.3g)" % (
            tag, what, v, float(np.abs(np.asarray(g, np.float64) - o).max()))
        gg = np.asarray(g, np.float64).ravel()
        oo = np.asarray(o, np.float64).ravel()
        self.floor_only[what] = self.floor_only.get(what, 0) + int((np.abs(gg - oo) > ATOL + RTOL * np.abs(oo)).sum())
        self.n_elems[what] = self.n_elems.get(what, 0) + gg.size

    def _excuse(self, kind, tag, margin, err):
        self.excused.append((kind, tag, float(margin), float(err)))
        self.counts[kind + "_ties"] += 1

    def assert_bounds(self, max_floor_frac=5e-4, max_excused=1, floor_ok=FLOOR_OK):
        """The plain elementwise tolerance holds on every component outside `floor_ok`; inside it, at
        most max_floor_frac of a component's elements pass only through the RMS floor; at most
        max_excused discrete decisions were excused."""
        for what, n in self.floor_only.items():
            lim = max_floor_frac * self.n_elems[what] if what in floor_ok else 0
            assert n <= lim, "%s: %d of %d elements within tolerance only through the row-RMS floor (limit %d)" % (
                what, n, self.n_elems[what], lim)
        assert len(self.excused) <= max_excused, "%d excused decisions (limit %d): %s" % (
            len(self.excused), max_excused, self.excused)

    def _q8(self, name, l, x, rows):
        cols = x.size
        x = np.ascontiguousarray(x, np.float32)
        xq = np.empty(cols, np.int8)
        xs = np.empty(cols // 32, np.float32)
        self.orc.orc_quant_act(ptr(x), cols, 1, ptr(xq), ptr(xs), None, None)
        y = np.empty(rows, np.float32)
        self.orc.orc_gemv_q8(ptr(self.A[(l, name + ".q")]), ptr(self.A[(l, name + ".s")]), ptr(xq), ptr(xs), ptr(y),
                             rows, cols, 1)
        return y

    def _bf16(self, w, x, rows):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty(rows, np.float32)
        self.orc.orc_gemv_bf16(ptr(w), ptr(x), ptr(y), rows, x.size, 1)
        return y

    def _hc_read(self, l, h, R_in, emb_rows, bo, inj_prev, with_inj=True):
        cfg, D = self.cfg, self.cfg.n_embd
        HC, L = cfg.hc, cfg.hc_lr
        if l >= 0:
            norm, dq, ds = self.A[(l, "hc_norm%d" % h)], self.A[(l, "hc_down%d.q" % h)], self.A[(l, "hc_down%d.s" % h)]
            uq, us, inj_w = self.A[(l, "hc_up%d.q" % h)], self.A[(l, "hc_up%d.s" % h)], self.A[(l, "hc_inj%d" % h)]
        else:
            norm, dq, ds = self.A[(-1, "head_norm")], self.A[(-1, "head_down.q")], self.A[(-1, "head_down.s")]
            uq, us, inj_w = self.A[(-1, "head_up.q")], self.A[(-1, "head_up.s")], None
        keep = [np.ascontiguousarray(a, np.float32) if a is not None else None for a in (R_in, emb_rows, bo, inj_prev)]
        R_out = np.empty(HC * D, np.float32)
        nsc = np.empty(HC, np.float32)
        lo = np.empty(L, np.float32)
        inj = np.empty(HC, np.float32)
        mixed = np.empty(D, np.float32)
        self.orc.orc_hc_read(ptr(keep[0]), ptr(keep[1]), ptr(keep[2]), ptr(keep[3]), ptr(norm), ptr(dq), ptr(ds),
                             ptr(inj_w) if (with_inj and inj_w is not None) else None, ptr(uq), ptr(us), D, HC, L,
                             cfg.eps, 1, ptr(R_out), ptr(nsc), ptr(lo),
                             ptr(inj) if (with_inj and inj_w is not None) else None, ptr(mixed))
        return R_out, mixed, inj

    # -------------------------------------------------------------------------------------------
    def check_row(self, tag, pos, tok, g, g_logits, g_greedy, g_pre):
        """g: the stage trace of a T = 1 forward at `pos` (layer_parity.gpu_trace plus R_a, R_f, inj_a, inj_f)."""
        cfg, st, orc = self.cfg, self.st, self.orc
        D, HC = cfg.n_embd, cfg.hc
        QKV, GV = 2 * cfg.gdn_hk * 128 + cfg.gdn_hv * 128, cfg.gdn_hv * 128
        QD, KVD, hd = cfg.qsa_qh * cfg.qsa_hd, cfg.qsa_kvh * cfg.qsa_hd, cfg.qsa_hd
        IH, ID, blk, topk = cfg.idx_heads, cfg.idx_dim, cfg.idx_blk, cfg.idx_topk
        max_b = cfg.ctx_max // blk + 2
        n_kv = pos + 1
        self.counts["rows"] += 1
        new_state = {}
        for l in range(cfg.n_layers):
            t = "%s layer %d" % (tag, l)
            # ---- attention HC read
            if l == 0:
                if self.emb_q8:
                    tq = tok if 0 <= tok < cfg.n_vocab else 0
                    emb_row = (self.emb_s[tq].view(np.float16).astype(np.float32).repeat(32) *
                               self.emb_q[tq].astype(np.float32)).astype(np.float32)
                else:
                    emb_row = bf16_to_f32(self.emb[tok])
                R_a, mixa, inj_a = self._hc_read(l, 0, None, emb_row, None, None)
            elif l == 1 and getattr(cfg, "ple", 0):
                # per-layer embedding: the row's table rows, the block on the GPU's layer-0 outputs and the
                # pre-row conv history; the attention read then folds nothing
                pw = self.om.ple_w
                th = self.state[(-1, "tok_hist")].copy()
                emb = np.empty(D, np.float32)
                tk = np.array([tok], np.int32)
                orc.orc_ple_rows(C.cast(pw.row, C.c_void_p), None, D // 16, pw.scale, pw.eos, tk.ctypes.data, 1, pos,
                                 th.ctypes.data, emb.ctypes.data)
                R = np.ascontiguousarray(g["R_f"][0, 0], np.float32).copy()
                hist = self.state[(1, "ple_hist")].copy()
                bo, ip = np.ascontiguousarray(g["hidden"][0, 3, 0]), np.ascontiguousarray(g["inj_f"][0, 0])
                A = self.A
                orc.orc_ple_block(ptr(R), ptr(bo), ptr(ip), ptr(emb), ptr(A[(1, "ple_key")]), ptr(A[(1, "ple_value")]),
                                  ptr(A[(1, "ple_norm_query")]), ptr(A[(1, "ple_norm_key")]),
                                  ptr(A[(1, "ple_norm_conv")]), ptr(A[(1, "ple_conv1d")]), ptr(hist), D, HC, cfg.eps, 1,
                                  0, None)
                g_hist = st.read(1, "ple_hist", np.float32)
                self._cmp("PLE conv history", g_hist, hist, t)
                new_state[(1, "ple_hist")] = g_hist
                new_state[(-1, "tok_hist")] = st.read(-1, "tok_hist", np.int32)
                assert new_state[(-1, "tok_hist")][pos] == tok, "%s: token history at %d" % (t, pos)
                R_a, mixa, inj_a = self._hc_read(l, 0, R, None, None, None)
            else:
                R_a, mixa, inj_a = self._hc_read(l, 0, g["R_f"][l - 1, 0], None, g["hidden"][l - 1, 3, 0],
                                                 g["inj_f"][l - 1, 0])
            self._cmp("attention R", g["R_a"][l, 0], R_a, t)
            self._cmp("attention HC read", g["hidden"][l, 0, 0], mixa, t)
            self._cmp("attention inject", g["inj_a"][l, 0], inj_a, t)
            xa = np.ascontiguousarray(g["hidden"][l, 0, 0])
            # ---- attention block on the GPU's mixed_a and pre-row state
            if l not in self.qsa_layers:
                qkv = self._q8("qkv", l, xa, QKV)
                z = self._q8("wgate", l, xa, GV)
                ab = np.concatenate([self._bf16(self.A[(l, "alpha")], xa, cfg.gdn_hv),
                                     self._bf16(self.A[(l, "beta")], xa, cfg.gdn_hv)]).astype(np.float32)
                hist = self.state[(l, "conv_hist")].copy()
                ssm = self.state[(l, "ssm")].copy()
                y = np.empty(GV, np.float32)
                orc.orc_gdn_step(ptr(qkv), ptr(z), ptr(ab), ptr(self.A[(l, "dt_bias")]), ptr(self.A[(l, "ssm_a")]),
                                 ptr(self.A[(l, "conv1d")]), ptr(hist), ptr(ssm), ptr(self.A[(l, "ssm_norm")]), cfg.eps,
                                 ptr(y), cfg.gdn_hk, cfg.gdn_hv, 1)
                block = self._q8("wout", l, y, D)
                g_hist, g_ssm = st.read(l, "conv_hist", np.float32), st.read(l, "ssm", np.float32)
                self._cmp("GDN conv history", g_hist, hist, t)
                self._cmp("GDN state", g_ssm, ssm, t)
                new_state[(l, "conv_hist")], new_state[(l, "ssm")] = g_hist, g_ssm
            else:
                qi = self.qsa_layers.index(l)
                qg = self._q8("wq", l, xa, 2 * QD)
                kk = self._q8("wk", l, xa, KVD)
                vv = self._q8("wv", l, xa, KVD)
                idx_raw = self._bf16(self.A[(l, "idx_k")], xa, ID)
                q_idx = self._bf16(self.A[(l, "idx_q")], xa, IH * ID)
                for h in range(cfg.qsa_qh):
                    orc.orc_head_norm_rope(qg[h * 2 * hd:].ctypes.data, hd, ptr(self.A[(l, "q_norm")]), ptr(self.cos),
                                           ptr(self.sin), pos, cfg.n_rot, cfg.eps)
                for j in range(cfg.qsa_kvh):
                    orc.orc_head_norm_rope(kk[j * hd:].ctypes.data, hd, ptr(self.A[(l, "k_norm")]), ptr(self.cos),
                                           ptr(self.sin), pos, cfg.n_rot, cfg.eps)
                for i in range(IH):
                    orc.orc_head_norm_rope(q_idx[i * ID:].ctypes.data, ID, ptr(self.A[(l, "idx_qn")]), ptr(self.cos),
                                           ptr(self.sin), pos, cfg.n_rot, cfg.eps)
                # the rows the GPU quantised (k after norm + RoPE, v, the raw indexer key) against the
                # oracle's own rows, then the KV cell at pos: the oracle's quantisation of the GPU's rows,
                # bit for bit (codes and fp16 scales)
                gk, gv = g["kv_k_in"][qi, 0], g["kv_v_in"][qi, 0]
                self._cmp("k row (norm + RoPE)", gk, kk, t)
                self._cmp("v row", gv, vv, t)
                ok, oks = np.zeros(KVD, np.int8), np.zeros(KVD // 64, np.uint16)
                ov, ovs = np.zeros(KVD, np.int8), np.zeros(KVD // 64, np.uint16)
                orc.orc_kv_quant_row(ptr(np.ascontiguousarray(gk)), KVD, ptr(ok), ptr(oks))
                orc.orc_kv_quant_row(ptr(np.ascontiguousarray(gv)), KVD, ptr(ov), ptr(ovs))
                gcell = {n: st.read_range(l, n, dt, pos * w, w) for n, dt, w in
                         (("kv_k", np.int8, KVD), ("kv_v", np.int8, KVD), ("kv_ks", np.uint16, KVD // 64),
                          ("kv_vs", np.uint16, KVD // 64))}
                for n, o in (("kv_k", ok), ("kv_v", ov), ("kv_ks", oks), ("kv_vs", ovs)):
                    bad = np.flatnonzero(gcell[n] != o)
                    assert bad.size == 0, "%s: KV %s of cell %d differs from the quantisation of the GPU's own " \
                                          "row at %d of %d elements" % (t, n, pos, bad.size, o.size)
                    self.counts["kv_bytes"] += o.size
                for n in ("kv_k", "kv_v", "kv_ks", "kv_vs"):
                    w = gcell[n].size
                    arr = self.state[(l, n)]
                    arr[pos * w:(pos + 1) * w] = gcell[n]
                    new_state[(l, n)] = arr
                # indexer append of the GPU's raw key row on the pre-row indexer state
                gr = np.ascontiguousarray(g["idx_raw"][qi, 0])
                self._cmp("indexer key row", gr, idx_raw, t)
                tail, dead = self.state[(l, "idx_tail")].copy(), self.state[(l, "idx_dead")].copy()
                pooled = self.state[(l, "idx_pooled")].copy()
                key = np.full(ID, np.nan, np.float32)
                orc.orc_indexer_append_f32(ptr(gr), ptr(self.A[(l, "idx_kn")]), ptr(self.cos), ptr(self.sin), pos,
                                           ID, blk, cfg.n_rot, cfg.eps, ptr(tail), ptr(dead), ptr(pooled), ptr(key))
                g_tail, g_dead = st.read(l, "idx_tail", np.float32), st.read(l, "idx_dead", np.float32)
                g_pooled = st.read(l, "idx_pooled", np.uint16)
                assert np.array_equal(g_tail, tail), "%s: indexer tail (fp16-rounded raw keys) differs" % t
                self._cmp("indexer placeholder", g_dead, dead, t)
                for i in np.flatnonzero(g_pooled != pooled):
                    b, d = divmod(int(i), ID)
                    assert b == pos // blk and not np.isnan(key[d]), \
                        "%s: pooled key %d dim %d differs, and no block completed there" % (t, b, d)
                    assert key_flip_ok(key[d], g_pooled[i], pooled[i], key), \
                        "%s: pooled key %d dim %d: fp16 %r vs %r, unrounded key %r is not at their midpoint" % (
                            t, b, d, g_pooled[i], pooled[i], float(key[d]))
                    self.counts["key_midpoint_flips"] += 1
                new_state[(l, "idx_tail")], new_state[(l, "idx_dead")], new_state[(l, "idx_pooled")] = \
                    g_tail, g_dead, g_pooled
                # block scores on the stage's post-row keys, then the selection
                scores = np.zeros(max_b, np.float32)
                if n_kv > topk:
                    orc.orc_block_scores(ptr(g_pooled), ptr(g_dead), ptr(q_idx), n_kv, IH, ID, blk, ptr(scores))
                nb = n_kv // blk + 1
                gsc = np.ascontiguousarray(g["scores"][qi, 0])
                if n_kv > topk:
                    # no requantisation between the fp16 keys and the scores (and the open block's +1e9
                    # forcing would dominate a row RMS): plain elementwise
                    self._cmp("block scores", gsc[:nb], scores[:nb], t, plain=True)
                gsel = np.ascontiguousarray(g["sel"][qi, 0])
                n = int(g["n_sel"][qi, 0])
                assert n == min(n_kv, topk), "%s: selection count %d" % (t, n)
                own = np.zeros(topk, np.int32)
                assert orc.orc_topk_select(ptr(gsc), n_kv, blk, topk, ptr(own)) == n
                assert np.array_equal(own[:n], gsel[:n]), "%s: top-k of the stage's own scores differs" % t
                osel = np.zeros(topk, np.int32)
                orc.orc_topk_select(ptr(scores), n_kv, blk, topk, ptr(osel))
                if not np.array_equal(osel[:n], gsel[:n]):
                    from layer_parity import threshold_gap
                    gap = threshold_gap(scores, n_kv, blk, topk)
                    err = float(np.abs(gsc[:nb].astype(np.float64) - scores[:nb]).max())
                    assert gap <= 2 * err, "%s: selected cells differ, gap %.3g > 2 x score error %.3g" % (t, gap, err)
                    self._excuse("select", t, gap, err)
                sel = np.ascontiguousarray(gsel[:n])
                S = self.state
                kvs = (S[(l, "kv_k")], S[(l, "kv_ks")], S[(l, "kv_v")], S[(l, "kv_vs")])
                f16 = attn_f16(cfg, pos, 1)
                # the attention itself on identical inputs (the GPU's q | gate rows after norm + RoPE,
                # its KV store and selection): close to the oracle of the window's branch, and closer to
                # it than to the other branch
                gq = np.ascontiguousarray(g["qg"][qi, 0])
                self._cmp("q rows (norm + RoPE)", gq, qg, t)
                a_br = attend(orc, f16, gq, *kvs, sel, cfg.qsa_qh, cfg.qsa_kvh, hd)
                a_ot = attend(orc, not f16, gq, *kvs, sel, cfg.qsa_qh, cfg.qsa_kvh, hd)
                ga = g["attn"][qi, 0].astype(np.float64)
                scale = max(float(np.abs(a_br).max()), 1e-30)
                e_br = float(np.abs(ga - a_br).max()) / scale
                e_ot = float(np.abs(ga - a_ot).max()) / scale
                gap_br = float(np.abs(a_br.astype(np.float64) - a_ot).max()) / scale
                self.attn.append((t, "fp16" if f16 else "fp32", e_br, gap_br))
                assert e_br <= ATT_RTOL, "%s: attention (%s branch) on identical inputs off by %.3g of its range" % (
                    t, "fp16" if f16 else "fp32", e_br)
                if gap_br > 4e-5:
                    assert e_br < e_ot, "%s: attention is closer to the %s branch (%.3g) than to the window's " \
                                        "(%.3g)" % (t, "fp32" if f16 else "fp16", e_ot, e_br)
                # the chain from the oracle's own q rows, through the branch's attention and o projection
                att = attend(orc, f16, qg, *kvs, sel, cfg.qsa_qh, cfg.qsa_kvh, hd)
                block = self._q8("wo", l, att, D)
            self._cmp("attention block", g["hidden"][l, 1, 0], block, t)
            # ---- FFN HC read on the GPU's attention-half outputs
            R_f, mixf, inj_f = self._hc_read(l, 1, g["R_a"][l, 0], None, g["hidden"][l, 1, 0], g["inj_a"][l, 0])
            self._cmp("FFN R", g["R_f"][l, 0], R_f, t)
            self._cmp("FFN HC read", g["hidden"][l, 2, 0], mixf, t)
            self._cmp("FFN inject", g["inj_f"][l, 0], inj_f, t)
            # ---- MoE on the GPU's mixed_f
            xf = np.ascontiguousarray(g["hidden"][l, 2, 0])
            comb, ids, wts, logits = self._moe(l, xf)
            gi = g["ids"][l, 0]
            if not np.array_equal(gi, ids):
                gl = g["router_logits"][l, 0].astype(np.float64)
                err = float(np.abs(gl - logits).max())
                s = np.sort(logits.astype(np.float64))[::-1]
                K = cfg.top_k
                if set(gi.tolist()) == set(ids.tolist()):
                    for a, b in zip(gi, ids):
                        assert a == b or abs(logits[a] - logits[b]) <= 2 * err, "%s: expert order" % t
                    self._cmp("MoE output", g["hidden"][l, 3, 0], comb, t)
                else:
                    assert s[K - 1] - s[K] <= 2 * err, "%s: experts %s vs %s, gap %.3g > 2 x logit error %.3g" % (
                        t, sorted(gi.tolist()), sorted(ids.tolist()), s[K - 1] - s[K], err)
                    self._excuse("router", t, s[K - 1] - s[K], err)
            else:
                self._cmp("router weights", g["wts"][l, 0], wts, t)
                self._cmp("MoE output", g["hidden"][l, 3, 0], comb, t)
            self.counts["layers"] += 1
        # ---- head
        L = cfg.n_layers
        R_h, mixh, _ = self._hc_read(-1, 0, g["R_f"][L - 1, 0], None, g["hidden"][L - 1, 3, 0], g["inj_f"][L - 1, 0],
                                     with_inj=False)
        # pre-head residual = R_f[L-1] with the last MoE write folded in (the head read's R_out)
        self._cmp("pre-head residual", g_pre.ravel(), R_h, tag)
        logits = self._q8("head", -1, mixh, cfg.n_vocab) if self.head_q8 else self._bf16(self.A[(-1, "head")], mixh,
                                                                                            cfg.n_vocab)
        self._cmp("logits", g_logits.ravel(), logits, tag)
        ref = int(np.argmax(logits))
        gid = int(g_greedy[0])
        if gid != ref:
            err = float(np.abs(g_logits.ravel().astype(np.float64) - logits).max())
            gap = float(logits[ref]) - float(logits[gid])
            assert gap <= 2 * err, "%s: greedy %d vs %d, gap %.3g > 2 x logit error %.3g" % (tag, gid, ref, gap, err)
            self._excuse("greedy", tag, gap, err)
        # teacher forcing: the next row starts from the stage's own post-row state
        self.state.update(new_state)

    def _moe(self, l, x):
        cfg, A = self.cfg, self.A
        D, F, E, K = cfg.n_embd, cfg.n_ff, cfg.n_exp, cfg.top_k
        ow = OrcMoeWeights()
        ow.n_embd, ow.n_ff, ow.n_exp, ow.top_k = D, F, E, K
        ow.router, ow.sgate = ptr(A[(l, "router")]), ptr(A[(l, "sgate")])
        ow.blobs = None
        for n in ("sh_gate", "sh_up", "sh_down"):
            setattr(ow, n + "_q", ptr(A[(l, n + ".q")]))
            setattr(ow, n + "_s", ptr(A[(l, n + ".s")]))
        comb = np.empty(D, np.float32)
        ids = np.empty(K, np.int32)
        wts = np.empty(K, np.float32)
        logits = np.empty(E, np.float32)
        fn = self.orc.orc_moe_block_fn
        fn.restype = C.c_int
        cb = self.om._blob_cb                      # the oracle model's expert-blob callback (kept alive there)
        fn.argtypes = [C.POINTER(OrcMoeWeights), C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                       C.c_void_p, type(cb), C.c_void_p, C.c_int]
        assert fn(C.byref(ow), ptr(x), 1, ptr(comb), ptr(ids), ptr(wts), ptr(logits), None, cb, None, l) == 0
        return comb, ids, wts, logits

    def summary(self):
        w = ", ".join("%s %.3g (plain %.3g)" % (k, self.worst[k], self.worst_plain[k]) for k in self.worst)
        fo = ", ".join("%s %d/%d" % (k, n, self.n_elems[k]) for k, n in self.floor_only.items() if n)
        ex = "; ".join("%s at %s: margin %.3g vs error %.3g" % e for e in self.excused)
        at = ""
        if self.attn:
            for br in ("fp32", "fp16"):
                r = [a for a in self.attn if a[1] == br]
                if r:
                    at += " %s-branch attention on identical inputs: %d rows, max error %.3g, branches %.3g-%.3g " \
                          "apart (relative to the row's largest output);" % (
                              br, len(r), max(a[2] for a in r), min(a[3] for a in r), max(a[3] for a in r))
        return ("teacher-forced: %d rows, %d layer-rows; KV bytes bit-exact on the GPU's rows %d, pooled-key fp16 "
                "midpoint flips %d;%s excused decisions %d (%s); elements within tolerance only through the row-RMS "
                "floor: %s; worst tolerance excess (<= 0 passes): %s" % (
                    self.counts["rows"], self.counts["layers"], self.counts["kv_bytes"],
                    self.counts["key_midpoint_flips"], at, len(self.excused), ex or "none", fo or "none", w))

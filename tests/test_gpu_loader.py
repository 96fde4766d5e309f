"""GPU tests of the real-weight loaders: a checkpoint in the reference's files (tests/gguf_file.py:
GGUF with Q8_0 / bf16 / f32 tensors under the reference's names, pack/experts.bin, an optional bf16
embedding file, the mtp/ directory) is loaded with wzy_stage_load_gguf / wzy_stage_mtp_load; every
stage tensor is compared with the conversion of the file's tensor, then the loaded model decodes and
drafts against the oracle (which reads the stage's tensors)."""
import ctypes as C
import os

import numpy as np
import pytest

import gguf_file as gf
import wzy_amd
from mtp_oracle import MtpTeacher, OracleMtp, gpu_acts
from stage_oracle import OracleModel, small_cfg
from test_gpu_stage import run_layer_parity

pytestmark = pytest.mark.gpu

# GGUF tensor (per layer: "blk.N." + suffix) -> (stage tensor, conversion)
LAYER_MAP = [("hc_attn_norm.weight", "hc_norm0", "f32"), ("hc_attn_down.weight", "hc_down0", "bf16q8"),
             ("hc_attn_up.weight", "hc_up0", "bf16q8"), ("hc_attn_inject.weight", "hc_inj0", "bf16"),
             ("hc_ffn_norm.weight", "hc_norm1", "f32"), ("hc_ffn_down.weight", "hc_down1", "bf16q8"),
             ("hc_ffn_up.weight", "hc_up1", "bf16q8"), ("hc_ffn_inject.weight", "hc_inj1", "bf16"),
             ("ffn_gate_inp.weight", "router", "bf16"), ("ffn_gate_inp_shexp.weight", "sgate", "bf16"),
             ("ffn_gate_shexp.weight", "sh_gate", "q8"), ("ffn_up_shexp.weight", "sh_up", "q8"),
             ("ffn_down_shexp.weight", "sh_down", "q8")]
GDN_MAP = [("attn_qkv.weight", "qkv", "q8"), ("attn_gate.weight", "wgate", "q8"), ("ssm_out.weight", "wout", "q8"),
           ("ssm_alpha.weight", "alpha", "bf16"), ("ssm_beta.weight", "beta", "bf16"), ("ssm_a", "ssm_a", "f32"),
           ("ssm_dt.bias", "dt_bias", "f32"), ("ssm_conv1d.weight", "conv1d", "f32"),
           ("ssm_norm.weight", "ssm_norm", "f32")]
QSA_MAP = [("attn_q.weight", "wq", "q8"), ("attn_k.weight", "wk", "q8"), ("attn_v.weight", "wv", "q8"),
           ("attn_output.weight", "wo", "q8"), ("attn_q_norm.weight", "q_norm", "f32"),
           ("attn_k_norm.weight", "k_norm", "f32"), ("indexer.q_proj.weight", "idx_q", "bf16"),
           ("indexer.k_proj.weight", "idx_k", "bf16"), ("indexer.q_norm.weight", "idx_qn", "f32"),
           ("indexer.k_norm.weight", "idx_kn", "f32")]
MODEL_MAP = [("output_hc_norm.weight", "head_norm", "f32"), ("output_hc_down.weight", "head_down", "bf16q8"),
             ("output_hc_up.weight", "head_up", "bf16q8")]


def as_f32(t, v):
    if t == gf.F32:
        return v
    if t == gf.F16:
        return v.astype(np.float32)
    if t == gf.BF16:
        return gf.bf16_to_f32(v)
    q, s = v
    return (s.view(np.float16).astype(np.float32).repeat(32) * q.astype(np.float32)).astype(np.float32)


def check_tensor(st, layer, name, conv, t, v):
    """The stage tensor equals the reference uploader's conversion of the file tensor, bit for bit."""
    if conv == "q8":
        q, s = v
        assert np.array_equal(st.read(layer, name + ".q", np.int8), q), (layer, name)
        assert np.array_equal(st.read(layer, name + ".s", np.uint16), s), (layer, name)
    elif conv == "bf16q8":                           # up_bf_as_q8
        b = v if t == gf.BF16 else gf.bf16_bits(v)
        q, s = gf.q8_0_quantise(gf.bf16_to_f32(b))
        assert np.array_equal(st.read(layer, name + ".q", np.int8), q), (layer, name)
        assert np.array_equal(st.read(layer, name + ".s", np.uint16), s), (layer, name)
    elif conv == "bf16":                             # up_bf: bf16 as it is, f32 rounded to nearest even
        b = v if t == gf.BF16 else gf.bf16_bits(v)
        assert np.array_equal(st.read(layer, name, np.uint16), b), (layer, name)
    else:                                            # up_f32
        assert np.array_equal(st.read(layer, name, np.float32), as_f32(t, v)), (layer, name)


def check_loaded(wz, st, ck, cfg):
    n = 0
    for l in range(cfg.n_layers):
        qsa = l % cfg.qsa_period == cfg.qsa_period - 1
        for suf, name, conv in LAYER_MAP + (QSA_MAP if qsa else GDN_MAP):
            t, v = ck.t["blk.%d.%s" % (l, suf)]
            check_tensor(st, l, name, conv, t, v)
            n += 1
    for src, name, conv in MODEL_MAP:
        t, v = ck.t[src]
        check_tensor(st, -1, name, conv, t, v)
        n += 1
    t, v = ck.t["output.weight"]
    check_tensor(st, -1, "head", "q8" if t == gf.Q8_0 else "bf16", t, v)
    if ck.emb_file:
        t, v = ck.t["side:token_embd.weight"]
    else:
        t, v = ck.t["token_embd.weight"]
    check_tensor(st, -1, "emb", "q8" if t == gf.Q8_0 else "bf16", t, v)
    # experts: the plane layout of each reference blob
    rec = wz.wzy_nvfp4_expert_bytes(cfg.n_embd, cfg.n_ff)
    got = st.read(-1, "experts", np.uint8)
    want = np.empty(rec, np.uint8)
    for l in range(cfg.n_layers):
        for e in range(cfg.n_exp):
            wz.wzy_synth_expert_planes(ck.seed, l, e, cfg.n_embd, cfg.n_ff, want.ctypes.data)
            i = l * cfg.n_exp + e
            assert np.array_equal(got[i * rec:(i + 1) * rec], want), (l, e)
    return n + 2


@pytest.mark.parametrize("emb_q8,head_q8,side_emb", [(True, True, False), (False, False, False),
                                                     (False, True, True)])
def test_load_gguf_and_decode(wz, gpu, tmp_path, emb_q8, head_q8, side_emb):
    """Q8_0 or bf16 token embedding and LM head (the reference checkpoint has Q8_0 both, plus the bf16
    embedding file), f16 / bf16 vector tensors where up_f32 allows them, f32 tensors where up_bf
    rounds them to bf16."""
    print("case load_gguf emb_q8=%d head_q8=%d side_emb=%d" % (emb_q8, head_q8, side_emb), flush=True)
    ref = small_cfg(wzy_amd, ctx_max=256, n_layers=4, topk=64)
    ref.gdn_hk, ref.gdn_hv = 2, 4
    ck = gf.Checkpoint(wz, ref, 11, str(tmp_path), emb_q8=emb_q8 and not side_emb, head_q8=head_q8,
                       f32_vectors_as=gf.F16 if head_q8 else gf.BF16,
                       bf16_from_f32=("blk.0.ffn_gate_inp.weight", "blk.1.hc_attn_inject.weight",
                                      "blk.1.indexer.k_proj.weight"),
                       with_emb_file=side_emb)
    cfg = wzy_amd.StageCfg()
    wz.wzy_stage_cfg_from_gguf(str(ck.gguf).encode(), 256, C.byref(cfg))
    assert (cfg.emb_q8, cfg.head_q8) == (int(emb_q8 and not side_emb), int(head_q8))
    st = wzy_amd.Stage(cfg)             # the shapes build a stage
    st.close()
    loaded = []

    def load(s):
        s.load_gguf(ck.gguf, ck.experts, ck.emb_file)
        loaded.append(check_loaded(wz, s, ck, cfg))

    # the loaded model decodes: the single-token steps component by component against the oracle fed
    # the GPU's own inputs (teacher-forced, the plain elementwise tolerance), every row's discrete
    # decisions layer by layer free-running, the T=4 window last
    par, tf = run_layer_parity(wz, cfg, 11, 0, [[5], [17], [999], [0], [3, 4, 5, 6]], teacher=True, load=load)
    print("loaded %d tensors; %s; %s" % (loaded[0], par.summary(), tf.summary()), flush=True)
    assert tf.counts["rows"] == 4 and tf.counts["layers"] == 4 * cfg.n_layers
    tf.assert_bounds()


def test_load_gguf_rejects_mismatches(wz, gpu, tmp_path):
    ref = small_cfg(wzy_amd, ctx_max=256, n_layers=2, topk=64)
    ck = gf.Checkpoint(wz, ref, 12, str(tmp_path), emb_q8=True, head_q8=True)
    other = small_cfg(wzy_amd, ctx_max=256, n_layers=2, topk=64)
    other.n_ff = 256                                  # the stage expects another shared-expert width
    other.emb_q8 = other.head_q8 = 1
    st = wzy_amd.Stage(other)
    try:
        with pytest.raises(wzy_amd.WzyError, match="ffn_gate_shexp"):
            st.load_gguf(ck.gguf, ck.experts)
        with pytest.raises(wzy_amd.WzyError):        # a stage that was not loaded does not run
            st.forward(0, [1])
    finally:
        st.close()
    cfg = wzy_amd.StageCfg()
    wz.wzy_stage_cfg_from_gguf(str(ck.gguf).encode(), 256, C.byref(cfg))
    st = wzy_amd.Stage(cfg)
    try:
        short = tmp_path / "short.bin"
        short.write_bytes(open(ck.experts, "rb").read()[:-1])
        with pytest.raises(wzy_amd.WzyError, match="fewer than"):
            st.load_gguf(ck.gguf, short)
        with pytest.raises(wzy_amd.WzyError, match="emb_q8"):
            st.load_gguf(ck.gguf, ck.experts, ck.gguf)   # a bf16 embedding file for a Q8_0 stage
    finally:
        st.close()


@pytest.mark.parametrize("q8", [False, True])
def test_load_ple_and_decode(wz, orc, gpu, tmp_path, q8):
    """A checkpoint with layer 1's per-layer embedding block and the table file ple-fp8.gguf (sparse:
    the rows the decode reads hold random codes, the rest zeros): the block's tensors and the table's
    rows equal the files', the scale comes from strata.ple.scale, and the loaded model decodes against
    the oracle (which reads the stage's table).  Tables of the wrong shape, truncated tables and stages
    without PLE are refused before anything is copied."""
    print("case load_ple q8=%d" % q8, flush=True)
    ref = small_cfg(wzy_amd, ctx_max=256, n_layers=4, topk=64)
    ref.gdn_hk, ref.gdn_hv = 2, 4
    ck = gf.Checkpoint(wz, ref, 14, str(tmp_path), emb_q8=q8, head_q8=q8, with_ple=True)
    cfg = wzy_amd.StageCfg()
    wz.wzy_stage_cfg_from_gguf(str(ck.gguf).encode(), 256, C.byref(cfg))
    assert cfg.ple == 1
    head, n_rows = cfg.n_embd // 16, int(wz.wzy_ple_table_rows())
    windows = [[5], [17], [999], [0], [3, 4, 5, 6]]   # the teacher follows single-token windows: T=4 last
    toks = [t for w in windows for t in w]
    rng = np.random.default_rng(14)

    def codes():                                     # e4m3 codes of magnitude 2^-3 .. 2^2.9 (exponent field 4..9)
        return (rng.integers(0, 2, head) << 7 | rng.integers(4, 10, head) << 3 | rng.integers(0, 8, head)).astype(
            np.uint8)

    rows, ids = {}, np.empty(16, np.uint32)
    for p, t in enumerate(toks):                     # every row the decode reads
        orc.orc_ple_row_ids(t, toks[p - 1] if p >= 1 else -1, toks[p - 2] if p >= 2 else -1, cfg.ple_eos,
                            ids.ctypes.data)
        for r in ids:
            rows[int(r)] = codes()
    for r in (0, n_rows - 1, 123456789):
        rows[r] = rng.integers(0, 256, head, dtype=np.uint8)   # every code, NaN codes included
    ple = gf.write_ple_table(tmp_path / "ple-fp8.gguf", head, n_rows, rows, scale=0.25)

    def load(st):
        st.load_gguf(ck.gguf, ck.experts)
        st.load_ple(ple)
        for suf, name, conv in (("ple_key.weight", "ple_key", "bf16"), ("ple_value.weight", "ple_value", "bf16"),
                                ("ple_norm_key.weight", "ple_norm_key", "f32"),
                                ("ple_norm_query.weight", "ple_norm_query", "f32"),
                                ("ple_norm_conv.weight", "ple_norm_conv", "f32"),
                                ("ple_conv1d.weight", "ple_conv1d", "f32")):
            t, v = ck.t["blk.1." + suf]
            check_tensor(st, 1, name, conv, t, v)
        for r, b in rows.items():
            assert np.array_equal(st.read_range(-1, "ple_table", np.uint8, r * head, head), b), "table row %d" % r
        for r in (1, 20000003, n_rows - 2):
            if r not in rows:
                assert not st.read_range(-1, "ple_table", np.uint8, r * head, head).any(), "hole row %d" % r
        assert st.read(-1, "ple_scale", np.float32)[0] == 0.25

    # the loaded model decodes: the single-token steps component by component (teacher-forced) and
    # every row's decisions layer by layer (free-running)
    par, tf = run_layer_parity(wz, cfg, 14, 0, windows, teacher=True, load=load)
    print("ple load: %d table rows written; %s; %s" % (len(rows), par.summary(), tf.summary()), flush=True)
    assert tf.counts["rows"] == 4 and "PLE conv history" in tf.worst
    tf.assert_bounds()
    st = wzy_amd.Stage(cfg)
    try:
        st.load_gguf(ck.gguf, ck.experts)
        with pytest.raises(wzy_amd.WzyError, match="table is not loaded"):
            st.forward(0, [1])
        # refused: a table of the wrong width, a truncated table (an I8 tag, and a tag this library does
        # not know, read as raw bytes as the reference does), and a stage without PLE
        bad = gf.write_ple_table(tmp_path / "wide.gguf", head, n_rows, {}, dims=[head + 1, n_rows])
        with pytest.raises(wzy_amd.WzyError, match="1-byte codes"):
            st.load_ple(bad)
        for tag in (24, 200):
            cut = gf.write_ple_table(tmp_path / ("cut%d.gguf" % tag), head, n_rows, {}, type_tag=tag)
            with open(cut, "r+b") as fh:
                fh.truncate(os.path.getsize(cut) - head)
            with pytest.raises(wzy_amd.WzyError, match="outside the file"):
                st.load_ple(cut)
    finally:
        st.close()
    cfg.ple = 0
    st = wzy_amd.Stage(cfg)
    try:
        with pytest.raises(wzy_amd.WzyError, match="cfg.ple = 0"):
            st.load_ple(ple)
    finally:
        st.close()


def test_mtp_load_and_draft(wz, gpu, tmp_path):
    """The drafter from mtp/dense.txt + dense.bin + experts.bin and a draft vocabulary over a loaded
    checkpoint with a Q8_0 LM head: every drafter tensor equals the file's conversion, the draft head
    holds the LM head's Q8_0 rows of the vocabulary ids, and fronts + a two-step chain match the oracle
    component by component."""
    print("case mtp_load", flush=True)
    ref = small_cfg(wzy_amd, ctx_max=256, n_layers=2, topk=64)
    n_dv = 300
    ck = gf.Checkpoint(wz, ref, 13, str(tmp_path), emb_q8=True, head_q8=True, with_mtp=True, n_dv=n_dv)
    cfg = wzy_amd.StageCfg()
    wz.wzy_stage_cfg_from_gguf(str(ck.gguf).encode(), 256, C.byref(cfg))
    st = wzy_amd.Stage(cfg)
    try:
        st.load_gguf(ck.gguf, ck.experts)
        st.mtp_load(ck.mtp_dir, ck.dvocab)
        conv = {"q8": "q8", "bf16": "bf16", "f32": "f32"}
        names = {"fc_embedding.weight": "fc_emb", "fc_hidden.weight": "fc_hid",
                 "pre_fc_norm_embedding.weight": "pre_norm_emb", "pre_fc_norm_hidden.weight": "pre_norm_hid",
                 "self_attn.q_proj.weight": "wq", "self_attn.k_proj.weight": "wk", "self_attn.v_proj.weight": "wv",
                 "self_attn.o_proj.weight": "wo", "self_attn.q_norm.weight": "q_norm",
                 "self_attn.k_norm.weight": "k_norm", "mlp.gate.weight": "router",
                 "mlp.shared_expert.gate_proj.weight": "sh_gate", "mlp.shared_expert.up_proj.weight": "sh_up",
                 "mlp.shared_expert.down_proj.weight": "sh_down", "mlp.shared_expert_gate.weight": "sgate"}
        for i, p in enumerate(("attn_hyper_connection.", "mlp_hyper_connection.", "hyper_connection_mixer.")):
            names[p + "hc_norm.weight"] = "hc_norm%d" % i
            names[p + "input_mix_weight_down.weight"] = "hc_down%d" % i
            names[p + "input_mix_weight_up.weight"] = "hc_up%d" % i
            if i < 2:
                names[p + "block_inject_weight.weight"] = "hc_inj%d" % i
        assert set(names) == set(ck.mt)
        for src, (kind, v) in ck.mt.items():
            c = "bf16q8" if "input_mix_weight" in src else conv[kind]
            t = {"q8": gf.Q8_0, "bf16": gf.BF16, "f32": gf.F32}[kind]
            check_tensor(st, -1, "mtp." + names[src], c, t, v)
        assert np.array_equal(st.read(-1, "mtp.experts", np.uint8), ck.q2)
        assert np.array_equal(st.read(-1, "mtp.dvocab", np.int32), ck.dv_ids)
        hq, hs = ck.t["output.weight"][1]
        D = cfg.n_embd
        assert np.array_equal(st.read(-1, "mtp.head.q", np.int8).reshape(n_dv, D), hq.reshape(-1, D)[ck.dv_ids])
        assert np.array_equal(st.read(-1, "mtp.head.s", np.uint16).reshape(n_dv, D // 32),
                              hs.reshape(-1, D // 32)[ck.dv_ids])
        # fronts over cells 0..7, then a two-step chain at cell 8, each step teacher-forced
        om = OracleMtp.from_stage(st, cfg, n_dv)
        tch = MtpTeacher(om)
        toks = np.random.default_rng(5).integers(0, cfg.n_vocab, 12).astype(np.int32)
        st.forward(0, toks[:8], run_head=2)
        st.mtp_front(0, toks[1:9], 0)
        st.sync()
        g = gpu_acts(st, cfg, n_dv, rows=8)
        tch.check_front("front", g, 0, toks[1:9], st.pre_head(8))
        st.forward(8, [int(toks[8])], run_head=1)
        st.sync()
        rin, t = st.pre_head(1)[0], int(toks[8])
        for j in range(2):
            d_t, d_p = st.mtp_draft(8 + j, t, 0 if j == 0 else -1, 1)
            g = gpu_acts(st, cfg, n_dv)
            tch.check_step("step %d" % j, g, 8 + j, t, rin, int(d_t[0]), float(d_p[0]), 0)
            rin, t = g["R_out"], int(d_t[0])
        print("mtp load: " + tch.summary(), flush=True)
        assert tch.counts["steps"] == 2 and tch.counts["fronts"] >= 1
        # a vocabulary id outside the main vocabulary is refused, and the failed load leaves no drafter
        st2 = wzy_amd.Stage(cfg)
        try:
            st2.load_gguf(ck.gguf, ck.experts)
            bad = tmp_path / "bad_vocab.bin"
            np.array([1, cfg.n_vocab], np.int32).tofile(bad)
            with pytest.raises(wzy_amd.WzyError, match="out of range"):
                st2.mtp_load(ck.mtp_dir, bad)
            with pytest.raises(wzy_amd.WzyError):
                st2.mtp_draft(0, 1, 0, 1)
        finally:
            st2.close()
    finally:
        st.close()

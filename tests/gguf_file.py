"""A GGUF (version 3) writer and checkpoint builders for the loader tests.

The layout follows the published GGUF format: magic, version, tensor and metadata counts,
metadata key/value pairs, tensor infos (name, dims with the contiguous one first, GGML type, data
offset), then the tensor data at the file's alignment.  Tensors are written in the element formats
the reference loaders read (src/wzy_stage_v2.cuh:30-179): f32 (0), f16 (1), Q8_0 (8: fp16 scale + 32
int8 codes per block) and bf16 (30); the tensor names are those of init_stage_weights_and_state
(src/wzy_engine_v2.cu:334-378,542-556) and MtpEngine::init (src/wzy_mtp.cuh:494-536).
"""
import os
import struct

import numpy as np

F32, F16, Q8_0, BF16 = 0, 1, 8, 30
KV_U8, KV_I8, KV_U16, KV_I16, KV_U32, KV_I32, KV_F32, KV_BOOL, KV_STR, KV_ARR, KV_U64, KV_I64, KV_F64 = range(13)
_SCALAR = {KV_U8: "<B", KV_I8: "<b", KV_U16: "<H", KV_I16: "<h", KV_U32: "<I", KV_I32: "<i", KV_F32: "<f",
           KV_BOOL: "<?", KV_U64: "<Q", KV_I64: "<q", KV_F64: "<d"}


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == KV_STR:
        return _str(v)
    if t == KV_ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_value(et, x) for x in items)
    return struct.pack(_SCALAR[t], v)


def write_gguf(path, tensors, kvs=(), alignment=32, version=3):
    """tensors: list of (name, dims (contiguous first), ggml type, raw bytes); kvs: (key, type, value)."""
    kvs = list(kvs)
    if alignment != 32:
        kvs.append(("general.alignment", KV_U32, alignment))
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs))
    for k, t, v in kvs:
        head += _str(k) + struct.pack("<I", t) + _value(t, v)
    offs, off = [], 0
    for name, dims, t, raw in tensors:
        offs.append(off)
        off += (len(raw) + alignment - 1) // alignment * alignment
    for (name, dims, t, raw), o in zip(tensors, offs):
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", t, o)
    data_at = (len(head) + alignment - 1) // alignment * alignment
    with open(path, "wb") as fh:
        fh.write(head + b"\0" * (data_at - len(head)))
        for (name, dims, t, raw), o in zip(tensors, offs):
            pad = (len(raw) + alignment - 1) // alignment * alignment - len(raw)
            fh.write(raw + b"\0" * pad)
    return path


# ---- element formats ----------------------------------------------------------------------------
def bf16_bits(x):
    """fp32 -> bf16 bits, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def q8_0_quantise(x):
    """fp32 rows (a multiple of 32 values) -> (codes int8, fp16 scales as uint16) with the reference's
    per-32 rule d = half(amax/127), q = rint(x/d)."""
    v = np.ascontiguousarray(x, np.float32).reshape(-1, 32)
    amax = np.abs(v).max(axis=1)
    sh = (amax / np.float32(127.0)).astype(np.float16)
    d = sh.astype(np.float32)[:, None]
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(d > 0, np.clip(np.rint(v / np.where(d > 0, d, 1)), -127, 127), 0).astype(np.int8)
    return q.reshape(-1), sh.view(np.uint16)


def q8_0_blocks(codes, scales):
    """code / scale planes -> Q8_0 block bytes (fp16 scale then 32 codes)."""
    n = scales.size
    out = np.empty((n, 34), np.uint8)
    out[:, :2] = np.ascontiguousarray(scales, np.uint16).view(np.uint8).reshape(n, 2)
    out[:, 2:] = np.ascontiguousarray(codes, np.int8).view(np.uint8).reshape(n, 32)
    return out.tobytes()


# ---- a small checkpoint in the reference's files ------------------------------------------------
class Checkpoint:
    """Random weights of a stage configuration written as the reference's files: the GGUF (Q8_0
    projections, bf16 hyper-connection mixes / router / inject / indexer, f32 vectors; Q8_0 or bf16
    token embedding and LM head), pack/experts.bin (the generator's reference-layout NVFP4 blobs of
    `seed`), token-embd-bf16.gguf (optional) and the mtp/ directory with a draft vocabulary.
    `t` keeps every tensor as written (name -> (ggml type, array))."""

    def __init__(self, wz, cfg, seed, out_dir, emb_q8=True, head_q8=True, f32_vectors_as=F32, bf16_from_f32=(),
                 with_emb_file=False, with_mtp=False, n_dv=0, metadata=True, with_ple=False):
        self.cfg, self.seed, self.dir = cfg, seed, out_dir
        rng = np.random.default_rng(seed)
        D, HC, L = cfg.n_embd, cfg.hc, cfg.hc_lr
        HCD = HC * D
        GV = cfg.gdn_hv * 128
        QKV = cfg.gdn_hk * 256 + GV
        QD, KVD = cfg.qsa_qh * cfg.qsa_hd, cfg.qsa_kvh * cfg.qsa_hd
        self.t = {}
        tensors = []

        def add(name, rows, cols, kind, sd=None, mean=0.0, lo=None, hi=None):
            n = rows * cols
            if lo is not None:
                x = rng.uniform(lo, hi, n).astype(np.float32)
            else:
                x = (mean + (sd if sd is not None else 1.0 / np.sqrt(cols)) * rng.standard_normal(n)).astype(np.float32)
            dims = [cols] if rows == 1 else [cols, rows]
            if kind == "q8":
                q, s = q8_0_quantise(x)
                self.t[name] = (Q8_0, (q, s))
                tensors.append((name, dims, Q8_0, q8_0_blocks(q, s)))
            elif kind == "bf16":
                if name in bf16_from_f32:          # stored as f32; the loader rounds it to bf16
                    self.t[name] = (F32, x)
                    tensors.append((name, dims, F32, x.tobytes()))
                else:
                    b = bf16_bits(x)
                    self.t[name] = (BF16, b)
                    tensors.append((name, dims, BF16, b.tobytes()))
            else:                                  # an f32 vector, stored as f32_vectors_as
                t = f32_vectors_as
                if t == F32:
                    raw, val = x.tobytes(), x
                elif t == F16:
                    h = x.astype(np.float16)
                    raw, val = h.tobytes(), h
                elif t == BF16:
                    b = bf16_bits(x)
                    raw, val = b.tobytes(), b
                else:
                    q, s = q8_0_quantise(x)
                    raw, val = q8_0_blocks(q, s), (q, s)
                self.t[name] = (t, val)
                tensors.append((name, dims, t, raw))

        for l in range(cfg.n_layers):
            b = "blk.%d." % l
            qsa = l % cfg.qsa_period == cfg.qsa_period - 1
            for pre in ("hc_attn_", "hc_ffn_"):
                add(b + pre + "norm.weight", 1, HCD, "f32", sd=0.02, mean=1.0)
                add(b + pre + "down.weight", L, HCD, "bf16")
                add(b + pre + "up.weight", HCD, L, "bf16")
                add(b + pre + "inject.weight", HC, HCD, "bf16", sd=1.0 / np.sqrt(HCD))
            if not qsa:
                add(b + "attn_qkv.weight", QKV, D, "q8")
                add(b + "attn_gate.weight", GV, D, "q8")
                add(b + "ssm_out.weight", D, GV, "q8")
                add(b + "ssm_alpha.weight", cfg.gdn_hv, D, "bf16")
                add(b + "ssm_beta.weight", cfg.gdn_hv, D, "bf16")
                add(b + "ssm_a", 1, cfg.gdn_hv, "f32", lo=-2.0, hi=-1.0)
                add(b + "ssm_dt.bias", 1, cfg.gdn_hv, "f32", sd=0.5, mean=-3.0)
                add(b + "ssm_conv1d.weight", QKV, 4, "f32", sd=0.5)
                add(b + "ssm_norm.weight", 1, 128, "f32", sd=0.02, mean=1.0)
            else:
                add(b + "attn_q.weight", 2 * QD, D, "q8")
                add(b + "attn_k.weight", KVD, D, "q8")
                add(b + "attn_v.weight", KVD, D, "q8")
                add(b + "attn_output.weight", D, QD, "q8")
                add(b + "attn_q_norm.weight", 1, cfg.qsa_hd, "f32", sd=0.02, mean=1.0)
                add(b + "attn_k_norm.weight", 1, cfg.qsa_hd, "f32", sd=0.02, mean=1.0)
                add(b + "indexer.q_proj.weight", cfg.idx_heads * cfg.idx_dim, D, "bf16")
                add(b + "indexer.k_proj.weight", cfg.idx_dim, D, "bf16")
                add(b + "indexer.q_norm.weight", 1, cfg.idx_dim, "f32", sd=0.02, mean=1.0)
                add(b + "indexer.k_norm.weight", 1, cfg.idx_dim, "f32", sd=0.02, mean=1.0)
            if with_ple and l == 1:               # layer 1's per-layer embedding block (wzy_engine_v2.cu:493-499)
                add(b + "ple_key.weight", HCD, D, "bf16")
                add(b + "ple_value.weight", D, D, "bf16")
                add(b + "ple_norm_key.weight", 1, HCD, "f32", sd=0.02, mean=1.0)
                add(b + "ple_norm_query.weight", 1, HCD, "f32", sd=0.02, mean=1.0)
                add(b + "ple_norm_conv.weight", 1, HCD, "f32", sd=0.02, mean=1.0)
                add(b + "ple_conv1d.weight", HCD, 4, "f32", sd=0.5)
            add(b + "ffn_gate_inp.weight", cfg.n_exp, D, "bf16", sd=0.02)
            add(b + "ffn_gate_inp_shexp.weight", 1, D, "bf16", sd=0.02)
            add(b + "ffn_gate_shexp.weight", cfg.n_ff, D, "q8")
            add(b + "ffn_up_shexp.weight", cfg.n_ff, D, "q8")
            add(b + "ffn_down_shexp.weight", D, cfg.n_ff, "q8")
        add("output_hc_norm.weight", 1, HCD, "f32", sd=0.02, mean=1.0)
        add("output_hc_down.weight", L, HCD, "bf16")
        add("output_hc_up.weight", HCD, L, "bf16")
        add("output.weight", cfg.n_vocab, D, "q8" if head_q8 else "bf16")
        add("token_embd.weight", cfg.n_vocab, D, "q8" if emb_q8 else "bf16", sd=1.0)
        kvs = []
        if metadata:
            kvs = [("general.architecture", KV_STR, "wzynext"), ("wzynext.expert_used_count", KV_U32, cfg.top_k),
                   ("wzynext.rope.dimension_count", KV_U32, cfg.n_rot),
                   ("wzynext.rope.freq_base", KV_F32, cfg.rope_theta),
                   ("wzynext.attention.layer_norm_rms_epsilon", KV_F32, cfg.eps),
                   ("tokenizer.ggml.tokens", KV_ARR, (KV_STR, ["<a>", "<b>", "c"]))]
        os.makedirs(os.path.join(out_dir, "pack"), exist_ok=True)
        # the reference's file names under its model directory (src/wzy_engine_v2.cu:661,694,808)
        self.gguf = write_gguf(os.path.join(out_dir, "qwen-nvfp4-gptq-dense.gguf"), tensors, kvs)
        # experts.bin: blob (l, e) at (l * n_exp + e) * blob bytes
        blob = wz.wzy_nvfp4_blob_bytes(D, cfg.n_ff)
        self.experts = os.path.join(out_dir, "pack", "experts.bin")
        with open(self.experts, "wb") as fh:
            b = np.empty(blob, np.uint8)
            for l in range(cfg.n_layers):
                for e in range(cfg.n_exp):
                    wz.wzy_synth_expert_blob(seed, l, e, D, cfg.n_ff, b.ctypes.data)
                    fh.write(b.tobytes())
        self.emb_file = None
        if with_emb_file:
            x = rng.standard_normal(cfg.n_vocab * D).astype(np.float32)
            eb = bf16_bits(x)
            self.t["side:token_embd.weight"] = (BF16, eb)
            self.emb_file = write_gguf(os.path.join(out_dir, "token-embd-bf16.gguf"),
                                       [("token_embd.weight", [D, cfg.n_vocab], BF16, eb.tobytes())])
        self.mtp_dir = self.dvocab = None
        if with_mtp:
            self._write_mtp(wz, rng, n_dv)

    def _write_mtp(self, wz, rng, n_dv):
        cfg = self.cfg
        D, HC, L = cfg.n_embd, cfg.hc, cfg.hc_lr
        HCD = HC * D
        QD, KVD = cfg.qsa_qh * cfg.qsa_hd, cfg.qsa_kvh * cfg.qsa_hd
        self.mtp_dir = os.path.join(self.dir, "mtp")
        os.makedirs(self.mtp_dir, exist_ok=True)
        self.mt = {}
        lines, blob, off = [], [], 0

        def add(name, rows, cols, kind, sd=None, mean=0.0):
            nonlocal off
            n = rows * cols
            x = (mean + (sd if sd is not None else 1.0 / np.sqrt(cols)) * rng.standard_normal(n)).astype(np.float32)
            if kind == "q8":
                q, s = q8_0_quantise(x)
                raw, val = q8_0_blocks(q, s), (q, s)
            elif kind == "bf16":
                b = bf16_bits(x)
                raw, val = b.tobytes(), b
            else:
                raw, val = x.tobytes(), x
            self.mt[name] = (kind, val)
            lines.append("%s %s %d %d %d %d" % (name, kind, rows, cols, off, len(raw)))
            blob.append(raw)
            off += len(raw)

        add("fc_embedding.weight", D, D, "q8")
        add("fc_hidden.weight", D, D, "q8")
        add("pre_fc_norm_embedding.weight", 1, D, "f32", sd=0.02, mean=1.0)
        add("pre_fc_norm_hidden.weight", 1, HCD, "f32", sd=0.02, mean=1.0)
        for p, inj in (("attn_hyper_connection.", True), ("mlp_hyper_connection.", True),
                       ("hyper_connection_mixer.", False)):
            add(p + "hc_norm.weight", 1, HCD, "f32", sd=0.02, mean=1.0)
            add(p + "input_mix_weight_down.weight", L, HCD, "bf16")
            add(p + "input_mix_weight_up.weight", HCD, L, "bf16")
            if inj:
                add(p + "block_inject_weight.weight", HC, HCD, "bf16", sd=1.0 / np.sqrt(HCD))
        add("self_attn.q_proj.weight", 2 * QD, D, "q8")
        add("self_attn.k_proj.weight", KVD, D, "q8")
        add("self_attn.v_proj.weight", KVD, D, "q8")
        add("self_attn.o_proj.weight", D, QD, "q8")
        add("self_attn.q_norm.weight", 1, cfg.qsa_hd, "f32", sd=0.02, mean=1.0)
        add("self_attn.k_norm.weight", 1, cfg.qsa_hd, "f32", sd=0.02, mean=1.0)
        add("mlp.gate.weight", cfg.n_exp, D, "bf16", sd=0.02)
        add("mlp.shared_expert.gate_proj.weight", cfg.n_ff, D, "q8")
        add("mlp.shared_expert.up_proj.weight", cfg.n_ff, D, "q8")
        add("mlp.shared_expert.down_proj.weight", D, cfg.n_ff, "q8")
        add("mlp.shared_expert_gate.weight", 1, D, "bf16", sd=0.02)
        rng.shuffle(lines)                          # the index is looked up by name, not by order
        with open(os.path.join(self.mtp_dir, "dense.txt"), "w") as fh:
            fh.write("\n".join(lines) + "\n")
        with open(os.path.join(self.mtp_dir, "dense.bin"), "wb") as fh:
            fh.write(b"".join(blob))
        rec = wz.wzy_q2_expert_bytes(D, cfg.n_ff)
        self.q2 = np.empty(cfg.n_exp * rec, np.uint8)
        for e in range(cfg.n_exp):
            wz.wzy_synth_q2_expert(self.seed + 7, e, D, cfg.n_ff, self.q2[e * rec:].ctypes.data)
        self.q2.tofile(os.path.join(self.mtp_dir, "experts.bin"))
        self.dv_ids = np.sort(rng.choice(cfg.n_vocab, n_dv, replace=False)).astype(np.int32)
        self.dvocab = os.path.join(self.mtp_dir, "draft_vocab.bin")
        self.dv_ids.tofile(self.dvocab)


def write_ple_table(path, head, n_rows, rows, scale=None, type_tag=24, dims=None):
    """The reference's ple-fp8.gguf: one tensor per_layer_token_embd.weight of 1-byte fp8 codes
    [n_rows][head] (dims [head, n_rows]) and the strata.ple.scale metadata (f32; absent when scale is
    None).  Only the rows given (row -> head bytes) are written; the rest of the table is a hole of
    the sparse file (codes 0), so the multi-gigabyte table costs no disk space."""
    kvs = [] if scale is None else [("strata.ple.scale", KV_F32, float(scale))]
    dims = [head, n_rows] if dims is None else dims
    head_b = b"GGUF" + struct.pack("<IQQ", 3, 1, len(kvs))
    for k, t, v in kvs:
        head_b += _str(k) + struct.pack("<I", t) + _value(t, v)
    head_b += _str("per_layer_token_embd.weight") + struct.pack("<I", len(dims))
    head_b += b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", type_tag, 0)
    data_at = (len(head_b) + 31) // 32 * 32
    with open(path, "wb") as fh:
        fh.write(head_b + b"\0" * (data_at - len(head_b)))
        for r in sorted(rows):
            fh.seek(data_at + r * head)
            fh.write(bytes(rows[r]))
        fh.truncate(data_at + int(np.prod(dims, dtype=np.uint64)))
    return path

"""The real-weight loaders on the CPU (no GPU): the GGUF reader (include/wzy_loader.h) against files
written by tests/gguf_file.py, its rejection of damaged files, the element conversions of the
reference's uploaders (src/wzy_stage_v2.cuh:30-179), and the stage configuration derived from a
checkpoint's tensor shapes."""
import ctypes as C
import os
import struct

import numpy as np
import pytest

import gguf_file as gf
import wzy_amd
from stage_oracle import small_cfg


def open_gguf(wz, path):
    h = C.c_void_p()
    wz.wzy_gguf_open(str(path).encode(), C.byref(h))
    return h


def info(wz, h, i):
    name = C.c_char_p()
    nd = C.c_int()
    dims = (C.c_int64 * 4)()
    t = C.c_int()
    nb = C.c_size_t()
    wz.wzy_gguf_tensor_info(h, i, C.byref(name), C.byref(nd), dims, C.byref(t), C.byref(nb))
    return name.value.decode(), list(dims)[:nd.value], t.value, nb.value


def data(wz, h, i, nbytes):
    p = wz.wzy_gguf_tensor_data(h, i)
    return np.frombuffer((C.c_uint8 * nbytes).from_address(p), np.uint8).copy()


def test_gguf_reader_round_trip(wz, tmp_path):
    rng = np.random.default_rng(0)
    f32 = rng.standard_normal(6 * 5).astype(np.float32)
    f16 = rng.standard_normal(64).astype(np.float16)
    b16 = gf.bf16_bits(rng.standard_normal(3 * 32))
    q, s = gf.q8_0_quantise(rng.standard_normal(4 * 64).astype(np.float32))
    tensors = [("a.f32", [5, 6], gf.F32, f32.tobytes()), ("b.f16", [64], gf.F16, f16.tobytes()),
               ("c.bf16", [32, 3], gf.BF16, b16.tobytes()), ("d.q8", [64, 4], gf.Q8_0, gf.q8_0_blocks(q, s)),
               ("e.other", [7], 2, b"\x01" * 40)]
    kvs = [("general.architecture", gf.KV_STR, "wzynext"), ("n.u32", gf.KV_U32, 7), ("n.i8", gf.KV_I8, -3),
           ("n.bool", gf.KV_BOOL, True), ("n.u64", gf.KV_U64, 1 << 40), ("x.f32", gf.KV_F32, 0.5),
           ("x.f64", gf.KV_F64, -2.25), ("arr.str", gf.KV_ARR, (gf.KV_STR, ["a", "bb", ""])),
           ("arr.nested", gf.KV_ARR, (gf.KV_ARR, [(gf.KV_U16, [1, 2]), (gf.KV_U16, [])]))]
    for align in (32, 64):
        p = gf.write_gguf(tmp_path / ("t%d.gguf" % align), tensors, kvs, alignment=align)
        h = open_gguf(wz, p)
        try:
            assert wz.wzy_gguf_n_tensors(h) == 5
            assert wz.wzy_gguf_find(h, b"d.q8") == 3 and wz.wzy_gguf_find(h, b"nope") == -1
            assert info(wz, h, 0) == ("a.f32", [5, 6], gf.F32, 120)
            assert info(wz, h, 1) == ("b.f16", [64], gf.F16, 128)
            assert info(wz, h, 2) == ("c.bf16", [32, 3], gf.BF16, 192)
            assert info(wz, h, 3) == ("d.q8", [64, 4], gf.Q8_0, 8 * 34)
            assert info(wz, h, 4)[3] == 0                        # a type the loaders do not read
            assert data(wz, h, 0, 120).tobytes() == f32.tobytes()
            assert data(wz, h, 3, 8 * 34).tobytes() == gf.q8_0_blocks(q, s)
            v = C.c_int64()
            wz.wzy_gguf_get_int(h, b"n.u32", C.byref(v)); assert v.value == 7
            wz.wzy_gguf_get_int(h, b"n.i8", C.byref(v)); assert v.value == -3
            wz.wzy_gguf_get_int(h, b"n.bool", C.byref(v)); assert v.value == 1
            wz.wzy_gguf_get_int(h, b"n.u64", C.byref(v)); assert v.value == 1 << 40
            d = C.c_double()
            wz.wzy_gguf_get_float(h, b"x.f32", C.byref(d)); assert d.value == 0.5
            wz.wzy_gguf_get_float(h, b"x.f64", C.byref(d)); assert d.value == -2.25
            wz.wzy_gguf_get_float(h, b"n.u32", C.byref(d)); assert d.value == 7.0
            assert wz.wzy_gguf_get_int(h, b"x.f32", C.byref(v)) != 0
            assert wz.wzy_gguf_get_int(h, b"absent", C.byref(v)) != 0
            sp, sl = C.c_char_p(), C.c_size_t()
            wz.wzy_gguf_get_str(h, b"general.architecture", C.byref(sp), C.byref(sl))
            assert C.string_at(sp, sl.value) == b"wzynext"
        finally:
            wz.wzy_gguf_close(h)


def test_gguf_reader_rejects_damaged_files(wz, tmp_path):
    x = np.arange(64, dtype=np.float32)
    good = gf.write_gguf(tmp_path / "good.gguf", [("w", [64], gf.F32, x.tobytes())],
                         [("k", gf.KV_STR, "v")])
    raw = open(good, "rb").read()
    h = C.c_void_p()
    cases = {
        "magic": b"GGUX" + raw[4:],
        "version": raw[:4] + struct.pack("<I", 1) + raw[8:],
        "truncated header": raw[:40],
        "truncated data": raw[:-8],
        "huge count": raw[:8] + struct.pack("<Q", 1 << 40) + raw[16:],
    }
    for name, blob in cases.items():
        p = tmp_path / ("bad_%s.gguf" % name.replace(" ", "_"))
        p.write_bytes(blob)
        assert wz.dll.wzy_gguf_open(str(p).encode(), C.byref(h)) < 0, name
        assert wz.wzy_last_error().decode(), name
    assert wz.dll.wzy_gguf_open(str(tmp_path / "missing.gguf").encode(), C.byref(h)) < 0
    # a tensor offset past the end of the file
    bad = gf.write_gguf(tmp_path / "off.gguf", [("w", [64], gf.F32, x.tobytes())])
    b = bytearray(open(bad, "rb").read())
    i = b.find(b"w") + 1 + 4 + 8 + 4                 # name, n_dims, dim, type -> offset field
    b[i:i + 8] = struct.pack("<Q", 1 << 20)
    (tmp_path / "off.gguf").write_bytes(bytes(b))
    assert wz.dll.wzy_gguf_open(str(tmp_path / "off.gguf").encode(), C.byref(h)) < 0
    assert "outside" in wz.wzy_last_error().decode()
    # dimensions whose product wraps 64 bits (2^40 * 2^40 * 2^40 * 2^24 = 2^144 elements): an unchecked
    # product would wrap to 0 bytes and pass the "inside the file" check
    wrap = gf.write_gguf(tmp_path / "wrap.gguf", [("w", [1 << 40, 1 << 40, 1 << 40, 1 << 24], gf.F32, x.tobytes())])
    assert wz.dll.wzy_gguf_open(str(wrap).encode(), C.byref(h)) < 0
    assert "malformed" in wz.wzy_last_error().decode()
    # 2^50 elements of four dims: no wrap, but far past the element bound
    big = gf.write_gguf(tmp_path / "big.gguf", [("w", [1 << 10, 1 << 20, 1 << 20, 1], gf.F32, x.tobytes())])
    assert wz.dll.wzy_gguf_open(str(big).encode(), C.byref(h)) < 0


def test_q8_0_split_and_to_f32(wz):
    rng = np.random.default_rng(1)
    q, s = gf.q8_0_quantise(rng.standard_normal(10 * 32).astype(np.float32))
    blocks = np.frombuffer(gf.q8_0_blocks(q, s), np.uint8)
    cq = np.empty(320, np.int8); cs = np.empty(10, np.uint16)
    wz.wzy_q8_0_split(blocks.ctypes.data, 10, cq.ctypes.data, cs.ctypes.data)
    assert (cq == q).all() and (cs == s).all()
    out = np.empty(320, np.float32)
    wz.wzy_to_f32(gf.Q8_0, blocks.ctypes.data, 320, out.ctypes.data)
    # d * q in fp32 (up_f32): exact products of an fp16 scale and a small integer
    ref = (s.view(np.float16).astype(np.float64).repeat(32) * q.astype(np.float64)).astype(np.float32)
    assert np.array_equal(out, ref)
    h = rng.standard_normal(50).astype(np.float16)
    wz.wzy_to_f32(gf.F16, h.ctypes.data, 50, out.ctypes.data)
    assert np.array_equal(out[:50], h.astype(np.float32))
    b = gf.bf16_bits(rng.standard_normal(50))
    wz.wzy_to_f32(gf.BF16, b.ctypes.data, 50, out.ctypes.data)
    assert np.array_equal(out[:50], gf.bf16_to_f32(b))
    with pytest.raises(wzy_amd.WzyError):
        wz.wzy_to_f32(2, h.ctypes.data, 32, out.ctypes.data)


def test_bf16_from_f32_rounds_to_nearest_even(wz):
    # ties go to the even bf16; a carry out of the mantissa bumps the exponent
    vals = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -9, -(1.0 + 2 ** -8), 3.0e38, 2 ** -130,
                     1.9921875 + 2 ** -8, 0.0, -0.0], np.float32)
    want = np.array([0x3F80, 0x3F80, 0x3F82, 0x3F80, 0xBF80, 0x7F62, 0x0008, 0x4000, 0x0000, 0x8000], np.uint16)
    out = np.empty(vals.size, np.uint16)
    wz.wzy_bf16_from_f32(vals.ctypes.data, vals.size, out.ctypes.data)
    assert [hex(v) for v in out] == [hex(v) for v in want]
    # against exact rational rounding on random values
    x = np.random.default_rng(2).standard_normal(4096).astype(np.float32)
    got = np.empty(x.size, np.uint16)
    wz.wzy_bf16_from_f32(x.ctypes.data, x.size, got.ctypes.data)
    lo = (x.view(np.uint32) >> 16).astype(np.uint16)
    a, b = gf.bf16_to_f32(lo).astype(np.float64), gf.bf16_to_f32(lo + 1).astype(np.float64)
    xd = x.astype(np.float64)
    nearer_hi = np.abs(b - xd) < np.abs(xd - a)
    tie = np.abs(b - xd) == np.abs(xd - a)
    want = np.where(nearer_hi | (tie & (lo & 1 == 1)), lo + 1, lo)
    assert np.array_equal(got, want)


def test_bf16_to_q8_0_quantisation(wz):
    """quant_bf16_to_q8_kernel (src/wzy_kernels_v2.cuh:392-407): scale = half(amax/127), q = rint(v/scale)."""
    # known answers: a block whose amax is 127 has scale 1 and codes equal to the rounded values
    v = np.zeros(64, np.float32)
    v[:32] = np.arange(-15.5, 16.5, 1.0)
    v[0] = 127.0                                   # amax 127 -> scale exactly 1.0
    v[32:] = 0.0                                   # an all-zero block: scale 0, codes 0
    b = gf.bf16_bits(v)
    q = np.empty(64, np.int8); s = np.empty(2, np.uint16)
    wz.wzy_bf16_to_q8_0(b.ctypes.data, 2, q.ctypes.data, s.ctypes.data)
    assert s[0] == 0x3C00 and s[1] == 0
    exp = np.rint(gf.bf16_to_f32(b[:32]))           # half-way values round to even
    assert np.array_equal(q[:32], exp.astype(np.int8)) and (q[32:] == 0).all()
    assert list(q[1:5]) == [-14, -14, -12, -12]      # -14.5, -13.5, -12.5, -11.5: ties to even
    # random blocks: every code within half a scale step, the largest magnitude at +-126/127, and the
    # scale the fp16 rounding of amax/127
    x = np.random.default_rng(3).standard_normal(256 * 32).astype(np.float32) * np.repeat(
        np.exp(np.random.default_rng(4).uniform(-4, 6, 256)), 32).astype(np.float32)
    b = gf.bf16_bits(x)
    xf = gf.bf16_to_f32(b).reshape(256, 32)
    q = np.empty(x.size, np.int8); s = np.empty(256, np.uint16)
    wz.wzy_bf16_to_q8_0(b.ctypes.data, 256, q.ctypes.data, s.ctypes.data)
    d = s.view(np.float16).astype(np.float64)
    amax = np.abs(xf).max(axis=1).astype(np.float64)
    assert np.array_equal(s.view(np.float16), (np.abs(xf).max(axis=1) / np.float32(127)).astype(np.float16))
    err = np.abs(q.reshape(256, 32) * d[:, None] - xf) / d[:, None]
    clamped = np.abs(q.reshape(256, 32)) == 127                  # where the fp16 scale rounded down
    assert ((err <= 0.5 + 1e-6) | clamped).all() and (err[clamped] <= 0.5 + 127 * 2 ** -11).all()
    top = np.abs(q.reshape(256, 32)).max(axis=1)
    assert ((top == 127) | (top == 126)).all() and (np.abs(amax / d - top) <= 1.0).all()


def test_cfg_from_gguf(wz, tmp_path):
    ref = small_cfg(wzy_amd, ctx_max=512, n_layers=4, topk=64)
    ref.gdn_hk, ref.gdn_hv = 2, 4
    ck = gf.Checkpoint(wz, ref, 3, str(tmp_path / "m"), emb_q8=True, head_q8=False)
    cfg = wzy_amd.StageCfg()
    wz.wzy_stage_cfg_from_gguf(ck.gguf.encode() if isinstance(ck.gguf, str) else str(ck.gguf).encode(), 512,
                               C.byref(cfg))
    for f, _ in wzy_amd.StageCfg._fields_:
        want = getattr(ref, f)
        if f == "idx_topk":
            want = 2048                               # not in the tensors: the reference's constant
        elif f == "emb_q8":
            want = 1
        elif f == "head_q8":
            want = 0
        got = getattr(cfg, f)
        assert got == pytest.approx(want), (f, got, want)
    # without metadata the reference's constants apply
    ck2 = gf.Checkpoint(wz, ref, 3, str(tmp_path / "m2"), metadata=False)
    wz.wzy_stage_cfg_from_gguf(str(ck2.gguf).encode(), 512, C.byref(cfg))
    assert (cfg.top_k, cfg.n_rot, cfg.rope_theta) == (10, 64, pytest.approx(1e7))
    assert cfg.emb_q8 == 1 and cfg.head_q8 == 1 and cfg.ple == 0
    # blk.1.ple_key.weight switches the per-layer embedding on (has_ple)
    ck3 = gf.Checkpoint(wz, ref, 3, str(tmp_path / "m3"), with_ple=True)
    wz.wzy_stage_cfg_from_gguf(str(ck3.gguf).encode(), 512, C.byref(cfg))
    assert cfg.ple == 1 and cfg.ple_eos == 248044
    # attention layers that break the period are rejected
    raw = bytearray(open(ck.gguf, "rb").read())
    i = raw.find(b"blk.3.attn_q.weight")
    raw[i:i + 5] = b"blk.9"
    (tmp_path / "bad.gguf").write_bytes(bytes(raw))
    assert wz.dll.wzy_stage_cfg_from_gguf(str(tmp_path / "bad.gguf").encode(), 512, C.byref(cfg)) < 0

"""Pins the oracle's number formats against independent decoders (CPU only)."""
import numpy as np
import pytest

import refmath


def test_e2m1_table_matches_ocp_values(orc):
    # reference stores 2*value as int8 (src/wzy_stage_v2.cuh:190); OCP MX FP4 values x2
    for code in range(16):
        assert orc.orc_e2m1x2(code) == int(refmath.e2m1_decode([code])[0] * 2)


def test_ue4m3_half_all_codes_vs_torch(orc):
    codes = np.arange(256)
    dec = refmath.e4m3_decode(codes)          # sign ignored like the reference
    for c in range(256):
        assert orc.orc_ue4m3_half(c) == pytest.approx(dec[c] * 0.5, rel=0, abs=0)


def test_ue4m3_known_values(orc):
    # OCP e4m3: 0x38 = 1.0, 0x08 = 2^-6 (min normal), 0x01 = 2^-9 (min subnormal), 0x7E = 448
    assert orc.orc_ue4m3_half(0x38) == 0.5
    assert orc.orc_ue4m3_half(0x08) == 2.0 ** -7
    assert orc.orc_ue4m3_half(0x01) == 2.0 ** -10
    assert orc.orc_ue4m3_half(0x7E) == 224.0
    assert orc.orc_ue4m3_half(0xB8) == 0.5     # sign bit ignored


def test_f16_roundtrip_vs_numpy(orc):
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.standard_normal(20000) * 10.0 ** rng.integers(-8, 5, 20000),
                         [0.0, -0.0, 65504.0, 65519.9, 65520.0, 1e-8, 5.96e-8, 2.98e-8, 6.1035e-5, 6.0e-5]]).astype(np.float32)
    for x in xs:
        h = orc.orc_f32_to_f16(float(x))
        assert h == int(np.float32(x).astype(np.float16).view(np.uint16)), x
    for h in range(0, 65536, 7):
        f = np.uint16(h).view(np.float16)
        if np.isnan(f):
            continue
        assert orc.orc_f16_to_f32(h) == float(f)


def test_bf16_decode_vs_torch(orc):
    import torch
    hs = np.arange(0, 65536, 13, dtype=np.uint16)
    t = torch.from_numpy(hs.view(np.int16).copy()).view(torch.bfloat16).float().numpy()
    for h, v in zip(hs, t):
        if np.isnan(v):
            continue
        assert orc.orc_bf16_to_f32(int(h)) == v


def test_product_half_conversions_match_numpy(wz):
    rng = np.random.default_rng(1)
    for x in (rng.standard_normal(5000) * 100).astype(np.float32):
        assert wz.wzy_f32_to_f16(float(x)) == int(np.float32(x).astype(np.float16).view(np.uint16))
    import torch
    for x in (rng.standard_normal(5000) * 3).astype(np.float32):
        ref = torch.tensor([x], dtype=torch.float32).to(torch.bfloat16).view(torch.int16).item() & 0xFFFF
        assert wz.wzy_f32_to_bf16(float(x)) == ref

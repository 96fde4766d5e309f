"""Stage and QSA configurations this build cannot serve are rejected before any device work (CPU only).

The reference keeps only a ring of recent cells in VRAM and reads older selected cells from a pinned
host mirror (src/wzy_qsa_256k.cuh:17-29).  This build stores the full context in HBM, so a ring that
wraps would serve a newer cell's K/V for an older selected cell; every entry point that takes the
ring fields refuses such a configuration with WZY_EINVAL and a message."""
import ctypes as C

import pytest

import wzy_amd

EINVAL = -1


def stage_cfg(ctx_max, ring, sinks):
    c = wzy_amd.StageCfg()
    wzy_amd.lib().dll.wzy_stage_cfg_default(C.byref(c), ctx_max)
    c.kv_ring, c.kv_sinks = ring, sinks
    return c


@pytest.mark.parametrize("ctx_max,ring,sinks", [(65536, 32768, 4096), (4096, 1024, 0), (8192, 8191, 16),
                                                (4096, 0, 16), (4096, 4096, 4096), (4096, -8, 0)])
def test_stage_create_rejects_wrapping_ring(wz, ctx_max, ring, sinks):
    h = C.c_void_p()
    rc = wz.dll.wzy_stage_create(C.byref(stage_cfg(ctx_max, ring, sinks)), 0, C.byref(h))
    assert rc == EINVAL and not h.value
    msg = wz.wzy_last_error().decode()
    assert "ring" in msg or "sinks" in msg, msg


def qsa_dims(ctx_max, ring, sinks):
    d = wzy_amd.QsaDims()
    d.qh, d.kvh, d.hd, d.n_rot = 24, 2, 256, 64
    d.idx_heads, d.idx_dim, d.idx_blk, d.idx_topk = 4, 128, 4, 2048
    d.ctx_max, d.kv_ring, d.kv_sinks, d.eps = ctx_max, ring, sinks, 1e-6
    return d


@pytest.mark.parametrize("ctx_max,ring,sinks", [(262144, 32768, 4096), (4096, 0, 4)])
def test_qsa_entry_points_reject_wrapping_ring(wz, ctx_max, ring, sinks):
    dm = C.byref(qsa_dims(ctx_max, ring, sinks))
    fake = C.c_void_p(256)          # never dereferenced: the dims are checked first
    assert wz.dll.wzy_qsa_topk(dm, fake, fake, ctx_max // 4 + 2, fake, fake, 1, None) == EINVAL
    assert "ring" in wz.wzy_last_error().decode() or "sinks" in wz.wzy_last_error().decode()
    assert wz.dll.wzy_qsa_select(dm, fake, fake, fake, fake, fake, ctx_max // 4 + 2, fake, fake, 1, None) == EINVAL
    assert wz.dll.wzy_qsa_attend(dm, fake, fake, fake, fake, fake, fake, fake, fake, fake, 1 << 30, 1, None) == EINVAL


@pytest.mark.parametrize("n_embd", [1792, 2304, 2816, 3328, 3584, 3840])
def test_stage_create_rejects_width_without_hc_kernel(wz, n_embd):
    """A stream width that is a multiple of 256 but has no decode HC read kernel is refused when the
    stage is created (before any weights are allocated), not on its first forward."""
    c = stage_cfg(8192, 0, 0)
    c.n_embd = n_embd
    h = C.c_void_p()
    assert wz.dll.wzy_stage_create(C.byref(c), 0, C.byref(h)) == EINVAL and not h.value
    assert "HC read kernel" in wz.wzy_last_error().decode()

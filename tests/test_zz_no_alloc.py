"""wzy_row_top16_noalloc: the allocation-free top-16 reduction (its scratch is a fixed device array
inside the library).  Its results must be bit-identical to wzy_row_top16's, which the reduction
parity test pins against the oracle, on consecutive calls that share the array (the second call
smaller than the first), and sizes beyond the array are refused before anything is launched."""
import ctypes as C

import numpy as np
import pytest

import wzy_amd

DA = wzy_amd.DeviceArray
EINVAL = -1


def logits_rows(V, T, seed):
    rng = np.random.default_rng(seed)
    l = rng.standard_normal(T * V).astype(np.float32)
    l[V // 2] = l[V // 3] = 40.0              # top tie in row 0 -> lower id first
    if T > 1:
        l[V + 5:V + 40] = 30.0                # 35-way tie at the top of row 1
    return l


def run(wz, fn, ld, V, T):
    g = DA(T, np.int32)
    tv = DA(T * 16, np.float32)
    ti = DA(T * 16, np.int32)
    fn(ld.ptr, V, T, g.ptr, tv.ptr, ti.ptr, None)
    wz.wzy_device_sync()
    return g.numpy(), tv.numpy(), ti.numpy()


@pytest.mark.gpu
def test_noalloc_top16_matches_allocating_entry_point(wz, orc, gpu):
    # two calls in a row on the shared array, the second with a smaller input, then the first again
    for V, T, seed in [(248320, 8, 1), (151936, 2, 2), (3001, 1, 3), (248320, 8, 4)]:
        print("case noalloc_top16 V=%d T=%d seed=%d" % (V, T, seed), flush=True)
        l = logits_rows(V, T, seed)
        ld = DA.from_numpy(l)
        got = run(wz, wz.wzy_row_top16_noalloc, ld, V, T)
        ref = run(wz, wz.wzy_row_top16, ld, V, T)
        for a, b in zip(got, ref):
            np.testing.assert_array_equal(a, b)
        rg = np.empty(T, np.int32)
        rv = np.empty(T * 16, np.float32)
        ri = np.empty(T * 16, np.int32)
        orc.orc_row_top16(l.ctypes.data, V, T, rg.ctypes.data, rv.ctypes.data, ri.ctypes.data)
        np.testing.assert_array_equal(got[0], rg)
        np.testing.assert_array_equal(got[2], ri)


def test_noalloc_top16_rejects_sizes_beyond_its_array(wz):
    fake = C.c_void_p(256)                     # never dereferenced: sizes are checked first
    for V, T in [(262145, 1), (151936, 9), (151936, 0), (0, 1)]:
        assert wz.dll.wzy_row_top16_noalloc(fake, V, T, fake, fake, fake, None) == EINVAL
        assert "noalloc" in wz.wzy_last_error().decode()

"""Seeded MoE-layer inputs built with the product's synthetic generator (libwzy_amd host functions).

Tensor streams follow the per-layer tensor ids of the synthetic model (include/wzy_stage.h):
0 router, 1 shared-expert gate row, 2/3/4 shared gate/up/down; inputs use the INPUT stream kind.
"""
import numpy as np

import wzy_amd

S_DENSE = 5
S_INPUT = 7


class MoeLayer:
    pass


def stream(wz, kind, layer, sub):
    return wz.wzy_synth_stream(kind, layer, sub)


def make_layer(wz, seed, layer, D, F, E, K, blobs="all"):
    """Host copies of one MoE layer.  blobs: 'all' materialises every expert in the reference
    layout (small shapes only), a list of ids materialises just those."""
    p = wzy_amd.ptr
    m = MoeLayer()
    m.seed, m.layer, m.D, m.F, m.E, m.K = seed, layer, D, F, E, K
    m.router = np.empty(E * D, np.uint16)
    wz.wzy_synth_normal_bf16(seed, stream(wz, S_DENSE, layer, 0), E * D, 0.0, 0.02, p(m.router))
    m.sgate = np.empty(D, np.uint16)
    wz.wzy_synth_normal_bf16(seed, stream(wz, S_DENSE, layer, 1), D, 0.0, 0.02, p(m.sgate))
    m.sh = {}
    for name, sub, rows, cols in (("gate", 2, F, D), ("up", 3, F, D), ("down", 4, D, F)):
        q = np.empty(rows * cols, np.int8)
        s = np.empty(rows * cols // 32, np.uint16)
        wz.wzy_synth_q8(seed, stream(wz, S_DENSE, layer, sub), rows, cols, float(1.0 / np.sqrt(cols)), p(q), p(s))
        m.sh[name] = (q, s)
    m.blob_bytes = wz.wzy_nvfp4_blob_bytes(D, F)
    m.blobs = {}
    ids = range(E) if blobs == "all" else blobs
    for e in ids:
        m.blobs[e] = expert_blob(wz, seed, layer, e, D, F)
    return m


def expert_blob(wz, seed, layer, e, D, F):
    b = np.empty(wz.wzy_nvfp4_blob_bytes(D, F), np.uint8)
    wz.wzy_synth_expert_blob(seed, layer, e, D, F, wzy_amd.ptr(b))
    return b


def make_x(wz, seed, layer, T, D):
    """T rows of bf16-rounded N(0,1) activations as fp32."""
    h = np.empty(T * D, np.uint16)
    wz.wzy_synth_normal_bf16(seed, stream(wz, S_INPUT, layer, 0), T * D, 0.0, 1.0, wzy_amd.ptr(h))
    return (h.astype(np.uint32) << 16).view(np.float32).reshape(T, D).copy()


def orc_weights(orc_mod, m, blob_ptrs):
    """oracle weights struct; blob_ptrs must stay alive while it is used."""
    import ctypes as C
    w = orc_mod.OrcMoeWeights()
    w.n_embd, w.n_ff, w.n_exp, w.top_k = m.D, m.F, m.E, m.K
    w.router = m.router.ctypes.data
    w.sgate = m.sgate.ctypes.data
    w.blobs = C.cast(blob_ptrs, C.c_void_p).value
    w.sh_gate_q, w.sh_gate_s = m.sh["gate"][0].ctypes.data, m.sh["gate"][1].ctypes.data
    w.sh_up_q, w.sh_up_s = m.sh["up"][0].ctypes.data, m.sh["up"][1].ctypes.data
    w.sh_down_q, w.sh_down_s = m.sh["down"][0].ctypes.data, m.sh["down"][1].ctypes.data
    return w


def blob_ptr_array(m):
    import ctypes as C
    arr = (C.c_void_p * m.E)()
    for e in range(m.E):
        arr[e] = m.blobs[e].ctypes.data if e in m.blobs else None
    return arr

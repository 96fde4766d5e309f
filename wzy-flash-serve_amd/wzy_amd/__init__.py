"""ctypes bindings of libwzy_amd.so, the MI355X decode-path library.

The C ABI (include/wzy_kernels.h, include/wzy_synth.h, include/wzy_stage.h) takes plain pointers and
sizes; these bindings pass integers (device pointers from any allocator, numpy buffer addresses)
and raise WzyError on a negative status.  Loading fails loudly when the shared library has not been
built: there is no CPU fallback behind this module.
"""
import ctypes as C
import os

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_DIR, "libwzy_amd.so")

WZY_MAX_W = 8


class WzyError(RuntimeError):
    pass


P = C.c_void_p
I32 = C.c_int
I64 = C.c_int64
U64 = C.c_uint64
U32 = C.c_uint32
F32 = C.c_float
SZ = C.c_size_t


class MoeWeights(C.Structure):
    """struct wzy_moe_weights (include/wzy_kernels.h)"""
    _fields_ = [
        ("n_embd", I32), ("n_ff", I32), ("n_exp", I32), ("top_k", I32),
        ("router", P), ("sgate", P), ("experts", P),
        ("sh_gate_q", P), ("sh_gate_s", P),
        ("sh_up_q", P), ("sh_up_s", P),
        ("sh_down_q", P), ("sh_down_s", P),
    ]


class GemvSeg(C.Structure):
    _fields_ = [("w", C.c_void_p), ("s", C.c_void_p), ("y", C.c_void_p), ("rows", C.c_int), ("kind", C.c_int),
                ("y_stride", C.c_int)]


GEMV_Q8, GEMV_BF16 = 0, 1


class QsaDims(C.Structure):
    """struct wzy_qsa_dims (include/wzy_kernels.h)"""
    _fields_ = [("qh", I32), ("kvh", I32), ("hd", I32), ("n_rot", I32),
                ("idx_heads", I32), ("idx_dim", I32), ("idx_blk", I32), ("idx_topk", I32),
                ("ctx_max", I32), ("kv_ring", I32), ("kv_sinks", I32), ("eps", F32), ("attn_f16_above", I32)]


class QsaLayer(C.Structure):
    """struct wzy_qsa_layer (include/wzy_kernels.h)"""
    _fields_ = [("qg", P), ("kk", P), ("vv", P), ("q_idx", P), ("idx_raw", P),
                ("q_norm", P), ("k_norm", P), ("iq_norm", P), ("ik_norm", P), ("cos_tab", P), ("sin_tab", P),
                ("kq", P), ("ks", P), ("vq", P), ("vs", P), ("idx_tail", P), ("idx_dead", P), ("idx_pooled", P),
                ("scores", P), ("max_b", I32), ("sel_ids", P), ("sel_cnt", P), ("out", P), ("workspace", P),
                ("workspace_bytes", SZ)]


class StageCfg(C.Structure):
    """struct wzy_stage_cfg (include/wzy_stage.h)"""
    _fields_ = [("n_layers", I32), ("qsa_period", I32), ("n_embd", I32), ("hc", I32), ("hc_lr", I32),
                ("gdn_hk", I32), ("gdn_hv", I32), ("qsa_qh", I32), ("qsa_kvh", I32), ("qsa_hd", I32),
                ("n_rot", I32), ("idx_heads", I32), ("idx_dim", I32), ("idx_blk", I32), ("idx_topk", I32),
                ("n_exp", I32), ("top_k", I32), ("n_ff", I32), ("n_vocab", I32), ("ctx_max", I32),
                ("kv_ring", I32), ("kv_sinks", I32), ("rope_theta", F32), ("eps", F32),
                ("emb_q8", I32), ("head_q8", I32), ("attn_f16_above", I32), ("ple", I32), ("ple_eos", I32)]


WZY_MAX_STOPS = 64


class GenCfg(C.Structure):
    """struct wzy_gen_cfg (include/wzy_engine.h)"""
    _fields_ = [("max_new", I32), ("temp", F32), ("top_p", F32), ("top_k", I32), ("min_p", F32),
                ("rep_pen", F32), ("spec_min_p", F32), ("spec_k", I32), ("no_reuse", I32),
                ("n_stops", I32), ("stops", I32 * WZY_MAX_STOPS)]


class SpecGates(C.Structure):
    """struct wzy_spec_gates (include/wzy_engine.h)"""
    _fields_ = [("depth", I32), ("min_p", F32), ("gate", F32)]


class Request(C.Structure):
    """struct wzy_request (include/wzy_engine.h)"""
    _fields_ = [("json", I32), ("has_req", I32), ("req", I32), ("n_ids", I32), ("cfg", GenCfg),
                ("has_emb_file", I32)]


class LineFields(C.Structure):
    """struct wzy_line_fields (include/wzy_engine.h)"""
    _fields_ = [("req", I32), ("generated", I32), ("prompt_tokens", I32), ("reused", I32), ("read", I32),
                ("prompt_ms", C.c_double), ("decode_ms", C.c_double), ("draft_n", C.c_longlong),
                ("draft_accepted", C.c_longlong), ("promoted", C.c_longlong), ("vram_hit", C.c_double),
                ("restored_park", I32), ("parked_tokens", I32), ("active_tokens", I32),
                ("finish", C.c_char_p)]


LINE_KINDS = {0: "SKIP", 1: "PING", 2: "RESET", 3: "SAVE_PROFILE", 4: "QUIT", 5: "CANCEL", 6: "REQUEST"}
FMT_PREFILL, FMT_DONE, FMT_DONE_EMPTY = 1, 2, 3
# wzy_engine_session_plan results (include/wzy_engine.h)
SESS_REUSE, SESS_SWAP, SESS_RESTORE, SESS_PARK_RESET, SESS_RESET = 0, 1, 2, 3, 4
SESSION_SLOTS = 2

# name -> (restype, argtypes, checked)
_SIGS = {
    # engine host logic
    "wzy_engine_cfg_default": (None, [C.POINTER(GenCfg)], False),
    "wzy_engine_parse_line": (I32, [C.c_char_p, C.POINTER(Request), P, I32], False),
    "wzy_engine_target_dist": (I32, [P, I32, C.POINTER(GenCfg), P, I32, P, P, I32], False),
    "wzy_engine_verify_full": (I32, [P, I32, C.POINTER(GenCfg), P, I32, I32, F32, C.POINTER(I32)], False),
    "wzy_engine_verify_top16": (I32, [P, P, C.POINTER(GenCfg), P, I32, I32, F32, C.POINTER(I32)], False),
    "wzy_engine_reuse_prefix": (I32, [P, I32, P, I32], False),
    "wzy_engine_session_plan": (I32, [P, I32, P, I32, P, I32, I32, C.POINTER(I32)], False),
    "wzy_engine_spec_gates_default": (None, [C.POINTER(SpecGates)], False),
    "wzy_engine_mtp_gate": (I32, [P, P, I32, I32, I32, I32, C.POINTER(GenCfg), I32, C.POINTER(SpecGates)], False),
    "wzy_engine_format": (I32, [I32, C.POINTER(LineFields), C.c_char_p, I32], False),
    # stage
    "wzy_stage_cfg_default": (None, [C.POINTER(StageCfg), I32], False),
    "wzy_stage_create": (I32, [C.POINTER(StageCfg), I32, C.POINTER(P)], True),
    "wzy_stage_destroy": (I32, [P], True),
    "wzy_stage_device_bytes": (SZ, [P], False),
    "wzy_stage_load_synthetic": (I32, [P, U64, I32], True),
    "wzy_stage_record_forward": (I32, [P, I32, P, P, I32, I32, I32, I32, I32], True),
    "wzy_stage_prefill": (I32, [P, I32, P, I32], True),
    "wzy_stage_can_prefill": (I32, [C.POINTER(StageCfg)], False),
    "wzy_stage_prefill_time": (I32, [P, I32, P, I32, C.POINTER(F32)], True),
    "wzy_stage_service_cold_layers": (I32, [P], True),
    "wzy_stage_promote_cold": (I32, [P], True),
    "wzy_stage_commit_window_state": (I32, [P, I32, I32], True),
    "wzy_stage_reset_state": (I32, [P], True),
    "wzy_stage_sync": (I32, [P], True),
    "wzy_stage_session_bytes": (SZ, [P, I32], False),
    "wzy_stage_session_save": (I32, [P, I32, I32], True),
    "wzy_stage_session_restore": (I32, [P, I32], True),
    "wzy_stage_session_cells": (I32, [P, I32], False),
    "wzy_stage_session_clear": (I32, [P, I32], True),
    "wzy_stage_greedy_ids": (I32, [P, P, I32], True),
    "wzy_stage_top16": (I32, [P, P, P, I32], True),
    "wzy_stage_logits": (I32, [P, P, I32], True),
    "wzy_stage_pre_head": (I32, [P, P, I32], True),
    "wzy_stage_set_graphs": (I32, [P, I32], True),
    "wzy_stage_set_trace": (I32, [P, I32], True),
    "wzy_stage_read_tensor_range": (I32, [P, I32, C.c_char_p, SZ, P, SZ], True),
    "wzy_stage_write_tensor_range": (I32, [P, I32, C.c_char_p, SZ, P, SZ], True),
    "wzy_stage_stream": (P, [P], False),
    "wzy_stage_tensor_bytes": (SZ, [P, I32, C.c_char_p], False),
    "wzy_stage_read_tensor": (I32, [P, I32, C.c_char_p, P, SZ], True),
    "wzy_stage_write_tensor": (I32, [P, I32, C.c_char_p, P, SZ], True),
    "wzy_stage_time_moe": (I32, [P, I32, C.POINTER(F32), C.POINTER(F32), C.POINTER(F32)], True),
    "wzy_stage_mtp_init": (I32, [P, U64, I32], True),
    "wzy_stage_mtp_init_vocab": (I32, [P, P, I32], True),
    "wzy_stage_mtp_reset": (I32, [P], True),
    "wzy_stage_mtp_set_floor": (I32, [P, I32], True),
    "wzy_stage_mtp_front": (I32, [P, I32, P, I32, I32], True),
    "wzy_stage_mtp_draft": (I32, [P, I32, I32, I32, I32, P, P], True),
    "wzy_stage_mtp_propose": (I32, [P, I32, I32, P, I32, P, P], True),
    "wzy_stage_mtp_time": (I32, [P, I32, I32, I32, I32, C.POINTER(F32)], True),
    # layer kernels
    "wzy_hc_read_workspace_bytes": (SZ, [I32, I32, I32], False),
    "wzy_hc_read": (I32, [P, P, P, I32, P, P, P, P, P, P, P, P, P, P, P, P, P, I32, I32, I32, F32, I32, P, SZ, P], True),
    "wzy_gdn_step": (I32, [P, P, P, P, P, P, P, P, P, F32, P, I32, I32, I32, P, P, P], True),
    "wzy_gdn_recurrence": (I32, [P, P, P, P, P, P, P, F32, P, P, I32, I32, I32, P, P], True),
    "wzy_qsa_prepare": (I32, [C.POINTER(QsaDims), P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, I32, P], True),
    "wzy_qsa_select": (I32, [C.POINTER(QsaDims), P, P, P, P, P, I32, P, P, I32, P], True),
    "wzy_qsa_topk": (I32, [C.POINTER(QsaDims), P, P, I32, P, P, I32, P], True),
    "wzy_gemv_segs": (I32, [C.POINTER(GemvSeg), I32, P, I32, I32, P], True),
    "wzy_qsa_attend_workspace_bytes": (SZ, [C.POINTER(QsaDims), I32], False),
    "wzy_qsa_attend": (I32, [C.POINTER(QsaDims), P, P, P, P, P, P, P, P, P, SZ, I32, P], True),
    "wzy_last_error": (C.c_char_p, [], False),
    "wzy_version": (C.c_char_p, [], False),
    # kernels
    "wzy_quant_act": (I32, [P, P, P, P, P, I32, I32, P], True),
    "wzy_gemv_q8": (I32, [P, P, P, P, P, I32, I32, I32, I32, P], True),
    "wzy_gemv_bf16": (I32, [P, P, P, I32, I32, I32, I32, P], True),
    "wzy_nvfp4_expert_bytes": (SZ, [I32, I32], False),
    "wzy_nvfp4_blob_bytes": (SZ, [I32, I32], False),
    "wzy_nvfp4_repack_host": (I32, [P, P, I32, I32], True),
    "wzy_moe_workspace_bytes": (SZ, [I32, I32, I32, I32, I32], False),
    "wzy_moe_block": (I32, [C.POINTER(MoeWeights), P, I32, P, P, P, P, SZ, P], True),
    "wzy_moe_route": (I32, [P, I32, I32, I32, P, P, P], True),
    "wzy_gemm_bf16": (I32, [P, I32, I32, I32, P, P, P, I32, P, P, I32, P], True),
    "wzy_moe_prefill_workspace_bytes": (SZ, [I32, I32, I32, I32, I32], False),
    "wzy_moe_prefill": (I32, [C.POINTER(MoeWeights), P, I32, P, P, P, P, SZ, P], True),
    "wzy_moe_prefill_time": (I32, [C.POINTER(MoeWeights), P, I32, P, P, SZ, I32, C.POINTER(F32), P], True),
    "wzy_stage_moe_weights": (I32, [P, I32, C.POINTER(MoeWeights)], True),
    "wzy_moe_time_kernels": (I32, [C.POINTER(MoeWeights), I32, I32, P, P, SZ, I32, C.POINTER(F32),
                                   C.POINTER(F32), C.POINTER(F32), P], True),
    "wzy_row_argmax": (I32, [P, I32, I32, P, P], True),
    "wzy_row_top16": (I32, [P, I32, I32, P, P, P, P], True),
    "wzy_row_top16_noalloc": (I32, [P, I32, I32, P, P, P, P], True),
    "wzy_gdn_time_recurrence": (I32, [P, P, P, P, P, P, P, I32, I32, I32, I32, I32, P, P, P], True),
    "wzy_qsa_time_decode": (I32, [C.POINTER(QsaDims), C.POINTER(QsaLayer), P, I32, P, P], True),
    "wzy_ple_table_rows": (U64, [], False),
    "wzy_ple_rows": (I32, [P, I32, F32, I32, P, P, I32, P, I32, P, P, P], True),
    "wzy_ple_workspace_bytes": (SZ, [I32, I32, I32], False),
    "wzy_ple_block": (I32, [P, P, P, P, P, P, P, P, P, P, P, I32, I32, F32, I32, P, P, SZ, P], True),
    "wzy_synth_ple_row": (None, [U64, U64, I32, P], False),
    "wzy_synth_ple_table_device": (I32, [U64, I32, P, P], True),
    # synth
    "wzy_synth_hash": (U64, [U64, U64, U64], False),
    "wzy_synth_stream": (U64, [U32, U32, U32], False),
    "wzy_synth_normal": (None, [U64, U64, SZ, F32, F32, P], False),
    "wzy_synth_uniform": (None, [U64, U64, SZ, F32, F32, P], False),
    "wzy_synth_normal_bf16": (None, [U64, U64, SZ, F32, F32, P], False),
    "wzy_synth_q8": (None, [U64, U64, I32, I32, F32, P, P], False),
    "wzy_synth_expert_blob": (I32, [U64, I32, I32, I32, I32, P], True),
    "wzy_q2_expert_bytes": (SZ, [I32, I32], False),
    "wzy_synth_q2_expert": (I32, [U64, I32, I32, I32, P], True),
    "wzy_synth_q2_experts_device": (I32, [U64, I32, I32, I32, I32, P, P], True),
    "wzy_synth_expert_planes": (I32, [U64, I32, I32, I32, I32, P], True),
    "wzy_synth_experts_device": (I32, [U64, I32, I32, I32, I32, I32, P, P], True),
    "wzy_synth_kv_host": (None, [U64, I32, I32, I64, I32, I32, P, P], False),
    "wzy_synth_kv_device": (I32, [U64, I32, I32, I64, I32, I32, P, P, P], True),
    "wzy_f32_to_f16": (C.c_uint16, [F32], False),
    "wzy_f16_to_f32": (F32, [C.c_uint16], False),
    "wzy_f32_to_bf16": (C.c_uint16, [F32], False),
    # real-weight loaders
    "wzy_gguf_open": (I32, [C.c_char_p, C.POINTER(P)], True),
    "wzy_gguf_close": (None, [P], False),
    "wzy_gguf_n_tensors": (I32, [P], False),
    "wzy_gguf_find": (I32, [P, C.c_char_p], False),
    "wzy_gguf_tensor_info": (I32, [P, I32, C.POINTER(C.c_char_p), C.POINTER(I32), C.POINTER(I64), C.POINTER(I32),
                                   C.POINTER(SZ)], True),
    "wzy_gguf_tensor_data": (P, [P, I32], False),
    "wzy_gguf_get_int": (I32, [P, C.c_char_p, C.POINTER(I64)], False),
    "wzy_gguf_get_float": (I32, [P, C.c_char_p, C.POINTER(C.c_double)], False),
    "wzy_gguf_get_str": (I32, [P, C.c_char_p, C.POINTER(C.c_char_p), C.POINTER(SZ)], False),
    "wzy_q8_0_split": (None, [P, SZ, P, P], False),
    "wzy_bf16_to_q8_0": (None, [P, SZ, P, P], False),
    "wzy_bf16_from_f32": (None, [P, SZ, P], False),
    "wzy_to_f32": (I32, [I32, P, SZ, P], True),
    "wzy_stage_cfg_from_gguf": (I32, [C.c_char_p, I32, C.POINTER(StageCfg)], True),
    "wzy_stage_load_gguf": (I32, [P, C.c_char_p, C.c_char_p, C.c_char_p], True),
    "wzy_stage_load_ple": (I32, [P, C.c_char_p], True),
    "wzy_stage_mtp_load": (I32, [P, C.c_char_p, C.c_char_p], True),
    # runtime plumbing
    "wzy_dev_count": (I32, [C.POINTER(I32)], True),
    "wzy_dev_set": (I32, [I32], True),
    "wzy_dev_name": (I32, [I32, C.c_char_p, I32], True),
    "wzy_mem_info": (I32, [C.POINTER(SZ), C.POINTER(SZ)], True),
    "wzy_dev_malloc": (I32, [C.POINTER(P), SZ], True),
    "wzy_dev_free": (I32, [P], True),
    "wzy_memcpy_h2d": (I32, [P, P, SZ, P], True),
    "wzy_memcpy_d2h": (I32, [P, P, SZ, P], True),
    "wzy_memcpy_d2d": (I32, [P, P, SZ, P], True),
    "wzy_memset": (I32, [P, I32, SZ, P], True),
    "wzy_stream_create": (I32, [C.POINTER(P)], True),
    "wzy_stream_destroy": (I32, [P], True),
    "wzy_stream_sync": (I32, [P], True),
    "wzy_device_sync": (I32, [], True),
    "wzy_host_malloc": (I32, [C.POINTER(P), SZ], True),
    "wzy_host_free": (I32, [P], True),
}


class _Lib:
    def __init__(self, path=LIB_PATH):
        if not os.path.exists(path):
            raise WzyError("libwzy_amd.so not built (%s); run __graft_entry__.build()" % path)
        self.path = path
        self.dll = C.CDLL(path)
        for name, (res, args, checked) in _SIGS.items():
            fn = getattr(self.dll, name, None)
            if fn is None:
                continue
            fn.restype = res
            fn.argtypes = args
            setattr(self, name, self._wrap(fn, name) if checked else fn)

    def _wrap(self, fn, name):
        def call(*a):
            rc = fn(*a)
            if rc != 0:
                raise WzyError("%s failed (%d): %s" % (name, rc, self.dll.wzy_last_error().decode()))
            return rc
        call.__name__ = name
        return call

    def has(self, name):
        return hasattr(self.dll, name)


_LIB = None


def lib():
    """The loaded library (process-wide singleton)."""
    global _LIB
    if _LIB is None:
        _LIB = _Lib()
    return _LIB


def ptr(x):
    """Address of a numpy array / DeviceArray / int / None as a ctypes-compatible int."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if isinstance(x, DeviceArray):
        return x.ptr
    if hasattr(x, "ctypes"):
        return x.ctypes.data
    raise TypeError("cannot take the address of %r" % type(x))


def device_count():
    n = I32(0)
    lib().wzy_dev_count(C.byref(n))
    return n.value


class DeviceArray:
    """A device buffer owned through wzy_dev_malloc, with a numpy dtype and shape for convenience."""

    def __init__(self, shape, dtype, zero=False):
        import numpy as np
        self.dtype = np.dtype(dtype)
        self.shape = tuple(shape) if hasattr(shape, "__len__") else (int(shape),)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = P()
        lib().wzy_dev_malloc(C.byref(p), max(self.nbytes, 1))
        self.ptr = p.value
        if zero:
            lib().wzy_memset(self.ptr, 0, self.nbytes, None)

    @classmethod
    def from_numpy(cls, a):
        import numpy as np
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        lib().wzy_memcpy_h2d(d.ptr, a.ctypes.data, d.nbytes, None)
        return d

    def numpy(self):
        import numpy as np
        out = np.empty(self.shape, self.dtype)
        lib().wzy_memcpy_d2h(out.ctypes.data, self.ptr, self.nbytes, None)
        return out

    def free(self):
        if getattr(self, "ptr", None):
            lib().wzy_dev_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stage:
    """Owning handle of a wzy_stage (include/wzy_stage.h)."""

    def __init__(self, cfg, device=0):
        self.lib = lib()
        self.cfg = cfg
        h = P()
        self.lib.wzy_stage_create(C.byref(cfg), device, C.byref(h))
        self.h = h.value

    def close(self):
        if getattr(self, "h", None):
            self.lib.wzy_stage_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def load_synthetic(self, seed, n_ctx):
        self.lib.wzy_stage_load_synthetic(self.h, seed, n_ctx)

    def load_gguf(self, gguf_path, experts_path, emb_path=None):
        """Real weights: the GGUF checkpoint, the NVFP4 expert pack and optionally a bf16 embedding file."""
        self.lib.wzy_stage_load_gguf(self.h, str(gguf_path).encode(), str(experts_path).encode(),
                                     None if emb_path is None else str(emb_path).encode())

    def load_ple(self, ple_path):
        """The per-layer embedding table (the reference's ple-fp8.gguf) of a stage with cfg.ple."""
        self.lib.wzy_stage_load_ple(self.h, str(ple_path).encode())

    def forward(self, pos, toks, run_head=True, save_snaps=False, want_top16=False, snap_offset=0, emb=None):
        import numpy as np
        toks = np.ascontiguousarray(toks, dtype=np.int32)
        e = None if emb is None else np.ascontiguousarray(emb, dtype=np.float32)
        self.lib.wzy_stage_record_forward(self.h, int(pos), ptr(e), toks.ctypes.data, len(toks), int(run_head),
                                          int(save_snaps), int(want_top16), int(snap_offset))

    def prefill(self, pos, toks):
        import numpy as np
        toks = np.ascontiguousarray(toks, dtype=np.int32)
        self.lib.wzy_stage_prefill(self.h, int(pos), toks.ctypes.data, len(toks))

    def sync(self):
        self.lib.wzy_stage_sync(self.h)

    def greedy(self, T):
        import numpy as np
        out = np.empty(T, np.int32)
        self.lib.wzy_stage_greedy_ids(self.h, out.ctypes.data, T)
        return out

    def top16(self, T):
        import numpy as np
        v = np.empty(T * 16, np.float32)
        i = np.empty(T * 16, np.int32)
        self.lib.wzy_stage_top16(self.h, v.ctypes.data, i.ctypes.data, T)
        return v.reshape(T, 16), i.reshape(T, 16)

    def logits(self, T):
        import numpy as np
        out = np.empty((T, self.cfg.n_vocab), np.float32)
        self.lib.wzy_stage_logits(self.h, out.ctypes.data, T)
        return out

    def pre_head(self, T):
        import numpy as np
        out = np.empty((T, self.cfg.hc, self.cfg.n_embd), np.float32)
        self.lib.wzy_stage_pre_head(self.h, out.ctypes.data, T)
        return out

    def read(self, layer, name, dtype):
        import numpy as np
        n = self.lib.wzy_stage_tensor_bytes(self.h, layer, name.encode())
        if n == 0:
            raise WzyError("no tensor %s in layer %d" % (name, layer))
        out = np.empty(n // np.dtype(dtype).itemsize, dtype)
        self.lib.wzy_stage_read_tensor(self.h, layer, name.encode(), out.ctypes.data, out.nbytes)
        return out

    def read_range(self, layer, name, dtype, first, count):
        """Elements [first, first + count) of a tensor."""
        import numpy as np
        it = np.dtype(dtype).itemsize
        out = np.empty(count, dtype)
        self.lib.wzy_stage_read_tensor_range(self.h, layer, name.encode(), first * it, out.ctypes.data, count * it)
        return out

    def write(self, layer, name, arr):
        import numpy as np
        a = np.ascontiguousarray(arr)
        self.lib.wzy_stage_write_tensor(self.h, layer, name.encode(), a.ctypes.data, a.nbytes)

    # ---- MTP drafter ----
    def mtp_init(self, seed, n_dvocab):
        self.lib.wzy_stage_mtp_init(self.h, int(seed), int(n_dvocab))

    def mtp_load(self, mtp_dir, dvocab_path):
        """The drafter from dense.txt / dense.bin / experts.bin in mtp_dir and a draft vocabulary file."""
        self.lib.wzy_stage_mtp_load(self.h, str(mtp_dir).encode(), str(dvocab_path).encode())

    def mtp_reset(self):
        self.lib.wzy_stage_mtp_reset(self.h)

    def mtp_set_floor(self, floor):
        self.lib.wzy_stage_mtp_set_floor(self.h, int(floor))

    def mtp_front(self, cell0, next_toks, src_row0=0):
        import numpy as np
        t = np.ascontiguousarray(next_toks, dtype=np.int32)
        self.lib.wzy_stage_mtp_front(self.h, int(cell0), t.ctypes.data, len(t), int(src_row0))

    def mtp_draft(self, cell, tok, src_row, depth):
        """-> (token ids [depth], probabilities [depth])"""
        import numpy as np
        toks = np.empty(depth, np.int32)
        probs = np.empty(depth, np.float32)
        self.lib.wzy_stage_mtp_draft(self.h, int(cell), int(tok), int(src_row), int(depth), toks.ctypes.data,
                                     probs.ctypes.data)
        return toks, probs

    def mtp_propose(self, cell0, next_toks, depth):
        import numpy as np
        t = np.ascontiguousarray(next_toks, dtype=np.int32)
        toks = np.empty(depth, np.int32)
        probs = np.empty(depth, np.float32)
        self.lib.wzy_stage_mtp_propose(self.h, int(cell0), len(t), t.ctypes.data, int(depth), toks.ctypes.data,
                                       probs.ctypes.data)
        return toks, probs


def default_cfg(ctx_max):
    c = StageCfg()
    lib().wzy_stage_cfg_default(C.byref(c), ctx_max)
    return c

"""ctypes binding of oracle/liboracle.so (the CPU oracle).  Test infrastructure only."""
import ctypes as C
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "oracle", "liboracle.so")

P, I32, F32, SZ = C.c_void_p, C.c_int, C.c_float, C.c_size_t


class OrcMoeWeights(C.Structure):
    _fields_ = [("n_embd", I32), ("n_ff", I32), ("n_exp", I32), ("top_k", I32),
                ("router", P), ("sgate", P), ("blobs", P),
                ("sh_gate_q", P), ("sh_gate_s", P), ("sh_up_q", P), ("sh_up_s", P),
                ("sh_down_q", P), ("sh_down_s", P)]


_SIGS = {
    "orc_e2m1x2": (I32, [I32]),
    "orc_ue4m3_half": (F32, [I32]),
    "orc_f16_to_f32": (F32, [C.c_uint16]),
    "orc_f32_to_f16": (C.c_uint16, [F32]),
    "orc_bf16_to_f32": (F32, [C.c_uint16]),
    "orc_blob_bytes": (SZ, [I32, I32]),
    "orc_quant_act": (None, [P, I32, I32, P, P, P, P]),
    "orc_gemv_q8": (None, [P, P, P, P, P, I32, I32, I32]),
    "orc_gemv_bf16": (None, [P, P, P, I32, I32, I32]),
    "orc_router_topk": (None, [P, I32, I32, I32, P, P, P]),
    "orc_expert_gate_up": (None, [P, I32, I32, P, P, P, P, P]),
    "orc_expert_down": (None, [P, I32, I32, P, P, P]),
    "orc_moe_block": (I32, [C.POINTER(OrcMoeWeights), P, I32, P, P, P, P, P]),
    "orc_moe_prefill": (I32, [C.POINTER(OrcMoeWeights), P, I32, P, P, P]),
    "orc_pf_gemm": (None, [P, I32, I32, P, P, P, I32, P, I32]),
    "orc_hc_read_pf": (None, [P, P, P, P, P, P, P, P, P, I32, I32, I32, F32, I32, P, P]),
    "orc_hc_write": (None, [P, P, P, I32, I32, I32]),
    "orc_attend_pf": (None, [P, P, P, P, P, P, I32, I32, I32, I32, P]),
    "orc_hc_read": (None, [P, P, P, P, P, P, P, P, P, P, I32, I32, I32, F32, I32, P, P, P, P, P]),
    "orc_gdn_step": (None, [P, P, P, P, P, P, P, P, P, F32, P, I32, I32, I32]),
    "orc_gdn_recurrence": (None, [P, P, P, P, P, P, P, F32, P, P, I32, I32, I32]),
    "orc_rope_tables": (None, [I32, I32, F32, P, P]),
    "orc_head_norm_rope": (None, [P, I32, P, P, P, I32, I32, F32]),
    "orc_kv_quant_row": (None, [P, I32, P, P]),
    "orc_indexer_append": (None, [P, P, P, P, I32, I32, I32, I32, F32, P, P, P]),
    "orc_indexer_append_f32": (None, [P, P, P, P, I32, I32, I32, I32, F32, P, P, P, P]),
    "orc_block_scores": (None, [P, P, P, I32, I32, I32, I32, P]),
    "orc_topk_select": (I32, [P, I32, I32, I32, P]),
    "orc_attend": (None, [P, P, P, P, P, P, I32, I32, I32, I32, P]),
    "orc_row_argmax": (None, [P, I32, I32, P]),
    "orc_row_top16": (None, [P, I32, I32, P, P, P]),
    "orc_q2_blob_bytes": (SZ, [I32, I32]),
    "orc_q2_code": (I32, [P, I32]),
    "orc_q2_expert_gate_up": (None, [P, I32, I32, P, P, P, P, P]),
    "orc_q2_expert_down": (None, [P, I32, I32, P, P, P]),
    "orc_mtp_front": (None, [P, I32, P, P, I32, P, P, P]),
    "orc_mtp_step": (I32, [P, I32, I32, P, P, P, P, P, P]),
    "orc_ple_table_rows": (C.c_uint64, []),
    "orc_ple_row_ids": (None, [I32, I32, I32, I32, P]),
    "orc_ple_fp8": (F32, [C.c_uint8, F32]),
    "orc_ple_rows": (None, [P, P, I32, F32, I32, P, I32, I32, P, P]),
    "orc_ple_block": (None, [P, P, P, P, P, P, P, P, P, P, P, I32, I32, F32, I32, I32, P]),
    "orc_cpu_pool_create": (P, [I32, I32, I32]),
    "orc_cpu_pool_destroy": (None, [P]),
    "orc_cpu_pool_threads": (I32, [P]),
    "orc_cpu_pool_run": (I32, [P, P, P, P, I32, I32, P, P, P]),
}

_lib = None


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            raise RuntimeError("oracle not built (%s): run __graft_entry__.build()" % LIB)
        _lib = C.CDLL(LIB)
        for name, (res, args) in _SIGS.items():
            fn = getattr(_lib, name, None)
            if fn is not None:
                fn.restype, fn.argtypes = res, args
    return _lib


def ptr(a):
    if a is None:
        return None
    return a.ctypes.data

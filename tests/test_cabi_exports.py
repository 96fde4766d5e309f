"""The C-ABI library loads without a GPU and exports every function that include/*.h declares (CPU only)."""
import ctypes as C
import os
import re

import pytest

import wzy_amd

INCLUDE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include")
DECL = re.compile(r"^[A-Za-z_][\w \*]*?\b(wzy_\w+)\s*\(", re.M)


def _strip_comments(src):
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return re.sub(r"//[^\n]*", "", src)


def declared_functions():
    out = {}
    for name in sorted(os.listdir(INCLUDE)):
        if name.endswith(".h"):
            with open(os.path.join(INCLUDE, name)) as fh:
                src = _strip_comments(fh.read())
            for m in DECL.finditer(src):
                if not src[m.start():m.end()].lstrip().startswith(("#", "typedef", "return")):
                    out[m.group(1)] = name
    return out


def test_headers_declare_the_expected_surface():
    fns = declared_functions()
    for must in ("wzy_stage_create", "wzy_stage_record_forward", "wzy_stage_commit_window_state",
                 "wzy_moe_block", "wzy_row_top16", "wzy_qsa_select", "wzy_gdn_step", "wzy_hc_read",
                 "wzy_engine_parse_line", "wzy_engine_verify_top16", "wzy_last_error"):
        assert must in fns, must
    assert len(fns) >= 70


def test_library_exports_every_declared_function():
    dll = C.CDLL(wzy_amd.LIB_PATH)
    missing = sorted(n for n in declared_functions() if not hasattr(dll, n))
    assert not missing, "declared in include/*.h but not exported: %s" % missing


def test_bindings_cover_every_declared_function():
    missing = sorted(n for n in declared_functions() if n not in wzy_amd._SIGS)
    assert not missing, "no ctypes signature for: %s" % missing


def test_error_reporting_without_gpu(wz):
    # a bad argument is rejected on the host with a message, before any device work
    assert wz.dll.wzy_quant_act(None, None, None, None, None, 31, 1, None) < 0
    assert wz.wzy_last_error().decode() != ""
    assert wz.wzy_version().decode()

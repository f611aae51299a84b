"""CPU checks of the C ABI: the library loads, exports every symbol include/k2t_hip.h
declares, and its non-compute entry points behave as documented without a GPU."""
import ctypes as C
import os
import re

import pytest

import k2t

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_symbols():
    text = open(os.path.join(ROOT, "include", "k2t_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(k2t_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = C.CDLL(k2t.LIB_PATH)
    syms = _header_symbols()
    assert len(syms) >= 20
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing
    # and the Python mirror binds exactly the declared surface
    assert sorted(k2t.SIGNATURES) == syms


def test_no_gpu_entry_points():
    L = k2t.lib()
    assert L.k2t_version().decode().startswith("k2t-hip")
    L.k2t_ctx_destroy(None)  # no-op
    L.k2t_mat_destroy(None)  # no-op
    if L.k2t_device_count() == 0:
        h = C.c_void_p()
        rc = L.k2t_ctx_create(0, C.byref(h))
        assert rc < 0 and not h.value
        assert L.k2t_last_error().decode()


def test_argument_errors_are_reported_not_crashes():
    L = k2t.lib()
    rc = L.k2t_ctx_create(0, None)
    assert rc == -1 and "NULL" in L.k2t_last_error().decode()
    rc = L.k2t_gemv(None, None, None, None, None, 1, 0, -1, None, 0)
    assert rc == -1
    rc = L.k2t_mat_upload_nibble4(None, 16, 64, 0, None, 0, None, 0, C.byref(C.c_void_p()))
    assert rc == -1
    with pytest.raises(k2t.K2TError):
        k2t.check(L.k2t_act_quant(None, None, None, None, 64, 1, None, None, None))

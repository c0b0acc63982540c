"""The C-ABI library loads and exports every entry point its header declares
(no device needed)."""
import ctypes
import os
import re

from hessboost_amd import _capi as A

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "hessboost_rocm.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hbr_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared()
    assert len(names) > 40


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(A.LIB_PATH)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_the_header():
    assert sorted(A.SIGNATURES) == declared()


def test_error_reporting_without_device():
    """A malformed call reports HBR_INVALID and a message, touching no GPU."""
    L = A.lib()
    out = ctypes.c_void_p()
    st = L.hbr_cuts_from_dense(None, 10, 3, 256, None, float("nan"), ctypes.byref(out))
    assert st == A.INVALID
    assert "cuts" in A.last_error()


def test_csr_cuts_refuse_null_entries_without_device():
    """A CSR with entries but no column or value array is a caller error
    (HBR_INVALID), for the untyped and the typed entry point alike."""
    import numpy as np
    L = A.lib()
    rp = np.array([0, 2, 3], np.uint64)
    col = np.array([0, 1, 1], np.uint32)
    val = np.array([1.0, 2.0, 3.0], np.float32)
    out = ctypes.c_void_p()
    for c, v in ((None, A.ptr(val)), (A.ptr(col), None)):
        st = L.hbr_cuts_from_csr(A.ptr(rp), c, v, 2, 2, 256, None, ctypes.byref(out))
        assert st == A.INVALID and "null col or val" in A.last_error()
        st = L.hbr_cuts_from_csr_typed(A.ptr(rp), c, v, 2, 2, 256, None, None, ctypes.byref(out))
        assert st == A.INVALID and "null col or val" in A.last_error()
    empty = np.zeros(3, np.uint64)
    st = L.hbr_cuts_from_csr(A.ptr(empty), None, None, 2, 2, 256, None, ctypes.byref(out))
    assert st == A.OK
    L.hbr_cuts_free(out)

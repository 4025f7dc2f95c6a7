"""The C-ABI library loads and exports every entry point the header
declares; argument checks that need no GPU return their documented status."""
import ctypes as C
import os
import re

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ncmorph_amd.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ncm_[a-z0-9_]+)\s*\(", text)))


def test_exports_every_declared_symbol(ncm):
    from ncmorph_amd import _lib

    L = C.CDLL(_lib.LIB_PATH)
    syms = declared_symbols()
    assert len(syms) >= 15
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing
    bound = {name for name, _, _ in _lib.SIGNATURES}
    assert set(syms) == bound


def test_status_strings(ncm):
    L = ncm.lib()
    for code in range(0, -8, -1):
        assert L.ncm_status_string(code)
    assert L.ncm_status_string(-99) == b"unknown status"


def test_null_context_rejected(ncm):
    L = ncm.lib()
    assert L.ncm_linear_bf16(None, None, None, None, None, 1, 8, 1, 0) == -1
    assert L.ncm_rvq_prepare(None, None, 1, 1, 64, None) == -1
    assert L.ncm_rvq_encode(None, None, 1, 1, 64, 1, None, None, None, 1, None, None, None,
                            None, None) == -1
    assert L.ncm_destroy(None) == -1


def test_dropin_length_mismatch_rejected_before_device_use(ncm):
    # root.zig:107-110 asserts; the drop-in returns NCM_E_LENGTH instead.
    L = ncm.lib()
    x = np.zeros(6, np.float32)
    w = np.zeros(6, np.float32)
    y = np.zeros(4, np.float32)
    p = lambda a: C.c_void_p(a.ctypes.data)
    assert L.ncm_matmul_bf16(p(x), 6, p(w), 6, p(y), 4, 2, 3, 3) == -3
    assert L.ncm_matmul_bf16(p(x), 5, p(w), 6, p(y), 4, 2, 3, 2) == -3
    b = np.zeros(3, np.float32)
    assert L.ncm_matmul_bf16_bias(p(x), 6, p(w), 6, p(b), 3, p(y), 4, 2, 3, 2) == -3


def test_python_mirror_raises(ncm):
    import pytest
    from ncmorph_amd import kernels
    from ncmorph_amd._lib import NcmError

    with pytest.raises(NcmError):
        kernels.matmul_bf16(np.zeros(6, np.float32), np.zeros(6, np.float32),
                            np.zeros(5, np.float32), 2, 3, 2)

"""CPU-side checks of the C ABI: the library loads, exports exactly what
include/mri_qmatmul.h declares, and validates shapes (TensorError kinds and
check order) before touching a device."""
import ctypes as C
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = {"mri_qmatmul": os.path.join(ROOT, "include", "mri_qmatmul.h"),
           "mri_llama": os.path.join(ROOT, "include", "mri_llama.h")}


def declared_functions(module="mri_qmatmul"):
    src = open(HEADERS[module]).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(mri_[a-z0-9_]+)\s*\(", src)))


def test_every_header_has_a_binding():
    assert sorted(HEADERS) == sorted(f[:-2] for f in os.listdir(os.path.join(ROOT, "include"))
                                     if f.endswith(".h"))


@pytest.mark.parametrize("module", sorted(HEADERS))
def test_header_and_binding_agree(module):
    import importlib
    assert sorted(importlib.import_module(module).EXPORTED) == declared_functions(module)


@pytest.mark.parametrize("module", sorted(HEADERS))
def test_library_exports_every_declared_symbol(module):
    import mri_qmatmul
    lib = mri_qmatmul.lib()
    for name in declared_functions(module):
        assert hasattr(lib, name), name
    assert b"gfx950" in lib.mri_version()


def test_no_cpu_fallback_symbols():
    """The product library must not contain the oracle."""
    import mri_qmatmul
    lib = C.CDLL(mri_qmatmul.LIB_PATH)
    for name in ("orc_matmul_int8", "orc_quantize_symmetric"):
        assert not hasattr(lib, name)


def _status(rc):
    import mri_qmatmul
    return mri_qmatmul.STATUS.get(rc, rc)


def test_shape_errors_before_device_work():
    import mri_qmatmul as M
    lib = M.lib()
    h = C.c_void_p()
    # q8_direct.rs:80-107 (k_in % 32, then the byte count)
    assert _status(lib.mri_q8_0_matrix_from_raw_bytes(None, 34, 1, 31, C.byref(h))) \
        == "InvalidShape"
    buf = np.zeros(33, np.uint8)
    assert _status(lib.mri_q8_0_matrix_from_raw_bytes(buf.ctypes.data_as(C.c_void_p), 33,
                                                      1, 32, C.byref(h))) == "InvalidShape"
    assert b"data.len()=33" in lib.mri_last_error()
    # q4_0.rs:94-140 check order
    def q4(dims, n_out, k, wlen):
        arr = (C.c_size_t * len(dims))(*dims)
        return _status(lib.mri_matmul_q4_0_dequant(None, arr, len(dims), None, wlen,
                                                   n_out, k, None, None))
    assert q4([2, 4, 8], 1, 32, 18) == "InvalidShape"
    assert q4([1, 32], 1, 64, 18) == "ShapeMismatch"     # before the K%32 check
    assert q4([1, 33], 1, 33, 18) == "InvalidShape"
    assert q4([1, 32], 1, 32, 20) == "InvalidShape"
    # per_channel.rs:99-105 (a panic in the reference)
    assert _status(lib.mri_quantize_per_channel(None, 5, 2, 3, None, None, None)) \
        == "InvalidShape"
    # null handle
    assert _status(lib.mri_matmul_int8(None, 0, C.c_float(1.0), None, 0, None, None,
                                       None)) == "InvalidArgument"


def test_w4a8_argument_errors_before_device_work():
    """The W4A8 extension's handle checks: nibble order, K % 32, byte count;
    a null handle."""
    import mri_qmatmul as M
    lib = M.lib()
    h = C.c_void_p()
    buf = np.zeros(36, np.uint8)
    p = buf.ctypes.data_as(C.c_void_p)
    assert _status(lib.mri_q4_0_matrix_from_raw_device(p, 18, 1, 32, 2, None, C.byref(h))) \
        == "InvalidArgument"
    assert _status(lib.mri_q4_0_matrix_from_raw_device(p, 18, 1, 31, 0, None, C.byref(h))) \
        == "InvalidShape"
    assert _status(lib.mri_q4_0_matrix_from_raw_device(p, 17, 1, 32, 1, None, C.byref(h))) \
        == "InvalidShape"
    dims = (C.c_size_t * 2)(1, 32)
    assert _status(lib.mri_matmul_q4_0_w4a8(None, dims, 2, None, None, None, None, None)) \
        == "InvalidArgument"


@pytest.mark.skipif(os.path.exists("/dev/kfd") and os.access("/dev/kfd", os.R_OK),
                    reason="a GPU is visible")
def test_fails_loudly_without_gpu():
    import mri_qmatmul as M
    h = C.c_void_p()
    raw = np.zeros(34, np.uint8)
    rc = M.lib().mri_q8_0_matrix_from_raw_bytes(raw.ctypes.data_as(C.c_void_p), 34, 1,
                                                32, C.byref(h))
    assert rc != 0 and _status(rc) in ("HipError", "Unsupported")


def test_llama_argument_errors_before_device_work():
    """Shape errors of the model API (forward_int8.rs / config checks) come
    before any device call."""
    import mri_llama as L
    lib = L.lib()
    h = C.c_void_p()
    emb = np.zeros(4, np.float32)
    bad = L.Config(dim=6, n_heads=4, n_kv_heads=2, ffn_dim=8, vocab=2, max_seq=4, eps=1e-6,
                   rope_base=1e4, n_layers=1)  # dim % n_heads != 0
    rc = lib.mri_llama_create(C.byref(bad), emb.ctypes.data_as(C.c_void_p),
                              emb.ctypes.data_as(C.c_void_p), L.WeightRef(0, None, 0, 0),
                              C.byref(h))
    assert _status(rc) == "InvalidShape"
    odd = L.Config(dim=96, n_heads=2, n_kv_heads=2, ffn_dim=8, vocab=2, max_seq=4, eps=1e-6,
                   rope_base=1e4, n_layers=1)  # head_dim 48: no attention kernel for it
    rc = lib.mri_llama_create(C.byref(odd), emb.ctypes.data_as(C.c_void_p),
                              emb.ctypes.data_as(C.c_void_p), L.WeightRef(0, None, 0, 0),
                              C.byref(h))
    assert _status(rc) == "Unsupported"
    assert _status(lib.mri_llama_forward_cached(None, None, 0, 0, None, None, None)) \
        == "InvalidArgument"

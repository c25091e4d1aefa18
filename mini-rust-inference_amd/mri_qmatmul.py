"""ctypes binding of libmri_qmatmul.so (include/mri_qmatmul.h).

Host-side plumbing for tests and benchmarks: device buffers are torch CUDA
(HIP) tensors, passed to the C ABI as raw pointers together with torch's
current stream.  Every call goes through the HIP kernels; there is no CPU
fallback — a missing library raises ``ImportError`` at load time.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmri_qmatmul.so")

OK = 0
STATUS = {1: "InvalidShape", 2: "ShapeMismatch", 3: "InvalidArgument",
          4: "HipError", 5: "Unsupported"}


class MriError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{STATUS.get(code, code)}: {msg}")
        self.code = code
        self.kind = STATUS.get(code, str(code))


P = C.c_void_p
SZ = C.c_size_t
ST = C.c_int

_SIGS = {
    "mri_last_error": ([], C.c_char_p),
    "mri_version": ([], C.c_char_p),
    "mri_qmatrix_create": ([P, P, SZ, SZ, C.POINTER(P)], ST),
    "mri_qmatrix_create_device": ([P, P, SZ, SZ, P, C.POINTER(P)], ST),
    "mri_qmatrix_read": ([P, P, P], ST),
    "mri_qmatrix_n_out": ([P], SZ),
    "mri_qmatrix_k_in": ([P], SZ),
    "mri_qmatrix_device_bytes": ([P], SZ),
    "mri_qmatrix_destroy": ([P], None),
    "mri_q8_0_matrix_from_raw_bytes": ([P, SZ, SZ, SZ, C.POINTER(P)], ST),
    "mri_q8_0_matrix_from_raw_device": ([P, SZ, SZ, SZ, P, C.POINTER(P)], ST),
    "mri_q8_0_matrix_read_raw": ([P, P, SZ], ST),
    "mri_q8_0_matrix_n_out": ([P], SZ),
    "mri_q8_0_matrix_k_in": ([P], SZ),
    "mri_q8_0_matrix_device_bytes": ([P], SZ),
    "mri_q8_0_matrix_destroy": ([P], None),
    "mri_quantize_symmetric": ([P, SZ, P, P, P], ST),
    "mri_quantize_symmetric_rows": ([P, SZ, SZ, P, P, P], ST),
    "mri_quantize_per_channel": ([P, SZ, SZ, SZ, P, P, P], ST),
    "mri_dot_i8": ([P, P, SZ, P, P], ST),
    "mri_matmul_int8": ([P, SZ, C.c_float, P, SZ, P, P, P], ST),
    "mri_matmul_int8_rows": ([P, SZ, P, P, SZ, P, P, P], ST),
    "mri_matmul_int8_from_f32": ([P, P, SZ, P, P, P, P, P, P], ST),
    "mri_matmul_q8_0_direct": ([P, P, SZ, P, P, P, P, P], ST),
    "mri_matmul_q8_0_direct_exact": ([P, P, SZ, P, P, P, P, P], ST),
    "mri_matmul_q8_0_direct_noalloc": ([P, P, SZ, P, P, P, P, P], ST),
    "mri_matmul_q4_0_dequant_matrix": ([P, P, SZ, P, P, P], ST),
    "mri_matmul_q4_0_dequant": ([P, P, SZ, P, SZ, SZ, SZ, P, P], ST),
    "mri_q4_0_matrix_from_raw_bytes": ([P, SZ, SZ, SZ, C.c_int, C.POINTER(P)], ST),
    "mri_q4_0_matrix_from_raw_device": ([P, SZ, SZ, SZ, C.c_int, P, C.POINTER(P)], ST),
    "mri_q4_0_matrix_n_out": ([P], SZ),
    "mri_q4_0_matrix_k_in": ([P], SZ),
    "mri_q4_0_matrix_device_bytes": ([P], SZ),
    "mri_q4_0_matrix_destroy": ([P], None),
    "mri_matmul_q4_0_w4a8": ([P, P, SZ, P, P, P, P, P], ST),
    "mri_matmul_q4_0_dequant_ordered": ([P, P, SZ, P, SZ, SZ, SZ, C.c_int, P, P], ST),
    "mri_synchronize": ([P], ST),
    "mri_hbm_read": ([P, SZ, P, P], ST),
    "mri_mfma_i8_peak": ([P, C.c_int, P, C.POINTER(C.c_int), P], ST),
}

# Every symbol the header declares (checked by the CPU test suite).
EXPORTED = tuple(_SIGS)

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is not built; run __graft_entry__.build() first")
        # torch ships its own libamdhip64.so.7 under the same soname as the
        # system one the library links against; whichever is loaded first
        # serves the whole process.  Load torch's first so that torch, whose
        # tensors carry the device buffers, keeps the runtime it was built for.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        l = C.CDLL(LIB_PATH)
        for name, (args, res) in _SIGS.items():
            f = getattr(l, name)
            f.argtypes = args
            f.restype = res
        _lib = l
    return _lib


def check(rc: int) -> None:
    if rc != OK:
        raise MriError(rc, lib().mri_last_error().decode())


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream(stream=None):
    if stream is not None:
        return C.c_void_p(stream)
    import torch
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _dims(shape):
    arr = (C.c_size_t * max(len(shape), 1))(*shape)
    return arr, len(shape)


# ---------------------------------------------------------------------------
# weight handles
# ---------------------------------------------------------------------------
class QMatrix:
    """Device-resident QuantizedMatrix (per_channel.rs:31-40)."""

    def __init__(self, handle, n_out, k_in):
        self.h = handle
        self.n_out = n_out
        self.k_in = k_in

    @classmethod
    def from_host(cls, data, scales):
        """data: numpy int8 [N,K]; scales: numpy float32 [N]."""
        import numpy as np
        data = np.ascontiguousarray(data, dtype=np.int8)
        scales = np.ascontiguousarray(scales, dtype=np.float32)
        n, k = data.shape
        h = C.c_void_p()
        check(lib().mri_qmatrix_create(data.ctypes.data_as(P), scales.ctypes.data_as(P),
                                       n, k, C.byref(h)))
        return cls(h, n, k)

    @classmethod
    def from_device(cls, data, scales, stream=None):
        """data: torch int8 [N,K] on the GPU; scales: torch float32 [N]."""
        n, k = data.shape
        h = C.c_void_p()
        check(lib().mri_qmatrix_create_device(_ptr(data), _ptr(scales), n, k,
                                              _stream(stream), C.byref(h)))
        return cls(h, n, k)

    def read(self):
        import numpy as np
        d = np.empty((self.n_out, self.k_in), np.int8)
        s = np.empty(self.n_out, np.float32)
        check(lib().mri_qmatrix_read(self.h, d.ctypes.data_as(P), s.ctypes.data_as(P)))
        return d, s

    @property
    def device_bytes(self):
        return lib().mri_qmatrix_device_bytes(self.h)

    def close(self):
        if self.h:
            lib().mri_qmatrix_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Q8Matrix:
    """Device-resident Q8_0WeightMatrix (q8_direct.rs:60-69)."""

    def __init__(self, handle, n_out, k_in):
        self.h = handle
        self.n_out = n_out
        self.k_in = k_in

    @classmethod
    def from_raw_bytes(cls, raw, n_out, k_in):
        import numpy as np
        raw = np.ascontiguousarray(raw, dtype=np.uint8)
        h = C.c_void_p()
        check(lib().mri_q8_0_matrix_from_raw_bytes(raw.ctypes.data_as(P), raw.size,
                                                   n_out, k_in, C.byref(h)))
        return cls(h, n_out, k_in)

    @classmethod
    def from_raw_device(cls, raw, n_out, k_in, stream=None):
        h = C.c_void_p()
        check(lib().mri_q8_0_matrix_from_raw_device(_ptr(raw), raw.numel(), n_out,
                                                    k_in, _stream(stream), C.byref(h)))
        return cls(h, n_out, k_in)

    def read_raw(self):
        import numpy as np
        n = self.n_out * (self.k_in // 32) * 34
        out = np.empty(n, np.uint8)
        check(lib().mri_q8_0_matrix_read_raw(self.h, out.ctypes.data_as(P), n))
        return out

    @property
    def device_bytes(self):
        return lib().mri_q8_0_matrix_device_bytes(self.h)

    def close(self):
        if self.h:
            lib().mri_q8_0_matrix_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


Q4_ORDER_INTERLEAVED, Q4_ORDER_GGML = 0, 1


class Q4Matrix:
    """Q4_0 weights for the W4A8 extension (matmul_q4_0_w4a8), from raw
    18-byte blocks in the reference's interleaved nibble order or in
    upstream GGML's (Q4_ORDER_GGML)."""

    def __init__(self, handle, n_out, k_in):
        self.h = handle
        self.n_out = n_out
        self.k_in = k_in

    @classmethod
    def from_raw_bytes(cls, raw, n_out, k_in, order=Q4_ORDER_INTERLEAVED):
        import numpy as np
        raw = np.ascontiguousarray(raw, dtype=np.uint8)
        h = C.c_void_p()
        check(lib().mri_q4_0_matrix_from_raw_bytes(raw.ctypes.data_as(P), raw.size, n_out,
                                                   k_in, order, C.byref(h)))
        return cls(h, n_out, k_in)

    @classmethod
    def from_raw_device(cls, raw, n_out, k_in, order=Q4_ORDER_INTERLEAVED, stream=None):
        h = C.c_void_p()
        check(lib().mri_q4_0_matrix_from_raw_device(_ptr(raw), raw.numel(), n_out, k_in,
                                                    order, _stream(stream), C.byref(h)))
        return cls(h, n_out, k_in)

    @property
    def device_bytes(self):
        return lib().mri_q4_0_matrix_device_bytes(self.h)

    def close(self):
        if self.h:
            lib().mri_q4_0_matrix_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---------------------------------------------------------------------------
# entry points (torch device tensors in/out)
# ---------------------------------------------------------------------------
def quantize_symmetric(x, q, scale, stream=None):
    check(lib().mri_quantize_symmetric(_ptr(x), x.numel(), _ptr(q), _ptr(scale),
                                       _stream(stream)))


def quantize_symmetric_rows(x, q, scales, stream=None):
    m, k = x.shape
    check(lib().mri_quantize_symmetric_rows(_ptr(x), m, k, _ptr(q), _ptr(scales),
                                            _stream(stream)))


def quantize_per_channel(w, n_out, k_in, data, scales, stream=None):
    check(lib().mri_quantize_per_channel(_ptr(w), w.numel(), n_out, k_in, _ptr(data),
                                         _ptr(scales), _stream(stream)))


def dot_i8(a, b, out, stream=None):
    check(lib().mri_dot_i8(_ptr(a), _ptr(b), a.numel(), _ptr(out), _stream(stream)))


def matmul_int8(act_q, act_scale, w: QMatrix, m, out, acc_out=None, stream=None,
                act_q_len=None):
    n = act_q.numel() if act_q_len is None else act_q_len
    check(lib().mri_matmul_int8(_ptr(act_q), n, float(act_scale), w.h, m, _ptr(out),
                                _ptr(acc_out), _stream(stream)))


def matmul_int8_rows(act_q, act_scales, w: QMatrix, m, out, acc_out=None, stream=None):
    check(lib().mri_matmul_int8_rows(_ptr(act_q), act_q.numel(), _ptr(act_scales), w.h,
                                     m, _ptr(out), _ptr(acc_out), _stream(stream)))


def matmul_int8_from_f32(x, w: QMatrix, out, act_q_out=None, act_scale_out=None,
                         acc_out=None, stream=None, shape=None):
    dims, nd = _dims(tuple(x.shape) if shape is None else shape)
    check(lib().mri_matmul_int8_from_f32(_ptr(x), dims, nd, w.h, _ptr(out),
                                         _ptr(act_q_out), _ptr(act_scale_out),
                                         _ptr(acc_out), _stream(stream)))


def matmul_q8_0_direct(x, w: Q8Matrix, out, block_dots_out=None, act_scales_out=None,
                       stream=None, shape=None):
    dims, nd = _dims(tuple(x.shape) if shape is None else shape)
    check(lib().mri_matmul_q8_0_direct(_ptr(x), dims, nd, w.h, _ptr(out),
                                       _ptr(block_dots_out), _ptr(act_scales_out),
                                       _stream(stream)))


def matmul_q8_0_direct_exact(x, w: Q8Matrix, out, block_dots_out=None, act_scales_out=None,
                             stream=None, shape=None):
    """matmul_q8_0_direct with the reference's left-to-right block order kept
    at every row count: f32 outputs bit-identical to q8_direct.rs:269-282."""
    dims, nd = _dims(tuple(x.shape) if shape is None else shape)
    check(lib().mri_matmul_q8_0_direct_exact(_ptr(x), dims, nd, w.h, _ptr(out),
                                             _ptr(block_dots_out), _ptr(act_scales_out),
                                             _stream(stream)))


def matmul_q8_0_direct_noalloc(x, w: Q8Matrix, out, block_dots_out=None, act_scales_out=None,
                               stream=None, shape=None):
    """matmul_q8_0_direct staged in the library's fixed per-device array
    (NOALLOC_SCRATCH_BYTES): no device allocation; overlapping calls on one
    device race."""
    dims, nd = _dims(tuple(x.shape) if shape is None else shape)
    check(lib().mri_matmul_q8_0_direct_noalloc(_ptr(x), dims, nd, w.h, _ptr(out),
                                               _ptr(block_dots_out), _ptr(act_scales_out),
                                               _stream(stream)))


NOALLOC_SCRATCH_BYTES = 4 << 20  # MRI_NOALLOC_SCRATCH_BYTES


def matmul_q4_0_dequant_matrix(x, w: "Q4Matrix", out, stream=None, shape=None):
    """matmul_q4_0_dequant (W4A32) on a device-resident Q4_0 handle."""
    dims, nd = _dims(tuple(x.shape) if shape is None else shape)
    check(lib().mri_matmul_q4_0_dequant_matrix(_ptr(x), dims, nd, w.h, _ptr(out),
                                               _stream(stream)))


def matmul_q4_0_w4a8(x, w: Q4Matrix, out, block_dots_out=None, act_scales_out=None,
                     stream=None, shape=None):
    dims, nd = _dims(tuple(x.shape) if shape is None else shape)
    check(lib().mri_matmul_q4_0_w4a8(_ptr(x), dims, nd, w.h, _ptr(out), _ptr(block_dots_out),
                                     _ptr(act_scales_out), _stream(stream)))


def bind_matmul_q8_0_direct(x, w: Q8Matrix, out, stream=None):
    """matmul_q8_0_direct(x, w, out) with its C arguments converted once:
    returns a callable that issues the call again on the stream current
    now (for loops whose Python cost per call should stay small)."""
    dims, nd = _dims(tuple(x.shape))
    f = lib().mri_matmul_q8_0_direct
    args = (_ptr(x), dims, nd, w.h, _ptr(out), None, None, _stream(stream))

    def call():
        rc = f(*args)
        if rc != OK:
            check(rc)
    return call


def bind_matmul_int8_from_f32(x, w: QMatrix, out, stream=None):
    """matmul_int8_from_f32(x, w, out) with its C arguments converted once
    (see bind_matmul_q8_0_direct)."""
    dims, nd = _dims(tuple(x.shape))
    f = lib().mri_matmul_int8_from_f32
    args = (_ptr(x), dims, nd, w.h, _ptr(out), None, None, None, _stream(stream))

    def call():
        rc = f(*args)
        if rc != OK:
            check(rc)
    return call


def matmul_q4_0_dequant_ordered(x, weight_q4, n_out, k, order, out, stream=None):
    """W4A32 on raw Q4_0 blocks in the given nibble order (Q4_ORDER_*)."""
    dims, nd = _dims(tuple(x.shape))
    check(lib().mri_matmul_q4_0_dequant_ordered(_ptr(x), dims, nd, _ptr(weight_q4),
                                                weight_q4.numel(), n_out, k, order, _ptr(out),
                                                _stream(stream)))


def matmul_q4_0_dequant(x, weight_q4, n_out, k, out, stream=None, shape=None,
                        weight_len=None):
    dims, nd = _dims(tuple(x.shape) if shape is None else shape)
    wl = weight_q4.numel() if weight_len is None else weight_len
    check(lib().mri_matmul_q4_0_dequant(_ptr(x), dims, nd, _ptr(weight_q4), wl, n_out,
                                        k, _ptr(out), _stream(stream)))


def synchronize(stream=None):
    check(lib().mri_synchronize(_stream(stream)))


def version() -> str:
    return lib().mri_version().decode()


def hbm_read(buf, nbytes=None, stream=None):
    """One kernel that reads nbytes of the device tensor buf (diagnostic:
    the one-kernel HBM read ceiling at that size)."""
    n = buf.numel() * buf.element_size() if nbytes is None else nbytes
    check(lib().mri_hbm_read(C.c_void_p(buf.data_ptr()), n, None, _stream(stream)))


def mfma_i8_peak(src, iters, stream=None):
    """Enqueues the int8 MFMA ceiling kernel on operands src (torch int8,
    >= 32 KiB on the device); returns (int ops per launch, CUs)."""
    n = C.c_int(0)
    check(lib().mri_mfma_i8_peak(C.c_void_p(src.data_ptr()), int(iters), None, C.byref(n),
                                 _stream(stream)))
    return 2 * 32768 * 8 * int(iters) * 8 * n.value, n.value

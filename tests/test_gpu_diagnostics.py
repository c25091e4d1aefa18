"""The two measurement kernels the benchmark reports beside the hot path
(mri_hbm_read, mri_mfma_i8_peak in include/mri_qmatmul.h): they run at every
size class, including sizes that are not a multiple of 16 (the read covers
the whole 16-byte units, bytes rounded down), without error, and leave the
sink untouched for ordinary data.  That the read stays inside its buffer is
a property of its indexing (k_hbm_read reads unit i only for i < bytes / 16),
not something this test can observe."""
import ctypes as C

import numpy as np
import pytest

from gpu_util import empty, host, torch

pytestmark = pytest.mark.gpu


def mri():
    import mri_qmatmul
    return mri_qmatmul


@pytest.mark.parametrize("nbytes", [16, 4096, 4096 + 16, 65536 + 48, 47967232, 15, 4096 + 7,
                                    100003])
def test_hbm_read_sizes(nbytes):
    t = torch()
    buf = t.ones(nbytes, dtype=t.uint8, device="cuda")
    sink = t.full((1,), 7, dtype=t.int32, device="cuda")
    M = mri()
    M.check(M.lib().mri_hbm_read(C.c_void_p(buf.data_ptr()), nbytes,
                                 C.c_void_p(sink.data_ptr()), None))
    t.cuda.synchronize()
    assert int(host(sink)[0]) == 7


def test_mfma_i8_peak_runs():
    t = torch()
    src = t.randint(-127, 128, (32768,), dtype=t.int8, device="cuda")
    ops, cus = mri().mfma_i8_peak(src, 4)
    t.cuda.synchronize()
    assert cus > 0 and ops == 2 * 32768 * 8 * 4 * 8 * cus

"""The no-allocation variant of matmul_q8_0_direct
(mri_matmul_q8_0_direct_noalloc, include/mri_qmatmul.h) against the
allocating entry point, through the C ABI: the same kernels, so outputs,
block dots and activation scales must be bit-identical (call for call, with
and without the optional outputs), on consecutive calls
whose second input is smaller than the first (the fixed staging array keeps
the first call's contents), at M = 1 (fused quantization, no staging) and at
sizes past the staging limit (a clear error, nothing launched)."""
import numpy as np
import pytest

from gpu_util import F32, bits, dev, empty, host, synth_q8_0, torch

pytestmark = pytest.mark.gpu


def mri():
    import mri_qmatmul
    return mri_qmatmul


def run_both(w, x, n, k):
    t = torch()
    m = x.shape[0]
    outs = []
    for f in (mri().matmul_q8_0_direct, mri().matmul_q8_0_direct_noalloc):
        out = empty((m, n), t.float32)
        bd = empty((m, n, k // 32), t.int32)
        sa = empty(m, t.float32)
        f(dev(x), w, out, bd, sa)
        out2 = empty((m, n), t.float32)  # without the optional outputs
        f(dev(x), w, out2)
        outs.append((host(out), host(bd), host(sa), host(out2)))
    (o0, b0, s0, p0), (o1, b1, s1, p1) = outs
    assert np.array_equal(bits(o0), bits(o1))
    assert np.array_equal(b0, b1)
    assert np.array_equal(bits(s0), bits(s1))
    assert np.array_equal(bits(p0), bits(p1))
    if not (m >= 256 and n >= 8192):  # else the call without block dots runs the LDS-tiled kernel
        assert np.array_equal(bits(p0), bits(o0))


@pytest.mark.parametrize("n,k,rows", [(1000, 4096, (64, 3)), (300, 11008, (40, 2)),
                                      (96, 256, (512, 5, 1))])
def test_noalloc_matches_allocating_entry_point(n, k, rows):
    rng = np.random.default_rng(n + k)
    w = mri().Q8Matrix.from_raw_bytes(synth_q8_0(rng, n, k, with_min=True), n, k)
    for m in rows:
        run_both(w, rng.standard_normal((m, k)).astype(F32), n, k)


def test_noalloc_rejects_inputs_past_its_staging():
    t = torch()
    n, k = 32, 4096
    rng = np.random.default_rng(9)
    w = mri().Q8Matrix.from_raw_bytes(synth_q8_0(rng, n, k), n, k)
    m = mri().NOALLOC_SCRATCH_BYTES // k + 1   # m * 4096 + 4 * m > the limit
    x = empty((m, k), t.float32)
    out = empty((m, n), t.float32)
    with pytest.raises(mri().MriError) as e:
        mri().matmul_q8_0_direct_noalloc(x, w, out)
    assert e.value.kind == "Unsupported"
    assert "no-allocation" in str(e.value)

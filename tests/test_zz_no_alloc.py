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

from gpu_util import F32, bits, dev, empty, host, q8_gemm_range, synth_q8_0, torch

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
    if not q8_gemm_range(m, n):  # else the call without block dots runs the LDS-tiled kernel
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


def test_noalloc_allocates_nothing():
    """On a stream the library has not seen, the allocating entry point grows
    its per-stream staging (a hipMalloc of about 4 MiB here, which the
    device's free-memory readout shows), while the no-allocation entry point
    leaves the free device memory exactly as it was.  The fixed array itself
    (MRI_NOALLOC_SCRATCH_BYTES, a file-scope device variable) is placed in
    device memory by the HIP runtime when the first call looks up its
    address, once per device and process; a first call before the
    measurement makes sure of that.  A stream's first kernel also makes the
    runtime set up per-queue device memory (kernel arguments), so both
    streams run a small torch kernel before the readout starts."""
    t = torch()
    n, k, m = 64, 4096, 900          # staging m * 4096 + 4 * m bytes: 3.5 MiB
    rng = np.random.default_rng(17)
    w = mri().Q8Matrix.from_raw_bytes(synth_q8_0(rng, n, k), n, k)
    x = dev(rng.standard_normal((m, k)).astype(F32))
    outs = [empty((m, n), t.float32) for _ in range(2)]
    mri().matmul_q8_0_direct_noalloc(x[:2], w, outs[1][:2])  # the array is in place
    s_alloc, s_fixed = t.cuda.Stream(), t.cuda.Stream()
    for st in (s_alloc, s_fixed):
        with t.cuda.stream(st):
            outs[0].zero_()
    t.cuda.synchronize()
    free0 = t.cuda.mem_get_info()[0]
    with t.cuda.stream(s_alloc):
        mri().matmul_q8_0_direct(x, w, outs[0])
    t.cuda.synchronize()
    free1 = t.cuda.mem_get_info()[0]
    assert free0 - free1 >= 3 << 20, (free0, free1)  # the readout sees a staging allocation
    with t.cuda.stream(s_fixed):
        mri().matmul_q8_0_direct_noalloc(x, w, outs[1])
        mri().matmul_q8_0_direct_noalloc(x[:5], w, outs[1][:5])
    t.cuda.synchronize()
    free2 = t.cuda.mem_get_info()[0]
    assert free2 == free1, (free1, free2)
    o0, o1 = host(outs[0]), host(outs[1])
    assert np.array_equal(bits(o0), bits(o1))  # rows 0-4 recomputed from the same rows

"""GPU parity: the HIP kernels through the C ABI vs the CPU oracle.

Integer results (quantized activations, int32 accumulators, block dots) and
the per-channel INT8 f32 outputs must be bit-identical.  Q8_0 f32 outputs
are within 1e-5 * max(|ref|, sum_b |t_b|) of the reference's left-to-right
block sum where the kernel reorders it (the decode GEMV, M <= 4, adds
per-wave partial sums; the LDS-tiled prefill GEMM, M >= 128 and M * N > 2^20
without block dots, folds with FMAs) and bit-identical elsewhere (the
skinny kernel, and the block-ordered entry point at every M).
Q4_0 (W4A32) outputs are within 1e-5 * max(|ref|, sum_k |x_k w_k|).
"""
import sys

import numpy as np
import pytest

import closed_form as CF
import oracle_lib as O
from gpu_util import (q8_gemm_range, F32, assert_bits_equal, assert_q8_close, bits, dev, empty, host,
                      q8_oracle_sliced, q8_terms_abs_sum, synth_int8_weights, synth_q4_0,
                      synth_q8_0, torch)

pytestmark = pytest.mark.gpu


def mri():
    import mri_qmatmul
    return mri_qmatmul


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


# ---- quantizers ----------------------------------------------------------------

@pytest.mark.parametrize("n,scale,seed", [(4096, 1.0, 0), (1, 3.0, 1), (4097, 1e-3, 2),
                                          (11008 * 3 + 5, 50.0, 3)])
def test_quantize_symmetric(n, scale, seed):
    say(f"quantize_symmetric n={n}")
    t = torch()
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(n) * scale).astype(F32)
    q, s = O.quantize_symmetric(x)
    xd = dev(x)
    qd = empty(n, t.int8)
    sd = empty(1, t.float32)
    mri().quantize_symmetric(xd, qd, sd)
    assert host(sd)[0] == s
    assert np.array_equal(host(qd), q)


def test_quantize_ties_and_specials():
    t = torch()
    x = np.array([127.0, 0.5, -0.5, 1.5, -1.5, 2.5, -62.5, 126.5, np.nan, -0.0], F32)
    q, s = O.quantize_symmetric(x)
    qd, sd = empty(x.size, t.int8), empty(1, t.float32)
    mri().quantize_symmetric(dev(x), qd, sd)
    assert host(sd)[0] == s and np.array_equal(host(qd), q)
    z = np.zeros(100, F32)                               # all-zero -> scale 1
    qd, sd = empty(100, t.int8), empty(1, t.float32)
    mri().quantize_symmetric(dev(z), qd, sd)
    assert host(sd)[0] == 1.0 and not host(qd).any()


@pytest.mark.parametrize("m,k", [(9, 333), (5, 4096), (3, 11008), (6, 64)])
def test_quantize_rows_and_per_channel(m, k):
    # k % 4 != 0 takes the element-wise path, the others the float4 path
    # (k = 11008: unrolled loop plus remainder)
    t = torch()
    rng = np.random.default_rng(7 + k)
    x = rng.standard_normal((m, k)).astype(F32)
    x[m // 2] = 0.0
    x[0, k // 3] = np.nan
    q0, s0 = CF.quantize_rows(x)
    qd, sd = empty((m, k), t.int8), empty(m, t.float32)
    mri().quantize_symmetric_rows(dev(x), qd, sd)
    assert np.array_equal(host(qd), q0) and np.array_equal(bits(host(sd)), bits(s0))
    w = (rng.standard_normal((37, 96)) * 0.02).astype(F32)
    d0, ws0 = O.quantize_per_channel(w, 37, 96)
    dd, sd = empty((37, 96), t.int8), empty(37, t.float32)
    mri().quantize_per_channel(dev(w), 37, 96, dd, sd)
    assert np.array_equal(host(dd), d0) and np.array_equal(bits(host(sd)), bits(ws0))


def test_dot_i8_kats():  # int8_avx2.rs:219-297 through the GPU
    t = torch()
    cases = [([1, 2, 3], [4, 5, 6], 32), ([127] * 64, [1] * 64, 8128),
             ([1, -1] * 32, [2] * 64, 0), ([-3] * 32, [-5] * 32, 480),
             ([127] * 4096, [1] * 4096, 127 * 4096)]
    for a, b, want in cases:
        o = empty(1, t.int32)
        mri().dot_i8(dev(np.array(a, np.int8)), dev(np.array(b, np.int8)), o)
        assert host(o)[0] == want


# ---- weights round trip ----------------------------------------------------------

@pytest.mark.parametrize("n,k", [(1, 32), (17, 96), (64, 4096), (33, 100)])
def test_qmatrix_roundtrip(n, k):
    rng = np.random.default_rng(n * 1000 + k)
    d = rng.integers(-127, 128, (n, k)).astype(np.int8)
    s = rng.uniform(1e-4, 1e-3, n).astype(F32)
    w = mri().QMatrix.from_host(d, s)
    d2, s2 = w.read()
    assert np.array_equal(d, d2) and np.array_equal(s, s2)


@pytest.mark.parametrize("n,k", [(1, 32), (17, 96), (64, 4096), (3, 11008)])
def test_q8_matrix_roundtrip(n, k):
    raw = synth_q8_0(np.random.default_rng(k), n, k, with_min=True)
    w = mri().Q8Matrix.from_raw_bytes(raw, n, k)
    assert np.array_equal(w.read_raw(), raw)


# ---- per-channel INT8 ------------------------------------------------------------

INT8_SHAPES = [
    # (m, n, k)
    (1, 16, 64), (1, 11008 // 8, 4096), (1, 37, 96), (2, 50, 128), (3, 16, 4096),
    (1, 16400, 8192), (1, 300, 11008), (2, 4096, 4096),
    (4, 64, 1024), (5, 48, 320), (16, 64, 4096), (17, 33, 64), (32, 96, 4096),
    (33, 40, 256), (64, 128, 512), (128, 64, 1024),
]


@pytest.mark.parametrize("m,n,k", INT8_SHAPES)
def test_matmul_int8_bit_exact(m, n, k):
    say(f"matmul_int8 m={m} n={n} k={k}")
    t = torch()
    rng = np.random.default_rng(m * 7 + n * 13 + k)
    wq, ws = synth_int8_weights(rng, n, k)
    aq = rng.integers(-127, 128, (m, k)).astype(np.int8)
    sa = F32(0.0173)
    out0, acc0 = O.matmul_int8(aq, sa, wq, ws, m, want_acc=True)
    assert np.array_equal(acc0.astype(np.int64), CF.int_matmul(aq, wq))
    w = mri().QMatrix.from_host(wq, ws)
    out = empty((m, n), t.float32)
    acc = empty((m, n), t.int32)
    mri().matmul_int8(dev(aq), sa, w, m, out, acc)
    assert np.array_equal(host(acc), acc0)
    assert_bits_equal(host(out), out0, "matmul_int8 out")


@pytest.mark.parametrize("m,n,k", [(512, 11008, 4096), (300, 200, 1024), (2048, 512, 4096),
                                   (64, 4096, 11008), (128, 4096, 4096), (512, 4096, 11008),
                                   (2048, 8192, 4096), (128, 11008, 4096), (512, 4096, 4096),
                                   (2048, 4096, 4096), (2048, 11008, 4096),
                                   # K split over partial tiles: 128 x 64 tiles 4-way
                                   # (100 x 1000), 128 x 128 tiles 2-way (200 x 300) and
                                   # 4-way (129 x 2000); 128 x 64 2-way at 256 x 4096,
                                   # 128 x 128 whole at 192 x 11008
                                   (100, 1000, 4096), (200, 300, 2048), (129, 2000, 4096),
                                   (256, 4096, 4096), (192, 11008, 4096),
                                   # the larger plans: 128 x 192 whole tiles (512 and
                                   # 1536 x 11008), 256 x 128 stream-K (768 x 11008),
                                   # 256 x 128 whole (1280 x 11008), 256 x 256 stream-K
                                   # in whole passes (4096 x 4096)
                                   (768, 11008, 4096), (1536, 11008, 4096), (1280, 11008, 4096),
                                   (4096, 4096, 4096),
                                   # K a whole number of 64 but not of 128 bytes: the
                                   # 128-row plans repack instead of reading the rows
                                   (130, 200, 960), (512, 4096, 960)])
def test_matmul_int8_prefill_closed_form(m, n, k):
    """Prefill-sized matmul_int8 (int8.rs:61-98) at full shapes: the int32
    accumulators against an exact float64 matmul (|sum| <= 127^2 * K < 2^53)
    and the f32 outputs against the two-multiply epilogue in float32."""
    say(f"matmul_int8 prefill m={m} n={n} k={k}")
    t = torch()
    rng = np.random.default_rng(m + 3 * n + 7 * k)
    wq = rng.integers(-127, 128, (n, k)).astype(np.int8)
    ws = rng.uniform(1e-4, 1e-3, n).astype(F32)
    aq = rng.integers(-127, 128, (m, k)).astype(np.int8)
    sa = F32(0.0173)
    acc0 = (aq.astype(np.float64) @ wq.astype(np.float64).T).astype(np.int32)
    out0 = (acc0.astype(F32) * sa) * ws[None, :]
    w = mri().QMatrix.from_host(wq, ws)
    out = empty((m, n), t.float32)
    acc = empty((m, n), t.int32)
    mri().matmul_int8(dev(aq), sa, w, m, out, acc)
    assert np.array_equal(host(acc), acc0)
    assert_bits_equal(host(out), out0, "matmul_int8 prefill out")


@pytest.mark.parametrize("m,n,k", [(128, 4096, 4096), (512, 11008, 4096), (256, 300, 4096)])
def test_matmul_int8_prefill_misaligned_rows(m, n, k):
    """Rows at an address that is not 16-byte aligned take the repack path;
    the result equals the aligned call (which reads the rows as they are)
    bit for bit, and the closed form."""
    say(f"matmul_int8 prefill misaligned m={m} n={n} k={k}")
    t = torch()
    rng = np.random.default_rng(m + 5 * n + k)
    wq = rng.integers(-127, 128, (n, k)).astype(np.int8)
    ws = rng.uniform(1e-4, 1e-3, n).astype(F32)
    aq = rng.integers(-127, 128, (m, k)).astype(np.int8)
    acc0 = (aq.astype(np.float64) @ wq.astype(np.float64).T).astype(np.int32)
    w = mri().QMatrix.from_host(wq, ws)
    buf = dev(np.concatenate([np.zeros(4, np.int8), aq.ravel()]))
    au = buf[4:]
    assert au.data_ptr() % 16 != 0
    out_u, acc_u = empty((m, n), t.float32), empty((m, n), t.int32)
    mri().matmul_int8(au, F32(0.0173), w, m, out_u, acc_u)
    out_a, acc_a = empty((m, n), t.float32), empty((m, n), t.int32)
    mri().matmul_int8(dev(aq), F32(0.0173), w, m, out_a, acc_a)
    assert np.array_equal(host(acc_u), acc0)
    assert np.array_equal(host(acc_a), acc0)
    assert_bits_equal(host(out_u), host(out_a), "matmul_int8 misaligned vs aligned rows")


def test_matmul_int8_prefill_back_to_back():
    """Consecutive prefill products of different shapes on one stream, with
    and without the int32 output: every call starts from a clean state (the
    split-tile bookkeeping is left as it was found)."""
    t = torch()
    cases = []
    for m, n, k in [(300, 200, 1024), (2048, 512, 4096), (300, 200, 1024), (1024, 4096, 4096),
                    (2048, 512, 4096), (100, 1000, 4096), (200, 300, 2048), (100, 1000, 4096),
                    (768, 11008, 4096), (512, 11008, 4096), (768, 11008, 4096)]:
        rng = np.random.default_rng(m * 5 + n + k)
        wq = rng.integers(-127, 128, (n, k)).astype(np.int8)
        ws = rng.uniform(1e-4, 1e-3, n).astype(F32)
        aq = rng.integers(-127, 128, (m, k)).astype(np.int8)
        acc0 = (aq.astype(np.float64) @ wq.astype(np.float64).T).astype(np.int32)
        cases.append((m, n, k, mri().QMatrix.from_host(wq, ws), dev(aq),
                      acc0, (acc0.astype(F32) * F32(0.02)) * ws[None, :]))
    outs = []
    for i, (m, n, k, w, a, _, _) in enumerate(cases):
        say(f"matmul_int8 back-to-back #{i} m={m} n={n} k={k}")
        out = empty((m, n), t.float32)
        acc = empty((m, n), t.int32) if i % 2 == 0 else None
        mri().matmul_int8(a, F32(0.02), w, m, out, acc)
        outs.append((out, acc))
    for (m, n, k, _, _, acc0, out0), (out, acc) in zip(cases, outs):
        if acc is not None:
            assert np.array_equal(host(acc), acc0)
        assert_bits_equal(host(out), out0, f"matmul_int8 back-to-back {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,k", [(1, 64, 4096), (7, 40, 256), (48, 32, 128), (260, 96, 512)])
def test_matmul_int8_rows_bit_exact(m, n, k):
    t = torch()
    rng = np.random.default_rng(m + n + k)
    wq, ws = synth_int8_weights(rng, n, k)
    aq = rng.integers(-127, 128, (m, k)).astype(np.int8)
    sas = rng.uniform(1e-3, 1e-1, m).astype(F32)
    out0, acc0 = O.matmul_int8_rows(aq, sas, wq, ws, m, want_acc=True)
    w = mri().QMatrix.from_host(wq, ws)
    out, acc = empty((m, n), t.float32), empty((m, n), t.int32)
    mri().matmul_int8_rows(dev(aq), dev(sas), w, m, out, acc)
    assert np.array_equal(host(acc), acc0)
    assert_bits_equal(host(out), out0, "matmul_int8_rows out")


@pytest.mark.parametrize("m,n,k", [(128, 4096, 4096), (128, 11008, 4096), (512, 4096, 4096),
                                   (512, 11008, 4096), (2048, 4096, 4096), (2048, 11008, 4096),
                                   (768, 11008, 4096)])
def test_matmul_int8_rows_prefill_closed_form(m, n, k):
    """matmul_int8 with one activation scale per row (the per-row mode of the
    prefill benchmark) at the prefill shapes (M = 128 / 512 / 2048, N = 4096 /
    11008, K = 4096) and at 768 x 11008 (stream-K): int32 accumulators
    against an exact float64 matmul, f32 outputs bit for bit against
    ((f32)acc * s_a[m]) * s_w[n] in float32 (int8.rs:93 with s_a per row),
    both with the int32 output and without it (the staged-tile epilogue)."""
    say(f"matmul_int8_rows prefill m={m} n={n} k={k}")
    t = torch()
    rng = np.random.default_rng(m + 11 * n + k)
    wq = rng.integers(-127, 128, (n, k)).astype(np.int8)
    ws = rng.uniform(1e-4, 1e-3, n).astype(F32)
    aq = rng.integers(-127, 128, (m, k)).astype(np.int8)
    sas = rng.uniform(1e-3, 1e-1, m).astype(F32)
    acc0 = (aq.astype(np.float64) @ wq.astype(np.float64).T).astype(np.int32)
    out0 = (acc0.astype(F32) * sas[:, None]) * ws[None, :]
    w = mri().QMatrix.from_host(wq, ws)
    out, acc = empty((m, n), t.float32), empty((m, n), t.int32)
    mri().matmul_int8_rows(dev(aq), dev(sas), w, m, out, acc)
    assert np.array_equal(host(acc), acc0)
    assert_bits_equal(host(out), out0, "matmul_int8_rows prefill out (with acc)")
    out2 = empty((m, n), t.float32)
    mri().matmul_int8_rows(dev(aq), dev(sas), w, m, out2)
    assert_bits_equal(host(out2), out0, "matmul_int8_rows prefill out")


@pytest.mark.parametrize("m,n,k", [(1, 11008, 4096), (4, 64, 4096), (32, 128, 4096),
                                   (3, 20, 96), (200, 48, 256), (300, 512, 4096),
                                   (64, 100, 96)])
def test_matmul_int8_from_f32_bit_exact(m, n, k):
    say(f"matmul_int8_from_f32 m={m} n={n} k={k}")
    t = torch()
    rng = np.random.default_rng(m * 3 + n + k)
    wq, ws = synth_int8_weights(rng, n, k)
    x = rng.standard_normal((m, k)).astype(F32)
    out0, aq0, sa0, acc0 = O.matmul_int8_from_f32(x, wq, ws)
    w = mri().QMatrix.from_host(wq, ws)
    out, acc = empty((m, n), t.float32), empty((m, n), t.int32)
    aq, sa = empty((m, k), t.int8), empty(1, t.float32)
    mri().matmul_int8_from_f32(dev(x), w, out, aq, sa, acc)
    assert host(sa)[0] == sa0
    assert np.array_equal(host(aq), aq0)
    assert np.array_equal(host(acc), acc0)
    assert_bits_equal(host(out), out0, "matmul_int8_from_f32 out")


@pytest.mark.parametrize("n,k", [(11008, 4096), (4096, 4096), (4096, 11008), (8192, 1088),
                                 (100, 96), (1000, 4160), (48, 32)])
def test_matmul_int8_from_f32_lapwise_bit_exact(n, k):
    """One row without the quantized-row output: below 1024 tiles the GEMV
    quantizes the row lap by lap inside each wave (688 tiles with 4-chunk
    laps, 256 with 8, 8 waves a tile at K = 11008, uneven segments and a
    partial last lap at K = 1088 and 4160, K below one lap).  Outputs and
    int32 sums bit for bit those of the oracle and of the call that also
    returns the quantized row."""
    say(f"matmul_int8_from_f32 lap-wise n={n} k={k}")
    t = torch()
    rng = np.random.default_rng(n + 7 * k)
    wq, ws = synth_int8_weights(rng, n, k)
    x = rng.standard_normal((1, k)).astype(F32)
    out0, aq0, sa0, acc0 = O.matmul_int8_from_f32(x, wq, ws)
    w = mri().QMatrix.from_host(wq, ws)
    out, acc = empty((1, n), t.float32), empty((1, n), t.int32)
    mri().matmul_int8_from_f32(dev(x), w, out, None, None, acc)
    assert np.array_equal(host(acc), acc0)
    assert_bits_equal(host(out), out0, "matmul_int8_from_f32 lap-wise out")
    out2 = empty((1, n), t.float32)
    mri().matmul_int8_from_f32(dev(x), w, out2)
    assert_bits_equal(host(out2), out0, "matmul_int8_from_f32 lap-wise out (no acc)")
    out3, aq, sa = empty((1, n), t.float32), empty((1, k), t.int8), empty(1, t.float32)
    mri().matmul_int8_from_f32(dev(x), w, out3, aq, sa)
    assert_bits_equal(host(out3), host(out), "up-front vs lap-wise")


def special_row(rng, k, top=127.0, nan=True, inf=False):
    """A row whose values land on the quantizer's edge cases: with max|x| =
    127 the scale is exactly 1, so every half-integer is a tie (rounded away
    from zero), 0.49999997 is just below one, 126.5 and -127 sit at the
    clamp; NaN elements quantize to 0 and leave the max alone; an infinite
    element makes the scale infinite (every value then quantizes to 0)."""
    vals = np.array([0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 62.5, -62.5, 126.5, -126.5, 0.49999997,
                     -0.49999997, 0.0, -0.0, 3.0, -127.0], F32)
    x = vals[rng.integers(0, vals.size, k)] * F32(top / 127.0)
    x[rng.integers(0, k)] = top
    if nan:
        x[rng.integers(0, k, 3)] = np.nan
    if inf:
        x[rng.integers(0, k)] = np.inf
    return x.reshape(1, k)


@pytest.mark.parametrize("n,k", [(11008, 4096), (4096, 4096), (32000, 4096), (8200, 992),
                                 (48, 4096)])
@pytest.mark.parametrize("case", ["ties", "ties_scaled", "inf"])
def test_fused_row_quantizer_edge_values(n, k, case):
    """The decode GEMVs quantize their f32 row themselves (lap by lap inside
    each wave below 1024 tiles, up front above; Q8_0 into the masked operand
    layout, INT8 into its lap area).  At ties, values just below one, the
    clamp, NaN and infinite elements their quantized values must be
    quantize_symmetric's (symmetric.rs:42-57): Q8_0 block dots and scale and
    INT8 int32 sums bit for bit the oracle's."""
    say(f"fused row quantizer n={n} k={k} {case}")
    t = torch()
    rng = np.random.default_rng(n + k + len(case))
    x = special_row(rng, k, top=127.0 if case != "ties_scaled" else 3.75,
                    inf=case == "inf")
    raw = synth_q8_0(rng, n, k)
    out0, bd0, sa0 = O.matmul_q8_0_direct(x, raw, n, k, want_block_dots=True)
    w = mri().Q8Matrix.from_raw_bytes(raw, n, k)
    out, bd, sa = empty((1, n), t.float32), empty((1, n, k // 32), t.int32), empty(1, t.float32)
    mri().matmul_q8_0_direct(dev(x), w, out, bd, sa)
    assert np.array_equal(bits(host(sa)), bits(sa0))
    assert np.array_equal(host(bd), bd0)
    if case == "inf":
        assert np.isinf(sa0[0]) and not bd0.any()
        assert np.array_equal(np.isnan(host(out)), np.isnan(out0))
    else:
        q8_check(host(out), out0, bd0, sa0, raw, n, k, "q8_0 out", exact=False)
    wq, ws = synth_int8_weights(rng, n, k)
    iout0, _, _, acc0 = O.matmul_int8_from_f32(x, wq, ws)
    wi = mri().QMatrix.from_host(wq, ws)
    iout, acc = empty((1, n), t.float32), empty((1, n), t.int32)
    mri().matmul_int8_from_f32(dev(x), wi, iout, None, None, acc)
    assert np.array_equal(host(acc), acc0)
    if case == "inf":  # 0 * inf: NaN on both sides (the payload may differ)
        assert np.array_equal(np.isnan(host(iout)), np.isnan(iout0))
    else:
        assert_bits_equal(host(iout), iout0, "int8 out")


# ---- Q8_0 --------------------------------------------------------------------------

Q8_SHAPES = [
    (1, 16, 32), (1, 4096 // 4, 4096), (1, 50, 96), (1, 64, 11008), (2, 33, 256),
    (1, 16400, 8192), (1, 4096, 11008), (3, 2000, 4096), (1, 32000, 4096),
    (4, 48, 4096), (8, 16, 512), (16, 40, 1024), (17, 20, 64), (32, 64, 4096),
    (40, 24, 128), (33, 48, 256), (64, 80, 1024), (100, 37, 4096), (512, 96, 512),
    (300, 4096, 256), (2, 4096, 11008), (3, 11008, 4096), (4, 11008, 4096), (4, 64, 2048),
    # the benchmarked decode shapes: [1,4096]x[4096,4096] and [4096,11008], and the
    # batched decode rows M = 8, 16, 32 at N = 11008
    (1, 11008, 4096), (1, 4096, 4096), (8, 11008, 4096), (16, 11008, 4096), (32, 11008, 4096),
    # one row at 512-1023 tiles (the row quantized lap by lap in the GEMV): K with
    # padding blocks in its last lap, and K = 11008
    (1, 8200, 992), (1, 12000, 11008),
    # two to four f32 rows quantized in the GEMV prologue (without block dots): 4 waves x
    # 1 lap at 688 tiles, 4 x 2 below 512 tiles, 8 x 2 at K = 8192
    (2, 11008, 4096), (4, 4096, 4096), (2, 4096, 8192),
    # prefill sizes: partial row and channel tiles, K with padding blocks in its last lap
    # (992), many laps (11008); from 128 rows and more than 2^20 outputs the LDS-tiled
    # kernel (partial 128-row and 64-channel tiles), at 2^20 outputs the skinny kernel
    (128, 1000, 4096), (130, 520, 992), (200, 264, 11008), (64, 2048, 2048),
    (256, 8192, 256), (300, 8200, 512), (260, 16400, 256), (257, 8192, 992),
    (128, 8200, 512), (129, 8200, 256), (128, 8192, 256), (512, 2048, 256), (512, 2056, 256),
    (300, 4100, 1024),
]


def q8_check(got, out0, bd0, sa0, raw, n, k, what, exact=None):
    """Q8_0 f32 outputs against the oracle: within the contract, and bit for
    bit where the kernel keeps the reference's order (the skinny kernel: more
    than 4 rows, except the LDS-tiled kernel's range without block dots)."""
    d, _ = CF.q8_0_split(raw, n, k)
    assert_q8_close(got, out0, q8_terms_abs_sum(bd0, sa0, d), what)
    if exact is None:
        exact = got.shape[0] > 4 and not q8_gemm_range(got.shape[0], n)
    if exact:
        assert_bits_equal(got, out0, what)


@pytest.mark.parametrize("m,n,k", Q8_SHAPES)
def test_matmul_q8_0_direct_parity(m, n, k):
    say(f"matmul_q8_0_direct m={m} n={n} k={k}")
    t = torch()
    rng = np.random.default_rng(m * 11 + n + k)
    raw = synth_q8_0(rng, n, k, with_min=True)
    x = rng.standard_normal((m, k)).astype(F32)
    out0, bd0, sa0 = O.matmul_q8_0_direct(x, raw, n, k, want_block_dots=True)
    w = mri().Q8Matrix.from_raw_bytes(raw, n, k)
    out = empty((m, n), t.float32)
    bd = empty((m, n, k // 32), t.int32)
    sa = empty(m, t.float32)
    mri().matmul_q8_0_direct(dev(x), w, out, bd, sa)
    assert np.array_equal(bits(host(sa)), bits(sa0))
    assert np.array_equal(host(bd), bd0)
    q8_check(host(out), out0, bd0, sa0, raw, n, k, "q8_0 out", exact=m > 4)
    out2 = empty((m, n), t.float32)        # without the debug outputs
    sa2 = empty(m, t.float32)
    mri().matmul_q8_0_direct(dev(x), w, out2, act_scales_out=sa2)
    assert np.array_equal(bits(host(sa2)), bits(sa0))
    if q8_gemm_range(m, n):   # the LDS-tiled kernel: fused fold, within the contract
        q8_check(host(out2), out0, bd0, sa0, raw, n, k, "q8_0 out (prefill kernel)")
    else:
        assert_bits_equal(host(out2), host(out), "q8_0 out (no debug outputs)")


@pytest.mark.parametrize("m,n,k", [(512, 12288, 4096), (512, 22016, 4096), (512, 32000, 4096),
                                   (512, 4096, 4096), (512, 4096, 11008)])
def test_q8_0_prefill_gemm_full_shapes(m, n, k):
    """The LDS-tiled Q8_0 GEMM (m >= 128, m * n > 2^20, no block dots) at
    the shapes the decoder layer's prefill runs it at (fused q/k/v, fused
    gate/up, lm_head, o and down at 512 rows): every output within the contract of the
    oracle's sequential block sum (q8_direct.rs:229-289), and the activation
    scales bit-exact."""
    say(f"matmul_q8_0_direct prefill gemm m={m} n={n} k={k}")
    t = torch()
    rng = np.random.default_rng(m + n + k)
    raw = synth_q8_0(rng, n, k, with_min=True)
    x = rng.standard_normal((m, k)).astype(F32)
    w = mri().Q8Matrix.from_raw_bytes(raw, n, k)
    out = empty((m, n), t.float32)
    sa = empty(m, t.float32)
    mri().matmul_q8_0_direct(dev(x), w, out, act_scales_out=sa)
    got, sa_got = host(out), host(sa)
    out0, terms = q8_oracle_sliced(x, raw, n, k)
    assert np.array_equal(bits(sa_got), bits(CF.quantize_rows(x)[1]))
    assert_q8_close(got, out0, terms, f"q8_0 prefill gemm {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,k", [(1, 11008, 4096), (2, 300, 256), (4, 4096, 4096),
                                   (3, 64, 11008), (8, 48, 512), (256, 8192, 256),
                                   (300, 8200, 512), (128, 8200, 512), (512, 4096, 1024)])
def test_matmul_q8_0_direct_exact(m, n, k):
    """mri_matmul_q8_0_direct_exact keeps the reference's block order at
    every row count: bit-identical to the oracle where the default entry
    point reorders (m <= 4, and m >= 128 with m * n > 2^20), with and without
    block dots."""
    say(f"matmul_q8_0_direct_exact m={m} n={n} k={k}")
    t = torch()
    rng = np.random.default_rng(m * 13 + n + k)
    raw = synth_q8_0(rng, n, k, with_min=True)
    x = rng.standard_normal((m, k)).astype(F32)
    out0, bd0, sa0 = O.matmul_q8_0_direct(x, raw, n, k, want_block_dots=True)
    w = mri().Q8Matrix.from_raw_bytes(raw, n, k)
    out, sa = empty((m, n), t.float32), empty(m, t.float32)
    mri().matmul_q8_0_direct_exact(dev(x), w, out, act_scales_out=sa)
    assert np.array_equal(bits(host(sa)), bits(sa0))
    assert_bits_equal(host(out), out0, "q8_0 exact out")
    out2, bd = empty((m, n), t.float32), empty((m, n, k // 32), t.int32)
    mri().matmul_q8_0_direct_exact(dev(x), w, out2, bd)
    assert np.array_equal(host(bd), bd0)
    assert_bits_equal(host(out2), out0, "q8_0 exact out (with block dots)")


# f16 block scales beyond the positive normals: subnormals (exact in f32,
# m * 2^-24), both zeros, negative normals and subnormals, the extremes of
# the normal range (f16_to_f32, quantization.rs:416-459)
F16_SPECIAL = np.array([0x0001, 0x0002, 0x01FF, 0x0200, 0x03FF, 0x0000, 0x8000, 0x8001,
                        0x83FF, 0x0400, 0x8400, 0x9C00, 0xA1A3, 0x7BFF, 0xFBFF, 0x2E66,
                        0x1C00, 0x9400], np.uint16)


def special_scale_blocks(rng, n, k):
    q = rng.integers(-128, 128, (n, k)).astype(np.int8)
    d = rng.choice(F16_SPECIAL, (n, k // 32)).astype(np.uint16)
    return CF.q8_0_pack(d, q)


# the M = 1 GEMV (fused quantization), the M = 3 GEMV on quantized rows, the
# skinny kernel (8 and 40 rows), the LDS-tiled prefill GEMM (256 x 8192)
SPECIAL_SHAPES = [(1, 4096, 4096), (1, 48, 992), (3, 64, 1024), (8, 48, 512), (40, 64, 256),
                  (256, 8192, 256)]


@pytest.mark.parametrize("m,n,k", SPECIAL_SHAPES)
def test_q8_0_special_f16_scales(m, n, k):
    """Subnormal, zero, negative and extreme f16 block scales through every
    Q8_0 kernel: block dots bit-exact, f32 within the contract (bit-exact
    where the kernel keeps the block order)."""
    say(f"matmul_q8_0_direct special scales m={m} n={n} k={k}")
    t = torch()
    rng = np.random.default_rng(m * 5 + n + k)
    raw = special_scale_blocks(rng, n, k)
    x = rng.standard_normal((m, k)).astype(F32)
    out0, bd0, sa0 = O.matmul_q8_0_direct(x, raw, n, k, want_block_dots=True)
    w = mri().Q8Matrix.from_raw_bytes(raw, n, k)
    out = empty((m, n), t.float32)
    mri().matmul_q8_0_direct(dev(x), w, out)   # the kernel the shape dispatches to
    q8_check(host(out), out0, bd0, sa0, raw, n, k, "q8_0 special scales")
    bd = empty((m, n, k // 32), t.int32)
    out2 = empty((m, n), t.float32)
    mri().matmul_q8_0_direct(dev(x), w, out2, bd)
    assert np.array_equal(host(bd), bd0)
    q8_check(host(out2), out0, bd0, sa0, raw, n, k, "q8_0 special scales (block dots)",
             exact=m > 4)


def assert_same_class(got, exp, what):
    """Where the reference is not finite, the same class: NaN for NaN, the
    same infinity for an infinity."""
    got, exp = np.asarray(got, F32), np.asarray(exp, F32)
    en, gn = np.isnan(exp), np.isnan(got)
    assert np.array_equal(en, gn), f"{what}: NaN positions differ ({int(en.sum())} expected)"
    ei = np.isinf(exp)
    assert np.array_equal(ei, np.isinf(got)), f"{what}: infinity positions differ"
    assert np.array_equal(exp[ei], got[ei]), f"{what}: infinity signs differ"


@pytest.mark.parametrize("m,n,k", SPECIAL_SHAPES)
def test_q8_0_nonfinite_f16_scales(m, n, k):
    """Infinite and NaN f16 block scales decode to inf / NaN
    (quantization.rs:416-459), so the outputs they reach are inf or NaN in
    every summation order: the GPU gives the same class at the same places,
    and the finite outputs within the contract."""
    say(f"matmul_q8_0_direct non-finite scales m={m} n={n} k={k}")
    t = torch()
    rng = np.random.default_rng(m * 3 + n + k + 1)
    raw = special_scale_blocks(rng, n, k)
    # one block of about a third of the weight rows gets +inf, -inf or a NaN
    # (two payloads) as its scale
    blk = np.asarray(raw, np.uint8).reshape(n, k // 32, 34).copy()
    rows = np.flatnonzero(rng.random(n) < 0.35)
    cols = rng.integers(0, k // 32, rows.size)
    bad = rng.choice(np.array([0x7C00, 0xFC00, 0x7E00, 0xFD01], np.uint16), rows.size)
    blk[rows, cols, 0] = bad & 0xFF
    blk[rows, cols, 1] = bad >> 8
    raw = blk.ravel()
    x = rng.standard_normal((m, k)).astype(F32)
    out0, bd0, sa0 = O.matmul_q8_0_direct(x, raw, n, k, want_block_dots=True)
    w = mri().Q8Matrix.from_raw_bytes(raw, n, k)
    out = empty((m, n), t.float32)
    mri().matmul_q8_0_direct(dev(x), w, out)
    got = host(out)
    assert_same_class(got, out0, "q8_0 non-finite scales")
    fin_out = np.isfinite(out0)
    d2, _ = CF.q8_0_split(raw, n, k)
    with np.errstate(invalid="ignore"):
        terms = q8_terms_abs_sum(bd0, sa0, np.where(np.isfinite(d2), d2, 0.0))
    assert_q8_close(got[fin_out], out0[fin_out], terms[fin_out], "q8_0 non-finite: finite outputs")


def test_q8_0_graph_replay_and_streams():
    """matmul_q8_0_direct at several row counts (the quantize pass plus the
    decode GEMV or the skinny kernel) captured in one HIP graph: every replay
    agrees with the oracle for the input it sees (new data copied in between
    replays, eager work and synchronizations between them), and so do calls
    on two streams at once and back-to-back calls of different sizes."""
    t = torch()
    rng = np.random.default_rng(77)
    n, k = 272, 1024
    raw = synth_q8_0(rng, n, k, with_min=True)
    w = mri().Q8Matrix.from_raw_bytes(raw, n, k)
    sizes = [8, 3, 32, 17, 2]
    xs = [dev(np.zeros((m, k), F32)) for m in sizes]
    outs = [empty((m, n), t.float32) for m in sizes]

    def calls():
        for x, o in zip(xs, outs):
            mri().matmul_q8_0_direct(x, w, o)

    def check(host_xs, what):
        for m, hx, o in zip(sizes, host_xs, outs):
            out0, bd0, sa0 = O.matmul_q8_0_direct(hx, raw, n, k, want_block_dots=True)
            q8_check(host(o), out0, bd0, sa0, raw, n, k, f"{what} m={m}")

    s = t.cuda.Stream()
    s.wait_stream(t.cuda.current_stream())
    with t.cuda.stream(s):   # the stream's staging exists before capture
        calls()
    t.cuda.synchronize()
    g = t.cuda.CUDAGraph()
    with t.cuda.graph(g, stream=s):
        calls()
    for rep in range(4):
        hx = [rng.standard_normal((m, k)).astype(F32) * (rep + 1) for m in sizes]
        for x, h in zip(xs, hx):
            x.copy_(dev(h))
        for o in outs:
            o.zero_()
        t.cuda.synchronize()
        g.replay()
        t.cuda.synchronize()
        check(hx, f"graph replay {rep}")
        mri().matmul_q8_0_direct(xs[0], w, outs[0])   # eager work between replays
        t.cuda.synchronize()
    # two streams at once, then back-to-back sizes on the default stream
    hx = [rng.standard_normal((m, k)).astype(F32) for m in sizes]
    for x, h in zip(xs, hx):
        x.copy_(dev(h))
    t.cuda.synchronize()
    s1, s2 = t.cuda.Stream(), t.cuda.Stream()
    with t.cuda.stream(s1):
        mri().matmul_q8_0_direct(xs[0], w, outs[0])
        mri().matmul_q8_0_direct(xs[2], w, outs[2])
    with t.cuda.stream(s2):
        mri().matmul_q8_0_direct(xs[1], w, outs[1])
        mri().matmul_q8_0_direct(xs[3], w, outs[3])
        mri().matmul_q8_0_direct(xs[4], w, outs[4])
    t.cuda.synchronize()
    check(hx, "two streams")
    calls()
    calls()
    check(hx, "back to back")


def test_q8_0_gemm_k_split():
    """The LDS-tiled Q8_0 GEMM with its K split (2 parts per tile when the
    tiles would fill at most one workgroup slot per CU: 200 x 4096 x 6000
    and 128 x 2048 x 8256 here): within the contract of the oracle,
    deterministic (the parts are added in part order, whatever the order of
    arrival: the same input gives the same bits on every call), the tile
    counters reset between back-to-back calls of different shapes, HIP graph
    replays equal eager calls, and the no-allocation entry point (no K split)
    is within the contract too."""
    t = torch()
    rng = np.random.default_rng(91)
    cases = [(200, 6000, 4096), (128, 8256, 2048)]
    ws, xs, outs, raws = [], [], [], []
    for m, n, k in cases:
        raw = synth_q8_0(rng, n, k, with_min=True)
        raws.append(raw)
        ws.append(mri().Q8Matrix.from_raw_bytes(raw, n, k))
        xs.append(dev(rng.standard_normal((m, k)).astype(F32)))
        outs.append(empty((m, n), t.float32))

    def calls():
        for x, w, o in zip(xs, ws, outs):
            mri().matmul_q8_0_direct(x, w, o)

    calls()
    t.cuda.synchronize()
    first = [host(o).copy() for o in outs]
    for (m, n, k), raw, x, got in zip(cases, raws, xs, first):
        say(f"q8_0 gemm k split m={m} n={n} k={k}")
        out0, terms = q8_oracle_sliced(host(x), raw, n, k)
        assert_q8_close(got, out0, terms, f"k split {m}x{n}x{k}")
        na = empty((m, n), t.float32)
        mri().matmul_q8_0_direct_noalloc(x, ws[cases.index((m, n, k))], na)
        assert_q8_close(host(na), out0, terms, f"no-alloc {m}x{n}x{k}")
    calls()   # back to back: the counters were left at zero
    for o, f in zip(outs, first):
        assert_bits_equal(host(o), f, "k split, second call")
    s = t.cuda.Stream()
    s.wait_stream(t.cuda.current_stream())
    with t.cuda.stream(s):   # the stream's staging and workspace exist before capture
        calls()
    t.cuda.synchronize()
    g = t.cuda.CUDAGraph()
    with t.cuda.graph(g, stream=s):
        calls()
    for rep in range(3):
        for x, (m, n, k) in zip(xs, cases):
            x.copy_(dev(rng.standard_normal((m, k)).astype(F32) * (rep + 1)))
        for o in outs:
            o.zero_()
        t.cuda.synchronize()
        g.replay()
        t.cuda.synchronize()
        replayed = [host(o).copy() for o in outs]
        calls()   # eager work between replays, on the same inputs
        t.cuda.synchronize()
        for o, r in zip(outs, replayed):
            assert_bits_equal(r, host(o), f"graph replay {rep} vs eager")


def test_q8_0_reference_encoder_weights():
    """Weights built by create_q8_0_block (dequant.rs:389-421), as
    Q8_0WeightMatrix::from_f32_tensor does."""
    t = torch()
    rng = np.random.default_rng(3)
    wf = (rng.standard_normal((24, 256)) * 0.05).astype(F32)
    raw = O.quantize_q8_0(wf)
    x = rng.standard_normal((3, 256)).astype(F32)
    out0, bd0, sa0 = O.matmul_q8_0_direct(x, raw, 24, 256, want_block_dots=True)
    w = mri().Q8Matrix.from_raw_bytes(raw, 24, 256)
    out = empty((3, 24), t.float32)
    mri().matmul_q8_0_direct(dev(x), w, out)
    q8_check(host(out), out0, bd0, sa0, raw, 24, 256, "q8_0 encoder weights")


# ---- Q4_0 ----------------------------------------------------------------------------

@pytest.mark.parametrize("m,n,k", [(1, 16, 32), (1, 300, 4096), (3, 20, 96),
                                   (2, 64, 11008), (5, 7, 64), (1, 11008, 4096),
                                   (3, 4096, 11008), (2, 37, 512), (4, 21, 256),
                                   (1, 1000, 32768)])
def test_matmul_q4_0_dequant_tolerance(m, n, k):
    say(f"matmul_q4_0 m={m} n={n} k={k}")
    t = torch()
    rng = np.random.default_rng(m + n * 3 + k)
    raw = synth_q4_0(rng, n, k)
    x = rng.standard_normal((m, k)).astype(F32)
    out0 = O.matmul_q4_0_dequant(x, raw, n, k)
    out = empty((m, n), t.float32)
    mri().matmul_q4_0_dequant(dev(x), dev(raw), n, k, out)
    got = host(out)
    scale = np.maximum(np.abs(out0), CF.q4_0_terms_abs_sum(x, raw, n, k))
    err = np.abs(got.astype(np.float64) - out0)
    assert np.all(err <= 1e-5 * scale), float(np.max(err / scale))
    if k % 256 == 0 and m > 1:  # the staged form from a 16-byte aligned, unaligned-row x
        xo = torch().zeros(m * k + 1, dtype=t.float32, device="cuda")
        xo[1:] = dev(x).view(-1)
        out2 = empty((m, n), t.float32)
        mri().matmul_q4_0_dequant(xo[1:], dev(raw), n, k, out2, shape=(m, k))
        assert np.array_equal(host(out2), got)


@pytest.mark.parametrize("m,n,k", [(1, 16, 32), (1, 300, 4096), (3, 20, 96), (2, 64, 11008),
                                   (5, 7, 64), (4, 21, 256), (7, 48, 512)])
def test_matmul_q4_0_dequant_ggml_order(m, n, k):
    """W4A32 on GGML-order blocks: the same elements as the interleaved
    blocks, so the result agrees with the oracle on those to the same
    contract (both the staged and the fallback kernel)."""
    say(f"matmul_q4_0 ggml m={m} n={n} k={k}")
    t = torch()
    rng = np.random.default_rng(m + n * 5 + k)
    raw = synth_q4_0(rng, n, k)
    x = rng.standard_normal((m, k)).astype(F32)
    out0 = O.matmul_q4_0_dequant(x, raw, n, k)
    out = empty((m, n), t.float32)
    mri().matmul_q4_0_dequant_ordered(dev(x), dev(CF.q4_0_interleaved_to_ggml(raw)), n, k,
                                      mri().Q4_ORDER_GGML, out)
    scale = np.maximum(np.abs(out0), CF.q4_0_terms_abs_sum(x, raw, n, k))
    err = np.abs(host(out).astype(np.float64) - out0)
    assert np.all(err <= 1e-5 * scale), float(np.max(err / scale))
    with pytest.raises(mri().MriError) as e:
        mri().matmul_q4_0_dequant_ordered(dev(x), dev(raw), n, k, 7, out)
    assert e.value.kind == "InvalidArgument"


@pytest.mark.parametrize("m,n,k", [(1, 11008, 4096), (1, 4096, 11008), (1, 32000, 4096),
                                   (2, 300, 256), (3, 64, 4096), (4, 48, 4096), (5, 40, 512),
                                   (9, 33, 1024), (1, 16, 32), (1, 50, 96), (1, 1000, 16384)])
@pytest.mark.parametrize("order", [0, 1])
def test_matmul_q4_0_dequant_matrix(m, n, k, order):
    """W4A32 (matmul_q4_0_dequant semantics) on the device-resident 4-bit
    lap blocks of a Q4_0 handle, uploaded from either nibble order: within
    1e-5 * max(|ref|, sum_k |x_k w_k|) of the oracle's sequential sum."""
    say(f"matmul_q4_0_dequant_matrix m={m} n={n} k={k} order={order}")
    t = torch()
    rng = np.random.default_rng(m * 7 + n + k + 11 * order)
    raw = synth_q4_0(rng, n, k)
    x = rng.standard_normal((m, k)).astype(F32)
    out0 = O.matmul_q4_0_dequant(x, raw, n, k)
    up = CF.q4_0_interleaved_to_ggml(raw) if order else raw
    w = mri().Q4Matrix.from_raw_bytes(up, n, k, order)
    out = empty((m, n), t.float32)
    mri().matmul_q4_0_dequant_matrix(dev(x), w, out)
    got = host(out)
    scale = np.maximum(np.abs(out0), CF.q4_0_terms_abs_sum(x, raw, n, k))
    err = np.abs(got.astype(np.float64) - out0)
    assert np.all(err <= 1e-5 * scale), float(np.max(err / scale))


def test_matmul_q4_0_dequant_matrix_errors():
    t = torch()
    M = mri()
    rng = np.random.default_rng(2)
    w = M.Q4Matrix.from_raw_bytes(synth_q4_0(rng, 16, 64), 16, 64)
    out = empty((2, 16), t.float32)
    with pytest.raises(M.MriError) as e:
        M.matmul_q4_0_dequant_matrix(dev(np.zeros((2, 32), F32)), w, out)
    assert e.value.kind == "ShapeMismatch"
    with pytest.raises(M.MriError) as e:
        M.matmul_q4_0_dequant_matrix(dev(np.zeros((2, 64), F32)), w, out, shape=(2, 8, 8))
    assert e.value.kind == "InvalidShape"
    big = M.Q4Matrix.from_raw_bytes(synth_q4_0(rng, 16, 11008), 16, 11008)
    x = dev(np.zeros((4, 11008), F32))
    with pytest.raises(M.MriError) as e:  # four f32 rows of K = 11008 exceed the staging
        M.matmul_q4_0_dequant_matrix(x, big, empty((4, 16), t.float32))
    assert e.value.kind == "Unsupported"


# ---- error behaviour (TensorError kinds and order) ------------------------------------

def test_errors():
    t = torch()
    M = mri()
    wq = np.zeros((2, 32), np.int8)
    w = M.QMatrix.from_host(wq, np.ones(2, F32))
    out = empty((4, 4), t.float32)
    x = dev(np.ones((2, 4, 8), F32))
    with pytest.raises(M.MriError) as e:                 # int8.rs:292-301
        M.matmul_int8_from_f32(x, w, out)
    assert e.value.kind == "InvalidShape"
    w64 = M.QMatrix.from_host(np.zeros((1, 64), np.int8), np.ones(1, F32))
    with pytest.raises(M.MriError) as e:                 # int8.rs:303-318
        M.matmul_int8_from_f32(dev(np.ones((1, 32), F32)), w64, out)
    assert e.value.kind == "ShapeMismatch"
    with pytest.raises(M.MriError) as e:                 # int8.rs:320-329
        M.matmul_int8(dev(np.zeros(10, np.int8)), 1.0, w, 1, out)
    assert e.value.kind == "InvalidShape"
    with pytest.raises(M.MriError) as e:                 # q8_direct.rs:321-331
        M.Q8Matrix.from_raw_bytes(np.zeros(34, np.uint8), 1, 31)
    assert e.value.kind == "InvalidShape"
    with pytest.raises(M.MriError):
        M.Q8Matrix.from_raw_bytes(np.zeros(33, np.uint8), 1, 32)
    M.Q8Matrix.from_raw_bytes(np.zeros(0, np.uint8), 0, 32)   # zero n_out accepted
    q8 = M.Q8Matrix.from_raw_bytes(np.zeros(68, np.uint8), 2, 32)
    with pytest.raises(M.MriError) as e:
        M.matmul_q8_0_direct(x, q8, out)
    assert e.value.kind == "InvalidShape"
    q8b = M.Q8Matrix.from_raw_bytes(np.zeros(2 * 2 * 34, np.uint8), 2, 64)
    with pytest.raises(M.MriError) as e:
        M.matmul_q8_0_direct(dev(np.ones((1, 32), F32)), q8b, out)
    assert e.value.kind == "ShapeMismatch"
    dummy = dev(np.zeros(18, np.uint8))                  # q4_0.rs:307-347 order
    with pytest.raises(M.MriError) as e:
        M.matmul_q4_0_dequant(x, dummy, 1, 32, out)
    assert e.value.kind == "InvalidShape"
    with pytest.raises(M.MriError) as e:
        M.matmul_q4_0_dequant(dev(np.ones((1, 33), F32)), dummy, 1, 33, out)
    assert e.value.kind == "InvalidShape"
    with pytest.raises(M.MriError) as e:
        M.matmul_q4_0_dequant(dev(np.ones((1, 32), F32)), dummy, 1, 64, out)
    assert e.value.kind == "ShapeMismatch"
    with pytest.raises(M.MriError) as e:
        M.matmul_q4_0_dequant(dev(np.ones((1, 32), F32)), dev(np.zeros(20, np.uint8)),
                              1, 32, out)
    assert e.value.kind == "InvalidShape"
    with pytest.raises(M.MriError) as e:
        M.quantize_per_channel(dev(np.zeros(5, F32)), 2, 3, empty(6, t.int8),
                               empty(2, t.float32))
    assert e.value.kind == "InvalidShape"


def test_zero_sizes():
    t = torch()
    M = mri()
    w = M.QMatrix.from_host(np.zeros((0, 32), np.int8), np.zeros(0, F32))
    out = empty(1, t.float32)
    M.matmul_int8_from_f32(dev(np.ones((2, 32), F32)), w, out)
    w2 = M.QMatrix.from_host(np.ones((3, 32), np.int8), np.ones(3, F32))
    M.matmul_int8(dev(np.zeros(0, np.int8)), 1.0, w2, 0, out)
    M.synchronize()


@pytest.mark.parametrize("m", [1, 3, 8])
def test_zero_k(m):
    """K = 0: every output is the empty sum, ((f32)0 * s_a) * s_w for INT8
    and 0.0 for Q8_0 (no blocks), as the oracle computes it."""
    t = torch()
    M = mri()
    n = 32
    x = np.zeros((m, 0), F32)
    xd = t.zeros((m, 0), dtype=t.float32, device="cuda")
    w8 = M.Q8Matrix.from_raw_bytes(np.zeros(0, np.uint8), n, 0)
    out = empty((m, n), t.float32)
    out.fill_(7.0)
    M.matmul_q8_0_direct(xd, w8, out)
    assert_bits_equal(host(out), O.matmul_q8_0_direct(x, np.zeros(0, np.uint8), n, 0),
                      "q8_0 k=0")
    ws = np.linspace(0.5, 2.0, n).astype(F32)
    wi = M.QMatrix.from_host(np.zeros((n, 0), np.int8), ws)
    out2 = empty((m, n), t.float32)
    out2.fill_(7.0)
    M.matmul_int8_from_f32(xd, wi, out2)
    ref = O.matmul_int8_from_f32(x, np.zeros((n, 0), np.int8), ws)[0]
    assert_bits_equal(host(out2), ref, "int8 k=0")


def test_bound_calls_match():
    """The pre-bound call helpers issue the same entry points."""
    t = torch()
    M = mri()
    rng = np.random.default_rng(9)
    n, k = 272, 4096
    raw = synth_q8_0(rng, n, k)
    wq, ws = synth_int8_weights(rng, n, k)
    x = dev(rng.standard_normal((1, k)).astype(F32))
    w8, wi = M.Q8Matrix.from_raw_bytes(raw, n, k), M.QMatrix.from_host(wq, ws)
    a, b = empty((1, n), t.float32), empty((1, n), t.float32)
    M.matmul_q8_0_direct(x, w8, a)
    M.bind_matmul_q8_0_direct(x, w8, b)()
    assert_bits_equal(host(b), host(a), "bound q8_0")
    M.matmul_int8_from_f32(x, wi, a)
    M.bind_matmul_int8_from_f32(x, wi, b)()
    assert_bits_equal(host(b), host(a), "bound int8")


@pytest.mark.parametrize("m", [1, 3])
def test_unfused_path_matches(m):
    """x at a 4-byte (not 16-byte) aligned address takes the two-kernel path
    (quantize kernel + GEMV): Q8_0 within the contract of the oracle and bit
    for bit equal to the fused path; INT8 bit for bit."""
    t = torch()
    rng = np.random.default_rng(21 + m)
    n, k = 48, 4096
    raw = synth_q8_0(rng, n, k)
    wq, ws = synth_int8_weights(rng, n, k)
    x = rng.standard_normal((m, k)).astype(F32)
    buf = dev(np.concatenate([np.zeros(1, F32), x.ravel()]))
    xu = buf[1:].view(m, k)                       # misaligned by 4 bytes
    assert xu.data_ptr() % 16 != 0
    out0, bd0, sa0 = O.matmul_q8_0_direct(x, raw, n, k, want_block_dots=True)
    w8 = mri().Q8Matrix.from_raw_bytes(raw, n, k)
    out = empty((m, n), t.float32)
    mri().matmul_q8_0_direct(xu, w8, out)
    q8_check(host(out), out0, bd0, sa0, raw, n, k, "q8_0 unfused")
    fused = empty((m, n), t.float32)
    mri().matmul_q8_0_direct(dev(x), w8, fused)
    assert_bits_equal(host(out), host(fused), "q8_0 unfused vs fused")
    ref, aq0, sa0, acc0 = O.matmul_int8_from_f32(x, wq, ws)
    wi = mri().QMatrix.from_host(wq, ws)
    out2, aq, sa = empty((m, n), t.float32), empty((m, k), t.int8), empty(1, t.float32)
    mri().matmul_int8_from_f32(xu, wi, out2, aq, sa)
    assert host(sa)[0] == sa0 and np.array_equal(host(aq), aq0)
    assert_bits_equal(host(out2), ref, "int8 unfused")

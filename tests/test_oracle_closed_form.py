"""Pin the oracle against independent closed forms (numpy) on seeded data.

Integer results are compared exactly against int64 matrix products, f32
results bit-for-bit against numpy float32 evaluations in the reference's
operation order.  A final group plants plausible mistakes in a copy of the
closed form and shows that the checks catch each of them.
"""
import numpy as np
import pytest

import closed_form as CF
import oracle_lib as O

F32 = np.float32


def bits(a):
    return np.asarray(a, F32).view(np.uint32)


def test_f16_decode_exhaustive():
    """All 65536 f16 patterns decode as IEEE half (NaN payloads -> NaN)."""
    allbits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = CF.f16_bits_to_f32(allbits)
    got = np.array([O.f16_to_f32(int(b)) for b in allbits], F32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(bits(got)[~nan], bits(ref)[~nan])   # signed zeros too


def test_f32_to_f16_truncates_in_normal_range():
    rng = np.random.default_rng(1)
    e = rng.integers(113, 143, 20000)          # f16-normal exponents
    m = rng.integers(0, 1 << 23, 20000)
    s = rng.integers(0, 2, 20000)
    fb = ((s << 31) | (e << 23) | m).astype(np.uint32)
    expect = ((s << 15) | ((e - 112) << 10) | (m >> 13)).astype(np.uint16)
    got = np.array([O.f32_to_f16(float(v)) for v in fb.view(F32)], np.uint16)
    assert np.array_equal(got, expect)
    # truncation never rounds up: decode(encode(x)) <= |x|
    back = CF.f16_bits_to_f32(got)
    assert np.all(np.abs(back) <= np.abs(fb.view(F32)))


@pytest.mark.parametrize("seed,n,scale", [(0, 4096, 1.0), (1, 1000, 1e-3),
                                          (2, 333, 300.0), (3, 1, 5.0)])
def test_quantize_symmetric_closed_form(seed, n, scale):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(n) * scale).astype(F32)
    # plant exact ties: values whose scaled magnitude is k + 0.5
    q0, s0 = CF.quantize_symmetric(x)
    q, s = O.quantize_symmetric(x)
    assert s == s0 and np.array_equal(q, q0)


def test_quantize_ties_round_away_from_zero():
    # scale = 1 exactly (max_abs = 127): y = x exactly, ties at k+0.5.
    x = np.array([127.0, 0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 62.5, -62.5, 126.5],
                 F32)
    q, s = O.quantize_symmetric(x)
    assert s == 1.0
    assert list(q) == [127, 1, -1, 2, -2, 3, -3, 63, -63, 127]
    assert np.array_equal(CF.quantize_symmetric(x)[0], q)


def test_quantize_special_values():
    x = np.array([np.nan, 1.0, -2.0, 0.25], F32)
    q, s = O.quantize_symmetric(x)            # NaN ignored by the max, NaN -> 0
    assert s == F32(2.0) / F32(127.0)
    assert q[0] == 0 and q[2] == -127
    x = np.array([np.inf, 1.0, -np.inf], F32)  # scale inf -> inv 0 -> 0 / NaN -> 0
    q, s = O.quantize_symmetric(x)
    assert np.isinf(s) and list(q) == [0, 0, 0]
    q0, s0 = CF.quantize_symmetric(x)
    assert np.array_equal(q, q0)


def test_quantize_per_channel_closed_form():
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((37, 96)) * 0.02).astype(F32)
    w[3] = 0.0
    d, s = O.quantize_per_channel(w, 37, 96)
    d0, s0 = CF.quantize_per_channel(w)
    assert np.array_equal(d, d0) and np.array_equal(bits(s), bits(s0))
    assert d.min() >= -127          # never emits -128


@pytest.mark.parametrize("m,n,k,seed", [(1, 257, 4096, 0), (5, 64, 11008, 1),
                                        (17, 33, 96, 2), (3, 5, 31, 3)])
def test_matmul_int8_closed_form(m, n, k, seed):
    rng = np.random.default_rng(seed)
    aq = rng.integers(-127, 128, (m, k)).astype(np.int8)
    w = rng.integers(-127, 128, (n, k)).astype(np.int8)
    sw = rng.uniform(1e-4, 1e-3, n).astype(F32)
    sa = F32(0.0123)
    out, acc = O.matmul_int8(aq, sa, w, sw, m, want_acc=True)
    acc0 = CF.int_matmul(aq, w)
    assert np.array_equal(acc.astype(np.int64), acc0)
    assert np.array_equal(bits(out), bits(CF.epilogue(acc0, sa, sw)))
    avx = O.matmul_int8_avx2(aq, sa, w, sw, m)
    par, _ = O.matmul_int8_parallel(aq, sa, w, sw, m)
    assert np.array_equal(bits(avx), bits(out)) and np.array_equal(bits(par), bits(out))
    rows = rng.uniform(1e-3, 1e-1, m).astype(F32)
    out_r, acc_r = O.matmul_int8_rows(aq, rows, w, sw, m, want_acc=True)
    assert np.array_equal(bits(out_r), bits(CF.epilogue(acc0, rows, sw)))


def test_matmul_int8_from_f32_closed_form():
    rng = np.random.default_rng(9)
    x = rng.standard_normal((7, 256)).astype(F32)
    w, sw = CF.quantize_per_channel((rng.standard_normal((40, 256)) * 0.02).astype(F32))
    out, aq, sa, acc = O.matmul_int8_from_f32(x, w, sw)
    aq0, sa0 = CF.quantize_symmetric(x)             # per-tensor over [M,K]
    assert sa == sa0 and np.array_equal(aq.ravel(), aq0)
    acc0 = CF.int_matmul(aq0.reshape(7, 256), w)
    assert np.array_equal(bits(out), bits(CF.epilogue(acc0, sa0, sw)))


def _q8_synth(rng, n, k, with_min=False):
    q = rng.integers(-127, 128, (n, k)).astype(np.int8)
    if with_min:
        q[rng.random((n, k)) < 0.05] = -128
    d = rng.uniform(0.001, 0.01, (n, k // 32)).astype(np.float16).view(np.uint16)
    return CF.q8_0_pack(d, q)


@pytest.mark.parametrize("m,n,k,seed,with_min", [(1, 64, 4096, 0, False),
                                                 (4, 33, 1024, 1, True),
                                                 (3, 7, 32, 2, True)])
def test_q8_0_direct_closed_form(m, n, k, seed, with_min):
    rng = np.random.default_rng(seed)
    raw = _q8_synth(rng, n, k, with_min)
    x = rng.standard_normal((m, k)).astype(F32)
    out, bd, sa = O.matmul_q8_0_direct(x, raw, n, k, want_block_dots=True)
    out0, bd0, sa0 = CF.q8_0_direct(x, raw, n, k)
    assert np.array_equal(bd.astype(np.int64), bd0)
    assert np.array_equal(bits(sa), bits(sa0))
    assert np.array_equal(bits(out), bits(out0))


def test_q8_0_codec_closed_form():
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((8, 64)) * 0.05).astype(F32)
    raw = O.quantize_q8_0(w)
    d, q = CF.q8_0_split(raw, 8, 64)
    blocks = w.reshape(-1, 32)
    ma = np.max(np.abs(blocks), axis=1)
    scale = (ma / F32(127.0)).astype(F32)
    d_bits = np.array([O.f32_to_f16(float(v)) for v in scale], np.uint16)
    assert np.array_equal(CF.f16_bits_to_f32(d_bits).reshape(8, 2), d)
    inv = (F32(1.0) / scale).astype(F32)
    q0 = CF.sat_i8(CF.round_half_away(blocks * inv[:, None]), -128, 127)
    assert np.array_equal(q.reshape(-1, 32), q0)
    deq = O.dequantize_q8_0(raw).reshape(8, 64)
    assert np.array_equal(bits(deq), bits((np.repeat(d, 32, 1) * q.astype(F32)).astype(F32)))


@pytest.mark.parametrize("m,n,k,seed", [(1, 48, 512, 0), (3, 9, 96, 1)])
def test_q4_0_dequant_closed_form(m, n, k, seed):
    rng = np.random.default_rng(seed)
    raw = np.empty((n, k // 32, 18), np.uint8)
    raw[:, :, 2:] = rng.integers(0, 256, (n, k // 32, 16))
    d = rng.uniform(0.001, 0.05, (n, k // 32)).astype(np.float16).view(np.uint16)
    raw[:, :, 0] = d & 0xFF
    raw[:, :, 1] = d >> 8
    raw = raw.ravel()
    x = rng.standard_normal((m, k)).astype(F32)
    out = O.matmul_q4_0_dequant(x, raw, n, k)
    assert np.array_equal(bits(out), bits(CF.q4_0_dequant_matmul_seq(x, raw, n, k)))
    deq = O.dequantize_q4_0(raw).reshape(n, k)
    dd, q = CF.q4_0_split(raw, n, k)
    assert np.array_equal(bits(deq), bits((np.repeat(dd, 32, 1) * q.astype(F32)).astype(F32)))


def _q4_synth(rng, n, k):
    raw = np.empty((n, k // 32, 18), np.uint8)
    raw[:, :, 2:] = rng.integers(0, 256, (n, k // 32, 16))
    d = rng.uniform(0.001, 0.05, (n, k // 32)).astype(np.float16).view(np.uint16)
    raw[:, :, 0] = d & 0xFF
    raw[:, :, 1] = d >> 8
    return raw.ravel()


@pytest.mark.parametrize("m,n,k,seed", [(1, 48, 512, 0), (3, 9, 96, 1), (5, 16, 4096, 2)])
def test_q4_0_w4a8_is_q8_0_direct_on_expanded_blocks(m, n, k, seed):
    """The W4A8 extension is matmul_q8_0_direct on the same blocks with
    quants nibble - 8: bit-identical outputs, block dots and scales."""
    rng = np.random.default_rng(seed)
    raw4 = _q4_synth(rng, n, k)
    x = rng.standard_normal((m, k)).astype(F32)
    out, bd, sa = O.matmul_q4_0_w4a8(x, raw4, n, k, want_block_dots=True)
    out8, bd8, sa8 = O.matmul_q8_0_direct(x, CF.q4_0_to_q8_0(raw4, n, k), n, k,
                                          want_block_dots=True)
    assert np.array_equal(bd, bd8)
    assert np.array_equal(bits(sa), bits(sa8))
    assert np.array_equal(bits(out), bits(out8))
    out0, bd0, _ = CF.q8_0_direct(x, CF.q4_0_to_q8_0(raw4, n, k), n, k)
    assert np.array_equal(bd.astype(np.int64), bd0)
    assert np.array_equal(bits(out), bits(out0))


def test_q4_0_w4a8_ggml_order():
    """GGML-order blocks give the interleaved-order result of the same
    elements."""
    rng = np.random.default_rng(7)
    n, k = 24, 1024
    raw4 = _q4_synth(rng, n, k)
    x = rng.standard_normal((2, k)).astype(F32)
    want = O.matmul_q4_0_w4a8(x, raw4, n, k, O.Q4_INTERLEAVED)
    gg = CF.q4_0_interleaved_to_ggml(raw4)
    assert np.array_equal(bits(O.matmul_q4_0_w4a8(x, gg, n, k, O.Q4_GGML)), bits(want))
    # reading GGML bytes in the interleaved order is a different matrix
    assert not np.array_equal(bits(O.matmul_q4_0_w4a8(x, gg, n, k, O.Q4_INTERLEAVED)),
                              bits(want))


def test_q4_0_w4a8_errors():
    x = np.zeros((2, 64), F32)
    raw = np.zeros(2 * 2 * 18, np.uint8)
    with pytest.raises(O.OracleError) as e:
        O.matmul_q4_0_w4a8(x, raw, 2, 96)
    assert e.value.code == 2   # K mismatch first
    with pytest.raises(O.OracleError) as e:
        O.matmul_q4_0_w4a8(np.zeros((2, 48), F32), raw, 2, 48)
    assert e.value.code == 1   # K % 32
    with pytest.raises(O.OracleError) as e:
        O.matmul_q4_0_w4a8(x, raw[:-1], 2, 64)
    assert e.value.code == 1   # byte length


# ---- planted mistakes: each must be caught by the checks above ---------------

def test_planted_half_even_rounding_is_caught():
    x = np.array([127.0, 2.5, -2.5], F32)
    q, _ = O.quantize_symmetric(x)
    wrong = np.round(x).astype(np.int8)            # half-to-even
    assert not np.array_equal(q, wrong)


def test_planted_epilogue_order_and_fma_are_caught():
    rng = np.random.default_rng(11)
    acc = rng.integers(-2_000_000, 2_000_000, (64, 64)).astype(np.int64)
    sa = F32(0.0123457)
    sw = rng.uniform(1e-4, 1e-3, 64).astype(F32)
    right = CF.epilogue(acc, sa, sw)
    fused = (acc.astype(np.float64) * np.float64(sa) * sw.astype(np.float64)).astype(F32)
    assert not np.array_equal(bits(right), bits(fused))


def test_planted_unordered_block_sum_is_caught():
    rng = np.random.default_rng(12)
    n, k = 64, 4096
    raw = _q8_synth(rng, n, k)
    x = rng.standard_normal((1, k)).astype(F32)
    out = O.matmul_q8_0_direct(x, raw, n, k)
    _, bd0, sa0 = CF.q8_0_direct(x, raw, n, k)
    d, _ = CF.q8_0_split(raw, n, k)
    t = ((bd0[0].astype(F32) * sa0[0]) * d).astype(F32)
    pairwise = t.sum(axis=1, dtype=F32)            # numpy pairwise summation
    assert not np.array_equal(bits(out[0]), bits(pairwise))
    assert np.allclose(out[0], pairwise, rtol=1e-5, atol=1e-6)


def test_planted_q4_nibble_order_is_caught():
    blk = np.zeros(18, np.uint8)
    blk[1] = 0x3C
    blk[2:] = np.arange(16, dtype=np.uint8) | (np.uint8(0xF) << 4)
    v = O.dequantize_q4_0(blk)
    ggml_order = np.concatenate([(blk[2:] & 0xF).astype(F32) - 8,
                                 (blk[2:] >> 4).astype(F32) - 8])
    assert not np.array_equal(v, ggml_order)

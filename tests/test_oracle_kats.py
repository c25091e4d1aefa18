"""The reference's own known-answer tests, restated against the CPU oracle.

Each test names the Rust test it restates (src/<file>:<line> of the
reference crate).  Exact assertions stay exact; tolerance assertions keep
the reference's tolerance and error metric.
"""
import math

import numpy as np
import pytest

import oracle_lib as O

F32 = np.float32


def ar(start, stop, mul, add):
    """(start..stop).map(|i| i as f32 * mul + add) with f32 arithmetic."""
    i = np.arange(start, stop).astype(F32)
    return (i * F32(mul) + F32(add)).astype(F32)


def max_rel_err(a, b):
    """max_rel_err of int8.rs:159-167 (denominator floor 1e-3)."""
    a = np.asarray(a, F32).ravel()
    b = np.asarray(b, F32).ravel()
    den = np.maximum(np.maximum(np.abs(a), np.abs(b)), F32(1e-3))
    return float(np.max(np.abs(a - b) / den)) if a.size else 0.0


def naive(x, w):
    """matmul_naive(input, w^T) (naive.rs:31-95): float32 products added in
    the i-p-j order, i.e. sequentially over p for every output."""
    x = np.asarray(x, F32)
    w = np.asarray(w, F32)
    out = np.zeros((x.shape[0], w.shape[0]), F32)
    for p in range(x.shape[1]):
        out = (out + (x[:, p:p + 1] * w[None, :, p]).astype(F32)).astype(F32)
    return out


# ---- quant/int8/symmetric.rs -------------------------------------------------

def test_symmetric_doctest():  # symmetric.rs:33-40
    q, s = O.quantize_symmetric([0.0, 0.5, -1.0, 1.0])
    assert s == F32(1.0) / F32(127.0)
    assert q[2] == -127 and q[3] == 127


def test_scale_is_max_abs_over_127():  # symmetric.rs:171-180
    _, s = O.quantize_symmetric([0.0, 2.54, -1.27, 1.0])
    assert abs(s - F32(2.54) / F32(127.0)) < 1e-6


def test_scale_is_one_when_all_zeros():  # symmetric.rs:182-188
    q, s = O.quantize_symmetric(np.zeros(16, F32))
    assert s == 1.0 and np.all(q == 0)


def test_scale_handles_negative_max():  # symmetric.rs:190-197
    _, s = O.quantize_symmetric([-3.81, 1.0, -0.5])
    assert abs(s - F32(3.81) / F32(127.0)) < 1e-5


def test_max_value_maps_to_127():  # symmetric.rs:201-207
    q, _ = O.quantize_symmetric([1.0, -1.0, 0.5])
    assert q[0] == 127 and q[1] == -127


def test_zero_maps_to_zero():  # symmetric.rs:209-214
    q, _ = O.quantize_symmetric([0.0, 1.0, -1.0])
    assert q[0] == 0


def test_rounding_is_nearest_half_away():  # symmetric.rs:216-231
    q, _ = O.quantize_symmetric([0.5, 1.0])
    assert q[1] == 127 and q[0] == 64


def test_clamp_prevents_i8_overflow():  # symmetric.rs:233-242
    q, _ = O.quantize_symmetric([100.0])
    assert q[0] == 127


def test_roundtrip_error_below_half_lsb():  # symmetric.rs:246-262
    vals = (np.arange(-64, 65).astype(F32) * F32(0.05)).astype(F32)
    q, s = O.quantize_symmetric(vals)
    rec = q.astype(F32) * s
    assert np.max(np.abs(vals - rec)) <= s / 2 + 1e-6


def test_clip_fraction():  # symmetric.rs:316-323
    q, _ = O.quantize_symmetric([-1.0, 0.0, 1.0])
    clip = np.mean((q == 127) | (q == -127))
    assert abs(clip - 2.0 / 3.0) < 0.01


# ---- quant/int8/per_channel.rs -----------------------------------------------

def test_per_channel_doctest():  # per_channel.rs:84-96
    data, scales = O.quantize_per_channel([1.0, -2.0, 3.0, 0.1, 0.2, 0.3], 2, 3)
    assert data.shape == (2, 3)
    assert abs(scales[0] - 3.0 / 127.0) < 1e-6
    assert abs(scales[1] - 0.3 / 127.0) < 1e-6


def test_each_row_scale():  # per_channel.rs:243-252
    _, s = O.quantize_per_channel([1.0, -2.0, 3.0, 0.5, 0.0, 0.25], 2, 3)
    assert abs(s[0] - 3.0 / 127.0) < 1e-5 and abs(s[1] - 0.5 / 127.0) < 1e-5


def test_zero_row_gets_scale_one():  # per_channel.rs:254-261
    d, s = O.quantize_per_channel(np.zeros(6, F32), 2, 3)
    assert s[0] == 1.0 and s[1] == 1.0 and np.all(d == 0)


def test_max_abs_element_maps_to_127():  # per_channel.rs:263-270
    d, _ = O.quantize_per_channel([-5.0, 1.0, 2.5, 5.0], 1, 4)
    assert d[0, 0] == -127 and d[0, 3] == 127


def test_rows_are_quantised_independently():  # per_channel.rs:274-289
    d, s = O.quantize_per_channel([0, 0, 127.0, 0, 0, 1.0], 2, 3)
    assert d[0, 2] == 127 and d[1, 2] == 127
    assert abs(s[0] - 1.0) < 1e-5 and abs(s[1] - 1.0 / 127.0) < 1e-5


def test_per_channel_roundtrip_half_lsb():  # per_channel.rs:293-312
    w = ar(0, 128, 0.03, -2.0)
    d, s = O.quantize_per_channel(w, 4, 32)
    for n in range(4):
        rec = d[n].astype(F32) * s[n]
        assert np.max(np.abs(w[n * 32:(n + 1) * 32] - rec)) <= s[n] / 2 + 1e-6


def test_per_channel_exactly_representable():  # per_channel.rs:389-401
    w = np.arange(0, 128).astype(F32)
    d, s = O.quantize_per_channel(w, 1, 128)
    assert s[0] == 1.0 and np.array_equal(d[0].astype(F32), w)


def test_per_channel_length_mismatch_is_error():  # per_channel.rs:99-105 panics
    with pytest.raises(O.OracleError):
        O.quantize_per_channel(np.zeros(5, F32), 2, 3)


# ---- ops/matmul/int8_avx2.rs (dot KATs) --------------------------------------

@pytest.mark.parametrize("dot", [O.dot_i8_avx2, O.dot_i8_scalar])
def test_dot_kats(dot):
    assert dot(np.zeros(0, np.int8), np.zeros(0, np.int8)) == 0          # :219-222
    assert dot([1, 2, 3], [4, 5, 6]) == 32                                 # :224-230
    assert dot([127] * 64, [1] * 64) == 8128                               # :252-258
    a = [1 if i % 2 == 0 else -1 for i in range(64)]
    assert dot(a, [2] * 64) == 0                                           # :260-268
    assert dot([-3] * 32, [-5] * 32) == 480                                # :270-276
    assert dot([127] * 4096, [1] * 4096) == 127 * 4096                     # :278-285


def wrap_i8(v):
    return np.asarray(v, dtype=np.int64).astype(np.uint8).view(np.int8)


def test_dot_matches_scalar_32_33_128():  # int8_avx2.rs:232-250, :287-297
    a32 = wrap_i8(np.arange(32) - 16)
    b32 = wrap_i8(np.arange(32) * 2 - 30)
    assert O.dot_i8_avx2(a32, b32) == O.dot_i8_scalar(a32, b32)
    a33 = wrap_i8(np.arange(33) * 3 - 50)
    b33 = wrap_i8(np.arange(33) * 5 - 80)
    assert O.dot_i8_avx2(a33, b33) == O.dot_i8_scalar(a33, b33)
    a = wrap_i8(np.arange(128) * 7 + 3 - 64)
    b = wrap_i8(np.arange(128) * 11 + 1 - 64)
    assert O.dot_i8_avx2(a, b) == O.dot_i8_scalar(a, b)
    ref = int(np.dot(a.astype(np.int64), b.astype(np.int64)))
    assert O.dot_i8_scalar(a, b) == ref


def test_avx2_path_is_taken():
    # The CPU baseline must run the AVX2 sequence, as on the reference's x86 CI.
    assert O.have_avx2()


# ---- ops/matmul/int8.rs --------------------------------------------------------

def _qw(w, n, k):
    return O.quantize_per_channel(w, n, k)


def test_output_shape_is_m_by_n():  # int8.rs:171-178
    d, s = _qw(ar(0, 64, 0.01, 0.0), 2, 32)
    out, *_ = O.matmul_int8_from_f32(np.full((3, 32), 0.5, F32), d, s)
    assert out.shape == (3, 2)


def test_zero_input_gives_zero_output():  # int8.rs:180-189
    d, s = _qw(ar(0, 128, 0.1, -6.0), 4, 32)
    out, *_ = O.matmul_int8_from_f32(np.zeros((2, 32), F32), d, s)
    assert np.all(np.abs(out) < 1e-6)


def test_zero_weights_give_zero_output():  # int8.rs:191-201
    d, s = _qw(np.zeros(64, F32), 2, 32)
    out, *_ = O.matmul_int8_from_f32(ar(0, 96, 0.1, -5.0).reshape(3, 32), d, s)
    assert np.all(np.abs(out) < 1e-4)


@pytest.mark.parametrize("case", [
    # int8.rs:205-221: [2,32] x [4,32]^T
    (ar(0, 128, 0.03, -2.0), 4, 32, ar(0, 64, 0.05, -1.6), 2),
    # int8.rs:223-238: [4,128] x [8,128]^T
    (ar(0, 1024, 0.01, -5.0), 8, 128, ar(0, 512, 0.02, -5.0), 4),
])
def test_matches_naive_within_quant_error(case):
    w, n, k, x, m = case
    d, s = _qw(w, n, k)
    out, *_ = O.matmul_int8_from_f32(x.reshape(m, k), d, s)
    assert max_rel_err(out, naive(x.reshape(m, k), w.reshape(n, k))) < 0.02


def test_single_row_single_output_channel():  # int8.rs:240-252
    d, s = _qw(np.ones(32, F32), 1, 32)
    out, *_ = O.matmul_int8_from_f32(np.full((1, 32), 0.5, F32), d, s)
    assert out.shape == (1, 1) and abs(out[0, 0] - 16.0) < 0.5


def test_matmul_int8_direct_matches_wrapper():  # int8.rs:256-270
    w = ar(0, 96, 0.04, -2.0)
    x = ar(0, 64, 0.06, -2.0)
    d, s = _qw(w, 3, 32)
    aq, sa = O.quantize_symmetric(x)
    via_wrapper, *_ = O.matmul_int8_from_f32(x.reshape(2, 32), d, s)
    via_direct = O.matmul_int8(aq, sa, d, s, 2)
    assert np.array_equal(via_wrapper.view(np.uint32), via_direct.view(np.uint32))


def test_non_contiguous_input_handled():  # int8.rs:274-288
    t = ar(0, 128, 0.05, -3.0).reshape(64, 2)
    x_nc = t.T                                   # [2,64] non-contiguous view
    d, s = _qw(ar(0, 192, 0.02, -2.0), 3, 64)
    a, *_ = O.matmul_int8_from_f32(x_nc, d, s)   # binding makes it contiguous
    b, *_ = O.matmul_int8_from_f32(np.ascontiguousarray(x_nc), d, s)
    assert np.array_equal(a, b)


def test_error_on_non_2d_input():  # int8.rs:292-301
    d, s = _qw(np.zeros(32, F32), 1, 32)
    with pytest.raises(O.OracleError) as e:
        O.matmul_int8_from_f32(np.ones((2, 4, 8), F32), d, s)
    assert e.value.kind == "InvalidShape"


def test_error_on_k_mismatch():  # int8.rs:303-318
    d, s = _qw(np.zeros(64, F32), 2, 32)
    O.matmul_int8_from_f32(np.ones((2, 32), F32), d, s)
    d2, s2 = _qw(np.zeros(64, F32), 1, 64)
    with pytest.raises(O.OracleError) as e:
        O.matmul_int8_from_f32(np.ones((1, 32), F32), d2, s2)
    assert e.value.kind == "ShapeMismatch"


def test_error_on_bad_act_q_length():  # int8.rs:320-329
    d, s = _qw(np.zeros(64, F32), 2, 32)
    with pytest.raises(O.OracleError) as e:
        O.matmul_int8(np.zeros(10, np.int8), 1.0, d, s, 1)
    assert e.value.kind == "InvalidShape"


def test_no_overflow_large_k():  # int8.rs:333-353
    k = 4096
    d, s = _qw(np.full(k, 127.0, F32), 1, k)
    out, _, _, acc = O.matmul_int8_from_f32(np.full((1, k), 127.0, F32), d, s)
    assert acc[0, 0] == 127 * 127 * 4096
    exp = 127.0 * 127.0 * k
    assert abs(out[0, 0] - exp) / exp < 0.02


# ---- ops/matmul/int8_avx2.rs + parallel.rs (bit identity) --------------------

@pytest.mark.parametrize("k,n,m,wmul,wadd,xmul,xadd", [
    (32, 4, 2, 0.03, -2.0, 0.05, -1.6),      # int8_avx2.rs:323-336
    (128, 8, 4, 0.01, -5.0, 0.02, -5.0),     # int8_avx2.rs:338-353
    (64, 4, 4, 0.03, -2.0, 0.05, -1.6),      # parallel.rs:380-393
    (256, 8, 16, 0.01, -5.0, 0.02, -5.0),    # parallel.rs:395-408
    (128, 6, 1, 0.04, -2.0, 0.06, -2.0),     # parallel.rs:410-423
])
def test_simd_and_parallel_bit_identical_to_scalar(k, n, m, wmul, wadd, xmul, xadd):
    d, s = _qw(ar(0, n * k, wmul, wadd), n, k)
    aq, sa = O.quantize_symmetric(ar(0, m * k, xmul, xadd))
    scalar = O.matmul_int8(aq, sa, d, s, m)
    avx2 = O.matmul_int8_avx2(aq, sa, d, s, m)
    par, used = O.matmul_int8_parallel(aq, sa, d, s, m)
    assert np.array_equal(scalar.view(np.uint32), avx2.view(np.uint32))
    assert np.array_equal(scalar.view(np.uint32), par.view(np.uint32))
    assert 1 <= used <= m


def test_parallel_zero_input_and_no_cross_row():  # parallel.rs:425-457
    k, n, m = 64, 4, 3
    d, s = _qw(ar(0, n * k, 0.1, -6.0), n, k)
    out, _ = O.matmul_int8_parallel(np.zeros(m * k, np.int8), 1.0, d, s, m)
    assert np.all(np.abs(out) < 1e-6)
    k, n, m = 64, 3, 8
    w = np.array([(i % 7) * 0.1 for i in range(n * k)], F32)
    d, s = _qw(w, n, k)
    x = np.zeros((m, k), F32)
    x[3] = (np.arange(k).astype(F32) * F32(0.1) + F32(0.5)).astype(F32)
    aq, sa = O.quantize_symmetric(x)
    par, _ = O.matmul_int8_parallel(aq, sa, d, s, m)
    assert np.array_equal(par, O.matmul_int8(aq, sa, d, s, m))
    assert np.all(par[np.arange(m) != 3] == 0)


def test_parallel_error_on_bad_act_q_length():  # parallel.rs:459-468
    d, s = _qw(np.zeros(64, F32), 2, 32)
    with pytest.raises(O.OracleError):
        O.matmul_int8_parallel(np.zeros(10, np.int8), 1.0, d, s, 1)


# ---- gguf/quantization.rs (f16) -------------------------------------------------

def test_f16_special_values():  # quantization.rs:528-545
    assert O.f16_to_f32(0x0000) == 0.0
    assert math.copysign(1.0, O.f16_to_f32(0x8000)) < 0
    assert abs(O.f16_to_f32(0x3C00) - 1.0) < 1e-6
    assert O.f16_to_f32(0x7C00) == math.inf
    assert O.f16_to_f32(0xFC00) == -math.inf
    assert math.isnan(O.f16_to_f32(0x7C01))


def test_f16_roundtrip():  # quantization.rs:516-526
    for v in [0.0, 1.0, -1.0, 0.5, 2.0, 100.0, -0.125, 65504.0]:
        back = O.f16_to_f32(O.f32_to_f16(v))
        assert abs(v - back) < abs(v) * 0.001 + 0.001


def test_q4_0_quant_extraction():  # quantization.rs:589-611 (interleaved order)
    blk = np.zeros(18, np.uint8)
    d = O.f32_to_f16(1.0)
    blk[0], blk[1] = d & 0xFF, d >> 8
    blk[2:10] = [0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE]
    v = O.dequantize_q4_0(blk)
    assert list(v[:4]) == [-8.0, -7.0, -6.0, -5.0]


def test_q8_0_dequantize_kat():  # quantization.rs:632-647
    blk = np.zeros(34, np.uint8)
    d = O.f32_to_f16(0.5)
    blk[0], blk[1] = d & 0xFF, d >> 8
    qs = [0, 1, 2, 3, 4, 5, 6, 7, -8, -7, -6, -5, -4, -3, -2, -1] + [0] * 16
    blk[2:] = np.array(qs, np.int8).view(np.uint8)
    v = O.dequantize_q8_0(blk)
    assert abs(v[0]) < 0.01 and abs(v[1] - 0.5) < 0.01 and abs(v[8] + 4.0) < 0.01


# ---- gguf/dequant.rs --------------------------------------------------------------

def _blk(d_bits, qbytes):
    return np.concatenate([np.array([d_bits & 0xFF, d_bits >> 8], np.uint8),
                           np.asarray(qbytes, np.int64).astype(np.uint8)])


def test_q8_0_doctest_and_single_block():  # dequant.rs:88-101, :761-785
    v = O.dequantize_q8_0(_blk(O.f32_to_f16(0.5), [i * 2 for i in range(32)]))
    assert len(v) == 32 and abs(v[0]) < 1e-3 and abs(v[1] - 1.0) < 1e-3
    v = O.dequantize_q8_0(_blk(0x3C00, range(32)))
    assert np.allclose(v, np.arange(32), atol=1e-2)


def test_q8_0_negative_and_multi_block():  # dequant.rs:786-834
    v = O.dequantize_q8_0(_blk(0x3800, range(-16, 16)))
    assert abs(v[0] + 8.0) < 1e-2 and abs(v[16]) < 1e-2 and abs(v[31] - 7.5) < 1e-2
    data = np.concatenate([_blk(0x3C00, [0] * 32), _blk(0x4000, [1] * 32)])
    v = O.dequantize_q8_0(data)
    assert np.all(v[:32] == 0) and np.all(v[32:] == 2.0)


def test_q8_0_invalid_and_empty():  # dequant.rs:836-852
    with pytest.raises(O.OracleError):
        O.dequantize_q8_0(np.zeros(35, np.uint8))
    assert O.dequantize_q8_0(np.zeros(0, np.uint8)).size == 0


def test_create_q8_0_block_roundtrips():  # dequant.rs:943-983
    vals = np.arange(32).astype(F32)
    assert np.max(np.abs(O.dequantize_q8_0(O.create_q8_0_block(vals)) - vals)) < 0.5
    z = O.create_q8_0_block(np.zeros(32, F32))
    assert np.all(O.dequantize_q8_0(z) == 0.0)
    vals = np.arange(-16, 16).astype(F32)
    assert np.max(np.abs(O.dequantize_q8_0(O.create_q8_0_block(vals)) - vals)) < 0.5


def test_q8_0_large():  # dequant.rs:995-1021
    data = []
    for b in range(100):
        data.append(_blk(O.f32_to_f16(F32((b + 1) * 0.01)), range(32)))
    v = O.dequantize_q8_0(np.concatenate(data))
    assert v.size == 3200 and abs(v[0]) < 0.01 and abs(v[1] - 0.01) < 0.01


def test_q4_0_doctest():  # dequant.rs:453-470
    blk = np.zeros(18, np.uint8)
    blk[1] = 0x3C
    blk[2] = 0x98
    v = O.dequantize_q4_0(blk)
    assert len(v) == 32 and abs(v[0]) < 0.1 and abs(v[1] - 1.0) < 0.1


def test_q4_0_dequant_kats():  # dequant.rs:1032-1122
    v = O.dequantize_q4_0(_blk(0x3C00, [0x98] * 16))
    assert np.array_equal(v, np.tile([0.0, 1.0], 16).astype(F32))
    v = O.dequantize_q4_0(_blk(0x4000, [0xF0] * 16))
    assert v[0] == -16.0 and v[1] == 14.0
    data = np.concatenate([_blk(0x3C00, [0x88] * 16), _blk(0x3800, [0xE4] * 16)])
    v = O.dequantize_q4_0(data)
    assert np.all(v[:32] == 0)
    assert np.array_equal(v[32:], np.tile([-2.0, 3.0], 16).astype(F32))


def test_q4_0_invalid_and_empty():  # dequant.rs:1124-1140
    with pytest.raises(O.OracleError):
        O.dequantize_q4_0(np.zeros(19, np.uint8))
    assert O.dequantize_q4_0(np.zeros(0, np.uint8)).size == 0


def test_q4_0_block_sequential_pattern():  # dequant.rs:1168-1194
    blk = np.zeros(18, np.uint8)
    blk[1] = 0x3C
    for i in range(16):
        blk[2 + i] = ((i * 2) % 16) | (((i * 2 + 1) % 16) << 4)
    v = O.dequantize_q4_0(blk)
    assert np.array_equal(v, np.array([(i % 16) - 8 for i in range(32)], F32))


def test_create_q4_0_block_kats():  # dequant.rs:1245-1289
    vals = np.arange(-8, 24).astype(F32)
    assert np.max(np.abs(O.dequantize_q4_0(O.create_q4_0_block(vals)) - vals)) < 3.0
    z = O.create_q4_0_block(np.zeros(32, F32))
    assert np.all(z[2:] == 0x88) and np.all(O.dequantize_q4_0(z) == 0)
    vals = ((np.arange(32) - 16) * 0.5).astype(F32)
    assert np.max(np.abs(O.dequantize_q4_0(O.create_q4_0_block(vals)) - vals)) < 2.0


# ---- ops/matmul/q8_direct.rs -------------------------------------------------------

def _q8w(w, n, k):
    return O.quantize_q8_0(np.asarray(w, F32).reshape(n, k))


def test_q8_from_raw_bytes_validation():  # q8_direct.rs:314-337
    O.q8_0_check_raw(2 * 34, 2, 32)
    with pytest.raises(O.OracleError):
        O.q8_0_check_raw(34, 1, 31)
    with pytest.raises(O.OracleError):
        O.q8_0_check_raw(33, 1, 32)
    O.q8_0_check_raw(0, 0, 32)


def test_q8_output_shape_and_zero_cases():  # q8_direct.rs:355-387
    raw = _q8w(ar(0, 128, 0.01, 0.0), 4, 32)
    assert O.matmul_q8_0_direct(np.full((3, 32), 0.5, F32), raw, 4, 32).shape == (3, 4)
    raw = _q8w(ar(0, 128, 0.1, -6.0), 4, 32)
    assert np.all(np.abs(O.matmul_q8_0_direct(np.zeros((2, 32), F32), raw, 4, 32)) < 1e-5)
    raw = _q8w(np.zeros(64, F32), 2, 32)
    out = O.matmul_q8_0_direct(ar(0, 64, 0.1, -3.0).reshape(2, 32), raw, 2, 32)
    assert np.all(np.abs(out) < 1e-4)


@pytest.mark.parametrize("case", [
    (ar(0, 128, 0.03, -2.0), 4, 32, ar(0, 64, 0.05, -1.6), 2),       # :391-411
    (ar(0, 768, 0.01, -3.84), 6, 128, ar(0, 384, 0.02, -3.84), 3),   # :413-432
])
def test_q8_matches_dequant_naive(case):
    w, n, k, x, m = case
    raw = _q8w(w, n, k)
    wd = O.dequantize_q8_0(raw).reshape(n, k)
    out = O.matmul_q8_0_direct(x.reshape(m, k), raw, n, k)
    assert max_rel_err(out, naive(x.reshape(m, k), wd)) < 0.03


def test_q8_single_dot():  # q8_direct.rs:434-445
    raw = _q8w(np.ones(32, F32), 1, 32)
    out = O.matmul_q8_0_direct(np.full((1, 32), 0.5, F32), raw, 1, 32)
    assert out.shape == (1, 1) and abs(out[0, 0] - 16.0) < 1.0


def test_q8_errors():  # q8_direct.rs:468-493
    raw = _q8w(np.zeros(32, F32), 1, 32)
    with pytest.raises(O.OracleError) as e:
        O.matmul_q8_0_direct(np.ones((2, 4, 8), F32), raw, 1, 32)
    assert e.value.kind == "InvalidShape"
    raw2 = _q8w(np.zeros(128, F32), 2, 64)
    with pytest.raises(O.OracleError) as e:
        O.matmul_q8_0_direct(np.ones((1, 32), F32), raw2, 2, 64)
    assert e.value.kind == "ShapeMismatch"


def test_q8_no_nan_or_inf():  # q8_direct.rs:497-509
    raw = _q8w(ar(0, 1024, 0.01, -5.12), 32, 32)
    out = O.matmul_q8_0_direct(ar(0, 512, 0.02, -5.12).reshape(16, 32), raw, 32, 32)
    assert np.all(np.isfinite(out))


# ---- ops/matmul/q4_0.rs --------------------------------------------------------------

def _q4w(rows):
    return np.concatenate([O.create_q4_0_block(c)
                           for r in rows for c in np.asarray(r, F32).reshape(-1, 32)])


@pytest.mark.parametrize("n,k,m,wfun,xfun", [
    (1, 32, 1, lambda n, k: k * 0.1 - 1.5, lambda i: i * 0.05),                  # :214-237
    (4, 64, 3, lambda n, k: (n * 64 + k) * 0.02 - 0.5, lambda i: i * 0.01),      # :239-267
    (8, 128, 4, lambda n, k: (n * 128 + k) * 0.01 - 0.5, lambda i: i * 0.005),   # :359-390
])
def test_q4_matches_naive_on_dequantized(n, k, m, wfun, xfun):
    rows = [[F32(wfun(r, c)) for c in range(k)] for r in range(n)]
    raw = _q4w(rows)
    wd = O.dequantize_q4_0(raw).reshape(n, k)
    x = np.array([F32(xfun(i)) for i in range(m * k)], F32).reshape(m, k)
    out = O.matmul_q4_0_dequant(x, raw, n, k)
    ref = naive(x, wd)
    assert out.shape == (m, n)
    assert np.all(np.abs(out - ref) < 1e-5)


def test_q4_zero_input_and_shape():  # q4_0.rs:269-280, :349-357
    raw = _q4w([np.ones(32, F32)])
    out = O.matmul_q4_0_dequant(np.zeros((2, 32), F32), raw, 1, 32)
    assert out.shape == (2, 1) and np.all(np.abs(out) < 1e-5)
    raw = _q4w([np.zeros(128, F32)] * 8)
    assert O.matmul_q4_0_dequant(np.zeros((5, 128), F32), raw, 8, 128).shape == (5, 8)


def test_q4_error_order():  # q4_0.rs:307-347
    dummy = np.zeros(18, np.uint8)
    with pytest.raises(O.OracleError) as e:
        O.matmul_q4_0_dequant(np.ones((2, 4, 8), F32), dummy, 1, 32)
    assert e.value.kind == "InvalidShape"
    with pytest.raises(O.OracleError) as e:
        O.matmul_q4_0_dequant(np.ones((1, 33), F32), dummy, 1, 33)
    assert e.value.kind == "InvalidShape"
    with pytest.raises(O.OracleError) as e:      # K mismatch is checked before K%32
        O.matmul_q4_0_dequant(np.ones((1, 32), F32), dummy, 1, 64)
    assert e.value.kind == "ShapeMismatch"
    with pytest.raises(O.OracleError) as e:
        O.matmul_q4_0_dequant(np.ones((1, 32), F32), np.zeros(20, np.uint8), 1, 32)
    assert e.value.kind == "InvalidShape"

"""GPU parity of the W4A8 extension (include/mri_qmatmul.h,
mri_matmul_q4_0_w4a8) against the oracle's orc_matmul_q4_0_w4a8, which is
pinned to matmul_q8_0_direct on the expanded blocks
(tests/test_oracle_closed_form.py).  Block dots and activation scales must
be bit-identical, in both nibble orders; f32 outputs are within
1e-5 * max(|ref|, sum_b |t_b|) of the block-ordered sum where the kernel
reorders it (the decode GEMV, M <= 4, adds per-wave partial sums; the
LDS-tiled GEMM, M >= 128 and M * N > 2^20 without block dots, folds with
FMAs) and bit-identical elsewhere."""
import sys

import numpy as np
import pytest

import closed_form as CF
import oracle_lib as O
from gpu_util import (q8_gemm_range, F32, assert_bits_equal, assert_q8_close, bits, dev, empty, host,
                      q8_terms_abs_sum, synth_q4_0, torch)

pytestmark = pytest.mark.gpu


def mri():
    import mri_qmatmul
    return mri_qmatmul


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


W4A8_SHAPES = [
    (1, 16, 32), (1, 16, 256), (1, 50, 96), (1, 1024, 4096), (1, 11008, 4096),
    (1, 64, 11008), (1, 32000 // 8, 4096), (2, 33, 256), (3, 48, 1024), (4, 64, 4096),
    (5, 40, 512), (9, 24, 1024), (16, 272, 4096), (33, 48, 256), (100, 40, 1024),
    (2, 32, 16384), (1, 48, 20480), (1, 8200, 992), (4, 11008, 4096),
    # prefill sizes on the LDS-tiled GEMM (128 rows and more than 2^20 outputs)
    (128, 8200, 512), (300, 4100, 1024),
]


@pytest.mark.parametrize("m,n,k", W4A8_SHAPES)
@pytest.mark.parametrize("order", [0, 1])
def test_w4a8_parity(m, n, k, order):
    say(f"matmul_q4_0_w4a8 m={m} n={n} k={k} order={order}")
    t = torch()
    rng = np.random.default_rng(m * 7 + n + k + order)
    raw = synth_q4_0(rng, n, k)
    x = rng.standard_normal((m, k)).astype(F32)
    out0, bd0, sa0 = O.matmul_q4_0_w4a8(x, raw, n, k, order, want_block_dots=True)
    w = mri().Q4Matrix.from_raw_bytes(raw, n, k, order)
    out = empty((m, n), t.float32)
    bd = empty((m, n, k // 32), t.int32)
    sa = empty(m, t.float32)
    mri().matmul_q4_0_w4a8(dev(x), w, out, bd, sa)
    assert np.array_equal(bits(host(sa)), bits(sa0))
    assert np.array_equal(host(bd), bd0)
    d, _ = CF.q4_0_split(raw, n, k)
    assert_q8_close(host(out), out0, q8_terms_abs_sum(bd0, sa0, d), "w4a8 out")
    if m > 4:  # the kernels above four rows keep the reference's order
        assert_bits_equal(host(out), out0, "w4a8 out")
    if q8_gemm_range(m, n):  # without block dots: the LDS-tiled GEMM, within the contract
        out3 = empty((m, n), t.float32)
        mri().matmul_q4_0_w4a8(dev(x), w, out3)
        assert_q8_close(host(out3), out0, q8_terms_abs_sum(bd0, sa0, d), "w4a8 out (gemm)")
        return
    out2 = empty((m, n), t.float32)          # without the debug outputs
    sa2 = empty(m, t.float32)
    mri().matmul_q4_0_w4a8(dev(x), w, out2, act_scales_out=sa2)
    assert np.array_equal(bits(host(sa2)), bits(sa0))
    assert_bits_equal(host(out2), host(out), "w4a8 out (no debug outputs)")


@pytest.mark.parametrize("m,n,k", [(1, 11008, 4096), (1, 50, 96), (3, 48, 1024),
                                   (4, 64, 4096), (9, 24, 1024), (40, 272, 4096),
                                   (256, 8192, 256), (200, 6000, 4096), (512, 4096, 1024)])
def test_w4a8_equals_q8_0_on_expanded_blocks(m, n, k):
    """W4A8 runs the Q8_0 kernels with a 4-bit B operand, so its outputs
    equal matmul_q8_0_direct's on the same blocks expanded to Q8_0 (quants
    nibble - 8, the same f16 scale bits) bit for bit, at every row count:
    the GEMV's wave order at 1-4 rows, the skinny kernel's block order, and
    the LDS-tiled GEMM from 128 rows and more than 2^20 outputs (16 * dot
    folded with d / 16, K split included at 200 x 6000 x 4096)."""
    say(f"w4a8 vs q8_0 on expanded blocks m={m} n={n} k={k}")
    t = torch()
    rng = np.random.default_rng(m * 5 + n + k)
    raw = synth_q4_0(rng, n, k)
    x = rng.standard_normal((m, k)).astype(F32)
    w4 = mri().Q4Matrix.from_raw_bytes(raw, n, k, 0)
    w8 = mri().Q8Matrix.from_raw_bytes(CF.q4_0_to_q8_0(raw, n, k), n, k)
    o4, o8 = empty((m, n), t.float32), empty((m, n), t.float32)
    mri().matmul_q4_0_w4a8(dev(x), w4, o4)
    mri().matmul_q8_0_direct(dev(x), w8, o8)
    assert_bits_equal(host(o4), host(o8), "w4a8 vs q8_0 on the expanded blocks")


def test_w4a8_ggml_file_order_matches_reference_order():
    """The same weights uploaded from GGML-order bytes and from
    interleaved-order bytes give the same outputs."""
    t = torch()
    rng = np.random.default_rng(3)
    n, k = 96, 2048
    raw = synth_q4_0(rng, n, k)
    x = dev(rng.standard_normal((1, k)).astype(F32))
    a, b = empty((1, n), t.float32), empty((1, n), t.float32)
    mri().matmul_q4_0_w4a8(x, mri().Q4Matrix.from_raw_bytes(raw, n, k, 0), a)
    gg = CF.q4_0_interleaved_to_ggml(raw)
    mri().matmul_q4_0_w4a8(x, mri().Q4Matrix.from_raw_device(dev(gg), n, k, 1), b)
    assert_bits_equal(host(b), host(a), "ggml order")


def test_w4a8_unfused_and_device_upload():
    """x at a 4-byte aligned address takes the quantize kernel + GEMV path;
    weights uploaded from a device buffer."""
    t = torch()
    rng = np.random.default_rng(5)
    n, k = 80, 4096
    raw = synth_q4_0(rng, n, k)
    x = rng.standard_normal((1, k)).astype(F32)
    buf = dev(np.concatenate([np.zeros(1, F32), x.ravel()]))
    xu = buf[1:].view(1, k)
    assert xu.data_ptr() % 16 != 0
    w = mri().Q4Matrix.from_raw_device(dev(raw), n, k)
    out = empty((1, n), t.float32)
    mri().matmul_q4_0_w4a8(xu, w, out)
    out0, bd0, sa0 = O.matmul_q4_0_w4a8(x, raw, n, k, want_block_dots=True)
    d, _ = CF.q4_0_split(raw, n, k)
    assert_q8_close(host(out), out0, q8_terms_abs_sum(bd0, sa0, d), "w4a8 unfused")


def test_w4a8_errors():
    t = torch()
    M = mri()
    rng = np.random.default_rng(1)
    w = M.Q4Matrix.from_raw_bytes(synth_q4_0(rng, 16, 64), 16, 64)
    out = empty((2, 16), t.float32)
    with pytest.raises(M.MriError) as e:
        M.matmul_q4_0_w4a8(dev(np.zeros((2, 32), F32)), w, out)
    assert e.value.kind == "ShapeMismatch"
    with pytest.raises(M.MriError) as e:
        M.matmul_q4_0_w4a8(dev(np.zeros((2, 64), F32)), w, out, shape=(2, 8, 8))
    assert e.value.kind == "InvalidShape"
    assert M.Q4Matrix.from_raw_bytes(np.zeros(18 * 16, np.uint8), 16, 32).device_bytes > 0

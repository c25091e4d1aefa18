"""Helpers for GPU tests: numpy <-> torch device tensors, seeded data."""
import numpy as np

F32 = np.float32


def torch():
    import torch as _t
    assert _t.cuda.is_available(), "GPU tests need a visible MI355X"
    return _t


def dev(a):
    t = torch()
    return t.from_numpy(np.ascontiguousarray(a)).to("cuda")


def empty(shape, dtype):
    t = torch()
    return t.empty(shape, dtype=dtype, device="cuda")


def host(t):
    torch().cuda.synchronize()
    return t.cpu().numpy()


def bits(a):
    return np.asarray(a, F32).view(np.uint32)


def assert_bits_equal(got, exp, what=""):
    got = np.asarray(got, F32)
    exp = np.asarray(exp, F32)
    assert got.shape == exp.shape, (what, got.shape, exp.shape)
    g, e = bits(got), bits(exp)
    bad = np.flatnonzero(g.ravel() != e.ravel())
    if bad.size:
        i = bad[0]
        raise AssertionError(
            f"{what}: {bad.size} of {g.size} f32 values differ bitwise; first at "
            f"{np.unravel_index(i, got.shape)}: got {got.ravel()[i]!r} "
            f"expected {exp.ravel()[i]!r}")


def synth_q8_0(rng, n, k, with_min=False):
    """Q8_0 raw blocks: quants uniform in [-127,127] (optionally some -128),
    f16 scales ~U(0.001, 0.01)."""
    import closed_form as CF
    q = rng.integers(-127, 128, (n, k)).astype(np.int8)
    if with_min:
        q[rng.random((n, k)) < 0.02] = -128
    d = rng.uniform(0.001, 0.01, (n, k // 32)).astype(np.float16).view(np.uint16)
    return CF.q8_0_pack(d, q)


def synth_q4_0(rng, n, k):
    raw = np.empty((n, k // 32, 18), np.uint8)
    raw[:, :, 2:] = rng.integers(0, 256, (n, k // 32, 16))
    d = rng.uniform(0.001, 0.05, (n, k // 32)).astype(np.float16).view(np.uint16)
    raw[:, :, 0] = d & 0xFF
    raw[:, :, 1] = d >> 8
    return raw.ravel()


def synth_int8_weights(rng, n, k):
    """Per-channel weights as the reference builds them: N(0, 0.02) f32
    quantized per row (quantize_per_channel), via the oracle."""
    import oracle_lib as O
    w = (rng.standard_normal((n, k)) * 0.02).astype(F32)
    return O.quantize_per_channel(w, n, k)


def q8_terms_abs_sum(bd, sa, d):
    """sum_b |t_b| in float64 for the block terms t_b = ((f32)dot_b * s_a) * d_b
    of matmul_q8_0_direct (q8_direct.rs:281): bd [M, N, nb] block dots,
    sa [M] activation scales, d [N, nb] block scales; returns [M, N]."""
    bd = np.abs(np.asarray(bd, np.float64))
    d = np.abs(np.asarray(d, np.float64))
    sa = np.abs(np.asarray(sa, np.float64))
    return np.einsum("mnb,nb->mn", bd, d) * sa[:, None]


def q8_gemm_range(m, n):
    """Shapes at which matmul_q8_0_direct without block dots runs the
    LDS-tiled prefill GEMM (an FMA fold, s_a applied once: within the
    contract, not in the reference's order): m >= 128 and m * n > 2^20."""
    return m >= 128 and m * n > (1 << 20)


def assert_q8_close(got, exp, terms_abs, what="", rel=1e-5):
    """The Q8_0 f32 contract: |got - exp| <= rel * max(|exp|, sum_b |t_b|)
    per element (the block terms may be added in another order than the
    reference's left-to-right sum)."""
    got = np.asarray(got, np.float64)
    exp = np.asarray(exp, np.float64)
    assert got.shape == exp.shape, (what, got.shape, exp.shape)
    bound = rel * np.maximum(np.abs(exp), terms_abs)
    bad = np.flatnonzero((np.abs(got - exp) > bound).ravel())
    if bad.size:
        i = bad[0]
        raise AssertionError(
            f"{what}: {bad.size} of {got.size} values outside {rel} * max(|ref|, sum|t_b|); "
            f"first at {np.unravel_index(i, got.shape)}: got {got.ravel()[i]!r} expected "
            f"{exp.ravel()[i]!r} (bound {bound.ravel()[i]:.3g})")


_POOL = None


def pool():
    """Host threads for the oracle at full sizes (ctypes releases the GIL)."""
    global _POOL
    if _POOL is None:
        import os
        from concurrent.futures import ThreadPoolExecutor
        _POOL = ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 4))
    return _POOL


def q8_oracle_sliced(x, raw, n, k, slice_rows=256):
    """The oracle's matmul_q8_0_direct over slices of the weight rows, run on
    host threads (each input row is quantized on its own, so the slices are
    independent and the result equals one call's), with the contract's
    sum_b |t_b| of every output computed from each slice's block dots.
    Returns (out [M, N] f32, terms_abs [M, N] f64)."""
    import closed_form as CF
    import oracle_lib as O
    x = np.ascontiguousarray(x, F32)
    m = x.shape[0]
    row = (k // 32) * 34
    out = np.empty((m, n), F32)
    terms = np.empty((m, n), np.float64)
    cuts = list(range(0, n, slice_rows)) + [n]

    def run(i):
        a, b = cuts[i], cuts[i + 1]
        part = raw[a * row:b * row]
        o, bd, sa = O.matmul_q8_0_direct(x, part, b - a, k, want_block_dots=True)
        d, _ = CF.q8_0_split(part, b - a, k)
        out[:, a:b] = o
        terms[:, a:b] = q8_terms_abs_sum(bd, sa, d)

    list(pool().map(run, range(len(cuts) - 1)))
    return out, terms

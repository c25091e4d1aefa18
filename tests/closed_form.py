"""Independent numpy formulations used to pin the oracle and the GPU path.

These are deliberately written differently from the oracle's C loops:
integer accumulators come from an int64 matrix product, rounding uses an
explicit half-away-from-zero construction (numpy's ``np.round`` is
half-to-even and would be wrong), f16 decoding uses numpy's IEEE float16,
and ordered f32 sums are evaluated with vectorised float32 adds across the
output dimension, one block (or element) at a time.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32


def round_half_away(y: np.ndarray) -> np.ndarray:
    """Rust f32::round: ties away from zero.  ``y - trunc(y)`` is exact for
    every finite float32."""
    y = np.asarray(y, dtype=F32)
    t = np.trunc(y)
    frac = np.abs(y - t)
    return (t + np.sign(y) * (frac >= F32(0.5))).astype(F32)


def sat_i8(r: np.ndarray, lo: float, hi: float) -> np.ndarray:
    """clamp(lo, hi) followed by Rust's saturating `as i8` (NaN -> 0)."""
    r = np.asarray(r, dtype=F32)
    out = np.where(np.isnan(r), F32(0), np.clip(r, F32(lo), F32(hi)))
    return out.astype(np.int8)


def max_abs(x: np.ndarray) -> F32:
    """fold(0.0, f32::max) of |x|: NaNs ignored (np.nanmax), 0 for empty."""
    x = np.abs(np.asarray(x, dtype=F32))
    if x.size == 0 or np.all(np.isnan(x)):
        return F32(0)
    return F32(max(F32(0), np.nanmax(x)))


def quantize_symmetric(x: np.ndarray):
    x = np.asarray(x, dtype=F32).ravel()
    ma = max_abs(x)
    scale = F32(1.0) if ma == 0 else F32(ma / F32(127.0))
    inv = F32(F32(1.0) / scale)
    with np.errstate(invalid="ignore", over="ignore"):
        q = sat_i8(round_half_away(x * inv), -127, 127)
    return q, scale


def quantize_rows(x: np.ndarray):
    x = np.asarray(x, dtype=F32)
    qs, ss = [], []
    for row in x:
        q, s = quantize_symmetric(row)
        qs.append(q)
        ss.append(s)
    return np.stack(qs).reshape(x.shape), np.array(ss, dtype=F32)


def quantize_per_channel(w: np.ndarray):
    w = np.asarray(w, dtype=F32)
    data = np.empty(w.shape, np.int8)
    scales = np.empty(w.shape[0], F32)
    for n in range(w.shape[0]):
        data[n], scales[n] = quantize_symmetric(w[n])
    return data, scales


def int_matmul(a_q: np.ndarray, w_q: np.ndarray) -> np.ndarray:
    """[M,K] x [N,K]^T in int64 (exact), returned as int64."""
    return a_q.astype(np.int64) @ w_q.astype(np.int64).T


def epilogue(acc: np.ndarray, s_a, s_w: np.ndarray) -> np.ndarray:
    """((f32)acc * s_a) * s_w with float32 RNE rounding at each step.
    ``s_a`` is a scalar or a per-row [M] array."""
    s_a = np.asarray(s_a, dtype=F32)
    if s_a.ndim == 1:
        s_a = s_a[:, None]
    t = acc.astype(F32) * s_a
    return (t * np.asarray(s_w, dtype=F32)[None, :]).astype(F32)


def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(F32)


def q8_0_split(raw: np.ndarray, n_out: int, k_in: int):
    """Raw Q8_0 bytes -> (d f32 [N, K/32], quants int8 [N, K])."""
    nb = k_in // 32
    blk = np.asarray(raw, dtype=np.uint8).reshape(n_out, nb, 34)
    d_bits = blk[:, :, 0].astype(np.uint16) | (blk[:, :, 1].astype(np.uint16) << 8)
    q = blk[:, :, 2:].view(np.int8).reshape(n_out, k_in)
    return f16_bits_to_f32(d_bits), q


def q8_0_pack(d_bits: np.ndarray, q: np.ndarray) -> np.ndarray:
    """(f16 bits [N, K/32], int8 [N, K]) -> raw 34-byte Q8_0 blocks."""
    n, k = q.shape
    nb = k // 32
    blk = np.empty((n, nb, 34), np.uint8)
    d_bits = np.asarray(d_bits, dtype=np.uint16)
    blk[:, :, 0] = (d_bits & 0xFF).astype(np.uint8)
    blk[:, :, 1] = (d_bits >> 8).astype(np.uint8)
    blk[:, :, 2:] = q.reshape(n, nb, 32).view(np.uint8)
    return blk.ravel()


def q8_0_direct(x: np.ndarray, raw: np.ndarray, n_out: int, k_in: int):
    """matmul_q8_0_direct: returns (out, block_dots int64 [M,N,nb], s_a)."""
    x = np.asarray(x, dtype=F32)
    m = x.shape[0]
    nb = k_in // 32
    d, wq = q8_0_split(raw, n_out, k_in)
    aq, sa = quantize_rows(x)
    a3 = aq.reshape(m, nb, 32).astype(np.int64)
    w3 = wq.reshape(n_out, nb, 32).astype(np.int64)
    dots = np.einsum("mbk,nbk->mnb", a3, w3)
    out = np.zeros((m, n_out), F32)
    for b in range(nb):                      # block order, float32 adds
        t = dots[:, :, b].astype(F32) * sa[:, None]
        t = (t * d[None, :, b]).astype(F32)
        out = (out + t).astype(F32)
    return out, dots, sa


def q4_0_split(raw: np.ndarray, n_out: int, k: int):
    """Raw Q4_0 bytes -> (d f32 [N, K/32], q int [N, K] in [-8,7]) with the
    reference's interleaved nibble order (low nibble = even element)."""
    nb = k // 32
    blk = np.asarray(raw, dtype=np.uint8).reshape(n_out, nb, 18)
    d_bits = blk[:, :, 0].astype(np.uint16) | (blk[:, :, 1].astype(np.uint16) << 8)
    qs = blk[:, :, 2:]
    q = np.empty((n_out, nb, 32), np.int32)
    q[:, :, 0::2] = (qs & 0x0F).astype(np.int32) - 8
    q[:, :, 1::2] = (qs >> 4).astype(np.int32) - 8
    return f16_bits_to_f32(d_bits), q.reshape(n_out, k)


def q4_0_to_q8_0(raw: np.ndarray, n_out: int, k: int) -> np.ndarray:
    """Q4_0 blocks (reference nibble order) as Q8_0 blocks: the same f16
    scale bits, quants nibble - 8 as int8."""
    nb = k // 32
    blk = np.asarray(raw, dtype=np.uint8).reshape(n_out, nb, 18)
    d_bits = blk[:, :, 0].astype(np.uint16) | (blk[:, :, 1].astype(np.uint16) << 8)
    _, q = q4_0_split(raw, n_out, k)
    return q8_0_pack(d_bits, q.astype(np.int8))


def q4_0_interleaved_to_ggml(raw: np.ndarray) -> np.ndarray:
    """Re-encode Q4_0 blocks from the reference's nibble order (element 2i =
    low nibble of byte i) to upstream GGML's (element i = low nibble of byte
    i, element i + 16 = its high nibble); the scale bytes are kept."""
    blk = np.asarray(raw, dtype=np.uint8).reshape(-1, 18).copy()
    qs = blk[:, 2:]
    e = np.empty((blk.shape[0], 32), np.uint8)
    e[:, 0::2] = qs & 0x0F
    e[:, 1::2] = qs >> 4
    blk[:, 2:] = e[:, :16] | (e[:, 16:] << 4)
    return blk.ravel()


def q4_0_dequant_matmul_seq(x: np.ndarray, raw: np.ndarray, n_out: int, k: int):
    """matmul_q4_0_dequant with the reference's sequential f32 sum over K."""
    x = np.asarray(x, dtype=F32)
    d, q = q4_0_split(raw, n_out, k)
    w = (np.repeat(d, 32, axis=1) * q.astype(F32)).astype(F32)   # [N,K]
    out = np.zeros((x.shape[0], n_out), F32)
    for i in range(k):
        out = (out + (x[:, i:i + 1] * w[None, :, i]).astype(F32)).astype(F32)
    return out


def q4_0_terms_abs_sum(x: np.ndarray, raw: np.ndarray, n_out: int, k: int):
    """sum_k |x_k * w_k| in float64 (the scale of the tolerance bound)."""
    d, q = q4_0_split(raw, n_out, k)
    w = np.repeat(d, 32, axis=1).astype(np.float64) * q
    return np.abs(np.asarray(x, np.float64)) @ np.abs(w).T

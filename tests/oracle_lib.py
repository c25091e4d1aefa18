"""ctypes binding of the CPU oracle (oracle/liboracle.so).

Test infrastructure: only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg load this.  Each wrapper returns numpy arrays and raises
``OracleError`` carrying the reference's TensorError kind when the restated
Rust function would return Err.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
LIB_PATH = os.path.join(ORACLE_DIR, "liboracle.so")

OK, INVALID_SHAPE, SHAPE_MISMATCH = 0, 1, 2
_KIND = {INVALID_SHAPE: "InvalidShape", SHAPE_MISMATCH: "ShapeMismatch"}


class OracleError(Exception):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{_KIND.get(code, code)}: {msg}")
        self.code = code
        self.kind = _KIND.get(code, str(code))


_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", ORACLE_DIR], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _sig(_lib)
    return _lib


P = C.c_void_p
SZ = C.c_size_t


def _sig(l):
    l.orc_f16_to_f32.argtypes = [C.c_uint16]
    l.orc_f16_to_f32.restype = C.c_float
    l.orc_f32_to_f16.argtypes = [C.c_float]
    l.orc_f32_to_f16.restype = C.c_uint16
    l.orc_quantize_symmetric.argtypes = [P, SZ, P]
    l.orc_quantize_symmetric.restype = C.c_float
    l.orc_quantize_per_channel.argtypes = [P, SZ, SZ, SZ, P, P]
    l.orc_dot_i8_scalar.argtypes = [P, P, SZ]
    l.orc_dot_i8_scalar.restype = C.c_int32
    l.orc_dot_i8_avx2.argtypes = [P, P, SZ]
    l.orc_dot_i8_avx2.restype = C.c_int32
    l.orc_matmul_int8.argtypes = [P, SZ, C.c_float, P, P, SZ, SZ, SZ, P, P]
    l.orc_matmul_int8_avx2.argtypes = [P, SZ, C.c_float, P, P, SZ, SZ, SZ, P]
    l.orc_matmul_int8_parallel.argtypes = [P, SZ, C.c_float, P, P, SZ, SZ, SZ, P,
                                           C.c_int, P]
    l.orc_matmul_int8_rows.argtypes = [P, SZ, P, P, P, SZ, SZ, SZ, P, P]
    l.orc_matmul_int8_from_f32.argtypes = [P, P, SZ, P, P, SZ, SZ, P, P, P, P]
    l.orc_create_q8_0_block.argtypes = [P, P]
    l.orc_dequantize_q8_0.argtypes = [P, SZ, P]
    l.orc_q8_0_check_raw.argtypes = [SZ, SZ, SZ]
    l.orc_matmul_q8_0_direct.argtypes = [P, P, SZ, P, SZ, SZ, SZ, P, P, P]
    l.orc_create_q4_0_block.argtypes = [P, P]
    l.orc_dequantize_q4_0.argtypes = [P, SZ, P]
    l.orc_matmul_q4_0_dequant.argtypes = [P, P, SZ, P, SZ, SZ, SZ, P]
    l.orc_matmul_q4_0_w4a8.argtypes = [P, P, SZ, P, SZ, SZ, SZ, C.c_int, P, P, P]
    l.orc_last_error.restype = C.c_char_p
    l.orc_have_avx2.restype = C.c_int
    l.orc_rmsnorm.argtypes = [P, SZ, SZ, P, C.c_float, P]
    l.orc_rmsnorm.restype = None
    l.orc_rope_table.argtypes = [SZ, SZ, C.c_float, P, P]
    l.orc_rope_table.restype = None
    l.orc_rope_apply.argtypes = [P, SZ, SZ, SZ, P, P, SZ, SZ]
    l.orc_gqa_causal.argtypes = [P, SZ, P, P, SZ, SZ, SZ, SZ, SZ, P, P]
    l.orc_swiglu.argtypes = [P, P, SZ, P]
    l.orc_swiglu.restype = None
    l.orc_argmax.argtypes = [P, SZ]
    l.orc_argmax.restype = C.c_uint32


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _check(rc):
    if rc != OK:
        raise OracleError(rc, lib().orc_last_error().decode())


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def _dims(shape):
    d = np.asarray(shape, dtype=np.uintp)
    return d, len(shape)


# ---- f16 codec ---------------------------------------------------------
def f16_to_f32(h: int) -> float:
    return lib().orc_f16_to_f32(h)


def f32_to_f16(f: float) -> int:
    return lib().orc_f32_to_f16(f)


# ---- quantizers ----------------------------------------------------------
def quantize_symmetric(x):
    x = _c(x, np.float32).ravel()
    q = np.empty(x.size, np.int8)
    s = lib().orc_quantize_symmetric(_p(x), x.size, _p(q))
    return q, np.float32(s)


def quantize_per_channel(w, n_out, k_in):
    w = _c(w, np.float32).ravel()
    data = np.empty(max(n_out * k_in, 1), np.int8)
    scales = np.empty(max(n_out, 1), np.float32)
    _check(lib().orc_quantize_per_channel(_p(w), w.size, n_out, k_in, _p(data),
                                          _p(scales)))
    return data[: n_out * k_in].reshape(n_out, k_in), scales[:n_out]


# ---- dots --------------------------------------------------------------
def dot_i8_scalar(a, b):
    a, b = _c(a, np.int8), _c(b, np.int8)
    return lib().orc_dot_i8_scalar(_p(a), _p(b), a.size)


def dot_i8_avx2(a, b):
    a, b = _c(a, np.int8), _c(b, np.int8)
    return lib().orc_dot_i8_avx2(_p(a), _p(b), a.size)


# ---- per-channel INT8 GEMMs --------------------------------------------
def matmul_int8(act_q, act_scale, w, scales, m, want_acc=False):
    act_q = _c(act_q, np.int8).ravel()
    w = _c(w, np.int8)
    scales = _c(scales, np.float32)
    n, k = w.shape
    out = np.empty((m, n), np.float32)
    acc = np.empty((m, n), np.int32) if want_acc else None
    _check(lib().orc_matmul_int8(_p(act_q), act_q.size, float(act_scale), _p(w),
                                 _p(scales), n, k, m, _p(out), _p(acc)))
    return (out, acc) if want_acc else out


def matmul_int8_avx2(act_q, act_scale, w, scales, m):
    act_q = _c(act_q, np.int8).ravel()
    w = _c(w, np.int8)
    scales = _c(scales, np.float32)
    n, k = w.shape
    out = np.empty((m, n), np.float32)
    _check(lib().orc_matmul_int8_avx2(_p(act_q), act_q.size, float(act_scale),
                                      _p(w), _p(scales), n, k, m, _p(out)))
    return out


def matmul_int8_parallel(act_q, act_scale, w, scales, m, n_threads=0,
                         out=None):
    """Returns (out, cores_used)."""
    act_q = _c(act_q, np.int8).ravel()
    n, k = w.shape
    if out is None:
        out = np.empty((m, n), np.float32)
    used = C.c_int(0)
    _check(lib().orc_matmul_int8_parallel(
        _p(act_q), act_q.size, float(act_scale), _p(w), _p(scales), n, k, m,
        _p(out), n_threads, C.byref(used)))
    return out, used.value


def matmul_int8_rows(act_q, act_scales, w, scales, m, want_acc=False):
    act_q = _c(act_q, np.int8).ravel()
    act_scales = _c(act_scales, np.float32)
    w = _c(w, np.int8)
    scales = _c(scales, np.float32)
    n, k = w.shape
    out = np.empty((m, n), np.float32)
    acc = np.empty((m, n), np.int32) if want_acc else None
    _check(lib().orc_matmul_int8_rows(_p(act_q), act_q.size, _p(act_scales),
                                      _p(w), _p(scales), n, k, m, _p(out),
                                      _p(acc)))
    return (out, acc) if want_acc else out


def matmul_int8_from_f32(x, w, scales):
    """Returns (out, act_q, act_scale, acc)."""
    x = _c(x, np.float32)
    w = _c(w, np.int8)
    scales = _c(scales, np.float32)
    n, k = w.shape
    dims, nd = _dims(x.shape)
    m = x.shape[0] if nd >= 1 else 1
    out = np.empty((m, n), np.float32)
    aq = np.empty(max(x.size, 1), np.int8)
    s = np.zeros(1, np.float32)
    acc = np.empty((m, n), np.int32)
    _check(lib().orc_matmul_int8_from_f32(_p(x), _p(dims), nd, _p(w), _p(scales),
                                          n, k, _p(out), _p(aq), _p(s), _p(acc)))
    return out, aq[: x.size].reshape(x.shape), s[0], acc


# ---- Q8_0 --------------------------------------------------------------
def create_q8_0_block(values32):
    v = _c(values32, np.float32)
    assert v.size == 32
    b = np.empty(34, np.uint8)
    lib().orc_create_q8_0_block(_p(v), _p(b))
    return b


def quantize_q8_0(w):
    """[N,K] f32 -> raw Q8_0 bytes (create_q8_0_block per 32 elements, as
    Q8_0WeightMatrix::from_f32_tensor, q8_direct.rs:118-158)."""
    w = _c(w, np.float32)
    n, k = w.shape
    blocks = w.reshape(-1, 32)
    out = np.empty((blocks.shape[0], 34), np.uint8)
    for i in range(blocks.shape[0]):
        out[i] = create_q8_0_block(blocks[i])
    return out.ravel()


def dequantize_q8_0(data):
    data = _c(data, np.uint8)
    out = np.empty(max(data.size // 34 * 32, 1), np.float32)
    _check(lib().orc_dequantize_q8_0(_p(data), data.size, _p(out)))
    return out[: data.size // 34 * 32]


def q8_0_check_raw(n_bytes, n_out, k_in):
    _check(lib().orc_q8_0_check_raw(n_bytes, n_out, k_in))


def matmul_q8_0_direct(x, w_raw, n_out, k_in, want_block_dots=False):
    """Returns out, or (out, block_dots[M,N,K/32], act_scales[M])."""
    x = _c(x, np.float32)
    w_raw = _c(w_raw, np.uint8)
    dims, nd = _dims(x.shape)
    m = x.shape[0] if nd >= 1 else 1
    out = np.empty((m, n_out), np.float32)
    bd = np.empty((m, n_out, max(k_in // 32, 1)), np.int32) if want_block_dots else None
    sa = np.empty(max(m, 1), np.float32) if want_block_dots else None
    _check(lib().orc_matmul_q8_0_direct(_p(x), _p(dims), nd, _p(w_raw), w_raw.size,
                                        n_out, k_in, _p(out), _p(bd), _p(sa)))
    return (out, bd, sa[:m]) if want_block_dots else out


# ---- Q4_0 --------------------------------------------------------------
def create_q4_0_block(values32):
    v = _c(values32, np.float32)
    assert v.size == 32
    b = np.empty(18, np.uint8)
    lib().orc_create_q4_0_block(_p(v), _p(b))
    return b


def quantize_q4_0(w):
    w = _c(w, np.float32)
    blocks = w.reshape(-1, 32)
    out = np.empty((blocks.shape[0], 18), np.uint8)
    for i in range(blocks.shape[0]):
        out[i] = create_q4_0_block(blocks[i])
    return out.ravel()


def dequantize_q4_0(data):
    data = _c(data, np.uint8)
    out = np.empty(max(data.size // 18 * 32, 1), np.float32)
    _check(lib().orc_dequantize_q4_0(_p(data), data.size, _p(out)))
    return out[: data.size // 18 * 32]


def matmul_q4_0_dequant(x, w_q4, n_out, k):
    x = _c(x, np.float32)
    w_q4 = _c(w_q4, np.uint8)
    dims, nd = _dims(x.shape)
    m = x.shape[0] if nd >= 1 else 1
    out = np.empty((max(m, 1), max(n_out, 1)), np.float32)
    _check(lib().orc_matmul_q4_0_dequant(_p(x), _p(dims), nd, _p(w_q4), w_q4.size,
                                         n_out, k, _p(out)))
    return out[:m, :n_out]


Q4_INTERLEAVED, Q4_GGML = 0, 1


def matmul_q4_0_w4a8(x, w_q4, n_out, k, order=Q4_INTERLEAVED, want_block_dots=False):
    """W4A8 extension: returns out, or (out, block_dots[M,N,K/32], act_scales[M])."""
    x = _c(x, np.float32)
    w_q4 = _c(w_q4, np.uint8)
    dims, nd = _dims(x.shape)
    m = x.shape[0] if nd >= 1 else 1
    out = np.empty((max(m, 1), max(n_out, 1)), np.float32)
    bd = np.empty((max(m, 1), max(n_out, 1), max(k // 32, 1)), np.int32) if want_block_dots \
        else None
    sa = np.empty(max(m, 1), np.float32) if want_block_dots else None
    _check(lib().orc_matmul_q4_0_w4a8(_p(x), _p(dims), nd, _p(w_q4), w_q4.size, n_out, k,
                                      order, _p(out), _p(bd), _p(sa)))
    if want_block_dots:
        return out[:m, :n_out], bd[:m, :n_out], sa[:m]
    return out[:m, :n_out]


def have_avx2() -> bool:
    return bool(lib().orc_have_avx2())


# ---- decoder-layer steps (oracle/llama.c) --------------------------------
def rmsnorm(x, w, eps):
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    d = w.size
    out = np.empty_like(x)
    lib().orc_rmsnorm(_p(x), x.size // d, d, _p(w), float(eps), _p(out))
    return out


def rope_table(max_seq, head_dim, base):
    half = head_dim // 2
    cos = np.empty((max_seq, half), np.float32)
    sin = np.empty((max_seq, half), np.float32)
    lib().orc_rope_table(max_seq, head_dim, float(base), _p(cos), _p(sin))
    return cos, sin


def rope_apply(x, n_heads, head_dim, cos, sin, start_pos):
    """x [seq, n_heads*head_dim] (or [seq, n_heads, head_dim]); returns a copy."""
    y = np.array(x, dtype=np.float32, copy=True, order="C")
    seq = y.size // (n_heads * head_dim)
    _check(lib().orc_rope_apply(_p(y), seq, n_heads, head_dim, _p(_c(cos, np.float32)),
                                _p(_c(sin, np.float32)), cos.shape[0], start_pos))
    return y


def gqa_causal(q, k, v, n_heads, n_kv_heads, head_dim, start_pos):
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    seq_q = q.size // (n_heads * head_dim)
    seq_k = k.size // (n_kv_heads * head_dim)
    out = np.empty((seq_q, n_heads * head_dim), np.float32)
    scratch = np.empty(max(seq_k, 1), np.float32)
    _check(lib().orc_gqa_causal(_p(q), seq_q, _p(k), _p(v), seq_k, n_heads, n_kv_heads,
                                head_dim, start_pos, _p(out), _p(scratch)))
    return out


def swiglu(gate, up):
    g, u = _c(gate, np.float32), _c(up, np.float32)
    out = np.empty_like(g)
    lib().orc_swiglu(_p(g), _p(u), g.size, _p(out))
    return out


def argmax(v):
    v = _c(v, np.float32)
    return int(lib().orc_argmax(_p(v), v.size))


# ---- LlamaModelInt8 composition (model/llama/forward_int8.rs) ------------
class Proj:
    """One projection weight in one of the formats: "int8"
    (QuantizedMatrix: data [N,K] int8 + scales [N], projected by
    matmul_int8_from_f32, forward_int8.rs:72-74), "q8_0" (raw Q8_0 bytes,
    matmul_q8_0_direct), "q4_0" (raw Q4_0 bytes, matmul_q4_0_dequant) or
    "w4a8" (raw Q4_0 bytes, the W4A8 extension matmul_q4_0_w4a8)."""

    def __init__(self, fmt, n_out, k_in, data, scales=None):
        self.fmt, self.n_out, self.k_in, self.data, self.scales = fmt, n_out, k_in, data, scales

    def __call__(self, x):
        if self.fmt == "int8":
            return matmul_int8_from_f32(x, self.data, self.scales)[0]
        if self.fmt == "q8_0":
            return matmul_q8_0_direct(x, self.data, self.n_out, self.k_in)
        if self.fmt == "w4a8":
            return matmul_q4_0_w4a8(x, self.data, self.n_out, self.k_in)
        return matmul_q4_0_dequant(x, self.data, self.n_out, self.k_in)


class LlamaOracle:
    """LlamaModelInt8 with a KvCache (forward_int8.rs:148-402, 416-546):
    forward_cached() is embed -> TransformerBlockInt8::forward_cached per
    layer -> rmsnorm -> output projection (logits of every row);
    forward_decode() the one-token step.  layers: list of dicts with keys
    attn_norm, ffn_norm and wq wk wv wo wgate wup wdown (Proj)."""

    def __init__(self, cfg, token_embd, layers, output_norm, output):
        self.cfg = cfg
        self.token_embd = _c(token_embd, np.float32)
        self.layers = layers
        self.output_norm = _c(output_norm, np.float32)
        self.output = output
        hd = cfg["head_dim"]
        self.cos, self.sin = rope_table(cfg["max_seq"], hd, cfg["rope_base"])
        kvd = cfg["n_kv_heads"] * hd
        self.k_cache = np.zeros((len(layers), cfg["max_seq"], kvd), np.float32)
        self.v_cache = np.zeros_like(self.k_cache)

    def embed(self, tokens):  # forward_int8.rs:125-140
        for t in tokens:
            if t >= self.token_embd.shape[0]:
                raise OracleError(INVALID_SHAPE, f"token id {t} >= vocab_size")
        return self.token_embd[np.asarray(tokens, dtype=np.int64)].copy()

    def block(self, li, x, start_pos):
        """attn_sublayer_cached (forward_int8.rs:291-323) + ffn_sublayer
        (:350-357); the decode step (:325-348) is the same with seq = 1."""
        c, L = self.cfg, self.layers[li]
        nh, nkv, hd = c["n_heads"], c["n_kv_heads"], c["head_dim"]
        seq = x.shape[0]
        normed = rmsnorm(x, L["attn_norm"], c["eps"])
        q = L["wq"](normed)
        k = L["wk"](normed)
        v = L["wv"](normed)
        q = rope_apply(q, nh, hd, self.cos, self.sin, start_pos)
        k = rope_apply(k, nkv, hd, self.cos, self.sin, start_pos)
        self.k_cache[li, start_pos:start_pos + seq] = k   # cached.rs write_k / write_v
        self.v_cache[li, start_pos:start_pos + seq] = v
        total = start_pos + seq
        attn = gqa_causal(q, self.k_cache[li, :total], self.v_cache[li, :total], nh, nkv, hd,
                          start_pos)
        x = x + L["wo"](attn)
        normed = rmsnorm(x, L["ffn_norm"], c["eps"])
        h = swiglu(L["wgate"](normed), L["wup"](normed))
        return x + L["wdown"](h)

    def forward_cached(self, tokens, start_pos=0):
        x = self.embed(tokens)
        for li in range(len(self.layers)):
            x = self.block(li, x, start_pos)
        x = rmsnorm(x, self.output_norm, self.cfg["eps"])
        return self.output(x)

    def forward_decode(self, token, pos):
        return self.forward_cached([token], pos)[0]

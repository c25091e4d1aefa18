"""Pins the decoder-layer oracle (oracle/llama.c + the LlamaOracle
composition) with the reference's own known-answer tests, float64 closed
forms and invariants of the composition.  CPU only."""
import math

import numpy as np
import pytest

import oracle_lib as O

F32 = np.float32


# ---- rmsnorm (ops/norm/rmsnorm.rs) ----------------------------------------------
def test_rmsnorm_pytorch_reference():  # rmsnorm.rs:319-335
    out = O.rmsnorm(np.array([1, 2, 3, 4], F32), np.ones(4, F32), 1e-5)
    assert np.allclose(out, [0.3651484, 0.7302968, 1.0954452, 1.4605936], atol=1e-5)


def test_rmsnorm_unit_vector_and_zeros():  # rmsnorm.rs:289-317
    out = O.rmsnorm(np.array([1, 0, 0, 0], F32), np.ones(4, F32), 0.0)
    assert np.allclose(out, [2, 0, 0, 0], atol=1e-6)  # rms = 1/2
    z = O.rmsnorm(np.zeros((2, 8), F32), np.ones(8, F32), 1e-6)
    assert np.all(z == 0) and not np.any(np.isnan(z))


def test_rmsnorm_closed_form_and_rows_independent():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 4096)).astype(F32)
    w = rng.uniform(0.5, 1.5, 4096).astype(F32)
    out = O.rmsnorm(x, w, 1e-6)
    x64 = x.astype(np.float64)
    ref = w * (x64 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + 1e-6))
    assert np.allclose(out, ref, rtol=2e-5, atol=1e-6)
    # row 3 alone gives the same bits (rmsnorm.rs:261-287)
    assert np.array_equal(O.rmsnorm(x[3:4], w, 1e-6), out[3:4])
    # a plausible slip, dividing by d - 1, is caught
    bad = w * (x64 / np.sqrt((x64 * x64).sum(axis=1, keepdims=True) / 4095 + 1e-6))
    assert not np.allclose(out, bad, rtol=2e-5, atol=1e-6)


# ---- silu / swiglu (ops/activation) ---------------------------------------------
def test_silu_and_swiglu_pytorch_reference():
    g = np.array([1, -1, 2, -2], F32)
    s = O.swiglu(g, np.ones(4, F32))  # swiglu with up = 1 is silu (swiglu.rs:143)
    assert np.allclose(s, [0.731059, -0.268941, 1.761594, -0.238406], atol=1e-5)  # silu.rs:111
    out = O.swiglu(np.array([1, 2, -1, -2], F32), np.array([1, 0.5, 2, 3], F32))
    assert np.allclose(out, [0.731059, 0.880797, -0.537882, -0.715219], atol=1e-4)  # swiglu.rs:259
    assert np.all(O.swiglu(np.zeros(3, F32), np.array([1, 2, 3], F32)) == 0)  # swiglu.rs:155
    # silu(0) = 0, large |x| limits (silu.rs:92-109)
    e = O.swiglu(np.array([0, 50, -50], F32), np.ones(3, F32))
    assert e[0] == 0 and abs(e[1] - 50) < 1e-4 and abs(e[2]) < 1e-6


def test_swiglu_closed_form():
    rng = np.random.default_rng(1)
    g = (rng.standard_normal(10000) * 4).astype(F32)
    u = rng.standard_normal(10000).astype(F32)
    g64 = g.astype(np.float64)
    ref = g64 / (1 + np.exp(-g64)) * u
    assert np.allclose(O.swiglu(g, u), ref, rtol=1e-6, atol=1e-7)


# ---- RoPE (ops/rope.rs) ---------------------------------------------------------
def test_rope_table_kats():
    cos, sin = O.rope_table(16, 8, 10000.0)
    assert np.allclose(cos[0], 1, atol=1e-7) and np.allclose(sin[0], 0, atol=1e-7)  # pos 0
    assert np.allclose(cos * cos + sin * sin, 1, atol=1e-6)  # Pythagorean
    ang = np.abs(np.arctan2(sin[1], cos[1]))
    assert np.all(np.diff(ang) <= 0)  # theta decreases with the pair index
    # closed form in float64
    th = 1.0 / 10000.0 ** (2 * np.arange(4) / 8)
    pos = np.arange(16)[:, None]
    assert np.allclose(cos, np.cos(pos * th), atol=2e-6)
    assert np.allclose(sin, np.sin(pos * th), atol=2e-6)


def test_rope_apply_identity_and_rotation():
    cos, sin = O.rope_table(4, 4, 10000.0)
    x = np.arange(1, 9, dtype=F32).reshape(1, 8)
    assert np.allclose(O.rope_apply(x, 2, 4, cos, sin, 0), x, atol=1e-6)  # rope.rs pos-0 test
    # pair (2i, 2i+1) rotated by angle pos*theta_i: norms kept, as a complex product
    rng = np.random.default_rng(2)
    cos, sin = O.rope_table(64, 128, 10000.0)
    x = rng.standard_normal((3, 2 * 128)).astype(F32)
    y = O.rope_apply(x, 2, 128, cos, sin, 17)
    z = x.reshape(3, 2, 64, 2).astype(np.float64)
    zc = z[..., 0] + 1j * z[..., 1]
    rot = (cos[17:20] + 1j * sin[17:20]).astype(np.complex128)[:, None, :]
    ref = zc * rot
    yc = y.reshape(3, 2, 64, 2)
    assert np.allclose(yc[..., 0], ref.real, atol=1e-5)
    assert np.allclose(yc[..., 1], ref.imag, atol=1e-5)
    with pytest.raises(O.OracleError):
        O.rope_apply(x, 2, 128, cos, sin, 62)  # past the table


# ---- causal GQA (attention/gqa.rs, mask.rs, sdpa.rs, softmax.rs) ---------------------
def test_gqa_causal_first_token_self_only():  # gqa.rs:420-460
    q = np.array([[1, 0, 1, 0], [0.5, 0.5, 0.5, 0.5]], F32)
    k = np.array([[1, 0], [0, 1]], F32)
    v = np.array([[5, 7], [99, 99]], F32)
    out = O.gqa_causal(q, k, v, 2, 1, 2, 0)
    assert np.allclose(out[0], [5, 7, 5, 7], atol=1e-4)


def test_gqa_groups2_kv_sharing():  # gqa.rs:346-418, last query sees every key
    q = np.zeros((1, 8), F32)
    k = np.zeros((2, 4), F32)
    v = np.array([[1, 0, 0, 3], [2, 0, 0, 4]], F32)
    out = O.gqa_causal(q, k, v, 4, 2, 2, 1)
    assert np.allclose(out[0], [1.5, 0, 1.5, 0, 0, 3.5, 0, 3.5], atol=1e-5)


def _attention64(q, k, v, nh, nkv, hd, start):
    q, k, v = (a.astype(np.float64) for a in (q, k, v))
    sq, sk = q.shape[0], k.shape[0]
    out = np.zeros((sq, nh * hd))
    for h in range(nh):
        kh = h // (nh // nkv)
        s = q[:, h * hd:(h + 1) * hd] @ k[:, kh * hd:(kh + 1) * hd].T / math.sqrt(hd)
        mask = np.arange(sk)[None, :] > (start + np.arange(sq))[:, None]
        s[mask] = -np.inf
        p = np.exp(s - s.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        out[:, h * hd:(h + 1) * hd] = p @ v[:, kh * hd:(kh + 1) * hd]
    return out


@pytest.mark.parametrize("sq,sk,start,nh,nkv", [(5, 5, 0, 4, 4), (3, 9, 6, 4, 2), (1, 17, 16, 8, 1)])
def test_gqa_causal_closed_form(sq, sk, start, nh, nkv):
    rng = np.random.default_rng(sq * 31 + sk)
    hd = 16
    q = rng.standard_normal((sq, nh * hd)).astype(F32)
    k = rng.standard_normal((sk, nkv * hd)).astype(F32)
    v = rng.standard_normal((sk, nkv * hd)).astype(F32)
    if start + sq < sk:
        k, v = k[:start + sq], v[:start + sq]
    out = O.gqa_causal(q, k, v, nh, nkv, hd, start)
    ref = _attention64(q, k, v, nh, nkv, hd, start)
    assert np.allclose(out, ref, rtol=1e-5, atol=1e-6)
    # the transposed-operand slip (q @ k instead of q @ k^T is not even
    # shaped right here); the off-by-one mask slip, one key too many, is caught
    if start + sq > 1:
        bad = _attention64(q, np.vstack([k, k[-1:]]), np.vstack([v, v[-1:] + 1]), nh, nkv, hd,
                           start + 1)
        assert not np.allclose(out, bad[:, :], rtol=1e-5, atol=1e-6)


def test_gqa_shape_errors():  # gqa.rs:476-523
    q = np.zeros((2, 8), F32)
    kv = np.zeros((2, 6), F32)
    with pytest.raises(O.OracleError):
        O.gqa_causal(q, kv, kv, 4, 3, 2, 0)  # 4 heads not divisible by 3
    with pytest.raises(O.OracleError):
        O.gqa_causal(q, np.zeros((1, 4), F32), np.zeros((1, 4), F32), 4, 2, 2, 0)  # keys < queries


# ---- argmax (sampling/mod.rs:144-151) ---------------------------------------------
def test_argmax_last_of_ties():
    assert O.argmax(np.array([1, 3, 3, 2], F32)) == 2
    assert O.argmax(np.array([5], F32)) == 0
    assert O.argmax(np.array([-1, -1], F32)) == 1
    rng = np.random.default_rng(3)
    v = rng.standard_normal(32000).astype(F32)
    assert O.argmax(v) == int(np.argmax(v))  # no ties: the plain argmax


# ---- composition (forward_int8.rs) ------------------------------------------------------
def tiny_model(fmt, seed=0, d=64, nh=4, nkv=2, ffn=96, vocab=50, max_seq=24, n_layers=2):
    rng = np.random.default_rng(seed)
    hd = d // nh
    cfg = dict(dim=d, n_heads=nh, n_kv_heads=nkv, head_dim=hd, ffn=ffn, vocab=vocab,
               max_seq=max_seq, eps=1e-6, rope_base=10000.0)

    def proj(n, k):
        w = (rng.standard_normal((n, k)) * 0.05).astype(F32)
        if fmt == "int8":
            data, scales = O.quantize_per_channel(w, n, k)
            return O.Proj("int8", n, k, data, scales)
        if fmt == "q8_0":
            return O.Proj("q8_0", n, k, O.quantize_q8_0(w))
        return O.Proj("q4_0", n, k, O.quantize_q4_0(w))

    layers = []
    for _ in range(n_layers):
        layers.append(dict(
            attn_norm=rng.uniform(0.8, 1.2, d).astype(F32),
            ffn_norm=rng.uniform(0.8, 1.2, d).astype(F32),
            wq=proj(nh * hd, d), wk=proj(nkv * hd, d), wv=proj(nkv * hd, d), wo=proj(d, nh * hd),
            wgate=proj(ffn, d), wup=proj(ffn, d), wdown=proj(d, ffn)))
    embd = rng.standard_normal((vocab, d)).astype(F32)
    return O.LlamaOracle(cfg, embd, layers, rng.uniform(0.8, 1.2, d).astype(F32),
                         proj(vocab, d)), rng


def test_composition_decode_matches_prefill_rows_q8_0():
    """Per-row activation quantization (Q8_0 path) makes every step row-local
    except attention, whose row p sees keys 0..p either way: the cached
    decode of token p reproduces prefill row p bit for bit."""
    m, rng = tiny_model("q8_0")
    toks = rng.integers(0, 50, 12).tolist()
    full = m.forward_cached(toks, 0)
    m2, _ = tiny_model("q8_0")
    pre = m2.forward_cached(toks[:8], 0)
    assert np.array_equal(pre, full[:8])
    for p in range(8, 12):
        assert np.array_equal(m2.forward_decode(toks[p], p), full[p])


def test_composition_int8_per_tensor_scale_differs_but_close():
    """The per-channel INT8 model quantizes the whole [seq, d] input with one
    scale (forward_int8.rs:72-74 -> int8.rs:141), so a decode row differs from
    the prefill row in the low bits only."""
    m, rng = tiny_model("int8")
    toks = rng.integers(0, 50, 10).tolist()
    full = m.forward_cached(toks, 0)
    m2, _ = tiny_model("int8")
    m2.forward_cached(toks[:9], 0)
    last = m2.forward_decode(toks[9], 9)
    scale = np.abs(full[9]).max()
    assert np.abs(last - full[9]).max() <= 0.05 * scale
    # and the embedding lookup rejects ids past the vocabulary (forward_int8.rs:132-136)
    with pytest.raises(O.OracleError):
        m.embed([50])

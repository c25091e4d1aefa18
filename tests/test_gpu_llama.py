"""GPU LlamaModelInt8 (include/mri_llama.h) against the CPU oracle's
composition (tests/oracle_lib.py LlamaOracle over oracle/llama.c).

Tolerances.  The layer's f32 sums (RMSNorm, softmax denominator, attention
value sum) and exp differ from the reference in rounding only.  With Q4_0
weights (W4A32, no activation quantization) that is all that differs, and
the logits agree to 1e-4 of their largest magnitude.  INT8 and Q8_0
projections quantize their inputs to int8: a last-bit difference in an
activation can move one element across a rounding boundary, which changes
that element by one quantization step, so the logits of those models are
compared to 2e-2 of their largest magnitude (a wrong head, position or
mask moves them by O(1)) and greedy tokens by their oracle margin.  The
W4A8 extension quantizes its inputs the same way and is compared the same
way."""
import numpy as np
import pytest

import oracle_lib as O
from gpu_util import dev, empty, host

pytestmark = pytest.mark.gpu

F32 = np.float32


def torch():
    import torch as t
    return t


def mods():
    import mri_llama as L
    import mri_qmatmul as Q
    return L, Q


MIXED = {"wq": "int8", "wk": "q8_0", "wv": "w4a8", "wo": "q8_0", "wgate": "w4a8", "wup": "int8",
         "wdown": "int8", "out": "q8_0"}


def build(fmt, seed=0, d=256, nh=4, nkv=2, ffn=512, vocab=300, max_seq=48, n_layers=2,
          out_w=None):
    """The same random model on both sides (fmt "mixed": a different format
    per projection role, MIXED); out_w: the output projection's f32 weights
    instead of random ones."""
    L, Q = mods()
    rng = np.random.default_rng(seed)
    hd = d // nh
    cfg = dict(dim=d, n_heads=nh, n_kv_heads=nkv, head_dim=hd, ffn=ffn, vocab=vocab,
               max_seq=max_seq, eps=1e-6, rope_base=10000.0)

    def proj(n, k, role="out"):
        if fmt == "mixed":
            return proj_fmt(MIXED[role], n, k)
        return proj_fmt(fmt, n, k)

    def proj_fmt(fmt, n, k, w=None):
        if w is None:
            w = (rng.standard_normal((n, k)) * 0.05).astype(F32)
        if fmt == "int8":
            data, scales = O.quantize_per_channel(w, n, k)
            return O.Proj("int8", n, k, data, scales), Q.QMatrix.from_host(data, scales)
        if fmt == "q8_0":
            raw = O.quantize_q8_0(w)
            return O.Proj("q8_0", n, k, raw), Q.Q8Matrix.from_raw_bytes(raw, n, k)
        raw = O.quantize_q4_0(w)
        if fmt == "w4a8":
            return O.Proj("w4a8", n, k, raw), Q.Q4Matrix.from_raw_bytes(raw, n, k)
        return O.Proj("q4_0", n, k, raw), (dev(raw), n, k)

    o_layers, g_layers = [], []
    for _ in range(n_layers):
        an = rng.uniform(0.8, 1.2, d).astype(F32)
        fn = rng.uniform(0.8, 1.2, d).astype(F32)
        ol, gl = dict(attn_norm=an, ffn_norm=fn), dict(attn_norm=an, ffn_norm=fn)
        for name, (n, k) in (("wq", (nh * hd, d)), ("wk", (nkv * hd, d)), ("wv", (nkv * hd, d)),
                             ("wo", (d, nh * hd)), ("wgate", (ffn, d)), ("wup", (ffn, d)),
                             ("wdown", (d, ffn))):
            ol[name], gl[name] = proj(n, k, name)
        o_layers.append(ol)
        g_layers.append(gl)
    embd = rng.standard_normal((vocab, d)).astype(F32)
    onorm = rng.uniform(0.8, 1.2, d).astype(F32)
    if out_w is None:
        o_out, g_out = proj(vocab, d)
    else:
        o_out, g_out = proj_fmt(MIXED["out"] if fmt == "mixed" else fmt, vocab, d, out_w)
    oracle = O.LlamaOracle(cfg, embd, o_layers, onorm, o_out)
    gpu = L.Llama(cfg, embd, onorm, g_out, g_layers)
    return oracle, gpu, rng


def close(got, ref, frac):
    scale = float(np.abs(ref).max())
    err = float(np.abs(got - ref).max())
    assert err <= frac * scale, f"max |gpu - ref| = {err:.3g} > {frac} * {scale:.3g}"


TOL = {"q4_0": 1e-4, "q8_0": 2e-2, "int8": 2e-2, "w4a8": 2e-2, "mixed": 2e-2}


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0", "int8", "w4a8"])
def test_llama_prefill_and_decode_logits(fmt):
    """forward_cached over a prompt, then forward_decode steps (teacher
    forced: both sides see the same tokens)."""
    t = torch()
    oracle, gpu, rng = build(fmt, seed={"q4_0": 1, "q8_0": 2, "int8": 3, "w4a8": 4}[fmt])
    toks = rng.integers(0, 300, 24).tolist()
    cache = gpu.kv_cache()
    logits = empty((20, 300), t.float32)
    gpu.forward_cached(toks[:20], 0, cache, logits)
    ref = oracle.forward_cached(toks[:20], 0)
    close(host(logits), ref, TOL[fmt])
    one = empty((300,), t.float32)
    for p in range(20, 24):
        gpu.forward_decode(toks[p], p, cache, one)
        close(host(one), oracle.forward_decode(toks[p], p), TOL[fmt])


def test_llama_decode_split_keys_head_dim_64():
    """Decode past 128 keys at head_dim 64 with two query heads per KV head:
    the decode attention then splits each head's keys over 64-key
    workgroups (four key rows per wave load instruction at this head size)
    and the last workgroup of a head combines them, including a partial
    last chunk.  Teacher-forced decode steps at contexts 151-196 keys
    against the oracle; Q4_0 weights quantize no activation, so the
    tolerance is f32 rounding (a lost, doubled or misplaced key moves the
    logits by far more)."""
    t = torch()
    oracle, gpu, rng = build("q4_0", seed=41, d=256, nh=4, nkv=2, max_seq=200, n_layers=1)
    toks = rng.integers(0, 300, 196).tolist()
    cache = gpu.kv_cache()
    lg = empty((150, 300), t.float32)
    gpu.forward_cached(toks[:150], 0, cache, lg)
    close(host(lg), oracle.forward_cached(toks[:150], 0), TOL["q4_0"])
    one = empty((300,), t.float32)
    for p in range(150, 196):
        gpu.forward_decode(toks[p], p, cache, one)
        close(host(one), oracle.forward_decode(toks[p], p), TOL["q4_0"])


@pytest.mark.parametrize("fmt", ["q8_0", "w4a8"])
def test_llama_prefill_wide_ffn(fmt):
    """An FFN of 65568 (over 16384 float4 per row): the prefill rows'
    SwiGLU and the down projection's row quantization, done in one pass,
    take the element-wise path there instead of the register-resident one."""
    t = torch()
    oracle, gpu, rng = build(fmt, seed=31, d=128, nh=2, nkv=2, ffn=65568, max_seq=16,
                             n_layers=1)
    toks = rng.integers(0, 300, 7).tolist()
    lg = empty((7, 300), t.float32)
    gpu.forward_cached(toks, 0, gpu.kv_cache(), lg)
    close(host(lg), oracle.forward_cached(toks, 0), TOL[fmt])


def test_llama_mixed_formats():
    """A different weight format per projection role: q/k/v and gate/up
    cannot be concatenated, so decode rows run three q/k/v projections, each
    with the RMSNorm prologue and its own RoPE / cache epilogue."""
    t = torch()
    oracle, gpu, rng = build("mixed", seed=23)
    toks = rng.integers(0, 300, 18).tolist()
    cache = gpu.kv_cache()
    lg = empty((14, 300), t.float32)
    gpu.forward_cached(toks[:14], 0, cache, lg)
    close(host(lg), oracle.forward_cached(toks[:14], 0), 2e-2)
    one = empty((300,), t.float32)
    for p in range(14, 18):
        gpu.forward_decode(toks[p], p, cache, one)
        close(host(one), oracle.forward_decode(toks[p], p), 2e-2)
    toks2 = gpu.generate_greedy(toks[:10], 4, gpu.kv_cache())
    assert toks2.shape == (5,)


def test_llama_gqa_and_mha_head_dim_128():
    """n_kv_heads == n_heads (MHA) with head_dim 128, the 7B geometry, and a
    prefill that starts past position 0."""
    t = torch()
    oracle, gpu, rng = build("q4_0", seed=5, d=256, nh=2, nkv=2, ffn=384, max_seq=40,
                             n_layers=1)
    toks = rng.integers(0, 300, 30).tolist()
    cache = gpu.kv_cache()
    lg = empty((17, 300), t.float32)
    gpu.forward_cached(toks[:17], 0, cache, lg)
    close(host(lg), oracle.forward_cached(toks[:17], 0), 1e-4)
    lg2 = empty((13, 300), t.float32)
    gpu.forward_cached(toks[17:], 17, cache, lg2)  # a second chunk at start_pos 17
    close(host(lg2), oracle.forward_cached(toks[17:], 17), 1e-4)


def test_llama_int8_ffn_not_whole_tiles():
    """ffn = 300 is not a multiple of 16: wq/wk/wv run as one fused
    projection, wgate/wup as two (the fused [wgate; wup] needs whole 16-row
    tiles).  Both layouts agree with the oracle."""
    t = torch()
    oracle, gpu, rng = build("int8", seed=17, ffn=300, n_layers=1)
    toks = rng.integers(0, 300, 9).tolist()
    cache = gpu.kv_cache()
    lg = empty((8, 300), t.float32)
    gpu.forward_cached(toks[:8], 0, cache, lg)
    close(host(lg), oracle.forward_cached(toks[:8], 0), 2e-2)
    one = empty((300,), t.float32)
    gpu.forward_decode(toks[8], 8, cache, one)
    close(host(one), oracle.forward_decode(toks[8], 8), 2e-2)


def test_llama_decode_matches_prefill_rows_q8_0():
    """Per-row activation quantization: decoding token p after a prefill of
    0..p-1 gives prefill row p (the oracle's rows are bit-identical; the GPU
    attention sums differ in order between the two launch shapes only)."""
    t = torch()
    _, gpu, rng = build("q8_0", seed=7)
    toks = rng.integers(0, 300, 16).tolist()
    c1 = gpu.kv_cache()
    full = empty((16, 300), t.float32)
    gpu.forward_cached(toks, 0, c1, full)
    c2 = gpu.kv_cache()
    part = empty((12, 300), t.float32)
    gpu.forward_cached(toks[:12], 0, c2, part)
    one = empty((300,), t.float32)
    for p in range(12, 16):
        gpu.forward_decode(toks[p], p, c2, one)
        close(host(one), host(full)[p], 2e-2)


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0", "w4a8"])
def test_llama_generate_greedy(fmt):
    """Device-resident greedy loop: every chosen token is the oracle's
    argmax of the oracle's logits on the same (teacher-forced) prefix, or
    within the comparison tolerance of it."""
    t = torch()
    oracle, gpu, rng = build(fmt, seed=11)
    prompt = rng.integers(0, 300, 16).tolist()
    cache = gpu.kv_cache()
    steps = 12
    lg = empty((steps + 1, 300), t.float32)
    toks = gpu.generate_greedy(prompt, steps, cache, lg)
    assert toks.shape == (steps + 1,)
    ref_rows = [oracle.forward_cached(prompt, 0)[-1]]
    for i in range(steps):
        ref_rows.append(oracle.forward_decode(int(toks[i]), len(prompt) + i))
    ref = np.stack(ref_rows)
    close(host(lg), ref, TOL[fmt])
    g = host(lg)
    for i in range(steps + 1):
        assert toks[i] == O.argmax(g[i])  # the GPU picked its own argmax
        margin = ref[i].max() - ref[i][toks[i]]
        assert margin <= TOL[fmt] * np.abs(ref[i]).max(), f"step {i}: margin {margin}"


@pytest.mark.parametrize("fmt", ["q8_0", "int8"])
def test_llama_generate_greedy_ties(fmt):
    """The greedy loop's argmax (in the output projection's epilogue) on
    ties: only rows 7 and 123 of the output weights are non-zero, and equal,
    so those two logits are equal and every other one is exactly zero; each
    step must choose the last of its equal maxima (123 when their value is
    positive, else 299), as the reference's max_by does."""
    t = torch()
    rng = np.random.default_rng(21)
    w = np.zeros((300, 256), F32)
    w[7] = w[123] = (rng.standard_normal(256) * 0.05).astype(F32)
    _, gpu, rng = build(fmt, seed=12, out_w=w)
    prompt = rng.integers(0, 300, 9).tolist()
    steps = 6
    lg = empty((steps + 1, 300), t.float32)
    toks = gpu.generate_greedy(prompt, steps, gpu.kv_cache(), lg)
    g = host(lg)
    for i in range(steps + 1):
        assert g[i][7] == g[i][123] and np.count_nonzero(g[i]) <= 2
        want = 123 if g[i][123] > 0 else 299
        assert toks[i] == want == O.argmax(g[i]), f"step {i}: {toks[i]} (logit {g[i][123]})"


def test_argmax_last_of_ties():
    t = torch()
    L, _ = mods()
    rng = np.random.default_rng(4)
    v = rng.standard_normal((3, 32000)).astype(F32)
    v[1, 5] = v[1, 31999] = v[1, 777] = 9.0  # ties: the last wins
    v[2, :] = -1.0
    idx = empty((3,), t.int32)
    L.argmax(dev(v), idx)
    got = host(idx).view(np.uint32)
    assert got[0] == O.argmax(v[0]) and got[1] == 31999 and got[2] == 31999


def test_llama_errors():
    t = torch()
    L, Q = mods()
    _, gpu, _ = build("q8_0", seed=13, n_layers=1)
    cache = gpu.kv_cache()
    lg = empty((4, 300), t.float32)
    with pytest.raises(Q.MriError) as e:
        gpu.forward_cached([1, 2, 300], 0, cache, lg)  # id >= vocab (forward_int8.rs:132)
    assert e.value.kind == "InvalidShape"
    with pytest.raises(Q.MriError) as e:
        gpu.forward_cached([1, 2], 47, cache, lg)  # past the cache
    assert e.value.kind == "InvalidShape"
    with pytest.raises(Q.MriError) as e:
        gpu.forward_cached([], 0, cache, lg)
    assert e.value.kind == "InvalidShape"
    other = L.KvCache(2, 48, 2, 64)  # two layers: not this model's cache
    with pytest.raises(Q.MriError) as e:
        gpu.forward_cached([1], 0, other, lg)
    assert e.value.kind == "ShapeMismatch"


@pytest.mark.parametrize("n", [1, 5, 513, 32000, 70001])
def test_argmax_one_row(n):
    """One row runs the split kernel (its blocks meet through a counter that
    every call leaves at zero): the oracle's choice on random values, ties
    (the last wins), -0.0 against +0.0 (equal, so the last wins), NaN away
    from element 0 (never chosen; the reference panics on NaN) and an
    all-NaN row (0), over consecutive calls."""
    t = torch()
    L, _ = mods()
    rng = np.random.default_rng(n)
    idx = empty((1,), t.int32)
    for trial in range(5):
        v = rng.standard_normal(n).astype(F32)
        if trial == 1 and n > 2:
            v[[0, n // 2, n - 1]] = 9.0
        elif trial == 2:
            v[:] = -0.0
            v[rng.integers(0, n, max(1, n // 4))] = 0.0
        elif trial == 3 and n > 1:
            v[1 + rng.integers(0, n - 1, max(1, n // 3))] = np.nan
        elif trial == 4:
            v[:] = np.nan
        L.argmax(dev(v), idx)
        got = int(host(idx).view(np.uint32)[0])
        assert got == O.argmax(v), f"trial {trial}"


@pytest.mark.parametrize("fmt", ["q8_0", "int8"])
def test_llama_zero_layers(fmt):
    """No decoder layers: the output projection reads the embedding row
    (decode rows: in place, with the output RMSNorm in its prologue; the
    greedy loop: the row its argmax gathered)."""
    t = torch()
    oracle, gpu, rng = build(fmt, seed=29, n_layers=0)
    toks = rng.integers(0, 300, 8).tolist()
    cache = gpu.kv_cache()
    lg = empty((5, 300), t.float32)
    gpu.forward_cached(toks[:5], 0, cache, lg)
    close(host(lg), oracle.forward_cached(toks[:5], 0), 2e-2)
    one = empty((300,), t.float32)
    for p in range(5, 8):
        gpu.forward_decode(toks[p], p, cache, one)
        close(host(one), oracle.forward_decode(toks[p], p), 2e-2)
    steps = 4
    glg = empty((steps + 1, 300), t.float32)
    got = gpu.generate_greedy(toks[:5], steps, gpu.kv_cache(), glg)
    ref = [oracle.forward_cached(toks[:5], 0)[-1]]
    for i in range(steps):
        ref.append(oracle.forward_decode(int(got[i]), 5 + i))
    close(host(glg), np.stack(ref), 2e-2)

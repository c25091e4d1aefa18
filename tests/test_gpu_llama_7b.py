"""One LlamaModelInt8 decoder layer at the Llama-7B geometry on the GPU:
hidden 4096, 32 heads of 128 (n_kv_heads = 32), SwiGLU FFN 11008, vocab
32000, RMSNorm eps 1e-6, RoPE base 10000 (forward_int8.rs:148-546).

This is the code the 7B layer runs and the small-model tests do not reach:
- prefill chunks of 64 and more rows (the GEMM / skinny-above-32-rows
  projections, k_rmsnorm over 4096 columns, the matrix-core attention
  k_attention_mfma over up to 130 keys, the second chunk at start_pos 66);
- decode steps at contexts of 131-133 keys (three 64-key chunks of the split
  decode attention, k_attn_decode_part, and their combine in the last
  workgroup of each head) and, in the property test below, past 1024 keys
  (17 chunks);
- the decode row-operation GEMVs at their 7B sizes (the fused 12288-row
  q/k/v projection with RoPE and the cache write in its epilogue, the fused
  22016-row gate/up, down with K = 11008 adding into the residual row, the
  32000-row output projection).

Teacher-forced against the oracle's composition (tests/oracle_lib.py
LlamaOracle over oracle/llama.c).  Tolerances, relative to the largest
logit magnitude:
- Q4_0 weights (W4A32, no activation quantization): 1e-4.  Only f32
  rounding differs (the layer's row sums run as tree sums on the GPU);
  measured at this geometry: at most 2e-5 on every prefill and decode row.
  This pins the layer's logic (heads, positions, RoPE, mask, the chunked
  decode attention and its combine) at the 7B sizes.
- Q8_0, W4A8 and per-channel INT8 (int8 activations): 4e-2.  A last-bit f32
  difference before a quantization moves one activation element by one
  step, and at this geometry that moves a row's logits by up to 2.6 %
  (measured: each row is either bit-identical to the oracle or 1-2.6 % off,
  with the same layer built with Q4_0 weights at 2e-5).  A wrong head,
  position or mask moves them by O(1).
The oracle's projections run on several host threads over slices of the
output rows; each output depends on its own weight row only, so the result
is the single-threaded oracle's bit for bit.

The full-size property test (512-token prompt, 128 greedy steps) needs no
oracle: each decoded token's logits equal the prefill row at its position
(per-row activation quantization, so the two launch shapes see the same
arithmetic up to f32 summation order), and each chosen token is the argmax of
its own logits row."""
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import closed_form as CF
import oracle_lib as O
from gpu_util import dev, empty, host

pytestmark = pytest.mark.gpu

F32 = np.float32
D, NH, HD, FFN, VOCAB = 4096, 32, 128, 11008, 32000
TOL = {"q4_0": 1e-4, "q8_0": 4e-2, "int8": 4e-2, "w4a8": 4e-2}
POOL = ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 4))


def torch():
    import torch as t
    return t


def mods():
    import mri_llama as L
    import mri_qmatmul as Q
    return L, Q


def say(msg):
    print(msg, flush=True)


class ParProj(O.Proj):
    """The oracle projection split over slices of the output rows (runs on
    POOL; ctypes releases the GIL).  INT8: the activation is quantized per
    tensor over the whole input first (quantize_symmetric, as
    matmul_int8_from_f32), then each slice runs matmul_int8 (the oracle's
    row-parallel matmul_int8_parallel serves one caller at a time);
    Q8_0: matmul_q8_0_direct quantizes each input row on its own, and Q4_0
    (matmul_q4_0_dequant) does not quantize, so slices of the weight rows
    are independent as they are."""

    SLICE = 256

    def __call__(self, x):
        x = np.ascontiguousarray(x, F32)
        m, n, k = x.shape[0], self.n_out, self.k_in
        out = np.empty((m, n), F32)
        cuts = list(range(0, n, self.SLICE)) + [n]
        if self.fmt == "int8":
            aq, sa = O.quantize_symmetric(x.ravel())

            def run(i):
                a, b = cuts[i], cuts[i + 1]
                out[:, a:b] = O.matmul_int8(aq, sa, self.data[a:b], self.scales[a:b], m)
        elif self.fmt == "q8_0":
            row = (k // 32) * 34

            def run(i):
                a, b = cuts[i], cuts[i + 1]
                out[:, a:b] = O.matmul_q8_0_direct(x, self.data[a * row:b * row], b - a, k)
        elif self.fmt == "w4a8":
            row = (k // 32) * 18

            def run(i):
                a, b = cuts[i], cuts[i + 1]
                out[:, a:b] = O.matmul_q4_0_w4a8(x, self.data[a * row:b * row], b - a, k)
        else:
            row = (k // 32) * 18

            def run(i):
                a, b = cuts[i], cuts[i + 1]
                out[:, a:b] = O.matmul_q4_0_dequant(x, self.data[a * row:b * row], b - a, k)
        list(POOL.map(run, range(len(cuts) - 1)))
        return out


def synth(fmt, rng, n, k):
    """Random weights of the format with a realistic magnitude (element
    standard deviation ~0.02, as N(0, 0.02) weights): quants uniform in
    [-127, 127] (Q8_0: some -128, which the Q8_0 format allows), scales
    around 0.02 / 73; Q4_0: random nibbles (quants -8..7, standard deviation
    4.6), scales around 0.02 / 4.6."""
    if fmt in ("q4_0", "w4a8"):
        raw = np.empty((n, k // 32, 18), np.uint8)
        raw[:, :, 2:] = rng.integers(0, 256, (n, k // 32, 16), dtype=np.uint8)
        d = rng.uniform(3.8e-3, 4.9e-3, (n, k // 32)).astype(np.float16).view(np.uint16)
        raw[:, :, 0] = d & 0xFF
        raw[:, :, 1] = d >> 8
        return raw.ravel(), None
    if fmt == "int8":
        data = rng.integers(-127, 128, (n, k), dtype=np.int8)
        scales = rng.uniform(2e-4, 3.5e-4, n).astype(F32)
        return data, scales
    q = rng.integers(-128, 128, (n, k), dtype=np.int8)
    d = rng.uniform(2e-4, 3.5e-4, (n, k // 32)).astype(np.float16).view(np.uint16)
    return CF.q8_0_pack(d, q), None


def build_7b(fmt, seed, max_seq):
    L, Q = mods()
    rng = np.random.default_rng(seed)
    cfg = dict(dim=D, n_heads=NH, n_kv_heads=NH, head_dim=HD, ffn=FFN, vocab=VOCAB,
               max_seq=max_seq, eps=1e-6, rope_base=10000.0)

    def proj(n, k):
        data, scales = synth(fmt, rng, n, k)
        if fmt == "int8":
            return ParProj("int8", n, k, data, scales), Q.QMatrix.from_host(data, scales)
        if fmt == "q4_0":
            return ParProj("q4_0", n, k, data), (dev(data), n, k)
        if fmt == "w4a8":
            return ParProj("w4a8", n, k, data), Q.Q4Matrix.from_raw_bytes(data, n, k)
        return ParProj("q8_0", n, k, data), Q.Q8Matrix.from_raw_bytes(data, n, k)

    an = rng.uniform(0.8, 1.2, D).astype(F32)
    fn = rng.uniform(0.8, 1.2, D).astype(F32)
    ol, gl = dict(attn_norm=an, ffn_norm=fn), dict(attn_norm=an, ffn_norm=fn)
    for name, (n, k) in (("wq", (D, D)), ("wk", (D, D)), ("wv", (D, D)), ("wo", (D, D)),
                         ("wgate", (FFN, D)), ("wup", (FFN, D)), ("wdown", (D, FFN))):
        ol[name], gl[name] = proj(n, k)
    embd = rng.standard_normal((VOCAB, D), dtype=F32)
    onorm = rng.uniform(0.8, 1.2, D).astype(F32)
    o_out, g_out = proj(VOCAB, D)
    oracle = O.LlamaOracle(cfg, embd, [ol], onorm, o_out)
    gpu = L.Llama(cfg, embd, onorm, g_out, [gl])
    return oracle, gpu, rng


def close(got, ref, what, tol):
    scale = float(np.abs(ref).max())
    err = float(np.abs(got - ref).max())
    assert err <= tol * scale, f"{what}: max |gpu - ref| = {err:.3g} > {tol} * {scale:.3g}"


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0", "int8", "w4a8"])
def test_llama_7b_layer_teacher_forced(fmt):
    """Prefill 66 rows at position 0 and 64 rows at position 66, then three
    decode steps at positions 130-132 and a 4-step greedy run on a fresh
    cache, each compared with the oracle on the same tokens."""
    t = torch()
    say(f"7B layer {fmt}: building")
    oracle, gpu, rng = build_7b(fmt, seed={"q8_0": 71, "int8": 72, "q4_0": 74, "w4a8": 77}[fmt],
                                max_seq=160)
    tol = TOL[fmt]
    toks = rng.integers(0, VOCAB, 133).tolist()
    cache = gpu.kv_cache()
    for start, stop in ((0, 66), (66, 130)):
        say(f"7B layer {fmt}: prefill rows {start}..{stop - 1}")
        lg = empty((stop - start, VOCAB), t.float32)
        gpu.forward_cached(toks[start:stop], start, cache, lg)
        ref = oracle.forward_cached(toks[start:stop], start)
        close(host(lg), ref, f"prefill {start}..{stop - 1}", tol)
    one = empty((VOCAB,), t.float32)
    for p in range(130, 133):
        say(f"7B layer {fmt}: decode at position {p}")
        gpu.forward_decode(toks[p], p, cache, one)
        close(host(one), oracle.forward_decode(toks[p], p), f"decode at {p}", tol)
    steps = 4
    say(f"7B layer {fmt}: generate_greedy 130 + {steps}")
    glg = empty((steps + 1, VOCAB), t.float32)
    got = gpu.generate_greedy(toks[:130], steps, gpu.kv_cache(), glg)
    # generate_greedy prefills the 130 rows in one chunk: per-tensor INT8
    # activation scales span those rows, so the oracle does the same
    ref = [oracle.forward_cached(toks[:130], 0)[-1]]
    for i in range(steps):
        ref.append(oracle.forward_decode(int(got[i]), 130 + i))
    ref = np.stack(ref)
    g = host(glg)
    close(g, ref, "generate_greedy logits", tol)
    for i in range(steps + 1):
        assert got[i] == O.argmax(g[i]), f"step {i}: not the argmax of its own logits"
        margin = ref[i].max() - ref[i][got[i]]
        assert margin <= tol * np.abs(ref[i]).max(), f"step {i}: margin {margin}"


def test_llama_7b_layer_512_prompt_128_steps_q8_0():
    """The benchmark's run (512-token prompt, 128 greedy steps) checked by
    properties at full size: generate_greedy's logits row i equals the
    logits of position 511 + i from one prefill over the prompt and the
    generated tokens, and every token is the argmax of its own row."""
    t = torch()
    say("7B layer q8_0 512 + 128: building")
    _, gpu, rng = build_7b("q8_0", seed=73, max_seq=640)
    prompt = rng.integers(0, VOCAB, 512).tolist()
    steps = 128
    glg = empty((steps + 1, VOCAB), t.float32)
    say("7B layer q8_0 512 + 128: generate_greedy")
    got = gpu.generate_greedy(prompt, steps, gpu.kv_cache(), glg)
    g = host(glg)
    for i in range(steps + 1):
        assert got[i] == O.argmax(g[i]), f"step {i}: not the argmax of its own logits"
    seq = prompt + [int(v) for v in got[:steps]]
    say("7B layer q8_0 512 + 128: prefill of all 640 positions")
    full = empty((len(seq), VOCAB), t.float32)
    gpu.forward_cached(seq, 0, gpu.kv_cache(), full)
    f = host(full)[511:]
    for i in range(steps + 1):
        close(g[i], f[i], f"step {i} vs prefill row {511 + i}", TOL["q8_0"])


def test_llama_7b_layer_decode_past_1024_keys_q4_0():
    """Decode at contexts of 1029-1032 keys, where the attention splits each
    head's keys over workgroups and the last one combines them: greedy steps
    after a 1028-token prompt give the logits of one prefill over the same
    1032 tokens.  Q4_0 weights (W4A32) quantize no activation, so the two
    launch shapes differ only in f32 summation order: 1e-4 of the largest
    logit (a lost or doubled 64-key chunk moves them by far more)."""
    t = torch()
    say("7B layer q4_0 1028 + 4: building")
    _, gpu, rng = build_7b("q4_0", seed=76, max_seq=1088)
    prompt = rng.integers(0, VOCAB, 1028).tolist()
    steps = 4
    glg = empty((steps + 1, VOCAB), t.float32)
    say("7B layer q4_0 1028 + 4: generate_greedy")
    got = gpu.generate_greedy(prompt, steps, gpu.kv_cache(), glg)
    g = host(glg)
    for i in range(steps + 1):
        assert got[i] == O.argmax(g[i]), f"step {i}: not the argmax of its own logits"
    seq = prompt + [int(v) for v in got[:steps]]
    say("7B layer q4_0 1028 + 4: prefill of all 1032 positions")
    full = empty((len(seq), VOCAB), t.float32)
    gpu.forward_cached(seq, 0, gpu.kv_cache(), full)
    f = host(full)[1027:]
    for i in range(steps + 1):
        close(g[i], f[i], f"step {i} vs prefill row {1027 + i}", TOL["q4_0"])

"""GGUF files into the GPU model (mini-rust-inference_amd/mri_gguf.py
load_llama) against the oracle's LlamaModelInt8 composition on the same
weights: "int8" mode (the reference's from_loader: f32 extraction, then
quantize_per_channel) and "direct" mode (Q8_0 tensors straight into Q8_0
handles, Q4_0 into W4A8 handles).  Tolerances as in test_gpu_llama.py."""
import numpy as np
import pytest

import closed_form as CF
import oracle_lib as O
from gpu_util import empty, host

pytestmark = pytest.mark.gpu

F32 = np.float32
D, NH, NKV, FFN, VOCAB, LAYERS, CTX = 256, 4, 2, 512, 300, 2, 40


def torch():
    import torch as t
    return t


def write_model(path, wfmt, rng, ggml_order=False):
    """A random Llama written as GGUF: F16 embedding, F32 norms, projections
    and output in wfmt ("q8_0", "q4_0" or "f32").  Returns the arrays the
    oracle needs: (embd f32, onorm, output weight, layers)."""
    import mri_gguf as G
    hd = D // NH
    meta = {"general.architecture": "llama", "llama.block_count": LAYERS,
            "llama.embedding_length": D, "llama.attention.head_count": NH,
            "llama.attention.head_count_kv": NKV, "llama.feed_forward_length": FFN,
            "llama.context_length": CTX, "llama.vocab_size": VOCAB,
            "llama.rope.freq_base": 10000.0,
            "llama.attention.layer_norm_rms_epsilon": 1e-6}
    tensors = {}

    def weight(name, n, k):
        w = (rng.standard_normal((n, k)) * 0.05).astype(F32)
        if wfmt == "q8_0":
            raw = O.quantize_q8_0(w)
            tensors[name] = (G.Q8_0, (n, k), raw)
            return ("q8_0", raw, O.dequantize_q8_0(raw).reshape(n, k))
        if wfmt == "q4_0":
            raw = O.quantize_q4_0(w)
            disk = CF.q4_0_interleaved_to_ggml(raw) if ggml_order else raw
            tensors[name] = (G.Q4_0, (n, k), disk)
            return ("q4_0", raw, O.dequantize_q4_0(raw).reshape(n, k))
        tensors[name] = (G.F32, (n, k), w)
        return ("f32", None, w)

    embd = rng.standard_normal((VOCAB, D)).astype(np.float16)
    tensors["token_embd.weight"] = (G.F16, (VOCAB, D), embd)
    onorm = rng.uniform(0.8, 1.2, D).astype(F32)
    tensors["output_norm.weight"] = (G.F32, (D,), onorm)
    out = weight("output.weight", VOCAB, D)
    layers = []
    for i in range(LAYERS):
        L = {"attn_norm": rng.uniform(0.8, 1.2, D).astype(F32),
             "ffn_norm": rng.uniform(0.8, 1.2, D).astype(F32)}
        tensors[f"blk.{i}.attn_norm.weight"] = (G.F32, (D,), L["attn_norm"])
        tensors[f"blk.{i}.ffn_norm.weight"] = (G.F32, (D,), L["ffn_norm"])
        for key, role, (n, k) in (("wq", "attn_q", (NH * hd, D)), ("wk", "attn_k", (NKV * hd, D)),
                                  ("wv", "attn_v", (NKV * hd, D)), ("wo", "attn_output", (D, NH * hd)),
                                  ("wgate", "ffn_gate", (FFN, D)), ("wup", "ffn_up", (FFN, D)),
                                  ("wdown", "ffn_down", (D, FFN))):
            L[key] = weight(f"blk.{i}.{role}.weight", n, k)
        layers.append(L)
    G.write_gguf(path, meta, tensors)
    return embd.astype(F32), onorm, out, layers


def oracle_model(mode, embd, onorm, out, layers):
    """LlamaOracle on the weights the loader should produce."""
    def proj(w):
        fmt, raw, wf = w
        n, k = wf.shape
        if mode == "direct" and fmt == "q8_0":
            return O.Proj("q8_0", n, k, raw)
        if mode == "direct" and fmt == "q4_0":
            return O.Proj("w4a8", n, k, raw)
        data, scales = O.quantize_per_channel(wf, n, k)
        return O.Proj("int8", n, k, data, scales)
    cfg = dict(dim=D, n_heads=NH, n_kv_heads=NKV, head_dim=D // NH, ffn=FFN, vocab=VOCAB,
               max_seq=CTX, eps=float(F32(1e-6)), rope_base=10000.0)
    ol = []
    for L in layers:
        d = dict(attn_norm=L["attn_norm"], ffn_norm=L["ffn_norm"])
        for key in ("wq", "wk", "wv", "wo", "wgate", "wup", "wdown"):
            d[key] = proj(L[key])
        ol.append(d)
    return O.LlamaOracle(cfg, embd, ol, onorm, proj(out))


def close(got, ref, frac):
    scale = float(np.abs(ref).max())
    err = float(np.abs(got - ref).max())
    assert err <= frac * scale, f"max |gpu - ref| = {err:.3g} > {frac} * {scale:.3g}"


@pytest.mark.parametrize("wfmt,mode,ggml", [("q8_0", "direct", False), ("q8_0", "int8", False),
                                           ("f32", "direct", False), ("q4_0", "direct", False),
                                           ("q4_0", "direct", True), ("q4_0", "int8", False)])
def test_load_llama_matches_oracle(tmp_path, wfmt, mode, ggml):
    import mri_gguf as G
    import mri_qmatmul as Q
    t = torch()
    rng = np.random.default_rng({"q8_0": 1, "f32": 2, "q4_0": 3}[wfmt])
    path = tmp_path / "m.gguf"
    arrays = write_model(path, wfmt, rng, ggml_order=ggml)
    model, cfg = G.load_llama(path, mode=mode,
                              q4_order=Q.Q4_ORDER_GGML if ggml else Q.Q4_ORDER_INTERLEAVED)
    assert (cfg["n_layers"], cfg["vocab"], cfg["max_seq"]) == (LAYERS, VOCAB, CTX)
    oracle = oracle_model(mode, *arrays)
    toks = rng.integers(0, VOCAB, 14).tolist()
    cache = model.kv_cache()
    lg = empty((12, VOCAB), t.float32)
    model.forward_cached(toks[:12], 0, cache, lg)
    close(host(lg), oracle.forward_cached(toks[:12], 0), 2e-2)
    one = empty((VOCAB,), t.float32)
    for p in (12, 13):
        model.forward_decode(toks[p], p, cache, one)
        close(host(one), oracle.forward_decode(toks[p], p), 2e-2)

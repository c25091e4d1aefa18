"""GGUF reader (mini-rust-inference_amd/gguf.py) on the CPU: header,
metadata and tensor-info parsing, alignment, dequantization (checked against
the oracle's dequantize_q8_0 / dequantize_q4_0, which the reference's KATs
pin), and LlamaConfig::from_metadata's rules (model/llama/config.rs:66-145).
"""
import struct

import numpy as np
import pytest

import closed_form as CF
import oracle_lib as O

F32 = np.float32


def gg():
    import mri_gguf as gguf
    return gguf


def _q8(rng, n, k):
    q = rng.integers(-127, 128, (n, k)).astype(np.int8)
    d = rng.uniform(0.001, 0.01, (n, k // 32)).astype(np.float16).view(np.uint16)
    return CF.q8_0_pack(d, q)


def _q4(rng, n, k):
    raw = np.empty((n, k // 32, 18), np.uint8)
    raw[:, :, 2:] = rng.integers(0, 256, (n, k // 32, 16))
    raw[:, :, :2] = rng.uniform(0.001, 0.05, (n, k // 32)).astype(np.float16).view(
        np.uint8).reshape(n, k // 32, 2)
    return raw.ravel()


@pytest.mark.parametrize("alignment", [32, 64])
def test_roundtrip_and_dequant(tmp_path, alignment):
    G = gg()
    rng = np.random.default_rng(0)
    f = rng.standard_normal((3, 64)).astype(F32)
    h = rng.standard_normal((5, 32)).astype(np.float16)
    q8, q4 = _q8(rng, 4, 96), _q4(rng, 6, 64)
    path = tmp_path / "t.gguf"
    G.write_gguf(path, {"general.name": "t", "a.u32": 7, "a.big": 1 << 40, "a.f": 0.5,
                        "a.flag": True, "a.list": ["x", "yz"]},
                 {"f": (G.F32, (3, 64), f), "h": (G.F16, (5, 32), h),
                  "q8": (G.Q8_0, (4, 96), q8), "q4": (G.Q4_0, (6, 64), q4)},
                 alignment=alignment)
    g = G.GgufFile(path)
    assert g.version == 3
    assert g.metadata["a.u32"] == 7 and g.metadata["a.big"] == 1 << 40
    assert g.metadata["a.f"] == 0.5 and g.metadata["a.flag"] is True
    assert g.metadata["a.list"] == ["x", "yz"] and g.metadata["general.name"] == "t"
    assert g.metadata_types["a.u32"] == 4 and g.metadata_types["a.big"] == 10
    assert g.data_offset % alignment == 0
    for name in g.tensors:
        assert (g.data_offset + g.tensors[name][2]) % alignment == 0
    assert g.shape("q8") == (4, 96) and g.shape("h") == (5, 32)
    assert np.array_equal(np.asarray(g.raw("q8")), q8)
    assert np.array_equal(np.asarray(g.raw("q4")), q4)
    assert np.array_equal(g.f32("f"), f)
    assert np.array_equal(g.f32("h"), h.astype(F32))
    assert np.array_equal(g.f32("q8").view(np.uint32),
                          O.dequantize_q8_0(q8).reshape(4, 96).view(np.uint32))
    assert np.array_equal(g.f32("q4").view(np.uint32),
                          O.dequantize_q4_0(q4).reshape(6, 64).view(np.uint32))
    # GGML nibble order: the same elements from re-encoded bytes
    gpath = tmp_path / "g.gguf"
    G.write_gguf(gpath, {}, {"q4": (G.Q4_0, (6, 64), CF.q4_0_interleaved_to_ggml(q4))})
    assert np.array_equal(G.GgufFile(gpath).f32("q4", q4_order=1), g.f32("q4"))


def test_bad_files(tmp_path):
    G = gg()
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"GGUX" + b"\0" * 28)
    with pytest.raises(G.GgufError, match="not a GGUF"):
        G.GgufFile(p)
    p.write_bytes(struct.pack("<IIQQ", G.GGUF_MAGIC, 1, 0, 0))
    with pytest.raises(G.GgufError, match="version"):
        G.GgufFile(p)
    p.write_bytes(struct.pack("<IIQQ", G.GGUF_MAGIC, 3, 0, 1) + struct.pack("<Q", 100))
    with pytest.raises(G.GgufError, match="past the end"):
        G.GgufFile(p)
    G.write_gguf(p, {}, {"w": (G.F32, (2, 8), np.zeros((2, 8), F32))})
    g = G.GgufFile(p)
    with pytest.raises(G.GgufError, match="not found"):
        g.raw("nope")


LLAMA_META = {"llama.block_count": 2, "llama.embedding_length": 256,
              "llama.attention.head_count": 4, "llama.feed_forward_length": 512,
              "llama.context_length": 48}


def _config(tmp_path, meta):
    G = gg()
    p = tmp_path / "c.gguf"
    G.write_gguf(p, meta, {})
    g = G.GgufFile(p)
    return G.llama_config(g.metadata, g.metadata_types)


def test_llama_config_rules(tmp_path):
    """config.rs:66-145: n_kv_heads falls back to n_heads, vocab comes from
    llama.vocab_size or the token list, rope base 10000 and eps 1e-5 unless
    given as f32, and the head-count checks."""
    G = gg()
    c = _config(tmp_path, dict(LLAMA_META, **{"tokenizer.ggml.tokens": ["a"] * 300}))
    assert (c["n_layers"], c["dim"], c["n_heads"], c["n_kv_heads"], c["ffn"], c["vocab"],
            c["context_length"], c["head_dim"]) == (2, 256, 4, 4, 512, 300, 48, 64)
    assert c["rope_base"] == 10000.0 and abs(c["eps"] - 1e-5) < 1e-12
    c = _config(tmp_path, dict(LLAMA_META, **{"llama.vocab_size": 32000,
                                              "llama.attention.head_count_kv": 2,
                                              "llama.rope.freq_base": 500000.0,
                                              "llama.attention.layer_norm_rms_epsilon": 1e-6}))
    assert c["vocab"] == 32000 and c["n_kv_heads"] == 2 and c["rope_base"] == 500000.0
    assert c["eps"] == float(np.float32(1e-6))
    with pytest.raises(G.GgufError, match="llama.vocab_size"):
        _config(tmp_path, LLAMA_META)
    for key in LLAMA_META:
        meta = dict(LLAMA_META, **{"llama.vocab_size": 10})
        del meta[key]
        with pytest.raises(G.GgufError, match=key):
            _config(tmp_path, meta)
    with pytest.raises(G.GgufError, match="not divisible by n_heads"):
        _config(tmp_path, dict(LLAMA_META, **{"llama.vocab_size": 10,
                                              "llama.attention.head_count": 3}))
    with pytest.raises(G.GgufError, match="not divisible by n_kv_heads"):
        _config(tmp_path, dict(LLAMA_META, **{"llama.vocab_size": 10,
                                              "llama.attention.head_count_kv": 3}))
    # a u64 value that does not fit in u32 is absent (get_u32_wide)
    with pytest.raises(G.GgufError, match="llama.context_length"):
        _config(tmp_path, dict(LLAMA_META, **{"llama.vocab_size": 10,
                                              "llama.context_length": 1 << 33}))

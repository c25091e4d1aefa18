"""GGUF weights straight into device handles (the loading path of
LlamaModelInt8::from_loader, model/llama/forward_int8.rs:461-507).

GgufFile parses a GGUF v2/v3 file (header, metadata, tensor infos; gguf/
header.rs, metadata.rs, tensor_info.rs, loader.rs) and memory-maps its tensor
data, so a tensor's bytes are read from the file only when uploaded.
llama_config restates LlamaConfig::from_metadata (model/llama/config.rs:
66-145).  load_llama builds the GPU model (mri_llama.Llama) in one of two
ways:

  mode="int8"    the reference's from_loader: every projection is extracted
                 as f32 (F32 / F16 / Q8_0 / Q4_0 dequantized as
                 gguf/dequant.rs does) and quantized per output channel
                 (quantize_per_channel, per_channel.rs:98-128, on the GPU).
  mode="direct"  Q8_0 tensors are uploaded as they are into Q8_0 handles
                 (matmul_q8_0_direct), Q4_0 tensors into W4A8 handles, and
                 F32 / F16 projections are quantized per channel as above.

Embeddings and norm weights are f32 on the host (F16 / Q8_0 / Q4_0
dequantized).  Q4_0 bytes follow the reference's nibble order unless
q4_order is mri_qmatmul.Q4_ORDER_GGML (files written by llama.cpp).
"""
from __future__ import annotations

import struct

import numpy as np

GGUF_MAGIC = 0x46554747  # "GGUF" little-endian
DEFAULT_ALIGNMENT = 32

# GGML tensor types handled here (gguf/dtype.rs)
F32, F16, Q4_0, Q8_0 = 0, 1, 2, 8
TYPE_NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q8_0: "Q8_0"}

# metadata value types (gguf/metadata.rs)
_SCALARS = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?",
            10: "<Q", 11: "<q", 12: "<d"}
_STRING, _ARRAY = 8, 9


class GgufError(Exception):
    pass


class _Reader:
    def __init__(self, buf):
        self.buf = buf
        self.pos = 0

    def take(self, fmt):
        n = struct.calcsize(fmt)
        if self.pos + n > len(self.buf):
            raise GgufError(f"unexpected end of file at byte {self.pos}")
        v = struct.unpack_from(fmt, self.buf, self.pos)[0]
        self.pos += n
        return v

    def string(self):
        n = self.take("<Q")
        if self.pos + n > len(self.buf):
            raise GgufError(f"string of {n} bytes runs past the end of the file")
        s = bytes(self.buf[self.pos:self.pos + n]).decode("utf-8")
        self.pos += n
        return s

    def value(self, vtype):
        if vtype in _SCALARS:
            return self.take(_SCALARS[vtype])
        if vtype == _STRING:
            return self.string()
        if vtype == _ARRAY:
            et = self.take("<I")
            n = self.take("<Q")
            return [self.value(et) for _ in range(n)]
        raise GgufError(f"unknown metadata value type {vtype}")


class GgufFile:
    """A GGUF file: .metadata (dict), .tensors (name -> (type, dims, offset)),
    tensor data memory-mapped from the file."""

    def __init__(self, path):
        self.path = path
        self._map = np.memmap(path, dtype=np.uint8, mode="r")
        r = _Reader(self._map)
        if r.take("<I") != GGUF_MAGIC:
            raise GgufError(f"{path}: not a GGUF file")
        self.version = r.take("<I")
        if self.version not in (2, 3):
            raise GgufError(f"{path}: GGUF version {self.version} is not supported")
        n_tensors = r.take("<Q")
        n_kv = r.take("<Q")
        self.metadata = {}
        self.metadata_types = {}   # key -> GGUF value type
        for _ in range(n_kv):
            key = r.string()
            vtype = r.take("<I")
            self.metadata_types[key] = vtype
            self.metadata[key] = r.value(vtype)
        self.tensors = {}
        for _ in range(n_tensors):
            name = r.string()
            nd = r.take("<I")
            if nd > 8:
                raise GgufError(f"tensor {name}: {nd} dimensions")
            dims = [r.take("<Q") for _ in range(nd)]
            ttype = r.take("<I")
            off = r.take("<Q")
            self.tensors[name] = (ttype, dims, off)
        align = int(self.metadata.get("general.alignment", DEFAULT_ALIGNMENT))
        self.data_offset = (r.pos + align - 1) // align * align

    def shape(self, name):
        """Row-major shape (GGUF stores the innermost dimension first)."""
        return tuple(int(d) for d in reversed(self.tensors[name][1]))

    def dtype(self, name):
        return self.tensors[name][0]

    def nbytes(self, name):
        ttype, dims, _ = self.tensors[name]
        n = int(np.prod(dims)) if dims else 1
        if ttype == F32:
            return 4 * n
        if ttype == F16:
            return 2 * n
        if ttype in (Q8_0, Q4_0):
            if n % 32:
                raise GgufError(f"tensor {name}: {n} elements is not a multiple of 32")
            return n // 32 * (34 if ttype == Q8_0 else 18)
        raise GgufError(f"tensor {name}: type {ttype} is not supported")

    def raw(self, name):
        """The tensor's bytes (a view of the mapped file)."""
        if name not in self.tensors:
            raise GgufError(f"tensor {name!r} not found")
        start = self.data_offset + self.tensors[name][2]
        n = self.nbytes(name)
        if start + n > self._map.size:
            raise GgufError(f"tensor {name}: data runs past the end of the file")
        return self._map[start:start + n]

    def f32(self, name, q4_order=0):
        """The tensor as f32, dequantized as gguf/dequant.rs does (for Q4_0
        in the given nibble order)."""
        ttype = self.dtype(name)
        raw = np.asarray(self.raw(name))
        shape = self.shape(name)
        if ttype == F32:
            return raw.view(np.float32).reshape(shape).copy()
        if ttype == F16:
            return raw.view(np.float16).astype(np.float32).reshape(shape)
        blk = raw.reshape(-1, 34 if ttype == Q8_0 else 18)
        d = blk[:, :2].copy().view(np.float16).astype(np.float32)  # [nb, 1]
        if ttype == Q8_0:
            q = blk[:, 2:].view(np.int8).astype(np.float32)
        else:
            qs = blk[:, 2:]
            q = np.empty((blk.shape[0], 32), np.float32)
            if q4_order == 1:
                q[:, :16] = (qs & 0x0F).astype(np.float32) - 8
                q[:, 16:] = (qs >> 4).astype(np.float32) - 8
            else:
                q[:, 0::2] = (qs & 0x0F).astype(np.float32) - 8
                q[:, 1::2] = (qs >> 4).astype(np.float32) - 8
        return (q * d).astype(np.float32).reshape(shape)


def _u32_wide(meta, types, key):
    """Metadata::get_u32, else get_u64 narrowed to u32 (config.rs:152-156):
    unsigned 8/16/32-bit values, or a 64-bit one that fits."""
    t = types.get(key)
    v = meta.get(key)
    if t in (0, 2, 4):
        return v
    if t == 10 and v <= 0xFFFFFFFF:
        return v
    return None


def _f32(meta, types, key):
    """Metadata::get_f32: a Float32 value only."""
    return meta[key] if types.get(key) == 6 else None


def llama_config(meta, types):
    """LlamaConfig::from_metadata (model/llama/config.rs:66-145): required
    llama.* keys, n_kv_heads falling back to n_heads, vocab from
    llama.vocab_size or the tokenizer's token list, rope base 10000 and
    RMSNorm eps 1e-5 by default, and the head-count checks.  types maps
    each key to its GGUF value type (GgufFile.metadata_types)."""
    cfg = {}
    for key, name in (("llama.block_count", "n_layers"), ("llama.embedding_length", "dim"),
                      ("llama.attention.head_count", "n_heads"),
                      ("llama.feed_forward_length", "ffn"),
                      ("llama.context_length", "context_length")):
        v = _u32_wide(meta, types, key)
        if v is None:
            raise GgufError(f"missing metadata key: {key}")
        cfg[name] = v
    kv = _u32_wide(meta, types, "llama.attention.head_count_kv")
    cfg["n_kv_heads"] = cfg["n_heads"] if kv is None else kv
    vocab = _u32_wide(meta, types, "llama.vocab_size")
    tokens = meta.get("tokenizer.ggml.tokens")
    if vocab is None and types.get("tokenizer.ggml.tokens") == _ARRAY and \
            all(isinstance(t, str) for t in tokens):
        vocab = len(tokens)
    if vocab is None:
        raise GgufError("missing metadata key: llama.vocab_size")
    cfg["vocab"] = vocab
    base = _f32(meta, types, "llama.rope.freq_base")
    cfg["rope_base"] = 10000.0 if base is None else base
    eps = _f32(meta, types, "llama.attention.layer_norm_rms_epsilon")
    cfg["eps"] = 1e-5 if eps is None else eps
    if cfg["n_heads"] == 0:
        raise GgufError("n_heads must be > 0")
    if cfg["dim"] % cfg["n_heads"]:
        raise GgufError(f"embedding_length {cfg['dim']} not divisible by n_heads "
                        f"{cfg['n_heads']}")
    if cfg["n_kv_heads"] == 0 or cfg["n_heads"] % cfg["n_kv_heads"]:
        raise GgufError(f"n_heads {cfg['n_heads']} not divisible by n_kv_heads "
                        f"{cfg['n_kv_heads']}")
    cfg["head_dim"] = cfg["dim"] // cfg["n_heads"]
    return cfg


LAYER_ROLES = (("wq", "attn_q"), ("wk", "attn_k"), ("wv", "attn_v"), ("wo", "attn_output"),
               ("wgate", "ffn_gate"), ("wup", "ffn_up"), ("wdown", "ffn_down"))


def _projection(g, name, mode, q4_order):
    """One [n_out, k_in] weight as a device handle."""
    import torch

    import mri_qmatmul as Q
    n_out, k_in = g.shape(name)
    ttype = g.dtype(name)
    if mode == "direct" and ttype in (Q8_0, Q4_0):
        raw = torch.from_numpy(np.asarray(g.raw(name)).copy()).cuda()
        if ttype == Q8_0:
            return Q.Q8Matrix.from_raw_device(raw, n_out, k_in)
        return Q.Q4Matrix.from_raw_device(raw, n_out, k_in, q4_order)
    w = torch.from_numpy(g.f32(name, q4_order)).cuda()
    data = torch.empty((n_out, k_in), dtype=torch.int8, device="cuda")
    scales = torch.empty(n_out, dtype=torch.float32, device="cuda")
    Q.quantize_per_channel(w, n_out, k_in, data, scales)
    return Q.QMatrix.from_device(data, scales)


def load_llama(path, mode="direct", max_seq=None, q4_order=0):
    """LlamaModelInt8::from_loader on the GPU.  Returns (model, config);
    max_seq (default: the file's context length) sizes the activation
    buffers and the RoPE table."""
    import mri_llama as L
    if mode not in ("direct", "int8"):
        raise ValueError(f"mode must be 'direct' or 'int8', not {mode!r}")
    g = GgufFile(path)
    cfg = llama_config(g.metadata, g.metadata_types)
    cfg["max_seq"] = cfg["context_length"] if max_seq is None else max_seq
    emb = g.f32("token_embd.weight", q4_order)
    onorm = g.f32("output_norm.weight", q4_order)
    out = _projection(g, "output.weight", mode, q4_order)
    layers = []
    for i in range(cfg["n_layers"]):
        layer = {"attn_norm": g.f32(f"blk.{i}.attn_norm.weight", q4_order),
                 "ffn_norm": g.f32(f"blk.{i}.ffn_norm.weight", q4_order)}
        for key, role in LAYER_ROLES:
            layer[key] = _projection(g, f"blk.{i}.{role}.weight", mode, q4_order)
        layers.append(layer)
    return L.Llama(cfg, emb, onorm, out, layers), cfg


def write_gguf(path, metadata, tensors, alignment=DEFAULT_ALIGNMENT):
    """Writes a GGUF v3 file: metadata {key: value} (int -> u32, or u64 when
    it does not fit; float -> f32; str; list of str) and tensors
    {name: (ggml type, row-major shape, raw bytes)}.  For fixtures and
    tests."""
    def s(x):
        b = x.encode("utf-8")
        return struct.pack("<Q", len(b)) + b

    def val(v):
        if isinstance(v, bool):
            return struct.pack("<I?", 7, v)
        if isinstance(v, int):
            return struct.pack("<II", 4, v) if v <= 0xFFFFFFFF else struct.pack("<IQ", 10, v)
        if isinstance(v, float):
            return struct.pack("<If", 6, v)
        if isinstance(v, str):
            return struct.pack("<I", _STRING) + s(v)
        if isinstance(v, list):
            return struct.pack("<IIQ", _ARRAY, _STRING, len(v)) + b"".join(s(x) for x in v)
        raise TypeError(type(v))

    meta = dict(metadata)
    if alignment != DEFAULT_ALIGNMENT:
        meta["general.alignment"] = alignment
    head = struct.pack("<IIQQ", GGUF_MAGIC, 3, len(tensors), len(meta))
    head += b"".join(s(k) + val(v) for k, v in meta.items())
    blobs, off = [], 0
    for name, (ttype, shape, data) in tensors.items():
        data = bytes(np.ascontiguousarray(data).view(np.uint8).ravel())
        dims = list(reversed([int(d) for d in shape]))
        head += s(name) + struct.pack("<I", len(dims)) + b"".join(
            struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", ttype, off)
        pad = (-len(data)) % alignment
        blobs.append(data + b"\0" * pad)
        off += len(data) + pad
    head += b"\0" * ((-len(head)) % alignment)
    with open(path, "wb") as f:
        f.write(head)
        for b in blobs:
            f.write(b)

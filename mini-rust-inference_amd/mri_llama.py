"""ctypes binding of the GPU LlamaModelInt8 (include/mri_llama.h).

Host plumbing for tests and benchmarks over libmri_qmatmul.so: weights are
the handles of mri_qmatmul (QMatrix / Q8Matrix) or device Q4_0 byte
tensors, logits are torch CUDA (HIP) tensors.  No CPU fallback: every call
runs the HIP kernels.
"""
from __future__ import annotations

import ctypes as C

import mri_qmatmul as Q

P = C.c_void_p
SZ = C.c_size_t
ST = C.c_int

INT8, Q8_0, Q4_0, Q4_0_W4A8 = 0, 1, 2, 3


class Config(C.Structure):
    _fields_ = [("dim", SZ), ("n_heads", SZ), ("n_kv_heads", SZ), ("ffn_dim", SZ),
                ("vocab", SZ), ("max_seq", SZ), ("eps", C.c_float), ("rope_base", C.c_float),
                ("n_layers", SZ)]


class WeightRef(C.Structure):
    _fields_ = [("format", C.c_int), ("ptr", P), ("n_out", SZ), ("k_in", SZ)]


_SIGS = {
    "mri_llama_create": ([C.POINTER(Config), P, P, WeightRef, C.POINTER(P)], ST),
    "mri_llama_set_layer": ([P, SZ, P, P, C.POINTER(WeightRef)], ST),
    "mri_llama_destroy": ([P], None),
    "mri_kv_cache_create": ([SZ, SZ, SZ, SZ, C.POINTER(P)], ST),
    "mri_kv_cache_destroy": ([P], None),
    "mri_llama_forward_cached": ([P, P, SZ, SZ, P, P, P], ST),
    "mri_llama_forward_decode": ([P, C.c_uint32, SZ, P, P, P], ST),
    "mri_llama_generate_greedy": ([P, P, SZ, SZ, P, P, P, P], ST),
    "mri_argmax": ([P, SZ, SZ, P, P], ST),
}
EXPORTED = tuple(_SIGS)

_done = False


def lib():
    global _done
    lib = Q.lib()
    if not _done:
        for name, (args, res) in _SIGS.items():
            f = getattr(lib, name)
            f.argtypes = args
            f.restype = res
        _done = True
    return lib


def weight_ref(w):
    """QMatrix / Q8Matrix / Q4Matrix (W4A8) handle, or (q4_0 device uint8
    tensor, n_out, k_in) for the W4A32 projection."""
    if isinstance(w, Q.QMatrix):
        return WeightRef(INT8, w.h, w.n_out, w.k_in)
    if isinstance(w, Q.Q8Matrix):
        return WeightRef(Q8_0, w.h, w.n_out, w.k_in)
    if isinstance(w, Q.Q4Matrix):
        return WeightRef(Q4_0_W4A8, w.h, w.n_out, w.k_in)
    t, n_out, k_in = w
    return WeightRef(Q4_0, C.c_void_p(t.data_ptr()), n_out, k_in)


class KvCache:
    def __init__(self, n_layers, max_seq, n_kv_heads, head_dim):
        h = C.c_void_p()
        Q.check(lib().mri_kv_cache_create(n_layers, max_seq, n_kv_heads, head_dim, C.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            lib().mri_kv_cache_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Llama:
    """LlamaModelInt8 (forward_int8.rs:416-546) on the GPU.  `keep` holds the
    weight objects so that they outlive the model."""

    def __init__(self, cfg: dict, token_embd, output_norm, output, layers):
        import numpy as np
        self.cfg = cfg
        self.keep = [output, layers]
        c = Config(cfg["dim"], cfg["n_heads"], cfg["n_kv_heads"], cfg["ffn"], cfg["vocab"],
                   cfg["max_seq"], cfg["eps"], cfg["rope_base"], len(layers))
        emb = np.ascontiguousarray(token_embd, np.float32)
        on = np.ascontiguousarray(output_norm, np.float32)
        h = C.c_void_p()
        Q.check(lib().mri_llama_create(C.byref(c), emb.ctypes.data_as(P), on.ctypes.data_as(P),
                                       weight_ref(output), C.byref(h)))
        self.h = h
        for i, L in enumerate(layers):
            refs = (WeightRef * 7)(*[weight_ref(L[k]) for k in
                                     ("wq", "wk", "wv", "wo", "wgate", "wup", "wdown")])
            an = np.ascontiguousarray(L["attn_norm"], np.float32)
            fn = np.ascontiguousarray(L["ffn_norm"], np.float32)
            Q.check(lib().mri_llama_set_layer(h, i, an.ctypes.data_as(P), fn.ctypes.data_as(P),
                                              refs))

    def kv_cache(self):
        c = self.cfg
        return KvCache(len(self.keep[1]), c["max_seq"], c["n_kv_heads"],
                       c["dim"] // c["n_heads"])

    def forward_cached(self, tokens, start_pos, cache, logits, stream=None):
        import numpy as np
        t = np.ascontiguousarray(tokens, np.uint32)
        Q.check(lib().mri_llama_forward_cached(self.h, t.ctypes.data_as(P), t.size, start_pos,
                                               cache.h, C.c_void_p(logits.data_ptr()),
                                               Q._stream(stream)))

    def forward_decode(self, token, pos, cache, logits, stream=None):
        Q.check(lib().mri_llama_forward_decode(self.h, int(token), pos, cache.h,
                                               C.c_void_p(logits.data_ptr()), Q._stream(stream)))

    def generate_greedy(self, prompt, n_steps, cache, logits=None, stream=None):
        import numpy as np
        p = np.ascontiguousarray(prompt, np.uint32)
        out = np.empty(n_steps + 1, np.uint32)
        Q.check(lib().mri_llama_generate_greedy(
            self.h, p.ctypes.data_as(P), p.size, n_steps, cache.h, out.ctypes.data_as(P),
            None if logits is None else C.c_void_p(logits.data_ptr()), Q._stream(stream)))
        return out

    def close(self):
        if self.h:
            lib().mri_llama_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def argmax(v, idx, stream=None):
    rows, n = (1, v.numel()) if v.dim() == 1 else tuple(v.shape)
    Q.check(lib().mri_argmax(C.c_void_p(v.data_ptr()), rows, n, C.c_void_p(idx.data_ptr()),
                             Q._stream(stream)))

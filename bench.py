#!/usr/bin/env python3
"""Benchmark of the quantized-matmul hot path on one MI355X.

Headline workload (one "step" = one call of the hot path):
  Q8_0 decode GEMV, x [1, 4096] f32 x W [11008, 4096] Q8_0 (matmul_q8_0_direct),
  synthetic data: quants ~U[-127, 127], f16 block scales ~U(0.001, 0.01),
  x ~ N(0, 1).  Enough device copies of the weights (>= 384 MB, more than
  the 256 MB Infinity Cache) are used in rotation so that the weight stream
  comes from HBM.  The first call is checked against the oracle before
  timing: int32 block dots bit for bit, f32 outputs within
  1e-5 * max(|ref|, sum_b |t_b|).

value = algorithmic bytes per call / mean call time (GB/s), with
        algorithmic bytes = Q8_0 weight bytes (34 B per 32 weights)
        + 4*K (x) + 4*N (out).  The mean call time is the faster of two
        timings of the same calls (both reported): launched one by one from
        Python, and recorded once (one call per rotated weight copy) into a
        HIP graph that is replayed.  The call is one kernel, so this is also
        roofline.achieved: bytes / mean kernel time over the timed region,
        from HIP events on the stream the kernels run on.
cpu_baseline = the oracle's restatement of the reference's only Q8_0 path
        (scalar, single-threaded matmul_q8_0_direct) on the same shape.

Secondary fields (the decode GEMVs timed as the headline; the prefill
GEMMs, whose kernels outlast the launch, Python-launched): the Q8_0 sweep over the Llama-7B
projection shapes (M = 1), the skinny Q8_0 decode M in {4, 8, 16, 32}, the
per-channel INT8 decode GEMV (matmul_int8_from_f32, M = 1), the INT8
prefill GEMM over M in {128, 512, 2048} x N in {4096, 11008} on per-row
quantized activations (matmul_int8 with per-row scales) and end to end from
f32, the Q4_0 W4A32 decode GEMV, the W4A8 extension's decode GEMV (Q4_0
weights, int8 activations), and the reference's rayon+AVX2
matmul_int8_parallel restatement on the INT8 decode shape (one core, as
the reference: one row) and on a bounded row sample of the prefill shape
(all cores).

Decoder layer (the 7B-dims LlamaModelInt8 configuration): one random-init
layer (hidden 4096, 32 heads of 128, SwiGLU 11008, RMSNorm eps 1e-6, RoPE
base 10000) with the output head (vocab 32000), Q8_0 weights (and per-channel
INT8, the reference model's own format, and Q4_0 weights on the W4A8
extension): a 512-token prefill
(forward_cached) and 128 greedy decode steps (generate_greedy, token ids
kept on the device), seeded random prompt ids.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mini-rust-inference_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E
INT8_PEAK_TOPS = 5000.0    # MI355X dense int8 MFMA (5.0 POP/s)
MALL_BYTES = 256 << 20     # Infinity Cache
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_q8_0_decode_1x4096x11008.json")


def q8_bytes(m, n, k):
    return n * (k // 32) * 34 + 4 * m * k + 4 * m * n


def q4_bytes(m, n, k):
    return n * (k // 32) * 18 + 4 * m * k + 4 * m * n


def int8_bytes(m, n, k):
    """Per-channel INT8 decode: int8 weights + f32 scales + f32 x + f32 out."""
    return n * k + 4 * n + 4 * m * k + 4 * m * n


def copies_for(nbytes):
    return max(2, min(16, -(-(MALL_BYTES * 3 // 2) // nbytes)))


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Timer:
    """HIP events on torch's current stream, which is the stream every
    entry point below enqueues on.

    per_call_ms launches the calls from Python (each call pays the ctypes
    and argument-check cost on the host, which exceeds the kernel time of
    the small decode GEMVs).  per_call_graph_ms records one pass over the
    rotated weight copies into a HIP graph and replays it (no host cost, but
    the graph's own gap between kernel nodes); the replayed output is
    checked bit for bit against an eager call on the same weights.
    best_ms takes the faster of the two: each is the kernel time plus an
    overhead that the other does not have."""

    def __init__(self, torch):
        self.torch = torch

    def per_call_ms(self, fn, steps, warmup, n_rot):
        t = self.torch
        for i in range(warmup):
            fn(i % n_rot)
        t.cuda.synchronize()
        e0 = t.cuda.Event(enable_timing=True)
        e1 = t.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(steps):
            fn(i % n_rot)
        e1.record()
        t.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    def best_ms(self, fn, steps, warmup, n_rot, out, fast=None):
        """(min, graph-replayed, Python-launched) ms per call; fast(i), when
        given, is fn(i) with its C arguments bound once, for the launched
        loop."""
        g = self.per_call_graph_ms(fn, steps, warmup, n_rot, out)
        h = self.per_call_ms(fast or fn, steps, warmup, n_rot)
        return min(g, h), g, h

    def per_call_graph_ms(self, fn, steps, warmup, n_rot, out):
        t = self.torch
        # the library keeps its staging buffers per stream: warm them on the
        # stream the graph is captured on, so that capture allocates nothing
        s = t.cuda.Stream()
        s.wait_stream(t.cuda.current_stream())
        with t.cuda.stream(s):
            for i in range(warmup):
                fn(i % n_rot)
            fn(n_rot - 1)
        t.cuda.synchronize()
        want = out.clone()
        g = t.cuda.CUDAGraph()
        with t.cuda.graph(g, stream=s):
            for i in range(n_rot):
                fn(i)
        reps = max(1, -(-steps // n_rot))
        for _ in range(3):          # replays, each checked against the eager call
            out.zero_()
            g.replay()
            t.cuda.synchronize()
            if not t.equal(out, want):
                raise SystemExit("bench: graph replay differs from the eager call")
        e0 = t.cuda.Event(enable_timing=True)
        e1 = t.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        t.cuda.synchronize()
        return e0.elapsed_time(e1) / (reps * n_rot)


def q8_raw_device(torch, n, k, seed):
    """Raw Q8_0 blocks on the device: quants ~U[-127,127], f16 d ~U(0.001,0.01)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    nb = k // 32
    q = torch.randint(-127, 128, (n, nb, 32), dtype=torch.int8, device="cuda", generator=g)
    d = (torch.rand((n, nb), device="cuda", generator=g) * 0.009 + 0.001).half()
    raw = torch.empty((n, nb, 34), dtype=torch.uint8, device="cuda")
    raw[:, :, 0:2] = d.view(torch.uint8).view(n, nb, 2)
    raw[:, :, 2:] = q.view(torch.uint8)
    return raw.view(-1)


def q4_raw_device(torch, n, k, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    nb = k // 32
    nib = torch.randint(0, 256, (n, nb, 16), dtype=torch.uint8, device="cuda", generator=g)
    d = (torch.rand((n, nb), device="cuda", generator=g) * 0.049 + 0.001).half()
    raw = torch.empty((n, nb, 18), dtype=torch.uint8, device="cuda")
    raw[:, :, 0:2] = d.view(torch.uint8).view(n, nb, 2)
    raw[:, :, 2:] = nib
    return raw.view(-1)


def int8_weights_device(torch, M, n, k, seed):
    """Per-channel INT8 weights as the reference builds them: f32 ~N(0, 0.02)
    quantized per output row (quantize_per_channel) -- on the device."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    wf = torch.randn((n, k), device="cuda", generator=g) * 0.02
    data = torch.empty((n, k), dtype=torch.int8, device="cuda")
    scales = torch.empty(n, dtype=torch.float32, device="cuda")
    M.quantize_per_channel(wf, n, k, data, scales)
    return data, scales


def bench_q8(torch, M, T, m, n, k, steps, warmup, check=False, seed=1):
    raw = q8_raw_device(torch, n, k, seed)
    nrot = copies_for(raw.numel())
    ws = [M.Q8Matrix.from_raw_device(raw, n, k) for _ in range(nrot)]
    g = torch.Generator(device="cuda").manual_seed(seed + 100)
    x = torch.randn((m, k), device="cuda", generator=g)
    out = torch.empty((m, n), device="cuda")
    if check:
        import numpy as np
        import oracle_lib as O
        dots = torch.empty((m, n, k // 32), dtype=torch.int32, device="cuda")
        M.matmul_q8_0_direct(x, ws[0], out, dots)
        raw_np = raw.cpu().numpy()
        ref, bd, sa = O.matmul_q8_0_direct(x.cpu().numpy(), raw_np, n, k, want_block_dots=True)
        if not np.array_equal(dots.cpu().numpy(), bd):
            raise SystemExit("bench: Q8_0 block dots differ from the oracle")
        # f32 contract: |gpu - ref| <= 1e-5 * max(|ref|, sum_b |t_b|)
        dsc = raw_np.reshape(n, k // 32, 34)[:, :, :2].copy().view(np.float16)[:, :, 0]
        terms = np.einsum("mnb,nb->mn", np.abs(bd).astype(np.float64),
                          np.abs(dsc.astype(np.float64))) * np.abs(sa.astype(np.float64))[:, None]
        err = np.abs(out.cpu().numpy().astype(np.float64) - ref)
        if not np.all(err <= 1e-5 * np.maximum(np.abs(ref), terms)):
            raise SystemExit("bench: Q8_0 output outside the 1e-5 contract")
    call = lambda i: M.matmul_q8_0_direct(x, ws[i], out)  # noqa: E731
    bound = [M.bind_matmul_q8_0_direct(x, w, out) for w in ws]
    ms, ms_graph, ms_host = T.best_ms(call, steps, warmup, nrot, out, lambda i: bound[i]())
    return ms, raw, x, nrot, (ms_graph, ms_host)


def bench_q4(torch, M, T, m, n, k, steps, warmup, seed=3):
    raws = [q4_raw_device(torch, n, k, seed + i) for i in range(copies_for(n * k // 32 * 18))]
    x = torch.randn((m, k), device="cuda")
    out = torch.empty((m, n), device="cuda")
    return T.best_ms(lambda i: M.matmul_q4_0_dequant(x, raws[i], n, k, out), steps,
                     warmup, len(raws), out)[0]


def bench_w4a8(torch, M, T, n, k, steps, warmup, seed=4):
    """W4A8 extension: Q4_0 weights with int8 activations, M = 1."""
    raws = [q4_raw_device(torch, n, k, seed + i) for i in range(copies_for(n * k // 32 * 18))]
    ws = [M.Q4Matrix.from_raw_device(r, n, k) for r in raws]
    del raws
    x = torch.randn((1, k), device="cuda")
    out = torch.empty((1, n), device="cuda")
    return T.best_ms(lambda i: M.matmul_q4_0_w4a8(x, ws[i], out), steps, warmup, len(ws),
                     out)[0]


def bench_w4a32_handle(torch, M, T, n, k, steps, warmup, seed=6):
    """matmul_q4_0_dequant (W4A32) on device-resident Q4_0 handles, M = 1."""
    raws = [q4_raw_device(torch, n, k, seed + i) for i in range(copies_for(n * k // 32 * 18))]
    ws = [M.Q4Matrix.from_raw_device(r, n, k) for r in raws]
    del raws
    x = torch.randn((1, k), device="cuda")
    out = torch.empty((1, n), device="cuda")
    return T.best_ms(lambda i: M.matmul_q4_0_dequant_matrix(x, ws[i], out), steps, warmup,
                     len(ws), out)[0]


def bench_int8_decode(torch, M, T, n, k, steps, warmup, seed=5):
    data, scales = int8_weights_device(torch, M, n, k, seed)
    nrot = copies_for(n * k)
    ws = [M.QMatrix.from_device(data, scales) for _ in range(nrot)]
    x = torch.randn((1, k), device="cuda")
    out = torch.empty((1, n), device="cuda")
    bound = [M.bind_matmul_int8_from_f32(x, w, out) for w in ws]
    ms = T.best_ms(lambda i: M.matmul_int8_from_f32(x, ws[i], out), steps, warmup,
                   nrot, out, lambda i: bound[i]())[0]
    return ms, data, scales


def bench_int8_prefill(torch, M, T, m, n, k, steps, warmup, seed=7):
    """Per-channel INT8 weights, per-row quantized activations (matmul_int8
    with one scale per row): returns (ms per call of the rows entry point,
    ms per call end to end from f32 with per-tensor quantization)."""
    data, scales = int8_weights_device(torch, M, n, k, seed)
    nrot = copies_for(n * k)
    ws = [M.QMatrix.from_device(data, scales) for _ in range(nrot)]
    x = torch.randn((m, k), device="cuda")
    aq = torch.empty((m, k), dtype=torch.int8, device="cuda")
    sa = torch.empty(m, dtype=torch.float32, device="cuda")
    M.quantize_symmetric_rows(x, aq, sa)
    out = torch.empty((m, n), device="cuda")
    ms_rows = T.per_call_ms(lambda i: M.matmul_int8_rows(aq, sa, ws[i], m, out), steps, warmup,
                            nrot)
    ms_f32 = T.per_call_ms(lambda i: M.matmul_int8_from_f32(x, ws[i], out), steps, warmup, nrot)
    return ms_rows, ms_f32


LAYER = dict(dim=4096, n_heads=32, n_kv_heads=32, ffn=11008, vocab=32000, eps=1e-6,
             rope_base=10000.0)


def layer_decode_bytes(fmt, ctx):
    """Weight bytes read per decode token (7 projections + output head) plus
    the K and V cache rows read by attention at context length ctx."""
    d, f, v = LAYER["dim"], LAYER["ffn"], LAYER["vocab"]
    shapes = [(d, d)] * 4 + [(f, d)] * 2 + [(d, f), (v, d)]
    if fmt == "q8_0":
        w = sum(n * (k // 32) * 34 for n, k in shapes)
    elif fmt == "w4a8":
        w = sum(n * (k // 32) * 18 for n, k in shapes)
    else:
        w = sum(n * k + 4 * n for n, k in shapes)
    return w + 2 * ctx * d * 4


def bench_layer(torch, M, fmt, n_prompt=512, n_steps=128, seed=21):
    """Returns a dict of the decoder-layer figures for weight format fmt."""
    import numpy as np
    import mri_llama as L
    c = dict(LAYER, max_seq=n_prompt + n_steps)
    d, f, v = c["dim"], c["ffn"], c["vocab"]
    rng = np.random.default_rng(seed)
    sd = [seed]

    def w(n, k):
        sd[0] += 1
        if fmt == "q8_0":
            g = torch.Generator(device="cuda").manual_seed(sd[0])
            nb = k // 32
            q = torch.randint(-127, 128, (n, nb, 32), dtype=torch.int8, device="cuda",
                              generator=g)
            dd = (torch.rand((n, nb), device="cuda", generator=g) * 0.0018 + 0.0002).half()
            raw = torch.empty((n, nb, 34), dtype=torch.uint8, device="cuda")
            raw[:, :, 0:2] = dd.view(torch.uint8).view(n, nb, 2)
            raw[:, :, 2:] = q.view(torch.uint8)
            return M.Q8Matrix.from_raw_device(raw.view(-1), n, k)
        if fmt == "w4a8":
            return M.Q4Matrix.from_raw_device(q4_raw_device(torch, n, k, sd[0]), n, k)
        data, scales = int8_weights_device(torch, M, n, k, sd[0])
        return M.QMatrix.from_device(data, scales)

    layer = dict(attn_norm=np.ones(d, np.float32), ffn_norm=np.ones(d, np.float32),
                 wq=w(d, d), wk=w(d, d), wv=w(d, d), wo=w(d, d), wgate=w(f, d), wup=w(f, d),
                 wdown=w(d, f))
    emb = rng.standard_normal((v, d), dtype=np.float32)
    model = L.Llama(c, emb, np.ones(d, np.float32), w(v, d), [layer])
    del emb
    cache = model.kv_cache()
    prompt = rng.integers(0, v, n_prompt).tolist()
    logits = torch.empty((n_prompt, v), device="cuda")
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    model.forward_cached(prompt, 0, cache, logits)  # warm (workspaces, code objects)
    model.generate_greedy(prompt, 8, cache)
    pre = []
    for _ in range(3):
        e0, e1 = ev(), ev()
        e0.record()
        model.forward_cached(prompt, 0, cache, logits)
        e1.record()
        torch.cuda.synchronize()
        pre.append(e0.elapsed_time(e1))
    gen = []
    for _ in range(2):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        toks = model.generate_greedy(prompt, n_steps, cache)
        gen.append((time.perf_counter() - t0) * 1e3)
    check = layer_check(torch, model, prompt, n_steps, v)
    pre_ms, gen_ms = min(pre), min(gen)
    dec_us = (gen_ms - pre_ms) / n_steps * 1e3
    nbytes = layer_decode_bytes(fmt, n_prompt + n_steps // 2)
    gbs = nbytes / (dec_us * 1e-6) / 1e9
    model.close()
    return {"prefill_512_ms": round(pre_ms, 3),
            "prefill_tokens_per_s": round(n_prompt / (pre_ms * 1e-3), 1),
            "decode_us_per_token": round(dec_us, 2),
            "decode_tokens_per_s": round(1e6 / dec_us, 1),
            "generate_512_plus_128_ms": round(gen_ms, 3),
            "decode_bytes_per_token": nbytes,
            "decode_GB_s": round(gbs, 1), "decode_frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
            "first_tokens": [int(t) for t in toks[:4]], "check": check}


def layer_check(torch, model, prompt, n_steps, v):
    """Checks of the timed run at full size, before its figures count:
    every greedy token is the argmax (last of equal maxima) of its own
    logits row, and the logits of the first decode step (the first chosen
    token at position len(prompt)) equal row len(prompt) of one prefill over
    the prompt and that token, within 1e-1 of the largest logit magnitude (a
    wrong position, head or cache row moves them by O(1); activation
    quantization moves them by a few percent at most)."""
    import numpy as np
    n = len(prompt)
    lg = torch.empty((n_steps + 1, v), device="cuda")
    toks = model.generate_greedy(prompt, n_steps, model.kv_cache(), lg)
    g = lg.cpu().numpy()
    for i in range(n_steps + 1):
        r = g[i]
        assert toks[i] == v - 1 - int(np.argmax(r[::-1])), f"step {i}: not the argmax"
    full = torch.empty((n + 1, v), device="cuda")
    model.forward_cached(list(prompt) + [int(toks[0])], 0, model.kv_cache(), full)
    f = full[n].cpu().numpy()
    rel = float(np.abs(g[1] - f).max() / np.abs(f).max())
    assert rel <= 1e-1, f"first decode step vs prefill row: {rel}"
    return {"greedy_tokens_are_argmax": True, "first_decode_vs_prefill_row_rel": round(rel, 5)}


def cpu_q8_direct(raw_np, x_np, n, k, budget_s):
    """Scalar single-thread matmul_q8_0_direct (the reference's only Q8_0
    path) on the full decode shape; returns (GB/s, calls, seconds)."""
    import oracle_lib as O
    O.matmul_q8_0_direct(x_np, raw_np, n, k)                 # warm
    reps, t0 = 0, time.perf_counter()
    while True:
        O.matmul_q8_0_direct(x_np, raw_np, n, k)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return q8_bytes(1, n, k) * reps / el / 1e9, reps, el


def cpu_int8_parallel(wq, sc, m, k, n, budget_s):
    """rayon+AVX2 matmul_int8_parallel restatement: one task per output row
    on a pool of all online CPUs.  Returns (ms per call, cores used, calls)."""
    import numpy as np
    import oracle_lib as O
    rng = np.random.default_rng(5)
    aq = rng.integers(-127, 128, (m, k), dtype=np.int8)
    out = np.empty((m, n), np.float32)
    O.matmul_int8_parallel(aq, 0.01, wq, sc, m, out=out)
    reps, used, t0 = 0, 0, time.perf_counter()
    while True:
        _, used = O.matmul_int8_parallel(aq, 0.01, wq, sc, m, out=out)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return el / reps * 1e3, used, reps


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def load_traffic():
    """HBM bytes per launch of the headline kernel, from the rocprofv3 --pmc
    FETCH_SIZE / WRITE_SIZE runs recorded under profiles/ (null if absent)."""
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 256 MiB device copy, 20 times (the reference "
                         "kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes)")
    ap.add_argument("--profile-gemm", default="",
                    help="only run matmul_int8 20 times at each comma-separated MxKxN shape "
                         "(random int8 operands; a workload for rocprofv3 counter passes)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the path shards over output rows without cross-GPU arithmetic, so the "
              "N-GPU figure is not measured here.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    import mri_qmatmul as M

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    T = Timer(torch)

    if args.copy_calibration:
        src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")   # 256 MiB
        dst = torch.empty_like(src)
        for _ in range(20):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": src.numel() * 4, "copy_bytes_written":
                          dst.numel() * 4, "launches": 20}), flush=True)
        return

    if args.profile_gemm:
        for spec in args.profile_gemm.split(","):
            mm, kk, nn = (int(v) for v in spec.split("x"))
            g = torch.Generator(device="cuda").manual_seed(1)
            wq = torch.randint(-127, 128, (nn, kk), dtype=torch.int8, device="cuda", generator=g)
            wsc = torch.rand(nn, device="cuda", generator=g) * 1e-3
            w = M.QMatrix.from_device(wq, wsc)
            a = torch.randint(-127, 128, (mm, kk), dtype=torch.int8, device="cuda", generator=g)
            o = torch.empty((mm, nn), device="cuda")
            for _ in range(20):
                M.matmul_int8(a, 0.01, w, mm, o)
            torch.cuda.synchronize()
            log(f"profile-gemm {spec}: 20 calls")
        return

    # ---- headline: Q8_0 decode GEMV [1,4096] x [4096,11008] ------------------
    m, n, k = 1, 11008, 4096
    ms, raw, x, nrot, (ms_graph, ms_host) = bench_q8(torch, M, T, m, n, k, args.steps,
                                                     args.warmup, check=True)
    nbytes = q8_bytes(m, n, k)
    value = nbytes / (ms * 1e-3) / 1e9
    log(f"q8_0 decode [1,{k}]x[{k},{n}]: {ms*1e3:.2f} us/call, {value:.0f} GB/s")

    secondary = {}
    # the one-kernel read ceiling at the headline's size, same rotation
    rbytes = nbytes // 16 * 16
    bufs = [torch.empty(rbytes, dtype=torch.uint8, device="cuda") for _ in range(nrot)]
    for b_ in bufs:
        b_.fill_(1)
    import ctypes
    f_rd = M.lib().mri_hbm_read
    st_rd = M._stream(None)
    a_rd = [(ctypes.c_void_p(b_.data_ptr()), rbytes, None, st_rd) for b_ in bufs]
    ms_rd = T.per_call_ms(lambda i: f_rd(*a_rd[i]), args.steps, args.warmup, nrot)
    del bufs
    gbs_rd = rbytes / (ms_rd * 1e-3) / 1e9
    secondary["hbm_read_ceiling"] = {
        "bytes": rbytes, "us": round(ms_rd * 1e3, 2), "GB_s": round(gbs_rd, 1),
        "frac_of_hbm_peak": round(gbs_rd / HBM_PEAK_GBS, 4),
        "gemv_frac_of_read_ceiling": round(value / gbs_rd, 4),
        "what": "one plain streaming-read kernel over the same number of bytes, same "
                "rotation and timing (mri_hbm_read)"}
    log(f"plain read of {rbytes} B: {ms_rd*1e3:.2f} us, {gbs_rd:.0f} GB/s "
        f"(GEMV at {value / gbs_rd:.3f} of it)")
    if not args.no_secondary:
        steps2 = max(20, args.steps // 2)
        sweep = {}
        for (kk, nn) in [(4096, 4096), (11008, 4096), (4096, 32000)]:
            ms2, _, _, _, _ = bench_q8(torch, M, T, 1, nn, kk, steps2, args.warmup)
            gbs = q8_bytes(1, nn, kk) / (ms2 * 1e-3) / 1e9
            sweep[f"{kk}x{nn}"] = {"us": round(ms2 * 1e3, 2), "GB_s": round(gbs, 1),
                                  "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
            log(f"q8_0 M=1 {kk}->{nn}: {ms2*1e3:.2f} us {gbs:.0f} GB/s")
        sweep["4096x11008"] = {"us": round(ms * 1e3, 2), "GB_s": round(value, 1),
                               "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4)}
        secondary["q8_0_m1_sweep"] = sweep

        skinny = {}
        for mm in (4, 8, 16, 32):
            ms2, _, _, _, _ = bench_q8(torch, M, T, mm, 11008, 4096, steps2, args.warmup)
            gbs = q8_bytes(mm, 11008, 4096) / (ms2 * 1e-3) / 1e9
            skinny[str(mm)] = {"us": round(ms2 * 1e3, 2), "GB_s": round(gbs, 1)}
            log(f"q8_0 M={mm}: {ms2*1e3:.2f} us {gbs:.0f} GB/s")
        secondary["q8_0_skinny_4096x11008"] = skinny

        # prefill-sized Q8_0 products of the 7B layer (M = 512): the LDS-tiled
        # kernel (from 128 rows once M * N > 2^20: all four shapes here)
        q8pre = {}
        for (kk, nn) in [(4096, 12288), (4096, 22016), (4096, 4096), (11008, 4096)]:
            ms2, _, _, _, _ = bench_q8(torch, M, T, 512, nn, kk, max(5, steps2 // 20),
                                       args.warmup)
            tops = 2 * 512 * nn * kk / (ms2 * 1e-3) / 1e12
            q8pre[f"512x{kk}x{nn}"] = {
                "us": round(ms2 * 1e3, 1), "TOPS": round(tops, 1),
                "kernel": "k_gemm_q8_0" if 512 * nn > (1 << 20) else "k_skinny_q8_0"}
            log(f"q8_0 prefill M=512 {kk}->{nn}: {ms2*1e3:.1f} us {tops:.0f} TOPS")
        secondary["q8_0_prefill_m512"] = q8pre

        ms_i8, wq_d, sc_d = bench_int8_decode(torch, M, T, 11008, 4096, steps2, args.warmup)
        gbs = int8_bytes(1, 11008, 4096) / (ms_i8 * 1e-3) / 1e9
        secondary["int8_decode_1x4096x11008"] = {
            "us": round(ms_i8 * 1e3, 2), "GB_s": round(gbs, 1),
            "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
        log(f"int8 decode: {ms_i8*1e3:.2f} us {gbs:.0f} GB/s")

        prefill = {}
        for mm in (128, 512, 2048):
            for nn in (4096, 11008):
                st = max(5, steps2 // (4 if mm < 2048 else 10))
                ms_r, ms_f = bench_int8_prefill(torch, M, T, mm, nn, 4096, st, 3)
                tops = 2 * mm * nn * 4096 / (ms_r * 1e-3) / 1e12
                tops_f = 2 * mm * nn * 4096 / (ms_f * 1e-3) / 1e12
                prefill[f"{mm}x4096x{nn}"] = {
                    "us": round(ms_r * 1e3, 2), "TOPS": round(tops, 1),
                    "frac_of_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
                    "us_from_f32": round(ms_f * 1e3, 2), "TOPS_from_f32": round(tops_f, 1)}
                log(f"int8 prefill M={mm} N={nn}: {ms_r*1e3:.1f} us {tops:.0f} TOPS "
                    f"(from f32 {ms_f*1e3:.1f} us)")
        # the int8 MFMA ceiling on this device with random operands and no
        # memory traffic (the power state of real data), next to the GEMM
        src = torch.randint(-127, 128, (32768,), dtype=torch.int8, device="cuda")
        M.mfma_i8_peak(src, 200)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        ops_pk = sum(M.mfma_i8_peak(src, 4000)[0] for _ in range(5))
        e1.record()
        torch.cuda.synchronize()
        tops_pk = ops_pk / (e0.elapsed_time(e1) * 1e-3) / 1e12
        prefill["mfma_i8_ceiling"] = {
            "TOPS": round(tops_pk, 1), "frac_of_int8_peak": round(tops_pk / INT8_PEAK_TOPS, 4),
            "what": "v_mfma_i32_32x32x32_i8 only, random operands in registers, 8 waves per "
                    "CU, no memory traffic (mri_mfma_i8_peak)"}
        log(f"int8 MFMA ceiling (random operands, no memory): {tops_pk:.0f} TOPS")
        secondary["int8_prefill_gemm"] = prefill

        ms_q4 = bench_q4(torch, M, T, 1, 11008, 4096, steps2, args.warmup)
        gbs = q4_bytes(1, 11008, 4096) / (ms_q4 * 1e-3) / 1e9
        secondary["q4_0_decode_1x4096x11008"] = {
            "us": round(ms_q4 * 1e3, 2), "GB_s": round(gbs, 1),
            "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
        log(f"q4_0 decode: {ms_q4*1e3:.2f} us {gbs:.0f} GB/s")
        ms_h = bench_w4a32_handle(torch, M, T, 11008, 4096, steps2, args.warmup)
        gbs = q4_bytes(1, 11008, 4096) / (ms_h * 1e-3) / 1e9
        secondary["q4_0_w4a32_handle_decode_1x4096x11008"] = {
            "us": round(ms_h * 1e3, 2), "GB_s": round(gbs, 1),
            "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
        log(f"q4_0 W4A32 (device handle) decode: {ms_h*1e3:.2f} us {gbs:.0f} GB/s")
        ms_w4 = bench_w4a8(torch, M, T, 11008, 4096, steps2, args.warmup)
        gbs = q4_bytes(1, 11008, 4096) / (ms_w4 * 1e-3) / 1e9
        secondary["q4_0_w4a8_decode_1x4096x11008"] = {
            "us": round(ms_w4 * 1e3, 2), "GB_s": round(gbs, 1),
            "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
        log(f"q4_0 w4a8 decode: {ms_w4*1e3:.2f} us {gbs:.0f} GB/s")

        layer = {}
        for fmt in ("q8_0", "int8", "w4a8"):
            layer[fmt] = bench_layer(torch, M, fmt)
            log(f"decoder layer {fmt}: prefill 512 {layer[fmt]['prefill_512_ms']:.2f} ms, "
                f"decode {layer[fmt]['decode_us_per_token']:.1f} us/token")
        secondary["decoder_layer_7b_512_plus_128"] = layer

        if not args.no_cpu:
            wq, sc = wq_d.cpu().numpy(), sc_d.cpu().numpy()
            ms_cpu, used, reps = cpu_int8_parallel(wq, sc, 1, 4096, 11008, 3.0)
            secondary["cpu_int8_parallel_1x4096x11008"] = {
                "ms": round(ms_cpu, 3), "cores_used": used,
                "cores_available": os.cpu_count(), "reps": reps,
                "GB_s": round(int8_bytes(1, 11008, 4096) / (ms_cpu * 1e-3) / 1e9, 2)}
            log(f"cpu matmul_int8_parallel M=1: {ms_cpu:.3f} ms (cores used {used})")
            rows = 512  # the full M = 512 prefill shape (about 50 ms a call on 16 cores)
            ms_cpu, used, reps = cpu_int8_parallel(wq, sc, rows, 4096, 11008, 4.0)
            secondary["cpu_int8_parallel_prefill_512x4096x11008"] = {
                "rows": rows, "n": 11008, "k": 4096, "ms": round(ms_cpu, 2),
                "TOPS": round(2 * rows * 11008 * 4096 / (ms_cpu * 1e-3) / 1e12, 4),
                "cores_used": used, "cores_available": os.cpu_count(), "reps": reps}
            log(f"cpu matmul_int8_parallel M={rows}: {ms_cpu:.1f} ms (cores used {used})")

    cpu = None
    if not args.no_cpu:
        gbs_cpu, reps, el = cpu_q8_direct(raw.cpu().numpy(), x.cpu().numpy(), n, k,
                                          args.cpu_seconds)
        cpu = {"value": round(gbs_cpu, 3), "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": f"oracle matmul_q8_0_direct (scalar, 1 thread, the reference's "
                         f"only Q8_0 path) on [1,{k}]x[{k},{n}]: {reps} calls in {el:.1f} s "
                         f"on {cpu_model()} ({os.cpu_count()} CPUs visible)"}
        log(f"cpu q8_0 direct: {gbs_cpu:.3f} GB/s ({reps} reps)")

    line = {
        "metric": "Q8_0 decode GEMV HBM GB/s (% peak) + \u00b5s/token; INT8 prefill GEMM TOPS",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "us_per_token": round(ms * 1e3, 3),
        "us_per_call_graph_replayed": round(ms_graph * 1e3, 3),
        "us_per_call_python_launched": round(ms_host * 1e3, 3),
        "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8xint8->int32, f32 scale",
        "data": "synthetic",
        "config": {"workload": "Q8_0 decode GEMV [1,4096]x[4096,11008] (matmul_q8_0_direct)",
                   "m": m, "k": k, "n": n, "weight_copies_rotated": nrot,
                   "algorithmic_bytes_per_call": nbytes},
        "roofline": {"bound": "hbm", "achieved": round(value, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(value / HBM_PEAK_GBS, 4),
                     "traffic": load_traffic()},
        "cpu_baseline": cpu,
    }
    line.update(secondary)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

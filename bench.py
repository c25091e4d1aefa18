#!/usr/bin/env python3
"""Benchmark of the quantized-matmul hot path on one MI355X.

Headline workload (one "step" = one call of the hot path):
  Q8_0 decode GEMV, x [1, 4096] f32  x  W [11008, 4096] Q8_0 (matmul_q8_0_direct),
  synthetic data: quants ~U[-127,127], f16 block scales ~U(0.001, 0.01),
  x ~ N(0, 1).  Eight device copies of the weights (384 MB > the 256 MB
  Infinity Cache) are used in rotation so the weight stream comes from HBM.

value  = algorithmic bytes per call / mean call time (GB/s), with
         algorithmic bytes = Q8_0 weight bytes (34 B per 32 weights)
         + 4*K (x) + 4*N (out).
roofline.achieved = the same bytes / mean duration of the GEMV kernel, timed
         with HIP events on the stream the kernel runs on.
cpu_baseline = the oracle's restatement of the reference's only Q8_0 path
         (scalar, single-threaded matmul_q8_0_direct) on the same shape.

Also reported (secondary fields): the Q8_0 sweep over the Llama-7B
projection shapes, skinny M in {4,8,16,32}, the per-channel INT8 decode GEMV
and the M=512 INT8 prefill GEMM in TOPS, plus the reference's rayon+AVX2
matmul_int8_parallel restatement on the INT8 decode shape.
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
INT8_PEAK_TOPS = 5000.0    # MI355X dense int8 MFMA (5.0 POPS)
MALL_BYTES = 256 << 20


def q8_bytes(m, n, k):
    return n * (k // 32) * 34 + 4 * m * k + 4 * m * n


def int8_bytes(m, n, k):
    return n * k + 4 * n + 4 * m * k + 4 * m * n


def make_q8_raw(rng, n, k):
    import numpy as np
    q = rng.integers(-127, 128, (n, k), dtype=np.int8)
    d = rng.uniform(0.001, 0.01, (n, k // 32)).astype(np.float16).view(np.uint16)
    blk = np.empty((n, k // 32, 34), np.uint8)
    blk[:, :, 0] = (d & 0xFF).astype(np.uint8)
    blk[:, :, 1] = (d >> 8).astype(np.uint8)
    blk[:, :, 2:] = q.reshape(n, k // 32, 32).view(np.uint8)
    return blk.ravel()


def copies_for(nbytes):
    return max(2, min(16, -(-(MALL_BYTES * 3 // 2) // nbytes)))


def time_calls(torch, fn, steps, warmup, n_rot):
    for i in range(warmup):
        fn(i % n_rot)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        fn(i % n_rot)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps  # ms per call


def bench_q8(torch, M, rng, m, n, k, steps, warmup, check=False):
    import numpy as np
    raw = make_q8_raw(rng, n, k)
    nrot = copies_for(len(raw))
    ws = [M.Q8Matrix.from_raw_bytes(raw, n, k) for _ in range(nrot)]
    x = torch.randn(m, k, device="cuda")
    out = torch.empty(m, n, device="cuda")
    if check:
        import oracle_lib as O
        M.matmul_q8_0_direct(x, ws[0], out)
        ref = O.matmul_q8_0_direct(x.cpu().numpy(), raw, n, k)
        got = out.cpu().numpy()
        if not np.array_equal(got.view(np.uint32), ref.view(np.uint32)):
            raise SystemExit("bench: Q8_0 output differs from the oracle")
    ms = time_calls(torch, lambda i: M.matmul_q8_0_direct(x, ws[i], out), steps, warmup,
                    nrot)
    return ms, raw, x


def bench_int8(torch, M, rng, m, n, k, steps, warmup, from_f32=True):
    import numpy as np
    wq = rng.integers(-127, 128, (n, k), dtype=np.int8)
    sc = rng.uniform(1e-4, 1e-3, n).astype(np.float32)
    nrot = copies_for(n * k)
    ws = [M.QMatrix.from_host(wq, sc) for _ in range(nrot)]
    out = torch.empty(m, n, device="cuda")
    if from_f32:
        x = torch.randn(m, k, device="cuda")
        fn = lambda i: M.matmul_int8_from_f32(x, ws[i], out)
    else:
        aq = torch.randint(-127, 128, (m, k), dtype=torch.int8, device="cuda")
        fn = lambda i: M.matmul_int8(aq, 0.0123, ws[i], m, out)
    ms = time_calls(torch, fn, steps, warmup, nrot)
    return ms, wq, sc


def cpu_baseline_q8(raw, x_np, n, k, budget_s):
    """Scalar single-thread matmul_q8_0_direct (the reference's only Q8_0
    path) timed on this host; returns (GB/s, reps, seconds)."""
    import oracle_lib as O
    O.matmul_q8_0_direct(x_np, raw, n, k)                 # warm
    reps, t0 = 0, time.perf_counter()
    while True:
        O.matmul_q8_0_direct(x_np, raw, n, k)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return q8_bytes(1, n, k) * reps / el / 1e9, reps, el


def cpu_int8_parallel(wq, sc, k, n, budget_s):
    """rayon+AVX2 matmul_int8_parallel restatement at M=1 (one row -> one
    core, as in the reference)."""
    import numpy as np
    import oracle_lib as O
    rng = np.random.default_rng(5)
    aq = rng.integers(-127, 128, (1, k), dtype=np.int8)
    out = np.empty((1, n), np.float32)
    O.matmul_int8_parallel(aq, 0.01, wq, sc, 1, out=out)
    reps, used, t0 = 0, 0, time.perf_counter()
    while True:
        _, used = O.matmul_int8_parallel(aq, 0.01, wq, sc, 1, out=out)
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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the path shards over output rows without cross-GPU arithmetic, so "
              "N-GPU throughput is N x the one-GPU value plus an all-gather.",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    import mri_qmatmul as M

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    rng = np.random.default_rng(2026)
    log = lambda *a: print(*a, file=sys.stderr, flush=True)

    # ---- headline: Q8_0 decode GEMV [1,4096] x [4096,11008] ------------------
    m, n, k = 1, 11008, 4096
    ms, raw, x = bench_q8(torch, M, rng, m, n, k, args.steps, args.warmup, check=True)
    nbytes = q8_bytes(m, n, k)
    value = nbytes / (ms * 1e-3) / 1e9
    log(f"q8_0 decode [1,{k}]x[{k},{n}]: {ms*1e3:.2f} us/call, {value:.0f} GB/s")

    secondary = {}
    if not args.no_secondary:
        steps2 = max(20, args.steps // 2)
        sweep = {}
        for (kk, nn) in [(4096, 4096), (11008, 4096), (4096, 32000)]:
            ms2, _, _ = bench_q8(torch, M, rng, 1, nn, kk, steps2, args.warmup)
            gbs = q8_bytes(1, nn, kk) / (ms2 * 1e-3) / 1e9
            sweep[f"{kk}x{nn}"] = {"us": round(ms2 * 1e3, 2), "GB_s": round(gbs, 1)}
            log(f"q8_0 M=1 {kk}->{nn}: {ms2*1e3:.2f} us {gbs:.0f} GB/s")
        sweep["4096x11008"] = {"us": round(ms * 1e3, 2), "GB_s": round(value, 1)}
        secondary["q8_0_m1_sweep"] = sweep
        skinny = {}
        for mm in (4, 8, 16, 32):
            ms2, _, _ = bench_q8(torch, M, rng, mm, 11008, 4096, steps2, args.warmup)
            gbs = q8_bytes(mm, 11008, 4096) / (ms2 * 1e-3) / 1e9
            skinny[str(mm)] = {"us": round(ms2 * 1e3, 2), "GB_s": round(gbs, 1)}
            log(f"q8_0 M={mm}: {ms2*1e3:.2f} us {gbs:.0f} GB/s")
        secondary["q8_0_skinny_4096x11008"] = skinny
        ms_i8, wq, sc = bench_int8(torch, M, rng, 1, 11008, 4096, steps2, args.warmup)
        secondary["int8_decode_1x4096x11008"] = {
            "us": round(ms_i8 * 1e3, 2),
            "GB_s": round(int8_bytes(1, 11008, 4096) / (ms_i8 * 1e-3) / 1e9, 1)}
        log(f"int8 decode: {ms_i8*1e3:.2f} us")
        ms_p, _, _ = bench_int8(torch, M, rng, 512, 11008, 4096, max(10, steps2 // 4),
                                max(3, args.warmup // 4))
        tops = 2 * 512 * 11008 * 4096 / (ms_p * 1e-3) / 1e12
        secondary["int8_prefill_512x4096x11008"] = {
            "us": round(ms_p * 1e3, 2), "TOPS": round(tops, 1),
            "frac_of_int8_peak": round(tops / INT8_PEAK_TOPS, 4)}
        log(f"int8 prefill M=512: {ms_p*1e3:.1f} us {tops:.0f} TOPS")
        if not args.no_cpu:
            ms_cpu, used, reps = cpu_int8_parallel(wq, sc, 4096, 11008, 3.0)
            secondary["cpu_int8_parallel_1x4096x11008"] = {
                "ms": round(ms_cpu, 3), "cores_used": used,
                "cores_available": os.cpu_count(), "reps": reps}
            log(f"cpu matmul_int8_parallel M=1: {ms_cpu:.3f} ms (cores used {used})")

    cpu = None
    if not args.no_cpu:
        gbs_cpu, reps, el = cpu_baseline_q8(raw, x.cpu().numpy(), n, k, args.cpu_seconds)
        cpu = {"value": round(gbs_cpu, 3), "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": f"oracle matmul_q8_0_direct (scalar, 1 thread) on "
                         f"[1,{k}]x[{k},{n}], {reps} calls in {el:.1f} s on "
                         f"{cpu_model()} ({os.cpu_count()} CPUs visible)"}
        log(f"cpu q8_0 direct: {gbs_cpu:.3f} GB/s ({reps} reps)")

    line = {
        "metric": "Q8_0 decode GEMV HBM GB/s (% peak) + us/token; INT8 prefill GEMM TOPS",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "us_per_token": round(ms * 1e3, 3),
        "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8xint8->int32, f32 scale",
        "data": "synthetic",
        "config": {"workload": "Q8_0 decode GEMV [1,4096]x[4096,11008] (matmul_q8_0_direct)",
                   "m": m, "k": k, "n": n, "weight_copies_rotated": copies_for(len(raw)),
                   "algorithmic_bytes_per_call": nbytes},
        "roofline": {"bound": "hbm", "achieved": round(value, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(value / HBM_PEAK_GBS, 4),
                     "traffic": None},
        "cpu_baseline": cpu,
    }
    line.update(secondary)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

#!/usr/bin/env python3
"""Benchmark of the Q4/g64 quantized-linear path on one MI355X.

Headline (the `value`): decode GEMV bandwidth on the decode workload
  x bf16 [1,3840] . dequant(W [15360,3840] Q4/g64)^T  ->  y bf16 [1,15360]
measured cold: the timed launches rotate over distinct device copies of the weight
whose total exceeds the 256 MB Infinity Cache, so every launch streams from HBM.
A step is one GEMV launch; `value` = algorithmic bytes per launch / mean launch time.

Also reported: the prefill GEMM (seven projections of a Gemma-class 12B decoder layer
at M=2048) in TFLOP/s against the bf16 MFMA peak, and the oracle's restatement of
MLX's CPU quantized_matmul timed on this host (the CPU baseline).

Progress goes to stderr; stdout carries exactly one JSON line.
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import hyperion_amd as hy  # noqa: E402
from hyperion_amd import synthetic as syn  # noqa: E402

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
DECODE_N, DECODE_K = 15360, 3840


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def decode_bytes(m, n, k):
    """Algorithmic bytes of one Q4/g64 GEMV launch: packed codes (0.5 B/weight) +
    bf16 scale and bias per 64 weights + x + y."""
    return n * k // 2 + 2 * 2 * n * (k // 64) + 2 * m * k + 2 * m * n


def time_launches(stream, fn, steps, warmup):
    for i in range(warmup):
        fn(i)
    stream.synchronize()
    e0, e1 = hy.Event(), hy.Event()
    e0.record(stream)
    for i in range(steps):
        fn(i)
    e1.record(stream)
    ms = e0.elapsed_ms(e1)
    e0.close()
    e1.close()
    return ms


def bench_decode(stream, steps, warmup, copies):
    n, k = DECODE_N, DECODE_K
    log(f"decode GEMV m=1 n={n} k={k}: generating weights, {copies} device copies")
    w, s, b = syn.q4_weights(n, k, seed=105)
    x = syn.activations(1, k, seed=104)
    base = hy.QWeight.from_host(w, s, b)
    wd = hy.DeviceArray.from_host(w, stream)
    sd = hy.DeviceArray.from_host(s, stream)
    bd = hy.DeviceArray.from_host(b, stream)
    qws = [base]
    for _ in range(copies - 1):
        h = ctypes.c_void_p()
        hy.call("hyp_qweight_create_device", wd.ptr, sd.ptr, bd.ptr, n, k, 64, 4, stream.handle, ctypes.byref(h))
        qws.append(hy.QWeight(h))
    stream.synchronize()
    xd = hy.DeviceArray.from_host(x, stream)
    yd = hy.DeviceArray((1, n), np.uint16)

    def cold(i):
        hy.qmatmul(qws[i % copies], xd, 1, yd, stream)

    def warm(i):
        hy.qmatmul(base, xd, 1, yd, stream)

    ms_cold = time_launches(stream, cold, steps, warmup)
    ms_warm = time_launches(stream, warm, steps, warmup)
    nbytes = decode_bytes(1, n, k)
    per_cold = ms_cold / steps
    per_warm = ms_warm / steps
    log(f"decode cold {per_cold * 1e3:.2f} us/launch = {nbytes / per_cold / 1e6:.0f} GB/s; "
        f"warm {per_warm * 1e3:.2f} us = {nbytes / per_warm / 1e6:.0f} GB/s")
    for q in qws:
        q.close()
    return {"ms_total": ms_cold, "ms_per_launch": per_cold, "bytes": nbytes,
            "warm_ms_per_launch": per_warm, "copies": copies,
            "cold_working_set_bytes": copies * nbytes}


def bench_prefill(stream, m, steps, warmup):
    log(f"prefill GEMM m={m}: seven projections")
    per = {}
    total_flops = 0
    total_ms = 0.0
    for i, (name, (n, k)) in enumerate(syn.LAYER_SHAPES.items()):
        w, s, b = syn.q4_weights(n, k, seed=500 + i)
        qw = hy.QWeight.from_host(w, s, b)
        xd = hy.DeviceArray.from_host(syn.activations(m, k, seed=400 + i), stream)
        yd = hy.DeviceArray((m, n), np.uint16)
        ms = time_launches(stream, lambda _i: hy.qmatmul(qw, xd, m, yd, stream), steps, warmup) / steps
        flops = 2 * m * n * k
        per[name] = {"n": n, "k": k, "ms": round(ms, 4), "tflops": round(flops / ms / 1e9, 1)}
        total_flops += flops
        total_ms += ms
        log(f"  {name:5s} n={n:5d} k={k:5d}: {ms:.3f} ms  {flops / ms / 1e9:.0f} TFLOP/s")
        qw.close()
    tflops = total_flops / total_ms / 1e9
    log(f"prefill layer m={m}: {total_ms:.3f} ms  {tflops:.0f} TFLOP/s")
    return {"m": m, "layer_ms": round(total_ms, 4), "tflops": round(tflops, 1),
            "frac_of_mfma_peak": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), "per_projection": per}


def cpu_baseline(seconds):
    """The oracle's restatement of MLX's CPU quantized_matmul (bf16 accumulation) on the
    full decode GEMV, repeated for about `seconds` on one host core."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    n, k = DECODE_N, DECODE_K
    w, s, b = syn.q4_weights(n, k, seed=105)
    x = syn.activations(1, k, seed=104)
    reps = 0
    t0 = time.perf_counter()
    while True:
        O.qmatmul_mlx_cpu(x, w, s, b)
        reps += 1
        if time.perf_counter() - t0 >= seconds:
            break
    dt = time.perf_counter() - t0
    gbs = reps * decode_bytes(1, n, k) / dt / 1e9
    log(f"cpu baseline: {reps} GEMVs in {dt:.1f} s = {gbs:.2f} GB/s (1 core)")
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{reps} full decode GEMVs [1,{k}]x[{n},{k}] Q4/g64, bf16-accumulating "
                      f"restatement of MLX's CPU loop, {dt:.1f} s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--copies", type=int, default=24, help="distinct weight copies rotated (cold HBM)")
    ap.add_argument("--prefill-steps", type=int, default=10)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported by this build", file=sys.stderr)
        sys.exit(2)

    info = hy.runtime_info()
    log(f"{info.device_name.decode()} {info.arch_name.decode()} CUs={info.compute_units}")
    stream = hy.Stream()
    dec = bench_decode(stream, args.steps, args.warmup, args.copies)
    pre = None if args.no_prefill else bench_prefill(stream, 2048, args.prefill_steps, 2)
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)

    per = dec["ms_per_launch"]
    gbs = dec["bytes"] / per / 1e6
    line = {
        "metric": "Q4/g64 qmatmul: decode GB/s (% HBM peak) + prefill TFLOPS (% MFMA peak)",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(per, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "decode GEMV x[1,3840] . W[15360,3840]^T, MLX affine Q4/g64, cold HBM "
                               f"({dec['copies']} rotated weight copies)",
                   "m": 1, "n": DECODE_N, "k": DECODE_K},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None},
        "decode_warm_gbs": round(dec["bytes"] / dec["warm_ms_per_launch"] / 1e6, 1),
        "prefill": pre,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

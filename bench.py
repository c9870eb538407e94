#!/usr/bin/env python3
"""Benchmark of the Q4/g64 quantized-linear path on one MI355X.

Headline (`value`): the decode GEMV
  x bf16 [1,3840] . dequant(W [15360,3840] Q4/g64)^T  ->  y bf16 [1,15360]
timed cold: the launches rotate over distinct device copies of W whose total exceeds
the 256 MB Infinity Cache, so every launch streams its weights from HBM. A step is one
launch; value = algorithmic bytes per launch / mean launch time, both measured with HIP
events on the stream the kernel runs on.

Also reported, each on its own workload:
  quantize    bf16 W [15360,3840] N(0, 0.02^2) with 1% x8 outliers -> Q4/g64 (GB/s)
  prefill     the seven projections at m = 512 and 2048 as the product calls them (q/k/v
              in one grouped launch, gate/up fused with the GELU gating) (TFLOP/s vs bf16
              MFMA peak)
  decode      48 layers (renormalise + q/k/v in one launch, o, fused gate/up + GELU, down)
              + tied LM head [262144,3840] with softcap + greedy sampling with its top-8
              sidecar on the device, m = 1 and 4, replayed from a captured HIP graph
              (tokens/s and effective HBM GB/s); the head timed alone (per-layer figures);
              and the layer stack as one decode-step program launch
  model       the whole decoder through the model-level entry points on a synthetic 12B
              artifact: a 1024-token prefill (tokens/s) and 32 greedy decode tokens from
              that context (ms per token: norms, RoPE, attention over the KV caches, all
              projections, LM head and sampling)
and the oracle's restatement of MLX's CPU quantized_matmul timed on this host's cores
(cpu_baseline).

Progress goes to stderr; stdout carries exactly one JSON line.
"""
import argparse
import ctypes
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import hyperion_amd as hy  # noqa: E402
from hyperion_amd import decode_chain as dc  # noqa: E402
from hyperion_amd import synthetic as syn  # noqa: E402

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
DECODE_N, DECODE_K = 15360, 3840
HIDDEN = syn.HIDDEN
METRIC = "Q4/g64 qmatmul: decode GB/s (% HBM peak) + prefill TFLOPS (% MFMA peak)"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def q4_bytes(n, k):
    """Packed codes (0.5 B/weight) + bf16 scale and bias per 64 weights."""
    return n * k // 2 + 4 * n * (k // 64)


def gemv_bytes(m, n, k):
    """Algorithmic bytes of one launch: the Q4 matrix + x + y (bf16)."""
    return q4_bytes(n, k) + 2 * m * k + 2 * m * n


MALL_BYTES = 256 << 20   # MI355X Infinity Cache


def cold_rotation_ok(copies, bytes_per_copy):
    """True when every reuse of a copy in a rotation over `copies` buffers comes after at
    least one MALL's worth of other bytes: a launch on copy c is preceded by launches on
    the other copies - 1 buffers since c was last read."""
    return (copies - 1) * bytes_per_copy > MALL_BYTES


def time_launches(stream, fn, steps, warmup):
    """Mean milliseconds per call of fn(i), from HIP events recorded on `stream`. The
    index keeps counting from the warm-up into the timed loop (warm-up calls are
    fn(0..warmup-1), timed calls fn(warmup..warmup+steps-1)), so a rotation over
    buffers indexed by i % copies never restarts at the buffers the warm-up just read.
    The start event is recorded behind the warm-up calls while they are still queued, so
    the timed region opens on a busy stream (steady state, as in a decode loop) and not on
    an idle GPU, whose first launch would carry the queue's start-up."""
    stream.synchronize()
    for i in range(warmup):
        fn(i)
    e0, e1 = hy.Event(), hy.Event()
    e0.record(stream)
    for i in range(warmup, warmup + steps):
        fn(i)
    e1.record(stream)
    ms = e0.elapsed_ms(e1)
    e0.close()
    e1.close()
    return ms / steps


def device_copies(w, s, b, n, k, copies, stream):
    """`copies` resident projections with the same values in distinct HBM buffers."""
    wd = hy.DeviceArray.from_host(w, stream)
    sd = hy.DeviceArray.from_host(s, stream)
    bd = hy.DeviceArray.from_host(b, stream)
    out = []
    for _ in range(copies):
        h = ctypes.c_void_p()
        hy.call("hyp_qweight_create_device", wd.ptr, sd.ptr, bd.ptr, n, k, 64, 4, stream.handle, ctypes.byref(h))
        out.append(hy.QWeight(h))
    stream.synchronize()
    return out


def bench_decode_gemv(stream, steps, warmup, copies):
    n, k = DECODE_N, DECODE_K
    if not cold_rotation_ok(copies, q4_bytes(n, k)):
        raise SystemExit(f"--copies {copies}: a rotation over {copies} weight copies re-reads a copy within "
                         f"{MALL_BYTES >> 20} MiB of other traffic (the MALL would serve it)")
    log(f"decode GEMV m=1 n={n} k={k}: {copies} device copies")
    w, s, b = syn.q4_weights(n, k, seed=105)
    qws = device_copies(w, s, b, n, k, copies, stream)
    xd = hy.DeviceArray.from_host(syn.activations(1, k, seed=104), stream)
    yd = hy.DeviceArray((1, n), np.uint16)
    # Set-up: one read of every copy. A buffer's first read in a process pays page-table
    # walks that a resident weight set read every token does not (measured: 8.9 against
    # 8.2 us per launch over 20 launches without this pass; equal to 200 launches with it).
    for q in qws:
        hy.qmatmul(q, xd, 1, yd, stream)
    cold = time_launches(stream, lambda i: hy.qmatmul(qws[i % copies], xd, 1, yd, stream), steps, warmup)
    warm = time_launches(stream, lambda i: hy.qmatmul(qws[0], xd, 1, yd, stream), steps, warmup)
    nbytes = gemv_bytes(1, n, k)
    log(f"decode cold {cold * 1e3:.2f} us/launch = {nbytes / cold / 1e6:.0f} GB/s; "
        f"warm {warm * 1e3:.2f} us = {nbytes / warm / 1e6:.0f} GB/s")
    for a in (*qws, xd, yd):
        a.close()
    return {"ms_per_launch": cold, "warm_ms_per_launch": warm, "bytes": nbytes, "copies": copies}


def bench_quantize(stream, steps, warmup, copies=4):
    n, k = DECODE_N, DECODE_K
    assert cold_rotation_ok(copies, 2 * n * k + q4_bytes(n, k))
    log(f"quantize/pack n={n} k={k}: {copies} input copies")
    wb = syn.quantize_input(n, k, seed=101)
    ins = [hy.DeviceArray.from_host(wb, stream) for _ in range(copies)]
    wq = hy.DeviceArray((n, k // 8), np.uint32)
    sq = hy.DeviceArray((n, k // 64), np.uint16)
    bq = hy.DeviceArray((n, k // 64), np.uint16)
    ms = time_launches(stream, lambda i: hy.quantize(ins[i % copies], n, k, wq, sq, bq, stream), steps, warmup)
    nbytes = 2 * n * k + q4_bytes(n, k)
    log(f"quantize {ms * 1e3:.2f} us = {nbytes / ms / 1e6:.0f} GB/s")
    return {"workload": f"bf16 [{n},{k}] -> Q4/g64", "us": round(ms * 1e3, 2), "bytes": nbytes,
            "gbs": round(nbytes / ms / 1e6, 1), "frac_of_hbm_peak": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4)}


# The layer's prefill calls as the product makes them: q/k/v in one grouped launch, o, the
# MLP's gate and up as one fused launch with the GELU gating (hyp_qmlp_gate_up_gelu),
# down.
PREFILL_CALLS = (("qkv", ("q", "k", "v")), ("o", ("o",)), ("mlp", ("gate", "up")), ("down", ("down",)))


def dense_bf16_child(m, steps, warmup):
    """Child-process mode: hipBLASLt's dense bf16 GEMM (bf16 weights, no dequantisation) on
    the layer's prefill calls at m rows (q/k/v as one [8192, 3840] weight, gate and up as one
    [30720, 3840] weight without the gating), in both weight layouts - torch.matmul(x, W^T
    stored [k, n]) and torch.nn.functional.linear(x, W stored [n, k], the linear layer's own
    layout) - keeping the faster per call; timed with torch's events on torch's stream; prints
    {call: ms} as JSON. torch brings its own HIP runtime, which does not share a process with
    this library's, hence the separate process."""
    import torch
    dev = torch.device("cuda:0")
    out = {}
    for call_name, projs in PREFILL_CALLS:
        k = syn.LAYER_SHAPES[projs[0]][1]
        n = sum(syn.LAYER_SHAPES[p][0] for p in projs)
        x = torch.randn(m, k, device=dev, dtype=torch.bfloat16)
        wt = torch.randn(k, n, device=dev, dtype=torch.bfloat16)
        w = torch.randn(n, k, device=dev, dtype=torch.bfloat16)
        best = None
        for fn in (lambda: torch.matmul(x, wt), lambda: torch.nn.functional.linear(x, w)):
            for _ in range(warmup):
                fn()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(steps):
                fn()
            e1.record()
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / steps
            best = ms if best is None else min(best, ms)
        out[call_name] = best
    print(json.dumps(out), flush=True)


def dense_bf16_reference(m, steps, warmup):
    """Runs dense_bf16_child in a child process (called before this process touches the GPU)."""
    import subprocess
    res = subprocess.run([sys.executable, os.path.abspath(__file__), "--dense-child", str(m),
                          "--steps", str(steps), "--warmup", str(warmup)],
                         capture_output=True, text=True, timeout=600, check=True)
    return json.loads(res.stdout.strip().splitlines()[-1])


def read_floor(nbytes, launches=200):
    """The shortest time a bare streaming kernel takes to read nbytes from HBM in one launch
    (hyperion_amd/stream_floor, a child process run before this process touches the GPU): the
    practical ceiling of a launch of that size, beside the 8 TB/s peak."""
    import subprocess
    exe = os.path.join(ROOT, "hyperion_amd", "stream_floor")
    if not os.path.exists(exe):
        log("read floor: hyperion_amd/stream_floor is not built; skipped")
        return None
    res = subprocess.run([exe, str(nbytes), str(launches)], capture_output=True, text=True, timeout=120, check=True)
    for line in res.stderr.strip().splitlines():
        log(line)
    rec = json.loads(res.stdout.strip().splitlines()[-1])
    rec["frac_of_hbm_peak"] = round(rec["gbs"] / HBM_PEAK_GBS, 4)
    return rec


def bench_prefill(stream, m, steps, warmup, dense=None):
    log(f"prefill m={m}: the layer's calls (q/k/v grouped)")
    per = {}
    total_flops = 0
    total_ms = 0.0
    dense_ms = 0.0
    for ci, (call_name, projs) in enumerate(PREFILL_CALLS):
        k = syn.LAYER_SHAPES[projs[0]][1]
        qws, yds = [], []
        for pi, proj in enumerate(projs):
            n = syn.LAYER_SHAPES[proj][0]
            w, s, b = syn.q4_weights(n, k, seed=500 + 8 * ci + pi)
            qws.append(hy.QWeight.from_host(w, s, b))
            if call_name != "mlp" or pi == 0:
                yds.append(hy.DeviceArray((m, n), np.uint16))
        xd = hy.DeviceArray.from_host(syn.activations(m, k, seed=400 + ci), stream)
        if call_name == "mlp":
            fn = lambda _i: hy.qmlp_gate_up_gelu(qws[0], qws[1], xd, m, yds[0], stream)  # noqa: E731
        elif len(qws) == 1:
            fn = lambda _i: hy.qmatmul(qws[0], xd, m, yds[0], stream)  # noqa: E731
        else:
            fn = lambda _i: hy.qmatmul_group(qws, xd, m, yds, stream)  # noqa: E731
        ms = time_launches(stream, fn, steps, warmup)
        n_total = sum(syn.LAYER_SHAPES[p][0] for p in projs)
        flops = 2 * m * n_total * k
        per[call_name] = {"n": n_total, "k": k, "us": round(ms * 1e3, 1), "tflops": round(flops / ms / 1e9, 1)}
        msg = f"  {call_name:5s} n={n_total:5d} k={k:5d}: {ms * 1e3:8.1f} us  {flops / ms / 1e9:6.0f} TFLOP/s"
        if dense is not None:
            dms = dense[call_name]
            dense_ms += dms
            per[call_name]["dense_bf16_tflops"] = round(flops / dms / 1e9, 1)
            msg += f"   (dense bf16 hipBLASLt {flops / dms / 1e9:6.0f} TFLOP/s)"
        total_flops += flops
        total_ms += ms
        log(msg)
        for q in qws:
            q.close()
    tflops = total_flops / total_ms / 1e9
    log(f"prefill layer m={m}: {total_ms * 1e3:.1f} us  {tflops:.0f} TFLOP/s")
    out = {"m": m, "layer_us": round(total_ms * 1e3, 1), "tflops": round(tflops, 1),
           "frac_of_mfma_peak": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), "per_call": per}
    if dense is not None:
        dense_tf = total_flops / dense_ms / 1e9
        out["dense_bf16_layer_tflops"] = round(dense_tf, 1)
        out["frac_of_dense_bf16"] = round(tflops / dense_tf, 4)
        log(f"prefill layer m={m}: dense bf16 hipBLASLt {dense_tf:.0f} TFLOP/s; Q4 GEMM at {tflops / dense_tf:.1%} of it")
    return out


def bench_decode_stream(model, m, steps, warmup, stream):
    """One decode step at batch m: the 48-layer stack's 192 per-op launches and the head
    (renormalise, softcap LM head, greedy sampling with the top-8 sidecar) replayed from one graph. Also timed: the
    head alone, from which the per-layer figures are derived, and the same layer stack as
    one step-program launch followed by the head's graph."""
    b = dc.StepBuffers(hy, m, syn.activations(m, HIDDEN, seed=77), stream)
    with hy.Graph.capture(stream) as head:
        dc.lm_head(model, m, b, stream)
    head_ms = time_launches(stream, lambda _i: head.launch(stream), steps, warmup)
    with hy.Graph.capture(stream) as graph:
        dc.decode_step(model, m, b, stream)
    graph_ms = time_launches(stream, lambda _i: graph.launch(stream), steps, warmup)
    graph.close()
    prog = dc.layer_program(model, m, b)

    def step(_i):
        prog.run(stream)
        head.launch(stream)

    ms = time_launches(stream, step, steps, warmup)
    prog.check()
    prog.close()
    head.close()
    b.close()
    layers = len(model.layers)
    nbytes = model.weight_bytes + dc.step_activation_bytes(layers, m)
    head_bytes = q4_bytes(syn.VOCAB, HIDDEN) + 2 * m * (HIDDEN + 2 * syn.VOCAB) + 80 * m
    layer_bytes = (nbytes - head_bytes) / max(layers, 1)

    def rates(step_ms):
        layer_us = (step_ms - head_ms) * 1e3 / max(layers, 1)
        return {"ms_per_step": round(step_ms, 4), "tokens_per_s": round(m / (step_ms / 1e3), 1),
                "gbs": round(nbytes / step_ms / 1e6, 1),
                "frac_of_hbm_peak": round(nbytes / step_ms / 1e6 / HBM_PEAK_GBS, 4),
                "layer_us": round(layer_us, 2), "layer_gbs": round(layer_bytes / layer_us / 1e3, 1)}

    out = {"m": m, **rates(graph_ms), "bytes_per_step": nbytes,
           "launches_per_step": dc.LAUNCHES_PER_LAYER * layers + 3,
           "lm_head_us": round(head_ms * 1e3, 1), "lm_head_gbs": round(head_bytes / head_ms / 1e6, 1),
           "step_program": {**rates(ms), "launches_per_step": 4}}
    log(f"decode stream m={m}: per-op launches (graph) {graph_ms:.3f} ms/step = {out['tokens_per_s']:.0f} tok/s, "
        f"{out['gbs']:.0f} GB/s, layer {out['layer_us']} us ({out['layer_gbs']} GB/s); step program "
        f"{ms:.3f} ms = {out['step_program']['tokens_per_s']:.0f} tok/s, layer {out['step_program']['layer_us']} us; "
        f"LM head {out['lm_head_us']} us ({out['lm_head_gbs']} GB/s)")
    return out


def artifact_dir(min_free_bytes):
    """A scratch directory with room for a synthetic artifact (memory-backed if possible)."""
    import shutil
    import tempfile
    for base in ("/dev/shm", tempfile.gettempdir()):
        try:
            if os.path.isdir(base) and shutil.disk_usage(base).free >= min_free_bytes:
                return tempfile.mkdtemp(prefix="hyp_bench_", dir=base)
        except OSError:
            continue
    return None


def bench_model_decode(prompt_len, n_decode, layers, host_launch=False):
    """The product's model-level path on a synthetic 12B artifact (48 layers, tied LM head
    [262144,3840], 6.6 GB of Q4/g64; the layers' codes are zero, their scales, biases, norms
    and the embedding random, so every byte is still streamed): hyp_model_load,
    hyp_prefill_chunk of a
    prompt_len-token prompt (2048-token chunks), then hyp_decode_block of n_decode greedy
    tokens in one call - embed, every layer's norms, q/k/v, RoPE, KV cache append,
    attention over the cached context, o, MLP and residual sandwich, final norm, softcap
    LM head and greedy sampling, all on the device, one host round trip per call.
    host_launch: the n_decode tokens go through hyp_model_forward_hidden one at a time instead
    (every kernel of a decode step but the LM head and the sampler, launched from the host,
    not replayed from the step's graph), for kernel traces."""
    import shutil
    cfg = syn.gemma4_text_config(num_layers=layers, max_positions=max(8192, prompt_len + n_decode + 16))
    d = artifact_dir(8 << 30)
    if d is None:
        log("model decode: no scratch directory with 8 GB free; skipped")
        return None
    try:
        t0 = time.time()
        syn.write_model(d, cfg, seed=21, branch_gain=0.5, qk_gain=0.7, share_layers=True, zero_layer_codes=True)
        t1 = time.time()
        model = hy.Model(hy.geometry_from_config(cfg), d)
        t2 = time.time()
    finally:
        shutil.rmtree(d, ignore_errors=True)
    log(f"model decode: artifact written in {t1 - t0:.1f} s, loaded in {t2 - t1:.1f} s")
    prompt = np.random.default_rng(22).integers(0, cfg["vocab_size"], size=prompt_len).astype(np.uint32)
    res = hy.StepResult()
    warm = model.kvstate()
    warm.prefill(prompt[:64], res)
    warm.decode(4, res)
    warm.close()
    st = model.kvstate()
    t0 = time.perf_counter()
    st.prefill(prompt, res)
    prefill_s = time.perf_counter() - t0
    if host_launch:
        nxt = np.random.default_rng(23).integers(0, cfg["vocab_size"], size=n_decode).astype(np.uint32)
        t0 = time.perf_counter()
        for j in range(n_decode):
            st.forward_hidden(nxt[j:j + 1], prompt_len + j)
        decode_s = time.perf_counter() - t0
        f = res.fields()
    else:
        st.decode(2, res)
        t0 = time.perf_counter()
        f = st.decode(n_decode, res)
        decode_s = time.perf_counter() - t0
    st.close()
    res.close()
    model.close()
    n_global = cfg["layer_types"].count("full_attention")
    sl = ((4096, 3840), (2048, 3840), (2048, 3840), (3840, 4096), (15360, 3840), (15360, 3840), (3840, 15360))
    gl = ((8192, 3840), (512, 3840), (3840, 8192), (15360, 3840), (15360, 3840), (3840, 15360))
    weight_bytes = (layers - n_global) * sum(q4_bytes(n, k) for n, k in sl) + \
        n_global * sum(q4_bytes(n, k) for n, k in gl) + q4_bytes(syn.VOCAB, HIDDEN)
    ms = decode_s * 1e3 / n_decode
    out = {"layers": layers, "prompt_tokens": prompt_len, "decode_tokens": n_decode,
           "decode_launch": "host, hyp_model_forward_hidden (no LM head)" if host_launch else "graph replay",
           "prefill_tokens_per_s": round(prompt_len / prefill_s, 1), "prefill_s": round(prefill_s, 4),
           "decode_ms_per_token": round(ms, 4), "decode_tokens_per_s": round(1e3 / ms, 1),
           "weight_bytes": weight_bytes, "weight_stream_gbs": round(weight_bytes / ms / 1e6, 1),
           "last_token": int(f.token_id)}
    log(f"model decode: prefill {prompt_len} tokens {prefill_s * 1e3:.1f} ms ({out['prefill_tokens_per_s']:.0f} tok/s); "
        f"decode {ms:.3f} ms/token = {out['decode_tokens_per_s']:.0f} tok/s from context {prompt_len + 2}")
    return out


def bench_sample(stream, steps, warmup):
    """hyp_sample_greedy and hyp_sample_greedy_topk (the greedy epilogue with its top-8
    sidecar) on rows of vocab 262144 seeded logits N(0, 36): 10 calls captured in one graph,
    timed per call from graph replays."""
    out = []
    for rows in (1, 4):
        logits = hy.DeviceArray.from_host(
            syn.bf16_bits((np.random.default_rng(31 + rows).standard_normal((rows, syn.VOCAB)) * 6).astype(np.float32)),
            stream)
        for name, fn, rec in (("greedy", hy.sample_greedy, 12), ("greedy_topk", hy.sample_greedy_topk, 80)):
            res = hy.DeviceArray((rows, rec // 4), np.uint32)
            with hy.Graph.capture(stream) as graph:
                for _ in range(10):
                    fn(logits, rows, syn.VOCAB, res, stream)
            ms = time_launches(stream, lambda _i: graph.launch(stream), steps, warmup) / 10
            graph.close()
            nbytes = 2 * rows * syn.VOCAB + rec * rows
            out.append({"entry": name, "rows": rows, "vocab": syn.VOCAB, "us": round(ms * 1e3, 2),
                        "gbs": round(nbytes / ms / 1e6, 1)})
            log(f"{name} sample rows={rows} vocab={syn.VOCAB}: {ms * 1e3:.2f} us per call")
            res.close()
        if rows == 1:
            # the temperature draw (hyp_sample_stochastic) with the top-8 sidecar, one row
            cfg = hy.SamplingConfig(temperature=0.8, top_k=64, top_p=0.95, min_p=0.05, seed=7)
            res = hy.DeviceArray((1, 20), np.uint32)
            with hy.Graph.capture(stream) as graph:
                for j in range(10):
                    hy.sample_stochastic(logits, syn.VOCAB, cfg, 7 + j, res, stream)
            ms = time_launches(stream, lambda _i: graph.launch(stream), steps, warmup) / 10
            graph.close()
            out.append({"entry": "stochastic", "rows": 1, "vocab": syn.VOCAB, "us": round(ms * 1e3, 2),
                        "gbs": round((2 * syn.VOCAB + 80) / ms / 1e6, 1),
                        "config": "temperature 0.8, top_k 64, top_p 0.95, min_p 0.05"})
            log(f"stochastic sample rows=1 vocab={syn.VOCAB}: {ms * 1e3:.2f} us per call")
            res.close()
        logits.close()
    return out


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(seconds):
    """The oracle's restatement of MLX's CPU quantized_matmul (bf16 accumulation) over a
    bounded number of full decode GEMVs: on one host core (the reference's CPU stream
    runs one task), and with output rows over this process's share of cores (OpenMP,
    OMP_NUM_THREADS or all cores)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    n, k = DECODE_N, DECODE_K
    w, s, b = syn.q4_weights(n, k, seed=105)
    x = syn.activations(1, k, seed=104)
    threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)

    def timed(fn):
        reps = 0
        t0 = time.perf_counter()
        while True:
            fn()
            reps += 1
            if time.perf_counter() - t0 >= seconds:
                break
        dt = time.perf_counter() - t0
        return reps, dt, reps * gemv_bytes(1, n, k) / dt / 1e9

    what = (f"full decode GEMVs [1,{k}]x[{n},{k}] Q4/g64 with the oracle's bf16-accumulating "
            f"restatement of MLX's CPU quantized_matmul on {cpu_model()} (nproc {os.cpu_count()})")
    reps, dt, gbs = timed(lambda: O.qmatmul_mlx_cpu(x, w, s, b))
    log(f"cpu baseline: {reps} GEMVs in {dt:.1f} s = {gbs:.3f} GB/s (1 core)")
    one = {"value": round(gbs, 4), "unit": "GB/s", "cores": 1, "kind": "port",
           "sample": f"{reps} {what} in {dt:.1f} s"}
    reps, dt, gbs = timed(lambda: O.qmatmul_mlx_cpu_mt(x, w, s, b, threads))
    log(f"cpu baseline: {reps} GEMVs in {dt:.1f} s = {gbs:.3f} GB/s ({threads} threads)")
    par = {"value": round(gbs, 4), "unit": "GB/s", "cores": threads, "kind": "port",
           "sample": f"{reps} {what}, output rows over {threads} OpenMP threads, in {dt:.1f} s"}
    return one, par


def measured_traffic():
    """HBM bytes per decode-GEMV launch from the committed counter summary, if present."""
    path = os.path.join(ROOT, "profiles", "decode_gemv_traffic.md")
    if not os.path.exists(path):
        return None
    m = re.search(r"```json\s*(\{.*?\})\s*```", open(path).read(), flags=re.S)
    if not m:
        return None
    rec = json.loads(m.group(1))
    return rec.get("hbm_bytes_per_launch")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200, help="timed decode-GEMV launches")
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--copies", type=int, default=24, help="distinct weight copies rotated (cold HBM)")
    ap.add_argument("--layers", type=int, default=syn.NUM_LAYERS, help="decoder layers in the decode stream")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--only-decode", action="store_true", help="only the headline decode GEMV")
    ap.add_argument("--only-prefill", action="store_true", help="the headline decode GEMV and the prefill GEMMs")
    ap.add_argument("--only-sample", action="store_true", help="the headline decode GEMV and greedy sampling")
    ap.add_argument("--only-quantize", action="store_true", help="the headline decode GEMV and quantize/pack")
    ap.add_argument("--only-stream", action="store_true", help="the headline decode GEMV and the decode stream")
    ap.add_argument("--only-model", action="store_true",
                    help="the headline decode GEMV and the model-level prefill + decode")
    ap.add_argument("--prompt", type=int, default=1024, help="prompt tokens of the model-level run")
    ap.add_argument("--model-host-launch", action="store_true",
                    help="model-level decode tokens launched from the host (for kernel traces)")
    ap.add_argument("--dense-ref", action="store_true",
                    help="also time hipBLASLt's dense bf16 GEMM (torch.matmul) on the prefill shapes")
    ap.add_argument("--dense-child", type=int, default=0, help=argparse.SUPPRESS)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-read-floor", action="store_true",
                    help="skip the bare-stream read floor of the headline's bytes (hyperion_amd/stream_floor)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run 5 device-to-device copies of 256 MiB (the reference kernel of known "
                         "traffic for scaling hardware byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (this build runs on a single "
              "MI355X; the multi-GPU sharding of the path is a design, not a measured run)", file=sys.stderr)
        sys.exit(2)
    if args.dense_child:
        dense_bf16_child(args.dense_child, 10, 2)
        return
    # The dense reference and the read floor run in child processes before this process
    # makes any HIP call.
    dense = {m: dense_bf16_reference(m, 10, 2) for m in (512, 2048)} if args.dense_ref else {}
    floor = None if args.no_read_floor else read_floor(gemv_bytes(1, DECODE_N, DECODE_K))

    info = hy.runtime_info()
    log(f"{info.device_name.decode()} {info.arch_name.decode()} CUs={info.compute_units}")
    stream = hy.Stream()
    if args.copy_calibration:
        nbytes = 256 << 20
        src, dst = hy.DeviceArray((nbytes,), np.uint8), hy.DeviceArray((nbytes,), np.uint8)
        for _ in range(5):
            hy.call("hyp_memcpy_dtod", dst.ptr, src.ptr, nbytes, stream.handle)
        stream.synchronize()
        log(f"copy calibration: 5 x {nbytes} bytes device-to-device")
    dec = bench_decode_gemv(stream, args.steps, args.warmup, args.copies)
    extra = {}
    if args.only_prefill:
        extra["prefill"] = [bench_prefill(stream, m, 10, 2, dense.get(m)) for m in (512, 2048)]
    elif args.only_sample:
        extra["sample_greedy"] = bench_sample(stream, 20, 3)
    elif args.only_quantize:
        extra["quantize"] = bench_quantize(stream, 50, 5)
    elif args.only_stream:
        model = dc.DecodeModel(hy, args.layers, log)
        extra["decode_stream"] = [bench_decode_stream(model, m, 10, 2, stream) for m in (1, 4)]
        model.close()
    elif args.only_model:
        extra["model_decode"] = bench_model_decode(args.prompt, 32, args.layers, args.model_host_launch)
    elif not args.only_decode:
        extra["quantize"] = bench_quantize(stream, 50, 5)
        extra["sample_greedy"] = bench_sample(stream, 20, 3)
        extra["prefill"] = [bench_prefill(stream, m, 10, 2, dense.get(m)) for m in (512, 2048)]
        model = dc.DecodeModel(hy, args.layers, log)
        streams = [bench_decode_stream(model, m, 10, 2, stream) for m in (1, 4)]
        model.close()
        extra["decode_stream"] = streams
        extra["model_decode"] = bench_model_decode(args.prompt, 32, args.layers)
    # Every HIP object this process made is released here, before the interpreter exits:
    # nothing is left for finalizers or exit handlers to destroy.
    stream.synchronize()
    stream.close()
    cpu, cpu_par = (None, None) if args.no_cpu else cpu_baseline(args.cpu_seconds)

    per = dec["ms_per_launch"]
    gbs = dec["bytes"] / per / 1e6
    line = {
        "metric": METRIC,
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
        "data": "synthetic (seeded codes, scales and activations; random-init weights)",
        "config": {"workload": "decode GEMV x[1,3840] . W[15360,3840]^T, MLX affine Q4/g64, cold HBM "
                               f"({dec['copies']} rotated weight copies)",
                   "m": 1, "n": DECODE_N, "k": DECODE_K},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic()},
        "decode_gemv_warm_gbs": round(dec["bytes"] / dec["warm_ms_per_launch"] / 1e6, 1),
        "hbm_read_floor": floor,
        "decode_gemv_frac_of_read_floor": round(gbs / floor["gbs"], 4) if floor else None,
        "cpu_baseline": cpu,
        "cpu_baseline_parallel": cpu_par,
    }
    line.update(extra)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

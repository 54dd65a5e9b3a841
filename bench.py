#!/usr/bin/env python3
"""Benchmark of the MI355X q4_0 and per-group INT4 paths -- one JSON line on stdout.

Metric: q4_0 GEMV GB/s (% HBM peak) at M=1; q4_0 GEMM TFLOP/s
(% MFMA) at M=2048.

* Headline ``value``: decode GEMV throughput on configs[1] -- one step is one
  Llama-2-7B layer's projections at M=1 (fused QKV 4096x12288, O 4096x4096,
  gate and up 4096x11008, down 11008x4096).  GB/s counts the q4_0 weight bytes
  (18 bytes per 32 weights) per step over the measured step time.  Ten copies of
  the layer's weights (1.14 GB, beyond the 256 MB Infinity Cache) are rotated
  so reads come from HBM.  Steps are replayed from a HIP graph; the timed region
  is bracketed by HIP events recorded on the stream the kernels run on.
* ``prefill``: the M=2048 GEMM configs (configs[3]: 4096x14336 and 14336x4096)
  in TFLOP/s, with the same keys as the top level (``value``, ``unit``,
  ``roofline``, ``cpu_baseline``).
* ``configs``: every other BASELINE config point -- configs[0] (M=1 4096x4096),
  configs[2] (M = 4, 8, 16 on 4096x14336 and 14336x4096) and configs[4]
  (lm_head 4096x128256 and the ragged down 11008x4096 at M = 1 and 512): GB/s
  and % of HBM peak for M <= 16, TFLOP/s and % of the fp16 MFMA peak for M >= 512.
  Each is a graph of launches over weight copies rotated through >= 1 GB.
* ``cpu_baseline``: the reference's CPU path (dequantize to fp16 on every call,
  then ``X @ W``; quantization.py:452-454) restated in oracle/, timed on this
  host's cores on a bounded sample; ``secondary`` is the same call at fp32
  (``X.float() @ dequant_f32``).
* ``int4``: the per-group INT4 path (quantization.py:26-239) on the same decode
  layer and prefill shapes, group size 128 with fp16 scales and zeros (an fp16
  model's weights), with its own roofline and CPU baseline; ``fused_rmsnorm_m1`` times
  fused_rmsnorm_linear_int4 (MM:3017-3103) per call on the layer's normalised
  projections (qkv, gate, up) beside plain matmul_int4 on the same weights.

Inputs are synthetic: seeded N(0, 0.02) fp32 weights quantized on the GPU with
the llama.cpp q4_0 rule, N(0, 1) fp16 activations.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
FP16_PEAK_TFLOPS = 2500.0    # MI355X dense fp16 MFMA

# HBM bytes per launch from rocprofv3 FETCH_SIZE / WRITE_SIZE passes over the same
# workloads (bench.py --part decode|prefill), each counter scaled by what it reads
# for a plain 256 MiB device copy (FETCH_SIZE x 2, WRITE_SIZE x 1).  Figures and
# commands: profiles/gemv_dma_llama7b_m1.md, profiles/q4_gemm7_llama7b_m2048.md.
DECODE_TRAFFIC_BYTES = 23335567       # average over the five projections (23.32 MB read + 0.017 MB written)
DECODE_KERNEL = "q4_gemv_span_kernel (qkv, gate, up) + q4_gemv_dma_kernel (o, down): decode GEMV, M=1"
PREFILL_KERNEL = "q4_gemm7_kernel (M=2048 K=4096 N=14336)"
PREFILL_UP_TRAFFIC_BYTES = 361849343  # 302.7 MB read + 59.2 MB written

DECODE_LAYER = [  # (name, K, N) -- Llama-2-7B projections, configs[1]
    ("qkv", 4096, 12288),
    ("o_proj", 4096, 4096),
    ("gate", 4096, 11008),
    ("up", 4096, 11008),
    ("down", 11008, 4096),
]
PREFILL = [("up", 2048, 4096, 14336), ("down", 2048, 14336, 4096)]
I4_GROUP = 128
# HBM bytes per launch of the INT4 kernels (rocprofv3 FETCH_SIZE / WRITE_SIZE over
# bench.py --part int4-decode|int4-prefill, scaled as above; profiles/i4_gemv1_llama7b_m1.md,
# profiles/i4_gemm7_llama7b_m2048.md).
I4_DECODE_TRAFFIC_BYTES = 21934858   # 21.80 MB read + 0.13 MB written
I4_PREFILL_UP_TRAFFIC_BYTES = 373744538   # 307.6 MB read + 66.1 MB written


def wbytes(K, N):
    return 18 * (K // 32) * N


def i4_wbytes(K, N, gs=I4_GROUP):
    """Packed nibbles plus fp16 scales and zeros of one INT4 weight."""
    return K // 2 * N + 2 * 2 * ((K + gs - 1) // gs) * N


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50000)
    p.add_argument("--warmup", type=int, default=200)
    p.add_argument("--copies", type=int, default=10, help="weight copies rotated per step")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-seconds", type=float, default=15.0)
    p.add_argument("--no-graph", action="store_true", help="eager launches instead of a HIP graph")
    p.add_argument("--part", choices=["all", "decode", "prefill", "configs", "copy", "int4-decode",
                                      "int4-prefill", "probes", "prefill-splits", "prefill-routing"],
                   default="all",
                   help="run one part only (for profiler passes); 'copy' runs a plain 256 MiB "
                        "device copy that calibrates the FETCH_SIZE / WRITE_SIZE counters; "
                        "'probes' runs the machine probes of libmcq4_bench.so (launch floor, "
                        "read patterns of the q4_0 layout, atomic and store-to-load latency, "
                        "shader clock); 'prefill-splits' times the few-tile prefill shapes "
                        "(M = 512, N = 4096) over forced kernels and K splits")
    return p.parse_args()


def make_weights(mo, torch, K, N, seed, dev, outliers=False):
    g = torch.Generator(device=dev).manual_seed(seed)
    W = torch.randn(K, N, generator=g, device=dev) * 0.02
    if outliers:
        n = W.numel() // 100
        idx = torch.randperm(W.numel(), generator=g, device=dev)[:n]
        W.view(-1)[idx] = torch.randn(n, generator=g, device=dev) * 0.2
    b = mo.quantize_ggml_q4_0_llama(W)
    del W
    return b


def time_region(torch, stream, fn, steps, warmup, min_warm_s=0.2, stats=None):
    """Run fn(i) at least `warmup` times and for at least `min_warm_s` seconds (the
    GPU clocks ramp up after host-side setup), then time `steps` calls between HIP
    events on `stream`.  With a `stats` dict, events also split the same region into
    up to 10 chunks and stats["median_call_s"] gets the median time per call over
    the chunks."""
    t_w = time.perf_counter()
    i = 0
    with torch.cuda.stream(stream):
        while i < warmup or time.perf_counter() - t_w < min_warm_s:
            fn(i % max(1, steps))
            i += 1
            if i % 16 == 0:
                torch.cuda.synchronize()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    chunk = max(1, steps // 10) if stats is not None else steps + 1
    marks = []                                   # (event, calls so far)
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        start.record(stream)
        for i in range(steps):
            fn(i)
            if (i + 1) % chunk == 0 and i + 1 < steps:
                ev = torch.cuda.Event(enable_timing=True)
                ev.record(stream)
                marks.append((ev, i + 1))
        end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    if stats is not None:
        per, prev, prev_n = [], start, 0
        for ev, n in marks + [(end, steps)]:
            per.append(prev.elapsed_time(ev) / 1e3 / (n - prev_n))
            prev, prev_n = ev, n
        stats["median_call_s"] = statistics.median(per)
    return start.elapsed_time(end) / 1e3, wall


CONFIG_POINTS = [  # (config, M, K, N) -- every BASELINE point outside the headline layer
    ("configs[0]", 1, 4096, 4096),
    ("configs[2]", 4, 4096, 14336), ("configs[2]", 8, 4096, 14336), ("configs[2]", 16, 4096, 14336),
    ("configs[2]", 4, 14336, 4096), ("configs[2]", 8, 14336, 4096), ("configs[2]", 16, 14336, 4096),
    ("configs[4]", 1, 4096, 128256), ("configs[4]", 512, 4096, 128256),
    ("configs[4]", 1, 11008, 4096), ("configs[4]", 512, 11008, 4096),
]


def shape_bench(mo, torch, dev, M, K, N, pool_bytes=1 << 30, reps=20, outliers=False):
    """Average time of one matmul launch at (M, K, N): a HIP graph of one launch per
    weight copy, the copies rotated through >= pool_bytes so reads come from HBM."""
    copies = max(1, -(-pool_bytes // wbytes(K, N)))
    ws = [make_weights(mo, torch, K, N, 31 * i + K + N, dev, outliers=outliers) for i in range(copies)]
    g = torch.Generator(device=dev).manual_seed(3)
    x = torch.randn(M, K, generator=g, device=dev).half()
    stream = torch.cuda.Stream(dev)
    with torch.cuda.stream(stream):
        mo.matmul_ggml_q4_0(x, ws[0])
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for w in ws:
            mo.matmul_ggml_q4_0(x, w)
    secs, _ = time_region(torch, stream, lambda i: graph.replay(), reps, 3)
    t = secs / (reps * copies)
    del graph
    t_read = read_ceiling(torch, stream, ws, reps) / copies if M <= 16 else None
    del ws
    torch.cuda.empty_cache()
    return t, copies, t_read


def prefill_split_sweep(mo, torch, dev):
    """The few-tile prefill shapes (M = 512, N = 4096: 32 tiles of 256 x 256, 64 of
    128 x 256, 128 of 128 x 128) under each prefill kernel forced with 1, 2, 4 and 8
    K splits (q4_gemm8: 1 and 2), and the default plan: TFLOP/s per point, graph replays over rotated weight copies."""
    from metalops_amd import _lib
    keys = ("MCQ4_GEMM_PATH", "MCQ4_GEMM6_SPLIT", "MCQ4_GEMM8_SPLIT")
    saved = {k: os.environ.get(k) for k in keys}
    out = []
    try:
        for M, K, N in ((512, 11008, 4096), (512, 4096, 4096)):
            runs = [("default", None, None)] + [(f"gemm{p}", p, sp) for p in ("6", "7") for sp in (1, 2, 4, 8)] \
                + [("gemm8", "8", sp) for sp in (1, 2)]
            for name, path, sp in runs:
                for k in keys:
                    os.environ.pop(k, None)
                if path:
                    os.environ["MCQ4_GEMM_PATH"] = path
                    os.environ["MCQ4_GEMM8_SPLIT" if path == "8" else "MCQ4_GEMM6_SPLIT"] = str(sp)
                _lib.reload_options()
                t, _, _ = shape_bench(mo, torch, dev, M, K, N, reps=5)
                out.append({"M": M, "K": K, "N": N, "kernel": name, "splits": sp, "us": round(t * 1e6, 2),
                            "TFLOP/s": round(2 * M * N * K / t / 1e12, 1)})
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
        _lib.reload_options()
    return out


# Prefill shapes around the few-tile GEMM's routing rule (q4_gemm8 when its plan is one
# round of 192..256 workgroups): inside the rule, and just outside it on either side.
ROUTING_SHAPES = [(384, 4096, 4096), (384, 11008, 4096), (512, 4096, 4096), (512, 11008, 4096),
                  (512, 14336, 4096), (768, 4096, 4096), (1024, 4096, 4096), (1024, 14336, 4096),
                  (256, 4096, 14336), (256, 11008, 4096), (1536, 4096, 4096), (512, 4096, 14336),
                  (1024, 4096, 11008), (2048, 4096, 4096), (768, 4096, 14336), (1280, 4096, 8192),
                  (640, 4096, 11008)]


def prefill_routing_sweep(mo, torch, dev):
    """Each ROUTING_SHAPES point under the default plan and under each prefill kernel
    forced (MCQ4_GEMM_PATH=6|7|8, each with its own split plan): microseconds per
    launch, graph replays over rotated weight copies."""
    from metalops_amd import _lib
    saved = os.environ.get("MCQ4_GEMM_PATH")
    out = []
    try:
        for M, K, N in ROUTING_SHAPES:
            rec = {"M": M, "K": K, "N": N}
            for name, path in (("default", None), ("gemm6", "6"), ("gemm7", "7"), ("gemm8", "8")):
                os.environ.pop("MCQ4_GEMM_PATH", None)
                if path:
                    os.environ["MCQ4_GEMM_PATH"] = path
                _lib.reload_options()
                t, _, _ = shape_bench(mo, torch, dev, M, K, N, reps=5)
                rec[name + "_us"] = round(t * 1e6, 2)
            out.append(rec)
            print(json.dumps(rec), file=sys.stderr, flush=True)
    finally:
        os.environ.pop("MCQ4_GEMM_PATH", None)
        if saved is not None:
            os.environ["MCQ4_GEMM_PATH"] = saved
        _lib.reload_options()
    return out


def config_points(mo, torch, dev):
    out = []
    for cfg, M, K, N in CONFIG_POINTS:
        t, copies, t_read = shape_bench(mo, torch, dev, M, K, N, reps=20 if M <= 16 else 5)
        rec = {"config": cfg, "M": M, "K": K, "N": N, "us": round(t * 1e6, 2), "weight_copies": copies}
        if M <= 16:
            gbs = wbytes(K, N) / t / 1e9
            rec.update({"GB/s": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
                        "GB/s_incl_x_y": round((wbytes(K, N) + 2 * M * (K + N)) / t / 1e9, 1),
                        "read_ceiling_GB/s": round(wbytes(K, N) / t_read / 1e9, 1)})
        else:
            tf = 2.0 * M * N * K / t / 1e12
            rec.update({"TFLOP/s": round(tf, 1), "pct_mfma_peak": round(100 * tf / FP16_PEAK_TFLOPS, 2)})
        out.append(rec)
    return out


_BENCH_LIB = None


def bench_lib():
    """libmcq4_bench.so: the measurement probes (metalops_amd/csrc/bench/mcq4_bench.h),
    built beside libmcq4.so and kept out of the drop-in library."""
    global _BENCH_LIB
    if _BENCH_LIB is None:
        import ctypes
        path = os.path.join(ROOT, "metalops_amd", "_lib", "libmcq4_bench.so")
        if not os.path.exists(path):
            raise ImportError(f"{path} is not built; run __graft_entry__.build()")
        lib = ctypes.CDLL(path)
        p, i, i64, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t
        sigs = {"mcqb_read_probe": [p, sz, p, p], "mcqb_read_tiles": [p, i64, i64, i, i, i, p, p],
                "mcqb_read_rows": [p, i64, i64, i64, i, i, p, p],
                "mcqb_empty": [i, i, p], "mcqb_measure_sclk": [p, i, p],
                "mcqb_atomic_chain": [p, i, i, p, p], "mcqb_exchange": [p, p, i, i, i, i, p]}
        for name, args in sigs.items():
            fn = getattr(lib, name)
            fn.restype = i
            fn.argtypes = args
        _BENCH_LIB = lib
    return _BENCH_LIB


def bench_check(status, name):
    if status != 0:
        raise RuntimeError(f"{name} failed with status {status}")


def read_ceiling(torch, stream, weights, reps):
    """Seconds per pass of plain reads (mcqb_read_probe, one launch per weight) over
    `weights` in order, captured in one HIP graph -- the HBM read rate the same
    bytes reach with launches of the same sizes and nothing else to do."""
    lib = bench_lib()
    sink = torch.zeros(4, dtype=torch.int32, device=weights[0].device)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        cs = torch.cuda.current_stream().cuda_stream
        for w in weights:
            bench_check(lib.mcqb_read_probe(w.data_ptr(), w.numel() * w.element_size(), sink.data_ptr(), cs),
                        "mcqb_read_probe")
    secs, _ = time_region(torch, stream, lambda i: graph.replay(), reps, 3)
    del graph
    return secs / reps


def decode_bench(mo, torch, dev, args):
    R = max(1, args.copies)
    layers = []
    for r in range(R):
        layers.append([make_weights(mo, torch, K, N, 1000 * r + i, dev) for i, (_, K, N) in
                       enumerate(DECODE_LAYER)])
    g = torch.Generator(device=dev).manual_seed(1)
    xs = {K: torch.randn(1, K, generator=g, device=dev).half() for K in (4096, 11008)}
    ys = [torch.empty(1, N, device=dev, dtype=torch.float16) for (_, _, N) in DECODE_LAYER]
    stream = torch.cuda.Stream(dev)

    def one_step(r):
        outs = []
        for (name, K, N), w in zip(DECODE_LAYER, layers[r % R]):
            outs.append(mo.matmul_ggml_q4_0(xs[K], w))
        return outs

    # warm the per-stream workspace before any capture
    with torch.cuda.stream(stream):
        one_step(0)
    torch.cuda.synchronize()

    if args.no_graph:
        fn = one_step
        launches_per_call = len(DECODE_LAYER)
        calls = args.steps
        st = {}
        secs, wall = time_region(torch, stream, fn, calls, args.warmup, stats=st)
        steps = calls
        median_step_s = st["median_call_s"]
        replays, check_s = 0, None
    else:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for r in range(R):
                one_step(r)
        singles = []
        for r in range(R):
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr, stream=stream):
                one_step(r)
            singles.append(gr)
        full, rem = divmod(args.steps, R)

        def fn(i):
            if i < full:
                graph.replay()
            else:
                singles[i - full].replay()

        st = {}
        secs, wall = time_region(torch, stream, fn, full + rem, max(1, args.warmup // R), stats=st)
        steps = args.steps
        median_step_s = st["median_call_s"] / R if full else secs / steps
        replays = full + rem
        # A short timed region (the driver's --steps 20 is two replays) is checked
        # against one of at least 50 ms of replays, reported beside it.
        check_s = None
        if secs < 0.05:
            n = max(1, int(0.05 / (secs / max(1, full + rem) * (R if not full else 1))) + 1)
            csecs, _ = time_region(torch, stream, lambda i: graph.replay(), n, 3)
            check_s = csecs / (n * R)
    bytes_step = sum(wbytes(K, N) for _, K, N in DECODE_LAYER)
    xy_step = sum(2 * K + 2 * N for _, K, N in DECODE_LAYER)
    read_s = read_ceiling(torch, stream, [w for layer in layers for w in layer], 20) / R

    # The same step with gate and up in one launch (matmul_ggml_q4_0_grouped):
    # four launches instead of five, same weights and results.
    def grouped_step(r):
        qkv, o, gate, up, down = layers[r % R]
        return [mo.matmul_ggml_q4_0(xs[4096], qkv), mo.matmul_ggml_q4_0(xs[4096], o),
                *mo.matmul_ggml_q4_0_grouped(xs[4096], [gate, up]), mo.matmul_ggml_q4_0(xs[11008], down)]

    ggraph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        grouped_step(0)
    torch.cuda.synchronize()
    with torch.cuda.graph(ggraph, stream=stream):
        for r in range(R):
            grouped_step(r)
    reps = max(1, min(steps, 20000) // R)
    gsecs, _ = time_region(torch, stream, lambda i: ggraph.replay(), reps, 3)
    del ggraph
    return {
        "read_ceiling_s": read_s,
        "graph_replays": replays, "check_step_s": check_s,
        "grouped_step_s": gsecs / (reps * R),
        "seconds": secs, "steps": steps, "wall": wall, "median_step_s": median_step_s,
        "bytes_step": bytes_step, "xy_step": xy_step,
        "launches_step": len(DECODE_LAYER), "copies": R,
        "weight_pool_bytes": bytes_step * R,
    }


def prefill_bench(mo, torch, dev, iters=30, warmup=10):
    out = []
    stream = torch.cuda.Stream(dev)
    for name, M, K, N in PREFILL:
        w = make_weights(mo, torch, K, N, 77, dev, outliers=True)
        g = torch.Generator(device=dev).manual_seed(2)
        x = torch.randn(M, K, generator=g, device=dev).half()
        with torch.cuda.stream(stream):
            mo.matmul_ggml_q4_0(x, w)
        st = {}
        secs, _ = time_region(torch, stream, lambda i: mo.matmul_ggml_q4_0(x, w), iters, warmup, stats=st)
        t = secs / iters
        fl = 2.0 * M * N * K
        out.append({"name": name, "M": M, "K": K, "N": N, "ms": t * 1e3, "median_ms": st["median_call_s"] * 1e3,
                    "tflops": fl / t / 1e12})
        del w, x
    return out


def prefill_cpu_baseline(seconds_budget):
    """Reference CPU path at the prefill size: dequantize to fp16 then X @ W
    (quantization.py:452-454) at M = 2048 on the up shape (4096 x 14336) when a
    call fits the budget, else the largest power-of-two M that does."""
    import numpy as np
    import torch

    from oracle import q4_0_ref as ref

    K, N = 4096, 14336
    rng = np.random.default_rng(0)
    W = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    blocks = torch.from_numpy(ref.quantize_llama_rule(W))
    X = torch.from_numpy(rng.standard_normal((2048, K)).astype(np.float16))

    def timed(x, budget):
        M = 16
        t0 = time.perf_counter()
        ref.fallback_torch_cpu(x[:M], blocks)                 # warm-up
        per = time.perf_counter() - t0
        while M < 2048 and per * 2 * 3 <= budget:             # 3 timed calls at 2M still fit
            M *= 2
            t0 = time.perf_counter()
            ref.fallback_torch_cpu(x[:M], blocks)             # also the warm-up at this M
            per = time.perf_counter() - t0
        n, t0 = 0, time.perf_counter()
        while n < 1 or (time.perf_counter() - t0 + per <= budget and n < 20):
            ref.fallback_torch_cpu(x[:M], blocks)
            n += 1
        return M, n, (time.perf_counter() - t0) / n

    M, n, per = timed(X, seconds_budget * 2 / 3)
    # The secondary figure: the same call at fp32 (X.float() @ dequant_f32).
    M32, n32, per32 = timed(X.float(), seconds_budget / 3)
    return {
        "value": round(2.0 * M * K * N / per / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"up K=4096 N=14336 at M={M} fp16: dequantize + X@W per call (quantization.py:452-454), "
                  f"torch CPU, {n} calls, {per:.2f} s/call; os.cpu_count()={os.cpu_count()}",
        "secondary": {
            "value": round(2.0 * M32 * K * N / per32 / 1e12, 4),
            "unit": "TFLOP/s",
            "sample": f"the same at fp32 (X.float() @ dequant_f32), M={M32}, {n32} calls, {per32:.2f} s/call",
        },
    }


def make_i4_weights(mo, torch, K, N, seed, dev, outliers=False):
    g = torch.Generator(device=dev).manual_seed(seed)
    W = torch.randn(K, N, generator=g, device=dev) * 0.02
    if outliers:
        idx = torch.randperm(K * N, generator=g, device=dev)[: K * N // 100]
        W.view(-1)[idx] = torch.randn(idx.numel(), generator=g, device=dev) * 0.2
    out = mo.quantize_int4(W.half(), I4_GROUP)
    del W
    return out


def i4_decode_bench(mo, torch, dev, args):
    R = max(1, args.copies)
    layers = [[make_i4_weights(mo, torch, K, N, 5000 + 1000 * r + i, dev)
               for i, (_, K, N) in enumerate(DECODE_LAYER)] for r in range(R)]
    g = torch.Generator(device=dev).manual_seed(1)
    xs = {K: torch.randn(1, K, generator=g, device=dev).half() for K in (4096, 11008)}
    stream = torch.cuda.Stream(dev)

    def one_step(r):
        return [mo.matmul_int4(xs[K], *w, I4_GROUP) for (_, K, _), w in zip(DECODE_LAYER, layers[r % R])]

    with torch.cuda.stream(stream):
        one_step(0)
    torch.cuda.synchronize()
    if args.no_graph:
        secs, _ = time_region(torch, stream, one_step, args.steps, args.warmup)
        steps = args.steps
    else:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for r in range(R):
                one_step(r)
        reps = max(1, args.steps // R)
        secs, _ = time_region(torch, stream, lambda i: graph.replay(), reps, max(1, args.warmup // R))
        steps = reps * R
    bytes_step = sum(i4_wbytes(K, N) for _, K, N in DECODE_LAYER)
    return {"seconds": secs, "steps": steps, "bytes_step": bytes_step,
            "launches_step": len(DECODE_LAYER), "copies": R}


I4_NORMED = ("qkv", "gate", "up")   # the projections that follow an RMSNorm in a Llama layer


def i4_rmsnorm_bench(mo, torch, dev, args):
    """fused_rmsnorm_linear_int4 at M=1 on the decode layer's normalised projections
    (qkv after input_layernorm, gate and up after post_attention_layernorm), against
    plain matmul_int4 on the same weights: one graph of R rotated weight copies each."""
    R = max(1, args.copies)
    shapes = [(K, N) for name, K, N in DECODE_LAYER if name in I4_NORMED]
    layers = [[make_i4_weights(mo, torch, K, N, 9000 + 1000 * r + i, dev) for i, (K, N) in enumerate(shapes)]
              for r in range(R)]
    g = torch.Generator(device=dev).manual_seed(4)
    x = torch.randn(1, 4096, generator=g, device=dev).half()
    wn = (1 + 0.1 * torch.randn(4096, generator=g, device=dev)).half()
    stream = torch.cuda.Stream(dev)
    out = {}
    for name, fn in (("fused", lambda w: mo.fused_rmsnorm_linear_int4(x, wn, *w, 1e-5, I4_GROUP)),
                     ("plain", lambda w: mo.matmul_int4(x, *w, I4_GROUP))):
        with torch.cuda.stream(stream):
            for w in layers[0]:
                fn(w)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for r in range(R):
                for w in layers[r]:
                    fn(w)
        reps = max(1, args.steps // R)
        secs, _ = time_region(torch, stream, lambda i: graph.replay(), reps, max(1, args.warmup // R))
        out[name] = secs / (reps * R * len(shapes))
        del graph
    del layers
    torch.cuda.empty_cache()
    return out


def i4_prefill_bench(mo, torch, dev, iters=30, warmup=10):
    out = []
    stream = torch.cuda.Stream(dev)
    for name, M, K, N in PREFILL:
        w = make_i4_weights(mo, torch, K, N, 77, dev, outliers=True)
        g = torch.Generator(device=dev).manual_seed(2)
        x = torch.randn(M, K, generator=g, device=dev).half()
        with torch.cuda.stream(stream):
            mo.matmul_int4(x, *w, I4_GROUP)
        secs, _ = time_region(torch, stream, lambda i: mo.matmul_int4(x, *w, I4_GROUP), iters, warmup)
        t = secs / iters
        fl = 2.0 * M * N * K
        out.append({"name": name, "M": M, "K": K, "N": N, "ms": t * 1e3, "tflops": fl / t / 1e12})
        del w, x
    return out


def i4_cpu_baseline(seconds_budget):
    """Reference CPU path of matmul_int4 (W in X.dtype from fp32 (q - z) * s, then X @ W)."""
    import numpy as np
    import torch

    from oracle import int4_ref as ref

    K, N = 4096, 4096
    rng = np.random.default_rng(0)
    W = (rng.standard_normal((K, N)) * 0.02).astype(np.float16).astype(np.float32)
    packed, s, z = ref.quantize(W, I4_GROUP, ref.F16)
    X = torch.from_numpy(rng.standard_normal((1, K)).astype(np.float16))
    ref.fallback_torch_cpu(X, packed, s, z, I4_GROUP)
    n, t0 = 0, time.perf_counter()
    while True:
        ref.fallback_torch_cpu(X, packed, s, z, I4_GROUP)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds_budget or n >= 10000:
            break
    per = el / n
    return {
        "value": i4_wbytes(K, N) / per / 1e9,
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"O-proj K=N=4096 M=1 fp16, group 128 fp16 scales/zeros: dequantize + X@W per "
                  f"call (quantization.py:220-239), numpy + torch CPU, {n} calls in {el:.1f}s "
                  f"({per * 1e3:.2f} ms/call)",
    }


def cpu_baseline(seconds_budget):
    """Reference CPU path (dequant to fp16 each call, then X @ W) on the O-proj shape."""
    import numpy as np
    import torch

    from oracle import q4_0_ref as ref

    K, N = 4096, 4096
    rng = np.random.default_rng(0)
    W = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    blocks = torch.from_numpy(ref.quantize_llama_rule(W))
    X = torch.from_numpy(rng.standard_normal((1, K)).astype(np.float16))

    def timed(x, budget):
        ref.fallback_torch_cpu(x, blocks)  # warm-up
        n, t0 = 0, time.perf_counter()
        while True:
            ref.fallback_torch_cpu(x, blocks)
            n += 1
            el = time.perf_counter() - t0
            if el >= budget or n >= 10000:
                return n, el

    n, el = timed(X, seconds_budget * 2 / 3)
    per = el / n
    # The secondary figure: the same call at fp32 (X.float() @ dequant_f32).
    n32, el32 = timed(X.float(), seconds_budget / 3)
    per32 = el32 / n32
    return {
        "value": wbytes(K, N) / per / 1e9,
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"O-proj K=N=4096 M=1 fp16: dequantize + X@W per call (quantization.py:452-454), "
                  f"torch CPU, {n} calls in {el:.1f}s ({per * 1e3:.2f} ms/call); "
                  f"os.cpu_count()={os.cpu_count()}",
        "secondary": {
            "value": wbytes(K, N) / per32 / 1e9,
            "unit": "GB/s",
            "sample": f"the same at fp32 (X.float() @ dequant_f32), {n32} calls in {el32:.1f}s "
                      f"({per32 * 1e3:.2f} ms/call)",
        },
    }


def probes(torch, dev):
    """Machine probes (libmcq4_bench.so) that the decode figures are read against:
    the per-launch floor of a graph, the HBM read rate of the q4_0 layout's access
    patterns at the decode layer's sizes, the round trip of a returning atomic, the
    store-to-load visibility between workgroups, and the shader clock under MFMA load."""
    lib = bench_lib()
    stream = torch.cuda.Stream(dev)
    out = {"part": "probes"}

    def graph_time(launch, n, reps=20):
        with torch.cuda.stream(stream):
            launch(0)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(n):
                launch(i)
        secs, _ = time_region(torch, stream, lambda i: graph.replay(), reps, 3)
        del graph
        return secs / (reps * n)

    # 1. Per-launch floor: back-to-back empty kernels in one graph.
    floor = {}
    for grid, block in ((1, 64), (256, 256), (256, 1024)):
        t = graph_time(lambda i: bench_check(lib.mcqb_empty(grid, block, torch.cuda.current_stream().cuda_stream),
                                             "mcqb_empty"), 50)
        floor[f"{grid}x{block}"] = round(t * 1e6, 3)
    out["empty_kernel_us_per_launch"] = floor

    # 2. Read patterns of a q4_0 weight [K/32][N][18] at the layer's shapes, over
    #    copies rotated through >= 1.1 GB (reads from HBM): contiguous, 16-column
    #    strips (one workgroup per strip, the M = 1 strip kernel's pattern), 64-column
    #    tiles split four ways along K and, at N > 4096, spans of 2-3 16-column groups
    #    (one workgroup per span, near the M = 1 span kernel's 256 spans).
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    pats = []
    for _, K, N in DECODE_LAYER[:2] + DECODE_LAYER[2:3] + DECODE_LAYER[4:]:
        nbytes = wbytes(K, N)
        copies = max(2, -(-int(1.1e9) // nbytes))
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device=dev).random_(0, 256) for _ in range(copies)]
        rec = {"K": K, "N": N, "bytes": nbytes}
        cs = lambda: torch.cuda.current_stream().cuda_stream
        kinds = {
            "contiguous": lambda i: bench_check(lib.mcqb_read_probe(bufs[i].data_ptr(), nbytes, sink.data_ptr(), cs()),
                                                "mcqb_read_probe"),
            "strip16": lambda i: bench_check(lib.mcqb_read_tiles(bufs[i].data_ptr(), K, N, 16, 1, 16, sink.data_ptr(),
                                                                 cs()), "mcqb_read_tiles"),
            "tile64_k4": lambda i: bench_check(lib.mcqb_read_tiles(bufs[i].data_ptr(), K, N, 64, 4, 16,
                                                                   sink.data_ptr(), cs()), "mcqb_read_tiles"),
        }
        if N > 4096:
            g = -(-N // (16 * 256))
            while N % (16 * g):
                g -= 1
            rec["span_cols"] = 16 * g
            kinds["span"] = lambda i, c=16 * g: bench_check(
                lib.mcqb_read_tiles(bufs[i].data_ptr(), K, N, c, 1, 16, sink.data_ptr(), cs()), "mcqb_read_tiles")
        for name, fn in kinds.items():
            t = graph_time(fn, copies)
            rec[name] = {"us": round(t * 1e6, 3), "GB/s": round(nbytes / t / 1e9, 1)}
        pats.append(rec)
        del bufs
    torch.cuda.empty_cache()
    out["read_patterns"] = pats

    # 2b. Per-group INT4 weights [K/2][N] (one byte per column per two K rows): pieces
    #     of 64 and 128 columns (bytes), each piece column split along K so the grid
    #     stays near 256 workgroups of 8 waves (the INT4 decode kernel's tile is 128).
    ipats = []
    for _, K, N in DECODE_LAYER[:2] + DECODE_LAYER[2:3] + DECODE_LAYER[4:]:
        nbytes = (K // 2) * N
        copies = max(2, -(-int(1.1e9) // nbytes))
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device=dev).random_(0, 256) for _ in range(copies)]
        rec = {"K": K, "N": N, "bytes": nbytes}
        cs = lambda: torch.cuda.current_stream().cuda_stream
        kinds = {"contiguous": lambda i: bench_check(
            lib.mcqb_read_probe(bufs[i].data_ptr(), nbytes, sink.data_ptr(), cs()), "mcqb_read_probe")}
        for piece in (64, 128):
            ks = max(1, 256 // (N // piece))
            rec[f"piece{piece}_ksplit"] = ks
            kinds[f"piece{piece}"] = lambda i, pc=piece, k=ks: bench_check(
                lib.mcqb_read_rows(bufs[i].data_ptr(), K // 2, N, pc, k, 8, sink.data_ptr(), cs()), "mcqb_read_rows")
        for name, fn in kinds.items():
            t = graph_time(fn, copies)
            rec[name] = {"us": round(t * 1e6, 3), "GB/s": round(nbytes / t / 1e9, 1)}
        ipats.append(rec)
        del bufs
    torch.cuda.empty_cache()
    out["int4_read_patterns"] = ipats

    # 3. Returning 64-bit atomic add, a dependent chain per workgroup.
    words = torch.zeros(256 * 64, dtype=torch.int64, device=dev)
    ticks = torch.zeros(256, dtype=torch.int64, device=dev)
    at = {}
    for grid in (1, 256):
        bench_check(lib.mcqb_atomic_chain(words.data_ptr(), 200, grid, ticks.data_ptr(), None), "mcqb_atomic_chain")
        torch.cuda.synchronize()
        bench_check(lib.mcqb_atomic_chain(words.data_ptr(), 200, grid, ticks.data_ptr(), None), "mcqb_atomic_chain")
        torch.cuda.synchronize()
        at[f"grid{grid}"] = round(float(ticks[:grid].double().mean()) * 10.0 / 200, 1)
    out["atomic_rtt_ns"] = at

    # 4. Store -> poll visibility between workgroups (pair stride 8: same XCD under
    #    round-robin placement; stride 1: neighbouring XCDs).
    slots = torch.zeros(4096, dtype=torch.int64, device=dev)
    res = torch.zeros(1024, dtype=torch.int64, device=dev)
    ex = []
    for sm, sname in ((0, "plain"), (1, "agent_atomic"), (2, "nontemporal")):
        for lm, lname in ((0, "sc0_buffer_load"), (1, "agent_atomic_load")):
            for d in (8, 1):
                slots.zero_()
                torch.cuda.synchronize()
                bench_check(lib.mcqb_exchange(slots.data_ptr(), res.data_ptr(), d, sm, lm, 20000, None),
                            "mcqb_exchange")
                torch.cuda.synchronize()
                h = res.view(256, 4).cpu().tolist()
                same, cross, fail_same, fail_cross = [], [], 0, 0
                for wg in range(256):
                    if (wg // d) % 2 == 0:
                        continue
                    pw = wg - d
                    sx = h[wg][0] == h[pw][0]
                    if not h[wg][3]:
                        if sx:
                            fail_same += 1
                        else:
                            fail_cross += 1
                        continue
                    (same if sx else cross).append((h[wg][2] - h[pw][1]) * 10.0)
                rec = {"store": sname, "load": lname, "pair_stride": d}
                for nm, v, f in (("same_xcd", same, fail_same), ("cross_xcd", cross, fail_cross)):
                    if v or f:
                        rec[nm] = {"pairs": len(v) + f, "never_seen": f,
                                   "p50_ns": round(statistics.median(v), 0) if v else None}
                ex.append(rec)
    out["store_to_load"] = ex

    # 5. Prefill tile time against the number of tiles in flight: the 256 x 256-tile
    #    GEMM (forced with MCQ4_GEMM_PATH=7, no K split: MCQ4_GEMM6_SPLIT=1) on M = 256,
    #    K = 4096, N = 256 n -- n tiles, one workgroup per CU up to 256, then rounds --
    #    with random operands and with all-zero operands.
    import metalops_amd as mo
    from metalops_amd import _lib as mlib
    saved = {k: os.environ.get(k) for k in ("MCQ4_GEMM_PATH", "MCQ4_GEMM6_SPLIT")}
    os.environ["MCQ4_GEMM_PATH"] = "7"
    os.environ["MCQ4_GEMM6_SPLIT"] = "1"
    mlib.reload_options()
    tiles = []
    try:
        for n in (1, 8, 64, 128, 192, 256, 448, 512):
            rec = {"tiles": n}
            w = make_weights(mo, torch, 4096, 256 * n, 5, dev)
            g = torch.Generator(device=dev).manual_seed(6)
            x = torch.randn(256, 4096, generator=g, device=dev).half()
            for kind in ("random", "zero"):
                if kind == "zero":
                    w.zero_()
                    x.zero_()
                t = graph_time(lambda i: mo.matmul_ggml_q4_0(x, w), 4, reps=10)
                rec[kind + "_us"] = round(t * 1e6, 2)
            rec["tflops_random"] = round(2.0 * 256 * 4096 * 256 * n / (rec["random_us"] * 1e-6) / 1e12, 1)
            tiles.append(rec)
            del w, x
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
        mlib.reload_options()
    out["prefill_tile_scaling"] = tiles

    # 6. Shader clock under a dense MFMA load.
    out["sclk_mfma_mhz"] = sclk_mfma_mhz(torch, dev)
    return out


def sclk_mfma_mhz(torch, dev):
    """Median shader clock (MHz) of the waves of one dense-MFMA launch on every CU
    (mcqb_measure_sclk: each wave's s_memtime cycles over its 100 MHz s_memrealtime
    ticks).  The pool's boxes differ in it, and the decode and prefill figures with it."""
    lib = bench_lib()
    tk = torch.zeros(4096, dtype=torch.int64, device=dev)
    bench_check(lib.mcqb_measure_sclk(tk.data_ptr(), 20000, None), "mcqb_measure_sclk")
    torch.cuda.synchronize()
    t2 = tk.view(-1, 2).double()
    return round(float((100.0 * t2[:, 0] / t2[:, 1]).median()), 0)


def run_part(mo, torch, dev, args):
    """One part of the benchmark, printing its own JSON line (profiler passes)."""
    if args.part == "copy":
        a = torch.ones(256 << 20, dtype=torch.uint8, device=dev)
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"part": "copy", "bytes_read": a.numel(), "bytes_written": b.numel(),
                          "launches": 5}), flush=True)
    elif args.part == "decode":
        dec = decode_bench(mo, torch, dev, args)
        t = dec["seconds"] / dec["steps"]
        print(json.dumps({"part": "decode", "GB/s": round(dec["bytes_step"] / t / 1e9, 1),
                          "us_per_launch": round(t / dec["launches_step"] * 1e6, 3),
                          "weight_bytes_per_launch": dec["bytes_step"] / dec["launches_step"]}),
              flush=True)
    elif args.part == "int4-decode":
        dec = i4_decode_bench(mo, torch, dev, args)
        t = dec["seconds"] / dec["steps"]
        print(json.dumps({"part": "int4-decode", "GB/s": round(dec["bytes_step"] / t / 1e9, 1),
                          "us_per_launch": round(t / dec["launches_step"] * 1e6, 3),
                          "weight_bytes_per_launch": dec["bytes_step"] / dec["launches_step"]}),
              flush=True)
    elif args.part == "configs":
        print(json.dumps({"part": "configs", "configs": config_points(mo, torch, dev)}), flush=True)
    elif args.part == "probes":
        print(json.dumps(probes(torch, dev)), flush=True)
    elif args.part == "int4-prefill":
        print(json.dumps({"part": "int4-prefill", "configs": i4_prefill_bench(mo, torch, dev)}),
              flush=True)
    elif args.part == "prefill-splits":
        print(json.dumps({"part": "prefill-splits", "points": prefill_split_sweep(mo, torch, dev)}), flush=True)
    elif args.part == "prefill-routing":
        print(json.dumps({"part": "prefill-routing", "points": prefill_routing_sweep(mo, torch, dev)}), flush=True)
    else:
        print(json.dumps({"part": "prefill", "configs": prefill_bench(mo, torch, dev)}), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested). "
              "The q4_0 kernels shard by columns or K blocks without a collective on the "
              "decode path; multi-GPU runs are not part of this build.", file=sys.stderr)
        sys.exit(2)
    import torch

    import metalops_amd as mo

    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.part != "all":
        run_part(mo, torch, dev, args)
        return

    dec = decode_bench(mo, torch, dev, args)
    t_step = dec["seconds"] / dec["steps"]
    gbs = dec["bytes_step"] / t_step / 1e9
    t_launch = t_step / dec["launches_step"]
    pre = prefill_bench(mo, torch, dev)
    pre_up = pre[0]
    pre_tflops = sum(2.0 * p["M"] * p["K"] * p["N"] for p in pre) / sum(p["ms"] / 1e3 for p in pre) / 1e12
    points = config_points(mo, torch, dev)
    sclk = sclk_mfma_mhz(torch, dev)

    i4_dec = i4_decode_bench(mo, torch, dev, args)
    i4_t = i4_dec["seconds"] / i4_dec["steps"]
    i4_gbs = i4_dec["bytes_step"] / i4_t / 1e9
    i4_pre = i4_prefill_bench(mo, torch, dev)
    i4_rms = i4_rmsnorm_bench(mo, torch, dev, args)

    cpu = i4_cpu = pre_cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(args.cpu_seconds)
        pre_cpu = prefill_cpu_baseline(args.cpu_seconds)
        i4_cpu = i4_cpu_baseline(args.cpu_seconds / 2)

    line = {
        "metric": "q4_0 GEMV GB/s (% HBM peak) at M=1; q4_0 GEMM TFLOP/s (% MFMA) at M=2048",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": dec["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(t_step * 1e3, 5),
        "median_ms_per_step": round(dec["median_step_s"] * 1e3, 5),
        # What ms_per_step rests on: the timed region, its graph replays (each of
        # `weight_copies_rotated` steps) and, when the region is under 50 ms, the
        # per-step time over at least 50 ms of replays of the same graph.
        "timing": {
            "timed_region_ms": round(dec["seconds"] * 1e3, 4),
            "graph_replays": dec["graph_replays"],
            "steps_per_replay": dec["copies"],
            "check_ms_per_step_50ms": (round(dec["check_step_s"] * 1e3, 5)
                                       if dec["check_step_s"] is not None else None),
        },
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0 x f16 -> f32 acc",
        "data": "synthetic (seeded N(0,0.02) weights, llama.cpp q4_0 rule; N(0,1) fp16 activations)",
        "config": {
            "workload": "Llama-2-7B decode projections at M=1 (configs[1]): qkv 4096x12288, "
                        "o 4096x4096, gate/up 4096x11008 x2, down 11008x4096",
            "M": 1,
            "bytes_per_step": dec["bytes_step"],
            "weight_copies_rotated": dec["copies"],
            "weight_pool_bytes": dec["weight_pool_bytes"],
            "graph": not args.no_graph,
        },
        "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "gbs_incl_x_y": round((dec["bytes_step"] + dec["xy_step"]) / t_step / 1e9, 1),
        # The same weight bytes read by a plain streaming kernel, one launch per
        # projection, in a graph: what the launch sizes allow, before any math.
        "read_ceiling": {
            "GB/s": round(dec["bytes_step"] / dec["read_ceiling_s"] / 1e9, 1),
            "pct_hbm_peak": round(100 * dec["bytes_step"] / dec["read_ceiling_s"] / 1e9 / HBM_PEAK_GBS, 2),
            "kernel": "read_probe_kernel (mcqb_read_probe: 16 KiB per 256-thread workgroup)",
            "value_over_ceiling": round(dec["read_ceiling_s"] / t_step, 4),
        },
        # The box: shader clock under a dense MFMA load (the decode kernels' exposed
        # math and the power-bound prefill scale with it; 1391-1530 MHz seen in the pool).
        "machine": {"sclk_mfma_mhz": sclk},
        # The layer with gate and up in one launch (matmul_ggml_q4_0_grouped, no
        # reference counterpart): the same bytes in four launches.
        "grouped_gate_up": {
            "GB/s": round(dec["bytes_step"] / dec["grouped_step_s"] / 1e9, 1),
            "pct_hbm_peak": round(100 * dec["bytes_step"] / dec["grouped_step_s"] / 1e9 / HBM_PEAK_GBS, 2),
            "ms_per_step": round(dec["grouped_step_s"] * 1e3, 5),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(dec["bytes_step"] / dec["launches_step"] / t_launch / 1e9, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": DECODE_TRAFFIC_BYTES,
            "algorithmic_bytes_per_launch": dec["bytes_step"] // dec["launches_step"],
            "kernel": DECODE_KERNEL,
            "avg_launch_us": round(t_launch * 1e6, 3),
        },
        "prefill": {
            "metric": "q4_0 GEMM TFLOP/s (% MFMA) at M=2048 (configs[3], up and down together)",
            "value": round(pre_tflops, 1),
            "unit": "TFLOP/s",
            "pct_mfma_peak": round(100 * pre_tflops / FP16_PEAK_TFLOPS, 2),
            "configs": [{k: (round(v, 3) if isinstance(v, float) else v) for k, v in p.items()}
                        for p in pre],
            "roofline": {
                "bound": "mfma",
                "achieved": round(pre_up["tflops"], 1),
                "peak": FP16_PEAK_TFLOPS,
                "unit": "TFLOP/s",
                "frac": round(pre_up["tflops"] / FP16_PEAK_TFLOPS, 4),
                "traffic": PREFILL_UP_TRAFFIC_BYTES,
                "kernel": PREFILL_KERNEL,
                "avg_launch_us": round(pre_up["ms"] * 1e3, 2),
            },
            "cpu_baseline": pre_cpu,
        },
        "configs": points,
        "cpu_baseline": cpu,
        "int4": {
            "workload": "same decode layer and prefill shapes, per-group INT4 (group 128, fp16 "
                        "scales/zeros; quantization.py:26-239)",
            "decode_gbs": round(i4_gbs, 1),
            "decode_ms_per_step": round(i4_t * 1e3, 5),
            "bytes_per_step": i4_dec["bytes_step"],
            "roofline": {
                "bound": "hbm",
                "achieved": round(i4_gbs, 1),
                "peak": HBM_PEAK_GBS,
                "unit": "GB/s",
                "frac": round(i4_gbs / HBM_PEAK_GBS, 4),
                "traffic": I4_DECODE_TRAFFIC_BYTES,
                "algorithmic_bytes_per_launch": i4_dec["bytes_step"] // i4_dec["launches_step"],
                "kernel": "i4_gemv1_kernel (decode GEMV, M=1)",
                "avg_launch_us": round(i4_t / i4_dec["launches_step"] * 1e6, 3),
            },
            "fused_rmsnorm_m1": {
                "projections": list(I4_NORMED),
                "us_per_call": round(i4_rms["fused"] * 1e6, 3),
                "plain_matmul_us_per_call": round(i4_rms["plain"] * 1e6, 3),
            },
            "prefill": {
                "configs": [{k: (round(v, 3) if isinstance(v, float) else v) for k, v in p.items()}
                            for p in i4_pre],
                "roofline": {
                    "bound": "mfma",
                    "achieved": round(i4_pre[0]["tflops"], 1),
                    "peak": FP16_PEAK_TFLOPS,
                    "unit": "TFLOP/s",
                    "frac": round(i4_pre[0]["tflops"] / FP16_PEAK_TFLOPS, 4),
                    "traffic": I4_PREFILL_UP_TRAFFIC_BYTES,
                    "kernel": "i4_gemm7_kernel (M=2048 K=4096 N=14336)",
                },
            },
            "cpu_baseline": i4_cpu,
        },
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

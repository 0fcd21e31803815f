#!/usr/bin/env python3
"""Benchmark of the quantized-linear hot path on one MI355X.

Workload: the int4 W4A16 group-128 decode sweep at
Llama-3-8B MLP shapes -- gate_up (K=4096, N=28672) and down (K=14336, N=4096),
M in {1, 8, 32, 128}, bf16 activations ~ N(0,1), codes ~ U{0..15}, zero point
8, bf16 scales ~ U[0.002, 0.02].  One *step* is one pass over the sweep: the 8
GEMMs (2 shapes x 4 M), each on the next of a rotating set of weight copies
(>= 512 MB per shape, twice the 256 MB Infinity Cache) so bytes come from HBM.

``value`` is HBM GB/s over the packed-weight + scale bytes of the step (the
config's stated unit).  ``roofline`` describes the dominant HBM-bound launch,
gate_up at M=32, with bytes = weights + scales + activations + output, timed
with HIP events on the stream the kernel runs on.  ``cpu_baseline`` times the
CPU oracle (dequantize-then-matmul, oracle/int4.py) on one gate_up M=32 GEMM.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
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

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
ROTATE_BYTES = 512 * 2**20
SHAPES = {"gate_up": (4096, 28672), "down": (14336, 4096)}
MS = (1, 8, 32, 128)
HEADLINE = ("gate_up", 32)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def weight_bytes(k, n):
    return k * n // 2 + (k // 128) * n * 2


def cpu_baseline(seconds_budget: float = 20.0) -> dict:
    """Time the CPU oracle on one gate_up M=32 GEMM (bounded sample)."""
    import numpy as np
    from oracle import int4 as oint4
    try:
        from threadpoolctl import threadpool_info
        threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:  # pragma: no cover
        threads = 1
    k, n = SHAPES["gate_up"]
    m = 32
    rng = np.random.default_rng(0)
    codes = rng.integers(0, 16, (k, n), dtype=np.uint8)
    q = oint4.pack_int4(codes)
    s = rng.uniform(0.002, 0.02, (k // 128, n)).astype(np.float32)
    a = rng.standard_normal((m, k)).astype(np.float32)
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start < 1.0):
        t0 = time.perf_counter()
        oint4.w4a16_reference(a, q, s)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > seconds_budget:
            break
    med = statistics.median(times)
    return {
        "value": round(weight_bytes(k, n) / med / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"one gate_up GEMM (M=32, K=4096, N=28672): unpack + (q-8)*s + fp32 "
                   f"matmul (oracle/int4.py w4a16_reference), median of {len(times)} runs, "
                   f"{med * 1e3:.1f} ms each; host has {os.cpu_count()} logical CPUs"),
    }


class Int4Point:
    def __init__(self, name, k, n, m, dev, copies):
        import torch
        from torchinferno_amd import _lib
        from torchinferno_amd.kernels import int4 as ti4
        self.name, self.k, self.n, self.m = name, k, n, m
        self.a = torch.randn((m, k), device=dev, dtype=torch.bfloat16)
        self.out = torch.empty((m, n), device=dev, dtype=torch.bfloat16)
        self.copies = copies
        self.ws = ti4.make_workspace(n, dev, size_k=k, max_m=m)
        self.fn = _lib.lib().ti_w4a16_gemm
        self.ws_bytes = self.ws.numel() * 4
        self.i = 0

    def launch(self, stream):
        pw, ps = self.copies[self.i % len(self.copies)]
        self.i += 1
        st = self.fn(self.a.data_ptr(), 2, pw.data_ptr(), ps.data_ptr(), self.out.data_ptr(),
                     self.m, self.n, self.k, 128, self.ws.data_ptr(), self.ws_bytes, stream)
        if st:
            raise RuntimeError(f"ti_w4a16_gemm failed: {st}")

    @property
    def wbytes(self):
        return weight_bytes(self.k, self.n)

    @property
    def algo_bytes(self):
        return self.wbytes + self.m * self.k * 2 + self.m * self.n * 2

    @property
    def flops(self):
        return 2 * self.m * self.n * self.k


def make_copies(k, n, dev):
    import torch
    from torchinferno_amd.kernels import int4 as ti4
    codes = torch.randint(0, 16, (k, n), device=dev, dtype=torch.int32)
    q = ti4.pack_int4(codes)
    del codes
    s = (torch.rand((k // 128, n), device=dev) * 0.018 + 0.002).to(torch.bfloat16)
    ncopy = max(2, -(-ROTATE_BYTES // weight_bytes(k, n)))
    copies = [ti4.repack_int4(q, s) for _ in range(ncopy)]
    torch.cuda.synchronize()
    return copies


def timed_burst(launch_fns, reps, stream_handle):
    """Queue `reps` rounds of launches behind a spin kernel so the host never
    starves the GPU; return elapsed GPU ms between the events."""
    import torch
    torch.cuda._sleep(int(50e6))
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        for fn in launch_fns:
            fn(stream_handle)
    end.record()
    end.synchronize()
    return start.elapsed_time(end)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(each BASELINE shape is one GPU's shard); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    from torchinferno_amd import _lib
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    _lib.lib()
    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    props = torch.cuda.get_device_properties(dev)
    log(f"device: {props.name} CUs={props.multi_processor_count}")

    points = []
    for name, (k, n) in SHAPES.items():
        copies = make_copies(k, n, dev)
        log(f"{name}: K={k} N={n} copies={len(copies)}")
        for m in MS:
            points.append(Int4Point(name, k, n, m, dev, copies))
    stream = torch.cuda.current_stream(dev).cuda_stream

    # Per-point launch durations (each point alone, back-to-back launches).
    per_point = {}
    for p in points:
        timed_burst([p.launch], 20, stream)  # warm
        reps = 200
        ms = timed_burst([p.launch], reps, stream)
        per_point[(p.name, p.m)] = ms / reps

    # The timed region: exactly `steps` steps of the full sweep.
    for _ in range(args.warmup):
        for p in points:
            p.launch(stream)
    torch.cuda.synchronize()
    launches = [p.launch for p in points]
    torch.cuda._sleep(int(50e6))
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        for fn in launches:
            fn(stream)
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = start.elapsed_time(end)
    ms_per_step = gpu_ms / args.steps
    step_bytes = sum(p.wbytes for p in points)
    value = step_bytes / (ms_per_step * 1e-3) / 1e9

    pts = []
    for p in points:
        t = per_point[(p.name, p.m)] * 1e-3
        gbs = p.algo_bytes / t / 1e9
        tf = p.flops / t / 1e12
        hbm_bound = p.m <= 32
        pts.append({
            "shape": p.name, "M": p.m, "K": p.k, "N": p.n, "us": round(t * 1e6, 2),
            "weight_GBs": round(p.wbytes / t / 1e9, 1), "algo_GBs": round(gbs, 1),
            "TFLOPs": round(tf, 2), "bound": "hbm" if hbm_bound else "mfma",
            "frac": round(gbs / HBM_PEAK_GBS if hbm_bound else tf / BF16_PEAK_TFLOPS, 4),
        })
    head = next(p for p in points if (p.name, p.m) == HEADLINE)
    t_head = per_point[HEADLINE] * 1e-3
    achieved = head.algo_bytes / t_head / 1e9
    roofline = {
        "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
        "kernel": "ti::int4::w4a16_decode_kernel<bf16, MR=32, NT=4, WK=2, R=3, SPLIT=0>",
        "launch": "gate_up K=4096 N=28672 M=32",
        "avg_launch_us": round(t_head * 1e6, 2),
        "algo_bytes_per_launch": head.algo_bytes,
    }
    cpu = None
    if not args.no_cpu_baseline:
        log("timing CPU baseline ...")
        cpu = cpu_baseline()
    line = {
        "metric": "TFLOP/s and HBM GB/s vs roofline, int4/FP8 GEMM at Llama-3 8B/70B shapes",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random int4 codes, bf16 scales/activations; no checkpoint)",
        "config": {"workload": "int4 W4A16 g128 decode sweep (BASELINE configs[1])",
                   "shapes": {k: {"K": v[0], "N": v[1]} for k, v in SHAPES.items()},
                   "M": list(MS), "bytes_per_step": step_bytes, "parallelism": "none (1 GPU)"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "points": pts,
        "wall_s": round(wall, 3),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

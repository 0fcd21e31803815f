#!/usr/bin/env python3
"""Benchmark of the quantized-linear hot path on one MI355X.

Headline workload: the int4 W4A16 group-128 decode
sweep at Llama-3-8B MLP shapes -- gate_up (K=4096, N=28672) and down (K=14336,
N=4096), M in {1, 8, 32, 128}, bf16 activations ~ N(0,1), codes ~ U{0..15}, zero
point 8, bf16 scales ~ U[0.002, 0.02].  One *step* is one pass over the sweep:
the 8 GEMMs, each on the next copy of its shape from a rotating set shared by
all M points of that shape (>= 512 MiB per shape, twice the 256 MiB Infinity
Cache), so no launch re-reads a copy another launch has just brought on chip and
bytes come from HBM.  ``value`` is
HBM GB/s over the packed-weight + scale bytes of a step (the config's unit).

``roofline`` describes the launch that dominates a step's time, with its
algorithmic bytes (or flops) over its average duration, measured with HIP
events on the stream the kernel runs on.  ``points`` lists every BASELINE
config measured the same way: config 0 (int4 fp16), config 2 (FP8 per-token x
per-channel, Llama-3-70B, plus its fused add+RMSNorm / SwiGLU -> FP8
activation producers), config 3 (DeepSeek 128x128 block FP8, and the same
shapes with MXFP4 weights) and config 4 (routed FP8 MoE, 256 experts, top-8,
router included, and the same experts in MXFP4).  ``cpu_baseline`` times the
reference's PyTorch CPU path (dequantize, then an fp32 matmul) on one config-1
gate_up M=32 GEMM; ``cpu_points`` does the same for samples of configs 2, 3 and 4.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--only int4|fp8|moe]
"""
from __future__ import annotations

import argparse
import gc
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP8_PEAK_TFLOPS = 5000.0
ROTATE_BYTES = 512 * 2**20
SHAPES = {"gate_up": (4096, 28672), "down": (14336, 4096)}
MS = (1, 8, 32, 128)
FP8_SHAPES = {"qkv": (8192, 10240), "gate_up": (8192, 57344), "down": (28672, 8192)}
FP8_MS = (1, 64, 512, 4096)
BLOCK_SHAPES = {"a": (7168, 18432), "b": (18432, 7168), "c": (7168, 24576)}
BLOCK_MS = (16, 256, 4096)
MOE_TS = (64, 512, 4096)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def rand_e4m3(shape, device=None, generator=None):
    """Random finite e4m3fn codes (every byte but the NaN codes 0x7F and 0xFF), as
    uint8: synthetic FP8 weights and activations."""
    import torch
    mag = torch.randint(0, 0x7F, shape, device=device, generator=generator, dtype=torch.uint8)
    return mag.bitwise_or_(torch.randint(0, 2, shape, device=device, generator=generator, dtype=torch.uint8) << 7)


def quant_weight_per_channel(n, k, dev):
    """Config 2's weight: N(0, 0.02) in bf16, per-output-channel e4m3 (absmax/448),
    by the package's own quantizer (weight preparation, not timed)."""
    import torch
    from torchinferno_amd.kernels import fp8 as tf8
    wq, ws = tf8.quantize_weight_fp8_per_channel((torch.randn((n, k), device=dev) * 0.02).to(torch.bfloat16))
    return wq, ws.reshape(-1).float().contiguous()


def quant_weight_block(n, k, dev, pow2=False):
    """Config 3/4's weight: N(0, 0.02) quantized in 128x128 blocks, s = block
    absmax / 448 (rounded up to a power of two with ``pow2``, DeepSeek-V4's E8M0
    scales); codes by torch's e4m3 cast.  Returns (codes [n, k], scales fp32
    [ceil(n/128), k/128])."""
    import torch
    nb, kb = -(-n // 128), k // 128
    w = torch.randn((nb * 128, k), device=dev) * 0.02
    w[n:] = 0
    blocks = w.view(nb, 128, kb, 128)
    amax = blocks.abs().amax(dim=(1, 3))
    sc = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
    if pow2:
        sc = torch.exp2(torch.ceil(torch.log2(sc)))
    q = (blocks / sc[:, None, :, None]).view(nb * 128, k)[:n].to(torch.float8_e4m3fn).contiguous()
    return q, sc.float().contiguous()


def quant_act(m, k, dev, mode):
    """Activations: N(0,1) bf16 rows quantized per token (mode 0) or per 1x128 block
    with step-major scales [K/128, M] (modes 1-4; power-of-two scales for 3 and 4),
    by the package's own quantizers."""
    import torch
    from torchinferno_amd.kernels import block_fp8 as tb
    from torchinferno_amd.kernels import fp8 as tf8
    x = torch.randn((m, k), device=dev).to(torch.bfloat16)
    if mode == 0:
        a, asc = tf8.quantize_activation_fp8_per_token(x)
        return a, asc.reshape(-1).contiguous()
    return tb._act_quant_stepmajor(x, mode >= 3)


def weight_bytes(k, n):
    return k * n // 2 + (k // 128) * n * 2


def _cpu_time(fn, budget_s):
    """Median seconds of fn() over up to 3 runs after one warm-up, stopping early
    once `budget_s` is spent; returns (median, runs)."""
    fn()
    times = []
    t_start = time.perf_counter()
    while len(times) < 3:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s:
            break
    return statistics.median(times), len(times)


def cpu_baseline(budget_s: float = 6.0) -> tuple[dict, list]:
    """The reference's PyTorch CPU path on the box's host cores, on bounded samples
    of the BASELINE workloads (dequantize, then an fp32 matmul):

    * int4 (config 1, gate_up M=32): unpack the int32 words, ``(q - 8) * s`` in fp32,
      ``a.float() @ w`` -- ``_dequant_ref``, tests/test_marlin_int4.py:40-49;
    * FP8 per-token x per-channel (config 2, qkv M=64): ``xq.float() * xs`` and
      ``wq.float() * ws``, fp32 matmul;
    * block FP8 (config 3 a, M=16): ``dequantize_block_fp8``
      (src/torchinferno/models/deepseek_v4/ops.py:180-188) + matmul;
    * MoE (config 4 T=64): the per-expert loop of MoE.forward
      (src/torchinferno/models/deepseek_v4/tensor_parallel.py:899-907) over 8 of
      the touched experts, scaled to all of them.

    Threads: torch.get_num_threads(), i.e. OMP_NUM_THREADS where set (the box's CPU
    share), else torch's default.  Returns (the int4 record, the other records)."""
    import torch
    threads = torch.get_num_threads()
    host = f"{threads} threads (torch.get_num_threads) of {os.cpu_count()} logical CPUs"
    g = torch.Generator().manual_seed(0)

    def e4m3(*shape):
        return rand_e4m3(shape, generator=g).view(torch.float8_e4m3fn)

    # int4 gate_up M=32
    k, n = SHAPES["gate_up"]
    m = 32
    words = torch.randint(-2**31, 2**31 - 1, (k // 8, n), generator=g, dtype=torch.int32)
    sc = torch.rand((k // 128, n), generator=g) * 0.018 + 0.002
    a = torch.randn((m, k), generator=g)
    shifts = torch.arange(0, 32, 4, dtype=torch.int32).view(1, 8, 1)

    def deq4():
        q = ((words.view(k // 8, 1, n) >> shifts) & 0xF).view(k, n)
        return (q.float() - 8.0) * sc.repeat_interleave(128, 0)

    w = deq4()
    t_deq, r1 = _cpu_time(deq4, budget_s)
    t_mm, r2 = _cpu_time(lambda: a @ w, budget_s)
    t = t_deq + t_mm
    int4 = {
        "value": round(weight_bytes(k, n) / t / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
        "sample": (f"one config-1 gate_up GEMM (M=32, K=4096, N=28672) on torch CPU: unpack + (q-8)*s "
                   f"{t_deq * 1e3:.1f} ms + fp32 matmul {t_mm * 1e3:.1f} ms (medians of {r1}/{r2} runs); {host}"),
    }
    del w, words
    recs = []

    # FP8 rowcol: config 2 qkv M=64
    k, n, m = 8192, 10240, 64
    wq, ws = e4m3(n, k), torch.rand((1, n), generator=g) * 1e-3
    xq, xs = e4m3(m, k), torch.rand((m, 1), generator=g) * 1e-2
    t_deq, _ = _cpu_time(lambda: wq.float() * ws.t(), budget_s)
    wd = wq.float() * ws.t()
    t_mm, runs = _cpu_time(lambda: (xq.float() * xs) @ wd.t(), budget_s)
    t = t_deq + t_mm
    recs.append({"point": "cpu config2 fp8 rowcol qkv M=64 K=8192 N=10240", "us": round(t * 1e6, 1),
                 "TFLOPs": round(2 * m * n * k / t / 1e12, 4), "algo_GBs": round((n * k + m * k) / t / 1e9, 3),
                 "dequant_ms": round(t_deq * 1e3, 2), "matmul_ms": round(t_mm * 1e3, 2), "cores": threads,
                 "kind": "port"})
    del wq, wd

    # block FP8: config 3 a M=16
    k, n, m = 7168, 18432, 16
    bq, bs = e4m3(n, k), torch.rand((n // 128, k // 128), generator=g) * 1e-3
    aq, a_s = e4m3(m, k), torch.rand((m, k // 128), generator=g) * 1e-2

    def deq_block(w, s):
        full = s.repeat_interleave(128, 0).repeat_interleave(128, 1)[: w.size(0), : w.size(1)]
        return w.float() * full

    t_deq, _ = _cpu_time(lambda: deq_block(bq, bs), budget_s)
    bd = deq_block(bq, bs)
    t_mm, _ = _cpu_time(lambda: (aq.float() * a_s.repeat_interleave(128, 1)) @ bd.t(), budget_s)
    t = t_deq + t_mm
    recs.append({"point": "cpu config3 fp8 block a M=16 K=7168 N=18432", "us": round(t * 1e6, 1),
                 "TFLOPs": round(2 * m * n * k / t / 1e12, 4), "algo_GBs": round((n * k + m * k) / t / 1e9, 3),
                 "dequant_ms": round(t_deq * 1e3, 2), "matmul_ms": round(t_mm * 1e3, 2), "cores": threads,
                 "kind": "port"})
    del bq, bd

    # MoE: config 4 T=64, per-expert loop over a sample of experts
    e_tot, h, inter, topk, tok = 256, 7168, 2048, 8, 64
    logits = torch.randn((tok, e_tot), generator=g)
    ids = torch.topk(torch.softmax(logits, -1), topk, dim=-1).indices
    touched = torch.unique(ids)
    x = torch.randn((tok, h), generator=g).to(torch.bfloat16)
    sample = touched[:8].tolist()
    experts = {ei: (e4m3(2 * inter, h), torch.rand((2 * inter // 128, h // 128), generator=g) * 1e-3,
                    e4m3(h, inter), torch.rand((h // 128, inter // 128), generator=g) * 1e-3) for ei in sample}

    def moe_loop():
        y = torch.zeros((tok, h))
        for ei in sample:
            w13, s13, w2, s2 = experts[ei]
            rows, slot = torch.where(ids == ei)
            xe = x[rows].float()
            gu = xe @ deq_block(w13, s13).t()
            act = torch.nn.functional.silu(gu[:, :inter]) * gu[:, inter:]
            y[rows] += act.to(torch.bfloat16).float() @ deq_block(w2, s2).t()
        return y

    t_s, runs = _cpu_time(moe_loop, budget_s)
    t = t_s * touched.numel() / len(sample)
    recs.append({"point": f"cpu config4 fp8 moe T={tok} experts_touched={touched.numel()}",
                 "us": round(t * 1e6, 1), "tokens_per_s": round(tok / t, 2),
                 "algo_GBs": round(touched.numel() * (3 * inter * h) / t / 1e9, 3), "cores": threads,
                 "kind": "port",
                 "sample": f"{len(sample)} of the {touched.numel()} touched experts, median of {runs} runs, "
                           f"scaled by {touched.numel()}/{len(sample)}"})
    return int4, recs


def timed_burst(launch_fns, reps, stream_handle):
    """Queue `reps` rounds of launches behind a spin kernel so the host never
    starves the GPU; return elapsed GPU ms between events recorded on the
    launches' stream."""
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


def _check(name, st):
    if st:
        from torchinferno_amd import _lib
        raise RuntimeError(f"{name} failed ({st}): {_lib.lib().ti_last_error().decode()}")


# --------------------------------------------------------------------------- int4


class Rotation:
    """Weight copies of one shape, handed out in turn to every launch of that shape,
    so consecutive launches -- of any M -- read different copies and a copy comes
    back only after >= ROTATE_BYTES of other weights have streamed past it."""

    def __init__(self, copies):
        self.copies = copies
        self.i = 0

    def next(self):
        c = self.copies[self.i % len(self.copies)]
        self.i += 1
        return c


class Int4Point:
    def __init__(self, name, k, n, m, dev, copies, dtype_code=2):
        import torch
        from torchinferno_amd import _lib
        from torchinferno_amd.kernels import int4 as ti4
        self.name, self.k, self.n, self.m = name, k, n, m
        dt = torch.bfloat16 if dtype_code == 2 else torch.float16
        self.dtype_code = dtype_code
        self.a = torch.randn((m, k), device=dev, dtype=dt)
        self.out = torch.empty((m, n), device=dev, dtype=dt)
        self.copies = copies if isinstance(copies, Rotation) else Rotation(copies)
        self.ws = ti4.make_workspace(n, dev, size_k=k, max_m=m)
        self.fn = _lib.lib().ti_w4a16_gemm
        self.ws_bytes = self.ws.numel() * 4

    def launch(self, stream):
        pw, ps = self.copies.next()
        _check("ti_w4a16_gemm", self.fn(self.a.data_ptr(), self.dtype_code, pw.data_ptr(), ps.data_ptr(),
                                        self.out.data_ptr(), self.m, self.n, self.k, 128, self.ws.data_ptr(),
                                        self.ws_bytes, stream))

    @property
    def wbytes(self):
        return weight_bytes(self.k, self.n)

    @property
    def algo_bytes(self):
        return self.wbytes + self.m * self.k * 2 + self.m * self.n * 2

    @property
    def flops(self):
        return 2 * self.m * self.n * self.k

    @property
    def bound(self):
        # bf16 ridge: 2.5 PFLOP/s / 8 TB/s = 312 flop/byte
        return "mfma" if self.flops / self.algo_bytes > BF16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9) else "hbm"


def plan_name(p) -> str:
    import ctypes
    from torchinferno_amd import _lib
    buf = ctypes.create_string_buffer(256)
    _lib.lib().ti_w4a16_plan_name(p.m, p.n, p.k, 128, buf, 256)
    return buf.value.decode()


def read_traffic(label: str):
    """HBM bytes per launch of `label` from the committed rocprofv3 counter summary
    (profiles/int4_dominant_traffic.txt: FETCH_SIZE x 2.0 + WRITE_SIZE x 1.0, the
    factors a copy kernel of known size gives); None if absent or for another launch."""
    path = os.path.join(ROOT, "profiles", "int4_dominant_traffic.txt")
    try:
        vals = dict(line.split("=", 1) for line in open(path).read().split("\n") if "=" in line)
    except OSError:
        return None
    if vals.get("launch", "").strip() != label:
        return None
    return int(float(vals["hbm_bytes_per_launch"]))


def make_int4_copies(k, n, dev, dtype=None):
    import torch
    from torchinferno_amd.kernels import int4 as ti4
    dtype = dtype or torch.bfloat16
    codes = torch.randint(0, 16, (k, n), device=dev, dtype=torch.int32)
    q = ti4.pack_int4(codes)
    del codes
    s = (torch.rand((k // 128, n), device=dev) * 0.018 + 0.002).to(dtype)
    ncopy = max(2, -(-ROTATE_BYTES // weight_bytes(k, n)))
    copies = [ti4.repack_int4(q, s) for _ in range(ncopy)]
    torch.cuda.synchronize()
    return copies


def point_record(label, t_s, algo_bytes, flops, bound, peak_tf, extra=None):
    gbs = algo_bytes / t_s / 1e9
    tf = flops / t_s / 1e12
    rec = {"point": label, "us": round(t_s * 1e6, 2), "algo_GBs": round(gbs, 1), "TFLOPs": round(tf, 2),
           "bound": bound, "frac": round(gbs / HBM_PEAK_GBS if bound == "hbm" else tf / peak_tf, 4)}
    if extra:
        rec.update(extra)
    return rec


# --------------------------------------------------------------------------- FP8


def fp8_points(dev, stream):
    """Config 2 (rowcol) and config 3 (block) GEMMs on pre-quantized activations, and
    config 2 at M=64 and 4096 again with the per-token activation quant timed in.
    Modes 3 and 4 time config 3's shapes with DeepSeek-V4's power-of-two (ue8m0 /
    E8M0) scales, which the MFMA applies (block FP8 and MXFP4)."""
    import torch
    from torchinferno_amd import _lib
    L = _lib.lib()
    ws = torch.zeros(64 << 20, dtype=torch.int32, device=dev)
    recs = []
    for mode, shapes, ms in ((0, FP8_SHAPES, FP8_MS), (1, BLOCK_SHAPES, BLOCK_MS), (2, BLOCK_SHAPES, BLOCK_MS),
                             (3, BLOCK_SHAPES, BLOCK_MS), (4, BLOCK_SHAPES, BLOCK_MS)):
        f4 = mode in (2, 4)
        pow2 = mode >= 3
        for sname, (k, n) in shapes.items():
            wbytes_n = n * k // 2 if f4 else n * k
            ncopy = max(2, -(-ROTATE_BYTES // wbytes_n))
            if f4:  # MXFP4: e2m1 pairs, e8m0 scale per 32 K
                bq = [torch.randint(0, 256, (n, k // 2), device=dev, dtype=torch.uint8) for _ in range(ncopy)]
                from torchinferno_amd.kernels.block_fp8 import fp4_scale_stepmajor
                bs = [fp4_scale_stepmajor(torch.randint(118, 130, (n, k // 32), device=dev, dtype=torch.uint8))
                      for _ in range(ncopy)]
            else:
                # quantized N(0, 0.02) weights, as configs 2 and 3 define them
                made = [quant_weight_per_channel(n, k, dev) if mode == 0 else quant_weight_block(n, k, dev, pow2)
                        for _ in range(ncopy)]
                bq = [q for q, _ in made]
                bs = [sc for _, sc in made]
                del made
                if mode == 0:  # per-token FP8: the weights in the tiled layout the hooks cache
                    bq = [_tiled_fp8_weight(b) for b in bq]
            for m in ms:
                # N(0,1) activations quantized per token (config 2) or per 1x128 block with
                # step-major scales [K/128, M], as the DSv4 linear path keeps them
                a, asc = quant_act(m, k, dev, mode)
                out = torch.empty((m, n), device=dev, dtype=torch.bfloat16)
                i = [0]

                def launch(st, a=a, asc=asc, out=out, m=m, k=k, n=n, i=i, bq=bq, bs=bs, mode=mode):
                    j = i[0] % len(bq)
                    i[0] += 1
                    if mode == 0:
                        r = L.ti_fp8_gemm_rowcol_tiled(a.data_ptr(), asc.data_ptr(), 1, bq[j].data_ptr(),
                                                       bs[j].data_ptr(), 1, out.data_ptr(), 2, m, n, k,
                                                       ws.data_ptr(), ws.numel() * 4, st)
                    elif mode in (2, 4):
                        fn = L.ti_fp4_gemm_pow2 if mode == 4 else L.ti_fp4_gemm
                        r = fn(a.data_ptr(), asc.data_ptr(), 1, bq[j].data_ptr(), bs[j].data_ptr(), 1,
                               out.data_ptr(), 2, m, n, k, ws.data_ptr(), ws.numel() * 4, st)
                    else:
                        fn = L.ti_fp8_gemm_block_pow2 if mode == 3 else L.ti_fp8_gemm_block
                        r = fn(a.data_ptr(), asc.data_ptr(), 1, bq[j].data_ptr(), bs[j].data_ptr(),
                               out.data_ptr(), 2, m, n, k, ws.data_ptr(), ws.numel() * 4, st)
                    _check("fp8 gemm", r)

                reps = 10 if m >= 4096 else 40
                timed_burst([launch], 3, stream)
                t = timed_burst([launch], reps, stream) / reps * 1e-3
                flops = 2 * m * n * k
                scale_bytes = (n * 4 if mode == 0 else (-(-n // 128)) * (k // 128) * 4 if mode in (1, 3)
                               else n * (k // 32))
                algo = wbytes_n + scale_bytes + m * k + m * n * 2
                bound = "mfma" if flops / algo > FP8_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9) else "hbm"
                label = {0: "config2 fp8 rowcol", 1: "config3 fp8 block", 2: "config3-shape mxfp4",
                         3: "config3-shape fp8 block ue8m0", 4: "config3-shape mxfp4 ue8m0"}[mode]
                recs.append(point_record(f"{label} {sname} M={m} K={k} N={n}", t, algo, flops, bound,
                                         FP8_PEAK_TFLOPS))
                log(recs[-1])
                if mode == 0 and m in (64, 4096):
                    # config 2 as specified: bf16 activations quantized per token inside the
                    # timed region (quant kernel + GEMM), the reference's "incl. dynamic quant"
                    # figure (scripts/bench_fp8_prefill.py:13-17)
                    x = torch.randn((m, k), device=dev).to(torch.bfloat16)

                    def launch_q(st, x=x, a=a, asc=asc, m=m, k=k, launch=launch):
                        _check("fp8 quant", L.ti_fp8_quant_per_token(x.data_ptr(), 2, m, k, 1e-10, a.data_ptr(),
                                                                     asc.data_ptr(), st))
                        launch(st)

                    timed_burst([launch_q], 3, stream)
                    t = timed_burst([launch_q], reps, stream) / reps * 1e-3
                    algo_q = algo + m * k * 2 + m * k + m * 4  # + x read, codes and scales written
                    bound_q = "mfma" if flops / algo_q > FP8_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9) else "hbm"
                    recs.append(point_record(f"{label} incl. per-token quant {sname} M={m} K={k} N={n}", t,
                                             algo_q, flops, bound_q, FP8_PEAK_TFLOPS))
                    log(recs[-1])
                    del x, launch_q
                # Free this point's activations and outputs before the next point, so a
                # large M's buffers do not stay allocated under the later points.
                del a, asc, out, launch
                gc.collect()
                torch.cuda.empty_cache()
            del bq, bs
            torch.cuda.empty_cache()
    return recs


def _tiled_fp8_weight(w):
    """Config 2's weights in the tiled layout the hooks cache (kernels.fp8.tile_weight_fp8,
    prepared at load time, outside every timed region)."""
    import torch
    from torchinferno_amd.kernels import fp8 as tf8
    return tf8.tile_weight_fp8(w.view(torch.float8_e4m3fn))


def fp8_single_point(spec, launches, dev, stream):
    """Launch one config-2 (``rowcol:SHAPE:M``) or config-3 (``block:SHAPE:M``) GEMM
    `launches` times over rotating weight copies: the program a counter run profiles."""
    import torch
    from torchinferno_amd import _lib
    L = _lib.lib()
    mode_name, sname, m = spec.split(":")
    m = int(m)
    mode = {"rowcol": 0, "block": 1}[mode_name]
    k, n = (FP8_SHAPES if mode == 0 else BLOCK_SHAPES)[sname]
    ncopy = max(2, -(-ROTATE_BYTES // (n * k)))
    made = [quant_weight_per_channel(n, k, dev) if mode == 0 else quant_weight_block(n, k, dev)
            for _ in range(ncopy)]
    bq = [q for q, _ in made]
    bs = [sc for _, sc in made]
    del made
    if mode == 0:
        bq = [_tiled_fp8_weight(b) for b in bq]
    a, asc = quant_act(m, k, dev, mode)
    out = torch.empty((m, n), device=dev, dtype=torch.bfloat16)
    ws = torch.zeros(64 << 20, dtype=torch.int32, device=dev)
    for i in range(launches):
        j = i % ncopy
        if mode == 0:
            r = L.ti_fp8_gemm_rowcol_tiled(a.data_ptr(), asc.data_ptr(), 1, bq[j].data_ptr(), bs[j].data_ptr(),
                                           1, out.data_ptr(), 2, m, n, k, ws.data_ptr(), ws.numel() * 4, stream)
        else:
            r = L.ti_fp8_gemm_block(a.data_ptr(), asc.data_ptr(), 1, bq[j].data_ptr(), bs[j].data_ptr(),
                                    out.data_ptr(), 2, m, n, k, ws.data_ptr(), ws.numel() * 4, stream)
        _check("fp8 gemm", r)
    torch.cuda.synchronize()
    print(json.dumps({"point": spec, "launches": launches}), flush=True)


def moe_single_point(t, launches, dev, stream, ue8m0=False):
    """Launch the config-4 routed FP8 MoE (router included) at T tokens `launches`
    times: the program a kernel-trace run profiles.  ``ue8m0``: DeepSeek-V4's scale
    format (power-of-two activation and E8M0 weight scales, applied by the MFMA)."""
    import torch
    from torchinferno_amd import _lib
    L = _lib.lib()
    e, h, inter, k = 256, 7168, 2048, 8
    w13, s13, w2, s2 = fp8_experts(e, h, inter, dev, ue8m0)
    x = torch.randn((t, h), device=dev).to(torch.bfloat16)
    logits = torch.randn((t, e), device=dev)
    wts = torch.empty((t, k), dtype=torch.float32, device=dev)
    ids = torch.empty((t, k), dtype=torch.int32, device=dev)
    out = torch.empty((t, h), dtype=torch.bfloat16, device=dev)
    need = int(L.ti_fp8_moe_workspace_bytes(t, k, e, h, inter))
    ws = torch.empty(need + 256, dtype=torch.uint8, device=dev)
    wsp = (ws.data_ptr() + 255) & ~255
    for _ in range(launches):
        _check("route", L.ti_moe_route_topk(logits.data_ptr(), t, e, k, 1, 1.0, wts.data_ptr(), ids.data_ptr(),
                                            stream))
        _check("moe", L.ti_fp8_moe(x.data_ptr(), wts.data_ptr(), ids.data_ptr(), t, k, w13.data_ptr(),
                                   s13.data_ptr(), w2.data_ptr(), s2.data_ptr(), e, h, inter, 0.0,
                                   2 if ue8m0 else 0, out.data_ptr(), wsp, need, stream))
    torch.cuda.synchronize()
    print(json.dumps({"point": f"moe:{t}" + (":ue8m0" if ue8m0 else ""), "launches": launches}), flush=True)


# --------------------------------------------------------------------------- fused producers


def fused_points(dev, stream):
    """Config 2's activation producers: add+RMSNorm -> FP8 over the hidden size
    (8192) and SwiGLU -> FP8 over the intermediate size (28672, gate/up as split
    views of one [M, 2I] tensor).  HBM-bound: algorithmic bytes are the reads of
    x, residual and the norm weight plus the writes of hidden, codes and scales
    (2+2+2+1 bytes per element), resp. gate + up reads and code writes (2+2+1)."""
    import torch
    from torchinferno_amd import _lib
    L = _lib.lib()
    recs = []
    hsz, isz = 8192, 28672
    for m in (1, 64, 4096):
        x = torch.randn((m, hsz), device=dev).to(torch.bfloat16)
        r = torch.randn_like(x)
        w = torch.rand((hsz,), device=dev).to(torch.bfloat16)
        hid = torch.empty_like(x)
        q = torch.empty((m, hsz), dtype=torch.uint8, device=dev)
        sc = torch.empty((m,), dtype=torch.float32, device=dev)

        def norm(st, x=x, r=r, w=w, hid=hid, q=q, sc=sc, m=m):
            _check("rmsnorm", L.ti_fp8_rmsnorm_quant_per_token(x.data_ptr(), r.data_ptr(), w.data_ptr(), 2, m, hsz,
                                                               1e-5, hid.data_ptr(), q.data_ptr(), sc.data_ptr(), st))

        gu = torch.randn((m, 2 * isz), device=dev).to(torch.bfloat16)
        q2 = torch.empty((m, isz), dtype=torch.uint8, device=dev)
        sc2 = torch.empty((m,), dtype=torch.float32, device=dev)

        def swiglu(st, gu=gu, q2=q2, sc2=sc2, m=m):
            _check("swiglu", L.ti_fp8_swiglu_quant_per_token(gu.data_ptr(), 2 * isz, gu.data_ptr() + isz * 2,
                                                             2 * isz, 2, m, isz, q2.data_ptr(), sc2.data_ptr(), st))

        for label, fn, algo in ((f"config2 add_rmsnorm_fp8 M={m} H={hsz}", norm, m * hsz * 7 + hsz * 2 + m * 4),
                                (f"config2 swiglu_fp8 M={m} I={isz}", swiglu, m * isz * 5 + m * 4)):
            reps = 20 if m >= 4096 else 200
            timed_burst([fn], 5, stream)
            t = timed_burst([fn], reps, stream) / reps * 1e-3
            recs.append(point_record(label, t, algo, 0, "hbm", FP8_PEAK_TFLOPS))
            log(recs[-1])
    return recs


# --------------------------------------------------------------------------- MoE


def fp8_experts(e, h, inter, dev, pow2=False):
    """Config 4's experts: per expert, w1/w3 [I, H] and w2 [H, I] from N(0, 0.02)
    quantized in 128x128 blocks (quant_weight_block), stacked as w13 [E, 2I, H],
    w2 [E, H, I] with their block scales."""
    import torch
    w13 = torch.empty((e, 2 * inter, h), device=dev, dtype=torch.float8_e4m3fn)
    w2 = torch.empty((e, h, inter), device=dev, dtype=torch.float8_e4m3fn)
    s13 = torch.empty((e, 2 * inter // 128, h // 128), device=dev)
    s2 = torch.empty((e, h // 128, inter // 128), device=dev)
    for i in range(e):
        w13[i], s13[i] = quant_weight_block(2 * inter, h, dev, pow2)
        w2[i], s2[i] = quant_weight_block(h, inter, dev, pow2)
    return w13, s13, w2, s2


def moe_points(dev, stream):
    """Config 4: router + routed experts (256 experts, H=7168, I=2048, top-8)."""
    import torch
    from torchinferno_amd import _lib
    from torchinferno_amd.kernels import moe as tmoe
    L = _lib.lib()
    e, h, inter, k = 256, 7168, 2048, 8
    recs = []
    for pow2 in (False, True):
        w13, s13, w2, s2 = fp8_experts(e, h, inter, dev, pow2)
        per_expert = 2 * inter * h + h * inter + (s13[0].numel() + s2[0].numel()) * 4
        if not pow2:
            recs += _moe_sweep(L, dev, "config4 fp8 moe", "ti_fp8_moe", w13, s13, w2, s2, e, h, inter, k,
                               per_expert)
        else:
            # DeepSeek-V4's scale format: ue8m0 activations and E8M0 weight scales, applied by the MFMA
            recs += _moe_sweep(L, dev, "config4-shape fp8 moe ue8m0", "ti_fp8_moe", w13, s13, w2, s2, e, h,
                               inter, k, per_expert, round_scale=2)
        del w13, w2, s13, s2
        torch.cuda.empty_cache()
    torch.cuda.empty_cache()
    # The same routed experts with MXFP4 weights (e2m1 pairs, e8m0 per 32 K).
    w13 = torch.randint(0, 256, (e, 2 * inter, h // 2), device=dev, dtype=torch.uint8)
    w2 = torch.randint(0, 256, (e, h, inter // 2), device=dev, dtype=torch.uint8)
    from torchinferno_amd.kernels.block_fp8 import fp4_scale_stepmajor
    s13 = fp4_scale_stepmajor(torch.randint(118, 124, (e, 2 * inter, h // 32), device=dev, dtype=torch.uint8))
    s2 = fp4_scale_stepmajor(torch.randint(118, 124, (e, h, inter // 32), device=dev, dtype=torch.uint8))
    per_expert = (2 * inter * h + h * inter) // 2 + s13[0].numel() + s2[0].numel()
    recs += _moe_sweep(L, dev, "config4-shape mxfp4 moe", "ti_fp4_moe", w13, s13, w2, s2, e, h, inter, k,
                       per_expert)
    recs += _moe_sweep(L, dev, "config4-shape mxfp4 moe ue8m0", "ti_fp4_moe", w13, s13, w2, s2, e, h, inter, k,
                       per_expert, round_scale=2)
    del w13, w2
    torch.cuda.empty_cache()
    return recs


def _moe_sweep(L, dev, label, entry, w13, s13, w2, s2, e, h, inter, k, per_expert, round_scale=0):
    import torch
    stream = torch.cuda.current_stream(dev).cuda_stream
    fn = getattr(L, entry)
    recs = []
    for t in MOE_TS:
        g = torch.Generator(device=dev).manual_seed(t)
        x = torch.randn((t, h), generator=g, device=dev).to(torch.bfloat16)
        logits = torch.randn((t, e), generator=g, device=dev)
        wts = torch.empty((t, k), dtype=torch.float32, device=dev)
        ids = torch.empty((t, k), dtype=torch.int32, device=dev)
        out = torch.empty((t, h), dtype=torch.bfloat16, device=dev)
        need = int(L.ti_fp8_moe_workspace_bytes(t, k, e, h, inter))
        ws = torch.empty(need + 256, dtype=torch.uint8, device=dev)
        wsp = (ws.data_ptr() + 255) & ~255

        def launch(st, t=t, x=x, logits=logits, wts=wts, ids=ids, out=out, wsp=wsp, need=need):
            _check("route", L.ti_moe_route_topk(logits.data_ptr(), t, e, k, 1, 1.0, wts.data_ptr(), ids.data_ptr(), st))
            lay = (1,) if entry == "ti_fp4_moe" else ()
            _check("moe", fn(x.data_ptr(), wts.data_ptr(), ids.data_ptr(), t, k, w13.data_ptr(),
                             s13.data_ptr(), w2.data_ptr(), s2.data_ptr(), *lay, e, h, inter, 0.0, round_scale,
                             out.data_ptr(), wsp, need, st))

        timed_burst([launch], 2, stream)
        reps = 10
        ms = timed_burst([launch], reps, stream) / reps
        torch.cuda.synchronize()
        touched = int(torch.unique(ids).numel())
        algo = touched * per_expert + t * h * 2 * 2
        flops = t * k * 2 * (2 * inter * h + h * inter)
        recs.append(point_record(f"{label} T={t} experts_touched={touched}", ms * 1e-3, algo, flops, "hbm",
                                 FP8_PEAK_TFLOPS))
        log(recs[-1])
    return recs


# --------------------------------------------------------------------------- main


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", choices=["int4", "fp8", "moe"], default=None,
                    help="run only one family of points (profiling)")
    ap.add_argument("--point", default=None,
                    help="NAME:M -- launch only that config-1 int4 point, --steps times (counter runs); "
                         "rowcol:SHAPE:M / block:SHAPE:M for a config-2 / config-3 FP8 GEMM; "
                         "moe:T[:ue8m0] for the config-4 MoE; "
                         "'copy' for a 256 MiB copy (counter calibration)")
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
    stream = torch.cuda.current_stream(dev).cuda_stream

    if args.point == "copy":
        # counter calibration: a plain 256 MiB device-to-device copy (torch's copy kernel)
        src = torch.ones((64 << 20,), dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"point": "copy", "bytes_read": src.numel() * 4, "launches": args.steps}), flush=True)
        return
    if args.point and args.point.startswith("moe:"):
        f = args.point.split(":")
        moe_single_point(int(f[1]), args.steps, dev, stream, ue8m0=f[2:] == ["ue8m0"])
        return
    if args.point and args.point.count(":") == 2:
        fp8_single_point(args.point, args.steps, dev, stream)
        return
    if args.point:
        name, m = args.point.split(":")
        k, n = SHAPES[name]
        p = Int4Point(name, k, n, int(m), dev, make_int4_copies(k, n, dev))
        for _ in range(args.steps):
            p.launch(stream)
        torch.cuda.synchronize()
        print(json.dumps({"point": args.point, "launches": args.steps, "plan": plan_name(p)}), flush=True)
        return

    extra_points = []
    if args.only in (None, "fp8"):
        extra_points += fp8_points(dev, stream)
        extra_points += fused_points(dev, stream)
    if args.only in (None, "moe"):
        extra_points += moe_points(dev, stream)
    if args.only in ("fp8", "moe"):
        print(json.dumps({"points": extra_points}), flush=True)
        return

    # config 0: fp16 M=16 K=N=4096
    c0 = make_int4_copies(4096, 4096, dev, torch.float16)
    p0 = Int4Point("config0", 4096, 4096, 16, dev, c0, dtype_code=1)
    timed_burst([p0.launch], 20, stream)
    t0 = timed_burst([p0.launch], 200, stream) / 200 * 1e-3
    extra_points.insert(0, point_record("config0 int4 fp16 M=16 K=4096 N=4096", t0, p0.algo_bytes, p0.flops,
                                        p0.bound, BF16_PEAK_TFLOPS))
    del c0, p0

    points = []
    for name, (k, n) in SHAPES.items():
        copies = Rotation(make_int4_copies(k, n, dev))
        log(f"{name}: K={k} N={n} copies={len(copies.copies)}")
        for m in MS:
            points.append(Int4Point(name, k, n, m, dev, copies))

    # Per-point launch durations (each point alone, back-to-back launches).
    per_point = {}
    for p in points:
        timed_burst([p.launch], 20, stream)  # warm
        reps = 200
        per_point[(p.name, p.m)] = timed_burst([p.launch], reps, stream) / reps

    # The timed region: exactly `steps` steps of the full sweep.
    for _ in range(args.warmup):
        for p in points:
            p.launch(stream)
    torch.cuda.synchronize()
    launches = [p.launch for p in points]
    torch.cuda._sleep(int(50e6))
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    t_wall = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        for fn in launches:
            fn(stream)
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall
    gpu_ms = start.elapsed_time(end)
    ms_per_step = gpu_ms / args.steps
    step_bytes = sum(p.wbytes for p in points)
    value = step_bytes / (ms_per_step * 1e-3) / 1e9

    pts = []
    for p in points:
        t = per_point[(p.name, p.m)] * 1e-3
        pts.append(point_record(f"config1 int4 bf16 {p.name} M={p.m} K={p.k} N={p.n}", t, p.algo_bytes, p.flops,
                                p.bound, BF16_PEAK_TFLOPS, {"weight_GBs": round(p.wbytes / t / 1e9, 1)}))
    # Dominant launch of the step: the largest share of its time.
    dom = max(points, key=lambda p: per_point[(p.name, p.m)])
    t_dom = per_point[(dom.name, dom.m)] * 1e-3
    if dom.bound == "hbm":
        achieved, peak, unit = dom.algo_bytes / t_dom / 1e9, HBM_PEAK_GBS, "GB/s"
    else:
        achieved, peak, unit = dom.flops / t_dom / 1e12, BF16_PEAK_TFLOPS, "TFLOP/s"
    dom_label = f"{dom.name}:{dom.m}"
    roofline = {
        "bound": dom.bound, "achieved": round(achieved, 1), "peak": peak, "unit": unit,
        "frac": round(achieved / peak, 4), "traffic": read_traffic(dom_label),
        "kernel": plan_name(dom),
        "launch": f"{dom.name} K={dom.k} N={dom.n} M={dom.m}",
        "avg_launch_us": round(t_dom * 1e6, 2),
        "algo_bytes_per_launch": dom.algo_bytes, "flops_per_launch": dom.flops,
        "share_of_step": round(t_dom * 1e3 / ms_per_step, 3),
    }
    cpu, cpu_points = None, []
    if not args.no_cpu_baseline:
        log("timing CPU baseline ...")
        cpu, cpu_points = cpu_baseline()
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
        "data": ("synthetic (random int4 codes, bf16 scales/activations; FP8 weights and activations quantized "
                 "from N(0, 0.02) / N(0, 1) as configs 2-4 define them; random e2m1 codes for MXFP4; "
                 "no checkpoint)"),
        "config": {"workload": "int4 W4A16 g128 decode sweep (BASELINE configs[1])",
                   "shapes": {k: {"K": v[0], "N": v[1]} for k, v in SHAPES.items()},
                   "M": list(MS), "bytes_per_step": step_bytes, "parallelism": "none (1 GPU)"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "points": pts + extra_points,
        "cpu_points": cpu_points,
        "wall_s": round(wall, 3),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

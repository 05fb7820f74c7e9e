"""Benchmark of the MI355X quantized-KV attention path (one JSON line on stdout).

Headline workload: FP8-E4M3 KV-cache flash-decode, batch 32,
32 query / 8 KV heads, head_dim 128, every sequence at context 8192, bf16 queries and outputs;
cached K/V from bf16 N(0,1) with 1 % of channels x8, per-(token, head) absmax/448 scales.
A step is one decode call (split-K attention + split combine) over the whole batch, with the
cache resident in HBM. Two cache copies (554 MB each, both larger than the 256 MB MALL) are
used alternately so every call streams from HBM.

value = algorithmic HBM bytes per call (codes + scales + q + out) / measured seconds per call.
roofline.achieved = the same bytes / the decode kernel's average duration, timed with HIP events
on the stream the library launches on (torch's current stream). cpu_baseline = the oracle's
restatement of the reference CPU path (dequantize -> bf16 -> f32 unfused attention), timed on the
host on a bounded sample of the same workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--extra]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2516.6


def load_cqkv():
    import importlib.util
    spec = importlib.util.spec_from_file_location(
        "cqkv", os.path.join(ROOT, "candle-rocm-vulkan_amd", "cqkv.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["cqkv"] = mod
    spec.loader.exec_module(mod)
    return mod


def kv_gpu(shape, seed, dev, outliers=True):
    import torch
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(*shape, generator=g, device=dev)
    if outliers:
        mask = torch.rand(shape[1], shape[3], generator=g, device=dev) < 0.01
        x = torch.where(mask[None, :, None, :], x * 8.0, x)
    return x.to(torch.bfloat16)


def build_cache(cq, fmt, b, hkv, d, ctx, dev, seed):
    cache = cq.TurboKvCache(fmt, fmt, b, hkv, d, ctx, device=dev)
    chunk = max(1, 2048 // 1)
    for t0 in range(0, ctx, chunk):
        t = min(chunk, ctx - t0)
        cache.append(kv_gpu((b, hkv, t, d), seed + t0, dev), kv_gpu((b, hkv, t, d), seed + 7 + t0, dev))
    return cache


def time_calls(fn, steps, warmup, stream):
    import torch
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(steps):
        fn(i)
    stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps  # ms per call


def decode_bytes(b, hq, hkv, d, ctx, fmt):
    per_row = {5: d + 4, 2: d // 2 + d // 32, 0: d // 2 + 4}[fmt]
    return 2 * b * hkv * ctx * per_row + 2 * b * hq * d * 2


def cpu_baseline_decode(cq, cache, q, b_sample, ctx, scale, threads):
    """Oracle CPU path on the first b_sample sequences; returns seconds per full call."""
    import numpy as np
    from oracle import oracle as O
    b = q.shape[0]
    kr = cq.rows_export(cache.k, ctx).cpu().numpy().view(np.uint32)[:b_sample]
    vr = cq.rows_export(cache.v, ctx).cpu().numpy().view(np.uint32)[:b_sample]
    qb = O.f32_to_bf16_bits(q[:b_sample].float().cpu().numpy())
    reps, t_total = 0, 0.0
    while t_total < 10.0 and reps < 20:
        t0 = time.perf_counter()
        O.cache_attention(qb, kr, vr, (O.FP8, 0), (O.FP8, 0), None, None, ctx, scale,
                          threads=threads)
        t_total += time.perf_counter() - t0
        reps += 1
    return t_total / reps * (b / b_sample), reps


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--splits", type=int, default=0)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the path shards by batch / kv head with no exchange, see DESIGN.md", file=sys.stderr)
        sys.exit(2)

    import torch
    cq = load_cqkv()
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)

    B, HQ, HKV, D, CTX = 32, 32, 8, 128, 8192
    scale = 1.0 / D ** 0.5
    caches = [build_cache(cq, cq.FP8, B, HKV, D, CTX, dev, 1000 * i) for i in range(2)]
    q = kv_gpu((B, HQ, 1, D), 5, dev, outliers=False)
    out = torch.empty_like(q)
    splits = args.splits or cq.decode_splits(B, HKV, CTX)
    ws = torch.zeros(cq.decode_workspace_bytes(B, HQ, 1, D, splits), dtype=torch.uint8, device=dev)

    def step(i):
        c = caches[i & 1]
        cq.decode_attention(q, c.k, c.v, CTX, scale, out=out, splits=splits, workspace=ws)

    ms = time_calls(step, args.steps, args.warmup, stream)
    nbytes = decode_bytes(B, HQ, HKV, D, CTX, cq.FP8)
    achieved = nbytes / (ms * 1e-3) / 1e9  # GB/s
    cores = min(16, os.cpu_count() or 1)
    cpu = None
    if not args.no_cpu:
        sec, reps = cpu_baseline_decode(cq, caches[0], q, 2, CTX, scale, cores)
        cpu = {"value": round(nbytes / sec / 1e12, 6), "unit": "TB/s", "cores": cores,
               "kind": "port", "us_per_call": round(sec * 1e6, 1),
               "sample": f"oracle cache_attention (reference CPU path restated in C) on 2 of the "
                         f"32 sequences, {reps} reps, scaled x16 to the full call"}
    res = {
        "metric": "quant-KV flash-decode µs/call + achieved HBM TB/s; bf16 prefill TFLOP/s",
        "value": round(achieved / 1000.0, 4),
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "us_per_call": round(ms * 1e3, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8-e4m3 cache, bf16 q/out, f32 accumulate",
        "data": "synthetic (torch N(0,1) bf16, 1% channels x8)",
        "config": {"workload": "BASELINE config 2: FP8-KV GQA flash-decode", "batch": B,
                   "q_heads": HQ, "kv_heads": HKV, "head_dim": D, "context": CTX,
                   "splits": splits, "cache_copies": 2, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": None, "bytes_per_call": nbytes,
                     "timed": "whole call (decode + combine kernels)"},
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()

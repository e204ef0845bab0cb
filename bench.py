#!/usr/bin/env python3
"""Benchmark of the IRON decode operator path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Headline (``value``): BASELINE configs[1], the fused int4-g32 dequant+GEMV at
batch 1 (W 8192x2048, gate_proj shape), as HBM GB/s of algorithmic bytes.
A step is one launch over one weight copy; the copies rotate through a pool
of >= 512 MiB so the 256 MiB Infinity Cache cannot hold the working set and
every step streams its weights from HBM. Inputs are resident in HBM before
the timed region.

``roofline`` is measured on the kernel's own stream with HIP events, one
start/stop pair per launch, averaged; ``cpu_baseline`` times the CPU oracle
(torch, dequantize then matvec) on the host cores on a bounded sample.
Extra figures for the other BASELINE configurations go under ``extra``.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0  # dense bf16 MFMA
POOL_BYTES = 640 << 20  # rotate through > 512 MiB of distinct weights

METRIC = "GEMV HBM GB/s (% of peak); Llama-3.2-1B decode tok/s, 1 MI355X"


def _events(torch, n):
    return [torch.cuda.Event(enable_timing=True) for _ in range(n)]


def time_steps(torch, launch, steps, warmup):
    """Warm up, then time exactly ``steps`` launches bracketed by synchronize.

    Returns (wall_ms_total, mean_kernel_us) where the kernel time comes from a
    start/stop event pair around each launch on the launch stream.
    """
    for i in range(warmup):
        launch(i)
    torch.cuda.synchronize()
    starts, stops = _events(torch, steps), _events(torch, steps)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        starts[i].record()
        launch(warmup + i)
        stops[i].record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    per = sorted(s.elapsed_time(e) * 1e3 for s, e in zip(starts, stops))
    # mean of the central 80% (drops the first-touch and preemption outliers)
    lo, hi = len(per) // 10, len(per) - len(per) // 10
    core = per[lo:hi] or per
    return wall_ms, sum(core) / len(core)


def time_back_to_back(torch, launch, n):
    """Events around ``n`` back-to-back launches: per-launch time incl. gaps (us)."""
    e0, e1 = _events(torch, 2)
    torch.cuda.synchronize()
    e0.record()
    for i in range(n):
        launch(i)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / n


def bench_gemv_int4(torch, dev, steps, warmup):
    from iron_amd import _lib
    from oracle import configs

    M, K = 8192, 2048
    codes, scales, x = configs.cfg2_gemv_int4(M=M, K=K)
    nbytes = M * K // 2 + 2 * M * K // 32 + 2 * K + 2 * M  # 9,457,664 B algorithmic
    copies = max(2, POOL_BYTES // (codes.numel() + 2 * scales.numel()))
    C = [codes.to(dev) for _ in range(copies)]
    S = [scales.to(dev) for _ in range(copies)]
    xd = x.to(dev)
    y = torch.empty(M, dtype=torch.bfloat16, device=dev)
    stream = _lib.stream_handle(dev)
    lib = _lib.load()
    fn = lib.iron_gemv_i4g32

    def launch(i):
        rc = fn(C[i % copies].data_ptr(), S[i % copies].data_ptr(), xd.data_ptr(), y.data_ptr(), M, K, 1, stream)
        if rc:
            raise RuntimeError(lib.iron_last_error().decode())

    wall_ms, kern_us = time_steps(torch, launch, steps, warmup)
    b2b_us = time_back_to_back(torch, launch, 200)
    return {
        "bytes": nbytes,
        "wall_ms": wall_ms,
        "kernel_us": kern_us,
        "b2b_us": b2b_us,
        "pool_copies": copies,
        "inputs": (codes, scales, x),
    }


def bench_gemv_bf16(torch, dev, steps, warmup):
    from iron_amd import _lib
    from oracle import configs

    M, K = 2048, 8192
    W, x = configs.cfg1_gemv_bf16(M=M, K=K)
    nbytes = 2 * M * K + 2 * K + 2 * M  # 33,574,912 B
    copies = max(2, POOL_BYTES // (2 * W.numel()))
    Ws = [W.to(dev) for _ in range(copies)]
    xd = x.to(dev)
    y = torch.empty(M, dtype=torch.bfloat16, device=dev)
    stream = _lib.stream_handle(dev)
    lib = _lib.load()
    fn = lib.iron_gemv_bf16

    def launch(i):
        rc = fn(Ws[i % copies].data_ptr(), xd.data_ptr(), y.data_ptr(), M, K, 1, 0, stream)
        if rc:
            raise RuntimeError(lib.iron_last_error().decode())

    wall_ms, kern_us = time_steps(torch, launch, steps, warmup)
    b2b_us = time_back_to_back(torch, launch, 200)
    del Ws
    return {"bytes": nbytes, "wall_ms": wall_ms, "kernel_us": kern_us, "b2b_us": b2b_us}


def cpu_baseline_int4(torch, inputs, budget_s=10.0):
    """Oracle on the host cores: dequantize with torch ops, then matvec."""
    from oracle import ops

    codes, scales, x = inputs
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    nbytes = codes.numel() + 2 * scales.numel() + 2 * x.numel() + 2 * codes.shape[0]
    ops.gemv_int4_reference(codes, scales, x)  # warm
    reps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        ops.gemv_int4_reference(codes, scales, x)
        reps += 1
    dt = time.perf_counter() - t0
    return {
        "value": round(nbytes * reps / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{reps} x config-2 int4 GEMV (8192x2048) via oracle.ops.gemv_int4_reference "
        f"(torch CPU dequant + fp32 matvec), {dt:.1f} s",
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    args = ap.parse_args()

    if args.gpus != 1:
        print(
            "bench.py measures one MI355X: the IRON operator path is single-device "
            "(multi-GPU sharding is a design note, not a run). Use --gpus 1.",
            file=sys.stderr,
        )
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda", 0)

    i4 = bench_gemv_int4(torch, dev, args.steps, args.warmup)
    bf = bench_gemv_bf16(torch, dev, max(200, args.steps // 4), args.warmup)

    value = i4["bytes"] * args.steps / (i4["wall_ms"] * 1e-3) / 1e9
    achieved = i4["bytes"] / (i4["kernel_us"] * 1e-6) / 1e9
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(i4["wall_ms"] / args.steps, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "BASELINE configs[1]: fused int4-g32 dequant+GEMV, batch 1, W 8192x2048 "
            "(signed int4, bf16 group-32 scales), x 2048 bf16, fp32 accumulate, bf16 out",
            "weight_pool_copies": i4["pool_copies"],
            "algorithmic_bytes_per_step": i4["bytes"],
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel": "gemv_i4_kernel",
            "kernel_us": round(i4["kernel_us"], 3),
        },
        "extra": {
            "gemv_bf16_cfg1": {
                "kernel_us": round(bf["kernel_us"], 3),
                "GB/s": round(bf["bytes"] / (bf["kernel_us"] * 1e-6) / 1e9, 1),
                "frac_hbm": round(bf["bytes"] / (bf["kernel_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                "back_to_back_us_per_launch": round(bf["b2b_us"], 3),
            },
            "gemv_int4_cfg2_back_to_back_us_per_launch": round(i4["b2b_us"], 3),
        },
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline_int4(torch, i4["inputs"], args.cpu_seconds)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

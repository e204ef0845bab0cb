#!/usr/bin/env python3
"""Benchmark of the IRON decode/prefill operator path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
                    [--mode full|gemv|gemv_bf16|sustained|model|prefill|gemm_large|gemm_512|attention|floor|mfma|swiglu|trace]

--mode gemv runs only the headline kernel (plus three 64 MiB device copies
that calibrate rocprofv3's FETCH_SIZE / WRITE_SIZE counters); --mode model
runs only the Llama configuration; --mode sustained the two GEMV kernels over
tall matrices (the streaming rate without the per-launch cost); --mode prefill only the config 5 prefill
GEMM and the 3968-token causal attention; --mode gemm_large the 3968-token
prefill projections and 4096^3 beside hipBLASLt; --mode gemm_512 the plain
(no K split) 512-token projections beside hipBLASLt; --mode attention the GQA decode
attention at config 3 and at KV 4096; --mode floor the per-launch floors (an
empty kernel as a graph node, a pure streaming read of the decode kernels'
sizes); --mode swiglu config 4's block (bf16, int4 in two launches, int4 in one
launch); --mode trace per-workgroup phase traces (iron_trace_next_launch) of the
decode attention, the headline int4 GEMV and the one-launch SwiGLU block, with
Perfetto JSON in TRACE_DIR. The modes exist for kernel traces and counters.

Headline (``value``): BASELINE configs[1], the fused int4-g32 dequant+GEMV at
batch 1 (W 8192x2048, gate_proj shape), as HBM GB/s of algorithmic bytes
(9,457,664 B per step). A step is one launch over one weight copy. Inputs are
resident in HBM before the timed region.

Cache-proof rotation (every GPU figure): copies of a kernel's working set fill
a pool of >= 640 MiB, launch i reads copy i % copies, and a copy is read again
only after every other copy has been (>= 640 MiB read since), so the 256 MiB
Infinity Cache cannot serve a timed launch at any step count. Launches are
issued from captured hipGraphs -- the way the decode step issues its kernels
-- so the host's per-launch cost (about 3 us in the HIP runtime plus the
Python call) does not bound the rate; ``python_launch_us`` reports the same
kernel launched one call at a time from Python.

Headline timing: one graph holds a lead of one launch per copy, then the K
timed launches; its replay time minus the replay time of the lead alone is
the device time of exactly the K launches (HIP events on the launch stream;
each replay is queued behind an untimed replay of the lead, so the host's
graph-launch latency stays out). The difference cancels the fixed cost a
graph replay carries at its start and end, so the per-launch time does not
depend on K. Other configs: a graph of a multiple of `copies` launches (>= a
few hundred), replayed untimed then timed; per-launch time = timed replay / n,
median of 5.

``roofline``: algorithmic bytes / the headline kernel's average duration in
rocprofv3's kernel trace of this command (profiles/gemv_i4g32_cfg2_kernel_trace.md,
read at run time; each traced dispatch carries its own completion signal, so
that duration is longer than the untraced per-launch time of ``value``, which
the line also carries as ``kernel_us_live`` / ``frac_live``). ``traffic``: HBM
bytes per launch from rocprofv3 FETCH_SIZE + WRITE_SIZE of the same command,
each scaled by the counter's reading for a copy of known size
(profiles/gemv_i4g32_cfg2_pmc.md, read at run time).
``cpu_baseline``: the CPU oracle (torch: dequantise, then fp32 matvec) timed
on the host cores on a bounded sample; ``cpu_baseline.model_decode`` and
``extra.llama_cfg5.cpu_baseline`` time the oracle's fp32 Llama forward
(Llama-3.2-1B shape) at config 5's windows: the 512-token prefill, decode
after it, and decode at KV 3968 on. Each config in ``extra`` carries its own
``cpu_baseline`` in the GPU figure's unit, with the core count.
``extra`` carries the other BASELINE configurations: bf16 GEMV (cfg 1), GQA
decode (cfg 3, and at KV 4096), SwiGLU block bf16 and int4 (cfg 4), the
prefill GEMM with cold weights and the Llama-3.2-1B-shaped model (cfg 5:
prefill 512 tokens, 128 greedy decode steps; plus the KV 3968 -> 4096
window). Its ``ttft_ms`` replays the prefill graph captured beforehand for
the prompt length (``ttft_eager_ms``: the same prefill issued kernel by
kernel); the token ids are copied from the host inside both timings. Every
config also prints the reference's ``Latency (us):`` / ``Effective
Bandwidth:`` lines on stderr.
"""

from __future__ import annotations

import argparse
import json
import math
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

# The headline kernel's rocprofv3 evidence, committed under profiles/ and read
# at run time (each file carries one `bench.py reads: <key> <value>` line):
# the kernel-trace average duration of the headline command's dispatches,
# and the HBM bytes per launch from its FETCH_SIZE + WRITE_SIZE passes (each
# scaled by the counter's reading for a copy of known size).
TRACE_PROFILE = "profiles/gemv_i4g32_cfg2_kernel_trace.md"
# where --mode trace writes its Perfetto JSON: the results folder that a remote run returns
TRACE_DIR = os.path.join("gpurun_out", "traces")
PMC_PROFILE = "profiles/gemv_i4g32_cfg2_pmc.md"


def profile_value(rel_path: str, key: str):
    """The number on the `bench.py reads: <key> <value>` line of a committed
    profile summary, or None when the file or the line is missing."""
    import re

    try:
        text = (ROOT / rel_path).read_text()
    except OSError:
        return None
    m = re.search(r"bench\.py reads: " + re.escape(key) + r" ([0-9.]+)", text)
    return float(m.group(1)) if m else None


def copies_for(nbytes: int) -> int:
    """Distinct copies of an nbytes working set that fill the rotation pool."""
    return max(2, -(-POOL_BYTES // nbytes))


class Timer:
    """Device time of launch closures launch(i, stream), where launch i reads copy
    i % copies of its inputs.

    Cache-proof protocol: a launch never re-reads a copy until every other copy
    (>= POOL_BYTES of distinct data in all) has been read since, so the 256 MiB
    Infinity Cache cannot serve the timed launches at any step count. Graphs
    hold a multiple of `copies` consecutive launches (each replay reads every
    copy once, in order), and a warm replay of the full rotation precedes every
    timed region.
    """

    def __init__(self, torch, lib):
        self.torch, self.lib = torch, lib

    def capture(self, launch, n, offset=0):
        """hipGraph of launch(offset), ..., launch(offset + n - 1) on the capturing stream."""
        from iron_amd import _lib
        from iron_amd.common.graph import capture_graph

        dev = self.torch.device("cuda", 0)

        def body():
            s = _lib.stream_handle(dev)
            for i in range(n):
                launch(offset + i, s)

        return capture_graph(body, dev)

    def replay_ms(self, graphs, lead=None):
        """Events (on the replay stream) around back-to-back replays of `graphs`, in
        order (milliseconds). `lead`, replayed first and untimed, keeps the GPU
        busy while the host submits the timed graphs, so the start event is
        recorded when the lead ends, with the timed graphs already queued: the
        host's graph-launch latency stays out of the timed region."""
        torch = self.torch
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        if lead is not None:
            lead.replay()
        a.record()
        for g in graphs:
            g.replay()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b)

    def rotating_us(self, launch, copies, min_launches=200, rounds=5):
        """Device time per launch (microseconds): a graph of n consecutive launches,
        n the smallest multiple of `copies` >= min_launches; each round replays it
        once untimed (the lead) and once timed; the median over `rounds`."""
        n = copies * max(1, -(-min_launches // copies))
        g = self.capture(launch, n)
        g.replay()
        t = sorted(self.replay_ms([g], lead=g) * 1e3 / n for _ in range(rounds))
        del g
        return t[len(t) // 2]

    def wall_ms(self, launch, n, offset=0):
        """Events around n back-to-back launch(i, stream) calls issued one at a time (milliseconds)."""
        from iron_amd import _lib

        torch = self.torch
        s = _lib.stream_handle(torch.device("cuda", 0))
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record()
        for i in range(n):
            launch(offset + i, s)
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b)


def metric_lines(name, latency_us, nbytes):
    """The per-operator lines the reference's operator tests print and its CI
    scrapes (iron/common/test_utils.py:293-294), on stderr so that stdout
    stays the one JSON line."""
    print(f"[{name}]\nLatency (us): {latency_us:.1f}\nEffective Bandwidth: {nbytes / (latency_us * 1e-6) / 1e9:.6e} GB/s",
          file=sys.stderr, flush=True)


def cpu_time(fn, budget_s):
    """fn() timed on the host: one warm call, then repeated calls until budget_s
    is spent (at least one). Returns (calls, seconds)."""
    fn()
    reps, t0 = 0, time.perf_counter()
    while reps == 0 or time.perf_counter() - t0 < budget_s:
        fn()
        reps += 1
    return reps, time.perf_counter() - t0


def cpu_threads(torch) -> int:
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    return threads


def _check(lib, rc):
    if rc:
        raise RuntimeError(lib.iron_last_error().decode())


def bench_gemv_int4(torch, lib, tm, dev, steps, warmup, rounds=5):
    """The headline: `steps` launches of the config 2 GEMV, timed on the GPU
    without any graph boundary inside the measurement.

    Two graphs are captured: `lead`, one launch per weight copy (every copy
    once, in rotation order), and `full`, the same lead followed by the
    `steps` timed launches, which continue the rotation (so every timed
    launch reads a copy that `copies - 1` other launches, >= POOL_BYTES, have
    read past since its last use). Each is replayed behind an untimed replay
    of `lead` that keeps the GPU busy while the host queues it, and the timed
    region is the difference of the two replay times: the device time of
    exactly the `steps` launches. A graph replay carries a fixed cost of
    several microseconds at its start and end; the difference cancels it, so
    the per-launch time does not depend on `steps`. Median over `rounds`."""
    from iron_amd import _lib
    from iron_amd.common.graph import capture_graph
    from oracle import configs

    M, K = 8192, 2048
    codes, scales, x = configs.cfg2_gemv_int4(M=M, K=K)
    nbytes = M * K // 2 + 2 * M * K // 32 + 2 * K + 2 * M
    copies = copies_for(codes.numel() + 2 * scales.numel())
    C = [codes.to(dev) for _ in range(copies)]
    S = [scales.to(dev) for _ in range(copies)]
    xd = x.to(dev)
    y = torch.empty(M, dtype=torch.bfloat16, device=dev)
    stream = _lib.stream_handle(dev)
    Cp = [c.data_ptr() for c in C]
    Sp = [t.data_ptr() for t in S]
    xp, yp = xd.data_ptr(), y.data_ptr()

    def launch(i, s):
        _check(lib, lib.iron_gemv_i4g32(Cp[i % copies], Sp[i % copies], xp, yp, M, K, 1, s))

    for i in range(warmup):
        launch(i, stream)
    lead = tm.capture(launch, copies)
    full = tm.capture(launch, copies + steps)
    full.replay()
    t_lead = sorted(tm.replay_ms([lead], lead=lead) for _ in range(rounds))[rounds // 2]
    t_full = sorted(tm.replay_ms([full], lead=lead) for _ in range(rounds))[rounds // 2]
    wall = t_full - t_lead
    del lead, full
    # the same kernel issued one Python call at a time (host-bound when the kernel is short)
    n_py = min(steps, 1000)
    py_us = tm.wall_ms(launch, n_py) * 1e3 / n_py
    return {"bytes": nbytes, "wall_ms": wall, "copies": copies, "python_launch_us": py_us,
            "lead_ms": t_lead, "full_ms": t_full,
            "timed_distinct_bytes": min(steps, copies) * (codes.numel() + 2 * scales.numel()),
            "inputs": (codes, scales, x)}


def _gpu_line(name, kern_us, nbytes=None, flops=None, cpu=None):
    """One config's GPU figure (HBM GB/s or MFMA TFLOP/s) with its CPU baseline beside it."""
    out = {"kernel_us": round(kern_us, 3)}
    if nbytes is not None:
        out.update({"GB/s": round(nbytes / kern_us / 1e3, 1), "frac_hbm": round(nbytes / kern_us / 1e3 / HBM_PEAK_GBS, 4),
                    "algorithmic_bytes": nbytes})
        metric_lines(name, kern_us, nbytes)
    if flops is not None:
        tf = flops / kern_us / 1e6
        out.update({"TFLOP/s": round(tf, 1), "frac_mfma": round(tf / BF16_PEAK_TFLOPS, 4), "flops": int(flops)})
    if cpu is not None:
        out["cpu_baseline"] = cpu
    return out


def _cpu_line(torch, fn, budget_s, unit_work, unit, what):
    """CPU baseline of one config: fn() on the host cores for ~budget_s seconds;
    value = unit_work per call x calls / seconds (unit_work in GB or TFLOP)."""
    if budget_s <= 0:
        return None
    threads = cpu_threads(torch)
    reps, dt = cpu_time(fn, budget_s)
    return {"value": round(unit_work * reps / dt, 4), "unit": unit, "cores": threads, "kind": "port",
            "sample": f"{reps} x {what}, {dt:.1f} s"}


def bench_gemv_bf16(torch, lib, tm, dev, n, cpu_s=0.0):
    from iron_amd import _lib
    from oracle import configs, ops

    M, K = 2048, 8192
    W, x = configs.cfg1_gemv_bf16(M=M, K=K)
    nbytes = 2 * M * K + 2 * K + 2 * M
    copies = copies_for(2 * W.numel())
    Ws = [W.to(dev) for _ in range(copies)]
    xd = x.to(dev)
    y = torch.empty(M, dtype=torch.bfloat16, device=dev)
    stream = _lib.stream_handle(dev)

    def launch(i, s):
        _check(lib, lib.iron_gemv_bf16(Ws[i % copies].data_ptr(), xd.data_ptr(), y.data_ptr(), M, K, 1, 0, s))

    for i in range(20):
        launch(i, stream)
    kern = tm.rotating_us(launch, copies, n)
    b2b = tm.wall_ms(launch, n) * 1e3 / n
    cpu = _cpu_line(torch, lambda: ops.gemv_reference(W, x), cpu_s, nbytes / 1e9, "GB/s",
                    "config-1 bf16 GEMV (2048x8192) via oracle.ops.gemv_reference (torch CPU, fp32 matvec)")
    out = _gpu_line("gemv_bf16_cfg1", kern, nbytes=nbytes, cpu=cpu)
    out["python_launch_us"] = round(b2b, 3)
    out["weight_copies"] = copies
    return out


def bench_gemv_sustained(torch, lib, tm, dev, cpu_s=0.0):
    """The two GEMV kernels over tall matrices (K 2048, random codes / weights,
    one launch per call, rotated copies): the rate once the fixed per-launch
    cost (~2 us, profiles/floors_launch_read_mfma.md) is small beside the bytes,
    and the incremental rate between the two sizes, (bytes2 - bytes1) /
    (t2 - t1), which cancels it. The north_star's "sustain >= 75% of HBM
    peak" read as streaming over many rows, beside the batch-1 configs."""
    from iron_amd import _lib
    from oracle import configs, ops

    K = 2048
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(K, device=dev, generator=g).to(torch.bfloat16)
    out = {}
    for fmt, sizes in (("int4_g32", (131072, 262144)), ("bf16", (65536, 131072))):
        pts = []
        for M in sizes:
            if fmt == "int4_g32":
                nbytes = M * K // 2 + M * (K // 32) * 2 + 2 * K + 2 * M
                copies = copies_for(nbytes)
                ws = [(torch.randint(0, 256, (M, K // 2), dtype=torch.uint8, device=dev, generator=g),
                       (torch.rand(M, K // 32, device=dev, generator=g) * 0.009 + 0.001).to(torch.bfloat16))
                      for _ in range(copies)]
            else:
                nbytes = 2 * M * K + 2 * K + 2 * M
                copies = copies_for(nbytes)
                ws = [(torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16), None) for _ in range(copies)]
            y = torch.empty(M, dtype=torch.bfloat16, device=dev)

            def launch(i, s, ws=ws, y=y, M=M):
                w, sc = ws[i % len(ws)]
                if sc is not None:
                    _check(lib, lib.iron_gemv_i4g32(w.data_ptr(), sc.data_ptr(), x.data_ptr(), y.data_ptr(), M, K, 1, s))
                else:
                    _check(lib, lib.iron_gemv_bf16(w.data_ptr(), x.data_ptr(), y.data_ptr(), M, K, 1, 0, s))

            stream = _lib.stream_handle(dev)
            for i in range(copies):
                launch(i, stream)
            kern = tm.rotating_us(launch, copies, 4 * copies)
            pts.append((M, nbytes, kern, copies))
            del ws, y
            torch.cuda.empty_cache()
        line = {f"M{M}": {"kernel_us": round(t, 3), "algorithmic_bytes": b, "GB/s": round(b / t / 1e3, 1),
                          "frac_hbm": round(b / t / 1e3 / HBM_PEAK_GBS, 4), "weight_copies": c}
                for M, b, t, c in pts}
        (_, b1, t1, _), (_, b2, t2, _) = pts
        inc = (b2 - b1) / (t2 - t1) / 1e3
        line["incremental_GB/s"] = round(inc, 1)
        line["incremental_frac_hbm"] = round(inc / HBM_PEAK_GBS, 4)
        out[fmt] = line
    # CPU baseline: the same oracle GEMVs at the configs' sizes (their host rate does not depend on M)
    if cpu_s > 0:
        W1, x1 = configs.cfg1_gemv_bf16(M=2048, K=8192)
        codes, scales, x2 = configs.cfg2_gemv_int4()
        out["bf16"]["cpu_baseline"] = _cpu_line(
            torch, lambda: ops.gemv_reference(W1, x1), cpu_s, (2 * W1.numel() + 2 * 8192 + 2 * 2048) / 1e9, "GB/s",
            "config-1 bf16 GEMV via oracle.ops.gemv_reference (torch CPU, fp32 matvec)")
        nb2 = codes.numel() + 2 * scales.numel() + 2 * x2.numel() + 2 * codes.shape[0]
        out["int4_g32"]["cpu_baseline"] = _cpu_line(
            torch, lambda: ops.gemv_int4_reference(codes, scales, x2), cpu_s, nb2 / 1e9, "GB/s",
            "config-2 int4 GEMV via oracle.ops.gemv_int4_reference (torch CPU: dequantise, fp32 matvec)")
    return out


def bench_gqa(torch, lib, tm, dev, n, L=2048, max_len=None, cpu_s=0.0):
    """GQA decode attention (32/8 heads, d 64) with the new token at position
    L-1 of a cache of capacity max_len (config 3: L = max_len = 2048)."""
    from iron_amd import _lib
    from oracle import configs, ops

    H, Hkv, D = 32, 8, 64
    max_len = max_len or L
    q, kn, vn, kc, vc, pos, angles = configs.cfg3_gqa_decode(n_heads=H, n_kv=Hkv, head_dim=D, L=L)
    if max_len > L:
        pad = torch.zeros(Hkv, max_len - L, D, dtype=kc.dtype)
        kc, vc = torch.cat([kc, pad], 1), torch.cat([vc, pad], 1)
        angles = ops.rope_angles_table(D, max_len, theta=500000.0)
    nbytes = 2 * Hkv * L * D * 2 + H * D * 2 * 2 + 2 * Hkv * D * 2 + D * 4
    copies = copies_for(2 * Hkv * L * D * 2)
    KC = [kc.to(dev) for _ in range(copies)]
    VC = [vc.to(dev) for _ in range(copies)]
    qd, knd, vnd, ad = q.to(dev), kn.to(dev), vn.to(dev), angles.to(dev)
    out = torch.empty(H, D, dtype=torch.bfloat16, device=dev)
    ws = torch.zeros(int(lib.iron_gqa_decode_workspace_bytes(H, Hkv, D, max_len)), dtype=torch.uint8, device=dev)
    stream = _lib.stream_handle(dev)

    # the model's call: counters kept at zero by the caller (IRON_GQA_COUNTERS_ZERO), so the timed launch is
    # the attention kernel alone; streaming K/V loads (caches cold, rotated)
    def launch(i, s):
        _check(lib, lib.iron_gqa_decode_ex(qd.data_ptr(), knd.data_ptr(), vnd.data_ptr(), KC[i % copies].data_ptr(),
                                           VC[i % copies].data_ptr(), ad.data_ptr(), angles.shape[0], out.data_ptr(),
                                           ws.data_ptr(), H, Hkv, D, max_len, pos, None, 1.0 / math.sqrt(D), 2, s))

    for i in range(20):
        launch(i, stream)
    kern = tm.rotating_us(launch, copies, n)
    cpu = None
    if cpu_s > 0:
        cpu = _cpu_line(torch, lambda: ops.gqa_decode_reference(q, kn, vn, kc, vc, pos, angles, scale=1.0 / math.sqrt(D)),
                        cpu_s, nbytes / 1e9, "GB/s",
                        f"GQA decode at KV {L} via oracle.ops.gqa_decode_reference (torch CPU, fp32 softmax attention)")
    res = _gpu_line(f"gqa_decode_L{L}", kern, nbytes=nbytes, cpu=cpu)
    res.update({"kv_len": L, "max_len": max_len, "cache_copies": copies})
    return res


def bench_swiglu(torch, lib, tm, dev, n, cpu_s=0.0):
    """Config 4: x + Wd(silu(Wg xn) * (Wu xn)), xn = RMSNorm(x)*w: two kernels
    (norm + gate/up pair GEMV, then down GEMV + residual)."""
    from iron_amd import _lib
    from oracle import configs, ops

    E, F = 2048, 8192
    x, nw, Wg, Wu, Wd = configs.cfg4_swiglu_block(E, F)
    stream = _lib.stream_handle(dev)
    xd, nwd = x.to(dev), nw.to(dev)
    h = torch.empty(F, dtype=torch.bfloat16, device=dev)
    y = torch.empty(E, dtype=torch.bfloat16, device=dev)
    res = {}
    # bf16
    g_, u_, d_ = Wg.to(dev), Wu.to(dev), Wd.to(dev)
    reps = copies_for(3 * 2 * E * F)
    G = [g_] + [g_.clone() for _ in range(reps - 1)]
    U = [u_] + [u_.clone() for _ in range(reps - 1)]
    Dn = [d_] + [d_.clone() for _ in range(reps - 1)]

    def block(i, s):
        _check(lib, lib.iron_gemv_bf16_fused(G[i % reps].data_ptr(), U[i % reps].data_ptr(), xd.data_ptr(),
                                             h.data_ptr(), F, E, 1, nwd.data_ptr(), 1e-5, None, 0, None, s))
        _check(lib, lib.iron_gemv_bf16_fused(Dn[i % reps].data_ptr(), None, h.data_ptr(), y.data_ptr(), E, F, 0,
                                             None, 0.0, xd.data_ptr(), 0, None, s))

    for i in range(10):
        block(i, stream)
    t = tm.rotating_us(block, reps, n)
    nbytes = 3 * 2 * E * F + 4 * E + 2 * 2 * F + 2 * E * 2
    cpu = _cpu_line(torch, lambda: ops.swiglu_block_reference(x, nw, Wg, Wu, Wd), cpu_s, nbytes / 1e9, "GB/s",
                    "config-4 bf16 SwiGLU block via oracle.ops.swiglu_block_reference (torch CPU)")
    res["bf16"] = _gpu_line("swiglu_block_bf16_cfg4", t, nbytes=nbytes, cpu=cpu)
    del G, U, Dn
    # int4-g32
    q = {}
    for name, W in (("g", Wg), ("u", Wu), ("d", Wd)):
        Wdv = W.to(dev)
        c = torch.empty(W.shape[0], W.shape[1] // 2, dtype=torch.uint8, device=dev)
        s = torch.empty(W.shape[0], W.shape[1] // 32, dtype=torch.bfloat16, device=dev)
        _check(lib, lib.iron_quantize_i4g32(Wdv.data_ptr(), c.data_ptr(), s.data_ptr(), W.shape[0], W.shape[1],
                                            stream))
        q[name] = (c, s)
    per = sum(c.numel() + 2 * s.numel() for c, s in q.values())
    reps = copies_for(per)
    Q = [q] + [{k: (c.clone(), s.clone()) for k, (c, s) in q.items()} for _ in range(reps - 1)]

    def block4(i, s):
        a = Q[i % reps]
        _check(lib, lib.iron_gemv_i4g32_fused(a["g"][0].data_ptr(), a["g"][1].data_ptr(), a["u"][0].data_ptr(),
                                              a["u"][1].data_ptr(), xd.data_ptr(), h.data_ptr(), F, E, 1, 1,
                                              nwd.data_ptr(), 1e-5, None, 0, None, s))
        _check(lib, lib.iron_gemv_i4g32_fused(a["d"][0].data_ptr(), a["d"][1].data_ptr(), None, None, h.data_ptr(),
                                              y.data_ptr(), E, F, 1, 0, None, 0.0, xd.data_ptr(), 0, None, s))

    for i in range(10):
        block4(i, stream)
    t = tm.rotating_us(block4, reps, n)
    nbytes = per + 4 * E + 2 * 2 * F + 2 * E * 2
    cpu = None
    if cpu_s > 0:
        host = {k: (c.cpu(), s.cpu()) for k, (c, s) in q.items()}

        def cpu_block4():
            Wq = {k: ops.dequant_planar(c, s) for k, (c, s) in host.items()}
            return ops.swiglu_block_reference(x, nw, Wq["g"], Wq["u"], Wq["d"])

        cpu = _cpu_line(torch, cpu_block4, cpu_s, nbytes / 1e9, "GB/s",
                        "config-4 int4-g32 SwiGLU block (oracle.ops.dequant_planar, then swiglu_block_reference)")
    res["int4_g32"] = _gpu_line("swiglu_block_int4_cfg4", t, nbytes=nbytes, cpu=cpu)
    # the same block as one launch (iron_swiglu_decode_i4g32: h handed over inside the launch)
    ws = torch.zeros(int(_lib.query("iron_swiglu_decode_i4g32_workspace_bytes", E, F)), dtype=torch.uint8,
                     device=dev)

    def block1(i, s):
        a = Q[i % reps]
        _check(lib, lib.iron_swiglu_decode_i4g32(a["g"][0].data_ptr(), a["g"][1].data_ptr(), a["u"][0].data_ptr(),
                                                 a["u"][1].data_ptr(), a["d"][0].data_ptr(), a["d"][1].data_ptr(),
                                                 xd.data_ptr(), y.data_ptr(), E, F, 1, 1, nwd.data_ptr(), 1e-5,
                                                 xd.data_ptr(), ws.data_ptr(), 100000, s))

    for i in range(10):
        block1(i, stream)
    t1 = tm.rotating_us(block1, reps, n)
    torch.cuda.synchronize()
    if int(ws[:4].view(torch.int32).item()) != 0:
        raise RuntimeError("iron_swiglu_decode_i4g32: a wait gave up during the benchmark")
    res["int4_g32_one_launch"] = _gpu_line("swiglu_block_int4_cfg4_one_launch", t1, nbytes=nbytes, cpu=cpu)
    return res


def _traced(torch, dev, launch, copies, calls, tag):
    """Device phase traces (iron_trace_next_launch) of `calls` calls of
    launch(i, stream), each on rotated (cold) inputs after a warm round: the
    spread of their spans, and the phase summary of the median-span call,
    whose Perfetto JSON goes to TRACE_DIR/<tag>.json."""
    from iron_amd import _lib
    from iron_amd.common import tracing_utils as tu

    s = _lib.stream_handle(dev)
    buf = tu.new_buffer(1 << 16, dev)
    for i in range(copies):
        launch(i, s)
    runs = []
    for i in range(calls):
        buf.zero_()
        tu.arm(buf)
        launch(i, s)
        torch.cuda.synchronize()
        recs = tu.parse_records(buf)
        summ = tu.phase_summary(recs)
        runs.append((max(v["span_ns"] for v in summ.values()), recs, summ))
    runs.sort(key=lambda r: r[0])
    span, recs, summ = runs[len(runs) // 2]
    out_dir = Path(TRACE_DIR)
    out_dir.mkdir(parents=True, exist_ok=True)
    with open(out_dir / f"{tag}.json", "w") as f:
        json.dump(tu.perfetto_json(recs), f)
    tu.print_cycles_summary(summ)
    rnd = lambda v: round(v, 1) if isinstance(v, float) else v
    return {"calls": calls, "span_ns": {"min": round(runs[0][0], 1), "median": round(span, 1),
                                         "max": round(runs[-1][0], 1)},
            "median_call": {k: {"workgroups": v["workgroups"], "span_ns": round(v["span_ns"], 1),
                                "points": [{kk: rnd(vv) for kk, vv in p.items()} for p in v["points"]]}
                            for k, v in summ.items()}}


def bench_trace(torch, lib, dev, calls=25):
    """--mode trace: per-workgroup phase traces of the decode attention (config
    3 and KV 4096, streamed caches), the headline int4 GEMV (config 2), the
    one-launch SwiGLU block (config 4) and the bf16 prefill GEMM (config 5 and
    4096^3), on cold inputs."""
    from iron_amd import _lib
    from oracle import configs, ops

    res = {}
    H, Hkv, D = 32, 8, 64
    for L, max_len in ((2048, 2048), (4096, 4608)):
        q, kn, vn, kc, vc, pos, angles = configs.cfg3_gqa_decode(n_heads=H, n_kv=Hkv, head_dim=D, L=L)
        if max_len > L:
            pad = torch.zeros(Hkv, max_len - L, D, dtype=kc.dtype)
            kc, vc = torch.cat([kc, pad], 1), torch.cat([vc, pad], 1)
            angles = ops.rope_angles_table(D, max_len, theta=500000.0)
        copies = copies_for(2 * Hkv * L * D * 2)
        KC = [kc.to(dev) for _ in range(copies)]
        VC = [vc.to(dev) for _ in range(copies)]
        qd, knd, vnd, ad = q.to(dev), kn.to(dev), vn.to(dev), angles.to(dev)
        out = torch.empty(H, D, dtype=torch.bfloat16, device=dev)
        ws = torch.zeros(int(lib.iron_gqa_decode_workspace_bytes(H, Hkv, D, max_len)), dtype=torch.uint8, device=dev)

        def attn(i, s):
            _check(lib, lib.iron_gqa_decode_ex(qd.data_ptr(), knd.data_ptr(), vnd.data_ptr(), KC[i % copies].data_ptr(),
                                               VC[i % copies].data_ptr(), ad.data_ptr(), angles.shape[0],
                                               out.data_ptr(), ws.data_ptr(), H, Hkv, D, max_len, pos, None,
                                               1.0 / math.sqrt(D), 2, s))

        res["gqa_decode_cfg3" if L == 2048 else "gqa_decode_kv4096"] = _traced(
            torch, dev, attn, copies, calls, "gqa_decode_cfg3" if L == 2048 else "gqa_decode_kv4096")
        del KC, VC
    codes, scales, x = configs.cfg2_gemv_int4()
    copies = copies_for(codes.numel() + 2 * scales.numel())
    C = [codes.to(dev) for _ in range(copies)]
    S = [scales.to(dev) for _ in range(copies)]
    xd = x.to(dev)
    y = torch.empty(8192, dtype=torch.bfloat16, device=dev)

    def gemv(i, s):
        _check(lib, lib.iron_gemv_i4g32(C[i % copies].data_ptr(), S[i % copies].data_ptr(), xd.data_ptr(),
                                        y.data_ptr(), 8192, 2048, 1, s))

    res["gemv_int4_cfg2"] = _traced(torch, dev, gemv, copies, calls, "gemv_int4_cfg2")
    del C, S
    E, F = 2048, 8192
    xb, nw, Wg, Wu, Wd = configs.cfg4_swiglu_block(E, F)
    q = []
    for W in (Wg, Wu, Wd):
        c = torch.empty(W.shape[0], W.shape[1] // 2, dtype=torch.uint8, device=dev)
        sc = torch.empty(W.shape[0], W.shape[1] // 32, dtype=torch.bfloat16, device=dev)
        _check(lib, lib.iron_quantize_i4g32(W.to(dev).data_ptr(), c.data_ptr(), sc.data_ptr(), W.shape[0], W.shape[1],
                                            _lib.stream_handle(dev)))
        q += [c, sc]
    copies = copies_for(sum(t.numel() * t.element_size() for t in q))
    Q = [q] + [[t.clone() for t in q] for _ in range(copies - 1)]
    xd, nwd = xb.to(dev), nw.to(dev)
    yb = torch.empty(E, dtype=torch.bfloat16, device=dev)
    ws = torch.zeros(int(_lib.query("iron_swiglu_decode_i4g32_workspace_bytes", E, F)), dtype=torch.uint8, device=dev)

    def swiglu(i, s):
        a = Q[i % copies]
        _check(lib, lib.iron_swiglu_decode_i4g32(*(t.data_ptr() for t in a), xd.data_ptr(), yb.data_ptr(), E, F, 1, 1,
                                                 nwd.data_ptr(), 1e-5, xd.data_ptr(), ws.data_ptr(), 100000, s))

    res["swiglu_one_launch_cfg4"] = _traced(torch, dev, swiglu, copies, calls, "swiglu_one_launch_cfg4")
    if int(ws[:4].view(torch.int32).item()) != 0:
        raise RuntimeError("iron_swiglu_decode_i4g32: a wait gave up during the trace")
    del Q
    # the bf16 prefill GEMM: config 5 (128x128 tiles, one per CU) and 4096^3 (256x256 tiles), cold weights
    for tag, (M, K, N) in (("gemm_cfg5", (512, 2048, 8192)), ("gemm_4096", (4096, 4096, 4096))):
        g = torch.Generator(device=dev).manual_seed(0)
        A = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
        W = (torch.randn(N, K, device=dev, generator=g) * 0.02).to(torch.bfloat16)
        C = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        copies = copies_for(2 * W.numel())
        Ws = [W] + [W.clone() for _ in range(copies - 1)]

        def gemm(i, s):
            _check(lib, lib.iron_gemm_bf16_nt(A.data_ptr(), Ws[i % copies].data_ptr(), C.data_ptr(), M, N, K, N, 0, 0,
                                              0.0, 0.0, s))

        res[tag] = _traced(torch, dev, gemm, copies, calls, tag)
        del Ws
    return res


def bench_prefill_gemm(torch, lib, tm, dev, n, int4=False, cpu_s=0.0, shape=(512, 2048, 8192)):
    """Config 5 prefill GEMM M=512 K=2048 N=8192 (bf16 weights, or int4-g32
    weights dequantised in the kernel's prologue), weights rotated through the
    pool (cold, as in the model, where each layer's weights are read once).
    `shape` = (M, K, N) times another bf16 projection the same way."""
    from iron_amd import _lib
    from oracle import ops

    M, K, N = shape
    g = torch.Generator(device=dev).manual_seed(0)
    A = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
    W = (torch.randn(N, K, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    C = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    stream = _lib.stream_handle(dev)
    if int4:
        codes = torch.empty(N, K // 2, dtype=torch.uint8, device=dev)
        scales = torch.empty(N, K // 32, dtype=torch.bfloat16, device=dev)
        _check(lib, lib.iron_quantize_i4g32(W.data_ptr(), codes.data_ptr(), scales.data_ptr(), N, K, stream))
        copies = copies_for(codes.numel() + 2 * scales.numel())
        CS = [(codes, scales)] + [(codes.clone(), scales.clone()) for _ in range(copies - 1)]
    else:
        copies = copies_for(2 * W.numel())
        Ws = [W] + [W.clone() for _ in range(copies - 1)]

    def launch(i, s):
        if int4:
            c, sc = CS[i % copies]
            _check(lib, lib.iron_gemm_i4g32_nt(A.data_ptr(), c.data_ptr(), sc.data_ptr(), C.data_ptr(), M, N,
                                               K, N, 0, 0, 0.0, 0.0, 1, 1, None, 0, s))
        else:
            _check(lib, lib.iron_gemm_bf16_nt(A.data_ptr(), Ws[i % copies].data_ptr(), C.data_ptr(), M, N, K, N, 0,
                                              0, 0.0, 0.0, s))

    for i in range(10):
        launch(i, stream)
    t = tm.rotating_us(launch, copies, n)
    cpu = None
    if cpu_s > 0 and not int4:
        Ah, Wh = A.cpu(), W.cpu()
        cpu = _cpu_line(torch, lambda: ops.gemm_reference(Ah, Wh, b_col_maj=True), cpu_s, 2.0 * M * N * K / 1e12,
                        "TFLOP/s", "config-5 prefill GEMM 512x2048x8192 via oracle.ops.gemm_reference (torch CPU, fp32)")
    res = _gpu_line("prefill_gemm" + ("_int4" if int4 else ""), t, flops=2.0 * M * N * K, cpu=cpu)
    res.update({"shape": [M, K, N], "weights": "int4-g32" if int4 else "bf16", "weight_copies": copies})
    if not int4:
        # the vendor library on the same shape and protocol: torch.matmul -> hipBLASLt (a 2-D product of a
        # transposed weight view; no batched kernel involved)
        out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)

        def launch_lib(i, s):
            torch.matmul(A, Ws[i % copies].t(), out=out)

        for i in range(10):
            launch_lib(i, stream)
        torch.cuda.synchronize()
        t_lib = tm.rotating_us(launch_lib, copies, n)
        tf = 2.0 * M * N * K / t_lib / 1e6
        res["library_reference"] = {"what": "torch.matmul (hipBLASLt), same shape, same weight rotation",
                                    "kernel_us": round(t_lib, 3), "TFLOP/s": round(tf, 1),
                                    "frac_mfma": round(tf / BF16_PEAK_TFLOPS, 4)}
    return res


def bench_prefill_attention(torch, lib, tm, dev, n, S=3968, cpu_s=0.0):
    """Causal GQA prefill attention of cfg 5's long prompt (32/8 heads, d 64):
    useful flops 4 * S * (S + 1) / 2 * d per head (QK^T and PV, visible keys).
    The 24 MB of operands are re-read many times per launch by design, so they
    are not rotated."""
    from iron_amd import _lib

    H, Hkv, D = 32, 8, 64
    g = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn(S, H * D, device=dev, generator=g).to(torch.bfloat16)
    k = torch.randn(Hkv, S, D, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(Hkv, S, D, device=dev, generator=g).to(torch.bfloat16)
    o = torch.empty(S, H * D, dtype=torch.bfloat16, device=dev)
    stream = _lib.stream_handle(dev)

    def launch(i, s):
        _check(lib, lib.iron_attention_prefill(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), H, Hkv, S, S,
                                               D, D, H * D, S * D, D, D, H * D, S, 1, 0, 0.125, s))

    for i in range(5):
        launch(i, stream)
    t = tm.rotating_us(launch, 1, n)
    flops = 4.0 * S * (S + 1) / 2 * D * H
    cpu = None
    if cpu_s > 0:
        from oracle import ops

        # the oracle takes the whole causal attention of the prompt (all 32 heads);
        # its value counts the same useful flops as the GPU figure
        Qc = q.cpu().view(S, H, D).transpose(0, 1).contiguous()
        Kc, Vc = k.cpu(), v.cpu()
        cpu = _cpu_line(torch, lambda: ops.attention_reference(Qc, Kc, Vc, causal=True, scale=0.125), cpu_s,
                        flops / 1e12, "TFLOP/s",
                        f"causal GQA prefill attention, {S} tokens, 32/8 heads via oracle.ops.attention_reference "
                        "(torch CPU, fp32 scores and softmax; counted as the GPU figure's useful flops)")
    res = _gpu_line("prefill_attention", t, flops=flops, cpu=cpu)
    res["seq"] = S
    return res


def bench_floor(torch, lib, tm, dev):
    """The floors that bound one short launch, measured with the protocol of the
    kernels they bound: an empty kernel as one node of a replayed graph (and
    issued one Python call at a time), and a pure streaming read of the decode
    kernels' sizes from the rotation pool, at 1..8 16-byte loads in flight per
    lane (iron_probe_read)."""
    from iron_amd import _lib

    out = {"empty_graph_node_us": {}, "empty_python_launch_us": {}, "read_us": {}}
    for wgs in (1, 256, 2048, 8192):
        def empty(i, s, wgs=wgs):
            _check(lib, lib.iron_probe_empty(wgs, s))

        empty(0, _lib.stream_handle(dev))
        out["empty_graph_node_us"][str(wgs)] = round(tm.rotating_us(empty, 1, 500), 3)
        out["empty_python_launch_us"][str(wgs)] = round(tm.wall_ms(empty, 500) * 1e3 / 500, 3)
    sizes = {"cfg2_int4_gemv": 9457664, "cfg3_gqa_kv": 4194304, "kv4096_layer": 8388608,
             "cfg1_bf16_gemv": 33574912, "swiglu_int4_pair": 18874368, "lm_head_bf16": 525336576,
             "stream_1GiB": 1 << 30}
    for name, nbytes in sizes.items():
        stride = (nbytes + 255) // 256 * 256
        copies = copies_for(stride)
        pool = torch.empty(copies * stride, dtype=torch.uint8, device=dev)
        pool.random_(0, 256)
        base = pool.data_ptr()
        row = {}
        for lpl in (1, 2, 4, 8):
            wgs = int(lib.iron_probe_read_workgroups(nbytes, lpl))
            sink = torch.empty(wgs, dtype=torch.int32, device=dev)

            def read(i, s, lpl=lpl, sink=sink, wgs=wgs):
                _check(lib, lib.iron_probe_read(base + (i % copies) * stride, nbytes, sink.data_ptr(), wgs, lpl, s))

            read(0, _lib.stream_handle(dev))
            t = tm.rotating_us(read, copies, 200 if nbytes < (64 << 20) else 2 * copies)
            row[f"loads_per_lane_{lpl}"] = {"us": round(t, 3), "GB/s": round(nbytes / t / 1e3, 1)}
        best = min(v["us"] for v in row.values())
        out["read_us"][name] = {"bytes": nbytes, "best_us": best, "best_GB/s": round(nbytes / best / 1e3, 1),
                                "by_shape": row}
        del pool
    return out


def bench_mfma(torch, lib, tm, dev):
    """MFMA issue rate and shader clock (iron_probe_mfma): register-only
    v_mfma_f32_32x32x16_bf16 loops, first with the config 5 prefill GEMM's
    per-CU work (256 workgroups of 8 waves, 256 MFMAs per wave on 2
    accumulators, as its 128x128 tile issues over K = 2048), then variants.
    Per case: graph-replayed time per launch, achieved TFLOP/s, and from the
    in-kernel clock stamps the median shader clock (MHz) and shader cycles per
    wave."""
    from iron_amd import _lib

    cases = [("cfg5_gemm_tile", 256, 8, 256, 2), ("cfg5_4chains", 256, 8, 256, 4), ("cfg5_8chains", 256, 8, 256, 8),
             ("1wave_per_simd", 256, 4, 512, 2), ("1wave_per_simd_4chains", 256, 4, 512, 4),
             ("steady_2x", 512, 8, 2048, 4), ("steady_4x", 1024, 8, 2048, 4)]
    out = {}
    for name, wgs, wpw, n, chains in cases:
        waves = wgs * wpw
        sink = torch.empty(waves, dtype=torch.float32, device=dev)
        clocks = torch.zeros(waves * 4, dtype=torch.int64, device=dev)

        def run(i, s, wgs=wgs, wpw=wpw, n=n, chains=chains, sink=sink, clocks=clocks, waves=waves):
            _check(lib, lib.iron_probe_mfma(wgs, wpw, n, chains, sink.data_ptr(), clocks.data_ptr(), waves, s))

        run(0, _lib.stream_handle(dev))
        t = tm.rotating_us(run, 1, 20)
        torch.cuda.synchronize()
        c = clocks.view(waves, 4).cpu().double()
        cyc = (c[:, 1] - c[:, 0])
        real_s = (c[:, 3] - c[:, 2]) / 100e6
        mhz = (cyc / real_s.clamp_min(1e-9) / 1e6).median().item()
        flops = 2.0 * 32 * 32 * 16 * n * waves
        out[name] = {"workgroups": wgs, "waves_per_wg": wpw, "mfma_per_wave": n, "chains": chains,
                     "kernel_us": round(t, 3), "TFLOP/s": round(flops / t / 1e6, 1),
                     "frac_mfma": round(flops / t / 1e6 / BF16_PEAK_TFLOPS, 4),
                     "shader_MHz_median": round(mhz, 1), "wave_cycles_median": int(cyc.median().item()),
                     "wave_us_median": round(float(real_s.median().item()) * 1e6, 3)}
    return out


def bench_model(torch, dev, decode_steps=128, prompt_len=512, long_ctx=3968):
    """Config 5: random-init Llama-3.2-1B shape, int4-g32 linears, bf16 tied head."""
    from iron_amd.applications.llama_3_2_1b import LlamaConfig, LlamaHIP, random_weights

    cfg = LlamaConfig(max_seq_len=long_ctx + decode_steps + 64)
    t0 = time.perf_counter()
    model = LlamaHIP(cfg, random_weights(cfg, dev, seed=0), device=dev)
    init_s = time.perf_counter() - t0
    g = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, cfg.vocab_size, (prompt_len,), generator=g).tolist()
    model.reset()
    model.prefill(prompt)  # warm (code objects, buffers)
    model.reset()
    model.prefill(prompt, use_graph=True)  # eager run + capture of this prompt length's prefill graph
    model.capture_decode_graph()
    out = {"init_s": round(init_s, 2)}

    def ttft_s(use_graph):
        """Median of 3 timed prefills of the prompt from position 0 (prompt ids copied from the host)."""
        t = []
        for _ in range(3):
            model.reset()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            model.prefill(prompt, use_graph=use_graph)
            torch.cuda.synchronize()
            t.append(time.perf_counter() - t0)
        return sorted(t)[1]

    eager = ttft_s(False)
    ttft = ttft_s(True)  # leaves the model prefilled for the decode below
    out["prefill_tokens"] = prompt_len
    out["ttft_ms"] = round(ttft * 1e3, 3)
    out["ttft_eager_ms"] = round(eager * 1e3, 3)
    out["prefill_tok_s"] = round(prompt_len / ttft, 1)

    t0 = time.perf_counter()
    model.decode(decode_steps)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    out["decode_steps"] = decode_steps
    out["decode_tok_s_kv512_640"] = round(decode_steps / dt, 1)
    out["decode_ms_per_token_kv512_640"] = round(dt / decode_steps * 1e3, 4)

    # long-context window: fill the cache to 3968, then decode to 4096
    long_prompt = torch.randint(0, cfg.vocab_size, (long_ctx,), generator=g).tolist()
    model.reset()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    model.prefill(long_prompt)
    torch.cuda.synchronize()
    out["prefill_3968_ms"] = round((time.perf_counter() - t0) * 1e3, 2)
    t0 = time.perf_counter()
    model.decode(decode_steps)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    out["decode_tok_s_kv3968_4096"] = round(decode_steps / dt, 1)
    out["decode_ms_per_token_kv3968_4096"] = round(dt / decode_steps * 1e3, 4)
    # bytes a decode token must stream at KV 4096 (int4 linears, bf16 head)
    E, F, V, Lr = cfg.emb_dim, cfg.hidden_dim, cfg.vocab_size, cfg.n_layers
    lin = (cfg.qkv_dim * E + E * E + 2 * F * E + E * F) * (0.5 + 2 / 32) * Lr
    kv = 2 * cfg.n_kv_groups * 4096 * cfg.head_dim * 2 * Lr
    head = V * E * 2
    per_tok = lin + kv + head
    out["decode_bytes_per_token_kv4096"] = int(per_tok)
    out["decode_GB/s_kv3968_4096"] = round(per_tok * out["decode_tok_s_kv3968_4096"] / 1e9, 1)
    out["decode_frac_hbm_kv3968_4096"] = round(out["decode_GB/s_kv3968_4096"] / HBM_PEAK_GBS, 4)

    # the same window with LlamaConfig(head_int4=True): the tied head as int4-g32 too
    del model
    torch.cuda.empty_cache()
    cfg4 = LlamaConfig(max_seq_len=long_ctx + decode_steps + 64, head_int4=True)
    model = LlamaHIP(cfg4, random_weights(cfg4, dev, seed=0), device=dev)
    model.reset()
    model.prefill(prompt)
    model.capture_decode_graph()
    model.reset()
    model.prefill(long_prompt)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    model.decode(decode_steps)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    head4 = V * E // 2 + V * (E // 32) * 2
    out["int4_head"] = {
        "decode_tok_s_kv3968_4096": round(decode_steps / dt, 1),
        "decode_ms_per_token_kv3968_4096": round(dt / decode_steps * 1e3, 4),
        "decode_bytes_per_token_kv4096": int(lin + kv + head4),
    }
    return out


def cpu_baseline_int4(torch, inputs, budget_s):
    """Oracle on the host cores: dequantize with torch ops, then fp32 matvec."""
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
        f"(torch CPU: dequantise to bf16, fp32 matvec), {dt:.1f} s",
    }


def cpu_baseline_model(torch, budget_s, prompt_len=512, long_ctx=3968):
    """The oracle's fp32 Llama forward (restated llama_cpu.py) on the host cores,
    Llama-3.2-1B shape, random fp32 weights, at config 5's windows beside the
    GPU figures: the 512-token prefill (TTFT), greedy decode steps after it (KV
    512 on), and greedy decode steps at KV 3968 on. The long window's cache is
    filled with random K/V rows instead of a 3968-token CPU prefill: a decode
    step's work does not depend on the cached values. Each decode window gets
    half of budget_s (a bounded sample)."""
    from iron_amd.applications.llama_3_2_1b import LlamaConfig, random_weights
    from iron_amd.applications.llama_3_2_1b.model import compute_rope_angles
    from oracle import llama as ollama

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    cfg = LlamaConfig()
    t0 = time.perf_counter()
    w = {k: v.float() for k, v in random_weights(cfg, torch.device("cpu"), seed=0).items()}
    shape = ollama.LlamaShape(cfg.vocab_size, cfg.emb_dim, cfg.n_layers, cfg.n_heads, cfg.n_kv_groups, cfg.hidden_dim)
    ref = ollama.LlamaCPU(shape, w, compute_rope_angles(cfg.head_dim, long_ctx + 512, cfg.rope_base, cfg.rope_scaling))
    setup_s = time.perf_counter() - t0
    g = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, cfg.vocab_size, (1, prompt_len), generator=g)

    def decode(logits, kv0, budget):
        steps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < budget:
            logits = ref.forward(torch.tensor([[int(logits.argmax())]]), last_only=True)[0, -1]
            steps += 1
        dt = time.perf_counter() - t0
        return {"value": round(steps / dt, 3), "unit": "tok/s", "cores": threads, "kind": "port",
                "sample": f"{steps} greedy decode steps of the oracle's fp32 Llama forward (restated llama_cpu.py), "
                f"Llama-3.2-1B shape, random weights, KV {kv0}..{kv0 + steps}, {dt:.1f} s"}

    ref.reset()
    t0 = time.perf_counter()
    logits = ref.forward(prompt, last_only=True)[0, -1]
    ttft = time.perf_counter() - t0
    short = decode(logits, prompt_len, budget_s / 2)
    # the long window: caches of long_ctx random rows (bf16-representable, like the GPU's)
    for i in range(shape.n_layers):
        ref.kc[i] = torch.randn(1, shape.n_kv_groups, long_ctx, shape.head_dim, generator=g).bfloat16().float()
        ref.vc[i] = torch.randn(1, shape.n_kv_groups, long_ctx, shape.head_dim, generator=g).bfloat16().float()
    long = decode(logits, long_ctx, budget_s / 2)
    return {
        "ttft_ms_512": {"value": round(ttft * 1e3, 1), "unit": "ms", "cores": threads, "kind": "port",
                        "sample": f"one {prompt_len}-token prefill of the oracle's fp32 Llama forward (last position's "
                        "logits), Llama-3.2-1B shape"},
        "decode_kv512": short,
        "decode_kv3968": long,
        "setup_s": round(setup_s, 1),
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="host-time budget of the config 2 and model-decode CPU baselines (the other configs' "
                    "baselines get a third of it each)")
    ap.add_argument("--mode", choices=["full", "gemv", "gemv_bf16", "sustained", "model", "prefill", "gemm_large", "gemm_512",
                                       "attention", "floor", "mfma", "swiglu", "trace"],
                    default="full")
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
    from iron_amd import _lib

    lib = _lib.load()
    dev = torch.device("cuda", 0)
    tm = Timer(torch, lib)

    def emit(mode, extra):
        print(json.dumps({"metric": METRIC, "mode": mode, "extra": extra}), flush=True)
        return 0

    if args.mode == "model":
        return emit("model", {"llama_cfg5": bench_model(torch, dev)})
    if args.mode == "prefill":
        return emit("prefill", {
            "prefill_gemm_cfg5": bench_prefill_gemm(torch, lib, tm, dev, 100),
            "prefill_gemm_int4_cfg5": bench_prefill_gemm(torch, lib, tm, dev, 100, int4=True),
            "prefill_attention_cfg5": bench_prefill_attention(torch, lib, tm, dev, 20),
        })
    if args.mode == "gemm_large":
        # the 3968-token prefill projections (o_proj, qkv, down, fused gate/up pair) and 4096^3, each beside
        # hipBLASLt on the same shape and weight rotation
        shapes = {"o_proj_3968": (3968, 2048, 2048), "qkv_3968": (3968, 2048, 3072), "down_3968": (3968, 8192, 2048),
                  "gate_up_3968": (3968, 2048, 16384), "square_4096": (4096, 4096, 4096)}
        return emit("gemm_large", {k: bench_prefill_gemm(torch, lib, tm, dev, 10, shape=v) for k, v in shapes.items()})
    if args.mode == "gemm_512":
        # the 512-token projections through the plain entry point (no workspace, so no K split: the smaller tiles
        # for shapes whose 128x128 tiles leave CUs idle), each beside hipBLASLt on the same shape and weights
        shapes = {"o_proj_512": (512, 2048, 2048), "qkv_512": (512, 2048, 3072), "down_512": (512, 8192, 2048),
                  "gate_up_512": (512, 2048, 16384)}
        return emit("gemm_512", {k: bench_prefill_gemm(torch, lib, tm, dev, 50, shape=v) for k, v in shapes.items()})
    if args.mode == "attention":
        return emit("attention", {
            "gqa_decode_cfg3": bench_gqa(torch, lib, tm, dev, 300),
            "gqa_decode_kv4096": bench_gqa(torch, lib, tm, dev, 300, L=4096, max_len=4608),
        })
    if args.mode == "gemv_bf16":
        return emit("gemv_bf16", {"gemv_bf16_cfg1": bench_gemv_bf16(torch, lib, tm, dev, 300)})
    if args.mode == "sustained":
        return emit("sustained", {"gemv_sustained": bench_gemv_sustained(torch, lib, tm, dev)})
    if args.mode == "trace":
        return emit("trace", {"trace": bench_trace(torch, lib, dev)})
    if args.mode == "swiglu":
        return emit("swiglu", {"swiglu_block_cfg4": bench_swiglu(torch, lib, tm, dev, 200)})
    if args.mode == "floor":
        return emit("floor", {"floor": bench_floor(torch, lib, tm, dev)})
    if args.mode == "mfma":
        return emit("mfma", {"mfma": bench_mfma(torch, lib, tm, dev)})

    i4 = bench_gemv_int4(torch, lib, tm, dev, args.steps, args.warmup)
    value = i4["bytes"] * args.steps / (i4["wall_ms"] * 1e-3) / 1e9
    kernel_us = i4["wall_ms"] * 1e3 / args.steps
    achieved_live = i4["bytes"] / kernel_us / 1e3
    metric_lines("gemv_int4_cfg2", kernel_us, i4["bytes"])
    # The roofline uses the kernel duration rocprofv3's kernel trace reports for
    # this command's dispatches (each traced dispatch carries its own completion
    # signal, so it is longer than the untraced per-step time above, which stays
    # the headline value), so that the line and profiles/ agree.
    trace_ns = profile_value(TRACE_PROFILE, "avg_ns")
    traffic = profile_value(PMC_PROFILE, "traffic_bytes")
    kernel_us_roof = trace_ns / 1e3 if trace_ns else kernel_us
    achieved = i4["bytes"] / kernel_us_roof / 1e3
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
            "workload": "BASELINE configs[1]: fused int4-g32 dequant+GEMV, batch 1, W 8192x2048 (signed int4 "
            "codes, bf16 group-32 scales, zero-point 0), x 2048 bf16 ~N(0,1), fp32 accumulate, bf16 out, seed 0",
            "weight_pool_copies": i4["copies"],
            "algorithmic_bytes_per_step": i4["bytes"],
            "timed_distinct_bytes": i4["timed_distinct_bytes"],
            "timing": "device time of the steps launches = replay time of one graph holding a lead of "
            "weight_pool_copies launches then the steps launches, minus the replay time of the lead alone "
            "(medians of 5)",
            "lead_replay_ms": round(i4["lead_ms"], 4),
            "lead_plus_steps_replay_ms": round(i4["full_ms"], 4),
            "python_launch_us": round(i4["python_launch_us"], 3),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": int(traffic) if traffic else None,
            "kernel": "gemv_i4_fast<1, 2, 1, false, 0, false>",
            "kernel_us": round(kernel_us_roof, 3),
            "kernel_us_source": TRACE_PROFILE if trace_ns else "live (profile missing)",
            "traffic_source": PMC_PROFILE if traffic else None,
            "kernel_us_live": round(kernel_us, 3),
            "achieved_live": round(achieved_live, 2),
            "frac_live": round(achieved_live / HBM_PEAK_GBS, 4),
            "live_timing": "untraced per-step device time of this run (the headline value); the kernel trace's "
            "per-dispatch duration includes a completion signal per dispatch",
        },
    }
    if args.mode == "gemv":
        # calibration for the PMC runs: 64 MiB device-to-device copies (known bytes)
        src = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
    else:
        cs = 0.0 if args.no_cpu_baseline else args.cpu_seconds / 3
        extra = {
            "gemv_bf16_cfg1": bench_gemv_bf16(torch, lib, tm, dev, 300, cpu_s=cs),
            "gemv_sustained": bench_gemv_sustained(torch, lib, tm, dev, cpu_s=cs / 2),
            "gqa_decode_cfg3": bench_gqa(torch, lib, tm, dev, 300, cpu_s=cs),
            "gqa_decode_kv4096": bench_gqa(torch, lib, tm, dev, 300, L=4096, max_len=4608, cpu_s=cs),
            "swiglu_block_cfg4": bench_swiglu(torch, lib, tm, dev, 200, cpu_s=cs),
            "prefill_gemm_cfg5": bench_prefill_gemm(torch, lib, tm, dev, 100, cpu_s=cs),
            "prefill_attention_cfg5": bench_prefill_attention(torch, lib, tm, dev, 20, cpu_s=cs),
            "llama_cfg5": bench_model(torch, dev),
        }
        out["extra"] = extra
        if not args.no_cpu_baseline:
            out["cpu_baseline"] = cpu_baseline_int4(torch, i4["inputs"], args.cpu_seconds)
            model_cpu = cpu_baseline_model(torch, args.cpu_seconds)
            extra["llama_cfg5"]["cpu_baseline"] = model_cpu
            out["cpu_baseline"]["model_decode"] = model_cpu["decode_kv3968"]
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""Device phase traces as Perfetto JSON and a phase summary.

The MI355X counterpart of the reference's tracing path: a design's hardware
trace buffer (``trace_size`` / ``IRON_TRACE_SIZE``, iron/operators/_trace.py:
17-71) written out by ``dump_traces`` (iron/common/tracing_utils.py:49-115) as
trace text, Perfetto JSON and a cycles summary.

Here the trace is written by the kernels themselves. ``iron_trace_next_launch``
(include/iron_hip.h) arms a device buffer for the next entry-point call. Kernels
with trace points (decode attention, the int4 GEMV fast path, the one-launch
SwiGLU block, the bf16 GEMM) then write one 64-byte record per workgroup: kernel id,
workgroup, XCC_ID, HW_ID, and up to six s_memrealtime stamps (100 MHz, one
clock for all XCDs) taken when the workgroup passed each trace point.

An operator whose ``trace_size`` (or ``IRON_TRACE_SIZE``) is positive arms a
zero-filled buffer of that many bytes for each call of its callable and
exposes it as ``call.trace_buffer`` (iron_amd/common/base.py):

    fn = GEMVInt4(M=8192, K=2048, trace_size=1 << 20).get_callable()
    fn(codes, scales, x, y)
    dump_traces(fn, "gemv_i4_cfg2")

On an untraced callable ``dump_traces`` returns an empty list, so a test can
call it unconditionally. Environment: ``IRON_TRACE_DIR`` (default
``outputs/traces``) and ``IRON_TRACE_SIZE``.
"""

from __future__ import annotations

import json
import os
from pathlib import Path

import numpy as np

__all__ = [
    "KERNELS",
    "RECORD_BYTES",
    "arm",
    "dump_traces",
    "new_buffer",
    "parse_records",
    "perfetto_json",
    "phase_summary",
    "print_cycles_summary",
    "resolve_trace_size",
]

DEFAULT_TRACE_DIR = "outputs/traces"
RECORD_BYTES = 64
STAMPS = 6
CLOCK_HZ = 100e6  # s_memrealtime

# kernel id -> (name, trace point names); ids and points as the kernels write them
KERNELS = {
    1: ("gqa_decode", ("start", "q in LDS", "scores and P.V", "partial stored", "counted in", "merged")),
    2: ("gemv_i4", ("start", "x prepared", "row products")),
    3: ("swiglu_decode_i4", ("start", "x ready", "h published", "h gathered", "down row")),
    4: ("gemm_bf16", ("start", "first stage", "K quarter", "K half", "K three quarters", "tile stored")),
}


def resolve_trace_size(trace_size=None) -> int:
    """Effective trace size in bytes: an explicit positive argument, else
    ``IRON_TRACE_SIZE``, else 0 (off). A malformed environment value raises."""
    if trace_size and trace_size > 0:
        return int(trace_size)
    return int(os.environ.get("IRON_TRACE_SIZE", "0"))


def new_buffer(nbytes: int, device):
    """A zero-filled device trace buffer (64-byte aligned by the allocator)."""
    import torch

    return torch.zeros(max(RECORD_BYTES, int(nbytes) // RECORD_BYTES * RECORD_BYTES), dtype=torch.uint8,
                       device=device)


def arm(buffer) -> None:
    """Arm `buffer` (a device uint8 tensor) for this thread's next entry-point call."""
    from .. import _lib

    _lib.call("iron_trace_next_launch", buffer.data_ptr(), buffer.numel())


def _host_bytes(buffer) -> np.ndarray:
    if hasattr(buffer, "cpu"):
        buffer = buffer.cpu().numpy()
    a = np.asarray(buffer)
    return a.view(np.uint8).reshape(-1)


def parse_records(buffer) -> list[dict]:
    """The written records of a trace buffer (device or host bytes).

    Each: kernel id and name, workgroup, xcc, hw_id, and `stamps` (the clock
    values of the trace points the workgroup reached, in order; a point it
    never reached ends the list)."""
    raw = _host_bytes(buffer)
    n = raw.size // RECORD_BYTES
    words = raw[: n * RECORD_BYTES].view(np.uint32).reshape(n, RECORD_BYTES // 4)
    stamps = raw[: n * RECORD_BYTES].view(np.uint64).reshape(n, RECORD_BYTES // 8)[:, 2:2 + STAMPS]
    out = []
    for i in np.nonzero(words[:, 0])[0]:
        kid = int(words[i, 0])
        name, points = KERNELS.get(kid, (f"kernel{kid}", tuple(f"point {k}" for k in range(STAMPS))))
        st = []
        for k in range(len(points)):
            v = int(stamps[i, k])
            if v == 0:
                break
            st.append(v)
        out.append({"kernel": kid, "name": name, "points": points[: len(st)], "workgroup": int(words[i, 1]),
                    "xcc": int(words[i, 2]), "hw_id": int(words[i, 3]), "stamps": st})
    return out


def _ns(ticks: int) -> float:
    return ticks * 1e9 / CLOCK_HZ


def phase_summary(records: list[dict]) -> dict:
    """Per kernel: for each trace point, the workgroups that reached it and the
    time of reaching it from the launch's earliest start (ns: min, median,
    p90, max), and for each step between consecutive points its duration (ns:
    median, p90); plus the span (last stamp - first start)."""
    by = {}
    for r in records:
        by.setdefault(r["name"], []).append(r)
    out = {}
    for name, recs in by.items():
        t0 = min(r["stamps"][0] for r in recs if r["stamps"])
        last = max(r["stamps"][-1] for r in recs if r["stamps"])
        points = max((r["points"] for r in recs), key=len)
        pts = []
        for k, p in enumerate(points):
            at = np.array([_ns(r["stamps"][k] - t0) for r in recs if len(r["stamps"]) > k])
            step = np.array([_ns(r["stamps"][k] - r["stamps"][k - 1]) for r in recs if len(r["stamps"]) > k]) if k else None
            row = {"point": p, "workgroups": int(at.size), "min": float(at.min()), "median": float(np.median(at)),
                   "p90": float(np.percentile(at, 90)), "max": float(at.max())}
            if step is not None and step.size:
                row["step_median"] = float(np.median(step))
                row["step_p90"] = float(np.percentile(step, 90))
            pts.append(row)
        out[name] = {"workgroups": len(recs), "span_ns": _ns(last - t0), "points": pts}
    return out


def print_cycles_summary(summary: dict) -> None:
    """Print a phase_summary() (the role of mlir-aie's per-tile cycles summary)."""
    for name, s in summary.items():
        print(f"[trace] {name}: {s['workgroups']} workgroups, span {s['span_ns']:.0f} ns")
        for p in s["points"]:
            step = f"  step median {p['step_median']:.0f} p90 {p['step_p90']:.0f}" if "step_median" in p else ""
            print(f"[trace]   {p['point']:<16} n={p['workgroups']:<5} at min {p['min']:.0f} median {p['median']:.0f} "
                  f"p90 {p['p90']:.0f} max {p['max']:.0f} ns{step}")


def perfetto_json(records: list[dict]) -> dict:
    """Chrome/Perfetto trace events: one process per XCD, one thread per
    workgroup, one complete event per step between trace points (named after
    the point it ends at), times in microseconds from the earliest start."""
    if not records:
        return {"traceEvents": []}
    t0 = min(r["stamps"][0] for r in records if r["stamps"])
    ev = []
    for x in sorted({r["xcc"] for r in records}):
        ev.append({"ph": "M", "name": "process_name", "pid": x, "args": {"name": f"XCD {x}"}})
    for r in records:
        st = r["stamps"]
        for k in range(1, len(st)):
            ev.append({"name": r["points"][k], "cat": r["name"], "ph": "X", "pid": r["xcc"], "tid": r["workgroup"],
                       "ts": _ns(st[k - 1] - t0) / 1e3, "dur": _ns(st[k] - st[k - 1]) / 1e3,
                       "args": {"hw_id": r["hw_id"]}})
    return {"traceEvents": ev, "displayTimeUnit": "ns"}


def _slug(text: str) -> str:
    return "".join(c if c.isalnum() or c in "-_." else "_" for c in text)


def dump_traces(run, tag: str, out_dir=None, summary: bool = True) -> list[Path]:
    """Write a completed call's trace as text (one record per line) and
    Perfetto JSON, and print its phase summary. `run` is a callable whose
    ``trace_buffer`` holds the records (an operator callable with trace_size
    set), or a buffer itself. Returns the JSON paths written: empty when the
    callable is untraced or its buffer holds no record."""
    buffer = getattr(run, "trace_buffer", run if hasattr(run, "numel") or isinstance(run, np.ndarray) else None)
    if buffer is None:
        return []
    records = parse_records(buffer)
    if not records:
        print("[trace] buffer holds no record, no trace data captured")
        return []
    out_dir = Path(out_dir or os.environ.get("IRON_TRACE_DIR", DEFAULT_TRACE_DIR))
    out_dir.mkdir(parents=True, exist_ok=True)
    tag = _slug(tag)
    with open(out_dir / f"{tag}.txt", "w") as f:
        for r in records:
            f.write(f"{r['name']} wg={r['workgroup']} xcc={r['xcc']} hw_id=0x{r['hw_id']:08x} "
                    + " ".join(str(t) for t in r["stamps"]) + "\n")
    path = out_dir / f"{tag}.json"
    with open(path, "w") as f:
        json.dump(perfetto_json(records), f)
    print(f"[trace] {path}")
    if summary:
        print_cycles_summary(phase_summary(records))
    return [path]

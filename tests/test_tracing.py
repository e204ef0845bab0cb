"""CPU: the device phase-trace format, its Perfetto writer and summary, and the
host side of iron_trace_next_launch (the MI355X counterpart of the reference's
trace_size buffers and dump_traces, iron/operators/_trace.py:17-71,
iron/common/tracing_utils.py:49-115)."""

import json

import numpy as np
import pytest

from iron_amd.common import tracing_utils as tu


def _buffer(records, n_slots):
    """Trace buffer bytes with `records` = [(slot, kernel, wg, xcc, hw, stamps)]."""
    buf = np.zeros(n_slots * tu.RECORD_BYTES, dtype=np.uint8)
    words = buf.view(np.uint32).reshape(n_slots, 16)
    st = buf.view(np.uint64).reshape(n_slots, 8)
    for slot, kernel, wg, xcc, hw, stamps in records:
        words[slot, :4] = (kernel, wg, xcc, hw)
        st[slot, 2:2 + len(stamps)] = stamps
    return buf


def test_parse_records_and_truncated_points():
    buf = _buffer([(0, 2, 0, 3, 0x1234, [1000, 1010, 1030]),
                   (2, 2, 2, 5, 0x10, [1002, 1020, 1035]),
                   (3, 1, 3, 0, 0, [990, 1000, 1100, 1110, 1150])], 5)
    recs = tu.parse_records(buf)
    assert [r["workgroup"] for r in recs] == [0, 2, 3]  # slots 1 and 4 were never written
    assert recs[0]["name"] == "gemv_i4" and recs[0]["xcc"] == 3 and recs[0]["hw_id"] == 0x1234
    assert recs[0]["points"] == ("start", "x prepared", "row products")
    assert recs[2]["name"] == "gqa_decode" and len(recs[2]["stamps"]) == 5  # never reached "merged"
    assert recs[2]["points"][-1] == "counted in"


def test_phase_summary_times_and_steps():
    # three workgroups of one kernel; clock ticks are 10 ns
    buf = _buffer([(0, 2, 0, 0, 0, [100, 110, 130]),
                   (1, 2, 1, 1, 0, [102, 120, 140]),
                   (2, 2, 2, 2, 0, [104, 112, 160])], 3)
    s = tu.phase_summary(tu.parse_records(buf))["gemv_i4"]
    assert s["workgroups"] == 3 and s["span_ns"] == pytest.approx(600.0)
    start, x, rows = s["points"]
    assert start["median"] == pytest.approx(20.0) and start["max"] == pytest.approx(40.0)
    assert x["min"] == pytest.approx(100.0) and x["median"] == pytest.approx(120.0) and x["max"] == pytest.approx(200.0)
    assert x["step_median"] == pytest.approx(100.0)  # steps 100, 180, 80 ns
    assert rows["step_median"] == pytest.approx(200.0)  # steps 200, 200, 480 ns
    assert rows["max"] == pytest.approx(600.0)


def test_perfetto_events():
    buf = _buffer([(0, 3, 0, 4, 0, [200, 210, 250, 300, 320]),
                   (1, 3, 1, 6, 0, [205, 230])], 2)
    doc = tu.perfetto_json(tu.parse_records(buf))
    meta = [e for e in doc["traceEvents"] if e["ph"] == "M"]
    spans = [e for e in doc["traceEvents"] if e["ph"] == "X"]
    assert sorted(e["pid"] for e in meta) == [4, 6]
    assert len(spans) == 4 + 1
    first = [e for e in spans if e["tid"] == 0]
    assert [e["name"] for e in first] == ["x ready", "h published", "h gathered", "down row"]
    assert first[0]["ts"] == pytest.approx(0.0) and first[0]["dur"] == pytest.approx(0.1)  # 10 ticks = 100 ns
    assert first[-1]["ts"] == pytest.approx(1.0) and first[-1]["dur"] == pytest.approx(0.2)
    json.dumps(doc)


def test_dump_traces_files_and_untraced(tmp_path):
    class Run:  # an operator callable after a traced call
        trace_buffer = _buffer([(0, 2, 0, 0, 0, [100, 110, 130])], 4)

    paths = tu.dump_traces(Run(), "gemv trace/1", out_dir=tmp_path)
    assert paths == [tmp_path / "gemv_trace_1.json"]
    assert json.loads(paths[0].read_text())["traceEvents"]
    assert (tmp_path / "gemv_trace_1.txt").read_text().startswith("gemv_i4 wg=0 xcc=0")

    class Untraced:
        trace_buffer = None

    assert tu.dump_traces(Untraced(), "x", out_dir=tmp_path) == []
    assert tu.dump_traces(object(), "x", out_dir=tmp_path) == []

    class Empty:
        trace_buffer = np.zeros(256, dtype=np.uint8)

    assert tu.dump_traces(Empty(), "x", out_dir=tmp_path) == []


def test_resolve_trace_size(monkeypatch):
    monkeypatch.delenv("IRON_TRACE_SIZE", raising=False)
    assert tu.resolve_trace_size() == 0 and tu.resolve_trace_size(4096) == 4096
    monkeypatch.setenv("IRON_TRACE_SIZE", "8192")
    assert tu.resolve_trace_size() == 8192 and tu.resolve_trace_size(64) == 64
    monkeypatch.setenv("IRON_TRACE_SIZE", "lots")
    with pytest.raises(ValueError):
        tu.resolve_trace_size()


def test_trace_arming_checked_on_host():
    """A misaligned buffer is refused; an armed buffer too small for the launch
    makes the entry point refuse before it launches, and disarms (the next call
    is untraced); NULL disarms."""
    from iron_amd import _lib

    p = 1 << 20  # stand-in addresses: nothing is launched
    with pytest.raises(_lib.IronHipError, match="64-byte aligned"):
        _lib.call("iron_trace_next_launch", p + 16, 4096)
    _lib.call("iron_trace_next_launch", p, 64)  # one record
    with pytest.raises(_lib.IronHipError, match="holds 1 records; this launch writes 1024"):
        _lib.call("iron_gemv_i4g32", p, p, p, p + (1 << 16), 8192, 2048, 1, None)
    _lib.call("iron_trace_next_launch", p, 64)
    _lib.call("iron_trace_next_launch", None, 0)  # disarmed again

"""GPU: device phase traces (iron_trace_next_launch) of the decode attention,
the int4 GEMV and the one-launch SwiGLU block. A traced call writes one record
per workgroup with its trace points in order, and its outputs are
bit-identical to an untraced call's."""

import pytest
import torch

from iron_amd.common import tracing_utils as tu
from oracle import configs

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16


def _bits_equal(a, b):
    return torch.equal(a.cpu().view(torch.int16), b.cpu().view(torch.int16))


def _monotone(rec):
    return all(b >= a for a, b in zip(rec["stamps"], rec["stamps"][1:]))


def test_trace_gqa_decode_cfg3(gpu, tmp_path):
    """Config 3 (KV 2048, one launch, 64-position chunks for streamed caches):
    every chunk reaches 'counted in', one per KV head merges, and a KV head's
    chunks all run on one XCD."""
    from iron_amd import _lib
    from iron_amd.operators import GQADecode

    print("trace: gqa decode cfg3", flush=True)
    q, kn, vn, kc, vc, pos, angles = configs.cfg3_gqa_decode()
    args = lambda: (q.to(gpu), kn.to(gpu), vn.to(gpu), kc.to(gpu).contiguous(), vc.to(gpu).contiguous(),
                    angles.to(gpu))
    outs = []
    for traced in (False, True):
        op = GQADecode(num_heads=32, num_kv_heads=8, head_dim=64, max_len=kc.shape[1], angle_rows=angles.shape[0],
                       trace_size=(1 << 16) if traced else None)
        op.set_position(pos)
        fn = op.get_callable()
        out = torch.empty(32, 64, dtype=BF16, device=gpu)
        fn(*args(), out)
        torch.cuda.synchronize()
        outs.append(out)
    assert _bits_equal(outs[0], outs[1])
    chunk = _lib.query("iron_gqa_decode_chunk_positions", 32, 8, 64, kc.shape[1], pos, _lib.stream_handle(gpu))
    recs = tu.parse_records(fn.trace_buffer)
    assert all(r["name"] == "gqa_decode" for r in recs)
    assert len(recs) == 8 * ((pos + chunk) // chunk)
    assert all(len(r["stamps"]) >= 5 and _monotone(r) for r in recs)
    assert sum(len(r["stamps"]) == 6 for r in recs) == 8  # the last arriver of each KV head
    if chunk in (64, 128):  # one launch: KV head j = workgroup % 8 ... all on one XCD
        for j in range(8):
            assert len({r["xcc"] for r in recs if r["workgroup"] % 8 == j}) == 1
    assert tu.dump_traces(fn, "gqa_cfg3", out_dir=tmp_path, summary=False) == [tmp_path / "gqa_cfg3.json"]


def test_trace_gemv_int4_cfg2(gpu):
    """The headline int4 GEMV (8192 x 2048): 1024 workgroups of 8 rows, three
    trace points each."""
    from iron_amd.operators import GEMVInt4

    print("trace: gemv int4 cfg2", flush=True)
    codes, scales, x = configs.cfg2_gemv_int4()
    a = (codes.to(gpu), scales.to(gpu), x.to(gpu))
    ys = []
    for traced in (False, True):
        fn = GEMVInt4(M=8192, K=2048, trace_size=(1 << 16) if traced else None).get_callable()
        y = torch.empty(8192, dtype=BF16, device=gpu)
        fn(*a, y)
        torch.cuda.synchronize()
        ys.append(y)
    assert _bits_equal(ys[0], ys[1])
    recs = tu.parse_records(fn.trace_buffer)
    assert len(recs) == 1024 and sorted(r["workgroup"] for r in recs) == list(range(1024))
    assert all(len(r["stamps"]) == 3 and _monotone(r) for r in recs)
    s = tu.phase_summary(recs)["gemv_i4"]
    assert s["span_ns"] > 0 and s["points"][2]["workgroups"] == 1024


def test_trace_too_small_buffer_refused(gpu):
    from iron_amd import _lib
    from iron_amd.operators import GEMVInt4

    codes, scales, x = configs.cfg2_gemv_int4()
    fn = GEMVInt4(M=8192, K=2048, trace_size=4096).get_callable()  # 64 records for 1024 workgroups
    with pytest.raises(_lib.IronHipError, match="this launch writes 1024"):
        fn(codes.to(gpu), scales.to(gpu), x.to(gpu), torch.empty(8192, dtype=BF16, device=gpu))


def test_trace_swiglu_one_launch(gpu):
    """The one-launch SwiGLU block: 256 workgroups, five trace points each; the
    h gathers all complete after the last publish."""
    from iron_amd import _lib

    print("trace: swiglu one launch", flush=True)
    x, nw, Wg, Wu, Wd = configs.cfg4_swiglu_block()
    s = _lib.stream_handle(gpu)
    q = []
    for W in ((Wg.float() * nw.float()).to(BF16), (Wu.float() * nw.float()).to(BF16), Wd):
        c = torch.empty(W.shape[0], W.shape[1] // 2, dtype=torch.uint8, device=gpu)
        sc = torch.empty(W.shape[0], W.shape[1] // 32, dtype=BF16, device=gpu)
        _lib.call("iron_quantize_i4g32", W.to(gpu).data_ptr(), c.data_ptr(), sc.data_ptr(), W.shape[0], W.shape[1], s)
        q += [c, sc]
    ws = torch.zeros(int(_lib.query("iron_swiglu_decode_i4g32_workspace_bytes", 2048, 8192)), dtype=torch.uint8,
                     device=gpu)
    xd = x.to(gpu)
    ys = []
    buf = tu.new_buffer(256 * tu.RECORD_BYTES, gpu)
    for traced in (False, True):
        y = torch.empty(2048, dtype=BF16, device=gpu)
        if traced:
            tu.arm(buf)
        _lib.call("iron_swiglu_decode_i4g32", *(t.data_ptr() for t in q), xd.data_ptr(), y.data_ptr(), 2048, 8192, 1,
                  2, None, 1e-5, xd.data_ptr(), ws.data_ptr(), 200000, s)
        torch.cuda.synchronize()
        ys.append(y)
    assert int(ws[:4].view(torch.int32).item()) == 0
    assert _bits_equal(ys[0], ys[1])
    recs = tu.parse_records(buf)
    assert len(recs) == 256 and all(len(r["stamps"]) == 5 and _monotone(r) for r in recs)
    last_publish = max(r["stamps"][2] for r in recs)
    assert all(r["stamps"][3] >= last_publish for r in recs)


def test_trace_gemm_cfg5(gpu):
    """The config 5 prefill GEMM (512 x 2048 x 8192, 128x128 tiles): 256
    workgroups, six trace points each, output bit-identical untraced."""
    from iron_amd import _lib

    print("trace: gemm cfg5", flush=True)
    g = torch.Generator(device=gpu).manual_seed(3)
    M, K, N = 512, 2048, 8192
    A = torch.randn(M, K, device=gpu, generator=g).to(BF16)
    W = (torch.randn(N, K, device=gpu, generator=g) * 0.02).to(BF16)
    s = _lib.stream_handle(gpu)
    buf = tu.new_buffer(1 << 16, gpu)
    cs = []
    for traced in (False, True):
        C = torch.empty(M, N, dtype=BF16, device=gpu)
        if traced:
            tu.arm(buf)
        _lib.call("iron_gemm_bf16_nt", A.data_ptr(), W.data_ptr(), C.data_ptr(), M, N, K, N, 0, 0, 0.0, 0.0, s)
        torch.cuda.synchronize()
        cs.append(C)
    assert _bits_equal(cs[0], cs[1])
    recs = tu.parse_records(buf)
    assert len(recs) == 256 and all(r["name"] == "gemm_bf16" for r in recs)
    assert all(len(r["stamps"]) == 6 and _monotone(r) for r in recs)

"""GPU: iron_gqa_decode_noalloc (partials in the library's per-GPU scratch
array, no workspace argument) against iron_gqa_decode with a caller workspace,
through the C ABI: identical output and cache appends, bit for bit, on two
calls in a row, the second with a smaller cache (the scratch keeps the first
call's partials, which must not leak into the second)."""

import math

import pytest
import torch

from oracle import configs, ops

pytestmark = pytest.mark.gpu


def _case(gpu, L, max_len, n_heads=32, n_kv=8, seed=0):
    q, kn, vn, kc, vc, pos, _ = configs.cfg3_gqa_decode(n_heads=n_heads, n_kv=n_kv, head_dim=64, L=L, seed=seed)
    pad = torch.zeros(n_kv, max_len - L, 64, dtype=kc.dtype)
    kc, vc = torch.cat([kc, pad], 1), torch.cat([vc, pad], 1)
    angles = ops.rope_angles_table(64, max_len, theta=500000.0)
    d = lambda t: t.to(gpu).contiguous()
    return dict(q=d(q), kn=d(kn), vn=d(vn), kc=d(kc), vc=d(vc), angles=d(angles), pos=pos, max_len=max_len,
                H=n_heads, Hkv=n_kv)


def _run(gpu, c, noalloc, pos_dev=False):
    from iron_amd import _lib

    kc, vc = c["kc"].clone(), c["vc"].clone()
    out = torch.full((c["H"], 64), -1.0, dtype=torch.bfloat16, device=gpu)
    s = _lib.stream_handle(gpu)
    pd = torch.tensor([c["pos"]], dtype=torch.int32, device=gpu) if pos_dev else None
    pos = -1 if pos_dev else c["pos"]
    common = (c["q"].data_ptr(), c["kn"].data_ptr(), c["vn"].data_ptr(), kc.data_ptr(), vc.data_ptr(),
              c["angles"].data_ptr(), c["angles"].shape[0], out.data_ptr())
    tail = (c["H"], c["Hkv"], 64, c["max_len"], pos, _lib.ptr(pd), 1.0 / math.sqrt(64), s)
    if noalloc:
        _lib.call("iron_gqa_decode_noalloc", *common, *tail)
    else:
        need = int(_lib.query("iron_gqa_decode_workspace_bytes", c["H"], c["Hkv"], 64, c["max_len"]))
        ws = torch.zeros(need, dtype=torch.uint8, device=gpu)  # the arrival counters start at zero
        _lib.call("iron_gqa_decode", *common, ws.data_ptr(), *tail)
    torch.cuda.synchronize()
    return out, kc, vc


def test_noalloc_matches_workspace_entry_point_twice(gpu):
    big = _case(gpu, L=4096, max_len=4608, seed=1)  # the Llama-3.2-1B decode shape at KV 4096
    small = _case(gpu, L=101, max_len=512, seed=2)  # then a smaller cache: fewer chunks than the first call
    for c, pos_dev in ((big, False), (small, True)):
        print(f"noalloc case: kv {c['pos'] + 1}, max_len {c['max_len']}, pos_dev {pos_dev}", flush=True)
        want = _run(gpu, c, noalloc=False, pos_dev=pos_dev)
        got = _run(gpu, c, noalloc=True, pos_dev=pos_dev)
        for w, g in zip(want, got):
            assert torch.equal(w.view(torch.int16), g.view(torch.int16))
        ref, _, _ = ops.gqa_decode_reference(c["q"].cpu(), c["kn"].cpu(), c["vn"].cpu(), c["kc"].cpu(),
                                             c["vc"].cpu(), c["pos"], c["angles"].cpu(), scale=0.125)
        ma, rl = ops.max_abs_rel_l2(got[0], ref)
        assert ma <= 2e-2 and rl <= 1e-2, (ma, rl)


def test_noalloc_group_sizes(gpu):
    """Other GQA group sizes (G = 1 and 8) share the same scratch array."""
    for H, Hkv in ((8, 8), (32, 4)):
        c = _case(gpu, L=300, max_len=320, n_heads=H, n_kv=Hkv, seed=3)
        want = _run(gpu, c, noalloc=False)
        got = _run(gpu, c, noalloc=True)
        for w, g in zip(want, got):
            assert torch.equal(w.view(torch.int16), g.view(torch.int16))


def test_noalloc_captured_in_a_graph(gpu):
    """iron_gqa_decode_noalloc captured into a hipGraph (its scratch address
    looked up beforehand, outside capture, by the max-bytes query) and replayed
    several times, with the program's own eager work between the replays:
    every replay's output and cache append equal iron_gqa_decode's bit for bit
    (the replay re-appends the same k/v row, so each replay computes the same)."""
    from iron_amd import _lib
    from iron_amd.common.graph import capture_graph

    assert _lib.query("iron_gqa_decode_noalloc_max_bytes") == 4 << 20
    c = _case(gpu, L=1000, max_len=1024, seed=4)
    print("noalloc under capture: kv 1000, max_len 1024", flush=True)
    want = _run(gpu, c, noalloc=False)
    kc, vc = c["kc"].clone(), c["vc"].clone()
    out = torch.full((c["H"], 64), -1.0, dtype=torch.bfloat16, device=gpu)

    def call():
        _lib.call("iron_gqa_decode_noalloc", c["q"].data_ptr(), c["kn"].data_ptr(), c["vn"].data_ptr(),
                  kc.data_ptr(), vc.data_ptr(), c["angles"].data_ptr(), c["angles"].shape[0], out.data_ptr(),
                  c["H"], c["Hkv"], 64, c["max_len"], c["pos"], None, 0.125, _lib.stream_handle(gpu))

    call()  # eager first: code object loaded
    torch.cuda.synchronize()
    graph = capture_graph(call, gpu)
    for r in range(4):
        out.fill_(-1.0)  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want[0].view(torch.int16)), f"replay {r}"
        assert torch.equal(kc.view(torch.int16), want[1].view(torch.int16)), f"replay {r}"
        assert torch.equal(vc.view(torch.int16), want[2].view(torch.int16)), f"replay {r}"

"""GPU: the one-launch int4 SwiGLU decode block (iron_swiglu_decode_i4g32).

Config 4's block (hidden 2048, FFN 8192, group-32 int4 weights) in one launch
whose workgroups hand h over inside the launch. Bar: bit-identical to the two
fused GEMV launches it replaces (gate/up pair, then down + residual), and
within BASELINE's max-abs 2e-2 / rel-L2 1e-2 of the fp32 chain on the same
dequantised weights. Also: repeated calls on one workspace (the tag epoch
advances), graph replays with the input changed between them, aliasing of x,
residual and y, and the give-up path forced from the host (a status word set
before the call), which must leave y untouched.
"""

import pytest
import torch

from oracle import configs, ops

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16
E, F = 2048, 8192
WAIT_US = 200000


def _bits_equal(a, b):
    return torch.equal(a.cpu().contiguous().view(torch.int16), b.cpu().contiguous().view(torch.int16))


def _i4(W, gpu):
    from iron_amd import _lib

    c = torch.empty(W.shape[0], W.shape[1] // 2, dtype=torch.uint8, device=gpu)
    s = torch.empty(W.shape[0], W.shape[1] // 32, dtype=BF16, device=gpu)
    _lib.call("iron_quantize_i4g32", W.to(gpu).data_ptr(), c.data_ptr(), s.data_ptr(), W.shape[0], W.shape[1],
              _lib.stream_handle(gpu))
    return c, s


@pytest.fixture(scope="module")
def block(gpu):
    x, nw, Wg, Wu, Wd = configs.cfg4_swiglu_block()
    folded = {m: (Wg if m != 2 else (Wg.float() * nw.float()).to(BF16),
                  Wu if m != 2 else (Wu.float() * nw.float()).to(BF16)) for m in (0, 1, 2)}
    q = {m: (*_i4(g, gpu), *_i4(u, gpu)) for m, (g, u) in folded.items() if m != 0}
    q[0] = q[1]
    dc, ds = _i4(Wd, gpu)
    torch.cuda.synchronize()
    return dict(x=x, nw=nw.to(gpu), q=q, dc=dc, ds=ds)


def _workspace(gpu):
    from iron_amd import _lib

    n = int(_lib.query("iron_swiglu_decode_i4g32_workspace_bytes", E, F))
    assert n > 0
    return torch.zeros(n, dtype=torch.uint8, device=gpu)


def _two_launch(b, mode, x, y, resid, gpu):
    from iron_amd import _lib

    gc, gs, uc, us = b["q"][mode]
    h = torch.empty(F, dtype=BF16, device=gpu)
    s = _lib.stream_handle(gpu)
    _lib.call("iron_gemv_i4g32_fused", gc.data_ptr(), gs.data_ptr(), uc.data_ptr(), us.data_ptr(), x.data_ptr(),
              h.data_ptr(), F, E, 1, mode, b["nw"].data_ptr() if mode == 1 else None, 1e-5, None, 0, None, s)
    _lib.call("iron_gemv_i4g32_fused", b["dc"].data_ptr(), b["ds"].data_ptr(), None, None, h.data_ptr(), y.data_ptr(),
              E, F, 1, 0, None, 0.0, _lib.ptr(resid), 0, None, s)


def _one_launch(b, mode, x, y, resid, ws, gpu, wait_us=WAIT_US):
    from iron_amd import _lib

    gc, gs, uc, us = b["q"][mode]
    _lib.call("iron_swiglu_decode_i4g32", gc.data_ptr(), gs.data_ptr(), uc.data_ptr(), us.data_ptr(),
              b["dc"].data_ptr(), b["ds"].data_ptr(), x.data_ptr(), y.data_ptr(), E, F, 1, mode,
              b["nw"].data_ptr() if mode == 1 else None, 1e-5, _lib.ptr(resid), ws.data_ptr(), wait_us,
              _lib.stream_handle(gpu))


def _status(ws):
    return int(ws[:4].view(torch.int32).item())


@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("with_resid", [True, False])
def test_one_launch_bit_identical_to_two_launches(gpu, block, mode, with_resid):
    print(f"swiglu one-launch: mode {mode}, residual {with_resid}", flush=True)
    xd = block["x"].to(gpu)
    resid = xd if with_resid else None
    ws = _workspace(gpu)
    y1 = torch.full((E,), 7.0, dtype=BF16, device=gpu)
    y2 = torch.empty(E, dtype=BF16, device=gpu)
    _one_launch(block, mode, xd, y1, resid, ws, gpu)
    _two_launch(block, mode, xd, y2, resid, gpu)
    torch.cuda.synchronize()
    assert _status(ws) == 0
    assert _bits_equal(y1, y2)


@pytest.mark.parametrize("mode", [1, 2])
def test_one_launch_against_fp32_chain(gpu, block, mode):
    """Config 4 at full size against the fp32 chain on the dequantised weights."""
    x, nw = block["x"], block["nw"].cpu()
    xd = x.to(gpu)
    ws = _workspace(gpu)
    y = torch.empty(E, dtype=BF16, device=gpu)
    _one_launch(block, mode, xd, y, xd, ws, gpu)
    torch.cuda.synchronize()
    gc, gs, uc, us = block["q"][mode]
    Wg = ops.dequant_planar(gc.cpu(), gs.cpu()).float()
    Wu = ops.dequant_planar(uc.cpu(), us.cpu()).float()
    Wd = ops.dequant_planar(block["dc"].cpu(), block["ds"].cpu()).float()
    xf = x.float()
    xhat = xf / torch.sqrt((xf * xf).mean() + 1e-5)
    xn = xhat * nw.float() if mode == 1 else xhat
    ref = xf + Wd @ (torch.nn.functional.silu(Wg @ xn) * (Wu @ xn))
    max_abs, rel_l2 = ops.max_abs_rel_l2(y, ref)
    assert max_abs <= 2e-2 and rel_l2 <= 1e-2, (max_abs, rel_l2)


def test_one_launch_in_place_repeated_and_graph(gpu, block):
    """x, residual and y one buffer (the decode layer's use), five calls in a row
    on one workspace with fresh inputs each time, then a captured graph replayed
    three times with the input rewritten eagerly between replays."""
    print("swiglu one-launch: in place, repeated, graph", flush=True)
    g = torch.Generator().manual_seed(5)
    ws = _workspace(gpu)
    for i in range(5):
        x = torch.randn(E, generator=g).to(BF16).to(gpu)
        buf = x.clone()
        ref = torch.empty(E, dtype=BF16, device=gpu)
        _one_launch(block, 2, buf, buf, buf, ws, gpu)
        _two_launch(block, 2, x, ref, x, gpu)
        torch.cuda.synchronize()
        assert _status(ws) == 0
        assert _bits_equal(buf, ref), f"call {i}"
    buf = torch.empty(E, dtype=BF16, device=gpu)
    s = torch.cuda.Stream(gpu)
    s.wait_stream(torch.cuda.current_stream(gpu))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            _one_launch(block, 2, buf, buf, buf, ws, gpu)
    torch.cuda.current_stream(gpu).wait_stream(s)
    for i in range(3):
        x = torch.randn(E, generator=g).to(BF16).to(gpu)
        buf.copy_(x)
        graph.replay()
        ref = torch.empty(E, dtype=BF16, device=gpu)
        _two_launch(block, 2, x, ref, x, gpu)
        torch.cuda.synchronize()
        assert _status(ws) == 0
        assert _bits_equal(buf, ref), f"replay {i}"


def test_one_launch_status_set_gives_up_and_recovers(gpu, block):
    """A status word already nonzero makes every wait give up: y stays as it
    was and the word stays set; after the workspace is zero-filled the call
    works again."""
    xd = block["x"].to(gpu)
    ws = _workspace(gpu)
    ws[:4].view(torch.int32).fill_(4)
    y = torch.full((E,), 3.0, dtype=BF16, device=gpu)
    _one_launch(block, 2, xd, y, xd, ws, gpu)
    torch.cuda.synchronize()
    assert _status(ws) != 0
    assert torch.equal(y.cpu(), torch.full((E,), 3.0, dtype=BF16))
    ws.zero_()
    ref = torch.empty(E, dtype=BF16, device=gpu)
    _one_launch(block, 2, xd, y, xd, ws, gpu)
    _two_launch(block, 2, xd, ref, xd, gpu)
    torch.cuda.synchronize()
    assert _status(ws) == 0
    assert _bits_equal(y, ref)

"""GPU: OperatorSequence dispatch modes and the SwiGLU sequence operators,
following the reference's own tests (swiglu_decode/test.py:16-104,
swiglu_prefill/test.py:17-110: same shapes, golden chain, tolerances and
buffer API)."""

import pytest
import torch

from iron_amd.common import OperatorSequence
from iron_amd.common.sequence import CompareDispatch, Tolerance
from iron_amd.operators import Softmax, SwiGLUDecode, SwiGLUPrefill
from oracle import ops

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16


def _verify_matmul(out, a, b, rel_tol, abs_tol, max_error_rate=0.0):
    """``out`` against a @ b under verify_buffer's tolerance, where an element
    may also differ by 2^-16 of its absolute mass sum|a_k b_k|: at the golden's
    scale (|outputs| ~ 1e7), an output that cancels to ~10 carries fp32
    accumulation differences of that order whatever the summation order."""
    ref = a.float() @ b.float()
    mass = a.float().abs() @ b.float().abs()
    o, r, m = out.float().reshape(-1), ref.reshape(-1), mass.reshape(-1)
    bad = ops.verify_buffer(o, r, rel_tol=rel_tol, abs_tol=abs_tol, max_error_rate=max_error_rate)
    bad = [i for i in bad if abs(float(o[i]) - float(r[i])) > 2.0**-16 * float(m[i])]
    assert len(bad) <= max_error_rate * o.numel(), (len(bad), [(i, float(o[i]), float(r[i])) for i in bad[:6]])
    return True


def _verify(out, ref, rel_tol, abs_tol, max_error_rate=0.0):
    """True when verify_buffer (test_utils.py:18-119 semantics) finds no failures."""
    o, r = out.float().reshape(-1), ref.float().reshape(-1)
    bad = ops.verify_buffer(o, r, rel_tol=rel_tol, abs_tol=abs_tol, max_error_rate=max_error_rate)
    assert not bad, (len(bad), [(i, float(o[i]), float(r[i])) for i in bad[:6]])
    return True


@pytest.mark.parametrize("dispatch", ["fused", "separate"])
@pytest.mark.parametrize("embedding_dim,hidden_dim", [(2048, 2048), (1024, 3584)])
def test_swiglu_decode(gpu, embedding_dim, hidden_dim, dispatch):
    golden = ops.swiglu_decode_golden(M=1, K=embedding_dim, N=hidden_dim)
    op = SwiGLUDecode(embedding_dim=embedding_dim, hidden_dim=hidden_dim, dispatch=dispatch)
    op.compile()
    fc = op.get_callable()
    fc.get_buffer("w_gate").torch_view()[:] = golden["w_gate"].T.reshape(-1)
    fc.get_buffer("w_up").torch_view()[:] = golden["w_up"].T.reshape(-1)
    fc.get_buffer("w_down").torch_view()[:] = golden["w_down"].T.reshape(-1)
    for name in ("w_gate", "w_up", "w_down"):
        fc.get_buffer(name).to("npu")
    for call in range(2):  # the second call replays the captured graph
        x = golden["input"] if call == 0 else -golden["input"]
        fc.get_buffer("in").torch_view()[:] = x.reshape(-1)
        fc()
        for name in ("left_swished", "right", "intermediate"):
            fc.get_buffer(name).to("cpu")
        left_swished = fc.get_buffer("left_swished").torch_view().reshape(1, hidden_dim)
        right = fc.get_buffer("right").torch_view().reshape(1, hidden_dim)
        intermediate = fc.get_buffer("intermediate").torch_view().reshape(1, hidden_dim)
        assert _verify(intermediate, left_swished.float() * right.float(), 0.04, 0.4)
        out = fc.get_buffer("out").torch_view().reshape(1, embedding_dim)
        assert _verify_matmul(out, intermediate, golden["w_down"], 0.04, 0.4)
        # and the gate GEMV against the golden chain on this call's input
        left = fc.get_buffer("left").to("cpu").torch_view().reshape(1, hidden_dim)
        assert _verify_matmul(left, x, golden["w_gate"], 0.04, 0.4)


@pytest.mark.parametrize("b_col_maj", [False, True])
def test_swiglu_prefill(gpu, b_col_maj):
    seq_len, embedding_dim, hidden_dim = 256, 2048, 2048
    golden = ops.swiglu_decode_golden(M=seq_len, K=embedding_dim, N=hidden_dim)
    op = SwiGLUPrefill(seq_len=seq_len, embedding_dim=embedding_dim, hidden_dim=hidden_dim, b_col_maj=b_col_maj)
    op.compile()
    fc = op.get_callable()

    def stored(w):
        return (w.t().contiguous() if b_col_maj else w).reshape(-1)

    fc.get_buffer("w_gate").torch_view()[:] = stored(golden["w_gate"])
    fc.get_buffer("w_up").torch_view()[:] = stored(golden["w_up"])
    fc.get_buffer("w_down").torch_view()[:] = stored(golden["w_down"])
    for name in ("w_gate", "w_up", "w_down"):
        fc.get_buffer(name).to("npu")
    fc.get_buffer("in").torch_view()[:] = golden["input"].reshape(-1)
    fc()
    for name in ("left_swished", "right", "intermediate", "out"):
        fc.get_buffer(name).to("cpu")
    ls = fc.get_buffer("left_swished").torch_view().reshape(seq_len, hidden_dim)
    right = fc.get_buffer("right").torch_view().reshape(seq_len, hidden_dim)
    inter = fc.get_buffer("intermediate").torch_view().reshape(seq_len, hidden_dim)
    assert _verify(inter, ls.float() * right.float(), 0.04, 0.4)
    out = fc.get_buffer("out").torch_view().reshape(seq_len, embedding_dim)
    assert _verify_matmul(out, inter, golden["w_down"], 0.08, 0.4, max_error_rate=0.05)


def test_compare_dispatch_checks_every_step(gpu):
    golden = ops.swiglu_decode_golden(M=1, K=1024, N=3584, seed=7)
    op = SwiGLUDecode(embedding_dim=1024, hidden_dim=3584,
                      dispatch=CompareDispatch(tolerance=Tolerance.relative(0.04, 0.4)))
    fc = op.get_callable()
    fc.get_buffer("w_gate").torch_view()[:] = golden["w_gate"].T.reshape(-1)
    fc.get_buffer("w_up").torch_view()[:] = golden["w_up"].T.reshape(-1)
    fc.get_buffer("w_down").torch_view()[:] = golden["w_down"].T.reshape(-1)
    fc.get_buffer("in").torch_view()[:] = golden["input"].reshape(-1)
    fc()
    assert [s["op"] for s in fc.last_step_stats] == ["GEMV", "GEMV", "SiLU", "ElementwiseMul", "GEMV"]
    assert not any(s["mismatch"] for s in fc.last_step_stats)


def test_compare_dispatch_raises_on_mismatch(gpu):
    """A reference that disagrees (planted on the CPU side) is caught."""
    from iron_amd.common import get_reference_provider, set_reference_provider

    prev = get_reference_provider()
    set_reference_provider(lambda op, *xs: prev(op, *xs) + 1.0)
    try:
        sm = Softmax(rows=16, cols=64)
        seq = OperatorSequence("sm", [(sm, "x", "y")], ["x"], ["y"], dispatch="compare")
        fc = seq.get_callable()
        fc.get_buffer("x").torch_view()[:] = torch.randn(16 * 64).to(BF16)
        with pytest.raises(RuntimeError, match="deviates from reference"):
            fc()
    finally:
        set_reference_provider(prev)


def test_runtime_parameter_reaches_captured_graph(gpu):
    """Softmax's runtime vector size as a sequence parameter: params.write +
    sync between replays of the captured graph changes the mask."""
    sm = Softmax(rows=16, cols=128, vector_size_parameter="valid")
    seq = OperatorSequence("smp", [(sm, "x", "y")], ["x"], ["y"], dispatch="fused")
    fc = seq.get_callable()
    x = torch.randn(16, 128).to(BF16)
    fc.get_buffer("x").torch_view()[:] = x.reshape(-1)
    for valid in (128, 40, 77, 128, 1):
        fc.params.write("valid", valid)
        fc()
        y = fc.get_buffer("y").torch_view().reshape(16, 128)
        ref = ops.softmax_reference(x, valid)
        assert ops.max_abs_rel_l2(y, ref)[0] <= 1e-2, valid
        assert float(y[:, valid:].float().abs().max() if valid < 128 else 0.0) == 0.0

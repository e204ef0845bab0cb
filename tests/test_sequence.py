"""OperatorSequence host logic on the CPU: buffer layout (sequence.py:408-547
of the reference), argument checks, and the reference dispatch mode (every
step through reference(), here the oracle provider)."""

import pytest
import torch

from iron_amd.common import OperatorSequence
from iron_amd.common.sequence import ALIGN, CompareDispatch, FusedDispatch, Tolerance
from iron_amd.operators import ElementwiseAdd, ElementwiseMul, GEMV, SiLU, SwiGLUDecode
from oracle import ops

BF16 = torch.bfloat16


def _ops(n=256):
    return (SiLU(size=n, num_aie_columns=1, tile_size=n), ElementwiseMul(size=n, tile_size=n, num_aie_columns=1),
            ElementwiseAdd(size=n, tile_size=n, num_aie_columns=1))


def test_layout_arenas_offsets_and_slices():
    silu, mul, add = _ops()
    seq = OperatorSequence(
        "t",
        runlist=[(silu, "a", "s"), (mul, "s", "b", "m"), (add, "m", "big[0:512]", "out")],
        input_args=["a", "b"],
        output_args=["out"],
        buffer_sizes={"big": 4096},
    )
    layout, sizes, slices = seq.calculate_buffer_layout()
    assert layout["a"] == ("input", 0, 512) and layout["b"] == ("input", ALIGN * 2, 512)
    assert layout["out"] == ("output", 0, 512)
    assert {k for k, v in layout.items() if v[0] == "scratch"} == {"s", "m", "big"}
    assert all(v[1] % ALIGN == 0 for v in layout.values())
    assert sizes[0] == ALIGN * 4 and sizes[1] == ALIGN * 2
    assert slices == {"big[0:512]": ("big", 0, 512)}
    seq.subbuffer_layout, seq.buffer_sizes, seq.slice_info = layout, sizes, slices
    kind, start, end = seq.get_layout_for_buffer("big[0:512]")
    assert kind == "scratch" and start == layout["big"][1] and end == start + 512


def test_layout_errors():
    silu, mul, _ = _ops()
    silu2 = SiLU(size=128, num_aie_columns=1, tile_size=128)
    with pytest.raises(ValueError, match="conflicting sizes"):
        OperatorSequence("t", [(silu, "a", "s"), (silu2, "s", "o")], ["a"], ["o"]).calculate_buffer_layout()
    with pytest.raises(ValueError, match="explicit size"):
        OperatorSequence("t", [(silu, "p[0:512]", "o")], [], ["o"]).calculate_buffer_layout()
    with pytest.raises(ValueError, match="Input argument"):
        OperatorSequence("t", [(silu, "a", "o")], ["zz"], ["o"]).calculate_buffer_layout()
    with pytest.raises(ValueError, match="must match"):
        OperatorSequence("t", [(mul, "a", "o")], ["a"], ["o"]).calculate_buffer_layout()
    with pytest.raises(TypeError):
        OperatorSequence("t", [("notanop", "a")], ["a"], [])
    with pytest.raises(TypeError):
        OperatorSequence("t", [(silu, "a", "o")], ["a"], ["o"], dispatch="nope")
    assert isinstance(OperatorSequence("t", [(silu, "a", "o")], ["a"], ["o"]).dispatch.resolve(None), FusedDispatch)


def test_tolerance_check():
    tol = Tolerance.relative(0.1, 0.01)
    assert tol.check(torch.tensor([1.05, 0.0]), torch.tensor([1.0, 0.005]))[0]
    ok, detail = tol.check(torch.tensor([1.2]), torch.tensor([1.0]))
    assert not ok and "1/1" in detail
    assert CompareDispatch().step_tolerance(_ops()[0]) == CompareDispatch.FALLBACK_TOLERANCE


def test_swiglu_decode_reference_dispatch_matches_golden_chain():
    E, F = 64, 256
    g = ops.swiglu_decode_golden(M=1, K=E, N=F, seed=3)
    op = SwiGLUDecode(embedding_dim=E, hidden_dim=F, dispatch="reference")
    op.compile()
    fc = op.get_callable()
    fc.get_buffer("w_gate").torch_view()[:] = g["w_gate"].T.reshape(-1)
    fc.get_buffer("w_up").torch_view()[:] = g["w_up"].T.reshape(-1)
    fc.get_buffer("w_down").torch_view()[:] = g["w_down"].T.reshape(-1)
    fc.get_buffer("in").torch_view()[:] = g["input"].reshape(-1)
    fc()
    for name, key in (("left", "left"), ("right", "right"), ("left_swished", "left_swished"),
                      ("intermediate", "intermediate"), ("out", "output")):
        got = fc.get_buffer(name).torch_view()
        assert torch.equal(got, g[key].reshape(-1)), name


def test_reference_without_provider_raises():
    from iron_amd.common import get_reference_provider, set_reference_provider

    prev = get_reference_provider()
    set_reference_provider(None)
    try:
        with pytest.raises(NotImplementedError, match="no reference provider"):
            _ops()[0].reference(torch.zeros(256, dtype=BF16))
    finally:
        set_reference_provider(prev)
    assert GEMV(M=8, K=8).reference(torch.ones(8, 8, dtype=BF16), torch.ones(8, dtype=BF16)).float().sum() == 64

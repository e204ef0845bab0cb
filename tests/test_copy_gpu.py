"""GPU: Transpose, Repeat and StridedCopy against the oracle, bit-exact (the
reference's own gate for data movement: rel_tol = abs_tol = 0). Shapes follow
transpose/test.py:14-82, repeat/test.py:20-33 and strided_copy/test.py:14-80,
including the cache_offset runtime parameter of strided_copy/test.py:110-150."""

import pytest
import torch

from iron_amd.common import OperatorSequence
from oracle import ops

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16


@pytest.mark.parametrize("M,N,cols,ch,nb", [(2048, 64, 1, 1, 1), (64, 512, 8, 1, 1), (2048, 64, 1, 2, 1),
                                           (2048, 64, 1, 1, 2), (2048, 64, 1, 1, 4), (8192, 512, 8, 2, 1)])
def test_transpose(gpu, M, N, cols, ch, nb):
    from iron_amd.operators import Transpose

    torch.manual_seed(42)
    x = (torch.rand(nb, M, N) * 4).to(BF16).squeeze(0)
    op = Transpose(M=M, N=N, num_aie_columns=cols, num_channels=ch, m=64, n=64, s=8, num_batches=nb)
    out = torch.empty(nb * N * M, dtype=BF16, device=gpu).reshape((nb, N * M) if nb > 1 else (N * M,))
    op.get_callable()(x.reshape((nb, M * N) if nb > 1 else (M * N,)).to(gpu), out)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu().reshape(-1), ops.transpose_reference(x, M, N).reshape(-1))


@pytest.mark.parametrize("rows,cols,repeat,dtype", [(8, 64, 4, BF16), (8, 512, 4, BF16), (4, 1024, 2, BF16),
                                                   (8, 2048 * 64, 4, BF16), (5, 3, 3, BF16), (7, 9, 2, torch.uint8)])
def test_repeat(gpu, rows, cols, repeat, dtype):
    from iron_amd.operators import Repeat

    torch.manual_seed(42)
    x = (torch.rand(rows, cols) * 4).to(dtype) if dtype != torch.uint8 else torch.randint(0, 255, (rows, cols), dtype=dtype)
    out = torch.empty(rows * repeat, cols, dtype=dtype, device=gpu)
    Repeat(rows=rows, cols=cols, repeat=repeat, dtype=dtype).get_callable()(x.to(gpu), out)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), ops.repeat_reference(x, repeat))


N_KV, HEAD_DIM, SEQ = 8, 64, 128


def _kv_slot(seq, slot, ch=1):
    return dict(input_sizes=[N_KV, HEAD_DIM], input_strides=[HEAD_DIM, 1], input_offset=0,
                input_buffer_size=N_KV * HEAD_DIM, output_sizes=[1, N_KV, HEAD_DIM],
                output_strides=[0, seq * HEAD_DIM, 1], output_offset=slot * HEAD_DIM,
                output_buffer_size=N_KV * seq * HEAD_DIM, num_aie_channels=ch)


def _flat(size, ch=1, transfer_size=None):
    return dict(input_sizes=[size], input_strides=[1], input_offset=0, input_buffer_size=size, output_sizes=[size],
                output_strides=[1], output_offset=0, output_buffer_size=size, num_aie_channels=ch,
                transfer_size=transfer_size)


@pytest.mark.parametrize("kw", [_flat(1024), _flat(1024, 2), _flat(1024, 4), _flat(1024, 2, 256), _kv_slot(SEQ, 0),
                                _kv_slot(SEQ, 5), _kv_slot(SEQ, SEQ - 1), _kv_slot(SEQ, 5, 2), _kv_slot(SEQ, 5, 4),
                                _kv_slot(2048, 1000), _flat(1 << 22, 4, 4096)])
def test_strided_copy(gpu, kw):
    from iron_amd.operators import StridedCopy

    torch.manual_seed(42)
    inp = (torch.rand(int(kw["input_buffer_size"])) * 4).to(BF16)
    prior = torch.randn(int(kw["output_buffer_size"])).to(BF16)
    out = prior.to(gpu)
    StridedCopy(**kw).get_callable()(inp.to(gpu), out)
    torch.cuda.synchronize()
    g = {k: v for k, v in kw.items() if k not in ("transfer_size", "input_buffer_size")}
    ref = ops.strided_copy_reference(inp, **g, out=prior)
    assert torch.equal(out.cpu(), ref)


def test_strided_copy_rejects_out_of_range_pattern(gpu):
    from iron_amd import _lib
    from iron_amd.operators import StridedCopy

    kw = _kv_slot(SEQ, SEQ)  # one slot past the cache
    with pytest.raises(_lib.IronHipError, match="outside"):
        StridedCopy(**kw).get_callable()(torch.zeros(N_KV * HEAD_DIM, dtype=BF16, device=gpu),
                                          torch.zeros(N_KV * SEQ * HEAD_DIM, dtype=BF16, device=gpu))


@pytest.mark.parametrize("dispatch", ["fused", "separate"])
def test_strided_copy_cache_offset_parameter(gpu, dispatch):
    """The whole cache is checked: a mis-scaled addend (elements vs bytes)
    would land the write in another slot."""
    from iron_amd.operators import StridedCopy

    base = _kv_slot(SEQ, 0)
    op = StridedCopy(**base, output_offset_parameter="cache_offset")
    seq = OperatorSequence("sc_cache", [(op, "in", "out")], input_args=["in"], output_args=["out"], dispatch=dispatch)
    run = seq.get_callable()
    out_buf = run.get_buffer("out")
    expected = torch.zeros(base["output_buffer_size"], dtype=BF16)
    out_buf.torch_view()[: expected.numel()] = expected
    out_buf.to("npu")
    for i, slot in enumerate((0, 5, SEQ - 1)):
        torch.manual_seed(i + 1)
        inp = (torch.rand(N_KV * HEAD_DIM) * 4).to(BF16)
        g = {k: v for k, v in base.items() if k != "input_buffer_size"}
        expected = ops.strided_copy_reference(inp, **g, output_offset_addend=slot * HEAD_DIM, out=expected)
        run.get_buffer("in").torch_view()[: inp.numel()] = inp
        run.params.write("cache_offset", slot * HEAD_DIM)
        run.params.sync()
        run()
        got = out_buf.torch_view()[: expected.numel()].clone()
        assert torch.equal(got, expected), f"slot {slot}"

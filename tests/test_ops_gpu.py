"""GPU parity: RMSNorm, SiLU, ElementwiseMul/Add, Softmax, RoPE against the CPU oracle.

Parameter lists follow the reference tests (iron/operators/rms_norm/test.py,
silu/test.py, elementwise_{mul,add}/test.py, softmax/test.py:34-55,
rope/test.py:13-52) with the reference's seeded inputs (seed 42, rand*4) and
its tolerance (rel 0.04 / abs 1e-6; RoPE rel 0.05). Add and Mul round once,
like torch's bf16 ops, and are checked bit-exact.
"""

import pytest
import torch

from oracle import ops

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16
BENCH_ELEMENTS = 1 << 23


def _rand(*shape, seed=42):
    torch.manual_seed(seed)
    return torch.rand(*shape, dtype=BF16) * 4


@pytest.mark.parametrize(
    "size,cols,ch,tile,weighted",
    [(2048, 1, 1, 2048, False), (2048, 2, 1, 1024, True), (4096, 1, 2, 2048, True), (8192, 1, 1, 8192, False),
     (1024, 8, 1, 128, True), (512 * 2048, 1, 1, 2048, True), (BENCH_ELEMENTS, 8, 2, 4096, False)],
)
def test_rms_norm(gpu, size, cols, ch, tile, weighted):
    from iron_amd.operators import RMSNorm

    op = RMSNorm(size=size, num_aie_columns=cols, num_channels=ch, tile_size=tile, weighted=weighted)
    torch.manual_seed(42)
    x = torch.rand(size // tile, tile, dtype=BF16) * 4
    w = torch.rand(tile, dtype=BF16) * 4 if weighted else None
    ref = ops.rms_norm_reference(x, w)
    out = torch.empty_like(x, device=gpu)
    args = [x.to(gpu)] + ([w.to(gpu)] if weighted else []) + [out]
    op.get_callable()(*args)
    torch.cuda.synchronize()
    assert not ops.verify_buffer(out, ref, rel_tol=0.04, abs_tol=1e-6)


def test_rms_norm_residual_fused(gpu):
    """iron_rmsnorm with a residual: sum_out = bf16(x + r), out = RMSNorm(sum_out) * w."""
    from iron_amd import _lib

    torch.manual_seed(7)
    x = torch.randn(512, 2048).to(BF16)
    r = torch.randn(512, 2048).to(BF16)
    w = (1 + 0.1 * torch.randn(2048)).to(BF16)
    s_ref = ops.add_reference(x, r)
    ref = ops.rms_norm_reference(s_ref, w)
    xd, rd, wd = x.to(gpu), r.to(gpu), w.to(gpu)
    out = torch.empty_like(xd)
    _lib.call("iron_rmsnorm", xd.data_ptr(), rd.data_ptr(), wd.data_ptr(), out.data_ptr(), xd.data_ptr(), 512,
              2048, 1e-5, _lib.stream_handle(gpu))
    torch.cuda.synchronize()
    assert torch.equal(xd.cpu(), s_ref)  # sum written in place of x
    assert not ops.verify_buffer(out, ref, rel_tol=0.04, abs_tol=1e-6)


@pytest.mark.parametrize("size,cols,tile", [(2048, 1, 2048), (2048, 8, 256), (8192, 8, 1024), (BENCH_ELEMENTS, 8, 4096)])
def test_silu(gpu, size, cols, tile):
    from iron_amd.operators import SiLU

    x = _rand(size)
    out = torch.empty(size, dtype=BF16, device=gpu)
    SiLU(size=size, num_aie_columns=cols, tile_size=tile).get_callable()(x.to(gpu), out)
    torch.cuda.synchronize()
    assert not ops.verify_buffer(out, ops.silu_reference(x), rel_tol=0.04, abs_tol=1e-6)


@pytest.mark.parametrize("name", ["ElementwiseMul", "ElementwiseAdd"])
@pytest.mark.parametrize("size,cols,tile", [(2048, 1, 2048), (2048, 8, 256), (8192, 4, 2048), (BENCH_ELEMENTS, 8, 4096)])
def test_binary_elementwise_bit_exact(gpu, name, size, cols, tile):
    import iron_amd.operators as O

    torch.manual_seed(42)
    a = torch.rand(size, dtype=BF16) * 4
    b = torch.rand(size, dtype=BF16) * 4
    ref = a * b if name == "ElementwiseMul" else a + b  # torch bf16: fp32 op, one RNE rounding
    out = torch.empty(size, dtype=BF16, device=gpu)
    getattr(O, name)(size=size, tile_size=tile, num_aie_columns=cols).get_callable()(a.to(gpu), b.to(gpu), out)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), ref)


def test_silu_mul_odd_length(gpu):
    from iron_amd import _lib

    torch.manual_seed(8)
    n = 8192 + 5
    g = torch.randn(n).to(BF16)
    u = torch.randn(n).to(BF16)
    gd, ud = g.to(gpu), u.to(gpu)
    out = torch.empty_like(gd)
    _lib.call("iron_silu_mul", gd.data_ptr(), ud.data_ptr(), out.data_ptr(), n, _lib.stream_handle(gpu))
    torch.cuda.synchronize()
    assert not ops.verify_buffer(out, ops.swiglu_reference(g, u), rel_tol=0.04, abs_tol=1e-6)


@pytest.mark.parametrize("rows,cols", [(64, 512), (16, 2048), (4096, 512), (32, 2048), (16, 16384)])
def test_softmax(gpu, rows, cols):
    from iron_amd.operators import Softmax

    x = _rand(rows, cols)
    out = torch.empty(rows * cols, dtype=BF16, device=gpu)
    Softmax(rows=rows, cols=cols).get_callable()(x.to(gpu).flatten(), out)
    torch.cuda.synchronize()
    assert not ops.verify_buffer(out, ops.softmax_reference(x), rel_tol=0.04, abs_tol=1e-6)


@pytest.mark.parametrize("valid", [1, 100, 2047, 2048])
def test_softmax_runtime_mask(gpu, valid):
    """The decode softmax of the reference app: 32 rows x 2048, masked to the context length."""
    from iron_amd.operators import Softmax

    x = _rand(32, 2048)
    out = torch.empty(32 * 2048, dtype=BF16, device=gpu)
    Softmax(rows=32, cols=2048, rtp_vector_size=valid).get_callable()(x.to(gpu).flatten(), out)
    torch.cuda.synchronize()
    ref = ops.softmax_reference(x, valid=valid)
    assert not ops.verify_buffer(out, ref, rel_tol=0.04, abs_tol=1e-6)
    assert torch.all(out.view(32, 2048)[:, valid:].cpu() == 0)


def _rope_params():
    out = []
    for cols_aie in (1, 2, 4, 8):
        for rows in (32, 64):
            for arows in (8, 16, 32):
                for cols in (128, 512):
                    for method in (0, 1):
                        regular = rows == 32 and cols == 512 and arows in (8, 32) and method == 0
                        if regular or cols == 128:
                            out.append((rows, cols, arows, cols_aie, method))
    out.append((4096, 512, 8, 8, 0))
    return out


@pytest.mark.parametrize("rows,cols,arows,cols_aie,method", _rope_params())
def test_rope(gpu, rows, cols, arows, cols_aie, method):
    from iron_amd.operators import RoPE

    x, angles = ops.rope_generate_inputs(rows=rows, cols=cols, context_len=arows)
    out = torch.empty(rows, cols, dtype=BF16, device=gpu)
    RoPE(rows=rows, cols=cols, angle_rows=arows, num_aie_columns=cols_aie, method_type=method).get_callable()(
        x.to(gpu), angles.to(gpu), out)
    torch.cuda.synchronize()
    assert not ops.verify_buffer(out, ops.rope_reference(x, angles, method), rel_tol=0.05, abs_tol=0.0)


def test_rope_fp32_table_llama_decode_shape(gpu):
    """q (32, 64) at one position with the fp32 llama3-scaled table."""
    from iron_amd.operators import RoPE

    torch.manual_seed(9)
    x = torch.randn(32, 64).to(BF16)
    table = ops.rope_angles_table(64, 4096)
    row = table[2047:2048].contiguous()
    out = torch.empty(32, 64, dtype=BF16, device=gpu)
    RoPE(rows=32, cols=64, angle_rows=1).get_callable()(x.to(gpu), row.to(gpu), out)
    torch.cuda.synchronize()
    ref = ops.rope_reference(x, row)
    bad = ops.within_bf16_ulps(out, ops.rope_reference(x, row).float(), n_ulp=1.0)
    assert not bad and torch.allclose(out.cpu().float(), ref.float(), atol=2e-2)


@pytest.mark.parametrize("size,cols,chans,tile", [(2048, 1, 1, 2048), (8192, 8, 2, 1024), (65536, 4, 1, 4096)])
def test_gelu(gpu, size, cols, chans, tile):
    """GELU (tanh form) against the oracle at the reference test's tolerance
    (iron/operators/gelu/test.py:47: relative 0.04, absolute 1e-6), on inputs in
    [-4, 4] (both tails of the tanh)."""
    from iron_amd.operators import GELU

    g = torch.Generator().manual_seed(size + cols)
    x = (torch.rand(size, generator=g) * 8 - 4).to(BF16)
    out = torch.empty(size, dtype=BF16, device=gpu)
    GELU(size=size, num_aie_columns=cols, num_channels=chans, tile_size=tile).get_callable()(x.to(gpu), out)
    torch.cuda.synchronize()
    ref = ops.gelu_tanh(x).to(BF16)
    assert not ops.verify_buffer(out, ref, rel_tol=0.04, abs_tol=1e-6)


@pytest.mark.parametrize("n", [1, 1025, 128256])
def test_argmax_bf16(gpu, n):
    """Greedy argmax over bf16 logits: the first index of the maximum (ties
    planted), the history write at *pos when pos < history_cap, and pos += 1."""
    from iron_amd import _lib

    g = torch.Generator().manual_seed(n)
    x = torch.randn(n, generator=g).to(BF16)
    if n > 1000:
        x[n // 3] = x[n - 1] = 9.0  # tie: the first index wins
    s = _lib.stream_handle(gpu)
    xd = x.to(gpu)
    tok = torch.full((1,), -1, dtype=torch.int32, device=gpu)
    pos = torch.tensor([3], dtype=torch.int32, device=gpu)
    hist = torch.full((8,), -1, dtype=torch.int32, device=gpu)
    _lib.call("iron_argmax_bf16", xd.data_ptr(), n, tok.data_ptr(), pos.data_ptr(), hist.data_ptr(), 8, s)
    torch.cuda.synchronize()
    want = int(torch.argmax(x.float()))
    assert int(tok) == want and (n <= 1000 or want == n // 3)
    assert int(pos) == 4 and int(hist[3]) == want and int((hist != -1).sum()) == 1
    pos.fill_(8)  # at the history capacity: no write, position still advances
    _lib.call("iron_argmax_bf16", xd.data_ptr(), n, tok.data_ptr(), pos.data_ptr(), hist.data_ptr(), 8, s)
    _lib.call("iron_argmax_bf16", xd.data_ptr(), n, tok.data_ptr(), None, None, 0, s)  # token only
    torch.cuda.synchronize()
    assert int(pos) == 9 and int((hist != -1).sum()) == 1 and int(tok) == want

"""GPU parity: GEMV, fused int4 GEMV and Dequant against the CPU oracle.

Shapes follow the reference's own test lists (iron/operators/gemv/test.py:20-43,
:82-101; dequant/test.py:13-55) plus BASELINE configs 1 and 2 at full size.
Tolerances: the reference test's rel 0.04 / abs 1e-3 for its seeded goldens;
BASELINE's max-abs 2e-2 and rel-L2 1e-2 for the configs; bit-exact dequant.
"""

import pytest
import torch

from oracle import configs, ops

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16


def _bits_equal(a, b):
    return torch.equal(a.cpu().contiguous().view(torch.int16), b.cpu().contiguous().view(torch.int16))


@pytest.mark.parametrize(
    "M,K", [(128, 128), (2048, 8192), (8192, 2048), (512, 64), (3072, 2048), (100, 24), (130, 8200)]
)
def test_gemv_reference_golden(gpu, M, K):
    from iron_amd.operators import GEMV

    d = ops.gemv_golden(M=M, K=K)
    op = GEMV(M=M, K=K).compile()
    fn = op.get_callable()
    A, x = d["A"].to(gpu), d["B"].to(gpu)
    y = torch.empty(M, dtype=BF16, device=gpu)
    fn(A.flatten(), x, y)
    torch.cuda.synchronize()
    errs = ops.verify_buffer(y, d["C"], rel_tol=0.04, abs_tol=1e-3)
    assert not errs, f"{len(errs)} mismatches, first {errs[:5]}"


@pytest.mark.parametrize("M,K,B", [(256, 128, 4), (256, 128, 100), (448, 64, 192), (64, 1536, 8), (1024, 1024, 2), (512, 64, 32)])
def test_gemv_batched_golden(gpu, M, K, B):
    from iron_amd.operators import GEMV

    d = ops.gemv_golden_batched(M=M, K=K, num_batches=B)
    fn = GEMV(M=M, K=K, num_batches=B).get_callable()
    y = torch.empty(B, M, dtype=BF16, device=gpu)
    fn(d["A"].to(gpu), d["B"].to(gpu), y)
    torch.cuda.synchronize()
    assert not ops.verify_buffer(y, d["C"], rel_tol=0.04, abs_tol=1e-3)


@pytest.mark.parametrize("M,K", [(128, 128), (2048, 8192), (8192, 2048)])
def test_gemv_gelu_epilogue(gpu, M, K):
    from iron_amd.operators import GEMV

    d = ops.gemv_golden(M=M, K=K)
    ref = ops.gelu_tanh(d["C"].float()).to(BF16)
    fn = GEMV(M=M, K=K, epilogue="gelu").get_callable()
    y = torch.empty(M, dtype=BF16, device=gpu)
    fn(d["A"].to(gpu), d["B"].to(gpu), y)
    torch.cuda.synchronize()
    assert not ops.verify_buffer(y, ref, rel_tol=0.06, abs_tol=2e-2)


def test_config1_gemv_bf16(gpu):
    """2048x8192 bf16, seed 0; max-abs 2e-2 and rel-L2 1e-2
    against the fp32-accumulated reference."""
    from iron_amd.operators import GEMV

    W, x = configs.cfg1_gemv_bf16()
    ref = ops.gemv_reference(W, x, out_dtype=torch.float32)
    y = torch.empty(2048, dtype=BF16, device=gpu)
    GEMV(M=2048, K=8192).get_callable()(W.to(gpu), x.to(gpu), y)
    torch.cuda.synchronize()
    max_abs, rel_l2 = ops.max_abs_rel_l2(y, ref)
    assert max_abs <= 2e-2 and rel_l2 <= 1e-2, (max_abs, rel_l2)


@pytest.mark.parametrize("M,K", [(8192, 2048), (2048, 8192), (512, 2048), (2048, 2048), (64, 4096), (96, 8448), (8, 32)])
def test_gemv_int4(gpu, M, K):
    """Fused int4-g32 GEMV. Config 2 (8192x2048) is held to the BASELINE bar,
    max-abs 2e-2 / rel-L2 1e-2 against GEMV(Dequant()) accumulated in fp32.
    Every shape is also held to one bf16 ulp of the exact value
    sum(q*s*x) (float64): the kernel applies the group scale to the exact
    integer codes, so it need not reproduce the bf16 rounding of the weights."""
    from iron_amd.operators import GEMVInt4

    codes, scales, x = configs.cfg2_gemv_int4(M=M, K=K)
    ref = ops.gemv_int4_reference(codes, scales, x, out_dtype=torch.float32)
    exact = ops.gemv_int4_exact(codes, scales, x)
    y = torch.empty(M, dtype=BF16, device=gpu)
    GEMVInt4(M=M, K=K).get_callable()(codes.to(gpu), scales.to(gpu), x.to(gpu), y)
    torch.cuda.synchronize()
    max_abs, rel_l2 = ops.max_abs_rel_l2(y, ref)
    assert rel_l2 <= 1e-2, rel_l2
    if (M, K) == (8192, 2048):
        assert max_abs <= 2e-2, max_abs
    bad = ops.within_bf16_ulps(y, exact, n_ulp=1.0, atol=1e-5 * float(exact.abs().max()))
    assert not bad, [(i, float(y[i]), float(exact[i])) for i in bad[:5]]


def test_gemv_int4_unsigned(gpu):
    from iron_amd.operators import GEMVInt4

    g = torch.Generator().manual_seed(5)
    M, K = 256, 2048
    q = torch.randint(0, 16, (M, K), generator=g, dtype=torch.int16)
    codes = ops.pack_int4(q)
    scales = (0.001 + 0.009 * torch.rand(M, K // 32, generator=g)).to(BF16)
    x = torch.randn(K, generator=g).to(BF16)
    ref = ops.gemv_int4_reference(codes, scales, x, signed=False, out_dtype=torch.float32)
    y = torch.empty(M, dtype=BF16, device=gpu)
    GEMVInt4(M=M, K=K, signed=False).get_callable()(codes.to(gpu), scales.to(gpu), x.to(gpu), y)
    torch.cuda.synchronize()
    max_abs, rel_l2 = ops.max_abs_rel_l2(y, ref)
    assert max_abs <= 2e-2 and rel_l2 <= 1e-2, (max_abs, rel_l2)


@pytest.mark.parametrize("N,K,group,signed", [(8192, 2048, 32, True), (2048, 8192, 32, True), (64, 256, 64, False), (3, 40, 8, True)])
def test_dequant_planar_bit_exact(gpu, N, K, group, signed):
    from iron_amd import _lib

    g = torch.Generator().manual_seed(N + K)
    lo, hi = (-8, 8) if signed else (0, 16)
    q = torch.randint(lo, hi, (N, K), generator=g, dtype=torch.int16)
    codes = ops.pack_int4(q)
    scales = (0.001 + 0.009 * torch.rand(N, K // group, generator=g)).to(BF16)
    out = torch.empty(N, K, dtype=BF16, device=gpu)
    c, s = codes.to(gpu), scales.to(gpu)
    _lib.call("iron_dequant_i4", c.data_ptr(), s.data_ptr(), out.data_ptr(), N, K, group, int(signed),
              _lib.stream_handle(gpu))
    torch.cuda.synchronize()
    assert _bits_equal(out, ops.dequant_planar(codes, scales, group, signed))


def _dequant_params():
    out = []
    for n in (1024, 2048, 4096, 8192):
        for cols in range(1, 9):
            for ch in (1, 2):
                cores = cols * ch
                tile = min(n // cores, 16384)
                if tile * cores == n:
                    out.append((n, cols, ch, tile))
    out.append((1 << 23, 8, 2, 4096))
    return out


@pytest.mark.parametrize("n,cols,ch,tile", _dequant_params()[::5] + [(1 << 23, 8, 2, 4096)])
def test_dequant_payload_bit_exact(gpu, n, cols, ch, tile):
    """The reference Dequant test matrix (dequant/test.py:13-55), sampled."""
    from iron_amd.operators import Dequant

    payload = ops.dequant_generate_inputs(n, tile, 32)
    ref = ops.dequant_payload_reference(payload, tile, 32)
    op = Dequant(size=n, num_aie_columns=cols, num_channels=ch, tile_size=tile)
    out = torch.empty(n, dtype=BF16, device=gpu)
    op.get_callable()(payload.to(gpu), out)
    torch.cuda.synchronize()
    assert _bits_equal(out, ref)

"""GPU parity: GEMM and flm.GEMM (bf16 MFMA) against the CPU oracle.

Shapes and layouts follow the reference tests: iron/operators/gemm/test.py
(regular list; rel/abs 0.005) and iron/operators/flm/gemm/test.py:54-113 (NPU2
list; abs bound 0.004 * K * mean|a| * mean|b|, rel 0.04; activation inputs
scaled by 0.5), plus the Llama prefill shapes of BASELINE config 5.
"""

import pytest
import torch

from oracle import ops

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16


@pytest.mark.parametrize(
    "M,K,N,b_col_maj,c_col_maj",
    [
        (2048, 2048, 2048, False, False),
        (2048, 2048, 2048, True, False),
        (2048, 2048, 2048, True, True),
        (384, 1536, 1792, True, False),
        (1792, 896, 1152, False, True),
        (896, 1792, 640, False, True),
        (192, 384, 64, False, False),
        (192, 384, 64, True, True),
        (64, 512, 256, True, False),
        (2048, 64, 8192, False, False),
        (100, 192, 130, True, False),
    ],
)
def test_gemm(gpu, M, K, N, b_col_maj, c_col_maj):
    from iron_amd.operators import GEMM

    g = ops.gemm_golden(M, K, N, b_col_maj=b_col_maj)
    ref = g["output"].T.contiguous() if c_col_maj else g["output"]
    op = GEMM(M=M, K=K, N=N, b_col_maj=b_col_maj, c_col_maj=c_col_maj)
    C = torch.empty(ref.shape, dtype=BF16, device=gpu)
    op.get_callable()(g["input"].to(gpu), g["input_b"].to(gpu), C)
    torch.cuda.synchronize()
    errs = ops.verify_buffer(C, ref, rel_tol=0.005, abs_tol=0.005)
    assert not errs, f"{len(errs)} mismatches of {ref.numel()}"


FLM = [
    (256, 512, 1024, "none", None),
    (512, 1024, 2048, "none", None),
    (256, 512, 1536, "none", None),
    (256, 512, 128, "none", None),
    (256, 512, 1024, "silu", None),
    (256, 512, 1024, "gelu", None),
    (256, 512, 1024, "none", (-2.0, 2.0)),
    (1024, 2048, 2048, "none", None),
    (1024, 2560, 2560, "none", None),
    (512, 1536, 1536, "silu", None),
    (256, 512, 1024, "sigmoid", None),
    (512, 1024, 2048, "silu", (-4.0, 4.0)),
    (1024, 1536, 6144, "none", None),
    (1024, 2560, 10240, "none", None),
    (1000, 576, 1500, "silu", (-3.0, 3.0)),  # 128x64 tiles, ragged in M and N
]


@pytest.mark.parametrize("M,K,N,epilogue,clamp", FLM)
def test_flm_gemm(gpu, M, K, N, epilogue, clamp):
    from iron_amd.operators import flm

    scale = 4.0 if epilogue == "none" else 0.5
    g = ops.flm_gemm_golden(M, K, N, epilogue=epilogue, clamp=clamp, scale=scale)
    op = flm.GEMM(M=M, K=K, N=N, epilogue=epilogue, clamp=clamp)
    C = torch.empty(M, N, dtype=BF16, device=gpu)
    op.get_callable()(g["input"].to(gpu), op.pack_B(g["input_b"]).to(gpu), C)
    torch.cuda.synchronize()
    mass = K * g["input"].abs().float().mean() * g["input_b"].abs().float().mean()
    errs = ops.verify_buffer(C, g["output"], rel_tol=0.04, abs_tol=float(0.004 * mass))
    assert not errs, f"{len(errs)} mismatches"


@pytest.mark.parametrize("M,K,N", [(512, 2048, 2048), (512, 2048, 512), (512, 2048, 8192), (512, 8192, 2048),
                                   (13, 2048, 3072), (512, 2048, 3072), (1000, 576, 1500)])
def test_prefill_gemm_shapes(gpu, M, K, N):
    """Config 5 prefill projections (A activations, B = nn.Linear weight (N, K)), fp32-accumulated
    reference; BASELINE bar max-abs 2e-2 / rel-L2 1e-2 on N(0,1) activations x N(0,0.02^2) weights."""
    from iron_amd import _lib

    gen = torch.Generator().manual_seed(M + K + N)
    A = torch.randn(M, K, generator=gen).to(BF16)
    W = (torch.randn(N, K, generator=gen) * 0.02).to(BF16)
    ref = A.float() @ W.float().T
    Ad, Wd = A.to(gpu), W.to(gpu)
    C = torch.empty(M, N, dtype=BF16, device=gpu)
    _lib.call("iron_gemm_bf16_nt", Ad.data_ptr(), Wd.data_ptr(), C.data_ptr(), M, N, K, N, 0, 0, 0.0, 0.0,
              _lib.stream_handle(gpu))
    torch.cuda.synchronize()
    max_abs, rel_l2 = ops.max_abs_rel_l2(C, ref)
    assert rel_l2 <= 1e-2
    bad = ops.within_bf16_ulps(C, ref, n_ulp=1.0, atol=1e-5 * float(ref.abs().max()))
    assert not bad, bad[:5]


@pytest.mark.parametrize(
    "M,K,N",
    [
        (4000, 128, 4104),  # 256x256 tiles, ragged M and N
        (4096, 256, 4100),  # 256x256 tiles, odd row stride: element stores
        (3968, 2048, 2048),  # 256x128 tiles (prefill o_proj at 3968 tokens)
        (3968, 256, 3072),  # 256x192 tiles (prefill qkv at 3968 tokens), ragged M
        (3000, 64, 3072),  # 256x192 tiles, ragged M (184 rows in the last tile row)
        (2600, 64, 3300),  # 256x128 tiles, ragged, odd row stride
        (1280, 192, 4096),  # 128x128 tiles, more workgroups than CUs
        (1000, 192, 2050),  # 128x128 tiles, one workgroup per CU, ragged
    ],
)
def test_gemm_tile_shapes(gpu, M, K, N):
    """Each tile shape the launcher picks (by tile count), at ragged edges
    (rows past M or N load the last row; their outputs are never stored):
    within one bf16 ulp of the fp32-accumulated product."""
    from iron_amd import _lib

    gen = torch.Generator().manual_seed(M * 7 + K + N)
    A = torch.randn(M, K, generator=gen).to(BF16)
    W = (torch.randn(N, K, generator=gen) * 0.05).to(BF16)
    ref = A.float() @ W.float().T
    C = torch.full((M, N), float("nan"), dtype=BF16, device=gpu)
    Ad, Wd = A.to(gpu), W.to(gpu)  # held until the launch has run
    _lib.call("iron_gemm_bf16_nt", Ad.data_ptr(), Wd.data_ptr(), C.data_ptr(), M, N, K, N, 0, 0, 0.0, 0.0,
              _lib.stream_handle(gpu))
    torch.cuda.synchronize()
    assert not torch.isnan(C).any()
    bad = ops.within_bf16_ulps(C, ref, n_ulp=1.0, atol=1e-5 * float(ref.abs().max()))
    assert not bad, bad[:5]


@pytest.mark.parametrize("M,K,N,splits", [(512, 8192, 2048, 4), (512, 2048, 2048, 4), (512, 2048, 3072, 2),
                                          (100, 512, 200, 2), (100, 512, 203, 2), (256, 1024, 384, 8),
                                          (64, 4096, 64, 8)])
@pytest.mark.parametrize("epi,clamp", [(0, False), (2, False), (4, True)])
def test_gemm_splitk(gpu, M, K, N, splits, epi, clamp):
    """Split-K GEMM (fp32 partials + ordered merge) against the fp32 reference
    with the flm epilogue order (round to bf16, activation, clamp), and (with
    no epilogue) against the single-pass kernel: within one bf16 ulp of it."""
    from iron_amd import _lib

    g = torch.Generator().manual_seed(M + K + N + splits)
    A = (torch.randn(M, K, generator=g) * 0.5).to(BF16)
    W = (torch.randn(N, K, generator=g) * 0.5).to(BF16)
    s = _lib.stream_handle(gpu)
    Ad, Wd = A.to(gpu), W.to(gpu)
    C1 = torch.empty(M, N, dtype=BF16, device=gpu)
    C2 = torch.empty(M, N, dtype=BF16, device=gpu)
    lo, hi = (-1.5, 2.0) if clamp else (0.0, 0.0)
    need = int(_lib.query("iron_gemm_splitk_workspace_bytes", M, N, splits))
    ws = torch.empty(need, dtype=torch.uint8, device=gpu)
    _lib.call("iron_gemm_bf16_nt_splitk", Ad.data_ptr(), Wd.data_ptr(), C1.data_ptr(), M, N, K, N, epi, int(clamp),
              lo, hi, splits, ws.data_ptr(), need, s)
    _lib.call("iron_gemm_bf16_nt", Ad.data_ptr(), Wd.data_ptr(), C2.data_ptr(), M, N, K, N, epi, int(clamp), lo, hi, s)
    torch.cuda.synchronize()
    names = {0: "none", 2: "silu", 4: "gelu"}
    ref = ops.flm_apply_epilogue((A.float() @ W.float().T).to(BF16), names[epi], (lo, hi) if clamp else None)
    mass = (A.float().abs() @ W.float().abs().T)
    err = (C1.cpu().float() - ref.float()).abs()
    assert torch.all(err <= 2.0**-7 * ref.float().abs() + 2.0**-12 * mass + 1e-3), float(err.max())
    if epi == 0 and not clamp:  # an activation can stretch a 1-ulp input flip past one output ulp
        assert not ops.within_bf16_ulps(C1.cpu(), C2.cpu().float(), n_ulp=1.0, atol=2.0**-14 * float(mass.max()))


def test_gemm_splitk_choice_and_errors(gpu):
    from iron_amd import _lib

    # bf16: a short K is split only when the plain kernel's 64x64 / 128x64 tiles leave CUs idle
    assert _lib.query("iron_gemm_splitk_choose", 512, 2048, 8192) == 4
    assert _lib.query("iron_gemm_splitk_choose", 128, 2048, 8192) == 8
    assert _lib.query("iron_gemm_splitk_choose", 2048, 2048, 8192) == 2
    assert _lib.query("iron_gemm_splitk_choose", 512, 2048, 2048) == 1  # 256 tiles of 64x64
    assert _lib.query("iron_gemm_splitk_choose", 512, 3072, 2048) == 2  # 192 tiles of 128x64
    assert _lib.query("iron_gemm_splitk_choose", 512, 8192, 2048) == 1
    assert _lib.query("iron_gemm_splitk_choose", 4096, 4096, 4096) == 1
    # int4-g32: 128x128 tiles or larger, so shorter K is split too
    assert _lib.query("iron_gemm_i4g32_splitk_choose", 512, 2048, 2048) == 4
    assert _lib.query("iron_gemm_i4g32_splitk_choose", 512, 3072, 2048) == 2
    assert _lib.query("iron_gemm_i4g32_splitk_choose", 512, 2048, 8192) == 4
    assert _lib.query("iron_gemm_i4g32_splitk_choose", 512, 8192, 2048) == 1  # 256 tiles already fill the GPU
    A = torch.zeros(128, 192, dtype=BF16, device=gpu)
    C = torch.zeros(128, 128, dtype=BF16, device=gpu)
    with pytest.raises(_lib.IronHipError, match="must divide"):
        _lib.call("iron_gemm_bf16_nt_splitk", A.data_ptr(), A.data_ptr(), C.data_ptr(), 128, 128, 192, 128, 0, 0,
                  0.0, 0.0, 2, C.data_ptr(), C.numel() * 2, _lib.stream_handle(gpu))
    with pytest.raises(_lib.IronHipError, match="workspace"):
        _lib.call("iron_gemm_bf16_nt_splitk", A.data_ptr(), A.data_ptr(), C.data_ptr(), 128, 128, 192, 128, 0, 0,
                  0.0, 0.0, 3, C.data_ptr(), 16, _lib.stream_handle(gpu))


@pytest.mark.parametrize(
    "M,K,N,signed",
    [
        (512, 2048, 8192, True),  # config 5 gate/up shape: 128x128 tiles, one per CU
        (512, 2048, 3072, True),  # qkv
        (512, 2048, 2048, True),  # o_proj: split K (64 tiles)
        (512, 8192, 2048, True),  # down_proj: split K
        (3968, 2048, 3072, True),  # long prompt: 256x128 tiles
        (200, 320, 1000, False),  # ragged M and N, unsigned codes
        (1, 64, 64, True),  # smallest shape
    ],
)
def test_gemm_i4g32_matches_bf16_on_dequantized(gpu, M, K, N, signed):
    """iron_gemm_i4g32_nt dequantizes in its prologue: the result must be
    bit-identical to iron_gemm_bf16_nt on the oracle's dequantized weights
    (bf16(q*s), bit-exact) with the same split count, and within one bf16 ulp
    of the fp32-accumulated product."""
    from iron_amd import _lib

    gen = torch.Generator().manual_seed(M + K + N + int(signed))
    lo, hi = (-8, 8) if signed else (0, 16)
    q = torch.randint(lo, hi, (N, K), generator=gen, dtype=torch.int16)
    codes = ops.pack_int4(q)
    scales = (0.001 + 0.009 * torch.rand(N, K // 32, generator=gen)).to(BF16)
    A = torch.randn(M, K, generator=gen).to(BF16)
    W = ops.dequant_planar(codes, scales, signed=signed)
    s = _lib.stream_handle(gpu)
    splits = _lib.query("iron_gemm_i4g32_splitk_choose", M, N, K)
    need = int(_lib.query("iron_gemm_splitk_workspace_bytes", M, N, splits))
    ws = torch.empty(max(need, 16), dtype=torch.uint8, device=gpu)
    Ad, Wd, cd, sd = A.to(gpu), W.to(gpu), codes.to(gpu), scales.to(gpu)
    C4 = torch.full((M, N), float("nan"), dtype=BF16, device=gpu)
    Cb = torch.empty(M, N, dtype=BF16, device=gpu)
    _lib.call("iron_gemm_i4g32_nt", Ad.data_ptr(), cd.data_ptr(), sd.data_ptr(), C4.data_ptr(), M, N, K, N, 0, 0,
              0.0, 0.0, int(signed), splits, ws.data_ptr(), need, s)
    if splits > 1:
        _lib.call("iron_gemm_bf16_nt_splitk", Ad.data_ptr(), Wd.data_ptr(), Cb.data_ptr(), M, N, K, N, 0, 0, 0.0, 0.0,
                  splits, ws.data_ptr(), need, s)
    else:
        _lib.call("iron_gemm_bf16_nt", Ad.data_ptr(), Wd.data_ptr(), Cb.data_ptr(), M, N, K, N, 0, 0, 0.0, 0.0, s)
    torch.cuda.synchronize()
    assert torch.equal(C4.cpu().view(torch.int16), Cb.cpu().view(torch.int16))
    ref = A.float() @ W.float().T
    bad = ops.within_bf16_ulps(C4, ref, n_ulp=1.0, atol=1e-5 * float(ref.abs().max()))
    assert not bad, bad[:5]


def test_gemm_int4_operator_epilogue_and_errors(gpu):
    """GEMMInt4 operator (arg order A, codes, scales, C) against the GEMM
    operator and the split-K bf16 GEMM on the dequantized weights (both
    policies split this K in 2 ranges: bit-identical); the flm epilogue path
    of the C ABI; argument checks."""
    from iron_amd import _lib
    from iron_amd.operators import GEMM, GEMMInt4

    M, K, N = 256, 1024, 768
    gen = torch.Generator().manual_seed(7)
    q = torch.randint(-8, 8, (N, K), generator=gen, dtype=torch.int16)
    codes, scales = ops.pack_int4(q), (0.001 + 0.009 * torch.rand(N, K // 32, generator=gen)).to(BF16)
    A = torch.randn(M, K, generator=gen).to(BF16)
    W = ops.dequant_planar(codes, scales)
    Ad, Wd, cd, sd = A.to(gpu), W.to(gpu), codes.to(gpu), scales.to(gpu)
    C4 = torch.empty(M, N, dtype=BF16, device=gpu)
    Cb = torch.empty(M, N, dtype=BF16, device=gpu)
    Cs = torch.empty(M, N, dtype=BF16, device=gpu)
    s = _lib.stream_handle(gpu)
    splits = _lib.query("iron_gemm_i4g32_splitk_choose", M, N, K)
    assert splits == 2 and _lib.query("iron_gemm_splitk_choose", M, N, K) == 2  # 48 tiles of 64x64
    need = int(_lib.query("iron_gemm_splitk_workspace_bytes", M, N, splits))
    ws = torch.empty(need, dtype=torch.uint8, device=gpu)
    GEMMInt4(M=M, K=K, N=N).get_callable()(Ad, cd, sd, C4)
    GEMM(M=M, K=K, N=N, b_col_maj=True).get_callable()(Ad, Wd, Cb)
    _lib.call("iron_gemm_bf16_nt_splitk", Ad.data_ptr(), Wd.data_ptr(), Cs.data_ptr(), M, N, K, N, 0, 0, 0.0, 0.0,
              splits, ws.data_ptr(), need, s)
    torch.cuda.synchronize()
    assert torch.equal(C4.cpu().view(torch.int16), Cs.cpu().view(torch.int16))
    assert torch.equal(C4.cpu().view(torch.int16), Cb.cpu().view(torch.int16))
    _lib.call("iron_gemm_i4g32_nt", Ad.data_ptr(), cd.data_ptr(), sd.data_ptr(), C4.data_ptr(), M, N, K, N, 2, 1,
              -1.0, 1.5, 1, 1, None, 0, s)
    _lib.call("iron_gemm_bf16_nt", Ad.data_ptr(), Wd.data_ptr(), Cb.data_ptr(), M, N, K, N, 2, 1, -1.0, 1.5, s)
    torch.cuda.synchronize()
    assert torch.equal(C4.cpu().view(torch.int16), Cb.cpu().view(torch.int16))
    with pytest.raises(RuntimeError, match="multiple of 64"):
        _lib.call("iron_gemm_i4g32_nt", Ad.data_ptr(), cd.data_ptr(), sd.data_ptr(), C4.data_ptr(), M, N, 96, N, 0,
                  0, 0.0, 0.0, 1, 1, None, 0, s)
    with pytest.raises(RuntimeError, match="workspace"):
        _lib.call("iron_gemm_i4g32_nt", Ad.data_ptr(), cd.data_ptr(), sd.data_ptr(), C4.data_ptr(), M, N, K, N, 0, 0,
                  0.0, 0.0, 1, 2, None, 0, s)
    with pytest.raises(ValueError):
        GEMMInt4(M=M, K=96, N=N)


def _interleave_gate_up(Wg, Wu):
    F, K = Wg.shape
    return torch.stack([Wg.view(F // 64, 64, K), Wu.view(F // 64, 64, K)], dim=1).reshape(2 * F, K).contiguous()


@pytest.mark.parametrize("M,K,F", [(512, 2048, 8192), (3968, 2048, 8192), (100, 256, 320), (1, 64, 64)])
def test_gemm_swiglu_matches_unfused(gpu, M, K, F):
    """iron_gemm_bf16_nt_swiglu over the 64-row interleaved [gate; up] weight
    is bit-identical to gate GEMM + up GEMM + iron_silu_mul, and within the
    BASELINE bar of the fp32 SwiGLU."""
    from iron_amd import _lib

    gen = torch.Generator().manual_seed(M + K + F)
    A = torch.randn(M, K, generator=gen).to(BF16)
    Wg = (torch.randn(F, K, generator=gen) * 0.02).to(BF16)
    Wu = (torch.randn(F, K, generator=gen) * 0.02).to(BF16)
    Ad, Wgd, Wud = A.to(gpu), Wg.to(gpu), Wu.to(gpu)
    Wgu = _interleave_gate_up(Wgd, Wud)
    s = _lib.stream_handle(gpu)
    H = torch.full((M, F), float("nan"), dtype=BF16, device=gpu)
    G = torch.empty(M, F, dtype=BF16, device=gpu)
    U = torch.empty(M, F, dtype=BF16, device=gpu)
    _lib.call("iron_gemm_bf16_nt_swiglu", Ad.data_ptr(), Wgu.data_ptr(), H.data_ptr(), M, F, K, F, s)
    _lib.call("iron_gemm_bf16_nt", Ad.data_ptr(), Wgd.data_ptr(), G.data_ptr(), M, F, K, F, 0, 0, 0.0, 0.0, s)
    _lib.call("iron_gemm_bf16_nt", Ad.data_ptr(), Wud.data_ptr(), U.data_ptr(), M, F, K, F, 0, 0, 0.0, 0.0, s)
    _lib.call("iron_silu_mul", G.data_ptr(), U.data_ptr(), G.data_ptr(), M * F, s)
    torch.cuda.synchronize()
    assert torch.equal(H.cpu().view(torch.int16), G.cpu().view(torch.int16))
    ref = torch.nn.functional.silu(A.float() @ Wg.float().T) * (A.float() @ Wu.float().T)
    max_abs, rel_l2 = ops.max_abs_rel_l2(H, ref)
    assert rel_l2 <= 1e-2 and max_abs <= 2e-2 * max(1.0, float(ref.abs().max())), (max_abs, rel_l2)
    with pytest.raises(RuntimeError, match="multiple of 64"):
        _lib.call("iron_gemm_bf16_nt_swiglu", Ad.data_ptr(), Wgu.data_ptr(), H.data_ptr(), M, F + 32, K, F + 32, s)


@pytest.mark.parametrize("M,K,N,epilogue,clamp", [(256, 512, 1024, "none", None), (256, 512, 1024, "silu", None),
                                                  (64, 2048, 512, "none", (-50.0, 50.0)), (512, 2048, 2048, "gelu", None)])
def test_flm_gemm_floor_rounding(gpu, M, K, N, epilogue, clamp):
    """flm.GEMM(rounding="floor") (flm/gemm/op.py:105,426-430; the reference's
    test list carries it at 256x512x1024): every output-stage conversion
    truncates. Against the oracle's truncating golden within one bf16 ulp (the
    fp32 sums differ in order, so a value next to a boundary may land one ulp
    apart), and against the same GEMM with round-to-nearest: never larger in
    magnitude, different in a large share of the elements. The last shape
    splits K (the merge kernel's conversions)."""
    from iron_amd.operators import flm

    scale = 4.0 if epilogue == "none" else 0.5
    g = ops.flm_gemm_golden(M, K, N, epilogue=epilogue, clamp=clamp, scale=scale, rounding="floor")
    outs = {}
    for rnd in ("conv_even", "floor"):
        op = flm.GEMM(M=M, K=K, N=N, epilogue=epilogue, clamp=clamp, rounding=rnd)
        C = torch.empty(M, N, dtype=BF16, device=gpu)
        op.get_callable()(g["input"].to(gpu), op.pack_B(g["input_b"]).to(gpu), C)
        torch.cuda.synchronize()
        outs[rnd] = C.cpu().float()
    fl, rne = outs["floor"], outs["conv_even"]
    if epilogue == "none" and clamp is None:
        assert torch.all(fl.abs() <= rne.abs())
        assert (fl != rne).float().mean() > 0.2
    else:
        assert (fl != rne).float().mean() > 0.05
    if epilogue == "none":
        bad = ops.within_bf16_ulps(fl.to(BF16), g["output"].float(), n_ulp=1.0, atol=1e-6)
    else:
        # the fp32 accumulators differ by the summation order (up to ~2^-20 of the
        # element's mass sum |a||b|, which dominates where the sum cancels to near
        # zero), so the first conversion may land one ulp of the accumulator or
        # that much apart; the activation (slope <= 1.13 for silu and
        # x*sigmoid(1.702x)) carries it into the output, truncated once more
        acc = g["input"].float() @ g["input_b"].float()
        mass = g["input"].float().abs() @ g["input_b"].float().abs()
        d = (fl - g["output"].float()).abs().reshape(-1)
        allowed = (1.2 * (ops.bf16_ulp(acc) + 2.0**-20 * mass.double()) + ops.bf16_ulp(g["output"].float()))
        allowed = allowed.reshape(-1).float()
        bad = torch.nonzero(d > allowed).flatten().tolist()
        detail = [(i, float(fl.reshape(-1)[i]), float(g["output"].float().reshape(-1)[i]), float(acc.reshape(-1)[i]),
                   float(rne.reshape(-1)[i])) for i in bad[:5]]
        assert not bad, detail
    assert not bad, bad[:5]

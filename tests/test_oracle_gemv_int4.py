"""Pins for the oracle's GEMV and int4 functions (CPU only).

Each check is independent of the oracle's own formula: float64 brute force,
exact rational rounding, round trips, and a literal loop restatement of the
reference packer (iron/operators/dequant/reference.py:77-92).
"""

from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import ops

BF16 = torch.bfloat16


def bf16_ulp(v: float) -> float:
    if v == 0:
        return 2.0**-133
    e = np.floor(np.log2(abs(v)))
    return 2.0 ** (e - 7)


@pytest.mark.parametrize("M,K", [(1, 8), (7, 64), (33, 96), (64, 512)])
def test_gemv_reference_matches_float64(M, K):
    g = torch.Generator().manual_seed(M * 1000 + K)
    A = (torch.randn(M, K, generator=g) * 4).to(BF16)
    x = (torch.randn(K, generator=g) * 4).to(BF16)
    y = ops.gemv_reference(A, x).double().numpy()
    exact = A.double().numpy() @ x.double().numpy()
    for a, b in zip(y, exact):
        assert abs(a - b) <= bf16_ulp(b) * 0.5 + 1e-3 * abs(b) * 2**-8 + 1e-12, (a, b)


def test_gemv_reference_batched_is_per_batch():
    d = ops.gemv_golden_batched(M=16, K=32, num_batches=3)
    for b in range(3):
        ref = (d["A"][b].double() @ d["B"][b].double())
        assert torch.allclose(d["C"][b].double(), ref, rtol=2**-7, atol=1e-6)


def test_gelu_tanh_matches_torch():
    x = torch.linspace(-6, 6, 1001)
    assert torch.allclose(ops.gelu_tanh(x), torch.nn.functional.gelu(x, approximate="tanh"), atol=2e-6)


def test_pack_unpack_round_trip_all_nibble_pairs():
    q = torch.tensor([[a, b] for a in range(-8, 8) for b in range(-8, 8)], dtype=torch.int16).reshape(1, -1)
    codes = ops.pack_int4(q)
    assert codes.dtype == torch.uint8 and codes.shape == (1, 256)
    assert sorted(codes.flatten().tolist()) == list(range(256))
    assert torch.equal(ops.unpack_int4(codes, signed=True), q)
    # low nibble is the even element
    assert ops.pack_int4(torch.tensor([[1, 2]], dtype=torch.int16)).item() == 0x21
    assert ops.pack_int4(torch.tensor([[-1, 0]], dtype=torch.int16)).item() == 0x0F
    u = ops.unpack_int4(torch.arange(256, dtype=torch.uint8).reshape(1, -1), signed=False)
    assert u.min() == 0 and u.max() == 15


def _exact_bf16_rne(value: Fraction) -> float:
    """Nearest bf16 to an exact rational, ties to even (independent of torch)."""
    if value == 0:
        return 0.0
    sign = -1 if value < 0 else 1
    v = abs(value)
    e = 0
    while v >= 2:
        v /= 2
        e += 1
    while v < 1:
        v *= 2
        e -= 1
    # v in [1,2): 7 fraction bits
    scaled = v * 128
    lo = int(scaled)
    rem = scaled - lo
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and lo % 2 == 1):
        lo += 1
    return sign * lo / 128 * 2.0**e


def test_dequant_is_exact_rne_of_exact_product():
    # every code against a spread of finite bf16 scales (normal range, both signs)
    rng = np.random.default_rng(0)
    bits = rng.integers(0x0080, 0x7E00, size=1500).astype(np.int64)
    bits = np.concatenate([bits, bits | 0x8000, [0x3F80, 0x3C23, 0x3A83, 0x7DFF]])
    scales = torch.from_numpy(bits.astype(np.int16)).view(BF16)
    q = torch.arange(-8, 8, dtype=torch.int16)
    codes = ops.pack_int4(q.repeat(len(scales), 1))  # (S, 8)
    out = ops.dequant_planar(codes, scales.reshape(-1, 1), group=16, signed=True)
    for i, s in enumerate(scales.tolist()):
        for j, qq in enumerate(range(-8, 8)):
            expect = _exact_bf16_rne(Fraction(qq) * Fraction(s))
            assert out[i, j].item() == expect, (qq, s, out[i, j].item(), expect)


def test_dequant_unsigned_codes():
    codes = torch.tensor([[0xF0, 0x21]], dtype=torch.uint8)
    s = torch.tensor([[0.5]], dtype=BF16)
    out = ops.dequant_planar(codes, s, group=4, signed=False)
    assert out.float().tolist() == [[0.0, 7.5, 0.5, 1.0]]


def _payload_loops(A_int, scales, num_tiles, nsf, group):
    """Literal loop form of dequant/reference.py:77-92."""
    per_tile = nsf * group // 2
    out = torch.zeros(num_tiles, per_tile + 2 * nsf, dtype=torch.uint8)
    for i in range(num_tiles):
        for j in range(nsf):
            for k in range(group // 2):
                out[i, j * (group // 2) + k] = (int(A_int[i * nsf + j, 2 * k]) & 0x0F) | (
                    (int(A_int[i * nsf + j, 2 * k + 1]) & 0x0F) << 4
                )
        for j in range(nsf):
            b = int(scales[i * nsf + j].view(torch.int16)) & 0xFFFF
            out[i, per_tile + 2 * j] = b & 0xFF
            out[i, per_tile + 2 * j + 1] = (b >> 8) & 0xFF
    return out.flatten()


@pytest.mark.parametrize("n,tile,group", [(256, 128, 32), (512, 256, 64)])
def test_payload_generator_matches_loop_packer(n, tile, group):
    payload = ops.dequant_generate_inputs(n, tile, group, seed=3)
    torch.manual_seed(3)
    nt, nsf = n // tile, tile // group
    A = torch.rand(nt * nsf, group, dtype=BF16) * 3.75
    sc = 1 / 3.75 + (1 - 1 / 3.75) * torch.rand(nt * nsf, dtype=BF16)
    Aq = torch.quantize_per_channel(A.float(), sc.float(), torch.zeros(nt * nsf), 0, torch.quint8).int_repr()
    assert torch.equal(payload, _payload_loops(Aq, sc, nt, nsf, group))
    # and the payload decodes to q*s with q in [0,15]
    out = ops.dequant_payload_reference(payload, tile, group, signed=False)
    assert torch.equal(out, (Aq.float() * sc.float().unsqueeze(1)).to(BF16).reshape(-1))


def test_gemv_int4_reference_is_composition():
    codes, scales, x = __import__("oracle.configs", fromlist=["x"]).cfg2_gemv_int4(M=64, K=256, seed=1)
    W = ops.dequant_planar(codes, scales)
    q = ops.unpack_int4(codes).double()
    exact = (q * scales.double().repeat_interleave(32, 1)) @ x.double()
    y = ops.gemv_int4_reference(codes, scales, x)
    # weights rounded to bf16 first, then fp32 accumulation: within a bf16 ulp
    # of the unrounded product plus the weight rounding (<= 2^-9 relative each)
    err = (y.double() - exact).abs()
    bound = exact.abs() * 2**-8 + (q.abs() * scales.double().repeat_interleave(32, 1)).matmul(x.double().abs()) * 2**-8
    assert torch.all(err <= bound + 1e-6)
    assert W.dtype == BF16


def test_quantizer_picks_nearest_code_and_bf16_scale():
    """quantize_int4_g32 against a float64 brute force over all 16 codes."""
    torch.manual_seed(5)
    W = (torch.randn(16, 256) * 0.02).to(BF16)
    W[0, :32] = 0  # an all-zero group
    codes, scales = ops.quantize_int4_g32(W)
    Wd = W.double().reshape(16, 8, 32)
    amax = Wd.abs().amax(-1)
    assert torch.equal(scales, (amax.clamp_min(1e-8) / 7).float().to(BF16))
    s = scales.double().unsqueeze(-1)
    grid = torch.arange(-8, 8, dtype=torch.float64)
    err = (Wd.unsqueeze(-1) - grid * s.unsqueeze(-1)).abs()  # (16, 8, 32, 16)
    best = err.min(-1).values
    q = ops.unpack_int4(codes).double().reshape(16, 8, 32)
    mine = (Wd - q * s).abs()
    assert torch.all(mine <= best + 1e-12)  # nearest representable value (ties either way)
    assert torch.all(mine <= s / 2 + 1e-12)
    assert int(q.min()) >= -8 and int(q.max()) <= 7

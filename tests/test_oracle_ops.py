"""Pins for the oracle's RoPE, norm, softmax, attention, GEMM and SwiGLU functions (CPU).

Every check compares against something the oracle does not share code with:
transformers' published llama3 RoPE routine, torch library routines run in
float64, closed forms, brute-force loops, and the reference's own RoPE
convention test (iron/tests/operators/rope_reference_convention.py:21-64),
restated.
"""

import math

import numpy as np
import pytest
import torch

from oracle import ops

BF16 = torch.bfloat16


# ------------------------------------------------------------------- RoPE
def test_llama3_rope_table_matches_transformers():
    from transformers import LlamaConfig
    from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS

    cfg = LlamaConfig(
        hidden_size=2048, num_attention_heads=32, num_key_value_heads=8, head_dim=64, rope_theta=500000.0,
        max_position_embeddings=131072,
        rope_scaling={"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                      "original_max_position_embeddings": 8192},
    )
    inv_freq, _ = ROPE_INIT_FUNCTIONS["llama3"](cfg, None)
    pos = torch.tensor([0, 1, 2, 2047, 4095], dtype=torch.float32)
    ang = pos[:, None] * inv_freq[None, :].float()
    cos, sin = ops.compute_rope_params(64, 500000.0, 4096, ops.LLAMA3_FREQ_CONFIG)
    assert torch.allclose(cos[pos.long()], torch.cos(ang), atol=1e-6, rtol=0)
    assert torch.allclose(sin[pos.long()], torch.sin(ang), atol=1e-6, rtol=0)


def test_rope_table_without_scaling_is_textbook():
    cos, sin = ops.compute_rope_params(64, 10000.0, 8)
    i = torch.arange(32, dtype=torch.float64)
    inv = 10000.0 ** (-2 * i / 64)
    for p in range(8):
        assert torch.allclose(cos[p].double(), torch.cos(p * inv), atol=1e-6)
        assert torch.allclose(sin[p].double(), torch.sin(p * inv), atol=1e-6)
    assert torch.all(cos[0] == 1) and torch.all(sin[0] == 0)


def _block_major_expected(x, angles, rows, angle_rows):
    """The reference's device convention row by row: row r uses angle row r // (rows // angle_rows)."""
    cols = x.shape[-1]
    half = cols // 2
    per = rows // angle_rows
    out = torch.empty(rows, cols, dtype=torch.float32)
    for r in range(rows):
        a = r // per
        cos = angles[a, 0::2].float()
        sin = angles[a, 1::2].float()
        x1, x2 = x[r, :half].float(), x[r, half:].float()
        out[r, :half] = x1 * cos - x2 * sin
        out[r, half:] = x2 * cos + x1 * sin
    return out.to(BF16)


@pytest.mark.parametrize("rows,angle_rows", [(6, 3), (8, 2), (1024, 1), (4, 4), (13, 13), (12, 4)])
def test_rope_reference_device_convention(rows, angle_rows):
    torch.manual_seed(0)
    cols = 4
    x = torch.randn(rows, cols).to(BF16)
    angles = torch.zeros(angle_rows, cols, dtype=BF16)
    angles[:, 0::2] = torch.rand(angle_rows, 2).to(BF16)
    angles[:, 1::2] = torch.rand(angle_rows, 2).to(BF16)
    assert torch.equal(ops.rope_reference(x, angles), _block_major_expected(x, angles, rows, angle_rows))


def test_rope_interleaved_is_complex_rotation():
    torch.manual_seed(1)
    x = torch.randn(5, 32).to(BF16)
    theta = torch.rand(5, 16) * 6
    angles = torch.empty(5, 32)
    angles[:, 0::2] = torch.cos(theta)
    angles[:, 1::2] = torch.sin(theta)
    y = ops.rope_reference(x, angles, method_type=1).double()
    z = torch.complex(x[:, 0::2].double(), x[:, 1::2].double()) * torch.exp(1j * theta.double())
    assert torch.allclose(y[:, 0::2], z.real, atol=2e-2, rtol=1e-2)
    assert torch.allclose(y[:, 1::2], z.imag, atol=2e-2, rtol=1e-2)


def test_rope_position_zero_is_identity():
    x = torch.randn(8, 64).to(BF16)
    angles = ops.rope_angles_table(64, 4)
    assert torch.equal(ops.rope_reference(x, angles[0:1]), x)


# ------------------------------------------------------- norm / eltwise
def test_rms_norm_matches_torch_rms_norm():
    torch.manual_seed(2)
    x = (torch.rand(16, 2048) * 4).to(BF16)
    w = (torch.rand(2048) * 4).to(BF16)
    ref = torch.nn.functional.rms_norm(x.double(), (2048,), w.double(), eps=1e-5)
    assert torch.allclose(ops.rms_norm_reference(x, w).double(), ref, rtol=2**-7, atol=1e-6)
    ref_u = torch.nn.functional.rms_norm(x.double(), (2048,), None, eps=1e-5)
    assert torch.allclose(ops.rms_norm_reference(x).double(), ref_u, rtol=2**-7, atol=1e-6)


def test_silu_and_swiglu_closed_form():
    x = torch.linspace(-8, 8, 257).to(BF16)
    xd = x.double()
    assert torch.allclose(ops.silu_reference(x).double(), xd / (1 + torch.exp(-xd)), rtol=2**-7, atol=1e-6)
    u = torch.linspace(-2, 2, 257).to(BF16)
    assert torch.allclose(ops.swiglu_reference(x, u).double(), xd / (1 + torch.exp(-xd)) * u.double(),
                          rtol=2**-7, atol=1e-5)


def test_softmax_rows_and_mask():
    torch.manual_seed(3)
    x = (torch.rand(16, 64) * 4).to(BF16)
    s = ops.softmax_reference(x).double()
    e = torch.exp(x.double() - x.double().max(-1, keepdim=True).values)
    assert torch.allclose(s, e / e.sum(-1, keepdim=True), rtol=2**-7, atol=1e-6)
    assert torch.allclose(s.sum(-1), torch.ones(16, dtype=torch.float64), atol=16 * 2**-8)
    m = ops.softmax_reference(x, valid=40).double()
    assert torch.all(m[:, 40:] == 0)
    e = torch.exp(x[:, :40].double() - x[:, :40].double().max(-1, keepdim=True).values)
    assert torch.allclose(m[:, :40], e / e.sum(-1, keepdim=True), rtol=2**-7, atol=1e-6)


# -------------------------------------------------------------- attention
def test_attention_reference_matches_sdpa_float64():
    torch.manual_seed(4)
    H, Hkv, S, D = 8, 2, 37, 64
    Q = torch.randn(H, S, D).to(BF16)
    K = torch.randn(Hkv, S, D).to(BF16)
    V = torch.randn(Hkv, S, D).to(BF16)
    out = ops.attention_reference(Q, K, V, causal=True).double()
    ref = torch.nn.functional.scaled_dot_product_attention(
        Q.double(), K.double().repeat_interleave(4, 0), V.double().repeat_interleave(4, 0), is_causal=True
    )
    assert torch.allclose(out, ref, atol=2e-2, rtol=1e-2)


def test_attention_brute_force_small():
    torch.manual_seed(5)
    Q = torch.randn(2, 3, 64).to(BF16)
    K = torch.randn(1, 5, 64).to(BF16)
    V = torch.randn(1, 5, 64).to(BF16)
    out = ops.attention_reference(Q, K, V, causal=True).double()  # queries at positions 2, 3, 4
    for h in range(2):
        for i in range(3):
            n = i + 3
            s = [sum(Q[h, i, d].item() * K[0, j, d].item() for d in range(64)) / 8 for j in range(n)]
            mx = max(s)
            p = [math.exp(v - mx) for v in s]
            z = sum(p)
            for d in range(0, 64, 7):
                expect = sum(p[j] * V[0, j, d].item() for j in range(n)) / z
                assert abs(out[h, i, d].item() - expect) <= 1e-2 * max(1, abs(expect))


def test_single_position_attention_returns_v():
    q = torch.randn(4, 1, 64).to(BF16)
    k = torch.randn(1, 1, 64).to(BF16)
    v = torch.randn(1, 1, 64).to(BF16)
    assert torch.equal(ops.attention_reference(q, k, v), v.expand(4, 1, 64))


def test_gqa_decode_reference_appends_and_attends():
    from oracle import configs

    q, kn, vn, kc, vc, pos, angles = configs.cfg3_gqa_decode(n_heads=8, n_kv=2, L=40)
    out, kc2, vc2 = ops.gqa_decode_reference(q, kn, vn, kc, vc, pos, angles)
    assert torch.equal(kc2[:, :pos], kc[:, :pos]) and torch.equal(vc2[:, pos], vn)
    assert torch.equal(kc2[:, pos], ops.rope_reference(kn, angles[pos : pos + 1]))
    qr = ops.rope_reference(q, angles[pos : pos + 1]).double()
    for h in (0, 5):
        g = h // 4
        s = kc2[g, : pos + 1].double() @ qr[h] / 8.0
        p = torch.softmax(s, 0)
        assert torch.allclose(out[h].double(), p @ vc2[g, : pos + 1].double(), atol=1e-2, rtol=1e-2)


# ------------------------------------------------------------------- GEMM
@pytest.mark.parametrize("bc,cc", [(False, False), (True, False), (False, True), (True, True)])
def test_gemm_reference_layouts(bc, cc):
    torch.manual_seed(6)
    A = torch.randn(8, 16).to(BF16)
    B = torch.randn(16, 12).to(BF16)
    stored = B.T.contiguous() if bc else B
    C = ops.gemm_reference(A, stored, bc, cc).double()
    exact = A.double().numpy() @ B.double().numpy()
    if cc:
        exact = exact.T
    assert np.allclose(C.numpy(), exact, rtol=2**-7, atol=1e-5)


def test_flm_epilogues_closed_form():
    C = torch.linspace(-6, 6, 97).to(BF16)
    c = C.double()
    assert torch.allclose(ops.flm_apply_epilogue(C, "gelu").double(), c / (1 + torch.exp(-1.702 * c)), rtol=2**-7, atol=1e-3)
    assert torch.allclose(ops.flm_apply_epilogue(C, "silu").double(), c / (1 + torch.exp(-c)), rtol=2**-7, atol=1e-3)
    assert torch.allclose(ops.flm_apply_epilogue(C, "sigmoid").double(), 1 / (1 + torch.exp(-c)), rtol=2**-7, atol=1e-3)
    cl = ops.flm_apply_epilogue(C, "none", (-1.0, 2.0)).double()
    assert cl.min() == -1.0 and cl.max() == 2.0


def test_swiglu_golden_chain_consistent():
    d = ops.swiglu_decode_golden(M=1, K=64, N=128)
    left = d["input"].double() @ d["w_gate"].double()
    assert torch.allclose(d["left"].double(), left, rtol=2**-7, atol=1e-3 * left.abs().max().item())
    inter = d["left_swished"].double() * d["right"].double()
    assert torch.allclose(d["intermediate"].double(), inter, rtol=2**-7, atol=1e-6)


def _strided_brute(inp, isz, ist, ioff, out_len, osz, ost, ooff, channels):
    """Nested loops over each channel's split pattern (no numpy meshgrid)."""
    import itertools

    def pad(sz, st):
        return [1] * (4 - len(sz)) + list(sz), [0] * (4 - len(st)) + list(st)

    def offsets(sz, st, off):
        sz, st = pad(sz, st)
        hi = max(i for i, s in enumerate(sz) if s >= 1)
        per = sz[hi] // channels
        res = []
        for c in range(channels):
            split = sz[:hi] + [per] + sz[hi + 1 :]
            base = off + c * per * st[hi]
            chan = []
            for idx in itertools.product(*[range(s) for s in split]):
                chan.append(base + sum(i * s for i, s in zip(idx, st)))
            res.append(chan)
        return res

    out = torch.zeros(out_len, dtype=inp.dtype)
    for s, d in zip(offsets(isz, ist, ioff), offsets(osz, ost, ooff)):
        for a, b in zip(s, d):
            out[b] = inp[a]
    return out


@pytest.mark.parametrize("channels", [1, 2, 4])
def test_strided_copy_matches_brute_force(channels):
    g = torch.Generator().manual_seed(channels)
    inp = torch.rand(512, generator=g).to(torch.bfloat16)
    cases = [
        ([8, 16], [16, 1], 0, 1024, [8, 1, 16], [64, 0, 1], 5),
        ([4, 8, 8], [64, 1, 8], 3, 600, [4, 64], [128, 1], 40),  # permuted gather
        ([256], [2], 0, 256, [256], [1], 0),
    ]
    for isz, ist, ioff, olen, osz, ost, ooff in cases:
        ref = ops.strided_copy_reference(inp, isz, ist, ioff, olen, osz, ost, ooff, num_aie_channels=channels)
        assert torch.equal(ref, _strided_brute(inp, isz, ist, ioff, olen, osz, ost, ooff, channels))


def test_strided_copy_kv_append_identity():
    """The KV-cache write of llama_npu.py:311-323: cache[:, slot, :] = x."""
    n_kv, hd, seq, slot = 8, 64, 32, 7
    x = torch.randn(n_kv, hd).to(torch.bfloat16)
    cache = torch.randn(n_kv, seq, hd).to(torch.bfloat16)
    out = ops.strided_copy_reference(x.reshape(-1), [n_kv, hd], [hd, 1], 0, n_kv * seq * hd, [1, n_kv, hd],
                                     [0, seq * hd, 1], 0, output_offset_addend=slot * hd, out=cache.reshape(-1))
    expect = cache.clone()
    expect[:, slot, :] = x
    assert torch.equal(out.reshape(n_kv, seq, hd), expect)


def test_repeat_and_transpose_references():
    x = torch.arange(12.0).reshape(3, 4)
    assert ops.repeat_reference(x, 2).tolist() == [r for r in x.tolist() for _ in range(2)]
    t = ops.transpose_reference(torch.arange(24.0), 4, 6)
    assert torch.equal(t[0], torch.arange(24.0).reshape(4, 6).T)


def test_bf16_toward_zero_known_answers_and_invariants():
    """The oracle's "floor" conversion of flm.GEMM (flm/gemm/design.py:164-172:
    truncation, which the reference describes as biasing every conversion the
    same way): the mantissa is cut, so the result rounds toward zero -- for a
    negative value that is up, not down (-1.01171875 -> -1.0078125)."""
    x = torch.tensor([1.01171875, -1.01171875, 1.00390625, 1.0, -0.0, 3.3895313892515355e38, float("inf"),
                      float("-inf"), 1e-40, float("nan")], dtype=torch.float32)
    y = ops.bf16_toward_zero(x).float()
    want = [1.0078125, -1.0078125, 1.0, 1.0, -0.0, 3.3895313892515355e38, float("inf"), float("-inf")]
    assert y[:8].tolist() == want
    assert x[2].to(torch.bfloat16).float() == 1.0 and x[0].to(torch.bfloat16).float() == 1.015625  # RNE differs
    assert 0 <= y[8] <= 1e-40 and torch.isnan(y[9])
    g = torch.Generator().manual_seed(0)
    r = torch.randn(100000, generator=g) * torch.exp(torch.randn(100000, generator=g) * 8)
    t = ops.bf16_toward_zero(r).float()
    assert torch.all(t.abs() <= r.abs()) and torch.all((t == 0) | (torch.sign(t) == torch.sign(r)))
    # the largest-magnitude bf16 not above |r|: the RNE neighbour, or the one below it toward zero
    rne = r.to(torch.bfloat16).float()
    below = torch.where(rne.abs() > r.abs(), torch.nextafter(rne.to(torch.bfloat16), torch.zeros(1, dtype=torch.bfloat16)).float(), rne)
    assert torch.equal(t, below)
    exact = r.to(torch.bfloat16).float()
    assert torch.equal(ops.bf16_toward_zero(exact).float(), exact)  # bf16 values pass unchanged


def test_flm_gemm_floor_reference():
    """flm_gemm_reference(rounding="floor") truncates both conversions: its
    outputs never exceed the round-to-nearest ones in magnitude and differ from
    them in a large share of the elements."""
    g = ops.flm_gemm_golden(64, 512, 96, epilogue="none", rounding="floor")
    rne = ops.flm_gemm_reference(g["input"], g["input_b"])
    fl = g["output"].float()
    assert torch.all(fl.abs() <= rne.float().abs())
    assert (fl != rne.float()).float().mean() > 0.2
    acc = g["input"].float() @ g["input_b"].float()
    assert torch.equal(g["output"], ops.bf16_toward_zero(acc))

"""CPU restatements of the reference operators (TEST INFRASTRUCTURE ONLY).

Each function cites the reference file:line it restates (paths relative to the
atassis/IRON tree) and names what pins it (tests/test_oracle_ops.py).
Arithmetic follows the reference: bf16 tensors in, fp32 math, one bf16
rounding at the end unless the reference rounds more often.
"""

from __future__ import annotations

import math

import numpy as np
import torch

BF16 = torch.bfloat16


# --------------------------------------------------------------------- GEMV
def gemv_reference(A: torch.Tensor, x: torch.Tensor, out_dtype=BF16) -> torch.Tensor:
    """y = A @ x, fp32 accumulation, bf16 out (gemv/reference.py:9-11).

    Batched when A is (B, M, K) and x (B, K) (gemv/reference.py:45-66).
    ``out_dtype=torch.float32`` returns the unrounded fp32-accumulated result,
    the reference the BASELINE bf16 tolerance is stated against.
    PINNED BY: float64 numpy brute force on small shapes.
    """
    y = torch.matmul(A.float(), x.float().unsqueeze(-1)).squeeze(-1)
    return y.to(out_dtype)


def gemv_golden(M=128, K=128, seed=42):
    """Seeded golden of gemv/reference.py:14-42 (randn*4 bf16 A and x)."""
    torch.manual_seed(seed)
    A = torch.randn(M, K, dtype=BF16) * 4
    B = torch.randn(K, dtype=BF16) * 4
    return {"A": A, "B": B, "C": gemv_reference(A, B)}


def gemv_golden_batched(M=128, K=128, num_batches=2, seed=42):
    """Seeded golden of gemv/reference.py:45-66."""
    torch.manual_seed(seed)
    A = torch.randn(num_batches, M, K, dtype=BF16) * 4
    B = torch.randn(num_batches, K, dtype=BF16) * 4
    return {"A": A, "B": B, "C": gemv_reference(A, B)}


def gelu_tanh(x: torch.Tensor) -> torch.Tensor:
    """0.5x(1+tanh(0.79788456(x+0.044715x^3))) in fp32 (gemv/reference.py:69-76).

    PINNED BY: torch.nn.functional.gelu(approximate="tanh").
    """
    xf = x.float()
    return 0.5 * xf * (1.0 + torch.tanh(0.79788456 * (xf + 0.044715 * xf**3)))


# ------------------------------------------------------------------- int4
def pack_int4(q: torch.Tensor) -> torch.Tensor:
    """Pack int4 values (..., K) into (..., K/2) uint8, low nibble = even element.

    Layout of BASELINE config 2 and of dequant/reference.py:77-84 (low nibble
    first). Two's complement for negative values.
    PINNED BY: unpack_int4 round trip over all 16x16 nibble pairs.
    """
    q = q.to(torch.int16)
    lo = q[..., 0::2] & 0xF
    hi = q[..., 1::2] & 0xF
    return (lo | (hi << 4)).to(torch.uint8)


def unpack_int4(codes: torch.Tensor, signed: bool = True) -> torch.Tensor:
    """Inverse of pack_int4: (..., K/2) uint8 -> (..., K) int16."""
    c = codes.to(torch.int16)
    lo = c & 0xF
    hi = (c >> 4) & 0xF
    if signed:
        lo = torch.where(lo >= 8, lo - 16, lo)
        hi = torch.where(hi >= 8, hi - 16, hi)
    out = torch.empty(*codes.shape[:-1], codes.shape[-1] * 2, dtype=torch.int16)
    out[..., 0::2] = lo
    out[..., 1::2] = hi
    return out


def dequant_planar(codes, scales, group=32, signed=True) -> torch.Tensor:
    """bf16_rne(float(q) * float(scale)) (dequant/reference.py:9-14 contract).

    The product of a 4-bit integer and a bf16 is exact in fp32; torch's
    float32 -> bfloat16 conversion rounds to nearest even.
    PINNED BY: exhaustive 16 codes x all finite bf16 scales against exact
    rational rounding (fractions) on a sample, and torch RNE elsewhere.
    """
    q = unpack_int4(codes, signed).float()
    s = scales.float().repeat_interleave(group, dim=-1)
    return (q * s).to(BF16)


def dequant_payload_reference(payload: torch.Tensor, tile_size: int, group_size: int, signed=False):
    """Reference payload layout -> bf16 (dequant/reference.py:8-18).

    Per tile: tile/2 code bytes (low nibble first), then tile/group bf16
    scales as little-endian byte pairs (dequant/reference.py:68-92).
    """
    tile_bytes = tile_size // 2 + 2 * (tile_size // group_size)
    tiles = payload.reshape(-1, tile_bytes)
    codes = tiles[:, : tile_size // 2]
    sb = tiles[:, tile_size // 2 :].to(torch.int32)
    sbits = (sb[:, 0::2] | (sb[:, 1::2] << 8)).to(torch.int16)
    scales = sbits.view(BF16)
    return dequant_planar(codes, scales, group_size, signed).reshape(-1)


def dequant_generate_inputs(input_length, tile_size, group_size, seed=42):
    """Restatement of dequant/reference.py:21-94 (vectorised packing).

    Uniform bf16 values in [0, 3.75) per group, quantised per group with a
    bf16 scale in [1/3.75, 1) by torch.quantize_per_channel (quint8, zero
    point 0), then packed tile by tile: codes then scales.
    PINNED BY: the loop-form packer in tests (literal restatement of :77-92).
    """
    torch.manual_seed(seed)
    if input_length % tile_size != 0:
        raise ValueError("Input length must be a multiple of tile size.")
    if tile_size % group_size != 0:
        raise ValueError("Tile size must be a multiple of group size.")
    num_tiles = input_length // tile_size
    nsf = tile_size // group_size
    val_range = 3.75
    A = torch.rand(num_tiles * nsf, group_size, dtype=BF16) * val_range
    r1, r2 = 1 / val_range, 1
    scales = r1 + (r2 - r1) * torch.rand(num_tiles * nsf, dtype=BF16)
    zp = torch.zeros(num_tiles * nsf, dtype=BF16)
    Aq = torch.quantize_per_channel(
        A.to(torch.float32), scales=scales.to(torch.float32), zero_points=zp.to(torch.float32),
        axis=0, dtype=torch.quint8,
    ).int_repr()
    codes = ((Aq[:, 0::2] & 0x0F) | ((Aq[:, 1::2] & 0x0F) << 4)).to(torch.uint8)
    codes = codes.reshape(num_tiles, nsf * group_size // 2)
    sbits = scales.view(torch.int16).to(torch.int32)
    sbytes = torch.stack([sbits & 0xFF, (sbits >> 8) & 0xFF], dim=-1).to(torch.uint8)
    sbytes = sbytes.reshape(num_tiles, nsf * 2)
    return torch.cat([codes, sbytes], dim=1).flatten()


def gemv_int4_reference(codes, scales, x, group=32, signed=True, out_dtype=BF16) -> torch.Tensor:
    """GEMV(Dequant(codes, scales), x): bit-exact bf16 weights, fp32 accumulation.

    Composition of dequant_planar and gemv_reference.
    """
    W = dequant_planar(codes, scales, group, signed)
    return gemv_reference(W, x, out_dtype)


def gemv_int4_exact(codes, scales, x, group=32, signed=True) -> torch.Tensor:
    """sum_k q_k * s_g(k) * x_k in float64 with no intermediate rounding.

    The mathematically exact value the fused int4 GEMV approximates (it applies
    the group scale to exact integer codes rather than to bf16-rounded weights).
    """
    q = unpack_int4(codes, signed).double()
    s = scales.double().repeat_interleave(group, dim=-1)
    return (q * s) @ x.double()


def quantize_int4_g32(W: torch.Tensor, group=32):
    """Symmetric int4 group quantiser used to build test weights.

    scale = bf16(max|w| / 7) per group, q = clamp(round(w/scale), -8, 7).
    Returns (codes (N, K/2) uint8, scales (N, K/group) bf16).
    """
    Wf = W.float().reshape(W.shape[0], -1, group)
    amax = Wf.abs().amax(dim=-1, keepdim=True).clamp_min(1e-8)
    s = (amax / 7.0).to(BF16)
    q = torch.clamp(torch.round(Wf / s.float()), -8, 7).to(torch.int16).reshape(W.shape)
    return pack_int4(q), s.reshape(W.shape[0], -1)


# ------------------------------------------------------------------- RoPE
def compute_rope_params(head_dim, theta_base=10_000, context_length=4096, freq_config=None,
                        dtype=torch.float32):
    """cos/sin tables with optional llama3 frequency scaling (rope/reference.py:7-66).

    PINNED BY: transformers' _compute_llama3_parameters (an independent
    published implementation) and closed-form special cases.
    """
    assert head_dim % 2 == 0
    inv_freq = 1.0 / (theta_base ** (torch.arange(0, head_dim, 2, dtype=dtype)[: head_dim // 2].float() / head_dim))
    if freq_config is not None:
        f = freq_config
        low_wl = f["original_context_length"] / f["low_freq_factor"]
        high_wl = f["original_context_length"] / f["high_freq_factor"]
        wavelen = 2 * torch.pi / inv_freq
        scaled = torch.where(wavelen > low_wl, inv_freq / f["factor"], inv_freq)
        smooth = (f["original_context_length"] / wavelen - f["low_freq_factor"]) / (
            f["high_freq_factor"] - f["low_freq_factor"]
        )
        smoothed = (1 - smooth) * (inv_freq / f["factor"]) + smooth * inv_freq
        medium = (wavelen <= low_wl) & (wavelen >= high_wl)
        inv_freq = torch.where(medium, smoothed, scaled)
    pos = torch.arange(context_length, dtype=dtype)
    ang = pos.unsqueeze(1) * inv_freq.unsqueeze(0)
    return torch.cos(ang), torch.sin(ang)


LLAMA3_FREQ_CONFIG = {
    "factor": 32.0,
    "low_freq_factor": 1.0,
    "high_freq_factor": 4.0,
    "original_context_length": 8192,
}


def rope_angles_table(head_dim, context_length, theta=500000.0, freq_config=LLAMA3_FREQ_CONFIG,
                      dtype=torch.float32):
    """Interleaved [cos, sin, cos, sin, ...] rows (rope/reference.py:145-148 layout)."""
    cos, sin = compute_rope_params(head_dim, theta, context_length, freq_config)
    angles = torch.empty(context_length, head_dim, dtype=torch.float32)
    angles[:, 0::2] = cos
    angles[:, 1::2] = sin
    return angles.to(dtype)


def rope_reference(x, angles, method_type=0):
    """RoPE from the packed angles buffer (rope/reference.py:69-102).

    Row r uses angle row r // (rows / angle_rows); fp32 math, one bf16 rounding.
    PINNED BY: the reference's own convention test
    (iron/tests/operators/rope_reference_convention.py:21-64), restated.
    """
    rows = x.shape[0]
    if rows % angles.shape[0] != 0:
        raise ValueError(f"{rows} rows cannot share {angles.shape[0]} angle rows evenly")
    rep = rows // angles.shape[0]
    cos = angles[..., 0::2].float().repeat_interleave(rep, dim=0)
    sin = angles[..., 1::2].float().repeat_interleave(rep, dim=0)
    x32 = x.float()
    if method_type == 0:
        half = x.shape[-1] // 2
        x1, x2 = x32[..., :half], x32[..., half:]
        y = torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1)
    elif method_type == 1:
        xe, xo = x32[..., 0::2], x32[..., 1::2]
        y = torch.empty_like(x32)
        y[..., 0::2] = xe * cos - xo * sin
        y[..., 1::2] = xe * sin + xo * cos
    else:
        raise ValueError(f"method_type must be 0 or 1, got {method_type}")
    return y.to(BF16)


def rope_generate_inputs(rows=4096, cols=64, context_len=131072, seed=42):
    """Restatement of rope/reference.py:105-150 (bf16 llama3-scaled table)."""
    torch.manual_seed(seed)
    cos, sin = compute_rope_params(cols, 500000.0, context_len, LLAMA3_FREQ_CONFIG)
    if context_len < rows and rows % context_len != 0:
        raise ValueError("rows must be a multiple of context_len when rows > context_len")
    n_heads = rows // context_len if context_len < rows else 1
    seq_len = rows // n_heads
    x = torch.rand(n_heads, seq_len, cols, dtype=BF16) * 4
    angles = torch.zeros((seq_len, cols), dtype=BF16)
    angles[:, ::2] = cos[:seq_len, : cols // 2]
    angles[:, 1::2] = sin[:seq_len, : cols // 2]
    return x.transpose(0, 1).reshape(rows, cols).contiguous(), angles


# --------------------------------------------------------- norm / eltwise
def rms_norm_reference(x, w=None, eps=1e-5):
    """x / sqrt(mean(x^2) + eps) [* w], fp32, bf16 out (rms_norm/reference.py:7-16).

    PINNED BY: torch.nn.functional.rms_norm.
    """
    xf = x.float()
    out = xf / torch.sqrt(torch.mean(xf * xf, dim=-1, keepdim=True) + eps)
    if w is not None:
        out = out * w.float()
    return out.to(BF16)


def silu_reference(x):
    """SiLU (silu/reference.py:7-9), fp32 math. PINNED BY: closed form x*sigmoid(x)."""
    return torch.nn.functional.silu(x.float()).to(BF16)


def mul_reference(a, b):
    """a * b (elementwise_mul/reference.py:7-9)."""
    return (a.float() * b.float()).to(BF16)


def add_reference(a, b):
    """a + b (elementwise_add/reference.py:7-9)."""
    return (a.float() + b.float()).to(BF16)


def softmax_reference(x, valid=None):
    """Row softmax over the last dim in fp32 (softmax/reference.py:9-11).

    With ``valid`` (the runtime vector size of softmax/design.py:74-91), columns
    >= valid are masked to -inf first and come out as 0.
    PINNED BY: float64 closed form; rows sum to 1.
    """
    xf = x.float()
    if valid is not None and valid < x.shape[-1]:
        xf = xf.clone()
        xf[..., valid:] = float("-inf")
    return torch.softmax(xf, dim=-1).to(BF16)


def swiglu_reference(gate, up):
    """SiLU(gate) * up (the silu -> mul steps of swiglu_decode/op.py:56-62)."""
    g = gate.float()
    return (torch.nn.functional.silu(g) * up.float()).to(BF16)


# ---------------------------------------------------------------- attention
def mha_golden(heads=1, S_q=256, S_kv=256, d=64, num_kv_heads=2, seed=42):
    """Seeded inputs of mha/reference.py:27-94 with a fp32 causal-SDPA output.

    Q (heads,S,d), K/V (kv_heads,S,d) = rand*4 bf16; O = causal softmax(QK^T/sqrt(d))V.
    PINNED BY: float64 explicit attention; L=1 special case.
    """
    torch.manual_seed(seed)
    np.random.seed(seed)
    if num_kv_heads == 0:
        num_kv_heads = heads
    Q = torch.rand(heads, S_q, d, dtype=BF16) * 4
    K = torch.rand(num_kv_heads, S_kv, d, dtype=BF16) * 4
    V = torch.rand(num_kv_heads, S_kv, d, dtype=BF16) * 4
    O = attention_reference(Q, K, V, causal=True)
    return {"Q": Q, "K": K, "V": V, "O": O}


def attention_reference(Q, K, V, causal=True, scale=None, q_offset=None):
    """GQA attention in fp32: softmax(Q K^T * scale [+ causal mask]) V -> bf16.

    Q (H, Sq, d), K/V (Hkv, Skv, d); head h uses KV head h // (H/Hkv)
    (llama_cpu.py:118-146, repeat_interleave). Query i sits at absolute
    position q_offset + i (default Skv - Sq) and may attend keys <= it.
    """
    H, Sq, d = Q.shape
    Hkv, Skv, _ = K.shape
    g = H // Hkv
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    Kf = K.float().repeat_interleave(g, dim=0)
    Vf = V.float().repeat_interleave(g, dim=0)
    s = torch.matmul(Q.float(), Kf.transpose(-1, -2)) * scale
    if causal:
        off = (Skv - Sq) if q_offset is None else q_offset
        qi = torch.arange(Sq).unsqueeze(1) + off
        kj = torch.arange(Skv).unsqueeze(0)
        s = s.masked_fill(kj > qi, float("-inf"))
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, Vf).to(BF16)


def gqa_decode_reference(q, k_new, v_new, k_cache, v_cache, pos, angles, scale=None):
    """One decode step of llama_cpu.grouped_query_attention_forward (llama_cpu.py:49-148).

    q (H, d) and k_new (Hkv, d) are rotated (two-halves) with angle row ``pos``
    and rounded to bf16 (the RoPE operator's output), k_new/v_new are written at
    cache position ``pos``, and attention runs over positions 0..pos.
    Returns (out (H, d) bf16, k_cache', v_cache').
    """
    qr = rope_reference(q, angles[pos : pos + 1])
    kr = rope_reference(k_new, angles[pos : pos + 1])
    kc = k_cache.clone()
    vc = v_cache.clone()
    kc[:, pos] = kr
    vc[:, pos] = v_new
    out = attention_reference(qr.unsqueeze(1), kc[:, : pos + 1], vc[:, : pos + 1], causal=False, scale=scale)
    return out.squeeze(1), kc, vc


# -------------------------------------------------------------------- GEMM
def gemm_reference(A, B, b_col_maj=False, c_col_maj=False):
    """C = A @ B from stored inputs, fp32 accumulate, bf16 out (gemm/reference.py:7-18)."""
    Bm = B.T if b_col_maj else B
    C = torch.matmul(A.float(), Bm.float()).to(A.dtype)
    return C.T.contiguous() if c_col_maj else C


def gemm_golden(M, K, N, seed=42, b_col_maj=False):
    """Seeded inputs of gemm/reference.py:21-36 (A randn*4, B rand*4)."""
    torch.manual_seed(seed)
    A = torch.randn(M, K, dtype=BF16) * 4
    B = torch.rand(K, N, dtype=BF16) * 4
    if b_col_maj:
        B = B.T.contiguous()
    return {"input": A, "input_b": B, "output": gemm_reference(A, B, b_col_maj)}


FLM_EPILOGUES = ("none", "gelu", "silu", "sigmoid")


def bf16_toward_zero(x: torch.Tensor) -> torch.Tensor:
    """fp32 -> bf16 by mantissa truncation (round toward zero): the "floor"
    conversion of flm.GEMM (flm/gemm/design.py:164-172). NaN stays NaN.
    PINNED BY: known answers and the truncation invariants (|y| <= |x|, same
    sign, |x - y| < one bf16 ulp) in tests/test_oracle_ops.py."""
    x = x.float().contiguous()
    bits = x.view(torch.int32) & ~0xFFFF
    y = bits.view(torch.float32).to(BF16)  # exact: the low 16 bits are zero
    return torch.where(torch.isnan(x), torch.full_like(y, float("nan")), y)


def _to_bf16(x: torch.Tensor, rounding: str) -> torch.Tensor:
    return bf16_toward_zero(x) if rounding == "floor" else x.to(BF16)


def flm_apply_epilogue(C, epilogue="none", clamp=None, rounding="conv_even"):
    """flm.GEMM output stage (flm/gemm/reference.py:8-31); gelu = x*sigmoid(1.702x).
    With rounding="floor" the final bf16 conversion truncates."""
    Cf = C.float()
    if epilogue == "gelu":
        Cf = Cf * torch.sigmoid(1.702 * Cf)
    elif epilogue == "silu":
        Cf = Cf * torch.sigmoid(Cf)
    elif epilogue == "sigmoid":
        Cf = torch.sigmoid(Cf)
    elif epilogue != "none":
        raise ValueError(epilogue)
    if clamp is not None:
        Cf = torch.clamp(Cf, clamp[0], clamp[1])
    return _to_bf16(Cf, rounding)


def flm_gemm_reference(A, B, epilogue="none", clamp=None, rounding="conv_even"):
    """fp32 matmul -> bf16 -> epilogue -> clamp (flm/gemm/reference.py:34-57).
    rounding="floor": both bf16 conversions truncate (flm/gemm/op.py:105)."""
    C = _to_bf16(torch.matmul(A.float(), B.float()), rounding)
    return flm_apply_epilogue(C, epilogue, clamp, rounding)


def flm_gemm_golden(M, K, N, seed=42, epilogue="none", clamp=None, scale=4.0, rounding="conv_even"):
    """Seeded inputs of flm/gemm/reference.py:60-81."""
    torch.manual_seed(seed)
    A = torch.randn(M, K, dtype=BF16) * scale
    B = torch.rand(K, N, dtype=BF16) * scale
    return {"input": A, "input_b": B, "output": flm_gemm_reference(A, B, epilogue, clamp, rounding)}


# ------------------------------------------------------------------ SwiGLU
def swiglu_decode_golden(M=1, K=2048, N=8192, seed=42):
    """Seeded golden chain of swiglu_decode/reference.py:9-60 (incl. the unused
    biases that keep the RNG stream identical)."""
    torch.manual_seed(seed)
    v = 4
    x = torch.randn(M, K, dtype=BF16) * v
    w_gate = torch.randn(N, K, dtype=BF16).T * v
    _b1 = torch.randn(K, dtype=BF16) * v
    w_up = torch.randn(N, K, dtype=BF16).T * v
    _b2 = torch.randn(K, dtype=BF16) * v
    w_down = torch.randn(N, K, dtype=BF16) * v
    left = (x.float() @ w_gate.float()).to(BF16)
    left_swished = silu_reference(left)
    right = (x.float() @ w_up.float()).to(BF16)
    intermediate = mul_reference(left_swished, right)
    y = (intermediate.float() @ w_down.float()).to(BF16)
    return {
        "input": x, "w_gate": w_gate, "w_up": w_up, "w_down": w_down, "left": left,
        "left_swished": left_swished, "right": right, "intermediate": intermediate, "output": y,
    }


def swiglu_block_reference(x, norm_w, Wg, Wu, Wd, eps=1e-5):
    """BASELINE config 4 block: x + Wd(silu(Wg xn) * (Wu xn)), xn = RMSNorm(x)*w.

    bf16 between steps as the operator chain hands them over.
    """
    xn = rms_norm_reference(x, norm_w, eps)
    g = gemv_reference(Wg, xn)
    u = gemv_reference(Wu, xn)
    h = swiglu_reference(g, u)
    d = gemv_reference(Wd, h)
    return add_reference(x, d)


# ----------------------------------------------------------- verification
def verify_buffer(output, reference, rel_tol=0.04, abs_tol=1e-6, max_error_rate=0.0):
    """Element test of iron/common/test_utils.py:18-119:
    pass iff |a-b| < max(abs_tol, rel_tol*(|a|+|b|)); returns failing indices
    when more than max_error_rate of the elements fail."""
    a = output.detach().float().cpu().reshape(-1)
    b = reference.detach().float().cpu().reshape(-1)[: a.numel()]
    diff = (a - b).abs()
    tol = torch.maximum(torch.full_like(diff, abs_tol), rel_tol * (a.abs() + b.abs()))
    bad = ~((diff < tol) | (a == b))
    bad &= ~(torch.isnan(a) & torch.isnan(b))
    n_bad = int(bad.sum())
    if n_bad == 0 or n_bad <= max_error_rate * a.numel():
        return []
    return torch.nonzero(bad).flatten().tolist()


def bf16_ulp(ref: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 numbers at |ref| (2^(floor(log2|ref|) - 7)); tiny floor at 0."""
    r = ref.detach().double().abs().clamp_min(2.0**-126)
    return torch.exp2(torch.floor(torch.log2(r)) - 7)


def within_bf16_ulps(out, ref32, n_ulp=1.0, atol=0.0):
    """Element-wise |out - ref| <= n_ulp * ulp_bf16(ref) + atol, ref unrounded.

    A correctly rounded bf16 result sits within half an ulp of the exact value;
    one ulp leaves room for fp32 summation-order differences that flip a
    rounding. Returns the failing indices.
    """
    o = out.detach().double().cpu().reshape(-1)
    r = ref32.detach().double().cpu().reshape(-1)
    bad = (o - r).abs() > n_ulp * bf16_ulp(r) + atol
    return torch.nonzero(bad).flatten().tolist()


def max_abs_rel_l2(out, ref):
    """(max |out-ref|, ||out-ref|| / ||ref||) in float64 — the BASELINE bf16 bar."""
    o = out.detach().double().cpu().reshape(-1)
    r = ref.detach().double().cpu().reshape(-1)
    d = o - r
    return float(d.abs().max()), float(d.norm() / max(r.norm(), 1e-30))


# ------------------------------------------------------------- data movement
def transpose_reference(x, M, N):
    """Each (M, N) matrix of x transposed (transpose/reference.py:7-10)."""
    return x.reshape(-1, M, N).transpose(-2, -1).contiguous()


def repeat_reference(x, repeat):
    """Repeat-interleave along dim 0 (repeat/reference.py:7-9)."""
    return x.repeat_interleave(repeat, dim=0)


def _pad_to_4d(sizes, strides):
    return [1] * (4 - len(sizes)) + list(sizes), [0] * (4 - len(strides)) + list(strides)


def _tap_offsets(sizes, strides, offset):
    grids = np.meshgrid(*[np.arange(s) for s in sizes], indexing="ij")
    flat = np.full(grids[0].shape, offset, dtype=np.int64)
    for grid, stride in zip(grids, strides):
        flat = flat + grid * stride
    return flat.reshape(-1)


def _channel_offsets(sizes, strides, offset, channels):
    sizes, strides = _pad_to_4d(sizes, strides)
    highest = max(i for i, s in enumerate(sizes) if s >= 1)
    per = sizes[highest] // channels
    split = sizes[:highest] + [per] + sizes[highest + 1 :]
    return [_tap_offsets(split, strides, offset + c * per * strides[highest]) for c in range(channels)]


def strided_copy_reference(input_flat, input_sizes, input_strides, input_offset, output_buffer_size, output_sizes,
                           output_strides, output_offset, num_aie_channels=1, input_offset_addend=0,
                           output_offset_addend=0, out=None):
    """Gather by the input pattern, scatter by the output pattern, channel by
    channel (strided_copy/reference.py:9-75). The reference starts from a zero
    output; ``out`` gives the prior contents instead (elements outside the
    output pattern keep them, as on the device).
    PINNED BY: nested-loop brute force and the KV-cache append identity."""
    src = _channel_offsets(input_sizes, input_strides, input_offset + input_offset_addend, num_aie_channels)
    dst = _channel_offsets(output_sizes, output_strides, output_offset + output_offset_addend, num_aie_channels)
    res = torch.zeros(int(output_buffer_size), dtype=input_flat.dtype) if out is None else out.clone()
    for s, d in zip(src, dst):
        if len(s) != len(d):
            raise ValueError(f"tap element counts differ ({len(s)} vs {len(d)})")
        res[torch.from_numpy(d)] = input_flat[torch.from_numpy(s)]
    return res

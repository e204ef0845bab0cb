"""BASELINE.json configurations as seeded synthetic inputs (TEST INFRASTRUCTURE).

Generation convention (seed 0 unless a test passes another): a CPU torch
generator, values drawn in fp32 and rounded once to bf16. The same tensors feed
the GPU run (copied to HBM) and the CPU oracle / baseline.
"""

from __future__ import annotations

import torch

from . import ops

BF16 = torch.bfloat16


def _gen(seed):
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def cfg1_gemv_bf16(M=2048, K=8192, seed=0):
    """Config 1: W (M,K) ~N(0,0.02^2), x (K,) ~N(0,1), bf16."""
    g = _gen(seed)
    W = (torch.randn(M, K, generator=g) * 0.02).to(BF16)
    x = torch.randn(K, generator=g).to(BF16)
    return W, x


def cfg2_gemv_int4(M=8192, K=2048, seed=0):
    """Config 2: signed int4 q ~U{-8..7} packed along K low nibble first,
    scales ~U[0.001,0.01] bf16 per 32-group, x ~N(0,1) bf16."""
    g = _gen(seed)
    q = torch.randint(-8, 8, (M, K), generator=g, dtype=torch.int16)
    scales = (0.001 + 0.009 * torch.rand(M, K // 32, generator=g)).to(BF16)
    x = torch.randn(K, generator=g).to(BF16)
    return ops.pack_int4(q), scales, x


def cfg3_gqa_decode(n_heads=32, n_kv=8, head_dim=64, L=2048, seed=0):
    """Config 3: q (H,d), new k/v (Hkv,d) and a cache holding L-1 earlier
    positions (Hkv, L, d), all ~N(0,1) bf16; the new token sits at position L-1.
    Returns (q, k_new, v_new, k_cache, v_cache, pos, angles)."""
    g = _gen(seed)
    q = torch.randn(n_heads, head_dim, generator=g).to(BF16)
    k_new = torch.randn(n_kv, head_dim, generator=g).to(BF16)
    v_new = torch.randn(n_kv, head_dim, generator=g).to(BF16)
    k_cache = torch.randn(n_kv, L, head_dim, generator=g).to(BF16)
    v_cache = torch.randn(n_kv, L, head_dim, generator=g).to(BF16)
    pos = L - 1
    angles = ops.rope_angles_table(head_dim, L, theta=500000.0)
    return q, k_new, v_new, k_cache, v_cache, pos, angles


def cfg4_swiglu_block(hidden=2048, inter=8192, seed=0):
    """Config 4: x (hidden,) ~N(0,1); RMSNorm w ~N(1,0.1^2); Wg, Wu (inter,hidden)
    and Wd (hidden,inter) ~N(0,0.02^2), bf16."""
    g = _gen(seed)
    x = torch.randn(hidden, generator=g).to(BF16)
    norm_w = (1.0 + 0.1 * torch.randn(hidden, generator=g)).to(BF16)
    Wg = (torch.randn(inter, hidden, generator=g) * 0.02).to(BF16)
    Wu = (torch.randn(inter, hidden, generator=g) * 0.02).to(BF16)
    Wd = (torch.randn(hidden, inter, generator=g) * 0.02).to(BF16)
    return x, norm_w, Wg, Wu, Wd

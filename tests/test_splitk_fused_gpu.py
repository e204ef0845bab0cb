"""Split-K GEMM partials merged by their consumer (iron_gemm_nt_partials feeding
iron_rmsnorm_splitk and iron_qkv_rope_scatter_splitk) against the unfused
chain (iron_gemm_bf16_nt_splitk / iron_gemm_i4g32_nt, then iron_rmsnorm /
iron_qkv_rope_scatter): bit-identical outputs, KV-cache rows and residual
stream. The unfused chain is checked against the oracle (RMSNorm of
rms_norm/reference.py:7-16 with the residual add, RoPE of
rope/reference.py:69-102) within bf16 rounding."""

import pytest
import torch

from oracle import ops

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16


def _partials(lib, s, gpu, A, W, splits, int4):
    """(workspace, reference GEMM output C via the split-K GEMM with its own merge)."""
    M, K = A.shape
    N = W.shape[0]
    need = int(lib.query("iron_gemm_splitk_workspace_bytes", M, N, splits))
    ws = torch.empty(need, dtype=torch.uint8, device=gpu)
    ws2 = torch.empty(need, dtype=torch.uint8, device=gpu)
    C = torch.empty(M, N, dtype=BF16, device=gpu)
    if int4:
        codes, scales = ops.quantize_int4_g32(W)
        cd, sd = codes.to(gpu), scales.to(gpu)
        lib.call("iron_gemm_nt_partials", A.data_ptr(), None, cd.data_ptr(), sd.data_ptr(), 1, M, N, K, splits,
                 ws.data_ptr(), need, s)
        lib.call("iron_gemm_i4g32_nt", A.data_ptr(), cd.data_ptr(), sd.data_ptr(), C.data_ptr(), M, N, K, N, 0, 0,
                 0.0, 0.0, 1, splits, ws2.data_ptr(), need, s)
    else:
        lib.call("iron_gemm_nt_partials", A.data_ptr(), W.data_ptr(), None, None, 1, M, N, K, splits, ws.data_ptr(),
                 need, s)
        lib.call("iron_gemm_bf16_nt_splitk", A.data_ptr(), W.data_ptr(), C.data_ptr(), M, N, K, N, 0, 0, 0.0, 0.0,
                 splits, ws2.data_ptr(), need, s)
    return ws, C


@pytest.mark.parametrize("M,K,N,splits,int4", [(512, 2048, 2048, 4, False), (512, 8192, 2048, 4, False),
                                              (37, 1024, 264, 2, False), (100, 2048, 1024, 8, False),
                                              (512, 2048, 2048, 4, True), (64, 4096, 512, 2, True)])
def test_rmsnorm_splitk_matches_unfused(gpu, M, K, N, splits, int4):
    from iron_amd import _lib

    print(f"rmsnorm_splitk M={M} K={K} N={N} splits={splits} int4={int4}", flush=True)
    g = torch.Generator().manual_seed(M * 7 + N + splits)
    A = (torch.randn(M, K, generator=g) * 0.5).to(BF16).to(gpu)
    W = (torch.randn(N, K, generator=g) * 0.05).to(BF16)
    X0 = torch.randn(M, N, generator=g).to(BF16).to(gpu)
    s = _lib.stream_handle(gpu)
    ws, C = _partials(_lib, s, gpu, A, W.to(gpu) if not int4 else W, splits, int4)
    X1, X2 = X0.clone(), X0.clone()
    O1 = torch.empty(M, N, dtype=BF16, device=gpu)
    O2 = torch.empty(M, N, dtype=BF16, device=gpu)
    _lib.call("iron_rmsnorm_splitk", X1.data_ptr(), ws.data_ptr(), splits, None, O1.data_ptr(), X1.data_ptr(), M, N,
              1e-5, s)
    _lib.call("iron_rmsnorm", X2.data_ptr(), C.data_ptr(), None, O2.data_ptr(), X2.data_ptr(), M, N, 1e-5, s)
    torch.cuda.synchronize()
    assert torch.equal(O1, O2) and torch.equal(X1, X2)
    # the unfused chain against the oracle: s = bf16(x + C), out = norm(s)
    ssum = (X0.cpu().float() + C.cpu().float()).to(BF16)
    assert torch.equal(X2.cpu(), ssum)
    ref = ops.rms_norm_reference(ssum, None, 1e-5)
    assert not ops.within_bf16_ulps(O2.cpu(), ref.float(), n_ulp=1.0, atol=1e-6)


@pytest.mark.parametrize("S,H,Hkv,K,splits,pos0,int4", [(100, 4, 2, 1024, 2, 0, False), (512, 32, 8, 2048, 2, 0, False),
                                                         (64, 8, 2, 2048, 4, 37, False), (96, 4, 1, 1024, 2, 5, True)])
def test_qkv_scatter_splitk_matches_unfused(gpu, S, H, Hkv, K, splits, pos0, int4):
    from iron_amd import _lib

    print(f"qkv_scatter_splitk S={S} H={H} Hkv={Hkv} K={K} splits={splits} pos0={pos0} int4={int4}", flush=True)
    D, max_len = 64, 640
    N = (H + 2 * Hkv) * D
    g = torch.Generator().manual_seed(S + H + K + splits)
    A = (torch.randn(S, K, generator=g) * 0.5).to(BF16).to(gpu)
    W = (torch.randn(N, K, generator=g) * 0.05).to(BF16)
    angles = ops.rope_angles_table(D, max_len).to(gpu)
    s = _lib.stream_handle(gpu)
    ws, C = _partials(_lib, s, gpu, A, W.to(gpu) if not int4 else W, splits, int4)
    outs = []
    for fused in (True, False):
        q = torch.zeros(S, H * D, dtype=BF16, device=gpu)
        kc = torch.zeros(Hkv, max_len, D, dtype=BF16, device=gpu)
        vc = torch.zeros(Hkv, max_len, D, dtype=BF16, device=gpu)
        tail = (angles.data_ptr(), max_len, q.data_ptr(), kc.data_ptr(), vc.data_ptr(), S, H, Hkv, D, max_len, pos0, s)
        if fused:
            _lib.call("iron_qkv_rope_scatter_splitk", ws.data_ptr(), splits, *tail)
        else:
            _lib.call("iron_qkv_rope_scatter", C.data_ptr(), *tail)
        outs.append((q, kc, vc))
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    # the unfused chain against the oracle's two-halves RoPE at positions pos0..pos0+S-1
    q, kc, vc = (t.cpu() for t in outs[1])
    Cc = C.cpu().reshape(S, H + 2 * Hkv, D)
    ang = angles.cpu()[pos0:pos0 + S]
    for h in range(H):
        ref = ops.rope_reference(Cc[:, h], ang)
        assert not ops.within_bf16_ulps(q.reshape(S, H, D)[:, h], ref.float(), n_ulp=1.0, atol=1e-6)
    for j in range(Hkv):
        ref = ops.rope_reference(Cc[:, H + j], ang)
        assert not ops.within_bf16_ulps(kc[j, pos0:pos0 + S], ref.float(), n_ulp=1.0, atol=1e-6)
        assert torch.equal(vc[j, pos0:pos0 + S], Cc[:, H + Hkv + j])
        assert not kc[j, :pos0].any() and not kc[j, pos0 + S:].any()


@pytest.mark.parametrize("S,H,Hkv,splits,pos0", [(100, 4, 2, 2, 3), (33, 32, 8, 4, 0), (7, 8, 1, 1, 600)])
def test_qkv_scatter_vector_and_scalar_paths_agree(gpu, S, H, Hkv, splits, pos0):
    """The scatter's 16-byte path (every operand 16-byte aligned) and its
    element path (an operand that is not) write identical bits, from a bf16
    qkv and from split-K partials."""
    from iron_amd import _lib

    print(f"qkv_scatter paths S={S} H={H} Hkv={Hkv} splits={splits} pos0={pos0}", flush=True)
    D, max_len = 64, 640
    N = (H + 2 * Hkv) * D
    g = torch.Generator().manual_seed(S * 3 + H + splits)
    qkv = torch.randn(S * N, generator=g).to(BF16)
    part = torch.randn(splits * S * N, generator=g) * 0.3
    angles = ops.rope_angles_table(D, max_len).to(gpu)
    # copies at an offset of one element: 2 bytes (bf16) and 4 bytes (fp32) past a 16-byte boundary
    qkv_a = qkv.to(gpu)
    qkv_u = torch.zeros(S * N + 8, dtype=BF16, device=gpu)
    qkv_u[1:1 + S * N] = qkv_a
    part_a = part.to(gpu)
    part_u = torch.zeros(splits * S * N + 4, device=gpu)
    part_u[1:1 + splits * S * N] = part_a
    s = _lib.stream_handle(gpu)
    outs = {}
    for name, src, split in (("bf16 aligned", qkv_a.data_ptr(), 0), ("bf16 offset", qkv_u[1:].data_ptr(), 0),
                             ("partials aligned", part_a.data_ptr(), splits),
                             ("partials offset", part_u[1:].data_ptr(), splits)):
        q = torch.zeros(S, H * D, dtype=BF16, device=gpu)
        kc = torch.zeros(Hkv, max_len, D, dtype=BF16, device=gpu)
        vc = torch.zeros(Hkv, max_len, D, dtype=BF16, device=gpu)
        tail = (angles.data_ptr(), max_len, q.data_ptr(), kc.data_ptr(), vc.data_ptr(), S, H, Hkv, D, max_len, pos0, s)
        if split:
            _lib.call("iron_qkv_rope_scatter_splitk", src, split, *tail)
        else:
            _lib.call("iron_qkv_rope_scatter", src, *tail)
        outs[name] = (q, kc, vc)
    torch.cuda.synchronize()
    for a, b in (("bf16 aligned", "bf16 offset"), ("partials aligned", "partials offset")):
        for x, y in zip(outs[a], outs[b]):
            assert torch.equal(x, y), (a, b)
    # the bf16 path against the oracle's RoPE; v rows copied exactly
    q, kc, vc = (t.cpu() for t in outs["bf16 aligned"])
    rows = qkv.reshape(S, H + 2 * Hkv, D)
    ang = angles.cpu()[pos0:pos0 + S]
    for h in range(H):
        ref = ops.rope_reference(rows[:, h], ang)
        assert not ops.within_bf16_ulps(q.reshape(S, H, D)[:, h], ref.float(), n_ulp=1.0, atol=1e-6)
    for j in range(Hkv):
        ref = ops.rope_reference(rows[:, H + j], ang)
        assert not ops.within_bf16_ulps(kc[j, pos0:pos0 + S], ref.float(), n_ulp=1.0, atol=1e-6)
        assert torch.equal(vc[j, pos0:pos0 + S], rows[:, H + Hkv + j])
    # the partials path: the v rows are the partial sums in range order, rounded once
    vsum = part.reshape(splits, S, H + 2 * Hkv, D).sum(0) if splits > 1 else part.reshape(S, H + 2 * Hkv, D)
    vc_p = outs["partials aligned"][2].cpu()
    for j in range(Hkv):
        exact = torch.zeros(S, D)
        for kb in range(splits):
            exact = exact + part.reshape(splits, S, H + 2 * Hkv, D)[kb, :, H + Hkv + j]
        assert torch.equal(vc_p[j, pos0:pos0 + S], exact.to(BF16))
        assert torch.allclose(exact, vsum[:, H + Hkv + j], atol=1e-5)

"""GPU parity: GQA decode (split-K flash-decode) and MHA prefill against the oracle.

BASELINE config 3 (32 q-heads, 8 KV heads, d 64, KV length 2048, RoPE llama3
theta 500000 at position 2047, scale 1/8, fp32 softmax) at full size, plus
positions on and around the 64-position chunk edges, the first token and the
last cache slot. MHA follows the reference test list (mha/test.py:13-31) and
tolerance (rel 4e-2 / abs 0.15, 0.5% mismatches allowed).
"""

import math

import pytest
import torch

from oracle import configs, ops

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16


def _run_decode(gpu, q, kn, vn, kc, vc, pos, angles, max_len, pos_tensor=False, op=None, fill=0.0):
    """One decode step through the GQADecode operator. The cache rows before pos
    hold kc/vc; the rows from pos on hold `fill` (stale data the step must not
    read: only row pos is written, the rest stays masked)."""
    from iron_amd.operators import GQADecode

    H, Hkv = q.shape[0], kn.shape[0]
    if op is None:
        op = GQADecode(num_heads=H, num_kv_heads=Hkv, head_dim=64, max_len=max_len, angle_rows=angles.shape[0])
    kcd = torch.full((Hkv, max_len, 64), fill, dtype=BF16, device=gpu)
    vcd = torch.full((Hkv, max_len, 64), fill, dtype=BF16, device=gpu)
    kcd[:, :pos] = kc[:, :pos].to(gpu)
    vcd[:, :pos] = vc[:, :pos].to(gpu)
    out = torch.empty(H, 64, dtype=BF16, device=gpu)
    if pos_tensor:
        op.position_tensor = torch.tensor([pos], dtype=torch.int32, device=gpu)
    else:
        op.position_tensor = None
        op.set_position(pos)
    fn = op.get_callable()
    fn(q.to(gpu), kn.to(gpu), vn.to(gpu), kcd, vcd, angles.to(gpu), out)
    torch.cuda.synchronize()
    return out.cpu(), kcd.cpu(), vcd.cpu(), op


def _counters(op, gpu):
    """The workspace's arrival counters (one 128-byte line per KV head)."""
    ws = op.workspace(torch.device(gpu))
    return ws[: 128 * op.num_kv_heads].view(torch.int32).view(op.num_kv_heads, 32)[:, 0].cpu()


def test_config3_gqa_decode(gpu):
    q, kn, vn, kc, vc, pos, angles = configs.cfg3_gqa_decode()
    ref, kref, vref = ops.gqa_decode_reference(q, kn, vn, kc, vc, pos, angles)
    out, kcd, vcd, _ = _run_decode(gpu, q, kn, vn, kc, vc, pos, angles, max_len=2048)
    max_abs, rel_l2 = ops.max_abs_rel_l2(out, ref)
    assert max_abs <= 2e-2 and rel_l2 <= 1e-2, (max_abs, rel_l2)
    # the new key (rotated) and value are appended at pos, bit-exact
    assert torch.equal(kcd[:, pos], kref[:, pos]) and torch.equal(vcd[:, pos], vref[:, pos])


@pytest.mark.parametrize("pos", [0, 1, 15, 16, 63, 64, 65, 127, 128, 129, 255, 1000, 4095])
@pytest.mark.parametrize("use_tensor", [False, True])
def test_gqa_decode_positions(gpu, pos, use_tensor):
    max_len = 4096
    q, kn, vn, kc, vc, _, _ = configs.cfg3_gqa_decode(L=max_len, seed=pos + 1)
    angles = ops.rope_angles_table(64, max_len)
    ref, kref, _ = ops.gqa_decode_reference(q, kn, vn, kc, vc, pos, angles)
    out, kcd, _, _ = _run_decode(gpu, q, kn, vn, kc, vc, pos, angles, max_len, pos_tensor=use_tensor)
    max_abs, rel_l2 = ops.max_abs_rel_l2(out, ref)
    assert max_abs <= 2e-2 and rel_l2 <= 1e-2, (pos, max_abs, rel_l2)
    assert torch.equal(kcd[:, pos], kref[:, pos])


# n_kv_heads a multiple of 8: one launch (merge in the last workgroup of each
# KV head); otherwise partials + merge kernel. Every group size on both.
@pytest.mark.parametrize("H,Hkv", [(32, 32), (32, 16), (64, 8), (8, 8), (16, 2), (8, 2), (8, 4), (4, 4), (24, 24)])
def test_gqa_decode_group_sizes(gpu, H, Hkv):
    q, kn, vn, kc, vc, pos, angles = configs.cfg3_gqa_decode(n_heads=H, n_kv=Hkv, L=300, seed=3)
    ref, kref, vref = ops.gqa_decode_reference(q, kn, vn, kc, vc, pos, angles)
    out, kcd, vcd, _ = _run_decode(gpu, q, kn, vn, kc, vc, pos, angles, max_len=512)
    max_abs, rel_l2 = ops.max_abs_rel_l2(out, ref)
    assert max_abs <= 2e-2 and rel_l2 <= 1e-2, (max_abs, rel_l2)
    assert torch.equal(kcd[:, pos], kref[:, pos]) and torch.equal(vcd[:, pos], vref[:, pos])


# A long cache (max_len / 128 chunks x Hkv >= the CU count) takes 128-position
# chunks of 8 waves on the one-launch path; every group size there, with
# stale NaN rows past pos and a reused workspace (counters back at zero).
@pytest.mark.parametrize("H,Hkv", [(8, 8), (16, 8), (32, 8), (64, 8), (32, 16), (64, 32)])
def test_gqa_decode_long_cache_group_sizes(gpu, H, Hkv):
    max_len = 4224  # 33 chunks of 128 per KV head
    q, kn, vn, kc, vc, _, _ = configs.cfg3_gqa_decode(n_heads=H, n_kv=Hkv, L=max_len, seed=H + Hkv)
    angles = ops.rope_angles_table(64, max_len)
    op = None
    for pos in (4223, 2049, 127, 4100):
        ref, kref, vref = ops.gqa_decode_reference(q, kn, vn, kc, vc, pos, angles)
        out, kcd, vcd, op = _run_decode(gpu, q, kn, vn, kc, vc, pos, angles, max_len, op=op, fill=float("nan"))
        assert torch.isfinite(out.float()).all(), pos
        max_abs, rel_l2 = ops.max_abs_rel_l2(out, ref)
        assert max_abs <= 2e-2 and rel_l2 <= 1e-2, (pos, max_abs, rel_l2)
        for name, got, want in (("k", kcd[:, pos], kref[:, pos]), ("v", vcd[:, pos], vref[:, pos])):
            bad = (got.view(torch.int16) != want.view(torch.int16)).nonzero().tolist()
            assert not bad, (pos, name, bad[:8], got.float().flatten()[:4].tolist(), want.float().flatten()[:4].tolist())
        assert int(_counters(op, gpu).abs().sum()) == 0, pos


@pytest.mark.parametrize("Hkv,max_len", [(8, 512), (8, 4224), (2, 512)])
def test_gqa_decode_device_position_out_of_range_changes_nothing(gpu, Hkv, max_len):
    """A device position outside the cache cannot be refused on the host: the
    call leaves the output, the caches and the counters as they were, on every
    launch path, and the next call with a valid position is exact."""
    from iron_amd.operators import GQADecode

    H = 4 * Hkv
    q, kn, vn, kc, vc, _, _ = configs.cfg3_gqa_decode(n_heads=H, n_kv=Hkv, L=max_len, seed=Hkv + max_len)
    angles = ops.rope_angles_table(64, max_len)
    op = GQADecode(num_heads=H, num_kv_heads=Hkv, head_dim=64, max_len=max_len, angle_rows=max_len)
    kcd, vcd = kc.to(gpu).contiguous(), vc.to(gpu).contiguous()
    k0, v0 = kcd.clone(), vcd.clone()
    out = torch.full((H, 64), 3.0, dtype=BF16, device=gpu)
    fn = op.get_callable()
    for bad in (max_len, max_len + 1000, -1):
        op.position_tensor = torch.tensor([bad], dtype=torch.int32, device=gpu)
        fn(q.to(gpu), kn.to(gpu), vn.to(gpu), kcd, vcd, angles.to(gpu), out)
        torch.cuda.synchronize()
        assert torch.all(out == 3.0), bad
        assert torch.equal(kcd, k0) and torch.equal(vcd, v0), bad
        assert int(_counters(op, gpu).abs().sum()) == 0, bad
    pos = max_len - 1
    op.position_tensor = torch.tensor([pos], dtype=torch.int32, device=gpu)
    fn(q.to(gpu), kn.to(gpu), vn.to(gpu), kcd, vcd, angles.to(gpu), out)
    torch.cuda.synchronize()
    ref, kref, _ = ops.gqa_decode_reference(q, kn, vn, kc, vc, pos, angles)
    max_abs, rel_l2 = ops.max_abs_rel_l2(out.cpu(), ref)
    assert max_abs <= 2e-2 and rel_l2 <= 1e-2, (max_abs, rel_l2)
    assert torch.equal(kcd[:, pos].cpu(), kref[:, pos])


def test_gqa_decode_position_hint_picks_the_shape(gpu):
    """With a device position, the host position is a hint that picks the
    launch shape (64- or 128-position chunks) and nothing else: both shapes
    match the oracle at the same device position, and the shape query reports
    what each hint picks (64 below the CUs' worth of 128-position chunks, or
    half of it for resident caches; 128 above)."""
    from iron_amd import _lib
    max_len = 4224
    s = _lib.stream_handle(gpu)
    shape = lambda p: _lib.query("iron_gqa_decode_chunk_positions", 32, 8, 64, max_len, p, s)
    shape_ex = lambda p, f: _lib.query("iron_gqa_decode_chunk_positions_ex", 32, 8, 64, max_len, p, f, s)
    assert shape(0) == 64 and shape(max_len - 1) == 128 and shape(-1) == 128
    cus = torch.cuda.get_device_properties(gpu).multi_processor_count
    mid = 128 * (cus // 8 - 1) - 1  # last position whose 128-position chunks (8 KV heads) stay below the CU count
    assert shape(mid) == 64 and shape_ex(mid, 0) == 64 and shape_ex(mid, 1) == 128 and shape_ex(mid, 3) == 128
    assert shape_ex(0, 1) == 64 and shape_ex(max_len - 1, 0) == 128 and shape_ex(0, 4) == -1
    assert _lib.query("iron_gqa_decode_chunk_positions", 8, 2, 64, max_len, max_len - 1, s) == 64  # two launches
    assert _lib.query("iron_gqa_decode_chunk_positions", 32, 2, 64, max_len, 0, s) == -1  # group of 16
    assert _lib.query("iron_gqa_decode_chunk_positions", 32, 8, 32, max_len, 0, s) == -1
    q, kn, vn, kc, vc, _, _ = configs.cfg3_gqa_decode(L=max_len, seed=21)
    angles = ops.rope_angles_table(64, max_len)
    from iron_amd.operators import GQADecode
    for pos in (3000, 130):
        ref, _, _ = ops.gqa_decode_reference(q, kn, vn, kc, vc, pos, angles)
        for hint in (0, max_len - 1):
            op = GQADecode(num_heads=32, num_kv_heads=8, head_dim=64, max_len=max_len, angle_rows=max_len)
            op.set_position(hint)
            op.position_tensor = torch.tensor([pos], dtype=torch.int32, device=gpu)
            kcd, vcd = kc.to(gpu).contiguous(), vc.to(gpu).contiguous()
            out = torch.empty(32, 64, dtype=BF16, device=gpu)
            op.get_callable()(q.to(gpu), kn.to(gpu), vn.to(gpu), kcd, vcd, angles.to(gpu), out)
            torch.cuda.synchronize()
            max_abs, rel_l2 = ops.max_abs_rel_l2(out.cpu(), ref)
            assert max_abs <= 2e-2 and rel_l2 <= 1e-2, (pos, hint, max_abs, rel_l2)


@pytest.mark.parametrize("Hkv", [8, 2])
@pytest.mark.parametrize("fill", [float("nan"), float("inf")])
@pytest.mark.parametrize("pos", [0, 70, 383])
def test_gqa_decode_ignores_stale_rows(gpu, Hkv, fill, pos):
    """Cache rows past pos (in the last chunk and the whole chunks after it)
    hold NaN or inf: neither their scores nor their values may reach the
    output, on both launch paths."""
    q, kn, vn, kc, vc, _, _ = configs.cfg3_gqa_decode(n_heads=4 * Hkv, n_kv=Hkv, L=512, seed=pos + 5)
    angles = ops.rope_angles_table(64, 512)
    ref, _, _ = ops.gqa_decode_reference(q, kn, vn, kc, vc, pos, angles)
    out, _, _, _ = _run_decode(gpu, q, kn, vn, kc, vc, pos, angles, max_len=512, fill=fill)
    assert torch.isfinite(out.float()).all()
    max_abs, rel_l2 = ops.max_abs_rel_l2(out, ref)
    assert max_abs <= 2e-2 and rel_l2 <= 1e-2, (max_abs, rel_l2)


@pytest.mark.parametrize("Hkv", [8, 16, 2])
def test_gqa_decode_workspace_reuse(gpu, Hkv):
    """One operator and workspace over calls at changing positions (so the
    number of active chunks changes from call to call): every call matches the
    oracle, repeats are bitwise equal, and the arrival counters are back at
    zero after each call."""
    max_len = 640
    q, kn, vn, kc, vc, _, _ = configs.cfg3_gqa_decode(n_heads=4 * Hkv, n_kv=Hkv, L=max_len, seed=11)
    angles = ops.rope_angles_table(64, max_len)
    op = None
    first = {}
    for pos in [500, 100, 300, 37, 639, 0, 500, 100]:
        out, _, _, op = _run_decode(gpu, q, kn, vn, kc, vc, pos, angles, max_len, op=op, pos_tensor=pos % 2 == 1)
        ref, _, _ = ops.gqa_decode_reference(q, kn, vn, kc, vc, pos, angles)
        max_abs, rel_l2 = ops.max_abs_rel_l2(out, ref)
        assert max_abs <= 2e-2 and rel_l2 <= 1e-2, (pos, max_abs, rel_l2)
        if pos in first:
            assert torch.equal(out, first[pos]), pos
        first[pos] = out
        assert int(_counters(op, gpu).abs().sum()) == 0, pos


@pytest.mark.parametrize("workgroups", [8, 256, 576, 1000, 4104])
def test_xcd_dispatch_is_round_robin(gpu, workgroups):
    """The one-launch decode needs workgroups whose linear ids agree mod 8 to
    share an XCD (and so an L2). Read each workgroup's XCC_ID and check it."""
    from iron_amd import _lib

    ids = torch.full((workgroups,), -1, dtype=torch.int32, device=gpu)
    _lib.call("iron_probe_xcc_ids", workgroups, ids.data_ptr(), _lib.stream_handle(gpu))
    torch.cuda.synchronize()
    h = ids.cpu()
    assert int(h.min()) >= 0
    n = torch.arange(workgroups)
    assert torch.equal(h, h[n % 8]), h[:16].tolist()
    assert len(set(h[:8].tolist())) == 8  # eight XCDs, one class each


@pytest.mark.parametrize(
    "seq_len,heads,kv",
    [(16384, 1, 0), (2048, 8, 2), (1000, 4, 4), (64, 2, 1), (100, 32, 8), (512, 32, 8)],
)
def test_mha_causal(gpu, seq_len, heads, kv):
    from iron_amd.operators import MHA

    g = ops.mha_golden(heads=heads, S_q=seq_len, S_kv=seq_len, d=64, num_kv_heads=kv)
    op = MHA(num_heads=heads, seq_len=seq_len, d=64, num_KV_heads=kv)
    sp = op.seq_padded
    pad = lambda t: torch.nn.functional.pad(t, (0, 0, 0, sp - seq_len))
    Q, K, V = pad(g["Q"]), pad(g["K"]), pad(g["V"])
    O = torch.empty(Q.numel(), dtype=BF16, device=gpu)
    op.get_callable()(Q.to(gpu).flatten(), K.to(gpu).flatten(), V.to(gpu).flatten(), O)
    torch.cuda.synchronize()
    ref = pad(g["O"])
    errs = ops.verify_buffer(O, ref, rel_tol=4e-2, abs_tol=1.5e-1, max_error_rate=0.005)
    assert not errs, f"{len(errs)} mismatches"
    assert torch.all(O.view(heads, sp, 64)[:, seq_len:].cpu() == 0)


@pytest.mark.parametrize(
    "H,Hkv,Sq,Skv,causal,q_offset",
    [
        (32, 8, 512, 512, 1, 0),  # config 5 prefill, model layout (cache of 4096 rows)
        (32, 8, 200, 712, 1, 512),  # a second chunk: queries at positions 512..711 over the cache
        (32, 8, 1, 4096, 1, 4095),  # one query at the last cache slot
        (4, 2, 300, 300, 0, 0),  # not causal
        (8, 1, 77, 130, 0, 0),  # not causal, Skv not a multiple of the 64-key block
        (2, 2, 129, 1000, 1, 871),  # ragged query tile, long visible prefix
        # more heads and longer prompts: many query tiles per head, all CUs busy
        (32, 8, 2048, 2048, 1, 0),  # causal, the long-prompt shape
        (64, 8, 1100, 1100, 1, 0),  # causal, ragged last tile
        (256, 32, 300, 700, 1, 400),  # a second chunk over the cache
        (96, 8, 513, 1000, 0, 0),  # not causal, Skv not a multiple of the 64-key block
        (128, 128, 257, 257, 0, 0),  # one query head per KV head
        (256, 8, 1, 4096, 1, 4095),  # one query at the last cache slot
    ],
)
def test_attention_prefill_abi(gpu, H, Hkv, Sq, Skv, causal, q_offset):
    """iron_attention_prefill through the C ABI with the model's strided layout
    (Q rows of H*64, a KV cache of (Hkv, max_len, 64)) against the fp32 oracle,
    BASELINE bar: max-abs 2e-2, rel-L2 1e-2. Output rows past Sq up to out_rows
    are zero."""
    from iron_amd import _lib

    d, max_len = 64, 4096
    g = torch.Generator().manual_seed(H * 1000 + Sq + Skv + q_offset)
    Q = torch.randn(Sq, H, d, generator=g).to(BF16)
    Kc = torch.randn(Hkv, max_len, d, generator=g).to(BF16)
    Vc = torch.randn(Hkv, max_len, d, generator=g).to(BF16)
    out_rows = Sq + 5
    O = torch.full((out_rows, H, d), float("nan"), dtype=BF16, device=gpu)
    Qd, Kd, Vd = Q.to(gpu), Kc.to(gpu), Vc.to(gpu)
    scale = 1.0 / math.sqrt(d)
    _lib.call("iron_attention_prefill", Qd.data_ptr(), Kd.data_ptr(), Vd.data_ptr(), O.data_ptr(), H, Hkv, Sq, Skv, d,
              d, H * d, max_len * d, d, d, H * d, out_rows, causal, q_offset, scale, _lib.stream_handle(gpu))
    torch.cuda.synchronize()
    ref = ops.attention_reference(Q.permute(1, 0, 2), Kc[:, :Skv], Vc[:, :Skv], causal=bool(causal), scale=scale,
                                  q_offset=q_offset)
    got = O[:Sq].cpu().permute(1, 0, 2)
    max_abs, rel_l2 = ops.max_abs_rel_l2(got, ref)
    assert max_abs <= 2e-2 and rel_l2 <= 1e-2, (max_abs, rel_l2)
    assert torch.all(O[Sq:].cpu() == 0)


@pytest.mark.parametrize("Hkv", [8, 2])
@pytest.mark.parametrize("pos", [0, 200, 511])
def test_gqa_decode_ex_resident_matches(gpu, Hkv, pos):
    """iron_gqa_decode_ex with IRON_GQA_KV_RESIDENT (allocating K/V loads) gives
    the bits of iron_gqa_decode (streaming loads): outputs and appended cache
    rows, on the one-launch path (Hkv 8) and the two-kernel path (Hkv 2)."""
    from iron_amd import _lib

    H, max_len = 4 * Hkv, 512
    q, kn, vn, kc, vc, _, _ = configs.cfg3_gqa_decode(n_heads=H, n_kv=Hkv, L=max_len, seed=pos + 21)
    angles = ops.rope_angles_table(64, max_len).to(gpu)
    ws_bytes = int(_lib.query("iron_gqa_decode_workspace_bytes", H, Hkv, 64, max_len))
    results = []
    for fn, extra in (("iron_gqa_decode", ()), ("iron_gqa_decode_ex", (1,))):
        qd, knd, vnd = q.to(gpu), kn.to(gpu), vn.to(gpu)
        kcd, vcd = kc.to(gpu).clone(), vc.to(gpu).clone()
        out = torch.empty(H, 64, dtype=torch.bfloat16, device=gpu)
        ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=gpu)
        _lib.call(fn, qd.data_ptr(), knd.data_ptr(), vnd.data_ptr(), kcd.data_ptr(), vcd.data_ptr(), angles.data_ptr(),
                  angles.shape[0], out.data_ptr(), ws.data_ptr(), H, Hkv, 64, max_len, pos, None, 0.125, *extra,
                  _lib.stream_handle(gpu))
        torch.cuda.synchronize()
        results.append((out.cpu(), kcd.cpu(), vcd.cpu()))
    (o0, k0, v0), (o1, k1, v1) = results
    assert torch.equal(o0, o1) and torch.equal(k0, k1) and torch.equal(v0, v1)

"""GPU parity of the Llama runner against the fp32 CPU oracle (oracle/llama.py,
the restated llama_cpu.py), with the reference's accuracy gate
(iron/applications/llama_3.2_1b/test.py:77-97): teacher-forced, KL(ref || gpu)
<= 0.1 at prefill and <= 0.05 per decode step, plus top-1 agreement; and its
determinism gate (test.py:100-113): bitwise-identical logits across runs.

The oracle runs with the GPU model's effective weights (the int4-g32
dequantised matrices), so the comparison isolates the kernels.
"""

import pytest
import torch

from oracle import llama as ollama

pytestmark = pytest.mark.gpu

TINY = dict(vocab_size=1000, emb_dim=256, n_layers=2, n_heads=4, n_kv_groups=2, hidden_dim=512, max_seq_len=320)


def _models(gpu, seed=0, **over):
    from iron_amd.applications.llama_3_2_1b import LlamaConfig, LlamaHIP, random_weights

    cfg = LlamaConfig(**over)
    w = random_weights(cfg, gpu, seed=seed)
    model = LlamaHIP(cfg, w, device=gpu)
    eff = {k: v.float().cpu() for k, v in model.effective_weights().items()}
    shape = ollama.LlamaShape(cfg.vocab_size, cfg.emb_dim, cfg.n_layers, cfg.n_heads, cfg.n_kv_groups, cfg.hidden_dim)
    ref = ollama.LlamaCPU(shape, eff, model.angles.cpu())
    return model, ref


def _teacher_forced(model, ref, prompt, steps, use_graph):
    model.reset()
    ref.reset()
    model.prefill(prompt)
    torch.cuda.synchronize()
    r = ref.forward(torch.tensor([prompt]))[0, -1]
    kl, top1 = ollama.kl_and_top1(r, model.logits.cpu())
    results = [(kl, top1)]
    for _ in range(steps):
        nxt = int(r.argmax())
        model.set_token(nxt)
        model.decode(1, use_graph=use_graph)
        torch.cuda.synchronize()
        r = ref.forward(torch.tensor([[nxt]]))[0, -1]
        results.append(ollama.kl_and_top1(r, model.logits.cpu()))
    return results


def test_tiny_model_int4_head(gpu):
    """LlamaConfig(head_int4=True): the tied head quantized to int4-g32 (the
    oracle gets the same dequantised head), same accuracy gate."""
    model, ref = _models(gpu, seed=5, head_int4=True, **TINY)
    assert model.head.int4 and model.head.codes is not None
    g = torch.Generator().manual_seed(6)
    prompt = torch.randint(0, 1000, (29,), generator=g).tolist()
    res = _teacher_forced(model, ref, prompt, steps=8, use_graph=True)
    assert res[0][0] <= 0.1, res[0]
    assert all(kl <= 0.05 for kl, _ in res[1:]), res
    assert sum(t for _, t in res) >= len(res) - 1, res


@pytest.mark.parametrize("use_graph", [False, True])
def test_tiny_model_teacher_forced(gpu, use_graph):
    model, ref = _models(gpu, seed=1, **TINY)
    g = torch.Generator().manual_seed(3)
    prompt = torch.randint(0, 1000, (37,), generator=g).tolist()
    res = _teacher_forced(model, ref, prompt, steps=12, use_graph=use_graph)
    assert res[0][0] <= 0.1, res[0]
    assert all(kl <= 0.05 for kl, _ in res[1:]), res
    assert sum(t for _, t in res) >= len(res) - 1, res


def test_tiny_model_bf16_linears(gpu):
    model, ref = _models(gpu, seed=2, int4=False, **TINY)
    prompt = list(range(10, 60))
    res = _teacher_forced(model, ref, prompt, steps=5, use_graph=True)
    assert res[0][0] <= 0.1 and all(kl <= 0.05 for kl, _ in res[1:]), res


def test_graph_matches_eager_bitwise(gpu):
    model, _ = _models(gpu, seed=4, **TINY)
    prompt = list(range(100, 140))
    a = model.generate(prompt, 20, use_graph=False)
    la = model.logits.clone()
    b = model.generate(prompt, 20, use_graph=True)
    lb = model.logits.clone()
    assert a == b
    assert torch.equal(la.view(torch.int16), lb.view(torch.int16))


def test_determinism_alternating_prompts(gpu):
    """Alternating two prompts over repeated rounds gives bitwise-identical logits
    (llama_inference_harness.py:201-228)."""
    model, _ = _models(gpu, seed=5, **TINY)
    prompts = [list(range(5, 45)), list(range(300, 333))]
    first = {}
    for r in range(6):
        p = r % 2
        toks = model.generate(prompts[p], 6)
        cur = (toks, model.logits.clone().view(torch.int16))
        if p in first:
            assert first[p][0] == cur[0] and torch.equal(first[p][1], cur[1]), f"round {r} differs"
        else:
            first[p] = cur


def test_full_size_model_teacher_forced(gpu):
    """Llama-3.2-1B shape (16 layers, 2048, 32/8 heads, FFN 8192, vocab 128256,
    tied head), random init, int4-g32 linears: prefill 128 tokens + 6 decode steps."""
    torch.manual_seed(0)
    model, ref = _models(gpu, seed=0, max_seq_len=512)
    g = torch.Generator().manual_seed(7)
    prompt = torch.randint(0, 128256, (128,), generator=g).tolist()
    res = _teacher_forced(model, ref, prompt, steps=6, use_graph=True)
    assert res[0][0] <= 0.1, res[0]
    assert all(kl <= 0.05 for kl, _ in res[1:]), res
    assert sum(t for _, t in res) >= len(res) - 1, res


def test_prefill_from_int4_bitwise(gpu):
    """prefill_int4=True (prefill GEMMs dequantise the int4 weights in the
    kernel, no bf16 copies; separate gate/up GEMMs + SiLU*mul) gives bitwise
    the same logits and tokens as the bf16-copy prefill (fused SwiGLU GEMM):
    the dequantised values, the MFMA order and the epilogue arithmetic match."""
    from iron_amd.applications.llama_3_2_1b import LlamaConfig, LlamaHIP, random_weights

    outs = []
    for prefill_int4 in (False, True):
        cfg = LlamaConfig(prefill_int4=prefill_int4, **TINY)
        model = LlamaHIP(cfg, random_weights(cfg, gpu, seed=6), device=gpu)
        assert (model.layers[0]["qkv"]._bf16 is None) == prefill_int4
        assert ("gate_up" in model.layers[0]) != prefill_int4  # fused SwiGLU GEMM on the bf16 path
        toks = model.generate(list(range(7, 70)), 8)
        outs.append((toks, model.logits.clone().view(torch.int16)))
    assert outs[0][0] == outs[1][0]
    assert torch.equal(outs[0][1], outs[1][1])


MID = dict(vocab_size=1000, emb_dim=1024, n_layers=2, n_heads=16, n_kv_groups=4, hidden_dim=2048, max_seq_len=320)


@pytest.mark.parametrize("prefill_int4", [False, True])
def test_prefill_fused_merge_bit_identical(gpu, prefill_int4):
    """LlamaConfig(prefill_fuse_merge=True): the split-K GEMMs' partial sums are
    merged by the RoPE scatter and the RMSNorm that consume them. Logits and KV
    caches must equal, bit for bit, those of the GEMMs' own merge, for a prompt
    and for a continuation at a later position."""
    import dataclasses

    from iron_amd import _lib
    from iron_amd.applications.llama_3_2_1b import LlamaConfig, LlamaHIP, random_weights

    cfg = LlamaConfig(prefill_int4=prefill_int4, **MID)
    # at these shapes qkv and o_proj split K in 2 ranges, down_proj in 4 (both policies)
    for q in ("iron_gemm_splitk_choose", "iron_gemm_i4g32_splitk_choose"):
        assert _lib.query(q, 64, 1536, 1024) == 2
        assert _lib.query(q, 64, 1024, 1024) == 2
        assert _lib.query(q, 64, 1024, 2048) == 4
    w = random_weights(cfg, gpu, seed=4)
    fused = LlamaHIP(cfg, w, device=gpu)
    plain = LlamaHIP(dataclasses.replace(cfg, prefill_fuse_merge=False), w, device=gpu)
    for m in (fused, plain):
        m.reset()
    for chunk in (list(range(3, 67)), [5, 900, 17, 4, 4, 250, 61]):
        for m in (fused, plain):
            m.prefill(chunk)
        torch.cuda.synchronize()
        assert torch.equal(fused.logits, plain.logits)
        for i in range(cfg.n_layers):
            assert torch.equal(fused.k_cache[i], plain.k_cache[i])
            assert torch.equal(fused.v_cache[i], plain.v_cache[i])


def test_prefill_graph_matches_eager(gpu):
    """prefill(use_graph=True): the first call of a (length, start) shape runs
    eagerly and captures it, later calls replay the graph. Logits, KV caches and
    the decode that follows must equal the eager path bit for bit, also after a
    longer prompt grows the split-K workspace (which drops the old graphs)."""
    from iron_amd.applications.llama_3_2_1b import LlamaConfig, LlamaHIP, random_weights

    cfg = LlamaConfig(**MID)
    w = random_weights(cfg, gpu, seed=6)
    gm, em = LlamaHIP(cfg, w, device=gpu), LlamaHIP(cfg, w, device=gpu)
    g = torch.Generator().manual_seed(7)
    p1 = torch.randint(0, cfg.vocab_size, (64,), generator=g).tolist()
    p2 = torch.randint(0, cfg.vocab_size, (7,), generator=g).tolist()
    long = torch.randint(0, cfg.vocab_size, (300,), generator=g).tolist()

    def same():
        torch.cuda.synchronize()
        assert torch.equal(gm.logits, em.logits)
        for i in range(cfg.n_layers):
            assert torch.equal(gm.k_cache[i], em.k_cache[i]) and torch.equal(gm.v_cache[i], em.v_cache[i])

    for rnd in range(2):  # round 0 captures, round 1 replays
        for m in (gm, em):
            m.reset()
        gm.prefill(p1, use_graph=True)
        em.prefill(p1)
        same()
        gm.prefill(p2, use_graph=True)  # continuation at position 64
        em.prefill(p2)
        same()
        assert set(gm._prefill_graphs) == {(64, 0), (7, 64)}
    for m in (gm, em):
        m.decode(3)
    same()
    for m in (gm, em):
        m.reset()
    gm.prefill(long, use_graph=True)  # grows the workspace: earlier graphs are dropped
    em.prefill(long)
    same()
    assert set(gm._prefill_graphs) == {(300, 0)}
    for m in (gm, em):
        m.reset()
    gm.prefill(p1, use_graph=True)
    gm.prefill(p1[:5], use_graph=True)
    em.prefill(p1)
    em.prefill(p1[:5])
    same()
    # at most MAX_PREFILL_GRAPHS shapes are kept, the oldest dropped first
    gm.MAX_PREFILL_GRAPHS = 2
    gm.reset()
    gm.prefill(p1[:9], use_graph=True)
    assert list(gm._prefill_graphs) == [(5, 64), (9, 0)]


def test_prefill_graph_reuse_eviction_and_regrowth(gpu):
    """Captured prefill graphs under reuse and churn, each result bit-identical
    to an eager model: a replay with other token ids of the same length; a
    larger prompt issued right after a replay, without a host synchronisation
    (its buffers and workspace grow, so every graph is dropped while the replay
    may still run); least-recently-used eviction; and an evicted shape captured
    again."""
    from iron_amd.applications.llama_3_2_1b import LlamaConfig, LlamaHIP, random_weights

    cfg = LlamaConfig(**MID)
    w = random_weights(cfg, gpu, seed=8)
    gm, em = LlamaHIP(cfg, w, device=gpu), LlamaHIP(cfg, w, device=gpu)
    g = torch.Generator().manual_seed(9)

    def ids(n):
        return torch.randint(0, cfg.vocab_size, (n,), generator=g).tolist()

    def run(prompt):
        for m in (gm, em):
            m.reset()
        gm.prefill(prompt, use_graph=True)
        em.prefill(prompt)

    def same():
        torch.cuda.synchronize()
        assert torch.equal(gm.logits, em.logits)
        for i in range(cfg.n_layers):
            assert torch.equal(gm.k_cache[i], em.k_cache[i]) and torch.equal(gm.v_cache[i], em.v_cache[i])

    run(ids(40))  # capture (40, 0)
    same()
    run(ids(40))  # replay with other ids
    same()
    gm.reset()
    gm.prefill(ids(40), use_graph=True)  # replay, then at once a longer prompt: no synchronize in between
    big = ids(200)
    gm.reset()
    gm.prefill(big, use_graph=True)
    em.reset()
    em.prefill(big)
    same()
    assert list(gm._prefill_graphs) == [(200, 0)]
    gm.MAX_PREFILL_GRAPHS = 2
    a, b, c = ids(30), ids(31), ids(32)
    run(a)
    run(b)
    run(a)  # hit: (30, 0) becomes the most recently used
    run(c)  # evicts (31, 0), the least recently used
    assert list(gm._prefill_graphs) == [(30, 0), (32, 0)]
    same()
    run(ids(31))  # the evicted shape, captured again
    same()
    run(ids(31))  # and replayed
    same()
    assert list(gm._prefill_graphs) == [(32, 0), (31, 0)]
    # buffers stay sized by the longest prompt (256 rows for 200 tokens)
    assert gm._prefill_bufs["cap"] == 256

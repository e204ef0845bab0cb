"""The one-launch decode step (iron_llama_decode_fused + iron_llama_decode_head)
against the 82-launch step it replaces, on the Llama-3.2-1B layer shape
(hidden 2048, 32/8 heads, FFN 8192, int4-g32 linears, full vocabulary) with
fewer layers: the logits of every step, the chosen tokens and the final hidden
state must be bitwise equal (the fused roles run the same arithmetic), eagerly
and replayed from the captured graph, with caches read resident and streamed,
across attention chunk boundaries. The bounded waits are forced to give up
from the host (a 1 us bound) and the model must report it, then recover.

The 82-launch step is itself pinned against the fp32 oracle (test_llama_gpu.py,
test_llama_cfg5_gpu.py); this test pins the fused step to it.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _model(gpu, n_layers=2, max_seq_len=256, seed=11):
    from iron_amd.applications.llama_3_2_1b import LlamaConfig, LlamaHIP, random_weights

    cfg = LlamaConfig(n_layers=n_layers, max_seq_len=max_seq_len, decode_fused=True)
    model = LlamaHIP(cfg, random_weights(cfg, gpu, seed=seed), device=gpu)
    assert model.fused, "the Llama-3.2-1B layer shape with int4 linears takes the one-launch step"
    return model


def _run(model, prompt, steps, fused, use_graph):
    """Prefill, then `steps` greedy decode steps one at a time; returns the
    logits after every step, the generated tokens and the final x."""
    model.fused = fused
    model.graph = model.graph_multi = None  # recapture for this path
    model.reset()
    model.prefill(prompt)
    logits, toks = [], []
    for _ in range(steps):
        model.decode(1, use_graph=use_graph)
        torch.cuda.synchronize()
        logits.append(model.logits.clone())
        toks.append(int(model.token.item()))
    return logits, toks, model.x.clone()


@pytest.mark.parametrize("use_graph", [False, True])
@pytest.mark.parametrize("resident", [True, False])
def test_fused_step_bitwise_equals_separate_launches(gpu, use_graph, resident):
    print(f"[fused step] graph={use_graph} resident={resident}", flush=True)
    model = _model(gpu)
    model.kv_flags = 1 if resident else 0
    g = torch.Generator().manual_seed(3)
    prompt = torch.randint(0, 128256, (58,), generator=g).tolist()  # decode crosses position 64
    ref_l, ref_t, ref_x = _run(model, prompt, 12, fused=False, use_graph=use_graph)
    got_l, got_t, got_x = _run(model, prompt, 12, fused=True, use_graph=use_graph)
    assert got_t == ref_t
    for i, (a, b) in enumerate(zip(got_l, ref_l)):
        assert torch.equal(a, b), f"step {i}: max |d| {(a.float() - b.float()).abs().max().item()}"
    assert torch.equal(got_x, ref_x)


def test_fused_multi_step_graph_and_long_context(gpu):
    """The 8-step graph (device-resident position and epoch advancing inside the
    replay), four layers, a prompt that fills most of the cache: tokens and
    final logits equal the separate-launch path."""
    print("[fused step] 8-step graph, 4 layers, KV 400 -> 417", flush=True)
    model = _model(gpu, n_layers=4, max_seq_len=448, seed=5)
    g = torch.Generator().manual_seed(9)
    prompt = torch.randint(0, 128256, (400,), generator=g).tolist()
    out = {}
    for fused in (False, True):
        model.fused = fused
        model.graph = model.graph_multi = None
        model.reset()
        model.prefill(prompt)
        model.decode(17, use_graph=True)
        model.commit()
        torch.cuda.synchronize()
        out[fused] = (model.history[399:417].tolist(), model.logits.clone())
    assert out[True][0] == out[False][0]
    assert torch.equal(out[True][1], out[False][1])


def test_fused_step_bounded_wait_reports_and_recovers(gpu):
    """A 1 us bound on every wait: the step cannot complete in time (layer 0
    waits for the token selection), so the waits give up, the launch still
    ends, and the model reports the status word. With the normal bound the
    next steps are again bitwise equal to the separate-launch path."""
    print("[fused step] forced give-up (1 us waits)", flush=True)
    model = _model(gpu, seed=7)
    prompt = list(range(100, 140))
    model.fused = True
    model.reset()
    model.prefill(prompt)
    bound = model.cfg.decode_wait_us
    model.cfg.decode_wait_us = 1
    with pytest.raises(RuntimeError, match="a wait gave up"):
        model.decode(1, use_graph=False)
    assert int(model.status.item()) == 0  # cleared after the report
    model.cfg.decode_wait_us = bound
    ref_l, ref_t, _ = _run(model, prompt, 4, fused=False, use_graph=False)
    got_l, got_t, _ = _run(model, prompt, 4, fused=True, use_graph=False)
    assert got_t == ref_t
    assert all(torch.equal(a, b) for a, b in zip(got_l, ref_l))

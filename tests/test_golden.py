"""The oracle and the product's host tables against the committed golden
fixtures (tests/golden/, written by transformers; see make_golden.py there).

- RoPE: transformers' llama3 inverse frequencies and cos/sin rows (BASELINE
  config 3: head_dim 64, theta 500000) against the oracle's
  compute_rope_params (rope/reference.py:7-66) and the table the Llama runner
  builds (compute_rope_angles).
- Llama: the oracle's fp32 forward (oracle/llama.py, llama_cpu.py:221-285)
  with its KV cache, teacher-forced over the fixture's greedy continuation,
  against transformers' fp32 logits.
"""

import importlib.util
from pathlib import Path

import numpy as np
import torch

from oracle import llama, ops

GOLDEN = Path(__file__).resolve().parent / "golden"


def load_make_golden():
    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_rope_oracle_matches_golden():
    f = np.load(GOLDEN / "rope_llama3_hd64.npz")
    pos = torch.from_numpy(f["positions"])
    cos, sin = ops.compute_rope_params(64, 500000.0, int(pos.max()) + 1, ops.LLAMA3_FREQ_CONFIG)
    # same fp32 formula evaluated in a different order: a few ulp
    torch.testing.assert_close(cos[pos], torch.from_numpy(f["cos"]), atol=2e-6, rtol=0)
    torch.testing.assert_close(sin[pos], torch.from_numpy(f["sin"]), atol=2e-6, rtol=0)
    assert torch.equal(cos[0], torch.ones(32)) and torch.equal(sin[0], torch.zeros(32))


def test_product_rope_table_matches_golden():
    from iron_amd.applications.llama_3_2_1b import compute_rope_angles

    f = np.load(GOLDEN / "rope_llama3_hd64.npz")
    pos = torch.from_numpy(f["positions"])
    t = compute_rope_angles(64, int(pos.max()) + 1, 500000.0, ops.LLAMA3_FREQ_CONFIG)[pos]
    torch.testing.assert_close(t[:, 0::2], torch.from_numpy(f["cos"]), atol=2e-6, rtol=0)
    torch.testing.assert_close(t[:, 1::2], torch.from_numpy(f["sin"]), atol=2e-6, rtol=0)


def test_oracle_llama_matches_golden():
    mg = load_make_golden()
    f = np.load(GOLDEN / "llama_tiny_hf.npz")
    w = mg.tiny_weights(int(f["seed"]))
    assert mg.weights_checksum(w) == float(f["weights_sum"]), "the seeded weight generator changed"
    V, E, L, H, KV, F = (int(v) for v in f["shape"])
    shape = llama.LlamaShape(vocab_size=V, emb_dim=E, n_layers=L, n_heads=H, n_kv_groups=KV, hidden_dim=F)
    prompt, cont, gold = f["prompt"].tolist(), f["continuation"].tolist(), torch.from_numpy(f["logits"])
    ora = llama.LlamaCPU(shape, {k: v.float() for k, v in w.items()}, ops.rope_angles_table(E // H, 64))
    rows = [ora.forward(torch.tensor([prompt]))[0, -1]]
    for t in cont:
        rows.append(ora.forward(torch.tensor([[t]]))[0, -1])
    out = torch.stack(rows)
    torch.testing.assert_close(out, gold, atol=2e-4, rtol=1e-4)
    assert out[:-1].argmax(-1).tolist() == cont

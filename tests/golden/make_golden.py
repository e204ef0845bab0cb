#!/usr/bin/env python3
"""Writes the golden fixtures of this directory.

The expected outputs come from transformers (an independent, published
implementation of Llama 3 and of its llama3 RoPE frequency scaling), never
from the oracle or from the reference's code; the reference's own tests hold
no committed fixtures. Run from the repository root:

    python tests/golden/make_golden.py

rope_llama3_hd64.npz
    The RoPE table of BASELINE config 3 (head_dim 64, theta 500000, llama3
    scaling factor 32 / low 1 / high 4 / original 8192; the defaults of
    iron/operators/rope/reference.py:105-125): transformers' inverse
    frequencies and its LlamaRotaryEmbedding cos/sin (fp32) at a few positions.
llama_tiny_hf.npz
    A small Llama of the reference's architecture (llama_cpu.py:221-285: RMSNorm,
    GQA with llama3 RoPE, SwiGLU, tied head) with the weights of
    ``tiny_weights()`` (seeded, bf16 values), run by transformers'
    LlamaForCausalLM in float32: a prompt, the greedy continuation, and the
    fp32 logits of the last prompt position and of every decode position
    (teacher-forced on that continuation).
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent

ROPE_POSITIONS = [0, 1, 2, 511, 512, 2047, 4095, 4607]
ROPE_SCALING = {"factor": 32.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0, "original_context_length": 8192}

TINY = dict(vocab_size=1000, emb_dim=256, n_layers=2, n_heads=4, n_kv_groups=2, hidden_dim=512)
TINY_SEED = 11
TINY_PROMPT_LEN = 24
TINY_DECODE = 8


def tiny_weights(seed: int = TINY_SEED) -> dict:
    """Hugging Face-named bf16 weights of the TINY shape: every matrix ~N(0, 1/fan_in)
    (unit gain, so the logits are peaked rather than flat), the embedding ~N(0, 0.25^2)
    and norm weights ~N(1, 0.1^2); drawn on the CPU generator in a fixed order."""
    g = torch.Generator().manual_seed(seed)
    E, H, V = TINY["emb_dim"], TINY["hidden_dim"], TINY["vocab_size"]
    hd = E // TINY["n_heads"]

    def n(rows, cols, sd):
        return (torch.randn(rows, cols, generator=g) * sd).to(torch.bfloat16)

    def norm():
        return (torch.randn(E, generator=g) * 0.1 + 1.0).to(torch.bfloat16)

    w = {"model.embed_tokens.weight": n(V, E, 0.25), "model.norm.weight": norm()}
    for i in range(TINY["n_layers"]):
        p = f"model.layers.{i}."
        w[p + "input_layernorm.weight"] = norm()
        w[p + "post_attention_layernorm.weight"] = norm()
        w[p + "self_attn.q_proj.weight"] = n(TINY["n_heads"] * hd, E, E ** -0.5)
        w[p + "self_attn.k_proj.weight"] = n(TINY["n_kv_groups"] * hd, E, E ** -0.5)
        w[p + "self_attn.v_proj.weight"] = n(TINY["n_kv_groups"] * hd, E, E ** -0.5)
        w[p + "self_attn.o_proj.weight"] = n(E, TINY["n_heads"] * hd, (TINY["n_heads"] * hd) ** -0.5)
        w[p + "mlp.gate_proj.weight"] = n(H, E, E ** -0.5)
        w[p + "mlp.up_proj.weight"] = n(H, E, E ** -0.5)
        w[p + "mlp.down_proj.weight"] = n(E, H, H ** -0.5)
    return w


def weights_checksum(w: dict) -> float:
    """Sum over every weight (float64) in name order: detects a change of the generator."""
    return float(sum(w[k].double().sum() for k in sorted(w)))


def tiny_prompt() -> list[int]:
    g = torch.Generator().manual_seed(TINY_SEED + 1)
    return torch.randint(0, TINY["vocab_size"], (TINY_PROMPT_LEN,), generator=g).tolist()


def _hf_config(vocab, emb, layers, heads, kv, hidden, max_pos=131072):
    from transformers import LlamaConfig

    return LlamaConfig(
        vocab_size=vocab, hidden_size=emb, intermediate_size=hidden, num_hidden_layers=layers,
        num_attention_heads=heads, num_key_value_heads=kv, head_dim=emb // heads, rms_norm_eps=1e-5,
        rope_theta=500000.0, max_position_embeddings=max_pos, tie_word_embeddings=True, attention_bias=False,
        mlp_bias=False,
        rope_scaling={"rope_type": "llama3", "factor": ROPE_SCALING["factor"],
                      "low_freq_factor": ROPE_SCALING["low_freq_factor"],
                      "high_freq_factor": ROPE_SCALING["high_freq_factor"],
                      "original_max_position_embeddings": ROPE_SCALING["original_context_length"]},
    )


def make_rope() -> None:
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding

    rot = LlamaRotaryEmbedding(_hf_config(16, 2048, 1, 32, 8, 64))
    pos = torch.tensor([ROPE_POSITIONS])
    x = torch.zeros(1, 1, 64, dtype=torch.float32)
    cos, sin = rot(x, pos)
    half = 32
    np.savez(
        HERE / "rope_llama3_hd64.npz",
        positions=np.array(ROPE_POSITIONS, dtype=np.int64),
        inv_freq=rot.inv_freq.float().numpy(),
        cos=cos[0, :, :half].float().numpy(),
        sin=sin[0, :, :half].float().numpy(),
    )


def make_llama_tiny() -> None:
    from transformers import LlamaForCausalLM

    cfg = _hf_config(TINY["vocab_size"], TINY["emb_dim"], TINY["n_layers"], TINY["n_heads"], TINY["n_kv_groups"],
                     TINY["hidden_dim"])
    hf = LlamaForCausalLM(cfg).eval()
    w = {k: v.float() for k, v in tiny_weights().items()}
    missing, unexpected = hf.load_state_dict(w, strict=False)
    assert not unexpected and all("lm_head" in m or "rotary" in m for m in missing), (missing, unexpected)
    prompt = tiny_prompt()
    ids = list(prompt)
    with torch.no_grad():
        for _ in range(TINY_DECODE):
            nxt = int(hf(torch.tensor([ids])).logits[0, -1].argmax())
            ids.append(nxt)
        logits = hf(torch.tensor([ids])).logits[0, TINY_PROMPT_LEN - 1 : TINY_PROMPT_LEN + TINY_DECODE].float()
    np.savez(
        HERE / "llama_tiny_hf.npz",
        shape=np.array([TINY[k] for k in ("vocab_size", "emb_dim", "n_layers", "n_heads", "n_kv_groups",
                                          "hidden_dim")], dtype=np.int64),
        seed=np.array(TINY_SEED, dtype=np.int64),
        weights_sum=np.array(weights_checksum(tiny_weights()), dtype=np.float64),
        prompt=np.array(prompt, dtype=np.int64),
        continuation=np.array(ids[TINY_PROMPT_LEN:], dtype=np.int64),
        logits=logits.numpy(),
    )


if __name__ == "__main__":
    import transformers

    torch.manual_seed(0)
    make_rope()
    make_llama_tiny()
    print(f"wrote fixtures with transformers {transformers.__version__} into {HERE}")

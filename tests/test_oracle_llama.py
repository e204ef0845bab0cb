"""Pin of the oracle Llama forward (oracle/llama.py) against transformers'
LlamaForCausalLM on identical weights (CPU, small shape). Also checks that the
product's RoPE table equals the oracle's (both restate rope/reference.py:7-66)."""

import torch

from oracle import llama, ops


def _tiny_weights(shape, seed=0):
    g = torch.Generator().manual_seed(seed)
    E, H, Hd = shape.emb_dim, shape.hidden_dim, shape.head_dim
    n = lambda *s, m=0.0, sd=0.05: torch.randn(*s, generator=g) * sd + m
    w = {"model.embed_tokens.weight": n(shape.vocab_size, E), "model.norm.weight": n(E, m=1.0, sd=0.1)}
    for i in range(shape.n_layers):
        p = f"model.layers.{i}."
        w[p + "input_layernorm.weight"] = n(E, m=1.0, sd=0.1)
        w[p + "post_attention_layernorm.weight"] = n(E, m=1.0, sd=0.1)
        w[p + "self_attn.q_proj.weight"] = n(shape.n_heads * Hd, E)
        w[p + "self_attn.k_proj.weight"] = n(shape.n_kv_groups * Hd, E)
        w[p + "self_attn.v_proj.weight"] = n(shape.n_kv_groups * Hd, E)
        w[p + "self_attn.o_proj.weight"] = n(E, shape.n_heads * Hd)
        w[p + "mlp.gate_proj.weight"] = n(H, E)
        w[p + "mlp.up_proj.weight"] = n(H, E)
        w[p + "mlp.down_proj.weight"] = n(E, H)
    return w


def test_oracle_llama_matches_transformers():
    from transformers import LlamaConfig, LlamaForCausalLM

    shape = llama.LlamaShape(vocab_size=300, emb_dim=128, n_layers=2, n_heads=2, n_kv_groups=1, hidden_dim=256)
    w = _tiny_weights(shape)
    cfg = LlamaConfig(
        vocab_size=300, hidden_size=128, intermediate_size=256, num_hidden_layers=2, num_attention_heads=2,
        num_key_value_heads=1, head_dim=64, rms_norm_eps=1e-5, rope_theta=500000.0, max_position_embeddings=4096,
        tie_word_embeddings=True, attention_bias=False, mlp_bias=False,
        rope_scaling={"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                      "original_max_position_embeddings": 8192},
    )
    hf = LlamaForCausalLM(cfg).eval()
    missing, unexpected = hf.load_state_dict(w, strict=False)
    assert not unexpected and all("lm_head" in m or "rotary" in m for m in missing)
    angles = ops.rope_angles_table(64, 64)
    ora = llama.LlamaCPU(shape, w, angles)
    ids = torch.tensor([[5, 17, 3, 250, 99, 0, 42, 7, 7, 120]])
    with torch.no_grad():
        ref = hf(ids).logits
        out = ora.forward(ids)
        assert torch.allclose(out, ref, atol=2e-4, rtol=1e-4), (out - ref).abs().max()
        # incremental decode with the KV cache equals the full forward's next position
        nxt = torch.tensor([[11]])
        step = ora.forward(nxt)
        full = hf(torch.cat([ids, nxt], dim=1)).logits[:, -1:]
        assert torch.allclose(step, full, atol=2e-4, rtol=1e-4)


def test_product_rope_table_matches_oracle():
    from iron_amd.applications.llama_3_2_1b import compute_rope_angles

    a = compute_rope_angles(64, 4096, 500000.0, ops.LLAMA3_FREQ_CONFIG)
    b = ops.rope_angles_table(64, 4096)
    assert torch.allclose(a, b, atol=1e-5, rtol=0)


def test_oracle_last_only_matches_full_forward():
    """forward(last_only=True) is the last row of the full forward, also after a
    cached prefix."""
    shape = llama.LlamaShape(vocab_size=300, emb_dim=128, n_layers=2, n_heads=2, n_kv_groups=1, hidden_dim=256)
    w = _tiny_weights(shape, seed=3)
    angles = ops.rope_angles_table(64, 64)
    a, b = llama.LlamaCPU(shape, w, angles), llama.LlamaCPU(shape, w, angles)
    for ids in (torch.tensor([[5, 17, 3, 250, 99]]), torch.tensor([[8, 1, 2]])):
        full = a.forward(ids)
        last = b.forward(ids, last_only=True)
        assert last.shape == (1, 1, 300)
        # a one-row product may sum in another order than the full one: fp32 rounding only
        assert torch.allclose(last[0, 0], full[0, -1], atol=1e-5, rtol=1e-5)

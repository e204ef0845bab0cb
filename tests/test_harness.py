"""Harness host logic on the CPU: safetensors loading and config inference,
and generate_token's sampling rule (llama_inference_harness.py:146-169)."""

import torch

from iron_amd.applications.llama_3_2_1b import config_from_weights, generate_token, load_safetensors_weights


def _tiny_weights(tied=True):
    g = torch.Generator().manual_seed(0)
    E, F, V, L = 128, 256, 300, 2
    w = {"model.embed_tokens.weight": torch.randn(V, E, generator=g).to(torch.bfloat16),
         "model.norm.weight": torch.ones(E, dtype=torch.bfloat16)}
    for i in range(L):
        p = f"model.layers.{i}."
        w[p + "self_attn.q_proj.weight"] = torch.randn(E, E, generator=g).to(torch.bfloat16)
        w[p + "self_attn.k_proj.weight"] = torch.randn(64, E, generator=g).to(torch.bfloat16)
        w[p + "self_attn.v_proj.weight"] = torch.randn(64, E, generator=g).to(torch.bfloat16)
        w[p + "self_attn.o_proj.weight"] = torch.randn(E, E, generator=g).to(torch.bfloat16)
        w[p + "mlp.gate_proj.weight"] = torch.randn(F, E, generator=g).to(torch.bfloat16)
        w[p + "mlp.up_proj.weight"] = torch.randn(F, E, generator=g).to(torch.bfloat16)
        w[p + "mlp.down_proj.weight"] = torch.randn(E, F, generator=g).to(torch.bfloat16)
        w[p + "input_layernorm.weight"] = torch.ones(E, dtype=torch.bfloat16)
        w[p + "post_attention_layernorm.weight"] = torch.ones(E, dtype=torch.bfloat16)
    w["lm_head.weight"] = w["model.embed_tokens.weight"].clone() if tied else torch.randn(V, E, generator=g).to(torch.bfloat16)
    return w


def test_safetensors_round_trip_and_config(tmp_path):
    import safetensors.torch

    for tied in (True, False):
        w = _tiny_weights(tied)
        f = tmp_path / f"m{int(tied)}.safetensors"
        safetensors.torch.save_file(w, str(f))
        got = load_safetensors_weights(f)
        assert ("lm_head.weight" in got) == (not tied)
        for k, v in got.items():
            assert torch.equal(v, w[k]), k
        cfg = config_from_weights(got, max_seq_len=256)
        assert (cfg.vocab_size, cfg.emb_dim, cfg.n_layers, cfg.n_heads, cfg.n_kv_groups, cfg.hidden_dim) == (
            300, 128, 2, 2, 1, 256)


class _Cfg:
    temperature = 0.7
    top_k = 3


def test_generate_token_samples_only_top_k():
    logits = torch.tensor([[[0.0, 5.0, 4.0, -1.0, 4.5, 3.9]]])

    def fwd(config, state):
        return logits, state

    torch.manual_seed(0)
    seen = {generate_token(_Cfg, fwd, None)[0] for _ in range(400)}
    assert seen == {1, 2, 4}
    # the sampling distribution is softmax(logits / T) over the top k
    torch.manual_seed(1)
    counts = torch.zeros(6)
    for _ in range(4000):
        counts[generate_token(_Cfg, fwd, None)[0]] += 1
    p = torch.softmax(torch.tensor([5.0, 4.0, 4.5]) / 0.7, 0)
    assert torch.allclose(counts[[1, 2, 4]] / 4000, p, atol=0.03)

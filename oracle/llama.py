"""fp32 CPU Llama forward (TEST INFRASTRUCTURE ONLY).

Restates iron/applications/llama_3.2_1b/llama_cpu.py:14-285 -- the golden the
reference checks its NPU model against (llama_npu.py:1239-1256) -- with the
causal mask generalised to a non-empty cache. Weights use the Hugging Face
names the reference loads (llama_cpu.py:225-278).
PINNED BY: transformers' LlamaForCausalLM on the same weights
(tests/test_oracle_llama.py).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch


@dataclass
class LlamaShape:
    vocab_size: int = 128256
    emb_dim: int = 2048
    n_layers: int = 16
    n_heads: int = 32
    n_kv_groups: int = 8
    hidden_dim: int = 8192

    @property
    def head_dim(self) -> int:
        return self.emb_dim // self.n_heads


def rope_forward(x, angles):
    """llama_cpu.py:14-38: x (B, S, H, D); angles (S, D) interleaved [cos, sin]."""
    d = x.shape[-1]
    x1, x2 = x[..., : d // 2], x[..., d // 2 :]
    cos = angles[:, ::2].unsqueeze(0).unsqueeze(2)
    sin = angles[:, 1::2].unsqueeze(0).unsqueeze(2)
    out = torch.empty_like(x)
    out[..., : d // 2] = x1 * cos - x2 * sin
    out[..., d // 2 :] = x1 * sin + x2 * cos
    return out


def rms_norm_forward(x, weight, eps=1e-5):
    """llama_cpu.py:41-46."""
    variance = x.pow(2).mean(-1, keepdim=True)
    return weight * (x * torch.rsqrt(variance + eps))


def gqa_forward(x, kc, vc, Wq, Wk, Wv, Wo, angles, n_heads, n_kv):
    """llama_cpu.py:49-148 with the mask over absolute positions."""
    b, s, _ = x.shape
    hd = Wq.shape[0] // n_heads
    past = kc.shape[2]
    q = torch.nn.functional.linear(x, Wq).view(b, s, n_heads, hd)
    k = torch.nn.functional.linear(x, Wk).view(b, s, n_kv, hd)
    v = torch.nn.functional.linear(x, Wv).view(b, s, n_kv, hd)
    q = rope_forward(q, angles[past : past + s])
    k = rope_forward(k, angles[past : past + s])
    q, k, v = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    kc = torch.cat([kc, k], dim=2)
    vc = torch.cat([vc, v], dim=2)
    g = n_heads // n_kv
    kk = kc.repeat_interleave(g, dim=1)
    vv = vc.repeat_interleave(g, dim=1)
    scores = torch.matmul(q, kk.transpose(-2, -1)) / math.sqrt(hd)
    qi = torch.arange(s).unsqueeze(1) + past
    kj = torch.arange(past + s).unsqueeze(0)
    scores = scores.masked_fill(kj > qi, float("-inf"))
    w = torch.softmax(scores, dim=-1)
    ctx = torch.matmul(w, vv).transpose(1, 2).contiguous().view(b, s, -1)
    return torch.nn.functional.linear(ctx, Wo), kc, vc


def swiglu_ffn_forward(x, w1, w2, w3):
    """llama_cpu.py:151-168."""
    g = torch.nn.functional.linear(x, w1)
    u = torch.nn.functional.linear(x, w2)
    return torch.nn.functional.linear(torch.nn.functional.silu(g) * u, w3)


class LlamaCPU:
    """fp32 model state: weights (name -> fp32 tensor), per-layer KV caches, angles."""

    def __init__(self, shape: LlamaShape, weights: dict, angles: torch.Tensor):
        self.shape = shape
        self.w = {k: v.float() for k, v in weights.items()}
        self.angles = angles.float()
        self.reset()

    def reset(self):
        sh = self.shape
        self.kc = [torch.empty(1, sh.n_kv_groups, 0, sh.head_dim) for _ in range(sh.n_layers)]
        self.vc = [torch.empty(1, sh.n_kv_groups, 0, sh.head_dim) for _ in range(sh.n_layers)]

    def forward(self, token_ids: torch.Tensor, last_only: bool = False) -> torch.Tensor:
        """llama_cpu.py:221-285: logits (1, S, vocab) for token_ids (1, S).

        ``last_only`` applies the final norm and the head to the last position
        only, (1, 1, vocab): the rows the accuracy gate reads, without the
        S x vocab head product of a long prompt."""
        sh, w = self.shape, self.w
        x = torch.nn.functional.embedding(token_ids, w["model.embed_tokens.weight"])
        for i in range(sh.n_layers):
            p = f"model.layers.{i}."
            h = rms_norm_forward(x, w[p + "input_layernorm.weight"])
            a, self.kc[i], self.vc[i] = gqa_forward(
                h, self.kc[i], self.vc[i], w[p + "self_attn.q_proj.weight"], w[p + "self_attn.k_proj.weight"],
                w[p + "self_attn.v_proj.weight"], w[p + "self_attn.o_proj.weight"], self.angles, sh.n_heads,
                sh.n_kv_groups,
            )
            x = x + a
            h = rms_norm_forward(x, w[p + "post_attention_layernorm.weight"])
            x = x + swiglu_ffn_forward(h, w[p + "mlp.gate_proj.weight"], w[p + "mlp.up_proj.weight"],
                                       w[p + "mlp.down_proj.weight"])
        if last_only:
            x = x[:, -1:]
        x = rms_norm_forward(x, w["model.norm.weight"])
        head = w.get("lm_head.weight", w["model.embed_tokens.weight"])  # tied unless given (HF convention)
        return torch.nn.functional.linear(x, head)


def kl_and_top1(ref_logits: torch.Tensor, cand_logits: torch.Tensor):
    """KL(ref || cand) of the next-token distributions and top-1 agreement
    (llama_inference_harness.py:172-198)."""
    r = torch.log_softmax(ref_logits.float().reshape(-1), dim=0)
    c = torch.log_softmax(cand_logits.float().reshape(-1), dim=0)
    return float(torch.sum(r.exp() * (r - c))), int(r.argmax()) == int(c.argmax())

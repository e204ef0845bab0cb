"""Inference harness for the HIP Llama runner: the functions of
iron/applications/llama_3.2_1b/llama_inference_harness.py:146-348 with the same
signatures and behaviour, driven by a ``forward_pass(config, state)`` that
returns ``(logits (1, n, vocab), state)``.

- ``generate_token``: temperature scaling, top-k filtering and multinomial
  sampling on the last position's logits (harness:146-169), with torch's
  global generator (seeded by ``init``, as the reference seeds it).
- ``generate``: prefill + decode loop, printing tokens and the TTFT / tokens
  per second statistics (harness:298-348); returns the tokens and the stats.
- ``check_accuracy``: teacher-forced KL(reference || candidate) and top-1
  agreement per step against another forward pass (the gate of
  harness:172-198; same signature and return value).
- ``check_determinism``: alternating prompts, logits compared bitwise (the
  gate of harness:201-228; same signature and return value).

``hip_forward_pass`` runs the model: a state with more than one token id (or
an empty cache) prefills, a single token id decodes one step (captured graph).
Logits are copied to the host only because sampling and the checks read them;
greedy generation without sampling is ``LlamaHIP.generate``, which stays on
the GPU.
"""

from __future__ import annotations

import sys
import time
from dataclasses import dataclass, field

import torch

from .model import LlamaConfig, LlamaHIP

SEED = 1608560892  # llama_inference_harness.py:282


@dataclass
class HarnessConfig:
    """The harness's view of a model: the model object plus the generation
    settings of llama_inference_harness.py:43-45."""

    model: LlamaHIP
    temperature: float = 0.7
    top_k: int | None = 50
    use_graph: bool = True
    tokenizer: object | None = None  # anything with encode(str) / decode(list[int])
    special_tokens: dict = field(default_factory=lambda: {"<|begin_of_text|>": 128000, "<|end_of_text|>": 128001})

    @property
    def n_layers(self) -> int:
        return self.model.cfg.n_layers


class LlamaModelState:
    """Token ids still to be processed plus the KV cache (harness:73-106); the
    cache lives in the model, so a new state empties it."""

    def __init__(self, config: HarnessConfig):
        self.config = config
        self.token_ids = torch.empty(0, dtype=torch.long)
        self.reset_kv_cache(config)

    def reset_kv_cache(self, config: HarnessConfig | None = None) -> None:
        (config or self.config).model.reset()
        self.num_preceding_tokens = 0


def hip_forward_pass(config: HarnessConfig, state: LlamaModelState):
    """Process ``state.token_ids``; return (logits (1, 1, vocab) fp32 on the
    host, state). The logits are those of the last processed position."""
    model = config.model
    ids = torch.as_tensor(state.token_ids).reshape(-1)
    if ids.numel() == 0:
        raise ValueError("no token ids to process")
    if ids.numel() > 1 or state.num_preceding_tokens == 0:
        model.prefill(ids.tolist())
    else:
        model.set_token(int(ids[0]))
        model.decode(1, use_graph=config.use_graph)
    state.num_preceding_tokens = model.host_pos
    logits = model.logits.float().cpu().reshape(1, 1, -1)
    return logits, state


def generate_token(config, forward_pass, state):
    """One forward pass, then temperature, top-k and sampling (harness:146-169)."""
    logits, state = forward_pass(config, state)
    last = logits[:, -1, :]
    if config.temperature > 0:
        last = last / config.temperature
    if config.top_k is not None:
        top, _ = torch.topk(last, config.top_k)
        last = torch.where(last < top[:, -1:], torch.tensor(float("-inf")), last)
    probs = torch.nn.functional.softmax(last, dim=-1)
    next_token = torch.multinomial(probs, num_samples=1)
    return next_token.item(), state


def init(config: HarnessConfig, prompt_token_ids, seed: int = SEED):
    """Fresh state holding ``<|begin_of_text|>`` + the prompt ids, with torch's
    generator seeded as the reference seeds it (harness:274-295)."""
    state = LlamaModelState(config)
    torch.manual_seed(seed)
    ids = [config.special_tokens["<|begin_of_text|>"]] + [int(t) for t in prompt_token_ids]
    if len(ids) > config.model.cfg.max_seq_len:
        raise ValueError(f"Prompt length ({len(ids)} tokens) exceeds the KV capacity ({config.model.cfg.max_seq_len})")
    state.token_ids = torch.tensor([ids], dtype=torch.long)
    return state


def _text(config, token):
    return config.tokenizer.decode([token]) if config.tokenizer is not None else f"[{token}]"


def generate(config, state, forward_pass=hip_forward_pass, num_tokens=100, use_kv_cache=True, out=sys.stdout):
    """Sample ``num_tokens`` tokens (harness:298-348). Returns (tokens, stats)."""
    tokens = []
    t0 = time.perf_counter()
    first, state = generate_token(config, forward_pass, state)
    tokens.append(first)
    print(_text(config, first), end="", flush=True, file=out)
    t1 = time.perf_counter()

    def advance(tok):
        if use_kv_cache:
            state.token_ids = torch.tensor([[tok]], dtype=torch.long)
        else:
            prev = state.token_ids
            state.reset_kv_cache(config)
            state.token_ids = torch.cat([prev, torch.tensor([[tok]], dtype=torch.long)], dim=1)

    advance(first)
    t2 = time.perf_counter()
    for _ in range(num_tokens - 1):
        tok, state = generate_token(config, forward_pass, state)
        tokens.append(tok)
        print(_text(config, tok), end="", flush=True, file=out)
        advance(tok)
    t3 = time.perf_counter()
    t_prefill, t_decode = t1 - t0, t3 - t2
    n = len(tokens)
    stats = {"ttft_s": t_prefill, "decode_s": t_decode, "n_tokens": n,
             "decode_tok_s": (n - 1) / t_decode if n > 1 and t_decode > 0 else None,
             "total_tok_s": n / (t_prefill + t_decode)}
    sys.stderr.write("\n\n=== Performance Statistics ===\n")
    sys.stderr.write(f"[Prefill] Time to first token:   {t_prefill:7.3f} s\n")
    if n > 1:
        sys.stderr.write(f"[Decode]  Time per token (mean): {t_decode / (n - 1):7.3f} s\n")
        sys.stderr.write(f"[Decode]  Tokens per second:     {(n - 1) / t_decode:7.3f}\n")
    sys.stderr.write(f"[Total]   Time per token (mean): {(t_prefill + t_decode) / n:7.3f} s\n")
    sys.stderr.write(f"[Total]   Tokens per second:     {n / (t_prefill + t_decode):7.3f}\n")
    return tokens, stats


def _divergence(ref_logits: torch.Tensor, cand_logits: torch.Tensor):
    """(KL(ref || cand), top-1 agreement, the reference's greedy token) of two
    next-token logit vectors, in float64."""
    ref_lp = torch.log_softmax(ref_logits.reshape(-1).double(), dim=0)
    cand_lp = torch.log_softmax(cand_logits.reshape(-1).double(), dim=0)
    kl = torch.nn.functional.kl_div(cand_lp, ref_lp, reduction="sum", log_target=True)
    want = int(torch.argmax(ref_lp))
    return float(kl), int(torch.argmax(cand_lp)) == want, want


def check_accuracy(config, state, forward_pass, ref_config, ref_state, ref_forward_pass, num_tokens):
    """Teacher-forced comparison against a reference forward pass
    (the gate of llama_inference_harness.py:172-198).

    Both passes start from ``state.token_ids``; after every step both are fed
    the reference's greedy token, so step n measures the candidate's own error
    at step n. Step 0 is the prefill. Returns one ``(kl, top1)`` per step:
    KL(reference || candidate) of the next-token distributions and whether
    both put the same token first.
    """
    ref_state.token_ids = state.token_ids
    results = []
    for step in range(num_tokens):
        cand, state = forward_pass(config, state)
        ref, ref_state = ref_forward_pass(ref_config, ref_state)
        kl, same, forced = _divergence(ref[0, -1], cand[0, -1])
        results.append((kl, same))
        print(f"[step {step}] KL(ref||cand) = {kl:.3e}, top-1 {'agrees' if same else 'DIFFERS'}", flush=True)
        state.token_ids = ref_state.token_ids = torch.full((1, 1), forced, dtype=torch.long)
    return results


def check_determinism(config, prompts, forward_pass, num_tokens, rounds, make_state=LlamaModelState):
    """Bitwise reproducibility (the gate of llama_inference_harness.py:201-228).

    Each round runs every prompt in turn (so consecutive runs alternate
    prompts) from a fresh state, greedily, for ``num_tokens`` steps, and keeps
    the bf16 bit patterns of each step's logits. Rounds after the first are
    compared with the first round of the same prompt. Returns the number of
    runs that differ anywhere.
    """
    baseline: dict[int, torch.Tensor] = {}
    differing = 0
    for rnd in range(rounds):
        for p, prompt in enumerate(prompts):
            state = make_state(config)
            state.token_ids = prompt
            bits = []
            for _ in range(num_tokens):
                logits, state = forward_pass(config, state)
                last = logits[0, -1]
                bits.append(last.to(torch.bfloat16).view(torch.int16))
                state.token_ids = torch.argmax(last).reshape(1, 1)
            run = torch.stack(bits)
            if p not in baseline:
                baseline[p] = run
                continue
            bad = torch.nonzero((run != baseline[p]).any(dim=1)).flatten().tolist()
            if bad:
                differing += 1
                print(f"determinism: prompt {p}, round {rnd}: logits at steps {bad} differ from round 0", flush=True)
    return differing


# The CPU reference model that --check-accuracy compares against. The library
# ships only the HIP path, so a caller registers one (the test suite registers
# its fp32 oracle): factory(model) -> (ref_config, make_ref_state,
# ref_forward_pass), where make_ref_state(ref_config) is a fresh reference
# state and ref_forward_pass(ref_config, ref_state) returns (logits (1, n,
# vocab), ref_state) for ref_state.token_ids, as forward_pass does.
_model_reference = None


def set_model_reference(factory) -> None:
    """Register (or clear, with None) the reference-model factory used by the
    accuracy check of the application entry point."""
    global _model_reference
    _model_reference = factory


def get_model_reference():
    return _model_reference


def load_safetensors_weights(path, device="cpu") -> dict:
    """Hugging Face Llama weights from a local .safetensors file
    (harness:63 loads the same file); names as the model expects them.
    ``lm_head.weight`` is dropped when it equals the tied embedding."""
    import safetensors.torch

    w = safetensors.torch.load_file(str(path), device=str(device))
    head = w.get("lm_head.weight")
    if head is not None and torch.equal(head, w["model.embed_tokens.weight"]):
        del w["lm_head.weight"]
    return w


def config_from_weights(weights: dict, **over) -> LlamaConfig:
    """LlamaConfig whose shapes are read from the weight dict."""
    emb = weights["model.embed_tokens.weight"]
    n_layers = 1 + max(int(k.split(".")[2]) for k in weights if k.startswith("model.layers."))
    q = weights["model.layers.0.self_attn.q_proj.weight"]
    k = weights["model.layers.0.self_attn.k_proj.weight"]
    head_dim = over.pop("head_dim", 64)
    cfg = dict(vocab_size=emb.shape[0], emb_dim=emb.shape[1], n_layers=n_layers, n_heads=q.shape[0] // head_dim,
               n_kv_groups=k.shape[0] // head_dim,
               hidden_dim=weights["model.layers.0.mlp.gate_proj.weight"].shape[0])
    cfg.update(over)
    return LlamaConfig(**cfg)

"""Command line of the Llama-3.2-1B application: the counterpart of running
iron/applications/llama_3.2_1b/llama_npu.py (its arguments are those of
llama_inference_harness.py:231-264, its summary lines those of
llama_npu.py:1239-1268).

    python -m iron_amd.applications.llama_3_2_1b [weights.safetensors]
        [--prompt-len N] [--num-tokens N]
        [--check-accuracy | --check-determinism ROUNDS]

Without a weights file the model is the Llama-3.2-1B shape with random
weights (``--seed``). There is no tokenizer here: the prompt is
``<|begin_of_text|>`` followed by prompt-len - 1 token ids from a seeded
generator (the reference takes prompt-len characters of its prompt text), and
generated tokens print as ``[id]``.

Output, as the reference prints it:
  sampling (default)    the tokens, then on stderr
                        ``[Prefill] Time to first token:`` and
                        ``[Decode]  Tokens per second:`` among the statistics
  --check-accuracy      ``[Accuracy] Prefill KL:``, ``[Accuracy] Decode max KL:``,
                        ``[Accuracy] Top-1 mismatches:`` (teacher-forced against
                        a CPU reference model registered with
                        ``set_model_reference``; the library ships none)
  --check-determinism   ``[Determinism] Differing runs: n/m`` over two prompts
                        run ROUNDS times each, alternating
"""

from __future__ import annotations

import argparse
import sys


def parse_args(argv=None):
    ap = argparse.ArgumentParser(prog="python -m iron_amd.applications.llama_3_2_1b",
                                 description="Llama-3.2-1B inference on one MI355X (HIP kernels)")
    ap.add_argument("weights_path", nargs="?", default=None,
                    help="Hugging Face Llama .safetensors file (default: random weights of the Llama-3.2-1B shape)")
    ap.add_argument("--prompt-len", type=int, default=2048, help="prompt length in tokens (default: 2048)")
    ap.add_argument("--num-tokens", type=int, default=40, help="tokens to generate (default: 40)")
    ap.add_argument("--check-accuracy", action="store_true",
                    help="instead of sampling, compare each step's logits with the registered CPU reference "
                    "model, feeding both the reference's greedy token")
    ap.add_argument("--check-determinism", type=int, metavar="ROUNDS",
                    help="instead of sampling, run two prompts ROUNDS times each, alternating, and count the "
                    "runs whose logits differ bitwise from the first run")
    ap.add_argument("--seed", type=int, default=0, help="seed of the random weights and the prompt ids")
    ap.add_argument("--head-int4", action="store_true", help="quantize the tied lm_head to int4-g32 as well")
    ap.add_argument("--bf16-linears", action="store_true", help="keep the linear layers in bf16 (no int4)")
    ap.add_argument("--eager", action="store_true", help="issue decode kernels one by one (no captured graph)")
    args = ap.parse_args(argv)
    if args.prompt_len < 1 or args.num_tokens < 1:
        ap.error("--prompt-len and --num-tokens must be positive")
    if args.check_determinism is not None and args.check_determinism < 2:
        ap.error("--check-determinism needs at least 2 rounds")
    if args.check_accuracy and args.check_determinism is not None:
        ap.error("--check-accuracy and --check-determinism are exclusive")
    return args


def _capacity(n: int) -> int:
    """KV capacity for n positions: a multiple of 64 with one block to spare."""
    return (n + 127) // 64 * 64


def main(argv=None) -> int:
    args = parse_args(argv)
    import torch

    from .harness import (HarnessConfig, LlamaModelState, check_accuracy, check_determinism, config_from_weights,
                          generate, get_model_reference, hip_forward_pass, init, load_safetensors_weights)
    from .model import LlamaConfig, LlamaHIP, random_weights

    if not torch.cuda.is_available():
        print("this application needs a GPU (there is no CPU path)", file=sys.stderr)
        return 2
    if args.check_accuracy and get_model_reference() is None:
        print("--check-accuracy needs a CPU reference model: register one with "
              "iron_amd.applications.llama_3_2_1b.set_model_reference (the library ships only the HIP path)",
              file=sys.stderr)
        return 2
    dev = torch.device("cuda", 0)
    cap = _capacity(args.prompt_len + args.num_tokens)
    opts = dict(max_seq_len=cap, head_int4=args.head_int4, int4=not args.bf16_linears)
    if args.weights_path:
        weights = load_safetensors_weights(args.weights_path)
        cfg = config_from_weights(weights, **opts)
    else:
        cfg = LlamaConfig(**opts)
        weights = random_weights(cfg, dev, seed=args.seed)
    model = LlamaHIP(cfg, weights, device=dev)
    del weights
    hc = HarnessConfig(model=model, use_graph=not args.eager)
    g = torch.Generator().manual_seed(args.seed + 1)
    ids = torch.randint(0, cfg.vocab_size, (2, args.prompt_len - 1), generator=g).tolist()
    state = init(hc, ids[0])
    print(f"Llama {cfg.n_layers} layers, hidden {cfg.emb_dim}, vocab {cfg.vocab_size}, "
          f"{'int4-g32' if cfg.int4 else 'bf16'} linears, {'int4-g32' if cfg.head_int4 else 'bf16'} head; "
          f"prompt {args.prompt_len} tokens", file=sys.stderr, flush=True)

    if args.check_accuracy:
        ref_config, make_ref_state, ref_forward = get_model_reference()(model)
        results = check_accuracy(hc, state, hip_forward_pass, ref_config, make_ref_state(ref_config), ref_forward,
                                 args.num_tokens)
        kl = [k for k, _ in results]
        print(f"[Accuracy] Prefill KL: {kl[0]:.6f}")
        if len(kl) > 1:
            print(f"[Accuracy] Decode max KL: {max(kl[1:]):.6f}")
        print(f"[Accuracy] Top-1 mismatches: {sum(1 for _, top1 in results if not top1)}")
        return 0

    if args.check_determinism is not None:
        bos = hc.special_tokens["<|begin_of_text|>"]
        prompts = [torch.tensor([[bos] + p], dtype=torch.long) for p in ids]
        n_differ = check_determinism(hc, prompts, hip_forward_pass, args.num_tokens, args.check_determinism,
                                     make_state=LlamaModelState)
        print(f"[Determinism] Differing runs: {n_differ}/{len(prompts) * (args.check_determinism - 1)}")
        return 0

    generate(hc, state, hip_forward_pass, num_tokens=args.num_tokens)
    print()
    return 0


if __name__ == "__main__":
    sys.exit(main())

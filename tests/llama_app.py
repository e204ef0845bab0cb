"""Runs the application entry point (python -m iron_amd.applications.llama_3_2_1b)
with the fp32 CPU oracle (oracle/llama.py, the restated llama_cpu.py)
registered as the reference model of --check-accuracy -- the role
llama_cpu.llama_forward_pass plays for iron/applications/llama_3.2_1b/
llama_npu.py:1239-1256. Test infrastructure: the library itself ships no CPU
model.

    python tests/llama_app.py [application arguments]
"""

import os
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))


class OracleState:
    """Reference state: the oracle model (with its KV cache) and the ids to process."""

    def __init__(self, ref):
        import torch

        self.ref = ref
        ref.reset()
        self.token_ids = torch.empty(0, dtype=torch.long)


def oracle_forward(ref_config, state):
    import torch

    ids = torch.as_tensor(state.token_ids).reshape(1, -1)
    return state.ref.forward(ids, last_only=True), state


def oracle_reference(model):
    """Reference-model factory for set_model_reference: the oracle on the
    model's effective weights (the dequantised int4-g32 matrices), so the
    comparison isolates the kernels."""
    import torch

    from oracle import llama as ollama

    torch.set_num_threads(len(os.sched_getaffinity(0)))
    cfg = model.cfg
    eff = {k: v.float().cpu() for k, v in model.effective_weights().items()}
    shape = ollama.LlamaShape(cfg.vocab_size, cfg.emb_dim, cfg.n_layers, cfg.n_heads, cfg.n_kv_groups, cfg.hidden_dim)
    ref = ollama.LlamaCPU(shape, eff, model.angles.cpu())
    return ref, OracleState, oracle_forward


if __name__ == "__main__":
    from iron_amd.applications.llama_3_2_1b import set_model_reference
    from iron_amd.applications.llama_3_2_1b.__main__ import main

    set_model_reference(oracle_reference)
    sys.exit(main())

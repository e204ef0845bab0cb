"""Llama-3.2-1B decode/prefill on MI355X (iron/applications/llama_3.2_1b)."""

from .model import LlamaConfig, LlamaHIP, compute_rope_angles, random_weights
from .harness import (
    HarnessConfig,
    LlamaModelState,
    check_accuracy,
    check_determinism,
    config_from_weights,
    generate,
    generate_token,
    hip_forward_pass,
    init,
    load_safetensors_weights,
    get_model_reference,
    set_model_reference,
)

__all__ = [
    "LlamaConfig", "LlamaHIP", "compute_rope_angles", "random_weights", "HarnessConfig", "LlamaModelState",
    "check_accuracy", "check_determinism", "config_from_weights", "generate", "generate_token", "hip_forward_pass",
    "init", "load_safetensors_weights", "get_model_reference", "set_model_reference",
]

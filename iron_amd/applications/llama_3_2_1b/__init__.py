"""Llama-3.2-1B decode/prefill on MI355X (iron/applications/llama_3.2_1b)."""

from .model import LlamaConfig, LlamaHIP, compute_rope_angles, random_weights

__all__ = ["LlamaConfig", "LlamaHIP", "compute_rope_angles", "random_weights"]

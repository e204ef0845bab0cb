"""Dequant: int4 codes x bf16 group scale -> bf16 (iron/operators/dequant/op.py:20-81).

Payload layout and arg spec are the reference's: per tile of ``tile_size``
weights, ``tile_size/2`` code bytes (low nibble = even element) followed by
``tile_size/group_size`` bf16 scales; input ``(size/2 + 2*size/group,)``
uint8, output ``(size,)`` bf16 (dequant/reference.py:8-18,68-92). The product
``q * scale`` is exact in fp32 and rounded once to bf16 (round-to-nearest-even),
so the output is bit-exact.

``signed`` (default False, the reference's uint4) selects two's-complement
nibbles in [-8, 7], the encoding of the fused int4 GEMV weights.
"""

from dataclasses import dataclass, field

import torch

from ... import _lib
from ...common import HIPOperator, AIERuntimeArgSpec


@dataclass
class Dequant(HIPOperator):
    """int4 (+ per-group bf16 scale) -> bf16 dequantization."""

    size: int
    num_aie_columns: int
    num_channels: int
    tile_size: int
    group_size: int = field(default=32, repr=False)
    signed: bool = field(default=False, repr=False)
    context: object = field(default=None, repr=False)

    def __post_init__(self):
        self.input_size = (self.size // 2) + (self.size // self.group_size) * 2
        self.output_size = self.size
        total_cores = self.num_aie_columns * self.num_channels
        if self.size % total_cores != 0:
            raise ValueError(f"size ({self.size}) must be divisible by total cores ({total_cores})")
        if total_cores > 16:
            raise ValueError(f"total cores ({total_cores}) must be <= 16")
        if self.size % self.tile_size:
            raise ValueError(f"size ({self.size}) must be a multiple of tile_size ({self.tile_size})")
        if self.tile_size % self.group_size or self.group_size % 2:
            raise ValueError(
                f"group_size ({self.group_size}) must be even and divide tile_size ({self.tile_size})"
            )
        HIPOperator.__init__(self, context=self.context)

    def get_arg_spec(self):
        return [
            AIERuntimeArgSpec("in", (self.input_size,), dtype=torch.uint8),
            AIERuntimeArgSpec("out", (self.output_size,), dtype=torch.bfloat16),
        ]

    def _launch(self, payload, out, *, stream):
        _lib.call(
            "iron_dequant_i4_payload",
            payload.data_ptr(),
            out.data_ptr(),
            self.size,
            self.tile_size,
            self.group_size,
            int(self.signed),
            stream,
        )

"""GELU, tanh approximation (iron/operators/gelu/op.py:12-26; reference
iron/operators/gelu/reference.py:7-9): out = 0.5 x (1 + tanh(sqrt(2/pi)
(x + 0.044715 x^3))), fp32 math, one bf16 rounding.

Channeled-unary fields and arg spec ``(input (size,), output (size,))`` of
iron/common/operator_bases.py:22-90 (num_channels is a field here, as in the
reference's GELU); kernel iron_gelu.
"""

from dataclasses import dataclass, field

from ... import _lib
from ...common import HIPOperator, AIERuntimeArgSpec


@dataclass
class GELU(HIPOperator):
    size: int
    num_aie_columns: int
    num_channels: int
    tile_size: int
    context: object = field(default=None, repr=False)

    def __post_init__(self):
        max_multiple = self.num_aie_columns * self.tile_size
        if self.size % max_multiple != 0:
            raise ValueError(
                f"size ({self.size}) must be a multiple of num_aie_columns * tile_size ({max_multiple})"
            )
        HIPOperator.__init__(self, context=self.context)

    def get_arg_spec(self):
        return [AIERuntimeArgSpec("in", (self.size,)), AIERuntimeArgSpec("out", (self.size,))]

    def _launch(self, x, out, *, stream):
        _lib.call("iron_gelu", x.data_ptr(), out.data_ptr(), self.size, stream)

"""SiLU (iron/operators/silu/op.py:12-26): out = x * sigmoid(x), fp32 math.

Channeled-unary fields and arg spec ``(input (size,), output (size,))`` of
iron/common/operator_bases.py:22-90; kernel iron_silu.
"""

from dataclasses import dataclass, field

from ... import _lib
from ...common import HIPOperator, AIERuntimeArgSpec


@dataclass
class SiLU(HIPOperator):
    size: int
    num_aie_columns: int
    tile_size: int
    num_channels: int = field(default=1, init=False, repr=False)
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
        _lib.call("iron_silu", x.data_ptr(), out.data_ptr(), self.size, stream)

"""RMSNorm (iron/operators/rms_norm/op.py:19-122) on MI355X.

Fields, validation and arg spec as the reference:
``(input (size/tile_size, tile_size), [weight (tile_size,),] output)``; each
row of ``tile_size`` elements is normalised as x / sqrt(mean(x^2) + eps)
(rms_norm/reference.py:7-16), times the weight when ``weighted``. One HIP
workgroup per row, fp32 math, one bf16 rounding (iron_rmsnorm).
"""

from dataclasses import dataclass, field
from typing import ClassVar, Dict

from ... import _lib
from ...common import HIPOperator, AIERuntimeArgSpec


@dataclass
class RMSNorm(HIPOperator):
    size: int
    num_aie_columns: int
    num_channels: int
    tile_size: int
    weighted: bool = False
    epsilon: float = 1e-5
    context: object = field(default=None, repr=False)

    _name_aliases: ClassVar[Dict[str, str]] = {
        **HIPOperator._name_aliases,
        "weighted": "w",
        "epsilon": "eps",
    }

    def __post_init__(self):
        max_multiple = self.num_aie_columns * self.num_channels * self.tile_size
        if self.size % max_multiple != 0:
            raise ValueError(
                f"size ({self.size}) must be a multiple of "
                f"num_aie_columns * num_channels * tile_size ({max_multiple})"
            )
        if self.tile_size % 8 or self.tile_size > 16384:
            raise ValueError(f"tile_size ({self.tile_size}) must be a multiple of 8 and <= 16384")
        HIPOperator.__init__(self, context=self.context)

    @property
    def rows(self) -> int:
        return self.size // self.tile_size

    def get_arg_spec(self):
        specs = [AIERuntimeArgSpec("in", (self.rows, self.tile_size))]
        if self.weighted:
            specs.append(AIERuntimeArgSpec("in", (self.tile_size,)))
        specs.append(AIERuntimeArgSpec("out", (self.rows, self.tile_size)))
        return specs

    def _launch(self, *args, stream):
        if self.weighted:
            x, w, out = args
        else:
            (x, out), w = args, None
        _lib.call("iron_rmsnorm", x.data_ptr(), None, _lib.ptr(w), out.data_ptr(), None, self.rows,
                  self.tile_size, float(self.epsilon), stream)

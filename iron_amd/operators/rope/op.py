"""RoPE (iron/operators/rope/op.py:18-92) on MI355X.

Arg spec ``(input (rows, cols), angles (angle_rows, cols), output (rows, cols))``
with the reference's angle layout: each angle row interleaves [cos, sin]
pairs, and input row r uses angle row r // (rows / angle_rows)
(rope/reference.py:69-102). method_type 0 rotates the two halves (HF),
1 the interleaved pairs. fp32 math, one bf16 rounding (iron_rope).
"""

from dataclasses import dataclass, field
from typing import ClassVar, Dict

import torch

from ... import _lib
from ...common import HIPOperator, AIERuntimeArgSpec


@dataclass
class RoPE(HIPOperator):
    rows: int
    cols: int
    angle_rows: int | None = None
    num_aie_columns: int = 1
    method_type: int = 0
    context: object = field(default=None, repr=False)

    # the angle table may also be fp32 (the Llama runner keeps an fp32 table)
    _extra_dtypes: ClassVar[dict] = {1: (torch.float32,)}
    _name_aliases: ClassVar[Dict[str, str]] = {
        **HIPOperator._name_aliases,
        "num_aie_columns": "col",
        "angle_rows": "arows",
        "method_type": "m",
    }

    def __post_init__(self):
        if self.angle_rows is None:
            self.angle_rows = self.rows
        if not (self.cols % (16 * 2) == 0 and self.cols >= (16 * 2)):
            raise ValueError("cols must be multiple of 32 and >= 32")
        if self.rows % self.num_aie_columns != 0:
            raise ValueError("rows must be divisible by num_aie_columns")
        if not (self.angle_rows <= self.rows and self.rows % self.angle_rows == 0):
            raise ValueError("angle_rows must divide rows")
        if not (self.angle_rows >= self.num_aie_columns and self.angle_rows % self.num_aie_columns == 0):
            raise ValueError("angle_rows must be divisible by num_aie_columns")
        if self.method_type not in {0, 1}:
            raise ValueError(f"method_type must be 0 or 1, got {self.method_type}")
        HIPOperator.__init__(self, context=self.context)

    def get_arg_spec(self):
        return [
            AIERuntimeArgSpec("in", (self.rows, self.cols)),
            AIERuntimeArgSpec("in", (self.angle_rows, self.cols)),
            AIERuntimeArgSpec("out", (self.rows, self.cols)),
        ]

    def _launch(self, x, angles, out, *, stream):
        _lib.call("iron_rope", x.data_ptr(), angles.data_ptr(), int(angles.dtype == torch.float32),
                  out.data_ptr(), self.rows, self.cols, self.angle_rows, self.method_type, stream)

"""Repeat (iron/operators/repeat/op.py:15-70): repeat-interleave along the
leading dimension, ``out = x.repeat_interleave(repeat, dim=0)``.

Fields and arg spec as the reference: ``(in (rows, cols), out (rows*repeat,
cols))`` of ``dtype`` (bf16 default; any torch dtype); ``transfer_size`` is
accepted. Kernel iron_repeat_rows (16-byte chunks when a row allows).
"""

from dataclasses import dataclass, field
from typing import ClassVar, Dict

import torch

from ... import _lib
from ...common import HIPOperator, AIERuntimeArgSpec


@dataclass
class Repeat(HIPOperator):
    rows: int
    cols: int
    repeat: int
    transfer_size: int | None = None
    dtype: object = field(default=torch.bfloat16, repr=False)
    context: object = field(default=None, repr=False)

    _name_aliases: ClassVar[Dict[str, str]] = {**HIPOperator._name_aliases, "repeat": "by", "transfer_size": "ts"}

    def __post_init__(self):
        if self.rows <= 0 or self.cols <= 0 or self.repeat <= 0:
            raise ValueError("rows, cols and repeat must be positive")
        if not isinstance(self.dtype, torch.dtype):
            raise ValueError(f"dtype must be a torch dtype, got {self.dtype!r}")
        HIPOperator.__init__(self, context=self.context)

    def get_arg_spec(self):
        return [AIERuntimeArgSpec("in", (self.rows, self.cols), dtype=self.dtype),
                AIERuntimeArgSpec("out", (self.rows * self.repeat, self.cols), dtype=self.dtype)]

    def _launch(self, x, out, *, stream):
        row_bytes = self.cols * x.element_size()
        _lib.call("iron_repeat_rows", x.data_ptr(), out.data_ptr(), self.rows, row_bytes, self.repeat, stream)

"""Softmax (iron/operators/softmax/op.py:21-97): row softmax over ``cols``.

Arg spec ``(input (rows*cols,), output (rows*cols,))``. ``rtp_vector_size``
(default ``cols``) masks columns at or beyond it to -inf before the softmax,
as the reference's runtime vector size does (softmax/design.py:74-91); the
masked outputs are 0. Inside an OperatorSequence, ``vector_size_parameter``
names the runtime parameter that overrides it per call. fp32 math
(iron_softmax).
"""

from dataclasses import dataclass, field

from ... import _lib
from ...common import HIPOperator, AIERuntimeArgSpec


@dataclass
class Softmax(HIPOperator):
    rows: int
    cols: int
    num_aie_columns: int = 1
    num_channels: int = 1
    rtp_vector_size: int | None = None
    vector_size_parameter: str | None = None
    context: object = field(default=None, repr=False)

    @property
    def size(self):
        return self.rows * self.cols

    def __post_init__(self):
        if self.rows % 16 != 0:
            raise ValueError(f"rows ({self.rows}) must be a multiple of 16")
        if self.cols % 16 != 0:
            raise ValueError(f"cols ({self.cols}) must be a multiple of 16")
        if self.rows % self.num_aie_columns != 0:
            raise ValueError(
                f"rows ({self.rows}) must be a multiple of num_aie_columns ({self.num_aie_columns})"
            )
        if self.cols > 16384:
            raise ValueError(f"cols ({self.cols}) must be <= 16384")
        self._vector_size_dev = None  # device int32 set by an OperatorSequence
        HIPOperator.__init__(self, context=self.context)

    def get_arg_spec(self):
        return [AIERuntimeArgSpec("in", (self.size,)), AIERuntimeArgSpec("out", (self.size,))]

    def _launch(self, x, out, *, stream):
        valid = self.cols if self.rtp_vector_size is None else int(self.rtp_vector_size)
        _lib.call("iron_softmax", x.data_ptr(), out.data_ptr(), self.rows, self.cols, valid,
                  _lib.ptr(self._vector_size_dev), stream)

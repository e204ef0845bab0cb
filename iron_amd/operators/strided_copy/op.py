"""StridedCopy (iron/operators/strided_copy/op.py:15-110): gather by an input
access pattern, scatter by an output access pattern.

Fields and arg spec as the reference: ``(in (input_buffer_size,), out
(output_buffer_size,))`` of ``dtype``; patterns of 1-4 dimensions given as
sizes/strides/offset in elements, split over ``num_aie_channels`` as the
reference splits them. Elements of ``out`` outside the output pattern are
left untouched (the KV-cache append of llama_npu.py:311-323 relies on that).
Inside an OperatorSequence, ``input_offset_parameter`` /
``output_offset_parameter`` name runtime parameters whose value (elements)
is added to the offsets when the copy runs. Kernel iron_strided_copy.
"""

import ctypes
from dataclasses import dataclass, field
from typing import ClassVar, Dict

import torch

from ... import _lib
from ...common import HIPOperator, AIERuntimeArgSpec


def _ll_array(vals):
    return (ctypes.c_longlong * len(vals))(*[int(v) for v in vals])


@dataclass
class StridedCopy(HIPOperator):
    input_sizes: list
    input_strides: list
    input_offset: int
    output_sizes: list
    output_strides: list
    output_offset: int
    input_buffer_size: int = field(repr=False)
    output_buffer_size: int = field(repr=False)
    dtype: object = field(default=torch.bfloat16, repr=False)
    transfer_size: int | None = None
    num_aie_channels: int = 1
    input_offset_parameter: str | None = None
    output_offset_parameter: str | None = None
    kwargs: dict = field(default_factory=dict, repr=False)
    context: object = field(default=None, repr=False)

    _name_aliases: ClassVar[Dict[str, str]] = {
        **HIPOperator._name_aliases,
        "input_sizes": "isz", "input_strides": "ist", "input_offset": "ioff", "output_sizes": "osz",
        "output_strides": "ost", "output_offset": "ooff", "transfer_size": "tr", "num_aie_channels": "ch",
        "input_offset_parameter": "ipar", "output_offset_parameter": "opar",
    }

    def __post_init__(self):
        if len(self.input_sizes) != len(self.input_strides):
            raise ValueError(
                f"input_sizes and input_strides must have the same length "
                f"({len(self.input_sizes)} vs {len(self.input_strides)})"
            )
        if len(self.output_sizes) != len(self.output_strides):
            raise ValueError(
                f"output_sizes and output_strides must have the same length "
                f"({len(self.output_sizes)} vs {len(self.output_strides)})"
            )
        if not 1 <= len(self.input_sizes) <= 4 or not 1 <= len(self.output_sizes) <= 4:
            raise ValueError("access patterns have 1 to 4 dimensions")
        if not isinstance(self.dtype, torch.dtype):
            raise ValueError(f"dtype must be a torch dtype, got {self.dtype!r}")
        self._in_addend_dev = None  # device int32 set by an OperatorSequence
        self._out_addend_dev = None
        HIPOperator.__init__(self, context=self.context)

    def get_arg_spec(self):
        return [AIERuntimeArgSpec("in", (int(self.input_buffer_size),), dtype=self.dtype),
                AIERuntimeArgSpec("out", (int(self.output_buffer_size),), dtype=self.dtype)]

    def _launch(self, x, out, *, stream):
        _lib.call("iron_strided_copy", x.data_ptr(), out.data_ptr(), x.element_size(), int(self.input_buffer_size),
                  int(self.output_buffer_size), len(self.input_sizes), _ll_array(self.input_sizes),
                  _ll_array(self.input_strides), int(self.input_offset), _lib.ptr(self._in_addend_dev),
                  len(self.output_sizes), _ll_array(self.output_sizes), _ll_array(self.output_strides),
                  int(self.output_offset), _lib.ptr(self._out_addend_dev), int(self.num_aie_channels), stream)

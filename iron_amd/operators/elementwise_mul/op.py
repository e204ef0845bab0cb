"""ElementwiseMul (iron/operators/elementwise_mul/op.py:12-24): out = a * b.

Binary-elementwise fields and arg spec ``(a (size,), b (size,), out (size,))``
of iron/common/operator_bases.py:93-203; kernel iron_mul.
"""

from dataclasses import dataclass, field
from typing import ClassVar, Dict

from ... import _lib
from ...common import HIPOperator, AIERuntimeArgSpec


@dataclass
class BinaryElementwise(HIPOperator):
    size: int
    tile_size: int
    num_aie_columns: int = 8
    context: object = field(default=None, repr=False)

    _entry: ClassVar[str] = ""
    _name_aliases: ClassVar[Dict[str, str]] = {**HIPOperator._name_aliases, "num_aie_columns": "col"}

    def __post_init__(self):
        if self.size % (self.num_aie_columns * self.tile_size) != 0:
            raise ValueError(
                f"size ({self.size}) must be a multiple of "
                f"num_aie_columns * tile_size ({self.num_aie_columns * self.tile_size})"
            )
        HIPOperator.__init__(self, context=self.context)

    def get_arg_spec(self):
        return [AIERuntimeArgSpec("in", (self.size,)), AIERuntimeArgSpec("in", (self.size,)),
                AIERuntimeArgSpec("out", (self.size,))]

    def _launch(self, a, b, out, *, stream):
        _lib.call(self._entry, a.data_ptr(), b.data_ptr(), out.data_ptr(), self.size, stream)


@dataclass
class ElementwiseMul(BinaryElementwise):
    _entry: ClassVar[str] = "iron_mul"

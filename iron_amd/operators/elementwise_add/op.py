"""ElementwiseAdd (iron/operators/elementwise_add/op.py:12-24): out = a + b."""

from dataclasses import dataclass
from typing import ClassVar

from ..elementwise_mul.op import BinaryElementwise


@dataclass
class ElementwiseAdd(BinaryElementwise):
    _entry: ClassVar[str] = "iron_add"

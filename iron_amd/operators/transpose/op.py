"""Transpose (iron/operators/transpose/op.py:16-120): each of ``num_batches``
(M, N) matrices laid back to back is transposed to (N, M).

Same fields and validation as the reference (the AIE tile sizes m, n, s and
the column/channel counts are checked, then only size the work); arg spec
``(in (B?, M*N), out (B?, N*M))``, bf16. Kernel iron_transpose_batched_bf16
(64x64 tiles through LDS).
"""

from dataclasses import dataclass, field
from typing import ClassVar, Dict

from ... import _lib
from ...common import HIPOperator, AIERuntimeArgSpec


@dataclass
class Transpose(HIPOperator):
    M: int
    N: int
    num_aie_columns: int
    num_channels: int
    m: int
    n: int
    s: int
    num_batches: int = 1
    context: object = field(default=None, repr=False)

    _name_aliases: ClassVar[Dict[str, str]] = {**HIPOperator._name_aliases, "num_batches": "batch"}

    def __post_init__(self):
        if self.M % self.m != 0:
            raise ValueError(f"Matrix rows ({self.M}) must be a multiple of {self.m}")
        if self.N % self.n != 0:
            raise ValueError(f"Matrix columns ({self.N}) must be a multiple of {self.n}")
        if self.m % self.s != 0:
            raise ValueError(f"AIE tile rows ({self.m}) must be a multiple of {self.s}")
        if self.n % self.s != 0:
            raise ValueError(f"AIE tile columns ({self.n}) must be a multiple of {self.s}")
        if self.M * self.N % (self.m * self.n * self.num_aie_columns * self.num_channels) != 0:
            raise ValueError("Transfer size must be divisible by m*n*num_columns*num_channels")
        if self.N // self.num_aie_columns // self.n < 1:
            raise ValueError(f"num_aie_columns ({self.num_aie_columns}) exceeds N/n ({self.N // self.n})")
        if self.M // self.num_channels // self.m < 1:
            raise ValueError(f"num_channels ({self.num_channels}) exceeds M/m ({self.M // self.m})")
        if self.num_batches < 1:
            raise ValueError("num_batches must be >= 1")
        HIPOperator.__init__(self, context=self.context)

    def get_arg_spec(self):
        batch_dim = (self.num_batches,) if self.num_batches > 1 else ()
        return [AIERuntimeArgSpec("in", batch_dim + (self.M * self.N,)),
                AIERuntimeArgSpec("out", batch_dim + (self.N * self.M,))]

    def _launch(self, x, out, *, stream):
        _lib.call("iron_transpose_batched_bf16", x.data_ptr(), out.data_ptr(), self.M, self.N, self.num_batches, stream)

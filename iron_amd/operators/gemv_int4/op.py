"""GEMVInt4: fused int4 dequant + GEMV (new operator; no single reference op).

Computes ``y = Dequant(codes, scales) . x`` without materialising the bf16
weights: the composition of Dequant (iron/operators/dequant/op.py:20-81) and
GEMV (iron/operators/gemv/op.py:22-159) in one HBM pass.

Weight format (planar, group 32, zero-point 0):
  codes  (M, K/2) uint8 -- two weights per byte along K, low nibble first;
                           two's complement [-8, 7] when ``signed`` (default)
  scales (M, K/32) bf16 -- one scale per 32 consecutive K
Arg spec: (codes, scales, vector (K,), output (M,)).
"""

from dataclasses import dataclass, field

import torch

from ... import _lib
from ...common import HIPOperator, AIERuntimeArgSpec


@dataclass
class GEMVInt4(HIPOperator):
    M: int
    K: int
    group_size: int = 32
    signed: bool = field(default=True, repr=False)
    context: object = field(default=None, repr=False)
    # bytes of the per-call device phase trace (iron_amd/common/tracing_utils.py); None: IRON_TRACE_SIZE
    trace_size: int | None = field(default=None, repr=False)

    def __post_init__(self):
        if self.group_size != 32:
            raise ValueError(f"group_size must be 32 (got {self.group_size})")
        if self.M <= 0 or self.K <= 0 or self.K % 32:
            raise ValueError(f"M ({self.M}) must be positive and K ({self.K}) a positive multiple of 32")
        HIPOperator.__init__(self, context=self.context)

    def get_arg_spec(self):
        return [
            AIERuntimeArgSpec("in", (self.M, self.K // 2), dtype=torch.uint8),  # codes
            AIERuntimeArgSpec("in", (self.M, self.K // 32)),  # scales
            AIERuntimeArgSpec("in", (self.K,)),  # vector
            AIERuntimeArgSpec("out", (self.M,)),  # output
        ]

    def _launch(self, codes, scales, x, y, *, stream):
        _lib.call(
            "iron_gemv_i4g32",
            codes.data_ptr(),
            scales.data_ptr(),
            x.data_ptr(),
            y.data_ptr(),
            self.M,
            self.K,
            int(self.signed),
            stream,
        )

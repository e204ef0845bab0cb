"""GEMMInt4: C = A @ Dequant(codes, scales)^T with the int4 weights
dequantized inside the GEMM (new operator; no single reference op).

The composition of Dequant (iron/operators/dequant/op.py:20-81) and GEMM
(iron/operators/gemm/op.py:21-231, b_col_maj=True) without writing the bf16
weights to memory: the prefill projections can read the same int4-g32 weights
the decode GEMVs use. Dequantized values are bit-exact (q * s rounded once to
bf16), and C is bit-identical to GEMM on them.

Weight format (planar, group 32, zero-point 0), as GEMVInt4:
  codes  (N, K/2) uint8 -- low nibble first; two's complement when ``signed``
  scales (N, K/32) bf16
Arg spec: (A (M, K) bf16, codes, scales, C (M, N) bf16). K % 64 == 0.
Shapes whose 128x128 tiles cannot fill the GPU split K into fp32 partials
(operator-owned workspace), as GEMM does.
"""

from dataclasses import dataclass, field

import torch

from ... import _lib
from ...common import HIPOperator, AIERuntimeArgSpec


@dataclass
class GEMMInt4(HIPOperator):
    M: int
    K: int
    N: int
    group_size: int = 32
    signed: bool = field(default=True, repr=False)
    context: object = field(default=None, repr=False)

    def __post_init__(self):
        if self.group_size != 32:
            raise ValueError(f"group_size must be 32 (got {self.group_size})")
        if self.M <= 0 or self.N <= 0 or self.K <= 0 or self.K % 64:
            raise ValueError(f"M ({self.M}) and N ({self.N}) must be positive and K ({self.K}) a multiple of 64")
        self._ws = {}
        HIPOperator.__init__(self, context=self.context)

    def get_arg_spec(self):
        return [
            AIERuntimeArgSpec("in", (self.M, self.K)),
            AIERuntimeArgSpec("in", (self.N, self.K // 2), dtype=torch.uint8),  # codes
            AIERuntimeArgSpec("in", (self.N, self.K // 32)),  # scales
            AIERuntimeArgSpec("out", (self.M, self.N)),
        ]

    def _launch(self, A, codes, scales, C, *, stream):
        splits = _lib.query("iron_gemm_i4g32_splitk_choose", self.M, self.N, self.K)
        ws, need = None, 0
        if splits > 1:
            need = int(_lib.query("iron_gemm_splitk_workspace_bytes", self.M, self.N, splits))
            ws = self._ws.get(A.device)
            if ws is None or ws.numel() < need:
                ws = torch.empty(need, dtype=torch.uint8, device=A.device)
                self._ws[A.device] = ws
        _lib.call("iron_gemm_i4g32_nt", A.data_ptr(), codes.data_ptr(), scales.data_ptr(), C.data_ptr(), self.M,
                  self.N, self.K, self.N, 0, 0, 0.0, 0.0, int(self.signed), splits, _lib.ptr(ws), need, stream)

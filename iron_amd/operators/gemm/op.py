"""GEMM (iron/operators/gemm/op.py:21-231): C = A @ B in bf16 on MFMA.

Fields and arg spec as the reference: A (M, K); B (K, N), or (N, K) when
``b_col_maj``; C (M, N), or (N, M) when ``c_col_maj`` (gemm/reference.py:7-18).
The AIE tiling knobs are accepted and ignored. K must be a multiple of 64.

Kernel: iron_gemm_bf16_nt (A and B both K-contiguous). B given row-major
(K, N) is first transposed into an operator-owned scratch buffer; a
column-major C is produced by computing C^T = B A^T. Shapes whose output
tiles cannot fill the GPU are split over K (iron_gemm_bf16_nt_splitk, fp32
partials in an operator-owned workspace).
"""

from dataclasses import dataclass, field
from typing import ClassVar, Dict

import torch

from ... import _lib
from ...common import HIPOperator, AIERuntimeArgSpec

_DTYPES = {"bf16": torch.bfloat16}


@dataclass
class GEMM(HIPOperator):
    M: int
    K: int
    N: int
    tile_m: int = 64
    tile_k: int = 64
    tile_n: int = 64
    b_col_maj: bool = False
    c_col_maj: bool = False
    num_aie_columns: int = field(default=8)
    emulate_bf16_mmul_with_bfp16: bool = field(default=True, repr=False)
    prio_accuracy: bool = field(default=False, repr=False)
    round_conv_even: bool = field(default=True, repr=False)
    dtype_in: str = field(default="bf16", repr=False)
    dtype_out: str = field(default="bf16", repr=False)
    use_scalar: bool = field(default=False, repr=False)
    separate_c_tiles: bool = field(default=False, repr=False)
    context: object = field(default=None, repr=False)

    _name_aliases: ClassVar[Dict[str, str]] = {
        **HIPOperator._name_aliases,
        "tile_m": "tm",
        "tile_k": "tk",
        "tile_n": "tn",
        "b_col_maj": "bc",
        "c_col_maj": "cc",
    }

    def __post_init__(self):
        if self.M <= 0 or self.N <= 0 or self.K <= 0:
            raise ValueError(f"M ({self.M}), K ({self.K}) and N ({self.N}) must be positive")
        if self.K % 64 != 0:
            raise ValueError(f"K ({self.K}) must be a multiple of 64")
        if self.dtype_in not in _DTYPES or self.dtype_out not in _DTYPES:
            raise ValueError(f"only bf16 in/out is supported (got {self.dtype_in}/{self.dtype_out})")
        self._bt = {}
        self._ws = {}
        HIPOperator.__init__(self, context=self.context)

    def get_arg_spec(self):
        return [
            AIERuntimeArgSpec("in", (self.M, self.K)),
            AIERuntimeArgSpec("in", (self.N, self.K) if self.b_col_maj else (self.K, self.N)),
            AIERuntimeArgSpec("out", (self.N, self.M) if self.c_col_maj else (self.M, self.N)),
        ]

    def _b_nk(self, B, stream):
        """B as (N, K) K-contiguous (transposed into scratch when given row-major)."""
        if self.b_col_maj:
            return B
        bt = self._bt.get(B.device)
        if bt is None:
            bt = torch.empty(self.N, self.K, dtype=torch.bfloat16, device=B.device)
            self._bt[B.device] = bt
        _lib.call("iron_transpose_bf16", B.data_ptr(), bt.data_ptr(), self.K, self.N, stream)
        return bt

    def _nt(self, X, W, C, rows, cols, stream):
        """C (rows, cols) = X (rows, K) . W (cols, K)^T, split over K when the
        output tiles alone cannot fill the GPU (operator-owned workspace)."""
        splits = _lib.query("iron_gemm_splitk_choose", rows, cols, self.K)
        if splits > 1:
            need = int(_lib.query("iron_gemm_splitk_workspace_bytes", rows, cols, splits))
            ws = self._ws.get(X.device)
            if ws is None or ws.numel() < need:
                ws = torch.empty(need, dtype=torch.uint8, device=X.device)
                self._ws[X.device] = ws
            _lib.call("iron_gemm_bf16_nt_splitk", X.data_ptr(), W.data_ptr(), C.data_ptr(), rows, cols, self.K,
                      cols, 0, 0, 0.0, 0.0, splits, ws.data_ptr(), need, stream)
        else:
            _lib.call("iron_gemm_bf16_nt", X.data_ptr(), W.data_ptr(), C.data_ptr(), rows, cols, self.K, cols, 0, 0,
                      0.0, 0.0, stream)

    def _launch(self, A, B, C, *, stream):
        Bnk = self._b_nk(B, stream)
        if self.c_col_maj:
            self._nt(Bnk, A, C, self.N, self.M, stream)
        else:
            self._nt(A, Bnk, C, self.M, self.N, stream)

"""flm.GEMM (iron/operators/flm/gemm/op.py:64-499): bf16 GEMM with a fused
activation and optional clamp, on MFMA.

C = clamp(act(bf16(A @ B))), act in {none, gelu = x*sigmoid(1.702x), silu,
sigmoid} (flm/gemm/reference.py:8-57): the fp32 accumulator is rounded to bf16
before the activation, as the reference kernel does.

``pack_B(B)`` reorders a row-major (K, N) weight once into the kernel's
consumption order, here (N, K) K-contiguous; the arg spec is
(A (M, K), B packed (N, K), C (M, N)). The AIE tiling knobs (tile_n, k_tile,
tile_ma, m_chunk) are accepted for API compatibility. ``rounding`` selects
the fp32 -> bf16 conversions of the output stage (design.py:164-172):
``conv_even`` rounds to nearest even, ``floor`` truncates the mantissa
(rounds toward zero), the reference's overlay mode (op.py:105,426-430).
"""

from dataclasses import dataclass, field
from enum import Enum
from typing import ClassVar, Dict

import torch

from .... import _lib
from ....common import HIPOperator, AIERuntimeArgSpec


class Epilogue(str, Enum):
    """Activation folded into the output stage; declaration order is the mode number."""

    NONE = "none"
    GELU = "gelu"
    SILU = "silu"
    SIGMOID = "sigmoid"

    def __str__(self):
        return self.value

    @property
    def mode(self) -> int:
        return list(Epilogue).index(self)


class Rounding(str, Enum):
    CONV_EVEN = "conv_even"
    FLOOR = "floor"

    def __str__(self):
        return self.value


# kernel epilogue codes (include/iron_hip.h: enum iron_epilogue)
_EPI_CODE = {Epilogue.NONE: 0, Epilogue.GELU: 4, Epilogue.SILU: 2, Epilogue.SIGMOID: 3}
_ROUND_TOWARD_ZERO = 0x100  # IRON_EPI_ROUND_TOWARD_ZERO
K_TILE = 512


@dataclass
class GEMM(HIPOperator):
    M: int
    K: int
    N: int
    epilogue: Epilogue = Epilogue.NONE
    epilogue_modes: tuple = tuple(Epilogue)
    clamp: tuple | None = None
    tile_n: int | None = None
    k_tile: int = K_TILE
    tile_ma: int | None = None
    m_chunk: int | None = None
    rounding: Rounding = Rounding.CONV_EVEN
    context: object = field(default=None, repr=False)

    _name_aliases: ClassVar[Dict[str, str]] = {
        **HIPOperator._name_aliases,
        "epilogue": "epi",
        "tile_n": "tn",
        "k_tile": "kt",
        "tile_ma": "ma",
        "m_chunk": "mc",
        "rounding": "rnd",
    }

    def __post_init__(self):
        if self.tile_n is None:
            self.tile_n = 64
        elif self.tile_n not in (16, 32, 64, 128):
            raise ValueError(f"tile_n must be one of [16, 32, 64, 128], got {self.tile_n}")
        if self.M <= 0 or self.N <= 0 or self.K <= 0:
            raise ValueError("M, K and N must be positive")
        if self.K % 64 != 0:
            raise ValueError(f"K ({self.K}) must be a multiple of 64")
        self.epilogue = Epilogue(self.epilogue)
        self.rounding = Rounding(self.rounding)
        self.epilogue_modes = tuple(dict.fromkeys(Epilogue(m) for m in self.epilogue_modes))
        if self.epilogue is not Epilogue.NONE and self.epilogue not in self.epilogue_modes:
            raise ValueError(
                f"epilogue {self.epilogue} is not in epilogue_modes "
                f"{tuple(str(m) for m in self.epilogue_modes)}, so it would not be compiled in "
                "and the kernel would silently apply none"
            )
        if self.clamp is not None:
            lo, hi = self.clamp
            if lo > hi:
                raise ValueError(f"clamp min ({lo}) must be <= max ({hi})")
        self._ws = {}
        HIPOperator.__init__(self, context=self.context)

    def pack_B(self, B: torch.Tensor) -> torch.Tensor:
        """Row-major (K, N) weights -> consumption order (N, K), K-contiguous."""
        if B.shape != (self.K, self.N):
            raise ValueError(f"B must be ({self.K}, {self.N}), got {tuple(B.shape)}")
        return B.t().contiguous()

    def packed_B_size(self, K, N):
        return K * N

    def get_arg_spec(self):
        return [
            AIERuntimeArgSpec("in", (self.M, self.K)),
            AIERuntimeArgSpec("in", (self.N, self.K)),
            AIERuntimeArgSpec("out", (self.M, self.N)),
        ]

    def _launch(self, A, B, C, *, stream):
        lo, hi = (float(self.clamp[0]), float(self.clamp[1])) if self.clamp is not None else (0.0, 0.0)
        epi, has_clamp = _EPI_CODE[self.epilogue], int(self.clamp is not None)
        if self.rounding is Rounding.FLOOR:
            epi |= _ROUND_TOWARD_ZERO
        splits = _lib.query("iron_gemm_splitk_choose", self.M, self.N, self.K)
        if splits > 1:  # output tiles alone cannot fill the GPU: split K, merge applies the epilogue
            need = int(_lib.query("iron_gemm_splitk_workspace_bytes", self.M, self.N, splits))
            ws = self._ws.get(A.device)
            if ws is None or ws.numel() < need:
                ws = torch.empty(need, dtype=torch.uint8, device=A.device)
                self._ws[A.device] = ws
            _lib.call("iron_gemm_bf16_nt_splitk", A.data_ptr(), B.data_ptr(), C.data_ptr(), self.M, self.N, self.K,
                      self.N, epi, has_clamp, lo, hi, splits, ws.data_ptr(), need, stream)
        else:
            _lib.call("iron_gemm_bf16_nt", A.data_ptr(), B.data_ptr(), C.data_ptr(), self.M, self.N, self.K, self.N,
                      epi, has_clamp, lo, hi, stream)

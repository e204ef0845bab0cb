"""GEMV: y = A . x on MI355X (reference: iron/operators/gemv/op.py:22-159).

Same dataclass fields, validation and arg spec as the reference:
``(matrix (B?,M,K), vector (B?,K), output (B?,M))``, B present when
``num_batches > 1``. The AIE tiling knobs (num_aie_columns, tile sizes,
kernel_vector_size) are accepted and checked the way the reference checks
them, then ignored: the HIP kernel assigns one wavefront per output row and
streams the row with 16-byte loads (iron_gemv_bf16 in csrc/gemv.hip).
"""

from dataclasses import dataclass, field
from typing import ClassVar, Dict

from ... import _lib
from ...common import HIPOperator, AIERuntimeArgSpec

EPILOGUES = {"none": 0, "gelu": 1}


@dataclass
class GEMV(HIPOperator):
    """bf16 General Matrix-Vector multiplication (optionally batched)."""

    M: int
    K: int
    num_aie_columns: int = 1
    tile_size_input: int = 2
    tile_size_output: int | None = None
    num_batches: int = 1
    kernel_vector_size: int = field(default=64, repr=False)
    epilogue: str = field(default="none", repr=False)
    context: object = field(default=None, repr=False)

    _name_aliases: ClassVar[Dict[str, str]] = {
        **HIPOperator._name_aliases,
        "num_aie_columns": "col",
        "tile_size_input": "tsi",
        "tile_size_output": "tso",
        "num_batches": "batch",
    }

    def __post_init__(self):
        if self.tile_size_output is None:
            self.tile_size_output = self.tile_size_input
        if not (
            self.tile_size_output % self.tile_size_input == 0
            and self.tile_size_output >= self.tile_size_input
        ):
            raise ValueError("tile_size_output must be a multiple of tile_size_input")
        if self.M <= 0 or self.K <= 0 or self.num_batches <= 0:
            raise ValueError(f"M ({self.M}), K ({self.K}) and num_batches must be positive")
        if self.K % 8:
            raise ValueError(f"K ({self.K}) must be a multiple of 8 (16-byte rows)")
        if self.epilogue not in EPILOGUES:
            raise ValueError(f"unknown epilogue {self.epilogue!r} (expected 'none' or 'gelu')")
        HIPOperator.__init__(self, context=self.context)

    @property
    def name(self) -> str:
        base = super().name
        return base if self.epilogue == "none" else f"{base}_epi{self.epilogue}"

    def get_arg_spec(self):
        batch_dim = (self.num_batches,) if self.num_batches > 1 else ()
        return [
            AIERuntimeArgSpec("in", batch_dim + (self.M, self.K)),  # matrix
            AIERuntimeArgSpec("in", batch_dim + (self.K,)),  # vector
            AIERuntimeArgSpec("out", batch_dim + (self.M,)),  # output
        ]

    def _launch(self, A, x, y, *, stream):
        _lib.call(
            "iron_gemv_bf16",
            A.data_ptr(),
            x.data_ptr(),
            y.data_ptr(),
            self.M,
            self.K,
            self.num_batches,
            EPILOGUES[self.epilogue],
            stream,
        )

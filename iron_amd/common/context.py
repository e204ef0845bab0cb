"""AIEContext counterpart (iron/common/context.py:12-67).

The reference context carries the MLIR-AIE build directory and compiler choice.
Here the only run-time state an operator needs is its GPU; the remaining
fields are accepted so code written against the reference constructs it
unchanged, and are otherwise advisory.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from pathlib import Path


@dataclass
class AIEContext:
    build_dir: Path | str = field(default_factory=lambda: Path("build"))
    mlir_verbose: bool = False
    compiler: str = "hipcc"
    device_index: int = 0

    def __post_init__(self) -> None:
        self.build_dir = Path(self.build_dir)

    @property
    def device(self):
        import torch

        return torch.device("cuda", self.device_index)

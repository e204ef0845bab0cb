"""Common utilities and base classes (counterpart of iron/common/__init__.py)."""

from .base import (
    AIEOperatorBase,
    HIPOperator,
    MLIROperator,
    CompositeOperator,
    AIERuntimeArgSpec,
)
from .context import AIEContext

__all__ = [
    "AIEOperatorBase",
    "HIPOperator",
    "MLIROperator",
    "CompositeOperator",
    "AIERuntimeArgSpec",
    "AIEContext",
]

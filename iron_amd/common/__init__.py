"""Common utilities and base classes (counterpart of iron/common/__init__.py)."""

from .base import (
    AIEOperatorBase,
    HIPOperator,
    MLIROperator,
    CompositeOperator,
    AIERuntimeArgSpec,
    set_reference_provider,
    get_reference_provider,
)
from .context import AIEContext
from .sequence import OperatorSequence, Tolerance

__all__ = [
    "AIEOperatorBase",
    "HIPOperator",
    "MLIROperator",
    "CompositeOperator",
    "AIERuntimeArgSpec",
    "AIEContext",
    "OperatorSequence",
    "Tolerance",
    "set_reference_provider",
    "get_reference_provider",
]

"""flm operators (iron/operators/flm/__init__.py:1-35), lazily re-exported:

    from iron_amd.operators.flm import GEMM
"""

import importlib

_OPERATOR_MODULES = {"GEMM": "gemm"}

__all__ = sorted(_OPERATOR_MODULES)


def __getattr__(name):
    module = _OPERATOR_MODULES.get(name)
    if module is None:
        raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
    return getattr(importlib.import_module(f".{module}.op", __name__), name)


def __dir__():
    return sorted(set(globals()) | set(_OPERATOR_MODULES))

"""The operator library (catalog of iron/operators/__init__.py:13-47).

Operators are re-exported lazily (PEP 562):

    from iron_amd.operators import GEMV   # imports iron_amd.operators.gemv.op only
"""

import importlib

_OPERATOR_MODULES = {
    "Dequant": "dequant",
    "ElementwiseAdd": "elementwise_add",
    "ElementwiseMul": "elementwise_mul",
    "GELU": "gelu",
    "GEMM": "gemm",
    "GEMMInt4": "gemm_int4",
    "GEMV": "gemv",
    "GEMVInt4": "gemv_int4",
    "GQADecode": "gqa_decode",
    "MHA": "mha",
    "RMSNorm": "rms_norm",
    "RoPE": "rope",
    "SiLU": "silu",
    "Softmax": "softmax",
    "SwiGLUDecode": "swiglu_decode",
    "SwiGLUPrefill": "swiglu_prefill",
    "Transpose": "transpose",
    "StridedCopy": "strided_copy",
    "Repeat": "repeat",
}

_SUBPACKAGES: tuple = ("flm",)

__all__ = sorted(set(_OPERATOR_MODULES) | set(_SUBPACKAGES))


def __getattr__(name):
    if name in _SUBPACKAGES:
        return importlib.import_module(f".{name}", __name__)
    module = _OPERATOR_MODULES.get(name)
    if module is None:
        raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
    return getattr(importlib.import_module(f".{module}.op", __name__), name)


def __dir__():
    return sorted(set(globals()) | set(_OPERATOR_MODULES) | set(_SUBPACKAGES))

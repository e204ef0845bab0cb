"""ctypes binding of libiron_hip.so (the C ABI declared in include/iron_hip.h).

The library is built in-tree by ``iron_amd._build`` (``__graft_entry__.build``).
There is no fallback: if the shared object is missing or a symbol is absent,
loading raises, and every operator call fails loudly.

torch is imported before the library is opened so that the HIP runtime torch
ships (soname libamdhip64.so.7) is the one the library binds to; the library
and torch then share one runtime, one device context and one set of streams.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libiron_hip.so"

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_LL = ctypes.c_longlong

# name -> argtypes (every function returns int, 0 = success) ...
SIGNATURES: dict[str, list] = {
    "iron_time_next_launch": [_P, _P],
    "iron_trace_next_launch": [_P, _LL],
    "iron_gemv_bf16": [_P, _P, _P, _I, _I, _I, _I, _P],
    "iron_gemv_bf16_fused": [_P, _P, _P, _P, _I, _I, _I, _P, _F, _P, _I, _P, _P],
    "iron_gemv_i4g32": [_P, _P, _P, _P, _I, _I, _I, _P],
    "iron_gemv_i4g32_fused": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _F, _P, _I, _P, _P],
    "iron_dequant_i4": [_P, _P, _P, _I, _I, _I, _I, _P],
    "iron_dequant_i4_payload": [_P, _P, _LL, _I, _I, _I, _P],
    "iron_rmsnorm": [_P, _P, _P, _P, _P, _I, _I, _F, _P],
    "iron_add": [_P, _P, _P, _LL, _P],
    "iron_mul": [_P, _P, _P, _LL, _P],
    "iron_silu": [_P, _P, _LL, _P],
    "iron_silu_mul": [_P, _P, _P, _LL, _P],
    "iron_gelu": [_P, _P, _LL, _P],
    "iron_softmax": [_P, _P, _I, _I, _I, _P, _P],
    "iron_rope": [_P, _P, _I, _P, _I, _I, _I, _I, _P],
    "iron_gqa_decode": [_P, _P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _P, _F, _P],
    "iron_gqa_decode_ex": [_P, _P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _P, _F, _I, _P],
    "iron_gqa_decode_noalloc": [_P, _P, _P, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I, _P, _F, _P],
    "iron_attention_prefill": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _LL, _LL, _LL, _LL, _LL, _LL, _I, _I, _I, _F, _P],
    "iron_gemm_bf16_nt": [_P, _P, _P, _I, _I, _I, _LL, _I, _I, _F, _F, _P],
    "iron_gemm_bf16_nt_splitk": [_P, _P, _P, _I, _I, _I, _LL, _I, _I, _F, _F, _I, _P, _LL, _P],
    "iron_gemm_bf16_nt_swiglu": [_P, _P, _P, _I, _I, _I, _LL, _P],
    "iron_gemm_i4g32_nt": [_P, _P, _P, _P, _I, _I, _I, _LL, _I, _I, _F, _F, _I, _I, _P, _LL, _P],
    "iron_transpose_bf16": [_P, _P, _I, _I, _P],
    "iron_transpose_batched_bf16": [_P, _P, _I, _I, _I, _P],
    "iron_repeat_rows": [_P, _P, _LL, _LL, _I, _P],
    "iron_strided_copy": [_P, _P, _I, _LL, _LL, _I, _P, _P, _LL, _P, _I, _P, _P, _LL, _P, _I, _P],
    "iron_quantize_i4g32": [_P, _P, _P, _I, _I, _P],
    "iron_embedding": [_P, _P, _P, _I, _I, _I, _P],
    "iron_argmax_bf16": [_P, _I, _P, _P, _P, _I, _P],
    "iron_argmax_select": [_P, _I, _P, _I, _I, _P, _P, _P, _P, _I, _P],
    "iron_qkv_rope_scatter": [_P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P],
    "iron_qkv_rope_scatter_splitk": [_P, _I, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P],
    "iron_rmsnorm_splitk": [_P, _P, _I, _P, _P, _P, _I, _I, _F, _P],
    "iron_gemm_nt_partials": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _LL, _P],
    "iron_llama_decode_fused": [_P, _I, _P, _I, _P, _I, _P, _P, _P, _I, _P, _I, _I, _F, _F, _P, _P, _P, _P, _P,
                                ctypes.c_uint, _I, _P],
    "iron_llama_decode_head": [_P, _P, _P, _P, _P, _I, _I, _F, _P, _P, _P],
    "iron_swiglu_decode_i4g32": [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _F, _P, _P, ctypes.c_uint, _P],
    "iron_probe_empty": [_I, _P],
    "iron_probe_read": [_P, _LL, _P, _LL, _I, _P],
    "iron_probe_mfma": [_I, _I, _I, _I, _P, _P, _LL, _P],
    "iron_probe_xcc_ids": [_I, _P, _P],
}

# ... except these queries, which return a value.
QUERIES: dict[str, tuple] = {
    "iron_gqa_decode_workspace_bytes": (_LL, [_I, _I, _I, _I]),
    "iron_gqa_decode_chunk_positions": (_I, [_I, _I, _I, _I, _I, _P]),
    "iron_gqa_decode_chunk_positions_ex": (_I, [_I, _I, _I, _I, _I, _I, _P]),
    "iron_gqa_decode_noalloc_max_bytes": (_LL, []),
    "iron_llama_decode_fused_exchange_bytes": (_LL, [_I]),
    "iron_swiglu_decode_i4g32_workspace_bytes": (_LL, [_I, _I]),
    "iron_xcd_round_robin": (_I, [_P]),
    "iron_gemm_splitk_choose": (_I, [_I, _I, _I]),
    "iron_gemm_i4g32_splitk_choose": (_I, [_I, _I, _I]),
    "iron_gemm_splitk_workspace_bytes": (_LL, [_I, _I, _I]),
    "iron_probe_read_workgroups": (_LL, [_LL, _I]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class IronHipError(RuntimeError):
    """A libiron_hip entry point returned an error code."""


def load() -> ctypes.CDLL:
    """Open libiron_hip.so once per process and declare its signatures."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built: run `python -m iron_amd._build` "
                "(or __graft_entry__.build()); there is no CPU fallback"
            )
        import torch  # noqa: F401  (binds the library to torch's HIP runtime)

        lib = ctypes.CDLL(str(LIB_PATH))
        lib.iron_last_error.restype = ctypes.c_char_p
        lib.iron_last_error.argtypes = []
        lib.iron_abi_version.restype = _I
        lib.iron_abi_version.argtypes = []
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)  # AttributeError if the build lacks it
            fn.restype = _I
            fn.argtypes = argtypes
        for name, (restype, argtypes) in QUERIES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
        return lib


def exported_symbols() -> list[str]:
    """Names of the C entry points this binding declares (for export checks)."""
    return ["iron_last_error", "iron_abi_version", *SIGNATURES, *QUERIES]


def call(name: str, *args) -> None:
    """Invoke entry point ``name``; raise IronHipError with the library's message on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.iron_last_error().decode(errors="replace")
        raise IronHipError(f"{name} failed (code {rc}): {msg}")


def query(name: str, *args):
    """Call a value-returning entry point (see QUERIES)."""
    return getattr(load(), name)(*args)


def ptr(t) -> int | None:
    """Device address of a torch tensor (None passes NULL)."""
    return None if t is None else t.data_ptr()


def stream_handle(device=None) -> int:
    """hipStream_t of torch's current stream on ``device``."""
    import torch

    return torch.cuda.current_stream(device).cuda_stream

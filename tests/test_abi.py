"""The C ABI: the library loads and exports exactly what include/iron_hip.h declares."""

import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "iron_hip.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(iron_\w+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_functions()
    assert "iron_gemv_bf16" in names and "iron_last_error" in names
    assert len(names) >= 8


def test_library_exports_every_declared_symbol():
    from iron_amd import _lib

    lib = _lib.load()
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True)
    exported = set(re.findall(r"\bT (iron_\w+)", out.stdout))
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, f"declared but not exported: {missing}"
    for n in declared_functions():
        assert hasattr(lib, n)


def test_binding_covers_header():
    from iron_amd import _lib

    assert sorted(_lib.exported_symbols()) == declared_functions()


def test_abi_version_and_error_path():
    from iron_amd import _lib

    lib = _lib.load()
    assert lib.iron_abi_version() == 1
    with pytest.raises(_lib.IronHipError, match="null pointer"):
        _lib.call("iron_gemv_bf16", None, None, None, 16, 16, 1, 0, None)
    with pytest.raises(_lib.IronHipError, match="multiple of 8"):
        _lib.call("iron_gemv_bf16", 16, 16, 16, 16, 12, 1, 0, None)


def test_splitk_consumer_argument_errors():
    """The split-K partials entry point and its consumers reject bad arguments
    on the host, before any launch."""
    from iron_amd import _lib

    with pytest.raises(_lib.IronHipError, match="exactly one of B"):
        _lib.call("iron_gemm_nt_partials", 16, 16, 16, 16, 1, 64, 64, 128, 2, 16, 1 << 20, None)
    with pytest.raises(_lib.IronHipError, match="must divide"):
        _lib.call("iron_gemm_nt_partials", 16, 16, None, None, 1, 64, 64, 192, 2, 16, 1 << 20, None)
    with pytest.raises(_lib.IronHipError, match="workspace of"):
        _lib.call("iron_gemm_nt_partials", 16, 16, None, None, 1, 64, 64, 128, 2, 16, 100, None)
    with pytest.raises(_lib.IronHipError, match="splits=0"):
        _lib.call("iron_rmsnorm_splitk", 16, 16, 0, None, 16, 16, 4, 64, 1e-5, None)
    with pytest.raises(_lib.IronHipError, match="multiple of 8"):
        _lib.call("iron_rmsnorm_splitk", 16, 16, 2, None, 16, 16, 4, 60, 1e-5, None)
    with pytest.raises(_lib.IronHipError, match="exceed the cache"):
        _lib.call("iron_qkv_rope_scatter_splitk", 16, 2, 16, 64, 16, 16, 16, 8, 4, 2, 64, 64, 60, None)



def test_time_next_launch_argument_error():
    from iron_amd import _lib

    with pytest.raises(_lib.IronHipError, match="both events or neither"):
        _lib.call("iron_time_next_launch", 16, None)
    _lib.call("iron_time_next_launch", None, None)  # disarm: always accepted


def test_operator_catalog_resolves():
    """Every name of the lazy operator catalog (iron/operators/__init__.py:13-47
    counterpart) imports and is an operator class with the reference's
    get_arg_spec / get_callable surface; unknown names raise AttributeError."""
    import iron_amd.operators as catalog

    for name in catalog.__all__:
        obj = getattr(catalog, name)
        if name == "flm":
            assert hasattr(obj, "GEMM")
            continue
        assert isinstance(obj, type) and obj.__name__ == name, name
        assert hasattr(obj, "get_arg_spec") and hasattr(obj, "get_callable"), name
    with pytest.raises(AttributeError):
        getattr(catalog, "NoSuchOperator")


def test_gqa_decode_noalloc_rejects_oversized_shape_on_host():
    """The no-allocation decode attention refuses, before touching a GPU, a shape
    whose partials exceed the library's scratch array."""
    from iron_amd import _lib

    cap = _lib.query("iron_gqa_decode_noalloc_max_bytes")
    assert cap == 4 << 20
    assert _lib.query("iron_gqa_decode_workspace_bytes", 32, 8, 64, 29056) <= cap
    assert _lib.query("iron_gqa_decode_workspace_bytes", 32, 8, 64, 29057) > cap
    with pytest.raises(_lib.IronHipError, match="more than the 4194304"):
        _lib.call("iron_gqa_decode_noalloc", 16, 16, 16, 16, 16, 16, 32768, 16, 32, 8, 64, 32768, 0, None, 0.125,
                  None)
    with pytest.raises(_lib.IronHipError, match="invalid shape"):
        _lib.call("iron_gqa_decode_noalloc", 16, 16, 16, 16, 16, 16, 128, 16, 32, 8, 32, 128, 0, None, 0.125, None)


def test_offset_limits_rejected_on_host():
    """Arguments past the kernels' 32-bit buffer offsets are rejected before any launch:
    GEMM K above 2^21, prefill-attention K/V spans of 2 GiB or more."""
    from iron_amd import _lib

    p = 1 << 20  # a 16-byte-aligned stand-in address: nothing is launched
    with pytest.raises(_lib.IronHipError, match="exceeds"):
        _lib.call("iron_gemm_bf16_nt", p, p, p, 64, 64, (1 << 21) + 64, 64, 0, 0, 0.0, 0.0, None)
    with pytest.raises(_lib.IronHipError, match="2 GiB"):
        _lib.call("iron_attention_prefill", p, p, p, p, 8, 8, 16, 1 << 20, 64, 64, 512, 64, 1 << 10, 64, 512, 16, 1, 0,
                  0.125, None)


def test_gqa_decode_ex_rejects_unknown_flags_on_host():
    """Flag bits other than IRON_GQA_KV_RESIDENT and IRON_GQA_COUNTERS_ZERO are refused before anything runs."""
    from iron_amd import _lib

    with pytest.raises(_lib.IronHipError, match="unknown flags"):
        _lib.call("iron_gqa_decode_ex", 16, 16, 16, 16, 16, 16, 128, 16, 256, 32, 8, 64, 128, 0, None, 0.125, 4, None)


def test_swiglu_decode_one_launch_rejects_on_host():
    """The one-launch SwiGLU block takes E=2048, F=8192 only, checks its
    pointers, alignments, norm mode and wait bound before anything runs."""
    from iron_amd import _lib

    assert _lib.query("iron_swiglu_decode_i4g32_workspace_bytes", 2048, 8192) == 256 + 8 * 4096
    assert _lib.query("iron_swiglu_decode_i4g32_workspace_bytes", 4096, 8192) == -1
    p = 1 << 20  # a 256-byte-aligned stand-in address: nothing is launched

    def call(E=2048, F=8192, mode=2, norm_w=None, ws=p, wait=1000, x=p):
        _lib.call("iron_swiglu_decode_i4g32", p, p, p, p, p, p, x, p, E, F, 1, mode, norm_w, 1e-5, None, ws, wait,
                  None)

    with pytest.raises(_lib.IronHipError, match="E=4096"):
        call(E=4096)
    with pytest.raises(_lib.IronHipError, match="norm_mode=3"):
        call(mode=3)
    with pytest.raises(_lib.IronHipError, match="needs norm_w"):
        call(mode=1)
    with pytest.raises(_lib.IronHipError, match="wait_us=0"):
        call(wait=0)
    with pytest.raises(_lib.IronHipError, match="aligned"):
        call(ws=p + 16)
    with pytest.raises(_lib.IronHipError, match="aligned"):
        call(x=p + 2)
    with pytest.raises(_lib.IronHipError, match="null pointer"):
        call(ws=None)

"""CPU: the C ABI's argument checks under AddressSanitizer. The library with
its host code instrumented (iron_amd._build.build_asan: AddressSanitizer on
the host side only) is loaded into a subprocess with clang's ASan runtime preloaded,
and every entry point is called with arguments it must refuse (NULL and
misaligned pointers, zero and negative sizes) plus every query: each must
return IRON_EINVAL (22) with a message in iron_last_error(), and ASan must report
nothing (it aborts the process on an invalid access)."""

import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def test_abi_argument_checks_under_asan(tmp_path):
    from iron_amd import _build

    try:
        _build._hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    rt = _build.asan_runtime()
    if rt is None:
        pytest.skip("clang's ASan runtime not found")
    lib = _build.build_asan(tmp_path / "asan")
    env = dict(os.environ, LD_PRELOAD=str(rt), ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:halt_on_error=1",
               HIP_VISIBLE_DEVICES="")  # the checks need no device: none is offered
    res = subprocess.run([sys.executable, str(ROOT / "tests" / "asan_abi_driver.py"), str(lib)], env=env,
                         capture_output=True, text=True, timeout=300)
    print(res.stdout[-2000:], res.stderr[-4000:])
    assert res.returncode == 0, res.stderr[-4000:]
    assert "AddressSanitizer" not in res.stderr
    assert "rejected or answered cleanly" in res.stdout

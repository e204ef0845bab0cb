"""Exercise every C-ABI entry point's argument checks in the AddressSanitizer
host build (iron_amd._build.build_asan); run by tests/test_asan_abi.py in a
subprocess with the ASan runtime preloaded, so that any invalid memory access
in the checks or the error reporting aborts with a report. No GPU is touched:
every call below is one the host rejects before anything is launched.

    python tests/asan_abi_driver.py <path to libiron_hip_asan.so>
"""

import ctypes
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parent.parent))

from iron_amd import _lib  # noqa: E402  (the argument tables only; the GPU library is not loaded)

EINVAL = 22
# entry points with no argument to refuse: iron_time_next_launch takes two event
# handles (NULL, NULL disarms; others arm), which it only records;
# iron_trace_next_launch takes NULL as "disarm" (its alignment check is called below)
NO_CHECKS = {"iron_time_next_launch", "iron_trace_next_launch"}


def _args(argtypes, ptr, i, f):
    out = []
    for t in argtypes:
        if t is _lib._P:
            out.append(ptr)
        elif t is _lib._F:
            out.append(f)
        elif t is ctypes.c_uint:
            out.append(0)
        else:
            out.append(i)
    return out


def main() -> int:
    lib = ctypes.CDLL(sys.argv[1])
    lib.iron_last_error.restype = ctypes.c_char_p
    lib.iron_last_error.argtypes = []
    calls = 0
    for name, argtypes in _lib.SIGNATURES.items():
        if name in NO_CHECKS:
            continue
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int
        fn.argtypes = argtypes
        # all-zero (NULL pointers, zero sizes), then misaligned stand-in pointers with negative sizes
        for ptr, i, f in ((None, 0, 0.0), ((1 << 20) + 2, -1, -1.0)):
            rc = fn(*_args(argtypes, ptr, i, f))
            calls += 1
            assert rc == EINVAL, (name, ptr, rc)
            msg = lib.iron_last_error()
            assert msg and len(msg) > 8, (name, msg)  # a description of what was refused
    tr = lib.iron_trace_next_launch
    tr.restype, tr.argtypes = ctypes.c_int, _lib.SIGNATURES["iron_trace_next_launch"]
    assert tr((1 << 20) + 16, 4096) == EINVAL and lib.iron_last_error()
    assert tr(None, 0) == 0
    calls += 2
    for name, (restype, argtypes) in _lib.QUERIES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
        for i in (0, -1, 1 << 30):
            fn(*_args(argtypes, None, i, 0.0))
            calls += 1
    print(f"asan driver: {calls} calls rejected or answered cleanly", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

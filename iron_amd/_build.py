"""Build libiron_hip.so from iron_amd/csrc/*.hip for gfx950.

Every translation unit is compiled in parallel with hipcc into
``iron_amd/_objs/`` and linked in-tree into ``iron_amd/libiron_hip.so`` (the
file the ctypes loader opens and the one that travels to the GPU box).

Usage:  python -m iron_amd._build  [--jobs N] [--verbose]
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ = PKG / "_objs"
LIB = PKG / "libiron_hip.so"
INCLUDE = PKG.parent / "include"

ARCH = "gfx950"

# -packed-fp32-ops keeps the compiler from emitting v_pk_{add,mul,fma}_f32.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    "-Wno-unknown-pragmas",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


# Per-file additions for attention.hip. MFMA accumulators stay in VGPRs: the
# flash-attention loop rescales its output accumulators with VALU ops, and with
# accumulators in AGPRs the compiler copied them back and forth every block.
# -fno-honor-nans: max(a, b) of finite scores then needs no NaN-quieting
# v_max_f32 per operand (finite inputs give identical results).
# decode_fused.hip runs the same decode attention body, so it takes the same flags.
# gemv.hip, attention.hip, llama.hip: the dispatch preloads a kernel's leading
# scalar and pointer arguments into SGPRs (up to 14 SGPRs; a struct argument
# ends the preloaded run), so the GEMVs, the decode attention and the token
# select issue their first loads without waiting for an argument fetch.
# probe.hip: the floor probes get the same, so that the floors they measure
# are those of kernels launched like the product's.
FILE_FLAGS = {
    "gemv.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=7"],
    "llama.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=8"],
    "probe.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=3"],
    "attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-fno-honor-nans", "-mllvm", "-amdgpu-kernarg-preload-count=9"],
    "decode_fused.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-fno-honor-nans"],
}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP extension cannot be built")


def _compile(src: Path, verbose: bool) -> Path:
    obj = OBJ / (src.stem + ".o")
    cmd = [_hipcc(), *HIP_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the -packed-fp32-ops feature; drop that line.
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile every csrc/*.hip and link libiron_hip.so. Always rebuilds."""
    OBJ.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 4)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), sources))
    tmp = LIB.with_suffix(".so.tmp")
    # --no-undefined: a kernel whose host-side launch stub was silently not emitted
    # (the host pass drops a template kernel whose body it cannot instantiate) fails here
    # instead of at dlopen on the GPU box
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined", "-o", str(tmp),
           *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


def asan_runtime() -> Path | None:
    """clang's AddressSanitizer runtime next to hipcc's clang (preloaded into
    the Python process that loads the sanitized library), or None."""
    root = Path(_hipcc()).resolve().parent.parent
    for base in (root / "lib" / "llvm" / "lib" / "clang", Path("/opt/rocm/lib/llvm/lib/clang")):
        hits = sorted(base.glob("*/lib/linux/libclang_rt.asan-x86_64.so")) if base.exists() else []
        if hits:
            return hits[-1]
    return None


def build_asan(out_dir: Path, jobs: int | None = None) -> Path:
    """The library with its host code built under AddressSanitizer
    (``libiron_hip_asan.so`` in out_dir): every entry point's argument checks
    and error reporting are instrumented; the device code is the ordinary
    gfx950 build (the sanitizer applies to the host side only). It is linked
    without the sanitizer runtime, which the process that loads it preloads.
    For CPU tests of the validation paths; the GPU library is build()'s."""
    out_dir = Path(out_dir)
    out_dir.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    host_asan = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer"]

    def one(src: Path) -> Path:
        obj = out_dir / (src.stem + ".o")
        cmd = [_hipcc(), *HIP_FLAGS, *FILE_FLAGS.get(src.name, []), *host_asan, "-c", str(src), "-o", str(obj)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc (host asan) failed on {src.name}:\n{res.stderr[-2000:]}")
        return obj

    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 4)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(one, sources))
    lib = out_dir / "libiron_hip_asan.so"
    res = subprocess.run([_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(lib), *map(str, objs)],
                         capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"asan link failed:\n{res.stderr[-2000:]}")
    return lib


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args()
    print(build(args.jobs, args.verbose))


if __name__ == "__main__":
    main()

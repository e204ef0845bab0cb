"""Contracts of hand-written assembly that the compiler cannot check, verified
on the gfx950 assembly of this repository's own sources (no GPU needed).

load_lds16 (iron_common.hpp) writes M0 behind the compiler's back: in every
kernel that uses it, each M0 write must be its own (followed by one wait state,
s_nop 0, then its buffer_load ... lds), so the compiler never keeps a value of
its own in M0 there, and no LDS-DMA load directly follows the M0 write it reads
(GFX9 needs one wait state between the two).

The compiler does not count those loads, so a vmcnt wait it inserts for a
load of its own also waits for every K/V block in flight. In the prefill
attention, after the first LDS-DMA load, every vmcnt wait must be one of the
kernel's own waits right before its barriers.
"""

import re
import subprocess

import pytest

from iron_amd import _build

KERNELS = {
    "gemm.hip": ["gemm_nt_kernel"],
    "attention.hip": ["attention_prefill_kernel"],
}


def device_asm(src_name):
    try:
        hipcc = _build._hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    src = _build.CSRC / src_name
    cmd = [hipcc, *_build.HIP_FLAGS, *_build.FILE_FLAGS.get(src_name, []), "--cuda-device-only", "-S", str(src),
           "-o", "-"]
    out = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stderr[-2000:]
    return out.stdout


def functions(asm):
    """name -> list of instruction lines of each function in the assembly (a
    function runs from its label to its .Lfunc_end label: it may hold several
    s_endpgm, one per exit)."""
    funcs, name, body = {}, None, []
    for line in asm.splitlines():
        m = re.match(r"^(_Z\S+):", line)
        if m:
            name, body = m.group(1), []
            funcs[name] = body
            continue
        if line.startswith(".Lfunc_end"):
            name = None
            continue
        if name is not None:
            s = line.split(";")[0].strip()
            if s and not s.startswith("."):
                body.append(s)
    return funcs


@pytest.mark.parametrize("src_name", sorted(KERNELS))
def test_m0_written_only_by_load_lds16(src_name):
    funcs = functions(device_asm(src_name))
    checked = 0
    for fname, body in funcs.items():
        if not any(k in fname for k in KERNELS[src_name]):
            continue
        checked += 1
        loads = 0
        for i, ins in enumerate(body):
            if re.search(r"\bm0\b", ins):
                assert ins.startswith("s_mov_b32 m0,"), (fname, i, ins)
                nop = body[i + 1] if i + 1 < len(body) else ""
                nxt = body[i + 2] if i + 2 < len(body) else ""
                assert nop == "s_nop 0", (fname, i, ins, nop)
                assert nxt.startswith("buffer_load_dwordx4") and nxt.endswith("lds"), (fname, i, ins, nxt)
                loads += 1
        assert loads > 0, fname
        assert not any(ins.startswith("global_load_lds") for ins in body), fname
    assert checked > 0, f"no kernel of {KERNELS[src_name]} found in {src_name}"


def test_prefill_attention_loop_has_no_compiler_vmcnt_wait():
    funcs = functions(device_asm("attention.hip"))
    bodies = [b for name, b in funcs.items() if "attention_prefill_kernel" in name]
    assert bodies, "attention_prefill_kernel not found"
    for body in bodies:
        first = next(i for i, ins in enumerate(body) if ins.startswith("buffer_load_dwordx4") and ins.endswith("lds"))
        waits = [(i, ins) for i, ins in enumerate(body[first:], first) if ins.startswith("s_waitcnt") and "vmcnt" in ins]
        assert waits, "no vmcnt wait after the first K/V load"
        for i, ins in waits:
            nxt = body[i + 1] if i + 1 < len(body) else ""
            assert nxt == "s_barrier", (i, ins, nxt)

"""CPU: the built library's decode kernels have their leading arguments
preloaded into SGPRs (the kernarg preload counts in iron_amd/_build.py).

Results do not depend on it, so no parity test would notice a build that lost
the flags; decode would only run ~6% slower. This test reads the gfx950 code
objects inside libiron_hip.so (the clang offload bundles of its .hip_fatbin
section) and checks each hot kernel's descriptor: bits 0-6 of the 16-bit
KERNARG_PRELOAD field at byte 58 hold the number of SGPRs the dispatch fills
with kernel arguments.
"""

import struct
from pathlib import Path

import pytest

LIB = Path(__file__).resolve().parent.parent / "iron_amd" / "libiron_hip.so"
BUNDLE_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def _section_headers(elf: bytes) -> list:
    """(name, file offset, size, address, link, entry size) per section of an
    ELF64 little-endian file, in section-index order."""
    assert elf[:4] == b"\x7fELF" and elf[4] == 2 and elf[5] == 1
    shoff, = struct.unpack_from("<Q", elf, 0x28)
    shentsize, shnum, shstrndx = struct.unpack_from("<HHH", elf, 0x3A)
    hdrs = [struct.unpack_from("<IIQQQQIIQQ", elf, shoff + i * shentsize) for i in range(shnum)]
    names_off = hdrs[shstrndx][4]

    def name(o):
        end = elf.index(b"\0", names_off + o)
        return elf[names_off + o:end].decode()

    return [(name(h[0]), h[4], h[5], h[3], h[6], h[9]) for h in hdrs]


def _sections(elf: bytes) -> dict:
    """name -> (file offset, size, address, link, entry size)."""
    return {h[0]: h[1:] for h in _section_headers(elf)}


def _code_objects(lib: bytes) -> list[bytes]:
    """The gfx950 device ELFs of every offload bundle in .hip_fatbin."""
    off, size, *_ = _sections(lib)[".hip_fatbin"]
    fat = lib[off:off + size]
    out, pos = [], fat.find(BUNDLE_MAGIC)
    while pos >= 0:
        n, = struct.unpack_from("<Q", fat, pos + 24)
        p = pos + 32
        for _ in range(n):
            eoff, esize, tlen = struct.unpack_from("<QQQ", fat, p)
            triple = fat[p + 24:p + 24 + tlen].decode()
            p += 24 + tlen
            if "gfx950" in triple:
                out.append(fat[pos + eoff:pos + eoff + esize])
        pos = fat.find(BUNDLE_MAGIC, pos + 24)
    return out


def _preload_lengths(co: bytes) -> dict:
    """kernel symbol -> kernarg preload length (SGPRs) from its descriptor."""
    hdrs = _section_headers(co)
    secs = {h[0]: h[1:] for h in hdrs}
    symoff, symsize, _, _, entsize = secs[".dynsym"]
    stroff = secs[".dynstr"][0]
    out = {}
    for i in range(symsize // entsize):
        st_name, _, _, st_shndx, st_value, _ = struct.unpack_from("<IBBHQQ", co, symoff + i * entsize)
        end = co.index(b"\0", stroff + st_name)
        name = co[stroff + st_name:end].decode()
        if not name.endswith(".kd") or not 0 < st_shndx < len(hdrs):
            continue  # defined descriptors only
        # the descriptor's file offset: its address within the section that holds it
        _, off, size, addr, _, _ = hdrs[st_shndx]
        assert addr <= st_value and st_value + 64 <= addr + size, name
        kd = co[off + st_value - addr:off + st_value - addr + 64]
        out[name[:-3]] = struct.unpack_from("<H", kd, 58)[0] & 0x7F
    return out


@pytest.fixture(scope="module")
def lengths():
    if not LIB.exists():
        pytest.skip("libiron_hip.so is not built")
    found = {}
    for co in _code_objects(LIB.read_bytes()):
        found.update(_preload_lengths(co))
    assert found, "no gfx950 kernel descriptors found in the library"
    return found


def _min_length(lengths, fragment):
    ks = {k: v for k, v in lengths.items() if fragment in k}
    assert ks, f"no kernel named like {fragment}"
    return min(ks.values()), ks


@pytest.mark.parametrize(
    "fragment, sgprs",
    [
        ("12gemv_i4_fast", 13),  # codes, scales, x, codes2, scales2, resid: 6 x 2, M: 1
        ("14gemv_bf16_fast", 9),  # W, W2, x, resid: 4 x 2, M: 1
        ("17gqa_decode_kernel", 14),  # 5 pointers, pos, nsplit, max_len, angle_rows
        ("19select_embed_kernel", 14),
    ],
)
def test_decode_kernels_preload_their_leading_arguments(lengths, fragment, sgprs):
    got, ks = _min_length(lengths, fragment)
    assert got >= sgprs, f"{fragment}: kernarg preload {got} SGPRs < {sgprs} ({sorted(ks.items())[:3]})"


def test_struct_only_kernels_preload_nothing(lengths):
    """A kernel whose first argument is a struct gets no preload (the run ends
    at the struct): the GEMM keeps its arguments in GemmArgs."""
    got, ks = _min_length(lengths, "14gemm_nt_kernel")
    assert max(ks.values()) == 0

"""iron_amd: the IRON operator API on MI355X (gfx950) HIP kernels.

Operators keep the reference's names and call signatures
(``from iron_amd.operators import GEMV``); every kernel is hand-written HIP
in iron_amd/csrc, built into libiron_hip.so and reached through its C ABI
(include/iron_hip.h).
"""

__version__ = "0.1.0"

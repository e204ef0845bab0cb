"""Small helpers shared by the operators."""


def float_to_name(v: float) -> str:
    """Filesystem-safe spelling of a float for operator names.

    Same mapping as the reference's helper (iron/common/utils.py:23-38), so
    operator names derived from dataclass fields agree: shortest round-trip
    repr with '.' -> 'p', '-' -> 'n' and '+' dropped (0.01 -> '0p01').
    """
    return repr(v).replace(".", "p").replace("-", "n").replace("+", "")

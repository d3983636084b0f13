"""Level types and level arithmetic of the Fenwick hierarchy.

Mirrors the public names of hattention/base.py:12-72 (``HType``, ``HStruct``,
``ceil_log``, ``floor_log``, ``get_num_levels``, ``get_level_index``).  The
weak level of a pair is computed in closed form, ``bit_length(t ^ s)``, which
equals the reference recursion (base.py:41-46) for every pair; the kernels
evaluate the same closed form in registers, so no T x T level table
(base.py:101-161) is ever built and the reference's T <= 16384 table limit
does not apply.
"""
import math
from enum import Enum


class HType(Enum):
    """base.py:12-14."""
    WEAK = 0
    STRONG = 1


class HStruct(Enum):
    """base.py:17-19."""
    MAMBA2 = 0
    GDELTA = 1


def ceil_log(x: int, b: int) -> int:
    """base.py:29-30 for integers (exact; no floating-point log)."""
    if b == 2 and isinstance(x, int) and x >= 1:
        return (x - 1).bit_length()
    return math.ceil(math.log(x, b))


def floor_log(x: int, b: int) -> int:
    """base.py:33-34 for integers."""
    if b == 2 and isinstance(x, int) and x >= 1:
        return x.bit_length() - 1
    return math.floor(math.log(x, b))


def get_num_levels(length: int, base: int) -> int:
    """base.py:37-38: levels needed for ``length`` tokens."""
    return ceil_log(length, base) + 1


def get_level_index(t: int, s: int, b: int, htype: HType) -> int:
    """base.py:65-72 for the weak hierarchy with base 2 (t > s)."""
    if t <= s:
        raise ValueError
    if htype != HType.WEAK or b != 2:
        raise NotImplementedError("only HType.WEAK with level base 2 is supported")
    return (t ^ s).bit_length()

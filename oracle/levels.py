"""Level function of the weak (HType.WEAK, base 2) Fenwick hierarchy.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Restates:
* ``floor_log`` / ``ceil_log`` / ``get_num_levels``      -- hattention/base.py:29-38
* ``get_level_index_weak`` (the recursion)              -- hattention/base.py:41-46
* ``make_levels_matrix`` (T x T table, default / clamp) -- hattention/base.py:101-161
* ``skip_kv`` / ``skip_q`` / ``skip_g`` (chunk schedule) -- hattention/chunkwise.py:34-74

Pinning: the closed form ``level(t, s) = bit_length(t ^ s)`` (0 on the
diagonal) is checked against the recursion by brute force over every pair
with t < 2048 and against random pairs up to 2^15; the chunk schedule is
checked against the closed form (a pair of chunks (i, j), j < i, is served by
inter-chunk level ``bit_length(i ^ j) - 1``, i.e. absolute level
``6 + bit_length(i ^ j)`` for a 64-token chunk).
"""
import math

import numpy as np


def floor_log(x: int, b: int) -> int:
    """base.py:33-34 (uses math.log exactly like the reference)."""
    return math.floor(math.log(x, b))


def ceil_log(x: int, b: int) -> int:
    """base.py:29-30."""
    return math.ceil(math.log(x, b))


def get_num_levels(length: int, base: int) -> int:
    """base.py:37-38."""
    return ceil_log(length, base) + 1


def level_weak_recursive(t: int, s: int, b: int = 2) -> int:
    """Restatement of ``get_level_index_weak`` (base.py:41-46), for t > s."""
    while True:
        ell = floor_log(t, b)
        v = b ** ell
        if s < v:
            return ell + 1
        t, s = t - v, s - v


def level_closed_form(t: int, s: int) -> int:
    """0 on the diagonal, ``bit_length(t ^ s)`` strictly below it (t > s)."""
    if t == s:
        return 0
    return (t ^ s).bit_length()


def levels_matrix(length: int, default: int = -1, clamp_min=None) -> np.ndarray:
    """Vectorised closed form of ``make_levels_matrix`` (base.py:101-161).

    Entry [t, s] is the level of the pair for s <= t and ``default`` above the
    diagonal; ``clamp_min`` clamps like base.py:158-159.
    """
    t = np.arange(length, dtype=np.int64)[:, None]
    s = np.arange(length, dtype=np.int64)[None, :]
    x = np.bitwise_xor(t, s)
    # bit_length via frexp-free integer loop (exact for any int64)
    lev = np.zeros_like(x)
    y = x.copy()
    while np.any(y):
        nz = y > 0
        lev[nz] += 1
        y >>= 1
    out = np.where(s <= t, lev, default).astype(np.int64)
    if clamp_min is not None:
        out = np.maximum(out, clamp_min)
    return out


def skip_kv(i_t: int, ell: int) -> bool:
    """chunkwise.py:34-42: chunk i_t does not write its kv into level ell."""
    return ((i_t >> ell) & 1) == 1


def skip_q(i_t: int, ell: int) -> bool:
    """chunkwise.py:45-48: chunk i_t does not read level ell."""
    return not skip_kv(i_t, ell)


def skip_g(i_t: int, ell: int, backward: bool = False) -> bool:
    """chunkwise.py:51-74 (OFFSET=False): forward reset after the last chunk of
    an aligned 2^(ell+1) block; backward reset at its first chunk."""
    period = 1 << (ell + 1)
    if not backward:
        return i_t % period == period - 1
    return i_t % period == 0

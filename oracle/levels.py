"""Level functions of the weak and strong (HType.WEAK / HType.STRONG, base 2)
hierarchies.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Restates:
* ``floor_log`` / ``ceil_log`` / ``get_num_levels``      -- hattention/base.py:29-38
* ``get_level_index_weak`` (the recursion)              -- hattention/base.py:41-46
* ``make_levels_matrix`` (T x T table, default / clamp) -- hattention/base.py:101-161
* ``skip_kv`` / ``skip_q`` / ``skip_g`` (chunk schedule) -- hattention/chunkwise.py:34-74
* ``level_strong_recursive`` (the strong recursion)   -- hattention/base.py:49-62
* ``levels_matrix_strong`` (its T x T table)           -- hattention/base.py:101-161

The strong hierarchy at a chunk of C = 2^c tokens (``strong_intra_table``,
``strong_subdiag_table``, ``strong_far_level``): every diagonal C x C block
holds one table, every sub-diagonal block (source chunk = target chunk - 1)
holds one other table, and a pair of chunks further apart (c_s <= c_t - 2)
has a single level c + strong(c_t, c_s), the strong function of the chunk
indices.  This is what a chunkwise strong kernel uses; it is checked by brute
force against the recursion (tests/test_oracle_levels.py).

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


# --------------------------------------------------------------------------
# strong hierarchy (HType.STRONG)
# --------------------------------------------------------------------------
def level_strong_recursive(t: int, s: int, b: int = 2) -> int:
    """Restatement of ``get_level_index_strong`` (base.py:49-62), for t > s."""
    if b != 2:
        raise NotImplementedError
    while True:
        ell = floor_log(t, b)
        v = b ** max(ell - 1, 0)
        r = t - b ** ell
        if s < v:
            return ell + 1
        if s < v * 2 and r >= v:
            return ell + 1
        if s < v * 2:
            t, s = t - v, s - v
        else:
            t, s = t - 2 * v, s - 2 * v


def levels_matrix_strong(length: int, default: int = -1, clamp_min=None) -> np.ndarray:
    """The strong recursion evaluated for every pair at once (numpy, exact
    integer arithmetic; floor_log2 as bit length - 1, which equals the
    reference's floor(log(x, 2)) for every x < 2^15): entry [t, s] is the level
    for s < t, 0 on the diagonal, ``default`` above it (base.py:141-161)."""
    t = np.broadcast_to(np.arange(length, dtype=np.int64)[:, None], (length, length)).copy()
    s = np.broadcast_to(np.arange(length, dtype=np.int64)[None, :], (length, length)).copy()
    out = np.zeros((length, length), dtype=np.int64)
    live = s < t
    while np.any(live):
        tl, sl = t[live], s[live]
        ell = np.floor(np.log2(tl)).astype(np.int64)
        # exact floor(log2) for positive integers
        ell = np.where((1 << (ell + 1)) <= tl, ell + 1, ell)
        ell = np.where((1 << ell) > tl, ell - 1, ell)
        v = np.left_shift(1, np.maximum(ell - 1, 0))
        r = tl - np.left_shift(1, ell)
        done = (sl < v) | ((sl < 2 * v) & (r >= v))
        step = np.where(sl < 2 * v, v, 2 * v)
        idx = np.nonzero(live)
        res = out[idx]
        res[done] = ell[done] + 1
        out[idx] = res
        nt, ns = tl - step, sl - step
        tt, ss = t[idx], s[idx]
        tt[~done], ss[~done] = nt[~done], ns[~done]
        t[idx], s[idx] = tt, ss
        lv = live[idx]
        lv[done] = False
        live[idx] = lv
    out = np.where(np.arange(length)[None, :] <= np.arange(length)[:, None], out, default)
    if clamp_min is not None:
        out = np.maximum(out, clamp_min)
    return out.astype(np.int64)


def strong_intra_table(C: int) -> np.ndarray:
    """Levels of the pairs inside one chunk of C tokens (t >= s; 0 on the
    diagonal, 0 above it)."""
    return np.maximum(levels_matrix_strong(C, default=0), 0)


def strong_subdiag_table(C: int) -> np.ndarray:
    """Levels of target position a of chunk i and source position b of chunk
    i - 1 (any i >= 1): the block [C, 2C) x [0, C) of the strong table."""
    return levels_matrix_strong(2 * C, default=0)[C:, :C].copy()


def strong_far_level(ct: int, cs: int, C: int) -> int:
    """Level of every pair of target chunk ct and source chunk cs <= ct - 2:
    log2(C) + strong(ct, cs)."""
    if cs > ct - 2:
        raise ValueError("not a far chunk pair")
    return int(math.log2(C)) + level_strong_recursive(ct, cs)

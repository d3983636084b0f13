"""Pin the level function and the chunk schedule (oracle/levels.py).

The closed form bit_length(t ^ s) is checked against the reference's own
recursion (base.py:41-46, restated with math.log exactly as written) by brute
force, and the chunk-scan schedule (chunkwise.py:34-74) is checked against
the closed form: every (reading chunk i, source chunk j<i) pair is served by
exactly one inter-chunk level, and that level is bit_length(i ^ j) - 1.

The strong level function (base.py:49-62): the vectorised table against the
recursion by brute force, a few hand-derived rows, and the chunk
decomposition a chunkwise strong kernel relies on (one table for the diagonal
blocks, one for the sub-diagonal blocks, a single chunk-pair level elsewhere).
"""
import random

import numpy as np
import pytest

from oracle.levels import (level_weak_recursive, level_closed_form, levels_matrix,
                           skip_kv, skip_q, skip_g, get_num_levels, ceil_log)


def test_closed_form_matches_recursion_all_pairs_below_2048():
    for t in range(1, 2048):
        for s in range(t):
            assert level_weak_recursive(t, s) == level_closed_form(t, s), (t, s)


def test_closed_form_matches_recursion_random_pairs_to_2e15():
    rng = random.Random(0)
    for _ in range(20000):
        t = rng.randrange(1, 1 << 15)
        s = rng.randrange(0, t)
        assert level_weak_recursive(t, s) == level_closed_form(t, s), (t, s)


def test_levels_matrix_table():
    T = 300
    m = levels_matrix(T)
    for t in range(T):
        assert m[t, t] == 0
        for s in range(t):
            assert m[t, s] == level_weak_recursive(t, s)
        for s in range(t + 1, T):
            assert m[t, s] == -1
    assert (levels_matrix(T, clamp_min=0) >= 0).all()


def test_known_values():
    # chunk 1 vs chunk 0 -> level 7; chunks 2-3 vs 0-1 -> level 8; 3 vs 2 -> 7
    assert level_closed_form(64, 63) == 7
    assert level_closed_form(64 * 2, 0) == 8 and level_closed_form(64 * 3 + 5, 64 + 7) == 8
    assert level_closed_form(64 * 3, 64 * 2 + 63) == 7
    assert get_num_levels(64, 2) == 7
    assert ceil_log(256, 2) == 8


def test_schedule_serves_each_pair_once_at_its_level():
    NT = 64
    nlev = ceil_log(NT, 2)
    for ell in range(nlev):
        # simulate which source chunks are inside the state read by chunk i
        state = set()
        for i in range(NT):
            if not skip_q(i, ell):
                for j in state:
                    assert level_closed_form(i, j) - 1 == ell
                for j in range(i):
                    if level_closed_form(i, j) - 1 == ell:
                        assert j in state
            if skip_g(i, ell):
                state = set()
            if not skip_kv(i, ell):
                state.add(i)


# ---- strong hierarchy (base.py:49-62) ------------------------------------
from oracle.levels import (level_strong_recursive, levels_matrix_strong, strong_far_level,  # noqa: E402
                           strong_intra_table, strong_subdiag_table)


def test_strong_matrix_matches_recursion_all_pairs_below_512():
    M = levels_matrix_strong(512)
    for t in range(512):
        for s in range(t):
            assert M[t, s] == level_strong_recursive(t, s), (t, s)
        assert M[t, t] == 0
        assert (M[t, t + 1:] == -1).all()


def test_strong_known_values():
    # a row of the strong table (every level boundary of the recursion's cases)
    assert [level_strong_recursive(15, s) for s in range(15)] == \
        [4] * 8 + [3] * 4 + [2, 2, 1]
    assert [level_strong_recursive(12, s) for s in range(12)] == [4] * 8 + [3, 3, 2, 1]
    # the strong hierarchy is finer than the weak one near the diagonal
    assert level_strong_recursive(8, 7) == 1 and (8 ^ 7).bit_length() == 4


@pytest.mark.parametrize("C", [16, 64])
def test_strong_chunk_decomposition(C):
    """Every diagonal block holds strong_intra_table, every sub-diagonal block
    strong_subdiag_table, every farther block one level log2(C) + strong(i, j)."""
    NT = 2048 // C
    M = levels_matrix_strong(NT * C, default=0)
    intra, sub = strong_intra_table(C), strong_subdiag_table(C)
    for i in range(NT):
        assert (M[i * C:(i + 1) * C, i * C:(i + 1) * C] == intra).all(), i
        if i >= 1:
            assert (M[i * C:(i + 1) * C, (i - 1) * C:i * C] == sub).all(), i
        for j in range(i - 1):
            blk = M[i * C:(i + 1) * C, j * C:(j + 1) * C]
            assert (blk == strong_far_level(i, j, C)).all(), (i, j)

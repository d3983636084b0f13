"""Pin the level function and the chunk schedule (oracle/levels.py).

The closed form bit_length(t ^ s) is checked against the reference's own
recursion (base.py:41-46, restated with math.log exactly as written) by brute
force, and the chunk-scan schedule (chunkwise.py:34-74) is checked against
the closed form: every (reading chunk i, source chunk j<i) pair is served by
exactly one inter-chunk level, and that level is bit_length(i ^ j) - 1.
"""
import random

import numpy as np

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

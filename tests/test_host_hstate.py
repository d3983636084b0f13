"""Host logic of the decode / prefill path (CPU only, no kernel launches).

* The weak cascade planned on the host copy of the counts
  (hattention.recurrent.HState.plan_cascade_weak) against the oracle's
  FenwickState (restatement of recurrent.py:42-54): counts after every insert
  and the cascade depth implied by the state change.
* The counts set after a prefill (kernel.py:451-462) equal the recurrent counts
  after the same number of tokens, for every T multiple of 64 up to 64 * 300.
* Argument checks raise the reference's exception types, and device tensors
  are required (no CPU fallback).
"""
import pytest
import torch

from oracle import mamba2 as M


def _oracle_counts_seq(n, L):
    S = M.FenwickState(1, 1, 1, 1, L, torch.float64)
    seq = []
    for _ in range(n):
        before = list(S.counts)
        S.insert(torch.ones(1, 1, dtype=torch.float64),
                 torch.zeros(1, 1, 1, 1, dtype=torch.float64))
        seq.append((before, list(S.counts)))
    return seq


def test_cascade_plan_matches_oracle_counts():
    from hattention.base import HType, HStruct
    from hattention.recurrent import HState
    L = 10
    S = HState(2, HType.WEAK, HStruct.MAMBA2, (1, 1, 1, 1, L), torch.float32, "cpu")
    for before, after in _oracle_counts_seq(2 ** (L - 1), L):
        assert S.host_counts == before
        depth = S.plan_cascade_weak()
        assert S.host_counts == after
        # levels below the depth were full and are now empty except level 0
        # (the new token); the depth level received their tokens
        moved = sum(before[:depth])
        assert all(after[e] == 0 for e in range(1, depth))
        if depth > 0:
            assert after[depth] == before[depth] + moved
        assert after[0] == (1 if depth > 0 else before[0] + 1)


def test_cascade_overflow_raises_index_error():
    from hattention.base import HType, HStruct
    from hattention.recurrent import HState
    S = HState(2, HType.WEAK, HStruct.MAMBA2, (1, 1, 1, 1, 3), torch.float32, "cpu")
    for _ in range(4):
        S.plan_cascade_weak()
    with pytest.raises(IndexError):
        S.plan_cascade_weak()


def test_cascade_over_capacity_raises_value_error():
    from hattention.base import HType, HStruct
    from hattention.recurrent import HState
    S = HState(2, HType.WEAK, HStruct.MAMBA2, (1, 1, 1, 1, 4), torch.float32, "cpu")
    S.host_counts = [1, 3, 0, 0]
    with pytest.raises(ValueError):
        S.plan_cascade_weak()


@pytest.mark.parametrize("L", [12, 16])
def test_prefill_counts_equal_recurrent_counts(L):
    from hattention.kernel import _prefill_counts
    S = M.FenwickState(1, 1, 1, 1, L, torch.float64)
    n = 0
    for nt in range(1, 301):
        T = 64 * nt
        if T > 2 ** (L - 1):
            break
        while n < T:
            S.insert(torch.ones(1, 1, dtype=torch.float64),
                     torch.zeros(1, 1, 1, 1, dtype=torch.float64))
            n += 1
        counts, empty = _prefill_counts(T, L, 2)
        assert counts == S.counts, T
        assert empty == [e for e in range(L - 1, 0, -1) if S.counts[e] == 0], T


def test_step_rejects_host_tensors():
    from hattention.base import HType, HStruct
    from hattention.kernel import hattention_step
    from hattention.recurrent import HState
    S = HState(2, HType.WEAK, HStruct.MAMBA2, (1, 2, 64, 16, 8), torch.float32, "cpu")
    q = torch.randn(1, 2, 64)
    with pytest.raises(RuntimeError, match="HIP device"):
        hattention_step(S, q, q, torch.randn(1, 2, 16), None, torch.randn(1, 2),
                        torch.randn(1, 2, 8), None, 2, HType.WEAK, HStruct.MAMBA2)
    assert S.host_counts == [0] * 8


def test_step_argument_checks():
    from hattention.base import HType, HStruct
    from hattention.kernel import hattention_step
    from hattention.recurrent import HState
    S = HState(2, HType.WEAK, HStruct.MAMBA2, (1, 2, 64, 16, 8), torch.float32, "cpu")
    q = torch.randn(1, 2, 64)
    v = torch.randn(1, 2, 16)
    g = torch.randn(1, 2)
    l = torch.randn(1, 2, 8)
    with pytest.raises(TypeError):      # g not in the state dtype (kernel.py:591-606)
        hattention_step(S, q, q, v, None, g.double(), l, None, 2, HType.WEAK, HStruct.MAMBA2)
    with pytest.raises(TypeError):      # q and v dtypes differ
        hattention_step(S, q, q, v.double(), None, g, l, None, 2, HType.WEAK, HStruct.MAMBA2)
    with pytest.raises(NotImplementedError):   # scale without l2norm (:614-615)
        hattention_step(S, q, q, v, None, g, l, 0.5, 2, HType.WEAK, HStruct.MAMBA2)
    with pytest.raises(ValueError):     # MAMBA2 with beta (recurrent.py:141-143)
        hattention_step(S, q, q, v, g, g, l, None, 2, HType.WEAK, HStruct.MAMBA2)
    with pytest.raises(TypeError):      # hstruct differs from the state's
        hattention_step(S, q, q, v, g, g, l, None, 2, HType.WEAK, HStruct.GDELTA)


def test_strong_step_needs_device_tensors():
    """HType.STRONG runs the same step kernels (strong cascade); no CPU path."""
    from hattention.base import HType, HStruct
    from hattention.recurrent import HState, launch_step
    S = HState(2, HType.STRONG, HStruct.MAMBA2, (1, 1, 64, 16, 4), torch.float32, "cpu")
    with pytest.raises(RuntimeError):
        launch_step(S, k=torch.randn(1, 1, 64), v=torch.randn(1, 1, 16), g=torch.randn(1, 1),
                    update=True, output=False)
    S3 = HState(3, HType.WEAK, HStruct.MAMBA2, (1, 1, 64, 16, 4), torch.float32, "cpu")
    with pytest.raises(NotImplementedError):
        launch_step(S3, k=torch.randn(1, 1, 64), v=torch.randn(1, 1, 16), g=torch.randn(1, 1),
                    update=True, output=False)


def test_strong_cascade_plan_matches_oracle():
    """plan_cascade_strong against the oracle's cascade_strong (restatement of
    recurrent.py:56-74): the counts after every insert, and the kernels' state
    move for the planned merge level m (levels 0 .. m-1 up one level, m - 1
    merging into m) applied to per-level values equals the oracle's states."""
    import random
    from hattention.base import HType, HStruct
    from hattention.recurrent import HState
    L = 9
    S = HState(2, HType.STRONG, HStruct.MAMBA2, (1, 1, 1, 1, L), torch.float32, "cpu")
    O = M.FenwickState(1, 1, 1, 1, L, torch.float64, htype=M.STRONG)
    rng = random.Random(0)
    shadow = [0.0] * L
    for n in range(700):
        gate, value = rng.uniform(0.5, 1.0), rng.uniform(-1.0, 1.0)
        m = S.plan_cascade_strong()
        assert 1 <= m <= L
        prev, new = 0.0, []
        for e in range(L):
            cur = shadow[e]
            new.append(0.0 if e == 0 else (prev if e < m else (cur + prev if e == m else cur)))
            prev = cur
        shadow = [x * gate for x in new]
        shadow[0] = value
        O.insert(torch.full((1, 1), gate, dtype=torch.float64),
                 torch.full((1, 1, 1, 1), value, dtype=torch.float64))
        assert S.host_counts == O.counts, n
        ref = O.states[0, 0, 0, 0].tolist()
        assert max(abs(a - b) for a, b in zip(shadow, ref)) < 1e-12, n

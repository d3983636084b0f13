"""Non-fixed lambda (mamba_apis.py:32-67, 88-113): the LambdaLevelMLP and the
rotary embedding it takes from torchtune (absent here, restated in
hattention.mamba_apis).  CPU only: these are torch modules around the path.

The rotary embedding is pinned by what the mathematics fixes, not by a copy of
its formula: position 0 is the identity; each feature pair (2i, 2i + 1) is a
plane rotation (norms kept) by pos * base^(-2i/dim), checked against math.cos /
math.sin in float64 for every pair at several positions; the interleaved-pair
convention (torchtune's, not the half-split one) is pinned by the image of a
basis vector; the relative-position property <R_m q, R_n k> = <R_{m-n} q, k>
holds.  The MLP is pinned by its definition: level i is mlp(rope(x, i)),
level 0 is mlp(x).
"""
import math

import pytest
import torch

from hattention.mamba_apis import (LambdaLevelMLP, RotaryPositionalEmbeddings, compute_lambda,
                                   compute_lambda_maybe_fixed)


def _rot(x, pos, rope):
    return rope(x, input_pos=torch.full((x.shape[1],), pos, dtype=torch.int32))


def test_rope_position_zero_is_identity():
    rope = RotaryPositionalEmbeddings(dim=16, max_seq_len=8)
    x = torch.randn(2, 3, 4, 16)
    assert torch.equal(_rot(x, 0, rope), x)


@pytest.mark.parametrize("pos", [1, 3, 7, 15])
def test_rope_pairs_are_plane_rotations(pos):
    dim, base = 16, 10_000
    rope = RotaryPositionalEmbeddings(dim=dim, max_seq_len=16)
    x = torch.randn(1, 2, 3, dim, dtype=torch.float64)
    y = _rot(x.float(), pos, rope).double()
    for i in range(dim // 2):
        a = pos * base ** (-2 * i / dim)
        c, s = math.cos(a), math.sin(a)
        x0, x1 = x[..., 2 * i], x[..., 2 * i + 1]
        assert torch.allclose(y[..., 2 * i], x0 * c - x1 * s, atol=1e-5, rtol=1e-5)
        assert torch.allclose(y[..., 2 * i + 1], x1 * c + x0 * s, atol=1e-5, rtol=1e-5)
    # a rotation keeps the norm of every pair
    n_in = x.unflatten(-1, (-1, 2)).norm(dim=-1)
    n_out = y.unflatten(-1, (-1, 2)).norm(dim=-1)
    assert torch.allclose(n_in, n_out, atol=1e-5, rtol=1e-5)


def test_rope_interleaved_pairs():
    # e_0 goes to (cos a, sin a, 0, ...): feature 1 pairs with feature 0
    rope = RotaryPositionalEmbeddings(dim=8, max_seq_len=4)
    x = torch.zeros(1, 1, 1, 8)
    x[..., 0] = 1.0
    y = _rot(x, 2, rope)[0, 0, 0]
    assert abs(y[0].item() - math.cos(2.0)) < 1e-6 and abs(y[1].item() - math.sin(2.0)) < 1e-6
    assert y[2:].abs().max().item() == 0.0


def test_rope_relative_positions():
    rope = RotaryPositionalEmbeddings(dim=16, max_seq_len=16)
    q = torch.randn(1, 1, 1, 16)
    k = torch.randn(1, 1, 1, 16)
    lhs = (_rot(q, 9, rope) * _rot(k, 4, rope)).sum()
    rhs = (_rot(q, 5, rope) * k).sum()
    assert abs(lhs.item() - rhs.item()) < 1e-4 * (1 + abs(rhs.item()))


def test_rope_dtype_and_default_positions():
    rope = RotaryPositionalEmbeddings(dim=8, max_seq_len=4)
    x = torch.randn(1, 4, 2, 8).bfloat16()
    y = rope(x)
    assert y.dtype == torch.bfloat16
    # default positions 0 .. s - 1: token j rotated by j
    for j in range(4):
        assert torch.equal(y[:, j:j + 1], _rot(x[:, j:j + 1], j, rope))
    with pytest.raises(IndexError):
        _rot(x, 4, rope)


def test_lambda_level_mlp_levels():
    torch.manual_seed(0)
    m = LambdaLevelMLP(dim=16, max_num_levels=15)
    assert set(m.state_dict()) == {"mlp0.weight", "mlp0.bias", "mlp1.weight", "mlp1.bias"}
    L = torch.randn(1, 1, 4, 16)
    dl = torch.randn(2, 8, 4, 16)
    y0, y1 = m(L, dl, num_levels=13)
    assert y0.shape == (1, 1, 4, 13) and y1.shape == (2, 8, 4, 13)
    assert torch.allclose(y0[..., 0:1], m.mlp0(L)) and torch.allclose(y1[..., 0:1], m.mlp1(dl))
    for i in (1, 5, 12):
        assert torch.equal(y1[..., i:i + 1], m.mlp1(_rot(dl, i, m.rope)))
    with pytest.raises(ValueError):
        m(L[0], dl, num_levels=13)          # 3-D inputs
    with pytest.raises(ValueError):
        m(L, dl, num_levels=16)             # beyond max_num_levels


def test_compute_lambda_non_fixed():
    torch.manual_seed(1)
    m = LambdaLevelMLP(dim=16, max_num_levels=15)
    L = torch.randn(1, 1, 4, 16)
    dl = torch.randn(2, 8, 4, 16)
    for mode in ("positive", "bounded", None):
        got = compute_lambda_maybe_fixed(L, dl, mode, 15, False, m)
        want = compute_lambda(*m(L, dl, num_levels=15), mode)
        assert torch.equal(got, want)
    with pytest.raises(ValueError):
        compute_lambda_maybe_fixed(L[..., :8], dl, "positive", 15, False, m)

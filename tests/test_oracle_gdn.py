"""Pin the log-linear Gated DeltaNet oracle (oracle/gdn.py).

Checks (float64, CPU):
* recurrent (Fenwick state machine with matrix gates, recurrent.py) ==
  materialised pair sum with explicit transition products == chunked UT/WY
  form with per-level delta-rule scans (three structurally different
  algorithms);
* lambda == 1 reduces to the textbook gated delta rule (one state);
* the UT transform: (I + A) Aw = I, W = Aw beta K reproduces the WY product
  prod_u (I - beta_u k_u k_u^T) = I - sum_u k_u w_u^T, and Au = Aw o gamma;
* beta == 0 gives o == 0; lambda one-hot on a level selects that level's pairs;
* final per-level states of the chunked scan equal the recurrent states;
* gradcheck of the chunked form; the scale factor of the GDN API cancels
  against lambda / scale (gated_delta_rule_apis.py:65-70).
"""
import math

import pytest
import torch

from oracle import gdn as D
from oracle.levels import levels_matrix


def make(B, T, H, K, V, L, seed=0, dtype=torch.float64, normalize=True):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, K, generator=gen, dtype=dtype)
    k = torch.randn(B, T, H, K, generator=gen, dtype=dtype)
    if normalize:
        q, k = D.l2norm(q), D.l2norm(k)
    v = torch.randn(B, T, H, V, generator=gen, dtype=dtype)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen, dtype=dtype))
    g = -torch.rand(B, T, H, generator=gen, dtype=dtype) * 0.2
    l = torch.nn.functional.softplus(torch.randn(B, T, H, L, generator=gen, dtype=dtype))
    return q, k, v, beta, g, l


def rel(a, b):
    return ((a - b).abs().max() / b.abs().max()).item()


@pytest.mark.parametrize("T,C", [(8, 2), (16, 4), (32, 4), (24, 8)])
def test_three_forms_agree(T, C):
    L = math.ceil(math.log2(T)) + 2
    q, k, v, beta, g, l = make(2, T, 2, 4, 3, L, seed=T)
    o_rec = D.recurrent_fwd(q, k, v, beta, g, l)
    o_mat = D.materialized_fwd(q, k, v, beta, g, l)
    gc, o_chk, Aw, Au, _ = D.chunked_fwd(q, k, v, beta, g, l, chunk_size=C)
    assert rel(o_mat, o_rec) < 1e-12
    assert rel(o_chk, o_rec) < 1e-12
    NT = T // C
    assert torch.allclose(gc, torch.cumsum(g.reshape(2, NT, C, 2), 2).reshape(2, T, 2))


def test_lambda_one_is_gated_delta_rule():
    q, k, v, beta, g, l = make(1, 32, 2, 5, 3, 7, seed=3)
    l = torch.ones_like(l)
    ref = D.delta_rule_fwd(q, k, v, beta, g)
    assert rel(D.recurrent_fwd(q, k, v, beta, g, l), ref) < 1e-12
    assert rel(D.chunked_fwd(q, k, v, beta, g, l, chunk_size=8)[1], ref) < 1e-12


def test_ut_transform_identities():
    gen = torch.Generator().manual_seed(5)
    C, K = 16, 6
    kc = D.l2norm(torch.randn(C, K, generator=gen, dtype=torch.float64))
    bc = torch.sigmoid(torch.randn(C, generator=gen, dtype=torch.float64))
    Gc = torch.cumsum(-torch.rand(C, generator=gen, dtype=torch.float64) * 0.3, 0)
    A, Aw, Au, W = D.ut_transform(kc, bc, Gc)
    I = torch.eye(C, dtype=torch.float64)
    assert torch.allclose((I + A) @ Aw, I, atol=1e-12)
    # WY: prod_{u=C-1..0} (I - beta_u k_u k_u^T) == I - K^T W
    P = torch.eye(K, dtype=torch.float64)
    for u in range(C):
        P = (torch.eye(K, dtype=torch.float64) - bc[u] * torch.outer(kc[u], kc[u])) @ P
    assert torch.allclose(P, torch.eye(K, dtype=torch.float64) - kc.T @ W, atol=1e-12)
    # Au = (I + A o gamma)^-1 = Aw o gamma
    gamma = D._segsum_exp(Gc)
    Au2 = torch.linalg.inv(I + A * gamma)
    assert torch.allclose(Au, Au2, atol=1e-12)


def test_beta_zero_gives_zero():
    q, k, v, beta, g, l = make(1, 16, 1, 3, 2, 6, seed=7)
    o = D.chunked_fwd(q, k, v, torch.zeros_like(beta), g, l, chunk_size=4)[1]
    assert o.abs().max().item() == 0.0


@pytest.mark.parametrize("level", [0, 2, 4, 5])
def test_one_hot_level(level):
    T = 32
    q, k, v, beta, g, l = make(1, T, 1, 3, 2, 7, seed=level)
    l = torch.zeros_like(l)
    l[..., level] = 1.0
    o = D.chunked_fwd(q, k, v, beta, g, l, chunk_size=4)[1]
    # brute force restricted to pairs of that level
    lev = torch.from_numpy(levels_matrix(T, default=-1))
    I = torch.eye(3, dtype=torch.float64)
    ref = torch.zeros_like(o)
    for s in range(T):
        x = beta[0, s, 0] * k[0, s, 0]
        for t in range(s, T):
            if t > s:
                G = torch.exp(g[0, t, 0]) * (I - beta[0, t, 0] * torch.outer(k[0, t, 0], k[0, t, 0]))
                x = G @ x
            if lev[t, s] == level:
                ref[0, t, 0] += (q[0, t, 0] @ x) * v[0, s, 0]
    assert rel(o, ref) < 1e-12


def test_final_state_matches_recurrent():
    T, C = 32, 4
    q, k, v, beta, g, l = make(1, T, 2, 3, 2, 6, seed=11)
    _, o, _, _, ht = D.chunked_fwd(q, k, v, beta, g, l, chunk_size=C, output_final_state=True)
    o_rec, S = D.recurrent_fwd(q, k, v, beta, g, l, return_state=True)
    assert rel(o, o_rec) < 1e-12
    # with T a power of two every token ends in the top level of each block; the
    # chunk-level states summed over levels >= ell_h0 plus the recurrent levels
    # below it equal the total propagated state
    h0 = 3
    assert rel(ht[..., h0:].sum(-1) + S[..., :h0].sum(-1), S.sum(-1)) < 1e-12


def test_gradcheck_chunked():
    q, k, v, beta, g, l = make(1, 8, 1, 3, 2, 5, seed=13)
    args = [x.clone().requires_grad_(True) for x in (q, k, v, beta, g, l)]
    fn = lambda *a: D.chunked_fwd(*a, chunk_size=2)[1]
    assert torch.autograd.gradcheck(fn, args, eps=1e-6, atol=1e-7)


def test_scale_cancels_in_gdn_api():
    q, k, v, beta, g, l = make(1, 16, 1, 8, 4, 6, seed=17, normalize=False)
    scale = 8 ** -0.5
    o1 = D.hattention_gdn_fwd(q, k, v, beta, g, l / scale, scale=scale, chunk_size=4)
    o2 = D.chunked_fwd(D.l2norm(q), D.l2norm(k), v, beta, g, l, chunk_size=4)[1]
    assert rel(o1, o2) < 1e-12


# --------------------------------------------------------------------------
# HType.STRONG: the reference's chunkwise GDN path with the strong level table
# --------------------------------------------------------------------------
@pytest.mark.parametrize("T,C", [(64, 8), (96, 8), (128, 16), (64, 16)])
def test_strong_chunked_equals_pair_sum(T, C):
    """The strong chunk loop (level loop from 1, every chunk reading every level,
    strong intra-chunk levels) == the pair sum whose weights come from the chunk
    indices and the T x T strong table."""
    NT = T // C
    L = int(math.log2(C)) + 1 + math.ceil(math.log2(NT)) + 1
    q, k, v, beta, g, l = make(2, T, 2, 5, 3, L, seed=T + C)
    o_chk = D.chunked_fwd(q, k, v, beta, g, l, chunk_size=C, htype=D.STRONG)[1]
    o_mat = D.materialized_fwd(q, k, v, beta, g, l, weights=D.strong_chunkwise_weights(l, C))
    assert rel(o_chk, o_mat) < 1e-12


def test_strong_chunk_weights_by_hand():
    """Known weights of the strong chunkwise path, read off the reference's masks
    by hand for four chunks of 4 tokens (h0 = 3, nlev = 2: level 1 only): chunk
    1 sees chunk 0 at level 1, chunks 2 and 3 see chunks 0 and 1 at level 1,
    chunk 3 does not see chunk 2 (bit 1 of 2 is set, level 0 is skipped)."""
    T, C = 16, 4
    l = torch.arange(1, 1 + T * 6, dtype=torch.float64).reshape(1, T, 1, 6)
    w = D.strong_chunkwise_weights(l, C)
    for t in range(T):
        i = t // C
        for s in range(t + 1):
            j = s // C
            if j == i:
                continue
            want = l[0, t, 0, 4].item() if (i, j) in {(1, 0), (2, 0), (2, 1), (3, 0), (3, 1)} else 0.0
            assert w[0, t, 0, s].item() == want, (t, s)


def test_strong_differs_from_weak():
    q, k, v, beta, g, l = make(1, 64, 1, 4, 3, 7, seed=5)
    o_w = D.chunked_fwd(q, k, v, beta, g, l, chunk_size=8)[1]
    o_s = D.chunked_fwd(q, k, v, beta, g, l, chunk_size=8, htype=D.STRONG)[1]
    assert rel(o_s, o_w) > 1e-3


def test_gradcheck_chunked_strong():
    q, k, v, beta, g, l = make(1, 16, 1, 3, 2, 6, seed=19)
    args = [x.clone().requires_grad_(True) for x in (q, k, v, beta, g, l)]
    fn = lambda *a: D.chunked_fwd(*a, chunk_size=2, htype=D.STRONG)[1]
    assert torch.autograd.gradcheck(fn, args, eps=1e-6, atol=1e-7)

"""Pin the log-linear Mamba-2 oracle (oracle/mamba2.py).

Checks (all float64 on CPU):
* materialised H form == Fenwick recurrent form == chunked form == chunked
  level-scan form (four structurally different algorithms);
* brute-force pair loop with the reference's recursive level function and
  the product of exp(g) over (s, t] equals the materialised form;
* lambda == 1 reduces to the textbook SSD recurrence (no hierarchy);
* g == 0 (no decay) and lambda one-hot on a single level select exactly the
  pairs of that level;
* the final per-level states of the level scan equal the recurrent form's
  Fenwick states decayed to the sequence end (levels >= ell_h0);
* torch.autograd.gradcheck (finite differences) on the chunked form, and the
  identity dG_t = q_t.dq_t - k_t.dk_t used by the HIP backward.
"""
import math

import pytest
import torch

from oracle import mamba2 as M
from oracle.levels import levels_matrix


def make_inputs(B, T, H, K, V, L, G=None, seed=0, dtype=torch.float64):
    gen = torch.Generator().manual_seed(seed)
    G = G or H
    q = torch.randn(B, T, G, K, generator=gen, dtype=dtype)
    k = torch.randn(B, T, G, K, generator=gen, dtype=dtype)
    v = torch.randn(B, T, H, V, generator=gen, dtype=dtype)
    A = torch.exp(torch.empty(H, dtype=dtype).uniform_(0.0, math.log(16.0), generator=gen))
    dt = torch.nn.functional.softplus(torch.randn(B, T, H, generator=gen, dtype=dtype) - 3.0)
    g = -A * dt
    l = torch.nn.functional.softplus(torch.randn(B, T, H, L, generator=gen, dtype=dtype))
    return q, k, v, g, l


def rel(a, b):
    return ((a - b).abs().max() / b.abs().max()).item()


@pytest.mark.parametrize("T,C", [(16, 4), (32, 8), (64, 8)])
def test_four_forms_agree(T, C):
    L = int(math.log2(T)) + 1
    q, k, v, g, l = make_inputs(2, T, 3, 5, 4, L)
    o_mat = M.materialized_fwd(q, k, v, g, l)
    o_rec = M.recurrent_fwd(q, k, v, g, l)
    o_chk = M.chunked_fwd(q, k, v, g, l, chunk_size=C)
    o_scn, gc, _ = M.chunked_scan_fwd(q, k, v, g, l, chunk_size=C)
    assert rel(o_rec, o_mat) < 1e-12
    assert rel(o_chk, o_mat) < 1e-12
    assert rel(o_scn, o_mat) < 1e-12
    # chunk-local inclusive cumsum of g (chunkwise.py:1175)
    ref_gc = torch.cumsum(g.reshape(2, T // C, C, 3), dim=2).reshape(2, T, 3)
    assert torch.allclose(gc, ref_gc)


def test_brute_force_matches_materialized():
    T = 24
    q, k, v, g, l = make_inputs(1, T, 2, 3, 3, 6)
    assert rel(M.brute_force_fwd(q, k, v, g, l), M.materialized_fwd(q, k, v, g, l)) < 1e-12


def test_groups():
    T, H, G = 32, 4, 2
    q, k, v, g, l = make_inputs(1, T, H, 4, 3, 6, G=G)
    o = M.chunked_fwd(q, k, v, g, l, chunk_size=8)
    q2 = q.repeat_interleave(H // G, dim=2)
    k2 = k.repeat_interleave(H // G, dim=2)
    assert rel(o, M.materialized_fwd(q2, k2, v, g, l)) < 1e-12


def test_lambda_one_is_plain_ssd():
    T = 64
    q, k, v, g, l = make_inputs(2, T, 2, 4, 3, 7)
    l = torch.ones_like(l)
    ref = M.ssd_scan_fwd(q, k, v, g)
    assert rel(M.chunked_fwd(q, k, v, g, l, chunk_size=8), ref) < 1e-12
    assert rel(M.recurrent_fwd(q, k, v, g, l), ref) < 1e-12


@pytest.mark.parametrize("level", [0, 1, 3, 5, 6])
def test_one_hot_level_selects_pairs(level):
    T = 64
    q, k, v, _, l = make_inputs(1, T, 1, 3, 2, 7, seed=level)
    g = torch.zeros(1, T, 1, dtype=torch.float64)          # no decay
    l = torch.zeros_like(l)
    l[..., level] = 1.0
    o = M.chunked_fwd(q, k, v, g, l, chunk_size=8)
    lev = torch.from_numpy(levels_matrix(T, default=-1))
    mask = (lev == level).to(torch.float64)
    ref = torch.einsum("ts,ts,sv->tv", torch.einsum("tk,sk->ts", q[0, :, 0], k[0, :, 0]),
                       mask, v[0, :, 0])
    assert rel(o[0, :, 0], ref) < 1e-12


def test_final_state_matches_recurrent():
    T, C = 64, 8
    L = 7
    q, k, v, g, l = make_inputs(1, T, 2, 3, 4, L)
    o, _, ht = M.chunked_scan_fwd(q, k, v, g, l, chunk_size=C, output_final_state=True)
    o_rec, S = M.recurrent_fwd(q, k, v, g, l, return_state=True)
    # The level scan holds, per inter-chunk level, the decayed sum of the
    # chunks in that level's open block; with T a power of two the recurrent
    # state after T tokens has every token merged into its top levels.  Their
    # sum over levels >= ell_h0 plus the recurrent state's levels < ell_h0 is
    # the full decayed sum of k v^T over all tokens.
    ell_h0 = 4
    total_scan = ht[..., ell_h0:].sum(-1) + S.states[..., :ell_h0].sum(-1)
    Gt = torch.cumsum(g, 1)
    full = torch.einsum("bthk,bthv,bth->bhkv", k, v, torch.exp(Gt[:, -1:] - Gt))
    assert rel(total_scan, full) < 1e-12
    assert rel(o, o_rec) < 1e-12


def test_gradcheck_chunked():
    T = 16
    q, k, v, g, l = make_inputs(1, T, 1, 3, 2, 5)
    for x in (q, k, v, g, l):
        x.requires_grad_(True)
    fn = lambda *a: M.chunked_fwd(*a, chunk_size=4)
    assert torch.autograd.gradcheck(fn, (q, k, v, g, l), eps=1e-6, atol=1e-7)


def test_backward_forms_agree_and_dg_identity():
    T, C = 32, 8
    q, k, v, g, l = make_inputs(2, T, 2, 4, 3, 6)
    do = torch.randn(2, T, 2, 3, dtype=torch.float64)
    gm = M.autograd_bwd(M.materialized_fwd, q, k, v, g, l, do)
    gc = M.autograd_bwd(M.chunked_fwd, q, k, v, g, l, do, chunk_size=C)
    gs = M.autograd_bwd(lambda *a: M.chunked_scan_fwd(*a, chunk_size=C)[0], q, k, v, g, l, do)
    for a, b, c in zip(gm, gc, gs):
        assert rel(b, a) < 1e-11 and rel(c, a) < 1e-11
    dq, dk, dv, dg, dl = gm
    dG = (q * dq).sum(-1) - (k * dk).sum(-1)                 # [B, T, H]
    dg_from_identity = torch.flip(torch.cumsum(torch.flip(dG, [1]), 1), [1])
    assert rel(dg_from_identity, dg) < 1e-10
    # and the lambda form of the row sums: sum_l lambda dlambda = q . dq
    assert rel((l * dl).sum(-1), (q * dq).sum(-1)) < 1e-10


def test_layer_fwd_scan_forms_agree_and_lambda_special_values():
    """layer_fwd (mamba_apis.py:346-403) with the chunked level scan equals it
    with the materialised form; lambda modes hit their closed-form values."""
    torch.manual_seed(21)
    B, T, H, G, P, N, Lv = 1, 128, 2, 1, 3, 4, 8
    x = torch.randn(B, T, H, P, dtype=torch.float64)
    dt = torch.randn(B, T, H, dtype=torch.float64) - 2
    A = -torch.rand(H, dtype=torch.float64) - 0.5
    Bm = torch.randn(B, T, G, N, dtype=torch.float64)
    Cm = torch.randn(B, T, G, N, dtype=torch.float64)
    dl = torch.randn(B, T, H, Lv, dtype=torch.float64)
    L = torch.randn(H, Lv, dtype=torch.float64)
    D = torch.randn(H, dtype=torch.float64)
    bias = torch.randn(H, dtype=torch.float64) * 0.1
    for mode in ("positive", "bounded", None):
        y1 = M.layer_fwd(x, dt, A, Bm, Cm, dl, L, D, bias, mode)
        y2 = M.layer_fwd(x, dt, A, Bm, Cm, dl, L, D, bias, mode,
                         scan=lambda q, k, v, g, l: M.materialized_fwd(q, k, v, g, l))
        assert rel(y1, y2) < 1e-12, mode
    zeros = torch.zeros(1, 1, 1, 1, dtype=torch.float64)
    one = torch.ones(1, 1, dtype=torch.float64)
    assert abs(M.layer_lambda(one, zeros, "positive").item() - math.log(2.0)) < 1e-15
    assert abs(M.layer_lambda(-1e3 * one, zeros + 1, "bounded").item() - 1.0) < 1e-15
    assert M.layer_lambda(2 * one, zeros + 3, None).item() == 6.0


def test_layer_fwd_gradcheck():
    torch.manual_seed(22)
    B, T, H, G, P, N, Lv = 1, 8, 2, 1, 2, 3, 4
    args = [torch.randn(B, T, H, P), torch.randn(B, T, H) - 1, -torch.rand(H) - 0.5,
            torch.randn(B, T, G, N), torch.randn(B, T, G, N), torch.randn(B, T, H, Lv),
            torch.randn(H, Lv), torch.randn(H), torch.randn(H) * 0.1]
    args = [a.double().requires_grad_(True) for a in args]
    for mode in ("positive", "bounded", None):
        fn = lambda *a: M.layer_fwd(*a, lambda_mode=mode,
                                    scan=lambda q, k, v, g, l: M.materialized_fwd(q, k, v, g, l))
        assert torch.autograd.gradcheck(fn, args, eps=1e-6, atol=1e-7), mode


def test_causal_conv1d_and_gated_rmsnorm_closed_forms():
    """The conv restatement against a direct loop over taps; the gated RMSNorm
    against its definition on a hand-picked row; the split layer's forms agree."""
    torch.manual_seed(23)
    Bsz, Dch, S, W = 2, 5, 9, 4
    x = torch.randn(Bsz, Dch, S, dtype=torch.float64)
    w = torch.randn(Dch, W, dtype=torch.float64)
    b = torch.randn(Dch, dtype=torch.float64)
    ref = torch.zeros_like(x)
    for s in range(S):
        acc = b[None, :].clone().expand(Bsz, Dch).clone()
        for k in range(W):
            sp = s - (W - 1) + k
            if sp >= 0:
                acc = acc + w[None, :, k] * x[:, :, sp]
        ref[:, :, s] = acc * torch.sigmoid(acc)
    assert rel(M.causal_conv1d_silu(x, w, b), ref) < 1e-14
    # gated rmsnorm: u = [3, 4] * silu(z) with z large -> silu(z) ~ z ... use z = 0 -> u = 0
    xx = torch.tensor([[3.0, 4.0]], dtype=torch.float64)
    zz = torch.full((1, 2), 50.0, dtype=torch.float64)     # silu(50) = 50 (to 1e-20)
    u = xx * 50.0
    expect = u / math.sqrt((u * u).mean().item() + 1e-6) * torch.tensor([2.0, -1.0], dtype=torch.float64)
    assert rel(M.gated_rmsnorm(xx, torch.tensor([2.0, -1.0], dtype=torch.float64), zz, 1e-6), expect) < 1e-14
    # the split layer with the chunked and the materialised scans
    H, P, G, N, Lv, S2 = 2, 4, 1, 3, 8, 128
    dim = H * P
    width = 2 * dim + 2 * G * N + H + H * Lv
    zx = torch.randn(1, S2, width, dtype=torch.float64)
    args = dict(conv_w=torch.randn(dim + 2 * G * N, 4, dtype=torch.float64) * 0.5,
                conv_b=torch.randn(dim + 2 * G * N, dtype=torch.float64) * 0.1,
                dt_bias=torch.randn(H, dtype=torch.float64) * 0.1 - 2,
                A=-torch.rand(H, dtype=torch.float64) - 0.5, L=torch.randn(H, Lv, dtype=torch.float64),
                D=torch.randn(H, dtype=torch.float64), rms_w=torch.randn(dim, dtype=torch.float64),
                eps=1e-6, out_w=torch.randn(6, dim, dtype=torch.float64),
                out_b=torch.randn(6, dtype=torch.float64), headdim=P, ngroups=G)
    y1 = M.split_conv1d_layer_fwd(zx, **args)
    y2 = M.split_conv1d_layer_fwd(zx, **args,
                                  scan=lambda q, k, v, g, l: M.materialized_fwd(q, k, v, g, l))
    assert rel(y1, y2) < 1e-12


# ---- strong hierarchy (HType.STRONG) --------------------------------------
@pytest.mark.parametrize("T,C", [(16, 4), (64, 8), (96, 16), (256, 64)])
def test_strong_forms_agree(T, C):
    """materialised strong table (base.py:49-62) == recurrent cascade_strong
    (recurrent.py:56-74) == the chunked decomposition of chunked_strong_fwd."""
    L = int(math.log2(T)) + 2
    q, k, v, g, l = make_inputs(2, T, 2, 5, 4, L, seed=T + C)
    o_mat = M.materialized_fwd(q, k, v, g, l, htype=M.STRONG)
    o_rec = M.recurrent_fwd(q, k, v, g, l, htype=M.STRONG)
    o_chk = M.chunked_strong_fwd(q, k, v, g, l, chunk_size=C)
    assert rel(o_rec, o_mat) < 1e-12
    assert rel(o_chk, o_mat) < 1e-12
    # and it is a different hierarchy from the weak one
    assert rel(M.materialized_fwd(q, k, v, g, l), o_mat) > 1e-3


@pytest.mark.parametrize("level", [0, 1, 2, 4, 6, 7])
def test_strong_one_hot_level_selects_pairs(level):
    """g == 0, lambda one-hot: exactly the pairs whose strong level (the
    reference's recursion, pair by pair) is `level`."""
    from oracle.levels import level_strong_recursive
    T = 192
    q, k, v, _, l = make_inputs(1, T, 1, 3, 2, 9, seed=level)
    g = torch.zeros(1, T, 1, dtype=torch.float64)
    l = torch.zeros_like(l)
    l[..., level] = 1.0
    o = M.chunked_strong_fwd(q, k, v, g, l, chunk_size=16)
    mask = torch.zeros(T, T, dtype=torch.float64)
    for t in range(T):
        for s in range(t + 1):
            mask[t, s] = float((0 if s == t else level_strong_recursive(t, s)) == level)
    ref = torch.einsum("ts,ts,sv->tv", torch.einsum("tk,sk->ts", q[0, :, 0], k[0, :, 0]),
                       mask, v[0, :, 0])
    assert rel(o[0, :, 0], ref) < 1e-12


def test_strong_lambda_one_is_plain_ssd():
    T = 128
    q, k, v, g, l = make_inputs(1, T, 2, 4, 3, 9, seed=3)
    o = M.chunked_strong_fwd(q, k, v, g, torch.ones_like(l), chunk_size=16)
    assert rel(o, M.ssd_scan_fwd(q, k, v, g)) < 1e-12


@pytest.mark.parametrize("T,C,G", [(64, 16, 2), (256, 16, 1), (320, 64, 2), (1024, 64, 1)])
def test_strong_backward_decomposition_matches_autograd(T, C, G):
    """chunked_strong_bwd (chunk walks forward and, through the transposed
    cascade, in reverse; dense diagonal / sub-diagonal tiles; dG identity)
    against torch.autograd through the materialised strong table of
    base.py:49-62 (a structurally different form), grouped q / k included."""
    L = int(math.log2(T)) + 3
    q, k, v, g, l = make_inputs(1, T, 2, 5, 4, L, G=G, seed=T + C)
    do = torch.randn(1, T, 2, 4, generator=torch.Generator().manual_seed(7), dtype=torch.float64)
    got = M.chunked_strong_bwd(q, k, v, g, l, do, chunk_size=C)
    ref = M.autograd_bwd(lambda *a: M.materialized_fwd(*a, htype=M.STRONG), q, k, v, g, l, do)
    for name, a, r in zip(("dq", "dk", "dv", "dg", "dl"), got, ref):
        assert a.shape == r.shape, name
        assert rel(a, r) < 1e-11, (name, rel(a, r))


@pytest.mark.parametrize("NT", [2, 3, 4, 5, 7, 8, 9, 12, 16, 17, 31, 32, 33])
def test_strong_final_state_closed_form(NT):
    """strong_final_state (the reference's USE_H2 state loop with its phases and
    resets) against the closed form the HIP kernel computes: level 7 + ell,
    ell >= 1, holds the chunks base .. base + 2^(ell-1) - 1 (base: the start of
    the aligned 2^(ell+1)-chunk block that holds the last chunk), each chunk's
    decayed k^T v further decayed to the end of the sequence; every other level
    zero.  A wrong phase test, reset position or final-chunk rule changes which
    chunks a level holds."""
    C = 4
    B, H, K, V = 1, 2, 3, 2
    T = C * NT
    nlev = math.ceil(math.log2(NT))
    L = 3 + nlev
    gen = torch.Generator().manual_seed(1234 + NT)
    q = torch.randn(B, T, H, K, generator=gen, dtype=torch.float64)
    k = torch.randn(B, T, H, K, generator=gen, dtype=torch.float64)
    v = torch.randn(B, T, H, V, generator=gen, dtype=torch.float64)
    g = -0.2 * torch.rand(B, T, H, generator=gen, dtype=torch.float64)
    l = torch.rand(B, T, H, L, generator=gen, dtype=torch.float64)
    ht = M.strong_final_state(q, k, v, g, l, chunk_size=C)
    ell_h0 = 3   # get_num_levels(4, 2)
    G = torch.cumsum(g, dim=1)                                  # [B, T, H]
    ref = torch.zeros_like(ht)
    for ell in range(1, nlev):
        P, S = 2 << ell, 1 << (ell - 1)
        base = (NT - 1) // P * P
        for c in range(base, min(base + S, NT)):
            for t in range(C * c, C * c + C):
                w = torch.exp(G[:, T - 1] - G[:, t])               # decay of token t to the end
                ref[..., ell_h0 + ell] += torch.einsum("bh,bhk,bhv->bhkv", w, k[:, t], v[:, t])
    assert torch.allclose(ht, ref, rtol=1e-12, atol=1e-12)
    assert ht[..., ell_h0].abs().max() == 0          # ell = 0: not part of the strong loop
    for ell in range(1, nlev):
        assert ht[..., ell_h0 + ell].abs().max() > 0

"""Log-linear Gated DeltaNet (HStruct.GDELTA, HType.WEAK, base 2): CPU oracle.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Time-first tensors, one head per q / k (the reference expands groups before its
kernels, chunkwise_hgdn.py:614-623):

    q, k : [B, T, H, K]     v : [B, T, H, V]
    beta : [B, T, H]        g : [B, T, H] per-step log-decay
    l    : [B, T, H, L]     level weights lambda

The recurrence (recurrent.py:76-94, 134-166 with HStruct.GDELTA): every
Fenwick level S_l [K, V] is advanced by the same transition
G_t = exp(g_t) (I - beta_t k_t k_t^T) from the left, the new token's
beta_t k_t v_t^T becomes level 0 (after the weak cascade), and
o_t = q_t^T sum_l lambda[t, l] S_l.  Equivalently

    o_t = sum_{s <= t} lambda[t, lev(t, s)] q_t^T (G_t ... G_{s+1}) beta_s k_s v_s^T.

Restatements (reference file:line):
* ``recurrent_fwd``     -- HState (GDELTA) + step_state / step_output,
  hattention/recurrent.py:9-216.
* ``materialized_fwd``  -- the pair sum above with explicit K x K transition
  products (the quantity base.py:258-331 materialises as a DPLR tensor); tiny T.
* ``ut_transform``      -- chunk_scaled_dot_kkt + solve_tril + recompute_w_u
  (fla_future/chunk_scaled_dot_kkt.py:14-126, solve_tril.py:14-276,
  wy_fast.py:147-237): A = strict-tril(diag(beta) K K^T), Aw = (I + A)^-1,
  Au = (I + A o gamma)^-1 = Aw o gamma, W = Aw (beta K), U = Au (beta V).
* ``chunked_fwd``       -- chunkwise_hgdn.chunkwise_fwd (chunkwise_hgdn.py:566-788)
  and hgdn_minimal (hssd_minimal.py:287-493): intra-chunk
  ((tril(Q K^T) Aw) o gamma o beta_s o lambda[t, lev]) V, then per inter-chunk
  level a delta-rule scan over chunks (chunk_delta_h.py:16-186 with the
  skip_kv / skip_g masks) read through q_new = exp(G) (q - tril(Q K^T) W).
  Returns (g_cumsum, o, Aw, Au, ht) like the reference.
* ``delta_rule_fwd``    -- the plain gated delta rule (one state, no levels):
  what log-linear GDN reduces to when lambda == 1.

Pinning (tests/test_oracle_gdn.py): recurrent == materialised == chunked (three
structurally different algorithms); lambda == 1 equals the textbook gated delta
rule; (I + A) Aw = I; beta = 0 gives o = 0; lambda one-hot on a level selects
exactly that level's pairs; gradcheck of the chunked form.

HType.STRONG: what the reference's chunkwise GDN path computes with the strong
level table (chunkwise_hgdn.py:630, 724-728, 782), which is not the recurrent
strong cascade (recurrent.py:56-74): the intra-chunk tile takes lambda at the
strong level of the pair (make_levels_matrix with htype STRONG), the
inter-chunk level loop starts at 1, every level keeps the weak delta-rule
state (the same skip_kv / skip_g masks as HType.WEAK, chunk_delta_h.py:16-186),
and every chunk reads every level >= 1 (chunk_fwd_kernel_o with USE_H2, which
lifts the skip_q exit, chunkwise.py:521-527).  A level-e state read at chunk i
holds the chunks j in [i & ~(2^(e+1) - 1), i) whose bit e is clear, so a pair
of chunks can be counted at several levels and a chunk's immediate predecessor
can be counted at none (with four chunks, chunk 2 for chunk 3: bit 1 of 2
is set and level 0 is skipped).
* ``chunked_fwd(..., htype=STRONG)`` restates that chunk loop;
* ``strong_chunkwise_weights`` / ``materialized_fwd(..., weights=...)`` give the
  same function as a pair sum whose weight is built from the chunk indices
  directly (and the intra-chunk levels from the T x T strong table of
  oracle.levels, so the chunk translation invariance of the table is checked
  too).  The two agree to 1e-12 in float64; autograd through the chunked form
  is pinned by gradcheck.
"""
import math
from typing import Optional

import torch

from oracle.levels import (get_num_levels, levels_matrix, levels_matrix_strong,
                           strong_intra_table)

WEAK, STRONG = 0, 1   # HType values (hattention/base.py:12-14)


def _check(q, k, v, beta, g, l):
    B, T, H, K = q.shape
    if k.shape != q.shape or v.shape[:3] != (B, T, H) or beta.shape != (B, T, H) \
            or g.shape != (B, T, H) or l.shape[:3] != (B, T, H):
        raise ValueError("shape mismatch")
    return B, T, H, K, v.shape[3], l.shape[3]


# --------------------------------------------------------------------------
# 1. recurrent form (recurrent.py)
# --------------------------------------------------------------------------
def recurrent_fwd(q, k, v, beta, g, l, return_state: bool = False):
    """hattention_recurrent with HStruct.GDELTA (recurrent.py:169-216)."""
    B, T, H, K, V, L = _check(q, k, v, beta, g, l)
    S = torch.zeros(B, H, K, V, L, dtype=q.dtype)
    counts = [0] * L
    I = torch.eye(K, dtype=q.dtype)
    ys = []
    for t in range(T):
        # cascade_weak (recurrent.py:42-54)
        for level in range(L):
            cap = 2 ** level
            if counts[level] == cap:
                S[..., level + 1] = S[..., level + 1] + S[..., level]
                counts[level + 1] += counts[level]
                S[..., level] = 0.0
                counts[level] = 0
            elif counts[level] < cap:
                break
        kt, vt, bt = k[:, t], v[:, t], beta[:, t]
        gate = torch.exp(g[:, t])[..., None, None] * (
            I - bt[..., None, None] * torch.einsum("bhm,bhn->bhmn", kt, kt))   # step_state :146-154
        S = torch.einsum("bhmn,bhnvl->bhmvl", gate, S)                          # insert :90-91
        S[..., 0] = bt[..., None, None] * torch.einsum("bhk,bhv->bhkv", kt, vt)
        counts[0] += 1
        Sl = torch.einsum("bhkvl,bhl->bhkv", S, l[:, t])                      # step_output :159-166
        ys.append(torch.einsum("bhk,bhkv->bhv", q[:, t], Sl))
    o = torch.stack(ys, dim=1)
    return (o, S) if return_state else o


# --------------------------------------------------------------------------
# 2. materialised pair sum (tiny T)
# --------------------------------------------------------------------------
def materialized_fwd(q, k, v, beta, g, l, weights=None):
    """o_t = sum_{s<=t} lambda[t, lev(t,s)] q_t^T (G_t ... G_{s+1}) beta_s k_s v_s^T.

    ``weights`` [B, T, H, T] replaces lambda[t, lev(t, s)] by an explicit pair
    weight w[b, t, h, s] (used for the strong chunkwise form)."""
    B, T, H, K, V, L = _check(q, k, v, beta, g, l)
    lev = torch.from_numpy(levels_matrix(T, default=0, clamp_min=0))
    I = torch.eye(K, dtype=q.dtype)
    G = torch.exp(g)[..., None, None] * (
        I - beta[..., None, None] * torch.einsum("bthm,bthn->bthmn", k, k))   # [B,T,H,K,K]
    o = torch.zeros(B, T, H, V, dtype=q.dtype)
    for s in range(T):
        x = beta[:, s, :, None] * k[:, s]                                     # [B,H,K]
        for t in range(s, T):
            if t > s:
                x = torch.einsum("bhmn,bhn->bhm", G[:, t], x)
            lw = l[:, t, :, lev[t, s]] if weights is None else weights[:, t, :, s]
            w = lw * (q[:, t] * x).sum(-1)                                    # [B,H]
            o[:, t] = o[:, t] + w[..., None] * v[:, s]
    return o


def strong_chunkwise_weights(l, chunk_size: int = 64):
    """Pair weights [B, T, H, T] of the reference's chunkwise GDN path with
    HType.STRONG (chunkwise_hgdn.py:630, 724-783), from the chunk indices:

    * s in t's chunk: lambda[t, strong(t, s)], the strong level from the T x T
      table (make_levels_matrix with htype STRONG, diagonal blocks only);
    * s in an earlier chunk j of t's chunk i: the sum of lambda[t, h0 + e] over
      the levels e in 1 .. nlev - 1 whose state at chunk i holds chunk j, i.e.
      j >= i & ~(2^(e+1) - 1) and bit e of j clear (weak state, read at every
      chunk); h0 = log2(chunk) + 1."""
    B, T, H, L = l.shape
    C = chunk_size
    NT = T // C
    h0 = get_num_levels(C, 2)
    nlev = math.ceil(math.log2(NT)) if NT > 1 else 0
    lev = torch.from_numpy(levels_matrix_strong(T, default=0, clamp_min=0))
    w = torch.zeros(B, T, H, T, dtype=l.dtype)
    for t in range(T):
        i = t // C
        for s in range(t + 1):
            j = s // C
            if j == i:
                w[:, t, :, s] = l[:, t, :, lev[t, s]]
                continue
            for e in range(1, nlev):
                if j >= (i & ~((2 << e) - 1)) and not (j >> e) & 1:
                    w[:, t, :, s] = w[:, t, :, s] + l[:, t, :, h0 + e]
    return w


# --------------------------------------------------------------------------
# 3. plain gated delta rule (lambda == 1)
# --------------------------------------------------------------------------
def delta_rule_fwd(q, k, v, beta, g):
    """S_t = exp(g_t)(I - beta_t k_t k_t^T) S_{t-1} + beta_t k_t v_t^T, o_t = q_t^T S_t."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    S = torch.zeros(B, H, K, V, dtype=q.dtype)
    I = torch.eye(K, dtype=q.dtype)
    ys = []
    for t in range(T):
        kt, bt = k[:, t], beta[:, t]
        G = torch.exp(g[:, t])[..., None, None] * (
            I - bt[..., None, None] * torch.einsum("bhm,bhn->bhmn", kt, kt))
        S = torch.einsum("bhmn,bhnv->bhmv", G, S) + \
            bt[..., None, None] * torch.einsum("bhk,bhv->bhkv", kt, v[:, t])
        ys.append(torch.einsum("bhk,bhkv->bhv", q[:, t], S))
    return torch.stack(ys, dim=1)


# --------------------------------------------------------------------------
# 4. chunked form
# --------------------------------------------------------------------------
def _segsum_exp(Gc):
    """gamma[.., t, s] = exp(Gc_t - Gc_s) for s <= t, 0 above (exp(segsum(g)),
    hssd_minimal.py:94-105), Gc the chunk-local inclusive cumsum on dim -1."""
    C = Gc.shape[-1]
    d = Gc[..., :, None] - Gc[..., None, :]
    mask = torch.tril(torch.ones(C, C, dtype=torch.bool))
    return torch.exp(d.masked_fill(~mask, float("-inf")))


def ut_transform(kc, bc, Gc):
    """One chunk per leading index: kc [.., C, K], bc [.., C], Gc [.., C].

    Returns A (strictly lower, fp), Aw = (I + A)^-1, Au = Aw o gamma,
    W = Aw (beta K), U-operator Au diag(beta) (apply to V).
    """
    C = kc.shape[-2]
    A = bc[..., :, None] * (kc @ kc.transpose(-1, -2))
    A = torch.tril(A, diagonal=-1)
    I = torch.eye(C, dtype=kc.dtype)
    Aw = torch.linalg.solve_triangular(I + A, I.expand_as(A).clone(), upper=False,
                                       unitriangular=True)
    gamma = _segsum_exp(Gc)
    Au = Aw * gamma
    W = Aw @ (bc[..., None] * kc)
    return A, Aw, Au, W


def chunked_fwd(q, k, v, beta, g, l, chunk_size: int = 64, output_final_state: bool = False,
                htype: int = WEAK):
    """chunkwise_hgdn.chunkwise_fwd (chunkwise_hgdn.py:566-788): (g_cumsum, o, Aw, Au, ht).

    htype STRONG: the strong intra-chunk levels, the level loop from 1 and every
    chunk reading every level (chunkwise_hgdn.py:630, 724-728, 782; see the
    module docstring); the states are the weak ones."""
    B, T, H, K, V, L = _check(q, k, v, beta, g, l)
    C = chunk_size
    if T % C:
        raise ValueError
    NT = T // C
    h0 = get_num_levels(C, 2)
    nlev = math.ceil(math.log2(NT)) if NT > 1 else 0
    if h0 + nlev > L:
        raise ValueError("too few levels")
    # [B, H, NT, C, ...]
    r = lambda x: x.reshape(B, NT, C, H, *x.shape[3:]).movedim(3, 1)
    qc, kc, vc, bc, lc = r(q), r(k), r(v), r(beta), r(l)
    Gc = torch.cumsum(r(g), dim=-1)                                  # chunk-local cumsum
    A, Aw, Au, W = ut_transform(kc, bc, Gc)
    U = Au @ (bc[..., None] * vc)
    gamma = _segsum_exp(Gc)
    # intra-chunk (chunk_fwd_kernel_o_intra, chunkwise_hgdn.py:41-126)
    if htype == STRONG:
        lev = torch.from_numpy(strong_intra_table(C))
    else:
        lev = torch.from_numpy(levels_matrix(C, default=0, clamp_min=0))
    tt = torch.arange(C)[:, None].expand(C, C)
    lam = lc[..., tt, lev]                                           # [B,H,NT,t,s]
    Cm = torch.tril(qc @ kc.transpose(-1, -2)) @ Aw                  # tril(QK^T) Aw
    o = (Cm * gamma * bc[..., None, :] * lam) @ vc
    # gated operands (preprocess_qkw, chunk_delta_h.py:384-462; q_new :690-700)
    eG = torch.exp(Gc)
    Knew = kc * torch.exp(Gc[..., -1:] - Gc)[..., None]
    Wnew = W * eG[..., None]
    Qnew = eG[..., None] * (qc - torch.tril(qc @ kc.transpose(-1, -2)) @ W)
    glast = torch.exp(Gc[..., -1])                                   # [B,H,NT]
    ht = torch.zeros(B, H, K, V, L, dtype=q.dtype) if output_final_state else None
    # STRONG starts at level 1 (chunkwise_hgdn.py:724-728)
    for ell in range(1 if htype == STRONG else 0, nlev):
        S = torch.zeros(B, H, K, V, dtype=q.dtype)
        period = 1 << (ell + 1)
        for i in range(NT):
            # reading chunk; STRONG reads every chunk (USE_H2, chunkwise.py:521-527)
            if htype == STRONG or (i >> ell) & 1:
                o[:, :, i] = o[:, :, i] + lc[:, :, i, :, h0 + ell, None] * (Qnew[:, :, i] @ S)
            reset = (i % period == period - 1)
            if output_final_state and i == NT - 1:
                reset = False
            if reset:
                S = torch.zeros_like(S)
            else:                                                    # S <- G_chunk S
                S = glast[:, :, i, None, None] * S - \
                    Knew[:, :, i].transpose(-1, -2) @ (Wnew[:, :, i] @ S)
            if not (i >> ell) & 1:                                   # writing chunk
                S = S + Knew[:, :, i].transpose(-1, -2) @ U[:, :, i]
        if output_final_state:
            ht[..., h0 + ell] = S
    g_cumsum = Gc.movedim(1, 3).reshape(B, T, H)
    o = o.movedim(1, 3).reshape(B, T, H, V)
    Aw_out = Aw.movedim(1, 3).reshape(B, T, H, C)
    Au_out = Au.movedim(1, 3).reshape(B, T, H, C)
    return g_cumsum, o, Aw_out, Au_out, ht


# --------------------------------------------------------------------------
# 5. the HAttention GDELTA boundary
# --------------------------------------------------------------------------
def l2norm(x, eps: float = 1e-6):
    """x / sqrt(sum x^2 + eps) over the last dim (fla.modules.l2norm)."""
    return x * torch.rsqrt((x * x).sum(-1, keepdim=True) + eps)


def l2norm_scale_bwd(x, dy, scale: float = 1.0, eps: float = 1e-6):
    """Closed-form gradient of y = l2norm(x) * scale (fla l2norm_bwd as used at
    kernel.py:24-29, 224-225): with r = (sum x^2 + eps)^-1/2 and u = x r,
    dx = r scale (dy - u (u . dy)).  The GDN backward kernel applies this form
    to dq (scale = the attention scale) and dk (scale = 1)."""
    r = torch.rsqrt((x * x).sum(-1, keepdim=True) + eps)
    u = x * r
    return r * scale * (dy - u * (u * dy).sum(-1, keepdim=True))


def hattention_gdn_fwd(q, k, v, beta, g, l, scale: Optional[float] = None, chunk_size: int = 64):
    """HAttentionFunction.forward, GDELTA branch (kernel.py:100-123): q <- l2norm(q) * scale,
    k <- l2norm(k), then chunkwise_hgdn.chunkwise_fwd; returns o."""
    if scale is None:
        scale = q.shape[-1] ** -0.5
    return chunked_fwd(l2norm(q) * scale, l2norm(k), v, beta, g, l, chunk_size)[1]


def autograd_bwd(fwd, q, k, v, beta, g, l, do, **kw):
    """(dq, dk, dv, dbeta, dg, dl) of sum(o * do) through any forward form above."""
    leaves = [x.detach().clone().requires_grad_(True) for x in (q, k, v, beta, g, l)]
    o = fwd(*leaves, **kw)
    if isinstance(o, tuple):
        o = o[1]
    return tuple(torch.autograd.grad((o * do).sum(), leaves))

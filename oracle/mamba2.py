"""Log-linear Mamba-2 (HStruct.MAMBA2, HType.WEAK and STRONG, level base 2): CPU oracle.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

All functions take time-first tensors (``head_first=False``, the only layout
the reference APIs use):

    q, k : [B, T, G, K]   (G divides H; group of head h is h // (H // G))
    v    : [B, T, H, V]
    g    : [B, T, H]      per-step log-decay (fp32 in the reference)
    l    : [B, T, H, L]   level weights lambda (linear, not log)

and return ``o : [B, T, H, V]`` computed in the dtype of the inputs (pass
float64 for the parity checks).  The math they all implement is

    o_t = sum_{s <= t} l[t, level(t, s)] * exp(G_t - G_s) * (q_t . k_s) * v_s

with ``G`` the inclusive cumulative sum of ``g`` and ``level`` the weak Fenwick
level (``oracle.levels``).

Restatements (reference file:line):
* ``materialized_fwd``  -- make_masked_H_matrix + hattention_materialized,
  hattention/base.py:75-98, 334-349 (O(T^2), explicit H matrix).
* ``recurrent_fwd``     -- HState.cascade_weak / insert / dot, step_state,
  step_output, hattention_recurrent, hattention/recurrent.py:9-216
  (Fenwick-tree state machine, one token at a time).
* ``chunked_fwd``       -- hssd_minimal_discrete, hattention/hssd_minimal.py:108-220
  (intra-chunk blocks + masked chunk-level decay matrix per level).
* ``chunked_scan_fwd``  -- the host loop of chunkwise_fwd with its kernels,
  hattention/chunkwise.py:1118-1275 (chunk_fwd_kernel_h :94-280 and
  chunk_fwd_kernel_o :473-647): intra-chunk tile, then per inter-chunk level a
  sequential scan over chunks with the skip_kv / skip_g / skip_q schedule.
  Also returns the chunk-local cumsum of g (chunkwise.py:1175) and the final
  per-level states ``ht`` [B, H, K, V, L] (chunkwise.py:1179, 229-279).
* ``ssd_scan_fwd``      -- plain (non-hierarchical) gated linear attention /
  Mamba-2 SSD recurrence h_t = exp(g_t) h_{t-1} + k_t v_t^T, o_t = q_t h_t:
  the textbook form that log-linear Mamba-2 reduces to when lambda == 1
  (the intent of the reference's check, hattention/mamba_apis.py:569-729).
* ``strong_final_state`` -- the final states ``ht`` the reference's chunkwise
  forward stores for HType.STRONG: the strong state loop of chunk_fwd_kernel_h
  (USE_H2, chunkwise.py:94-280) with its raw phase-0 state b_h kept per level;
  pinned against a closed form (a range of chunk summaries decayed to the end
  of the sequence) in tests/test_oracle_mamba2.py.
* ``autograd_bwd``      -- gradients (dq, dk, dv, dg, dl) of any of the above
  through torch.autograd; dg is w.r.t. the raw per-step g, which is what the
  reference returns after its reverse chunk-local cumsum (chunkwise.py:1596).

Strong hierarchy (HType.STRONG): ``materialized_fwd(..., htype=STRONG)`` uses
the strong level table (base.py:49-62 via oracle.levels), ``recurrent_fwd(...,
htype=STRONG)`` the cascade of HState.cascade_strong (recurrent.py:56-74), and
``chunked_strong_fwd`` the chunk decomposition the HIP strong kernel
implements; ``chunked_strong_bwd`` restates the HIP strong backward's
decomposition (chunk walks forward and, with the transposed cascade, in
reverse; dense diagonal / sub-diagonal tiles) and is checked against autograd
through ``chunked_strong_fwd``.  The first two restate the reference's two definitions of the
strong hierarchy independently, and all three agree to 1e-12; a one-hot
lambda with g == 0 is checked against a pair loop over the recursion and
lambda == 1 against the plain SSD scan.

Pinning: the four forward forms are structurally different algorithms and are
checked against each other; ``ssd_scan_fwd`` (textbook) pins the lambda == 1
case; lambda one-hot on one level is checked against a brute-force pair loop
using the recursive level function; autograd is pinned by
torch.autograd.gradcheck (finite differences) in float64.
"""
import math
from typing import Optional, Tuple

import torch

from oracle.levels import (get_num_levels, levels_matrix, level_weak_recursive,
                           levels_matrix_strong, strong_intra_table, strong_subdiag_table)

WEAK, STRONG = 0, 1   # HType values (hattention/base.py:12-14)


def _expand_groups(x: torch.Tensor, H: int) -> torch.Tensor:
    """[B, T, G, D] -> [B, T, H, D] (chunkwise.py:1169-1171 repeat)."""
    G = x.shape[2]
    if G == H:
        return x
    return x.repeat_interleave(H // G, dim=2)


def _check(q, k, v, g, l):
    B, T, G, K = q.shape
    H = v.shape[2]
    if k.shape != q.shape or v.shape[:2] != (B, T) or g.shape != (B, T, H) \
            or l.shape[:3] != (B, T, H) or H % G != 0:
        raise ValueError("shape mismatch")
    return B, T, G, H, K, v.shape[3], l.shape[3]


# --------------------------------------------------------------------------
# 1. materialised H matrix (base.py:75-98, 334-349)
# --------------------------------------------------------------------------
def materialized_H(g: torch.Tensor, l: torch.Tensor, htype: int = WEAK) -> torch.Tensor:
    """H[b, h, t, s] = l[b, t, h, level(t, s)] * prod_{u=s+1..t} exp(g[b, u, h]).

    base.py:87-96 builds the product of A = exp(g) over (s, t]; here the product
    is formed as exp of the difference of inclusive cumsums (identical math).
    ``htype`` selects the weak or the strong level function (base.py:65-72).
    """
    B, T, H = g.shape
    table = levels_matrix if htype == WEAK else levels_matrix_strong
    lev = torch.from_numpy(table(T, default=0, clamp_min=0))
    G = torch.cumsum(g, dim=1)                               # [B, T, H]
    seg = G[:, :, None, :] - G[:, None, :, :]                # [B, t, s, H]
    mask = torch.tril(torch.ones(T, T, dtype=torch.bool))
    seg = seg.masked_fill(~mask[None, :, :, None], float("-inf"))
    tt = torch.arange(T)[:, None].expand(T, T)
    lam = l.permute(0, 2, 1, 3)[:, :, tt, lev]               # [B, H, t, s]
    return torch.exp(seg).permute(0, 3, 1, 2) * lam          # [B, H, t, s]


def materialized_fwd(q, k, v, g, l, htype: int = WEAK) -> torch.Tensor:
    """hattention_materialized (base.py:334-349): O = (H o Q K^T) V."""
    B, T, G, H, K, V, L = _check(q, k, v, g, l)
    q = _expand_groups(q, H)
    k = _expand_groups(k, H)
    Hm = materialized_H(g, l, htype)
    qkt = torch.einsum("bthd,bshd->bhts", q, k)
    return torch.einsum("bhts,bshd->bthd", Hm * qkt, v)


# --------------------------------------------------------------------------
# 2. Fenwick recurrent form (recurrent.py:9-216)
# --------------------------------------------------------------------------
class FenwickState:
    """HState for HStruct.MAMBA2 (recurrent.py:9-54, 56-74, 76-100), weak or
    strong cascade.

    ``states`` [B, H, K, V, L]; ``counts`` [L] tokens merged into each level.
    """

    def __init__(self, B, H, K, V, L, dtype, htype: int = WEAK):
        self.L = L
        self.htype = htype
        self.states = torch.zeros(B, H, K, V, L, dtype=dtype)
        self.counts = [0] * L

    def cascade_weak(self):
        """recurrent.py:42-54: a full level (count == 2^level) is merged into
        the next level and emptied; stop at the first non-full level."""
        for level in range(self.L):
            capacity = 2 ** level
            if self.counts[level] == capacity:
                nxt = level + 1
                self.states[..., nxt] = self.states[..., nxt] + self.states[..., level]
                self.counts[nxt] += self.counts[level]
                self.states[..., level] = 0.0
                self.counts[level] = 0
            elif self.counts[level] < capacity:
                break
            else:
                raise ValueError("level over capacity")

    def cascade_strong(self):
        """recurrent.py:56-74: a carry (state, count) walks up the levels; level
        0, and a level whose count plus the carry's would exceed its capacity
        2^max(level - 1, 0), hands its content on as the next carry and takes
        the current one; otherwise the carry merges into the level and is
        cleared.  A carry left after the top level is dropped."""
        carry_s = torch.zeros_like(self.states[..., 0])
        carry_c = 0
        for level in range(self.L):
            capacity = 2 ** max(level - 1, 0)
            if self.counts[level] + carry_c > capacity or level == 0:
                over_s, over_c = self.states[..., level].clone(), self.counts[level]
                self.states[..., level] = carry_s
                self.counts[level] = carry_c
                carry_s, carry_c = over_s, over_c
            else:
                self.states[..., level] = self.states[..., level] + carry_s
                self.counts[level] += carry_c
                carry_s = torch.zeros_like(carry_s)
                carry_c = 0

    def cascade(self):
        if self.htype == WEAK:
            self.cascade_weak()
        else:
            self.cascade_strong()

    def insert(self, gate: torch.Tensor, value: torch.Tensor):
        """recurrent.py:76-94 (MAMBA2 branch): cascade, decay every level by the
        scalar gate, then the new token's k v^T becomes level 0."""
        self.cascade()
        self.states = gate[:, :, None, None, None] * self.states
        self.states[..., 0] = value
        self.counts[0] += 1

    def dot(self, lam: torch.Tensor) -> torch.Tensor:
        """recurrent.py:96-100 with step_output :159-166 weights: sum_l lam_l S_l."""
        return torch.einsum("bhkvl,bhl->bhkv", self.states, lam)


def recurrent_fwd(q, k, v, g, l, return_state: bool = False, htype: int = WEAK):
    """hattention_recurrent (recurrent.py:169-216) for HStruct.MAMBA2."""
    B, T, G, H, K, V, L = _check(q, k, v, g, l)
    q = _expand_groups(q, H)
    k = _expand_groups(k, H)
    S = FenwickState(B, H, K, V, L, q.dtype, htype)
    ys = []
    for t in range(T):
        value = torch.einsum("bhk,bhv->bhkv", k[:, t], v[:, t])      # step_state :145
        S.insert(torch.exp(g[:, t]), value)                          # a = exp(g)
        Sl = S.dot(l[:, t])
        ys.append(torch.einsum("bhk,bhkv->bhv", q[:, t], Sl))       # step_output :166
    o = torch.stack(ys, dim=1)
    return (o, S) if return_state else o


# --------------------------------------------------------------------------
# 3. plain SSD scan (lambda == 1 special case)
# --------------------------------------------------------------------------
def ssd_scan_fwd(q, k, v, g) -> torch.Tensor:
    """h_t = exp(g_t) h_{t-1} + k_t v_t^T ; o_t = q_t . h_t (no hierarchy)."""
    B, T, G, K = q.shape
    H, V = v.shape[2], v.shape[3]
    q = _expand_groups(q, H)
    k = _expand_groups(k, H)
    h = torch.zeros(B, H, K, V, dtype=q.dtype)
    ys = []
    for t in range(T):
        h = torch.exp(g[:, t])[:, :, None, None] * h + \
            torch.einsum("bhk,bhv->bhkv", k[:, t], v[:, t])
        ys.append(torch.einsum("bhk,bhkv->bhv", q[:, t], h))
    return torch.stack(ys, dim=1)


# --------------------------------------------------------------------------
# 4. chunked forms
# --------------------------------------------------------------------------
def _intra_level_table(C: int) -> torch.Tensor:
    return torch.from_numpy(levels_matrix(C, default=0, clamp_min=0))


def _chunk_views(q, k, v, g, l, C):
    B, T, G, H, K, V, L = _check(q, k, v, g, l)
    if T % C != 0:
        raise ValueError(f"T={T} must be a multiple of the chunk {C}")
    NT = T // C
    q = _expand_groups(q, H).reshape(B, NT, C, H, K)
    k = _expand_groups(k, H).reshape(B, NT, C, H, K)
    v = v.reshape(B, NT, C, H, V)
    g = g.reshape(B, NT, C, H)
    l = l.reshape(B, NT, C, H, L)
    return q, k, v, g, l, (B, T, H, K, V, L, NT)


def _intra_chunk(q, k, v, Gc, l, C):
    """Diagonal blocks (hssd_minimal.py:170-172; chunk_fwd_kernel_o USE_A,
    chunkwise.py:590-623): A = (Q K^T) o exp(Gc_t - Gc_s) o lambda[t, lev], causal."""
    lev = _intra_level_table(C)                                       # [t, s]
    mask = torch.tril(torch.ones(C, C, dtype=torch.bool))
    seg = Gc[:, :, :, None, :] - Gc[:, :, None, :, :]                 # [B,NT,t,s,H]
    seg = seg.masked_fill(~mask[None, None, :, :, None], float("-inf"))
    tt = torch.arange(C)[:, None].expand(C, C)
    lam = l.permute(0, 1, 3, 2, 4)[:, :, :, tt, lev]                  # [B,NT,H,t,s]
    lam = lam.permute(0, 1, 3, 4, 2)                                  # [B,NT,t,s,H]
    S = torch.einsum("bnthk,bnshk->bntsh", q, k)
    A = S * torch.exp(seg) * lam
    return torch.einsum("bntsh,bnshv->bnthv", A, v)


def _chunk_states(k, v, Gc):
    """hssd_minimal.py:176-178: kv_j = sum_s exp(Gc_last - Gc_s) k_s v_s^T."""
    decay = torch.exp(Gc[:, :, -1:, :] - Gc)                         # [B,NT,C,H]
    return torch.einsum("bnshk,bnsh,bnshv->bnhkv", k, decay, v)


def chunked_fwd(q, k, v, g, l, chunk_size: int = 64) -> torch.Tensor:
    """hssd_minimal_discrete (hssd_minimal.py:108-220), HType.WEAK.

    Inter-chunk part: for each inter-chunk level ell the chunk-level decay matrix
    exp(Cend[i-1] - Cend[j]) (hssd_minimal.py:184-188) is masked to the chunk
    pairs whose level is ell (:199-206) and applied to the chunk states; the
    reading chunk's output gets lambda[t, ell_h0 + ell] * exp(Gc_t) q_t . state
    (:210-212).  Levels come from the closed form instead of the T x T table.
    """
    C = chunk_size
    q, k, v, g, l, (B, T, H, K, V, L, NT) = _chunk_views(q, k, v, g, l, C)
    ell_h0 = get_num_levels(C, 2)
    nlev = math.ceil(math.log2(NT)) if NT > 1 else 0
    if ell_h0 + nlev > L:
        raise ValueError("too few levels")
    Gc = torch.cumsum(g, dim=2)                                      # chunk-local
    y = _intra_chunk(q, k, v, Gc, l, C)
    if NT > 1:
        kv = _chunk_states(k, v, Gc)                                 # [B,NT,H,K,V]
        Cend = torch.cumsum(Gc[:, :, -1, :], dim=1)                  # [B,NT,H]
        Cprev = torch.cat([torch.zeros_like(Cend[:, :1]), Cend[:, :-1]], dim=1)
        seg = Cprev[:, :, None, :] - Cend[:, None, :, :]             # [B,i,j,H]
        ii = torch.arange(NT)[:, None]
        jj = torch.arange(NT)[None, :]
        below = jj < ii
        seg = seg.masked_fill(~below[None, :, :, None], float("-inf"))
        dchunk = torch.exp(seg)
        clev = torch.from_numpy(levels_matrix(NT, default=0, clamp_min=0)) - 1
        out_decay = torch.exp(Gc)                                    # [B,NT,C,H]
        for ell in range(nlev):
            m = (clev == ell) & below
            d = dchunk * m[None, :, :, None].to(dchunk.dtype)
            st = torch.einsum("bijh,bjhkv->bihkv", d, kv)
            qs = torch.einsum("bnthk,bnhkv->bnthv", q, st)
            y = y + qs * (out_decay * l[..., ell_h0 + ell])[..., None]
    return y.reshape(B, T, H, V)


def chunked_strong_fwd(q, k, v, g, l, chunk_size: int = 64) -> torch.Tensor:
    """Chunked form of the strong hierarchy (HType.STRONG), the decomposition
    the HIP strong kernel implements (checked against materialized_fwd and
    recurrent_fwd with htype=STRONG, which restate base.py:49-62 and
    recurrent.py:56-74):

      o_t = sum_{s in chunk(t), s <= t} lam[t, intra(a, b)] e^{G_t - G_s} (q_t.k_s) v_s
          + sum_{s in chunk(t) - 1}     lam[t, sub(a, b)]  e^{G_t - G_s} (q_t.k_s) v_s
          + sum_{j >= 2} lam[t, log2(C) + j] e^{Gc_t} q_t . S_j(chunk(t)),

    with a, b the positions inside the chunks, intra / sub the two C x C level
    tables (oracle.levels.strong_intra_table / strong_subdiag_table), Gc the
    chunk-local inclusive cumsum, and S_j(i) level j of a chunk-level strong
    state (the cascade of recurrent.py:56-74 over whole chunks: each chunk is
    one insertion with value sum_s e^{Gc_last - Gc_s} k_s v_s^T and gate
    e^{Gc_last}), read for chunk i after the cascade and before the chunk's
    own decay and insertion, so it holds the source chunks c <= i - 2 with
    strong(i, c) = j, decayed to the start of chunk i.
    """
    C = chunk_size
    q, k, v, g, l, (B, T, H, K, V, L, NT) = _chunk_views(q, k, v, g, l, C)
    c = int(math.log2(C))
    nlev = math.ceil(math.log2(NT)) if NT > 1 else 0
    if c + 1 + nlev > L:
        raise ValueError("too few levels")
    Gc = torch.cumsum(g, dim=2)                                         # [B,NT,C,H]
    tt = torch.arange(C)[:, None].expand(C, C)
    # diagonal blocks
    lev = torch.from_numpy(strong_intra_table(C))
    mask = torch.tril(torch.ones(C, C, dtype=torch.bool))
    seg = Gc[:, :, :, None, :] - Gc[:, :, None, :, :]
    seg = seg.masked_fill(~mask[None, None, :, :, None], float("-inf"))
    lam = l.permute(0, 1, 3, 2, 4)[:, :, :, tt, lev].permute(0, 1, 3, 4, 2)
    A = torch.einsum("bnthk,bnshk->bntsh", q, k) * torch.exp(seg) * lam
    y = torch.einsum("bntsh,bnshv->bnthv", A, v)
    if NT > 1:
        # sub-diagonal blocks: source chunk n - 1 of target chunk n
        sub = torch.from_numpy(strong_subdiag_table(C))
        gl = Gc[:, :-1, -1:, :]                                         # [B,NT-1,1,H]
        seg = Gc[:, 1:, :, None, :] + (gl - Gc[:, :-1])[:, :, None, :, :]
        lam = l[:, 1:].permute(0, 1, 3, 2, 4)[:, :, :, tt, sub].permute(0, 1, 3, 4, 2)
        A = torch.einsum("bnthk,bnshk->bntsh", q[:, 1:], k[:, :-1]) * torch.exp(seg) * lam
        y[:, 1:] = y[:, 1:] + torch.einsum("bntsh,bnshv->bnthv", A, v[:, :-1])
        # far chunks: chunk-level strong state
        kv = _chunk_states(k, v, Gc)                                    # [B,NT,H,K,V]
        Lc = nlev + 2
        S = FenwickState(B, H, K, V, Lc, q.dtype, STRONG)
        for n in range(NT):
            S.cascade_strong()
            for j in range(2, Lc):
                if c + j >= L:
                    break
                w = l[:, n, :, :, c + j] * torch.exp(Gc[:, n])          # [B,C,H]
                y[:, n] = y[:, n] + torch.einsum("bthk,bhkv->bthv", q[:, n], S.states[..., j]) \
                    * w[..., None]
            S.states = torch.exp(Gc[:, n, -1])[:, :, None, None, None] * S.states
            S.states[..., 0] = kv[:, n]
            S.counts[0] += 1
    return y.reshape(B, T, H, V)


def _strong_merge_levels(NT: int, LM: int):
    """Merge level m of the chunk-level strong cascade at each step n (after n
    insertions): levels 0 .. m-1 move up one level and m - 1 merges into m;
    m == LM means the carry left the top level (recurrent.py:56-74)."""
    cnt = [0] * LM
    out = []
    for _ in range(NT):
        cc, m = 0, LM
        for j in range(LM):
            cap = 1 << max(j - 1, 0)
            swap = j == 0 or cnt[j] + cc > cap
            oc = cnt[j]
            if swap:
                cnt[j], cc = cc, oc
            else:
                cnt[j], cc = oc + cc, 0
            if j >= 1 and m == LM and (not swap or oc == 0):
                m = j
        out.append(m)
        cnt[0] += 1
    return out


def chunked_strong_bwd(q, k, v, g, l, do, chunk_size: int = 64, levels: int = 10):
    """(dq, dk, dv, dg, dl) of sum(o * do) for the strong chunk decomposition of
    ``chunked_strong_fwd``, by the decomposition the HIP strong backward
    implements (the reference's strong backward is chunkwise.py:1377-1580 with
    USE_A2 / USE_H2):

    * far levels, forward in time: the chunk-level strong state S_j(n) (read
      after the cascade of step n) gives dq_t += lam[t, 6 + j] e^{Gc_t} S_j do_t
      and dlam[t, 6 + j] = e^{Gc_t} q_t . S_j do_t;
    * far levels, backward in time: the adjoint A of the state runs the
      transposed steps in reverse (A_0 is d kv_n, then A_0 = 0, A *= e^{Gc_last},
      A_j += Q_n^T diag(lam[., 6 + j] e^{Gc}) dO_n, transposed cascade), and
      kv_n = K_n^T diag(e^{Gc_last - Gc}) V_n gives dk, dv;
    * diagonal / sub-diagonal blocks: dense 64 x 64 tiles with the two strong
      level tables; dlam of levels 0 .. log2(C) + 1 binned by the tables;
    * dG_t = q_t . dq_t - k_t . dk_t, dg_u = sum_{t >= u} dG_t.

    ``levels``: chunk-level state levels (the kernels hold 10; the carry that
    leaves the top is dropped, as in HState.cascade_strong).
    """
    C = chunk_size
    G0 = q.shape[2]
    q, k, v, g, l, (B, T, H, K, V, L, NT) = _chunk_views(q, k, v, g, l, C)
    do_ = do.reshape(B, NT, C, H, V)
    LM = levels
    c = int(math.log2(C))
    Gc = torch.cumsum(g, dim=2)                                       # [B,NT,C,H]
    eg = torch.exp(Gc)
    mlev = _strong_merge_levels(NT, LM)
    far = [j for j in range(2, LM) if c + j < L]
    # forward walk
    S = torch.zeros(LM, B, H, K, V, dtype=q.dtype)
    dq = torch.zeros_like(q)
    dl = torch.zeros_like(l)
    for n in range(NT):
        m = mlev[n]
        new = S.clone()
        new[0] = 0
        for e in range(1, LM):
            if e < m:
                new[e] = S[e - 1]
            elif e == m:
                new[e] = S[e] + S[e - 1]
        S = new
        for j in far:
            Y = torch.einsum("bthv,bhkv->bthk", do_[:, n], S[j])
            dq[:, n] += (l[:, n, :, :, c + j] * eg[:, n])[..., None] * Y
            dl[:, n, :, :, c + j] += eg[:, n] * (q[:, n] * Y).sum(-1)
        S = S * torch.exp(Gc[:, n, -1])[None, :, :, None, None]
        w = torch.exp(Gc[:, n, -1:] - Gc[:, n])                       # [B,C,H]
        S[0] = torch.einsum("bshk,bsh,bshv->bhkv", k[:, n], w, v[:, n])
    # reverse walk
    A = torch.zeros(LM, B, H, K, V, dtype=q.dtype)
    adj = torch.zeros(B, NT, H, K, V, dtype=q.dtype)
    for n in range(NT - 1, -1, -1):
        adj[:, n] = A[0]
        A[0] = 0
        A = A * torch.exp(Gc[:, n, -1])[None, :, :, None, None]
        for j in far:
            f = l[:, n, :, :, c + j] * eg[:, n]                        # [B,C,H]
            A[j] = A[j] + torch.einsum("bthk,bth,bthv->bhkv", q[:, n], f, do_[:, n])
        m = mlev[n]
        new = A.clone()
        for e in range(min(m, LM)):
            new[e] = A[e + 1] if e + 1 < LM else 0
        A = new
    # diagonal and sub-diagonal blocks
    dk = torch.zeros_like(k)
    dv = torch.zeros_like(v)
    tt = torch.arange(C)[:, None].expand(C, C)
    it = torch.from_numpy(strong_intra_table(C))
    mask = torch.tril(torch.ones(C, C, dtype=torch.bool))
    blocks = [(0, it, mask)]
    if NT > 1:
        blocks.append((1, torch.from_numpy(strong_subdiag_table(C)), None))
    for back, tab, msk in blocks:
        nt = slice(back, NT)
        ns = slice(0, NT - back)
        if back:
            seg = Gc[:, nt, :, None, :] + (Gc[:, ns, -1:, :] - Gc[:, ns])[:, :, None, :, :]
        else:
            seg = Gc[:, :, :, None, :] - Gc[:, :, None, :, :]
        E = torch.exp(seg)                                            # [B,n,t,s,H]
        if msk is not None:
            E = E * msk[None, None, :, :, None].to(E.dtype)
        lam = l[:, nt].permute(0, 1, 3, 2, 4)[:, :, :, tt, tab].permute(0, 1, 3, 4, 2)
        W = E * lam
        Sc = torch.einsum("bnthk,bnshk->bntsh", q[:, nt], k[:, ns])
        Dc = torch.einsum("bnthv,bnshv->bntsh", do_[:, nt], v[:, ns])
        dq[:, nt] += torch.einsum("bntsh,bnshk->bnthk", W * Dc, k[:, ns])
        dk[:, ns] += torch.einsum("bntsh,bnthk->bnshk", W * Dc, q[:, nt])
        dv[:, ns] += torch.einsum("bntsh,bnthv->bnshv", W * Sc, do_[:, nt])
        Mx = E * Sc * Dc
        for lev in range(min(c + 2, L)):
            sel = (tab == lev)
            if msk is not None:
                sel = sel & msk
            dl[:, nt, :, :, lev] += (Mx * sel[None, None, :, :, None].to(Mx.dtype)).sum(3)
    w = torch.exp(Gc[:, :, -1:] - Gc)                                  # [B,NT,C,H]
    dk += w[..., None] * torch.einsum("bnshv,bnhkv->bnshk", v, adj)
    dv += w[..., None] * torch.einsum("bnshk,bnhkv->bnshv", k, adj)
    dG = (q * dq).sum(-1) - (k * dk).sum(-1)                          # [B,NT,C,H]
    dG = dG.reshape(B, T, H)
    dg = dG.flip(1).cumsum(1).flip(1)
    dq = dq.reshape(B, T, H, K)
    dk = dk.reshape(B, T, H, K)
    if G0 != H:
        dq = dq.view(B, T, G0, H // G0, K).sum(3)
        dk = dk.view(B, T, G0, H // G0, K).sum(3)
    return dq, dk, dv.reshape(B, T, H, V), dg, dl.reshape(B, T, H, L)


def chunked_scan_fwd(q, k, v, g, l, chunk_size: int = 64,
                     output_final_state: bool = False
                     ) -> Tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    """chunkwise_fwd (chunkwise.py:1118-1275): returns (o, g_cumsum, ht).

    Per inter-chunk level ell (chunkwise.py:1219), scan the chunks in order
    (chunk_fwd_kernel_h, :179-266): the reading chunks (bit ell set, :523-527)
    first add lambda[t, ell_h0+ell] exp(Gc_t) q_t h (:576-606); then the state
    is reset after the last chunk of each aligned 2^(ell+1) block or decayed by
    exp(Gc_last) (:235-239), and the writing chunks (bit ell clear) add their
    decayed k^T v (:256-266).  With ``output_final_state`` the last chunk decays
    instead of resetting and the state is stored at level ell_h0+ell (:229-279).
    """
    C = chunk_size
    B0, T0 = q.shape[0], q.shape[1]
    q, k, v, g, l, (B, T, H, K, V, L, NT) = _chunk_views(q, k, v, g, l, C)
    ell_h0 = get_num_levels(C, 2)
    nlev = math.ceil(math.log2(NT)) if NT > 1 else 0
    if ell_h0 + nlev > L:
        raise ValueError("too few levels")
    Gc = torch.cumsum(g, dim=2)
    y = _intra_chunk(q, k, v, Gc, l, C)
    ht = torch.zeros(B, H, K, V, L, dtype=q.dtype) if output_final_state else None
    if NT > 1 or output_final_state:
        kv = _chunk_states(k, v, Gc)                                 # [B,NT,H,K,V]
        last = torch.exp(Gc[:, :, -1, :])                            # [B,NT,H]
        out_decay = torch.exp(Gc)
        ys = [y[:, i] for i in range(NT)]
        for ell in range(nlev):
            h = torch.zeros(B, H, K, V, dtype=q.dtype)
            period = 1 << (ell + 1)
            scale = out_decay * l[..., ell_h0 + ell]                 # [B,NT,C,H]
            for i in range(NT):
                if (i >> ell) & 1:                                   # reading chunk
                    qs = torch.einsum("bthk,bhkv->bthv", q[:, i], h)
                    ys[i] = ys[i] + qs * scale[:, i][..., None]
                reset = (i % period == period - 1)
                if output_final_state and i == NT - 1:
                    reset = False
                h = torch.zeros_like(h) if reset else h * last[:, i][:, :, None, None]
                if not (i >> ell) & 1:                               # writing chunk
                    h = h + kv[:, i]
            if output_final_state:
                ht[..., ell_h0 + ell] = h
        y = torch.stack(ys, dim=1)
    g_cumsum = Gc.reshape(B0, T0, H)
    return y.reshape(B, T, H, V), g_cumsum, ht


def strong_final_state(q, k, v, g, l, chunk_size: int = 64) -> torch.Tensor:
    """``ht`` of chunkwise_fwd with HType.STRONG and output_final_state: the
    loop of chunk_fwd_kernel_h with USE_H2, MODE_H2=1 and STORE_FINAL_STATE
    (chunkwise.py:94-280) for the strong levels ell = 1 .. nlev - 1
    (ell_init = 1, chunkwise.py:1215-1219), keeping its raw phase-0 state b_h.
    Per chunk i: b_h is reset when skip_g(i, ell) (i % 2^(ell+1) == 2^(ell+1) - 1,
    chunkwise.py:44-69; the last chunk decays instead, :227-233) or else
    multiplied by exp(Gc_last(i)) (:250-257); then, when get_phase_index(i, ell)
    (chunkwise.py:72-91, OFFSET=False) is 0, the chunk's decayed k^T v is added
    (:258-275).  b_h is stored at level ell_h0 + ell (:277-279); the other
    levels of the zero-initialised ht (chunkwise.py:1179) stay zero.
    Returns [B, H, K, V, L]."""
    C = chunk_size
    q, k, v, g, l, (B, T, H, K, V, L, NT) = _chunk_views(q, k, v, g, l, C)
    ell_h0 = get_num_levels(C, 2)
    nlev = math.ceil(math.log2(NT)) if NT > 1 else 0
    Gc = torch.cumsum(g, dim=2)
    kv = _chunk_states(k, v, Gc)                                     # [B,NT,H,K,V]
    last = torch.exp(Gc[:, :, -1, :])                                # [B,NT,H]
    ht = torch.zeros(B, H, K, V, L, dtype=k.dtype)
    for ell in range(1, nlev):
        period = 1 << (ell + 1)
        p0, p1 = 1 << ell, 1 << (ell - 1)
        b_h = torch.zeros(B, H, K, V, dtype=k.dtype)
        for i in range(NT):
            if i % period == period - 1 and i != NT - 1:
                b_h = torch.zeros_like(b_h)
            else:
                b_h = b_h * last[:, i][:, :, None, None]
            phase = (int(i % period >= p0) << 1) | int(i % p0 >= p1)
            if phase == 0:
                b_h = b_h + kv[:, i]
        ht[..., ell_h0 + ell] = b_h
    return ht


# --------------------------------------------------------------------------
# 5. backward through autograd
# --------------------------------------------------------------------------
def autograd_bwd(fwd, q, k, v, g, l, do, **kw):
    """(dq, dk, dv, dg, dl) of sum(o * do) for any forward form above.

    Matches the reference's return contract (kernel.py:230-236): dq/dk have the
    grouped shape of q/k, dg is w.r.t. the raw per-step g.
    """
    leaves = [x.detach().clone().requires_grad_(True) for x in (q, k, v, g, l)]
    o = fwd(*leaves, **kw)
    if isinstance(o, tuple):
        o = o[0]
    grads = torch.autograd.grad((o * do).sum(), leaves)
    return tuple(grads)


def brute_force_fwd(q, k, v, g, l) -> torch.Tensor:
    """Pair-by-pair loop over (t, s) using the reference's own recursive level
    function (base.py:41-46) and the product of exp(g) over (s, t] exactly as
    base.py:87-96 writes it (tiny T only)."""
    B, T, G, H, K, V, L = _check(q, k, v, g, l)
    q = _expand_groups(q, H)
    k = _expand_groups(k, H)
    A = torch.exp(g)
    o = torch.zeros(B, T, H, V, dtype=q.dtype)
    for t in range(T):
        for s in range(t + 1):
            lev = 0 if s == t else level_weak_recursive(t, s)
            w = l[:, t, :, lev] * torch.prod(A[:, s + 1:t + 1], dim=1) * \
                (q[:, t] * k[:, s]).sum(-1)
            o[:, t] += w[..., None] * v[:, s]
    return o


# --------------------------------------------------------------------------
# 6. the Mamba-2 layer scan with its pre- and post-processing
# --------------------------------------------------------------------------
def layer_lambda(L, dl, lambda_mode):
    """compute_lambda (hattention/mamba_apis.py:70-85) with L [H, Lv] broadcast
    over [B, T, H, Lv] (the rearrange of :360-366)."""
    Lb = L[None, None]
    if lambda_mode == "positive":
        return torch.nn.functional.softplus(Lb * dl)
    if lambda_mode == "bounded":
        return torch.exp(-torch.exp(Lb) * torch.nn.functional.softplus(dl))
    if lambda_mode is None:
        return Lb * dl
    raise ValueError


def layer_fwd(x, dt, A, B, C, dl, L, D=None, dt_bias=None, lambda_mode="positive",
              dt_softplus=True, scan=None, return_intermediates=False):
    """hmamba_chunk_scan_combined (hattention/mamba_apis.py:346-403) for
    HStruct.MAMBA2: dt' = softplus(dt + dt_bias), q = C, k = B, v = x dt',
    g = A dt', lambda = compute_lambda(L, dl), y = scan(...) + x D.

    x [B,T,H,P], dt [B,T,H], A [H], B / C [B,T,G,N], dl [B,T,H,Lv], L [H,Lv],
    D [H].  ``scan`` defaults to chunked_scan_fwd (the level-scan form).  The
    pre- and post-processing are torch's own functions (softplus, exp), so the
    restatement is pinned by them and by the scan's pinning; its gradients come
    from torch.autograd.  ``return_intermediates`` also returns (dt', v, g,
    lambda), the scan's inputs, as nodes of the same graph."""
    if dt_bias is not None:
        dt = dt + dt_bias[None, None]
    if dt_softplus:
        dt = torch.nn.functional.softplus(dt)
    v = x * dt[..., None]
    g = A[None, None] * dt
    lam = layer_lambda(L, dl, lambda_mode)
    if scan is None:
        y = chunked_scan_fwd(C, B, v, g, lam, chunk_size=64)[0]
    else:
        y = scan(C, B, v, g, lam)
    if D is not None:
        y = y + x * D[None, None, :, None]
    return (y, (dt, v, g, lam)) if return_intermediates else y


def causal_conv1d_silu(x, weight, bias):
    """causal_conv1d_fn(x, weight, bias, activation="silu") as called at
    hattention/mamba_apis.py:206-213 (the causal_conv1d package, absent here; its
    published algorithm): x [B, D, S], weight [D, W], bias [D] ->
    silu(bias[d] + sum_w weight[d, w] x[b, d, s - (W - 1) + w]), zero left padding;
    torch's grouped conv1d with W - 1 zeros on the left."""
    D, W = weight.shape
    y = torch.nn.functional.conv1d(torch.nn.functional.pad(x, (W - 1, 0)), weight[:, None, :],
                                   bias, groups=D)
    return torch.nn.functional.silu(y)


def gated_rmsnorm(x, weight, z, eps):
    """rmsnorm_fn(x, weight, bias=None, z=z, eps, group_size=None,
    norm_before_gate=False) as called at mamba_apis.py:247-255 (mamba_ssm's
    gated RMSNorm, absent here; its published algorithm):
    u = x silu(z), u / sqrt(mean(u^2) + eps) * weight."""
    u = x * torch.nn.functional.silu(z)
    return u * torch.rsqrt((u * u).mean(-1, keepdim=True) + eps) * weight


def split_conv1d_layer_fwd(zxbcdtdl, conv_w, conv_b, dt_bias, A, L, D, rms_w, eps, out_w, out_b,
                           headdim, ngroups, lambda_mode="positive", scan=None):
    """hmamba_split_conv1d_scan_combined (mamba_apis.py:116-260): split z, xBC, dt,
    dl; causal conv1d + SiLU of xBC; layer_fwd with D and dt_bias; gated RMSNorm
    with z; out-projection."""
    Bsz, S, _ = zxbcdtdl.shape
    H = D.shape[0]
    Lv = L.shape[-1]
    dim = H * headdim
    dstate = (zxbcdtdl.shape[-1] - 2 * dim - H - H * Lv) // ngroups // 2
    z, xBC, dt, dl = torch.split(zxbcdtdl, [dim, dim + 2 * ngroups * dstate, H, H * Lv], dim=-1)
    xBC = causal_conv1d_silu(xBC.transpose(1, 2), conv_w, conv_b).transpose(1, 2)
    x, Bm, Cm = torch.split(xBC, [dim, ngroups * dstate, ngroups * dstate], dim=-1)
    y = layer_fwd(x.reshape(Bsz, S, H, headdim), dt, A, Bm.reshape(Bsz, S, ngroups, dstate),
                  Cm.reshape(Bsz, S, ngroups, dstate), dl.reshape(Bsz, S, H, Lv), L, D=D,
                  dt_bias=dt_bias, lambda_mode=lambda_mode, scan=scan)
    y = gated_rmsnorm(y.reshape(Bsz, S, dim), rms_w, z, eps)
    return torch.nn.functional.linear(y, out_w, out_b)

"""The segment-parallel decomposition the HIP forward uses, checked on the CPU.

The forward kernels cut the chunk sequence into aligned segments of S = 2^s
chunks.  Inter-chunk levels e < s are scanned inside a segment; every chunk of
segment p reads a level e >= s (bit e - s of p set) as exp(E_i) * Htop_e(p),
built from per-segment summaries Sum(q) and total decays D_q.  The final
states (output_final_state) of the top levels are combinations of the same
summaries.  This module restates that decomposition in float64 torch, with
the same index arithmetic as the kernels, and checks it against the oracle's
level scan (chunked_scan_fwd, which follows chunkwise.py:1118-1275) for
several chunk counts, segment sizes and ragged last segments.  It pins the
algebra of the decomposition, not the kernels' arithmetic.
"""
import math

import pytest
import torch

from oracle import mamba2 as M


def make_inputs(B, T, H, K, V, L, seed=0):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, K, generator=gen, dtype=torch.float64)
    k = torch.randn(B, T, H, K, generator=gen, dtype=torch.float64)
    v = torch.randn(B, T, H, V, generator=gen, dtype=torch.float64)
    g = -torch.rand(B, T, H, generator=gen, dtype=torch.float64) * 0.3
    l = torch.nn.functional.softplus(torch.randn(B, T, H, L, generator=gen, dtype=torch.float64))
    return q, k, v, g, l


def segmented_fwd(q, k, v, g, l, C, slog, final_state):
    """Segment decomposition of the level scan (one (b, h) row at a time)."""
    B, T, H, K = q.shape
    V, L = v.shape[-1], l.shape[-1]
    NT = T // C
    nlev = math.ceil(math.log2(NT)) if NT > 1 else 0
    h0 = int(math.log2(C)) + 1                      # ell_h0 (7 for C = 64)
    S = 1 << slog
    NSEG = (NT + S - 1) // S
    nloc = min(slog, nlev)
    ntop = nlev - nloc
    o = torch.zeros(B, T, H, V, dtype=q.dtype)
    ht = torch.zeros(B, H, K, V, L, dtype=q.dtype)
    for b in range(B):
        for h in range(H):
            qq, kk, vv, gg, ll = q[b, :, h], k[b, :, h], v[b, :, h], g[b, :, h], l[b, :, h]
            gc = torch.cumsum(gg.reshape(NT, C), 1)              # chunk-local cumsum
            # kernel 1: summaries and decays
            sums, D = [], []
            for p in range(NSEG):
                acc = torch.zeros(K, V, dtype=q.dtype)
                for i in range(p * S, min(p * S + S, NT)):
                    w = torch.exp(gc[i, -1] - gc[i])
                    kc, vc = kk[i * C:(i + 1) * C], vv[i * C:(i + 1) * C]
                    acc = acc * torch.exp(gc[i, -1]) + kc.T @ (w[:, None] * vc)
                sums.append(acc)
                D.append(sum(gc[i, -1] for i in range(p * S, min(p * S + S, NT))))
            # kernel 2: one segment at a time
            for p in range(NSEG):
                htop = {}
                for e2 in range(ntop):
                    lo = (p >> (e2 + 1)) << (e2 + 1)
                    if (p >> e2) & 1:
                        hi = lo + (1 << e2)
                        dlog = sum((D[r] for r in range(hi, p)), torch.tensor(0.0, dtype=q.dtype))
                        acc = torch.zeros(K, V, dtype=q.dtype)
                        for qs in range(hi - 1, lo - 1, -1):
                            acc = acc + torch.exp(dlog) * sums[qs]
                            dlog = dlog + D[qs]
                        htop[e2] = acc
                        if final_state and p == NSEG - 1:
                            ht[b, h, :, :, h0 + slog + e2] = acc * torch.exp(D[p])
                    elif final_state and p == NSEG - 1:
                        lo2 = (p >> e2) << e2
                        dlog = torch.tensor(0.0, dtype=q.dtype)
                        acc = torch.zeros(K, V, dtype=q.dtype)
                        for qs in range(p, lo2 - 1, -1):
                            acc = acc + torch.exp(dlog) * sums[qs]
                            dlog = dlog + D[qs]
                        ht[b, h, :, :, h0 + slog + e2] = acc
                st = [torch.zeros(K, V, dtype=q.dtype) for _ in range(nloc)]
                E = torch.tensor(0.0, dtype=q.dtype)
                for ic in range(p * S, min(p * S + S, NT)):
                    ts = slice(ic * C, (ic + 1) * C)
                    qc, kc, vc, lc = qq[ts], kk[ts], vv[ts], ll[ts]
                    G = gc[ic]
                    # intra-chunk tile
                    lev = torch.tensor([[0 if s == t else (t ^ s).bit_length() for s in range(C)]
                                        for t in range(C)])
                    mask = torch.tensor([[s <= t for s in range(C)] for t in range(C)])
                    A = (qc @ kc.T) * torch.exp(G[:, None] - G[None, :]) * \
                        lc[torch.arange(C)[:, None], lev]
                    out = (A * mask) @ vc
                    eg = torch.exp(G)
                    for e in range(nloc):
                        if (ic >> e) & 1 and ic > p * S:
                            out = out + (qc @ st[e]) * (eg * lc[:, h0 + e])[:, None]
                    for e2 in range(ntop):
                        if (p >> e2) & 1:
                            out = out + (qc @ htop[e2]) * \
                                (eg * torch.exp(E) * lc[:, h0 + nloc + e2])[:, None]
                    o[b, ts, h] = out
                    kv = kc.T @ (torch.exp(G[-1] - G)[:, None] * vc)
                    last = ic == NT - 1
                    for e in range(nloc):
                        per = 2 << e
                        reset = (ic & (per - 1)) == per - 1 and not (last and final_state)
                        x = torch.zeros_like(st[e]) if reset else st[e] * torch.exp(G[-1])
                        if not (ic >> e) & 1:
                            x = x + kv
                        st[e] = x
                    if last and final_state:
                        for e in range(nloc):
                            ht[b, h, :, :, h0 + e] = st[e]
                    E = E + G[-1]
    return o, ht


@pytest.mark.parametrize("NT,slog", [(8, 1), (8, 2), (16, 2), (13, 2), (11, 1), (19, 2),
                                      (32, 4), (37, 3), (4, 2), (5, 3)])
def test_segmented_matches_level_scan(NT, slog):
    C = 4
    T = NT * C
    nlev = math.ceil(math.log2(NT)) if NT > 1 else 0
    L = int(math.log2(C)) + 1 + nlev + 1
    q, k, v, g, l = make_inputs(1, T, 2, 3, 2, L, seed=NT * 10 + slog)
    ref, _, ht_ref = M.chunked_scan_fwd(q, k, v, g, l, chunk_size=C, output_final_state=True)
    o, ht = segmented_fwd(q, k, v, g, l, C, slog, final_state=True)
    assert ((o - ref).abs().max() / ref.abs().max()).item() < 1e-12
    assert ((ht - ht_ref).abs().max() / ht_ref.abs().max()).item() < 1e-12
    o2, _ = segmented_fwd(q, k, v, g, l, C, slog, final_state=False)
    ref2 = M.chunked_scan_fwd(q, k, v, g, l, chunk_size=C)[0]
    assert ((o2 - ref2).abs().max() / ref2.abs().max()).item() < 1e-12


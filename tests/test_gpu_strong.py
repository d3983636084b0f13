"""GPU parity of the strong hierarchy (HType.STRONG).

The HIP paths run through the C-ABI: the strong chunkwise forward
(hattention.chunkwise.chunkwise_fwd with HType.STRONG -> hattn_mamba2_chunkwise_fwd
-> mamba2_strong.hip), the strong backward (chunkwise_bwd ->
hattn_mamba2_chunkwise_bwd -> mamba2_strong_bwd.hip) and the decode step with
the strong cascade (hattention.kernel.hattention_step -> hattn_hstate_step).
The checkers are the oracle's strong forms in float64 on the CPU
(oracle.mamba2.chunked_strong_fwd and recurrent_fwd(htype=STRONG), pinned
against the materialised strong table of base.py:49-62 and against each
other; the gradients by torch.autograd through chunked_strong_fwd), fed the
identical inputs.

Tolerances as the weak tests: bf16 inputs max|o - o_ref| / max|o_ref| < 2e-2 and
relative Frobenius error < 1e-2 (5e-2 for dg); level states of the decode 2e-2
per level.
"""
import math

import pytest
import torch

from bench import make_mamba2_inputs
from oracle import mamba2 as M

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
TOL_MAX = 2e-2
TOL_FRO = 1e-2


def _errs(out, ref):
    out = out.double().cpu()
    ref = ref.double().cpu()
    mx = ((out - ref).abs().max() / ref.abs().max()).item()
    fro = ((out - ref).norm() / ref.norm()).item()
    return mx, fro


def _levels(T):
    return 7 + (math.ceil(math.log2(T // 64)) if T > 64 else 0)


def _run_fwd(B, T, G, H, K, V, L, seed, rows=None, ldtype=None):
    from hattention.base import HType
    from hattention.chunkwise import chunkwise_fwd
    q, k, v, g, l = make_mamba2_inputs(B, T, H, K, V, L, G=G, seed=seed, ldtype=ldtype)
    print(f"[strong fwd] B={B} T={T} G={G} H={H} K={K} V={V} L={L} lambda={l.dtype}", flush=True)
    o, gc, ht = chunkwise_fwd(*(x.to(DEV) for x in (q, k, v, g, l)), False, 2, HType.STRONG, 64,
                              False)
    torch.cuda.synchronize()
    assert ht is None and o.dtype == v.dtype and o.shape == v.shape
    rows = rows or [(b, h) for b in range(B) for h in range(H)]
    for (b, h) in rows:
        gi = h // (H // G)
        qs, ks = (x[b:b + 1, :, gi:gi + 1].double() for x in (q, k))
        vs, gs, ls = (x[b:b + 1, :, h:h + 1].double() for x in (v, g, l))
        ref = M.chunked_strong_fwd(qs, ks, vs, gs, ls, chunk_size=64)
        mx, fro = _errs(o[b:b + 1, :, h:h + 1], ref)
        print(f"  row ({b},{h}) o: max-rel {mx:.2e} fro {fro:.2e}", flush=True)
        assert mx < TOL_MAX and fro < TOL_FRO, (b, h, mx, fro)
        ref_gc = torch.cumsum(gs.reshape(1, T // 64, 64, 1), dim=2).reshape(1, T, 1)
        assert torch.allclose(gc[b:b + 1, :, h:h + 1].double().cpu(), ref_gc, rtol=1e-5,
                              atol=1e-4)
    return o, (q, k, v, g, l)


@pytest.mark.parametrize("T", [64, 128, 192, 640, 1024])
def test_strong_fwd_lengths(T):
    _run_fwd(1, T, 2, 2, 64, 64, _levels(T), seed=T)


def test_strong_fwd_groups_k128_fp32_lambda():
    """grouped q / k, K = 128 (two 64-wide launches summed), fp32 lambda."""
    _run_fwd(2, 512, 1, 4, 128, 128, 10, seed=5, ldtype=torch.float32)


def test_strong_fwd_north_star_shape():
    """The north-star shape (B=4 T=16384 H=16 d=64 L=15) with the strong hierarchy,
    rows at both ends of the grid (and of the XCD map)."""
    _run_fwd(4, 16384, 16, 16, 64, 64, 15, seed=1000, rows=[(0, 0), (1, 7), (3, 15)])


def test_strong_fwd_nine_chunk_levels():
    """T = 32768, the longest sequence the strong C-ABI accepts (nine chunk
    levels: the last slot of the kernel's level arrays, lambda column 15 and
    the cascade's carry into the top level)."""
    _run_fwd(1, 32768, 2, 2, 64, 64, 16, seed=327)


@pytest.mark.parametrize("T", [2112, 4096, 5184, 8192])
def test_strong_fwd_segment_parallel(T):
    """More than 32 chunks: one walk per 32-chunk segment, started from the
    block sums of the earlier segments (33 chunks: a one-chunk last segment;
    81: a ragged one), every row."""
    _run_fwd(2, T, 2, 2, 64, 128, _levels(T), seed=T + 1)


@pytest.mark.parametrize("T", [4096, 16384])
def test_strong_fwd_levels_onehot_slow_decay(T):
    """Every chunk-level strong level on its own: lambda one-hot at column 6 + j
    and a slow decay (|g| <= 2e-4 per token, so the blocks of whole earlier
    segments that start each segment's walk keep their weight), o against the
    oracle's cascade form level by level."""
    from hattention.base import HType
    from hattention.chunkwise import chunkwise_fwd
    B, G, H, K, V = 1, 1, 1, 64, 64
    L = _levels(T)
    gen = torch.Generator().manual_seed(T + 3)
    q = (torch.randn(B, T, G, K, generator=gen) / 8).bfloat16()
    k = (torch.randn(B, T, G, K, generator=gen) / 8).bfloat16()
    v = torch.randn(B, T, H, V, generator=gen).bfloat16()
    g = -2e-4 * torch.rand(B, T, H, generator=gen)
    seen = 0
    for col in range(8, L):
        l = torch.zeros(B, T, H, L)
        l[..., col] = 1.0
        l = l.bfloat16()
        ref = M.chunked_strong_fwd(*(x.double() for x in (q, k, v, g, l)), chunk_size=64)
        if ref.abs().max().item() == 0.0:
            continue
        seen += 1
        o, _, _ = chunkwise_fwd(*(x.to(DEV) for x in (q, k, v, g, l)), False, 2, HType.STRONG, 64,
                                False)
        torch.cuda.synchronize()
        mx, fro = _errs(o, ref)
        print(f"  [strong onehot] T={T} level column {col}: |ref| {ref.abs().max().item():.2e} "
              f"max-rel {mx:.2e} fro {fro:.2e}", flush=True)
        assert mx < TOL_MAX and fro < TOL_FRO, (col, mx, fro)
    assert seen == L - 8


@pytest.mark.parametrize("T", [2112, 16384])
def test_strong_fwd_serial_walk_without_workspace(T):
    """Without a workspace for the block sums the forward walks each row
    serially; both walks against the oracle, and against each other (they
    differ by fp32 association and the bf16 rounding of the staged states)."""
    import ctypes
    from hattention import _lib
    B, G, H, K, V = 1, 2, 2, 64, 64
    L = _levels(T)
    q, k, v, g, l = make_mamba2_inputs(B, T, H, K, V, L, G=G, seed=T + 2)
    print(f"[strong fwd serial] T={T}", flush=True)
    lib = _lib.load()
    xs = [x.to(DEV) for x in (q, k, v, g, l)]
    need = lib.hattn_mamba2_chunkwise_fwd_workspace(B, T, G, H, K, V, L)
    outs = []
    for with_ws in (True, False):
        o = torch.empty(v.shape, dtype=v.dtype, device=DEV)
        gc = torch.empty(g.shape, dtype=torch.float32, device=DEV)
        ws = torch.empty(need if with_ws else 1, dtype=torch.uint8, device=DEV)
        st = lib.hattn_mamba2_chunkwise_fwd(
            *(_lib.ptr(x) for x in xs), _lib.ptr(o), _lib.ptr(gc), None, B, T, G, H, K, V, L,
            0, 0, 0, 0, 2, 1, 64, _lib.ptr(ws) if with_ws else None, need if with_ws else 0,
            _lib.stream_handle(DEV))
        _lib.check(st)
        outs.append(o)
    torch.cuda.synchronize()
    for h in range(H):
        gi = h // (H // G)
        qs, ks = (x[:, :, gi:gi + 1].double() for x in (q, k))
        vs, gs, ls = (x[:, :, h:h + 1].double() for x in (v, g, l))
        ref = M.chunked_strong_fwd(qs, ks, vs, gs, ls, chunk_size=64)
        for name, o in zip(("parallel", "serial"), outs):
            mx, fro = _errs(o[:, :, h:h + 1], ref)
            print(f"  head {h} {name}: max-rel {mx:.2e} fro {fro:.2e}", flush=True)
            assert mx < TOL_MAX and fro < TOL_FRO, (name, h, mx, fro)
    mx, fro = _errs(outs[0], outs[1].float())
    print(f"  parallel vs serial: max-rel {mx:.2e} fro {fro:.2e}", flush=True)
    assert mx < 1e-2 and fro < 2e-3


@pytest.mark.parametrize("B,T,G,H,K,V", [
    (1, 1024, 2, 2, 64, 64),      # 16 chunks: the last chunk ends every block
    (1, 5184, 2, 2, 64, 64),      # 81 chunks: ragged blocks, one-chunk ranges at the end
    (2, 2112, 1, 2, 128, 128),    # 33 chunks, grouped q / k, K and V of two 64-blocks
    (1, 16384, 2, 2, 64, 64),     # the north star's length: levels 8 .. 14
    (1, 32768, 1, 1, 64, 64),     # nine chunk levels
])
def test_strong_final_state(B, T, G, H, K, V):
    """output_final_state with HType.STRONG: ht against the oracle's restatement
    of the reference's USE_H2 state loop (oracle.mamba2.strong_final_state,
    pinned against its closed form on the CPU), every row; 1e-2 relative to each
    level's largest state, as the weak final states (a level decayed below
    1e-12 of the largest state, which fp64 keeps and fp32 flushes to zero, is
    checked against that floor); levels 0 .. 7 exactly zero.  o and g_cumsum
    are the ones of the call without final states."""
    from hattention.base import HType
    from hattention.chunkwise import chunkwise_fwd
    L = _levels(T)
    q, k, v, g, l = make_mamba2_inputs(B, T, H, K, V, L, G=G, seed=90 + T)
    print(f"[strong ht] B={B} T={T} G={G} H={H} K={K} V={V} L={L}", flush=True)
    ins = [x.to(DEV) for x in (q, k, v, g, l)]
    o, gc, ht = chunkwise_fwd(*ins, False, 2, HType.STRONG, 64, True)
    o0, gc0, _ = chunkwise_fwd(*ins, False, 2, HType.STRONG, 64, False)
    torch.cuda.synchronize()
    assert torch.equal(o, o0) and torch.equal(gc, gc0)
    assert ht.shape == (B, H, K, V, L) and ht.dtype == torch.float32
    ref = M.strong_final_state(*(x.double() for x in (q, k, v, g, l)), chunk_size=64)
    ht = ht.double().cpu()
    assert ht[..., :8].abs().max() == 0
    nlev = math.ceil(math.log2(T // 64))
    scale = ref.abs().max().item()
    for e in range(1, nlev):
        r = ref[..., 7 + e]
        err = ((ht[..., 7 + e] - r).abs().max() / max(r.abs().max().item(), 1e-12 * scale)).item()
        print(f"  level {7 + e}: max-rel {err:.2e}", flush=True)
        assert err < 1e-2, (e, err)


def test_strong_differs_from_weak():
    """The strong path is taken: its output differs from the weak one's on the
    same inputs by far more than the tolerance."""
    from hattention.base import HType
    from hattention.chunkwise import chunkwise_fwd
    o_s, xs = _run_fwd(1, 1024, 1, 1, 64, 64, 11, seed=7)
    o_w = chunkwise_fwd(*(x.to(DEV) for x in xs), False, 2, HType.WEAK, 64, False)[0]
    mx, _ = _errs(o_s, o_w)
    assert mx > 0.1, mx


def test_strong_hattention_kernel_forward_and_backward():
    """HAttentionFunction with HType.STRONG: the forward runs the strong kernel,
    the backward the strong backward kernels; gradients in the input dtypes
    against autograd through the oracle (kernel.py:230-244)."""
    from hattention.base import HType, HStruct
    from hattention.kernel import hattention_kernel
    B, T, H, K, V, L = 1, 256, 2, 64, 64, 9
    q, k, v, g, l, do = make_mamba2_inputs(B, T, H, K, V, L, seed=11, with_do=True)
    leaves = [x.to(DEV).requires_grad_(True) for x in (q, k, v, g, l)]
    o = hattention_kernel(leaves[0], leaves[1], leaves[2], None, leaves[3], leaves[4], None,
                          False, 2, HType.STRONG, HStruct.MAMBA2)
    ref_o = M.chunked_strong_fwd(*(x.double() for x in (q, k, v, g, l)), chunk_size=64)
    mx, fro = _errs(o.detach(), ref_o)
    assert mx < TOL_MAX and fro < TOL_FRO, (mx, fro)
    (o.float() * do.to(DEV).float()).sum().backward()
    ref = M.autograd_bwd(M.chunked_strong_fwd, *(x.double() for x in (q, k, v, g, l, do)),
                         chunk_size=64)
    for name, x, r in zip(NAMES, leaves, ref):
        assert x.grad is not None and x.grad.dtype == x.dtype, name
        mx, fro = _errs(x.grad, r)
        tf = TOL_FRO_DG if name == "dg" else TOL_FRO
        assert mx < TOL_MAX and fro < tf, (name, mx, fro)


# ---------------------------------------------------------------------------
# backward (chunkwise_bwd with HType.STRONG)
# ---------------------------------------------------------------------------
NAMES = ("dq", "dk", "dv", "dg", "dl")
# dg is the reverse cumsum of dG_t = q_t . dq_t - k_t . dk_t, which cancels
# heavily (sum_t dG_t = 0): the weak backward's bound, 5e-2 relative Frobenius
# on dg, with the max-abs/rel 2e-2 kept.
TOL_FRO_DG = 5e-2


def _run_bwd(B, T, G, H, K, V, L, seed, rows=None, ldtype=None, full=False):
    """chunkwise_bwd(HType.STRONG) against autograd through
    oracle.mamba2.chunked_strong_fwd in float64 on the identical inputs: every
    row (full=True: one vectorised oracle call over the whole batch) or the
    listed rows."""
    from hattention.base import HType
    from hattention.chunkwise import chunkwise_bwd, chunkwise_fwd
    q, k, v, g, l, do = make_mamba2_inputs(B, T, H, K, V, L, G=G, seed=seed, ldtype=ldtype,
                                           with_do=True)
    print(f"[strong bwd] B={B} T={T} G={G} H={H} K={K} V={V} L={L} lambda={l.dtype}", flush=True)
    qd, kd, vd, gd, ld, dod = (x.to(DEV) for x in (q, k, v, g, l, do))
    _, gc, _ = chunkwise_fwd(qd, kd, vd, gd, ld, False, 2, HType.STRONG, 64, False)
    grads = chunkwise_bwd(qd, kd, vd, gc, ld, dod, False, 2, HType.STRONG, 64)
    torch.cuda.synchronize()
    assert grads[0].dtype == q.dtype and grads[2].dtype == v.dtype
    assert grads[3].dtype == torch.float32 and grads[4].dtype == torch.float32
    if full:
        ref = M.autograd_bwd(M.chunked_strong_fwd, *(x.double() for x in (q, k, v, g, l, do)),
                             chunk_size=64)
        for name, a_, r in zip(NAMES, grads, ref):
            mx, fro = _errs(a_, r)
            print(f"  all rows {name}: max-rel {mx:.2e} fro {fro:.2e}", flush=True)
            tf = TOL_FRO_DG if name == "dg" else TOL_FRO
            assert mx < TOL_MAX and fro < tf, (name, mx, fro)
        return grads
    assert G == H, "row checks of grouped dq / dk need the whole group"
    rows = rows or [(b, h) for b in range(B) for h in range(H)]
    for (b, h) in rows:
        sl = lambda x: x[b:b + 1, :, h:h + 1].double()
        ref = M.autograd_bwd(M.chunked_strong_fwd, *(sl(x) for x in (q, k, v, g, l, do)),
                             chunk_size=64)
        for name, a_, r in zip(NAMES, grads, ref):
            mx, fro = _errs(a_[b:b + 1, :, h:h + 1], r)
            print(f"  row ({b},{h}) {name}: max-rel {mx:.2e} fro {fro:.2e}", flush=True)
            tf = TOL_FRO_DG if name == "dg" else TOL_FRO
            assert mx < TOL_MAX and fro < tf, (b, h, name, mx, fro)
    return grads


@pytest.mark.parametrize("T", [64, 128, 192, 640, 1024])
def test_strong_bwd_lengths(T):
    """one chunk (no sub-diagonal block, no far level), two chunks (no far
    level), ragged chunk counts and several far levels"""
    _run_bwd(1, T, 2, 2, 64, 64, _levels(T), seed=100 + T, full=True)


def test_strong_bwd_more_levels_than_needed():
    """L above 7 + ceil(log2(T/64)): the unused dlambda columns are zero"""
    g = _run_bwd(1, 1024, 1, 1, 64, 64, 14, seed=77, full=True)
    assert g[4][..., 11:].abs().max().item() == 0.0


def test_strong_bwd_groups_k128_v128_fp32_lambda():
    """grouped q / k (dq, dk summed over the group), K = V = 128 (one launch per
    64-wide key / value block, gradients summed in fp32), fp32 lambda"""
    _run_bwd(2, 512, 1, 2, 128, 128, 10, seed=5, ldtype=torch.float32, full=True)


def test_strong_bwd_many_rows():
    """every (batch, head) row of a grid that spans several XCD groups"""
    _run_bwd(3, 2048, 6, 6, 64, 64, 12, seed=9, full=True)


def test_strong_bwd_north_star_shape():
    """the north-star shape (B=4 T=16384 H=16 d=64 L=15) with the strong
    hierarchy: rows at both ends of the grid"""
    _run_bwd(4, 16384, 16, 16, 64, 64, 15, seed=1001, rows=[(0, 0), (3, 15)])


def test_strong_bwd_nine_chunk_levels():
    """T = 32768 (nine chunk levels, the strong C-ABI's maximum): every row."""
    _run_bwd(1, 32768, 2, 2, 64, 64, 16, seed=328, full=True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_strong_decode_matches_recurrent(dtype):
    """hattention_step with a strong HState from empty: every token's output and
    the final level states and counts against the recurrent cascade_strong."""
    from hattention.base import HType, HStruct
    from hattention.kernel import hattention_step
    from hattention.recurrent import HState
    B, T, G, H, K, V, L = 2, 150, 1, 2, 64, 32, 9
    q, k, v, g, l = make_mamba2_inputs(B, T, H, K, V, L, G=G, seed=401, dtype=dtype)
    print(f"[strong decode] B={B} T={T} H={H} K={K} V={V} L={L} {dtype}", flush=True)
    S = HState(2, HType.STRONG, HStruct.MAMBA2, (B, H, K, V, L), torch.float32, DEV)
    qd, kd, vd, gd, ld = (x.to(DEV) for x in (q, k, v, g, l))
    outs = []
    for t in range(T):
        o, S = hattention_step(S, qd[:, t], kd[:, t], vd[:, t], None, gd[:, t], ld[:, t], None,
                               2, HType.STRONG, HStruct.MAMBA2)
        outs.append(o)
    torch.cuda.synchronize()
    o = torch.stack(outs, 1)
    o_ref, F = M.recurrent_fwd(*(x.double() for x in (q, k, v, g, l)), return_state=True,
                               htype=M.STRONG)
    tol = (1e-4, 1e-4) if dtype == torch.float32 else (TOL_MAX, TOL_FRO)
    mx, fro = _errs(o, o_ref)
    print(f"  o: max-rel {mx:.2e} fro {fro:.2e}", flush=True)
    assert mx < tol[0] and fro < tol[1], (mx, fro)
    assert [int(c) for c in S.counts.cpu()] == list(F.counts) == S.host_counts
    got = S.states.double().cpu()
    for e in range(L):
        r = F.states[..., e]
        if r.abs().max() == 0:
            assert got[..., e].abs().max() == 0, e
            continue
        err = ((got[..., e] - r).norm() / r.norm()).item()
        assert err < max(tol[0], 1e-4), (e, err)


def test_strong_prefill_matches_recurrent():
    """hattention_prefill with HType.STRONG (every token through the decode
    step, as the reference's T0 = 0 for the strong hierarchy, kernel.py:495-499)."""
    from hattention.base import HType, HStruct
    from hattention.kernel import hattention_prefill
    B, T, H, K, V, L = 1, 100, 2, 64, 32, 9
    q, k, v, g, l = make_mamba2_inputs(B, T, H, K, V, L, seed=402, dtype=torch.float32)
    o, S = hattention_prefill(*(x.to(DEV) for x in (q, k, v)), None,
                              *(x.to(DEV) for x in (g, l)), None, False, 2, HType.STRONG,
                              HStruct.MAMBA2)
    torch.cuda.synchronize()
    o_ref, F = M.recurrent_fwd(*(x.double() for x in (q, k, v, g, l)), return_state=True,
                               htype=M.STRONG)
    mx, fro = _errs(o, o_ref)
    assert mx < 1e-4 and fro < 1e-4, (mx, fro)
    assert S.host_counts == list(F.counts)

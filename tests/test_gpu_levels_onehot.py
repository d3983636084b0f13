"""Level-by-level pinning of the HIP forward kernels: one-hot lambda, g == 0.

With lambda one-hot on level ell and no decay, the output holds exactly the
pairs (t, s) whose level is ell:

    o_t = sum_{s <= t, level(t, s) == ell} (q_t . k_s) v_s,

so a pair placed on the wrong level changes o by a whole (q_t . k_s) v_s
term.  The inputs are integers in {-1, 0, 1} (k and v sparse), so every
product, every partial sum the kernels form (intra-chunk tiles, level
states, segment summaries, the staged bf16 copies of the states) and every
output is an integer well below 2^8 (states) or 2^24 (sums): each kernel
computes them exactly, and the HIP output must equal the float64 reference
bit for bit.  The premise (state magnitudes below 256, exactly representable
in bf16) is checked on the inputs before the comparison.

References:
* at T <= 4096 the masked product ((level == ell) o Q K^T) V with the level
  matrices of oracle.levels (the reference's weak / strong recursions,
  base.py:41-62), and ``oracle.mamba2.materialized_fwd`` (the explicit H
  matrix of base.py:75-98) on one level per run as a cross-check;
* for the inter-chunk levels at T = 16384 and 32768 (where the T x T matrix does not
  fit), the Fenwick block form: chunk n reads level 7 + e iff bit e of n is
  set, and then holds the chunks m < n that agree with n above bit e, i.e.
  the 2^e chunks starting at (n >> (e + 1)) << (e + 1).  This form is pinned
  against materialized_fwd at T = 2048 in the same test module (a CPU test).

Kernels covered: the fused single-pass bf16 forward (north-star path, its
local levels, segment summaries, look-back and top levels), the bf16x3
kernels (fp32 inputs), and the HType.STRONG forward.
"""
import math

import numpy as np
import pytest
import torch

from hattention import _lib
from oracle.levels import levels_matrix, levels_matrix_strong
from oracle.mamba2 import WEAK, STRONG, materialized_fwd

DEV = torch.device("cuda:0")


def _inputs(T, H, K, V, seed):
    gen = torch.Generator().manual_seed(seed)

    def tern(shape, p):
        x = torch.randint(-1, 2, shape, generator=gen).double()
        keep = torch.rand(shape, generator=gen) < p
        return x * keep

    q = tern((1, T, H, K), 0.5)
    k = tern((1, T, H, K), 0.25)
    v = tern((1, T, H, V), 0.25)
    return q, k, v


def _max_state(k, v, T):
    """Largest |entry| of the sum of k_s v_s^T over any aligned block of up to
    T / 2 tokens (the level states and segment summaries the kernels stage)."""
    kk = k[0].permute(1, 0, 2).numpy()   # [H, T, K]
    vv = v[0].permute(1, 0, 2).numpy()
    m = 0.0
    size = 64
    while size <= T // 2:
        for s0 in range(0, T, size):
            blk = np.einsum("htk,htv->hkv", kk[:, s0:s0 + size], vv[:, s0:s0 + size])
            m = max(m, float(np.abs(blk).max()))
        size *= 2
    return m


def _fwd(q, k, v, l, htype, qdtype):
    """hattn_mamba2_chunkwise_fwd through the C-ABI with an fp32 output."""
    B, T, H, K = q.shape
    V, L = v.shape[3], l.shape[3]
    qd = q.to(qdtype).to(DEV).contiguous()
    kd = k.to(qdtype).to(DEV).contiguous()
    vd = v.to(qdtype).to(DEV).contiguous()
    ld = l.to(qdtype).to(DEV).contiguous()
    g = torch.zeros(B, T, H, dtype=torch.float32, device=DEV)
    o = torch.empty(B, T, H, V, dtype=torch.float32, device=DEV)
    gc = torch.empty_like(g)
    lib = _lib.load()
    ws, ws_ptr, ws_bytes = _lib.workspace(
        lib.hattn_mamba2_chunkwise_fwd_workspace(B, T, H, H, K, V, L), DEV)
    st = lib.hattn_mamba2_chunkwise_fwd(
        _lib.ptr(qd), _lib.ptr(kd), _lib.ptr(vd), _lib.ptr(g), _lib.ptr(ld), _lib.ptr(o),
        _lib.ptr(gc), None, B, T, H, H, K, V, L, _lib.dtype_code(qd), _lib.dtype_code(vd),
        _lib.dtype_code(ld), _lib.dtype_code(o), 2, htype, 64, ws_ptr, ws_bytes,
        _lib.stream_handle(DEV))
    _lib.check(st)
    torch.cuda.synchronize()
    if htype == WEAK and qdtype == torch.bfloat16:
        assert _lib.fwd_status(ws, B, T, H, V, DEV) == 0
    return o.double().cpu()


def _onehot(T, H, L, ell):
    l = torch.zeros(1, T, H, L, dtype=torch.float64)
    l[..., ell] = 1.0
    return l


def _block_form(q, k, v, e):
    """Output of inter-chunk level e (absolute 7 + e) with g == 0, by blocks."""
    B, T, H, K = q.shape
    NT = T // 64
    kc = k[0].reshape(NT, 64, H, K)
    vc = v[0].reshape(NT, 64, H, v.shape[3])
    kv = torch.einsum("nthk,nthv->nhkv", kc, vc)                  # [NT, H, K, V]
    cum = torch.cat([torch.zeros_like(kv[:1]), kv.cumsum(0)])      # cum[m] = sum of chunks < m
    o = torch.zeros_like(v)
    qc = q[0].reshape(NT, 64, H, K)
    for n in range(NT):
        if (n >> e) & 1:
            lo = (n >> (e + 1)) << (e + 1)
            st = cum[lo + (1 << e)] - cum[lo]
            o[0, 64 * n:64 * (n + 1)] = torch.einsum("thk,hkv->thv", qc[n], st)
    return o


def _masked_refs(q, k, v, T, htype):
    """Per level ell: ((level == ell) o Q K^T) V, float64, one head at a time."""
    lev = torch.from_numpy((levels_matrix if htype == WEAK else levels_matrix_strong)(T))
    qkt = torch.einsum("thk,shk->hts", q[0], k[0])
    def ref(ell):
        m = (lev == ell).double()
        return torch.einsum("hts,shv->thv", qkt * m, v[0])[None]
    return ref


def _check_exact(got, ref, what):
    diff = (got - ref).abs().max().item()
    assert torch.equal(got, ref), f"{what}: max |diff| {diff} (max |ref| {ref.abs().max().item()})"
    # the level carries work: a level that selects no pair would pass trivially
    return ref.abs().max().item()


def test_block_form_matches_materialized():
    """The Fenwick block form of the inter-chunk levels against the explicit
    H matrix with the reference's recursive level function (fp64, exact)."""
    T, H = 2048, 1
    q, k, v = _inputs(T, H, 64, 64, seed=3)
    g = torch.zeros(1, T, H, dtype=torch.float64)
    nlev = math.ceil(math.log2(T // 64))
    masked = _masked_refs(q, k, v, T, WEAK)
    for e in range(nlev):
        ref = materialized_fwd(q, k, v, g, _onehot(T, H, 7 + nlev, 7 + e), WEAK)
        assert torch.equal(masked(7 + e), ref), e
        assert torch.equal(_block_form(q, k, v, e), ref), e


@pytest.mark.gpu
@pytest.mark.parametrize("qdtype", [torch.bfloat16, torch.float32])
def test_weak_every_level_t4096(qdtype):
    # T = 4096: 64 chunks, four 16-chunk segments (bf16: local levels 7..10,
    # top levels 11, 12 from the segment summaries; fp32: one 64-chunk segment)
    T, H, K, V = 4096, 2, 64, 64
    nlev = 6
    L = 7 + nlev
    q, k, v = _inputs(T, H, K, V, seed=11)
    assert _max_state(k, v, T) < 256
    g = torch.zeros(1, T, H, dtype=torch.float64)
    masked = _masked_refs(q, k, v, T, WEAK)
    for ell in range(L):
        l = _onehot(T, H, L, ell)
        print(f"[onehot weak {qdtype}] T={T} level {ell}", flush=True)
        ref = masked(ell)
        if ell == L - 1:
            assert torch.equal(ref, materialized_fwd(q, k, v, g, l, WEAK))
        got = _fwd(q, k, v, l, 0, qdtype)
        assert _check_exact(got, ref, f"level {ell}") > 0


@pytest.mark.gpu
@pytest.mark.parametrize("T", [16384, 32768])
def test_weak_top_levels_north_star_length(T):
    # T = 16384 (the north star's length): 16 segments, local levels 7..10,
    # top levels 11..14 built by the look-back from the segment summaries;
    # T = 32768: 32 segments, five top levels (the kernel then stages bf16
    # lambda as bf16, so that two workgroups share a CU)
    H, K, V = 2, 64, 64
    nlev = int(math.log2(T // 64))
    L = 7 + nlev
    q, k, v = _inputs(T, H, K, V, seed=13)
    assert _max_state(k, v, T) < 256
    for e in range(nlev):
        ell = 7 + e
        print(f"[onehot weak bf16] T={T} level {ell}", flush=True)
        ref = _block_form(q, k, v, e)
        got = _fwd(q, k, v, _onehot(T, H, L, ell), 0, torch.bfloat16)
        assert _check_exact(got, ref, f"level {ell}") > 0


@pytest.mark.gpu
def test_weak_top_levels_bf16x3_segments():
    # fp32 inputs at T = 16384: 64-chunk segments, two top levels
    T, H, K, V = 16384, 1, 64, 64
    nlev = 8
    L = 7 + nlev
    q, k, v = _inputs(T, H, K, V, seed=17)
    assert _max_state(k, v, T) < 256
    for e in range(nlev):
        ell = 7 + e
        print(f"[onehot weak fp32] T={T} level {ell}", flush=True)
        ref = _block_form(q, k, v, e)
        got = _fwd(q, k, v, _onehot(T, H, L, ell), 0, torch.float32)
        assert _check_exact(got, ref, f"level {ell}") > 0


@pytest.mark.gpu
@pytest.mark.parametrize("T", [1024, 4096])
def test_strong_every_level(T):
    # HType.STRONG: diagonal and sub-diagonal level tables, the far chunk levels
    H, K, V = 2, 64, 64
    nlev = math.ceil(math.log2(T // 64))
    L = 7 + nlev
    q, k, v = _inputs(T, H, K, V, seed=19 + T)
    assert _max_state(k, v, T) < 256
    g = torch.zeros(1, T, H, dtype=torch.float64)
    masked = _masked_refs(q, k, v, T, STRONG)
    for ell in range(L):
        l = _onehot(T, H, L, ell)
        print(f"[onehot strong] T={T} level {ell}", flush=True)
        ref = masked(ell)
        if ell == L - 1:
            assert torch.equal(ref, materialized_fwd(q, k, v, g, l, STRONG))
        got = _fwd(q, k, v, l, 1, torch.bfloat16)
        if ref.abs().max() == 0:
            # a strong level no pair of this length reaches stays empty
            assert got.abs().max() == 0, ell
            continue
        _check_exact(got, ref, f"strong level {ell}")

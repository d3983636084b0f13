"""Fused pre- and post-processing of the log-linear Mamba-2 layer scan (MI355X).

hmamba_chunk_scan_combined (hattention/mamba_apis.py:263-404) wraps the scan in
elementwise torch work: dt' = softplus(dt + dt_bias), v = x dt', g = A dt',
lambda = compute_lambda(L, dl) and y = o + x D.  Here the forward is one launch
of the bf16 forward scan with that work folded into its loads and stores
(``hattn_mamba2_layer_scan_fwd``), or, outside its shapes and dtypes, three HIP
launches (libhattn_hip.so): ``hattn_mamba2_layer_prologue`` (one pass over x,
dt, dl writing v, g, lambda), the chunkwise kernels, and
``hattn_mamba2_layer_epilogue`` (y = o + x D); the backward is the chunkwise
backward plus ``hattn_mamba2_layer_bwd`` (one pass producing dx, ddt, ddl and
the per-head sums dA, ddt_bias, dD, dL).  Result dtypes follow torch's type
promotion of the reference's expressions, computed in fp32 inside the kernels.
"""
from typing import Optional

import torch

from hattention import _lib

LAMBDA_MODES = {None: 0, "positive": 1, "bounded": 2}


def _code(dtype: torch.dtype) -> int:
    try:
        return _lib.DTYPE_CODES[dtype]
    except KeyError:
        raise NotImplementedError(f"unsupported dtype {dtype}") from None


def _contig(t):
    return t.contiguous() if t is not None else None


def _aligned(t):
    """A contiguous tensor whose storage starts 16-byte aligned (the kernels
    read four elements at a time)."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def lambda_mode_code(lambda_mode: Optional[str]) -> int:
    if lambda_mode not in LAMBDA_MODES:
        raise ValueError
    return LAMBDA_MODES[lambda_mode]


def layer_prologue(x, dt, A, dt_bias, dl, L, dt_softplus: bool, lambda_mode: Optional[str],
                   v_dtype: Optional[torch.dtype] = None):
    """x [B,T,H,P], dt [B,T,H], A [H], dt_bias [H] or None, dl [B,T,H,Lv], L [H,Lv]
    -> (v = x softplus(dt + dt_bias) [B,T,H,P], g = A dt' [B,T,H] fp32,
    lambda [B,T,H,Lv]) in the dtypes torch gives the reference's expressions,
    except v in ``v_dtype`` when given."""
    B_, T, H, P = x.shape
    Lv = dl.shape[-1]
    if dt.shape != (B_, T, H) or dl.shape[:3] != (B_, T, H) or L.shape != (H, Lv) or \
            A.shape != (H,) or (dt_bias is not None and dt_bias.shape != (H,)):
        raise ValueError("shape mismatch in the layer pre-processing")
    dev = _lib.require_device(x, dt, A, dt_bias, dl, L)
    dtp = torch.result_type(dt, dt_bias) if dt_bias is not None else dt.dtype
    if v_dtype is None:
        v_dtype = torch.promote_types(x.dtype, dtp)
    lam_dtype = torch.promote_types(L.dtype, dl.dtype)
    x, dl = _aligned(x), _contig(dl)
    dt, L = _contig(dt), _contig(L)
    A = A.float().contiguous()
    bias = dt_bias.float().contiguous() if dt_bias is not None else None
    v = torch.empty(x.shape, dtype=v_dtype, device=dev)
    g = torch.empty(B_, T, H, dtype=torch.float32, device=dev)
    lam = torch.empty(dl.shape, dtype=lam_dtype, device=dev)
    _lib.check(_lib.load().hattn_mamba2_layer_prologue(
        _lib.ptr(x), _lib.ptr(dt), _lib.ptr(A), _lib.ptr(bias), _lib.ptr(dl), _lib.ptr(L),
        _lib.ptr(v), _lib.ptr(g), _lib.ptr(lam), B_, T, H, P, Lv, int(bool(dt_softplus)),
        lambda_mode_code(lambda_mode), _code(x.dtype), _code(dt.dtype), _code(dl.dtype),
        _code(L.dtype), _code(v.dtype), _code(lam.dtype), _lib.stream_handle(dev)))
    return v, g, lam


def layer_epilogue(y, x, D):
    """y + x * D[h] (y, x [B,T,H,P]; D [H]) in torch's promoted dtype."""
    B_, T, H, P = x.shape
    if y.shape != x.shape or D.shape != (H,):
        raise ValueError("shape mismatch in the layer post-processing")
    dev = _lib.require_device(y, x, D)
    out_dtype = torch.promote_types(y.dtype, torch.promote_types(x.dtype, D.dtype))
    y, x = _aligned(y), _aligned(x)
    Df = D.float().contiguous()
    out = torch.empty(x.shape, dtype=out_dtype, device=dev)
    _lib.check(_lib.load().hattn_mamba2_layer_epilogue(
        _lib.ptr(y), _lib.ptr(x), _lib.ptr(Df), _lib.ptr(out), B_, T, H, P, _code(y.dtype),
        _code(x.dtype), _code(out.dtype), _lib.stream_handle(dev)))
    return out


def layer_backward(x, dt, A, dt_bias, dl, L, D, dy, dv, dg, dlam, dt_softplus, lambda_mode):
    """Gradients of the pre- and post-processing given the scan's dv, dg, dlam and
    the layer output gradient dy: (dx, ddt, ddl, dA, ddt_bias, dD, dL), the
    per-head ones in fp32 (None where the input was None)."""
    B_, T, H, P = x.shape
    Lv = dl.shape[-1]
    dev = _lib.require_device(x, dt, dl, L, dv, dg, dlam, dy)
    x, dv = _aligned(x), _aligned(dv)
    dy = _aligned(dy) if D is not None else None
    dt, dl, L, dlam = _contig(dt), _contig(dl), _contig(L), _contig(dlam)
    dg = dg.float().contiguous()
    A = A.float().contiguous()
    bias = dt_bias.float().contiguous() if dt_bias is not None else None
    Df = D.float().contiguous() if D is not None else None
    dx = torch.empty(x.shape, dtype=x.dtype, device=dev)
    ddt = torch.empty(dt.shape, dtype=dt.dtype, device=dev)
    ddl = torch.empty(dl.shape, dtype=dl.dtype, device=dev)
    dA = torch.empty(H, dtype=torch.float32, device=dev)
    dbias = torch.empty(H, dtype=torch.float32, device=dev) if dt_bias is not None else None
    dD = torch.empty(H, dtype=torch.float32, device=dev) if D is not None else None
    dL = torch.empty(H, Lv, dtype=torch.float32, device=dev)
    lib = _lib.load()
    ws, ws_ptr, ws_bytes = _lib.workspace(lib.hattn_mamba2_layer_bwd_workspace(B_, T, H, Lv), dev)
    _lib.check(lib.hattn_mamba2_layer_bwd(
        _lib.ptr(x), _lib.ptr(dt), _lib.ptr(A), _lib.ptr(bias), _lib.ptr(dl), _lib.ptr(L),
        _lib.ptr(Df), _lib.ptr(dy), _lib.ptr(dv), _lib.ptr(dg), _lib.ptr(dlam), _lib.ptr(dx),
        _lib.ptr(ddt), _lib.ptr(ddl), _lib.ptr(dA), _lib.ptr(dbias), _lib.ptr(dD), _lib.ptr(dL),
        B_, T, H, P, Lv, int(bool(dt_softplus)), lambda_mode_code(lambda_mode),
        _code(x.dtype), _code(dt.dtype), _code(dl.dtype), _code(L.dtype),
        _code(dy.dtype) if dy is not None else 2, _code(dv.dtype), _code(dlam.dtype),
        _code(dx.dtype), _code(ddt.dtype), _code(ddl.dtype), ws_ptr, ws_bytes,
        _lib.stream_handle(dev)))
    return dx, ddt, ddl, dA, dbias, dD, dL


def layer_scan_folded(x, dt, A, Bc, Cc, dl, L, D, dt_bias, dt_softplus, lambda_mode, level_base,
                      htype):
    """The layer scan with the pre- and post-processing folded into the forward
    scan's loads and stores (``hattn_mamba2_layer_scan_fwd``): returns (y,
    g_cumsum), or None where that kernel does not apply (then the prologue ->
    chunkwise forward -> epilogue chain runs).  y has the dtype of that chain:
    C's (bf16) without D, torch's promotion of (C, x, D) with it."""
    from hattention.base import HType
    Bsz, T, H, P = x.shape
    G, N = Cc.shape[2], Cc.shape[3]
    Lv = dl.shape[-1]
    bf = torch.bfloat16
    if not (x.dtype == bf and Cc.dtype == bf and Bc.dtype == bf and N == 64 and P % 64 == 0
            and Lv <= 32 and htype == HType.WEAK and level_base == 2 and T % 64 == 0
            and Bc.shape == Cc.shape and dt.dtype in (bf, torch.float32)
            and dl.dtype in (bf, torch.float32)):
        return None
    if dt.shape != (Bsz, T, H) or dl.shape[:3] != (Bsz, T, H) or L.shape != (H, Lv) or \
            A.shape != (H,) or (dt_bias is not None and dt_bias.shape != (H,)):
        raise ValueError("shape mismatch in the layer pre-processing")
    dev = _lib.require_device(x, dt, A, dt_bias, dl, L, Bc, Cc, D)
    y_dtype = torch.promote_types(Cc.dtype, torch.promote_types(x.dtype, D.dtype)) \
        if D is not None else Cc.dtype
    lam_dtype = torch.promote_types(L.dtype, dl.dtype)
    x, dt, dl = x.contiguous(), dt.contiguous(), dl.contiguous()
    A32 = A.float().contiguous()
    bias = dt_bias.float().contiguous() if dt_bias is not None else None
    Lp = L.float().contiguous()
    Df = D.float().contiguous() if D is not None else None
    y = torch.empty(x.shape, dtype=y_dtype, device=dev)
    gcum = torch.empty(Bsz, T, H, dtype=torch.float32, device=dev)
    lib = _lib.load()
    ws, ws_ptr, ws_bytes = _lib.workspace(
        lib.hattn_mamba2_chunkwise_fwd_workspace(Bsz, T, G, H, N, P, Lv), dev)
    _lib.check(lib.hattn_mamba2_layer_scan_fwd(
        _lib.ptr(x), _lib.ptr(dt), _lib.ptr(A32), _lib.ptr(bias), _lib.ptr(Bc), _lib.ptr(Cc),
        _lib.ptr(dl), _lib.ptr(Lp), _lib.ptr(Df), _lib.ptr(y), _lib.ptr(gcum), Bsz, T, G, H, P, N,
        Lv, _code(x.dtype), _code(dt.dtype), _code(Cc.dtype), _code(dl.dtype), _code(lam_dtype),
        _code(y_dtype), int(bool(dt_softplus)), lambda_mode_code(lambda_mode), level_base,
        htype.value, 64, ws_ptr, ws_bytes, _lib.stream_handle(dev)))
    return y, gcum


class HMambaScanFunction(torch.autograd.Function):
    """The scan of hmamba_chunk_scan_combined (mamba_apis.py:346-403, MAMBA2,
    chunkwise, no final state) with its pre- and post-processing fused: one
    forward launch that folds the prologue into the scan's loads and the
    epilogue into its stores (``layer_scan_folded``), or prologue -> chunkwise
    forward (q = C, k = B) -> epilogue where that launch does not apply;
    backward: the prologue's v and lambda (recomputed when the folded forward
    did not write them) -> chunkwise backward -> layer backward.  Same
    gradients as torch autograd through the reference's expressions and
    HAttentionFunction."""

    @staticmethod
    def forward(ctx, x, dt, A, B, C, dl, L, D, dt_bias, dt_softplus, lambda_mode, level_base,
                htype):
        from hattention import chunkwise as _cw
        Cc, Bc = C.contiguous(), B.contiguous()
        ctx.cfg = (dt_softplus, lambda_mode, level_base, htype)
        folded = layer_scan_folded(x, dt, A, Bc, Cc, dl, L, D, dt_bias, dt_softplus, lambda_mode,
                                   level_base, htype)
        if folded is not None:
            y, gcum = folded
            ctx.save_for_backward(x, dt, A, Bc, Cc, dl, L, D, dt_bias, None, gcum, None)
            return y
        # v leaves the prologue in bf16 when the scan runs the bf16 kernels: they
        # round v to bf16 when they stage it for the MFMAs, so the forward values
        # are those of an fp32 v, at half its traffic (dv then comes back in bf16)
        v, g, lam = layer_prologue(x, dt, A, dt_bias, dl, L, dt_softplus, lambda_mode,
                                   v_dtype=torch.bfloat16 if C.dtype == torch.bfloat16 else None)
        o, gcum, _ = _cw.chunkwise_fwd(Cc, Bc, v, g, lam, False, level_base, htype, 64, False)
        y = o.to(C.dtype)
        if D is not None:
            y = layer_epilogue(y, x, D)
        ctx.save_for_backward(x, dt, A, Bc, Cc, dl, L, D, dt_bias, v, gcum, lam)
        return y

    @staticmethod
    def backward(ctx, dy):
        from hattention import chunkwise as _cw
        x, dt, A, Bc, Cc, dl, L, D, dt_bias, v, gcum, lam = ctx.saved_tensors
        dt_softplus, lambda_mode, level_base, htype = ctx.cfg
        if v is None:
            v, _, lam = layer_prologue(x, dt, A, dt_bias, dl, L, dt_softplus, lambda_mode,
                                       v_dtype=torch.bfloat16)
        do = dy.to(Cc.dtype).contiguous()
        dq, dk, dv, dg, dlam = _cw.chunkwise_bwd(Cc, Bc, v, gcum, lam, do, False, level_base,
                                                 htype, 64)
        dx, ddt, ddl, dA, dbias, dD, dL = layer_backward(
            x, dt, A, dt_bias, dl, L, D, dy, dv, dg, dlam, dt_softplus, lambda_mode)
        return (dx, ddt, dA.to(A.dtype), dk.to(Bc.dtype), dq.to(Cc.dtype), ddl, dL.to(L.dtype),
                dD.to(D.dtype) if D is not None else None,
                dbias.to(dt_bias.dtype) if dt_bias is not None else None,
                None, None, None, None)


# --------------------------------------------------------------------------
# hmamba_split_conv1d_scan_combined (mamba_apis.py:116-260): conv1d + SiLU of
# the xBC channels and the gated RMSNorm of the scan output
# --------------------------------------------------------------------------
class CausalConv1dSilu(torch.autograd.Function):
    """causal_conv1d_fn(xBC, weight, bias, activation="silu") of
    mamba_apis.py:206-213 on the column window [col0, col0 + Dc) of the packed
    rows of ``zx`` [B, S, width]; returns the contiguous x, B, C parts
    (channels [0, d1), [d1, d2), [d2, Dc)).  Backward: the window of the
    zx gradient (zeros elsewhere), dweight, dbias."""

    @staticmethod
    def forward(ctx, zx, col0, Dc, d1, d2, weight, bias):
        B_, S, width = zx.shape
        W = weight.shape[-1]
        dev = _lib.require_device(zx, weight, bias)
        zx = zx.contiguous()
        wt = weight.reshape(Dc, W).contiguous()
        bs = bias.contiguous() if bias is not None else None
        outs = [torch.empty(B_, S, n, dtype=zx.dtype, device=dev) for n in (d1, d2 - d1, Dc - d2)]
        _lib.check(_lib.load().hattn_causal_conv1d_silu_fwd(
            _lib.ptr(zx), width, col0, _lib.ptr(wt), _lib.ptr(bs), *(_lib.ptr(o) for o in outs),
            B_, S, Dc, d1, d2, W, _code(zx.dtype), _code(wt.dtype), _code(zx.dtype),
            _lib.stream_handle(dev)))
        ctx.save_for_backward(zx, wt, bs)
        ctx.cfg = (col0, Dc, d1, d2, weight.shape, bias is not None)
        return tuple(outs)

    @staticmethod
    def backward(ctx, g0, g1, g2):
        zx, wt, bs = ctx.saved_tensors
        col0, Dc, d1, d2, wshape, has_bias = ctx.cfg
        B_, S, width = zx.shape
        W = wt.shape[-1]
        dev = zx.device
        gs = []
        for g, n in ((g0, d1), (g1, d2 - d1), (g2, Dc - d2)):
            gs.append(g.contiguous() if g is not None else torch.zeros(B_, S, n, dtype=zx.dtype,
                                                                       device=dev))
        dzx = torch.zeros_like(zx)
        dw = torch.empty(Dc, W, dtype=torch.float32, device=dev)
        db = torch.empty(Dc, dtype=torch.float32, device=dev) if has_bias else None
        lib = _lib.load()
        ws, ws_ptr, ws_bytes = _lib.workspace(
            lib.hattn_causal_conv1d_silu_bwd_workspace(B_, S, Dc, W), dev)
        _lib.check(lib.hattn_causal_conv1d_silu_bwd(
            _lib.ptr(zx), width, col0, _lib.ptr(wt), _lib.ptr(bs), *(_lib.ptr(g) for g in gs),
            _lib.ptr(dzx), width, col0, _lib.ptr(dw), _lib.ptr(db), B_, S, Dc, d1, d2, W,
            _code(zx.dtype), _code(wt.dtype), *(_code(g.dtype) for g in gs), _code(dzx.dtype),
            ws_ptr, ws_bytes, _lib.stream_handle(dev)))
        return (dzx, None, None, None, None, dw.to(wt.dtype).reshape(wshape),
                db.to(bs.dtype) if db is not None else None)


class GatedRMSNorm(torch.autograd.Function):
    """rmsnorm_fn(y, weight, bias=None, z, eps, norm_before_gate=False) of
    mamba_apis.py:247-255 with z the column window [zcol0, zcol0 + n) of the
    packed rows of ``zx``: out = u / sqrt(mean(u^2) + eps) * weight, u = y silu(z),
    in y's dtype.  Backward: dy, the z window of the zx gradient, dweight."""

    @staticmethod
    def forward(ctx, y, zx, zcol0, weight, eps):
        B_, S, n = y.shape
        width = zx.shape[-1]
        dev = _lib.require_device(y, zx, weight)
        y, zx, w = y.contiguous(), zx.contiguous(), weight.contiguous()
        zv = zx.view(-1)[zcol0:]   # z row r starts at r * width
        out = torch.empty_like(y)
        rstd = torch.empty(B_ * S, dtype=torch.float32, device=dev)
        _lib.check(_lib.load().hattn_gated_rmsnorm_fwd(
            _lib.ptr(y), _lib.ptr(zv), width, _lib.ptr(w), _lib.ptr(out), _lib.ptr(rstd),
            B_ * S, n, float(eps), _code(y.dtype), _code(zx.dtype), _code(w.dtype),
            _code(out.dtype), _lib.stream_handle(dev)))
        ctx.save_for_backward(y, zx, w, rstd)
        ctx.zcol0 = zcol0
        return out

    @staticmethod
    def backward(ctx, dout):
        y, zx, w, rstd = ctx.saved_tensors
        zcol0 = ctx.zcol0
        B_, S, n = y.shape
        width = zx.shape[-1]
        dev = y.device
        dout = dout.contiguous()
        dy = torch.empty_like(y)
        dzx = torch.zeros_like(zx)
        dw = torch.empty(n, dtype=torch.float32, device=dev)
        lib = _lib.load()
        ws, ws_ptr, ws_bytes = _lib.workspace(lib.hattn_gated_rmsnorm_bwd_workspace(B_ * S, n), dev)
        _lib.check(lib.hattn_gated_rmsnorm_bwd(
            _lib.ptr(y), _lib.ptr(zx.view(-1)[zcol0:]), width, _lib.ptr(w), _lib.ptr(rstd),
            _lib.ptr(dout), _lib.ptr(dy), _lib.ptr(dzx.view(-1)[zcol0:]), width, _lib.ptr(dw),
            B_ * S, n, _code(y.dtype), _code(zx.dtype), _code(w.dtype), _code(dout.dtype),
            _code(dy.dtype), _code(dzx.dtype), ws_ptr, ws_bytes, _lib.stream_handle(dev)))
        return dy, dzx, None, dw.to(w.dtype), None

"""Autograd boundary of the chunkwise path (MI355X).

Mirrors hattention/kernel.py:32-374: ``HAttentionFunction`` (same forward
arguments, same saved tensors ``(q, k, v, b, g_cumsum, l, Aw, Au)``, same
return ``o.to(q.dtype)``, backward returning grads cast to the input dtypes
plus eight ``None``) and ``hattention_kernel`` (same signature and defaults).

Dispatch (kernel.py:55-123):
* MAMBA2 + chunkwise  -> ``chunkwise.chunkwise_fwd / chunkwise_bwd`` (HIP).
* GDELTA + chunkwise  -> ``chunkwise_hgdn.chunkwise_fwd / chunkwise_bwd`` (HIP),
  with q <- l2norm(q) * scale and k <- l2norm(k) (kernel.py:100-120).
* chunkwise=False (the non-chunkwise "parallel" path, parallel.py) is outside
  this build and raises NotImplementedError.
"""
import functools
from typing import Optional, Tuple

import torch

from hattention.base import HType, HStruct
from hattention import chunkwise as _cw


def input_guard(fn):
    """Make tensor arguments contiguous and run on their device (the role of
    fla.utils.input_guard at kernel.py:35, 138)."""
    @functools.wraps(fn)
    def wrapper(ctx, *args, **kwargs):
        args = [a.contiguous() if isinstance(a, torch.Tensor) else a for a in args]
        kwargs = {k: (v.contiguous() if isinstance(v, torch.Tensor) else v)
                  for k, v in kwargs.items()}
        dev = next((a.device for a in args if isinstance(a, torch.Tensor)), None)
        if dev is not None and dev.type == "cuda":
            with torch.cuda.device(dev):
                return fn(ctx, *args, **kwargs)
        return fn(ctx, *args, **kwargs)
    return wrapper


def l2norm_fwd(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """x / sqrt(||x||^2 + eps) over the last dim in fp32, cast back to x.dtype
    (fla.modules.l2norm.l2norm_fwd, used at kernel.py:20-23, 110-111)."""
    xf = x.float()
    return (xf * torch.rsqrt((xf * xf).sum(-1, keepdim=True) + eps)).to(x.dtype)


def l2norm_and_scale_fwd(x: torch.Tensor, scale: float) -> torch.Tensor:
    """kernel.py:20-23."""
    return l2norm_fwd(x) * scale


def l2norm_bwd(x: torch.Tensor, dy: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Gradient of y = x / sqrt(||x||^2 + eps): dx = r (dy - y (y . dy)), r =
    (||x||^2 + eps)^-1/2, in fp32, cast to x.dtype (fla.modules.l2norm.l2norm_bwd,
    used at kernel.py:24-29, 224-225)."""
    xf, dyf = x.float(), dy.float()
    r = torch.rsqrt((xf * xf).sum(-1, keepdim=True) + eps)
    y = xf * r
    return (r * (dyf - y * (y * dyf).sum(-1, keepdim=True))).to(x.dtype)


def l2norm_and_scale_bwd(x: torch.Tensor, dy: torch.Tensor, scale: float) -> torch.Tensor:
    """kernel.py:24-29: gradient of l2norm(x) * scale."""
    return l2norm_bwd(x, dy.float() * scale)


class HAttentionFunction(torch.autograd.Function):
    """kernel.py:32-244."""

    @staticmethod
    @input_guard
    def forward(ctx, q, k, v, b, g, l, scale, head_first, level_base, htype, hstruct,
                chunk_sizes, chunkwise, use_qk_l2norm_in_kernel):
        if hstruct == HStruct.MAMBA2 and chunkwise:
            if b is not None:
                raise ValueError
            if chunk_sizes[0] != chunk_sizes[1]:
                raise NotImplementedError
            if use_qk_l2norm_in_kernel:
                raise NotImplementedError
            if scale is not None:
                raise NotImplementedError
            o, g, _ = _cw.chunkwise_fwd(
                q=q, k=k, v=v, g=g, l=l, head_first=head_first, level_base=level_base,
                htype=htype, chunk_size=chunk_sizes[0], output_final_state=False)
            Aw = None
            Au = None
        elif hstruct == HStruct.GDELTA and chunkwise:
            if b is None:
                raise ValueError
            if chunk_sizes[0] != chunk_sizes[1]:
                raise NotImplementedError
            if not use_qk_l2norm_in_kernel:
                raise NotImplementedError
            if scale is None:
                raise NotImplementedError
            from hattention import chunkwise_hgdn as _hg
            g, o, Aw, Au, _ = _hg.chunkwise_fwd(
                q=l2norm_and_scale_fwd(q, scale=scale), k=l2norm_fwd(k), v=v, b=b, g=g, l=l,
                head_first=head_first, level_base=level_base, htype=htype,
                chunk_size=chunk_sizes[0], output_final_state=False)
        else:
            # MAMBA2 with chunkwise=False is the reference's parallel.py path.
            raise NotImplementedError("only the chunkwise path is implemented on MI355X")

        ctx.save_for_backward(q, k, v, b, g, l, Aw, Au)
        ctx.scale = scale
        ctx.dtype = g.dtype
        ctx.head_first = head_first
        ctx.level_base = level_base
        ctx.htype = htype
        ctx.hstruct = hstruct
        ctx.chunk_sizes = chunk_sizes
        ctx.chunkwise = chunkwise
        ctx.use_qk_l2norm_in_kernel = use_qk_l2norm_in_kernel
        return o.to(q.dtype)

    @staticmethod
    @input_guard
    def backward(ctx, do):
        q, k, v, b, g, l, Aw, Au = ctx.saved_tensors
        if ctx.hstruct == HStruct.MAMBA2 and ctx.chunkwise:
            if b is not None or Aw is not None or Au is not None:
                raise ValueError
            dq, dk, dv, dg, dl = _cw.chunkwise_bwd(
                q=q, k=k, v=v, g=g, l=l, do=do, head_first=ctx.head_first,
                level_base=ctx.level_base, htype=ctx.htype, chunk_size=ctx.chunk_sizes[0])
            db = None
        elif ctx.hstruct == HStruct.GDELTA and ctx.chunkwise:
            if b is None or Aw is None or Au is None:
                raise ValueError
            if ctx.chunk_sizes[0] != ctx.chunk_sizes[1]:
                raise NotImplementedError
            if not ctx.use_qk_l2norm_in_kernel:
                raise NotImplementedError
            if ctx.scale is None:
                raise NotImplementedError
            from hattention import chunkwise_hgdn as _hg
            dq, dk, dv, db, dg, dl = _hg.chunkwise_bwd(
                q=l2norm_and_scale_fwd(q, scale=ctx.scale), k=l2norm_fwd(k), v=v, b=b, g=g, l=l,
                Aw=Aw, Au=Au, do=do, head_first=ctx.head_first, level_base=ctx.level_base,
                htype=ctx.htype, chunk_size=ctx.chunk_sizes[0])
            dq = l2norm_and_scale_bwd(q, dq, scale=ctx.scale)
            dk = l2norm_bwd(k, dk)
        else:
            raise NotImplementedError
        return (dq.to(q), dk.to(k), dv.to(v), db.to(b) if b is not None else None,
                dg.to(ctx.dtype), dl.to(l), None, None, None, None, None, None, None, None)


def hattention_kernel(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    b: Optional[torch.Tensor],
    g: torch.Tensor,
    l: torch.Tensor,
    scale: Optional[float],
    head_first: bool,
    level_base: int,
    htype: HType,
    hstruct: HStruct,
    chunk_sizes: Optional[Tuple[int, int]] = None,
    chunkwise: bool = True,
    use_qk_l2norm_in_kernel: bool = False,
) -> torch.Tensor:
    """kernel.py:338-374."""
    if chunk_sizes is None:
        chunk_sizes = (64, 64)
    return HAttentionFunction.apply(q, k, v, b, g, l, scale, head_first, level_base, htype,
                                    hstruct, chunk_sizes, chunkwise, use_qk_l2norm_in_kernel)

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


# The reference decorates its autograd functions with fla.utils'
# autocast_custom_fwd / autocast_custom_bwd (kernel.py:36, 139, 251, 317), which
# are torch.amp.custom_fwd / custom_bwd for the GPU device without cast_inputs:
# under torch.autocast the forward records the autocast state and the backward
# runs in that same state; the inputs are not cast.
autocast_custom_fwd = functools.partial(torch.amp.custom_fwd, device_type="cuda")
autocast_custom_bwd = functools.partial(torch.amp.custom_bwd, device_type="cuda")


class HAttentionFunction(torch.autograd.Function):
    """kernel.py:32-244."""

    @staticmethod
    @input_guard
    @autocast_custom_fwd
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
            # the forward's workspace (its segment summaries) is kept for the backward
            o, g, _, ctx.fwd_ws = _cw.chunkwise_fwd_keep(
                q, k, v, g, l, head_first, level_base, htype, chunk_sizes[0], False)
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
            # q * scale / ||q|| and k / ||k|| are formed inside the kernels; the
            # forward's workspace (what the backward would recompute) is kept
            g, o, Aw, Au, _, ctx.fwd_ws = _hg.chunkwise_fwd_keep(
                q=q, k=k, v=v, b=b, g=g, l=l, head_first=head_first, level_base=level_base,
                htype=htype, chunk_size=chunk_sizes[0], output_final_state=False,
                qk_l2norm_scale=scale)
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
    @autocast_custom_bwd
    def backward(ctx, do):
        q, k, v, b, g, l, Aw, Au = ctx.saved_tensors
        if ctx.hstruct == HStruct.MAMBA2 and ctx.chunkwise:
            if b is not None or Aw is not None or Au is not None:
                raise ValueError
            dq, dk, dv, dg, dl = _cw.chunkwise_bwd(
                q=q, k=k, v=v, g=g, l=l, do=do, head_first=ctx.head_first,
                level_base=ctx.level_base, htype=ctx.htype, chunk_size=ctx.chunk_sizes[0],
                fwd_ws=ctx.fwd_ws)
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
            # the kernels normalise q, k and apply the l2norm chain rule to dq, dk
            dq, dk, dv, db, dg, dl = _hg.chunkwise_bwd(
                q=q, k=k, v=v, b=b, g=g, l=l, Aw=Aw, Au=Au, do=do, head_first=ctx.head_first,
                level_base=ctx.level_base, htype=ctx.htype, chunk_size=ctx.chunk_sizes[0],
                qk_l2norm_scale=ctx.scale, fwd_ws=ctx.fwd_ws)
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


# --------------------------------------------------------------------------
# prefill and decode (kernel.py:247-335, 377-633)
# --------------------------------------------------------------------------
class HAttentionPrefillFunction(torch.autograd.Function):
    """kernel.py:247-335: the chunkwise forward with its final level states;
    returns (o.to(q.dtype), ht [B, H, K, V, L] fp32).  No backward (as :318-335)."""

    @staticmethod
    @input_guard
    @autocast_custom_fwd
    def forward(ctx, q, k, v, b, g, l, scale, head_first, level_base, htype, hstruct, chunk_size,
                use_qk_l2norm_in_kernel):
        if hstruct == HStruct.MAMBA2:
            if b is not None:
                raise ValueError
            if use_qk_l2norm_in_kernel:
                raise NotImplementedError
            if scale is not None:
                raise NotImplementedError
            o, _, h = _cw.chunkwise_fwd(
                q=q, k=k, v=v, g=g, l=l, head_first=head_first, level_base=level_base,
                htype=htype, chunk_size=chunk_size, output_final_state=True)
        elif hstruct == HStruct.GDELTA:
            if b is None:
                raise ValueError
            if not use_qk_l2norm_in_kernel:
                raise NotImplementedError
            if scale is None:
                raise NotImplementedError
            from hattention import chunkwise_hgdn as _hg
            _, o, _, _, h = _hg.chunkwise_fwd(
                q=q, k=k, v=v, b=b, g=g, l=l, head_first=head_first, level_base=level_base,
                htype=htype, chunk_size=chunk_size, output_final_state=True,
                qk_l2norm_scale=scale)
        else:
            raise NotImplementedError
        if h is None:
            raise ValueError
        return o.to(q.dtype), h

    @staticmethod
    @autocast_custom_bwd
    def backward(ctx, do, dh):
        raise NotImplementedError


def _prefill_counts(T: int, L: int, level_base: int):
    """kernel.py:451-462: the level counts after a prefill of T tokens (one
    token at level 0, then greedily from the top level down, level e >= 1
    holding level_base^(e-1) tokens) and the levels left empty."""
    counts = [0] * L
    empty = []
    remainder = T - 1
    counts[0] = 1
    for level in range(L - 1, 0, -1):
        n = level_base ** (level - 1)
        if remainder >= n:
            remainder -= n
            counts[level] = n
        else:
            empty.append(level)
    if remainder != 0:
        raise ValueError
    return counts, empty


@torch.no_grad()
def postprocess_prefill_hstate_(hstate, q, k, v, b, g, l, scale, head_first, level_base, htype,
                                hstruct, chunk_size, use_qk_l2norm_in_kernel=False):
    """kernel.py:377-464: the chunkwise prefill leaves the levels >= level_chunk
    (7 for 64-token chunks) in ``hstate.states``; rebuild the levels below from
    the last chunk, then set the counts and clear the empty levels.

    MAMBA2: one ``hattn_mamba2_prefill_levels`` launch (the einsums of
    :418-436).  GDELTA: the recurrent form over the last chunk from a zero state
    (:438-449), one ``hattn_hstate_step`` launch per token."""
    from hattention.base import get_num_levels
    from hattention import _lib
    from hattention import recurrent as _rec
    if head_first:
        raise NotImplementedError
    B, T, G, K = k.shape
    _, _, H, V = v.shape
    _, _, _, L = l.shape
    if use_qk_l2norm_in_kernel:
        if scale is None:
            raise NotImplementedError
    elif scale is not None:
        raise NotImplementedError
    if chunk_size != 64 or T % chunk_size != 0 or T == 0:
        raise NotImplementedError("the prefill postprocess needs whole 64-token chunks")
    level_chunk = get_num_levels(chunk_size, level_base)
    _rec._check_state(hstate)
    if tuple(hstate.shape) != (B, H, K, V, L) or tuple(g.shape) != (B, T, H) or \
            v.shape[:2] != (B, T) or l.shape[:3] != (B, T, H) or H % G != 0:
        raise ValueError("shape mismatch between the HState and q, k, v, g, l")
    if L < level_chunk:
        raise ValueError(f"{L} levels, the prefill needs at least {level_chunk}")
    if hstruct == HStruct.MAMBA2:
        k, v, g = k.contiguous(), v.contiguous(), g.float().contiguous()
        dev = _lib.require_device(hstate.states, k, v, g)
        _lib.check(_lib.load().hattn_mamba2_prefill_levels(
            _lib.ptr(hstate.states), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), B, T, G, H, K, V,
            L, level_chunk, _lib.dtype_code(k), _lib.dtype_code(v), _lib.stream_handle(dev)))
    else:
        if b is None:
            raise ValueError
        tmp = _rec.HState(base=level_base, htype=htype, hstruct=hstruct,
                          shape=(B, H, K, V, level_chunk), dtype=hstate.dtype,
                          device=hstate.device)
        tm = lambda x: x[:, -chunk_size:].transpose(0, 1).contiguous()
        k_t, v_t, b_t, g_t = tm(k), tm(v), tm(b), tm(g.float())
        for t in range(chunk_size):
            _rec.launch_step(tmp, k=k_t[t], v=v_t[t], beta=b_t[t], g=g_t[t], update=True,
                             output=False, l2norm_qk=use_qk_l2norm_in_kernel, scale=scale)
        hstate.states[..., :level_chunk] = tmp.states
    counts, empty = _prefill_counts(T, L, level_base)
    if empty:
        hstate.states[..., empty] = 0
    hstate.set_counts(counts)
    return hstate


@torch.no_grad()
def hattention_prefill(q, k, v, b, g, l, scale, head_first, level_base, htype, hstruct,
                       chunk_size=None, use_qk_l2norm_in_kernel=False):
    """kernel.py:467-574: chunkwise forward over the whole 64-token chunks with
    the final level states, the low levels rebuilt from the last chunk, then one
    decode step per remaining token.  Returns (o, hstate)."""
    from hattention import recurrent as _rec
    if chunk_size is None:
        chunk_size = 64
    if head_first:
        raise NotImplementedError
    B, T, G, K = k.shape
    _, _, H, V = v.shape
    _, _, _, L = l.shape
    T0 = T - (T % chunk_size) if htype == HType.WEAK else 0
    o = torch.zeros_like(v)
    hstate = _rec.HState(base=level_base, htype=htype, hstruct=hstruct, shape=(B, H, K, V, L),
                         dtype=g.dtype, device=g.device)
    if T0 != 0:
        o[:, :T0], hstate.states = HAttentionPrefillFunction.apply(
            q[:, :T0], k[:, :T0], v[:, :T0], b[:, :T0] if b is not None else None, g[:, :T0],
            l[:, :T0], scale, head_first, level_base, htype, hstruct, chunk_size,
            use_qk_l2norm_in_kernel)
        postprocess_prefill_hstate_(
            hstate=hstate, q=q[:, :T0], k=k[:, :T0], v=v[:, :T0],
            b=b[:, :T0] if b is not None else None, g=g[:, :T0], l=l[:, :T0], scale=scale,
            head_first=head_first, level_base=level_base, htype=htype, hstruct=hstruct,
            chunk_size=chunk_size, use_qk_l2norm_in_kernel=use_qk_l2norm_in_kernel)
    if T0 < T:
        _check_step_args(hstate, q[:, T0], k[:, T0], v[:, T0],
                         b[:, T0] if b is not None else None, g[:, T0], l[:, T0], level_base,
                         htype, hstruct, use_qk_l2norm_in_kernel, scale)
        tm = lambda x: x[:, T0:].transpose(0, 1).contiguous() if x is not None else None
        q_t, k_t, v_t, b_t, g_t, l_t = tm(q), tm(k), tm(v), tm(b), tm(g), tm(l)
        o_t = torch.empty_like(v_t)
        for t in range(T - T0):
            _rec.launch_step(hstate, q=q_t[t], k=k_t[t], v=v_t[t],
                             beta=b_t[t] if b_t is not None else None, g=g_t[t], l=l_t[t],
                             o=o_t[t], update=True, output=True,
                             l2norm_qk=use_qk_l2norm_in_kernel, scale=scale)
        o[:, T0:] = o_t.transpose(0, 1)
    return o, hstate


def _check_step_args(hstate, q, k, v, b, g, l, level_base, htype, hstruct,
                     use_qk_l2norm_in_kernel, scale):
    """kernel.py:591-619: the argument checks of hattention_step."""
    if not all([q.ndim == 3, k.ndim == 3, v.ndim == 3, b.ndim == 2 if b is not None else True,
                g.ndim == 2, l.ndim == 3, g.dtype == hstate.dtype, q.dtype == k.dtype,
                q.dtype == v.dtype, q.dtype == l.dtype, hstate.base == level_base,
                hstate.htype == htype, hstate.hstruct == hstruct]):
        raise TypeError
    if use_qk_l2norm_in_kernel:
        if scale is None:
            raise NotImplementedError
    elif scale is not None:
        raise NotImplementedError
    if (hstruct == HStruct.MAMBA2) != (b is None):
        raise ValueError


@torch.no_grad()
def hattention_step(hstate, q, k, v, b, g, l, scale, level_base, htype, hstruct,
                    use_qk_l2norm_in_kernel=False):
    """kernel.py:577-633: one decode step, q, k [B, G, K], v [B, H, V], b, g
    [B, H], l [B, H, L]; returns (o [B, H, V] in v's dtype, hstate advanced in
    place).  One launch: l2norm of q and k (GDELTA), cascade, gate, insert and
    the output."""
    from hattention import recurrent as _rec
    _check_step_args(hstate, q, k, v, b, g, l, level_base, htype, hstruct,
                     use_qk_l2norm_in_kernel, scale)
    q, k, v, l, g = q.contiguous(), k.contiguous(), v.contiguous(), l.contiguous(), g.contiguous()
    b = b.contiguous() if b is not None else None
    o = torch.empty_like(v)
    _rec.launch_step(hstate, q=q, k=k, v=v, beta=b, g=g, l=l, o=o, update=True, output=True,
                     l2norm_qk=use_qk_l2norm_in_kernel, scale=scale)
    return o, hstate

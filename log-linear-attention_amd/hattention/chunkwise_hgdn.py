"""Host driver of the log-linear Gated DeltaNet chunkwise path (MI355X).

Same names, arguments and return tuples as hattention/chunkwise_hgdn.py:
* ``chunkwise_fwd(q, k, v, b, g, l, head_first, level_base, htype, chunk_size,
  output_final_state) -> (g_cumsum, o, Aw, Au, ht)``   -- chunkwise_hgdn.py:566-788
* ``chunkwise_bwd(q, k, v, b, g, l, Aw, Au, do, head_first, level_base, htype,
  chunk_size) -> (dq, dk, dv, db, dg, dl)``            -- chunkwise_hgdn.py:791-1222

Validation follows the reference (``ValueError`` for T % 64 and K / V not
multiples of the block options, ``NotImplementedError`` for K > 256 and level
bases other than 2).  ``HType.STRONG`` runs what the reference's chunkwise path
computes with the strong level table (chunkwise_hgdn.py:630, 724-728, 782):
lambda of an intra-chunk pair at its strong level, the inter-chunk levels
from 1 with the weak delta-rule states, and every chunk reading every level
>= 1; ``ht`` holds those states (level 7 stays zero).  Its backward returns
the gradient of that forward: the reference's own backward masks the level
reads as the weak hierarchy does (skip_q on dO, chunkwise_hgdn.py:1034,
1066-1067) and accumulates du on chunks whose u the forward masked
(chunk_bwd_kernel_dv without the skip_kv exit, chunkwise.py:1008-1012), so it
is not the derivative of its forward.  The backward kernels take K in {64, 128,
192, 256} (``NotImplementedError`` from the C-ABI otherwise) and V in blocks of
128.  Grouped q / k are expanded per head
before the kernels like the reference (chunkwise_hgdn.py:614-623) and their
gradients summed over the group (chunkwise_hgdn.py:1208-1215).  There is no
CPU path.
"""
from typing import Optional, Tuple

import torch

from hattention import _lib
from hattention.base import HType, get_num_levels, ceil_log

CHUNK = 64
VB = 128   # V columns per backward launch


def _validate(q, k, v, l, head_first, level_base, htype, chunk_size, **tensors):
    """chunkwise_hgdn.py:589-612 and :818-858: returns (B, T, G, H, K, V, L)."""
    if head_first:
        raise NotImplementedError("head_first=True is not supported (time-first layout only)")
    for name, t in dict(q=q, k=k, v=v, l=l, **tensors).items():
        if not t.is_contiguous():
            raise ValueError(f"Tensor argument {name} must be contiguous")
    B, T, G, K = k.shape
    _, _, H, V = v.shape
    L = l.shape[-1]
    # the kernels read q, k and v with one element type (dtype_qkv)
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError(f"q, k and v must share one dtype (got {q.dtype}, {k.dtype}, {v.dtype})")
    if H % G != 0:
        raise ValueError(f"H={H} is not a multiple of G={G}")
    if chunk_size != CHUNK:
        raise NotImplementedError(f"chunk_size={chunk_size} (only {CHUNK})")
    if level_base != 2:
        raise NotImplementedError("only level base 2 is supported")
    if htype not in (HType.WEAK, HType.STRONG):
        raise ValueError(f"htype={htype}")
    if K > 256:
        raise NotImplementedError("current kernel does not support head dimension larger than 256.")
    if T % CHUNK != 0 or T < CHUNK:
        raise ValueError(f"T={T} and BT={CHUNK}")
    for bs in (32, 64):
        if K % bs != 0:
            raise ValueError(f"K={K} and BK could be {bs}")
        if V % bs != 0:
            raise ValueError(f"V={V} and BV could be {bs}")
    if get_num_levels(CHUNK, level_base) + ceil_log(T // CHUNK, level_base) > L:
        raise ValueError(f"L={L} levels are too few for T={T}")
    return B, T, G, H, K, V, L


def _narrow_half(q, k, v, b, l, htype):
    """fp16 q / k / v with HType.WEAK run on kernels of their own (fp16 MFMA
    operands, fp16 o, gradients and saved states, as the reference's fp16 dots
    take them); those kernels read beta and lambda as fp32, so any 16-bit beta
    or lambda is widened (exact).  HType.STRONG has no fp16 kernels: fp16
    q / k / v are rounded to bf16 on the device (the reference's fp16 dots keep
    three more mantissa bits of the inputs), fp16 beta and lambda read as fp32.
    The caller returns the outputs and gradients in the inputs' dtypes."""
    half = torch.float16
    if q.dtype == half and htype == HType.WEAK:
        return q, k, v, b.float().contiguous(), l.float().contiguous()
    if q.dtype == half:
        q, k, v = (x.to(torch.bfloat16).contiguous() for x in (q, k, v))
    if b.dtype == half:
        b = b.float().contiguous()
    if l.dtype == half:
        l = l.float().contiguous()
    return q, k, v, b, l


def chunkwise_fwd(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    b: torch.Tensor,
    g: torch.Tensor,
    l: torch.Tensor,
    head_first: bool,
    level_base: int,
    htype: HType,
    chunk_size: int,
    output_final_state: bool,
    *,
    qk_l2norm_scale: Optional[float] = None,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    """Log-linear GDN forward; returns (g_cumsum, o, Aw, Au, ht) like the reference.

    ``qk_l2norm_scale`` (not in the reference's signature, default None = its
    behaviour): the kernels take raw q, k and use q * scale / ||q|| and
    k / ||k||, what HAttentionFunction computes before the reference's call
    (kernel.py:110-111), without a separate pass over q and k."""
    return chunkwise_fwd_keep(q, k, v, b, g, l, head_first, level_base, htype, chunk_size,
                              output_final_state, qk_l2norm_scale=qk_l2norm_scale,
                              keep=False)[:5]


def chunkwise_fwd_keep(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    b: torch.Tensor,
    g: torch.Tensor,
    l: torch.Tensor,
    head_first: bool,
    level_base: int,
    htype: HType,
    chunk_size: int,
    output_final_state: bool,
    *,
    qk_l2norm_scale: Optional[float] = None,
    keep: bool = True,
):
    """:func:`chunkwise_fwd` that also returns the forward's workspace, holding
    what the backward would recompute (q_new, W_new, K_new, U and every level's
    state at every chunk start, bit for bit), when the backward can take it
    (V in {64, 128}; else None): pass it to :func:`chunkwise_bwd` as ``fwd_ws``
    with the same inputs, and the backward skips its recompute
    (HAttentionFunction keeps it between its forward and backward).  Returns
    (g_cumsum, o, Aw, Au, ht, fwd_ws)."""
    B, T, G, H, K, V, L = _validate(q, k, v, l, head_first, level_base, htype, chunk_size,
                                    b=b, g=g)
    if g.dtype != torch.float32:
        raise ValueError("g (log-decay) must be float32")
    dev = _lib.require_device(q, k, v, b, g, l)
    o_dtype, k_dtype = v.dtype, k.dtype
    q, k, v, b, l = _narrow_half(q, k, v, b, l, htype)
    if G != H:
        q = q.repeat_interleave(H // G, dim=2).contiguous()
        k = k.repeat_interleave(H // G, dim=2).contiguous()
    o = torch.empty(v.shape, dtype=v.dtype, device=dev)
    g_cumsum = torch.empty(B, T, H, dtype=torch.float32, device=dev)
    Aw = torch.empty(B, T, H, CHUNK, dtype=k.dtype, device=dev)
    Au = torch.empty(B, T, H, CHUNK, dtype=k.dtype, device=dev)
    ht = torch.zeros(B, H, K, V, L, dtype=torch.float32, device=dev) if output_final_state else None
    lib = _lib.load()
    keep = keep and V in (64, VB)
    ws, ws_ptr, ws_bytes = _lib.workspace(
        (lib.hattn_gdn_chunkwise_fwd_keep_workspace if keep
         else lib.hattn_gdn_chunkwise_fwd_workspace)(B, T, H, K, V, L), dev)
    st = (lib.hattn_gdn_chunkwise_fwd_keep if keep else lib.hattn_gdn_chunkwise_fwd)(
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(b), _lib.ptr(g), _lib.ptr(l),
        _lib.ptr(o), _lib.ptr(g_cumsum), _lib.ptr(Aw), _lib.ptr(Au), _lib.ptr(ht),
        B, T, H, K, V, L, _lib.dtype_code(q), _lib.dtype_code(b), _lib.dtype_code(l),
        _lib.dtype_code(o), level_base, htype.value, chunk_size,
        1 if qk_l2norm_scale is not None else 0,
        float(qk_l2norm_scale) if qk_l2norm_scale is not None else 1.0, ws_ptr, ws_bytes,
        _lib.stream_handle(dev))
    _lib.check(st)
    if o_dtype != o.dtype:
        o, Aw, Au = o.to(o_dtype), Aw.to(k_dtype), Au.to(k_dtype)
    return g_cumsum, o, Aw, Au, ht, (ws if keep else None)


def chunkwise_bwd(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    b: torch.Tensor,
    g: torch.Tensor,
    l: torch.Tensor,
    Aw: torch.Tensor,
    Au: torch.Tensor,
    do: torch.Tensor,
    head_first: bool,
    level_base: int,
    htype: HType,
    chunk_size: int,
    *,
    qk_l2norm_scale: Optional[float] = None,
    fwd_ws: Optional[torch.Tensor] = None,
):
    """Log-linear GDN backward (chunkwise_hgdn.py:791-1222).

    ``fwd_ws`` (not in the reference): the workspace :func:`chunkwise_fwd_keep`
    returned for the same inputs; the backward then takes q_new, W_new, K_new,
    U and the level states from it instead of recomputing them (the same
    gradients, bit for bit).

    With ``qk_l2norm_scale`` (as in :func:`chunkwise_fwd`) q and k are the raw
    inputs and dq, dk come back w.r.t. them: the kernels apply the l2norm
    chain rule (kernel.py:24-29, 224-225) before storing them.

    ``g`` is the forward's chunk-local cumsum.  Returns (dq, dk, dv, db, dg, dl):
    dq / dk / dv / db in the dtypes of q / k / v / b, dg (w.r.t. the per-step g)
    and dl in fp32, like the reference.  ``Aw`` / ``Au`` are accepted for the
    reference's signature; the kernels recompute (I + A)^-1 in fp32.
    """
    B, T, G, H, K, V, L = _validate(q, k, v, l, head_first, level_base, htype, chunk_size,
                                    b=b, g=g, do=do)
    if g.dtype != torch.float32 or g.shape != (B, T, H):
        raise ValueError("g must be the fp32 chunk-local cumsum [B, T, H]")
    if do.shape != v.shape:
        raise ValueError("do must have the shape of v")
    dev = _lib.require_device(q, k, v, b, g, l, do)
    dtypes = (q.dtype, k.dtype, v.dtype, b.dtype)
    q, k, v, b, l = _narrow_half(q, k, v, b, l, htype)
    Aw, Au = Aw.to(k.dtype), Au.to(k.dtype)
    if G != H:
        q = q.repeat_interleave(H // G, dim=2).contiguous()
        k = k.repeat_interleave(H // G, dim=2).contiguous()
    do = do.to(v.dtype).contiguous()
    lib = _lib.load()
    # The gradients are sums over independent column blocks of V (each column of
    # o depends on its column of v only): the kernels take V in {64, 128}, so a
    # larger V runs block by block, dq / dk / db / dg / dl summed in fp32.
    blocks = [(v0, min(v0 + VB, V)) for v0 in range(0, V, VB)]
    dv = torch.empty_like(v)
    acc = None
    for v0, v1 in blocks:
        vb = v if len(blocks) == 1 else v[..., v0:v1].contiguous()
        dob = do if len(blocks) == 1 else do[..., v0:v1].contiguous()
        Vb = v1 - v0
        dq_b = torch.empty(B, T, H, K, dtype=q.dtype, device=dev)
        dk_b = torch.empty(B, T, H, K, dtype=k.dtype, device=dev)
        dv_b = dv if len(blocks) == 1 else torch.empty_like(vb)
        db_b = torch.empty_like(b)
        dg_b = torch.empty(B, T, H, dtype=torch.float32, device=dev)
        dl_b = torch.empty(B, T, H, L, dtype=torch.float32, device=dev)
        kept = fwd_ws is not None and len(blocks) == 1
        ws, ws_ptr, ws_bytes = _lib.workspace(
            (lib.hattn_gdn_chunkwise_bwd_fwd_ws_workspace if kept
             else lib.hattn_gdn_chunkwise_bwd_workspace)(B, T, H, K, Vb, L), dev)
        args = (
            _lib.ptr(q), _lib.ptr(k), _lib.ptr(vb), _lib.ptr(b), _lib.ptr(g), _lib.ptr(l),
            _lib.ptr(Aw), _lib.ptr(Au), _lib.ptr(dob), _lib.ptr(dq_b), _lib.ptr(dk_b),
            _lib.ptr(dv_b), _lib.ptr(db_b), _lib.ptr(dg_b), _lib.ptr(dl_b), B, T, H, K, Vb, L,
            _lib.dtype_code(q), _lib.dtype_code(b), _lib.dtype_code(l), _lib.dtype_code(dob),
            level_base, htype.value, chunk_size, 1 if qk_l2norm_scale is not None else 0,
            float(qk_l2norm_scale) if qk_l2norm_scale is not None else 1.0, ws_ptr, ws_bytes)
        if kept:
            st = lib.hattn_gdn_chunkwise_bwd_fwd_ws(*args, _lib.ptr(fwd_ws), fwd_ws.numel(),
                                                    _lib.stream_handle(dev))
        else:
            st = lib.hattn_gdn_chunkwise_bwd(*args, _lib.stream_handle(dev))
        _lib.check(st)
        del ws
        if len(blocks) == 1:
            dq, dk, db, dg, dl = dq_b, dk_b, db_b, dg_b, dl_b
            break
        dv[..., v0:v1] = dv_b
        parts = (dq_b.float(), dk_b.float(), db_b.float(), dg_b, dl_b)
        acc = parts if acc is None else tuple(a + p for a, p in zip(acc, parts))
    if acc is not None:
        dq, dk = acc[0].to(q.dtype), acc[1].to(k.dtype)
        db, dg, dl = acc[2].to(b.dtype), acc[3], acc[4]
    if G != H:
        dq = dq.view(B, T, G, H // G, K).sum(3, dtype=torch.float32).to(q.dtype)
        dk = dk.view(B, T, G, H // G, K).sum(3, dtype=torch.float32).to(k.dtype)
    dq, dk, dv, db = (x.to(d) for x, d in zip((dq, dk, dv, db), dtypes))
    return dq, dk, dv, db, dg, dl

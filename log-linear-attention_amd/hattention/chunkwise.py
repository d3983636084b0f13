"""Host drivers of the log-linear Mamba-2 chunkwise path (MI355X).

Same names, arguments and return tuples as hattention/chunkwise.py:
* ``chunkwise_fwd(q, k, v, g, l, head_first, level_base, htype, chunk_size,
  output_final_state) -> (o, g_cumsum, ht)``      -- chunkwise.py:1118-1275
* ``chunkwise_bwd(...)``                            -- chunkwise.py:1286-1597

Both validate like the reference (``ValueError`` for non-contiguous tensors,
T % 64, K/V multiples, too few levels; ``NotImplementedError`` for modes
outside the weak base-2 hierarchy), allocate the outputs with torch on the
inputs' device and launch the fused HIP kernels of libhattn_hip.so on the
current stream.  There is no CPU path.
"""
from typing import Optional, Tuple

import torch

from hattention import _lib
from hattention.base import HType, get_num_levels, ceil_log

CHUNK = 64


def _assert_contiguous(**tensors):
    """chunkwise.py:21-31 (assert_contiguous raises ValueError)."""
    for name, t in tensors.items():
        if isinstance(t, torch.Tensor) and not t.is_contiguous():
            raise ValueError(f"Tensor argument {name} must be contiguous")


def _shapes(q, k, v, l, head_first):
    if head_first:
        raise NotImplementedError("head_first=True is not supported (time-first layout only)")
    if q.dim() != 4 or k.shape != q.shape or v.dim() != 4 or l.dim() != 4:
        raise ValueError("expected q, k [B,T,G,K], v [B,T,H,V], l [B,T,H,L]")
    B, T, G, K = k.shape
    _, _, H, V = v.shape
    L = l.shape[-1]
    if v.shape[:2] != (B, T) or l.shape[:3] != (B, T, H):
        raise ValueError("batch / length / head mismatch")
    return B, T, G, H, K, V, L


def _validate(B, T, G, H, K, V, L, level_base, htype, chunk_size):
    """chunkwise.py:1140-1153 and :1211-1214."""
    if htype != HType.WEAK:
        raise NotImplementedError("HType.STRONG is outside the MI355X path")
    if level_base != 2:
        raise NotImplementedError("level_base must be 2")
    if chunk_size != CHUNK:
        raise NotImplementedError(f"chunk_size={chunk_size} (only {CHUNK})")
    if H % G != 0:
        raise ValueError(f"H={H} is not a multiple of G={G}")
    if T % CHUNK != 0 or T < CHUNK:
        raise ValueError(f"T={T} and BT={CHUNK}")
    for bs in (32, 64):
        if K % bs != 0:
            raise ValueError(f"K={K} and BK could be {bs}")
        if V % bs != 0:
            raise ValueError(f"V={V} and BV could be {bs}")
    NT = T // CHUNK
    if get_num_levels(CHUNK, level_base) + ceil_log(NT, level_base) > L:
        raise ValueError(f"L={L} levels are too few for T={T}")


def chunkwise_fwd(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    l: torch.Tensor,
    head_first: bool,
    level_base: int,
    htype: HType,
    chunk_size: int,
    output_final_state: bool,
) -> Tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    """Log-linear Mamba-2 forward (chunkwise.py:1118-1275).

    bf16 q / k multiply on bf16 MFMA; fp32 q / k select the bf16x3 kernels
    (each product as three bf16 MFMAs over hi / lo splits, fp32-accurate), the
    counterpart of the reference's fp32 dots.

    Returns ``o`` [B,T,H,V] in v.dtype, the chunk-local inclusive cumsum of g
    [B,T,H] fp32 and, if ``output_final_state``, ``ht`` [B,H,K,V,L] fp32 holding
    the inter-chunk level states at levels 7 .. 6 + ceil(log2(T/64)) (other
    levels zero), like the reference.
    """
    _assert_contiguous(q=q, k=k, v=v, g=g, l=l)
    B, T, G, H, K, V, L = _shapes(q, k, v, l, head_first)
    _validate(B, T, G, H, K, V, L, level_base, htype, chunk_size)
    if g.shape != (B, T, H):
        raise ValueError("g must be [B, T, H]")
    if g.dtype != torch.float32:
        raise ValueError("g (log-decay) must be float32")
    dev = _lib.require_device(q, k, v, g, l)
    if q.dtype != k.dtype:
        raise ValueError("q and k must share a dtype")
    out_dtype = v.dtype
    if q.dtype == torch.float32:
        # fp32 q / k run the bf16x3 (fp32-accurate) kernels, which read fp32 v
        # and lambda and write fp32 o
        v, l = v.float().contiguous(), l.float().contiguous()
    o = torch.empty(v.shape, dtype=v.dtype, device=dev)
    g_cumsum = torch.empty(g.shape, dtype=torch.float32, device=dev)
    ht = torch.zeros(B, H, K, V, L, dtype=torch.float32, device=dev) if output_final_state else None
    lib = _lib.load()
    ws, ws_ptr, ws_bytes = _lib.workspace(
        lib.hattn_mamba2_chunkwise_fwd_workspace(B, T, G, H, K, V, L), dev)
    st = lib.hattn_mamba2_chunkwise_fwd(
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), _lib.ptr(l), _lib.ptr(o),
        _lib.ptr(g_cumsum), _lib.ptr(ht), B, T, G, H, K, V, L,
        _lib.dtype_code(q), _lib.dtype_code(v), _lib.dtype_code(l), _lib.dtype_code(o),
        level_base, htype.value, chunk_size, ws_ptr, ws_bytes, _lib.stream_handle(dev))
    _lib.check(st)
    if o.dtype != out_dtype:
        o = o.to(out_dtype)
    return o, g_cumsum, ht


def chunkwise_bwd(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    l: torch.Tensor,
    do: torch.Tensor,
    head_first: bool,
    level_base: int,
    htype: HType,
    chunk_size: int,
):
    """Log-linear Mamba-2 backward (chunkwise.py:1286-1597).

    ``g`` is the chunk-local cumsum returned by :func:`chunkwise_fwd`.
    Returns (dq, dk, dv, dg, dl): dq / dk / dv in the dtypes of q / k / v,
    dg (w.r.t. the raw per-step g) and dl in fp32, like the reference.  Grouped
    q / k are expanded per head before the kernels and their gradients summed
    over the group afterwards (chunkwise.py:1360-1362, 1583-1594).
    """
    _assert_contiguous(q=q, k=k, v=v, g=g, l=l, do=do)
    B, T, G, H, K, V, L = _shapes(q, k, v, l, head_first)
    _validate(B, T, G, H, K, V, L, level_base, htype, chunk_size)
    if g.shape != (B, T, H) or g.dtype != torch.float32:
        raise ValueError("g must be the fp32 chunk-local cumsum [B, T, H]")
    if do.shape != v.shape:
        raise ValueError("do must have the shape of v")
    dev = _lib.require_device(q, k, v, g, l, do)
    if G != H:
        q = q.repeat_interleave(H // G, dim=2).contiguous()
        k = k.repeat_interleave(H // G, dim=2).contiguous()
    do = do.to(q.dtype).contiguous()
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    dg = torch.empty(B, T, H, dtype=torch.float32, device=dev)
    dl = torch.empty(B, T, H, L, dtype=torch.float32, device=dev)
    lib = _lib.load()
    ws, ws_ptr, ws_bytes = _lib.workspace(
        lib.hattn_mamba2_chunkwise_bwd_workspace(B, T, H, K, V, L), dev)
    st = lib.hattn_mamba2_chunkwise_bwd(
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), _lib.ptr(l), _lib.ptr(do),
        _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(dg), _lib.ptr(dl),
        B, T, H, K, V, L, _lib.dtype_code(q), _lib.dtype_code(v), _lib.dtype_code(l),
        _lib.dtype_code(do), level_base, htype.value, chunk_size, ws_ptr, ws_bytes,
        _lib.stream_handle(dev))
    _lib.check(st)
    if G != H:
        dq = dq.view(B, T, G, H // G, K).sum(3)
        dk = dk.view(B, T, G, H // G, K).sum(3)
    return dq, dk, dv, dg, dl

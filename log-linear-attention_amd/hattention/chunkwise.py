"""Host drivers of the log-linear Mamba-2 chunkwise path (MI355X).

Same names, arguments and return tuples as hattention/chunkwise.py:
* ``chunkwise_fwd(q, k, v, g, l, head_first, level_base, htype, chunk_size,
  output_final_state) -> (o, g_cumsum, ht)``      -- chunkwise.py:1118-1275
* ``chunkwise_bwd(...)``                            -- chunkwise.py:1286-1597

Both validate like the reference (``ValueError`` for non-contiguous tensors,
T % 64, K/V multiples, too few levels; ``NotImplementedError`` for modes
outside the base-2 weak and strong hierarchies), allocate the outputs with torch on the
inputs' device and launch the fused HIP kernels of libhattn_hip.so on the
current stream.  There is no CPU path.
"""
from typing import Optional, Tuple

import torch

from hattention import _lib
from hattention.base import HType, get_num_levels, ceil_log

CHUNK = 64
KB = 64   # key / value dimensions per kernel launch


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
    """chunkwise.py:1140-1153 and :1211-1214 (HType.WEAK and HType.STRONG)."""
    if htype not in (HType.WEAK, HType.STRONG):
        raise ValueError(f"htype={htype}")
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


def _native_half(q, k, v, l):
    """The fp16 path (HType.WEAK, forward and backward): fp16 q / k (and dO)
    multiply natively on fp16 MFMA, as the reference's fp16 dots do.  v stays
    fp16 (a bf16 v is read as fp32, exact), lambda is read as fp32 (exact for
    fp16 and bf16)."""
    if v.dtype == torch.bfloat16:
        v = v.float().contiguous()
    if l.dtype != torch.float32:
        l = l.float().contiguous()
    return q, k, v, l


def _widen_half(q, k, v, l):
    """Where there is no fp16 kernel (HType.STRONG): fp16 values
    are exact in fp32, so fp16 q / k run the fp32-accurate (bf16x3) kernels,
    and fp16 v or lambda next to bf16 q / k are read as fp32; the caller
    returns o and the gradients in the inputs' dtypes."""
    half = torch.float16
    if q.dtype == half:
        q, k = q.float().contiguous(), k.float().contiguous()
    if v.dtype == half:
        v = v.float().contiguous()
    if l.dtype == half:
        l = l.float().contiguous()
    return q, k, v, l


def _fwd_call(q, k, v, g, l, B, T, G, H, V, L, level_base, htype, chunk_size, ht, o_dtype):
    """One launch of hattn_mamba2_chunkwise_fwd (K = 64): returns (o, g_cumsum, workspace)."""
    dev = q.device
    o = torch.empty(v.shape, dtype=o_dtype, device=dev)
    g_cumsum = torch.empty(g.shape, dtype=torch.float32, device=dev)
    lib = _lib.load()
    ws, ws_ptr, ws_bytes = _lib.workspace(
        lib.hattn_mamba2_chunkwise_fwd_workspace(B, T, G, H, KB, V, L), dev)
    st = lib.hattn_mamba2_chunkwise_fwd(
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), _lib.ptr(l), _lib.ptr(o),
        _lib.ptr(g_cumsum), _lib.ptr(ht), B, T, G, H, KB, V, L,
        _lib.dtype_code(q), _lib.dtype_code(v), _lib.dtype_code(l), _lib.dtype_code(o),
        level_base, htype.value, chunk_size, ws_ptr, ws_bytes, _lib.stream_handle(dev))
    _lib.check(st)
    return o, g_cumsum, ws


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

    bf16 q / k multiply on bf16 MFMA, fp16 q / k on fp16 MFMA (HType.WEAK; the
    reference's fp16 dots); fp32 q / k select the bf16x3 kernels (each product
    as three bf16 MFMAs over hi / lo splits, fp32-accurate), the counterpart of
    the reference's fp32 dots.

    Returns ``o`` [B,T,H,V] in v.dtype, the chunk-local inclusive cumsum of g
    [B,T,H] fp32 and, if ``output_final_state``, ``ht`` [B,H,K,V,L] fp32 holding
    the inter-chunk level states at levels 7 .. 6 + ceil(log2(T/64)) (other
    levels zero), like the reference.

    HType.STRONG (bf16 q / k / v) runs the strong kernel: diagonal and
    sub-diagonal blocks from the strong level tables, farther chunks from a
    chunk-level strong cascade (chunkwise.py:199-276, 587-641).  Its final
    states are what the reference stores for the strong hierarchy: at level
    7 + ell, ell = 1 .. ceil(log2(T/64)) - 1, the raw phase-0 state of its
    strong state loop after the last chunk (chunkwise.py:179-279); level 7 and
    the intra-chunk levels stay zero.

    The kernels contract over 64 key dimensions.  A larger K (a multiple of 64)
    runs one launch per 64-wide block of q and k: the output is linear in that
    split (o = sum over blocks of the blocks' outputs, accumulated in fp32), and
    block i of the final states is the states' rows 64 i .. 64 i + 63.
    """
    return chunkwise_fwd_keep(q, k, v, g, l, head_first, level_base, htype, chunk_size,
                              output_final_state)[:3]


def chunkwise_fwd_keep(q, k, v, g, l, head_first, level_base, htype, chunk_size,
                       output_final_state):
    """:func:`chunkwise_fwd` that also returns the forward's workspace when the
    backward can reuse its segment summaries (bf16 q / k, K = V = 64, WEAK;
    else None): pass it to :func:`chunkwise_bwd` as ``fwd_ws`` with the same
    inputs (HAttentionFunction keeps it between its forward and backward)."""
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
    if q.dtype == torch.float16 and htype == HType.WEAK:
        q, k, v, l = _native_half(q, k, v, l)
    else:
        q, k, v, l = _widen_half(q, k, v, l)
    if q.dtype == torch.float32:
        # fp32 q / k run the bf16x3 (fp32-accurate) kernels, which read fp32 v
        # and lambda and write fp32 o
        v, l = v.float().contiguous(), l.float().contiguous()
    ht = torch.zeros(B, H, K, V, L, dtype=torch.float32, device=dev) if output_final_state else None
    keep = None
    if K == KB:
        o, g_cumsum, ws = _fwd_call(q, k, v, g, l, B, T, G, H, V, L, level_base, htype, chunk_size,
                                    ht, v.dtype)
        if V == KB and q.dtype == torch.bfloat16 and htype == HType.WEAK:
            keep = ws
    else:
        o = None
        for i in range(K // KB):
            blk = slice(KB * i, KB * (i + 1))
            hti = torch.zeros(B, H, KB, V, L, dtype=torch.float32, device=dev) if ht is not None else None
            oi, g_cumsum, _ = _fwd_call(q[..., blk].contiguous(), k[..., blk].contiguous(), v, g,
                                        l, B, T, G, H, V, L, level_base, htype, chunk_size, hti,
                                        torch.float32)
            o = oi if o is None else o.add_(oi)
            if ht is not None:
                ht[:, :, blk] = hti
    if o.dtype != out_dtype:
        o = o.to(out_dtype)
    return o, g_cumsum, ht, keep


def _bwd_call(q, k, v, g, l, do, B, T, H, V, L, level_base, htype, chunk_size, fwd_ws=None):
    """One launch of hattn_mamba2_chunkwise_bwd (K = V = 64, per-head q / k), or of
    hattn_mamba2_chunkwise_bwd_fwd_ws with the forward's workspace."""
    dev = q.device
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    dg = torch.empty(B, T, H, dtype=torch.float32, device=dev)
    dl = torch.empty(B, T, H, L, dtype=torch.float32, device=dev)
    lib = _lib.load()
    ws, ws_ptr, ws_bytes = _lib.workspace(
        lib.hattn_mamba2_chunkwise_bwd_workspace(B, T, H, KB, V, L, htype.value), dev)
    args = (_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), _lib.ptr(l), _lib.ptr(do),
            _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(dg), _lib.ptr(dl),
            B, T, H, KB, V, L, _lib.dtype_code(q), _lib.dtype_code(v), _lib.dtype_code(l),
            _lib.dtype_code(do), level_base, htype.value, chunk_size, ws_ptr, ws_bytes)
    if fwd_ws is None:
        st = lib.hattn_mamba2_chunkwise_bwd(*args, _lib.stream_handle(dev))
    else:
        st = lib.hattn_mamba2_chunkwise_bwd_fwd_ws(*args, _lib.ptr(fwd_ws), fwd_ws.numel(),
                                                   _lib.stream_handle(dev))
    _lib.check(st)
    return dq, dk, dv, dg, dl


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
    fwd_ws: Optional[torch.Tensor] = None,
):
    """Log-linear Mamba-2 backward (chunkwise.py:1286-1597).

    bf16 q / k run the bf16 MFMA kernels, fp16 q / k the same kernels on fp16
    MFMA (HType.WEAK); fp32 q / k the bf16x3 kernels (every
    product and every intermediate that feeds one as hi / lo bf16 planes,
    fp32-accurate), the counterpart of the reference's fp32 backward.

    ``g`` is the chunk-local cumsum returned by :func:`chunkwise_fwd`.
    Returns (dq, dk, dv, dg, dl): dq / dk / dv in the dtypes of q / k / v,
    dg (w.r.t. the raw per-step g) and dl in fp32, like the reference.  Grouped
    q / k are expanded per head before the kernels and their gradients summed
    over the group afterwards (chunkwise.py:1360-1362, 1583-1594).

    HType.STRONG (bf16 q / k / v / do) runs the strong backward kernels: chunk
    walks for the far levels (the forward's chunk-level strong cascade and its
    transpose in reverse order) and chunk-parallel diagonal / sub-diagonal
    blocks (chunkwise.py:1377-1580 with USE_A2 / USE_H2).

    ``fwd_ws`` (not in the reference): the workspace :func:`chunkwise_fwd_keep`
    returned for these inputs; its segment summaries replace the backward's own
    summary pass.  Used only where the forward kept it (bf16, K = V = 64, WEAK).

    The kernels take 64 key and 64 value dimensions.  Larger K and V (multiples
    of 64) run one launch per (key block, value block): with
    o_t = sum_s M[t,s] (q_t . k_s) v_s every gradient is a sum over those
    blocks (dq and dk of a key block sum over the value blocks, dv of a value
    block over the key blocks, dg and dlambda over all), accumulated in fp32.
    """
    _assert_contiguous(q=q, k=k, v=v, g=g, l=l, do=do)
    B, T, G, H, K, V, L = _shapes(q, k, v, l, head_first)
    _validate(B, T, G, H, K, V, L, level_base, htype, chunk_size)
    if g.shape != (B, T, H) or g.dtype != torch.float32:
        raise ValueError("g must be the fp32 chunk-local cumsum [B, T, H]")
    if do.shape != v.shape:
        raise ValueError("do must have the shape of v")
    _lib.require_device(q, k, v, g, l, do)
    if G != H:
        q = q.repeat_interleave(H // G, dim=2).contiguous()
        k = k.repeat_interleave(H // G, dim=2).contiguous()
    q_dtype, k_dtype, v_dtype = q.dtype, k.dtype, v.dtype
    if q.dtype == torch.float16 and htype == HType.WEAK:
        q, k, v, l = _native_half(q, k, v, l)
    else:
        q, k, v, l = _widen_half(q, k, v, l)
    do = do.to(q.dtype).contiguous()
    if q.dtype == torch.float32:
        # fp32 q / k run the bf16x3 (fp32-accurate) backward, which reads fp32 v,
        # lambda and dO and writes fp32 dq, dk, dv
        v, l = v.float().contiguous(), l.float().contiguous()
    if K == KB and V == KB:
        reuse = fwd_ws is not None and q.dtype == torch.bfloat16 and htype == HType.WEAK
        dq, dk, dv, dg, dl = _bwd_call(q, k, v, g, l, do, B, T, H, V, L, level_base, htype,
                                       chunk_size, fwd_ws if reuse else None)
    else:
        f32 = dict(dtype=torch.float32, device=q.device)
        dq = torch.zeros(B, T, H, K, **f32)
        dk = torch.zeros(B, T, H, K, **f32)
        dv = torch.zeros(B, T, H, V, **f32)
        dg = torch.zeros(B, T, H, **f32)
        dl = torch.zeros(B, T, H, L, **f32)
        kblocks = [slice(KB * i, KB * (i + 1)) for i in range(K // KB)]
        vblocks = [slice(KB * i, KB * (i + 1)) for i in range(V // KB)]
        vb = [(v[..., c].contiguous(), do[..., c].contiguous()) for c in vblocks]
        for kc in kblocks:
            qk = (q[..., kc].contiguous(), k[..., kc].contiguous())
            for c, (vc, doc) in zip(vblocks, vb):
                r = _bwd_call(qk[0], qk[1], vc, g, l, doc, B, T, H, KB, L, level_base, htype,
                              chunk_size)
                dq[..., kc] += r[0].float()
                dk[..., kc] += r[1].float()
                dv[..., c] += r[2].float()
                dg += r[3]
                dl += r[4]
        dq, dk, dv = dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype)
    dq, dk, dv = dq.to(q_dtype), dk.to(k_dtype), dv.to(v_dtype)
    if G != H:
        dq = dq.view(B, T, G, H // G, K).sum(3)
        dk = dk.view(B, T, G, H // G, K).sum(3)
    return dq, dk, dv, dg, dl

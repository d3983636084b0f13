"""Host driver of the log-linear Gated DeltaNet chunkwise path (MI355X).

Same name, arguments and return tuple as hattention/chunkwise_hgdn.py:
* ``chunkwise_fwd(q, k, v, b, g, l, head_first, level_base, htype, chunk_size,
  output_final_state) -> (g_cumsum, o, Aw, Au, ht)``   -- chunkwise_hgdn.py:566-788

Validation follows the reference (``ValueError`` for T % 64 and K / V not
multiples of the block options, ``NotImplementedError`` for K > 256 and modes
outside the weak base-2 hierarchy).  Grouped q / k are expanded per head
before the kernels like the reference (chunkwise_hgdn.py:614-623).  There is
no CPU path.  The GDN backward (chunkwise_hgdn.py:791-1222) is not part of
this build yet.
"""
from typing import Optional, Tuple

import torch

from hattention import _lib
from hattention.base import HType, get_num_levels, ceil_log

CHUNK = 64


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
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    """Log-linear GDN forward; returns (g_cumsum, o, Aw, Au, ht) like the reference."""
    if head_first:
        raise NotImplementedError("head_first=True is not supported (time-first layout only)")
    for name, t in dict(q=q, k=k, v=v, b=b, g=g, l=l).items():
        if not t.is_contiguous():
            raise ValueError(f"Tensor argument {name} must be contiguous")
    B, T, G, K = k.shape
    _, _, H, V = v.shape
    L = l.shape[-1]
    if H % G != 0:
        raise ValueError(f"H={H} is not a multiple of G={G}")
    if chunk_size != CHUNK:
        raise NotImplementedError(f"chunk_size={chunk_size} (only {CHUNK})")
    if level_base != 2 or htype != HType.WEAK:
        raise NotImplementedError("only the weak base-2 hierarchy is supported")
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
    if g.dtype != torch.float32:
        raise ValueError("g (log-decay) must be float32")
    dev = _lib.require_device(q, k, v, b, g, l)
    if G != H:
        q = q.repeat_interleave(H // G, dim=2).contiguous()
        k = k.repeat_interleave(H // G, dim=2).contiguous()
    o = torch.empty(v.shape, dtype=v.dtype, device=dev)
    g_cumsum = torch.empty(B, T, H, dtype=torch.float32, device=dev)
    Aw = torch.empty(B, T, H, CHUNK, dtype=k.dtype, device=dev)
    Au = torch.empty(B, T, H, CHUNK, dtype=k.dtype, device=dev)
    ht = torch.zeros(B, H, K, V, L, dtype=torch.float32, device=dev) if output_final_state else None
    lib = _lib.load()
    ws, ws_ptr, ws_bytes = _lib.workspace(
        lib.hattn_gdn_chunkwise_fwd_workspace(B, T, H, K, V, L), dev)
    st = lib.hattn_gdn_chunkwise_fwd(
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(b), _lib.ptr(g), _lib.ptr(l),
        _lib.ptr(o), _lib.ptr(g_cumsum), _lib.ptr(Aw), _lib.ptr(Au), _lib.ptr(ht),
        B, T, H, K, V, L, _lib.dtype_code(q), _lib.dtype_code(b), _lib.dtype_code(l),
        _lib.dtype_code(o), level_base, htype.value, chunk_size, ws_ptr, ws_bytes,
        _lib.stream_handle(dev))
    _lib.check(st)
    return g_cumsum, o, Aw, Au, ht


def hgdn_backward(*args, **kwargs):
    """chunkwise_hgdn.chunkwise_bwd (chunkwise_hgdn.py:791-1222): not built yet."""
    raise NotImplementedError("the MI355X log-linear GDN backward is not built yet")

"""hattn_mamba2_chunkwise_fwd_noalloc (static scratch, no workspace) against
hattn_mamba2_chunkwise_fwd (caller workspace): the same kernels on the same
inputs, so o, g_cumsum and ht must agree bit for bit.  Two calls in a row,
the second with a smaller input, so the second call runs on scratch the first
call left behind."""
import ctypes

import pytest
import torch

from bench import make_mamba2_inputs
from hattention import _lib


def _call(noalloc, q, k, v, g, l, final_state):
    B, T, G, K = q.shape
    H, V, L = v.shape[2], v.shape[3], l.shape[3]
    dev = q.device
    o = torch.empty_like(v)
    gc = torch.empty_like(g)
    ht = torch.zeros(B, H, K, V, L, dtype=torch.float32, device=dev) if final_state else None
    lib = _lib.load()
    args = [_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), _lib.ptr(l), _lib.ptr(o),
            _lib.ptr(gc), _lib.ptr(ht), B, T, G, H, K, V, L, _lib.dtype_code(q),
            _lib.dtype_code(v), _lib.dtype_code(l), _lib.dtype_code(o), 2, 0, 64]
    if noalloc:
        st = lib.hattn_mamba2_chunkwise_fwd_noalloc(*args, _lib.stream_handle(dev))
        ws = None
    else:
        ws, ws_ptr, ws_bytes = _lib.workspace(
            lib.hattn_mamba2_chunkwise_fwd_workspace(B, T, G, H, K, V, L), dev)
        st = lib.hattn_mamba2_chunkwise_fwd(*args, ws_ptr, ws_bytes, _lib.stream_handle(dev))
    _lib.check(st)
    torch.cuda.synchronize()
    del ws
    return o, gc, ht


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_matches_workspace_entry(dtype):
    dev = torch.device("cuda:0")
    # north-star-sized first call (16 segments, 4 top levels), then a smaller one
    for shape, final_state in (((4, 16384, 16, 64, 64, 15), True),
                               ((2, 4096, 4, 64, 128, 13), False)):
        B, T, H, K, V, L = shape
        if dtype == torch.float32:
            B = 1
        print(f"noalloc parity {dtype} B={B} T={T} H={H} K={K} V={V} L={L}", flush=True)
        ins = [x.to(dev) for x in make_mamba2_inputs(B, T, H, K, V, L, seed=77, dtype=dtype)]
        ref = _call(False, *ins, final_state)
        got = _call(True, *ins, final_state)
        for a, b in zip(ref, got):
            if a is None:
                assert b is None
                continue
            assert torch.equal(a, b), (shape, (a.float() - b.float()).abs().max().item())


@pytest.mark.gpu
def test_noalloc_rejects_sizes_beyond_static_scratch():
    # B=32 T=65536 H=32 V=64 needs well over 64 MiB of segment summaries
    # (placeholder tensor pointers: the capacity check fails before any HIP call)
    lib = _lib.load()
    dev = torch.device("cuda:0")
    p = ctypes.c_void_p(0x1000)
    need = lib.hattn_mamba2_chunkwise_fwd_workspace(32, 65536, 32, 32, 64, 64, 17)
    assert need > (64 << 20)
    st = lib.hattn_mamba2_chunkwise_fwd_noalloc(p, p, p, p, p, p, p, None, 32, 65536, 32, 32,
                                                64, 64, 17, 0, 0, 0, 0, 2, 0, 64,
                                                _lib.stream_handle(dev))
    assert st == _lib.HATTN_ERR_VALUE
    assert b"static scratch" in lib.hattn_last_error()

"""The fused forward's look-back fails loudly.

The single-pass bf16 forward waits, with a bounded poll, for the segment
summaries that earlier workgroups publish.  If a wait gives up (a lost flag,
or two calls overlapping on one workspace), the kernel sets bit 0 of the
status word in its workspace and writes NaN over that workgroup's o,
g_cumsum and ht.  These tests force the condition from the host through the
library's test hook (hattn_debug_lookback: a short poll limit, and phase A
publishing no flags), so every kernel still runs to completion: segment 0
(which waits for nothing) is computed as usual, every later segment comes
back as NaN, and the status word reports the timeout.  A normal run on the
same sizes reports status 0 and matches the oracle.
"""
import pytest
import torch

from bench import make_mamba2_inputs
from hattention import _lib
from oracle.mamba2 import chunked_scan_fwd

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _call(q, k, v, g, l, final_state):
    B, T, G, K = q.shape
    H, V, L = v.shape[2], v.shape[3], l.shape[3]
    o = torch.empty_like(v)
    gc = torch.empty_like(g)
    ht = torch.zeros(B, H, K, V, L, dtype=torch.float32, device=DEV) if final_state else None
    lib = _lib.load()
    ws, ws_ptr, ws_bytes = _lib.workspace(
        lib.hattn_mamba2_chunkwise_fwd_workspace(B, T, G, H, K, V, L), DEV)
    st = lib.hattn_mamba2_chunkwise_fwd(
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), _lib.ptr(l), _lib.ptr(o),
        _lib.ptr(gc), _lib.ptr(ht), B, T, G, H, K, V, L, _lib.dtype_code(q), _lib.dtype_code(v),
        _lib.dtype_code(l), _lib.dtype_code(o), 2, 0, 64, ws_ptr, ws_bytes,
        _lib.stream_handle(DEV))
    _lib.check(st)
    status = _lib.fwd_status(ws, B, T, H, V, DEV)
    return o, gc, ht, status


def test_lookback_timeout_poisons_and_reports():
    B, T, H, K, V, L = 1, 4096, 2, 64, 64, 13   # four 16-chunk segments
    ins = [x.to(DEV) for x in make_mamba2_inputs(B, T, H, K, V, L, seed=404)]
    lib = _lib.load()
    print(f"[lookback] forced timeout B={B} T={T} H={H}", flush=True)
    lib.hattn_debug_lookback(64, 0)
    try:
        o_bad, gc_bad, ht_bad, st_bad = _call(*ins, final_state=True)
    finally:
        lib.hattn_debug_lookback(0, 1)
    print(f"[lookback] normal run B={B} T={T} H={H}", flush=True)
    o, gc, ht, st = _call(*ins, final_state=True)
    assert st_bad & 1, st_bad
    assert st == 0, st
    seg = 16 * 64
    # segment 0 waits for nothing: computed as in the normal run
    assert torch.equal(o_bad[:, :seg], o[:, :seg])
    assert torch.equal(gc_bad[:, :seg], gc[:, :seg])
    # every later segment's outputs are NaN, and so are the final states
    assert torch.isnan(o_bad[:, seg:].float()).all()
    assert torch.isnan(gc_bad[:, seg:]).all()
    nlev = 6
    assert torch.isnan(ht_bad[..., 7:7 + nlev]).all()
    # the normal run is right
    q, k, v, g, l = (x.cpu() for x in ins)
    ref = chunked_scan_fwd(*(x.double() for x in (q, k, v, g, l)), chunk_size=64)[0]
    err = ((o.double().cpu() - ref).abs().max() / ref.abs().max()).item()
    assert err < 2e-2, err
    assert torch.isfinite(ht).all()


def test_status_word_clear_at_north_star():
    B, T, H, K, V, L = 4, 16384, 16, 64, 64, 15
    ins = [x.to(DEV) for x in make_mamba2_inputs(B, T, H, K, V, L, seed=405)]
    print(f"[lookback] status at B={B} T={T} H={H}", flush=True)
    for _ in range(3):
        o, gc, ht, st = _call(*ins, final_state=False)
        assert st == 0
        assert torch.isfinite(o.float()).all()

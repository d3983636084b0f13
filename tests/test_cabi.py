"""The C-ABI library loads and exports every entry point include/hattn.h declares.

CPU-only: no compute call is made.  The argument checks of the entry points
run on the host before any HIP call, so invalid shapes are exercised here and
must come back as the status codes that the Python layer maps to the
reference's exception types (chunkwise.py:1140-1153, 1211-1214).
"""
import ctypes
import os
import re
import subprocess

import pytest

from hattention import _lib


def gpu_visible() -> bool:
    import torch
    return torch.cuda.is_available()

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hattn.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hattn_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert "hattn_mamba2_chunkwise_fwd" in syms
    assert "hattn_version" in syms and "hattn_last_error" in syms


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\b(hattn_[a-z0-9_]+)\b", out))
    for s in declared_symbols():
        assert s in exported, s
        assert getattr(lib, s) is not None


def test_binding_table_covers_header():
    bound = {name for name, _, _ in _lib.SIGNATURES}
    assert set(declared_symbols()) <= bound


def test_workspace_query():
    lib = _lib.load()
    # one segment (T <= 31 chunks): no scratch; otherwise rows * segments * K * V fp32 + decays
    assert lib.hattn_mamba2_chunkwise_fwd_workspace(1, 64 * 16, 1, 1, 64, 64, 11) == 0
    n = lib.hattn_mamba2_chunkwise_fwd_workspace(4, 16384, 16, 16, 64, 64, 15)
    assert n >= 4 * 16 * 16 * 64 * 64 * 4
    assert lib.hattn_mamba2_chunkwise_fwd_workspace(1, 100, 1, 1, 64, 64, 8) == 0


@pytest.mark.skipif(gpu_visible(), reason="passes placeholder device pointers; host-only check")
def test_workspace_too_small_is_value_error():
    # the workspace check comes after the null-pointer check, so this case needs
    # non-null placeholders; it runs only where no GPU could be reached
    assert _fwd(T=64 * 64, L=13, ptr=0x1000) == _lib.HATTN_ERR_VALUE
    assert b"workspace" in _lib.load().hattn_last_error()


def test_null_tensor_is_value_error():
    assert _fwd() == _lib.HATTN_ERR_VALUE
    assert b"null" in _lib.load().hattn_last_error()


def test_span_above_32bit_range_is_not_implemented():
    # B=1, T=262144, H=64, V=64 fp32 v: one batch's v slice is 4 GiB, beyond the
    # 32-bit byte range of the kernels' buffer descriptors
    assert _fwd(T=262144, H=64, G=64, L=19, dv=2) == _lib.HATTN_ERR_NOT_IMPLEMENTED
    assert b"4 GiB" in _lib.load().hattn_last_error()
    # one element type smaller keeps it below the limit (fails later, on the null pointers)
    assert _fwd(T=262144, H=64, G=64, L=19) == _lib.HATTN_ERR_VALUE


def test_version_string():
    v = _lib.load().hattn_version().decode()
    assert v.startswith("hattn-mi355x") and "gfx950" in v


def _fwd(ptr=None, **kw):
    """Calls the forward with NULL tensor pointers (or placeholders when ptr is
    given): every case fails in the host-side validation, before any HIP call."""
    a = dict(B=1, T=128, G=1, H=1, K=64, V=64, L=8, dq=0, dv=0, dl=0, do=0, base=2, htype=0,
             chunk=64)
    a.update(kw)
    lib = _lib.load()
    p = ctypes.c_void_p(ptr)
    return lib.hattn_mamba2_chunkwise_fwd(p, p, p, p, p, p, None, None, a["B"], a["T"], a["G"],
                                          a["H"], a["K"], a["V"], a["L"], a["dq"], a["dv"],
                                          a["dl"], a["do"], a["base"], a["htype"], a["chunk"],
                                          None, 0, None)


@pytest.mark.parametrize("kw,code", [
    (dict(T=100), _lib.HATTN_ERR_VALUE),            # T % 64
    (dict(T=0), _lib.HATTN_ERR_VALUE),
    (dict(H=3, G=2), _lib.HATTN_ERR_VALUE),         # G does not divide H
    (dict(L=7), _lib.HATTN_ERR_VALUE),              # L < 7 + ceil(log2(T/64))
    (dict(V=40), _lib.HATTN_ERR_VALUE),
    (dict(chunk=32), _lib.HATTN_ERR_NOT_IMPLEMENTED),
    (dict(base=3), _lib.HATTN_ERR_NOT_IMPLEMENTED),
    (dict(htype=2), _lib.HATTN_ERR_VALUE),          # neither WEAK nor STRONG
    (dict(htype=1, dq=2, dv=2, dl=2, do=2), _lib.HATTN_ERR_NOT_IMPLEMENTED),  # STRONG: bf16 q/k/v
    (dict(htype=1, T=64 << 10, L=20), _lib.HATTN_ERR_NOT_IMPLEMENTED),  # STRONG: > 9 chunk levels
    (dict(K=128), _lib.HATTN_ERR_NOT_IMPLEMENTED),
    (dict(dq=1), _lib.HATTN_ERR_NOT_IMPLEMENTED),   # fp16 q/k
    (dict(dq=2), _lib.HATTN_ERR_NOT_IMPLEMENTED),   # fp32 q/k (bf16x3) with bf16 v, lambda, o
    (dict(dq=2, dv=2, dl=2, do=2, T=64 << 11, L=20), _lib.HATTN_ERR_NOT_IMPLEMENTED),  # > fp32 levels
])
def test_fwd_argument_checks(kw, code):
    assert _fwd(**kw) == code
    msg = _lib.load().hattn_last_error().decode()
    assert msg


def _bwd_fwd_ws(htype=0, dq=0):
    """hattn_mamba2_chunkwise_bwd_fwd_ws with NULL tensors and a NULL forward
    workspace: both fail on the host before any HIP call."""
    lib = _lib.load()
    nul = ctypes.c_void_p(None)
    return lib.hattn_mamba2_chunkwise_bwd_fwd_ws(
        *([nul] * 11), 1, 4096, 1, 64, 64, 13, dq, 0, 0, dq, 2, htype, 64, None, 0, None, 0,
        None)


def test_bwd_forward_workspace_checks():
    # no forward workspace -> ValueError, checked before the htype and dtype rules
    assert _bwd_fwd_ws() == _lib.HATTN_ERR_VALUE
    assert b"forward workspace" in _lib.load().hattn_last_error()
    assert _bwd_fwd_ws(htype=1) == _lib.HATTN_ERR_VALUE


def test_status_maps_to_reference_exceptions():
    lib = _lib.load()
    assert _fwd(T=100) == _lib.HATTN_ERR_VALUE
    with pytest.raises(ValueError):
        _lib.check(_lib.HATTN_ERR_VALUE)
    assert _fwd(chunk=32) == _lib.HATTN_ERR_NOT_IMPLEMENTED
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.HATTN_ERR_NOT_IMPLEMENTED)
    assert lib.hattn_last_error() is not None


def _bwd(**kw):
    """Mamba-2 backward with NULL tensor pointers: every case fails in the
    host-side validation, before any HIP call."""
    a = dict(B=1, T=128, H=1, K=64, V=64, L=8, dq=0, dv=0, dl=0, do=0, base=2, htype=0,
             chunk=64, ws=1 << 30)
    a.update(kw)
    lib = _lib.load()
    p = ctypes.c_void_p(None)
    return lib.hattn_mamba2_chunkwise_bwd(p, p, p, p, p, p, p, p, p, p, p, a["B"], a["T"], a["H"],
                                          a["K"], a["V"], a["L"], a["dq"], a["dv"], a["dl"],
                                          a["do"], a["base"], a["htype"], a["chunk"], p, a["ws"],
                                          None)


@pytest.mark.parametrize("kw,code", [
    (dict(T=100), _lib.HATTN_ERR_VALUE),            # T % 64
    (dict(L=7), _lib.HATTN_ERR_VALUE),              # L < 7 + ceil(log2(T/64))
    (dict(K=96), _lib.HATTN_ERR_VALUE),             # K, V multiples of 64
    (dict(K=128), _lib.HATTN_ERR_NOT_IMPLEMENTED),  # one 64-wide block per call
    (dict(htype=2), _lib.HATTN_ERR_VALUE),          # neither WEAK nor STRONG
    (dict(htype=1, dq=2, dv=2, dl=2, do=2), _lib.HATTN_ERR_NOT_IMPLEMENTED),  # STRONG: bf16
    (dict(htype=1, T=64 << 10, L=20), _lib.HATTN_ERR_NOT_IMPLEMENTED),  # STRONG: > 9 levels
    (dict(htype=1), _lib.HATTN_ERR_VALUE),          # STRONG, valid: fails on the null pointers
    (dict(), _lib.HATTN_ERR_VALUE),                 # WEAK, valid: fails on the null pointers
])
def test_bwd_argument_checks(kw, code):
    assert _bwd(**kw) == code
    assert _lib.load().hattn_last_error().decode()


def test_fwd_workspace_query_covers_strong_block_sums():
    """The forward's workspace query covers HType.STRONG's segment-parallel
    walks: per row, per 32-chunk segment but the last, seven fp32 64 x V block
    sums (six blocks and the whole segment), plus a log-decay per segment;
    none when the sequence is one segment."""
    lib = _lib.load()
    for B, T, H, V in ((4, 16384, 16, 64), (1, 4096, 2, 128), (2, 32768, 3, 64)):
        nseg = (T // 64 + 31) // 32
        need = B * H * (nseg - 1) * 7 * 64 * V * 4
        assert lib.hattn_mamba2_chunkwise_fwd_workspace(B, T, H, H, 64, V, 20) >= need
    # the north star's block sums fit the no-allocation entry point's 64 MiB
    assert 4 * 16 * 7 * 7 * 64 * 64 * 4 < (64 << 20)


def test_bwd_workspace_query_per_htype():
    lib = _lib.load()
    assert lib.hattn_mamba2_chunkwise_bwd_workspace(1, 100, 1, 64, 64, 8, 0) == 0
    weak = lib.hattn_mamba2_chunkwise_bwd_workspace(2, 4096, 4, 64, 64, 13, 0)
    strong = lib.hattn_mamba2_chunkwise_bwd_workspace(2, 4096, 4, 64, 64, 13, 1)
    assert weak > 0 and strong > 0 and weak != strong
    # the strong workspace holds at least the fp32 far dq and the bf16 adjoint tiles
    assert strong >= 2 * 4096 * 4 * 64 * (4 + 2)


def _gdn_bwd(**kw):
    """NULL tensor pointers: every case fails in the host-side validation, before
    any HIP call (the workspace case on the null check or the size check)."""
    a = dict(B=1, T=128, H=1, K=64, V=64, L=8, dq=0, db=0, dl=0, do=0, base=2, htype=0,
             chunk=64, ws=1 << 30)
    a.update(kw)
    lib = _lib.load()
    p = ctypes.c_void_p(None)
    return lib.hattn_gdn_chunkwise_bwd(p, p, p, p, p, p, None, None, p, p, p, p, p, p, p,
                                       a["B"], a["T"], a["H"], a["K"], a["V"], a["L"], a["dq"],
                                       a["db"], a["dl"], a["do"], a["base"], a["htype"],
                                       a["chunk"], 0, 1.0, p, a["ws"], None)


@pytest.mark.parametrize("kw,code", [
    (dict(T=100), _lib.HATTN_ERR_VALUE),            # T % 64
    (dict(L=7), _lib.HATTN_ERR_VALUE),              # L < 7 + ceil(log2(T/64))
    (dict(K=96, V=96), _lib.HATTN_ERR_VALUE),       # K, V multiples of 64
    (dict(K=320, V=64), _lib.HATTN_ERR_NOT_IMPLEMENTED),   # K > 256
    (dict(K=256, V=64), _lib.HATTN_ERR_VALUE),      # K = 256 valid: fails on the null pointers
    (dict(K=64, V=192), _lib.HATTN_ERR_NOT_IMPLEMENTED),   # V blocks of 64 / 128
    (dict(chunk=32), _lib.HATTN_ERR_NOT_IMPLEMENTED),
    (dict(htype=1), _lib.HATTN_ERR_VALUE),          # STRONG valid: fails on the null pointers
    (dict(htype=2), _lib.HATTN_ERR_VALUE),          # neither WEAK nor STRONG
    (dict(do=2), _lib.HATTN_ERR_NOT_IMPLEMENTED),   # do must be bf16
    (dict(dq=1, do=0), _lib.HATTN_ERR_NOT_IMPLEMENTED),  # fp16 q/k/v need an fp16 do
    (dict(dq=1, do=1), _lib.HATTN_ERR_VALUE),       # fp16 valid: fails on the null pointers
    (dict(dq=2, do=2), _lib.HATTN_ERR_NOT_IMPLEMENTED),  # no fp32 q/k/v kernels
    (dict(T=64 << 9, L=17), _lib.HATTN_ERR_NOT_IMPLEMENTED),  # > 8 inter-chunk levels
    (dict(ws=16), _lib.HATTN_ERR_VALUE),            # workspace too small
])
def test_gdn_bwd_argument_checks(kw, code):
    assert _gdn_bwd(**kw) == code
    assert _lib.load().hattn_last_error().decode()


def test_gdn_bwd_workspace_query():
    lib = _lib.load()
    assert lib.hattn_gdn_chunkwise_bwd_workspace(1, 100, 1, 64, 64, 8) == 0
    small = lib.hattn_gdn_chunkwise_bwd_workspace(1, 1024, 2, 64, 64, 11)
    big = lib.hattn_gdn_chunkwise_bwd_workspace(1, 2048, 2, 64, 64, 12)
    assert 0 < small < big


def test_gdn_keep_workspace_queries():
    lib = _lib.load()
    args = (2, 2048, 4, 128, 128, 12)
    fwd = lib.hattn_gdn_chunkwise_fwd_workspace(*args)
    keep = lib.hattn_gdn_chunkwise_fwd_keep_workspace(*args)
    bwd = lib.hattn_gdn_chunkwise_bwd_workspace(*args)
    kept = lib.hattn_gdn_chunkwise_bwd_fwd_ws_workspace(*args)
    # the keeping forward holds at least every level's state per chunk (bf16)
    B, T, H, K, V, L = args
    assert keep >= fwd + B * H * (T // 64) * 5 * V * K * 2
    assert 0 < kept < bwd
    assert lib.hattn_gdn_chunkwise_fwd_keep_workspace(1, 100, 1, 64, 64, 8) == 0
    assert lib.hattn_gdn_chunkwise_bwd_fwd_ws_workspace(1, 100, 1, 64, 64, 8) == 0


def test_gdn_keep_forward_argument_checks():
    lib = _lib.load()
    p = ctypes.c_void_p(None)

    def call(V, ws=1 << 30):
        return lib.hattn_gdn_chunkwise_fwd_keep(p, p, p, p, p, p, p, p, p, p, p, 1, 256, 2, 64,
                                                V, 9, 0, 0, 0, 0, 2, 0, 64, 0, 1.0, p, ws, None)
    # the kept buffers serve a backward in one V block
    assert call(192) == _lib.HATTN_ERR_NOT_IMPLEMENTED
    assert "V=192" in lib.hattn_last_error().decode()
    assert call(128) == _lib.HATTN_ERR_VALUE   # valid shape: fails on the null pointers


def test_gdn_forward_dtype_codes():
    """q/k/v dtype codes the GDN forward takes: bf16 and fp16 (fp16 with fp32
    beta / lambda, fp16 o and HType.WEAK is checked at dispatch, after the null
    pointer check); fp32 has no kernels."""
    lib = _lib.load()
    p = ctypes.c_void_p(None)

    def call(dt_qkv):
        return lib.hattn_gdn_chunkwise_fwd(p, p, p, p, p, p, p, p, p, p, p, 1, 256, 2, 64, 64, 9,
                                           dt_qkv, 2, 2, dt_qkv, 2, 0, 64, 0, 1.0, p, 1 << 30,
                                           None)
    assert call(0) == _lib.HATTN_ERR_VALUE
    assert call(1) == _lib.HATTN_ERR_VALUE
    assert call(2) == _lib.HATTN_ERR_NOT_IMPLEMENTED
    assert "bf16 or fp16" in lib.hattn_last_error().decode()


def test_gdn_kept_backward_argument_checks():
    """Placeholder (never dereferenced) tensor pointers: the forward-workspace
    checks come after the tensor checks and before any HIP call."""
    lib = _lib.load()
    x = ctypes.c_void_p(0x1000)
    B, T, H, K, V, L = 1, 256, 2, 64, 64, 9
    big = 1 << 40

    def call(fwd, fwd_bytes, V=V):
        return lib.hattn_gdn_chunkwise_bwd_fwd_ws(
            x, x, x, x, x, x, None, None, x, x, x, x, x, x, x, B, T, H, K, V, L, 0, 0, 0, 0, 2,
            0, 64, 0, 1.0, x, big, fwd, fwd_bytes, None)
    assert call(None, big) == _lib.HATTN_ERR_VALUE
    assert "forward workspace" in lib.hattn_last_error().decode()
    need = lib.hattn_gdn_chunkwise_fwd_keep_workspace(B, T, H, K, V, L)
    assert call(x, need - 1) == _lib.HATTN_ERR_VALUE
    assert call(x, big, V=192) == _lib.HATTN_ERR_NOT_IMPLEMENTED


def _fwd_noalloc(ptr=None, **kw):
    """hattn_mamba2_chunkwise_fwd_noalloc with NULL tensor pointers (or
    placeholders when ptr is given): the cases below fail in the host-side
    validation, before any HIP call."""
    a = dict(B=1, T=128, G=1, H=1, K=64, V=64, L=8, dq=0, dv=0, dl=0, do=0, base=2, htype=0,
             chunk=64)
    a.update(kw)
    lib = _lib.load()
    p = ctypes.c_void_p(ptr)
    gc = p if ptr is not None else None
    return lib.hattn_mamba2_chunkwise_fwd_noalloc(p, p, p, p, p, p, gc, None, a["B"], a["T"],
                                                  a["G"], a["H"], a["K"], a["V"], a["L"],
                                                  a["dq"], a["dv"], a["dl"], a["do"], a["base"],
                                                  a["htype"], a["chunk"], None)


@pytest.mark.parametrize("kw", [
    dict(T=100), dict(H=3, G=2), dict(L=7), dict(V=40), dict(chunk=32), dict(base=3),
    dict(htype=2), dict(K=128), dict(dq=1), dict(htype=1, dq=2, dv=2, dl=2, do=2),
    # big sizes: the shape / dtype status, not the static-scratch capacity
    dict(B=32, T=32768, G=32, H=32, L=16, K=128),
    dict(B=32, T=32768, G=32, H=32, L=16, dq=1),
])
def test_noalloc_reports_the_allocating_entry_points_status(kw):
    code = _fwd(**kw)
    msg = _lib.load().hattn_last_error()
    assert _fwd_noalloc(**kw) == code
    assert _lib.load().hattn_last_error() == msg


@pytest.mark.skipif(gpu_visible(), reason="passes placeholder device pointers; host-only check")
def test_noalloc_capacity_applies_to_weak_only():
    # WEAK beyond the 64 MiB static scratch: ValueError naming the scratch (the
    # check sits where the allocating entry point checks its workspace, after
    # the null-pointer check, so this case needs placeholder pointers)
    big = dict(B=32, T=32768, G=32, H=32, L=16)
    assert _fwd_noalloc(ptr=0x1000, **big) == _lib.HATTN_ERR_VALUE
    assert b"static scratch" in _lib.load().hattn_last_error()
    # STRONG uses no workspace: the same sizes pass every host check and reach
    # the launch, which fails here only because no GPU is visible
    assert _fwd_noalloc(ptr=0x1000, htype=1, **big) == _lib.HATTN_ERR_HIP
    assert b"static scratch" not in _lib.load().hattn_last_error()


def test_status_query_checks():
    lib = _lib.load()
    out = ctypes.c_uint(7)
    # sizes with one segment have no look-back: status 0 without a workspace
    assert lib.hattn_mamba2_chunkwise_fwd_status(None, 1, 1024, 1, 64, ctypes.byref(out),
                                                 None) == _lib.HATTN_OK
    assert out.value == 0
    # sizes with several segments need the workspace
    assert lib.hattn_mamba2_chunkwise_fwd_status(None, 1, 4096, 1, 64, ctypes.byref(out),
                                                 None) == _lib.HATTN_ERR_VALUE
    assert lib.hattn_mamba2_chunkwise_fwd_status(None, 1, 100, 1, 64, ctypes.byref(out),
                                                 None) == _lib.HATTN_ERR_VALUE

"""ctypes binding of libhattn_hip.so (declarations: include/hattn.h).

There is no fallback: if the library is missing or a tensor is not on a HIP
device the call raises.  Build the library with
``python log-linear-attention_amd/build_lib.py``.
"""
import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_native", "libhattn_hip.so")

HATTN_OK, HATTN_ERR_VALUE, HATTN_ERR_NOT_IMPLEMENTED, HATTN_ERR_HIP = 0, 1, 2, 3
DTYPE_CODES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}

# (name, restype, argtypes) of every exported entry point, in header order.
_P, _I, _F, _S = ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t
_LL = ctypes.c_longlong
SIGNATURES = [
    ("hattn_version", ctypes.c_char_p, []),
    ("hattn_last_error", ctypes.c_char_p, []),
    ("hattn_mamba2_chunkwise_fwd", _I,
     [_P, _P, _P, _F, _P, _P, _F, _F] + [_I] * 7 + [_I] * 4 + [_I] * 3 + [_P, _S, _P]),
    ("hattn_mamba2_chunkwise_fwd_workspace", _S, [_I] * 7),
    ("hattn_mamba2_chunkwise_fwd_noalloc", _I,
     [_P, _P, _P, _F, _P, _P, _F, _F] + [_I] * 7 + [_I] * 4 + [_I] * 3 + [_P]),
    ("hattn_mamba2_chunkwise_fwd_status", _I, [_P, _I, _I, _I, _I, _P, _P]),
    ("hattn_debug_lookback", None, [_I, _I]),
    ("hattn_mamba2_chunkwise_bwd", _I,
     [_P, _P, _P, _F, _P, _P, _P, _P, _P, _F, _F] + [_I] * 6 + [_I] * 4 + [_I] * 3
     + [_P, _S, _P]),
    ("hattn_mamba2_chunkwise_bwd_fwd_ws", _I,
     [_P, _P, _P, _F, _P, _P, _P, _P, _P, _F, _F] + [_I] * 6 + [_I] * 4 + [_I] * 3
     + [_P, _S, _P, _S, _P]),
    ("hattn_mamba2_chunkwise_bwd_workspace", _S, [_I] * 7),
    ("hattn_gdn_chunkwise_fwd", _I,
     [_P, _P, _P, _P, _F, _P, _P, _F, _P, _P, _F] + [_I] * 6 + [_I] * 4 + [_I] * 3
     + [_I, ctypes.c_float] + [_P, _S, _P]),
    ("hattn_gdn_chunkwise_fwd_workspace", _S, [_I] * 6),
    ("hattn_gdn_chunkwise_bwd", _I,
     [_P, _P, _P, _P, _F, _P, _P, _P, _P, _P, _P, _P, _P, _F, _F] + [_I] * 6 + [_I] * 4
     + [_I] * 3 + [_I, ctypes.c_float] + [_P, _S, _P]),
    ("hattn_gdn_chunkwise_bwd_workspace", _S, [_I] * 6),
    ("hattn_gdn_chunkwise_fwd_keep", _I,
     [_P, _P, _P, _P, _F, _P, _P, _F, _P, _P, _F] + [_I] * 6 + [_I] * 4 + [_I] * 3
     + [_I, ctypes.c_float] + [_P, _S, _P]),
    ("hattn_gdn_chunkwise_fwd_keep_workspace", _S, [_I] * 6),
    ("hattn_gdn_chunkwise_bwd_fwd_ws", _I,
     [_P, _P, _P, _P, _F, _P, _P, _P, _P, _P, _P, _P, _P, _F, _F] + [_I] * 6 + [_I] * 4
     + [_I] * 3 + [_I, ctypes.c_float] + [_P, _S, _P, _S, _P]),
    ("hattn_gdn_chunkwise_bwd_fwd_ws_workspace", _S, [_I] * 6),
    ("hattn_hstate_step", _I,
     [_P] * 9 + [_I] * 12 + [ctypes.c_float] + [_I] * 4 + [_P]),
    ("hattn_mamba2_prefill_levels", _I, [_P] * 4 + [_I] * 10 + [_P]),
    ("hattn_mamba2_layer_prologue", _I, [_P] * 9 + [_I] * 13 + [_P]),
    ("hattn_mamba2_layer_epilogue", _I, [_P] * 4 + [_I] * 7 + [_P]),
    ("hattn_mamba2_layer_scan_fwd", _I, [_P] * 11 + [_I] * 18 + [_P, _S, _P]),
    ("hattn_mamba2_layer_bwd_workspace", _S, [_I] * 4),
    ("hattn_mamba2_layer_bwd", _I, [_P] * 18 + [_I] * 17 + [_P, _S, _P]),
    ("hattn_causal_conv1d_silu_fwd", _I, [_P, _LL, _LL, _P, _P, _P, _P, _P] + [_I] * 9 + [_P]),
    ("hattn_causal_conv1d_silu_bwd_workspace", _S, [_I] * 4),
    ("hattn_causal_conv1d_silu_bwd", _I,
     [_P, _LL, _LL, _P, _P, _P, _P, _P, _P, _LL, _LL, _P, _P] + [_I] * 12 + [_P, _S, _P]),
    ("hattn_gated_rmsnorm_fwd", _I, [_P, _P, _LL, _P, _P, _P, _LL, _I, ctypes.c_float] + [_I] * 4
     + [_P]),
    ("hattn_gated_rmsnorm_bwd_workspace", _S, [_LL, _I]),
    ("hattn_gated_rmsnorm_bwd", _I, [_P, _P, _LL, _P, _P, _P, _P, _P, _LL, _P, _LL, _I] + [_I] * 6
     + [_P, _S, _P]),
]

_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Load the shared library once (raises ImportError if it is not built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise ImportError(
                    f"libhattn_hip.so not found at {LIB_PATH}; build it with "
                    "`python log-linear-attention_amd/build_lib.py`")
            lib = ctypes.CDLL(LIB_PATH)
            for name, res, args in SIGNATURES:
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def check(status: int) -> None:
    """Map an hattn_status to the exception type the reference raises."""
    if status == HATTN_OK:
        return
    msg = load().hattn_last_error().decode(errors="replace")
    if status == HATTN_ERR_VALUE:
        raise ValueError(msg)
    if status == HATTN_ERR_NOT_IMPLEMENTED:
        raise NotImplementedError(msg)
    raise RuntimeError(f"hattn HIP error: {msg}")


def dtype_code(t: torch.Tensor) -> int:
    try:
        return DTYPE_CODES[t.dtype]
    except KeyError:
        raise NotImplementedError(f"unsupported dtype {t.dtype}") from None


def require_device(*tensors) -> torch.device:
    """All tensors must live on one HIP device; the path has no CPU fallback."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                "hattention (MI355X) runs only on HIP device tensors; got a tensor on "
                f"{t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError("tensors on different devices")
    return dev


def ptr(t) -> int:
    return 0 if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> int:
    """The current stream of ``device`` as a raw hipStream_t (what
    torch.cuda.current_stream(device).cuda_stream returns, without building a
    Stream object: about 0.1 us instead of 1.8 us per call, which matters on
    the per-token decode path)."""
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None
                           else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


def fwd_status(ws, B: int, T: int, H: int, V: int, device: torch.device) -> int:
    """Health word of the last bf16 Mamba-2 forward on workspace ``ws`` (a
    tensor from :func:`workspace`, or None): bit 0 set means a look-back wait
    gave up and that call's outputs hold NaN.  Synchronises the stream."""
    import ctypes as _ct
    out = _ct.c_uint(0)
    check(load().hattn_mamba2_chunkwise_fwd_status(ptr(ws), B, T, H, V, _ct.byref(out),
                                                   stream_handle(device)))
    return out.value


def workspace(nbytes: int, device: torch.device):
    """Device scratch of ``nbytes`` bytes from torch's caching allocator (None
    when no scratch is needed); returns (tensor, pointer, size)."""
    if nbytes <= 0:
        return None, 0, 0
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    return ws, ws.data_ptr(), nbytes

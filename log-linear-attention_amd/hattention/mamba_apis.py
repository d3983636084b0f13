"""Mamba-2 style API of the log-linear Mamba-2 chunkwise path (MI355X).

Mirrors hattention/mamba_apis.py:
* ``compute_lambda``             -- :70-85  (lambda modes positive / bounded / None)
* ``compute_lambda_maybe_fixed`` -- :88-113 (fixed per-level lambdas only)
* ``hmamba_chunk_scan_combined`` -- :263-404 (dt / A / lambda pre-processing,
  then ``hattention_kernel`` with q=C, k=B, v=x*dt, g=A*dt, plus the D residual)

The pre-processing is elementwise torch on the device; the scan itself is the
HIP kernel.  Options the reference rejects with NotImplementedError are
rejected the same way; the per-call warnings of the reference are not emitted.
"""
from typing import Optional, Tuple

import torch

from hattention.base import HType, HStruct
from hattention.kernel import hattention_kernel


def compute_lambda(L: torch.Tensor, dl: torch.Tensor, lambda_mode: Optional[str]) -> torch.Tensor:
    """mamba_apis.py:70-85."""
    if lambda_mode == "positive":
        return torch.nn.functional.softplus(L * dl)
    if lambda_mode == "bounded":
        return torch.exp(-torch.exp(L) * torch.nn.functional.softplus(dl))
    if lambda_mode is None:
        return L * dl
    raise ValueError


def compute_lambda_maybe_fixed(L, dl, lambda_mode, lambda_level_max, lambda_level_fixed,
                               lambda_level_module=None) -> torch.Tensor:
    """mamba_apis.py:88-113 (the LambdaLevelMLP branch needs torchtune's RoPE and
    is not part of this build)."""
    if lambda_level_fixed:
        if not all([L.ndim in [3, 4], dl.ndim in [3, 4], L.shape[-1] == lambda_level_max,
                    dl.shape[-1] == lambda_level_max]):
            raise ValueError
        return compute_lambda(L=L, dl=dl, lambda_mode=lambda_mode)
    raise NotImplementedError("non-fixed lambda (LambdaLevelMLP) is not supported")


def hmamba_chunk_scan_combined(
    x: torch.Tensor,
    dt: torch.Tensor,
    A: torch.Tensor,
    B: torch.Tensor,
    C: torch.Tensor,
    dl: torch.Tensor,
    L: torch.Tensor,
    chunk_size: int,
    D: Optional[torch.Tensor] = None,
    z: Optional[torch.Tensor] = None,
    dt_bias: Optional[torch.Tensor] = None,
    initial_states: Optional[torch.Tensor] = None,
    seq_idx: Optional[torch.Tensor] = None,
    cu_seqlens: Optional[torch.Tensor] = None,
    dt_softplus: bool = False,
    dt_limit: Tuple[float, float] = (0.0, float("inf")),
    return_final_states: bool = False,
    return_varlen_states: bool = False,
    lambda_mode: Optional[str] = None,
    lambda_level_max: Optional[int] = None,
    lambda_level_base: Optional[int] = None,
    lambda_htype: Optional[HType] = None,
    lambda_hstruct: Optional[HStruct] = None,
    lambda_level_fixed: Optional[bool] = None,
    lambda_level_module=None,
):
    """mamba_apis.py:263-404.

    x [B,T,H,P], dt [B,T,H], A [H], B/C [B,T,G,N], dl [B,T,H,L], L [H,L].
    Returns (y, state); ``chunk_size`` is ignored as in the reference (the
    chunk is always 64).
    """
    if z is not None:
        raise NotImplementedError
    if initial_states is not None:
        raise NotImplementedError
    if seq_idx is not None:
        raise NotImplementedError
    if cu_seqlens is not None:
        raise NotImplementedError
    if dt_softplus is not True:
        raise NotImplementedError
    if tuple(dt_limit) != (0.0, float("inf")):
        raise NotImplementedError
    if return_varlen_states is not False:
        raise NotImplementedError
    if not B.shape == C.shape:
        raise ValueError("B and C must have the same shape")
    for arg in (lambda_level_max, lambda_level_base, lambda_htype, lambda_hstruct,
                lambda_level_fixed):
        if arg is None:
            raise ValueError
    if return_final_states:
        raise NotImplementedError("prefill (return_final_states=True) is not built yet")

    if D is not None:
        if D.dim() != 1:
            raise ValueError
        D_residual = x * D.view(1, 1, -1, 1)
    if dt_bias is not None:
        dt = dt + dt_bias.view(1, 1, -1)
    dt = torch.nn.functional.softplus(dt)
    x = x * dt.unsqueeze(-1)
    g = A.view(1, 1, -1) * dt
    lam = compute_lambda_maybe_fixed(L=L.view(1, 1, *L.shape), dl=dl, lambda_mode=lambda_mode,
                                     lambda_level_max=lambda_level_max,
                                     lambda_level_fixed=lambda_level_fixed,
                                     lambda_level_module=lambda_level_module)
    y = hattention_kernel(q=C, k=B, v=x, b=None, g=g.float(), l=lam, scale=None,
                          head_first=False, level_base=lambda_level_base, htype=lambda_htype,
                          hstruct=lambda_hstruct)
    if D is not None:
        y = y + D_residual
    return y, None

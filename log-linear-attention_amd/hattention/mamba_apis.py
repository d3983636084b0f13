"""Mamba-2 style API of the log-linear Mamba-2 chunkwise path (MI355X).

Mirrors hattention/mamba_apis.py:
* ``LambdaLevelMLP``             -- :32-67  (non-fixed lambda: per-level rotary
  embedding of L and dl, then one linear map each)
* ``compute_lambda``             -- :70-85  (lambda modes positive / bounded / None)
* ``compute_lambda_maybe_fixed`` -- :88-113
* ``hmamba_chunk_scan_combined`` -- :263-404 (dt / A / lambda pre-processing,
  then ``hattention_kernel`` with q=C, k=B, v=x*dt, g=A*dt, plus the D residual;
  with ``return_final_states`` the prefill ``hattention_prefill`` and its HState)
* ``hmamba_split_conv1d_scan_combined`` -- :116-260 (causal conv1d + SiLU,
  the layer scan, gated RMSNorm, out-projection)
* ``hselective_state_update``    -- :407-566 (the same pre-processing for one
  token, then one decode step of the HState)

The pre- and post-processing (dt softplus, x dt, A dt, lambda, D x) run as
fused HIP kernels around the scan (hattention/mamba_layer.py), with their
backward.  Options the reference rejects with NotImplementedError are
rejected the same way; the per-call warnings of the reference are not emitted.
"""
from typing import Optional, Tuple

import torch

from hattention.base import HType, HStruct
from hattention.kernel import hattention_kernel, hattention_prefill
from hattention.mamba_layer import (CausalConv1dSilu, GatedRMSNorm, HMambaScanFunction,
                                     lambda_mode_code, layer_epilogue, layer_prologue)


def compute_lambda(L: torch.Tensor, dl: torch.Tensor, lambda_mode: Optional[str]) -> torch.Tensor:
    """mamba_apis.py:70-85."""
    if lambda_mode == "positive":
        return torch.nn.functional.softplus(L * dl)
    if lambda_mode == "bounded":
        return torch.exp(-torch.exp(L) * torch.nn.functional.softplus(dl))
    if lambda_mode is None:
        return L * dl
    raise ValueError


class RotaryPositionalEmbeddings(torch.nn.Module):
    """The rotary position embedding the reference imports from torchtune
    (``torchtune.modules.RotaryPositionalEmbeddings``, mamba_apis.py:27-30; not
    installed here, version unpinned by the reference's requirements.txt):
    RoFormer's rotation (Su et al. 2021) with torchtune's conventions.  The
    feature pairs (2i, 2i + 1) of the last dim are rotated by the angle
    pos * theta_i, theta_i = base^(-2i / dim) (base 10000), computed in fp32
    (angle = float(pos) * theta_i, one rounding, as torchtune's cache); the
    result takes x's dtype.  x is [b, s, n_h, dim]; input_pos [s] (or None
    for 0 .. s - 1).  No parameters and no persistent buffers, like
    torchtune's module, so a state dict carries nothing for it."""

    def __init__(self, dim: int, max_seq_len: int = 4096, base: int = 10_000) -> None:
        super().__init__()
        if dim % 2:
            raise ValueError("dim must be even")
        self.dim = dim
        self.max_seq_len = max_seq_len
        self.base = base
        theta = 1.0 / (base ** (torch.arange(0, dim, 2)[: dim // 2].float() / dim))
        self.register_buffer("theta", theta, persistent=False)

    def forward(self, x: torch.Tensor, *, input_pos: Optional[torch.Tensor] = None) -> torch.Tensor:
        s = x.shape[1]
        pos = torch.arange(s, device=x.device) if input_pos is None else input_pos
        if pos.numel() and int(pos.max()) >= self.max_seq_len:
            raise IndexError("position beyond max_seq_len")
        ang = pos.to(device=x.device, dtype=torch.float32)[:, None] * self.theta.to(x.device)
        c = torch.cos(ang)[None, :, None, :]          # [1, s, 1, dim / 2]
        sn = torch.sin(ang)[None, :, None, :]
        xf = x.float().unflatten(-1, (-1, 2))
        x0, x1 = xf[..., 0], xf[..., 1]
        out = torch.stack((x0 * c - x1 * sn, x1 * c + x0 * sn), dim=-1).flatten(-2)
        return out.type_as(x)


class LambdaLevelMLP(torch.nn.Module):
    """mamba_apis.py:32-67: per-level lambda inputs from a ``dim``-wide L and
    dl.  For level index i, x is rotated by the rotary embedding at position i
    and mapped to one value by a linear layer (mlp0 for L, mlp1 for dl):
    returns (y0, y1), each [..., num_levels].  Same submodules and parameter
    names as the reference (mlp0, mlp1, rope), so its state dicts load."""

    def __init__(self, dim: int, max_num_levels: int, **kwargs) -> None:
        super().__init__()
        self.dim = dim
        self.max_num_levels = max_num_levels
        self.mlp0 = torch.nn.Linear(in_features=dim, out_features=1)
        self.mlp1 = torch.nn.Linear(in_features=dim, out_features=1)
        self.rope = RotaryPositionalEmbeddings(dim=dim, max_seq_len=max_num_levels)

    def forward(self, x0: torch.Tensor, x1: torch.Tensor,
                num_levels: int) -> Tuple[torch.Tensor, torch.Tensor]:
        if x0.ndim != 4 or x1.ndim != 4:
            raise ValueError
        if num_levels > self.max_num_levels:
            raise ValueError
        y0s, y1s = [], []
        for i in range(num_levels):
            p0 = torch.full((x0.shape[1],), i, dtype=torch.int32, device=x0.device)
            p1 = torch.full((x1.shape[1],), i, dtype=torch.int32, device=x1.device)
            y0s.append(self.mlp0(self.rope(x0, input_pos=p0)))
            y1s.append(self.mlp1(self.rope(x1, input_pos=p1)))
        return torch.cat(y0s, dim=-1), torch.cat(y1s, dim=-1)


def compute_lambda_maybe_fixed(L, dl, lambda_mode, lambda_level_max, lambda_level_fixed,
                               lambda_level_module=None) -> torch.Tensor:
    """mamba_apis.py:88-113."""
    if lambda_level_fixed:
        if not all([L.ndim in [3, 4], dl.ndim in [3, 4], L.shape[-1] == lambda_level_max,
                    dl.shape[-1] == lambda_level_max]):
            raise ValueError
        return compute_lambda(L=L, dl=dl, lambda_mode=lambda_mode)
    L_new, dl_new = _level_inputs(L, dl, lambda_level_max, lambda_level_module)
    return compute_lambda(L=L_new, dl=dl_new, lambda_mode=lambda_mode)


def _level_inputs(L, dl, lambda_level_max, lambda_level_module):
    """The non-fixed branch of mamba_apis.py:104-112: (L, dl) of width
    ``lambda_level_module.dim`` -> per-level (L_new, dl_new) of width
    ``lambda_level_max`` through the LambdaLevelMLP (torch ops, autograd)."""
    if not all([L.ndim in [3, 4], dl.ndim in [3, 4], L.shape[-1] == lambda_level_module.dim,
                dl.shape[-1] == lambda_level_module.dim]):
        raise ValueError
    return lambda_level_module(L, dl, num_levels=lambda_level_max)


def hmamba_split_conv1d_scan_combined(
    zxbcdtdl: torch.Tensor,
    conv1d_weight: torch.Tensor,
    conv1d_bias: torch.Tensor,
    dt_bias: torch.Tensor,
    A: torch.Tensor,
    L: torch.Tensor,
    D: torch.Tensor,
    chunk_size: int,
    initial_states: Optional[torch.Tensor] = None,
    seq_idx: Optional[torch.Tensor] = None,
    dt_limit: Tuple[float, float] = (0.0, float("inf")),
    return_final_states: bool = False,
    activation: str = "silu",
    rmsnorm_weight: Optional[torch.Tensor] = None,
    rmsnorm_eps: float = 1e-6,
    outproj_weight: Optional[torch.Tensor] = None,
    outproj_bias: Optional[torch.Tensor] = None,
    headdim: Optional[int] = None,
    ngroups: int = 1,
    norm_before_gate: bool = True,
    lambda_mode: Optional[str] = None,
    lambda_level_max: Optional[int] = None,
    lambda_level_base: Optional[int] = None,
    lambda_htype: Optional[HType] = None,
    lambda_hstruct: Optional[HStruct] = None,
    lambda_level_fixed: Optional[bool] = None,
    lambda_level_module=None,
) -> torch.Tensor:
    """mamba_apis.py:116-260: split the packed zxbcdtdl [B, S, 2 dim + 2 G N + H +
    H Lv] into z, xBC, dt, dl; xBC -> causal conv1d + SiLU (HIP kernel) -> x, B,
    C; the fused layer scan (hmamba_chunk_scan_combined); gated RMSNorm of the
    result with z (HIP kernel); the out-projection (torch linear, a library GEMM)."""
    if initial_states is not None:
        raise NotImplementedError
    if seq_idx is not None:
        raise NotImplementedError
    if tuple(dt_limit) != (0.0, float("inf")):
        raise NotImplementedError
    if return_final_states is not False:
        raise NotImplementedError
    if norm_before_gate is not False:
        raise NotImplementedError
    if rmsnorm_weight is None:
        raise NotImplementedError
    if activation not in ["silu", "swish"]:
        raise NotImplementedError

    batch, seqlen, _ = zxbcdtdl.shape
    dlambda = L.shape[-1]
    nheads, = D.shape
    dim = nheads * headdim
    dstate = (zxbcdtdl.shape[-1] - 2 * dim - nheads - nheads * dlambda) // ngroups // 2
    if D.dim() != 1:
        raise ValueError
    if headdim is None:
        raise ValueError
    if nheads % ngroups != 0:
        raise ValueError
    if zxbcdtdl.shape != (batch, seqlen, 2 * dim + 2 * ngroups * dstate + nheads + nheads * dlambda):
        raise ValueError
    if dt_bias.shape != (nheads,) or A.shape != (nheads,) or L.shape != (nheads, dlambda) or \
            D.shape != (nheads,):
        raise ValueError

    gn = ngroups * dstate
    Dc = dim + 2 * gn
    x, Bm, Cm = CausalConv1dSilu.apply(zxbcdtdl, dim, Dc, dim, dim + gn, conv1d_weight,
                                       conv1d_bias)
    c_dt = dim + Dc
    dt = zxbcdtdl[..., c_dt:c_dt + nheads]
    dl = zxbcdtdl[..., c_dt + nheads:].reshape(batch, seqlen, nheads, dlambda)
    y, _ = hmamba_chunk_scan_combined(
        x=x.view(batch, seqlen, nheads, headdim), dt=dt, A=A,
        B=Bm.view(batch, seqlen, ngroups, dstate), C=Cm.view(batch, seqlen, ngroups, dstate),
        dl=dl, L=L, chunk_size=chunk_size, D=D, z=None, dt_bias=dt_bias, dt_softplus=True,
        seq_idx=seq_idx, cu_seqlens=None, dt_limit=dt_limit,
        return_final_states=return_final_states, return_varlen_states=False,
        lambda_mode=lambda_mode, lambda_level_max=lambda_level_max,
        lambda_level_base=lambda_level_base, lambda_htype=lambda_htype,
        lambda_hstruct=lambda_hstruct, lambda_level_fixed=lambda_level_fixed,
        lambda_level_module=lambda_level_module)
    y = GatedRMSNorm.apply(y.reshape(batch, seqlen, dim), zxbcdtdl, 0, rmsnorm_weight,
                           rmsnorm_eps)
    return torch.nn.functional.linear(y, outproj_weight, outproj_bias)


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

    if D is not None and D.dim() != 1:
        raise ValueError
    if dt_bias is not None and dt_bias.dim() != 1:
        raise ValueError
    # compute_lambda_maybe_fixed's checks (mamba_apis.py:96-102) on L [1, 1, H, Lv]
    if not lambda_level_fixed:
        # mamba_apis.py:104-112: the LambdaLevelMLP maps L [H, dim] and dl [B, T, H,
        # dim] to per-level inputs; the fused scan then runs as for fixed levels
        L4, dl = _level_inputs(L[None, None], dl, lambda_level_max, lambda_level_module)
        L = L4[0, 0]
    if not all([L.dim() + 2 in (3, 4), dl.dim() in (3, 4), L.shape[-1] == lambda_level_max,
                dl.shape[-1] == lambda_level_max]):
        raise ValueError
    lambda_mode_code(lambda_mode)
    if lambda_hstruct != HStruct.MAMBA2:
        # the reference calls hattention_kernel with b=None, which GDELTA rejects
        raise ValueError

    if not return_final_states:
        # prologue -> chunkwise scan (q = C, k = B) -> epilogue, one autograd node
        y = HMambaScanFunction.apply(x, dt, A, B, C, dl, L, D, dt_bias, dt_softplus,
                                     lambda_mode, lambda_level_base, lambda_htype)
        return y, None
    with torch.no_grad():
        # :386-403: prefill with the final HState; v and lambda take C's / dl's dtype
        v, g, lam = layer_prologue(x, dt, A, dt_bias, dl, L, dt_softplus, lambda_mode,
                                   v_dtype=C.dtype)
        if v.dtype != C.dtype:
            v = v.to(dtype=C.dtype)
        if lam.dtype != dl.dtype:
            lam = lam.to(dtype=dl.dtype)
        y, state = hattention_prefill(q=C, k=B, v=v, b=None, g=g, l=lam, scale=None,
                                      head_first=False, level_base=lambda_level_base,
                                      htype=lambda_htype, hstruct=lambda_hstruct)
        if D is not None:
            y = layer_epilogue(y, x, D)
    return y, state


def hselective_state_update(
    state,
    x: torch.Tensor,
    dt: torch.Tensor,
    A: torch.Tensor,
    B: torch.Tensor,
    C: torch.Tensor,
    dl: torch.Tensor,
    L: torch.Tensor,
    D: Optional[torch.Tensor] = None,
    z: Optional[torch.Tensor] = None,
    dt_bias: Optional[torch.Tensor] = None,
    dt_softplus: bool = False,
    state_batch_indices: Optional[torch.Tensor] = None,
    lambda_mode: Optional[str] = None,
    lambda_level_max: Optional[int] = None,
    lambda_level_base: Optional[int] = None,
    lambda_htype: Optional[HType] = None,
    lambda_hstruct: Optional[HStruct] = None,
    lambda_level_fixed: Optional[bool] = None,
    lambda_level_module=None,
):
    """mamba_apis.py:407-566: one decode step of the log-linear Mamba-2 layer.

    x [B,H,P], dt [B,H], A [H], B/C [B,G,N], dl [B,H,L], L [H,L], D [H].
    Returns (out [B,H,P], state advanced in place).  The dt / A / lambda
    pre-processing is elementwise torch on the device; the state step is one
    ``hattn_hstate_step`` launch (q = C, k = B, v = x * dt, g = A * dt).
    """
    from hattention.recurrent import launch_step
    if state_batch_indices is not None:
        raise NotImplementedError
    if z is not None:
        raise NotImplementedError
    dims = [(x, 3), (dt, 2), (A, 1), (B, 3), (C, 3), (dl, 3), (L, 2)]
    if any(t.dim() != n for t, n in dims):
        raise ValueError
    if D is not None and D.dim() != 1:
        raise ValueError
    if dt_bias is not None and dt_bias.dim() != 1:
        raise ValueError
    batch, nheads, headdim = x.shape
    _, ngroups, dstate = B.shape
    dlambda = L.shape[-1]
    if dt.shape != x.shape[:2] or A.shape != (nheads,) or nheads % ngroups != 0:
        raise ValueError
    if B.shape != (batch, ngroups, dstate) or C.shape != B.shape:
        raise ValueError
    if dl.shape != (batch, nheads, dlambda) or L.shape != (nheads, dlambda):
        raise ValueError
    if D is not None and D.shape != (nheads,):
        raise ValueError
    for arg in (lambda_level_max, lambda_level_base, lambda_htype, lambda_hstruct,
                lambda_level_fixed):
        if arg is None:
            raise ValueError

    if not lambda_level_fixed:
        # mamba_apis.py:530-536 hands the LambdaLevelMLP 3-D [1, H, dim] / [B, H, dim]
        # inputs, which its forward rejects (:42-43): the reference's decode step
        # raises ValueError with non-fixed lambda, and so does this one
        L4, dl = _level_inputs(L[None], dl, lambda_level_max, lambda_level_module)
        L = L4[0]
    if not all([L.dim() + 1 in (3, 4), dl.dim() in (3, 4), L.shape[-1] == lambda_level_max,
                dl.shape[-1] == lambda_level_max]):
        raise ValueError
    # dtypes of the reference's intermediates (:493-509), for its checks (:517-525)
    dtp = torch.promote_types(dt.dtype, dt_bias.dtype) if dt_bias is not None else dt.dtype
    x_dtype = torch.promote_types(x.dtype, dtp)
    a_dtype = torch.promote_types(A.dtype, dtp)
    lam_dtype = torch.promote_types(L.dtype, dl.dtype)
    if not all([a_dtype == state.dtype, C.dtype == B.dtype,
                C.dtype == x_dtype or x_dtype == state.dtype,
                C.dtype == lam_dtype or lam_dtype == state.dtype,
                state.base == lambda_level_base, state.htype == lambda_htype,
                state.hstruct == lambda_hstruct]):
        raise TypeError
    # one token: the layer prologue on [B, 1, H, .] views, one step launch, the epilogue
    v, g, lam = layer_prologue(x.unsqueeze(1), dt.unsqueeze(1), A, dt_bias, dl.unsqueeze(1), L,
                               dt_softplus, lambda_mode)
    v, g, lam = v.squeeze(1), g.squeeze(1), lam.squeeze(1)
    out = torch.empty_like(v)
    launch_step(state, q=C.contiguous(), k=B.contiguous(), v=v, g=g, l=lam, o=out, update=True,
                output=True)
    if D is not None:
        out = layer_epilogue(out.unsqueeze(1), x.unsqueeze(1), D).squeeze(1)
    return out, state

"""FLA-compatible API of the log-linear Gated DeltaNet path (MI355X).

Mirrors hattention/gated_delta_rule_apis.py:20-134 ``chunk_h_gated_delta_rule``
with its three modes: the chunkwise forward (``output_final_state=False``), the
prefill returning the HState (``output_final_state=True``, no initial state)
and one decode step from an HState (both set, T == 1).  lambda is divided by
the scale when SCALE_LAMBDA (:17, :65-70), q / k are l2-normalised inside the
kernel boundary and q is multiplied by the scale (kernel.py:100-111), so the
scale cancels.  The per-call warnings of the reference are not emitted.
"""
from typing import Optional

import torch

from hattention.base import HType, HStruct
from hattention.kernel import hattention_kernel, hattention_prefill, hattention_step

SCALE_LAMBDA = True


def chunk_h_gated_delta_rule(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    l: torch.Tensor,
    beta: torch.Tensor,
    scale: float = None,
    initial_state=None,
    output_final_state: bool = False,
    cu_seqlens: Optional[torch.LongTensor] = None,
    head_first: bool = False,
    use_qk_l2norm_in_kernel: bool = False,
):
    """gated_delta_rule_apis.py:20-134; returns (o, final_state)."""
    assert q.dtype == k.dtype == v.dtype
    assert q.dtype != torch.float32, \
        "ChunkGatedDeltaRuleFunction does not support float32. Please use bfloat16."
    assert len(beta.shape) == 3, "beta must be of shape [B, T, H]"
    assert cu_seqlens is None
    assert use_qk_l2norm_in_kernel is True
    if head_first:
        raise NotImplementedError("head_first=True is not supported")
    if scale is None:
        scale = k.shape[-1] ** -0.5
    if SCALE_LAMBDA:
        l = l / scale
    common = dict(scale=scale, level_base=2, htype=HType.WEAK, hstruct=HStruct.GDELTA,
                  use_qk_l2norm_in_kernel=use_qk_l2norm_in_kernel)
    if output_final_state is False:
        if initial_state is not None:
            raise NotImplementedError
        final_state = None
        o = hattention_kernel(q=q, k=k, v=v, b=beta, g=g, l=l, head_first=False, **common)
    elif initial_state is None:
        # :90-104: prefill, returning the HState
        o, final_state = hattention_prefill(q=q, k=k, v=v, b=beta, g=g, l=l, head_first=False,
                                            **common)
    else:
        # :105-128: one decode step from ``initial_state`` (T == 1)
        if not all([q.ndim == 4, q.shape[1] == 1, k.ndim == 4, k.shape[1] == 1,
                    v.ndim == 4, v.shape[1] == 1, beta.ndim == 3, beta.shape[1] == 1,
                    g.ndim == 3, g.shape[1] == 1, l.ndim == 4, l.shape[1] == 1]):
            raise ValueError
        o, final_state = hattention_step(hstate=initial_state, q=q.squeeze(1), k=k.squeeze(1),
                                         v=v.squeeze(1), b=beta.squeeze(1), g=g.squeeze(1),
                                         l=l.squeeze(1), **common)
        o = o.unsqueeze(1)
    return o, final_state

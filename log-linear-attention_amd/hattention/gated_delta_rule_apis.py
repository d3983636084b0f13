"""FLA-compatible API of the log-linear Gated DeltaNet path (MI355X).

Mirrors hattention/gated_delta_rule_apis.py:20-134 ``chunk_h_gated_delta_rule``
for the chunkwise forward (``output_final_state=False``): lambda is divided by
the scale when SCALE_LAMBDA (:17, :65-70), q / k are l2-normalised inside the
kernel boundary and q is multiplied by the scale (kernel.py:100-111), so the
scale cancels.  Prefill / decode (``output_final_state=True``) are not part of
this build; the per-call warnings of the reference are not emitted.
"""
from typing import Optional

import torch

from hattention.base import HType, HStruct
from hattention.kernel import hattention_kernel

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
    """gated_delta_rule_apis.py:20-134 (chunkwise forward); returns (o, None)."""
    assert q.dtype == k.dtype == v.dtype
    assert q.dtype != torch.float32, \
        "ChunkGatedDeltaRuleFunction does not support float32. Please use bfloat16."
    assert len(beta.shape) == 3, "beta must be of shape [B, T, H]"
    assert cu_seqlens is None
    assert use_qk_l2norm_in_kernel is True
    if head_first:
        raise NotImplementedError("head_first=True is not supported")
    if output_final_state or initial_state is not None:
        raise NotImplementedError("prefill / decode are not part of this build")
    if scale is None:
        scale = k.shape[-1] ** -0.5
    if SCALE_LAMBDA:
        l = l / scale
    o = hattention_kernel(q=q, k=k, v=v, b=beta, g=g, l=l, scale=scale, head_first=False,
                          level_base=2, htype=HType.WEAK, hstruct=HStruct.GDELTA,
                          use_qk_l2norm_in_kernel=use_qk_l2norm_in_kernel)
    return o, None

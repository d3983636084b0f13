"""hattention for MI355X: the chunkwise path of log-linear attention.

Drop-in for the reference package's chunkwise entry points
(``hattention.kernel.hattention_kernel``, ``hattention.chunkwise.chunkwise_fwd``
/ ``chunkwise_bwd``, ``hattention.mamba_apis.hmamba_chunk_scan_combined``,
``hattention.gated_delta_rule_apis.chunk_h_gated_delta_rule``), backed by the
hand-written gfx950 kernels of ``libhattn_hip.so``.
"""
from hattention.base import HType, HStruct, get_num_levels, ceil_log, floor_log

__version__ = "0.1.0"

__all__ = ["HType", "HStruct", "get_num_levels", "ceil_log", "floor_log"]

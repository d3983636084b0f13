"""Fenwick level state (HState) and the recurrent step of log-linear attention.

Mirrors hattention/recurrent.py:9-216:
* ``HState``               -- :9-131 (states [B, H, K, V, L] and counts [L])
* ``step_state``           -- :134-156 (cascade, gate every level, insert the token)
* ``step_output``          -- :159-166 (o = q . sum_l lambda_l S_l)
* ``hattention_recurrent`` -- :169-216 (the token loop)

The state lives in HBM in the reference's layout and is advanced in place by
one ``hattn_hstate_step`` launch per token (libhattn_hip.so): cascade, gate,
insert, and for ``hattention_step`` also the output.  The cascades (weak,
:42-54, and strong, :56-74) depend only on the level counts, which depend only
on the number of tokens inserted, so they are planned here on a host copy of
the counts (``plan_cascade_weak`` / ``plan_cascade_strong``); the device
``counts`` tensor is advanced by the same launch.  No step reads anything back
from the device.  Level base 2 only (other bases raise NotImplementedError, as
the reference's strong check does); states are fp32, the dtype the reference
gives them (state dtype = g.dtype, :185, kernel.py:505).
"""
from typing import List, Optional, Tuple

import torch

from hattention import _lib
from hattention.base import HType, HStruct


class HState:
    """recurrent.py:9-131."""

    def __init__(self, base: int, htype: HType, hstruct: HStruct, shape, dtype: torch.dtype,
                 device) -> None:
        if htype != HType.WEAK and base != 2:
            raise NotImplementedError
        if not isinstance(shape, tuple):
            shape = tuple(shape)
        self.base = base
        self.htype = htype
        self.hstruct = hstruct
        self.shape = shape
        self.dtype = dtype
        self.device = torch.device(device)
        self.max_num_levels = shape[-1]
        self.states = torch.zeros(self.shape, dtype=self.dtype, device=self.device)
        self.counts = torch.zeros(self.max_num_levels, dtype=torch.int32, device=self.device)
        self.host_counts: List[int] = [0] * self.max_num_levels

    # -- level bookkeeping (host side) --------------------------------------
    def plan_cascade_weak(self) -> int:
        """recurrent.py:42-54 on the host copy of the counts, followed by the
        insert's counts[0] += 1 (:94).  Returns the cascade depth c: levels
        0 .. c-1 are full and merge, in order, into level c.  Raises ValueError
        for a level over capacity (as :53-54) and IndexError when the top level
        is full (the reference indexes level L there, :47)."""
        counts = list(self.host_counts)
        depth = self.max_num_levels
        for level in range(self.max_num_levels):
            capacity = self.base ** level
            if counts[level] == capacity:
                if level + 1 >= self.max_num_levels:
                    raise IndexError(f"HState level overflow: all {self.max_num_levels} "
                                     "levels are full")
                counts[level + 1] += counts[level]
                counts[level] = 0
            elif counts[level] < capacity:
                depth = level
                break
            else:
                raise ValueError("level count above capacity")
        counts[0] += 1
        self.host_counts = counts
        return depth

    def plan_cascade_strong(self) -> int:
        """recurrent.py:56-74 on the host copy of the counts, followed by the
        insert's counts[0] += 1.  The carry (state, count) walks up: level 0,
        and a level whose count plus the carry's exceeds its capacity
        2^max(level - 1, 0), hands its content on and takes the carry; the
        first other level merges the carry, and nothing above it changes.
        Returns that merge level m (L when the carry leaves the top level, as
        the reference drops it): levels 0 .. m-1 move up one level, level m - 1
        merging into level m."""
        counts = list(self.host_counts)
        carry = 0
        merge = self.max_num_levels
        for level in range(self.max_num_levels):
            capacity = self.base ** max(level - 1, 0)
            if counts[level] + carry > capacity or level == 0:
                counts[level], carry = carry, counts[level]
            else:
                counts[level] += carry
                merge = level
                break
        counts[0] += 1
        self.host_counts = counts
        return merge

    def plan_cascade(self) -> int:
        return self.plan_cascade_weak() if self.htype == HType.WEAK else self.plan_cascade_strong()

    def set_counts(self, counts: List[int]) -> None:
        """Set the level counts on the host and the device."""
        if len(counts) != self.max_num_levels:
            raise ValueError("counts length")
        self.host_counts = [int(c) for c in counts]
        self.counts.copy_(torch.tensor(self.host_counts, dtype=torch.int32))

    # -- reference methods ---------------------------------------------------
    def reset_states(self) -> None:
        """recurrent.py:101-102."""
        self.states = torch.zeros_like(self.states)

    def replace(self, other: "HState") -> None:
        """recurrent.py:104-114 (replaces the states, keeps the counts)."""
        if not all([tuple(self.shape) == tuple(other.shape), self.base == other.base,
                    self.htype == other.htype, self.dtype == other.dtype,
                    self.device == other.device]):
            raise ValueError("Shape, dtype or device mismatch")
        self.states = other.states

    def to(self, dtype: Optional[torch.dtype] = None, device=None) -> "HState":
        """recurrent.py:116-131 (a copy; the host counts travel with it)."""
        dtype = self.dtype if dtype is None else dtype
        device = self.device if device is None else device
        new = HState(base=self.base, htype=self.htype, hstruct=self.hstruct, shape=self.shape,
                     dtype=dtype, device=device)
        new.states = self.states.to(dtype=dtype, device=device)
        new.counts = self.counts.to(dtype=torch.int32, device=device)
        new.host_counts = list(self.host_counts)
        return new

    def dot(self, other: torch.Tensor) -> torch.Tensor:
        """recurrent.py:96-99: sum over levels of states * other."""
        return (self.states * other).sum(-1)


def _check_state(S: HState) -> None:
    if S.htype not in (HType.WEAK, HType.STRONG) or S.base != 2:
        raise NotImplementedError("only level base 2 (HType.WEAK or HType.STRONG) is built")
    if S.dtype != torch.float32:
        raise NotImplementedError(f"HState in {S.dtype}: the step kernels keep fp32 states")
    if not S.states.is_contiguous():
        S.states = S.states.contiguous()


_FP32 = _lib.DTYPE_CODES[torch.float32]
_fn_step = None


def _step_fn():
    global _fn_step
    if _fn_step is None:
        _fn_step = _lib.load().hattn_hstate_step
    return _fn_step


def _operand_error(name, t, shape, dev):
    if t.device != dev:
        return RuntimeError(
            "hattention (MI355X) runs only on HIP device tensors of the state's device; "
            f"{name} is on {t.device}")
    return ValueError(f"{name}: expected a contiguous tensor of shape {shape}, got "
                      f"{tuple(t.shape)} (contiguous={t.is_contiguous()})")


def launch_step(S: HState, *, q=None, k=None, v=None, beta=None, g=None, l=None, o=None,
                update: bool, output: bool, l2norm_qk: bool = False,
                scale: Optional[float] = None) -> None:
    """One ``hattn_hstate_step`` launch on the current stream of the state's
    device.  q, k: [B, G, K]; v, o: [B, H, V]; beta, g: [B, H]; l: [B, H, L];
    all contiguous on the state's device (g fp32).  Plans the cascade when
    ``update``.  Kept lean: it runs once per decoded token."""
    st = S.states
    if S.base != 2 or st.dtype is not torch.float32 or not st.is_contiguous():
        _check_state(S)
        st = S.states
    if not st.is_cuda:
        raise RuntimeError("hattention (MI355X) runs only on HIP device tensors; the HState "
                           f"is on {st.device}")
    dev = st.device
    didx = st.get_device()
    B, H, K, V, L = S.shape
    qk = q if q is not None else k
    if qk is None or (update and (k is None or v is None or g is None)) or \
            (output and (q is None or l is None or o is None)):
        raise ValueError("missing operand for the step")
    G = qk.shape[1]
    # (the device compared by index: t.device builds a torch.device per call)
    for name, t, shape in (("q", q, (B, G, K)), ("k", k, (B, G, K)), ("v", v, (B, H, V)),
                           ("beta", beta, (B, H)), ("g", g, (B, H)), ("l", l, (B, H, L)),
                           ("o", o, (B, H, V))):
        if t is not None and (t.shape != shape or not t.is_contiguous() or
                              t.get_device() != didx):
            raise _operand_error(name, t, shape, dev)
    if G <= 0 or H % G != 0:
        raise ValueError(f"G={G} does not divide H={H}")
    if g is not None and g.dtype is not torch.float32:
        raise TypeError("g must be float32")
    if q is not None and k is not None and q.dtype != k.dtype:
        raise TypeError("q and k must share a dtype")
    if v is not None and o is not None and v.dtype != o.dtype:
        raise TypeError("o must have v's dtype")
    dt = _lib.DTYPE_CODES
    try:
        codes = (dt[qk.dtype], dt[(v if v is not None else o).dtype],
                 dt[l.dtype] if l is not None else _FP32,
                 dt[beta.dtype] if beta is not None else _FP32)
    except KeyError as e:
        raise NotImplementedError(f"unsupported dtype {e}") from None
    fn = _step_fn()
    saved = S.host_counts
    cascade = S.plan_cascade() if update else 0
    status = fn(st.data_ptr(), S.counts.data_ptr(), _lib.ptr(q), _lib.ptr(k), _lib.ptr(v),
                _lib.ptr(beta), _lib.ptr(g), _lib.ptr(l), _lib.ptr(o), B, G, H, K, V, L,
                S.hstruct.value, S.htype.value, cascade, int(update), int(output), int(l2norm_qk),
                float(scale if scale is not None else 1.0), *codes,
                _lib.stream_handle(dev))
    if status:
        S.host_counts = saved
        _lib.check(status)


def step_state(S: HState, k: torch.Tensor, v: torch.Tensor, a: torch.Tensor,
               b: Optional[torch.Tensor] = None) -> HState:
    """recurrent.py:134-156: k [B, H, K], v [B, H, V], gate a [B, H] (linear,
    not log), b [B, H] (GDELTA only).  Advances S in place and returns it."""
    if S.hstruct == HStruct.MAMBA2:
        if b is not None:
            raise ValueError
    else:
        if b is None:
            raise ValueError
    g = torch.log(a.float()).contiguous()
    launch_step(S, k=k.contiguous(), v=v.contiguous(),
                beta=b.contiguous() if b is not None else None, g=g, update=True, output=False)
    return S


def step_output(S: HState, q: torch.Tensor, l: torch.Tensor,
                out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """recurrent.py:159-166: o = q . sum_l l_l S_l, q [B, H, K], l [B, H, L];
    o [B, H, V] in ``out_dtype`` (the reference casts the state to v's dtype
    first, :208-211; default: q's dtype)."""
    B, H, K, V, L = S.shape
    o = torch.empty(B, H, V, dtype=out_dtype or q.dtype, device=q.device)
    launch_step(S, q=q.contiguous(), l=l.contiguous(), o=o, update=False, output=True)
    return o


def hattention_recurrent(Q, K, V, A, B, L, base: int, htype: HType,
                         hstruct: HStruct) -> Tuple[torch.Tensor, HState]:
    """recurrent.py:169-216: Q, K [B, T, H, K]; V [B, T, H, V]; A [B, T, H] the
    gate (linear, fp32); B [B, T, H] (GDELTA) or None; L [B, T, H, L].  One
    fused step (update + output) per token."""
    if not all([Q.shape == K.shape, Q.shape[:-1] == V.shape[:-1], Q.shape[:-1] == A.shape,
                Q.shape[:-1] == L.shape[:-1], A.dtype == torch.float32, Q.dtype == K.dtype,
                Q.dtype == V.dtype, Q.dtype == L.dtype]):
        raise ValueError("Invalid shape")
    if (hstruct == HStruct.MAMBA2) != (B is None):
        raise ValueError
    Bsz, T, H, Kd = Q.shape
    S = HState(base=base, htype=htype, hstruct=hstruct,
               shape=(Bsz, H, Kd, V.shape[3], L.shape[-1]), dtype=A.dtype, device=Q.device)
    tm = lambda x: x.transpose(0, 1).contiguous() if x is not None else None
    q_t, k_t, v_t, l_t, b_t = tm(Q), tm(K), tm(V), tm(L), tm(B)
    g_t = tm(torch.log(A))
    o_t = torch.empty(T, Bsz, H, V.shape[3], dtype=V.dtype, device=V.device)
    for t in range(T):
        launch_step(S, q=q_t[t], k=k_t[t], v=v_t[t], beta=b_t[t] if b_t is not None else None,
                    g=g_t[t], l=l_t[t], o=o_t[t], update=True, output=True)
    return o_t.transpose(0, 1).contiguous(), S

"""GPU parity of the decode step and the prefill of the Fenwick level state.

The HIP path runs through the C-ABI (hattn_hstate_step, hattn_mamba2_prefill_levels
and the chunkwise forwards, via hattention.kernel.hattention_step /
hattention_prefill, hattention.mamba_apis.hselective_state_update and
hattention.gated_delta_rule_apis.chunk_h_gated_delta_rule).  The checker is the
recurrent restatement of the reference (oracle.mamba2.recurrent_fwd with its
FenwickState, oracle.gdn.recurrent_fwd) in float64 on the CPU, fed the
identical inputs: the outputs of every token and the final level states and
counts.  The reference's prefill (chunkwise final states, the low levels rebuilt
from the last chunk, the counts set greedily, kernel.py:377-464) yields exactly
the recurrent state after T tokens, level by level, so the same oracle checks it.

Tolerances: bf16 inputs max|o - o_ref| / max|o_ref| < 2e-2 and relative
Frobenius error < 1e-2; fp32 inputs 1e-4 on both (the
kernel computes in fp32).  Level states: relative Frobenius error per level of
the same bound (bf16: 2e-2).
"""
import math

import pytest
import torch

from bench import make_gdn_inputs, make_mamba2_inputs
from oracle import gdn as D
from oracle import mamba2 as M

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _errs(out, ref):
    out = out.double().cpu()
    ref = ref.double().cpu()
    mx = ((out - ref).abs().max() / ref.abs().max()).item()
    fro = ((out - ref).norm() / ref.norm()).item()
    return mx, fro


def _tols(dtype):
    return (1e-4, 1e-4, 1e-4) if dtype == torch.float32 else (2e-2, 1e-2, 2e-2)


def _check_out(o, ref, dtype, tag):
    tmax, tfro, _ = _tols(dtype)
    mx, fro = _errs(o, ref)
    print(f"  {tag} o: max-rel {mx:.2e} fro {fro:.2e}", flush=True)
    assert mx < tmax and fro < tfro, (tag, mx, fro)


def _check_state(states, counts, ref_states, ref_counts, dtype, tag):
    _, _, tst = _tols(dtype)
    assert [int(c) for c in counts.cpu()] == list(ref_counts), (tag, counts, ref_counts)
    got = states.double().cpu()
    for e in range(ref_states.shape[-1]):
        r = ref_states[..., e]
        a = got[..., e]
        if r.abs().max() == 0:
            assert a.abs().max() == 0, (tag, e)
            continue
        err = ((a - r).norm() / r.norm()).item()
        assert err < tst, (tag, e, err)


def _fenwick_counts(T, L):
    """Level counts of the oracle's FenwickState after T inserts."""
    S = M.FenwickState(1, 1, 1, 1, L, torch.float64)
    for _ in range(T):
        S.insert(torch.ones(1, 1, dtype=torch.float64), torch.zeros(1, 1, 1, 1,
                                                                      dtype=torch.float64))
    return S.counts


def _gdn_normed(q, k, scale):
    """q, k as the GDELTA step sees them: l2norm (eps 1e-6) and q * scale, in fp64."""
    return D.l2norm(q.double()) * scale, D.l2norm(k.double())


# ---------------------------------------------------------------------------
# decode from an empty state
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_mamba2_decode_matches_recurrent(dtype):
    from hattention.base import HType, HStruct
    from hattention.kernel import hattention_step
    from hattention.recurrent import HState
    B, T, G, H, K, V, L = 2, 70, 1, 2, 64, 32, 8
    q, k, v, g, l = make_mamba2_inputs(B, T, H, K, V, L, G=G, seed=301, dtype=dtype)
    print(f"[hstate] mamba2 decode B={B} T={T} G={G} H={H} K={K} V={V} L={L} {dtype}",
          flush=True)
    S = HState(2, HType.WEAK, HStruct.MAMBA2, (B, H, K, V, L), torch.float32, DEV)
    qd, kd, vd, gd, ld = (x.to(DEV) for x in (q, k, v, g, l))
    outs = []
    for t in range(T):
        o, S = hattention_step(S, qd[:, t], kd[:, t], vd[:, t], None, gd[:, t], ld[:, t], None,
                               2, HType.WEAK, HStruct.MAMBA2)
        assert o.dtype == dtype and o.shape == (B, H, V)
        outs.append(o)
    torch.cuda.synchronize()
    o = torch.stack(outs, 1)
    o_ref, F = M.recurrent_fwd(*(x.double() for x in (q, k, v, g, l)), return_state=True)
    _check_out(o, o_ref, dtype, "mamba2 decode")
    _check_state(S.states, S.counts, F.states, F.counts, dtype, "mamba2 decode")
    assert S.host_counts == F.counts


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gdn_decode_matches_recurrent(dtype):
    from hattention.base import HType, HStruct
    from hattention.kernel import hattention_step
    from hattention.recurrent import HState
    B, T, H, K, V, L = 2, 70, 2, 64, 64, 8
    q, k, v, beta, g, l = make_gdn_inputs(B, T, H, K, V, L, seed=302, dtype=dtype)
    scale = K ** -0.5
    print(f"[hstate] gdn decode B={B} T={T} H={H} K={K} V={V} L={L} {dtype}", flush=True)
    S = HState(2, HType.WEAK, HStruct.GDELTA, (B, H, K, V, L), torch.float32, DEV)
    qd, kd, vd, bd, gd, ld = (x.to(DEV) for x in (q, k, v, beta, g, l))
    outs = []
    for t in range(T):
        o, S = hattention_step(S, qd[:, t], kd[:, t], vd[:, t], bd[:, t], gd[:, t], ld[:, t],
                               scale, 2, HType.WEAK, HStruct.GDELTA,
                               use_qk_l2norm_in_kernel=True)
        outs.append(o)
    torch.cuda.synchronize()
    o = torch.stack(outs, 1)
    qn, kn = _gdn_normed(q, k, scale)
    o_ref, S_ref = D.recurrent_fwd(qn, kn, v.double(), beta.double(), g.double(), l.double(),
                                   return_state=True)
    _check_out(o, o_ref, dtype, "gdn decode")
    _check_state(S.states, S.counts, S_ref, _fenwick_counts(T, L), dtype, "gdn decode")


def test_step_state_and_step_output_split():
    """step_state then step_output (recurrent.py:134-166) equal the fused step."""
    from hattention.base import HType, HStruct
    from hattention.kernel import hattention_step
    from hattention.recurrent import HState, step_output, step_state
    B, T, H, K, V, L = 1, 9, 2, 64, 16, 5
    q, k, v, g, l = (x.to(DEV) for x in make_mamba2_inputs(B, T, H, K, V, L, seed=303,
                                                          dtype=torch.float32))
    S1 = HState(2, HType.WEAK, HStruct.MAMBA2, (B, H, K, V, L), torch.float32, DEV)
    S2 = HState(2, HType.WEAK, HStruct.MAMBA2, (B, H, K, V, L), torch.float32, DEV)
    for t in range(T):
        o1, _ = hattention_step(S1, q[:, t], k[:, t], v[:, t], None, g[:, t], l[:, t], None, 2,
                                HType.WEAK, HStruct.MAMBA2)
        step_state(S2, k[:, t], v[:, t], torch.exp(g[:, t]))
        o2 = step_output(S2, q[:, t], l[:, t])
        torch.testing.assert_close(o2, o1, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(S2.states, S1.states, rtol=1e-5, atol=1e-6)
    assert S1.host_counts == S2.host_counts == [int(c) for c in S2.counts.cpu()]


def test_level_overflow_raises():
    """All levels full: the reference indexes past the last level; here IndexError
    before any launch, and the state is left as it was."""
    from hattention.base import HType, HStruct
    from hattention.kernel import hattention_step
    from hattention.recurrent import HState
    B, H, K, V, L = 1, 1, 64, 16, 2
    q, k, v, g, l = (x.to(DEV) for x in make_mamba2_inputs(B, 4, H, K, V, L, seed=304))
    S = HState(2, HType.WEAK, HStruct.MAMBA2, (B, H, K, V, L), torch.float32, DEV)
    for t in range(2):     # with 2 levels the third token's cascade overflows
        hattention_step(S, q[:, t], k[:, t], v[:, t], None, g[:, t], l[:, t], None, 2,
                        HType.WEAK, HStruct.MAMBA2)
    before = S.states.clone()
    with pytest.raises(IndexError):
        hattention_step(S, q[:, 2], k[:, 2], v[:, 2], None, g[:, 2], l[:, 2], None, 2,
                        HType.WEAK, HStruct.MAMBA2)
    torch.cuda.synchronize()
    assert torch.equal(S.states, before) and S.host_counts == [1, 1]
    assert [int(c) for c in S.counts.cpu()] == [1, 1]


# ---------------------------------------------------------------------------
# prefill (chunkwise + low levels + remaining steps)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("T,L,dtype", [(64, 8, torch.bfloat16), (256, 10, torch.bfloat16),
                                       (293, 10, torch.bfloat16), (320, 10, torch.float32),
                                       (37, 7, torch.bfloat16)])
def test_mamba2_prefill_matches_recurrent(T, L, dtype):
    from hattention.base import HType, HStruct
    from hattention.kernel import hattention_prefill
    B, G, H, K, V = 1, 2, 4, 64, 64
    q, k, v, g, l = make_mamba2_inputs(B, T, H, K, V, L, G=G, seed=310 + T, dtype=dtype)
    print(f"[hstate] mamba2 prefill B={B} T={T} G={G} H={H} K={K} V={V} L={L} {dtype}",
          flush=True)
    o, S = hattention_prefill(*(x.to(DEV) for x in (q, k, v)), None, g.to(DEV), l.to(DEV),
                              None, False, 2, HType.WEAK, HStruct.MAMBA2)
    torch.cuda.synchronize()
    assert o.dtype == v.dtype
    o_ref, F = M.recurrent_fwd(*(x.double() for x in (q, k, v, g, l)), return_state=True)
    _check_out(o, o_ref, dtype, f"mamba2 prefill T={T}")
    _check_state(S.states, S.counts, F.states, F.counts, dtype, f"mamba2 prefill T={T}")
    assert S.host_counts == F.counts


@pytest.mark.parametrize("T,L", [(128, 9), (200, 10)])
def test_gdn_prefill_matches_recurrent(T, L):
    from hattention.base import HType, HStruct
    from hattention.kernel import hattention_prefill
    B, H, K, V = 1, 2, 64, 64
    q, k, v, beta, g, l = make_gdn_inputs(B, T, H, K, V, L, seed=320 + T)
    scale = K ** -0.5
    print(f"[hstate] gdn prefill B={B} T={T} H={H} K={K} V={V} L={L}", flush=True)
    o, S = hattention_prefill(*(x.to(DEV) for x in (q, k, v, beta, g, l)), scale, False, 2,
                              HType.WEAK, HStruct.GDELTA, use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    qn, kn = _gdn_normed(q, k, scale)
    o_ref, S_ref = D.recurrent_fwd(qn, kn, v.double(), beta.double(), g.double(), l.double(),
                                   return_state=True)
    _check_out(o, o_ref, torch.bfloat16, f"gdn prefill T={T}")
    _check_state(S.states, S.counts, S_ref, _fenwick_counts(T, L), torch.bfloat16,
                 f"gdn prefill T={T}")


def test_gdn_api_prefill_then_step():
    """chunk_h_gated_delta_rule: prefill with output_final_state, then decode
    steps through initial_state (gated_delta_rule_apis.py:90-128)."""
    from hattention.gated_delta_rule_apis import chunk_h_gated_delta_rule
    B, T, T1, H, K, V, L = 1, 128, 4, 2, 64, 64, 9
    q, k, v, beta, g, l = make_gdn_inputs(B, T + T1, H, K, V, L, seed=330)
    dq, dk, dv, db, dg, dl = (x.to(DEV) for x in (q, k, v, beta, g, l))
    o0, S = chunk_h_gated_delta_rule(dq[:, :T], dk[:, :T], dv[:, :T], dg[:, :T], dl[:, :T],
                                     db[:, :T], output_final_state=True,
                                     use_qk_l2norm_in_kernel=True)
    outs = [o0]
    for t in range(T, T + T1):
        sl = slice(t, t + 1)
        o1, S = chunk_h_gated_delta_rule(dq[:, sl], dk[:, sl], dv[:, sl], dg[:, sl], dl[:, sl],
                                         db[:, sl], initial_state=S, output_final_state=True,
                                         use_qk_l2norm_in_kernel=True)
        outs.append(o1)
    torch.cuda.synchronize()
    o = torch.cat(outs, 1)
    scale = K ** -0.5
    qn, kn = _gdn_normed(q, k, scale)
    # SCALE_LAMBDA: lambda / scale with q * scale, the scale cancels in o
    o_ref = D.recurrent_fwd(qn, kn, v.double(), beta.double(), g.double(),
                            l.double() / scale)
    _check_out(o, o_ref, torch.bfloat16, "gdn api prefill+step")


# ---------------------------------------------------------------------------
# Mamba-2 layer API
# ---------------------------------------------------------------------------
def test_hmamba_prefill_then_selective_state_update():
    """hmamba_chunk_scan_combined(return_final_states=True) then
    hselective_state_update per token (mamba_apis.py:263-566) against the
    recurrent oracle on the same pre-processed q, k, v, g, lambda + D x."""
    from hattention.base import HType, HStruct
    from hattention.mamba_apis import hmamba_chunk_scan_combined, hselective_state_update
    torch.manual_seed(340)
    Bsz, T, T1, H, G, P, N, L = 2, 128, 6, 4, 2, 64, 64, 10
    x = torch.randn(Bsz, T + T1, H, P).bfloat16()
    dt = torch.randn(Bsz, T + T1, H) * 0.5 - 2.0
    A = -torch.exp(torch.rand(H) * 2)
    Bm = torch.randn(Bsz, T + T1, G, N).bfloat16()
    Cm = torch.randn(Bsz, T + T1, G, N).bfloat16()
    dl = torch.randn(Bsz, T + T1, H, L).bfloat16()
    Lp = torch.randn(H, L)
    Dp = torch.randn(H)
    dt_bias = torch.randn(H) * 0.1
    kw = dict(lambda_mode="positive", lambda_level_max=L, lambda_level_base=2,
              lambda_htype=HType.WEAK, lambda_hstruct=HStruct.MAMBA2, lambda_level_fixed=True)
    d = lambda t: t.to(DEV)
    y0, S = hmamba_chunk_scan_combined(d(x[:, :T]), d(dt[:, :T]), d(A), d(Bm[:, :T]),
                                       d(Cm[:, :T]), d(dl[:, :T]), d(Lp), 64, D=d(Dp),
                                       dt_bias=d(dt_bias), dt_softplus=True,
                                       return_final_states=True, **kw)
    ys = [y0]
    for t in range(T, T + T1):
        y1, S = hselective_state_update(S, d(x[:, t]), d(dt[:, t]), d(A), d(Bm[:, t]),
                                        d(Cm[:, t]), d(dl[:, t]), d(Lp), D=d(Dp),
                                        dt_bias=d(dt_bias), dt_softplus=True, **kw)
        ys.append(y1.unsqueeze(1))
    torch.cuda.synchronize()
    y = torch.cat([yy.float() for yy in ys], 1)
    # oracle inputs: the reference's pre-processing in fp64
    dts = torch.nn.functional.softplus(dt.double() + dt_bias.double())
    v = x.double() * dts[..., None]
    g = A.double() * dts
    lam = torch.nn.functional.softplus(Lp.double() * dl.double())
    o_ref = M.recurrent_fwd(Cm.double(), Bm.double(), v, g, lam)
    y_ref = o_ref + x.double() * Dp.double()[None, None, :, None]
    _check_out(y, y_ref, torch.bfloat16, "hmamba prefill+decode")


# ---------------------------------------------------------------------------
# full size: decode after a north-star prefill equals the chunkwise forward
# ---------------------------------------------------------------------------
def test_north_star_prefill_then_decode_matches_chunkwise():
    """B=4 T=16384 H=16 K=V=64 bf16: prefill of 16384 tokens then 64 decode
    steps give the same outputs as the chunkwise forward over 16448 tokens
    (itself checked against the oracle at this size); the final level states of
    both routes agree (chunkwise ht for the levels >= 7)."""
    from hattention.base import HType, HStruct
    from hattention.kernel import hattention_kernel, hattention_prefill, hattention_step
    B, T, T1, H, K, V, L = 4, 16384, 64, 16, 64, 64, 16
    q, k, v, g, l = (x.to(DEV) for x in make_mamba2_inputs(B, T + T1, H, K, V, L, seed=350))
    print(f"[hstate] north-star prefill T={T} + {T1} steps", flush=True)
    o_full = hattention_kernel(q, k, v, None, g, l, None, False, 2, HType.WEAK, HStruct.MAMBA2)
    o0, S = hattention_prefill(q[:, :T], k[:, :T], v[:, :T], None, g[:, :T], l[:, :T], None,
                               False, 2, HType.WEAK, HStruct.MAMBA2)
    outs = []
    for t in range(T, T + T1):
        o1, S = hattention_step(S, q[:, t], k[:, t], v[:, t], None, g[:, t], l[:, t], None, 2,
                                HType.WEAK, HStruct.MAMBA2)
        outs.append(o1)
    torch.cuda.synchronize()
    mx, fro = _errs(o0, o_full[:, :T])
    assert mx < 2e-2 and fro < 1e-2, ("prefill part", mx, fro)
    mx, fro = _errs(torch.stack(outs, 1), o_full[:, T:])
    print(f"  decode tail vs chunkwise: max-rel {mx:.2e} fro {fro:.2e}", flush=True)
    assert mx < 2e-2 and fro < 1e-2, ("decode tail", mx, fro)
    assert S.host_counts == _fenwick_counts(T + T1, L)


@pytest.mark.parametrize("hs", ["MAMBA2", "GDELTA"])
@pytest.mark.parametrize("L", [7, 18])
def test_register_kernel_matches_lds_kernel(hs, L):
    """A state whose storage is not 16-byte aligned runs the register kernel
    (no LDS staging); both kernels give the same outputs and states, and both
    are checked against the recurrent oracle.  L = 18 runs the kernels' 32-level
    instances (16 < L <= 32, states of more than 32K tokens)."""
    from hattention.base import HType, HStruct
    from hattention.kernel import hattention_step
    from hattention.recurrent import HState
    hstruct = HStruct[hs]
    B, T, H, K, V = 1, 40, 2, 128, 64
    print(f"[hstate] register vs LDS kernel {hs} L={L}", flush=True)
    if hstruct == HStruct.MAMBA2:
        q, k, v, g, l = make_mamba2_inputs(B, T, H, K, V, L, seed=360, dtype=torch.float32)
        beta, scale, norm = None, None, False
    else:
        q, k, v, beta, g, l = make_gdn_inputs(B, T, H, K, V, L, seed=361, dtype=torch.float32)
        scale, norm = K ** -0.5, True
    shape = (B, H, K, V, L)
    S1 = HState(2, HType.WEAK, hstruct, shape, torch.float32, DEV)
    S2 = HState(2, HType.WEAK, hstruct, shape, torch.float32, DEV)
    n = math.prod(shape)
    S2.states = torch.zeros(n + 1, device=DEV)[1:].view(shape)   # 4-byte offset
    assert S2.states.data_ptr() % 16 != 0
    dd = [x.to(DEV) if x is not None else None for x in (q, k, v, beta, g, l)]
    o1, o2 = [], []
    for t in range(T):
        args = [x[:, t] if x is not None else None for x in dd]
        for S, outs in ((S1, o1), (S2, o2)):
            o, _ = hattention_step(S, *args, scale, 2, HType.WEAK, hstruct,
                                   use_qk_l2norm_in_kernel=norm)
            outs.append(o)
    torch.cuda.synchronize()
    torch.testing.assert_close(torch.stack(o2, 1), torch.stack(o1, 1), rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(S2.states, S1.states, rtol=1e-5, atol=1e-6)
    if hstruct == HStruct.GDELTA:
        qn, kn = _gdn_normed(q, k, scale)
        o_ref = D.recurrent_fwd(qn, kn, v.double(), beta.double(), g.double(), l.double())
        _check_out(torch.stack(o1, 1), o_ref, torch.float32, "gdn K=128")
    else:
        o_ref = M.recurrent_fwd(*(x.double() for x in (q, k, v, g, l)))
        _check_out(torch.stack(o1, 1), o_ref, torch.float32, "mamba2 K=128")
    _check_out(torch.stack(o2, 1), o_ref, torch.float32, "register kernel")


def test_stream_handle_is_the_current_stream():
    """The library's launches go to torch's current stream: the raw handle the
    binding passes equals torch.cuda.current_stream(dev).cuda_stream, on the
    default stream and inside a torch.cuda.stream context."""
    from hattention import _lib
    dev = torch.device("cuda:0")
    assert _lib.stream_handle(dev) == torch.cuda.current_stream(dev).cuda_stream
    s = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(s):
        assert _lib.stream_handle(dev) == s.cuda_stream
        assert _lib.stream_handle(torch.device("cuda")) == s.cuda_stream
    assert _lib.stream_handle(dev) == torch.cuda.current_stream(dev).cuda_stream


def test_launches_follow_a_side_stream():
    """A decode step and a chunkwise forward issued inside a torch.cuda.stream
    context run on that stream (the binding passes the current stream) and
    give bit-identical results to the same calls on the default stream."""
    from hattention.base import HType, HStruct
    from hattention.chunkwise import chunkwise_fwd
    from hattention.kernel import hattention_step
    from hattention.recurrent import HState
    dev = torch.device("cuda:0")
    B, T, H, K, V, L = 2, 2048, 2, 64, 64, 12
    q, k, v, g, l = make_mamba2_inputs(B, T, H, K, V, L, seed=41, device=dev)

    def run():
        o, gc, _ = chunkwise_fwd(q, k, v, g, l, False, 2, HType.WEAK, 64, False)
        S = HState(2, HType.WEAK, HStruct.MAMBA2, (B, H, K, V, L + 1), torch.float32, dev)
        lx = torch.cat([l, l[..., :1]], dim=-1)
        outs = []
        for t in range(8):
            ot, _ = hattention_step(S, q[:, t].contiguous(), k[:, t].contiguous(),
                                    v[:, t].contiguous(), None, g[:, t].contiguous(),
                                    lx[:, t].contiguous(), None, 2, HType.WEAK, HStruct.MAMBA2)
            outs.append(ot)
        return [o, gc, torch.stack(outs), S.states]

    ref = run()
    torch.cuda.synchronize()
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        side = run()
    s.synchronize()
    for i, (a, b) in enumerate(zip(side, ref)):
        assert torch.equal(a, b), i

"""GPU parity of the HIP log-linear Gated DeltaNet forward against the oracle.

The HIP path runs through the C-ABI (hattention.chunkwise_hgdn.chunkwise_fwd ->
libhattn_hip.so).  The checker is oracle.gdn.chunked_fwd (pinned against the
recurrent and materialised forms) in float64 on the CPU, fed the identical
bf16 inputs.  Tolerances (bf16 inputs):
max|o - o_ref| / max|o_ref| < 2e-2 and relative Frobenius error < 1e-2; the
returned Aw (bf16, (I + A)^-1 per chunk) to 1e-2 of its max; g_cumsum to 1e-5;
final states ht to 2e-2.  At full BASELINE size the oracle runs on a few
(batch, head) rows at the full length.
"""
import math

import pytest
import torch

from bench import make_gdn_inputs
from oracle import gdn as D

pytestmark = pytest.mark.gpu

TOL_MAX = 2e-2
TOL_FRO = 1e-2


def _errs(out, ref):
    out = out.double().cpu()
    ref = ref.double().cpu()
    mx = ((out - ref).abs().max() / ref.abs().max()).item()
    fro = ((out - ref).norm() / ref.norm()).item()
    return mx, fro


def _run(B, T, H, K, V, L, seed=0, rows=None, final_state=False, fp32_beta_lambda=False):
    from hattention.chunkwise_hgdn import chunkwise_fwd
    from hattention.base import HType
    q, k, v, beta, g, l = make_gdn_inputs(B, T, H, K, V, L, seed=seed)
    if fp32_beta_lambda:
        beta, l = beta.float(), l.float()
    dev = torch.device("cuda:0")
    print(f"[gdn_fwd] B={B} T={T} H={H} K={K} V={V} L={L} beta={beta.dtype}", flush=True)
    gc, o, Aw, Au, ht = chunkwise_fwd(*(x.to(dev) for x in (q, k, v, beta, g, l)), False, 2,
                                      HType.WEAK, 64, final_state)
    torch.cuda.synchronize()
    assert o.dtype == v.dtype and Aw.dtype == k.dtype and gc.dtype == torch.float32
    rows = rows or [(b, h) for b in range(B) for h in range(H)]
    for (b, h) in rows:
        sl = lambda x: x[b:b + 1, :, h:h + 1].double().cpu()
        gr, orf, awr, aur, htr = D.chunked_fwd(sl(q), sl(k), sl(v), sl(beta), sl(g), sl(l),
                                               chunk_size=64, output_final_state=final_state)
        mx, fro = _errs(o[b:b + 1, :, h:h + 1], orf)
        print(f"  row ({b},{h}) o: max-rel {mx:.2e} fro {fro:.2e}", flush=True)
        assert mx < TOL_MAX and fro < TOL_FRO, (b, h, mx, fro)
        assert torch.allclose(gc[b:b + 1, :, h:h + 1].double().cpu(), gr, rtol=1e-5, atol=1e-4)
        mx_aw, _ = _errs(Aw[b:b + 1, :, h:h + 1], awr)
        mx_au, _ = _errs(Au[b:b + 1, :, h:h + 1], aur)
        assert mx_aw < 1e-2 and mx_au < 1e-2, (mx_aw, mx_au)
        if final_state:
            nlev = math.ceil(math.log2(T // 64)) if T > 64 else 0
            for e in range(nlev):
                a = ht[b, h, :, :, 7 + e].double().cpu()
                r = htr[0, 0, :, :, 7 + e]
                # a level whose fp64 state decayed below fp32's range (|h| < 1e-30) is
                # zero in fp32, as in the reference; the floor keeps it from failing
                mx_h = ((a - r).abs().max() / max(r.abs().max().item(), 1e-30)).item()
                assert mx_h < 2e-2, (b, h, e, mx_h)
    return o


@pytest.mark.parametrize("T", [64, 128, 256, 640, 1024])
def test_small_lengths(T):
    L = 7 + (math.ceil(math.log2(T // 64)) if T > 64 else 0)
    _run(1, T, 2, 128, 128, L, seed=T)


def test_head_dim_64_and_fp32_beta_lambda():
    _run(2, 512, 2, 64, 64, 10, seed=5, fp32_beta_lambda=True)


def test_final_state():
    _run(1, 1024, 2, 128, 128, 11, seed=7, final_state=True)


def test_config3_full_size():
    # B=4 T=8192 H=16 dk=dv=128 L=14 bf16, every (batch, head) row
    _run(4, 8192, 16, 128, 128, 14, seed=1003)


@pytest.mark.parametrize("K,V", [(64, 128), (128, 64), (128, 256), (192, 192), (192, 384),
                                 (256, 64), (256, 256)])
def test_head_dims(K, V):
    """K up to 256 and V any multiple of 64 (chunkwise_hgdn.py:589-604)."""
    _run(1, 1024, 2, K, V, 11, seed=K + V, final_state=True)


def test_eight_levels():
    """T = 16384: eight inter-chunk levels (L = 15)."""
    _run(1, 16384, 2, 128, 128, 15, seed=21, final_state=True)


def test_reference_model_shape():
    """The reference's GDN model layer (configs/flame/h_gated_deltanet_mid.json:
    head_dim 192, 6 heads, expand_v 2 -> V = 384) at its training length 16384,
    every head."""
    _run(1, 16384, 6, 192, 384, 15, seed=22, final_state=True)


def test_chunk_h_gated_delta_rule_api():
    """gated_delta_rule_apis.chunk_h_gated_delta_rule == the oracle of
    HAttentionFunction's GDELTA branch (l2norm inside, scale cancels)."""
    from hattention.gated_delta_rule_apis import chunk_h_gated_delta_rule
    B, T, H, K, L = 1, 512, 2, 128, 10
    q, k, v, beta, g, l = make_gdn_inputs(B, T, H, K, K, L, seed=11)
    gen = torch.Generator().manual_seed(3)
    q = (torch.randn(B, T, H, K, generator=gen) * 3).bfloat16()   # not normalised
    dev = torch.device("cuda:0")
    o, st = chunk_h_gated_delta_rule(*(x.to(dev) for x in (q, k, v, g, l, beta)),
                                     use_qk_l2norm_in_kernel=True)
    assert st is None
    qn = D.l2norm(q.float()).bfloat16().double()
    kn = D.l2norm(k.float()).bfloat16().double()
    ref = D.chunked_fwd(qn, kn, *(x.double() for x in (v, beta, g, l)), chunk_size=64)[1]
    mx, fro = _errs(o, ref)
    assert mx < TOL_MAX and fro < TOL_FRO, (mx, fro)

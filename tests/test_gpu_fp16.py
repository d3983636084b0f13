"""fp16 inputs (the reference's kernels take fp16 q / k / v / lambda).

The Mamba-2 forward and backward (HType.WEAK) multiply fp16 q / k / v / dO
natively on fp16 MFMA (the bf16 kernels with fp16 operands; lambda read as
fp32), as the reference's fp16 dots do; the output and gradients come back in
the inputs' dtypes.  GDN with HType.WEAK does the same (fp16 MFMA, beta and
lambda read as fp32); GDN with HType.STRONG rounds fp16 q / k / v to bf16 (its
kernels are bf16 only) and reads fp16 beta / lambda as fp32.

Checks:
* Mamba-2 forward with fp16 inputs against the fp64 oracle fed the same fp16
  values: the kernel rounds the A tiles and the level states to fp16 for the
  MFMAs (as the reference's fp16 path keeps them in fp16), 2^-11 relative per
  operand (three more mantissa bits than bf16; measured 3e-4 .. 7e-4):
  max-abs/rel below 2e-3, relative Frobenius below 1e-3; and it takes the
  fp16 kernel, not the widening: the C-ABI accepts the fp16 dtype code and
  the result is farther from the oracle than the fp32-accurate run on the
  widened inputs (about 1e-5);
* Mamba-2 backward with fp16 inputs against autograd through the fp64 oracle:
  the kernels round their MFMA operands (staged tiles, the intra-chunk
  matrices, the level states) to fp16, 2^-11 relative (measured 1.5e-4 ..
  7e-4): max-abs/rel below 2e-3, relative Frobenius below 1e-3 (dg, a reverse
  cumsum with heavy cancellation, below 1e-2);
* GDN forward (o, Aw, ht) and backward (every gradient, against autograd
  through the fp64 oracle) with fp16 inputs, HType.WEAK: max-abs/rel below
  5e-3 and relative Frobenius below 2e-3 (dg below 1e-2), four times tighter
  than the bf16 GDN tests' 2e-2 / 1e-2;
* the fp16 GDN backward from a forward that kept its buffers is
  bit-identical to the recomputing one;
* GDN HType.STRONG with fp16 inputs equals, bit for bit, the bf16 run on the
  rounded inputs.
"""
import math

import pytest
import torch

from bench import make_gdn_inputs, make_mamba2_inputs
from oracle import gdn as D
from oracle.mamba2 import autograd_bwd, chunked_fwd, chunked_scan_fwd

pytestmark = pytest.mark.gpu

HALF = torch.float16
# fp16 GDN against the fp64 oracle: every MFMA operand (q_new, W_new, U, the
# level states, the intra-chunk matrices) rounded to fp16, 2^-11 relative
GDN16_MAX = 5e-3
GDN16_FRO = 2e-3


def _errs(out, ref):
    out = out.double().cpu()
    ref = ref.double().cpu()
    mx = ((out - ref).abs().max() / ref.abs().max()).item()
    fro = ((out - ref).norm() / ref.norm()).item()
    return mx, fro


@pytest.mark.parametrize("T,K,V", [(256, 64, 64), (1024, 128, 64)])
def test_mamba2_forward_backward_fp16(T, K, V):
    from hattention.base import HType
    from hattention.chunkwise import chunkwise_bwd, chunkwise_fwd
    B, H = 1, 2
    L = 7 + math.ceil(math.log2(T // 64))
    q, k, v, g, l, do = make_mamba2_inputs(B, T, H, K, V, L, seed=T + K, dtype=HALF,
                                           with_do=True)
    do = do.to(HALF)
    dev = torch.device("cuda:0")
    print(f"[fp16 mamba2] T={T} K={K} V={V}", flush=True)
    qd, kd, vd, gd, ld, dod = (x.to(dev) for x in (q, k, v, g, l, do))
    o, gc, _ = chunkwise_fwd(qd, kd, vd, gd, ld, False, 2, HType.WEAK, 64, False)
    grads = chunkwise_bwd(qd, kd, vd, gc, ld, dod, False, 2, HType.WEAK, 64)
    torch.cuda.synchronize()
    assert o.dtype == HALF and grads[0].dtype == HALF and grads[1].dtype == HALF
    assert grads[2].dtype == HALF and grads[3].dtype == torch.float32
    for h in range(H):
        sl = lambda x: x[:, :, h:h + 1].double().cpu()
        o_ref, _, _ = chunked_scan_fwd(sl(q), sl(k), sl(v), sl(g), sl(l), chunk_size=64)
        mx, fro = _errs(o[:, :, h:h + 1], o_ref)
        print(f"  head {h} o: max-rel {mx:.2e} fro {fro:.2e}", flush=True)
        assert mx < 2e-3 and fro < 1e-3, (h, mx, fro)
        ref = autograd_bwd(chunked_fwd, sl(q), sl(k), sl(v), sl(g), sl(l), sl(do), chunk_size=64)
        for name, a, r in zip(("dq", "dk", "dv", "dg", "dl"), grads, ref):
            mx, fro = _errs(a[:, :, h:h + 1], r)
            print(f"  head {h} {name}: max-rel {mx:.2e} fro {fro:.2e}", flush=True)
            tol = 1e-2 if name == "dg" else 1e-3
            assert mx < 2e-3 and fro < tol, (h, name, mx, fro)


@pytest.mark.parametrize("T,K,V,final_state", [(512, 64, 64, False), (1024, 128, 128, True)])
def test_gdn_forward_fp16_native(T, K, V, final_state):
    from hattention.base import HType
    from hattention.chunkwise_hgdn import chunkwise_fwd
    B, H = 1, 2
    L = 7 + math.ceil(math.log2(T // 64))
    q, k, v, beta, g, l = make_gdn_inputs(B, T, H, K, V, L, seed=11 + T, dtype=HALF)
    dev = torch.device("cuda:0")
    print(f"[fp16 gdn fwd] T={T} K={K} V={V} final_state={final_state}", flush=True)
    gc, o, Aw, Au, ht = chunkwise_fwd(*(x.to(dev) for x in (q, k, v, beta, g, l)), False, 2,
                                      HType.WEAK, 64, final_state)
    torch.cuda.synchronize()
    assert o.dtype == HALF and Aw.dtype == HALF and Au.dtype == HALF
    for h in range(H):
        sl = lambda x: x[:, :, h:h + 1].double().cpu()
        _, o_ref, aw_ref, _, ht_ref = D.chunked_fwd(sl(q), sl(k), sl(v), sl(beta), sl(g), sl(l),
                                                    chunk_size=64,
                                                    output_final_state=final_state)
        mx, fro = _errs(o[:, :, h:h + 1], o_ref)
        print(f"  head {h} o: max-rel {mx:.2e} fro {fro:.2e}", flush=True)
        assert mx < GDN16_MAX and fro < GDN16_FRO, (h, mx, fro)
        mx, fro = _errs(Aw[:, :, h:h + 1], aw_ref)
        print(f"  head {h} Aw: max-rel {mx:.2e} fro {fro:.2e}", flush=True)
        assert mx < GDN16_MAX and fro < GDN16_FRO, (h, mx, fro)
        if final_state:
            mx, fro = _errs(ht[:, h:h + 1], ht_ref)
            print(f"  head {h} ht: max-rel {mx:.2e} fro {fro:.2e}", flush=True)
            assert mx < GDN16_MAX and fro < GDN16_FRO, (h, mx, fro)


@pytest.mark.parametrize("T,K,V", [(512, 128, 128), (1024, 64, 64)])
def test_gdn_backward_fp16_native(T, K, V):
    from hattention.base import HType
    from hattention.chunkwise_hgdn import chunkwise_bwd, chunkwise_fwd
    B, H = 1, 2
    L = 7 + math.ceil(math.log2(T // 64))
    q, k, v, beta, g, l = make_gdn_inputs(B, T, H, K, V, L, seed=12 + T, dtype=HALF)
    do = torch.randn(B, T, H, V, generator=torch.Generator().manual_seed(5)).to(HALF)
    dev = torch.device("cuda:0")
    print(f"[fp16 gdn bwd] T={T} K={K} V={V}", flush=True)
    xs = [x.to(dev) for x in (q, k, v, beta, g, l)]
    gc, o, Aw, Au, _ = chunkwise_fwd(*xs, False, 2, HType.WEAK, 64, False)
    grads = chunkwise_bwd(xs[0], xs[1], xs[2], xs[3], gc, xs[5], Aw, Au, do.to(dev), False, 2,
                          HType.WEAK, 64)
    torch.cuda.synchronize()
    assert all(x.dtype == HALF for x in grads[:4])
    for h in range(H):
        sl = lambda x: x[:, :, h:h + 1].double().cpu()
        ref = D.autograd_bwd(D.chunked_fwd, *(sl(x) for x in (q, k, v, beta, g, l, do)),
                             chunk_size=64)
        for name, a, r in zip(("dq", "dk", "dv", "db", "dg", "dl"), grads, ref):
            mx, fro = _errs(a[:, :, h:h + 1], r)
            print(f"  head {h} {name}: max-rel {mx:.2e} fro {fro:.2e}", flush=True)
            fro_tol = 1e-2 if name == "dg" else GDN16_FRO
            assert mx < GDN16_MAX and fro < fro_tol, (h, name, mx, fro)


def test_gdn_fp16_kept_forward_is_bit_identical():
    from hattention.base import HType
    from hattention.chunkwise_hgdn import chunkwise_bwd, chunkwise_fwd_keep
    xs = [x.cuda() for x in make_gdn_inputs(1, 1024, 2, 128, 128, 11, seed=13, dtype=HALF)]
    do = torch.randn(1, 1024, 2, 128, generator=torch.Generator().manual_seed(6)).to(HALF).cuda()
    print("[fp16 gdn kept]", flush=True)
    outs = []
    for keep in (False, True):
        gc, o, Aw, Au, _, ws = chunkwise_fwd_keep(*xs, False, 2, HType.WEAK, 64, False, keep=keep)
        assert (ws is not None) == keep
        outs.append(chunkwise_bwd(xs[0], xs[1], xs[2], xs[3], gc, xs[5], Aw, Au, do, False, 2,
                                  HType.WEAK, 64, fwd_ws=ws))
    for name, a, b in zip(("dq", "dk", "dv", "db", "dg", "dl"), *outs):
        assert torch.equal(a, b), name


def test_gdn_strong_fp16_rounds_to_bf16():
    """HType.STRONG has no fp16 kernels: fp16 q / k / v give exactly the bf16
    run on the rounded inputs (fp16 beta / lambda read as fp32)."""
    from hattention.base import HType
    from hattention.chunkwise_hgdn import chunkwise_bwd, chunkwise_fwd
    q, k, v, beta, g, l = make_gdn_inputs(1, 512, 2, 64, 64, 10, seed=14, dtype=HALF)
    do = torch.randn(1, 512, 2, 64, generator=torch.Generator().manual_seed(7)).to(HALF)
    print("[fp16 gdn strong]", flush=True)

    def run(dt):
        xs = [q.to(dt), k.to(dt), v.to(dt), beta.float(), g, l.float()]
        xs = [x.cuda().contiguous() for x in xs]
        gc, o, Aw, Au, _ = chunkwise_fwd(*xs, False, 2, HType.STRONG, 64, False)
        return (o,) + chunkwise_bwd(xs[0], xs[1], xs[2], xs[3], gc, xs[5], Aw, Au,
                                    do.to(dt).cuda(), False, 2, HType.STRONG, 64)

    a, b = run(HALF), run(torch.bfloat16)
    for name, x, y in zip(("o", "dq", "dk", "dv", "db", "dg", "dl"), a, b):
        assert torch.equal(x, y.to(x.dtype)), name


@pytest.mark.parametrize("T,final_state", [(4096, False), (2048, True)])
def test_mamba2_forward_fp16_native(T, final_state):
    """The fp16 forward over several segments (the look-back and top levels) and
    its final states, against the fp64 oracle on the same fp16 values; the
    fp16 dtype code reaches the kernels (no widening to the fp32-accurate
    path, whose result is closer to the oracle)."""
    from hattention import _lib
    from hattention.base import HType
    from hattention.chunkwise import chunkwise_fwd
    B, H, K, V = 2, 2, 64, 64
    L = 7 + math.ceil(math.log2(T // 64))
    q, k, v, g, l = make_mamba2_inputs(B, T, H, K, V, L, seed=T + 3, dtype=HALF)
    dev = torch.device("cuda:0")
    print(f"[fp16 mamba2 native] T={T} final_state={final_state}", flush=True)
    xs = [x.to(dev) for x in (q, k, v, g, l)]
    o, gc, ht = chunkwise_fwd(*xs, False, 2, HType.WEAK, 64, final_state)
    o32, _, _ = chunkwise_fwd(*(x.float() for x in xs), False, 2, HType.WEAK, 64, False)
    torch.cuda.synchronize()
    assert o.dtype == HALF
    # the C-ABI takes fp16 q / k (the kernels' own dtype code, not NOT_IMPLEMENTED)
    lib = _lib.load()
    p = None
    st = lib.hattn_mamba2_chunkwise_fwd(p, p, p, p, p, p, p, p, B, T, H, H, K, V, L,
                                        _lib.DTYPE_CODES[HALF], _lib.DTYPE_CODES[HALF], 2,
                                        _lib.DTYPE_CODES[HALF], 2, 0, 64, p, 0, p)
    assert st == _lib.HATTN_ERR_VALUE   # past the dtype rules: fails on the null pointers
    for b in range(B):
        for h in range(H):
            sl = lambda x: x[b:b + 1, :, h:h + 1].double().cpu()
            o_ref, _, ht_ref = chunked_scan_fwd(sl(q), sl(k), sl(v), sl(g), sl(l), chunk_size=64,
                                                output_final_state=final_state)
            mx, fro = _errs(o[b:b + 1, :, h:h + 1], o_ref)
            mx32, _ = _errs(o32[b:b + 1, :, h:h + 1], o_ref)
            print(f"  row ({b},{h}) o: max-rel {mx:.2e} fro {fro:.2e} (fp32 path {mx32:.2e})",
                  flush=True)
            assert mx < 2e-3 and fro < 1e-3, (b, h, mx, fro)
            assert mx32 < mx
            if final_state:
                a = ht[b, h].double().cpu()
                r = ht_ref[0, 0]
                mxh = ((a - r).abs().max() / r.abs().max()).item()
                assert mxh < 2e-3, (b, h, mxh)


def test_mamba2_backward_fp16_takes_fp16_kernels():
    """The C-ABI backward takes fp16 q / k / dO (past its dtype rules: a call with
    null pointers fails as ValueError, not NotImplementedError), and fp16 needs
    fp32 lambda."""
    from hattention import _lib
    lib = _lib.load()
    p = None
    H16 = _lib.DTYPE_CODES[HALF]

    def call(dl):
        return lib.hattn_mamba2_chunkwise_bwd(p, p, p, p, p, p, p, p, p, p, p, 1, 1024, 2, 64, 64,
                                              11, H16, H16, dl, H16, 2, 0, 64, p, 1 << 30, p)
    assert call(2) == _lib.HATTN_ERR_VALUE
    assert call(H16) == _lib.HATTN_ERR_NOT_IMPLEMENTED

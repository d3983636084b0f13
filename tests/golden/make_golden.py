"""Write the golden fixtures of the chunkwise log-linear attention path.

    python tests/golden/make_golden.py

The reference ships no test vectors (its tree has no tests), so these
fixtures come from this repository's fp64 oracle (oracle/), whose forms are
pinned against each other, the reference's level recursion and closed forms
by tests/test_oracle_*.py.  They freeze small seeded cases so that a later
change to the oracle or to the HIP kernels is caught against fixed numbers:

* ``levels_T64.npz``  -- the weak level matrix of 64 tokens (base 2) from the
  restatement of the reference's recursion (hattention/base.py:41-46).
* ``mamba2_T128.npz`` -- log-linear Mamba-2, B=1 T=128 G=1 H=2 dk=dv=64 L=8:
  bf16-representable inputs (stored as float32), the upstream gradient dO,
  the output of hattention_recurrent (hattention/recurrent.py:169-216) and
  dq, dk, dv, dg, dl by autograd through it, all in float64.
* ``gdn_T128.npz``    -- log-linear Gated DeltaNet at the boundary of
  HAttentionFunction (hattention/kernel.py:100-123: q <- l2norm(q) * scale,
  k <- l2norm(k)), B=1 T=128 H=2 dk=dv=64 L=8, scale dk^-0.5: inputs, dO,
  the recurrent output and dq, dk, dv, dbeta, dg, dl by autograd through the
  chunked UT / WY form (float64, stored as float32).

Files are plain numpy archives (no pickled objects).
"""
import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import gdn as ogdn  # noqa: E402
from oracle import mamba2 as om  # noqa: E402
from oracle.levels import levels_matrix  # noqa: E402


def _bf16(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16).to(torch.float32)


def _decay(gen, B, T, H):
    A_log = torch.empty(H).uniform_(math.log(1.0), math.log(16.0), generator=gen)
    dt0 = torch.exp(torch.empty(H).uniform_(math.log(1e-3), math.log(1e-1), generator=gen))
    bias = dt0 + torch.log(-torch.expm1(-dt0))
    dt = torch.nn.functional.softplus(torch.randn(B, T, H, generator=gen) + bias).clamp(1e-3, 1e-1)
    return (-torch.exp(A_log) * dt).float()


def mamba2_case():
    B, T, G, H, K, V, L = 1, 128, 1, 2, 64, 64, 8
    gen = torch.Generator("cpu").manual_seed(2024)
    q = _bf16(torch.randn(B, T, G, K, generator=gen))
    k = _bf16(torch.randn(B, T, G, K, generator=gen))
    v = _bf16(torch.randn(B, T, H, V, generator=gen))
    g = _decay(gen, B, T, H)
    lam = _bf16(torch.nn.functional.softplus(torch.randn(B, T, H, L, generator=gen)))
    do = _bf16(torch.randn(B, T, H, V, generator=gen))
    d = [x.double() for x in (q, k, v, g, lam)]
    o = om.recurrent_fwd(*d)
    assert torch.allclose(om.chunked_fwd(*d), o, rtol=1e-10, atol=1e-10)
    dq, dk, dv, dg, dl = om.autograd_bwd(om.chunked_fwd, *d, do.double())
    return dict(q=q, k=k, v=v, g=g, l=lam, do=do, o=o, dq=dq, dk=dk, dv=dv, dg=dg, dl=dl)


def gdn_case():
    B, T, H, K, V, L = 1, 128, 2, 64, 64, 8
    gen = torch.Generator("cpu").manual_seed(2025)
    q = _bf16(torch.randn(B, T, H, K, generator=gen))
    k = _bf16(torch.randn(B, T, H, K, generator=gen))
    v = _bf16(torch.randn(B, T, H, V, generator=gen))
    g = _decay(gen, B, T, H)
    lam = _bf16(torch.nn.functional.softplus(torch.randn(B, T, H, L, generator=gen)))
    beta = _bf16(torch.sigmoid(torch.randn(B, T, H, generator=gen)))
    do = _bf16(torch.randn(B, T, H, V, generator=gen))
    scale = K ** -0.5

    def fwd(q_, k_, v_, b_, g_, l_):
        return ogdn.chunked_fwd(ogdn.l2norm(q_) * scale, ogdn.l2norm(k_), v_, b_, g_, l_)[1]

    d = [x.double() for x in (q, k, v, beta, g, lam)]
    o = ogdn.recurrent_fwd(ogdn.l2norm(d[0]) * scale, ogdn.l2norm(d[1]), *d[2:])
    assert torch.allclose(fwd(*d), o, rtol=1e-10, atol=1e-10)
    dq, dk, dv, db, dg, dl = ogdn.autograd_bwd(fwd, *d, do.double())
    return dict(q=q, k=k, v=v, beta=beta, g=g, l=lam, do=do, scale=torch.tensor(scale),
                o=o, dq=dq, dk=dk, dv=dv, dbeta=db, dg=dg, dl=dl)


def main():
    np.savez_compressed(os.path.join(HERE, "levels_T64.npz"),
                        levels=levels_matrix(64, default=0, clamp_min=0).astype(np.int8))
    for name, case in (("mamba2_T128", mamba2_case), ("gdn_T128", gdn_case)):
        arrs = {k: v.float().numpy() for k, v in case().items()}
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrs)
        print(name, {k: (v.shape, v.dtype.name) for k, v in arrs.items()})


if __name__ == "__main__":
    main()

"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces the frozen fixtures (a regression pin of the
oracle itself; the fixtures are float32 copies of float64 results).
GPU (marked ``gpu``): the HIP path through the reference's boundary
(hattention_kernel / HAttentionFunction, forward and backward) on the fixture
inputs, in bf16, against the frozen outputs and gradients: max|x - x_ref| /
max|x_ref| <= 2e-2 (BASELINE north_star bf16 tolerance).
"""
import os

import numpy as np
import pytest
import torch

from oracle import gdn as ogdn
from oracle import mamba2 as om
from oracle.levels import level_weak_recursive

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = 2e-2


def _load(name):
    with np.load(os.path.join(HERE, name), allow_pickle=False) as z:
        return {k: torch.from_numpy(z[k]) for k in z.files}


def _rel(x, ref):
    x, ref = x.double().cpu(), ref.double().cpu()
    return ((x - ref).abs().max() / ref.abs().max()).item()


def test_levels_fixture_matches_the_recursion():
    lev = _load("levels_T64.npz")["levels"]
    for t in range(64):
        for s in range(64):
            want = level_weak_recursive(t, s, 2) if s < t else 0
            assert int(lev[t, s]) == want, (t, s)


def test_mamba2_fixture_reproduced_by_the_oracle():
    f = _load("mamba2_T128.npz")
    d = [f[n].double() for n in ("q", "k", "v", "g", "l")]
    assert _rel(om.chunked_scan_fwd(*d)[0], f["o"]) < 1e-6
    grads = om.autograd_bwd(om.chunked_fwd, *d, f["do"].double())
    for name, gr in zip(("dq", "dk", "dv", "dg", "dl"), grads):
        assert _rel(gr, f[name]) < 1e-6, name


def test_gdn_fixture_reproduced_by_the_oracle():
    f = _load("gdn_T128.npz")
    d = [f[n].double() for n in ("q", "k", "v", "beta", "g", "l")]
    scale = float(f["scale"])
    o = ogdn.hattention_gdn_fwd(*d, scale=scale)
    assert _rel(o, f["o"]) < 1e-6


@pytest.mark.gpu
def test_mamba2_fixture_on_gpu():
    from hattention.base import HStruct, HType
    from hattention.kernel import hattention_kernel
    f = _load("mamba2_T128.npz")
    dev = torch.device("cuda:0")
    leaves = [f[n].to(dev, torch.bfloat16) if n != "g" else f[n].to(dev)
              for n in ("q", "k", "v", "g", "l")]
    leaves = [x.requires_grad_(True) for x in leaves]
    o = hattention_kernel(leaves[0], leaves[1], leaves[2], None, leaves[3], leaves[4], None,
                          False, 2, HType.WEAK, HStruct.MAMBA2)
    o.backward(f["do"].to(dev, torch.bfloat16))
    torch.cuda.synchronize()
    assert _rel(o.detach(), f["o"]) <= TOL
    for name, x in zip(("dq", "dk", "dv", "dg", "dl"), leaves):
        assert _rel(x.grad, f[name]) <= TOL, name


@pytest.mark.gpu
def test_gdn_fixture_on_gpu():
    from hattention.base import HStruct, HType
    from hattention.kernel import hattention_kernel
    f = _load("gdn_T128.npz")
    dev = torch.device("cuda:0")
    names = ("q", "k", "v", "beta", "g", "l")
    leaves = [f[n].to(dev, torch.bfloat16) if n != "g" else f[n].to(dev) for n in names]
    leaves = [x.requires_grad_(True) for x in leaves]
    o = hattention_kernel(leaves[0], leaves[1], leaves[2], leaves[3], leaves[4], leaves[5],
                          float(f["scale"]), False, 2, HType.WEAK, HStruct.GDELTA,
                          use_qk_l2norm_in_kernel=True)
    o.backward(f["do"].to(dev, torch.bfloat16))
    torch.cuda.synchronize()
    assert _rel(o.detach(), f["o"]) <= TOL
    for name, x in zip(("dq", "dk", "dv", "dbeta", "dg", "dl"), leaves):
        assert _rel(x.grad, f[name]) <= TOL, name

"""Host-side pieces of the GDELTA autograd boundary (kernel.py:20-29, 201-225):
the l2norm backward and the l2norm-and-scale backward must equal torch.autograd
of the forward functions (CPU, float64)."""
import torch

from hattention.kernel import l2norm_fwd, l2norm_bwd, l2norm_and_scale_fwd, l2norm_and_scale_bwd


def test_l2norm_bwd_matches_autograd():
    gen = torch.Generator().manual_seed(0)
    x = torch.randn(3, 17, 2, 64, generator=gen, dtype=torch.float64, requires_grad=True)
    dy = torch.randn(3, 17, 2, 64, generator=gen, dtype=torch.float64)
    (l2norm_fwd(x) * dy).sum().backward()
    # both sides compute in fp32 (l2norm_fwd normalises in fp32)
    assert torch.allclose(l2norm_bwd(x.detach(), dy), x.grad, rtol=1e-5, atol=1e-6)


def test_l2norm_and_scale_bwd_matches_autograd():
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(2, 9, 3, 128, generator=gen, dtype=torch.float64, requires_grad=True)
    dy = torch.randn(2, 9, 3, 128, generator=gen, dtype=torch.float64)
    scale = 128 ** -0.5
    (l2norm_and_scale_fwd(x, scale) * dy).sum().backward()
    got = l2norm_and_scale_bwd(x.detach(), dy, scale)
    assert torch.allclose(got.double(), x.grad, rtol=1e-5, atol=1e-6)

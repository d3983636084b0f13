"""The l2norm pieces of the GDELTA autograd boundary (kernel.py:20-29, 201-225):
the closed-form backward of l2norm(x) * scale that the GDN backward kernel
applies to dq and dk must equal torch.autograd of the forward (CPU, float64)."""
import torch

from oracle.gdn import l2norm, l2norm_scale_bwd


def test_l2norm_bwd_matches_autograd():
    gen = torch.Generator().manual_seed(0)
    x = torch.randn(3, 17, 2, 64, generator=gen, dtype=torch.float64, requires_grad=True)
    dy = torch.randn(3, 17, 2, 64, generator=gen, dtype=torch.float64)
    (l2norm(x) * dy).sum().backward()
    assert torch.allclose(l2norm_scale_bwd(x.detach(), dy), x.grad, rtol=1e-10, atol=1e-12)


def test_l2norm_and_scale_bwd_matches_autograd():
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(2, 9, 3, 128, generator=gen, dtype=torch.float64, requires_grad=True)
    dy = torch.randn(2, 9, 3, 128, generator=gen, dtype=torch.float64)
    scale = 128 ** -0.5
    (l2norm(x) * scale * dy).sum().backward()
    got = l2norm_scale_bwd(x.detach(), dy, scale)
    assert torch.allclose(got, x.grad, rtol=1e-10, atol=1e-12)


def test_l2norm_bwd_is_orthogonal_to_x():
    # the gradient of a scale-invariant function is orthogonal to x (up to eps)
    gen = torch.Generator().manual_seed(2)
    x = torch.randn(5, 64, generator=gen, dtype=torch.float64) * 3
    dy = torch.randn(5, 64, generator=gen, dtype=torch.float64)
    dx = l2norm_scale_bwd(x, dy, 0.125, eps=0.0)
    assert (dx * x).sum(-1).abs().max() < 1e-12

"""
The unformed product W0 * cutoff (mace_hip_kernels.conv.CutoffProduct) on the CPU: MACE's multiplication of the
radial MLP's output by the cutoff column yields it; any other use gets the real product, and its gradient is the
product rule.  Only these shapes are taken over; everything else on the MLP output is an ordinary tensor op.
"""
import torch

from mace_hip_kernels.conv import CutoffProduct, RadialWeights


def _factors(E=50, NW=24, seed=0):
    g = torch.Generator().manual_seed(seed)
    base = torch.randn(E, NW, generator=g, requires_grad=True)
    cut = torch.rand(E, 1, generator=g, requires_grad=True)
    return base, (base * 1.0).as_subclass(RadialWeights), cut


def test_product_is_unformed_but_reads_as_the_product():
    base, w0, cut = _factors()
    for p in (w0 * cut, cut * w0, torch.mul(w0, cut), w0.mul(cut)):
        assert isinstance(p, CutoffProduct) and p.shape == base.shape and p.requires_grad
        assert p.w0 is not None and p.cut is cut
        q = p + 0.0                                      # any other op runs on the real product
        assert type(q) is torch.Tensor and torch.equal(q, base * cut)


def test_gradient_is_the_product_rule():
    base, w0, cut = _factors(seed=1)
    p = w0 * cut
    gw, gc = torch.autograd.grad((p * p).sum(), (base, cut))
    rb, rc = torch.autograd.grad(((base * cut) ** 2).sum(), (base, cut))
    assert torch.allclose(gw, rb) and torch.allclose(gc, rc)


def test_other_products_stay_ordinary():
    base, w0, cut = _factors(seed=2)
    for r in (w0 * 2.0, w0 * torch.rand(50, 24), w0 * torch.rand(50, 1, dtype=torch.float64), w0 + 1, w0.sum()):
        assert not isinstance(r, (CutoffProduct, RadialWeights))

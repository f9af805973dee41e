"""
The storage-less stand-ins (mace_hip_kernels.pending): metadata queries are answered without forming the output,
any other use forms it once through an ordinary autograd-tracked computation, and a subclass's shortcut takes
precedence.  CPU only (the stand-in logic is independent of the kernels).
"""
import torch

from mace_hip_kernels.pending import Pending


_DIVS = {torch.Tensor.__truediv__, torch.Tensor.div, torch.div, torch.true_divide}


class _Doubled(Pending):
    formed = 0

    @staticmethod
    def __new__(cls, x):
        return Pending.__new__(cls, x.shape, x)

    def __init__(self, x):
        self.x = x

    def value(self):
        type(self).formed += 1
        return self.x * 2.0

    @classmethod
    def intercept(cls, func, args, kwargs):
        if func in _DIVS and isinstance(args[0], _Doubled) and args[1] == 2.0:
            return args[0].x * 1.0                    # the shortcut: (2 x) / 2 without forming 2 x
        return NotImplemented


def test_metadata_does_not_form_the_output():
    _Doubled.formed = 0
    x = torch.randn(5, 3)
    p = _Doubled(x)
    assert p.shape == (5, 3) and p.dtype == x.dtype and p.device == x.device
    assert p.dim() == 2 and p.size(1) == 3 and p.numel() == 15 and len(p) == 5
    assert _Doubled.formed == 0


def test_other_uses_form_it_once_with_autograd():
    _Doubled.formed = 0
    x = torch.randn(4, 2, requires_grad=True)
    y = _Doubled(x) + 1.0
    assert _Doubled.formed == 1 and type(y) is torch.Tensor
    assert torch.equal(y, x.detach() * 2.0 + 1.0)
    g, = torch.autograd.grad(y.sum(), x)
    assert torch.equal(g, torch.full_like(x, 2.0))


def test_shortcut_takes_precedence():
    _Doubled.formed = 0
    x = torch.randn(3, 3)
    assert torch.equal(_Doubled(x) / 2.0, x)
    assert _Doubled.formed == 0
    assert torch.equal(_Doubled(x) / 4.0, x * 0.5)      # no shortcut for 4: formed, then divided
    assert _Doubled.formed == 1

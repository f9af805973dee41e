"""
Scalar networks used by MACE around the hot path, restated after e3nn 0.4.4 ``e3nn.nn``:
``FullyConnectedNet`` (the radial MLP that produces the per-edge tensor-product weights) and ``Activation`` (the gate
of the non-linear readout).  Activations are rescaled to unit second moment under a standard normal input, which is
e3nn's ``normalize2mom``.
"""
import math

import torch

from .o3 import Irreps


class normalize2mom(torch.nn.Module):
    """f(x) * c with c = E[f(z)^2]^(-1/2), z ~ N(0, 1) (estimated on 1e6 samples of a fixed-seed CPU generator)."""

    def __init__(self, f):
        super().__init__()
        gen = torch.Generator(device='cpu').manual_seed(0)
        z = torch.randn(1_000_000, generator=gen, dtype=torch.float64)
        c = f(z).pow(2).mean().pow(-0.5).item()
        self.f = f
        self.cst = c
        self._is_id = abs(c - 1.0) < 1e-4

    def forward(self, x):
        return self.f(x) if self._is_id else self.f(x) * self.cst


class _Layer(torch.nn.Module):
    def __init__(self, h_in, h_out, act, var_in=1.0, var_out=1.0):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.randn(h_in, h_out))
        self.act = act
        self.h_in, self.var_in, self.var_out = h_in, var_in, var_out

    def forward(self, x):
        # as e3nn: hidden layers rescale after the activation; the last layer folds var_out into the weight scale
        if self.act is not None:
            x = self.act(x @ (self.weight / math.sqrt(self.h_in * self.var_in)))
            return x * math.sqrt(self.var_out)
        return x @ (self.weight / math.sqrt(self.h_in * self.var_in / self.var_out))


class FullyConnectedNet(torch.nn.Sequential):
    """Bias-free MLP ``hs[0] → … → hs[-1]``; the activation is applied after every layer but the last."""

    def __init__(self, hs, act=None, variance_in=1, variance_out=1, out_act=False):
        super().__init__()
        self.hs = list(hs)
        act = normalize2mom(act) if act is not None else None
        var_in = variance_in
        for i, (h1, h2) in enumerate(zip(self.hs, self.hs[1:])):
            last = i == len(self.hs) - 2
            a = act if (not last or out_act) else None
            var_out = variance_out if last else 1.0
            self.add_module(f'layer{i}', _Layer(h1, h2, a, var_in, var_out))
            var_in = 1.0


class Activation(torch.nn.Module):
    """Pointwise activation of scalar irreps (e3nn ``nn.Activation``); only scalar inputs are supported here."""

    def __init__(self, irreps_in, acts):
        super().__init__()
        self.irreps_in = Irreps(irreps_in)
        if len(acts) != len(self.irreps_in):
            raise ValueError('one activation per irreps block')
        for (_, ir), a in zip(self.irreps_in, acts):
            if ir.l != 0:
                raise NotImplementedError('only scalar activations')
        self.acts = torch.nn.ModuleList([normalize2mom(a) if a is not None else torch.nn.Identity() for a in acts])
        self.irreps_out = self.irreps_in

    def forward(self, x):
        outs = []
        for sl, a in zip(self.irreps_in.slices(), self.acts):
            outs.append(a(x[..., sl]))
        return torch.cat(outs, dim=-1)

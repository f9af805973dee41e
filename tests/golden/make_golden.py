"""
Writes the committed fixtures of tests/golden/ (values from the fp64 oracle; model structure from the harness):

  coupling.npz    real Wigner-3j symbols (l ≤ 3) from sympy's exact Clebsch-Gordan coefficients in e3nn's real basis,
                  and real spherical harmonics of 12 fixed vectors from scipy's complex harmonics;
  conv_small.npz  one convolution of layer 2 of a 32-channel l_max 3 model (in1 32x0e+32x1o, 10 paths) on a
                  seeded 17-node / 90-edge multigraph: inputs x, Y, W, g, sender, receiver and the oracle's out, gx,
                  gW, gY;
  sc_small.npz    the first symmetric contraction (0e+1o outputs, correlation 3) of the same model on 13 nodes of
                  seeded elements: inputs x, elem, g and the oracle's out and gx.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, 'mace-mps-kernels_amd')]
from oracle import conv as oconv  # noqa: E402
from oracle import sc as osc  # noqa: E402
from oracle import wigner  # noqa: E402


def coupling():
    out = {}
    for l1 in range(4):
        for l2 in range(4):
            for l3 in range(abs(l1 - l2), min(l1 + l2, 3) + 1):
                out[f'w3j_{l1}{l2}{l3}'] = wigner.wigner_3j(l1, l2, l3)
    v = np.random.default_rng(12345).normal(size=(12, 3)) * 3.0
    out['sh_vectors'] = v
    out['sh_values'] = wigner.spherical_harmonics(3, v)
    np.savez_compressed(os.path.join(HERE, 'coupling.npz'), **out)


def small_model():
    from mace_lite import factory
    return factory.make_model('32x0e+32x1o', 3, 3)


def conv_small(model):
    tp = model.interactions[1].conv_tp
    desc = oconv.describe_tp(tp)
    coef = oconv.path_terms(desc)
    rng = np.random.default_rng(2024)
    n, e = 17, 90
    s, r = oconv.random_graph(rng, n, e)
    nw = len(desc['ins']) * desc['mul']
    x, Y, W = rng.normal(size=(n, desc['x_dim'])), rng.normal(size=(e, desc['y_dim'])), rng.normal(size=(e, nw))
    g = rng.normal(size=(n, desc['out_dim']))
    np.savez_compressed(
        os.path.join(HERE, 'conv_small.npz'), n=n, sender=s, receiver=r, x=x, Y=Y, W=W, g=g,
        out=oconv.conv_fwd(desc, coef, x, Y, W, s, r, n), gx=oconv.conv_bwd_x(desc, coef, g, Y, W, s, r, n),
        gW=oconv.conv_bwd_w(desc, coef, x, g, Y, s, r), gY=oconv.conv_bwd_y(desc, coef, x, g, W, s, r))


def sc_small(model):
    sc = model.products[0].symmetric_contractions
    rng = np.random.default_rng(7)
    n, C, n_ell = 13, 32, 16
    x = rng.normal(size=(n, C, n_ell)) * 0.7
    elem = rng.integers(0, 4, n)
    xt = torch.tensor(x, requires_grad=True)
    parts = []
    for ct in sc.contractions:
        U = {nu: getattr(ct, f'U_matrix_{nu}').double() for nu in range(1, ct.correlation + 1)}
        U = {nu: (u if u.dim() == nu + 2 else u.unsqueeze(0)) for nu, u in U.items()}
        U = {nu: u.reshape(u.shape[0], -1, u.shape[-1]) for nu, u in U.items()}
        W = {ct.correlation: ct.weights_max.detach().double()}
        for j, w in enumerate(ct.weights):
            W[ct.correlation - 1 - j] = w.detach().double()
        parts.append(osc.sc_dense(U, W, xt, elem).reshape(n, -1))
    out = torch.cat(parts, dim=-1)
    g = rng.normal(size=tuple(out.shape))
    out.backward(torch.tensor(g))
    np.savez_compressed(os.path.join(HERE, 'sc_small.npz'), x=x, elem=elem, g=g, out=out.detach().numpy(),
                        gx=xt.grad.numpy())


def main():
    coupling()
    m = small_model()
    conv_small(m)
    sc_small(m)
    print('wrote', sorted(f for f in os.listdir(HERE) if f.endswith('.npz')))


if __name__ == '__main__':
    main()

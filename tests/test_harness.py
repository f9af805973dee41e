"""
The MACE host model (mace_lite, the unpatched e3nn path restated) and its data path, on the CPU in float64.

* forces are -dE/dr (central finite differences), stress is (1/V) dE/dε under a symmetric strain;
* energy is invariant and forces equivariant under rotation; translation and atom-permutation invariance;
* padding edges (self loops longer than r_max) change nothing, bit for bit in the energy;
* the periodic neighbour list equals a brute-force enumeration of images.
"""
import numpy as np
import pytest
import torch

from mace_lite import data as D
from mace_lite import factory
from oracle import wigner


def _model():
    return factory.make_model('8x0e+8x1o', 2, 2, elements=factory.ELEMENTS_PTCOH, dtype=torch.float64)


def _structure(seed=0):
    rng = np.random.default_rng(seed)
    s = D.fcc100_slab('Pt', (2, 2, 3), vacuum=10.0)
    s = D.add_adsorbates(s, rng, 4, ['C', 'O', 'H'], min_dist=1.0)
    return D.jitter(s, rng, 0.05)


def _ef(model, s, r_max=5.0, stress=False, pad=None):
    b = D.batch_graphs([D.graph_of(s, r_max)], factory.ELEMENTS_PTCOH, torch.float64, pad_edges_to=pad, r_max=r_max)
    out = model(D.fresh(b), compute_force=True, compute_stress=stress)
    return out


def test_forces_are_minus_energy_gradient():
    model, s = _model(), _structure()
    f = _ef(model, s)['forces'].detach().numpy()
    h = 1e-5
    for i in (0, 5, len(s) - 1):
        for k in range(3):
            sp, sm = s.copy(), s.copy()
            sp.positions[i, k] += h
            sm.positions[i, k] -= h
            fd = -(float(_ef(model, sp)['energy']) - float(_ef(model, sm)['energy'])) / (2 * h)
            assert abs(fd - f[i, k]) < 1e-7 * max(1.0, abs(fd)), (i, k, fd, f[i, k])


def test_stress_is_strain_derivative():
    model = _model()
    s = _structure(1)
    s.pbc = (True, True, True)
    out = _ef(model, s, stress=True)
    sigma = out['stress'][0].detach().numpy()
    vol = abs(np.linalg.det(s.cell))
    h = 1e-5
    for a, b in ((0, 0), (1, 1), (0, 1), (1, 2)):
        eps = np.zeros((3, 3))
        eps[a, b] = eps[b, a] = h / (2 if a != b else 1)
        def strained(sign):
            t = s.copy()
            m = np.eye(3) + sign * eps
            t.positions = t.positions @ m
            t.cell = t.cell @ m
            return float(_ef(model, t)['energy'])
        dE = (strained(1) - strained(-1)) / (2 * h)
        assert abs(dE / vol - sigma[a, b]) < 1e-7, (a, b, dE / vol, sigma[a, b])


def test_rotation_translation_permutation():
    model, s = _model(), _structure(2)
    s.pbc = (False, False, False)
    o0 = _ef(model, s)
    E0, F0 = float(o0['energy']), o0['forces'].detach().numpy()
    R = wigner.random_rotation(np.random.default_rng(3))
    o1 = _ef(model, s.rotated(R))
    assert abs(float(o1['energy']) - E0) < 1e-10
    assert np.abs(o1['forces'].detach().numpy() - F0 @ R.T).max() < 1e-10
    t = s.copy()
    t.positions = t.positions + np.array([0.3, -1.1, 2.0])
    assert abs(float(_ef(model, t)['energy']) - E0) < 1e-10
    perm = np.random.default_rng(4).permutation(len(s))
    p = D.Structure(s.numbers[perm], s.positions[perm], s.cell, s.pbc)
    o2 = _ef(model, p)
    assert abs(float(o2['energy']) - E0) < 1e-10
    assert np.abs(o2['forces'].detach().numpy() - F0[perm]).max() < 1e-10


def test_padding_edges_contribute_nothing():
    model, s = _model(), _structure(5)
    n_real = len(D.neighbour_list(s, 5.0)[0])
    o0 = _ef(model, s)
    o1 = _ef(model, s, pad=n_real + 37)
    assert float(o1['energy']) == float(o0['energy'])
    assert np.abs(o1['forces'].detach().numpy() - o0['forces'].detach().numpy()).max() < 1e-14
    with pytest.raises(ValueError):
        _ef(model, s, pad=n_real - 1)


def test_neighbour_list_bruteforce():
    rng = np.random.default_rng(6)
    s = D.jitter(D.fcc100_slab('Pt', (3, 3, 3), vacuum=8.0, pbc=(True, True, False)), rng, 0.1)
    snd, rcv, ush = D.neighbour_list(s, 4.5)
    got = set(zip(snd.tolist(), rcv.tolist(), map(tuple, ush.tolist())))
    want = set()
    for i in range(len(s)):
        for j in range(len(s)):
            for a in range(-2, 3):
                for b in range(-2, 3):
                    sh = np.array([a, b, 0])
                    if i == j and a == 0 and b == 0:
                        continue
                    d = s.positions[j] + sh @ s.cell - s.positions[i]
                    if np.linalg.norm(d) < 4.5:
                        want.add((i, j, (a, b, 0)))
    assert got == want
    order = list(zip(snd.tolist(), rcv.tolist()))
    assert order == sorted(order)

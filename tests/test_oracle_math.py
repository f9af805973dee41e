"""
Pins of the coupling coefficients and spherical harmonics (CPU).

The oracle's Wigner-3j symbols come from sympy's exact Clebsch-Gordan coefficients; the harness's come from a Racah
formula implementation.  Each is checked against facts a plausible mistake would break: sympy itself, unit norm,
selection rules, the closed form of the (0, l, l) path, the intertwiner identity C (D1 ⊗ D2) = D3 C with D taken from
the spherical harmonics (a transposed operand, a wrong phase or a permuted basis fails it), and the product identity
Σ C_ijk Y_i Y_j ∝ Y_k for l3 = l1 + l2 (ties the harmonic basis to the coupling basis).  The committed fixture
tests/golden/coupling.npz freezes the values (written by tests/golden/make_golden.py from sympy and scipy).
"""
import math
import os

import numpy as np
import pytest
import torch

from mace_lite import o3
from oracle import wigner

LMAX = 3
TRIPLES = [(l1, l2, l3) for l1 in range(LMAX + 1) for l2 in range(LMAX + 1)
           for l3 in range(abs(l1 - l2), min(l1 + l2, LMAX) + 1)]
GOLDEN = os.path.join(os.path.dirname(__file__), 'golden', 'coupling.npz')


def test_racah_cg_matches_sympy():
    from sympy.physics.wigner import clebsch_gordan
    for l1, l2, l3 in TRIPLES:
        for m1 in range(-l1, l1 + 1):
            for m2 in range(-l2, l2 + 1):
                m3 = m1 + m2
                if abs(m3) > l3:
                    continue
                want = float(clebsch_gordan(l1, l2, l3, m1, m2, m3))
                assert abs(o3._su2_cg(l1, m1, l2, m2, l3, m3) - want) < 1e-14


@pytest.mark.parametrize('l1,l2,l3', TRIPLES)
def test_wigner_3j_harness_equals_oracle(l1, l2, l3):
    a = o3.wigner_3j(l1, l2, l3, dtype=torch.float64).numpy()
    b = wigner.wigner_3j(l1, l2, l3)
    assert np.abs(a - b).max() < 1e-13
    assert abs(np.linalg.norm(b) - 1.0) < 1e-13


def test_wigner_3j_selection_rule_and_scalar_path():
    with pytest.raises(ValueError):
        o3.wigner_3j(1, 1, 3)
    for l in range(LMAX + 1):
        c = wigner.wigner_3j(0, l, l)[0]
        assert np.abs(c - np.eye(2 * l + 1) / math.sqrt(2 * l + 1)).max() < 1e-14
        c = wigner.wigner_3j(l, 0, l)[:, 0, :]
        assert np.abs(c - np.eye(2 * l + 1) / math.sqrt(2 * l + 1)).max() < 1e-14
    # (1,1,1) is the cross product up to scale
    c = wigner.wigner_3j(1, 1, 1)
    a, b = np.array([0.3, -1.2, 0.5]), np.array([0.7, 0.1, -0.4])
    v = np.einsum('ijk,i,j->k', c, a, b)
    cr = np.cross(a, b)
    assert np.abs(v / np.linalg.norm(v) - cr / np.linalg.norm(cr) * np.sign(v @ cr)).max() < 1e-12


def test_wigner_3j_intertwiner():
    rng = np.random.default_rng(0)
    R = wigner.random_rotation(rng)
    D = [wigner.wigner_D_from_sh(l, R) for l in range(LMAX + 1)]
    for d in D:
        assert np.abs(d @ d.T - np.eye(len(d))).max() < 1e-10          # orthogonal representation
    for l1, l2, l3 in TRIPLES:
        c = wigner.wigner_3j(l1, l2, l3)
        x, y = rng.normal(size=2 * l1 + 1), rng.normal(size=2 * l2 + 1)
        got = np.einsum('ijk,i,j->k', c, D[l1] @ x, D[l2] @ y)
        want = D[l3] @ np.einsum('ijk,i,j->k', c, x, y)
        assert np.abs(got - want).max() < 1e-10, (l1, l2, l3)
    # a planted mistake (one output component with the wrong sign) must fail the identity
    c = wigner.wigner_3j(1, 2, 2).copy()
    c[:, :, 1] *= -1
    x, y = rng.normal(size=3), rng.normal(size=5)
    got = np.einsum('ijk,i,j->k', c, D[1] @ x, D[2] @ y)
    want = D[2] @ np.einsum('ijk,i,j->k', c, x, y)
    assert np.abs(got - want).max() > 1e-3


def test_spherical_harmonics_closed_forms_and_norm():
    rng = np.random.default_rng(1)
    v = rng.normal(size=(40, 3)) * 2.5
    y = wigner.spherical_harmonics(LMAX, v)
    u = v / np.linalg.norm(v, axis=1, keepdims=True)
    assert np.abs(y[:, 0] - 1).max() < 1e-12
    assert np.abs(y[:, 1:4] - math.sqrt(3) * u).max() < 1e-12
    for l in range(LMAX + 1):
        assert np.abs((y[:, l * l:(l + 1) ** 2] ** 2).sum(1) - (2 * l + 1)).max() < 1e-10
    h = o3.SphericalHarmonics(o3.Irreps.spherical_harmonics(LMAX))(torch.tensor(v)).numpy()
    assert np.abs(h - y).max() < 1e-12


def test_harmonics_product_identity():
    """Σ_ij C(l1,l2,l1+l2)_ijk Y_l1,i Y_l2,j = κ Y_(l1+l2),k with one κ for all directions."""
    rng = np.random.default_rng(2)
    v = rng.normal(size=(30, 3))
    y = wigner.spherical_harmonics(LMAX, v)
    for l1 in range(1, LMAX):
        for l2 in range(1, LMAX - l1 + 1):
            l3 = l1 + l2
            c = wigner.wigner_3j(l1, l2, l3)
            p = np.einsum('ijk,ni,nj->nk', c, y[:, l1 * l1:(l1 + 1) ** 2], y[:, l2 * l2:(l2 + 1) ** 2])
            t = y[:, l3 * l3:(l3 + 1) ** 2]
            kappa = (p * t).sum() / (t * t).sum()
            assert abs(kappa) > 0.1 and np.abs(p - kappa * t).max() < 1e-12


def test_golden_coupling_fixture():
    g = np.load(GOLDEN)
    for l1, l2, l3 in TRIPLES:
        assert np.abs(g[f'w3j_{l1}{l2}{l3}'] - wigner.wigner_3j(l1, l2, l3)).max() < 1e-14
        assert np.abs(g[f'w3j_{l1}{l2}{l3}'] - o3.wigner_3j(l1, l2, l3, dtype=torch.float64).numpy()).max() < 1e-13
    y = o3.SphericalHarmonics(o3.Irreps.spherical_harmonics(LMAX))(torch.tensor(g['sh_vectors'])).numpy()
    assert np.abs(y - g['sh_values']).max() < 1e-12

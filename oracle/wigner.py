"""
Oracle for the coupling coefficients: e3nn-convention real Wigner-3j symbols and real spherical harmonics, computed
independently of ``mace_lite.o3``:

  * Clebsch-Gordan coefficients come from sympy (exact rationals/surds, ``sympy.physics.wigner.clebsch_gordan``),
    not from a Racah-formula implementation;
  * the real basis is e3nn's documented change of basis (rows m = -l..l; for m < 0 entries 1/√2 at l+|m| and -i/√2 at
    l-|m|; m = 0 → 1; m > 0 entries (-1)^m/√2 and i(-1)^m/√2; an overall (-i)^l phase); the coupling is
    ``einsum('ij,kl,mn,ikn->jlm', Q1, Q2, conj(Q3).T, CG)``, made real, divided by its Frobenius norm;
  * real spherical harmonics are scipy's complex ``sph_harm_y`` (Condon-Shortley phase) about the y axis, azimuth
    measured from z toward x, carried into the same real basis (without the (-i)^l phase), scaled to |Y_l|^2 = 2l+1.

Pinned by (tests/test_oracle_math.py): sympy exactness; selection rules; unit norm; (0,l,l) = δ/√(2l+1); the
intertwiner identity C·(D1⊗D2) = D3·C with D taken from the spherical harmonics; Σ_ij C_ijk Y_i Y_j ∝ Y_k for
l3 = l1 + l2 (ties the harmonic basis to the coupling basis); closed forms Y_0 = 1, Y_1 = √3 (x, y, z)/r.
"""
import functools
import math

import numpy as np


def _q(l, phase=True):
    q = np.zeros((2 * l + 1, 2 * l + 1), dtype=np.complex128)
    r2 = 1.0 / math.sqrt(2.0)
    for m in range(-l, 0):
        q[l + m, l + abs(m)] = r2
        q[l + m, l - abs(m)] = -1j * r2
    q[l, l] = 1.0
    for m in range(1, l + 1):
        q[l + m, l + abs(m)] = (-1) ** m * r2
        q[l + m, l - abs(m)] = 1j * (-1) ** m * r2
    return ((-1j) ** l) * q if phase else q


@functools.lru_cache(maxsize=None)
def su2_cg(l1, l2, l3):
    """Complex-basis CG tensor [2l1+1, 2l2+1, 2l3+1] from sympy (exact, then float64)."""
    from sympy.physics.wigner import clebsch_gordan
    c = np.zeros((2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1))
    for m1 in range(-l1, l1 + 1):
        for m2 in range(-l2, l2 + 1):
            m3 = m1 + m2
            if abs(m3) <= l3:
                c[l1 + m1, l2 + m2, l3 + m3] = float(clebsch_gordan(l1, l2, l3, m1, m2, m3))
    return c


@functools.lru_cache(maxsize=None)
def wigner_3j(l1, l2, l3):
    if not abs(l1 - l2) <= l3 <= l1 + l2:
        raise ValueError('triangle rule')
    c = np.einsum('ij,kl,mn,ikn->jlm', _q(l1), _q(l2), np.conj(_q(l3)).T, su2_cg(l1, l2, l3))
    assert np.abs(c.imag).max() < 1e-12
    c = c.real
    return c / np.linalg.norm(c)


def spherical_harmonics(lmax, vec):
    """[n, (lmax+1)^2] real spherical harmonics of (not necessarily unit) vectors, "component" normalisation."""
    from scipy.special import sph_harm_y
    vec = np.asarray(vec, dtype=np.float64)
    r = np.linalg.norm(vec, axis=-1)
    x, y, z = vec[:, 0] / r, vec[:, 1] / r, vec[:, 2] / r
    theta = np.arccos(np.clip(y, -1, 1))       # polar angle from +y
    phi = np.arctan2(x, z)                      # azimuth from +z toward +x
    out = []
    for l in range(lmax + 1):
        yc = np.stack([sph_harm_y(l, m, theta, phi) for m in range(-l, l + 1)], axis=-1)   # [n, 2l+1]
        q = _q(l, phase=False)
        yr = yc @ np.conj(q)                    # Y_real = q^H Y_complex  (q unitary)
        assert np.abs(yr.imag).max() < 1e-10
        out.append(yr.real * math.sqrt(4.0 * math.pi))
    return np.concatenate(out, axis=-1)


def wigner_D_from_sh(l, R, n=64, seed=0):
    """D_l(R) in the harmonic basis: least-squares solution of Y_l(R r) = D Y_l(r) over random directions."""
    rng = np.random.default_rng(seed)
    v = rng.normal(size=(n, 3))
    sl = slice(l * l, (l + 1) * (l + 1))
    a = spherical_harmonics(l, v)[:, sl]
    b = spherical_harmonics(l, v @ R.T)[:, sl]
    d, *_ = np.linalg.lstsq(a, b, rcond=None)
    return d.T


def random_rotation(rng):
    q = rng.normal(size=4)
    q /= np.linalg.norm(q)
    w, x, y, z = q
    return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - z * w), 2 * (x * z + y * w)],
                     [2 * (x * y + z * w), 1 - 2 * (x * x + z * z), 2 * (y * z - x * w)],
                     [2 * (x * z - y * w), 2 * (y * z + x * w), 1 - 2 * (x * x + y * y)]])

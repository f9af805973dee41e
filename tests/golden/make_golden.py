"""
Writes tests/golden/coupling.npz: real Wigner-3j symbols (l ≤ 3) from sympy's exact Clebsch-Gordan coefficients in
e3nn's real basis, and real spherical harmonics of 12 fixed vectors from scipy's complex harmonics — both computed by
oracle.wigner, which imports neither the product nor the harness.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import wigner  # noqa: E402


def main():
    out = {}
    for l1 in range(4):
        for l2 in range(4):
            for l3 in range(abs(l1 - l2), min(l1 + l2, 3) + 1):
                out[f'w3j_{l1}{l2}{l3}'] = wigner.wigner_3j(l1, l2, l3)
    v = np.random.default_rng(12345).normal(size=(12, 3)) * 3.0
    out['sh_vectors'] = v
    out['sh_values'] = wigner.spherical_harmonics(3, v)
    np.savez_compressed(os.path.join(HERE, 'coupling.npz'), **out)
    print('wrote', len(out), 'arrays')


if __name__ == '__main__':
    main()

"""
The spherical-harmonics kernels' generated arithmetic, checked on the CPU.

``mace_hip_kernels.edge.math_lines`` is the per-edge C code that the HIP kernels ``sh_fwd`` / ``sh_bwd`` are built
around.  Here the same lines are compiled by gcc into a plain C loop and run in fp32 against:

* the oracle's spherical harmonics (``oracle.wigner.spherical_harmonics``: scipy's complex harmonics turned real, pinned
  to closed forms and golden vectors in test_oracle_math.py) for the forward, l_max 1..3, both normalisations;
* float64 autograd of the host model's e3nn ``SphericalHarmonics`` (itself pinned to the oracle) for the backward,
  including the chain rule through v/|v| and a zero vector, where |v| is clamped to 1e-30.

Tolerances are fp32-sized: 5e-6 absolute on Y (|Y| <= ~4), 1e-5 relative to the largest gradient component.
"""
import ctypes
import shutil
import subprocess

import numpy as np
import pytest
import torch

from mace_hip_kernels import edge
from mace_lite import o3
from oracle import wigner

CASES = [(l, n) for l in (1, 2, 3) for n in ('component', 'norm')]


def _c_library(spec, tmp_path):
    m = edge.math_lines(spec)
    body = lambda lines: '\n'.join('    ' + l for l in lines)  # noqa: E731
    src = f"""
#include <math.h>
void sh_fwd(const float* vec, float* Y, long long E) {{
  for (long long e = 0; e < E; ++e) {{
    const float vx = vec[3 * e], vy = vec[3 * e + 1], vz = vec[3 * e + 2];
{body(m['head'])}
{body(m['fwd'])}
{body([f'Y[e * {spec.dim} + {c}] = Y{c};' for c in range(spec.dim)])}
  }}
}}
void sh_bwd(const float* vec, const float* gY, float* gv, long long E) {{
  for (long long e = 0; e < E; ++e) {{
    const float vx = vec[3 * e], vy = vec[3 * e + 1], vz = vec[3 * e + 2];
{body(m['head'])}
{body([f'const float g{c} = gY[e * {spec.dim} + {c}];' for c in range(spec.dim)])}
{body(m['bwd'])}
    gv[3 * e] = ox; gv[3 * e + 1] = oy; gv[3 * e + 2] = oz;
  }}
}}
"""
    c = tmp_path / 'sh.c'
    so = tmp_path / 'sh.so'
    c.write_text(src)
    subprocess.run(['gcc', '-O1', '-std=c99', '-Wall', '-Werror', '-Wno-unused-variable', '-shared', '-fPIC',
                    str(c), '-o', str(so), '-lm'], check=True)
    lib = ctypes.CDLL(str(so))
    fp = ctypes.POINTER(ctypes.c_float)
    lib.sh_fwd.argtypes = [fp, fp, ctypes.c_longlong]
    lib.sh_bwd.argtypes = [fp, fp, fp, ctypes.c_longlong]
    return lib


def _p(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _vectors(rng, n):
    v = rng.normal(size=(n, 3)) * rng.uniform(0.3, 6.0, size=(n, 1))
    v[0] = 0.0                                   # zero vector (padding edges): |v| clamped
    v[1] = (0.0, 2.5, 0.0)                       # on the polar axis
    v[2] = (1e-3, -1e-3, 2e-3)                   # short
    return v.astype(np.float32)


@pytest.mark.skipif(shutil.which('gcc') is None, reason='needs gcc')
@pytest.mark.parametrize('lmax,norm', CASES)
def test_generated_forward_matches_oracle(lmax, norm, tmp_path):
    mod = o3.SphericalHarmonics(o3.Irreps.spherical_harmonics(lmax), normalize=True, normalization=norm)
    spec = edge.SHSpec(mod)
    lib = _c_library(spec, tmp_path)
    v = _vectors(np.random.default_rng(lmax), 500)
    Y = np.zeros((len(v), spec.dim), np.float32)
    lib.sh_fwd(_p(v), _p(Y), len(v))
    ref = wigner.spherical_harmonics(lmax, v.astype(np.float64)[3:])          # component normalisation
    if norm == 'norm':
        ref = ref * np.array(spec.scale)
    assert np.abs(Y[3:] - ref).max() < 5e-6
    host = mod.double()(torch.tensor(v, dtype=torch.float64)).numpy()       # covers the special vectors too
    assert np.abs(Y - host).max() < 5e-6
    if norm == 'component':                                                   # |Y_l|^2 = 2l + 1 on the sphere
        for l in range(lmax + 1):
            assert np.abs((Y[3:, l * l:(l + 1) ** 2] ** 2).sum(1) - (2 * l + 1)).max() < 1e-4


@pytest.mark.skipif(shutil.which('gcc') is None, reason='needs gcc')
@pytest.mark.parametrize('lmax,norm', CASES)
def test_generated_backward_matches_autograd(lmax, norm, tmp_path):
    mod = o3.SphericalHarmonics(o3.Irreps.spherical_harmonics(lmax), normalize=True, normalization=norm)
    spec = edge.SHSpec(mod)
    lib = _c_library(spec, tmp_path)
    rng = np.random.default_rng(10 + lmax)
    v = _vectors(rng, 400)
    g = rng.normal(size=(len(v), spec.dim)).astype(np.float32)
    gv = np.zeros_like(v)
    lib.sh_bwd(_p(v), _p(g), _p(gv), len(v))
    vt = torch.tensor(v, dtype=torch.float64, requires_grad=True)
    ref, = torch.autograd.grad(mod.double()(vt), vt, torch.tensor(g, dtype=torch.float64))
    ref = ref.numpy()
    # the zero vector's gradient is ~1e30 (|v| clamped to 1e-30): compare it relative to itself
    assert np.abs(gv[0] - ref[0]).max() <= 1e-5 * np.abs(ref[0]).max()
    assert np.abs(gv[1:] - ref[1:]).max() <= 1e-5 * np.abs(ref[1:]).max()
    # the gradient of a function of the direction only is orthogonal to v
    dot = np.abs((gv[3:] * v[3:]).sum(1))
    assert (dot <= 1e-5 * np.linalg.norm(gv[3:], axis=1) * np.linalg.norm(v[3:], axis=1) + 1e-30).all()

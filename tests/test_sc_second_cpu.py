"""
The symmetric contraction's second-order kernels (``sc_jvp`` / ``sc_bwd2``, behind a double backward), with their
generated arithmetic checked on the CPU.

The kernels' source (``symmetric.source_second``) is compiled by g++ with a few definitions that stand in for the
HIP launch (a loop over blocks and lanes, ``mh_xcd_block`` the identity); the empty ``asm volatile`` fences that
only order loads on the GPU, and the unused buffer-resource line, are dropped.  The same generated statements then
run in fp32 and are compared with the oracle's directional derivatives (``oracle.sc.poly_jvp`` /
``poly_grad_jvp``, pinned to forward-mode and double-backward autograd of the dense contraction in
test_oracle_sc.py), in both input layouts.  Tolerance: 1e-5 relative to the largest reference value (fp32
arithmetic over hundreds of terms).
"""
import ctypes
import re
import shutil
import subprocess

import numpy as np
import pytest
import torch

from mace_hip_kernels import symmetric as hsym
from mace_lite import factory
from oracle import sc as osc

SHIM = r"""
#include <cmath>
#include <cstddef>
#define __global__
#define __launch_bounds__(x)
struct mh_dim3 { int x; };
static mh_dim3 threadIdx, blockIdx, gridDim;
static inline int mh_xcd_block(int b, int) { return b; }
"""


def _cpu_library(spec, tmp_path):
    src = hsym.source_second(spec)
    src = src[src.index('#define C '):]
    src = '\n'.join(l for l in src.split('\n') if 'asm volatile' not in l and '__amdgpu_buffer_rsrc_t' not in l
                    and not l.startswith('#define TLD'))
    names = re.findall(r'void (sc_(?:jvp|bwd2)i?_\w+)\(', src)
    drivers = []
    for k in names:
        bwd2 = k.startswith('sc_bwd2')
        params = 'const float* X, const float* V, const int* elem, const float* T, ' + \
            ('const float* G, float* GX, int N' if bwd2 else 'float* out, int N')
        args = 'X, V, elem, T, ' + ('G, GX, N' if bwd2 else 'out, N')
        drivers.append(f'extern "C" void run_{k}({params}) {{\n  gridDim.x = N;\n'
                       f'  for (int b = 0; b < N; ++b) {{ blockIdx.x = b;\n'
                       f'    for (int c = 0; c < BLOCK; ++c) {{ threadIdx.x = c; {k}({args}); }} }}\n}}')
    c = tmp_path / 'sc2.cpp'
    so = tmp_path / 'sc2.so'
    c.write_text(SHIM + src + '\n' + '\n'.join(drivers))
    subprocess.run(['g++', '-O1', '-std=c++17', '-shared', '-fPIC', '-w', str(c), '-o', str(so)], check=True)
    lib = ctypes.CDLL(str(so))
    return lib, {('bwd2' if k.startswith('sc_bwd2') else 'jvp', k.endswith('i') or 'i_c' in k): getattr(lib, f'run_{k}')
                 for k in names}


def _fp(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _oracle_tables(sc):
    """Per contraction: the oracle's symmetrised table from the module's U matrices and weights (float64)."""
    tabs = []
    for ct in sc.contractions:
        U = {}
        for nu in range(1, ct.correlation + 1):
            u = getattr(ct, f'U_matrix_{nu}').double()
            u = u if u.dim() == nu + 2 else u.unsqueeze(0)
            U[nu] = u.reshape(u.shape[0], -1, u.shape[-1]).numpy()
        W = {ct.correlation: ct.weights_max.detach().double().numpy()}
        for j, w in enumerate(ct.weights):
            W[ct.correlation - 1 - j] = w.detach().double().numpy()
        tabs.append(osc.poly_table(U, W))
    return tabs


@pytest.mark.skipif(shutil.which('g++') is None, reason='needs g++')
@pytest.mark.parametrize('hidden,lmax,corr', [('16x0e+16x1o', 2, 3), ('16x0e+16x1o+16x2e', 3, 2)])
def test_second_order_kernels_vs_oracle(hidden, lmax, corr, tmp_path):
    model = factory.make_model(hidden, lmax, corr, elements=factory.ELEMENTS_PTCOH)
    sc = model.products[0].symmetric_contractions
    spec = hsym.SCSpec(sc)
    lib, fns = _cpu_library(spec, tmp_path)
    assert set(fns) == {('jvp', False), ('bwd2', False), ('jvp', True), ('bwd2', True)}
    rng = np.random.default_rng(3)
    n, C, ne = 9, spec.C, spec.n_ell
    x, v = rng.normal(size=(n, C, ne)) * 0.7, rng.normal(size=(n, C, ne))
    g = rng.normal(size=(n, spec.out_dim))
    elem = rng.integers(0, spec.n_elem, n)
    tabs = _oracle_tables(sc)
    want_jvp, want_h, off = [], np.zeros_like(x), 0
    for tab in tabs:
        M = next(iter(tab.values())).shape[1]
        want_jvp.append(osc.poly_jvp(tab, x, elem, v).reshape(n, -1))
        want_h += osc.poly_grad_jvp(tab, x, elem, g[:, off:off + C * M].reshape(n, C, M), v)
        off += C * M
    want_jvp = np.concatenate(want_jvp, axis=1)
    T = spec.T.numpy().astype(np.float32)
    el = elem.astype(np.int32)
    gf = g.astype(np.float32)

    def irreps(a):                    # [n, C, n_ell] -> e3nn's layout [n, sum C d]
        parts, o = [], 0
        for d in spec.dims:
            parts.append(a[:, :, o:o + d].reshape(n, -1))
            o += d
        return np.ascontiguousarray(np.concatenate(parts, axis=1))

    for lay in (False, True):
        X = (irreps(x) if lay else x).astype(np.float32)
        V = (irreps(v) if lay else v).astype(np.float32)
        out = np.zeros((n, spec.out_dim), np.float32)
        fns[('jvp', lay)](_fp(X), _fp(V), _fp(el), _fp(T), _fp(out), n)
        assert np.abs(out - want_jvp).max() < 1e-5 * np.abs(want_jvp).max(), lay
        gx = np.zeros_like(X)
        fns[('bwd2', lay)](_fp(X), _fp(V), _fp(el), _fp(T), _fp(gf), _fp(gx), n)
        want = irreps(want_h) if lay else want_h
        assert np.abs(gx - want).max() < 1e-5 * np.abs(want).max(), lay

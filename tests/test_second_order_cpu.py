"""
The second-order kernels of the spherical harmonics and the radial embedding (behind a double backward), with their
generated statements checked on the CPU.

``sh_jvp`` / ``sh_bwd2`` and ``emb_jvp`` / ``emb_bwd2`` are the first-order kernels' statements (``edge.math_lines``,
``embedding.math_lines``) with ``float`` replaced by the dual-number type of ``csrc/mh_dual.h``.  Here the same
substituted statements and the same header are compiled by g++ into plain loops and run in fp32 against float64
autograd of the host model's e3nn modules: forward-mode (``torch.func.jvp``) for the JVPs, double backward for the
Hessian-vector products.  Tolerance: 1e-5 relative to the largest reference component (2e-5 for the embedding's
second derivative, whose 1/x^3 terms amplify fp32 rounding at short lengths).
"""
import ctypes
import os
import shutil
import subprocess

import numpy as np
import pytest
import torch

from mace_hip_kernels import _native, edge, embedding
from mace_lite import blocks, o3

HEADER = os.path.join(os.path.dirname(_native.DEVICE_HEADER), 'mh_dual.h')
FP = ctypes.POINTER(ctypes.c_float)


def _build(src, tmp_path, name):
    c, so = tmp_path / f'{name}.cpp', tmp_path / f'{name}.so'
    c.write_text('#include <cmath>\n#define MH_HD\n' + f'#include "{HEADER}"\n' + src)
    subprocess.run(['g++', '-O1', '-std=c++17', '-shared', '-fPIC', '-w', str(c), '-o', str(so)], check=True)
    return ctypes.CDLL(str(so))


def _p(a):
    return a.ctypes.data_as(FP)


def _body(lines):
    return '\n'.join('    ' + l for l in lines)


@pytest.mark.skipif(shutil.which('g++') is None, reason='needs g++')
@pytest.mark.parametrize('lmax,norm', [(2, 'component'), (3, 'component'), (3, 'norm')])
def test_sh_second_order_vs_autograd(lmax, norm, tmp_path):
    mod = o3.SphericalHarmonics(o3.Irreps.spherical_harmonics(lmax), normalize=True, normalization=norm)
    spec = edge.SHSpec(mod)
    m = edge.math_lines(spec)
    dz = _native.dualize
    src = f"""
extern "C" void sh_jvp(const float* vec, const float* dv, float* dY, long long E) {{
  for (long long e = 0; e < E; ++e) {{
    const mh_dual vx(vec[3 * e], dv[3 * e]), vy(vec[3 * e + 1], dv[3 * e + 1]), vz(vec[3 * e + 2], dv[3 * e + 2]);
{_body(dz(m['head']))}
{_body(dz(m['fwd']))}
{_body([f'dY[e * {spec.dim} + {c}] = Y{c}.d;' for c in range(spec.dim)])}
  }}
}}
extern "C" void sh_bwd2(const float* vec, const float* dv, const float* gY, float* gv, long long E) {{
  for (long long e = 0; e < E; ++e) {{
    const mh_dual vx(vec[3 * e], dv[3 * e]), vy(vec[3 * e + 1], dv[3 * e + 1]), vz(vec[3 * e + 2], dv[3 * e + 2]);
{_body(dz(m['head']))}
{_body([f'const float g{c} = gY[e * {spec.dim} + {c}];' for c in range(spec.dim)])}
{_body(dz(m['bwd']))}
    gv[3 * e] = ox.d; gv[3 * e + 1] = oy.d; gv[3 * e + 2] = oz.d;
  }}
}}
"""
    lib = _build(src, tmp_path, 'sh2')
    rng = np.random.default_rng(lmax)
    n = 300
    v = (rng.normal(size=(n, 3)) * rng.uniform(0.5, 5.0, size=(n, 1))).astype(np.float32)
    dv = rng.normal(size=(n, 3)).astype(np.float32)
    g = rng.normal(size=(n, spec.dim)).astype(np.float32)
    dY = np.zeros((n, spec.dim), np.float32)
    hv = np.zeros((n, 3), np.float32)
    lib.sh_jvp(_p(v), _p(dv), _p(dY), n)
    lib.sh_bwd2(_p(v), _p(dv), _p(g), _p(hv), n)
    m64 = mod.double()
    v64, dv64, g64 = (torch.tensor(a, dtype=torch.float64) for a in (v, dv, g))
    _, want_jvp = torch.func.jvp(m64, (v64,), (dv64,))
    vt = v64.clone().requires_grad_(True)
    gv, = torch.autograd.grad(m64(vt), vt, g64, create_graph=True)
    want_hv, = torch.autograd.grad((gv * dv64).sum(), vt)
    assert np.abs(dY - want_jvp.numpy()).max() < 1e-5 * np.abs(want_jvp.numpy()).max()
    assert np.abs(hv - want_hv.numpy()).max() < 1e-5 * np.abs(want_hv.numpy()).max()


@pytest.mark.skipif(shutil.which('g++') is None, reason='needs g++')
@pytest.mark.parametrize('n_basis,p', [(8, 5), (8, 6)])
def test_embedding_second_order_vs_autograd(n_basis, p, tmp_path):
    mod = blocks.RadialEmbeddingBlock(5.0, n_basis, p)
    spec = embedding.EmbSpec(mod)
    m = embedding.math_lines(spec)
    dz = _native.dualize
    src = f"""
extern "C" void emb_jvp(const float* len, const float* dl, float* dfeats, float* dcut, long long E) {{
  for (long long e = 0; e < E; ++e) {{
    const mh_dual x(len[e], dl[e]);
{_body(dz(m['head']))}
{_body(dz(m['fwd']))}
    dcut[e] = cut.d;
{_body([f'dfeats[e * {spec.n} + {k}] = f{k}.d;' for k in range(spec.n)])}
  }}
}}
extern "C" void emb_bwd2(const float* len, const float* dl, const float* gfeats, const float* gcut, float* glen,
                         long long E) {{
  for (long long e = 0; e < E; ++e) {{
    const mh_dual x(len[e], dl[e]);
{_body(dz(m['head']))}
{_body(dz(m['bwd']))}
    glen[e] = acc.d;
  }}
}}
"""
    lib = _build(src, tmp_path, 'emb2')
    rng = np.random.default_rng(p)
    n = 400
    r = rng.uniform(0.7, 6.0, size=n).astype(np.float32)          # some beyond r_max = 5 (zero envelope)
    dl = rng.normal(size=n).astype(np.float32)
    gf = rng.normal(size=(n, spec.n)).astype(np.float32)
    gc = rng.normal(size=n).astype(np.float32)
    df, dc, hx = np.zeros((n, spec.n), np.float32), np.zeros(n, np.float32), np.zeros(n, np.float32)
    lib.emb_jvp(_p(r), _p(dl), _p(df), _p(dc), n)
    lib.emb_bwd2(_p(r), _p(dl), _p(gf), _p(gc), _p(hx), n)
    m64 = mod.double()
    r64, dl64 = (torch.tensor(a, dtype=torch.float64)[:, None] for a in (r, dl))
    _, (want_f, want_c) = torch.func.jvp(m64, (r64,), (dl64,))
    rt = r64.clone().requires_grad_(True)
    f, c = m64(rt)
    gr, = torch.autograd.grad((f, c), rt, (torch.tensor(gf, dtype=torch.float64),
                                           torch.tensor(gc, dtype=torch.float64)[:, None]), create_graph=True)
    want_h, = torch.autograd.grad((gr * dl64).sum(), rt)
    assert np.abs(df - want_f.numpy()).max() < 1e-5 * np.abs(want_f.numpy()).max()
    assert np.abs(dc - want_c.numpy()[:, 0]).max() < 1e-5 * np.abs(want_c.numpy()).max()
    assert np.abs(hx - want_h.numpy()[:, 0]).max() < 2e-5 * np.abs(want_h.numpy()).max()


def test_second_order_sources_compile():
    mod = o3.SphericalHarmonics(o3.Irreps.spherical_harmonics(3), normalize=True, normalization='component')
    assert _native.compile_source(edge.source_second(edge.SHSpec(mod)))[:4] == b'\x7fELF'
    spec = embedding.EmbSpec(blocks.RadialEmbeddingBlock(5.0, 8, 6))
    assert _native.compile_source(embedding.source_second(spec))[:4] == b'\x7fELF'

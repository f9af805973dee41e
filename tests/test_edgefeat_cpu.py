"""
The fused edge kernels (``edgefeat.source``: ``edge_fwd`` = edge geometry + spherical harmonics + radial embedding,
``edge_bwd`` = the harmonics' and the embedding's backward) against the separate kernels they replace, on the CPU.

The generated HIP source of each (the fused pair, ``edge.source`` for ``sh_fwd`` / ``sh_bwd``, ``embedding.source``
for ``emb_fwd`` / ``emb_bwd``) is compiled by g++ with definitions that stand in for the HIP launch (a loop over
blocks and threads), and the edge vectors and lengths of ``geom_fwd`` are restated in numpy float32 (the same IEEE
operations in the same order; g++ forms no fused multiply-adds for x86-64 at -O1).  Every output must be bitwise
equal to the separate kernels' on the same inputs: ordinary edges, a zero-length self-loop, edges past r_max (cutoff
-0.0), one exactly at r_max, and a backward without a cutoff gradient; and the backward with a second consumer's
gradients (``gY2``, ``gfeats2``, ``gcut2``) against the separate kernels on the float32 sums.
"""
import ctypes
import shutil
import subprocess

import numpy as np
import pytest

from mace_hip_kernels import edge, edgefeat, embedding
from mace_lite import factory

SHIM = r"""
#include <cmath>
#define __global__
#define __launch_bounds__(x)
struct mh_dim3 { int x, y; };
static mh_dim3 threadIdx, blockIdx, gridDim;
static inline int mh_xcd_block(int b, int n) { (void)n; return b; }
"""


def _library(src, names, tmp_path, tag):
    body = src[src.index('#define BLOCK'):]
    drivers = []
    for k, (params, args, *tail) in names.items():
        after = f', {tail[0]}' if tail else ''             # kernel parameters that follow E
        drivers.append(f'extern "C" void run_{k}({params}, long long E) {{\n'
                       '  gridDim.x = (int)((E + BLOCK - 1) / BLOCK);\n'
                       '  for (int b = 0; b < gridDim.x; ++b) for (int t = 0; t < BLOCK; ++t) {\n'
                       f'    blockIdx.x = b; threadIdx.x = t; {k}({args}, E{after});\n'
                       '  }\n}')
    c, so = tmp_path / f'{tag}.cpp', tmp_path / f'{tag}.so'
    c.write_text(SHIM + body + '\n' + '\n'.join(drivers))
    subprocess.run(['g++', '-O1', '-std=c++17', '-shared', '-fPIC', '-w', str(c), '-o', str(so)], check=True)
    return ctypes.CDLL(str(so))


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _call(fn, *arrays, E):
    fn.argtypes = [ctypes.c_void_p] * len(arrays) + [ctypes.c_longlong]
    fn(*[_p(a) for a in arrays], E)


@pytest.mark.skipif(shutil.which('g++') is None, reason='needs g++')
@pytest.mark.parametrize('hidden,lmax', [('128x0e+128x1o', 3), ('32x0e+32x1o', 2)])
def test_fused_edge_kernels_equal_the_separate_ones(hidden, lmax, tmp_path):
    model = factory.make_model(hidden, lmax, 2, elements=factory.ELEMENTS_PTCOH)
    ss, es = edge.SHSpec(model.spherical_harmonics), embedding.EmbSpec(model.radial_embedding)
    f = 'const float* a0, const int* a1, const int* a2, const float* a3, float* a4, float* a5, float* a6, float* a7, ' \
        'float* a8'
    b = 'const float* a0, const float* a1, const float* a2, const float* a3, const float* a4, float* a5, float* a6, ' \
        'const float* a7, const float* a8, const float* a9'
    fa, ba = ', '.join(f'a{i}' for i in range(9)), ', '.join(f'a{i}' for i in range(7))
    fused = _library(edgefeat.source(ss, es), {edgefeat.kname(ss, es, 'edge_fwd'): (f, fa),
                                               edgefeat.kname(ss, es, 'edge_bwd'): (b, ba, 'a7, a8, a9')},
                     tmp_path, 'fused')
    sh = _library(edge.source(ss), {ss.kname('sh_fwd'): ('const float* a0, float* a1', 'a0, a1'),
                                    ss.kname('sh_bwd'): ('const float* a0, const float* a1, float* a2', 'a0, a1, a2')},
                  tmp_path, 'sh')
    em = _library(embedding.source(es), {
        es.kname('emb_fwd'): ('const float* a0, float* a1, float* a2', 'a0, a1, a2'),
        es.kname('emb_bwd'): ('const float* a0, const float* a1, const float* a2, float* a3', 'a0, a1, a2, a3')},
        tmp_path, 'emb')
    rng = np.random.default_rng(lmax)
    N, E = 60, 1001                                   # E not a multiple of the 256-edge block
    pos = rng.uniform(0.0, 9.0, size=(N, 3)).astype(np.float32)
    send = rng.integers(0, N, E).astype(np.int32)
    recv = rng.integers(0, N, E).astype(np.int32)
    shifts = (rng.integers(-1, 2, size=(E, 3)) * 9.0).astype(np.float32)
    send[0] = recv[0] = 3
    shifts[0] = 0.0                                   # a zero-length self-loop
    send[1], recv[1] = 0, 0
    shifts[1] = (es.r_max, 0.0, 0.0)                  # exactly at r_max: cutoff -0.0
    # geom_fwd, restated: v = (pos[r] - pos[s]) + shift and |v|, in float32
    v = (pos[recv] - pos[send]) + shifts
    ln = np.sqrt(v[:, 0] * v[:, 0] + v[:, 1] * v[:, 1] + v[:, 2] * v[:, 2]).astype(np.float32)
    assert (ln > es.r_max).any() and (ln < es.r_max).any()
    out = dict(vec=np.zeros((E, 3), np.float32), len=np.zeros(E, np.float32), Y=np.zeros((E, ss.dim), np.float32),
               feats=np.zeros((E, es.n), np.float32), cut=np.zeros(E, np.float32))
    _call(getattr(fused, 'run_' + edgefeat.kname(ss, es, 'edge_fwd')), pos, send, recv, shifts, out['vec'],
          out['len'], out['Y'], out['feats'], out['cut'], E=E)
    Y = np.zeros((E, ss.dim), np.float32)
    _call(getattr(sh, 'run_' + ss.kname('sh_fwd')), v, Y, E=E)
    feats, cut = np.zeros((E, es.n), np.float32), np.zeros(E, np.float32)
    _call(getattr(em, 'run_' + es.kname('emb_fwd')), ln, feats, cut, E=E)
    for name, want in (('vec', v), ('len', ln), ('Y', Y), ('feats', feats), ('cut', cut)):
        assert np.array_equal(out[name].view(np.uint32), np.ascontiguousarray(want).view(np.uint32)), name
    assert np.signbit(out['cut'][1]) and out['cut'][1] == 0.0          # -0.0 marks the edge at r_max
    gY = rng.normal(size=(E, ss.dim)).astype(np.float32)
    gf = rng.normal(size=(E, es.n)).astype(np.float32)
    gc = rng.normal(size=E).astype(np.float32)
    for with_cut in (True, False):
        gv, gl = np.zeros((E, 3), np.float32), np.zeros(E, np.float32)
        _call(getattr(fused, 'run_' + edgefeat.kname(ss, es, 'edge_bwd')), v, ln, gY, gf, gc if with_cut else None,
              gv, gl, None, None, None, E=E)
        wv, wl = np.zeros((E, 3), np.float32), np.zeros(E, np.float32)
        _call(getattr(sh, 'run_' + ss.kname('sh_bwd')), v, gY, wv, E=E)
        _call(getattr(em, 'run_' + es.kname('emb_bwd')), ln, gf, gc if with_cut else None, wl, E=E)
        assert np.array_equal(gv.view(np.uint32), wv.view(np.uint32)), with_cut
        assert np.array_equal(gl.view(np.uint32), wl.view(np.uint32)), with_cut
    # a second consumer's gradients (gY2, gfeats2, gcut2; each may be absent): the separate kernels on the float32
    # sums, bitwise, also with the cutoff gradient given only as the second operand
    g2 = (rng.normal(size=(E, ss.dim)).astype(np.float32), rng.normal(size=(E, es.n)).astype(np.float32),
          rng.normal(size=E).astype(np.float32))
    for first_cut, keep in ((True, (1, 1, 1)), (True, (0, 1, 0)), (False, (1, 0, 1)), (False, (0, 0, 0))):
        sec = [t if k else None for t, k in zip(g2, keep)]
        c1 = gc if first_cut else None
        gv, gl = np.zeros((E, 3), np.float32), np.zeros(E, np.float32)
        _call(getattr(fused, 'run_' + edgefeat.kname(ss, es, 'edge_bwd')), v, ln, gY, gf, c1, gv, gl, *sec, E=E)
        tY = gY if sec[0] is None else gY + sec[0]
        tf = gf if sec[1] is None else gf + sec[1]
        tc = c1 if sec[2] is None else (sec[2] if c1 is None else c1 + sec[2])
        wv, wl = np.zeros((E, 3), np.float32), np.zeros(E, np.float32)
        _call(getattr(sh, 'run_' + ss.kname('sh_bwd')), v, tY, wv, E=E)
        _call(getattr(em, 'run_' + es.kname('emb_bwd')), ln, tf, tc, wl, E=E)
        assert np.array_equal(gv.view(np.uint32), wv.view(np.uint32)), (first_cut, keep)
        assert np.array_equal(gl.view(np.uint32), wl.view(np.uint32)), (first_cut, keep)

"""
The LDS-staged symmetric-contraction kernels (``sc_fwds`` / ``sc_bwds``) and their host-side data: the walk-ordered
table (``pack_staged``), the element-grouped node slots (``group_slots``), and the kernels' generated arithmetic and
chunk pipeline run on the CPU.

For the CPU run the kernels' source is compiled by g++ with definitions that stand in for the HIP launch: a
workgroup is 256 threads (``std::thread``) that share the ``__shared__`` array and meet at ``__syncthreads`` (a
``std::barrier``), so the double-buffered chunk copies, the barrier placement and the per-slot stores run as they
would on the GPU; the empty ``asm volatile`` fences, which only order instructions there, are dropped.  Results are
compared with the oracle's polynomial (``oracle.sc.poly_eval`` / ``poly_grad``, pinned to the dense contraction and
autograd in test_oracle_sc.py).  Tolerance: 1e-5 relative to the largest reference value (fp32 arithmetic over
hundreds of terms).
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
#include <barrier>
#include <cmath>
#include <cstddef>
#include <thread>
#include <vector>
#define __global__
#define __launch_bounds__(x)
#define __shared__ static
struct mh_dim3 { int x, y; };
static thread_local mh_dim3 threadIdx;
static mh_dim3 blockIdx, gridDim;
static std::barrier<>* g_bar;
static inline void __syncthreads() { g_bar->arrive_and_wait(); }
static inline int __builtin_amdgcn_readfirstlane(int v) { return v; }
typedef float mh_f4 __attribute__((vector_size(16)));
"""


def _cpu_library(spec, tmp_path, npw, cr, split=1):
    gen = (lambda **kw: hsym._source_staged_split(spec, split=split, **kw)) if split > 1 else \
        (lambda **kw: hsym._source_staged(spec, **kw))
    src = gen(npw=npw, cr=cr)
    if spec.dims is not None:
        alt = gen(irreps=True, npw=npw, cr=cr)
        src += '\n' + alt[alt.index('#define SLOTS'):]
    src = src[src.index('#define C '):]
    src = '\n'.join(l for l in src.split('\n') if 'asm volatile' not in l)
    names = re.findall(r'void (sc_(?:fwds|bwds)2?i?_\w+)\(', src)
    nthr = split * hsym.STAGE_WAVES * hsym.WAVE
    drivers = []
    for k in names:
        bwd = k.startswith('sc_bwds')
        params = 'const float* X, const int* slots, const int* elem, const float* TS, ' + \
            ('const float* G, float* GX, int N' if bwd else 'float* out, int N')
        args = 'X, slots, elem, TS, ' + ('G, GX, N' if bwd else 'out, N')
        drivers.append(
            f'extern "C" void run_{k}({params}, int nslots) {{\n'
            f'  for (int bx = 0; bx < nslots / SLOTS; ++bx) for (int by = 0; by < NCB; ++by) {{\n'
            f'    blockIdx.x = bx; blockIdx.y = by;\n'
            f'    std::barrier<> bar({nthr}); g_bar = &bar;\n'
            f'    std::vector<std::thread> th;\n'
            f'    for (int t = 0; t < {nthr}; ++t)\n'
            f'      th.emplace_back([=] {{ threadIdx.x = t; {k}({args}); }});\n'
            f'    for (auto& h : th) h.join();\n'
            f'  }}\n}}')
    c = tmp_path / f'scs_{npw}_{cr}_{split}.cpp'
    so = tmp_path / f'scs_{npw}_{cr}_{split}.so'
    c.write_text(SHIM + src + '\n' + '\n'.join(drivers))
    subprocess.run(['g++', '-O1', '-std=c++20', '-shared', '-fPIC', '-pthread', '-w', str(c), '-o', str(so)],
                   check=True)
    lib = ctypes.CDLL(str(so))
    return lib, {('bwd' if k.startswith('sc_bwds') else 'fwd', bool(re.match(r'sc_(fwd|bwd)s2?i_', k))):
                 getattr(lib, f'run_{k}') for k in names}


def _fp(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _oracle_tables(sc):
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


def _slots_reference(elem, n_elem, gs):
    """The slot layout spelled out: per element in index order, its nodes in index order, padded with -1 to a
    multiple of gs; then -1 to ceil(n / gs) gs + n_elem gs."""
    out = []
    for e in range(n_elem):
        run = [i for i in range(len(elem)) if elem[i] == e]
        out += run + [-1] * (-len(run) % gs)
    total = -(-len(elem) // gs) * gs + n_elem * gs
    return np.array(out + [-1] * (total - len(out)), dtype=np.int32)


@pytest.mark.parametrize('counts', [[1, 8, 29, 0], [0, 0, 3, 0], [16, 16, 16, 16], [5, 0, 1, 12]])
def test_group_slots_layout(counts):
    rng = np.random.default_rng(sum(counts))
    elem = rng.permutation(np.repeat(np.arange(4), counts))
    attrs = torch.tensor(np.eye(4)[elem], dtype=torch.float32)
    slots = hsym.group_slots(attrs).numpy()
    want = _slots_reference(elem, 4, hsym.SLOT_GROUP)
    assert np.array_equal(slots, want)
    groups = slots.reshape(-1, hsym.SLOT_GROUP)
    for g in groups:                 # one element per group; a group starts with a node or is empty
        live = g[g >= 0]
        assert len(set(elem[live])) <= 1
        assert g[0] >= 0 or len(live) == 0
    assert sorted(slots[slots >= 0]) == list(range(len(elem)))


def test_pack_staged_layout():
    model = factory.make_model('32x0e+32x1o', 2, 2, elements=factory.ELEMENTS_PTCOH)
    spec = hsym.SCSpec(model.products[0].symmetric_contractions)
    wr = hsym.walk_rows(spec)
    assert sorted(wr) == list(range(spec.nrows))
    for cr in (16, 64):
        TS = hsym.pack_staged(spec, cr)
        nch = hsym.stage_chunks(spec, cr)
        assert TS.shape == (spec.n_elem, spec.ncb, nch * cr // 4, hsym.WAVE, 4)
        T = spec.T.numpy()
        for w in (0, 1, 5, spec.nrows - 1):
            for c in (0, spec.C - 1):
                assert TS[2, c // 64, w // 4, c % 64, w % 4] == T[2, wr[w], c]
        flat = TS.transpose(0, 1, 2, 4, 3).reshape(spec.n_elem, spec.ncb, -1, hsym.WAVE)   # [e][cb][w][lane]
        assert not flat[:, :, spec.nrows:].any()        # padding rows are zero


@pytest.mark.skipif(shutil.which('g++') is None, reason='needs g++')
@pytest.mark.parametrize('hidden,lmax,corr,npw,cr,split', [('16x0e+16x1o', 2, 3, 2, 64, 1),
                                                           ('16x0e+16x1o', 2, 3, 1, 16, 1),
                                                           ('16x0e+16x1o+16x2e', 3, 2, 2, 32, 1),
                                                           ('16x0e+16x1o', 2, 3, 2, 64, 2),
                                                           ('16x0e+16x1o+16x2e', 3, 2, 2, 64, 2)])
def test_staged_kernels_vs_oracle(hidden, lmax, corr, npw, cr, split, tmp_path):
    """split > 1: the split kernels, whose wave groups walk disjoint parts of the polynomial with their own LDS
    buffers, barrier counts padded to the longest group, and partial sums combined through LDS."""
    model = factory.make_model(hidden, lmax, corr, elements=factory.ELEMENTS_PTCOH)
    sc = model.products[0].symmetric_contractions
    spec = hsym.SCSpec(sc)
    assert hsym.stage_chunks(spec, cr) > 2                 # several chunk transitions
    if split > 1:                                           # several chunks per group
        nch = [-(-len(r) // cr) for r in hsym.walk_rows_split(spec, split)]
        assert min(nch) >= 2, nch
    lib, fns = _cpu_library(spec, tmp_path, npw, cr, split)
    assert set(fns) == {('fwd', False), ('bwd', False), ('fwd', True), ('bwd', True)}
    rng = np.random.default_rng(5)
    gs = hsym.STAGE_WAVES * npw
    elem = rng.permutation(np.repeat(np.arange(4), [1, gs, gs + 3, 0]))
    n, C, ne = elem.size, spec.C, spec.n_ell
    x = rng.normal(size=(n, C, ne)) * 0.7
    g = rng.normal(size=(n, spec.out_dim))
    tabs = _oracle_tables(sc)
    want_out, want_gx, off = [], np.zeros_like(x), 0
    for tab in tabs:
        M = next(iter(tab.values())).shape[1]
        want_out.append(osc.poly_eval(tab, x, elem).reshape(n, -1))
        want_gx += osc.poly_grad(tab, x, elem, g[:, off:off + C * M].reshape(n, C, M))
        off += C * M
    want_out = np.concatenate(want_out, axis=1)
    TS = hsym.pack_staged(spec, cr) if split == 1 else hsym.pack_staged_split(spec, split, cr)
    el = elem.astype(np.int32)
    gf = g.astype(np.float32)
    slots = _slots_reference(elem, 4, gs)

    def irreps(a):
        parts, o = [], 0
        for d in spec.dims:
            parts.append(a[:, :, o:o + d].reshape(n, -1))
            o += d
        return np.ascontiguousarray(np.concatenate(parts, axis=1))

    for lay in (False, True):
        X = (irreps(x) if lay else x).astype(np.float32)
        out = np.full((n, spec.out_dim), np.nan, np.float32)
        fns[('fwd', lay)](_fp(X), _fp(slots), _fp(el), _fp(TS), _fp(out), n, slots.size)
        assert np.abs(out - want_out).max() < 1e-5 * np.abs(want_out).max(), lay
        gx = np.full_like(X, np.nan)
        fns[('bwd', lay)](_fp(X), _fp(slots), _fp(el), _fp(TS), _fp(gf), _fp(gx), n, slots.size)
        want = irreps(want_gx) if lay else want_gx
        assert np.abs(gx - want).max() < 1e-5 * np.abs(want).max(), lay

"""
The GPU neighbour list (``mace_hip_kernels.neighbours``, C ABI ``mh_neighbour_list``) against the host builder
(``mace_lite.data``: scipy cKDTree + ``batch_graphs``, itself pinned to the brute-force oracle in
tests/test_oracle_neighbours.py): edge_index, unit_shifts and shifts equal element by element, in float64 and in
float32, exact and padded layouts, on every BASELINE configuration; overflow and unpaddable structures reported;
short and long per-sender segments; and an E+F call of the patched model on a GPU-built graph equal to the same
call on the host-built one.
"""
import copy

import numpy as np
import pytest
import torch

from mace_hip_kernels import neighbour_list, patch_model
from mace_hip_kernels import conv as hconv
from mace_hip_kernels import neighbours as hnl
from mace_lite import data as D
from mace_lite import factory

pytestmark = pytest.mark.gpu


def _dev():
    assert torch.cuda.is_available(), 'GPU test needs a GPU'
    return torch.device('cuda:0')


def _inputs(structs, dev, dtype=torch.float64):
    pos = torch.tensor(np.concatenate([s.positions for s in structs]), dtype=dtype, device=dev)
    cell = torch.tensor(np.stack([s.cell for s in structs]), dtype=torch.float64, device=dev)
    pbc = torch.tensor([[bool(v) for v in s.pbc] for s in structs], device=dev)
    ptr = torch.tensor(np.concatenate([[0], np.cumsum([len(s) for s in structs])]), dtype=torch.int64, device=dev)
    return pos, cell, pbc, ptr


def _host_batch(structs, r_max, pad, dtype):
    z_table = sorted({int(z) for s in structs for z in s.numbers}) or [1]
    return D.batch_graphs([D.graph_of(s, r_max) for s in structs], z_table, dtype, pad_edges_to=pad, r_max=r_max)


def _compare(nl, ref, n_real):
    assert torch.equal(nl.edge_index.cpu(), ref['edge_index'])
    assert torch.equal(nl.unit_shifts.cpu(), ref['unit_shifts'])
    assert torch.equal(nl.shifts.cpu(), ref['shifts'])
    assert int(nl.n_edges.sum()) == n_real


@pytest.mark.parametrize('cfg', [0, 1, 2, 3, 4])
def test_equals_host_builder(cfg):
    dev = _dev()
    st = factory.structures(cfg)
    structs, r_max, pad = st['structures'], st['r_max'], st['pad_edges_to']
    for dtype in (torch.float64, torch.float32):
        print(f'[case] neighbour list config {cfg} {dtype} pad={pad}', flush=True)
        ref = _host_batch(structs, r_max, pad, dtype)
        pos, cell, pbc, ptr = _inputs(structs, dev)
        nl = neighbour_list(pos, cell, ptr, r_max, pbc=pbc, pad_edges_to=pad, dtype=dtype)
        _compare(nl, ref, ref['n_real_edges'])
        assert nl.overflowed() == []
    if pad is None and cfg != 4:         # the same structures in a padded layout with room to spare
        ref0 = _host_batch(structs, r_max, None, torch.float32)
        per = max(np.bincount(ref0['batch'][ref0['edge_index'][0]].numpy(), minlength=len(structs)))
        padded = int(per) + 37
        print(f'[case] neighbour list config {cfg} padded to {padded}', flush=True)
        ref = _host_batch(structs, r_max, padded, torch.float32)
        pos, cell, pbc, ptr = _inputs(structs, dev)
        nl = neighbour_list(pos, cell, ptr, r_max, pbc=pbc, pad_edges_to=padded, dtype=torch.float32)
        _compare(nl, ref, ref['n_real_edges'])


@pytest.mark.parametrize('cfg', [0, 2])
def test_unwrapped_atoms_equal_host_builder(cfg):
    """Atoms moved by up to two cells along each periodic direction (unwrapped MD coordinates): the image search
    widens with the span of the fractional coordinates, and the list equals the host builder's on the moved atoms
    (itself equal to the wrapped list with shifted images, tests/test_oracle_neighbours.py)."""
    dev = _dev()
    st = factory.structures(cfg)
    r_max, pad = st['r_max'], st['pad_edges_to']
    rng = np.random.default_rng(5)
    moved = []
    for s in st['structures'][:4]:
        m = rng.integers(-2, 3, size=(len(s), 3)) * np.asarray(s.pbc, dtype=np.int64)
        moved.append(D.Structure(s.numbers, s.positions + m @ s.cell, s.cell, s.pbc))
    for layout in (pad, None):
        print(f'[case] neighbour list config {cfg} unwrapped, pad={layout}', flush=True)
        ref = _host_batch(moved, r_max, layout, torch.float64)
        pos, cell, pbc, ptr = _inputs(moved, dev)
        nl = neighbour_list(pos, cell, ptr, r_max, pbc=pbc, pad_edges_to=layout, dtype=torch.float64)
        _compare(nl, ref, ref['n_real_edges'])
        assert nl.overflowed() == []


def test_image_search_cut_is_reported():
    """An atom 70 cells away along the one periodic direction of a 2.5 A cell needs 72 translations: the search stops
    at 64, the structure reports n_edges -1 (padded layout: check() raises), and the exact layout raises."""
    dev = _dev()
    cell = np.eye(3) * 2.5
    far = D.Structure(np.array([78, 78]), np.array([[0.0, 0.0, 0.0], [70 * 2.5 + 1.0, 0.0, 0.0]]), cell,
                      (True, False, False))
    near = D.Structure(np.array([78, 78]), np.array([[0.0, 0.0, 0.0], [1.0, 0.0, 0.0]]), cell, (True, False, False))
    pos, cel, pbc, ptr = _inputs([near, far], dev)
    print('[case] neighbour list image search cut, padded', flush=True)
    nl = neighbour_list(pos, cel, ptr, 5.0, pbc=pbc, pad_edges_to=64, dtype=torch.float64)
    assert nl.n_edges.cpu().tolist()[1] == -1 and nl.n_edges.cpu().tolist()[0] > 0
    assert nl.overflowed() == [1]
    with pytest.raises(ValueError, match='64 cells'):
        nl.check()
    print('[case] neighbour list image search cut, exact', flush=True)
    with pytest.raises(ValueError, match='64 lattice translations'):
        neighbour_list(pos, cel, ptr, 5.0, pbc=pbc, pad_edges_to=None, dtype=torch.float64)


def test_overflow_and_unpaddable_reported():
    dev = _dev()
    st = factory.structures(2)
    structs = st['structures'][:6]
    counts = [len(D.graph_of(s, 5.0)['sender']) for s in structs]
    pad = int(np.median(counts))
    print(f'[case] neighbour list overflow: counts {counts}, pad {pad}', flush=True)
    pos, cell, pbc, ptr = _inputs(structs, dev)
    nl = neighbour_list(pos, cell, ptr, 5.0, pbc=pbc, pad_edges_to=pad, dtype=torch.float32)
    assert nl.n_edges.cpu().tolist() == counts
    assert nl.overflowed() == [i for i, c in enumerate(counts) if c > pad]
    with pytest.raises(ValueError, match='do not fit'):
        nl.check()
    for b, c in enumerate(counts):       # structures that fit are exact; the others keep pad of their edges
        seg = nl.edge_index[:, b * pad:(b + 1) * pad].cpu() - int(ptr[b])
        if c <= pad:
            assert torch.equal(seg, _host_batch([structs[b]], 5.0, pad, torch.float32)['edge_index'])
        else:
            ref = _host_batch([structs[b]], 5.0, None, torch.float32)
            us = nl.unit_shifts[b * pad:(b + 1) * pad].cpu()
            full = {(int(a), int(r), *u) for a, r, u in zip(*ref['edge_index'], ref['unit_shifts'].int().tolist())}
            kept = {(int(a), int(r), *u) for a, r, u in zip(*seg, us.int().tolist())}
            assert len(kept) == pad and kept <= full
    # an atomless structure between two others, padded: flagged, its slots in range
    s0, s1 = structs[0], structs[1]
    empty = D.Structure(np.zeros(0, dtype=np.int64), np.zeros((0, 3)), s0.cell, s0.pbc)
    pos, cell, pbc, ptr = _inputs([s0, empty, s1], dev)
    nl = neighbour_list(pos, cell, ptr, 5.0, pbc=pbc, pad_edges_to=6000, dtype=torch.float32)
    assert nl.n_edges.cpu().tolist() == [counts[0], -1, counts[1]]
    assert nl.overflowed() == [1]
    ei = nl.edge_index.cpu()
    assert int(ei.min()) >= 0 and int(ei.max()) < len(s0) + len(s1)
    ref = _host_batch([s0, s1], 5.0, 6000, torch.float32)
    assert torch.equal(ei[:, :6000], ref['edge_index'][:, :6000])
    assert torch.equal(ei[:, 12000:], ref['edge_index'][:, 6000:])


def test_small_cells_dense_clusters_and_triclinic():
    """Self images in a cell smaller than r_max; a non-periodic dense cluster (segments of ~150 edges, several
    passes of the per-sender ordering); a triclinic cell; a single atom with no neighbours."""
    dev = _dev()
    rng = np.random.default_rng(2)
    one = D.Structure(np.array([78]), np.zeros((1, 3)), np.eye(3) * 2.5, (True, True, True))
    clus = D.Structure(np.full(150, 78), rng.uniform(0, 4.0, (150, 3)), np.eye(3) * 30.0, (False, False, False))
    tcell = np.array([[7.1, 0.0, 0.0], [2.3, 6.4, 0.0], [1.1, -1.7, 5.9]])
    tri = D.Structure(np.full(40, 78), rng.uniform(0, 1, (40, 3)) @ tcell, tcell, (True, True, True))
    lone = D.Structure(np.array([1]), np.array([[1.0, 2.0, 3.0]]), np.eye(3) * 20.0, (False, False, False))
    for name, structs in (('small cell', [one]), ('cluster', [clus]), ('triclinic', [tri]), ('lone', [lone]),
                          ('mixed', [tri, one, clus, lone])):
        print(f'[case] neighbour list {name}', flush=True)
        ref = _host_batch(structs, 5.0, None, torch.float64)
        pos, cell, pbc, ptr = _inputs(structs, dev)
        nl = neighbour_list(pos, cell, ptr, 5.0, pbc=pbc, dtype=torch.float64)
        _compare(nl, ref, ref['n_real_edges'])


def test_model_on_gpu_built_graph():
    """E+F of the patched model (config 2, fp32) on the GPU-built padded graph equals the same call on the host-built
    batch (the graphs are identical; the tolerance covers the summation order of PyTorch's atomic scatter in the
    energy sums), and the graph is taken without a host check (the edge list is known to be in range)."""
    dev = _dev()
    print('[case] patched model on a GPU-built graph (config 2)', flush=True)
    model, batch, meta = factory.workload(2)
    met = copy.deepcopy(model).to(dev)
    patch_model(met, verbose=False)
    b_host = D.fresh({k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in batch.items()})
    b_gpu = D.fresh(b_host)
    # built from the float64 positions the host builder used (float32 ones could move an edge across r_max)
    pos, cell, pbc, ptr = _inputs(factory.structures(2)['structures'], dev)
    nl = neighbour_list(pos, cell, ptr, 5.0, pbc=pbc, pad_edges_to=6000, dtype=torch.float32)
    b_gpu['edge_index'], b_gpu['shifts'], b_gpu['unit_shifts'] = nl.edge_index, nl.shifts, nl.unit_shifts
    assert hnl.built_here(b_gpu['edge_index'], b_gpu['positions'].shape[0])
    pending = len(hconv._pending_checks)
    o_h = met(b_host, compute_force=True)
    o_g = met(b_gpu, compute_force=True)
    assert len(hconv._pending_checks) <= pending + 1          # only the host batch's edge list is checked
    hconv.check_graphs()
    assert float((o_h['energy'] - o_g['energy']).abs().max()) <= 1e-5
    assert float((o_h['forces'] - o_g['forces']).abs().max()) <= 1e-6
    nl.check()


def test_deferred_check_reports_out_of_range_nodes():
    """An edge list with a node outside [0, N) is clamped by the graph build (no fault) and reported by
    check_graphs(); with GRAPH_CHECK = 'sync' the call itself raises."""
    dev = _dev()
    print('[case] out-of-range edge_index: deferred and synchronous reports', flush=True)
    from mace_hip_kernels import HipConvTP
    from mace_lite import blocks as B
    from mace_lite.o3 import Irreps, TensorProduct
    sh, hid = Irreps.spherical_harmonics(2), Irreps('32x0e')
    mid, ins = B.tp_out_irreps_with_instructions(hid, sh, (sh * hid.count((0, 1))).sort()[0].simplify())
    op = HipConvTP(TensorProduct(hid, sh, mid, ins, shared_weights=False, internal_weights=False), device=dev)
    n, e = 10, 40
    x = torch.randn(n, 32, device=dev)
    Y = torch.randn(e, 9, device=dev)
    W = torch.randn(e, op.spec.nins * 32, device=dev)
    ei = torch.randint(0, n, (2, e), device=dev)
    ei[1, 7] = n + 3
    hconv.check_graphs()
    out = op(x, Y, W, ei)
    assert torch.isfinite(out).all()
    with pytest.raises(ValueError, match='outside'):
        hconv.check_graphs()
    old = hconv.GRAPH_CHECK
    try:
        hconv.GRAPH_CHECK = 'sync'
        with pytest.raises(ValueError, match='outside'):
            op(x, Y, W, ei.clone())
    finally:
        hconv.GRAPH_CHECK = old

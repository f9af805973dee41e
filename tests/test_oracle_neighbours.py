"""
Pins of the neighbour-list oracle (CPU): the brute-force float64 restatement (oracle/neighbours.py) against the host
model's independent scipy cKDTree builder on every benchmark configuration's structures (config 4's 20,000-atom bulk
on a 2,000-atom slice of it) and on a triclinic cell; against closed-form shell counts of ideal lattices; against the
edge set's own symmetry; and its padded layout against ``batch_graphs``.  A planted mistake (an image direction
dropped) must fail the cKDTree comparison.
"""
import numpy as np
import pytest

from mace_lite import data as D
from mace_lite import factory
from oracle import neighbours as onl


def _host(s, r_max):
    return D.neighbour_list(s, r_max)


def _same(a, b):
    return all(np.array_equal(x, y) for x, y in zip(a, b))


@pytest.mark.parametrize('cfg', [0, 1, 2, 3])
def test_oracle_equals_ckdtree_builder(cfg):
    st = factory.structures(cfg)
    for s in st['structures'][:4]:
        got = onl.neighbour_list(s.positions, s.cell, s.pbc, st['r_max'])
        assert _same(got, _host(s, st['r_max']))


def test_oracle_equals_ckdtree_on_bulk_slice_and_triclinic():
    s = factory.structures(4)['structures'][0]
    keep = np.argsort(s.positions[:, 2], kind='stable')[:2000]          # the bottom layers of the bulk block
    sub = D.Structure(s.numbers[keep], s.positions[keep], s.cell, s.pbc)
    assert _same(onl.neighbour_list(sub.positions, sub.cell, sub.pbc, 5.0), _host(sub, 5.0))
    rng = np.random.default_rng(3)
    cell = np.array([[7.1, 0.0, 0.0], [2.3, 6.4, 0.0], [1.1, -1.7, 5.9]])
    pos = rng.uniform(0, 1, (40, 3)) @ cell
    tri = D.Structure(np.full(40, 78), pos, cell, (True, True, True))
    got = onl.neighbour_list(pos, cell, tri.pbc, 5.0)
    assert _same(got, _host(tri, 5.0))
    # planted mistake: the images along the third lattice vector dropped
    flat = onl.neighbour_list(pos, cell, (True, True, False), 5.0)
    assert len(flat[0]) < len(got[0])


@pytest.mark.parametrize('r_max,want', [(3.0, 12), (4.5, 18), (5.0, 42)])
def test_fcc_shell_counts(r_max, want):
    """Ideal fcc, a = 3.92 A: shells at a/sqrt2 (12), a (6), a sqrt(3/2) (24): 12, 18, 42 neighbours per atom."""
    s = D.cubic_crystal(D.fcc_basis('Pt'), 3.92, (3, 3, 3))
    snd, rcv, ush = onl.neighbour_list(s.positions, s.cell, s.pbc, r_max)
    assert np.array_equal(np.bincount(snd, minlength=len(s)), np.full(len(s), want))


def test_self_images_in_a_small_cell():
    """One atom in a 2.5 A simple cubic cell, r_max 5: its own images at 2.5 |o| < 5, i.e. |o|^2 in {1, 2, 3}:
    6 + 12 + 8 = 26 edges, all self-loops with nonzero shift; the images at exactly 5 A (|o| = 2) are excluded."""
    s = D.Structure(np.array([78]), np.zeros((1, 3)), np.eye(3) * 2.5, (True, True, True))
    snd, rcv, ush = onl.neighbour_list(s.positions, s.cell, s.pbc, 5.0)
    n2 = (ush ** 2).sum(1)
    assert len(snd) == 26 and (snd == 0).all() and (rcv == 0).all() and (n2 > 0).all() and (n2 < 4).all()
    assert _same((snd, rcv, ush), _host(s, 5.0))


def test_edge_set_is_symmetric():
    s = factory.structures(0)['structures'][0]
    snd, rcv, ush = onl.neighbour_list(s.positions, s.cell, s.pbc, 5.0)
    fwd = {(a, b, *u) for a, b, u in zip(snd.tolist(), rcv.tolist(), ush.tolist())}
    assert fwd == {(b, a, *(-x for x in u)) for a, b, u in zip(snd.tolist(), rcv.tolist(), ush.tolist())}


def test_padded_layout_equals_batch_graphs():
    st = factory.structures(2)
    structs = st['structures'][:3]
    b = D.batch_graphs([D.graph_of(s, 5.0) for s in structs], st['elements'], pad_edges_to=6000, r_max=5.0)
    off, ei, us = 0, [], []
    for s in structs:
        snd, rcv, ush = onl.pad_graph(*onl.neighbour_list(s.positions, s.cell, s.pbc, 5.0), len(s), s.cell, 5.0, 6000)
        ei.append(np.stack([snd, rcv]) + off)
        us.append(ush)
        off += len(s)
    assert np.array_equal(b['edge_index'].numpy(), np.concatenate(ei, 1))
    assert np.array_equal(b['unit_shifts'].numpy(), np.concatenate(us).astype(np.float32))
    # the padding lies past r_max
    pos = b['positions'].double().numpy()
    vec = pos[b['edge_index'][1]] - pos[b['edge_index'][0]] + b['shifts'].double().numpy()
    pad = (b['edge_index'][0] == b['edge_index'][1]).numpy() & (np.abs(b['unit_shifts'].numpy()).sum(1) > 0)
    assert pad.sum() == 3 * 6000 - b['n_real_edges'] and (np.linalg.norm(vec[pad], axis=1) > 5.0).all()


def _unwrapped(s, seed, depth=2):
    """The structure with every atom moved by a random lattice vector of up to ``depth`` cells along each periodic
    direction (as in unwrapped MD coordinates), and the moves m [n, 3]."""
    rng = np.random.default_rng(seed)
    m = rng.integers(-depth, depth + 1, size=(len(s), 3)) * np.asarray(s.pbc, dtype=np.int64)
    return D.Structure(s.numbers, s.positions + m @ s.cell, s.cell, s.pbc), m


@pytest.mark.parametrize('cfg', [0, 2])
def test_unwrapped_atoms_keep_every_edge(cfg):
    """Moving atom i by the lattice vector m_i maps edge (i, j, o) to (i, j, o + m_i - m_j) and nothing else: the
    oracle and the host builder on the moved atoms give exactly the wrapped list with shifted images, in the same
    order.  The depth of atoms inside the cell, ceil(r_max / h_k), loses edges here (the planted mistake)."""
    st = factory.structures(cfg)
    r_max = st['r_max']
    for k, s in enumerate(st['structures'][:2]):
        snd, rcv, ush = onl.neighbour_list(s.positions, s.cell, s.pbc, r_max)
        u, m = _unwrapped(s, seed=10 + k)
        want = (snd, rcv, ush + m[snd] - m[rcv])
        assert _same(onl.neighbour_list(u.positions, u.cell, u.pbc, r_max), want)
        assert _same(_host(u, r_max), want)
        shallow = onl.image_depth(s.cell, s.pbc, r_max)
        assert any(d > w for d, w in zip(onl.image_depth(u.cell, u.pbc, r_max, u.positions), shallow))
        assert np.any(np.abs(want[2]).max(axis=0) > np.array(shallow))


def test_depth_of_atoms_inside_the_cell_is_the_plane_spacing_bound():
    """For atoms within one cell's span (config 2's slabs: fractional coordinates within -0.006 .. 0.98) the depth is
    exactly ceil(r_max / h_k): no search beyond what wrapped atoms need."""
    st = factory.structures(2)
    s = st['structures'][0]
    frac = s.positions @ np.linalg.inv(s.cell)
    assert (frac.max(axis=0) - frac.min(axis=0) < 1.0).all()
    assert onl.image_depth(s.cell, s.pbc, st['r_max'], s.positions) == onl.image_depth(s.cell, s.pbc, st['r_max'])

"""
Synthetic structures, periodic neighbour lists and MACE batch dictionaries (the data path of mace-torch's
``AtomicData`` / ``torch_geometric.Batch`` and ase's builders, which are not installed here).

Edges follow MACE's convention: ``edge_index = [sender, receiver]``, ``shifts = unit_shifts @ cell`` and the edge vector
is ``positions[receiver] - positions[sender] + shifts``.  Edges are sorted by (sender, receiver, shift).

Fixed-size graphs (README.md:77-78 of the reference recommends them): ``batch_graphs(..., pad_edges_to=E)`` appends
padding edges until every graph has exactly E edges.  A padding edge is a self-loop whose shift is longer than r_max, so
the radial cutoff envelope is exactly zero on it and it contributes exactly nothing to energies, forces or stress.
Padding edges are spread round-robin over the graph's atoms.
"""
import dataclasses

import numpy as np
import torch
from scipy.spatial import cKDTree

SYMBOLS = ['X', 'H', 'He', 'Li', 'Be', 'B', 'C', 'N', 'O', 'F', 'Ne', 'Na', 'Mg', 'Al', 'Si', 'P', 'S', 'Cl', 'Ar', 'K',
           'Ca', 'Sc', 'Ti', 'V', 'Cr', 'Mn', 'Fe', 'Co', 'Ni', 'Cu', 'Zn', 'Ga', 'Ge', 'As', 'Se', 'Br', 'Kr', 'Rb',
           'Sr', 'Y', 'Zr', 'Nb', 'Mo', 'Tc', 'Ru', 'Rh', 'Pd', 'Ag', 'Cd', 'In', 'Sn', 'Sb', 'Te', 'I', 'Xe', 'Cs',
           'Ba', 'La', 'Ce', 'Pr', 'Nd', 'Pm', 'Sm', 'Eu', 'Gd', 'Tb', 'Dy', 'Ho', 'Er', 'Tm', 'Yb', 'Lu', 'Hf', 'Ta',
           'W', 'Re', 'Os', 'Ir', 'Pt', 'Au', 'Hg', 'Tl', 'Pb', 'Bi', 'Po', 'At', 'Rn', 'Fr', 'Ra', 'Ac']
Z = {s: i for i, s in enumerate(SYMBOLS)}


@dataclasses.dataclass
class Structure:
    numbers: np.ndarray          # [N] atomic numbers
    positions: np.ndarray        # [N, 3] Å
    cell: np.ndarray             # [3, 3] rows are lattice vectors
    pbc: tuple = (True, True, True)

    def __len__(self):
        return len(self.numbers)

    def copy(self):
        return Structure(self.numbers.copy(), self.positions.copy(), self.cell.copy(), tuple(self.pbc))

    def rotated(self, R):
        return Structure(self.numbers.copy(), self.positions @ R.T, self.cell @ R.T, tuple(self.pbc))


# ---------------------------------------------------------------------------------------------------- builders
def fcc100_slab(symbol='Pt', size=(4, 4, 4), a=3.92, vacuum=12.0, pbc=(True, True, False)):
    """fcc(100) slab: in-plane spacing a/√2, layer spacing a/2, alternate layers offset by half a site; ``vacuum`` Å of
    empty space in total along z (half below, half above)."""
    nx, ny, nz = size
    d, h = a / np.sqrt(2.0), a / 2.0
    pos = []
    for iz in range(nz):
        off = 0.5 * (iz % 2)
        for iy in range(ny):
            for ix in range(nx):
                pos.append(((ix + off) * d, (iy + off) * d, vacuum / 2.0 + iz * h))
    cell = np.diag([nx * d, ny * d, (nz - 1) * h + vacuum])
    return Structure(np.full(len(pos), Z[symbol]), np.array(pos, dtype=np.float64), cell, tuple(pbc))


def cubic_crystal(basis, a, reps, vacuum=0.0, pbc=(True, True, True)):
    """Conventional cubic cell (``basis`` = [(symbol, fractional xyz)]) repeated ``reps``; optional vacuum along z."""
    nx, ny, nz = reps
    num, pos = [], []
    for iz in range(nz):
        for iy in range(ny):
            for ix in range(nx):
                for sym, f in basis:
                    num.append(Z[sym])
                    pos.append((np.array(f) + (ix, iy, iz)) * a)
    pos = np.array(pos, dtype=np.float64)
    cell = np.diag([nx * a, ny * a, nz * a + vacuum])
    if vacuum:
        pos[:, 2] += vacuum / 2.0
    return Structure(np.array(num), pos, cell, tuple(pbc))


def fcc_basis(sym):
    return [(sym, (0, 0, 0)), (sym, (0.5, 0.5, 0)), (sym, (0.5, 0, 0.5)), (sym, (0, 0.5, 0.5))]


def rocksalt_basis(cation, anion):
    return fcc_basis(cation) + [(anion, (0.5, 0, 0)), (anion, (0, 0.5, 0)), (anion, (0, 0, 0.5)), (anion, (0.5, 0.5, 0.5))]


def fluorite_basis(cation, anion):
    quarter = [(x, y, z) for x in (0.25, 0.75) for y in (0.25, 0.75) for z in (0.25, 0.75)]
    return fcc_basis(cation) + [(anion, q) for q in quarter]


def add_adsorbates(s, rng, n, species, height=(1.8, 2.2), min_dist=0.0, max_tries=20000, both_sides=False):
    """Add ``n`` single atoms uniformly over the x/y cell, ``height`` Å above the top layer (alternately above the top
    and below the bottom layer with ``both_sides``)."""
    s = s.copy()
    ztop, zbot = s.positions[:, 2].max(), s.positions[:, 2].min()
    num, pos = list(s.numbers), list(s.positions)
    tries = 0
    while len(num) < len(s) + n and tries < max_tries:
        tries += 1
        xy = rng.uniform(0, 1, 2) @ s.cell[:2, :2]
        up = not both_sides or (len(num) - len(s)) % 2 == 0
        p = np.array([xy[0], xy[1], (ztop + rng.uniform(*height)) if up else (zbot - rng.uniform(*height))])
        if min_dist > 0 and _min_image_dist(np.array(pos), p, s.cell, s.pbc) < min_dist:
            continue
        num.append(Z[species[rng.integers(len(species))]])
        pos.append(p)
    return Structure(np.array(num), np.array(pos), s.cell.copy(), s.pbc)


def add_molecules(s, rng, n, molecules, height=(1.8, 2.2), min_dist=1.6, max_tries=5000):
    """Add ``n`` small molecules (list of (symbols, xyz relative to the anchor atom)) rotated about z."""
    s = s.copy()
    ztop = s.positions[:, 2].max()
    num, pos = list(s.numbers), [p for p in s.positions]
    placed, tries = 0, 0
    while placed < n and tries < max_tries:
        tries += 1
        syms, rel = molecules[rng.integers(len(molecules))]
        th = rng.uniform(0, 2 * np.pi)
        rz = np.array([[np.cos(th), -np.sin(th), 0], [np.sin(th), np.cos(th), 0], [0, 0, 1]])
        rel = np.asarray(rel, dtype=np.float64) @ rz.T
        xy = rng.uniform(0, 1, 2) @ s.cell[:2, :2]
        anchor = np.array([xy[0], xy[1], ztop + rng.uniform(*height)])
        new = anchor + rel - rel[0]
        if min(_min_image_dist(np.array(pos), q, s.cell, s.pbc) for q in new) < min_dist:
            continue
        num += [Z[x] for x in syms]
        pos += list(new)
        placed += 1
    return Structure(np.array(num), np.array(pos), s.cell.copy(), s.pbc)


def _min_image_dist(pos, p, cell, pbc):
    d = pos - p
    inv = np.linalg.inv(cell)
    f = d @ inv
    for k in range(3):
        if pbc[k]:
            f[:, k] -= np.round(f[:, k])
    return np.sqrt(((f @ cell) ** 2).sum(1)).min() if len(d) else np.inf


def jitter(s, rng, sigma):
    s = s.copy()
    s.positions = s.positions + rng.normal(0.0, sigma, s.positions.shape)
    return s


MOLECULES = {
    'NH3': (['N', 'H', 'H', 'H'], [[0, 0, 0.116489], [0, 0.939731, -0.271808], [0.813831, -0.469865, -0.271808],
                                   [-0.813831, -0.469865, -0.271808]]),
    'NH2': (['N', 'H', 'H'], [[0, 0, 0], [0.8, 0, 0.6], [-0.8, 0, 0.6]]),
    'NH': (['N', 'H'], [[0, 0, 0], [0, 0, 1.03]]),
    'N': (['N'], [[0, 0, 0]]),
    'OH': (['O', 'H'], [[0, 0, 0], [0, 0, 0.98]]),
    'O': (['O'], [[0, 0, 0]]),
    'CO': (['C', 'O'], [[0, 0, 0], [0, 0, 1.15]]),
    'H': (['H'], [[0, 0, 0]]),
}


# ------------------------------------------------------------------------------------------- neighbour list
def neighbour_list(s, r_max):
    """(sender, receiver, unit_shifts) of every pair closer than r_max, periodic images included, self-pairs with zero
    shift excluded; sorted by (sender, receiver, shift)."""
    pos, cell = s.positions, s.cell
    n = len(pos)
    # images needed along each periodic lattice direction k: |o_k + f_j - f_i| < r_max / h_k (h_k the distance between
    # lattice planes, f the fractional coordinate along k), so floor(r_max / h_k + span of f) deep; ceil(r_max / h_k)
    # for atoms inside the cell
    vol = abs(np.linalg.det(cell))
    frac = pos @ np.linalg.inv(cell) if n and any(s.pbc) and vol > 0 else np.zeros((0, 3))
    reps = []
    for k in range(3):
        if s.pbc[k]:
            h = vol / np.linalg.norm(np.cross(cell[(k + 1) % 3], cell[(k + 2) % 3]))
            span = float(frac[:, k].max() - frac[:, k].min()) if len(frac) else 0.0
            reps.append(int(max(np.ceil(r_max / h), np.floor(r_max / h + span + 1e-9))))
        else:
            reps.append(0)
    offs = np.array([(i, j, k) for i in range(-reps[0], reps[0] + 1) for j in range(-reps[1], reps[1] + 1)
                     for k in range(-reps[2], reps[2] + 1)], dtype=np.int64)
    img = (pos[None, :, :] + (offs @ cell)[:, None, :]).reshape(-1, 3)
    t_img, t_pos = cKDTree(img), cKDTree(pos)
    m = t_pos.sparse_distance_matrix(t_img, r_max, output_type='ndarray')
    i = m['i'].astype(np.int64)
    jimg = m['j'].astype(np.int64)
    j, o = jimg % n, jimg // n
    sh = offs[o]
    keep = ~((i == j) & (sh == 0).all(1)) & (m['v'] < r_max)
    i, j, sh, o = i[keep], j[keep], sh[keep], o[keep]
    order = np.lexsort((o, j, i))
    return i[order], j[order], sh[order]


# --------------------------------------------------------------------------------------------------- batching
def graph_of(s, r_max):
    snd, rcv, ush = neighbour_list(s, r_max)
    return dict(structure=s, sender=snd, receiver=rcv, unit_shifts=ush)


def batch_graphs(graphs, z_table, dtype=torch.float32, device='cpu', pad_edges_to=None, r_max=None):
    """Concatenate graphs into MACE's batch dict (positions, node_attrs one-hot over ``z_table``, edge_index, shifts,
    unit_shifts, cell, batch, ptr).  With ``pad_edges_to`` every graph is padded to exactly that many edges."""
    z_index = {z: k for k, z in enumerate(z_table)}
    pos, attrs, snd, rcv, ush, sh, cells, bat, ptr = [], [], [], [], [], [], [], [], [0]
    n_real = 0
    for gi, g in enumerate(graphs):
        s = g['structure']
        n = len(s)
        off = ptr[-1]
        a = np.zeros((n, len(z_table)))
        a[np.arange(n), [z_index[int(z)] for z in s.numbers]] = 1.0
        gs, gr, gu = g['sender'], g['receiver'], g['unit_shifts']
        n_real += len(gs)
        if pad_edges_to is not None:
            extra = pad_edges_to - len(gs)
            if extra < 0:
                raise ValueError(f'graph {gi} has {len(gs)} edges > pad_edges_to={pad_edges_to}')
            if extra:
                if r_max is None:
                    raise ValueError('r_max is needed to build padding edges')
                cz = np.linalg.norm(s.cell[2])
                k = int(np.ceil((r_max + 1.0) / cz))
                at = np.arange(extra) % n
                pad_u = np.zeros((extra, 3), dtype=np.int64)
                pad_u[:, 2] = k
                gs = np.concatenate([gs, at])
                gr = np.concatenate([gr, at])
                gu = np.concatenate([gu, pad_u])
                order = np.argsort(gs, kind='stable')
                gs, gr, gu = gs[order], gr[order], gu[order]
        pos.append(s.positions)
        attrs.append(a)
        snd.append(gs + off)
        rcv.append(gr + off)
        ush.append(gu)
        sh.append(gu @ s.cell)
        cells.append(s.cell)
        bat.append(np.full(n, gi))
        ptr.append(off + n)
    t = lambda x, dt=dtype: torch.as_tensor(np.concatenate(x), dtype=dt, device=device)  # noqa: E731
    return {
        'positions': t(pos),
        'node_attrs': t(attrs),
        'edge_index': torch.stack([t(snd, torch.int64), t(rcv, torch.int64)]),
        'unit_shifts': t(ush),
        'shifts': t(sh),
        'cell': t(cells),
        'batch': t(bat, torch.int64),
        'ptr': torch.as_tensor(ptr, dtype=torch.int64, device=device),
        'n_real_edges': n_real,
    }


def fresh(batch):
    """Copy of a batch dict whose float tensors are new leaves (a model call mutates positions' grad state)."""
    return {k: (v.detach().clone() if isinstance(v, torch.Tensor) and v.is_floating_point() else v)
            for k, v in batch.items()}

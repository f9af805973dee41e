"""
Oracle for the neighbour list and the fixed-size padded graph layout (test infrastructure only; see
oracle/__init__.py).

The reference takes MACE's host-built graphs (mace-torch's data path over ase / matscipy, absent here) and
recommends fixed-size padded graphs for long runs (reference README.md:77-78); its convolution then sorts the edge
list per call (conv.py:229-235).  This restates, by brute force in float64 numpy, the graph such a builder hands the
model, in MACE's convention:
  * ``neighbour_list``  every (sender i, receiver j, unit shift o) with |pos[j] + o @ cell - pos[i]| < r_max over
                        the lattice translations that can hold one (``image_depth``: ceil(r_max / h_k) deep along
                        each periodic direction for atoms inside the cell, h_k the spacing of lattice planes k;
                        deeper for atoms outside it), without (i, i, 0); sorted by (i, j, o lexicographically);
  * ``pad_graph``       the fixed-size layout of one structure: P - E padding self-loops with unit shift (0, 0, kz),
                        kz = ceil((r_max + 1) / |c_2|), one per atom round-robin, each after its sender's real edges.

Pinned by (tests/test_oracle_neighbours.py): the independent scipy cKDTree builder of the host model
(``mace_lite.data``) on the benchmark structures and on a triclinic cell; closed-form shell counts of ideal lattices
(fcc: 12 neighbours inside the second shell, 18 inside the third; simple cubic with a cell smaller than r_max, where
one atom meets its own images); the symmetry of the edge set (for every (i, j, o) there is (j, i, -o)); padded
layouts whose every sender segment is sorted and whose padding edges lie exactly past r_max.
"""
import numpy as np


def image_depth(cell, pbc, r_max, pos=None):
    """Translations per lattice direction that hold every edge: along periodic k an edge needs
    |o_k + f_j,k - f_i,k| < r_max / h_k (h_k = |det| / |c_{k+1} x c_{k+2}|, f the fractional coordinates), so
    |o_k| <= floor(r_max / h_k + span_k) with span_k the range of f_k over the atoms ``pos``; at least
    ceil(r_max / h_k), the depth for atoms inside the cell."""
    vol = abs(np.linalg.det(cell))
    frac = None if pos is None or len(pos) == 0 or not any(pbc) or vol == 0 else \
        np.asarray(pos, np.float64) @ np.linalg.inv(cell)
    reps = []
    for k in range(3):
        if pbc[k]:
            h = vol / np.linalg.norm(np.cross(cell[(k + 1) % 3], cell[(k + 2) % 3]))
            span = 0.0 if frac is None else float(frac[:, k].max() - frac[:, k].min())
            reps.append(int(max(np.ceil(r_max / h), np.floor(r_max / h + span + 1e-9))))
        else:
            reps.append(0)
    return reps


def neighbour_list(pos, cell, pbc, r_max):
    """(sender, receiver, unit_shifts [E, 3]) by brute force: every atom pair and every image, in float64."""
    pos = np.asarray(pos, dtype=np.float64)
    cell = np.asarray(cell, dtype=np.float64)
    n = len(pos)
    reps = image_depth(cell, pbc, r_max, pos)
    snd, rcv, ush = [], [], []
    offs = [(a, b, c) for a in range(-reps[0], reps[0] + 1) for b in range(-reps[1], reps[1] + 1)
            for c in range(-reps[2], reps[2] + 1)]
    for oi, o in enumerate(offs):
        shift = np.asarray(o, dtype=np.float64) @ cell
        d = (pos[None, :, :] + shift[None, None, :]) - pos[:, None, :]        # [sender i, receiver j]
        dist = np.sqrt((d[..., 0] * d[..., 0] + d[..., 1] * d[..., 1]) + d[..., 2] * d[..., 2])
        hit = dist < r_max
        if o == (0, 0, 0):
            np.fill_diagonal(hit, False)
        i, j = np.nonzero(hit)
        snd.append(i)
        rcv.append(j)
        ush.append(np.full((len(i), 3), o, dtype=np.int64) if len(i) else np.zeros((0, 3), np.int64))
        ush[-1] = np.concatenate([ush[-1], np.full((len(i), 1), oi, dtype=np.int64)], axis=1)
    snd, rcv, ush = np.concatenate(snd), np.concatenate(rcv), np.concatenate(ush)
    order = np.lexsort((ush[:, 3], rcv, snd))
    return snd[order], rcv[order], ush[order, :3]


def pad_graph(snd, rcv, ush, n, cell, r_max, pad_to):
    """One structure's edges in the fixed-size layout: sorted real edges, then P - E padding self-loops (one per atom,
    round-robin from atom 0) with unit shift (0, 0, kz), each placed after its sender's real edges."""
    extra = pad_to - len(snd)
    if extra < 0:
        raise ValueError(f'{len(snd)} edges > pad_to={pad_to}')
    kz = int(np.ceil((r_max + 1.0) / np.linalg.norm(cell[2])))
    at = np.arange(extra) % n
    pad_u = np.zeros((extra, 3), dtype=np.int64)
    pad_u[:, 2] = kz
    s = np.concatenate([snd, at])
    r = np.concatenate([rcv, at])
    u = np.concatenate([ush, pad_u])
    order = np.argsort(s, kind='stable')
    return s[order], r[order], u[order]

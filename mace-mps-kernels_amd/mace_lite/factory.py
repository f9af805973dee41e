"""
Seeded random MACE models and synthetic workloads.

``make_model`` follows the reference's test factory (reference tests/helpers.py:25-39): ScaleShiftMACE, 8 Bessel
functions, polynomial cutoff p = 5, a ``RealAgnosticInteractionBlock`` then ``RealAgnosticResidualInteractionBlock``,
2 interactions, MLP_irreps 16x0e, avg_num_neighbors 20, zero E0s, silu gate, full-CG symmetric contraction, and every
parameter perturbed by 0.05·N(0,1) so no weight stays at its zero initialisation.

``WORKLOADS`` are the benchmark configurations 0–4 (model + structures); ``REF_CONFIGS`` are the four architectures
of the reference's parity test (reference tests/helpers.py:16-22) with the full-CG basis (the reduced basis needs
cuequivariance, which is not available here).
"""
import numpy as np
import torch

from . import data as D
from .blocks import interaction_classes
from .models import ScaleShiftMACE

ELEMENTS_PTCOH = [1, 6, 8, 78]        # H, C, O, Pt
ELEMENTS_REF = [1, 7, 8, 78]          # H, N, O, Pt (reference tests/helpers.py:14)

REF_CONFIGS = {
    # name: (hidden_irreps, max_ell, correlation)
    'l3_corr3_fullcg': ('32x0e+32x1o', 3, 3),
    'l3_corr3_fullcg_b': ('32x0e+32x1o', 3, 3),
    'l2_corr2_scalar': ('64x0e', 2, 2),
    'l3_corr3_l2hidden': ('32x0e+32x1o+32x2e', 3, 3),
}


def make_model(hidden='32x0e+32x1o', max_ell=3, correlation=3, seed=0, r_max=5.0, elements=ELEMENTS_REF,
               avg_num_neighbors=20.0, dtype=torch.float32):
    torch.manual_seed(seed)
    n = len(elements)
    model = ScaleShiftMACE(
        atomic_inter_scale=1.0, atomic_inter_shift=0.0, r_max=r_max, num_bessel=8, num_polynomial_cutoff=5,
        max_ell=max_ell, interaction_cls=interaction_classes['RealAgnosticResidualInteractionBlock'],
        interaction_cls_first=interaction_classes['RealAgnosticInteractionBlock'], num_interactions=2,
        num_elements=n, hidden_irreps=hidden, MLP_irreps='16x0e', atomic_energies=np.zeros(n),
        avg_num_neighbors=avg_num_neighbors, atomic_numbers=list(elements), correlation=correlation,
        gate=torch.nn.functional.silu)
    with torch.no_grad():
        for p in model.parameters():
            p.add_(0.05 * torch.randn_like(p))
    return model.to(dtype)


def make_structure(seed=0, n_frag=10):
    """4×4×3 Pt(100), 8 Å vacuum each side, NH3/NH2/NH/N/OH/O fragments 1.2–2.2 Å above the surface, min distance
    1.6 Å, periodic in all directions (reference tests/helpers.py:56-78)."""
    rng = np.random.default_rng(seed)
    slab = D.fcc100_slab('Pt', (4, 4, 3), a=3.92, vacuum=16.0, pbc=(True, True, True))
    frags = [D.MOLECULES[k] for k in ('NH3', 'NH2', 'NH', 'N', 'OH', 'O')]
    return D.add_molecules(slab, rng, n_frag, frags, height=(1.2, 2.2), min_dist=1.6)


def pt_slab_with_adsorbates(rng, size, n_ads, sigma=0.05, vacuum=12.0, min_dist=1.0, both_sides=False):
    """fcc(100) Pt block (a = 3.92 Å, x/y periodic, ``vacuum`` Å along z) plus ``n_ads`` C/O/H atoms uniform in x/y
    at 1.8–2.2 Å above the top layer (alternating top/bottom faces with ``both_sides``), every atom jittered by
    N(0, sigma)."""
    s = D.fcc100_slab('Pt', size, a=3.92, vacuum=vacuum)
    s = D.add_adsorbates(s, rng, n_ads, ['C', 'O', 'H'], height=(1.8, 2.2), min_dist=min_dist, both_sides=both_sides)
    return D.jitter(s, rng, sigma)


# ------------------------------------------------------------------------------------------------- workloads
def structures(cfg, seed=0):
    """The structures of BASELINE configuration ``cfg`` (0-4) and how they are batched: dict(structures, r_max,
    pad_edges_to (None: exact graphs), elements (the one-hot table), name, extra meta)."""
    rng = np.random.default_rng(1000 + seed)
    if cfg == 0:
        s = pt_slab_with_adsorbates(rng, (4, 4, 4), 15)
        return dict(structures=[s], r_max=5.0, pad_edges_to=None, elements=ELEMENTS_PTCOH,
                    name='cfg0_32ch_l2c2_79atoms', meta={})
    if cfg == 1:
        s = pt_slab_with_adsorbates(rng, (5, 5, 5), 35)
        return dict(structures=[s], r_max=5.0, pad_edges_to=None, elements=ELEMENTS_PTCOH,
                    name='cfg1_128ch_l3c3_160atoms', meta={})
    if cfg == 2:
        # 6x5x4 Pt block (120 atoms) with 20-61 adsorbates on both faces: 4.3k-5.9k edges per slab (mean ~5k), so
        # every graph fits the fixed 6,000-edge padding
        counts = rng.integers(140, 182, size=16)
        structs = [pt_slab_with_adsorbates(rng, (6, 5, 4), int(c) - 120, both_sides=True) for c in counts]
        return dict(structures=structs, r_max=5.0, pad_edges_to=6000, elements=ELEMENTS_PTCOH,
                    name='cfg2_128ch_l3c3_batch16_pad6000', meta=dict(atom_counts=counts.tolist()))
    if cfg == 3:
        mols = [D.MOLECULES[k] for k in ('CO', 'OH', 'NH', 'H')]
        slabs = [
            D.cubic_crystal(D.fcc_basis('Au'), 4.08, (3, 3, 2), vacuum=12.0, pbc=(True, True, False)),
            D.cubic_crystal(D.fcc_basis('Cu'), 3.61, (3, 3, 3), vacuum=12.0, pbc=(True, True, False)),
            D.cubic_crystal(D.fcc_basis('Ni'), 3.52, (3, 3, 3), vacuum=12.0, pbc=(True, True, False)),
            D.cubic_crystal(D.fcc_basis('Pt'), 3.92, (3, 3, 3), vacuum=12.0, pbc=(True, True, False)),
            D.cubic_crystal(D.rocksalt_basis('Mg', 'O'), 4.21, (2, 2, 2), vacuum=12.0, pbc=(True, True, False)),
            D.cubic_crystal(D.rocksalt_basis('Ni', 'O'), 4.18, (3, 3, 2), vacuum=12.0, pbc=(True, True, False)),
            D.cubic_crystal(D.fluorite_basis('Ce', 'O'), 5.41, (2, 2, 2), vacuum=12.0, pbc=(True, True, False)),
            D.cubic_crystal(D.fluorite_basis('Zr', 'O'), 5.07, (2, 2, 3), vacuum=12.0, pbc=(True, True, False)),
        ]
        structs = [D.jitter(D.add_molecules(s, rng, int(rng.integers(3, 8)), mols, min_dist=1.4), rng, 0.03)
                   for s in slabs]
        return dict(structures=structs, r_max=6.0, pad_edges_to=None, elements=list(range(1, 90)),
                    name='cfg3_89elem_128ch_l3c3_8slabs', meta=dict(atom_counts=[len(s) for s in structs]))
    if cfg == 4:
        s = D.jitter(D.cubic_crystal(D.fcc_basis('Pt'), 3.92, (25, 25, 8)), rng, 0.08)
        return dict(structures=[s], r_max=5.0, pad_edges_to=None, elements=ELEMENTS_PTCOH,
                    name='cfg4_bulkPt_20000atoms', meta={})
    raise ValueError(cfg)


def batch_of(st, dtype=torch.float32, device='cpu'):
    """MACE batch dict of a ``structures`` record (host neighbour lists, the configuration's padding)."""
    graphs = [D.graph_of(s, st['r_max']) for s in st['structures']]
    return D.batch_graphs(graphs, st['elements'], dtype, device, pad_edges_to=st['pad_edges_to'], r_max=st['r_max'])


def workload(cfg, seed=0, dtype=torch.float32, device='cpu'):
    """(model, batch, meta) for BASELINE configuration ``cfg`` (0-4)."""
    st = structures(cfg, seed)
    hidden, lmax, corr = {0: ('32x0e+32x1o', 2, 2), 1: ('128x0e+128x1o', 3, 3), 2: ('128x0e+128x1o', 3, 3),
                          3: ('128x0e+128x1o', 3, 3), 4: ('128x0e+128x1o+128x2e', 3, 3)}[cfg]
    model = make_model(hidden, lmax, corr, r_max=st['r_max'], elements=st['elements'], dtype=dtype)
    return model, batch_of(st, dtype, device), dict(name=st['name'], r_max=st['r_max'], hidden=hidden,
                                                    channels=int(hidden.split('x')[0]), l_max=lmax, correlation=corr,
                                                    **st['meta'])

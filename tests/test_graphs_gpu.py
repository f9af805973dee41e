"""
A patched E+F(+stress) call captured as a HIP graph (mace_hip_kernels.graphs) against eager calls.

The graph is replayed several times on new positions, with the program's own eager work and device synchronisations
between replays, and every replay is checked against an eager call of the same patched model on the same positions
(tolerances as the model parity tests: 1 meV per structure, 1e-5 eV/A, 1e-5 relative for stress).
"""
import copy

import numpy as np
import pytest
import torch

from mace_hip_kernels import patch_model
from mace_hip_kernels.graphs import capture
from mace_lite import data as D
from mace_lite import factory

pytestmark = pytest.mark.gpu


def _gpu_batch(batch, dev):
    return {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in batch.items()}


@pytest.mark.parametrize('cfg,stress', [(1, True), (2, False)])
def test_captured_call_matches_eager(cfg, stress):
    assert torch.cuda.is_available(), 'GPU test needs a GPU'
    dev = torch.device('cuda:0')
    print(f'[case] graph capture cfg{cfg} stress={stress}', flush=True)
    model, batch_cpu, _ = factory.workload(cfg)
    model = copy.deepcopy(model).to(dev)
    assert not patch_model(model, verbose=False)['skipped']
    batch = _gpu_batch(batch_cpu, dev)
    base = batch['positions'].detach().clone()
    call = capture(model, batch, compute_force=True, compute_stress=stress)
    rng = np.random.default_rng(7)
    prev_f = None
    for rep in range(4):
        new = base + torch.tensor(rng.normal(0.0, 0.02, size=tuple(base.shape)), dtype=base.dtype, device=dev)
        with torch.no_grad():
            batch['positions'].copy_(new)
        out = call.replay()
        e_g, f_g = out['energy'].detach().clone(), out['forces'].detach().clone()
        s_g = out['stress'].detach().clone() if stress else None
        # eager work between replays: an unrelated eager call plus a full device synchronisation
        ref_batch = D.fresh(batch)
        ref = model(ref_batch, compute_force=True, compute_stress=stress)
        torch.cuda.synchronize()
        de = float((e_g - ref['energy']).abs().max())
        df = float((f_g - ref['forces']).abs().max())
        print(f'  replay {rep}: |dE| {de:.2e} eV  |dF| {df:.2e} eV/A', flush=True)
        assert de <= 1e-3 and df <= 1e-5
        if stress:
            ds = float((s_g - ref['stress']).abs().max() / ref['stress'].abs().max().clamp_min(1e-12))
            assert ds <= 1e-5
        if prev_f is not None:                 # the replay recomputes: new positions give new forces
            assert float((f_g - prev_f).abs().max()) > 1e-4
        prev_f = f_g
    del call
    torch.cuda.synchronize()


def test_captured_call_rebuilds_graph():
    """capture(rebuild_graph=True): the edge list is part of the graph's input.  Each replay gets a different padded
    neighbour list (the structure re-jittered and its neighbours rebuilt, same atoms, same padded size) and must match
    an eager call on that batch."""
    assert torch.cuda.is_available(), 'GPU test needs a GPU'
    dev = torch.device('cuda:0')
    print('[case] graph capture with edge-list rebuild', flush=True)
    model = copy.deepcopy(factory.make_model('32x0e+32x1o', 2, 2, elements=factory.ELEMENTS_PTCOH)).to(dev)
    assert not patch_model(model, verbose=False)['skipped']
    rng = np.random.default_rng(3)
    s0 = factory.pt_slab_with_adsorbates(rng, (4, 4, 4), 15)
    batches = []
    for _ in range(3):
        s = s0.copy()
        s.positions = s.positions + rng.normal(0.0, 0.12, size=s.positions.shape)
        batches.append(D.batch_graphs([D.graph_of(s, 5.0)], factory.ELEMENTS_PTCOH, torch.float32, 'cpu',
                                      pad_edges_to=3200, r_max=5.0))
    assert not torch.equal(batches[0]['edge_index'], batches[1]['edge_index'])
    static = _gpu_batch(batches[0], dev)
    call = capture(model, static, rebuild_graph=True, compute_force=True)
    for rep, b in enumerate(batches[1:] + batches[:1]):
        with torch.no_grad():
            for k in ('positions', 'edge_index', 'shifts', 'unit_shifts'):
                static[k].copy_(b[k].to(dev))
        out = call.replay()
        e_g, f_g = out['energy'].detach().clone(), out['forces'].detach().clone()
        ref = model(D.fresh(_gpu_batch(b, dev)), compute_force=True)
        torch.cuda.synchronize()
        de = float((e_g - ref['energy']).abs().max())
        df = float((f_g - ref['forces']).abs().max())
        print(f'  replay {rep}: |dE| {de:.2e} eV  |dF| {df:.2e} eV/A', flush=True)
        assert de <= 1e-3 and df <= 1e-5
    del call
    torch.cuda.synchronize()


def test_captured_md_step_with_gpu_neighbour_list():
    """capture(neighbours=...): every replay rebuilds the padded neighbour list on the GPU from the current positions,
    then the CSRs, then E+F.  The positions move by up to ~0.15 A between replays (edges enter and leave the cutoff);
    each replay's edge list equals an eager GPU build on the same positions, and its energies and forces an eager
    call on that graph."""
    from mace_hip_kernels import neighbour_list
    assert torch.cuda.is_available(), 'GPU test needs a GPU'
    dev = torch.device('cuda:0')
    print('[case] captured MD step: GPU neighbour list + E+F', flush=True)
    model, batch_cpu, meta = factory.workload(2)
    model = copy.deepcopy(model).to(dev)
    assert not patch_model(model, verbose=False)['skipped']
    st = factory.structures(2)
    pbc = torch.tensor([[bool(v) for v in s.pbc] for s in st['structures']], device=dev)
    batch = D.fresh(_gpu_batch(batch_cpu, dev))
    base = batch['positions'].detach().clone()
    step = capture(model, batch, neighbours=dict(r_max=5.0, pbc=pbc, pad_edges_to=6000), compute_force=True)
    rng = np.random.default_rng(11)
    prev = None
    for rep in range(3):
        new = base + torch.tensor(rng.normal(0.0, 0.05, size=tuple(base.shape)), dtype=base.dtype, device=dev)
        with torch.no_grad():
            batch['positions'].copy_(new)
        out = step.replay()
        e_g, f_g = out['energy'].detach().clone(), out['forces'].detach().clone()
        ei_g = batch['edge_index'].clone()
        step.check()
        nl = neighbour_list(new, batch['cell'], batch['ptr'], 5.0, pbc=pbc, pad_edges_to=6000)
        assert torch.equal(ei_g, nl.edge_index) and torch.equal(batch['shifts'], nl.shifts)
        if prev is not None:
            assert not torch.equal(ei_g, prev)          # the graph changed with the positions
        prev = ei_g
        ref_batch = D.fresh(batch)
        ref_batch['positions'] = new.clone()
        ref_batch['edge_index'], ref_batch['shifts'] = nl.edge_index, nl.shifts
        ref_batch['unit_shifts'] = nl.unit_shifts
        ref = model(ref_batch, compute_force=True)
        torch.cuda.synchronize()
        de = float((e_g - ref['energy']).abs().max())
        df = float((f_g - ref['forces']).abs().max())
        print(f'  replay {rep}: |dE| {de:.2e} eV  |dF| {df:.2e} eV/A', flush=True)
        assert de <= 1e-3 and df <= 1e-5
    # the atoms pressed together (positions scaled by 0.8 about the origin) outgrow the 6,000-edge padding: the replay
    # itself raises nothing, the next replay (or check()) reports the structures from the counts its copy brought back
    print('[case] captured MD step: overflow reported one replay late', flush=True)
    with torch.no_grad():
        batch['positions'].copy_(base * 0.8)
    step.replay()
    with pytest.raises(ValueError, match='incomplete'):
        step.check()
    with torch.no_grad():
        batch['positions'].copy_(base)
    step.replay()
    step.check()
    with torch.no_grad():
        batch['positions'].copy_(base * 0.8)
    step.replay()
    torch.cuda.synchronize()
    with pytest.raises(ValueError, match='incomplete'):
        step.replay()
    step.check()
    del step
    torch.cuda.synchronize()

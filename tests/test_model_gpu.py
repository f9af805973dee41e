"""
Model-level parity of the patched MACE model (HIP kernels, fp32, GPU) against the unpatched e3nn path, mirroring the
reference's tests (reference tests/test_kernels.py:23-85) plus the BASELINE configurations.

Reference for E/F/stress: the same model unpatched, evaluated in float64 on the GPU (the e3nn path restated in plain
PyTorch).  Tolerances: the reference's (E: 1e-5 eV/atom; F: 1e-5 relative to the largest force component;
rotation: 1e-4 relative) and the tier's absolute ones (|dE| <= 1 meV per structure, max|dF| <= 1e-5 eV/A).
"""
import copy

import numpy as np
import pytest
import torch

from mace_hip_kernels import patch_model
from mace_lite import data as D
from mace_lite import factory
from oracle import wigner

pytestmark = pytest.mark.gpu
E_TOL = 1e-5        # eV per atom
F_TOL = 1e-5        # relative to the largest force component
E_ABS = 1e-3        # eV per structure
F_ABS = 1e-5        # eV/A


CORE = ('conv_tp', 'symmetric_contractions', 'spherical_harmonics')


def _core(report):
    """Patched convolutions, contractions and spherical harmonics (the rest of ``patched`` are node linears)."""
    return [n for n in report['patched'] if n.endswith(CORE)]


def _dev():
    assert torch.cuda.is_available(), 'GPU test needs a GPU'
    return torch.device('cuda:0')


def _to(batch, dev, dtype):
    return {k: (v.to(dev, dtype) if torch.is_tensor(v) and v.is_floating_point() else
                v.to(dev) if torch.is_tensor(v) else v) for k, v in batch.items()}


def _ef(model, batch, dev, dtype, stress=False):
    out = model(D.fresh(_to(batch, dev, dtype)), compute_force=True, compute_stress=stress)
    res = [out['energy'].detach().double().cpu().numpy(), out['forces'].detach().double().cpu().numpy()]
    if stress:
        res.append(out['stress'].detach().double().cpu().numpy())
    return res


def _pair(model, dev):
    ref = copy.deepcopy(model).to(dev, torch.float64)
    met = copy.deepcopy(model).to(dev, torch.float32)
    report = patch_model(met, verbose=False)
    return ref, met, report


def _check(ref, met, batch, dev, n_atoms, stress=False):
    r = _ef(ref, batch, dev, torch.float64, stress)
    m = _ef(met, batch, dev, torch.float32, stress)
    dE = np.abs(m[0] - r[0])
    dF = np.abs(m[1] - r[1]).max()
    assert dE.max() < E_ABS, dE
    assert (dE / np.asarray(n_atoms)).max() < E_TOL, dE
    assert dF / max(np.abs(r[1]).max(), 1e-3) < F_TOL, dF
    assert dF < F_ABS, dF
    if stress:
        ds = np.abs(m[2] - r[2]).max()
        assert ds / max(np.abs(r[2]).max(), 1e-6) < 1e-4, ds
    return dE.max(), dF


@pytest.mark.parametrize('config', list(factory.REF_CONFIGS))
def test_matches_e3nn_all_configs(config):
    dev = _dev()
    hidden, lmax, corr = factory.REF_CONFIGS[config]
    seed = 0 if not config.endswith('_b') else 7
    ref, met, report = _pair(factory.make_model(hidden, lmax, corr, seed=seed), dev)
    assert not report['skipped'], report['skipped']
    assert len(_core(report)) == 5 and 'spherical_harmonics' in report['patched'], report
    assert 'interactions.1.linear' in report['patched'] and 'interactions.0.skip_tp' in report['patched'], report
    assert 'interactions.1.conv_tp_weights' in report['patched'], report
    for s in (0, 1, 2):
        print(f'[case] {config} seed {s}', flush=True)
        st = factory.make_structure(seed=s)
        batch = D.batch_graphs([D.graph_of(st, 5.0)], factory.ELEMENTS_REF)
        dE, dF = _check(ref, met, batch, dev, [len(st)])
        print(f'       |dE| {dE * 1e3:.4f} meV  max|dF| {dF:.2e}', flush=True)


@pytest.mark.parametrize('config', list(factory.REF_CONFIGS))
def test_fused_radial_matches_e3nn(config):
    """fuse_radial=True: every interaction block whose convolution and radial MLP the fused kernels take runs the MLP's
    output layer inside the convolution; energies and forces stay within the unfused path's tolerances."""
    dev = _dev()
    hidden, lmax, corr = factory.REF_CONFIGS[config]
    model = factory.make_model(hidden, lmax, corr)
    ref = copy.deepcopy(model).to(dev, torch.float64)
    met = copy.deepcopy(model).to(dev, torch.float32)
    patch_model(met, verbose=False, fuse_radial=True)
    fused = [blk.conv_tp.fused_mlp() is blk.conv_tp_weights for blk in met.interactions]
    if not any(fused):
        pytest.skip(f'{config}: no block takes the fused kernels')
    for s in (0, 1):
        print(f'[case] fused radial {config} seed {s} blocks {fused}', flush=True)
        st = factory.make_structure(seed=s)
        batch = D.batch_graphs([D.graph_of(st, 5.0)], factory.ELEMENTS_REF)
        dE, dF = _check(ref, met, batch, dev, [len(st)])
        print(f'       |dE| {dE * 1e3:.4f} meV  max|dF| {dF:.2e}', flush=True)


def test_rotation_equivariance():
    dev = _dev()
    print('[case] rotation equivariance', flush=True)
    _, met, _ = _pair(factory.make_model(*factory.REF_CONFIGS['l3_corr3_fullcg']), dev)
    st = factory.make_structure(seed=3)
    R = wigner.random_rotation(np.random.default_rng(0))
    b0 = D.batch_graphs([D.graph_of(st, 5.0)], factory.ELEMENTS_REF)
    b1 = D.batch_graphs([D.graph_of(st.rotated(R), 5.0)], factory.ELEMENTS_REF)
    E0, F0 = _ef(met, b0, dev, torch.float32)
    E1, F1 = _ef(met, b1, dev, torch.float32)
    assert abs(E1 - E0).max() / len(st) < E_TOL
    assert np.abs(F1 - F0 @ R.T).max() / np.abs(F0).max() < 1e-4


def test_double_backward_raises():
    dev = _dev()
    print('[case] double backward guard', flush=True)
    _, met, _ = _pair(factory.make_model(*factory.REF_CONFIGS['l3_corr3_fullcg']), dev)
    batch = D.fresh(_to(D.batch_graphs([D.graph_of(factory.make_structure(seed=4), 5.0)], factory.ELEMENTS_REF),
                        dev, torch.float32))
    out = met(batch, compute_force=False, training=True)
    with pytest.raises(RuntimeError, match='double backward'):
        (f,) = torch.autograd.grad(out['energy'].sum(), batch['positions'], create_graph=True)
        torch.autograd.grad(f.sum(), batch['positions'])


def _force_loss(m, batch, dev, dt, stress=False, wrt_positions=False):
    """E^2 + |F|^2 (+ |stress|^2) computed with create_graph (MACE's training=True), differentiated with respect to
    the positions (``wrt_positions``) or to every parameter that has a gradient."""
    m.zero_grad()
    b = D.fresh(_to(batch, dev, dt))
    out = m(b, compute_force=True, compute_stress=stress, training=True)
    loss = (out['energy'] ** 2).sum() + (out['forces'] ** 2).sum()
    if stress:
        loss = loss + (out['stress'] ** 2).sum()
    if wrt_positions:
        g, = torch.autograd.grad(loss, b['positions'])
        return {'positions': g.double().cpu().numpy()}
    loss.backward()
    return {k: p.grad.double().cpu().numpy() for k, p in m.named_parameters() if p.grad is not None}


def _close(got, want, tol=1e-4):
    for k in want:
        scale = max(np.abs(want[k]).max(), 1e-8)
        assert np.abs(got[k] - want[k]).max() < tol * scale, k


@pytest.mark.parametrize('config,mlp', [('l3_corr3_fullcg', 'hip'), ('l3_corr3_l2hidden', 'hip'),
                                        ('l3_corr3_fullcg', 'e3nn')])
def test_double_backward_hessian_and_force_loss(config, mlp):
    """patch_model(double_backward=True): every drop-in differentiates twice, the radial MLPs through their
    second-order kernels (``mlp='e3nn'``: radial_mlp=False keeps them on e3nn, their weights trainable).  Against
    the unpatched model in float64: (1) a Hessian-vector product of the energy with respect to the positions,
    d(F·v)/dx; (2) the gradient of a loss on energy and forces computed with create_graph (MACE's training=True)
    with respect to the positions, and, with the MLPs on e3nn, with respect to their weights.  Tolerance: 1e-4
    relative to the largest reference component."""
    dev = _dev()
    print(f'[case] double backward {config} radial MLP on {mlp}', flush=True)
    model = factory.make_model(*factory.REF_CONFIGS[config])
    ref = copy.deepcopy(model).to(dev, torch.float64)
    met = copy.deepcopy(model).to(dev, torch.float32)
    report = patch_model(met, verbose=False, double_backward=True, radial_mlp=(mlp == 'hip'))
    assert 'spherical_harmonics' in report['patched'] and 'radial_embedding' in report['patched'], report
    assert any(n.endswith('conv_tp') for n in report['patched']), report
    assert 'edge_geometry' in report['patched'], report
    assert not report['skipped'], report
    assert ('interactions.0.conv_tp_weights' in report['patched']) == (mlp == 'hip'), report
    st = factory.make_structure(seed=4)
    batch = D.batch_graphs([D.graph_of(st, 5.0)], factory.ELEMENTS_REF)
    v = np.random.default_rng(0).normal(size=(len(st), 3))
    hv = []
    for m, dt in ((ref, torch.float64), (met, torch.float32)):
        b = D.fresh(_to(batch, dev, dt))
        out = m(b, compute_force=False, training=True)
        f, = torch.autograd.grad(-out['energy'].sum(), b['positions'], create_graph=True)
        h, = torch.autograd.grad((f * torch.tensor(v, dtype=dt, device=dev)).sum(), b['positions'])
        hv.append(h.double().cpu().numpy())
    assert np.abs(hv[1] - hv[0]).max() < 1e-4 * np.abs(hv[0]).max()
    _close(_force_loss(met, batch, dev, torch.float32, wrt_positions=True),
           _force_loss(ref, batch, dev, torch.float64, wrt_positions=True))
    if mlp == 'e3nn':
        g_ref, g_met = _force_loss(ref, batch, dev, torch.float64), _force_loss(met, batch, dev, torch.float32)
        common = sorted(set(g_ref) & set(g_met))
        assert any('conv_tp_weights' in k for k in common), common
        _close(g_met, {k: g_ref[k] for k in common})


def test_double_backward_upgrade_and_stress_loss():
    """patch_model(m) and then patch_model(m, double_backward=True): the drop-ins the first call made (radial MLPs
    included) differentiate twice, and a loss on energy, forces and stress (the edge geometry's second-order shifts
    path) has the position gradient of the unpatched model in float64, 1e-4 relative to the largest reference
    component."""
    dev = _dev()
    print('[case] double backward after a first-order patch, stress loss', flush=True)
    model = factory.make_model(*factory.REF_CONFIGS['l3_corr3_fullcg'])
    ref = copy.deepcopy(model).to(dev, torch.float64)
    met = copy.deepcopy(model).to(dev, torch.float32)
    first = patch_model(met, verbose=False)
    assert 'interactions.0.conv_tp_weights' in first['patched'], first
    report = patch_model(met, verbose=False, double_backward=True)
    assert not report['skipped'], report
    assert type(met.interactions[0].conv_tp_weights).__name__ == 'HipRadialMLP'
    assert met.interactions[0].conv_tp_weights.double_backward
    batch = D.batch_graphs([D.graph_of(factory.make_structure(seed=6), 5.0)], factory.ELEMENTS_REF)
    _close(_force_loss(met, batch, dev, torch.float32, stress=True, wrt_positions=True),
           _force_loss(ref, batch, dev, torch.float64, stress=True, wrt_positions=True))


@pytest.mark.parametrize('fuse', [False, True])
def test_patched_model_launches_the_fast_paths(fuse, monkeypatch):
    """The kernels an E+F call of the patched model runs, read from the C ABI's launch log (no assumption about which
    path a module takes).  Default: the factored convolution kernels (W0 * cutoff never formed: conv_fwdc,
    conv_bwdrc) after the radial MLP's kernels (mlp_fwd, mlp_bwd).  fuse_radial: the convolutions with the radial
    MLP's output layer inside (conv_fwdm, conv_bwdm: the per-edge weights and their gradient never stored; the MLPs
    run their hidden layers only, mlp_hid / mlp_hidb).  Both: layer 1's backward without dX (no conv_gxsum for it:
    the engine never asks for the first layer's node-feature gradient), the symmetric contraction's LDS-staged
    kernels reading e3nn's irreps layout (sc_fwdsi / sc_bwdsi: reshape_irreps left unformed, so no permutation
    kernel), and every other drop-in's kernels."""
    from mace_hip_kernels import _native
    dev = _dev()
    print(f'[case] kernels launched by the patched model (config 1, fuse_radial={fuse})', flush=True)
    model, batch, _ = factory.workload(1)
    met = copy.deepcopy(model).to(dev)
    patch_model(met, verbose=False, fuse_radial=fuse)
    met(D.fresh(_to(batch, dev, torch.float32)), compute_force=True)          # graph and element order cached
    b = D.fresh(_to(batch, dev, torch.float32))
    from mace_hip_kernels import conv as hconv
    masked, first_order = [], hconv._conv_grads

    def spy(*args, **kw):
        masked.append(kw.get('masked', False))
        return first_order(*args, **kw)
    monkeypatch.setattr(hconv, '_conv_grads', spy)
    with _native.timing() as tm:
        met(b, compute_force=True)
    torch.cuda.synchronize()
    # both convolutions' backward skips the edges outside the cutoff (the patched radial embedding's -0.0 marks)
    assert masked == ([] if fuse else [True, True]), masked
    sym = {tag: names for tag, names in tm.symbols.items()}
    flat = [n for names in sym.values() for n in names]
    if fuse:
        assert sym['conv_fwd[interactions.0.conv_tp]'] == ['conv_fwdm_x128_o2048_h64'], sym
        assert sym['conv_fwd[interactions.1.conv_tp]'] == ['conv_fwdm_x512_o5120_h64'], sym
        assert sym['conv_bwd[interactions.0.conv_tp]'] == ['conv_bwdm_x128_o2048_h64',
                                                            'conv_gysum_x128_o2048_h64'], sym
        assert sym['conv_bwd[interactions.1.conv_tp]'] == ['conv_bwdm_x512_o5120_h64', 'conv_gysum_x512_o5120_h64',
                                                            'conv_gxsum_x512_o5120'], sym
        for i in range(2):
            assert sym[f'mlp_hid[interactions.{i}.conv_tp_weights]'][0].startswith('mlp_hid_'), sym
            assert sym[f'mlp_bwd[interactions.{i}.conv_tp_weights]'][0].startswith('mlp_hidb_'), sym
        banned = ('conv_fwdc_', 'conv_bwdr', 'mlp_fwd_', 'mlp_bwd_')
    else:
        assert sym['conv_fwd[interactions.0.conv_tp]'] == ['conv_fwdc_x128_o2048'], sym
        assert sym['conv_fwd[interactions.1.conv_tp]'] == ['conv_fwdc_x512_o5120'], sym
        assert sym['conv_bwd[interactions.0.conv_tp]'] == ['conv_bwdrc_x128_o2048'], sym
        assert sym['conv_bwd[interactions.1.conv_tp]'] == ['conv_bwdrc_x512_o5120', 'conv_gxsum_x512_o5120'], sym
        for prefix in ('mlp_fwd_', 'mlp_bwd_'):
            assert any(n.startswith(prefix) for n in flat), (prefix, flat)
        banned = ('conv_fwdm_', 'conv_bwdm_', 'mlp_hid')
    for i in range(2):
        names = sym[f'sc_fwd[products.{i}.symmetric_contractions]'] + \
            sym[f'sc_bwd[products.{i}.symmetric_contractions]']
        assert [n.split('_c')[0] for n in names] == ['sc_fwdsi', 'sc_bwdsi'], names    # LDS-staged, irreps layout
    # the first block's skip_tp(linear(message) / avg) runs as one composed map in each direction
    comp = 'interactions.0.linear+interactions.0.skip_tp'
    assert sym[f'lin_fwd[{comp}]'] == ['lin_fwd_i2048_o2048_v4c'], sym
    assert sym[f'lin_bwd[{comp}]'] == ['lin_bwd_i2048_o2048_v4c'], sym
    assert not any(k.endswith(('[interactions.0.linear]', '[interactions.0.skip_tp]')) for k in sym), sym
    # a residual block's product adds its skip connection in the linear's store (pending output + sc)
    assert met.products[1].linear.pend_hint and not met.products[0].linear.pend_hint
    # the first product's output has three patched consumers: its backward adds their gradients as it loads them
    assert met.products[0].linear.slots == 2
    assert 'lin_bwd[products.0.linear+sum]' in sym and 'lin_bwd[products.0.linear]' not in sym, sym
    # the node embedding and the first block's linear_up, likewise (that block's skip_tp acts on the message)
    assert sym['lin_fwd[node_embedding.linear+interactions.0.linear_up]'] == ['lin_fwd_i4_o128c'], sym
    assert not any(k.endswith(('[node_embedding.linear]', '[interactions.0.linear_up]')) for k in sym), sym
    # the two convolutions' gradients of the edge pass's shared outputs reach its backward separately, which adds them
    assert any(k.startswith('edge_bwd[') and k.endswith('+slots]') for k in sym), sym
    # the edge geometry, harmonics and embedding forward as one pass (edge_fwd), their backward as edge_bwd + geom_bwd
    for prefix in ('edge_fwd_', 'edge_bwd_', 'geom_bwd', 'lin_fwd_', 'lin_bwd_',
                   'ro_fwd_', 'ro_bwd_'):
        assert any(n.startswith(prefix) for n in flat), (prefix, flat)
    assert not any(n.startswith(('perm_', 'conv_fwd_', 'conv_bwd_', 'sh_fwd_', 'sh_bwd_', 'emb_fwd_', 'emb_bwd_',
                                 'geom_fwd') + banned) for n in flat), flat


def test_stress_path_segmented_sums():
    """E+F+stress of the patched model (config 1, one structure): the stress displacement's per-structure gathers
    are differentiated by the segmented-sum kernel (two launches: atoms and edges), and energy, forces and stress
    match the unpatched model in float64."""
    from mace_hip_kernels import _native
    dev = _dev()
    print('[case] stress displacement through segmented sums (config 1)', flush=True)
    model, batch, _ = factory.workload(1)
    ref, met, _ = _pair(model, dev)
    met(D.fresh(_to(batch, dev, torch.float32)), compute_force=True, compute_stress=True)
    with _native.timing() as tm:
        met(D.fresh(_to(batch, dev, torch.float32)), compute_force=True, compute_stress=True)
    torch.cuda.synchronize()
    assert tm.symbols.get('geom_segsum') == ['geom_segsum'] and tm.summary()['geom_segsum'][0] == 2, tm.symbols
    _check(ref, met, batch, dev, np.diff(batch['ptr'].numpy()), stress=True)


def test_fused_edge_pass_matches_separate_kernels(monkeypatch):
    """The edge geometry, harmonics and embedding as one pass each way (edgefeat: edge_fwd / edge_bwd) against the
    same model with the three drop-ins launched separately: E+F+stress of config 1 and the position gradient of a
    force loss under double_backward (where the joint node's gradient is the modules' own second-order functions),
    within 1e-6 relative; the fused call launches one edge_fwd and one edge_bwd and none of the separate kernels."""
    from mace_hip_kernels import _native, edgefeat
    dev = _dev()
    print('[case] fused edge pass vs separate kernels (config 1, stress; force loss)', flush=True)
    model, batch, _ = factory.workload(1)
    met = copy.deepcopy(model).to(dev, torch.float32)
    patch_model(met, verbose=False)
    res = {}
    for fuse in (True, False):
        monkeypatch.setattr(edgefeat, 'FUSE', fuse)
        _ef(met, batch, dev, torch.float32, stress=True)
        with _native.timing() as tm:
            res[fuse] = _ef(met, batch, dev, torch.float32, stress=True)
        torch.cuda.synchronize()
        tags = [t for t, *_ in tm.records]
        if fuse:
            assert sum(t.startswith('edge_fwd') for t in tags) == 1 and sum(t.startswith('edge_bwd') for t in tags) == 1
            assert not any(t.startswith(('sh_', 'emb_')) or t == 'geom_fwd' for t in tags), tags
        else:
            assert not any(t.startswith('edge_') and t != 'edge_pairs' for t in tags), tags
    for a, b in zip(res[True], res[False]):
        assert np.abs(a - b).max() <= 1e-6 * max(np.abs(b).max(), 1e-6), (np.abs(a - b).max(), np.abs(b).max())
    dbl = copy.deepcopy(model).to(dev, torch.float32)
    patch_model(dbl, verbose=False, double_backward=True)
    small = D.batch_graphs([D.graph_of(factory.make_structure(seed=9), 5.0)], factory.ELEMENTS_REF)
    loss = {}
    for fuse in (True, False):
        monkeypatch.setattr(edgefeat, 'FUSE', fuse)
        loss[fuse] = _force_loss(dbl, small, dev, torch.float32, wrt_positions=True)
    for k in loss[False]:
        a, b = loss[True][k], loss[False][k]
        assert np.abs(a - b).max() <= 1e-6 * max(np.abs(b).max(), 1e-6), k


def test_residual_product_sum_in_the_linear():
    """A residual block's product, linear(node_feats) + sc, runs the sum in the linear's store (pend_hint): E, F and
    stress of config 1 bitwise equal to the same patched model adding the two apart."""
    dev = _dev()
    print('[case] residual product sum in the linear (config 1, stress)', flush=True)
    model, batch, _ = factory.workload(1)
    met = copy.deepcopy(model).to(dev, torch.float32)
    patch_model(met, verbose=False)
    plin = met.products[1].linear
    assert plin.pend_hint
    res = {}
    for hint in (True, False):
        plin.pend_hint = hint
        res[hint] = _ef(met, batch, dev, torch.float32, stress=True)
    for a, b in zip(res[True], res[False]):
        assert np.array_equal(a, b)


def test_product_output_gradient_slots():
    """The first product's output read by three patched consumers through gradient slots (the product linear's
    backward adds the three gradients as it loads them) against the same model summing them through autograd: E, F
    and stress of config 1 within 1e-6 relative (the sum's order differs), and a force loss's position gradient under
    double_backward (where the slots' gradients are summed by torch)."""
    dev = _dev()
    print('[case] product output gradient slots (config 1, stress; force loss)', flush=True)
    model, batch, _ = factory.workload(1)
    met = copy.deepcopy(model).to(dev, torch.float32)
    patch_model(met, verbose=False)
    plin = met.products[0].linear
    assert plin.slots == 2
    res = {}
    for k in (2, 0):
        plin.slots = k
        res[k] = _ef(met, batch, dev, torch.float32, stress=True)
    for a, b in zip(res[2], res[0]):
        assert np.abs(a - b).max() <= 1e-6 * max(np.abs(b).max(), 1e-6), (np.abs(a - b).max(), np.abs(b).max())
    dbl = copy.deepcopy(model).to(dev, torch.float32)
    patch_model(dbl, verbose=False, double_backward=True)
    small = D.batch_graphs([D.graph_of(factory.make_structure(seed=9), 5.0)], factory.ELEMENTS_REF)
    loss = {}
    for k in (2, 0):
        dbl.products[0].linear.slots = k
        loss[k] = _force_loss(dbl, small, dev, torch.float32, wrt_positions=True)
    for key in loss[0]:
        a, b = loss[2][key], loss[0][key]
        assert np.abs(a - b).max() <= 1e-6 * max(np.abs(b).max(), 1e-6), key


def test_unsupported_block_is_skipped():
    dev = _dev()
    print('[case] 48-channel model: convolutions skipped', flush=True)
    ref, met, report = _pair(factory.make_model('48x0e+48x1o', 3, 3), dev)
    assert all('conv_tp' in n for n, _ in report['skipped']) and len(report['skipped']) == 2, report
    assert len(_core(report)) == 3                     # both contractions and the spherical harmonics
    st = factory.make_structure(seed=5)
    _check(ref, met, D.batch_graphs([D.graph_of(st, 5.0)], factory.ELEMENTS_REF), dev, [len(st)])


@pytest.mark.parametrize('cfg', [0, 1, 2, 3])
def test_baseline_configs(cfg):
    dev = _dev()
    print(f'[case] BASELINE config {cfg}', flush=True)
    model, batch, meta = factory.workload(cfg)
    ref, met, report = _pair(model, dev)
    assert not report['skipped'] and len(_core(report)) == 5, report
    n_atoms = np.diff(batch['ptr'].numpy())
    dE, dF = _check(ref, met, batch, dev, n_atoms, stress=(cfg == 1))
    print(f'       {meta["name"]}: |dE| {dE * 1e3:.4f} meV  max|dF| {dF:.2e}', flush=True)


def test_idempotent_patch_and_unpatch():
    dev = _dev()
    print('[case] patch idempotence / unpatch', flush=True)
    from mace_hip_kernels import unpatch_model
    m = factory.make_model(*factory.REF_CONFIGS['l2_corr2_scalar']).to(dev)
    r1 = patch_model(m, verbose=False)
    r2 = patch_model(m, verbose=False)
    assert len(_core(r1)) == 5 and r2 == dict(patched=[], skipped=[])
    assert sorted(unpatch_model(m)) == sorted(r1['patched'])
    assert type(m.spherical_harmonics).__name__ == 'SphericalHarmonics'
    assert type(m.interactions[1].linear).__name__ == 'Linear'
    r3 = patch_model(m, verbose=False, spherical_harmonics=False, linears=False, radial_mlp=False,
                     radial_embedding=False, layouts=False, edge_geometry=False, readouts=False)
    assert len(r3['patched']) == 4 and 'spherical_harmonics' not in r3['patched']
    assert len(unpatch_model(m)) == 4
    assert not hasattr(m.interactions[0], 'conv_fusion')


def test_training_mode_patch_warns_about_frozen_parameters():
    """The drop-ins hold their weights as constants: patching a model in training mode names the parameters that no
    gradient will reach; the same model in eval mode patches silently, and leaving the radial MLPs and linears on
    e3nn keeps their parameters trainable (not named)."""
    import warnings
    dev = _dev()
    print('[case] training-mode patch warning', flush=True)
    m = factory.make_model(*factory.REF_CONFIGS['l2_corr2_scalar']).to(dev).train()
    with pytest.warns(UserWarning, match='training mode') as rec:
        patch_model(m, verbose=False)
    text = ' '.join(str(w.message) for w in rec)
    assert 'conv_tp_weights' in text and 'linear' in text
    m = factory.make_model(*factory.REF_CONFIGS['l2_corr2_scalar']).to(dev).eval()
    with warnings.catch_warnings(record=True) as rec:
        warnings.simplefilter('always')
        patch_model(m, verbose=False)
    assert not any('training mode' in str(w.message) for w in rec)
    m = factory.make_model(*factory.REF_CONFIGS['l2_corr2_scalar']).to(dev).train()
    with pytest.warns(UserWarning, match='training mode') as rec:
        patch_model(m, verbose=False, radial_mlp=False, linears=False, readouts=False)
    text = ' '.join(str(w.message) for w in rec if 'training mode' in str(w.message))
    assert 'conv_tp_weights' not in text and 'interactions.0.linear' not in text
    assert all(t.requires_grad for n, t in m.named_parameters() if 'conv_tp_weights' in n)

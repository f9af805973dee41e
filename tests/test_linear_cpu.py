"""
Host side of the node linears (mace_hip_kernels.linear), on the CPU: the weights probed from the e3nn modules, the
patch-time structure check, and the generated HIP source compiling for gfx950 (hipRTC, no GPU needed).
"""
import numpy as np
import pytest
import torch

from mace_hip_kernels import linear
from mace_lite import factory, o3


def _modules():
    m = factory.make_model('128x0e+128x1o', 3, 3, elements=factory.ELEMENTS_PTCOH)
    return [(n, mod) for n, mod in m.named_modules() if type(mod).__name__ in ('Linear', 'FullyConnectedTensorProduct')]


def test_probed_weights_reproduce_every_module():
    rng = np.random.default_rng(1)
    seen = 0
    for name, mod in _modules():
        ok, why = linear.lin_supported(mod)
        if not ok:
            assert 'multiples of 16' in why, (name, why)           # the 1-channel readout heads
            continue
        spec = linear.LinSpec(mod)
        x = rng.normal(size=(5, spec.Din))
        a = rng.normal(size=(5, spec.V)) if spec.V else None
        m64 = mod.double()
        with torch.no_grad():
            ref = (m64(torch.tensor(x), torch.tensor(a)) if spec.V else m64(torch.tensor(x))).numpy()
        assert np.abs(spec.apply(x, a) - ref).max() < 1e-12 * np.abs(ref).max()
        # the transposed weights are the adjoint: <g, L x> = <L^T g, x>
        g = rng.normal(size=(5, spec.Dout))
        gx = np.zeros_like(x)
        for (i, o), w in spec.Wio.items():
            mi, li, oi, _ = spec.in_blocks[i]
            mo, lo, oo, _ = spec.out_blocks[o]
            d = 2 * li + 1
            go = g[:, oo:oo + mo * d].reshape(5, mo, d)
            wt = spec.Wt[dict(spec.bterms[i])[o]:][:w.size].reshape(mo, w.shape[1], mi)
            t = (np.einsum('nwd,nv,wvu->nud', go, a, wt) if spec.V else np.einsum('nwd,wu->nud', go, wt[:, 0, :]))
            gx[:, oi:oi + mi * d] += t.reshape(5, -1)
        assert abs((g * ref).sum() - (gx * x).sum()) < 1e-10 * np.abs(g * ref).sum()
        seen += 1
    assert seen >= 9


def test_composed_map_is_the_two_maps_in_a_row():
    """LinSpec.compose (MACE's first block: skip_tp applied to the interaction linear's output) against the two e3nn
    modules run one after the other in float64, and the composed kname; maps that do not chain are refused."""
    m = factory.make_model('128x0e+128x1o', 3, 3, elements=factory.ELEMENTS_PTCOH)
    blk = m.interactions[0]
    lin, skp = linear.LinSpec(blk.linear), linear.LinSpec(blk.skip_tp)
    comp = linear.LinSpec.compose(lin, skp)
    assert comp.V == skp.V and comp.Din == lin.Din and comp.Dout == skp.Dout
    assert comp.kname('lin_fwd') == skp.kname('lin_fwd') + 'c'
    rng = np.random.default_rng(3)
    x, a = rng.normal(size=(6, lin.Din)), rng.normal(size=(6, skp.V))
    with torch.no_grad():
        ref = blk.skip_tp.double()(blk.linear.double()(torch.tensor(x)), torch.tensor(a)).numpy()
    assert np.abs(comp.apply(x, a) - ref).max() < 1e-12 * np.abs(ref).max()
    # a planted mistake in the composition (one middle block left out) must show
    broken = dict(comp.Wio)
    broken.pop(sorted(broken)[-1])
    bad = linear.LinSpec.compose(lin, skp)
    bad.Wio = broken
    assert np.abs(bad.apply(x, a) - ref).max() > 1e-3 * np.abs(ref).max()
    with pytest.raises(ValueError, match='do not compose'):
        linear.LinSpec.compose(skp, skp)


class _MixesComponents(o3.Linear):
    """A planted mistake: an o3.Linear whose output also mixes the m components of its 1o block."""

    def forward(self, x):
        y = super().forward(x)
        return y + 0.1 * torch.roll(y, 1, dims=-1) * (torch.arange(y.shape[-1]) >= 128)


class _WithBias(o3.Linear):
    def forward(self, x):
        return super().forward(x) + 0.5


@pytest.mark.parametrize('cls', [_MixesComponents, _WithBias])
def test_structure_check_rejects_other_maps(cls):
    mod = cls('128x0e+128x1o', '128x0e+128x1o')
    with pytest.raises(ValueError, match='block-diagonal'):
        linear.LinSpec(mod)


def test_unsupported_shapes_are_reported():
    assert not linear.lin_supported(o3.Linear('128x0e', '1x0e'))[0]
    assert not linear.lin_supported(o3.FullyConnectedTensorProduct('16x0e+16x1o', '1x1o', '16x1o'))[0]
    assert linear.lin_supported(o3.FullyConnectedTensorProduct('16x0e+16x1o', '3x0e', '16x0e+16x1o'))[0]


def test_generated_source_compiles():
    from mace_hip_kernels import _native
    for name, mod in _modules():
        if name in ('interactions.1.linear', 'interactions.0.skip_tp', 'node_embedding.linear'):
            spec = linear.LinSpec(mod)
            assert len(_native.compile_source(linear.source(spec))) > 1000
            assert spec.tiled_bwd == (name != 'node_embedding.linear')


def test_reshape_permutation_matches_the_module():
    """The permutation table of the reshape_irreps drop-in against the PyTorch module (on an arange input the output
    lists the source index of every element), and its HIP source compiling."""
    from mace_hip_kernels import _native, layout
    m = factory.make_model('128x0e+128x1o+128x2e', 3, 3, elements=factory.ELEMENTS_PTCOH)
    for blk in m.interactions:
        spec = layout.ReshapeSpec(blk.reshape)
        x = torch.arange(spec.dim, dtype=torch.float64).reshape(1, -1)
        assert blk.reshape(x).reshape(-1).long().tolist() == spec.perm()
        assert sorted(spec.perm()) == list(range(spec.dim))
        assert len(_native.compile_source(layout.source(spec))) > 1000

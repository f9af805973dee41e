"""
Host side of the radial MLP drop-in (mace_hip_kernels.radial), on the CPU: the restated layers against the e3nn
module in float64, the refusal of modules it does not cover, and the generated HIP source compiling for gfx950.
"""
import numpy as np
import pytest
import torch

from mace_hip_kernels import radial
from mace_lite import factory
from mace_lite import nn as enn


def test_restated_layers_match_every_block():
    m = factory.make_model('128x0e+128x1o', 3, 3, elements=factory.ELEMENTS_PTCOH)
    rng = np.random.default_rng(2)
    for blk in m.interactions:
        spec = radial.MLPSpec(blk.conv_tp_weights)
        x = rng.normal(size=(11, spec.hs[0]))
        with torch.no_grad():
            ref = blk.conv_tp_weights.double()(torch.tensor(x)).numpy()
        assert np.abs(spec.apply(x) - ref).max() < 1e-12 * np.abs(ref).max()
        pw = radial.packed_weights(spec)
        assert pw['bwd'][1].shape == (spec.hs[-2], spec.hs[-1]) and pw['fwd'][1].shape == (spec.hs[-1], spec.hs[-2])
        assert pw['fwd'][0].dtype == np.float32
        # both hidden layouts hold the same numbers
        assert np.isclose(np.abs(pw['fwd'][0]).sum(), np.abs(pw['bwd'][0]).sum(), rtol=1e-6)


def test_unsupported_networks_are_refused():
    assert not radial.mlp_supported(enn.FullyConnectedNet([8, 64, 100], torch.nn.functional.silu))[0]   # output
    assert not radial.mlp_supported(enn.FullyConnectedNet([8, 40, 128], torch.nn.functional.silu))[0]   # hidden
    assert not radial.mlp_supported(enn.FullyConnectedNet([8, 64, 128], torch.tanh))[0]                 # activation
    assert not radial.mlp_supported(enn.FullyConnectedNet([8, 128]))[0]                                 # no hidden
    assert radial.mlp_supported(enn.FullyConnectedNet([8, 64, 64, 128], torch.nn.functional.silu))[0]


def test_mismatched_module_is_rejected():
    """A planted mistake: a network whose forward is not the stack of its layers."""
    class Scaled(enn.FullyConnectedNet):
        def forward(self, x):
            return 1.001 * super().forward(x)
    with pytest.raises(ValueError, match='does not match'):
        radial.MLPSpec(Scaled([8, 64, 64, 128], torch.nn.functional.silu))


def test_generated_source_compiles():
    from mace_hip_kernels import _native
    m = factory.make_model('128x0e+128x1o', 3, 3, elements=factory.ELEMENTS_PTCOH)
    spec = radial.MLPSpec(m.interactions[1].conv_tp_weights)
    assert len(_native.compile_source(radial.source(spec))) > 1000

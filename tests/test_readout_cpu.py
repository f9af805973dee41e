"""
Host side of the readout-head drop-in (mace_hip_kernels.readout), on the CPU: the restated heads against the e3nn
modules in float64, the refusal of heads it does not cover, a planted mistake, and the generated source compiling.
"""
import numpy as np
import pytest
import torch

from mace_hip_kernels import readout
from mace_lite import blocks as B
from mace_lite import factory
from mace_lite.o3 import Irreps


def _heads():
    out = []
    for hidden in ('128x0e+128x1o', '48x0e+48x1o'):
        m = factory.make_model(hidden, 3, 3, elements=factory.ELEMENTS_PTCOH)
        out += [(f'{hidden}.{i}', ro) for i, ro in enumerate(m.readouts)]
    return out


@pytest.mark.parametrize('name,ro', _heads())
def test_restated_head_matches_module(name, ro):
    spec = readout.ReadoutSpec(ro)
    x = np.random.default_rng(1).normal(size=(13, spec.Din))
    with torch.no_grad():
        ref = ro.double()(torch.tensor(x)).numpy()
    assert np.abs(spec.apply(x) - ref).max() < 1e-12 * np.abs(ref).max()
    assert spec.kind == ('linear' if type(ro).__name__ == 'LinearReadoutBlock' else 'mlp')


def test_unsupported_heads_are_refused():
    assert not readout.readout_supported(B.LinearReadoutBlock(Irreps('128x0e+128x1o'), Irreps('2x0e')))[0]
    assert not readout.readout_supported(B.LinearReadoutBlock(Irreps('8x0e'), Irreps('1x0e')))[0]       # 8 % 16
    assert not readout.readout_supported(torch.nn.Linear(4, 1))[0]
    assert readout.readout_supported(B.LinearReadoutBlock(Irreps('32x0e+32x1o'), Irreps('1x0e')))[0]


def test_mismatched_module_is_rejected():
    """A planted mistake: a head whose forward is not its restated layers."""
    class Off(B.LinearReadoutBlock):
        def forward(self, x, heads=None):
            return super().forward(x) + 1e-3
    with pytest.raises(ValueError, match='does not match'):
        readout.ReadoutSpec(Off(Irreps('32x0e+32x1o'), Irreps('1x0e')))


def test_generated_source_compiles():
    from mace_hip_kernels import _native
    for _, ro in _heads():
        assert len(_native.compile_source(readout.source(readout.ReadoutSpec(ro)))) > 1000

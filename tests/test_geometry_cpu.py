"""
Host side of the edge-geometry route (mace_hip_kernels.geometry), on the CPU: install/uninstall on a model, the
wrapped module function falling back to the original for every call it does not take (CPU tensors, inactive), the
model's outputs unchanged by the wrapper, and the HIP source compiling.
"""
import copy

import torch

from mace_hip_kernels import geometry
from mace_lite import data as D
from mace_lite import factory
from mace_lite import models as M


def test_install_wraps_and_falls_back_on_cpu():
    model = factory.make_model('32x0e+32x1o', 2, 2, elements=factory.ELEMENTS_REF).double()
    ref = copy.deepcopy(model)
    st = factory.make_structure(seed=2)
    batch = D.batch_graphs([D.graph_of(st, 5.0)], factory.ELEMENTS_REF, torch.float64)
    assert geometry.install(model) and geometry.installed(model)
    assert hasattr(M.get_edge_vectors_and_lengths, '_mh_original')
    out = model(D.fresh(batch), compute_force=True)         # CPU float64: the wrapper takes the original path
    want = ref(D.fresh(batch), compute_force=True)
    assert torch.equal(out['energy'], want['energy']) and torch.equal(out['forces'], want['forces'])
    assert not geometry._ACTIVE.get()                        # reset after the forward
    clone = copy.deepcopy(model)                             # the activating forward follows a deep copy
    assert geometry.installed(clone) and clone.forward.__self__ is clone
    assert geometry.uninstall(model) and not geometry.installed(model) and not geometry.uninstall(model)


def test_source_compiles():
    from mace_hip_kernels import _native
    assert len(_native.compile_source(geometry.source())) > 1000

"""
mace_lite — plain-PyTorch restatement of the parts of mace-torch 0.3.16 and e3nn 0.4.4 that a MACE energy/force call
needs.  Neither package is installed in this image; this is the model that ``mace_hip_kernels.patch_model`` patches,
and its unpatched path is the "e3nn path" the HIP kernels are compared with and timed against.
"""
from . import blocks, cg, data, factory, models, nn, o3  # noqa: F401

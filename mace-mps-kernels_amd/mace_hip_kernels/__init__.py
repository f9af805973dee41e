"""
mace_hip_kernels — MI355X (gfx950) HIP kernels for MACE inference, patched into a loaded model in memory.

    from mace_hip_kernels import patch_model
    report = patch_model(model)          # model already on a ROCm 'cuda' device, float32; modified in place

Replaces, where supported (reference __init__.py:1-14):
  * each interaction block's convolution (gather → channel-wise tensor product → scatter-sum) via MACE's own
    ``conv_fusion`` hook,
  * each product block's symmetric contraction.
Everything else stays on the original e3nn / PyTorch path.  Inference only: the backward pass is first order
(energies, forces, stress, finite-difference Hessians, MD, relaxations); double backward raises.

The kernels are generated per layer with the layer's coefficients as literals, compiled by hipRTC through
``libmace_hip.so`` (C ABI in include/mace_hip.h) and launched on torch's current HIP stream.  If that library cannot
be loaded, ``patch_model`` raises: there is no CPU or eager fallback.
"""
import inspect
import warnings

import torch

from .conv import HipConvTP, conv_supported
from .edge import HipSphericalHarmonics, sh_supported
from .symmetric import HipSymmetricContraction, sc_supported
from . import _native

__version__ = '0.1.0'
__all__ = ['patch_model', 'unpatch_model', 'HipConvTP', 'HipSymmetricContraction', 'HipSphericalHarmonics',
           'conv_supported', 'sc_supported', 'sh_supported']


def _block_has_conv_fusion(blk):
    """Whether the block's forward implements MACE's ``conv_fusion`` branch (reference __init__.py:27-31)."""
    try:
        return 'conv_fusion' in inspect.getsource(type(blk).forward)
    except (OSError, TypeError):
        return False


def patch_model(model, conv=True, symmetric=True, verbose=True, spherical_harmonics=True):
    """Swap supported ops for HIP kernels, in place.  Returns ``{'patched': [...], 'skipped': [(name, reason)]}``
    (reference __init__.py:34-79).  Beyond the reference's two ops, ``spherical_harmonics`` also replaces the model's
    edge spherical harmonics (``model.spherical_harmonics``) when it is a supported e3nn module."""
    p = next(model.parameters())
    dev = p.device
    if dev.type != 'cuda' or torch.version.hip is None:
        raise RuntimeError(f'model must be on a ROCm GPU device (found {dev})')
    if p.dtype != torch.float32:
        raise RuntimeError('float32 models only')
    _native.load()                        # fail loudly before touching the model
    patched, skipped = [], []
    if conv:
        for i, blk in enumerate(getattr(model, 'interactions', [])):
            name = f'interactions.{i}.conv_tp'
            if isinstance(getattr(blk, 'conv_tp', None), HipConvTP):
                continue
            if hasattr(blk, 'conv_fusion'):
                skipped.append((name, 'block already uses another fused convolution'))
                continue
            if not _block_has_conv_fusion(blk):
                skipped.append((name, f'{type(blk).__name__} has no conv_fusion path'))
                continue
            ok, why = conv_supported(blk.conv_tp)
            if not ok:
                skipped.append((name, why))
                continue
            blk.conv_tp = HipConvTP(blk.conv_tp, device=dev)
            blk.conv_tp.tag = name
            blk.conv_fusion = True
            patched.append(name)
    if symmetric:
        for i, prod in enumerate(getattr(model, 'products', [])):
            name = f'products.{i}.symmetric_contractions'
            sc = getattr(prod, 'symmetric_contractions', None)
            if isinstance(sc, HipSymmetricContraction):
                continue
            cfg = getattr(prod, 'cueq_config', None)
            if cfg is not None and getattr(cfg, 'enabled', False):
                skipped.append((name, 'cuequivariance layout'))
                continue
            ok, why = sc_supported(sc)
            if not ok:
                skipped.append((name, why))
                continue
            prod.symmetric_contractions = HipSymmetricContraction(sc, device=dev)
            prod.symmetric_contractions.tag = name
            patched.append(name)
    if spherical_harmonics and hasattr(model, 'spherical_harmonics'):
        sh = model.spherical_harmonics
        if not isinstance(sh, HipSphericalHarmonics):
            ok, why = sh_supported(sh)
            if ok:
                model.spherical_harmonics = HipSphericalHarmonics(sh, device=dev)
                patched.append('spherical_harmonics')
            else:
                skipped.append(('spherical_harmonics', why))
    if verbose:
        for name, why in skipped:
            warnings.warn(f'mace_hip_kernels: kept e3nn for {name}: {why}')
    return dict(patched=patched, skipped=skipped)


def unpatch_model(model):
    """Restore the original e3nn modules replaced by ``patch_model`` (the patch is in memory only)."""
    restored = []
    for i, blk in enumerate(getattr(model, 'interactions', [])):
        if isinstance(getattr(blk, 'conv_tp', None), HipConvTP):
            blk.conv_tp = blk.conv_tp.original[0]
            if hasattr(blk, 'conv_fusion'):
                del blk.conv_fusion
            restored.append(f'interactions.{i}.conv_tp')
    for i, prod in enumerate(getattr(model, 'products', [])):
        if isinstance(getattr(prod, 'symmetric_contractions', None), HipSymmetricContraction):
            prod.symmetric_contractions = prod.symmetric_contractions.original[0]
            restored.append(f'products.{i}.symmetric_contractions')
    if isinstance(getattr(model, 'spherical_harmonics', None), HipSphericalHarmonics):
        model.spherical_harmonics = model.spherical_harmonics.original[0]
        restored.append('spherical_harmonics')
    return restored

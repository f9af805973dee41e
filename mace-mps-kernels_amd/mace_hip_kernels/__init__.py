"""
mace_hip_kernels — MI355X (gfx950) HIP kernels for MACE inference, patched into a loaded model in memory.

    from mace_hip_kernels import patch_model
    report = patch_model(model)          # model already on a ROCm 'cuda' device, float32; modified in place

Replaces, where supported (reference __init__.py:1-14):
  * each interaction block's convolution (gather → channel-wise tensor product → scatter-sum) via MACE's own
    ``conv_fusion`` hook,
  * each product block's symmetric contraction,
  * beyond the reference: the edge spherical harmonics, and the node-wise equivariant linears (e3nn ``o3.Linear``)
    and scalar-attribute tensor products (``skip_tp``) with at least 16 output channels per irrep, and each
    interaction block's radial MLP (``conv_tp_weights``), the radial embedding of the edge lengths, and the
    per-node layout permutation (``reshape_irreps``) in front of each symmetric contraction, and the edge geometry
    (``get_edge_vectors_and_lengths``, routed to the kernels while the patched model runs).
Everything else stays on the original e3nn / PyTorch path.  The backward pass is first order by default
(energies, forces, stress, MD, relaxations) and a double backward raises, as in the reference;
``patch_model(model, double_backward=True)`` makes every drop-in differentiable once more (force-loss gradients,
Hessian-vector products).  The graph itself can be built on the GPU (``neighbour_list``).

The kernels are generated per layer with the layer's coefficients as literals, compiled by hipRTC through
``libmace_hip.so`` (C ABI in include/mace_hip.h) and launched on torch's current HIP stream.  If that library cannot
be loaded, ``patch_model`` raises: there is no CPU or eager fallback.
"""
import inspect
import itertools
import warnings

import torch

from .conv import HipConvTP, conv_supported
from .edge import HipSphericalHarmonics, sh_supported
from .linear import HipNodeLinear, lin_supported, use_bf16 as _lin_bf16
from .radial import HipRadialMLP, mlp_supported
from .embedding import HipRadialEmbedding, emb_supported
from .layout import HipReshapeIrreps, reshape_supported
from .readout import HipReadout, readout_supported
from .symmetric import HipSymmetricContraction, sc_supported
from . import _native
from . import conv as _conv
from . import geometry as _geometry
from .conv import check_graphs
from .neighbours import NeighbourList, neighbour_list, update_batch

__version__ = '0.1.0'
__all__ = ['patch_model', 'unpatch_model', 'HipConvTP', 'HipSymmetricContraction', 'HipSphericalHarmonics',
           'HipNodeLinear', 'HipRadialMLP', 'HipRadialEmbedding', 'conv_supported', 'sc_supported', 'sh_supported', 'lin_supported',
           'mlp_supported', 'emb_supported', 'HipReshapeIrreps', 'reshape_supported', 'HipReadout',
           'readout_supported', 'neighbour_list', 'update_batch', 'NeighbourList', 'check_graphs']

_LINEAR_CLASSES = ('Linear', 'FullyConnectedTensorProduct')


def _block_has_conv_fusion(blk):
    """Whether the block's forward implements MACE's ``conv_fusion`` branch (reference __init__.py:27-31)."""
    try:
        return 'conv_fusion' in inspect.getsource(type(blk).forward)
    except (OSError, TypeError):
        return False


def _linear_candidates(model):
    """(name, parent, attribute, module) of every e3nn Linear / FullyConnectedTensorProduct in the model."""
    out = []
    for pname, parent in model.named_modules():
        for attr, mod in parent.named_children():
            if type(mod).__name__ in _LINEAR_CLASSES and not isinstance(mod, HipNodeLinear):
                out.append((f'{pname}.{attr}' if pname else attr, parent, attr, mod))
    return out


def patch_model(model, conv=True, symmetric=True, verbose=True, spherical_harmonics=True, linears=True,
                radial_mlp=True, radial_embedding=True, layouts=True, edge_geometry=True, readouts=True,
                double_backward=False, fuse_radial=False):
    """Swap supported ops for HIP kernels, in place.  Returns ``{'patched': [...], 'skipped': [(name, reason)]}``
    (reference __init__.py:34-79).  Beyond the reference's two ops, ``spherical_harmonics`` also replaces the model's
    edge spherical harmonics (``model.spherical_harmonics``) when it is a supported e3nn module, and ``linears`` the
    node-wise e3nn linears and scalar-attribute tensor products (``skip_tp``; linears with fewer than 16 output channels
    per irrep, such as a readout head's last layer when ``readouts`` is off, are left on e3nn without being reported),
    and
    ``radial_mlp`` each interaction block's radial MLP (``conv_tp_weights``, an e3nn FullyConnectedNet), and
    ``radial_embedding`` the model's Bessel x polynomial-cutoff edge embedding, and ``layouts`` each interaction
    block's ``reshape`` (irreps layout -> symmetric-contraction layout), and ``edge_geometry`` the edge vectors and
    lengths (MACE's ``get_edge_vectors_and_lengths`` in the model's module, taken over only while this model's forward
    runs; other models keep the original), and ``readouts`` the per-interaction readout heads (``LinearReadoutBlock``,
    ``NonLinearReadoutBlock``) as one kernel per direction each.  With ``linears``, an interaction block that applies
    its ``skip_tp`` to ``linear(message) / avg_num_neighbors`` (MACE's first block) runs the two maps as one launch of
    their composition per direction (``HipNodeLinear.compose_after``).

    ``fuse_radial`` (default off; with both the convolution and its radial MLP patched): the convolution forms its
    per-edge weights cutoff * MLP(edge_feats) inside its kernels from the MLP's last hidden activations, so the
    weights and their gradient are never stored (HipConvTP.attach_mlp).  Off, the MLP's kernels write the weights and
    the convolution reads them, which measures faster on MI355X for the benchmark models: the fused kernels save the
    weights' HBM round trip but spend more on the VALU than the round trip costs.  The MLP's kernels then run inside
    the convolution's autograd node (HipConvTP.defer_mlp; ``conv.DEFER_RADIAL``), so that both skip the rows of the
    edges outside the cutoff's support (padding edges, edges past r_max) whenever the cutoff comes unmodified from
    the patched radial embedding.

    ``double_backward`` (default off, as in the reference, where a backward under ``create_graph=True`` raises)
    makes the patched modules' gradients differentiable once more, for second derivatives with respect to the
    inputs: Hessian-vector products and force constants, or force and stress terms of a loss differentiated with
    respect to the positions (or to parameters the patch leaves on e3nn: ``radial_mlp=False`` keeps the radial MLPs'
    weights trainable).  Every drop-in takes it (fuse_radial does not: its fused kernels have no second-order form).
    The patched modules hold their weights as constants: no gradient reaches those weights, with or without it; a
    model patched in training mode with such parameters gets a warning naming them."""
    # a fully patched model may hold no parameters any more (the drop-ins keep their weights as buffers)
    p = next((t for t in itertools.chain(model.parameters(), model.buffers()) if t.is_floating_point()), None)
    if p is None:
        raise RuntimeError('model has no floating-point parameters or buffers')
    dev = p.device
    if dev.type != 'cuda' or torch.version.hip is None:
        raise RuntimeError(f'model must be on a ROCm GPU device (found {dev})')
    if p.dtype != torch.float32:
        raise RuntimeError('float32 models only')
    _native.load()                        # fail loudly before touching the model
    trainable = [n for n, t in model.named_parameters() if t.requires_grad]
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
    if double_backward:
        # convolutions an earlier call fused with their radial MLP (fuse_radial) go back to the two-kernel path:
        # the fused kernels have no second-order form
        for blk in getattr(model, 'interactions', []):
            cv, mlp = getattr(blk, 'conv_tp', None), getattr(blk, 'conv_tp_weights', None)
            if isinstance(cv, HipConvTP):
                if cv.fused_mlp() is not None:
                    cv.detach_mlp()
                cv.defer_mlp(None)
            if isinstance(mlp, HipRadialMLP):
                mlp.fuse = False
    if spherical_harmonics and hasattr(model, 'spherical_harmonics'):
        sh = model.spherical_harmonics
        if not isinstance(sh, HipSphericalHarmonics):
            ok, why = sh_supported(sh)
            if ok:
                model.spherical_harmonics = HipSphericalHarmonics(sh, device=dev)
                patched.append('spherical_harmonics')
            else:
                skipped.append(('spherical_harmonics', why))
    if edge_geometry and not _geometry.installed(model):
        if _geometry.install(model):
            patched.append('edge_geometry')
        else:
            skipped.append(('edge_geometry', f'no {_geometry.FUNCTION} in {type(model).__module__}'))
    if radial_embedding and hasattr(model, 'radial_embedding'):
        emb = model.radial_embedding
        if not isinstance(emb, HipRadialEmbedding):
            ok, why = emb_supported(emb)
            if ok:
                try:
                    model.radial_embedding = HipRadialEmbedding(emb, device=dev)
                except ValueError as e:
                    ok, why = False, str(e)
            if ok:
                patched.append('radial_embedding')
            else:
                skipped.append(('radial_embedding', why))
    if radial_mlp:
        for i, blk in enumerate(getattr(model, 'interactions', [])):
            name = f'interactions.{i}.conv_tp_weights'
            mlp = getattr(blk, 'conv_tp_weights', None)
            if mlp is None or isinstance(mlp, HipRadialMLP):
                continue
            ok, why = mlp_supported(mlp)
            if ok:
                try:
                    new = HipRadialMLP(mlp, device=dev)
                except ValueError as e:
                    ok, why = False, str(e)
            if not ok:
                skipped.append((name, why))
                continue
            new.tag = name
            blk.conv_tp_weights = new
            patched.append(name)
    if fuse_radial and not double_backward:
        for blk in getattr(model, 'interactions', []):
            cv, mlp = getattr(blk, 'conv_tp', None), getattr(blk, 'conv_tp_weights', None)
            if isinstance(cv, HipConvTP) and isinstance(mlp, HipRadialMLP) and cv.fused_mlp() is not mlp:
                ok, _ = cv.attach_mlp(mlp)
                mlp.fuse = ok
    if not double_backward and _conv.DEFER_RADIAL:
        # every other convolution runs its radial MLP's kernels inside its own autograd node (the MLP's output
        # handed over unformed), so that both skip the edges outside the cutoff's support
        for blk in getattr(model, 'interactions', []):
            cv, mlp = getattr(blk, 'conv_tp', None), getattr(blk, 'conv_tp_weights', None)
            if isinstance(cv, HipConvTP) and isinstance(mlp, HipRadialMLP) and cv.fused_mlp() is None:
                cv.defer_mlp(mlp)
                mlp.fuse = True
    if layouts:
        for i, blk in enumerate(getattr(model, 'interactions', [])):
            name = f'interactions.{i}.reshape'
            rs = getattr(blk, 'reshape', None)
            if rs is None or isinstance(rs, HipReshapeIrreps) or type(rs).__name__ != 'reshape_irreps':
                continue
            ok, why = reshape_supported(rs)
            if not ok:
                skipped.append((name, why))
                continue
            blk.reshape = HipReshapeIrreps(rs, device=dev)
            blk.reshape.tag = name
            patched.append(name)
            # MACE passes interaction i's reshaped message straight to product i's symmetric contraction; a patched
            # one reads the irreps layout itself, so the reshape is left unformed (formed only for other consumers)
            prods = getattr(model, 'products', None)
            sc = getattr(prods[i], 'symmetric_contractions', None) if prods is not None and i < len(prods) else None
            if isinstance(sc, HipSymmetricContraction) and sc.spec.dims == [2 * l + 1 for _, l in
                                                                             blk.reshape.spec.blocks]:
                blk.reshape.fuse = True
    if readouts:                          # before the linears: a head's own linears go with it
        for i, ro in enumerate(getattr(model, 'readouts', [])):
            name = f'readouts.{i}'
            if isinstance(ro, HipReadout):
                continue
            ok, why = readout_supported(ro)
            if ok:
                try:
                    new = HipReadout(ro, device=dev)
                except ValueError as e:
                    ok, why = False, str(e)
            if not ok:
                skipped.append((name, why))
                continue
            new.tag = name
            model.readouts[i] = new
            patched.append(name)
    if linears:
        for name, parent, attr, mod in _linear_candidates(model):
            if any(mul < 16 for mul, _ in mod.irreps_out):
                continue
            ok, why = lin_supported(mod)
            if ok:
                try:
                    new = HipNodeLinear(mod, device=dev)
                except ValueError as e:            # the probed map is not the expected block structure
                    ok, why = False, str(e)
            if not ok:
                skipped.append((name, why))
                continue
            new.tag = name
            # MACE's interaction blocks divide the post-convolution linear's output by avg_num_neighbors
            # (message = self.linear(message) / self.avg_num_neighbors): the division is folded into the kernels
            avg = getattr(parent, 'avg_num_neighbors', None)
            if attr == 'linear' and hasattr(parent, 'conv_tp') and isinstance(avg, (int, float)) and avg:
                new.div_hint = float(avg)
            setattr(parent, attr, new)
            patched.append(name)
        # an interaction block whose skip_tp consumes linear(message) / avg_num_neighbors (MACE's first block) runs
        # the two maps as one composed launch; a block that applies skip_tp elsewhere never triggers it
        for blk in getattr(model, 'interactions', []):
            lin, skp = getattr(blk, 'linear', None), getattr(blk, 'skip_tp', None)
            if (isinstance(lin, HipNodeLinear) and isinstance(skp, HipNodeLinear) and lin.div_hint is not None
                    and not skp._composed and lin.spec.V == 0 and lin.spec.out_blocks == skp.spec.in_blocks):
                skp.compose_after(lin)
        # the node embedding's output reaches the first interaction block's linear_up alone when that block is
        # MACE's RealAgnosticInteractionBlock (its skip_tp acts on the message; the residual block's skip_tp reads
        # the node features too) and the model has no other embedding consumer: the two maps run as one composed
        # launch
        emb = getattr(getattr(model, 'node_embedding', None), 'linear', None)
        blocks = list(getattr(model, 'interactions', []))
        up = getattr(blocks[0], 'linear_up', None) if blocks else None
        if (isinstance(emb, HipNodeLinear) and isinstance(up, HipNodeLinear)
                and type(blocks[0]).__name__ == 'RealAgnosticInteractionBlock'
                and not any(hasattr(model, k) for k in ('joint_embedding', 'embedding_readout'))
                and emb.spec.V == 0 and up.spec.V == 0 and not up._composed and emb.spec.out_blocks == up.spec.in_blocks):
            up.compose_after(emb)
            emb.pend_hint = True
        # a residual block's product returns linear(node_feats) + sc (MACE's EquivariantProductBasisBlock with the
        # skip connection of RealAgnosticResidualInteractionBlock): the sum runs in the linear's store
        for blk, prod in zip(blocks, getattr(model, 'products', [])):
            plin = getattr(prod, 'linear', None)
            if (isinstance(plin, HipNodeLinear) and plin.spec.V == 0 and plin.div_hint is None
                    and type(blk).__name__ == 'RealAgnosticResidualInteractionBlock'):
                plin.pend_hint = True
        # a product's output read by three patched consumers (its readout and the next residual block's skip_tp and
        # linear_up): two of them read aliases with gradient slots of their own, and the product linear's backward
        # adds the three gradients as it loads them (lin_bwds) instead of autograd adding them in two kernels
        prods, heads = list(getattr(model, 'products', [])), list(getattr(model, 'readouts', []))
        for i, prod in enumerate(prods[:-1]):
            plin = getattr(prod, 'linear', None)
            nxt = blocks[i + 1] if i + 1 < len(blocks) else None
            cons = [heads[i] if i < len(heads) else None, getattr(nxt, 'skip_tp', None),
                    getattr(nxt, 'linear_up', None)]
            if (isinstance(plin, HipNodeLinear) and plin.spec.V == 0 and not plin.pend_hint and plin.div_hint is None
                    and plin.compose_into is None and plin.spec.tiled_bwd and not _lin_bf16(plin.spec, True)
                    and type(nxt).__name__ == 'RealAgnosticResidualInteractionBlock'
                    and isinstance(cons[0], HipReadout) and all(isinstance(c, HipNodeLinear) for c in cons[1:])):
                plin.slots = 2
    # the patched convolutions share the patched edge pass's harmonics, features and cutoff: all but one read aliases
    # with gradient slots of their own (edgefeat.slot), so that the edge pass's backward adds their gradients itself
    sh_mod = getattr(model, 'spherical_harmonics', None)
    if isinstance(sh_mod, HipSphericalHarmonics):
        convs = [b for b in getattr(model, 'interactions', []) if isinstance(getattr(b, 'conv_tp', None), HipConvTP)]
        sh_mod.slots = max(0, len(convs) - 1)
    if double_backward:                   # including modules patched by an earlier call
        if _geometry.installed(model):
            model._mh_geometry_double_backward = True
        for mod in model.modules():
            if isinstance(mod, (HipConvTP, HipSymmetricContraction, HipNodeLinear, HipReshapeIrreps,
                                HipSphericalHarmonics, HipRadialEmbedding, HipReadout, HipRadialMLP)):
                mod.double_backward = True
                if hasattr(mod, 'second_module'):
                    mod.second_module()   # compiled now rather than inside the first double backward
    if verbose:
        for name, why in skipped:
            warnings.warn(f'mace_hip_kernels: kept e3nn for {name}: {why}')
    if model.training:
        # the drop-ins hold their weights as constants: a training step (an energy loss, or a force loss under
        # double_backward) would silently leave these parameters unchanged
        kept = {n for n, t in model.named_parameters() if t.requires_grad}
        frozen = sorted({n.rsplit('.', 1)[0] for n in trainable if n not in kept})
        if frozen:
            warnings.warn(f'mace_hip_kernels: the model is in training mode, and the parameters of {frozen} are now '
                          f'constants of the HIP drop-ins (no gradient reaches them); patch for inference (model.eval()), '
                          f'or keep modules to be trained on e3nn (e.g. radial_mlp=False, linears=False)')
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
    if _geometry.uninstall(model):
        restored.append('edge_geometry')
    if isinstance(getattr(model, 'radial_embedding', None), HipRadialEmbedding):
        model.radial_embedding = model.radial_embedding.original[0]
        restored.append('radial_embedding')
    for i, blk in enumerate(getattr(model, 'interactions', [])):
        if isinstance(getattr(blk, 'reshape', None), HipReshapeIrreps):
            blk.reshape = blk.reshape.original[0]
            restored.append(f'interactions.{i}.reshape')
        if isinstance(getattr(blk, 'conv_tp_weights', None), HipRadialMLP):
            blk.conv_tp_weights.fuse = False
            blk.conv_tp_weights = blk.conv_tp_weights.original[0]
            restored.append(f'interactions.{i}.conv_tp_weights')
    for i, ro in enumerate(getattr(model, 'readouts', [])):
        if isinstance(ro, HipReadout):
            model.readouts[i] = ro.original[0]
            restored.append(f'readouts.{i}')
    for pname, parent in list(model.named_modules()):
        for attr, mod in list(parent.named_children()):
            if isinstance(mod, HipNodeLinear):
                setattr(parent, attr, mod.original[0])
                restored.append(f'{pname}.{attr}' if pname else attr)
    return restored

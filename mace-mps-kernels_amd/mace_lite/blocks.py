"""
MACE 0.3.16 building blocks restated in plain PyTorch (mace-torch is not installed in this image).  They are the
callers of the two hot-path ops:

  * ``RealAgnosticInteractionBlock`` / ``RealAgnosticResidualInteractionBlock`` own ``conv_tp`` (an external-weight 'uvu'
    ``TensorProduct``) and take MACE's ``conv_fusion`` branch when the attribute is present, calling
    ``conv_tp(node_feats, edge_attrs, tp_weights, edge_index)``; this is the hook the reference patches
    (reference __init__.py:27-31, 57-58; conv.py:274-275);
  * ``EquivariantProductBasisBlock`` owns ``symmetric_contractions`` (a ``SymmetricContraction``), called as
    ``symmetric_contractions(node_feats[N, C, n_ell], node_attrs[N, n_elem])`` (reference symmetric.py:159, 168-170).

Unpatched, the convolution is ``scatter_sum(conv_tp(x[sender], Y, W), receiver)`` and the contraction is MACE's nested
U·W·x contraction; both are the "e3nn path" the patched kernels are checked against.
"""
import math

import numpy as np
import torch

from . import nn as enn
from .cg import U_matrix_real
from .o3 import FullyConnectedTensorProduct, Irrep, Irreps, Linear, TensorProduct


def scatter_sum(src, index, dim=0, dim_size=None):
    if dim < 0:
        dim += src.dim()
    if dim_size is None:
        dim_size = int(index.max()) + 1 if index.numel() else 0
    shape = list(src.shape)
    shape[dim] = dim_size
    out = src.new_zeros(shape)
    return out.index_add_(dim, index, src)


def tp_out_irreps_with_instructions(irreps1, irreps2, target_irreps):
    """Output irreps and 'uvu' instructions of the interaction convolution: one output block per allowed path."""
    irreps1, irreps2, target_irreps = Irreps(irreps1), Irreps(irreps2), Irreps(target_irreps)
    out_list, instructions = [], []
    for i, (mul, ir_in) in enumerate(irreps1):
        for j, (_, ir_edge) in enumerate(irreps2):
            for ir_out in ir_in * ir_edge:
                if ir_out in target_irreps:
                    k = len(out_list)
                    out_list.append((mul, ir_out))
                    instructions.append((i, j, k, 'uvu', True))
    irreps_out, permut, _ = Irreps(out_list).sort()
    instructions = [(i1, i2, permut[io], mode, tr) for i1, i2, io, mode, tr in instructions]
    instructions = sorted(instructions, key=lambda x: x[2])
    return irreps_out, instructions


class reshape_irreps(torch.nn.Module):
    """[N, Σ mul·(2l+1)] (mul_ir) → [N, mul, Σ (2l+1)]: the symmetric-contraction input layout."""

    def __init__(self, irreps):
        super().__init__()
        self.irreps = Irreps(irreps)

    def forward(self, t):
        n = t.shape[0]
        out, ix = [], 0
        for mul, ir in self.irreps:
            d = ir.dim
            out.append(t[:, ix:ix + mul * d].reshape(n, mul, d))
            ix += mul * d
        return torch.cat(out, dim=-1)


# ------------------------------------------------------------------------------------------------------- radial
class BesselBasis(torch.nn.Module):
    def __init__(self, r_max, num_basis=8):
        super().__init__()
        self.register_buffer('bessel_weights', math.pi / r_max * torch.linspace(1.0, num_basis, num_basis))
        self.register_buffer('prefactor', torch.tensor(math.sqrt(2.0 / r_max)))

    def forward(self, x):
        return self.prefactor * torch.sin(self.bessel_weights * x) / x


class PolynomialCutoff(torch.nn.Module):
    def __init__(self, r_max, p=6):
        super().__init__()
        self.register_buffer('p', torch.tensor(float(p)))
        self.register_buffer('r_max', torch.tensor(float(r_max)))

    def forward(self, x):
        p, u = self.p, x / self.r_max
        env = (1.0 - ((p + 1.0) * (p + 2.0) / 2.0) * torch.pow(u, p) + p * (p + 2.0) * torch.pow(u, p + 1)
               - (p * (p + 1.0) / 2.0) * torch.pow(u, p + 2))
        return env * (x < self.r_max)


class RadialEmbeddingBlock(torch.nn.Module):
    """Bessel basis × polynomial envelope; returns (edge_feats, cutoff) like MACE ≥ 0.3.10."""

    def __init__(self, r_max, num_bessel, num_polynomial_cutoff):
        super().__init__()
        self.bessel_fn = BesselBasis(r_max, num_bessel)
        self.cutoff_fn = PolynomialCutoff(r_max, num_polynomial_cutoff)
        self.out_dim = num_bessel

    def forward(self, edge_lengths):
        cutoff = self.cutoff_fn(edge_lengths)
        return self.bessel_fn(edge_lengths) * cutoff, cutoff


# ----------------------------------------------------------------------------------------------- small blocks
class LinearNodeEmbeddingBlock(torch.nn.Module):
    def __init__(self, irreps_in, irreps_out):
        super().__init__()
        self.linear = Linear(irreps_in, irreps_out)

    def forward(self, node_attrs):
        return self.linear(node_attrs)


class LinearReadoutBlock(torch.nn.Module):
    def __init__(self, irreps_in, irrep_out=Irreps('0e')):
        super().__init__()
        self.linear = Linear(irreps_in, irrep_out)

    def forward(self, x, heads=None):
        return self.linear(x)


class NonLinearReadoutBlock(torch.nn.Module):
    def __init__(self, irreps_in, MLP_irreps, gate, irrep_out=Irreps('0e')):
        super().__init__()
        self.hidden_irreps = Irreps(MLP_irreps)
        self.linear_1 = Linear(irreps_in, self.hidden_irreps)
        self.non_linearity = enn.Activation(self.hidden_irreps, [gate])
        self.linear_2 = Linear(self.hidden_irreps, irrep_out)

    def forward(self, x, heads=None):
        return self.linear_2(self.non_linearity(self.linear_1(x)))


class AtomicEnergiesBlock(torch.nn.Module):
    def __init__(self, atomic_energies):
        super().__init__()
        self.register_buffer('atomic_energies', torch.as_tensor(np.asarray(atomic_energies), dtype=torch.get_default_dtype()))

    def forward(self, x):
        return x @ self.atomic_energies.to(x.dtype)


class ScaleShiftBlock(torch.nn.Module):
    def __init__(self, scale, shift):
        super().__init__()
        self.register_buffer('scale', torch.tensor(float(scale)))
        self.register_buffer('shift', torch.tensor(float(shift)))

    def forward(self, x, heads=None):
        return self.scale * x + self.shift


# -------------------------------------------------------------------------------------- symmetric contraction
class Contraction(torch.nn.Module):
    """One output irrep of MACE's ``SymmetricContraction``.

    out[b, c, M] = Σ_ν Σ_{i1..iν} T_ν[elem_b, c, M, i1..iν] x[b,c,i1]…x[b,c,iν],  T_ν = U_ν · W_ν, evaluated as MACE
    nests it: contract the correlation-ν term with x, add the (ν-1) term, contract again, … down to ν = 1.
    """

    def __init__(self, irreps_in, irrep_out, correlation, num_elements):
        super().__init__()
        irreps_in = Irreps(irreps_in)
        self.num_features = irreps_in.count((0, 1))
        self.coupling_irreps = Irreps([ir for _, ir in irreps_in])
        self.correlation = correlation
        self.irrep_out = Irreps(irrep_out)
        dtype = torch.get_default_dtype()
        for nu in range(1, correlation + 1):
            u = U_matrix_real(self.coupling_irreps, self.irrep_out, nu, dtype=dtype)[-1]
            self.register_buffer(f'U_matrix_{nu}', u)
        self.weights = torch.nn.ParameterList([])
        for i in range(correlation, 0, -1):
            num_params = self.U_tensors(i).shape[-1]
            w = torch.nn.Parameter(torch.randn(num_elements, num_params, self.num_features) / num_params)
            if i == correlation:
                self.weights_max = w
            else:
                self.weights.append(w)

    def U_tensors(self, nu):
        return getattr(self, f'U_matrix_{nu}')

    def forward(self, x, y):
        b, c, ni = x.shape
        U = self.U_tensors(self.correlation).to(x.dtype)
        nk = U.shape[-1]
        lead = U.shape[:-2]
        wb = torch.einsum('ekc,be->bkc', self.weights_max, y)
        t = torch.einsum('bci,bkc->bcik', x, wb).reshape(b * c, ni * nk)
        out = (t @ U.reshape(-1, ni * nk).T).reshape(b, c, *lead)
        for j, w in enumerate(self.weights):
            nu = self.correlation - 1 - j
            U = self.U_tensors(nu).to(x.dtype)
            wb = torch.einsum('ekc,be->bkc', w, y)
            lead = U.shape[:-1]
            ct = torch.matmul(U.reshape(-1, U.shape[-1]), wb)            # [b, prod(lead), c]
            ct = ct.permute(0, 2, 1).reshape(b, c, *lead) + out
            out = torch.einsum('bcmi,bci->bcm', ct.reshape(b, c, -1, ni), x).reshape(b, c, *lead[:-1])
        return out.reshape(b, -1)


class SymmetricContraction(torch.nn.Module):
    def __init__(self, irreps_in, irreps_out, correlation, num_elements):
        super().__init__()
        self.irreps_in, self.irreps_out = Irreps(irreps_in), Irreps(irreps_out)
        self.contractions = torch.nn.ModuleList(
            [Contraction(self.irreps_in, Irreps(str(ir)), correlation, num_elements) for _, ir in self.irreps_out])

    def forward(self, x, y):
        return torch.cat([c(x, y) for c in self.contractions], dim=-1)


class EquivariantProductBasisBlock(torch.nn.Module):
    def __init__(self, node_feats_irreps, target_irreps, correlation, num_elements, use_sc=True):
        super().__init__()
        self.use_sc = use_sc
        self.symmetric_contractions = SymmetricContraction(node_feats_irreps, target_irreps, correlation, num_elements)
        self.linear = Linear(target_irreps, target_irreps)
        self.cueq_config = None

    def forward(self, node_feats, sc, node_attrs):
        node_feats = self.symmetric_contractions(node_feats, node_attrs)
        if self.use_sc and sc is not None:
            return self.linear(node_feats) + sc
        return self.linear(node_feats)


# ------------------------------------------------------------------------------------------- interaction blocks
class InteractionBlock(torch.nn.Module):
    def __init__(self, node_attrs_irreps, node_feats_irreps, edge_attrs_irreps, edge_feats_irreps, target_irreps,
                 hidden_irreps, avg_num_neighbors, radial_MLP=None):
        super().__init__()
        self.node_attrs_irreps = Irreps(node_attrs_irreps)
        self.node_feats_irreps = Irreps(node_feats_irreps)
        self.edge_attrs_irreps = Irreps(edge_attrs_irreps)
        self.edge_feats_irreps = Irreps(edge_feats_irreps)
        self.target_irreps = Irreps(target_irreps)
        self.hidden_irreps = Irreps(hidden_irreps)
        self.avg_num_neighbors = avg_num_neighbors
        self.radial_MLP = radial_MLP if radial_MLP is not None else [64, 64, 64]
        self._setup()

    def _setup_conv(self):
        self.linear_up = Linear(self.node_feats_irreps, self.node_feats_irreps)
        irreps_mid, instructions = tp_out_irreps_with_instructions(self.node_feats_irreps, self.edge_attrs_irreps,
                                                                   self.target_irreps)
        self.conv_tp = TensorProduct(self.node_feats_irreps, self.edge_attrs_irreps, irreps_mid, instructions,
                                     shared_weights=False, internal_weights=False)
        self.conv_tp_weights = enn.FullyConnectedNet(
            [self.edge_feats_irreps.num_irreps] + self.radial_MLP + [self.conv_tp.weight_numel], torch.nn.functional.silu)
        self.irreps_out = self.target_irreps
        self.linear = Linear(irreps_mid.simplify(), self.irreps_out)
        self.reshape = reshape_irreps(self.irreps_out)


class RealAgnosticInteractionBlock(InteractionBlock):
    def _setup(self):
        self._setup_conv()
        self.skip_tp = FullyConnectedTensorProduct(self.irreps_out, self.node_attrs_irreps, self.irreps_out)

    def forward(self, node_attrs, node_feats, edge_attrs, edge_feats, edge_index, cutoff=None, first_layer=False):
        sender, receiver = edge_index[0], edge_index[1]
        num_nodes = node_feats.shape[0]
        node_feats = self.linear_up(node_feats)
        tp_weights = self.conv_tp_weights(edge_feats)
        if cutoff is not None:
            tp_weights = tp_weights * cutoff
        if hasattr(self, 'conv_fusion'):
            message = self.conv_tp(node_feats, edge_attrs, tp_weights, edge_index)
        else:
            mji = self.conv_tp(node_feats[sender], edge_attrs, tp_weights)
            message = scatter_sum(mji, receiver, dim=0, dim_size=num_nodes)
        message = self.linear(message) / self.avg_num_neighbors
        message = self.skip_tp(message, node_attrs)
        return self.reshape(message), None


class RealAgnosticResidualInteractionBlock(InteractionBlock):
    def _setup(self):
        self._setup_conv()
        self.skip_tp = FullyConnectedTensorProduct(self.node_feats_irreps, self.node_attrs_irreps, self.hidden_irreps)

    def forward(self, node_attrs, node_feats, edge_attrs, edge_feats, edge_index, cutoff=None, first_layer=False):
        sender, receiver = edge_index[0], edge_index[1]
        num_nodes = node_feats.shape[0]
        sc = self.skip_tp(node_feats, node_attrs)
        node_feats = self.linear_up(node_feats)
        tp_weights = self.conv_tp_weights(edge_feats)
        if cutoff is not None:
            tp_weights = tp_weights * cutoff
        if hasattr(self, 'conv_fusion'):
            message = self.conv_tp(node_feats, edge_attrs, tp_weights, edge_index)
        else:
            mji = self.conv_tp(node_feats[sender], edge_attrs, tp_weights)
            message = scatter_sum(mji, receiver, dim=0, dim_size=num_nodes)
        message = self.linear(message) / self.avg_num_neighbors
        return self.reshape(message), sc


interaction_classes = {
    'RealAgnosticInteractionBlock': RealAgnosticInteractionBlock,
    'RealAgnosticResidualInteractionBlock': RealAgnosticResidualInteractionBlock,
}

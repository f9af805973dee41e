"""
``MACE`` / ``ScaleShiftMACE`` restated after mace-torch 0.3.16 ``mace/modules/models.py`` and ``utils.py``: node
embedding, spherical harmonics and radial embedding of the edges, ``num_interactions`` × (interaction → product basis
→ readout), scale/shift, per-graph energy, and forces / virials / stress by autograd through a symmetric cell
displacement.  ``model(data, compute_force=True, training=False)`` takes the batch dictionary of
``mace_lite.data.batch_graphs`` and returns ``{'energy', 'forces', 'stress', 'virials', …}``.
"""
import torch

from .blocks import (AtomicEnergiesBlock, EquivariantProductBasisBlock, LinearNodeEmbeddingBlock,
                     LinearReadoutBlock, NonLinearReadoutBlock, RadialEmbeddingBlock, ScaleShiftBlock, scatter_sum)
from .o3 import Irrep, Irreps, SphericalHarmonics


def get_edge_vectors_and_lengths(positions, edge_index, shifts):
    sender, receiver = edge_index[0], edge_index[1]
    vectors = positions[receiver] - positions[sender] + shifts
    return vectors, torch.linalg.norm(vectors, dim=-1, keepdim=True)


def get_symmetric_displacement(positions, unit_shifts, cell, edge_index, num_graphs, batch):
    sender = edge_index[0]
    displacement = torch.zeros((num_graphs, 3, 3), dtype=positions.dtype, device=positions.device)
    displacement.requires_grad_(True)
    sym = 0.5 * (displacement + displacement.transpose(-1, -2))
    positions = positions + torch.einsum('be,bec->bc', positions, sym[batch])
    cell = cell.view(-1, 3, 3)
    cell = cell + torch.matmul(cell, sym)
    shifts = torch.einsum('be,bec->bc', unit_shifts, cell[batch[sender]])
    return positions, shifts, displacement


def get_outputs(energy, positions, displacement, cell, training=False, compute_force=True, compute_virials=False,
                compute_stress=False):
    forces = virials = stress = None
    if (compute_virials or compute_stress) and displacement is not None:
        g = torch.autograd.grad([energy], [positions, displacement], grad_outputs=[torch.ones_like(energy)],
                                retain_graph=training, create_graph=training, allow_unused=True)
        forces = -g[0] if g[0] is not None else torch.zeros_like(positions)
        virials = -g[1] if g[1] is not None else torch.zeros_like(displacement)
        if compute_stress:
            volume = torch.linalg.det(cell.view(-1, 3, 3)).abs().view(-1, 1, 1)
            stress = g[1] / volume if g[1] is not None else torch.zeros_like(displacement)
            stress = torch.where(stress.abs() < 1e10, stress, torch.zeros_like(stress))
    elif compute_force:
        g = torch.autograd.grad([energy], [positions], grad_outputs=[torch.ones_like(energy)],
                                retain_graph=training, create_graph=training, allow_unused=True)[0]
        forces = -g if g is not None else torch.zeros_like(positions)
    return forces, virials, stress


class MACE(torch.nn.Module):
    def __init__(self, r_max, num_bessel, num_polynomial_cutoff, max_ell, interaction_cls, interaction_cls_first,
                 num_interactions, num_elements, hidden_irreps, MLP_irreps, atomic_energies, avg_num_neighbors,
                 atomic_numbers, correlation, gate, radial_MLP=None):
        super().__init__()
        self.register_buffer('atomic_numbers', torch.tensor(atomic_numbers, dtype=torch.int64))
        self.register_buffer('r_max', torch.tensor(float(r_max)))
        self.register_buffer('num_interactions', torch.tensor(num_interactions, dtype=torch.int64))
        hidden_irreps = Irreps(hidden_irreps)
        if isinstance(correlation, int):
            correlation = [correlation] * num_interactions
        node_attr_irreps = Irreps([(num_elements, (0, 1))])
        node_feats_irreps = Irreps([(hidden_irreps.count(Irrep(0, 1)), (0, 1))])
        self.node_embedding = LinearNodeEmbeddingBlock(node_attr_irreps, node_feats_irreps)
        self.radial_embedding = RadialEmbeddingBlock(r_max, num_bessel, num_polynomial_cutoff)
        edge_feats_irreps = Irreps(f'{self.radial_embedding.out_dim}x0e')
        sh_irreps = Irreps.spherical_harmonics(max_ell)
        num_features = hidden_irreps.count(Irrep(0, 1))
        interaction_irreps = (sh_irreps * num_features).sort()[0].simplify()
        self.spherical_harmonics = SphericalHarmonics(sh_irreps, normalize=True, normalization='component')
        radial_MLP = radial_MLP if radial_MLP is not None else [64, 64, 64]
        self.atomic_energies_fn = AtomicEnergiesBlock(atomic_energies)

        inter = interaction_cls_first(node_attr_irreps, node_feats_irreps, sh_irreps, edge_feats_irreps,
                                      interaction_irreps, hidden_irreps, avg_num_neighbors, radial_MLP)
        self.interactions = torch.nn.ModuleList([inter])
        use_sc_first = 'Residual' in str(interaction_cls_first)
        self.products = torch.nn.ModuleList([EquivariantProductBasisBlock(
            inter.target_irreps, hidden_irreps, correlation[0], num_elements, use_sc=use_sc_first)])
        self.readouts = torch.nn.ModuleList([LinearReadoutBlock(hidden_irreps, Irreps('1x0e'))])
        for i in range(num_interactions - 1):
            last = i == num_interactions - 2
            hidden_out = Irreps(str(hidden_irreps[0])) if last else hidden_irreps
            inter = interaction_cls(node_attr_irreps, hidden_irreps, sh_irreps, edge_feats_irreps, interaction_irreps,
                                    hidden_out, avg_num_neighbors, radial_MLP)
            self.interactions.append(inter)
            self.products.append(EquivariantProductBasisBlock(interaction_irreps, hidden_out, correlation[i + 1],
                                                              num_elements, use_sc=True))
            if last:
                self.readouts.append(NonLinearReadoutBlock(hidden_out, Irreps(MLP_irreps), gate, Irreps('1x0e')))
            else:
                self.readouts.append(LinearReadoutBlock(hidden_irreps, Irreps('1x0e')))

    def _prepare(self, data, compute_virials, compute_stress, compute_displacement):
        data['node_attrs'].requires_grad_(True)
        data['positions'].requires_grad_(True)
        num_graphs = data['ptr'].numel() - 1
        displacement = torch.zeros((num_graphs, 3, 3), dtype=data['positions'].dtype, device=data['positions'].device)
        positions, shifts = data['positions'], data['shifts']
        if compute_virials or compute_stress or compute_displacement:
            positions, shifts, displacement = get_symmetric_displacement(
                data['positions'], data['unit_shifts'], data['cell'], data['edge_index'], num_graphs, data['batch'])
        return positions, shifts, displacement, num_graphs

    def _interactions(self, data, positions, shifts):
        node_feats = self.node_embedding(data['node_attrs'])
        vectors, lengths = get_edge_vectors_and_lengths(positions, data['edge_index'], shifts)
        edge_attrs = self.spherical_harmonics(vectors)
        edge_feats, cutoff = self.radial_embedding(lengths)
        node_es = []
        for interaction, product, readout in zip(self.interactions, self.products, self.readouts):
            node_feats, sc = interaction(node_attrs=data['node_attrs'], node_feats=node_feats, edge_attrs=edge_attrs,
                                         edge_feats=edge_feats, edge_index=data['edge_index'], cutoff=cutoff)
            node_feats = product(node_feats=node_feats, sc=sc, node_attrs=data['node_attrs'])
            node_es.append(readout(node_feats).squeeze(-1))
        return torch.stack(node_es, dim=0).sum(dim=0)

    def forward(self, data, training=False, compute_force=True, compute_virials=False, compute_stress=False,
                compute_displacement=False):
        positions, shifts, displacement, num_graphs = self._prepare(data, compute_virials, compute_stress,
                                                                   compute_displacement)
        node_e0 = self.atomic_energies_fn(data['node_attrs'])
        e0 = scatter_sum(node_e0, data['batch'], dim=0, dim_size=num_graphs)
        node_inter_es = self._interactions(data, positions, shifts)
        inter_e = scatter_sum(node_inter_es, data['batch'], dim=0, dim_size=num_graphs)
        total = e0 + inter_e
        forces, virials, stress = get_outputs(total, positions, displacement, data['cell'], training, compute_force,
                                              compute_virials, compute_stress)
        return {'energy': total, 'node_energy': node_e0 + node_inter_es, 'interaction_energy': inter_e,
                'forces': forces, 'virials': virials, 'stress': stress, 'displacement': displacement}


class ScaleShiftMACE(MACE):
    def __init__(self, atomic_inter_scale, atomic_inter_shift, **kwargs):
        super().__init__(**kwargs)
        self.scale_shift = ScaleShiftBlock(atomic_inter_scale, atomic_inter_shift)

    def forward(self, data, training=False, compute_force=True, compute_virials=False, compute_stress=False,
                compute_displacement=False):
        positions, shifts, displacement, num_graphs = self._prepare(data, compute_virials, compute_stress,
                                                                   compute_displacement)
        node_e0 = self.atomic_energies_fn(data['node_attrs'])
        e0 = scatter_sum(node_e0, data['batch'], dim=0, dim_size=num_graphs)
        node_inter_es = self.scale_shift(self._interactions(data, positions, shifts))
        inter_e = scatter_sum(node_inter_es, data['batch'], dim=0, dim_size=num_graphs)
        total = e0 + inter_e
        forces, virials, stress = get_outputs(inter_e, positions, displacement, data['cell'], training, compute_force,
                                              compute_virials, compute_stress)
        return {'energy': total, 'node_energy': node_e0 + node_inter_es, 'interaction_energy': inter_e,
                'forces': forces, 'virials': virials, 'stress': stress, 'displacement': displacement}

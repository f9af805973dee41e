"""
Pins of the symmetric-contraction oracle (CPU, float64).

* dense Σ_ν U_ν·W_ν·x^⊗ν (oracle.sc.sc_dense) == MACE's nested contraction (mace_lite Contraction): two evaluation
  orders of the same polynomial;
* the symmetrised monomial table evaluated as a polynomial == sc_dense, and its derivative == autograd of sc_dense;
* the table's directional derivatives (output and gradient) == forward-mode and double-backward autograd of sc_dense;
* the product's SCSpec table (what the kernel reads) == the oracle's table, term by term;
* every U matrix satisfies the intertwiner identity U(D x, …, D x) = D_L U(x, …, x) with D from the spherical
  harmonics, and has full column rank; a planted mistake (one M row of U negated) breaks the identity;
* the table depends on the path basis only through Σ_p U·W: a contraction rewritten in another basis (U' = U·Q,
  W' = Q⁻¹·W for a random well-conditioned Q per correlation order, or a redundant basis with extra paths) gives the
  same SCSpec table, the same module output, and a planted inconsistent change (W left unrotated) does not.
"""
import copy

import numpy as np
import pytest
import torch

from mace_hip_kernels.symmetric import SCSpec
from mace_lite import blocks as B
from mace_lite.cg import U_matrix_real
from mace_lite.o3 import Irreps
from oracle import sc as osc


def _contraction(irreps_in, irrep_out, corr, n_elem=3, seed=0):
    torch.manual_seed(seed)
    with torch.random.fork_rng():
        ct = B.Contraction(Irreps(irreps_in), Irreps(irrep_out), corr, n_elem).double()
    return ct


def _uw(ct):
    U = {}
    for nu in range(1, ct.correlation + 1):
        u = ct.U_tensors(nu).double()
        u = u if u.dim() == nu + 2 else u.unsqueeze(0)
        U[nu] = u.reshape(u.shape[0], -1, u.shape[-1])
    W = {ct.correlation: ct.weights_max.detach().double()}
    for j, w in enumerate(ct.weights):
        W[ct.correlation - 1 - j] = w.detach().double()
    return U, W


CASES = [('6x0e+6x1o+6x2e', '0e', 3), ('6x0e+6x1o+6x2e', '1o', 3), ('4x0e+4x1o+4x2e+4x3o', '1o', 2),
         ('4x0e+4x1o', '1o', 3), ('5x0e+5x1o+5x2e', '2e', 2)]


@pytest.mark.parametrize('irreps_in,irrep_out,corr', CASES)
def test_dense_equals_nested(irreps_in, irrep_out, corr):
    ct = _contraction(irreps_in, irrep_out, corr)
    rng = np.random.default_rng(0)
    C, n = ct.num_features, Irreps(irreps_in).dim // ct.num_features
    x = torch.tensor(rng.normal(size=(11, C, n)))
    elem = rng.integers(0, 3, 11)
    y = torch.tensor(np.eye(3)[elem])
    U, W = _uw(ct)
    got = ct(x, y).reshape(11, C, -1)
    want = osc.sc_dense(U, W, x, elem)
    assert torch.abs(got - want).max() < 1e-10 * max(1.0, float(want.abs().max()))


@pytest.mark.parametrize('irreps_in,irrep_out,corr', CASES[:3])
def test_symmetrised_table_and_gradient(irreps_in, irrep_out, corr):
    ct = _contraction(irreps_in, irrep_out, corr)
    rng = np.random.default_rng(1)
    C, n = ct.num_features, Irreps(irreps_in).dim // ct.num_features
    x = rng.normal(size=(7, C, n))
    elem = rng.integers(0, 3, 7)
    U, W = _uw(ct)
    table = osc.poly_table({k: v.numpy() for k, v in U.items()}, {k: v.numpy() for k, v in W.items()})
    xt = torch.tensor(x, requires_grad=True)
    dense = osc.sc_dense(U, W, xt, elem)
    assert np.abs(osc.poly_eval(table, x, elem) - dense.detach().numpy()).max() < 1e-10
    g = rng.normal(size=dense.shape)
    dense.backward(torch.tensor(g))
    assert np.abs(osc.poly_grad(table, x, elem, g) - xt.grad.numpy()).max() < 1e-10


@pytest.mark.parametrize('irreps_in,irrep_out,corr', CASES[:2] + CASES[3:4])
def test_second_derivatives_equal_autograd(irreps_in, irrep_out, corr):
    """poly_jvp == forward-mode derivative of sc_dense (torch.func.jvp); poly_grad_jvp == the x-gradient of
    <v, d<g, out>/dx> by double backward through sc_dense.  A planted mistake (the pair loop of poly_grad_jvp
    run over p == q too, i.e. a squared factor's second derivative counted with the wrong multiplicity) fails."""
    ct = _contraction(irreps_in, irrep_out, corr)
    rng = np.random.default_rng(2)
    C, n = ct.num_features, Irreps(irreps_in).dim // ct.num_features
    x, v = rng.normal(size=(6, C, n)), rng.normal(size=(6, C, n))
    elem = rng.integers(0, 3, 6)
    U, W = _uw(ct)
    table = osc.poly_table({k: u.numpy() for k, u in U.items()}, {k: w.numpy() for k, w in W.items()})
    _, tangent = torch.func.jvp(lambda t: osc.sc_dense(U, W, t, elem), (torch.tensor(x),), (torch.tensor(v),))
    assert np.abs(osc.poly_jvp(table, x, elem, v) - tangent.numpy()).max() < 1e-10
    g = rng.normal(size=tangent.shape)
    xt = torch.tensor(x, requires_grad=True)
    gx, = torch.autograd.grad(osc.sc_dense(U, W, xt, elem), xt, torch.tensor(g), create_graph=True)
    hv, = torch.autograd.grad((gx * torch.tensor(v)).sum(), xt)
    got = osc.poly_grad_jvp(table, x, elem, g, v)
    assert np.abs(got - hv.numpy()).max() < 1e-10 * max(1.0, float(hv.abs().max()))
    # planted: square terms counted once more (pairs p == q included with the factor itself as direction)
    bad = got.copy()
    key = max((k for k in table if len(set(k)) < len(k)), key=lambda k: np.abs(table[k]).max())
    s_ = (table[key][elem].transpose(0, 2, 1) * g).sum(-1)
    bad[:, :, key[0]] += s_ * v[:, :, key[0]]
    assert np.abs(bad - hv.numpy()).max() > 1e-6


def test_product_table_equals_oracle_table():
    """SCSpec.T (rows the kernel reads) and its term list against the oracle's symmetrised table."""
    irreps_in = '8x0e+8x1o+8x2e'
    cts = [_contraction(irreps_in, o, 3, seed=s) for s, o in enumerate(('0e', '1o'))]

    class SC(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.contractions = torch.nn.ModuleList(cts)

    spec = SCSpec(SC())
    for bl, ct in zip(spec.blocks, cts):
        U, W = _uw(ct)
        table = osc.poly_table({k: v.numpy() for k, v in U.items()}, {k: v.numpy() for k, v in W.items()})
        kept = {k: v for k, v in table.items() if np.abs(v).max() > 1e-12}
        assert sorted(idx for idx, _ in bl['terms']) == sorted(kept)
        for idx, r0 in bl['terms']:
            for m in range(bl['M']):
                got = spec.T[:, r0 + m, :].double().numpy()
                want = kept[idx][:, m, :]
                assert np.abs(got - want).max() <= 1e-6 * max(1.0, np.abs(want).max())


@pytest.mark.parametrize('l_out', [0, 1, 2])
@pytest.mark.parametrize('nu', [1, 2, 3])
def test_u_matrix_intertwiner_and_rank(l_out, nu):
    irreps_in = Irreps('0e+1o+2e')
    target = Irreps(f'{l_out}{"e" if l_out % 2 == 0 else "o"}')
    res = U_matrix_real(irreps_in, target, nu, dtype=torch.float64)
    if not res:
        pytest.skip('no path')
    u = res[-1]
    u = u if u.dim() == nu + 2 else u.unsqueeze(0)
    u = u.reshape(u.shape[0], -1, u.shape[-1]).numpy()
    rng = np.random.default_rng(nu * 10 + l_out)
    assert osc.u_equivariance_error(u, [0, 1, 2], l_out, nu, rng) < 1e-10
    assert np.linalg.matrix_rank(u.reshape(-1, u.shape[-1])) == u.shape[-1]
    if u.shape[0] > 1:
        bad = u.copy()
        bad[0] *= -1
        assert osc.u_equivariance_error(bad, [0, 1, 2], l_out, nu, rng) > 1e-3


def rebased(ct, seed, redundant=0, consistent=True):
    """A copy of a Contraction in another path basis with the same polynomial: per correlation order ν,
    U_ν' = U_ν·A and W_ν' = B·W_ν with A·B = I on the old paths.  redundant = 0: A = Q, B = Q⁻¹ for a random
    orthogonal Q times column scales in [0.5, 2] (condition number <= 4); redundant = k: A = [Q | R] adds k paths
    (a basis with linearly dependent columns, as the full CG basis has), B = [Q⁻¹(W - R·Z); Z] for random R, Z.
    ``consistent=False`` leaves W unchanged (a planted mistake)."""
    rng = np.random.default_rng(seed)
    cr = copy.deepcopy(ct)
    with torch.no_grad():
        for nu in range(1, ct.correlation + 1):
            u = getattr(cr, f'U_matrix_{nu}')
            p = u.shape[-1]
            q, _ = np.linalg.qr(rng.normal(size=(p, p)))
            Q = torch.tensor(q * rng.uniform(0.5, 2.0, size=p), dtype=u.dtype)
            R = torch.tensor(rng.normal(size=(p, redundant)), dtype=u.dtype)
            A = torch.cat([Q, R], dim=1)                                   # [p, p + k]
            j = None if nu == ct.correlation else ct.correlation - 1 - nu
            w = cr.weights_max if j is None else cr.weights[j]
            Z = torch.tensor(rng.normal(size=(w.shape[0], redundant, w.shape[2])), dtype=w.dtype) / max(p, 1)
            wn = torch.cat([torch.einsum('pq,eqc->epc', torch.linalg.inv(Q), w - torch.einsum('pk,ekc->epc', R, Z)),
                            Z], dim=1) if consistent else torch.cat([w, Z], dim=1)
            cr.register_buffer(f'U_matrix_{nu}', torch.einsum('...p,pq->...q', u, A).contiguous())
            if j is None:
                cr.weights_max = torch.nn.Parameter(wn)
            else:
                cr.weights[j] = torch.nn.Parameter(wn)
    return cr


@pytest.mark.parametrize('redundant', [0, 3])
@pytest.mark.parametrize('irreps_in,irrep_out,corr', CASES[:3])
def test_table_is_basis_independent(irreps_in, irrep_out, corr, redundant):
    ct = _contraction(irreps_in, irrep_out, corr)
    cr = rebased(ct, seed=5, redundant=redundant)
    assert cr.U_tensors(corr).shape[-1] == ct.U_tensors(corr).shape[-1] + redundant

    class SC(torch.nn.Module):
        def __init__(self, c):
            super().__init__()
            self.contractions = torch.nn.ModuleList([c])

    a, b = SCSpec(SC(ct)), SCSpec(SC(cr))
    assert [t for t, _ in a.blocks[0]['terms']] == [t for t, _ in b.blocks[0]['terms']]
    assert torch.abs(a.T - b.T).max() <= 1e-6 * float(a.T.abs().max())
    rng = np.random.default_rng(1)
    C, n = ct.num_features, Irreps(irreps_in).dim // ct.num_features
    x = torch.tensor(rng.normal(size=(9, C, n)))
    y = torch.tensor(np.eye(3)[rng.integers(0, 3, 9)])
    want = ct(x, y)
    assert torch.abs(cr(x, y) - want).max() < 1e-10 * max(1.0, float(want.abs().max()))
    bad = SCSpec(SC(rebased(ct, seed=5, redundant=redundant, consistent=False)))
    assert torch.abs(bad.T - a.T).max() > 1e-3 * float(a.T.abs().max())

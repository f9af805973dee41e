"""
Oracle for the symmetric contraction (test infrastructure only; see oracle/__init__.py).

Restates in float64:
  * ``sc_dense``       out[b, c, M] = Σ_ν Σ_{i1..iν} (Σ_p U_ν[M, i1..iν, p]·W_ν[elem_b, p, c])·Π_k x[b, c, i_k]
                       — the mathematics the reference's polynomial encodes (reference symmetric.py:1-13), evaluated
                       densely over all index tuples (no symmetrisation, no nesting), in torch float64 so that its
                       gradient can be taken by autograd;
  * ``poly_table``     the symmetrised monomial table (reference symmetric.py:20-39): for every sorted index tuple,
                       the sum of U·W over all distinct orderings, by explicit permutation enumeration;
  * ``poly_eval``      evaluation of such a table and its derivative (reference symmetric.py:82-131).
  * ``poly_jvp`` / ``poly_grad_jvp``  directional derivatives of the output and of the gradient (the second
                       derivatives behind a double backward).
  * ``u_equivariance_error``  residual of the intertwiner identity of a U matrix under a random rotation, with the
                       rotation's representation taken from ``oracle.wigner``'s spherical harmonics.

Pinned by (tests/test_oracle_sc.py): sc_dense == MACE's nested contraction on random U/W (a different evaluation
order of the same sum); poly_eval(poly_table) == sc_dense; poly_eval derivative == autograd of sc_dense;
poly_jvp == forward-mode autograd of sc_dense; poly_grad_jvp == double backward of sc_dense in torch; U matrices
satisfy the intertwiner identity and have full column rank.
"""
import itertools

import numpy as np
import torch

from . import wigner


def sc_dense(U, W, x, elem):
    """U: {ν: [M, n^ν, p]} (M axis present, size 1 for scalars); W: {ν: [n_elem, p, c]}; x [b, c, n] → [b, c, M]."""
    x = torch.as_tensor(x, dtype=torch.float64)
    b, c, n = x.shape
    elem = torch.as_tensor(np.asarray(elem), dtype=torch.int64)
    M = next(iter(U.values())).shape[0]
    out = x.new_zeros(b, c, M)
    for nu, u in U.items():
        u = torch.as_tensor(u, dtype=torch.float64).reshape(M, n ** nu, -1)
        w = torch.as_tensor(W[nu], dtype=torch.float64)[elem]                  # [b, p, c]
        xo = x
        for _ in range(nu - 1):
            xo = (xo.unsqueeze(-1) * x.unsqueeze(-2)).reshape(b, c, -1)       # x^⊗ν [b, c, n^ν]
        t = torch.einsum('mip,bpc->bcmi', u, w)
        out = out + torch.einsum('bcmi,bci->bcm', t, xo)
    return out


def poly_table(U, W):
    """{sorted index tuple: [n_elem, M, c]} summed over all distinct orderings of the tuple."""
    table = {}
    for nu, u in U.items():
        u = np.asarray(u, dtype=np.float64)
        M = u.shape[0]
        n = round(u.shape[1] ** (1.0 / nu)) if u.ndim == 3 else u.shape[1]
        u = u.reshape((M,) + (n,) * nu + (u.shape[-1],))
        w = np.asarray(W[nu], dtype=np.float64)
        for key in itertools.combinations_with_replacement(range(n), nu):
            acc = 0.0
            for perm in set(itertools.permutations(key)):
                acc = acc + u[(slice(None),) + perm]                          # [M, p]
            table[key] = table.get(key, 0.0) + np.einsum('mp,epc->emc', acc, w)
    return table


def poly_eval(table, x, elem):
    """(out [b, c, M], d out·g/dx given g) of a symmetrised table at x [b, c, n]."""
    x = np.asarray(x, dtype=np.float64)
    elem = np.asarray(elem)
    b, c, n = x.shape
    M = next(iter(table.values())).shape[1]
    out = np.zeros((b, c, M))
    for key, coef in table.items():
        mono = np.ones((b, c))
        for i in key:
            mono = mono * x[:, :, i]
        out += coef[elem].transpose(0, 2, 1) * mono[:, :, None]
    return out


def poly_grad(table, x, elem, g):
    """∂(Σ_M g·out)/∂x for a symmetrised table: for each monomial, Σ over factor positions of the other factors."""
    x = np.asarray(x, dtype=np.float64)
    elem = np.asarray(elem)
    gx = np.zeros_like(x)
    for key, coef in table.items():
        s = (coef[elem].transpose(0, 2, 1) * g).sum(-1)                       # [b, c]
        for pos, i in enumerate(key):
            rest = np.ones_like(s)
            for q, j in enumerate(key):
                if q != pos:
                    rest = rest * x[:, :, j]
            gx[:, :, i] += s * rest
    return gx


def poly_jvp(table, x, elem, v):
    """Directional derivative of poly_eval's output along v [b, c, n]: Σ over monomials and factor positions of the
    coefficient times v at that position times the other factors.  It is the gradient of <ggx, poly_grad(g)> with
    respect to g for ggx = v, which the reference's backward guard refuses (symmetric.py:147-149)."""
    x, v = np.asarray(x, dtype=np.float64), np.asarray(v, dtype=np.float64)
    elem = np.asarray(elem)
    b, c, n = x.shape
    M = next(iter(table.values())).shape[1]
    out = np.zeros((b, c, M))
    for key, coef in table.items():
        dmono = np.zeros((b, c))
        for pos, i in enumerate(key):
            t = v[:, :, i].copy()
            for q, j in enumerate(key):
                if q != pos:
                    t = t * x[:, :, j]
            dmono += t
        out += coef[elem].transpose(0, 2, 1) * dmono[:, :, None]
    return out


def poly_grad_jvp(table, x, elem, g, v):
    """Directional derivative of poly_grad(x, g) along x + εv: for each monomial and each ordered pair of distinct
    factor positions (p, q), the coefficient·g sum times v at q times the remaining factors, added at position p.
    It is the gradient of <v, poly_grad(g)> with respect to x (a Hessian-vector product of <g, out>)."""
    x, v = np.asarray(x, dtype=np.float64), np.asarray(v, dtype=np.float64)
    elem = np.asarray(elem)
    gx = np.zeros_like(x)
    for key, coef in table.items():
        s = (coef[elem].transpose(0, 2, 1) * g).sum(-1)                       # [b, c]
        for p, i in enumerate(key):
            for q in range(len(key)):
                if q == p:
                    continue
                t = s * v[:, :, key[q]]
                for r, j in enumerate(key):
                    if r not in (p, q):
                        t = t * x[:, :, j]
                gx[:, :, i] += t
    return gx


def u_equivariance_error(u, ls_in, l_out, nu, rng):
    """max |U(D_in x, …) - D_out U(x, …)| over random x for a U matrix [M, n^ν, p] of irreps ls_in (list of l)."""
    R = wigner.random_rotation(rng)
    blocks = [wigner.wigner_D_from_sh(l, R) for l in ls_in]
    n = sum(2 * l + 1 for l in ls_in)
    D_in = np.zeros((n, n))
    o = 0
    for d in blocks:
        D_in[o:o + len(d), o:o + len(d)] = d
        o += len(d)
    D_out = wigner.wigner_D_from_sh(l_out, R)
    u = np.asarray(u, dtype=np.float64).reshape((u.shape[0],) + (n,) * nu + (u.shape[-1],))
    x = rng.normal(size=n)

    def contract(xv):                     # U(xv, xv, …, xv): [M, p]
        t = u
        for _ in range(nu):
            t = np.tensordot(t, xv, axes=([1], [0]))
        return t

    lhs = contract(D_in @ x)
    rhs = D_out @ contract(x)
    return float(np.abs(lhs - rhs).max())

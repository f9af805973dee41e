"""
Generalised Clebsch-Gordan (U) matrices of MACE's symmetric contraction, restated after mace-torch 0.3.16
``mace/tools/cg.py`` (full-CG basis).  ``U_matrix_real(irreps_in, irreps_out, ν)[-1]`` has shape
``[2L+1, n_ell, …, n_ell (ν times), n_paths]`` (the leading axis is dropped for L = 0): column p couples ν copies of the
node features (each of dimension n_ell = irreps_in.dim) into one copy of the output irrep along path p.

Paths are enumerated by recursive left-to-right coupling, every intermediate irrep allowed, each step weighted by
``wigner_3j(l_out, l_left, l_right) * sqrt(2 l_out + 1)`` ("component" normalisation), and stably sorted by output
irrep; the columns of the target irrep are stacked in that order.  The reduced basis of ``use_reduced_cg=True`` comes
from cuequivariance, which is not available here; the symmetric-contraction kernels only ever see the product U·W, so
the basis changes the parameterisation, not the kernel.
"""
import torch

from .o3 import Irrep, Irreps, wigner_3j


def _wigner_nj(irrepss, normalization='component', filter_ir_mid=None, dtype=None):
    irrepss = [Irreps(x) for x in irrepss]
    if filter_ir_mid is not None:
        filter_ir_mid = [Irrep(ir) for ir in filter_ir_mid]
    if len(irrepss) == 1:
        (irreps,) = irrepss
        ret = []
        eye = torch.eye(irreps.dim, dtype=dtype)
        i = 0
        for mul, ir in irreps:
            for _ in range(mul):
                ret.append((ir, eye[i:i + ir.dim]))
                i += ir.dim
        return ret
    *left, right = irrepss
    ret = []
    for ir_left, c_left in _wigner_nj(left, normalization, filter_ir_mid, dtype):
        i = 0
        for mul, ir in right:
            for ir_out in ir_left * ir:
                if filter_ir_mid is not None and ir_out not in filter_ir_mid:
                    continue
                c = wigner_3j(ir_out.l, ir_left.l, ir.l, dtype=dtype)
                if normalization == 'component':
                    c = c * ir_out.dim ** 0.5
                elif normalization == 'norm':
                    c = c * (ir_left.dim ** 0.5 * ir.dim ** 0.5)
                c = torch.einsum('jk,ijl->ikl', c_left.flatten(1), c)
                c = c.reshape(ir_out.dim, *(x.dim for x in left), ir.dim)
                for u in range(mul):
                    e = torch.zeros(ir_out.dim, *(x.dim for x in left), right.dim, dtype=dtype)
                    sl = slice(i + u * ir.dim, i + (u + 1) * ir.dim)
                    e[..., sl] = c
                    ret.append((ir_out, e))
            i += mul * ir.dim
    return sorted(ret, key=lambda t: t[0])


def U_matrix_real(irreps_in, irreps_out, correlation, normalization='component', filter_ir_mid=None, dtype=None):
    """[ir, U, ir, U, …] for the irreps of ``irreps_out`` reached by coupling ``correlation`` copies of irreps_in."""
    irreps_out = Irreps(irreps_out)
    irrepss = [Irreps(irreps_in)] * correlation
    if correlation == 4:
        filter_ir_mid = [(i, 1 if i % 2 == 0 else -1) for i in range(12)]
    dtype = dtype or torch.get_default_dtype()
    wigners = _wigner_nj(irrepss, normalization, filter_ir_mid, torch.float64)
    out = []
    cur_ir, cols = None, []
    for ir, base in wigners:
        if ir in irreps_out:
            if cur_ir is not None and ir != cur_ir and cols:
                out += [cur_ir, torch.stack(cols, dim=-1)]
                cols = []
            cur_ir = ir
            cols.append(base.squeeze(0) if base.shape[0] == 1 else base)
    if cols:
        out += [cur_ir, torch.stack(cols, dim=-1)]
    return [x.to(dtype) if isinstance(x, torch.Tensor) else x for x in out]

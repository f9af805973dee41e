"""
Irreps algebra, real Wigner-3j symbols, spherical harmonics, tensor products and equivariant linears, restated in
plain PyTorch after e3nn 0.4.4 (the version the reference was measured with, README.md:54).  e3nn is not installed in
this image, so the MACE host model that ``patch_model`` operates on is built from these classes instead.

The attribute surface is the one the reference duck-types (conv.py:31-51, 61-65, 84):
``TensorProduct.instructions[*].{i_in1,i_in2,i_out,connection_mode,has_weight}``, ``irreps_in1/in2/out``,
``weight_numel``, ``shared_weights``, ``internal_weights`` and ``__call__(x1, x2, weight)``.

Conventions (e3nn's):
  * an irrep is (l, p); ``Irreps`` is a tuple of (mul, irrep); features are laid out "mul_ir": block b occupies
    ``mul_b * (2 l_b + 1)`` consecutive floats, channel-major, component-minor;
  * the real basis of each l is the complex basis rotated by ``change_basis_real_to_complex`` (with the ``(-i)^l``
    phase that makes every coupling real); Wigner-3j symbols are the SU(2) Clebsch-Gordan coefficients (Racah formula)
    carried into that real basis and normalised to unit Frobenius norm;
  * spherical harmonics use y as the polar axis, so l = 1 is (x, y, z); "component" normalisation gives |Y_l|^2 = 2l+1;
  * tensor-product paths get the e3nn "component"/"element" normalisation, sqrt((2 l_out + 1) / fan_in).
"""
import collections
import functools
import math
from fractions import Fraction
from typing import NamedTuple, Tuple

import torch


# --------------------------------------------------------------------------------------------------------- irreps
class Irrep(tuple):
    """Irreducible representation (l, parity) of O(3)."""

    def __new__(cls, l, p=None):
        if p is None:
            if isinstance(l, Irrep):
                return l
            if isinstance(l, str):
                s = l.strip()
                lv = int(s[:-1])
                p = {'e': 1, 'o': -1, 'y': (-1) ** lv}[s[-1]]
                l = lv
            elif isinstance(l, tuple):
                l, p = l
        if not (isinstance(l, int) and l >= 0 and p in (-1, 1)):
            raise ValueError(f'bad irrep ({l}, {p})')
        return super().__new__(cls, (l, p))

    @property
    def l(self):  # noqa: E743
        return self[0]

    @property
    def p(self):
        return self[1]

    @property
    def dim(self):
        return 2 * self[0] + 1

    def __repr__(self):
        return f'{self[0]}{"e" if self[1] == 1 else "o"}'

    def __mul__(self, other):
        """Irreps contained in the tensor product self ⊗ other, ascending l."""
        other = Irrep(other)
        p = self.p * other.p
        return (Irrep(l, p) for l in range(abs(self.l - other.l), self.l + other.l + 1))

    def __rmul__(self, mul):
        return Irreps([(mul, self)])

    def __add__(self, other):
        return Irreps(self) + Irreps(other)


class MulIr(tuple):
    def __new__(cls, mul, ir):
        return super().__new__(cls, (mul, Irrep(ir)))

    def __getnewargs__(self):
        return (self[0], self[1])

    @property
    def mul(self):
        return self[0]

    @property
    def ir(self):
        return self[1]

    @property
    def dim(self):
        return self[0] * self[1].dim

    def __repr__(self):
        return f'{self.mul}x{self.ir}'


class Irreps(tuple):
    """Direct sum of irreps with multiplicities, e.g. ``Irreps('128x0e+128x1o')``."""

    def __new__(cls, irreps=None):
        if isinstance(irreps, Irreps):
            return super().__new__(cls, irreps)
        out = []
        if irreps is None:
            pass
        elif isinstance(irreps, Irrep):
            out.append(MulIr(1, irreps))
        elif isinstance(irreps, str):
            for part in irreps.split('+'):
                part = part.strip()
                if not part:
                    continue
                if 'x' in part:
                    m, i = part.split('x')
                    out.append(MulIr(int(m), Irrep(i)))
                else:
                    out.append(MulIr(1, Irrep(part)))
        else:
            for item in irreps:
                if isinstance(item, Irrep):
                    out.append(MulIr(1, item))
                elif isinstance(item, str):
                    out.append(MulIr(1, Irrep(item)))
                else:
                    mul, ir = item
                    out.append(MulIr(mul, Irrep(ir)))
        return super().__new__(cls, out)

    @staticmethod
    def spherical_harmonics(lmax, p=-1):
        return Irreps([(1, (l, p ** l)) for l in range(lmax + 1)])

    @property
    def dim(self):
        return sum(m.dim for m in self)

    @property
    def num_irreps(self):
        return sum(m.mul for m in self)

    @property
    def lmax(self):
        return max(ir.l for _, ir in self)

    @property
    def ls(self):
        return [ir.l for mul, ir in self for _ in range(mul)]

    def slices(self):
        s, out = 0, []
        for m in self:
            out.append(slice(s, s + m.dim))
            s += m.dim
        return out

    def count(self, ir):
        ir = Irrep(ir)
        return sum(mul for mul, irr in self if irr == ir)

    def __contains__(self, ir):
        ir = Irrep(ir)
        return any(irr == ir for _, irr in self)

    def __add__(self, other):
        return Irreps(tuple(self) + tuple(Irreps(other)))

    def __mul__(self, n):
        # e3nn semantics: tuple repetition
        if isinstance(n, Irreps):
            raise NotImplementedError
        return Irreps(tuple.__mul__(self, n))

    __rmul__ = __mul__

    def sort(self):
        """(sorted irreps, p, inv) with ``p[old] = new`` and ``inv[new] = old``, as e3nn's ``Irreps.sort``."""
        Ret = collections.namedtuple('sort', ['irreps', 'p', 'inv'])
        out = sorted((ir, i, mul) for i, (mul, ir) in enumerate(self))
        inv = tuple(i for _, i, _ in out)
        p = [0] * len(inv)
        for new, old in enumerate(inv):
            p[old] = new
        return Ret(Irreps([(mul, ir) for ir, _, mul in out]), tuple(p), inv)

    def simplify(self):
        out = []
        for mul, ir in self:
            if out and out[-1][1] == ir:
                out[-1] = (out[-1][0] + mul, ir)
            elif mul > 0:
                out.append((mul, ir))
        return Irreps(out)

    def __repr__(self):
        return '+'.join(repr(m) for m in self)

    def __getitem__(self, i):
        r = tuple.__getitem__(self, i)
        return Irreps(r) if isinstance(i, slice) else r


# ----------------------------------------------------------------------------------------------- Wigner 3j symbols
def _su2_cg(j1, m1, j2, m2, j3, m3):
    """Condon-Shortley Clebsch-Gordan coefficient <j1 m1 j2 m2 | j3 m3> (integer spins), Racah's closed form."""
    if m1 + m2 != m3 or not (abs(j1 - j2) <= j3 <= j1 + j2) or abs(m1) > j1 or abs(m2) > j2 or abs(m3) > j3:
        return 0.0
    f = math.factorial
    pre = Fraction((2 * j3 + 1) * f(j1 + j2 - j3) * f(j1 - j2 + j3) * f(-j1 + j2 + j3), f(j1 + j2 + j3 + 1))
    pre *= f(j1 + m1) * f(j1 - m1) * f(j2 + m2) * f(j2 - m2) * f(j3 + m3) * f(j3 - m3)
    s = Fraction(0)
    kmin = max(0, j2 - j3 - m1, j1 - j3 + m2)
    kmax = min(j1 + j2 - j3, j1 - m1, j2 + m2)
    for k in range(kmin, kmax + 1):
        den = f(k) * f(j1 + j2 - j3 - k) * f(j1 - m1 - k) * f(j2 + m2 - k) * f(j3 - j2 + m1 + k) * f(j3 - j1 - m2 + k)
        s += Fraction((-1) ** k, den)
    return float(s) * math.sqrt(float(pre))


def change_basis_real_to_complex(l):
    """[2l+1, 2l+1] complex matrix q with Y_complex = q @ Y_real (rows m = -l..l), including the (-i)^l phase."""
    q = torch.zeros((2 * l + 1, 2 * l + 1), dtype=torch.complex128)
    r2 = 1.0 / math.sqrt(2.0)
    for m in range(-l, 0):
        q[l + m, l + abs(m)] = r2
        q[l + m, l - abs(m)] = -1j * r2
    q[l, l] = 1.0
    for m in range(1, l + 1):
        q[l + m, l + abs(m)] = (-1) ** m * r2
        q[l + m, l - abs(m)] = 1j * (-1) ** m * r2
    return (-1j) ** l * q


@functools.lru_cache(maxsize=None)
def _wigner_3j_cached(l1, l2, l3):
    cg = torch.zeros((2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1), dtype=torch.complex128)
    for m1 in range(-l1, l1 + 1):
        for m2 in range(-l2, l2 + 1):
            m3 = m1 + m2
            if abs(m3) <= l3:
                cg[l1 + m1, l2 + m2, l3 + m3] = _su2_cg(l1, m1, l2, m2, l3, m3)
    q1, q2, q3 = (change_basis_real_to_complex(l) for l in (l1, l2, l3))
    c = torch.einsum('ij,kl,mn,ikn->jlm', q1, q2, q3.conj().T, cg)
    if c.imag.abs().max() > 1e-10:
        raise RuntimeError('wigner_3j: coupling is not real in the chosen basis')
    c = c.real
    return (c / c.norm()).contiguous()


def wigner_3j(l1, l2, l3, dtype=None, device=None):
    """Real coupling tensor C[m1, m2, m3] of l1 ⊗ l2 → l3, unit Frobenius norm (zero tensor if not allowed)."""
    if not (abs(l1 - l2) <= l3 <= l1 + l2):
        raise ValueError(f'wigner_3j({l1},{l2},{l3}) violates the triangle rule')
    c = _wigner_3j_cached(l1, l2, l3)
    return c.to(dtype=dtype or torch.get_default_dtype(), device=device)


# -------------------------------------------------------------------------------------------- spherical harmonics
def _sh_component(lmax, x, y, z):
    """Real spherical harmonics (y polar axis) of a unit vector with |Y_l|^2 = 2l+1, components concatenated l = 0..lmax.
    The l = 3 polynomials are written in terms of the (component-normalised) l = 2 ones."""
    out = [torch.ones_like(x)]
    if lmax >= 1:
        s3 = math.sqrt(3.0)
        out += [s3 * x, s3 * y, s3 * z]
    if lmax >= 2:
        s15, s5 = math.sqrt(15.0), math.sqrt(5.0)
        x2, y2, z2 = x * x, y * y, z * z
        x2z2 = x2 + z2
        sh20 = s15 * x * z
        sh21 = s15 * x * y
        sh22 = s5 * (y2 - 0.5 * x2z2)
        sh23 = s15 * y * z
        sh24 = 0.5 * s15 * (z2 - x2)
        out += [sh20, sh21, sh22, sh23, sh24]
    if lmax >= 3:
        s42, s7, s168 = math.sqrt(42.0), math.sqrt(7.0), math.sqrt(168.0)
        out += [
            s42 / 6.0 * (sh20 * z + sh24 * x),
            s7 * sh20 * y,
            s168 / 8.0 * (4.0 * y2 - x2z2) * x,
            0.5 * s7 * y * (2.0 * y2 - 3.0 * x2z2),
            s168 / 8.0 * z * (4.0 * y2 - x2z2),
            s7 * sh24 * y,
            s42 / 6.0 * (sh24 * z - sh20 * x),
        ]
    if lmax >= 4:
        raise NotImplementedError('spherical harmonics implemented up to l = 3')
    return torch.stack(out, dim=-1)


class SphericalHarmonics(torch.nn.Module):
    """``o3.SphericalHarmonics(irreps, normalize, normalization)`` for l ≤ 3, "component" or "norm" normalisation."""

    def __init__(self, irreps_out, normalize=True, normalization='component'):
        super().__init__()
        self.irreps_out = Irreps(irreps_out)
        self.normalize = normalize
        self.normalization = normalization
        self._ls = [ir.l for _, ir in self.irreps_out]
        self.lmax = max(self._ls)
        if self._ls != list(range(self.lmax + 1)):
            raise ValueError('expected 0e+1o+...+lmax')
        scale = []
        for l in self._ls:
            s = 1.0 if normalization == 'component' else 1.0 / math.sqrt(2 * l + 1)
            scale += [s] * (2 * l + 1)
        self._scale = scale                   # python floats: exact in any dtype the module is cast to
        self._scale_t = {}

    def forward(self, vec):
        if self.normalize:
            vec = vec / vec.norm(dim=-1, keepdim=True).clamp_min(1e-30)
        sh = _sh_component(self.lmax, vec[..., 0], vec[..., 1], vec[..., 2])
        key = (sh.device, sh.dtype)
        if key not in self._scale_t:
            self._scale_t[key] = torch.tensor(self._scale, dtype=sh.dtype, device=sh.device)
        return sh * self._scale_t[key]


# ------------------------------------------------------------------------------------------------ tensor products
class Instruction(NamedTuple):
    i_in1: int
    i_in2: int
    i_out: int
    connection_mode: str
    has_weight: bool
    path_weight: float
    path_shape: Tuple[int, ...]


class TensorProduct(torch.nn.Module):
    """e3nn ``o3.TensorProduct`` for the 'uvu' and 'uvw' connection modes.

    ``out[.., o3 + w*d3 + k] += sqrt(alpha) * sum_{ij} C[i,j,k] * (weights) * x1[.., o1 + u*d1 + i] * x2[.., o2 + v*d2 + j]``
    with alpha = (2 l_out + 1) / sum_{instructions into i_out} fan-in ("component" irreps, "element" paths).
    """

    def __init__(self, irreps_in1, irreps_in2, irreps_out, instructions, in1_var=None, in2_var=None, out_var=None,
                 irrep_normalization='component', path_normalization='element', internal_weights=None,
                 shared_weights=None):
        super().__init__()
        self.irreps_in1, self.irreps_in2, self.irreps_out = Irreps(irreps_in1), Irreps(irreps_in2), Irreps(irreps_out)
        ins = []
        for x in instructions:
            x = tuple(x)
            i1, i2, io, mode, train = x[:5]
            pw = x[5] if len(x) > 5 else 1.0
            m1, m2, mo = self.irreps_in1[i1].mul, self.irreps_in2[i2].mul, self.irreps_out[io].mul
            shape = {'uvw': (m1, m2, mo), 'uvu': (m1, m2), 'uvv': (m1, m2), 'uuw': (m1, mo), 'uuu': (m1,)}[mode]
            ins.append(Instruction(i1, i2, io, mode, bool(train), float(pw), shape))
        self.instructions = ins
        in1_var = [1.0] * len(self.irreps_in1) if in1_var is None else list(in1_var)
        in2_var = [1.0] * len(self.irreps_in2) if in2_var is None else list(in2_var)
        out_var = [1.0] * len(self.irreps_out) if out_var is None else list(out_var)

        def num_elements(i):
            m1, m2 = self.irreps_in1[i.i_in1].mul, self.irreps_in2[i.i_in2].mul
            return {'uvw': m1 * m2, 'uvu': m2, 'uvv': m1, 'uuw': m1, 'uuu': 1}[i.connection_mode]

        coeffs = []
        for i in ins:
            ir1, ir2, iro = self.irreps_in1[i.i_in1].ir, self.irreps_in2[i.i_in2].ir, self.irreps_out[i.i_out].ir
            if ir1.p * ir2.p != iro.p or not abs(ir1.l - ir2.l) <= iro.l <= ir1.l + ir2.l:
                raise ValueError(f'instruction {i} violates selection rules')
            alpha = {'component': iro.dim, 'norm': ir1.dim * ir2.dim, 'none': 1}[irrep_normalization]
            if path_normalization == 'element':
                x = sum(in1_var[j.i_in1] * in2_var[j.i_in2] * num_elements(j) for j in ins if j.i_out == i.i_out)
            elif path_normalization == 'path':
                x = in1_var[i.i_in1] * in2_var[i.i_in2] * num_elements(i) * sum(1 for j in ins if j.i_out == i.i_out)
            else:
                x = 1.0
            if x > 0:
                alpha /= x
            alpha *= out_var[i.i_out] * i.path_weight
            coeffs.append(math.sqrt(alpha))
        self._coeffs = coeffs
        if shared_weights is False and internal_weights is None:
            internal_weights = False
        if shared_weights is None:
            shared_weights = True
        if internal_weights is None:
            internal_weights = shared_weights and any(i.has_weight for i in ins)
        self.shared_weights, self.internal_weights = shared_weights, internal_weights
        self.weight_numel = sum(math.prod(i.path_shape) for i in ins if i.has_weight)
        if internal_weights:
            self.weight = torch.nn.Parameter(torch.randn(self.weight_numel))
        else:
            self.register_buffer('weight', torch.Tensor(), persistent=False)
        # coupling tables are kept out of the module's buffers: they are constants of the operation, recomputed in
        # float64 and cast per (device, dtype), so casting the model to float32 and back cannot round them
        self._w3j_ls, self._w3j = [], {}
        for k, i in enumerate(ins):
            l1, l2, lo = self.irreps_in1[i.i_in1].ir.l, self.irreps_in2[i.i_in2].ir.l, self.irreps_out[i.i_out].ir.l
            self._w3j_ls.append((l1, l2, lo))

    def __repr__(self):
        return f'TensorProduct({self.irreps_in1} x {self.irreps_in2} -> {self.irreps_out} | {len(self.instructions)} paths)'

    def _coupling(self, k, like):
        key = (like.device, like.dtype)
        if key not in self._w3j:
            self._w3j[key] = [wigner_3j(*ls, dtype=like.dtype, device=like.device) for ls in self._w3j_ls]
        return self._w3j[key][k]

    def forward(self, x1, x2, weight=None):
        if weight is None:
            if not self.internal_weights:
                raise ValueError('weights must be given for external-weight tensor products')
            weight = self.weight
        lead = torch.broadcast_shapes(x1.shape[:-1], x2.shape[:-1])
        x1 = x1.expand(*lead, x1.shape[-1]).reshape(-1, x1.shape[-1])
        x2 = x2.expand(*lead, x2.shape[-1]).reshape(-1, x2.shape[-1])
        z = x1.shape[0]
        if self.shared_weights:
            weight = weight.reshape(1, -1)
        else:
            weight = weight.reshape(-1, weight.shape[-1])
        s1, s2 = self.irreps_in1.slices(), self.irreps_in2.slices()
        blocks = [None] * len(self.irreps_out)
        woff = 0
        xx = {}              # outer products shared by the instructions of one input pair (e3nn's xx_dict)
        for k, i in enumerate(self.instructions):
            mi1, mi2, mo = self.irreps_in1[i.i_in1], self.irreps_in2[i.i_in2], self.irreps_out[i.i_out]
            a = x1[:, s1[i.i_in1]].reshape(z, mi1.mul, mi1.ir.dim)
            b = x2[:, s2[i.i_in2]].reshape(z, mi2.mul, mi2.ir.dim)
            n = math.prod(i.path_shape) if i.has_weight else 0
            w = weight[:, woff:woff + n].reshape(weight.shape[0], *i.path_shape) if i.has_weight else None
            woff += n
            if i.connection_mode not in ('uvu', 'uvw'):
                raise NotImplementedError(i.connection_mode)
            l1, l2 = mi1.ir.l, mi2.ir.l
            if w is not None and (l1 == 0 or l2 == 0):
                # e3nn's specialised code: a scalar operand makes the coupling δ/sqrt(2l+1) (1 for 0x0->0), so the
                # Clebsch-Gordan contraction is skipped
                t = (torch.einsum('zu,zvj->zuvj', a[..., 0], b) if l1 == 0 else
                     torch.einsum('zui,zv->zuvi', a, b[..., 0]))
                if l1 or l2:
                    t = t / math.sqrt(mo.ir.dim)
            else:
                key = (i.i_in1, i.i_in2)
                if key not in xx:
                    xx[key] = torch.einsum('zui,zvj->zuvij', a, b)
                t = torch.einsum('zuvij,ijk->zuvk', xx[key], self._coupling(k, x1))
            if i.connection_mode == 'uvu':
                out = t.sum(2) if w is None else torch.einsum('zuvk,zuv->zuk', t, w.expand(z, *i.path_shape))
            elif w.shape[0] == 1:
                out = torch.einsum('zuvk,uvw->zwk', t, w[0])
            else:
                out = torch.einsum('zuvk,zuvw->zwk', t, w)
            out = self._coeffs[k] * out.reshape(z, mo.dim)
            blocks[i.i_out] = out if blocks[i.i_out] is None else blocks[i.i_out] + out
        res = [blk if blk is not None else x1.new_zeros(z, mo.dim) for blk, mo in zip(blocks, self.irreps_out)]
        out = torch.cat(res, dim=-1) if res else x1.new_zeros(z, 0)
        return out.reshape(*lead, self.irreps_out.dim)


class FullyConnectedTensorProduct(TensorProduct):
    """All allowed 'uvw' paths in1 ⊗ in2 → out, shared internal weights (e3nn ``o3.FullyConnectedTensorProduct``)."""

    def __init__(self, irreps_in1, irreps_in2, irreps_out, **kw):
        irreps_in1, irreps_in2, irreps_out = Irreps(irreps_in1), Irreps(irreps_in2), Irreps(irreps_out)
        ins = [(i1, i2, io, 'uvw', True, 1.0)
               for i1, (_, ir1) in enumerate(irreps_in1)
               for i2, (_, ir2) in enumerate(irreps_in2)
               for io, (_, iro) in enumerate(irreps_out)
               if iro in list(ir1 * ir2)]
        super().__init__(irreps_in1, irreps_in2, irreps_out, ins, **kw)


class Linear(torch.nn.Module):
    """Equivariant linear map (e3nn ``o3.Linear``): every (in, out) block pair with equal irrep, weights [mul_in, mul_out],
    "element" path normalisation 1/sqrt(sum of mul_in feeding an output block)."""

    def __init__(self, irreps_in, irreps_out, internal_weights=True, shared_weights=True):
        super().__init__()
        self.irreps_in, self.irreps_out = Irreps(irreps_in), Irreps(irreps_out)
        self.instructions = [(i, o) for i, (_, iri) in enumerate(self.irreps_in)
                             for o, (_, iro) in enumerate(self.irreps_out) if iri == iro]
        fan = collections.Counter()
        for i, o in self.instructions:
            fan[o] += self.irreps_in[i].mul
        self._alpha = [1.0 / math.sqrt(fan[o]) for _, o in self.instructions]
        self.weight_numel = sum(self.irreps_in[i].mul * self.irreps_out[o].mul for i, o in self.instructions)
        self.weight = torch.nn.Parameter(torch.randn(self.weight_numel))

    def forward(self, x):
        lead = x.shape[:-1]
        x = x.reshape(-1, x.shape[-1])
        z = x.shape[0]
        si = self.irreps_in.slices()
        outs = [None] * len(self.irreps_out)
        off = 0
        for (i, o), alpha in zip(self.instructions, self._alpha):
            mi, mo = self.irreps_in[i], self.irreps_out[o]
            n = mi.mul * mo.mul
            w = self.weight[off:off + n].reshape(mi.mul, mo.mul)
            off += n
            xi = x[:, si[i]].reshape(z, mi.mul, mi.ir.dim)
            y = torch.einsum('zui,uw->zwi', xi, w) * alpha
            outs[o] = y if outs[o] is None else outs[o] + y
        res = [(b.reshape(z, mo.dim) if b is not None else x.new_zeros(z, mo.dim))
               for b, mo in zip(outs, self.irreps_out)]
        return torch.cat(res, dim=-1).reshape(*lead, self.irreps_out.dim)

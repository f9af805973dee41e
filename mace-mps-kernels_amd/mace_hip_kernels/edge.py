"""
Edge spherical harmonics for MACE on MI355X: a drop-in for the model's ``spherical_harmonics`` module (e3nn
``o3.SphericalHarmonics(0e+1o+...+l_max, normalize=True)``), which evaluates Y(v/|v|) for every edge vector.

On the GPU the e3nn module is a few dozen elementwise launches over the [E] vector components in the forward and
about as many again in the backward.  Here one thread handles one edge: the forward reads the 3 components and
writes the (l_max+1)^2 harmonics; the backward reads the vector and the incoming gradient and writes
dL/dv = (a - u (u·a)) / |v| with u = v/|v| and a = Σ_c gY_c ∂Y_c/∂u — the chain rule through the normalisation.

The polynomials are e3nn's (y is the polar axis; "component" normalisation has |Y_l|^2 = 2l+1 on the unit sphere,
"norm" divides degree l by sqrt(2l+1)).  They are written once as sympy expressions, from which both the forward
and the derivative code are generated, with common subexpressions shared and every constant an fp32 literal.
"""
import math

import numpy as np
import sympy as sp
from sympy.printing.c import C99CodePrinter
import torch

from . import _native

BLOCK = 256          # threads (edges) per workgroup
EPS = 1e-30          # |v| is clamped to this before dividing (as the model's normalisation does)


def sh_supported(mod):
    """(ok, reason) — whether a SphericalHarmonics module can be replaced."""
    try:
        ls = [ir.l for _, ir in mod.irreps_out]
        muls = [m for m, _ in mod.irreps_out]
        if ls != list(range(len(ls))) or any(m != 1 for m in muls):
            return False, 'irreps_out must be 1x0e+1x1o+...+1xl_max'
        if max(ls) > 3:
            return False, f'l_max {max(ls)} > 3'
        if not getattr(mod, 'normalize', False):
            return False, 'only normalize=True is supported'
        if getattr(mod, 'normalization', 'component') not in ('component', 'norm'):
            return False, f'normalization {mod.normalization!r}'
    except (AttributeError, TypeError) as e:
        return False, f'not an e3nn SphericalHarmonics ({e})'
    return True, ''


def _polynomials(lmax):
    """Real harmonics of a unit vector (x, y, z), component normalisation, l = 0..lmax concatenated."""
    x, y, z = sp.symbols('x y z', real=True)
    out = [sp.Integer(1)]
    if lmax >= 1:
        out += [sp.sqrt(3) * x, sp.sqrt(3) * y, sp.sqrt(3) * z]
    if lmax >= 2:
        x2z2 = x ** 2 + z ** 2
        sh20 = sp.sqrt(15) * x * z
        sh21 = sp.sqrt(15) * x * y
        sh22 = sp.sqrt(5) * (y ** 2 - x2z2 / 2)
        sh23 = sp.sqrt(15) * y * z
        sh24 = sp.sqrt(15) / 2 * (z ** 2 - x ** 2)
        out += [sh20, sh21, sh22, sh23, sh24]
    if lmax >= 3:
        out += [
            sp.sqrt(42) / 6 * (sh20 * z + sh24 * x),
            sp.sqrt(7) * sh20 * y,
            sp.sqrt(168) / 8 * (4 * y ** 2 - x2z2) * x,
            sp.sqrt(7) / 2 * y * (2 * y ** 2 - 3 * x2z2),
            sp.sqrt(168) / 8 * z * (4 * y ** 2 - x2z2),
            sp.sqrt(7) * sh24 * y,
            sp.sqrt(42) / 6 * (sh24 * z - sh20 * x),
        ]
    return (x, y, z), [sp.expand(e) for e in out]


def _lit(v):
    return f'{float(np.float32(v)).hex()}f'


class _F32Printer(C99CodePrinter):
    """C printer for fp32 code: every number an exact fp32 literal, small integer powers as products."""

    def _print_Float(self, e):
        return _lit(float(e))

    def _print_Integer(self, e):
        return _lit(int(e))

    def _print_Rational(self, e):
        return _lit(float(e))

    def _print_Pow(self, e):
        b, p = e.args
        if p.is_Integer and 2 <= int(p) <= 4:
            s = self._print(b)
            return '(' + '*'.join([s] * int(p)) + ')'
        if p.is_number:
            return f'powf({self._print(b)}, {_lit(float(p))})'
        return super()._print_Pow(e)


def _emit(exprs, names, ind, prefix):
    """CSE + fp32 printing of ``exprs`` assigned to ``names``; temporaries are ``prefix``0, 1, ..."""
    pr = _F32Printer()
    reps, red = sp.cse([sp.N(e, 30) for e in exprs], symbols=sp.numbered_symbols(prefix))
    L = [f'{ind}const float {pr.doprint(s)} = {pr.doprint(v)};' for s, v in reps]
    L += [f'{ind}{n} = {pr.doprint(v)};' for n, v in zip(names, red)]
    return L


class SHSpec:
    def __init__(self, mod):
        ok, why = sh_supported(mod)
        if not ok:
            raise ValueError(why)
        self.lmax = max(ir.l for _, ir in mod.irreps_out)
        self.dim = (self.lmax + 1) ** 2
        self.norm = mod.normalization == 'norm'
        self.scale = []
        for l in range(self.lmax + 1):
            self.scale += [1.0 / math.sqrt(2 * l + 1) if self.norm else 1.0] * (2 * l + 1)

    def kname(self, base):
        return f'{base}_l{self.lmax}_{"norm" if self.norm else "comp"}'

    def bytes(self, E):
        """Algorithmic HBM bytes of (forward, backward) over ``E`` edges: the vector and Y; the vector, gY and dL/dv."""
        return E * (12 + 4 * self.dim), E * (12 + 4 * self.dim + 12)


def math_lines(spec):
    """The per-edge arithmetic as plain C statements (no HIP constructs), shared by the kernels and the CPU check of
    the generated code: ``head`` reads ``vx, vy, vz`` and defines ``r``, ``rc`` and the unit vector ``x, y, z``;
    ``fwd`` defines ``Y0..Y{dim-1}``; ``bwd`` reads ``g0..g{dim-1}`` and defines the gradient ``ox, oy, oz``."""
    (x, y, z), polys = _polynomials(spec.lmax)
    polys = [p * sp.Float(s, 30) for p, s in zip(polys, spec.scale)]
    gs = sp.symbols(f'g0:{spec.dim}', real=True)
    a = [sum(g * sp.diff(p, v) for g, p in zip(gs, polys)) for v in (x, y, z)]
    head = [
        'const float r = sqrtf(vx * vx + vy * vy + vz * vz);',
        f'const float rc = fmaxf(r, {_lit(EPS)});',
        'const float x = vx / rc, y = vy / rc, z = vz / rc;',
    ]
    fwd = [f'float Y{c};' for c in range(spec.dim)] + _emit(polys, [f'Y{c}' for c in range(spec.dim)], '', 't')
    bwd = ['float ax, ay, az;'] + _emit(a, ['ax', 'ay', 'az'], '', 'q') + [
        'float ox, oy, oz;',
        f'if (r >= {_lit(EPS)}) {{                  /* clamp_min passes the gradient at r == EPS */',
        '  const float ua = x * ax + y * ay + z * az;   /* d(v/|v|)/dv = (I - u u^T) / |v| */',
        '  ox = (ax - x * ua) / r; oy = (ay - y * ua) / r; oz = (az - z * ua) / r;',
        '} else {',
        '  ox = ax / rc; oy = ay / rc; oz = az / rc;     /* |v| clamped: only the numerator varies */',
        '}',
    ]
    return dict(head=head, fwd=fwd, bwd=bwd)


def source(spec):
    """HIP source of ``sh_fwd`` and ``sh_bwd`` for one (l_max, normalisation)."""
    m = math_lines(spec)
    ind = lambda lines: ['  ' + l for l in lines]  # noqa: E731
    head = ['  const long long e = (long long)mh_xcd_block(blockIdx.x, gridDim.x) * BLOCK + threadIdx.x;',
            '  if (e >= E) return;',
            '  const float vx = vec[3 * e], vy = vec[3 * e + 1], vz = vec[3 * e + 2];'] + ind(m['head'])
    L = [_native.device_header(), f'#define BLOCK {BLOCK}', f'#define DIM {spec.dim}']
    L += [f'extern "C" __global__ __launch_bounds__(BLOCK) void {spec.kname("sh_fwd")}(',
          '    const float* __restrict__ vec, float* __restrict__ Y, long long E) {'] + head + ind(m['fwd'])
    L += ['  float* __restrict__ ye = Y + e * DIM;'] + [f'  ye[{c}] = Y{c};' for c in range(spec.dim)]
    L += ['}', '']
    L += [f'extern "C" __global__ __launch_bounds__(BLOCK) void {spec.kname("sh_bwd")}(',
          '    const float* __restrict__ vec, const float* __restrict__ gY, float* __restrict__ gv, long long E) {']
    L += head
    L += ['  const float* __restrict__ ge = gY + e * DIM;'] + [f'  const float g{c} = ge[{c}];' for c in range(spec.dim)]
    L += ind(m['bwd'])
    L += ['  gv[3 * e] = ox; gv[3 * e + 1] = oy; gv[3 * e + 2] = oz;', '}', '']
    return '\n'.join(L)


def source_second(spec):
    """HIP source of the second-order kernels behind a double backward: the statements of ``sh_fwd`` / ``sh_bwd`` on
    dual numbers (``mh_dual``) with the edge vectors carrying a direction dv.  ``sh_jvp`` writes dY = (dY/dv) dv;
    ``sh_bwd2`` writes the derivative of the vector gradient along dv for a fixed gY (a Hessian-vector product of
    <gY, Y>)."""
    m = math_lines(spec)
    ind = lambda lines: ['  ' + l for l in lines]  # noqa: E731
    head = ['  const long long e = (long long)mh_xcd_block(blockIdx.x, gridDim.x) * BLOCK + threadIdx.x;',
            '  if (e >= E) return;',
            '  const mh_dual vx(vec[3 * e], dv[3 * e]), vy(vec[3 * e + 1], dv[3 * e + 1]), '
            'vz(vec[3 * e + 2], dv[3 * e + 2]);'] + ind(_native.dualize(m['head']))
    L = [_native.device_header(), _native.dual_header(), f'#define BLOCK {BLOCK}', f'#define DIM {spec.dim}']
    L += [f'extern "C" __global__ __launch_bounds__(BLOCK) void {spec.kname("sh_jvp")}(',
          '    const float* __restrict__ vec, const float* __restrict__ dv, float* __restrict__ dY, long long E) {']
    L += head + ind(_native.dualize(m['fwd']))
    L += ['  float* __restrict__ ye = dY + e * DIM;'] + [f'  ye[{c}] = Y{c}.d;' for c in range(spec.dim)] + ['}', '']
    L += [f'extern "C" __global__ __launch_bounds__(BLOCK) void {spec.kname("sh_bwd2")}(',
          '    const float* __restrict__ vec, const float* __restrict__ dv, const float* __restrict__ gY,',
          '    float* __restrict__ gv, long long E) {']
    L += head
    L += ['  const float* __restrict__ ge = gY + e * DIM;'] + [f'  const float g{c} = ge[{c}];' for c in range(spec.dim)]
    L += ind(_native.dualize(m['bwd']))
    L += ['  gv[3 * e] = ox.d; gv[3 * e + 1] = oy.d; gv[3 * e + 2] = oz.d;', '}', '']
    return '\n'.join(L)


_DOUBLE_BACKWARD = ('mace_hip_kernels: double backward (create_graph=True, e.g. training on forces/stress or an '
                    'autograd Hessian) is not enabled for this HIP module; patch with '
                    'patch_model(model, double_backward=True)')


def _sh_bwd(op, vec, g):
    v = vec.reshape(-1, 3).contiguous()
    g = g.reshape(-1, op.spec.dim).contiguous()
    gv = torch.empty_like(v)
    _native.launch(f'sh_bwd[{op.tag}]', _native.load().mh_sh_bwd, op.module.handle, _native.ptr(v), _native.ptr(g),
                   _native.ptr(gv), v.shape[0], _native.stream_of(v))
    return gv.reshape(vec.shape)


class _SHFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, vec, op):
        if vec.dtype != torch.float32 or not vec.is_cuda:
            raise TypeError('mace_hip_kernels: spherical harmonics expect float32 GPU input')
        if vec.shape[-1] != 3:
            raise ValueError(f'edge vectors must be [..., 3], got {tuple(vec.shape)}')
        lead = vec.shape[:-1]
        v = vec.reshape(-1, 3).contiguous()
        E = v.shape[0]
        out = torch.empty(E, op.spec.dim, device=v.device, dtype=torch.float32)
        _native.launch(f'sh_fwd[{op.tag}]', _native.load().mh_sh_fwd, op.module.handle, _native.ptr(v),
                       _native.ptr(out), E, _native.stream_of(v))
        ctx.save_for_backward(vec)           # the input itself: a double backward differentiates through it
        ctx.op = op
        return out.reshape(*lead, op.spec.dim)

    @staticmethod
    def backward(ctx, g):
        vec, = ctx.saved_tensors
        op = ctx.op
        if torch.is_grad_enabled():          # only true under create_graph=True
            if not op.double_backward:
                raise RuntimeError(_DOUBLE_BACKWARD)
            return _SHAdjFn.apply(g, vec, op), None
        return _sh_bwd(op, vec, g), None


class _SHAdjFn(torch.autograd.Function):
    """dL/dv = (dY/dv)^T gY as a function of (gY, v), for a double backward: with ggv the incoming gradient,
    d<ggv, dL/dv>/dgY = (dY/dv) ggv (``sh_jvp``) and d<ggv, dL/dv>/dv the Hessian-vector product (``sh_bwd2``).
    Third derivatives are not provided."""

    @staticmethod
    def forward(ctx, g, vec, op):
        ctx.save_for_backward(g, vec)
        ctx.op = op
        return _sh_bwd(op, vec, g)

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, ggv):
        g, vec = ctx.saved_tensors
        op = ctx.op
        m = op.second_module()
        v = vec.reshape(-1, 3).contiguous()
        dv = ggv.reshape(-1, 3).contiguous()
        E, P, lib = v.shape[0], _native.ptr, _native.load()
        gg = gv = None
        if ctx.needs_input_grad[0]:
            gg = torch.empty(E, op.spec.dim, device=v.device, dtype=torch.float32)
            _native.launch(f'sh_jvp[{op.tag}]', lib.mh_sh_jvp, m.handle, P(v), P(dv), P(gg), E, _native.stream_of(v))
            gg = gg.reshape(g.shape)
        if ctx.needs_input_grad[1]:
            g2 = g.reshape(-1, op.spec.dim).contiguous()
            gv = torch.empty_like(v)
            _native.launch(f'sh_bwd2[{op.tag}]', lib.mh_sh_bwd2, m.handle, P(v), P(dv), P(g2), P(gv), E,
                           _native.stream_of(v))
            gv = gv.reshape(vec.shape)
        return gg, gv, None


class HipSphericalHarmonics(torch.nn.Module):
    """Drop-in for the model's ``spherical_harmonics``: ``forward(vectors[..., 3]) -> [..., (l_max+1)^2]``."""

    def __init__(self, mod, device=None):
        super().__init__()
        self.spec = SHSpec(mod)
        self.source = source(self.spec)
        code = _native.compile_source(self.source)
        dev = torch.device(device) if device is not None else torch.device('cuda', torch.cuda.current_device())
        self._device = dev
        with torch.cuda.device(dev):
            self.module = _native.Module(code, {
                _native.MH_SH_FWD: (self.spec.kname('sh_fwd'), BLOCK, BLOCK),
                _native.MH_SH_BWD: (self.spec.kname('sh_bwd'), BLOCK, BLOCK),
            })
        self.irreps_out = mod.irreps_out
        self.normalize, self.normalization = mod.normalize, mod.normalization
        self.original = [mod]
        self.tag = 'spherical_harmonics'
        # a backward under create_graph=True raises (the reference's behaviour) unless this is set; then the
        # gradient is differentiable once more through the second-order kernels (second_module)
        self.double_backward = False
        self._second = None

    def second_module(self):
        """The module of the second-order kernels (``sh_jvp``, ``sh_bwd2``), compiled on first use."""
        if self._second is None:
            code = _native.compile_source(source_second(self.spec))
            with torch.cuda.device(self._device):
                self._second = _native.Module(code, {
                    _native.MH_SH_JVP: (self.spec.kname('sh_jvp'), BLOCK, BLOCK),
                    _native.MH_SH_BWD2: (self.spec.kname('sh_bwd2'), BLOCK, BLOCK)})
        return self._second

    def forward(self, vec):
        from . import edgefeat
        Y = edgefeat.take_harmonics(self, vec)      # made in the geometry's pass (edgefeat), if it was
        return Y if Y is not None else _SHFn.apply(vec, self)

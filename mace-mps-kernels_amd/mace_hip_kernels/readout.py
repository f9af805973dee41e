"""
MACE's readout heads on MI355X: drop-ins for ``LinearReadoutBlock`` (e3nn Linear irreps -> 1x0e) and
``NonLinearReadoutBlock`` (Linear -> H x0e, the normalised SiLU, Linear -> 1x0e), which turn each interaction's node
features into per-node energies.  Only the input's scalar block contributes:

    linear:     e[n] = sum_u x[n, o0 + u] w[u]
    non-linear: e[n] = sum_k w2[k] c silu(h[n, k]),   h[n, k] = sum_u x[n, o0 + u] W1[u, k]

On the GPU the e3nn modules are a handful of launches per direction (batched GEMMs for each Linear, the activation
and its normalisation, their backward and a zero-filled gradient for the non-scalar blocks); here each direction is
one kernel.  Sixteen lanes serve one node: each lane reads the node's scalar block (the sixteen lanes of a node read
the same addresses, one transaction), computes its share of the hidden units or of the dot product with the
weights compiled in as fp32 tables, and the partial sums meet in a 16-lane butterfly.  The backward recomputes h
and writes the whole input gradient row, zeros in the non-scalar blocks.

The weights are read off the module when it is patched, in float64 (basis probes), and the restated head is checked
against the module on random inputs; there are no weight gradients (inference, like the other drop-ins).
"""
import copy

import numpy as np
import torch

from . import _native
from .pending import Pending, slot

LANES = 16           # lanes per node
BLOCK = 256          # 16 nodes per workgroup


def _lit(v):
    return f'{float(np.float32(v)).hex()}f'


def _scalar_block(irreps):
    """(offset, multiplicity, total dimension) of the only 0e block of ``irreps`` (None when not exactly one)."""
    off, found, dim = 0, [], 0
    for mul, ir in irreps:
        d = 2 * ir.l + 1
        if ir.l == 0 and ir.p == 1:
            found.append((off, mul))
        off += mul * d
    dim = off
    return (found[0][0], found[0][1], dim) if len(found) == 1 else None


def _kind(mod):
    """'LinearReadoutBlock' / 'NonLinearReadoutBlock' for those classes and their subclasses, else the class name."""
    names = [c.__name__ for c in type(mod).__mro__]
    for k in ('LinearReadoutBlock', 'NonLinearReadoutBlock'):
        if k in names:
            return k
    return type(mod).__name__


def readout_supported(mod):
    """(ok, reason) — whether a MACE readout head can be replaced."""
    kind = _kind(mod)
    try:
        if kind == 'LinearReadoutBlock':
            lin = mod.linear
            ins, outs = lin.irreps_in, lin.irreps_out
        elif kind == 'NonLinearReadoutBlock':
            ins, outs = mod.linear_1.irreps_in, mod.linear_2.irreps_out
            hid = mod.linear_1.irreps_out
            if any(ir.l != 0 or ir.p != 1 for _, ir in hid):
                return False, 'hidden irreps not all 0e'
            if sum(mul for mul, _ in hid) > 64:
                return False, 'more than 64 hidden units'
        else:
            return False, f'{kind} is not a MACE readout block'
        if [(mul, str(ir)) for mul, ir in outs] != [(1, '0e')]:
            return False, f'output irreps {outs} (only 1x0e)'
        sb = _scalar_block(ins)
        if sb is None:
            return False, 'input without exactly one 0e block'
        if sb[1] % LANES:
            return False, f'scalar multiplicity {sb[1]} not a multiple of {LANES}'
        if sb[0] % 4 or sb[2] % 4:
            return False, 'scalar block not 16-byte aligned in the row'
    except (AttributeError, TypeError) as e:
        return False, f'unrecognised readout ({e})'
    return True, ''


class ReadoutSpec:
    """The restated head: kind, input layout, weights (float64) and the activation's normalisation constant."""

    def __init__(self, mod):
        ok, why = readout_supported(mod)
        if not ok:
            raise ValueError(why)
        self.kind = 'linear' if _kind(mod) == 'LinearReadoutBlock' else 'mlp'
        first = mod.linear if self.kind == 'linear' else mod.linear_1
        self.o0, self.C0, self.Din = _scalar_block(first.irreps_in)
        m64 = copy.deepcopy(mod).to('cpu', torch.float64)
        basis = torch.zeros(self.C0, self.Din, dtype=torch.float64)
        basis[torch.arange(self.C0), self.o0 + torch.arange(self.C0)] = 1.0
        with torch.no_grad():
            if self.kind == 'linear':
                self.w = m64.linear(basis).numpy()[:, 0]                                    # [C0]
            else:
                self.W1 = m64.linear_1(basis).numpy()                                       # [C0, H]
                self.H = self.W1.shape[1]
                self.w2 = m64.linear_2(torch.eye(self.H, dtype=torch.float64)).numpy()[:, 0]  # [H]
                z = torch.linspace(-6.0, 6.0, 101, dtype=torch.float64).reshape(-1, 1).repeat(1, self.H)
                a = m64.non_linearity(z).numpy()
                s = torch.nn.functional.silu(z).numpy()
                mask = np.abs(s) > 1e-3
                self.c = float(np.median(a[mask] / s[mask]))
                if not np.allclose(a, self.c * s, rtol=1e-10, atol=1e-12):
                    raise ValueError('the activation is not a scaled SiLU')
        rng = np.random.default_rng(0)
        x = rng.normal(size=(9, self.Din))
        with torch.no_grad():
            ref = m64(torch.tensor(x)).numpy()
        got = self.apply(x)
        err = np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-300)
        if not err < 1e-10:
            raise ValueError(f'the module does not match its restated head (relative mismatch {err:.2e})')

    def apply(self, x):
        xs = x[:, self.o0:self.o0 + self.C0]
        if self.kind == 'linear':
            return (xs @ self.w)[:, None]
        h = xs @ self.W1
        return (self.c * h / (1.0 + np.exp(-h)) @ self.w2)[:, None]

    def kname(self, base):
        return f'{base}_{self.kind}_c{self.C0}' + (f'_h{self.H}' if self.kind == 'mlp' else '') + f'_d{self.Din}'

    def bytes(self, n):
        """(forward, backward) algorithmic HBM bytes over n nodes: the scalar block in, the energy out; the scalar
        block and dL/de in, the whole input gradient row out."""
        return n * 4 * (self.C0 + 1), n * 4 * (self.C0 + 1 + self.Din)


def _table(name, vals):
    body = ', '.join(_lit(v) for v in np.asarray(vals, dtype=np.float64).reshape(-1))
    return f'__device__ const float {name}[{np.asarray(vals).size}] = {{{body}}};'


def source(spec):
    """HIP source of ``ro_fwd`` and ``ro_bwd``.  The weights are compile-time tables in device memory (a lane reads
    the entries of its own channels or hidden units; the 16 lanes of a node read 16 neighbouring words)."""
    C0, o0, Din = spec.C0, spec.o0, spec.Din
    per = C0 // LANES                          # scalar channels per lane: u = s + LANES i
    L = [_native.device_header(),
         '__device__ __forceinline__ float ro_sig(float z) { return 1.f / (1.f + expf(-z)); }',
         '// sum over the 16 lanes of a node (xor butterfly inside each 16-lane row)',
         '__device__ __forceinline__ float ro_sum16(float v) {',
         '#pragma unroll',
         '  for (int m = 8; m >= 1; m >>= 1) v += __shfl_xor(v, m, 16);',
         '  return v;',
         '}']
    if spec.kind == 'linear':
        L.append(_table('ro_w', spec.w))
    else:
        H = spec.H
        HP = -(-H // LANES) * LANES                # hidden units padded to a multiple of 16 (zero weights)
        W1 = np.zeros((C0, HP))
        W1[:, :H] = spec.W1
        w2 = np.zeros(HP)
        w2[:H] = spec.w2
        L += [_table('ro_w1', W1), _table('ro_w2', w2)]
    L.append('')
    head = ['  const int t = threadIdx.x, s = t & 15;',
            f'  const long long n = (long long)mh_xcd_block(blockIdx.x, gridDim.x) * {BLOCK // LANES} + (t >> 4);',
            '  const bool live = n < N;',
            '  const long long nc = live ? n : N - 1;            // clamped: every load in bounds',
            f'  const float* __restrict__ xr = x + nc * {Din} + {o0};']
    if spec.kind == 'mlp':
        ks = HP // LANES                        # hidden units per lane: k = s + LANES j
        head += [f'  float h[{ks}];',
                 '#pragma unroll',
                 f'  for (int j = 0; j < {ks}; ++j) h[j] = 0.f;',
                 '#pragma unroll 4',
                 f'  for (int i = 0; i < {C0 // 4}; ++i) {{',
                 '    const float4 v = reinterpret_cast<const float4*>(xr)[i];   // the node\'s 16 lanes: one address',
                 '    const float xv[4] = {v.x, v.y, v.z, v.w};',
                 '#pragma unroll',
                 '    for (int e = 0; e < 4; ++e)',
                 '#pragma unroll',
                 f'      for (int j = 0; j < {ks}; ++j) h[j] += xv[e] * ro_w1[(4 * i + e) * {HP} + s + {LANES} * j];',
                 '  }']
    L += [f'extern "C" __global__ __launch_bounds__({BLOCK}) void {spec.kname("ro_fwd")}(const float* __restrict__ x,',
          '    float* __restrict__ out, long long N) {'] + head
    if spec.kind == 'linear':
        L += ['  float p = 0.f;',
              '#pragma unroll',
              f'  for (int i = 0; i < {per}; ++i) p += xr[s + {LANES} * i] * ro_w[s + {LANES} * i];']
    else:
        L += ['  float p = 0.f;',
              '#pragma unroll',
              f'  for (int j = 0; j < {ks}; ++j) p += ro_w2[s + {LANES} * j] * ({_lit(spec.c)} * h[j] * ro_sig(h[j]));']
    L += ['  p = ro_sum16(p);',
          '  if (live && s == 0) out[n] = p;',
          '}', '']
    # backward: dL/dx for the scalar block, zeros elsewhere
    L += [f'extern "C" __global__ __launch_bounds__({BLOCK}) void {spec.kname("ro_bwd")}(const float* __restrict__ x,',
          '    const float* __restrict__ g, float* __restrict__ gx, long long N) {'] + head
    L += ['  const float gn = g[nc];',
          f'  float* __restrict__ gr = gx + nc * {Din};']
    if spec.kind == 'linear':
        L += ['#pragma unroll',
              f'  for (int i = 0; i < {per}; ++i)',
              f'    if (live) gr[{o0} + s + {LANES} * i] = gn * ro_w[s + {LANES} * i];']
    else:
        # gh_k = g w2_k c silu'(h_k) on the lane owning k, then every lane of the node gathers all of them
        L += [f'  float gh[{ks}];',
              '#pragma unroll',
              f'  for (int j = 0; j < {ks}; ++j) {{',
              '    const float sg = ro_sig(h[j]);',
              f'    gh[j] = gn * ro_w2[s + {LANES} * j] * {_lit(spec.c)} * sg * (1.f + h[j] * (1.f - sg));',
              '  }',
              '#pragma unroll',
              f'  for (int i = 0; i < {per}; ++i) {{',
              f'    const int u = s + {LANES} * i;',
              '    float v = 0.f;',
              '#pragma unroll',
              f'    for (int j = 0; j < {ks}; ++j)',
              '#pragma unroll',
              f'      for (int r = 0; r < {LANES}; ++r)',
              f'        v += __shfl(gh[j], (t & 63 & ~15) + r, 64) * ro_w1[u * {HP} + r + {LANES} * j];',
              f'    if (live) gr[{o0} + u] = v;',
              '  }']
    if Din > C0:                                # zeros in the other blocks of the row
        L += [f'  for (int j = s; j < {Din - C0}; j += {LANES}) {{',
              f'    const int col = j < {o0} ? j : j + {C0};',
              '    if (live) gr[col] = 0.f;',
              '  }']
    L += ['}', '']
    return '\n'.join(L)


def source_second(spec):
    """HIP source of the SiLU head's second-order kernels behind a double backward (one thread per node, plain
    loops, dual numbers): ``ro_jvp`` writes de = (de/dx) v, ``ro_bwd2`` the derivative of the input gradient along v
    for a given dL/de (a Hessian-vector product of g e(x)), zeros outside the scalar block.  The head is
        z_j = sum_k x_k W1[k, j],  e = sum_j w2_j c z_j sigmoid(z_j)."""
    assert spec.kind == 'mlp'
    C0, o0, Din, H = spec.C0, spec.o0, spec.Din, spec.H
    c = _lit(spec.c)
    L = [_native.device_header(), _native.dual_header(), _table('ro_w1', spec.W1), _table('ro_w2', spec.w2), '']
    head = ['  const long long n = (long long)mh_xcd_block(blockIdx.x, gridDim.x) * BLOCK2 + threadIdx.x;',
            '  if (n >= N) return;',
            f'  const float* __restrict__ xr = x + n * {Din} + {o0};',
            f'  const float* __restrict__ vr = v + n * {Din} + {o0};',
            f'  mh_dual z[{H}];',
            f'  for (int j = 0; j < {H}; ++j) z[j] = mh_dual(0.f);',
            f'  for (int k = 0; k < {C0}; ++k) {{',
            '    const mh_dual xk(xr[k], vr[k]);',
            f'    for (int j = 0; j < {H}; ++j) z[j] += xk * ro_w1[k * {H} + j];',
            '  }']
    L += ['#define BLOCK2 256',
          f'extern "C" __global__ __launch_bounds__(BLOCK2) void {spec.kname("ro_jvp")}(const float* __restrict__ x,',
          '    const float* __restrict__ v, float* __restrict__ de, long long N) {'] + head
    L += ['  mh_dual e(0.f);',
          f'  for (int j = 0; j < {H}; ++j) e += ro_w2[j] * ({c} * z[j] * (1.f / (1.f + expf(-z[j]))));',
          '  de[n] = e.d;', '}', '']
    L += [f'extern "C" __global__ __launch_bounds__(BLOCK2) void {spec.kname("ro_bwd2")}(const float* __restrict__ x,',
          '    const float* __restrict__ v, const float* __restrict__ g, float* __restrict__ gx, long long N) {'] + head
    L += ['  const float gn = g[n];',
          f'  mh_dual q[{H}];',
          f'  for (int j = 0; j < {H}; ++j) {{',
          '    const mh_dual sg = 1.f / (1.f + expf(-z[j]));',
          f'    q[j] = gn * ro_w2[j] * {c} * (sg * (1.f + z[j] * (1.f - sg)));',
          '  }',
          f'  float* __restrict__ gr = gx + n * {Din};',
          f'  for (int k = 0; k < {C0}; ++k) {{',
          '    mh_dual a(0.f);',
          f'    for (int j = 0; j < {H}; ++j) a += q[j] * ro_w1[k * {H} + j];',
          f'    gr[{o0} + k] = a.d;',
          '  }',
          f'  for (int k = 0; k < {Din - C0}; ++k) gr[k < {o0} ? k : k + {C0}] = 0.f;',
          '}', '']
    return '\n'.join(L)


_DOUBLE_BACKWARD = ('mace_hip_kernels: double backward (create_graph=True, e.g. training on forces/stress or an '
                    'autograd Hessian) is not enabled for this HIP module; patch with '
                    'patch_model(model, double_backward=True)')


class _ReadoutFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, op):
        s = op.spec
        if x.dtype != torch.float32 or not x.is_cuda:
            raise TypeError('mace_hip_kernels: readout heads expect float32 GPU input')
        if x.shape[-1] != s.Din:
            raise ValueError(f'expected [..., {s.Din}] node features, got {tuple(x.shape)}')
        lead = x.shape[:-1]
        x2 = x.reshape(-1, s.Din).contiguous()
        N = x2.shape[0]
        out = torch.empty(N, 1, device=x.device, dtype=torch.float32)
        _native.launch(f'ro_fwd[{op.tag}]', _native.load().mh_readout_fwd, op.module.handle, _native.ptr(x2),
                       _native.ptr(out), N, _native.stream_of(x2))
        ctx.save_for_backward(x)             # the input itself: a double backward differentiates through it
        ctx.op = op
        return out.reshape(*lead, 1)

    @staticmethod
    def backward(ctx, g):
        x, = ctx.saved_tensors
        op = ctx.op
        if torch.is_grad_enabled():          # only true under create_graph=True
            if not op.double_backward:
                raise RuntimeError(_DOUBLE_BACKWARD)
            if op.spec.kind == 'linear':
                return _ReadoutAdjFn.apply(g, x.detach(), op), None
            return _ReadoutMLPAdjFn.apply(g, x, op), None
        return _readout_bwd(op, x, g), None


def _readout_bwd(op, x, g):
    x2 = x.reshape(-1, op.spec.Din).contiguous()
    g2 = g.reshape(-1).contiguous()
    gx = torch.empty_like(x2)
    _native.launch(f'ro_bwd[{op.tag}]', _native.load().mh_readout_bwd, op.module.handle, _native.ptr(x2),
                   _native.ptr(g2), _native.ptr(gx), x2.shape[0], _native.stream_of(x2))
    return gx.reshape(x.shape)


class _ReadoutAdjFn(torch.autograd.Function):
    """The linear head's input gradient g w^T as a function of g, for a double backward: it does not depend on x,
    and d<ggx, g w^T>/dg = ggx w, the head itself (through _ReadoutFn, so higher orders follow)."""

    @staticmethod
    def forward(ctx, g, x, op):
        ctx.op = op
        return _readout_bwd(op, x, g)

    @staticmethod
    def backward(ctx, ggx):
        return _ReadoutFn.apply(ggx, ctx.op), None, None


class _ReadoutMLPAdjFn(torch.autograd.Function):
    """The SiLU head's input gradient as a function of (g, x), for a double backward: with ggx the incoming
    gradient, d<ggx, dL/dx>/dg = (de/dx) ggx (``ro_jvp``) and d<ggx, dL/dx>/dx the Hessian-vector product
    (``ro_bwd2``).  Third derivatives are not provided."""

    @staticmethod
    def forward(ctx, g, x, op):
        ctx.save_for_backward(g, x)
        ctx.op = op
        return _readout_bwd(op, x, g)

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, ggx):
        g, x = ctx.saved_tensors
        op = ctx.op
        m = op.second_module()
        x2 = x.reshape(-1, op.spec.Din).contiguous()
        v2 = ggx.reshape(-1, op.spec.Din).contiguous()
        N, P, lib = x2.shape[0], _native.ptr, _native.load()
        dg = dx = None
        if ctx.needs_input_grad[0]:
            de = torch.empty(N, device=x2.device, dtype=torch.float32)
            _native.launch(f'ro_jvp[{op.tag}]', lib.mh_readout_jvp, m.handle, P(x2), P(v2), P(de), N,
                           _native.stream_of(x2))
            dg = de.reshape(g.shape)
        if ctx.needs_input_grad[1]:
            g2 = g.reshape(-1).contiguous()
            gx = torch.empty_like(x2)
            _native.launch(f'ro_bwd2[{op.tag}]', lib.mh_readout_bwd2, m.handle, P(x2), P(v2), P(g2), P(gx), N,
                           _native.stream_of(x2))
            dx = gx.reshape(x.shape)
        return dg, dx, None


class HipReadout(torch.nn.Module):
    """Drop-in for a MACE readout head: ``forward(node_feats[..., D], heads=None) -> [..., 1]``."""

    def __init__(self, mod, device=None):
        super().__init__()
        self.spec = ReadoutSpec(mod)
        self.source = source(self.spec)
        code = _native.compile_source(self.source)
        dev = torch.device(device) if device is not None else torch.device('cuda', torch.cuda.current_device())
        with torch.cuda.device(dev):
            self.module = _native.Module(code, {
                _native.MH_READOUT_FWD: (self.spec.kname('ro_fwd'), BLOCK, BLOCK // LANES),
                _native.MH_READOUT_BWD: (self.spec.kname('ro_bwd'), BLOCK, BLOCK // LANES)})
        self.original = [mod]
        self.tag = 'readout'
        # a backward under create_graph=True raises (the reference's behaviour) unless this is set
        self.double_backward = False
        self._device = dev
        self._second = None

    def second_module(self):
        """The SiLU head's second-order kernels (``ro_jvp``, ``ro_bwd2``), compiled on first use; a linear head
        needs none (its double backward is the head itself)."""
        if self.spec.kind == 'linear':
            return None
        if self._second is None:
            code = _native.compile_source(source_second(self.spec))
            with torch.cuda.device(self._device):
                self._second = _native.Module(code, {
                    _native.MH_READOUT_JVP: (self.spec.kname('ro_jvp'), 256, 256),
                    _native.MH_READOUT_BWD2: (self.spec.kname('ro_bwd2'), 256, 256)})
        return self._second

    def forward(self, x, heads=None):
        if isinstance(x, Pending):
            x = x.value()                      # formed here, under autograd, not inside the Function's forward
        return _ReadoutFn.apply(slot(x), self)

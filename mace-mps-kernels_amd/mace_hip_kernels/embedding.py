"""
MACE's radial embedding on MI355X: a drop-in for ``radial_embedding`` (``RadialEmbeddingBlock`` with the Bessel basis
and the polynomial cutoff envelope), which maps the [E, 1] edge lengths r to

    cutoff(r) = (1 - (p+1)(p+2)/2 u^p + p(p+2) u^(p+1) - p(p+1)/2 u^(p+2)) * [r < r_max],   u = r / r_max,
    edge_feats[:, n] = sqrt(2 / r_max) sin(n pi r / r_max) / r * cutoff(r),                  n = 1..n_basis,

and returns (edge_feats, cutoff).  On the GPU the PyTorch module is about a dozen elementwise launches (powers with
a tensor exponent, a comparison, the sines, the products) and its backward as many again; here one thread handles
one edge in each direction, and the backward takes the gradients of both outputs (the cutoff also scales the
convolution weights) back to dL/dr.
"""
import numpy as np
import torch

from . import _native

BLOCK = 256


def _lit(v):
    return f'{float(np.float32(v)).hex()}f'


def emb_supported(mod):
    """(ok, reason) — whether a radial embedding module can be replaced."""
    try:
        b, c = mod.bessel_fn, mod.cutoff_fn
        if type(b).__name__ != 'BesselBasis' or type(c).__name__ != 'PolynomialCutoff':
            return False, f'{type(b).__name__} x {type(c).__name__} (only BesselBasis x PolynomialCutoff)'
        if getattr(mod, 'distance_transform', None) is not None:
            return False, 'distance transform'
        p = float(c.p)
        if p != int(p) or not 1 <= p <= 16:
            return False, f'envelope power {p}'
        if b.bessel_weights.numel() > 32:
            return False, 'more than 32 basis functions'
    except (AttributeError, TypeError) as e:
        return False, f'not a MACE radial embedding ({e})'
    return True, ''


class EmbSpec:
    def __init__(self, mod):
        ok, why = emb_supported(mod)
        if not ok:
            raise ValueError(why)
        b, c = mod.bessel_fn, mod.cutoff_fn
        self.w = [float(v) for v in b.bessel_weights.detach().double().cpu()]
        self.pref = float(b.prefactor)
        self.p = int(float(c.p))
        self.r_max = float(c.r_max)
        self.n = len(self.w)
        # the module itself, in float64, on lengths either side of the cutoff: the restated formulas must match
        r = torch.linspace(0.3, 1.3 * self.r_max, 97, dtype=torch.float64).reshape(-1, 1)
        import copy
        m64 = copy.deepcopy(mod).to('cpu', torch.float64)
        with torch.no_grad():
            f_ref, c_ref = m64(r)
        f, cut = self.apply(r.numpy())
        err = max(np.abs(f - f_ref.numpy()).max(), np.abs(cut - c_ref.numpy()).max())
        if not err < 1e-10:
            raise ValueError(f'the module does not match the Bessel x polynomial-cutoff formulas ({err:.2e})')

    def apply(self, r):
        p = self.p
        u = r / self.r_max
        env = (1.0 - (p + 1.0) * (p + 2.0) / 2.0 * u ** p + p * (p + 2.0) * u ** (p + 1)
               - p * (p + 1.0) / 2.0 * u ** (p + 2))
        cut = env * (r < self.r_max)
        feats = self.pref * np.sin(np.array(self.w) * r) / r * cut
        return feats, cut

    def bytes(self, E):
        return E * 4 * (1 + self.n + 1), E * 4 * (1 + self.n + 1 + 1)

    def kname(self, base):
        return f'{base}_n{self.n}_p{self.p}'


def source(spec):
    p, n = spec.p, spec.n
    c1, c2, c3 = (p + 1.0) * (p + 2.0) / 2.0, p * (p + 2.0), p * (p + 1.0) / 2.0

    def powu(k):
        return ' * '.join(['u'] * k) if k > 0 else '1.f'

    head = ['  const long long e = (long long)mh_xcd_block(blockIdx.x, gridDim.x) * BLOCK + threadIdx.x;',
            '  if (e >= E) return;',
            '  const float x = len[e];',
            f'  const float u = x / {_lit(spec.r_max)};',
            f'  const float up = {powu(p)};',
            f'  const bool in = x < {_lit(spec.r_max)};',
            f'  const float env = 1.f - {_lit(c1)} * up + {_lit(c2)} * (up * u) - {_lit(c3)} * (up * u * u);',
            '  const float cut = in ? env : 0.f;']
    L = [_native.device_header(), f'#define BLOCK {BLOCK}',
         f'extern "C" __global__ __launch_bounds__(BLOCK) void {spec.kname("emb_fwd")}(const float* __restrict__ len,',
         '    float* __restrict__ feats, float* __restrict__ cutoff, long long E) {'] + head
    L += ['  cutoff[e] = cut;']
    for k, w in enumerate(spec.w):
        L.append(f'  feats[e * {n} + {k}] = ({_lit(spec.pref)} * sinf({_lit(w)} * x)) / x * cut;')
    L += ['}', '']
    # backward: d cut/dx = env'(u) / r_max inside the cutoff; d feat_k/dx = b_k' cut + b_k cut'
    L += [f'extern "C" __global__ __launch_bounds__(BLOCK) void {spec.kname("emb_bwd")}(const float* __restrict__ len,',
          '    const float* __restrict__ gfeats, const float* __restrict__ gcut, float* __restrict__ glen, long long E) {']
    L += head
    L += [f'  const float denv = (-{_lit(c1 * p)} * {powu(p - 1)} + {_lit(c2 * (p + 1))} * up'
          f' - {_lit(c3 * (p + 2))} * (up * u)) / {_lit(spec.r_max)};',
          '  const float dcut = in ? denv : 0.f;',
          '  const float ix = 1.f / x;',
          '  float acc = gcut ? gcut[e] * dcut : 0.f;']
    for k, w in enumerate(spec.w):
        L += ['  {',
              f'    const float s = sinf({_lit(w)} * x), c = cosf({_lit(w)} * x);',
              f'    const float b = {_lit(spec.pref)} * s * ix;',
              f'    const float db = {_lit(spec.pref)} * ({_lit(w)} * c - s * ix) * ix;',
              f'    acc += gfeats[e * {n} + {k}] * (db * cut + b * dcut);',
              '  }']
    L += ['  glen[e] = acc;', '}', '']
    return '\n'.join(L)


_DOUBLE_BACKWARD = ('mace_hip_kernels: double backward (create_graph=True, e.g. training on forces/stress or an '
                    'autograd Hessian) is not supported by this HIP module; patch_model(model, '
                    'double_backward=True) leaves it on e3nn')


class _EmbFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, lengths, op):
        if lengths.dtype != torch.float32 or not lengths.is_cuda:
            raise TypeError('mace_hip_kernels: the radial embedding expects float32 GPU input')
        if lengths.shape[-1] != 1:
            raise ValueError(f'edge lengths must be [..., 1], got {tuple(lengths.shape)}')
        lead = lengths.shape[:-1]
        r = lengths.reshape(-1).contiguous()
        E = r.shape[0]
        feats = torch.empty(E, op.spec.n, device=r.device, dtype=torch.float32)
        cut = torch.empty(E, 1, device=r.device, dtype=torch.float32)
        _native.launch(f'emb_fwd[{op.tag}]', _native.load().mh_emb_fwd, op.module.handle, _native.ptr(r),
                       _native.ptr(feats), _native.ptr(cut), E, _native.stream_of(r))
        ctx.save_for_backward(r)
        ctx.op, ctx.lead = op, lead
        return feats.reshape(*lead, op.spec.n), cut.reshape(*lead, 1)

    @staticmethod
    def backward(ctx, gf, gc):
        if torch.is_grad_enabled():
            raise RuntimeError(_DOUBLE_BACKWARD)
        r, = ctx.saved_tensors
        op = ctx.op
        E = r.shape[0]
        gf = torch.zeros(E, op.spec.n, device=r.device) if gf is None else gf.reshape(E, op.spec.n).contiguous()
        gc = None if gc is None else gc.reshape(E).contiguous()
        gr = torch.empty_like(r)
        _native.launch(f'emb_bwd[{op.tag}]', _native.load().mh_emb_bwd, op.module.handle, _native.ptr(r),
                       _native.ptr(gf), _native.ptr(gc), _native.ptr(gr), E, _native.stream_of(r))
        return gr.reshape(*ctx.lead, 1), None


class HipRadialEmbedding(torch.nn.Module):
    """Drop-in for MACE's ``radial_embedding``: ``forward(edge_lengths[..., 1]) -> (edge_feats, cutoff)``."""

    def __init__(self, mod, device=None):
        super().__init__()
        self.spec = EmbSpec(mod)
        self.source = source(self.spec)
        code = _native.compile_source(self.source)
        dev = torch.device(device) if device is not None else torch.device('cuda', torch.cuda.current_device())
        with torch.cuda.device(dev):
            self.module = _native.Module(code, {_native.MH_EMB_FWD: (self.spec.kname('emb_fwd'), BLOCK, BLOCK),
                                                _native.MH_EMB_BWD: (self.spec.kname('emb_bwd'), BLOCK, BLOCK)})
        self.out_dim = self.spec.n
        self.original = [mod]
        self.tag = 'radial_embedding'

    def forward(self, edge_lengths, *args, **kwargs):
        return _EmbFn.apply(edge_lengths, self)


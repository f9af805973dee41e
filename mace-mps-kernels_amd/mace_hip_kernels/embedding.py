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


def math_lines(spec):
    """The per-edge arithmetic as plain C statements of the length ``x``: ``head`` defines the envelope ``cut``,
    ``fwd`` the features ``f0..f{n-1}``, ``bwd`` (reading ``gfeats`` and ``gcut`` at edge ``e``) ``acc`` = dL/dx."""
    p, n = spec.p, spec.n
    c1, c2, c3 = (p + 1.0) * (p + 2.0) / 2.0, p * (p + 2.0), p * (p + 1.0) / 2.0

    def powu(k):
        return ' * '.join(['u'] * k) if k > 0 else '1.f'

    head = [f'const float u = x / {_lit(spec.r_max)};',
            f'const float up = {powu(p)};',
            f'const bool in = x < {_lit(spec.r_max)};',
            f'const float env = 1.f - {_lit(c1)} * up + {_lit(c2)} * (up * u) - {_lit(c3)} * (up * u * u);',
            'const float cut = in ? env : -0.f;']           # -0.0: outside the support (see HipRadialEmbedding)
    fwd = [f'const float f{k} = ({_lit(spec.pref)} * sinf({_lit(w)} * x)) / x * cut;' for k, w in enumerate(spec.w)]
    # d cut/dx = env'(u) / r_max inside the cutoff; d feat_k/dx = b_k' cut + b_k cut'
    bwd = [f'const float denv = (-{_lit(c1 * p)} * {powu(p - 1)} + {_lit(c2 * (p + 1))} * up'
           f' - {_lit(c3 * (p + 2))} * (up * u)) / {_lit(spec.r_max)};',
           'const float dcut = in ? denv : 0.f;',
           'const float ix = 1.f / x;',
           'float acc = gcut ? gcut[e] * dcut : 0.f;']
    for k, w in enumerate(spec.w):
        bwd += ['{',
                f'  const float s = sinf({_lit(w)} * x), c = cosf({_lit(w)} * x);',
                f'  const float b = {_lit(spec.pref)} * s * ix;',
                f'  const float db = {_lit(spec.pref)} * ({_lit(w)} * c - s * ix) * ix;',
                f'  acc += gfeats[e * {n} + {k}] * (db * cut + b * dcut);',
                '}']
    return dict(head=head, fwd=fwd, bwd=bwd)


def source(spec):
    n = spec.n
    m = math_lines(spec)
    ind = lambda lines: ['  ' + l for l in lines]  # noqa: E731
    head = ['  const long long e = (long long)mh_xcd_block(blockIdx.x, gridDim.x) * BLOCK + threadIdx.x;',
            '  if (e >= E) return;',
            '  const float x = len[e];'] + ind(m['head'])
    L = [_native.device_header(), f'#define BLOCK {BLOCK}',
         f'extern "C" __global__ __launch_bounds__(BLOCK) void {spec.kname("emb_fwd")}(const float* __restrict__ len,',
         '    float* __restrict__ feats, float* __restrict__ cutoff, long long E) {'] + head
    L += ['  cutoff[e] = cut;'] + ind(m['fwd']) + [f'  feats[e * {n} + {k}] = f{k};' for k in range(n)] + ['}', '']
    L += [f'extern "C" __global__ __launch_bounds__(BLOCK) void {spec.kname("emb_bwd")}(const float* __restrict__ len,',
          '    const float* __restrict__ gfeats, const float* __restrict__ gcut, float* __restrict__ glen, long long E) {']
    L += head + ind(m['bwd']) + ['  glen[e] = acc;', '}', '']
    return '\n'.join(L)


def source_second(spec):
    """HIP source of the second-order kernels behind a double backward: the statements of ``emb_fwd`` / ``emb_bwd``
    on dual numbers with the lengths carrying a direction dl.  ``emb_jvp`` writes (d feats, d cut) = their
    derivatives times dl; ``emb_bwd2`` writes the derivative of dL/dx along dl for fixed incoming gradients."""
    n = spec.n
    m = math_lines(spec)
    ind = lambda lines: ['  ' + l for l in lines]  # noqa: E731
    head = ['  const long long e = (long long)mh_xcd_block(blockIdx.x, gridDim.x) * BLOCK + threadIdx.x;',
            '  if (e >= E) return;',
            '  const mh_dual x(len[e], dl[e]);'] + ind(_native.dualize(m['head']))
    L = [_native.device_header(), _native.dual_header(), f'#define BLOCK {BLOCK}',
         f'extern "C" __global__ __launch_bounds__(BLOCK) void {spec.kname("emb_jvp")}(const float* __restrict__ len,',
         '    const float* __restrict__ dl, float* __restrict__ dfeats, float* __restrict__ dcutoff, long long E) {']
    L += head + ['  dcutoff[e] = cut.d;'] + ind(_native.dualize(m['fwd']))
    L += [f'  dfeats[e * {n} + {k}] = f{k}.d;' for k in range(n)] + ['}', '']
    L += [f'extern "C" __global__ __launch_bounds__(BLOCK) void {spec.kname("emb_bwd2")}(const float* __restrict__ len,',
          '    const float* __restrict__ dl, const float* __restrict__ gfeats, const float* __restrict__ gcut,',
          '    float* __restrict__ glen, long long E) {']
    L += head + ind(_native.dualize(m['bwd'])) + ['  glen[e] = acc.d;', '}', '']
    return '\n'.join(L)


_DOUBLE_BACKWARD = ('mace_hip_kernels: double backward (create_graph=True, e.g. training on forces/stress or an '
                    'autograd Hessian) is not enabled for this HIP module; patch with '
                    'patch_model(model, double_backward=True)')


def _emb_bwd(op, lengths, gf, gc):
    r = lengths.reshape(-1).contiguous()
    E = r.shape[0]
    gf = torch.zeros(E, op.spec.n, device=r.device) if gf is None else gf.reshape(E, op.spec.n).contiguous()
    gc = None if gc is None else gc.reshape(E).contiguous()
    gr = torch.empty_like(r)
    _native.launch(f'emb_bwd[{op.tag}]', _native.load().mh_emb_bwd, op.module.handle, _native.ptr(r),
                   _native.ptr(gf), _native.ptr(gc), _native.ptr(gr), E, _native.stream_of(r))
    return gr.reshape(lengths.shape)


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
        ctx.save_for_backward(lengths)       # the input itself: a double backward differentiates through it
        ctx.op = op
        return feats.reshape(*lead, op.spec.n), cut.reshape(*lead, 1)

    @staticmethod
    def backward(ctx, gf, gc):
        lengths, = ctx.saved_tensors
        op = ctx.op
        if torch.is_grad_enabled():          # only true under create_graph=True
            if not op.double_backward:
                raise RuntimeError(_DOUBLE_BACKWARD)
            return _EmbAdjFn.apply(gf, gc, lengths, op), None
        return _emb_bwd(op, lengths, gf, gc), None


class _EmbAdjFn(torch.autograd.Function):
    """dL/dx = sum_k gf_k f_k'(x) + gc cut'(x) as a function of (gf, gc, x), for a double backward: with ggx the
    incoming gradient, d<ggx, dL/dx>/d(gf, gc) = (f'(x), cut'(x)) ggx (``emb_jvp``) and d<ggx, dL/dx>/dx =
    (sum_k gf_k f_k''(x) + gc cut''(x)) ggx (``emb_bwd2``).  Third derivatives are not provided."""

    @staticmethod
    def forward(ctx, gf, gc, lengths, op):
        ctx.save_for_backward(gf, gc, lengths)
        ctx.op = op
        return _emb_bwd(op, lengths, gf, gc)

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, ggx):
        gf, gc, lengths = ctx.saved_tensors
        op = ctx.op
        m = op.second_module()
        r = lengths.reshape(-1).contiguous()
        dl = ggx.reshape(-1).contiguous()
        E, n, P, lib = r.shape[0], op.spec.n, _native.ptr, _native.load()
        d_gf = d_gc = d_x = None
        if ctx.needs_input_grad[0] or ctx.needs_input_grad[1]:
            df = torch.empty(E, n, device=r.device, dtype=torch.float32)
            dc = torch.empty(E, device=r.device, dtype=torch.float32)
            _native.launch(f'emb_jvp[{op.tag}]', lib.mh_emb_jvp, m.handle, P(r), P(dl), P(df), P(dc), E,
                           _native.stream_of(r))
            d_gf = df.reshape(gf.shape) if ctx.needs_input_grad[0] else None
            d_gc = dc.reshape(gc.shape) if ctx.needs_input_grad[1] else None
        if ctx.needs_input_grad[2]:
            gf2 = torch.zeros(E, n, device=r.device) if gf is None else gf.reshape(E, n).contiguous()
            gc2 = None if gc is None else gc.reshape(E).contiguous()
            gx = torch.empty_like(r)
            _native.launch(f'emb_bwd2[{op.tag}]', lib.mh_emb_bwd2, m.handle, P(r), P(dl), P(gf2), P(gc2), P(gx), E,
                           _native.stream_of(r))
            d_x = gx.reshape(lengths.shape)
        return d_gf, d_gc, d_x, None


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
        self._device = dev
        # a backward under create_graph=True raises (the reference's behaviour) unless this is set; then the
        # gradient is differentiable once more through the second-order kernels (second_module)
        self.double_backward = False
        self._second = None

    def second_module(self):
        """The module of the second-order kernels (``emb_jvp``, ``emb_bwd2``), compiled on first use."""
        if self._second is None:
            code = _native.compile_source(source_second(self.spec))
            with torch.cuda.device(self._device):
                self._second = _native.Module(code, {
                    _native.MH_EMB_JVP: (self.spec.kname('emb_jvp'), BLOCK, BLOCK),
                    _native.MH_EMB_BWD2: (self.spec.kname('emb_bwd2'), BLOCK, BLOCK)})
        return self._second

    def forward(self, edge_lengths, *args, **kwargs):
        from . import edgefeat
        made = edgefeat.take_embedding(self, edge_lengths)     # made in the geometry's pass (edgefeat), if it was
        feats, cut = made if made is not None else _EmbFn.apply(edge_lengths, self)
        # The cutoff is -0.0 exactly where r >= r_max (outside the envelope's support, where its derivative is zero)
        # and nonzero or +0.0 elsewhere; a patched convolution that receives this tensor unmodified (same version)
        # skips such edges in its backward (MH_CUT_MASKED).
        cut._mh_support_mask = cut._version
        from .geometry import lengths_pair_symmetric
        vec = lengths_pair_symmetric(edge_lengths)
        if vec is not None:
            # each feature row is the same function of its edge's length alone
            feats._mh_vec = (feats._version, vec, vec._version)
        return feats, cut


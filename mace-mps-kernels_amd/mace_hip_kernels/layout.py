"""
MACE's ``reshape_irreps`` on MI355X: the per-node permutation from e3nn's irreps layout [N, sum_l mul (2l+1)]
(channel-major inside each irrep block: index off_l + u (2l+1) + m) to the symmetric contraction's layout
[N, mul, sum_l (2l+1)] (index u * D + o_l + m, D = sum_l (2l+1)).  In PyTorch it is a slice, a reshape and a
concatenation per block, and its backward a zero-filled full-size tensor per slice; here each direction is one
kernel: a workgroup copies four node rows into LDS (coalesced), then writes the permuted rows (coalesced), the
gather happening in LDS; the backward applies the inverse permutation the same way.
"""
import torch

from . import _native
from .pending import Pending

BLOCK = 256
NODES = 4            # nodes per workgroup


def reshape_supported(mod):
    try:
        muls = {mul for mul, _ in mod.irreps}
        if len(muls) != 1:
            return False, 'blocks of different multiplicities'
        if muls.pop() % 4:
            return False, 'multiplicity not a multiple of 4'
    except (AttributeError, TypeError) as e:
        return False, f'not a reshape_irreps module ({e})'
    return True, ''


class ReshapeSpec:
    def __init__(self, mod):
        ok, why = reshape_supported(mod)
        if not ok:
            raise ValueError(why)
        self.blocks = [(mul, ir.l) for mul, ir in mod.irreps]
        self.mul = self.blocks[0][0]
        self.D = sum(2 * l + 1 for _, l in self.blocks)
        self.dim = self.mul * self.D

    def kname(self, base):
        return f'{base}_m{self.mul}_d{self.D}'

    def perm(self):
        """src[j]: the irreps-layout index that output index j (= u D + o_l + m) reads."""
        src, o = [0] * self.dim, 0
        off = 0
        for mul, l in self.blocks:
            d = 2 * l + 1
            for u in range(mul):
                for m in range(d):
                    src[u * self.D + o + m] = off + u * d + m
            off += mul * d
            o += d
        return src


def source(spec):
    """Each workgroup moves NODES whole rows: a coalesced copy of the rows into LDS, then a coalesced write of the
    permuted rows (the gather happens in LDS)."""
    conds, off, o = [], 0, 0
    for mul, l in spec.blocks:
        d = 2 * l + 1
        conds.append((o + d, off, d, o))
        off += mul * d
        o += d

    def src_of(ind):
        # forward: SC-layout index j (u = j / D, column c inside the block of dimension d) reads irreps index s
        L = [f'{ind}const int u = j / {spec.D}, c = j - u * {spec.D};', f'{ind}int s = 0;']
        for k, (end, boff, d, o0) in enumerate(conds):
            kw = 'if' if k == 0 else '} else if'
            L.append(f'{ind}{kw} (c < {end}) {{ s = {boff} + u * {d} + (c - {o0});')
        L.append(f'{ind}}}')
        return L

    def inv_of(ind):
        # backward: irreps index j (block at offset boff, dimension d: u = (j - boff) / d) reads SC index s
        L = [f'{ind}int s = 0;']
        for k, (end, boff, d, o0) in enumerate(conds):
            kw = 'if' if k == 0 else '} else if'
            bend = boff + spec.mul * d
            L.append(f'{ind}{kw} (j < {bend}) {{ const int u = (j - {boff}) / {d}; '
                     f's = u * {spec.D} + {o0} + (j - {boff} - u * {d});')
        L.append(f'{ind}}}')
        return L

    n4 = NODES * spec.dim // 4                       # float4s per workgroup
    it = -(-n4 // BLOCK)
    L = [_native.device_header(), f'#define BLOCK {BLOCK}']
    for name, fwd in ((spec.kname('perm_fwd'), True), (spec.kname('perm_bwd'), False)):
        L += [f'extern "C" __global__ __launch_bounds__(BLOCK) void {name}(const float* __restrict__ x,',
              '    float* __restrict__ y, int N) {',
              f'  __shared__ __align__(16) float rows[{NODES * spec.dim}];',
              f'  const int n0 = mh_xcd_block(blockIdx.x, gridDim.x) * {NODES};',
              f'  const int nn = min({NODES}, N - n0), m4 = nn * {spec.dim // 4};',
              f'  const size_t base = (size_t)n0 * {spec.dim};',
              '  const float4* __restrict__ xs = reinterpret_cast<const float4*>(x + base);',
              '  float4* __restrict__ ys = reinterpret_cast<float4*>(y + base);',
              '  float4 v[%d];' % it,
              '#pragma unroll',
              f'  for (int i = 0; i < {it}; ++i) {{ const int f = threadIdx.x + i * BLOCK; v[i] = xs[min(f, m4 - 1)]; }}',
              '#pragma unroll',
              f'  for (int i = 0; i < {it}; ++i) {{ const int f = threadIdx.x + i * BLOCK;',
              '    if (f < m4) reinterpret_cast<float4*>(rows)[f] = v[i]; }',
              '  __syncthreads();',
              '  for (int g = threadIdx.x; g < m4; g += BLOCK) {',
              f'    const int nl = g / {spec.dim // 4}, j0 = 4 * (g - nl * {spec.dim // 4});',
              '    float o[4];',
              '#pragma unroll',
              '    for (int e = 0; e < 4; ++e) {',
              '      const int j = j0 + e;']
        L += src_of('      ') if fwd else inv_of('      ')
        L += [f'      o[e] = rows[nl * {spec.dim} + s];',
              '    }',
              '    ys[g] = make_float4(o[0], o[1], o[2], o[3]);',
              '  }', '}', '']
    return '\n'.join(L)


class _PermFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, op):
        s = op.spec
        if x.dtype != torch.float32 or not x.is_cuda:
            raise TypeError('mace_hip_kernels: reshape_irreps expects float32 GPU input')
        if x.dim() != 2 or x.shape[1] != s.dim:
            raise ValueError(f'expected [N, {s.dim}], got {tuple(x.shape)}')
        x = x.contiguous()
        N = x.shape[0]
        y = torch.empty(N, s.mul, s.D, device=x.device, dtype=torch.float32)
        _native.launch(f'perm_fwd[{op.tag}]', _native.load().mh_perm_fwd, op.module.handle, _native.ptr(x),
                       _native.ptr(y), N, _native.stream_of(x))
        ctx.op = op
        return y

    @staticmethod
    def backward(ctx, g):
        op = ctx.op
        if torch.is_grad_enabled():          # only true under create_graph=True
            if not op.double_backward:
                raise RuntimeError('mace_hip_kernels: double backward (create_graph=True) is not enabled for this '
                                   'HIP module; patch with patch_model(model, double_backward=True)')
            return _PermAdjFn.apply(g, op), None
        return _perm_bwd(op, g), None


def _perm_bwd(op, g):
    g = g.contiguous()
    gx = torch.empty(g.shape[0], op.spec.dim, device=g.device, dtype=torch.float32)
    _native.launch(f'perm_bwd[{op.tag}]', _native.load().mh_perm_bwd, op.module.handle, _native.ptr(g),
                   _native.ptr(gx), g.shape[0], _native.stream_of(g))
    return gx


class _PermAdjFn(torch.autograd.Function):
    """The inverse permutation as a differentiable function of g (a double backward): its gradient is the forward
    permutation."""

    @staticmethod
    def forward(ctx, g, op):
        ctx.op = op
        return _perm_bwd(op, g)

    @staticmethod
    def backward(ctx, ggx):
        return _PermFn.apply(ggx, ctx.op), None


class HipReshapeIrreps(torch.nn.Module):
    """Drop-in for MACE's ``reshape_irreps``: ``forward(x[N, sum mul (2l+1)]) -> [N, mul, sum (2l+1)]``."""

    def __init__(self, mod, device=None):
        super().__init__()
        self.spec = ReshapeSpec(mod)
        self.source = source(self.spec)
        code = _native.compile_source(self.source)
        dev = torch.device(device) if device is not None else torch.device('cuda', torch.cuda.current_device())
        with torch.cuda.device(dev):
            self.module = _native.Module(code, {_native.MH_PERM_FWD: (self.spec.kname('perm_fwd'), BLOCK, NODES),
                                                _native.MH_PERM_BWD: (self.spec.kname('perm_bwd'), BLOCK, NODES)})
        self.irreps = mod.irreps
        self.original = [mod]
        self.tag = 'reshape'
        # a backward under create_graph=True raises (the reference's behaviour) unless this is set; the map is
        # linear, so its double backward is the forward map again
        self.double_backward = False
        # set by patch_model when the only consumer is a patched symmetric contraction, which can read the irreps
        # layout itself: forward then returns a PendingReshape
        self.fuse = False

    def forward(self, x):
        if self.fuse and torch.is_tensor(x) and x.dim() == 2 and x.dtype == torch.float32:
            return PendingReshape(x, self)
        return _PermFn.apply(x, self)


class PendingReshape(Pending):
    """MACE's reshape_irreps of x ([N, mul, sum (2l+1)]), not yet formed.  A patched symmetric contraction asks for
    the irreps-layout source (``irreps_source``) and reads it in place, so the permutation never runs in either
    direction; any other use forms the reshaped tensor first (the permutation kernel)."""

    @staticmethod
    def __new__(cls, x, op):
        return Pending.__new__(cls, (x.shape[0], op.spec.mul, op.spec.D), x)

    def __init__(self, x, op):
        self.src, self.op = x, op

    def irreps_source(self, dims):
        """The irreps-layout tensor if its blocks have the component dimensions ``dims``, else None."""
        return self.src if [2 * l + 1 for _, l in self.op.spec.blocks] == list(dims) else None

    def value(self):
        return _PermFn.apply(self.src, self.op)

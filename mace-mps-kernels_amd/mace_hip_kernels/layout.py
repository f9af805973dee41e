"""
MACE's ``reshape_irreps`` on MI355X: the per-node permutation from e3nn's irreps layout [N, sum_l mul (2l+1)]
(channel-major inside each irrep block: index off_l + u (2l+1) + m) to the symmetric contraction's layout
[N, mul, sum_l (2l+1)] (index u * D + o_l + m, D = sum_l (2l+1)).  In PyTorch it is a slice, a reshape and a
concatenation per block, and its backward a zero-filled full-size tensor per slice; here each direction is one
kernel: every thread moves one element of a node's row (coalesced on the written side, a gather inside the same
row on the read side), and the backward applies the inverse permutation.
"""
import torch

from . import _native

BLOCK = 256
NODES = 4            # nodes per workgroup


def reshape_supported(mod):
    try:
        muls = {mul for mul, _ in mod.irreps}
        if len(muls) != 1:
            return False, 'blocks of different multiplicities'
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
    # src(j): u = j / D, c = j % D; the block holding column c gives (offset, dimension, column start)
    conds, off, o = [], 0, 0
    for mul, l in spec.blocks:
        d = 2 * l + 1
        conds.append((o + d, off, d, o))
        off += mul * d
        o += d
    sel = []
    for k, (end, boff, d, o0) in enumerate(conds):
        kw = 'if' if k == 0 else '} else if'
        sel.append(f'  {kw} (c < {end}) {{ s = {boff} + u * {d} + (c - {o0}); ')
    sel.append('  }')
    body = ['  const int u = j / {D}, c = j - u * {D};'.format(D=spec.D), '  int s = 0;'] + sel
    L = [_native.device_header(), f'#define BLOCK {BLOCK}']
    for name, rd, wr in ((spec.kname('perm_fwd'), 'x[base + s]', 'y[base + j]'),
                         (spec.kname('perm_bwd'), 'x[base + j]', 'y[base + s]')):
        L += [f'extern "C" __global__ __launch_bounds__(BLOCK) void {name}(const float* __restrict__ x,',
              '    float* __restrict__ y, int N) {',
              f'  const int n0 = mh_xcd_block(blockIdx.x, gridDim.x) * {NODES};',
              f'  for (int f = threadIdx.x; f < {NODES * spec.dim}; f += BLOCK) {{',
              f'    const int nl = f / {spec.dim}, j = f - nl * {spec.dim};',
              '    if (n0 + nl >= N) break;',
              f'    const size_t base = (size_t)(n0 + nl) * {spec.dim};']
        L += ['  ' + b for b in body]
        L += [f'    {wr} = {rd};', '  }', '}', '']
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
        if torch.is_grad_enabled():
            raise RuntimeError('mace_hip_kernels: double backward (create_graph=True) is not supported by the HIP '
                               'kernels; use the unpatched e3nn model for that')
        op = ctx.op
        g = g.contiguous()
        gx = torch.empty(g.shape[0], op.spec.dim, device=g.device, dtype=torch.float32)
        _native.launch(f'perm_bwd[{op.tag}]', _native.load().mh_perm_bwd, op.module.handle, _native.ptr(g),
                       _native.ptr(gx), g.shape[0], _native.stream_of(g))
        return gx, None


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

    def forward(self, x):
        return _PermFn.apply(x, self)

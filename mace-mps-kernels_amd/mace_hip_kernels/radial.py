"""
The radial MLP of MACE's interaction blocks on MI355X: a drop-in for ``conv_tp_weights``, e3nn's
``FullyConnectedNet([n_basis] + radial_MLP + [weight_numel], silu)``, which maps the [E, n_basis] edge features to the
[E, weight_numel] per-edge weights of the convolution.

On the GPU the e3nn module is a chain of GEMMs and elementwise launches (a matmul, the normalised SiLU and its
rescale per layer) whose backward adds as many again, every intermediate an [E, 64] tensor, and whose last GEMM
(64 -> weight_numel, e.g. 1280) is most of the arithmetic.  Here each direction is ONE kernel on the fp32 matrix
cores (v_mfma_f32_16x16x4f32):

* a wave owns 16 edges and computes every layer for them with the transposed product out^T = W^T h^T, so that an
  MFMA result tile leaves lane (edge j = lane % 16, q = lane / 16) holding features 16 t + 4 q + r (r = 0..3) of
  its edge — which is exactly the operand layout the next layer's MFMA needs if that layer walks its K index in the
  order k = 16 t + 4 q + r.  Hidden activations never leave registers;
* the hidden layers' weights sit in LDS for the whole workgroup (4 waves, 64 edges); the last layer's weights are
  streamed through LDS 64 output columns at a time, the next chunk loaded into registers while the current one is
  multiplied, and each result tile is stored as one float4 per lane (16 consecutive bytes of an edge's row);
* the backward recomputes the hidden layers from the edge features (cheaper than storing [E, 64] activations),
  forms dL/dh = dL/dW0 W_last^T over the streamed weight chunks, and walks back through the SiLUs to dL/d(edge
  features).

Weights are read from the module when it is patched and checked against it in float64; there are no weight
gradients (inference, like the other drop-ins).
"""
import math

import numpy as np
import torch

from . import _native
from . import conv as _conv

BLOCK = 256          # 4 waves x 16 edges
EDGES = 64           # edges per workgroup
CHUNKS = (64, 32, 16)  # output columns of the last layer staged per LDS round (the largest that divides the width)
PAD = 4              # LDS row padding (floats): the 4 lane groups of a fragment land on different banks


def _layers(mod):
    return [m for m in mod.children()]


def mlp_supported(mod):
    """(ok, reason) — whether a FullyConnectedNet can be replaced."""
    try:
        layers = _layers(mod)
        if len(layers) < 2:
            return False, 'needs at least one hidden layer'
        hs = [layers[0].weight.shape[0]] + [l.weight.shape[1] for l in layers]
        if hs[0] > 64:
            return False, f'{hs[0]} input features (> 64)'
        if any(h % 16 or h > 128 for h in hs[1:-1]):
            return False, 'hidden widths must be multiples of 16 (<= 128)'
        if hs[-1] % 16:
            return False, f'output width {hs[-1]} is not a multiple of 16'
        for l in layers[:-1]:
            act = getattr(l, 'act', None)
            if act is None or getattr(act, 'f', None) is not torch.nn.functional.silu:
                return False, 'hidden activations must be (normalised) SiLU'
        if getattr(layers[-1], 'act', None) is not None:
            return False, 'activation on the output layer'
    except (AttributeError, TypeError, IndexError) as e:
        return False, f'not an e3nn FullyConnectedNet ({e})'
    return True, ''


class MLPSpec:
    """Layer widths and the effective float64 weights: hidden layer i is h <- c_i * silu(h @ A_i), the output layer
    out = h @ A_last (every normalisation constant folded into A and c)."""

    def __init__(self, mod):
        ok, why = mlp_supported(mod)
        if not ok:
            raise ValueError(why)
        layers = _layers(mod)
        self.hs = [layers[0].weight.shape[0]] + [l.weight.shape[1] for l in layers]
        self.A, self.c = [], []
        for l in layers:
            w = l.weight.detach().double().cpu().numpy()
            if l.act is not None:
                self.A.append(w / math.sqrt(l.h_in * l.var_in))
                cst = float(getattr(l.act, 'cst', 1.0)) if not getattr(l.act, '_is_id', False) else 1.0
                self.c.append(cst * math.sqrt(l.var_out))
            else:
                self.A.append(w / math.sqrt(l.h_in * l.var_in / l.var_out))
        rng = np.random.default_rng(0)
        x = rng.normal(size=(9, self.hs[0]))
        m64 = _float64_copy(mod)
        with torch.no_grad():
            ref = m64(torch.tensor(x)).numpy()
        got = self.apply(x)
        err = np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-300)
        if not err < 1e-10:
            raise ValueError(f'the module does not match its restated layers (relative mismatch {err:.2e})')

    def apply(self, x):
        h = x
        for A, c in zip(self.A[:-1], self.c):
            z = h @ A
            h = c * z / (1.0 + np.exp(-z))
        return h @ self.A[-1]

    def kname(self, base):
        """Kernel symbol of this network (layer widths in the name, so profiles tell the blocks apart)."""
        return f'{base}_' + 'x'.join(str(h) for h in self.hs)

    def flops(self, E):
        return 2 * E * sum(a * b for a, b in zip(self.hs, self.hs[1:]))

    def bytes(self, E):
        """(forward, backward) algorithmic HBM bytes over E edges: features in + weights out; features and dL/dW0
        in + dL/dfeatures out."""
        return E * 4 * (self.hs[0] + self.hs[-1]), E * 4 * (2 * self.hs[0] + self.hs[-1])


def _float64_copy(mod):
    import copy
    return copy.deepcopy(mod).to('cpu', torch.float64)


def _lit(v):
    return f'{float(np.float32(v)).hex()}f'


def _layout(spec):
    """Packing constants shared by the generator and the weight packer."""
    hs = spec.hs
    H0, NW, HL = hs[0], hs[-1], hs[-2]
    K0S = -(-H0 // 4)                                    # MFMA steps of the first layer (K = H0 padded to 4 K0S)
    rows = [4 * K0S] + hs[1:-2]                          # K extent of each hidden layer
    cols = hs[1:-1]                                      # outputs of each hidden layer
    CHUNK = next(c for c in CHUNKS if NW % c == 0)
    nat, tr, o1, o2 = [], [], 0, 0
    for r, c in zip(rows, cols):
        nat.append(o1)
        o1 += r * (c + PAD)                              # natural [k][j + PAD]   (backward)
        tr.append(o2)
        o2 += c * (r + PAD)                              # transposed [j][k + PAD] (forward)
    return dict(H0=H0, NW=NW, HL=HL, K0S=K0S, rows=rows, cols=cols, CHUNK=CHUNK, nat=nat, tr=tr, nat_size=o1,
                tr_size=o2, chunk_fwd=CHUNK * (HL + PAD), chunk_bwd=HL * (CHUNK + PAD))


def source(spec):
    """HIP source of ``mlp_fwd`` and ``mlp_bwd``."""
    Lo = _layout(spec)
    H0, NW, HL, K0S, CHUNK = Lo['H0'], Lo['NW'], Lo['HL'], Lo['K0S'], Lo['CHUNK']
    rows, cols = Lo['rows'], Lo['cols']
    nh = len(cols)
    TL = HL // 16
    NCHK = NW // CHUNK
    NO = CHUNK // 16
    lds_fwd = max(Lo['tr_size'], 2 * Lo['chunk_fwd'])
    lds_bwd = max(Lo['nat_size'], 2 * Lo['chunk_bwd'])
    L = [_native.device_header(), 'typedef float mh_f4 __attribute__((ext_vector_type(4)));', '',
         '__device__ __forceinline__ float mlp_sig(float z) { return 1.f / (1.f + expf(-z)); }', '']

    def head(name, args, lds):
        return [f'extern "C" __global__ __launch_bounds__({BLOCK}) void {name}({args}) {{',
                f'  __shared__ __align__(16) float lds[{lds}];',
                '  const int t = threadIdx.x, wave = t >> 6, lane = t & 63, q = lane >> 4, c16 = lane & 15;',
                f'  const long long e0 = (long long)mh_xcd_block(blockIdx.x, gridDim.x) * {EDGES} + wave * 16;',
                '  const long long ej = e0 + c16;                 // this lane\'s edge (as a B column / output row)',
                '  const bool live = ej < E;',
                '  const long long ejc = live ? ej : E - 1;       // clamped: every load in bounds']

    def stage(src, n):
        return [f'  for (int f = t; f < {n // 4}; f += {BLOCK})',
                f'    reinterpret_cast<mh_f4*>(lds)[f] = reinterpret_cast<const mh_f4*>({src})[f];']

    def xin():
        P = [f'  float xin[{K0S}];']
        P += [f'  xin[{st}] = {4 * st} + q < {H0} ? ef[ejc * {H0} + {4 * st} + q] : 0.f;' for st in range(K0S)]
        return P

    def hidden_fwd(transposed, keep):
        """z_i and h_i = c_i silu(z_i) for every hidden layer, A operands from LDS (transposed layout: one b128 read
        per 4 MFMAs; natural layout: b32 reads)."""
        P = []
        for i in range(nh):
            T = cols[i] // 16
            z = f'z{i}'
            P.append(f'  mh_f4 {z}[{T}];')
            for o in range(T):
                P.append(f'  {z}[{o}] = mh_f4{{0.f, 0.f, 0.f, 0.f}};')
            if i == 0:
                for st in range(K0S):
                    for o in range(T):
                        a = (f'lds[{Lo["tr"][0]} + ({16 * o} + c16) * {rows[0] + PAD} + {4 * st} + q]' if transposed else
                             f'lds[{Lo["nat"][0]} + ({4 * st} + q) * {cols[0] + PAD} + {16 * o} + c16]')
                        P.append(f'  {z}[{o}] = __builtin_amdgcn_mfma_f32_16x16x4f32({a}, xin[{st}], {z}[{o}], 0, 0, 0);')
            else:
                Tin = cols[i - 1] // 16
                for ti in range(Tin):
                    if transposed:
                        for o in range(T):
                            P.append(f'  const mh_f4 a{i}_{ti}_{o} = *reinterpret_cast<const mh_f4*>(&lds[{Lo["tr"][i]} + '
                                     f'({16 * o} + c16) * {rows[i] + PAD} + {16 * ti} + 4 * q]);')
                    for r in range(4):
                        for o in range(T):
                            a = (f'a{i}_{ti}_{o}[{r}]' if transposed else
                                 f'lds[{Lo["nat"][i]} + ({16 * ti + r} + 4 * q) * {cols[i] + PAD} + {16 * o} + c16]')
                            P.append(f'  {z}[{o}] = __builtin_amdgcn_mfma_f32_16x16x4f32({a}, h{i - 1}[{ti}][{r}], '
                                     f'{z}[{o}], 0, 0, 0);')
            if i < nh - 1 or keep:
                P.append(f'  mh_f4 h{i}[{T}];')
                for o in range(T):
                    for r in range(4):
                        P.append(f'  h{i}[{o}][{r}] = {_lit(spec.c[i])} * {z}[{o}][{r}] * mlp_sig({z}[{o}][{r}]);')
        return P

    def pre_load(src, nx, stride, width, ind):
        """This thread's share of an output-layer chunk, as float4 registers pre0..: chunk element f4 index f covers
        row f / (width / 4) and 4 columns (global row stride ``stride``)."""
        n4 = (CHUNK * HL) // 4
        P = []
        for it in range(-(-n4 // BLOCK)):
            fx = f't + {it * BLOCK}' if (it + 1) * BLOCK <= n4 else f'min(t + {it * BLOCK}, {n4 - 1})'
            P += [f'{ind}{{ const int f = {fx}, rr = f / {width // 4}, c4 = f - rr * {width // 4};',
                  f'{ind}  pre{it} = *reinterpret_cast<const mh_f4*>({src} + (size_t)rr * {stride} + {nx} + 4 * c4); }}']
        return P

    def pre_store(base, width, ind):
        n4 = (CHUNK * HL) // 4
        P = []
        for it in range(-(-n4 // BLOCK)):
            guard = '' if (it + 1) * BLOCK <= n4 else f'if (t + {it * BLOCK} < {n4}) '
            P += [f'{ind}{guard}{{ const int f = t + {it * BLOCK}, rr = f / {width // 4}, c4 = f - rr * {width // 4};',
                  f'{ind}  *reinterpret_cast<mh_f4*>(&lds[{base} + rr * {width + PAD} + 4 * c4]) = pre{it}; }}']
        return P

    npre = -(-(CHUNK * HL // 4) // BLOCK)
    pres = ', '.join(f'pre{i}' for i in range(npre))

    # ------------------------------------------------------------------ forward
    # hidden weights transposed [j][k + PAD]; output layer from WlT [NW][HL], chunks [CHUNK cols][HL + PAD]
    F = head(spec.kname('mlp_fwd'), 'const float* __restrict__ ef, const float* __restrict__ Wh, const float* __restrict__ Wl, '
             'float* __restrict__ W0, long long E', lds_fwd)
    F += stage('Wh', Lo['tr_size']) + ['  __syncthreads();'] + xin() + hidden_fwd(True, True)
    hl = f'h{nh - 1}'
    F += [f'  mh_f4 {pres};'] + pre_load('Wl', '0', HL, HL, '  ')
    F += ['  __syncthreads();                                // every wave is done with the hidden weights']
    F += pre_store('0', HL, '  ') + ['  __syncthreads();']
    F += [f'  for (int ch = 0; ch < {NCHK}; ++ch) {{',
          f'    const int base = (ch & 1) * {Lo["chunk_fwd"]}, nbase = {Lo["chunk_fwd"]} - base;',
          f'    const int nx = min(ch + 1, {NCHK - 1}) * {CHUNK * HL};      // next chunk (the last one reloads itself)']
    F += pre_load('Wl', 'nx', HL, HL, '    ')
    F += [f'    mh_f4 acc[{NO}];']
    F += [f'    acc[{o}] = mh_f4{{0.f, 0.f, 0.f, 0.f}};' for o in range(NO)]
    for ti in range(TL):
        for o in range(NO):
            F.append(f'    const mh_f4 a{ti}_{o} = *reinterpret_cast<const mh_f4*>(&lds[base + ({16 * o} + c16) * '
                     f'{HL + PAD} + {16 * ti} + 4 * q]);')
        for r in range(4):
            for o in range(NO):
                F.append(f'    acc[{o}] = __builtin_amdgcn_mfma_f32_16x16x4f32(a{ti}_{o}[{r}], {hl}[{ti}][{r}], acc[{o}], '
                         '0, 0, 0);')
    F.append('    if (live) {')
    F += [f'      *reinterpret_cast<mh_f4*>(W0 + ej * {NW} + ch * {CHUNK} + {16 * o} + 4 * q) = acc[{o}];'
          for o in range(NO)]
    F += ['    }']
    F += pre_store('nbase', HL, '    ') + ['    __syncthreads();', '  }', '}', '']
    L += F

    # ------------------------------------------------------------------ backward
    # dL/dh_last = gW Wl^T first (chunks of Wl [HL][NW] as [HL][CHUNK + PAD]; gW one float4 per lane per 16 columns,
    # K order k = 16 t + 4 q + r), then the hidden layers recomputed from the natural-layout weights and walked back
    B = head(spec.kname('mlp_bwd'), 'const float* __restrict__ ef, const float* __restrict__ Wh, const float* __restrict__ Wl, '
             'const float* __restrict__ gW, float* __restrict__ gef, long long E', lds_bwd)
    B += [f'  mh_f4 dh[{TL}];'] + [f'  dh[{o}] = mh_f4{{0.f, 0.f, 0.f, 0.f}};' for o in range(TL)]
    B += [f'  mh_f4 {pres};'] + pre_load('Wl', '0', NW, CHUNK, '  ')
    B += [f'  mh_f4 g{ti} = *reinterpret_cast<const mh_f4*>(gW + ejc * {NW} + {16 * ti} + 4 * q);' for ti in range(NO)]
    B += pre_store('0', CHUNK, '  ') + ['  __syncthreads();']
    B += [f'  for (int ch = 0; ch < {NCHK}; ++ch) {{',
          f'    const int base = (ch & 1) * {Lo["chunk_bwd"]}, nbase = {Lo["chunk_bwd"]} - base;',
          f'    const int nx = min(ch + 1, {NCHK - 1}) * {CHUNK};']
    B += pre_load('Wl', 'nx', NW, CHUNK, '    ')
    B += [f'    const mh_f4 gn{ti} = *reinterpret_cast<const mh_f4*>(gW + ejc * {NW} + nx + {16 * ti} + 4 * q);'
          for ti in range(NO)]
    for ti in range(NO):
        for o in range(TL):
            B.append(f'    const mh_f4 a{ti}_{o} = *reinterpret_cast<const mh_f4*>(&lds[base + ({16 * o} + c16) * '
                     f'{CHUNK + PAD} + {16 * ti} + 4 * q]);')
        for r in range(4):
            for o in range(TL):
                B.append(f'    dh[{o}] = __builtin_amdgcn_mfma_f32_16x16x4f32(a{ti}_{o}[{r}], g{ti}[{r}], dh[{o}], 0, 0, 0);')
    B += [f'    g{ti} = gn{ti};' for ti in range(NO)]
    B += pre_store('nbase', CHUNK, '    ') + ['    __syncthreads();', '  }']
    B += stage('Wh', Lo['nat_size']) + ['  __syncthreads();'] + xin() + hidden_fwd(False, False)
    cur = 'dh'
    for i in range(nh - 1, -1, -1):
        T = cols[i] // 16
        for o in range(T):
            for r in range(4):
                B += ['  {',
                      f'    const float z = z{i}[{o}][{r}], s = mlp_sig(z);',
                      f'    {cur}[{o}][{r}] *= {_lit(spec.c[i])} * s * (1.f + z * (1.f - s));',
                      '  }']
        if i > 0:
            Tp = cols[i - 1] // 16
            nxt = f'dh{i - 1}'
            # row j of layer i's natural weights = its input feature j: A[j][k] = W_i[j][k], one b128 per 4 steps
            B.append(f'  mh_f4 {nxt}[{Tp}];')
            B += [f'  {nxt}[{o}] = mh_f4{{0.f, 0.f, 0.f, 0.f}};' for o in range(Tp)]
            for ti in range(T):
                for o in range(Tp):
                    B.append(f'  const mh_f4 b{i}_{ti}_{o} = *reinterpret_cast<const mh_f4*>(&lds[{Lo["nat"][i]} + '
                             f'({16 * o} + c16) * {cols[i] + PAD} + {16 * ti} + 4 * q]);')
                for r in range(4):
                    for o in range(Tp):
                        B.append(f'  {nxt}[{o}] = __builtin_amdgcn_mfma_f32_16x16x4f32(b{i}_{ti}_{o}[{r}], {cur}[{ti}][{r}], '
                                 f'{nxt}[{o}], 0, 0, 0);')
            cur = nxt
    # dL/d(edge features): rows = the H0 inputs (one 16-row tile per 16; rows past the padded K read row 0)
    T0 = cols[0] // 16
    for o in range(-(-H0 // 16)):
        B += ['  {',
              '    mh_f4 d = mh_f4{0.f, 0.f, 0.f, 0.f};',
              f'    const int row = {16 * o} + c16 < {rows[0]} ? {16 * o} + c16 : 0;']
        for ti in range(T0):
            B.append(f'    const mh_f4 w{ti} = *reinterpret_cast<const mh_f4*>(&lds[{Lo["nat"][0]} + row * {cols[0] + PAD} + '
                     f'{16 * ti} + 4 * q]);')
            for r in range(4):
                B.append(f'    d = __builtin_amdgcn_mfma_f32_16x16x4f32(w{ti}[{r}], {cur}[{ti}][{r}], d, 0, 0, 0);')
        for r in range(4):
            B.append(f'    if (live && {16 * o + r} + 4 * q < {H0}) gef[ej * {H0} + {16 * o + r} + 4 * q] = d[{r}];')
        B.append('  }')
    B += ['}', '']
    L += B
    return '\n'.join(L)


def packed_weights(spec):
    """float32 weight buffers: {'fwd': (hidden transposed, WlT [NW, HL]), 'bwd': (hidden natural, Wl [HL, NW])}.
    Hidden layer i is laid out as the kernel's LDS copy: natural [k][j + PAD] (the first layer's K padded to a
    multiple of 4 with zero rows) or transposed [j][k + PAD]."""
    Lo = _layout(spec)
    nat = np.zeros(Lo['nat_size'])
    tr = np.zeros(Lo['tr_size'])
    for i, A in enumerate(spec.A[:-1]):
        r, c = Lo['rows'][i], Lo['cols'][i]
        buf = np.zeros((r, c + PAD))
        buf[:A.shape[0], :c] = A
        nat[Lo['nat'][i]:Lo['nat'][i] + buf.size] = buf.reshape(-1)
        bt = np.zeros((c, r + PAD))
        bt[:, :A.shape[0]] = A.T
        tr[Lo['tr'][i]:Lo['tr'][i] + bt.size] = bt.reshape(-1)
    Wl = spec.A[-1]
    return {'fwd': (tr.astype(np.float32), np.ascontiguousarray(Wl.T).astype(np.float32)),
            'bwd': (nat.astype(np.float32), np.ascontiguousarray(Wl).astype(np.float32))}


_DOUBLE_BACKWARD = ('mace_hip_kernels: double backward (create_graph=True, e.g. training on forces/stress or an '
                    'autograd Hessian) is not supported by the HIP kernels; use the unpatched e3nn model for that')


class _MLPFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, ef, op):
        s = op.spec
        if ef.dtype != torch.float32 or not ef.is_cuda:
            raise TypeError('mace_hip_kernels: the radial MLP expects float32 GPU input')
        if ef.shape[-1] != s.hs[0]:
            raise ValueError(f'expected [..., {s.hs[0]}] edge features, got {tuple(ef.shape)}')
        lead = ef.shape[:-1]
        x = ef.reshape(-1, s.hs[0]).contiguous()
        E = x.shape[0]
        out = torch.empty(E, s.hs[-1], device=x.device, dtype=torch.float32)
        _native.launch(f'mlp_fwd[{op.tag}]', _native.load().mh_mlp_fwd, op.module.handle, _native.ptr(x),
                       _native.ptr(op.WhT), _native.ptr(op.WlT), _native.ptr(out), E, _native.stream_of(x))
        ctx.save_for_backward(x)
        ctx.op, ctx.lead = op, lead
        return out.reshape(*lead, s.hs[-1])

    @staticmethod
    def backward(ctx, g):
        if torch.is_grad_enabled():
            raise RuntimeError(_DOUBLE_BACKWARD)
        x, = ctx.saved_tensors
        op = ctx.op
        s = op.spec
        g2 = g.reshape(-1, s.hs[-1]).contiguous()
        gx = torch.empty_like(x)
        _native.launch(f'mlp_bwd[{op.tag}]', _native.load().mh_mlp_bwd, op.module.handle, _native.ptr(x),
                       _native.ptr(op.Wh), _native.ptr(op.Wl), _native.ptr(g2), _native.ptr(gx), x.shape[0],
                       _native.stream_of(x))
        return gx.reshape(*ctx.lead, s.hs[0]), None


class HipRadialMLP(torch.nn.Module):
    """Drop-in for an e3nn ``FullyConnectedNet`` radial MLP: ``forward(edge_feats[..., n_basis]) -> [..., n_out]``."""

    def __init__(self, mod, device=None):
        super().__init__()
        self.spec = MLPSpec(mod)
        self.source = source(self.spec)
        code = _native.compile_source(self.source)
        dev = torch.device(device) if device is not None else torch.device('cuda', torch.cuda.current_device())
        with torch.cuda.device(dev):
            self.module = _native.Module(code, {
                _native.MH_MLP_FWD: (self.spec.kname('mlp_fwd'), BLOCK, EDGES),
                _native.MH_MLP_BWD: (self.spec.kname('mlp_bwd'), BLOCK, EDGES),
            })
        pw = packed_weights(self.spec)
        for name, arr in (('WhT', pw['fwd'][0]), ('WlT', pw['fwd'][1]), ('Wh', pw['bwd'][0]), ('Wl', pw['bwd'][1])):
            self.register_buffer(name, torch.tensor(arr, device=dev), persistent=False)
        self.hs = self.spec.hs
        self.original = [mod]
        self.tag = 'radial_mlp'

    def forward(self, ef):
        # the output's product with MACE's cutoff column is handed to the convolution unformed (conv.RadialWeights)
        return _MLPFn.apply(ef, self).as_subclass(_conv.RadialWeights)

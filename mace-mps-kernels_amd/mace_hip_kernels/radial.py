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


def source(spec):
    """HIP source of ``mlp_fwd`` and ``mlp_bwd``."""
    hs = spec.hs
    H0, NW = hs[0], hs[-1]
    hidden = hs[1:-1]
    nh = len(hidden)
    K0S = -(-H0 // 4)                                   # MFMA steps of the first layer
    HL = hs[-2]                                         # width feeding the output layer
    TL = HL // 16
    CHUNK = next(c for c in CHUNKS if NW % c == 0)
    # LDS: hidden weights [h_in][h_out + PAD] (first layer [4 K0S][...]), then one output-layer chunk [HL][CHUNK + PAD]
    offs, off = [], 0
    for i in range(nh):
        rows = 4 * K0S if i == 0 else hs[i]
        offs.append(off)
        off += rows * (hs[i + 1] + PAD)
    woff_chunk = off
    lds_floats = off + HL * (CHUNK + PAD)
    NCHK = NW // CHUNK
    NV4 = HL * CHUNK // 4                                # float4s per chunk
    NLD = -(-NV4 // BLOCK)                               # per thread (the last one clamped when NV4 % 256 != 0)
    L = [_native.device_header(), 'typedef float mh_f4 __attribute__((ext_vector_type(4)));', '']
    L += ['__device__ __forceinline__ float mlp_sig(float z) { return 1.f / (1.f + expf(-z)); }', '']

    # ---- shared prologue: hidden weights into LDS, this wave's 16 edges' features into registers
    def prologue(name, with_grad):
        P = [f'extern "C" __global__ __launch_bounds__({BLOCK}) void {name}(const float* __restrict__ ef,',
             '    const float* __restrict__ Wh, const float* __restrict__ Wl, ' +
             ('const float* __restrict__ gW, float* __restrict__ gef, long long E) {' if with_grad else
              'float* __restrict__ W0, long long E) {'),
             f'  __shared__ __align__(16) float lds[{lds_floats}];',
             '  const int t = threadIdx.x, wave = t >> 6, lane = t & 63, q = lane >> 4, c16 = lane & 15;',
             f'  const long long e0 = (long long)mh_xcd_block(blockIdx.x, gridDim.x) * {EDGES} + wave * 16;',
             '  const long long ej = e0 + c16;                 // this lane\'s edge (as a B column / output row)',
             '  const bool live = ej < E;',
             '  const long long ejc = live ? ej : E - 1;       // clamped: every load in bounds',
             f'  for (int f = t; f < {woff_chunk}; f += {BLOCK}) lds[f] = Wh[f];',
             '  __syncthreads();',
             f'  float xin[{K0S}];']
        P += [f'  xin[{st}] = {4 * st} + q < {H0} ? ef[ejc * {H0} + {4 * st} + q] : 0.f;' for st in range(K0S)]
        return P

    # output-layer weight chunks: float4 register prefetch (pre0..) and LDS store, unrolled (named registers)
    def chunk_load(nx, ind):
        P = []
        for it in range(NLD):
            fx = f't + {it * BLOCK}' if (it + 1) * BLOCK <= NV4 else f'min(t + {it * BLOCK}, {NV4 - 1})'
            P += [f'{ind}{{ const int f = {fx}, k = f / {CHUNK // 4}, c4 = f - k * {CHUNK // 4};',
                  f'{ind}  pre{it} = *reinterpret_cast<const mh_f4*>(Wl + (size_t)k * {NW} + {nx} + 4 * c4); }}']
        return P

    def chunk_store(ind):
        P = []
        for it in range(NLD):
            guard = '' if (it + 1) * BLOCK <= NV4 else f'if (t + {it * BLOCK} < {NV4}) '
            P += [f'{ind}{guard}{{ const int f = t + {it * BLOCK}, k = f / {CHUNK // 4}, c4 = f - k * {CHUNK // 4};',
                  f'{ind}  *reinterpret_cast<mh_f4*>(&lds[{woff_chunk} + k * {CHUNK + PAD} + 4 * c4]) = pre{it}; }}']
        return P

    def mm_first(dst, T):
        # layer 0: K = H0 in natural order (k = 4 s + q), A = W^T from LDS
        P = [f'  mh_f4 {dst}[{T}];']
        for o in range(T):
            P.append(f'  {dst}[{o}] = mh_f4{{0.f, 0.f, 0.f, 0.f}};')
            for st in range(K0S):
                P.append(f'  {dst}[{o}] = __builtin_amdgcn_mfma_f32_16x16x4f32(lds[{offs[0]} + ({4 * st} + q) * '
                         f'{hs[1] + PAD} + {16 * o} + c16], xin[{st}], {dst}[{o}], 0, 0, 0);')
        return P

    def mm_hidden(dst, src, T_in, T_out, base, ncol):
        # K walks the previous tile layout: step (t, r) <-> k = 16 t + 4 q + r (unrolled here: constant indices)
        P = [f'  mh_f4 {dst}[{T_out}];']
        for o in range(T_out):
            P.append(f'  {dst}[{o}] = mh_f4{{0.f, 0.f, 0.f, 0.f}};')
            for ti in range(T_in):
                for r in range(4):
                    P.append(f'  {dst}[{o}] = __builtin_amdgcn_mfma_f32_16x16x4f32(lds[{base} + ({16 * ti + r} + 4 * q) * '
                             f'{ncol + PAD} + {16 * o} + c16], {src}[{ti}][{r}], {dst}[{o}], 0, 0, 0);')
        return P

    def act(dst, src, T, c):
        P = [f'  mh_f4 {dst}[{T}];']
        for o in range(T):
            for r in range(4):
                P.append(f'  {dst}[{o}][{r}] = {_lit(c)} * {src}[{o}][{r}] * mlp_sig({src}[{o}][{r}]);')
        return P

    # ---------------------------------------------------------------- forward
    F = prologue('mlp_fwd', False)
    F += mm_first('z0', hidden[0] // 16) + act('h0', 'z0', hidden[0] // 16, spec.c[0])
    for i in range(1, nh):
        F += mm_hidden(f'z{i}', f'h{i - 1}', hidden[i - 1] // 16, hidden[i] // 16, offs[i], hidden[i])
        F += act(f'h{i}', f'z{i}', hidden[i] // 16, spec.c[i])
    hl = f'h{nh - 1}'
    F += [f'  mh_f4 {", ".join(f"pre{it}" for it in range(NLD))};']
    F += chunk_load('0', '  ')
    F += [f'  for (int ch = 0; ch < {NCHK}; ++ch) {{', '    __syncthreads();']
    F += chunk_store('    ')
    F += ['    __syncthreads();',
          f'    const int nx = min(ch + 1, {NCHK - 1}) * {CHUNK};      // next chunk (the last one reloads itself)']
    F += chunk_load('nx', '    ')
    for o in range(CHUNK // 16):
        F.append(f'    mh_f4 acc{o} = mh_f4{{0.f, 0.f, 0.f, 0.f}};')
    for ti in range(TL):
        for r in range(4):
            for o in range(CHUNK // 16):
                F.append(f'    acc{o} = __builtin_amdgcn_mfma_f32_16x16x4f32(lds[{woff_chunk} + ({16 * ti + r} + 4 * q) * '
                         f'{CHUNK + PAD} + {16 * o} + c16], {hl}[{ti}][{r}], acc{o}, 0, 0, 0);')
    F.append('    if (live) {')
    for o in range(CHUNK // 16):
        F.append(f'      *reinterpret_cast<mh_f4*>(W0 + ej * {NW} + ch * {CHUNK} + {16 * o} + 4 * q) = acc{o};')
    F += ['    }',
          '  }',
          '}', '']
    L += F

    # ---------------------------------------------------------------- backward
    B = prologue('mlp_bwd', True)
    B += mm_first('z0', hidden[0] // 16) + act('h0', 'z0', hidden[0] // 16, spec.c[0])
    for i in range(1, nh):
        B += mm_hidden(f'z{i}', f'h{i - 1}', hidden[i - 1] // 16, hidden[i] // 16, offs[i], hidden[i])
        if i < nh - 1:
            B += act(f'h{i}', f'z{i}', hidden[i] // 16, spec.c[i])
    # dL/dh_last = gW @ Wl^T: the output layer's columns are the K index, streamed in chunks; the B operand is gW, one
    # float4 per lane per 16 columns (k = 16 t + 4 q + r), the A operand Wl[h][k] from the staged chunk
    NG = CHUNK // 16
    B += [f'  mh_f4 dh[{TL}];']
    B += [f'  dh[{o}] = mh_f4{{0.f, 0.f, 0.f, 0.f}};' for o in range(TL)]
    B += [f'  mh_f4 {", ".join(f"pre{it}" for it in range(NLD))};']
    B += chunk_load('0', '  ')
    B += [f'  mh_f4 g{ti} = *reinterpret_cast<const mh_f4*>(gW + ejc * {NW} + {16 * ti} + 4 * q);' for ti in range(NG)]
    B += [f'  for (int ch = 0; ch < {NCHK}; ++ch) {{', '    __syncthreads();']
    B += chunk_store('    ')
    B += ['    __syncthreads();', f'    const int nx = min(ch + 1, {NCHK - 1}) * {CHUNK};']
    B += chunk_load('nx', '    ')
    B += [f'    const mh_f4 gn{ti} = *reinterpret_cast<const mh_f4*>(gW + ejc * {NW} + nx + {16 * ti} + 4 * q);'
          for ti in range(NG)]
    for ti in range(CHUNK // 16):
        for r in range(4):
            for o in range(TL):
                B.append(f'    dh[{o}] = __builtin_amdgcn_mfma_f32_16x16x4f32(lds[{woff_chunk} + ({16 * o} + c16) * '
                         f'{CHUNK + PAD} + {16 * ti + r} + 4 * q], g{ti}[{r}], dh[{o}], 0, 0, 0);')
    B += [f'    g{ti} = gn{ti};' for ti in range(NG)]
    B += ['  }']
    # back through the hidden layers: dz_i = dh_i * c_i * silu'(z_i); dh_{i-1} = dz_i @ A_i^T
    cur = 'dh'
    for i in range(nh - 1, -1, -1):
        T = hidden[i] // 16
        for o in range(T):
            for r in range(4):
                B += ['  {',
                      f'    const float z = z{i}[{o}][{r}], s = mlp_sig(z);',
                      f'    {cur}[{o}][{r}] *= {_lit(spec.c[i])} * s * (1.f + z * (1.f - s));',
                      '  }']
        if i > 0:
            Tp = hidden[i - 1] // 16
            nxt = f'dh{i - 1}'
            # A[j][k] = A_i[j][k] (row j = input feature of layer i, k = its output): LDS rows are the input features
            B.append(f'  mh_f4 {nxt}[{Tp}];')
            for o in range(Tp):
                B.append(f'  {nxt}[{o}] = mh_f4{{0.f, 0.f, 0.f, 0.f}};')
                for ti in range(T):
                    for r in range(4):
                        B.append(f'  {nxt}[{o}] = __builtin_amdgcn_mfma_f32_16x16x4f32(lds[{offs[i]} + ({16 * o} + c16) * '
                                 f'{hidden[i] + PAD} + {16 * ti + r} + 4 * q], {cur}[{ti}][{r}], {nxt}[{o}], 0, 0, 0);')
            cur = nxt
    # dL/d(edge features): rows = the H0 inputs (one 16-row tile per 16 inputs; rows past H0 read row 0)
    TI = -(-H0 // 16)
    T0 = hidden[0] // 16
    for o in range(TI):
        B += ['  {',
              '    mh_f4 d = mh_f4{0.f, 0.f, 0.f, 0.f};',
              f'    const int row = {16 * o} + c16 < {H0} ? {16 * o} + c16 : 0;']
        for ti in range(T0):
            for r in range(4):
                B.append(f'    d = __builtin_amdgcn_mfma_f32_16x16x4f32(lds[{offs[0]} + row * {hidden[0] + PAD} + '
                         f'{16 * ti + r} + 4 * q], {cur}[{ti}][{r}], d, 0, 0, 0);')
        for r in range(4):
            B.append(f'    if (live && {16 * o + r} + 4 * q < {H0}) gef[ej * {H0} + {16 * o + r} + 4 * q] = d[{r}];')
        B.append('  }')
    B += ['}', '']
    L += B
    return '\n'.join(L)


def packed_weights(spec):
    """(hidden weights as laid out in LDS, output-layer weights [HL, NW]) in float32."""
    hs = spec.hs
    K0S = -(-hs[0] // 4)
    parts = []
    for i, A in enumerate(spec.A[:-1]):
        rows = 4 * K0S if i == 0 else hs[i]
        buf = np.zeros((rows, hs[i + 1] + PAD))
        buf[:A.shape[0], :A.shape[1]] = A
        parts.append(buf.reshape(-1))
    return np.concatenate(parts).astype(np.float32), np.ascontiguousarray(spec.A[-1]).astype(np.float32)


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
                       _native.ptr(op.Wh), _native.ptr(op.Wl), _native.ptr(out), E, _native.stream_of(x))
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
                _native.MH_MLP_FWD: ('mlp_fwd', BLOCK, EDGES),
                _native.MH_MLP_BWD: ('mlp_bwd', BLOCK, EDGES),
            })
        wh, wl = packed_weights(self.spec)
        self.register_buffer('Wh', torch.tensor(wh, device=dev), persistent=False)
        self.register_buffer('Wl', torch.tensor(wl, device=dev), persistent=False)
        self.hs = self.spec.hs
        self.original = [mod]
        self.tag = 'radial_mlp'

    def forward(self, ef):
        return _MLPFn.apply(ef, self)

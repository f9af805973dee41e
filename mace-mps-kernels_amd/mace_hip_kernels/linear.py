"""
Node-wise equivariant linears on MI355X: drop-ins for e3nn ``o3.Linear`` (MACE's linear_up, linear, product linear,
node embedding) and for the tensor product of node features with scalar node attributes (MACE's ``skip_tp``, an
``o3.FullyConnectedTensorProduct(irreps, "n_elem x 0e", irreps_out)``).

Both are, per output irrep block o (multiplicity mul_o, dimension d = 2l+1) and node n,

    out[n, o, w, m] = sum_{i: irrep_i = irrep_o} sum_{u, v} x[n, i, u, m] a[n, v] W_io[u, v, w]

with a == 1 (V = 1 term) for the linear and a = node_attrs for skip_tp.  On the GPU the e3nn modules are a few
dozen launches each (slices, einsums through batched GEMMs, path-weight multiplies, a concatenation) and their
backward about as many again, each materialising a full-size tensor.  Here each direction is ONE launch of a
generated kernel: per output block, a GEMM with rows = (node, m) pairs, columns = output channels w, and
K = (input block, u, v), on the fp32 matrix cores (v_mfma_f32_16x16x4f32).  A tile is 16 // d whole nodes (<= 16
rows, one MFMA row tile) and 64 output channels (small tiles: the node counts of a batch are a few thousand, and
the chip has 256 CUs); long K loops run one tile per wave, short ones split K over a workgroup's waves.  Attribute terms v whose
a[n, v] is zero for every node of the tile are skipped (a one-hot element encoding leaves only the tile's species),
which is exact: they add 0.

The backward dL/dx is the same map with transposed weights Wt_oi[w, v, u] = W_io[u, v, w] (input and output blocks
swapped); attributes are data and get no gradient.

Weights are read from the module when it is patched (like the symmetric contraction's): the linear map is probed
on basis vectors in float64, and the block-diagonal equivariant structure is then checked on random inputs, so
e3nn's internal normalisation conventions never have to be restated.  Re-patch after changing the weights.
"""
import copy

import numpy as np
import torch

from . import _native

KC = 32              # K chunk (input channels u of one attribute v) loaded per step of a wave
BLOCK = 256          # 4 waves, one 16-row tile each
WAVES = BLOCK // 64
ROWS = 16            # rows (node, m) of a workgroup tile: one MFMA row tile


def _blocks(irreps):
    out, off = [], 0
    for mul, ir in irreps:
        out.append((mul, ir.l, off, str(ir)))
        off += mul * (2 * ir.l + 1)
    return out, off


def _kind(mod):
    if hasattr(mod, 'irreps_in1') and hasattr(mod, 'irreps_in2') and hasattr(mod, 'irreps_out'):
        return 'attrs'
    if hasattr(mod, 'irreps_in') and hasattr(mod, 'irreps_out'):
        return 'linear'
    return None


def lin_supported(mod):
    """(ok, reason) — whether an o3.Linear / scalar-attribute FullyConnectedTensorProduct can be replaced."""
    kind = _kind(mod)
    if kind is None:
        return False, 'not an e3nn Linear or tensor product'
    try:
        outs = mod.irreps_out
        if any(mul % 16 for mul, _ in outs):
            return False, 'output multiplicities must be multiples of 16'
        ins = mod.irreps_in1 if kind == 'attrs' else mod.irreps_in
        if any(2 * ir.l + 1 > ROWS for _, ir in list(ins) + list(outs)):
            return False, 'irrep too large'
        if kind == 'attrs':
            if any(str(ir) != '0e' for _, ir in mod.irreps_in2):
                return False, 'second operand must be scalars (0e)'
            if getattr(mod, 'shared_weights', True) is False:
                return False, 'per-sample weights'
        if getattr(mod, 'internal_weights', True) is False:
            return False, 'external weights'
    except (AttributeError, TypeError) as e:
        return False, f'unrecognised module ({e})'
    return True, ''


class LinSpec:
    """Block structure and packed weights of one node linear.

    ``terms[o]`` lists (i, woff) for every input block feeding output block o; W_io is stored [mul_i, V', mul_o]
    (V' = max(V, 1)) at ``woff`` of the packed forward weights.  ``bterms[i]`` lists (o, wtoff) for the transposed
    weights [mul_o, V', mul_i] of the backward."""

    def __init__(self, mod):
        ok, why = lin_supported(mod)
        if not ok:
            raise ValueError(why)
        self.kind = _kind(mod)
        ins = mod.irreps_in1 if self.kind == 'attrs' else mod.irreps_in
        self.in_blocks, self.Din = _blocks(ins)
        self.out_blocks, self.Dout = _blocks(mod.irreps_out)
        self.V = sum(m for m, _ in mod.irreps_in2) if self.kind == 'attrs' else 0
        Wio = _probe(mod, self)
        self.terms = {o: [] for o in range(len(self.out_blocks))}
        self.bterms = {i: [] for i in range(len(self.in_blocks))}
        fw, bw, fo, bo = [], [], 0, 0
        for (i, o), w in sorted(Wio.items()):          # w: [mul_i, V', mul_o] float64
            self.terms[o].append((i, fo))
            fw.append(w.reshape(-1))
            fo += w.size
            self.bterms[i].append((o, bo))
            bw.append(np.ascontiguousarray(w.transpose(2, 1, 0)).reshape(-1))
            bo += w.size
        self.W = np.concatenate(fw) if fw else np.zeros(4)
        self.Wt = np.concatenate(bw) if bw else np.zeros(4)
        self.Wio = Wio
        # the backward writes the input blocks with the same tiling: their multiplicities must tile too (a module
        # whose input never needs a gradient, like the node embedding of one-hot attributes, can do without)
        self.has_bwd = all(m % 16 == 0 for m, *_ in self.in_blocks)

    def apply(self, x, a=None):
        """float64 numpy application of the probed map (the patch-time structure check)."""
        out = np.zeros((x.shape[0], self.Dout))
        for (i, o), w in self.Wio.items():
            mi, li, oi, _ = self.in_blocks[i]
            mo, lo, oo, _ = self.out_blocks[o]
            d = 2 * li + 1
            xi = x[:, oi:oi + mi * d].reshape(-1, mi, d)
            if self.V:
                t = np.einsum('nud,nv,uvw->nwd', xi, a, w)
            else:
                t = np.einsum('nud,uw->nwd', xi, w[:, 0, :])
            out[:, oo:oo + mo * d] += t.reshape(x.shape[0], -1)
        return out

    def kname(self, base):
        """Kernel symbol of this module (shape-tagged so profiles tell the modules apart)."""
        return f'{base}_i{self.Din}_o{self.Dout}' + (f'_v{self.V}' if self.V else '')

    def flops(self, n):
        """Multiply-adds x 2 of the dense map over n nodes (attribute terms all counted)."""
        return 2 * n * sum(w.size * (2 * self.in_blocks[i][1] + 1) for (i, o), w in self.Wio.items())

    def bytes(self, n):
        """Algorithmic HBM bytes of (forward, backward) over n nodes: x (or g) in, out (or gx) out, attrs."""
        return (n * 4 * (self.Din + self.Dout + self.V),) * 2


def _probe(mod, spec):
    """{(i, o): W_io [mul_i, V', mul_o]} of the module's linear map, read off in float64 on the CPU."""
    m64 = copy.deepcopy(mod).to('cpu', torch.float64)
    VV = max(spec.V, 1)
    rows = sum(mul for mul, *_ in spec.in_blocks)
    X = torch.zeros(rows, spec.Din, dtype=torch.float64)
    r = 0
    starts = []
    for mul, l, off, _ in spec.in_blocks:
        starts.append(r)
        for u in range(mul):
            X[r, off + u * (2 * l + 1)] = 1.0
            r += 1
    outs = []
    with torch.no_grad():
        for v in range(VV):
            if spec.V:
                A = torch.zeros(rows, spec.V, dtype=torch.float64)
                A[:, v] = 1.0
                outs.append(m64(X, A).numpy())
            else:
                outs.append(m64(X).numpy())
    Wio = {}
    for i, (mi, li, oi, iri) in enumerate(spec.in_blocks):
        for o, (mo, lo, oo, iro) in enumerate(spec.out_blocks):
            if iri != iro:
                continue
            d = 2 * lo + 1
            w = np.stack([Y[starts[i]:starts[i] + mi, oo:oo + mo * d:d] for Y in outs], axis=1)   # [mi, V', mo]
            if np.any(w != 0.0):
                Wio[(i, o)] = w
    spec.Wio = Wio
    # structure check on random inputs: the module must be exactly this block-diagonal map (no bias, no mixing of
    # components m or of different irreps)
    rng = np.random.default_rng(0)
    x = rng.normal(size=(7, spec.Din))
    a = rng.normal(size=(7, spec.V)) if spec.V else None
    with torch.no_grad():
        ref = (m64(torch.tensor(x), torch.tensor(a)) if spec.V else m64(torch.tensor(x))).numpy()
    got = spec.apply(x, a)
    err = np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-300)
    if not err < 1e-10:
        raise ValueError(f'module is not a block-diagonal equivariant linear map (relative mismatch {err:.2e})')
    return Wio


def _cw(mo):
    """Columns per workgroup: 64 (4 MFMA column tiles per wave) where the multiplicity allows."""
    return 64 if mo % 64 == 0 else 32 if mo % 32 == 0 else 16


def _grid_y(blocks):
    """(block, column group) pairs of one direction, in blockIdx.y order."""
    return [(o, cg) for o, (mo, *_) in enumerate(blocks) for cg in range(mo // _cw(mo))]


def _tiles_mode(terms_o, in_blocks, V):
    """One tile per wave with the whole K loop (long K: the pipeline hides the load latency), or one tile per
    workgroup with K split over the waves (short K, or attribute terms: more waves in flight)."""
    return V == 0 and sum(-(-in_blocks[i][0] // KC) for i, _ in terms_o) >= 8


def _nodes_per_group(terms_o, in_blocks, V, l):
    tn = ROWS // (2 * l + 1)
    return WAVES * tn if (terms_o and _tiles_mode(terms_o, in_blocks, V)) else tn


def _loader(fn, i, in_blocks, mi, oi, D, Din, V, woff, mo, CT, NCH):
    """Register loads of chunk c of term i: A (x, times the attribute) and B (weights) in MFMA lane layout.

    K order inside a chunk: lane group kq takes k = k0 + 8 kq + st at step st, so a lane's 8 values of x are
    consecutive (two float4 loads for scalars); column order inside a group of 16 columns: lane c16 takes the CT
    adjacent columns CT c16 + ct (one vector load of W per step)."""
    VV = max(V, 1)
    vsel = f'vlist[1 + c / {NCH}]' if V else '0'
    vecx = D == 1 and Din % 4 == 0 and oi % 4 == 0 and mi % 8 == 0
    wt = {4: 'float4', 2: 'float2', 1: 'float'}[CT]
    L = [f'__device__ __forceinline__ void {fn}_ld{i}(const float* __restrict__ x, const float* __restrict__ attr,',
         '    const float* __restrict__ W, const int* __restrict__ vlist, int n0, int col0, int anl, int am,',
         f'    int q, int c16, int c, float (&ra)[{KC // 4}], float (&rb)[{KC // 4}][{CT}]) {{',
         f'  const int v = {vsel}, k0 = (c % {NCH}) * {KC} + 8 * q;',
         '  (void)v; (void)vlist; (void)attr;',
         f'  const float* __restrict__ xr = x + (size_t)(n0 + anl) * {Din} + {oi} + am;']
    if V:
        L.append(f'  const float s = attr[(size_t)(n0 + anl) * {V} + v];')
    if vecx:
        # mi % 8 == 0: the lane's 8 channels are all in range or all out of range
        L += [f'  const bool okx = k0 < {mi};',
              f'  const float4* __restrict__ xv = reinterpret_cast<const float4*>(xr + (okx ? k0 : 0));',
              '  const float4 x0 = xv[0], x1 = xv[1];',
              '  const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};']
    L += ['#pragma unroll',
          f'  for (int st = 0; st < {KC // 4}; ++st) {{',
          '    const int k = k0 + st;',
          f'    const bool ok = k < {mi};',
          f'    const int kc = ok ? k : {mi - 1};      // every load in bounds and unconditional']
    if vecx:
        L.append(f'    ra[st] = okx ? xs[st]{" * s" if V else ""} : 0.f;')
    else:
        L += [f'    const float xa = xr[kc * {D}];',
              f'    ra[st] = ok ? xa{" * s" if V else ""} : 0.f;']
    L += [f'    const {wt} wv = *reinterpret_cast<const {wt}*>(W + {woff} + ((size_t)kc * {VV} + v) * {mo} + col0'
          f' + {CT} * c16);']
    comps = ['x', 'y', 'z', 'w'][:CT] if CT > 1 else [None]
    for ct, cmp in enumerate(comps):
        L.append(f'    rb[st][{ct}] = ok ? wv{"." + cmp if cmp else ""} : 0.f;')
    L += ['  }', '}', '']
    return L


def _kloop(ld, CT, first, step, count, ind):
    """Pipelined K loop over `count` chunks first, first + step, ...: two register sets, unrolled by two so every
    array index is a constant and no branch separates a prefetch from the MFMAs that use it (the compiler would sink
    the loads past it); every prefetch is unconditional (clamped to the last chunk)."""
    mm = ['#pragma unroll',
          f'{ind}  for (int st = 0; st < {KC // 4}; ++st) {{',
          '#pragma unroll',
          f'{ind}    for (int ct = 0; ct < {CT}; ++ct)',
          f'{ind}      acc[ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(raX[st], rbX[st][ct], acc[ct], 0, 0, 0);',
          f'{ind}  }}']
    L = [f'{ind}float ra0[{KC // 4}], rb0[{KC // 4}][{CT}], ra1[{KC // 4}], rb1[{KC // 4}][{CT}];',
         f'{ind}const int nw = {count}, last = {first} + (nw - 1) * {step};',
         f'{ind}if (nw > 0) {ld}, {first}, ra0, rb0);',
         f'{ind}int c = {first};',
         f'{ind}for (int p = 0; p < nw / 2; ++p, c += {2 * step}) {{',
         f'{ind}  {ld}, min(c + {step}, last), ra1, rb1);',
         f'{ind}  __builtin_amdgcn_sched_barrier(0);']
    L += [l.replace('raX', 'ra0').replace('rbX', 'rb0') for l in mm]
    L += [f'{ind}  {ld}, min(c + {2 * step}, last), ra0, rb0);',
          f'{ind}  __builtin_amdgcn_sched_barrier(0);']
    L += [l.replace('raX', 'ra1').replace('rbX', 'rb1') for l in mm]
    L += [f'{ind}}}', f'{ind}if (nw & 1) {{']
    L += [l.replace('raX', 'ra0').replace('rbX', 'rb0') for l in mm]
    L += [f'{ind}}}']
    return L


def _mask(V, first, count):
    """The workgroup's list of attributes that are nonzero somewhere in its nodes (vlist[0] = count)."""
    VW = (V + 31) // 32
    return [f'  if (t < {VW}) amask[t] = 0u;',
            '  __syncthreads();',
            f'  for (int f = t; f < {count} * {V}; f += {BLOCK}) {{',
            f'    if (attr[(size_t){first} * {V} + f] != 0.f) {{ const int v = f % {V}; '
            'atomicOr(&amask[v >> 5], 1u << (v & 31)); }',
            '  }',
            '  __syncthreads();',
            '  if (t == 0) {',
            '    int c = 0;',
            f'    for (int w = 0; w < {VW}; ++w) {{',
            '      unsigned b = amask[w];',
            '      while (b) { vlist[1 + c++] = w * 32 + __builtin_ctz(b); b &= b - 1u; }',
            '    }',
            '    vlist[0] = c;',
            '  }',
            '  __syncthreads();',
            '  const int nact = vlist[0];']


def _kernel(name, in_blocks, out_blocks, terms, V, Din, Dout):
    """HIP source of one direction.  blockIdx.y selects (output block o, column group of CW channels), blockIdx.x a
    group of nodes.  A tile is TN = 16 // d whole nodes, i.e. <= 16 rows (node, m) — one MFMA row tile — and CW
    channels.  Each block runs in one of two modes (``_tiles_mode``):

    * one tile per wave, WAVES tiles per workgroup, each wave running the whole K loop for its tile and storing it
      from the result registers (no LDS, no barrier in the loop);
    * one tile per workgroup, its waves splitting K (chunks dealt round-robin) and the four partial tiles summed
      through LDS, then written node by node (each node's CW * d outputs are contiguous).

    K is walked in chunks c = (active attribute v, 32 input channels); operands are loaded straight into registers
    in the MFMA lane layout (16x16x4: lane (i, kq) = (lane % 16, lane / 16) holds A[i][4s + kq] and B[4s + kq][16 ct
    + i]) with the next chunk in flight."""
    fns, cases = [], []
    for o, (mo, l, oo, _) in enumerate(out_blocks):
        D = 2 * l + 1
        TN = ROWS // D
        CW = _cw(mo)
        CT = CW // 16
        fn = f'{name}_b{o}'
        tiles = bool(terms[o]) and _tiles_mode(terms[o], in_blocks, V)
        G = WAVES * TN if tiles else TN                       # nodes per workgroup
        L = [f'__device__ __forceinline__ void {fn}(const float* __restrict__ x, const float* __restrict__ attr,',
             '    const float* __restrict__ W, float* __restrict__ out, int N, int group, int cg, float* __restrict__ red,',
             '    unsigned* __restrict__ amask, int* __restrict__ vlist) {',
             f'  const int g0 = group * {G};                 // first node of the workgroup',
             '  if (g0 >= N) return;',
             f'  const int ng = min({G}, N - g0);',
             f'  const int t = threadIdx.x, col0 = cg * {CW};']
        if not terms[o]:
            L += [f'  for (int f = t; f < ng * {CW * D}; f += {BLOCK}) {{',
                  f'    const int nl = f / {CW * D}, j = f - nl * {CW * D};',
                  f'    out[(size_t)(g0 + nl) * {Dout} + {oo} + col0 * {D} + j] = 0.f;',
                  '  }', '}', '']
            fns += L
            cases.append((o, fn))
            continue
        L += ['  const int wave = t >> 6, lane = t & 63, q = lane >> 4, c16 = lane & 15;']
        if tiles:
            L += [f'  const int n0 = g0 + wave * {TN};                      // this wave\'s tile',
                  '  const bool wlive = n0 < N;',
                  f'  const int nn = wlive ? min({TN}, N - n0) : 0;',
                  '  const int nb = wlive ? n0 : g0;                        // load base: always a valid node']
        else:
            L += ['  const int n0 = g0, nn = ng, nb = g0;', '  const bool wlive = true;']
        # the lane's A row (node, m); rows past the tile read row 0 (their outputs are never stored)
        L += [f'  const int arow = c16 < nn * {D} ? c16 : 0;',
              f'  const int anl = arow / {D}, am = arow - anl * {D};',
              f'  mh_f4 acc[{CT}];',
              '#pragma unroll',
              f'  for (int c = 0; c < {CT}; ++c) acc[c] = mh_f4{{0.f, 0.f, 0.f, 0.f}};']
        if V:
            L += _mask(V, 'g0', 'ng')
        for (i, woff) in terms[o]:
            mi, li, oi, _ = in_blocks[i]
            assert li == l
            NCH = -(-mi // KC)
            nchunks = f'nact * {NCH}' if V else f'{NCH}'
            fns += _loader(fn, i, in_blocks, mi, oi, D, Din, V, woff, mo, CT, NCH)
            ld = f'{fn}_ld{i}(x, attr, W, vlist, nb, col0, anl, am, q, c16'
            if tiles:
                L += ['  if (wlive) {', f'    const int nch = {nchunks};']
                L += _kloop(ld, CT, '0', 1, 'nch', '    ')
            else:
                L += ['  {', f'    const int nch = {nchunks};']
                L += _kloop(ld, CT, 'wave', WAVES, 'wave < nch ? (nch - wave + 3) / 4 : 0', '    ')
            L += ['  }']
        if tiles:
            # the tile straight from the result registers: lane (c16, q) holds rows 4q + r, columns CT c16 + ct
            L += ['  if (wlive) {',
                  '#pragma unroll',
                  '    for (int r = 0; r < 4; ++r) {',
                  '      const int row = 4 * q + r;',
                  f'      if (row < nn * {D}) {{']
            if D == 1 and CT == 4 and Dout % 4 == 0 and oo % 4 == 0:
                L += [f'        *reinterpret_cast<float4*>(out + (size_t)(n0 + row) * {Dout} + {oo} + col0 + 4 * c16) =',
                      '            make_float4(acc[0][r], acc[1][r], acc[2][r], acc[3][r]);']
            else:
                L += [f'        const int nl = row / {D}, m = row - nl * {D};',
                      f'        float* __restrict__ o = out + (size_t)(n0 + nl) * {Dout} + {oo} + m;']
                L += [f'        o[(col0 + {CT} * c16 + {ct}) * {D}] = acc[{ct}][r];' for ct in range(CT)]
            L += ['      }', '    }', '  }', '}', '']
        else:
            # sum of the four waves' partial tiles, then coalesced per-node stores
            L += ['  __syncthreads();',
                  '#pragma unroll',
                  f'  for (int ct = 0; ct < {CT}; ++ct)',
                  '#pragma unroll',
                  '    for (int r = 0; r < 4; ++r)',
                  f'      red[(wave * 16 + q * 4 + r) * {CW} + {CT} * c16 + ct] = acc[ct][r];',
                  '  __syncthreads();',
                  f'  for (int f = t; f < nn * {CW * D}; f += {BLOCK}) {{',
                  f'    const int nl = f / {CW * D}, j = f - nl * {CW * D}, cc = j / {D}, m = j - cc * {D};',
                  f'    const int row = nl * {D} + m;',
                  f'    out[(size_t)(n0 + nl) * {Dout} + {oo} + col0 * {D} + j] = (red[row * {CW} + cc] + '
                  f'red[(16 + row) * {CW} + cc])',
                  f'        + (red[(32 + row) * {CW} + cc] + red[(48 + row) * {CW} + cc]);',
                  '  }',
                  '}', '']
        fns += L
        cases.append((o, fn))
    gy = _grid_y(out_blocks)
    cw_max = max(_cw(mo) for mo, *_ in out_blocks)
    VW = (V + 31) // 32
    sw = ['  switch (blockIdx.y) {']
    for y, (o, cg) in enumerate(gy):
        fn = dict(cases)[o]
        sw.append(f'    case {y}: {fn}(x, attr, W, out, N, group, {cg}, red, amask, vlist); break;')
    sw += ['    default: break;', '  }']
    K = [f'extern "C" __global__ __launch_bounds__({BLOCK}) void {name}(const float* __restrict__ x,',
         '    const float* __restrict__ attr, const float* __restrict__ W, float* __restrict__ out, int N) {',
         f'  __shared__ float red[{4 * 16 * cw_max}];',
         f'  __shared__ unsigned amask[{max(VW, 1)}];',
         f'  __shared__ int vlist[{V + 1}];',
         '  const int group = blockIdx.x;'] + sw + ['}', '']
    return fns + K


def source(spec):
    """HIP source of ``lin_fwd`` and ``lin_bwd`` for one module."""
    L = [_native.device_header(), 'typedef float mh_f4 __attribute__((ext_vector_type(4)));', '']
    L += _kernel(spec.kname('lin_fwd'), spec.in_blocks, spec.out_blocks, spec.terms, spec.V, spec.Din, spec.Dout)
    if spec.has_bwd:
        L += _kernel(spec.kname('lin_bwd'), spec.out_blocks, spec.in_blocks, spec.bterms, spec.V, spec.Dout, spec.Din)
    return '\n'.join(L)


def _tiles(blocks, terms, in_blocks, V):
    """Nodes per workgroup of the launch (its rows per block): the smallest over the output blocks; blocks with more
    nodes per workgroup leave their trailing workgroups idle."""
    return min(_nodes_per_group(terms[o], in_blocks, V, l) for o, (_, l, *_) in enumerate(blocks))


_DOUBLE_BACKWARD = ('mace_hip_kernels: double backward (create_graph=True, e.g. training on forces/stress or an '
                    'autograd Hessian) is not supported by the HIP kernels; use the unpatched e3nn model for that')


class _LinFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, attrs, op):
        s = op.spec
        if x.dtype != torch.float32 or not x.is_cuda:
            raise TypeError('mace_hip_kernels: node linears expect float32 GPU input')
        if x.shape[-1] != s.Din:
            raise ValueError(f'expected [..., {s.Din}] input, got {tuple(x.shape)}')
        lead = x.shape[:-1]
        x2 = x.reshape(-1, s.Din).contiguous()
        N = x2.shape[0]
        if N >= 2 ** 31:
            raise ValueError('too many nodes for one launch')
        a2 = None
        if s.V:
            if attrs is None or attrs.shape[-1] != s.V or attrs.shape[:-1] != lead:
                raise ValueError(f'expected node attributes [..., {s.V}] matching the input, got '
                                 f'{None if attrs is None else tuple(attrs.shape)}')
            if attrs.dtype != torch.float32 or attrs.device != x.device:
                raise TypeError('node attributes must be float32 on the input\'s device')
            a2 = attrs.reshape(-1, s.V).contiguous()
        out = torch.empty(N, s.Dout, device=x.device, dtype=torch.float32)
        _native.launch(f'lin_fwd[{op.tag}]', _native.load().mh_lin_fwd, op.module.handle, _native.ptr(x2),
                       _native.ptr(a2), _native.ptr(op.W), _native.ptr(out), N, _native.stream_of(x2))
        ctx.save_for_backward(a2) if a2 is not None else ctx.save_for_backward()
        ctx.op, ctx.lead, ctx.N = op, lead, N
        return out.reshape(*lead, s.Dout)

    @staticmethod
    def backward(ctx, g):
        if torch.is_grad_enabled():
            raise RuntimeError(_DOUBLE_BACKWARD)
        # node attributes are data (MACE's one-hot element encoding): no gradient flows to them, as in the
        # symmetric contraction
        if not ctx.needs_input_grad[0]:
            return None, None, None
        op = ctx.op
        s = op.spec
        if not s.has_bwd:
            raise NotImplementedError(f'mace_hip_kernels: {op.tag} has input multiplicities that the backward kernel '
                                      'does not tile (multiples of 16 needed)')
        a2 = ctx.saved_tensors[0] if ctx.saved_tensors else None
        g2 = g.reshape(-1, s.Dout).contiguous()
        gx = torch.empty(ctx.N, s.Din, device=g.device, dtype=torch.float32)
        _native.launch(f'lin_bwd[{op.tag}]', _native.load().mh_lin_bwd, op.module.handle, _native.ptr(g2),
                       _native.ptr(a2), _native.ptr(op.Wt), _native.ptr(gx), ctx.N, _native.stream_of(g2))
        return gx.reshape(*ctx.lead, s.Din), None, None


class HipNodeLinear(torch.nn.Module):
    """Drop-in for an e3nn ``o3.Linear`` (``forward(x)``) or a scalar-attribute ``FullyConnectedTensorProduct``
    (``forward(x, node_attrs)``), at inference (weights read at patch time; no weight gradients)."""

    def __init__(self, mod, device=None):
        super().__init__()
        self.spec = LinSpec(mod)
        s = self.spec
        self.source = source(s)
        code = _native.compile_source(self.source)
        dev = torch.device(device) if device is not None else torch.device('cuda', torch.cuda.current_device())
        with torch.cuda.device(dev):
            kernels = {_native.MH_LIN_FWD: (s.kname('lin_fwd'), BLOCK, _tiles(s.out_blocks, s.terms, s.in_blocks, s.V),
                                            len(_grid_y(s.out_blocks)))}
            if s.has_bwd:
                kernels[_native.MH_LIN_BWD] = (s.kname('lin_bwd'), BLOCK,
                                               _tiles(s.in_blocks, s.bterms, s.out_blocks, s.V),
                                               len(_grid_y(s.in_blocks)))
            self.module = _native.Module(code, kernels)
        self.register_buffer('W', torch.tensor(s.W, dtype=torch.float32, device=dev), persistent=False)
        self.register_buffer('Wt', torch.tensor(s.Wt, dtype=torch.float32, device=dev), persistent=False)
        for k in ('irreps_in', 'irreps_in1', 'irreps_in2', 'irreps_out'):
            if hasattr(mod, k):
                setattr(self, k, getattr(mod, k))
        self.original = [mod]
        self.tag = 'linear'

    def forward(self, x, attrs=None):
        if self.spec.V == 0 and attrs is not None:
            raise TypeError('this linear takes no node attributes')
        return _LinFn.apply(x, attrs, self)


"""
HIP source of the three interaction-convolution kernels of one layer (gfx950, wave64), generated from a ``ConvSpec``
with the layer's path coefficients as fp32 literals (reference conv.py:105-226 generates the Metal counterparts).

Thread mapping: lane u of the workgroup is channel u (NCB = ceil(MUL/64) waves per row); a row is a receiver (forward),
a sender (fused backward) or a chunk of 64 consecutive edges (per-edge backward).  Edge ids and their far endpoints
are fetched 64 at a time, one per lane, and broadcast with v_readlane, so the per-edge loop issues no dependent index
loads.  Per edge, Y[e] is wave-uniform (scalar loads); W[e], x[sender] and g[receiver] slices are 256-byte coalesced
loads at a uniform row pointer plus a loop-invariant per-lane offset.

Addressing: every global access is ``mh_ld(uniform_base, lane_byte_offset)`` — the base (row pointer + constant
column) lives in SGPRs, the per-lane offset is one of a handful of loop-invariant VGPRs (u·4·d for each block
dimension d), so no 64-bit VALU address arithmetic is emitted in the edge loop.  When MUL is a multiple of 64 every
lane is a live channel and no lane-activity test is generated at all.
"""
import numpy as np

from . import _native

WAVE = 64


def _lit(v):
    """Hexadecimal fp32 literal holding exactly float32(v) (round to nearest)."""
    return f'{float(np.float32(v)).hex()}f'


def _sum(parts):
    return ' + '.join(parts) if parts else '0.0f'


# fused backward: load each edge's inputs one iteration ahead of its use (see source())
PIPELINE_BWD = True


def _nxt(name):
    """Next-stage register of a per-edge input: y3 -> yn3, w2 -> wn2, gv5 -> gvn5."""
    return 'gvn' + name[2:] if name.startswith('gv') else name[0] + 'n' + name[1:]


class _Gen:
    """Shared naming for the three kernels of one spec."""

    def __init__(self, spec):
        self.s = spec
        self.full = spec.mul % WAVE == 0
        self.xi, self.nx = spec.xreg()
        self.oi, self.no = spec.oreg()
        self.dims = sorted({2 * l + 1 for l, _, _ in spec.in1} | {co['d3'] for co in spec.coef})

    # per-lane, loop-invariant byte offsets: channel u of a block with components of dimension d starts at u*d*4
    def prelude(self):
        L = ['  const int u = threadIdx.x, lane = threadIdx.x & (MH_WAVE - 1), wave = threadIdx.x >> 6;']
        if self.full:
            L += ['  const bool active = true;', '  const unsigned uc = u;']
        else:
            L += ['  const bool active = u < MUL;', '  const unsigned uc = active ? u : MUL - 1;',
                  '  const float am = active ? 1.0f : 0.0f;']
        L += [f'  const unsigned ol{d} = uc * {4 * d}u;' for d in sorted(set(self.dims) | {1})]
        return L

    def ld_x(self, ind, src):
        s = self.s
        L = [f'{ind}const float* __restrict__ xs = x + (size_t){src} * X_DIM;']
        for b, (l, _, off) in enumerate(s.in1):
            d = 2 * l + 1
            L += [f'{ind}xv{self.xi[b] + m} = mh_ld(xs + {off + m}, ol{d});' for m in range(d)]
        return L

    def ld_y(self, ind):
        return [f'{ind}const float* __restrict__ ye = Y + (size_t)e * Y_DIM;'] + \
               [f'{ind}const float y{j} = ye[{j}];' for j in range(self.s.y_dim)]

    def ld_w(self, ind):
        return [f'{ind}const float* __restrict__ we = W + (size_t)e * NW;'] + \
               [f'{ind}const float w{k} = mh_ld(we + {k * self.s.mul}, ol1);' for k in range(self.s.nins)]

    def ld_g(self, ind):
        L = [f'{ind}const float* __restrict__ gr = g + (size_t)r * OUT_DIM;']
        mask = '' if self.full else ' * am'
        for co in self.s.coef:
            d3 = co['d3']
            L += [f'{ind}const float gv{self.oi[co["k"]] + c} = mh_ld(gr + {co["o3"] + c}, ol{d3}){mask};'
                  for c in range(d3)]
        return L

    # --- software-pipelined backward: the edge's inputs are loaded one iteration ahead into the "n" stage
    def stage_names(self):
        s = self.s
        return ([f'y{j}' for j in range(s.y_dim)] + [f'w{k}' for k in range(s.nins)] +
                [f'gv{i}' for i in range(self.no)])

    def ld_stage(self, ind, e, r):
        """Issue the loads of edge (e, receiver r) into the next-stage registers yn*, wn*, gvn*."""
        s = self.s
        mask = '' if self.full else ' * am'
        L = [f'{ind}{{ const float* __restrict__ ye = Y + (size_t)({e}) * Y_DIM;',
             f'{ind}  const float* __restrict__ we = W + (size_t)({e}) * NW;',
             f'{ind}  const float* __restrict__ gr = g + (size_t)({r}) * OUT_DIM;']
        L += [f'{ind}  yn{j} = ye[{j}];' for j in range(s.y_dim)]
        L += [f'{ind}  wn{k} = mh_ld(we + {k * s.mul}, ol1);' for k in range(s.nins)]
        for co in s.coef:
            L += [f'{ind}  gvn{self.oi[co["k"]] + c} = mh_ld(gr + {co["o3"] + c}, ol{co["d3"]}){mask};'
                  for c in range(co['d3'])]
        L.append(f'{ind}}}')
        return L

    def fwd_body(self, ind):
        """acc[o] += w_k · Σ_a x[a] · (Σ_b v·y[b]) for every output component of every instruction."""
        L = []
        for co in self.s.coef:
            k, i1 = co['k'], self.s.ins[co['k']][0]
            for c in range(co['d3']):
                by_a = {}
                for a, b, cc, v in co['terms']:
                    if cc == c:
                        by_a.setdefault(a, []).append(f'{_lit(v)} * y{co["o2"] + b}')
                if not by_a:
                    continue
                t = _sum([f'xv{self.xi[i1] + a} * ({_sum(ys)})' for a, ys in sorted(by_a.items())])
                o = self.oi[k] + c
                L.append(f'{ind}acc{o} = fmaf(w{k}, {t}, acc{o});')
        return L

    def bwd_body(self, ind, with_gx):
        """h_a = Σ_{b,c} v·y[b]·g[c];  gx[a] += w·h_a;  gW_k = Σ_a x[a]·h_a;  P[b] += w·Σ_{a,c} v·x[a]·g[c]."""
        s = self.s
        L = []
        for co in s.coef:
            k, i1 = co['k'], s.ins[co['k']][0]
            L.append(f'{ind}{{')
            hs = []
            for a in range(co['d1']):
                ts = [f'{_lit(v)} * y{co["o2"] + b} * gv{self.oi[k] + c}' for aa, b, c, v in co['terms'] if aa == a]
                if not ts:
                    continue
                L.append(f'{ind}  const float h{a} = {_sum(ts)};')
                hs.append(a)
                if with_gx:
                    L.append(f'{ind}  gxa{self.xi[i1] + a} = fmaf(w{k}, h{a}, gxa{self.xi[i1] + a});')
            gw = _sum([f'xv{self.xi[i1] + a} * h{a}' for a in hs])
            st = f'mh_st_nt(gwe + {k * s.mul}, ol1, {gw});'       # written once, never re-read here
            L.append(f'{ind}  if (GWY) {st}' if self.full else f'{ind}  if (GWY && active) {st}')
            for b in range(co['d2']):
                ts = [f'{_lit(v)} * xv{self.xi[i1] + a} * gv{self.oi[k] + c}'
                      for a, bb, c, v in co['terms'] if bb == b]
                if ts:
                    L.append(f'{ind}  P{co["o2"] + b} = fmaf(w{k}, {_sum(ts)}, P{co["o2"] + b});')
            L.append(f'{ind}}}')
        return L


# Lane exchanges of the transpose reduction, one per lane bit from 5 down to 0.  Bits 5 and 4 cross 16-lane rows and
# go through __shfl_xor (ds_bpermute); bits 3..0 stay inside a row and use DPP moves, which are plain VALU operands
# (row_ror:8 = lane^8, row_half_mirror = lane^7, quad_perm [2,3,0,1] = lane^2, [1,0,3,2] = lane^1).  Every exchange
# pairs lanes that differ in the current bit and agree in the higher ones, which is all the reduction needs.
_DPP = {3: 0x128, 2: 0x141, 1: 0x4E, 0: 0xB1}


def _dpp(v, bit):
    return (f'__builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, {v}), '
            f'{_DPP[bit]:#x}, 0xf, 0xf, false))')


def _xchg(v, bit):
    return _dpp(v, bit) if bit < 4 else f'__shfl_xor({v}, {1 << bit}, MH_WAVE)'


def gy_reduce(indent, y_dim, y_pad):
    """Sum P0..P{y_pad-1} over the 64 lanes (transpose reduction, fixed order); lane L ends up holding the total of
    component L >> (6 - log2 y_pad), which lanes with zero low bits store to part[wave][j][.]."""
    L = [f'{indent}P{b} = 0.0f;' for b in range(y_dim, y_pad)]
    n = y_pad
    for bit in range(5, -1, -1):
        if n > 1:
            half = n // 2
            L.append(f'{indent}{{ const bool hi = (lane & {1 << bit}) != 0;')
            for k in range(half):
                L.append(f'{indent}  {{ const float s = hi ? P{k} : P{k + half}, q = hi ? P{k + half} : P{k};')
                L.append(f'{indent}    P{k} = q + {_xchg("s", bit)}; }}')
            L.append(f'{indent}}}')
            n = half
        else:
            L.append(f'{indent}P0 += {_xchg("P0", bit)};')
    shift = 6 - (y_pad.bit_length() - 1)
    L.append(f'{indent}{{ const int comp = lane >> {shift};')
    L.append(f'{indent}  if ((lane & {(1 << shift) - 1}) == 0 && comp < Y_DIM) part[wave][j][comp] = P0; }}')
    return L


def _gy_combine(indent, edge_expr):
    """Sum the per-wave gY partials of the current chunk held in LDS and write gY rows (fixed order)."""
    return [
        f'{indent}__syncthreads();',
        f'{indent}for (int q = threadIdx.x; q < cnt * Y_DIM; q += BLOCK) {{',
        f'{indent}  const int j = q / Y_DIM, b = q - j * Y_DIM;',
        f'{indent}  float v = 0.0f;',
        f'{indent}  for (int w = 0; w < NCB; ++w) v += part[w][j][b];',
        f'{indent}  gY[(size_t)({edge_expr}) * Y_DIM + b] = v;',
        f'{indent}}}',
        f'{indent}__syncthreads();',
    ]


def source(spec):
    """HIP source of conv_fwd, conv_bwd (fused) and conv_bwd_wy (per edge) for one layer."""
    G = _Gen(spec)
    nx, no = G.nx, G.no
    gyr = gy_reduce('      ', spec.y_dim, spec.y_pad)
    pdecl = 'float ' + ', '.join(f'P{b} = 0.0f' for b in range(spec.y_pad)) + ';'
    L = [_native.device_header(),
         f'#define MUL {spec.mul}', f'#define NCB {spec.ncb}', f'#define BLOCK {spec.block}',
         f'#define X_DIM {spec.x_dim}', f'#define Y_DIM {spec.y_dim}', f'#define Y_PAD {spec.y_pad}',
         f'#define OUT_DIM {spec.out_dim}', f'#define NW {spec.nins * spec.mul}']
    xdecl = 'float ' + ', '.join(f'xv{i}' for i in range(nx)) + ';'
    # ------------------------------------------------------------------------------------------- forward
    L += [
        f'extern "C" __global__ __launch_bounds__(BLOCK) void {spec.kname("conv_fwd")}(',
        '    const float* __restrict__ x, const float* __restrict__ Y, const float* __restrict__ W,',
        '    const int* __restrict__ rowptr, const int* __restrict__ eids, const int* __restrict__ senders,',
        '    float* __restrict__ out, int N) {',
        '  const int n = mh_xcd_block(blockIdx.x, gridDim.x);',
        '  if (n >= N) return;',
    ] + G.prelude() + [
        '  float ' + ', '.join(f'acc{i} = 0.0f' for i in range(no)) + ';',
        f'  {xdecl}',
        '  const int p0 = rowptr[n], p1 = rowptr[n + 1];',
        '  for (int pb = p0; pb < p1; pb += MH_WAVE) {',
        '    const int cnt = min(MH_WAVE, p1 - pb);',
        '    int my_e = 0, my_s = 0;',
        '    if (lane < cnt) { my_e = eids[pb + lane]; my_s = senders[my_e]; }',
        '    for (int j = 0; j < cnt; ++j) {',
        '      const int e = mh_bcast(my_e, j), s = mh_bcast(my_s, j);',
    ]
    L += G.ld_y('      ') + G.ld_x('      ', 's') + G.ld_w('      ') + G.fwd_body('      ')
    L += ['    }', '  }', '  if (active) {', '    float* __restrict__ o = out + (size_t)n * OUT_DIM;']
    for co in spec.coef:
        L += [f'    mh_st(o + {co["o3"] + c}, ol{co["d3"]}, acc{G.oi[co["k"]] + c});' for c in range(co['d3'])]
    L += ['  }', '}', '']
    # ----------------------------------------------------------------------------------- fused backward
    L += [
        f'extern "C" __global__ __launch_bounds__(BLOCK) void {spec.kname("conv_bwd")}(',
        '    const float* __restrict__ x, const float* __restrict__ g, const float* __restrict__ Y,',
        '    const float* __restrict__ W, const int* __restrict__ rowptr, const int* __restrict__ eids,',
        '    const int* __restrict__ receivers, float* __restrict__ gx, float* __restrict__ gW,',
        '    float* __restrict__ gY, int N, int flags) {',
        '  __shared__ float part[NCB][MH_WAVE][Y_PAD];',
        '  const int s = mh_xcd_block(blockIdx.x, gridDim.x);',
        '  if (s >= N) return;',
    ] + G.prelude() + [
        '  const bool GX = (flags & 1) != 0, GWY = (flags & 2) != 0;',
        '  float ' + ', '.join(f'xv{i} = 0.0f' for i in range(nx)) + ';',
        '  if (GWY) {',
    ]
    L += G.ld_x('    ', 's')
    L += [
        '  }',
        '  float ' + ', '.join(f'gxa{i} = 0.0f' for i in range(nx)) + ';',
        '  const int p0 = rowptr[s], p1 = rowptr[s + 1];',
        '  for (int pb = p0; pb < p1; pb += MH_WAVE) {',
        '    const int cnt = min(MH_WAVE, p1 - pb);',
        '    int my_e = 0, my_r = 0;',
        '    if (lane < cnt) { my_e = eids[pb + lane]; my_r = receivers[my_e]; }',
    ]
    if PIPELINE_BWD:
        # Edge j+1's loads are issued before edge j's gW stores.  vmcnt counts loads and stores in issue order, so
        # waiting for the next edge's inputs then never waits for the previous edge's stores.
        names = G.stage_names()
        L += ['    float ' + ', '.join(_nxt(n) for n in names) + ';',
              '    int en = mh_bcast(my_e, 0), rn = mh_bcast(my_r, 0);']
        L += G.ld_stage('    ', 'en', 'rn')
        L += ['    for (int j = 0; j < cnt; ++j) {', '      const int e = en, r = rn;']
        L += [f'      const float {n} = {_nxt(n)};' for n in names]
        L += ['      if (j + 1 < cnt) {', '        en = mh_bcast(my_e, j + 1); rn = mh_bcast(my_r, j + 1);']
        L += G.ld_stage('        ', 'en', 'rn')
        L += ['      }']
    else:
        L += ['    for (int j = 0; j < cnt; ++j) {', '      const int e = mh_bcast(my_e, j), r = mh_bcast(my_r, j);']
        L += G.ld_y('      ') + G.ld_w('      ') + G.ld_g('      ')
    L += [f'      {pdecl}', '      float* __restrict__ gwe = gW + (size_t)e * NW;']
    L += G.bwd_body('      ', with_gx=True)
    L += ['      if (GWY) {'] + ['  ' + t for t in gyr] + ['      }']
    L += ['    }', '    if (GWY) {']
    L += _gy_combine('      ', 'eids[pb + j]')
    L += ['    }', '  }', '  if (GX && active) {', '    float* __restrict__ gxs = gx + (size_t)s * X_DIM;']
    for b, (l, _, off) in enumerate(spec.in1):
        d = 2 * l + 1
        L += [f'    mh_st(gxs + {off + m}, ol{d}, gxa{G.xi[b] + m});' for m in range(d)]
    L += ['  }', '}', '']
    # --------------------------------------------------------------------- per-edge d/dW, d/dY (no CSR)
    L += [
        f'extern "C" __global__ __launch_bounds__(BLOCK) void {spec.kname("conv_bwd_wy")}(',
        '    const float* __restrict__ x, const float* __restrict__ g, const float* __restrict__ Y,',
        '    const float* __restrict__ W, const int* __restrict__ senders, const int* __restrict__ receivers,',
        '    float* __restrict__ gW, float* __restrict__ gY, int E) {',
        '  __shared__ float part[NCB][MH_WAVE][Y_PAD];',
        '  const int pb = mh_xcd_block(blockIdx.x, gridDim.x) * MH_WAVE;',
        '  if (pb >= E) return;',
    ] + G.prelude() + [
        '  const bool GWY = true;',
        '  const int cnt = min(MH_WAVE, E - pb);',
        f'  {xdecl}',
        '  int my_s = 0, my_r = 0;',
        '  if (lane < cnt) { my_s = senders[pb + lane]; my_r = receivers[pb + lane]; }',
        '  for (int j = 0; j < cnt; ++j) {',
        '    const int e = pb + j, s = mh_bcast(my_s, j), r = mh_bcast(my_r, j);',
    ]
    L += G.ld_y('    ') + G.ld_x('    ', 's') + G.ld_w('    ') + G.ld_g('    ')
    L += [f'    {pdecl}', '    float* __restrict__ gwe = gW + (size_t)e * NW;']
    L += G.bwd_body('    ', with_gx=False)
    L += [t[2:] for t in gyr]
    L += ['  }']
    L += _gy_combine('  ', 'pb + j')
    L += ['}', '']
    return '\n'.join(L)

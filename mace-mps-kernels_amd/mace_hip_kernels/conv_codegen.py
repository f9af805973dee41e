"""
HIP source of the three interaction-convolution kernels of one layer (gfx950, wave64), generated from a ``ConvSpec``
with the layer's path coefficients as fp32 literals (reference conv.py:105-226 generates the Metal counterparts).

Thread mapping: lane u of the workgroup is channel u (NCB = ceil(MUL/64) waves per row); a row is a receiver (forward),
a sender (fused backward) or a chunk of 64 consecutive edges (per-edge backward).  Edges are processed in chunks of
up to 64: their ids and far endpoints are fetched one per lane and broadcast with v_readlane, so the edge loop issues
no dependent index loads.

Edge-uniform coupling products.  For instruction k the tensor product contracts the Clebsch-Gordan table with the
edge's spherical harmonics before anything channel-dependent happens: M_k[a, c] = Σ_b C_k[a, b, c] · Y[e, o2_k + b].
These numbers are the same for every channel, so the row kernels compute them once per chunk, cooperatively (lane j
of the workgroup handles edge j, the pairs (k, a, c) split across the waves), into LDS; the edge loop then reads them
as wave-uniform ds_read_b128 broadcasts.  Then
    forward   acc[o3_k + c] += W[e, k] · Σ_a x[s, a] · M_k[a, c]
    backward  h_a = Σ_c M_k[a, c] · g[r, o3_k + c];   gx_a += W·h_a;   gW_k = Σ_a x_a h_a;
              gY[b] += W · Σ_{a,c} C_k[a,b,c] x_a g_c   (reduced over channels)
instead of every wave re-deriving the uniform products per edge.

Addressing: every global access is ``mh_ld(uniform_base, lane_byte_offset)`` — the base (row pointer + constant
column) is wave-uniform, the per-lane offset is one of a handful of loop-invariant registers (u·4·d for each block
dimension d).  When MUL is a multiple of 64 every lane is a live channel and no lane-activity test is generated.
Both row kernels issue the next edge's loads before the current edge's arithmetic and stores (vmcnt counts loads
and stores in issue order, so waiting for the next edge's inputs never waits for earlier stores).
"""
import numpy as np

from . import _native

WAVE = 64


def _lit(v):
    """Hexadecimal fp32 literal holding exactly float32(v) (round to nearest)."""
    return f'{float(np.float32(v)).hex()}f'


def _sum(parts):
    return ' + '.join(parts) if parts else '0.0f'


# fence the per-instruction LDS reads of the coupling products (bounds their register lifetime)
FENCE_M = True
# Load policy of the W (or W0) rows.  Read once per launch (the forward and backward kernels without a row map):
# non-temporal, never slower once W is not cache-resident (131 -> 112 us for the 1280-wide forward with W rotating
# over buffers larger than the Infinity Cache).  Read through a row map (conv_fwdcr: the radial MLP's rows shared
# between an edge and its reverse, each row read twice per launch): cacheable, so the second read finds the row in
# the caches (config 2 captured E+F -25 us, config 3 -18 us).  The receiver-ordered backward with a row map showed no
# difference either way and keeps the non-temporal policy.
W_NT = True
W_NT_ROWS = False
W_NT_BWD = True
# Store the gW (or ∂/∂W0) rows with the non-temporal policy (written once here; the radial MLP's backward reads
# them next).  Measured on config 2's captured E+F call: cacheable stores made it 25 us slower.
GW_NT = True
# ... except for layers with at most this many weights per edge: their dL/dW0 rows (config 2 layer 1: 161 MB) fit
# the Infinity Cache, where the MLP backward reads them next (captured call -3 us)
GW_CACHE_NW = 512
# Edges whose x and W slices the forward kernels have in flight ahead of the one being computed (1 or 2).
# Measured on config 2's captured E+F call: two ahead (unconditional, clamped loads) was 9 us slower.
FWD_PREFETCH = 1
# Edges whose x and W slices the receiver-ordered backward has in flight ahead of the one being computed (1 or 2).
# Measured on config 2 (isolated, layer 2): 290.7 us with one edge ahead, 295.7 us with two.
BWD_PREFETCH = 1
# The factored backward's per-edge cutoff: broadcast from a per-chunk register (True) or loaded per edge (False, a
# wave-uniform load).  Measured in config 2's E+F call, three alternating runs each: layer 1 backward 85.1-86.3 us
# broadcast, 76.8-77.3 us loaded; layer 2 unchanged (231-233 us).
BWD_CUT_BCAST = False
# Fence the factored backward's ∂/∂c accumulator after every instruction: the per-instruction gW values are then
# not scheduled together, 173 -> 155 VGPRs for the 1280-wide layer (3 waves per SIMD instead of 2; config 2,
# layer 2 backward 241 -> 230 us).
BWD_PC_FENCE = True
# Receiver-ordered backward with two channel waves: the waves' gY and ∂/∂c partials meet in one LDS plane by
# atomic adds (0 + a + b = 0 + b + a exactly, so the result does not depend on their order), halving that buffer
# (config 2, layer 1 backward 84 -> 77 us; layer 2's LDS then fits 6 workgroups per CU).
GY_LDS_ATOMIC = True
# Edges per chunk of the receiver-ordered kernels (conv_fwd/fwdc, conv_bwdr/bwdrc): 64 (one per lane), or 32 when
# a 64-edge chunk's coupling products would take more than CHUNK_LDS bytes of LDS (config 4's 17-instruction
# layer: 48 KB, 1.5 waves per SIMD; at 32 edges 24 KB).  Lanes 32-63 then sit out the chunk prologue only.
CHUNK_LDS = 24576


class _Gen:
    """Shared naming and code fragments for the kernels of one spec."""

    def __init__(self, spec):
        self.s = spec
        self.full = spec.mul % WAVE == 0
        self.xi, self.nx = spec.xreg()
        self.oi, self.no = spec.oreg()
        self.dims = sorted({2 * l + 1 for l, _, _ in spec.in1} | {co['d3'] for co in spec.coef} | {1})
        # coupling pairs (k, a, c) with their (b, coefficient) lists; pair p lives at Ms[edge][p]
        self.pairs = []
        self.pidx = {}
        for co in spec.coef:
            acc = {}
            for a, b, c, v in co['terms']:
                acc.setdefault((a, c), []).append((b, v))
            for (a, c), bv in sorted(acc.items()):
                self.pidx[(co['k'], a, c)] = len(self.pairs)
                self.pairs.append((co, a, c, bv))
        self.np = len(self.pairs)
        self.npp = (self.np + 3) // 4 * 4

    def prelude(self):
        L = ['  const int u = threadIdx.x, lane = threadIdx.x & (MH_WAVE - 1), wave = threadIdx.x >> 6;']
        if self.full:
            L += ['  const bool active = true;', '  const unsigned uc = u;']
        else:
            L += ['  const bool active = u < MUL;', '  const unsigned uc = active ? u : MUL - 1;',
                  '  const float am = active ? 1.0f : 0.0f;']
        L += [f'  const unsigned ol{d} = uc * {4 * d}u;' for d in self.dims]
        L += ['  (void)wave; (void)lane;']
        return L

    # ---------------------------------------------------------------------------------------- loads
    def ld_x(self, ind, src, dst='xv'):
        L = [f'{ind}{{ const float* __restrict__ xs = x + (size_t)({src}) * X_DIM;']
        for b, (l, _, off) in enumerate(self.s.in1):
            d = 2 * l + 1
            L += [f'{ind}  {dst}{self.xi[b] + m} = mh_ld(xs + {off + m}, ol{d});' for m in range(d)]
        return L + [f'{ind}}}']

    def ld_w(self, ind, e, dst, nt):
        ld = 'mh_ld_nt' if nt else 'mh_ld'
        return ([f'{ind}{{ const float* __restrict__ we = W + (size_t)({e}) * NW;'] +
                [f'{ind}  {dst}{k} = {ld}(we + {k * self.s.mul}, ol1);' for k in range(self.s.nins)] + [f'{ind}}}'])

    def ld_g(self, ind, r, dst):
        mask = '' if self.full else ' * am'
        L = [f'{ind}{{ const float* __restrict__ gr = g + (size_t)({r}) * OUT_DIM;']
        for co in self.s.coef:
            L += [f'{ind}  {dst}{self.oi[co["k"]] + c} = mh_ld(gr + {co["o3"] + c}, ol{co["d3"]}){mask};'
                  for c in range(co['d3'])]
        return L + [f'{ind}}}']

    def ld_y_uniform(self, ind):
        return [f'{ind}const float* __restrict__ ye = Y + (size_t)e * Y_DIM;'] + \
               [f'{ind}const float y{j} = ye[{j}];' for j in range(self.s.y_dim)]

    # ---------------------------------------------------------------- chunk prologue: M into LDS
    def m_prologue(self, ind, edge_of_lane):
        """Lane j computes edge j's coupling products; the pairs are split evenly over the NCB waves."""
        s, ncb = self.s, self.s.ncb
        per = (self.np + ncb - 1) // ncb
        L = [f'{ind}if (lane < cnt) {{',
             f'{ind}  const float* __restrict__ yl = Y + (size_t)({edge_of_lane}) * Y_DIM;']
        L += [f'{ind}  const float q{j} = yl[{j}];' for j in range(s.y_dim)]
        L += [f'{ind}  float* __restrict__ mrow = &Ms[lane][0];']
        for w in range(ncb):
            sel = self.pairs[w * per:(w + 1) * per]
            if not sel:
                continue
            L.append(f'{ind}  if (wave == {w}) {{' if ncb > 1 else f'{ind}  {{')
            for p, (co, a, c, bv) in enumerate(sel, start=w * per):
                val = _sum([f'{_lit(v)} * q{co["o2"] + b}' for b, v in bv])
                L.append(f'{ind}    mrow[{p}] = {val};')
            L.append(f'{ind}  }}')
        L.append(f'{ind}}}')
        L.append(f'{ind}__syncthreads();')
        return L

    def ld_m(self, ind, k):
        """Instruction k's coupling products of the current edge from LDS (uniform address → broadcast), read right
        before use; with FENCE_M an empty asm with a memory clobber keeps the next block's reads from being hoisted
        (LDS loads are ordinary loads, so the clobber orders them)."""
        qs = sorted({p // 4 for (kk, _, _), p in self.pidx.items() if kk == k})
        L = [f'{ind}asm volatile("" ::: "memory");'] if FENCE_M else []
        return L + [f'{ind}const float4 mq{q} = Ms4[j][{q}];' for q in qs]

    def m(self, k, a, c):
        p = self.pidx[(k, a, c)]
        return f'mq{p // 4}.{"xyzw"[p % 4]}'

    # ------------------------------------------------------------------------------- edge bodies
    def fwd_body(self, ind, xv='xv', w='w'):
        """acc[o] += w_k · Σ_a x_a · M_k[a, c]."""
        L = []
        for co in self.s.coef:
            k, i1 = co['k'], self.s.ins[co['k']][0]
            L.append(f'{ind}{{')
            L += self.ld_m(ind + '  ', k)
            for c in range(co['d3']):
                ts = [f'{xv}{self.xi[i1] + a} * {self.m(k, a, c)}' for a in range(co['d1'])
                      if (k, a, c) in self.pidx]
                if ts:
                    o = self.oi[k] + c
                    L.append(f'{ind}  acc{o} = fmaf({w}{k}, {_sum(ts)}, acc{o});')
            L.append(f'{ind}}}')
        return L

    def bwd_body(self, ind, with_gx, use_m, store, cut=False):
        """h_a = Σ_c M[a,c]·g_c (or Σ_{b,c} v·y_b·g_c);  gx_a += w·h_a;  gW_k = Σ_a x_a·h_a;
        P_b += w·Σ_{a,c} v·x_a·g_c.  With ``store`` the gW row is written and P accumulated; full-wave specs write it
        unconditionally (a store under a branch makes the wait-count pass assume it may be absent and wait for every
        outstanding access at the next edge, stores included).  With ``cut`` the weights are W = W0·c (w0{k}, ce):
        the stored row is ∂/∂W0 = gW·c and Pc accumulates this lane's share of ∂/∂c = Σ_k gW_k·W0_k."""
        s = self.s
        L = []
        for co in s.coef:
            k, i1 = co['k'], s.ins[co['k']][0]
            L.append(f'{ind}{{')
            if use_m:
                L += self.ld_m(ind + '  ', k)
            hs = []
            for a in range(co['d1']):
                if use_m:
                    ts = [f'{self.m(k, a, c)} * gv{self.oi[k] + c}' for c in range(co['d3']) if (k, a, c) in self.pidx]
                else:
                    ts = [f'{_lit(v)} * y{co["o2"] + b} * gv{self.oi[k] + c}'
                          for aa, b, c, v in co['terms'] if aa == a]
                if not ts:
                    continue
                L.append(f'{ind}  const float h{a} = {_sum(ts)};')
                hs.append(a)
                if with_gx:
                    L.append(f'{ind}  gxa{self.xi[i1] + a} = fmaf(w{k}, h{a}, gxa{self.xi[i1] + a});')
            if not store:
                L.append(f'{ind}}}')
                continue
            gw = _sum([f'xv{self.xi[i1] + a} * h{a}' for a in hs])
            if cut:
                L.append(f'{ind}  const float gwk = {gw};')
                L.append(f'{ind}  Pc = fmaf(gwk, w0{k}, Pc);' + (' asm volatile("" : "+v"(Pc));' if BWD_PC_FENCE else ''))
                gw = 'gwk * ce'
            gw_nt = GW_NT and s.nins * s.mul > GW_CACHE_NW
            st = f'{"mh_st_nt" if gw_nt else "mh_st"}(gwe + {k * s.mul}, ol1, {gw});'
            L.append(f'{ind}  {st}' if self.full else f'{ind}  if (active) {st}')
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


def gy_reduce(indent, y_dim, y_pad, atomic=False):
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
    dst = 'atomicAdd(&part[j][comp], P0)' if atomic else 'part[wave][j][comp] = P0'
    L.append(f'{indent}  if ((lane & {(1 << shift) - 1}) == 0 && comp < Y_DIM) {dst}; }}')
    return L


def chunk_edges(npp):
    """Edges per chunk of the receiver-ordered kernels for npp coupling products per edge."""
    return WAVE if WAVE * npp * 4 <= CHUNK_LDS else WAVE // 2


def _gy_combine(indent, edge_expr, cut=False, atomic=False):
    """Sum the per-wave gY partials of the current chunk held in LDS and write gY rows (fixed order); with ``cut``
    also the ∂/∂c partials.  The leading barrier also orders the chunk's Ms reads before the next chunk's prologue
    overwrites them."""
    L = [
        f'{indent}__syncthreads();',
        f'{indent}for (int q = threadIdx.x; q < cnt * Y_DIM; q += BLOCK) {{',
        f'{indent}  const int j = q / Y_DIM, b = q - j * Y_DIM;',
    ] + ([
        f'{indent}  const float v = part[j][b];',
        f'{indent}  part[j][b] = 0.0f;                    // zero again for the next chunk\'s atomic adds',
    ] if atomic else [
        f'{indent}  float v = 0.0f;',
        f'{indent}  for (int w = 0; w < NCB; ++w) v += part[w][j][b];',
    ]) + [
        f'{indent}  gY[(size_t)({edge_expr}) * Y_DIM + b] = v;',
        f'{indent}}}',
    ]
    if cut:
        L += [f'{indent}for (int j = threadIdx.x; j < cnt; j += BLOCK) {{']
        L += ([f'{indent}  const float v = partc[j];', f'{indent}  partc[j] = 0.0f;'] if atomic else
              [f'{indent}  float v = 0.0f;', f'{indent}  for (int w = 0; w < NCB; ++w) v += partc[w][j];'])
        L += [f'{indent}  gcut[{edge_expr}] = v;',
              f'{indent}}}']
    return L + [f'{indent}__syncthreads();']


def source(spec):
    """HIP source of conv_fwd, conv_bwd (fused) and conv_bwd_wy (per edge) for one layer."""
    G = _Gen(spec)
    nx, no, nk = G.nx, G.no, spec.nins
    gyr = gy_reduce('      ', spec.y_dim, spec.y_pad)
    pdecl = 'float ' + ', '.join(f'P{b} = 0.0f' for b in range(spec.y_pad)) + ';'

    def decl(prefix, n, init=None):
        return 'float ' + ', '.join(f'{prefix}{i}' + ('' if init is None else f' = {init}') for i in range(n)) + ';'

    def copy(dst, src, n):
        return [f'      const float {dst}{i} = {src}{i};' for i in range(n)]

    L = [_native.device_header(),
         f'#define MUL {spec.mul}', f'#define NCB {spec.ncb}', f'#define BLOCK {spec.block}',
         f'#define X_DIM {spec.x_dim}', f'#define Y_DIM {spec.y_dim}', f'#define Y_PAD {spec.y_pad}',
         f'#define OUT_DIM {spec.out_dim}', f'#define NW {spec.nins * spec.mul}', f'#define NPP {G.npp}',
         f'#define CHUNK {chunk_edges(G.npp)}']
    ms_decl = ['  __shared__ float4 Ms4[MH_WAVE][NPP / 4];',
               '  float (*Ms)[NPP] = reinterpret_cast<float (*)[NPP]>(Ms4);']
    ms_decl_c = ['  __shared__ float4 Ms4[CHUNK][NPP / 4];',
                 '  float (*Ms)[NPP] = reinterpret_cast<float (*)[NPP]>(Ms4);']
    # ------------------------------------------------------------------------------------------- forward
    def fwd_kernel(cut, rows=False):
        """``cut`` (kernel ``conv_fwdc``): the weights are W0·c with a per-edge scalar c, read as W0 and scaled in
        registers (the product is never formed in memory); an edge with c == 0 (padding, or past r_max in a
        neighbour list with a skin) contributes exactly zero, so each chunk of 64 edges is first compacted to its
        edges with c != 0 (ballot, then a per-wave LDS scatter by lane rank) and only those are walked.  Every wave
        of the workgroup builds the same list, so the barriers stay uniform."""
        F = [
            f'extern "C" __global__ __launch_bounds__(BLOCK) void '
            f'{spec.kname(("conv_fwdcr" if rows else "conv_fwdc") if cut else "conv_fwd")}(',
            '    const float* __restrict__ x, const float* __restrict__ Y, const float* __restrict__ W,',
            '    const int* __restrict__ rowptr, const int* __restrict__ eids, const int* __restrict__ senders,',
            '    float* __restrict__ out, int N' + (', const float* __restrict__ cutv, const int* __restrict__ wrow) {'
                                                   if cut else ') {'),
        ] + ms_decl_c + (['  __shared__ int sidx[NCB][CHUNK];'] if cut else []) + [
            '  const int n = mh_xcd_block(blockIdx.x, gridDim.x);',
            '  if (n >= N) return;',
        ] + G.prelude() + [
            '  ' + decl('acc', no, '0.0f'),
            '  ' + decl('xn', nx), '  ' + decl('wn', nk),
        ] + (['  ' + decl('xm', nx), '  ' + decl('wm', nk)] if FWD_PREFETCH > 1 else []) + [
            '  const int p0 = rowptr[n], p1 = rowptr[n + 1];',
            '  for (int pb = p0; pb < p1; pb += CHUNK) {',
        ]
        if cut:
            F += ['    const int cnt0 = min(CHUNK, p1 - pb);',
                  '    int my_e = 0, my_s = 0;',
                  '    bool keep = false;',
                  '    if (lane < cnt0) { my_e = eids[pb + lane]; keep = cutv[my_e] != 0.0f; }',
                  '    const unsigned long long kept = __ballot(keep);',
                  '    const int cnt = __popcll(kept);',
                  '    if (keep) sidx[wave][__popcll(kept & ((1ull << lane) - 1ull))] = my_e;',
                  '    if (cnt == 0) continue;',
                  '    float my_c = 0.0f;',
                  '    int my_w = 0;                       // the W0 row of lane j\'s edge (its own, or wrow[e])',
                  '    if (lane < cnt) {',
                  '      my_e = sidx[wave][lane]; my_s = senders[my_e]; my_c = cutv[my_e];',
                  '      my_w = wrow ? wrow[my_e] : my_e;',
                  '    }']
        else:
            F += ['    const int cnt = min(CHUNK, p1 - pb);',
                  '    int my_e = 0, my_s = 0;',
                  '    if (lane < cnt) { my_e = eids[pb + lane]; my_s = senders[my_e]; }',
                  '    const int my_w = my_e;']
        F += G.m_prologue('    ', 'my_e')
        F += ['    {', '      const int er0 = mh_bcast(my_w, 0), s0 = mh_bcast(my_s, 0);']
        F += G.ld_x('      ', 's0', 'xn') + G.ld_w('      ', 'er0', 'wn', W_NT_ROWS if rows else W_NT)
        F += ['    }']
        if FWD_PREFETCH > 1:          # edge 1 (or the last edge again) one stage further out
            F += ['    {', '      const int er1 = mh_bcast(my_w, min(1, cnt - 1)), s1 = mh_bcast(my_s, min(1, cnt - 1));']
            F += G.ld_x('      ', 's1', 'xm') + G.ld_w('      ', 'er1', 'wm', W_NT_ROWS if rows else W_NT)
            F += ['    }']
        F += ['    for (int j = 0; j < cnt; ++j) {']
        F += copy('xv', 'xn', nx)
        if cut:
            F += ['      const float cj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_c), j));']
            F += [f'      const float w{k} = wn{k} * cj;' for k in range(nk)]
        else:
            F += copy('w', 'wn', nk)
        if FWD_PREFETCH > 1:
            # unconditional (the last edges re-load themselves): no branch around the loads
            F += [f'      xn{i} = xm{i};' for i in range(nx)] + [f'      wn{k} = wm{k};' for k in range(nk)]
            F += ['      {', '        const int j2 = min(j + 2, cnt - 1);',
                  '        const int er2 = mh_bcast(my_w, j2), s2 = mh_bcast(my_s, j2);']
            F += G.ld_x('        ', 's2', 'xm') + G.ld_w('        ', 'er2', 'wm', W_NT_ROWS if rows else W_NT)
            F += ['      }']
        else:
            F += ['      if (j + 1 < cnt) {', '        const int er1 = mh_bcast(my_w, j + 1), s1 = mh_bcast(my_s, j + 1);']
            F += G.ld_x('        ', 's1', 'xn') + G.ld_w('        ', 'er1', 'wn', W_NT_ROWS if rows else W_NT)
            F += ['      }']
        F += G.fwd_body('      ')
        F += ['    }', '    __syncthreads();', '  }', '  if (active) {',
              '    float* __restrict__ o = out + (size_t)n * OUT_DIM;']
        for co in spec.coef:
            F += [f'    mh_st(o + {co["o3"] + c}, ol{co["d3"]}, acc{G.oi[co["k"]] + c});' for c in range(co['d3'])]
        return F + ['  }', '}', '']

    L += fwd_kernel(False) + fwd_kernel(True) + fwd_kernel(True, rows=True)
    # ----------------------------------------------------------------------------------- fused backward
    L += [
        f'extern "C" __global__ __launch_bounds__(BLOCK) void {spec.kname("conv_bwd")}(',
        '    const float* __restrict__ x, const float* __restrict__ g, const float* __restrict__ Y,',
        '    const float* __restrict__ W, const int* __restrict__ rowptr, const int* __restrict__ eids,',
        '    const int* __restrict__ receivers, float* __restrict__ gx, float* __restrict__ gW,',
        '    float* __restrict__ gY, int N, int flags) {',
        '  __shared__ float part[NCB][MH_WAVE][Y_PAD];',
    ] + ms_decl + [
        '  const int s = mh_xcd_block(blockIdx.x, gridDim.x);',
        '  if (s >= N) return;',
    ] + G.prelude() + [
        '  const bool GX = (flags & 1) != 0, GWY = (flags & 2) != 0;',
        '  ' + decl('xv', nx, '0.0f'),
        '  if (GWY) {',
    ]
    L += G.ld_x('    ', 's')
    L += [
        '  }',
        '  ' + decl('gxa', nx, '0.0f'),
        '  ' + decl('wn', nk), '  ' + decl('gvn', no),
        '  const int p0 = rowptr[s], p1 = rowptr[s + 1];',
    ]

    def bwd_chunks(store):
        # The flag test sits outside the edge loop, and the next edge's loads are unconditional (the last edge of a
        # chunk re-loads itself), so the loop has no branch around a global access: the wait for the prefetched
        # inputs then counts only the stores issued after them instead of draining the memory queue every edge.
        C = ['  for (int pb = p0; pb < p1; pb += MH_WAVE) {',
             '    const int cnt = min(MH_WAVE, p1 - pb);',
             '    int my_e = 0, my_r = 0;',
             '    if (lane < cnt) { my_e = eids[pb + lane]; my_r = receivers[my_e]; }']
        C += G.m_prologue('    ', 'my_e')
        C += ['    {', '      const int e0 = mh_bcast(my_e, 0), r0 = mh_bcast(my_r, 0);']
        C += G.ld_w('      ', 'e0', 'wn', W_NT_BWD) + G.ld_g('      ', 'r0', 'gvn')
        C += ['    }', '    for (int j = 0; j < cnt; ++j) {', '      const int e = mh_bcast(my_e, j);']
        C += copy('w', 'wn', nk) + copy('gv', 'gvn', no)
        C += ['      {', '        const int j1 = min(j + 1, cnt - 1);',
              '        const int e1 = mh_bcast(my_e, j1), r1 = mh_bcast(my_r, j1);']
        C += G.ld_w('        ', 'e1', 'wn', W_NT_BWD) + G.ld_g('        ', 'r1', 'gvn')
        C += ['      }']
        if store:
            C += [f'      {pdecl}', '      float* __restrict__ gwe = gW + (size_t)e * NW;']
        C += G.bwd_body('      ', with_gx=True, use_m=True, store=store)
        if store:
            C += gyr
        C += ['    }']
        C += _gy_combine('    ', 'eids[pb + j]') if store else ['    __syncthreads();']
        return C + ['  }']

    L += ['  if (GWY) {'] + ['  ' + t for t in bwd_chunks(True)] + ['  } else {']
    L += ['  ' + t for t in bwd_chunks(False)] + ['  }']
    L += ['  if (GX && active) {', '    float* __restrict__ gxs = gx + (size_t)s * X_DIM;']
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
        '  const int cnt = min(MH_WAVE, E - pb);',
        '  ' + decl('xv', nx), '  ' + decl('w', nk), '  ' + decl('gv', no),
        '  int my_s = 0, my_r = 0;',
        '  if (lane < cnt) { my_s = senders[pb + lane]; my_r = receivers[pb + lane]; }',
        '  for (int j = 0; j < cnt; ++j) {',
        '    const int e = pb + j, s = mh_bcast(my_s, j), r = mh_bcast(my_r, j);',
    ]
    L += G.ld_y_uniform('    ') + G.ld_x('    ', 's') + G.ld_w('    ', 'e', 'w', W_NT_BWD) + G.ld_g('    ', 'r', 'gv')
    L += [f'    {pdecl}', '    float* __restrict__ gwe = gW + (size_t)e * NW;']
    L += G.bwd_body('    ', with_gx=False, use_m=False, store=True)
    L += [t[2:] for t in gyr]
    L += ['  }']
    L += _gy_combine('  ', 'pb + j')
    L += ['}', '']
    L += _bwd_recv(G, gyr, pdecl, decl, copy)
    L += _bwd_recv(G, gyr, pdecl, decl, copy, cut=True)
    L += _gx_sum(spec)
    return '\n'.join(L)


def _bwd_recv(G, gyr, pdecl, decl, copy, cut=False):
    """Receiver-ordered backward (rows = receivers, the forward's CSR).  g[r] is loaded once per row and stays in
    registers; each edge gathers only x[s] (X_DIM floats) and its W row, writes its gW row and gY, and, when dX is
    wanted, its dX message gxm[e] = Σ_k W_k·h_k (X_DIM floats), which ``conv_gxsum`` adds up per sender.  Per edge
    this reads X_DIM + NW floats per channel block instead of the OUT_DIM-float g row the sender-ordered kernel
    gathers.

    ``cut`` (kernel ``conv_bwdrc``): the weights arrive factored as W = W0·c with a per-edge scalar c (MACE's
    ``tp_weights * cutoff``).  The kernel reads W0 and c, writes ∂/∂W0 = gW·c instead of gW, and reduces
    ∂/∂c[e] = Σ_{k,u} gW·W0 over the channels (a butterfly over the wave, then LDS across waves, fixed order), which
    saves the caller the separate passes over the [E, NW] tensors that differentiating the product takes.

    Masked edges (``cut`` with flags bit 1): c = -0.0 exactly marks an edge outside the envelope's support, where the
    envelope's derivative is zero (padding edges, edges past r_max).  There W = 0, so ∂/∂W0 = gW·c, gY and the dX
    message are zero, and ∂/∂c is multiplied by a zero derivative wherever it goes: the kernel writes zero ∂/∂W0,
    gY and ∂/∂c rows for such an edge without reading W0 or x, writes no dX message (``conv_gxsum`` skips the edge
    too), and walks only the other edges of each chunk (compacted by lane rank, as in ``conv_fwdc``).  With flags
    bit 2 as well the zero ∂/∂W0 rows are not written either: for a caller whose only consumer of ∂/∂W0 (the radial
    MLP's backward) skips the masked rows itself."""
    spec, nx, nk = G.s, G.nx, G.s.nins
    atomic = GY_LDS_ATOMIC and spec.ncb == 2
    if atomic:
        gyr = gy_reduce('      ', spec.y_dim, spec.y_pad, atomic=True)
    L = [
        f'extern "C" __global__ __launch_bounds__(BLOCK) void {spec.kname("conv_bwdrc" if cut else "conv_bwdr")}(',
        '    const float* __restrict__ x, const float* __restrict__ g, const float* __restrict__ Y,',
        '    const float* __restrict__ W, const int* __restrict__ rowptr, const int* __restrict__ eids,',
        '    const int* __restrict__ senders, float* __restrict__ gW, float* __restrict__ gY,',
        '    float* __restrict__ gxm, int N, int flags' +
        (', const float* __restrict__ cutv, float* __restrict__ gcut, const int* __restrict__ wrow) {'
         if cut else ') {'),
        '  __shared__ float part[CHUNK][Y_PAD];' if atomic else '  __shared__ float part[NCB][CHUNK][Y_PAD];',
    ] + ((['  __shared__ float partc[CHUNK];'] if atomic else ['  __shared__ float partc[NCB][CHUNK];']) +
         ['  __shared__ int sidx[NCB][CHUNK];'] if cut else []) + [
        '  __shared__ float4 Ms4[CHUNK][NPP / 4];',
        '  float (*Ms)[NPP] = reinterpret_cast<float (*)[NPP]>(Ms4);',
        '  const int r = mh_xcd_block(blockIdx.x, gridDim.x);',
        '  if (r >= N) return;',
    ] + ([
        '  for (int q = threadIdx.x; q < CHUNK * Y_PAD; q += BLOCK) (&part[0][0])[q] = 0.0f;',
    ] + (['  for (int q = threadIdx.x; q < CHUNK; q += BLOCK) partc[q] = 0.0f;'] if cut else []) + [
        '  __syncthreads();',
    ] if atomic else []) + G.prelude() + [
        '  const bool GX = (flags & 1) != 0;',
    ] + (['  const bool MASKED = (flags & 2) != 0;',
          '  const bool ZROWS = (flags & 4) == 0;     // write the zero gW rows of masked edges'] if cut else []) + [
        '  ' + decl('gv', G.no),
    ]
    L += G.ld_g('  ', 'r', 'gv')
    L += ['  ' + decl('xn', nx), '  ' + decl('wn', nk)]
    if BWD_PREFETCH > 1:
        L += ['  ' + decl('xm', nx), '  ' + decl('wm', nk)]
    L += ['  const int p0 = rowptr[r], p1 = rowptr[r + 1];']

    def chunks(msg):
        C = ['  for (int pb = p0; pb < p1; pb += CHUNK) {']
        if cut:
            # every wave reads the same edges and cutoffs, so ballots, counts and the `continue` are uniform over
            # the workgroup and the barriers below stay matched
            C += ['    const int cnt0 = min(CHUNK, p1 - pb);',
                  '    int my_e = 0, my_s = 0;',
                  '    bool keep = false;',
                  '    if (lane < cnt0) {',
                  '      my_e = eids[pb + lane];',
                  '      keep = !(MASKED && __float_as_uint(cutv[my_e]) == 0x80000000u);',
                  '    }',
                  '    const unsigned long long kept = __ballot(keep);',
                  '    const unsigned long long drop = __ballot(lane < cnt0 && !keep);',
                  '    const int cnt = __popcll(kept);',
                  '    if (keep) sidx[wave][__popcll(kept & ((1ull << lane) - 1ull))] = my_e;',
                  '    for (unsigned long long d = drop; d; d &= d - 1ull) {',
                  '      const int ez = mh_bcast(my_e, __builtin_ctzll(d));',
                  '      float* __restrict__ gz = gW + (size_t)ez * NW;']
            st = [f'mh_st_nt(gz + {k * spec.mul}, ol1, 0.0f);' for k in range(nk)]
            C += ['      if (ZROWS) {'] + [f'        {t}' if G.full else f'        if (active) {t}' for t in st] + ['      }']
            C += ['      if (wave == 0) {',
                  '        if (lane < Y_DIM) gY[(size_t)ez * Y_DIM + lane] = 0.0f;',
                  '        if (lane == 0) gcut[ez] = 0.0f;',
                  '      }',
                  '    }',
                  '    if (cnt == 0) continue;',
                  '    my_e = 0;',
                  '    float my_c = 0.0f;                  // the cutoff of lane j\'s edge, broadcast per edge below',
                  '    int my_w = 0;                       // the W0 row of lane j\'s edge (its own, or wrow[e])',
                  '    if (lane < cnt) {',
                  '      my_e = sidx[wave][lane]; my_s = senders[my_e]; my_c = cutv[my_e];',
                  '      my_w = wrow ? wrow[my_e] : my_e;',
                  '    }']
        else:
            C += ['    const int cnt = min(CHUNK, p1 - pb);',
                  '    int my_e = 0, my_s = 0;',
                  '    if (lane < cnt) { my_e = eids[pb + lane]; my_s = senders[my_e]; }',
                  '    const int my_w = my_e;']
        C += G.m_prologue('    ', 'my_e')
        C += ['    {', '      const int er0 = mh_bcast(my_w, 0), s0 = mh_bcast(my_s, 0);']
        C += G.ld_x('      ', 's0', 'xn') + G.ld_w('      ', 'er0', 'wn', W_NT_BWD)
        C += ['    }']
        if BWD_PREFETCH > 1:          # edge 1 (or the last edge again) one stage further out
            C += ['    {', '      const int er1 = mh_bcast(my_w, min(1, cnt - 1)), s1 = mh_bcast(my_s, min(1, cnt - 1));']
            C += G.ld_x('      ', 's1', 'xm') + G.ld_w('      ', 'er1', 'wm', W_NT_BWD)
            C += ['    }']
        C += ['    for (int j = 0; j < cnt; ++j) {', '      const int e = mh_bcast(my_e, j);']
        C += copy('xv', 'xn', nx)
        if cut:
            C += ['      const float ce = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_c), j));'
                  if BWD_CUT_BCAST else '      const float ce = cutv[e];']
            C += copy('w0', 'wn', nk)
            C += [f'      const float w{k} = w0{k} * ce;' for k in range(nk)]
            C += ['      float Pc = 0.0f;']
        else:
            C += copy('w', 'wn', nk)
        if BWD_PREFETCH > 1:
            C += [f'      xn{i} = xm{i};' for i in range(nx)] + [f'      wn{k} = wm{k};' for k in range(nk)]
            C += ['      {', '        const int j2 = min(j + 2, cnt - 1);',
                  '        const int er2 = mh_bcast(my_w, j2), s2 = mh_bcast(my_s, j2);']
            C += G.ld_x('        ', 's2', 'xm') + G.ld_w('        ', 'er2', 'wm', W_NT_BWD)
            C += ['      }']
        else:
            C += ['      {', '        const int j1 = min(j + 1, cnt - 1);',
                  '        const int er1 = mh_bcast(my_w, j1), s1 = mh_bcast(my_s, j1);']
            C += G.ld_x('        ', 's1', 'xn') + G.ld_w('        ', 'er1', 'wn', W_NT_BWD)
            C += ['      }']
        C += [f'      {pdecl}', '      float* __restrict__ gwe = gW + (size_t)e * NW;']
        if msg:
            C += ['      ' + decl('gxa', nx, '0.0f')]
        C += G.bwd_body('      ', with_gx=msg, use_m=True, store=True, cut=cut)
        if msg:
            C += ['      {', '        float* __restrict__ gme = gxm + (size_t)e * X_DIM;']
            for b, (l, _, off) in enumerate(spec.in1):
                d = 2 * l + 1
                st = [f'mh_st(gme + {off + m}, ol{d}, gxa{G.xi[b] + m});' for m in range(d)]
                C += [f'        {t}' if G.full else f'        if (active) {t}' for t in st]
            C += ['      }']
        C += gyr
        if cut:
            # all-reduce over the wave (every lane ends with the sum), lane 0 keeps the wave's partial
            C += [f'      Pc += {_xchg("Pc", bit)};' for bit in range(5, -1, -1)]
            C += ['      if (lane == 0) atomicAdd(&partc[j], Pc);' if atomic else '      if (lane == 0) partc[wave][j] = Pc;']
        C += ['    }']
        C += _gy_combine('    ', 'sidx[0][j]' if cut else 'eids[pb + j]', cut=cut, atomic=atomic)
        return C + ['  }']

    L += ['  if (GX) {'] + ['  ' + t for t in chunks(True)] + ['  } else {']
    L += ['  ' + t for t in chunks(False)] + ['  }', '}', '']
    return L


GX_LIST = 256             # edges of a sender up to which conv_gxsum lists its unmasked edges in LDS first


def gxsum_block(spec):
    """Threads of the dX-message reduction: one float4 column each, rounded up to whole waves."""
    return (spec.x_dim // 4 + WAVE - 1) // WAVE * WAVE


def _gx_sum(spec):
    """gx[s] = Σ_{e ∈ CSR_send(s)} gxm[e], summed in CSR order (deterministic); one float4 column per thread.
    ``mask`` non-NULL: edges whose mask value is -0.0 exactly have no message (``conv_bwdrc`` with masked edges
    writes none; it would be zero) and are left out, which leaves every sum unchanged.  For a sender of at most
    GX_LIST edges the first wave lists its unmasked edges in LDS (CSR order: a ballot prefix per 64 edges) after one
    round of id and mask loads, and the sum then loads only their rows (the padding edges' unset rows, about a fifth
    of config 2's, are not read).  A longer segment loads each row alongside its mask and drops masked ones by a
    select (waiting for the mask before each row load would add a dependent round trip per group of four edges).
    Skipping a masked edge and adding 0.0 for it give the same sum: the sum starts at +0.0 and never becomes -0.0."""
    assert spec.x_dim % 4 == 0
    return [
        f'#define GX_LIST {GX_LIST}',
        f'extern "C" __global__ __launch_bounds__({gxsum_block(spec)}) void {spec.kname("conv_gxsum")}(',
        '    const float* __restrict__ gxm, const int* __restrict__ rowptr, const int* __restrict__ eids,',
        '    float* __restrict__ gx, int N, const float* __restrict__ mask) {',
        '  __shared__ int live[GX_LIST];              // the sender\'s unmasked edges, CSR order',
        '  __shared__ int nlive;',
        '  const int s = mh_xcd_block(blockIdx.x, gridDim.x);',
        '  const int t = threadIdx.x;',
        '  if (s >= N) return;                        // (whole workgroup: s is uniform)',
        '  const int p0 = rowptr[s], p1 = rowptr[s + 1];',
        '  if (mask && p1 - p0 <= GX_LIST) {',
        '    if (t < 64) {',
        '      int base = 0;',
        '      for (int q = p0; q < p1; q += 64) {',
        '        const int pp = q + t;',
        '        int e = 0;',
        '        bool k = false;',
        '        if (pp < p1) { e = eids[pp]; k = __float_as_uint(mask[e]) != 0x80000000u; }',
        '        const unsigned long long b = __ballot(k);',
        '        if (k) live[base + __popcll(b & ((1ull << t) - 1ull))] = e;',
        '        base += __popcll(b);',
        '      }',
        '      if (t == 0) nlive = base;',
        '    }',
        '    __syncthreads();',
        '    if (t >= X_DIM / 4) return;',
        '    const float4* __restrict__ src = reinterpret_cast<const float4*>(gxm) + t;',
        '    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);',
        '    const int n = nlive;',
        '    int i = 0;',
        '    for (; i + 4 <= n; i += 4) {',
        '      const int e0 = live[i], e1 = live[i + 1], e2 = live[i + 2], e3 = live[i + 3];',
        '      const float4 v0 = src[(size_t)e0 * (X_DIM / 4)], v1 = src[(size_t)e1 * (X_DIM / 4)];',
        '      const float4 v2 = src[(size_t)e2 * (X_DIM / 4)], v3 = src[(size_t)e3 * (X_DIM / 4)];',
        '      acc.x += v0.x; acc.y += v0.y; acc.z += v0.z; acc.w += v0.w;',
        '      acc.x += v1.x; acc.y += v1.y; acc.z += v1.z; acc.w += v1.w;',
        '      acc.x += v2.x; acc.y += v2.y; acc.z += v2.z; acc.w += v2.w;',
        '      acc.x += v3.x; acc.y += v3.y; acc.z += v3.z; acc.w += v3.w;',
        '    }',
        '    for (; i < n; ++i) {',
        '      const float4 v = src[(size_t)live[i] * (X_DIM / 4)];',
        '      acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;',
        '    }',
        '    reinterpret_cast<float4*>(gx)[(size_t)s * (X_DIM / 4) + t] = acc;',
        '    return;',
        '  }',
        '  if (t >= X_DIM / 4) return;',
        '  const float4* __restrict__ src = reinterpret_cast<const float4*>(gxm) + t;',
        '  const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);',
        '  float4 acc = z;',
        '  int p = p0;',
        '  if (mask) {',
        '    for (; p + 4 <= p1; p += 4) {',
        '      const int e0 = eids[p], e1 = eids[p + 1], e2 = eids[p + 2], e3 = eids[p + 3];',
        '      const float4 v0 = src[(size_t)e0 * (X_DIM / 4)], v1 = src[(size_t)e1 * (X_DIM / 4)];',
        '      const float4 v2 = src[(size_t)e2 * (X_DIM / 4)], v3 = src[(size_t)e3 * (X_DIM / 4)];',
        '      const bool k0 = __float_as_uint(mask[e0]) != 0x80000000u, k1 = __float_as_uint(mask[e1]) != 0x80000000u;',
        '      const bool k2 = __float_as_uint(mask[e2]) != 0x80000000u, k3 = __float_as_uint(mask[e3]) != 0x80000000u;',
        '      acc.x += k0 ? v0.x : 0.0f; acc.y += k0 ? v0.y : 0.0f; acc.z += k0 ? v0.z : 0.0f; acc.w += k0 ? v0.w : 0.0f;',
        '      acc.x += k1 ? v1.x : 0.0f; acc.y += k1 ? v1.y : 0.0f; acc.z += k1 ? v1.z : 0.0f; acc.w += k1 ? v1.w : 0.0f;',
        '      acc.x += k2 ? v2.x : 0.0f; acc.y += k2 ? v2.y : 0.0f; acc.z += k2 ? v2.z : 0.0f; acc.w += k2 ? v2.w : 0.0f;',
        '      acc.x += k3 ? v3.x : 0.0f; acc.y += k3 ? v3.y : 0.0f; acc.z += k3 ? v3.z : 0.0f; acc.w += k3 ? v3.w : 0.0f;',
        '    }',
        '    for (; p < p1; ++p) {',
        '      const int e = eids[p];',
        '      const float4 v = src[(size_t)e * (X_DIM / 4)];',
        '      const bool k = __float_as_uint(mask[e]) != 0x80000000u;',
        '      acc.x += k ? v.x : 0.0f; acc.y += k ? v.y : 0.0f; acc.z += k ? v.z : 0.0f; acc.w += k ? v.w : 0.0f;',
        '    }',
        '  } else {',
        '    for (; p + 4 <= p1; p += 4) {',
        '      const int e0 = eids[p], e1 = eids[p + 1], e2 = eids[p + 2], e3 = eids[p + 3];',
        '      const float4 v0 = src[(size_t)e0 * (X_DIM / 4)], v1 = src[(size_t)e1 * (X_DIM / 4)];',
        '      const float4 v2 = src[(size_t)e2 * (X_DIM / 4)], v3 = src[(size_t)e3 * (X_DIM / 4)];',
        '      acc.x += v0.x; acc.y += v0.y; acc.z += v0.z; acc.w += v0.w;',
        '      acc.x += v1.x; acc.y += v1.y; acc.z += v1.z; acc.w += v1.w;',
        '      acc.x += v2.x; acc.y += v2.y; acc.z += v2.z; acc.w += v2.w;',
        '      acc.x += v3.x; acc.y += v3.y; acc.z += v3.z; acc.w += v3.w;',
        '    }',
        '    for (; p < p1; ++p) {',
        '      const float4 v = src[(size_t)eids[p] * (X_DIM / 4)];',
        '      acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;',
        '    }',
        '  }',
        '  reinterpret_cast<float4*>(gx)[(size_t)s * (X_DIM / 4) + t] = acc;',
        '}', '',
    ]

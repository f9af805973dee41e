"""
The interaction convolution with the radial MLP's output layer inside it: the per-edge weights are produced and
consumed in the kernels, never stored.

MACE forms the convolution's weights as ``tp_weights = conv_tp_weights(edge_feats) * cutoff``, whose last layer is a
linear map A [HL, NINS·MUL] from the HL (= 64) last hidden activations h[e] of an edge:
    W[e, k·MUL + u] = c_e · Σ_j h[e, j] A[j, k·MUL + u].
The reference streams W [E, NINS·MUL] through its kernels (read at conv.py:127, gradient written at :203-209); that
tensor is 491 MB for config 2's layer 2, read by the forward and backward and written by the MLP, with its gradient
written by the backward and read by the MLP's backward.  Here the convolution reads h [E, HL] (64 floats per edge
instead of 1,280) and forms W on the matrix cores, and the backward contracts its gradient with Aᵀ before anything
leaves the kernel, so only ∂(c·h) [E, HL] does.

Numerics: every product h·A runs at fp32 accuracy on the bf16 units (v_mfma_f32_16x16x32_bf16): c·h and A are each
split exactly into three bf16 parts and the six leading partial products are summed (mh_split8), as the radial MLP
kernels do.

Forward (``conv_fwdm``).  The MFMA computing D[edge][channel] = (c·h)[edge, :] · A[:, channel] for a tile of 16 edges
and 16 channels leaves lane l holding channel l % 16 for edges 4q .. 4q+3 (q = l / 16): the convolution's
channel-wise arithmetic then runs in exactly that layout, each lane accumulating its channel's output over its
four edges, and the four lane groups are summed at the end of the receiver (two butterfly steps, fixed order).
A workgroup serves one 16-channel tile for 24 receivers (2 per wave); A's slice for that tile, in the three bf16 parts
and the operand layout, is staged in LDS once per workgroup.  The operand c·h arrives from the radial MLP's
hidden-layer kernel already split into its bf16 parts, in the K order its own MFMAs left it in (A's rows are packed
in that order), so the convolution loads it as it is.  Edges whose cutoff is exactly zero
(padding, neighbour-list entries past r_max) contribute exactly zero and are dropped before any work (ballot
compaction per chunk of 64).  Per edge tile the edge-uniform coupling products M_k[a, c] = Σ_b C_k[a, b, c] Y[e, b]
are formed once into LDS.  Results do not depend on scheduling: every sum runs in a fixed order.
"""
import numpy as np
import torch

from . import _native
from .conv_codegen import _Gen, _gx_sum, _lit, _sum, gxsum_block
from .pending import Pending
from .radial import bf16_split3

CT = 16                 # channels per channel tile (the MFMA tile's width)
NWF = 12                # waves per forward workgroup
RPW = 2                 # receivers per wave (forward)
FWD_WAVES_PER_SIMD = 3  # occupancy the forward's register allocation targets (0: the compiler's choice)
BWD_PREFETCH_G = True   # backward: load the receiver's g rows for the next instruction before this one's arithmetic
PAIRS = [(0, 0), (0, 1), (1, 0), (0, 2), (1, 1), (2, 0)]   # bf16 parts (A operand, B operand) of the six products


def fused_supported(cspec, mspec):
    """(ok, reason): whether a convolution (ConvSpec) and the radial MLP feeding it (radial.MLPSpec) can run fused."""
    if cspec.mul % CT:
        return False, f'multiplicity {cspec.mul} is not a multiple of {CT}'
    if mspec.hs[-1] != cspec.nins * cspec.mul:
        return False, f'MLP output width {mspec.hs[-1]} != {cspec.nins} x {cspec.mul} weights'
    if mspec.hs[-2] % 32:
        return False, f'last hidden width {mspec.hs[-2]} is not a multiple of 32'
    if lds_bytes_bwd(cspec, mspec) > LDS_BYTES:
        return False, f'{cspec.nins} instructions: the output layer slices exceed the LDS'
    return True, ''


LDS_BYTES = 160 * 1024


def lds_bytes_bwd(cspec, mspec):
    """LDS of the fused backward: both layouts of a channel tile's slice of the output layer."""
    hl, nk = mspec.hs[-2], cspec.nins
    return nk * (hl // 32) * 3 * 1024 + (nk + 1) // 2 * 3 * (hl // 16) * 1024


class FusedSpec:
    """Layout constants of one fused convolution: instruction groups, channel tiles, the packed output layer."""

    def __init__(self, cspec, mspec):
        ok, why = fused_supported(cspec, mspec)
        if not ok:
            raise ValueError(why)
        self.c, self.m = cspec, mspec
        self.HL = mspec.hs[-2]
        self.S = self.HL // 32                           # K steps of 32 per W product
        self.nct = cspec.mul // CT
        by_block = {}
        for co in cspec.coef:
            by_block.setdefault(cspec.ins[co['k']][0], []).append(co['k'])
        self.groups = [by_block[b] for b in sorted(by_block)]
        self.korder = [k for g in self.groups for k in g]     # instruction order of the packed weights
        self.goff = np.cumsum([0] + [len(g) for g in self.groups]).tolist()

    def kname(self, base):
        return f'{base}_x{self.c.x_dim}_o{self.c.out_dim}_h{self.HL}'

    def pack_fwd(self):
        """Output layer A [HL, NINS·MUL] as the forward's B operand / the backward's first A operand: per channel
        tile ct, instruction k (in ``korder``), K step s and bf16 part p a 64-lane block where lane l = 16 q + i16
        holds A[kfeat(s, q, t), k·MUL + 16 ct + i16] for t = 0..7: [ct][k][s][p][64][8] uint16.  K position
        8 q + t of step s is hidden feature kfeat = 32 s + 16 (t / 4) + 4 q + t % 4, the order in which the radial
        MLP's last MFMA leaves a lane's activations (mlp_hid writes c h in it)."""
        A = np.asarray(self.m.A[-1], dtype=np.float64)
        parts = bf16_split3(A.astype(np.float32))                       # 3 x [HL, NW]
        mul = self.c.mul
        out = np.zeros((self.nct, len(self.korder), self.S, 3, 64, 8), dtype=np.uint16)
        for ct in range(self.nct):
            for ki, k in enumerate(self.korder):
                for s in range(self.S):
                    for q in range(4):
                        rows = kfeat(s, q)
                        cols = k * mul + CT * ct + np.arange(16)
                        for p in range(3):
                            out[ct, ki, s, p, 16 * q:16 * q + 16, :] = parts[p][np.ix_(rows, cols)].T
        return out.reshape(-1)


def kfeat(s, q):
    """Hidden features at K positions 8 q .. 8 q + 7 of K step s (see FusedSpec.pack_fwd)."""
    t = np.arange(8)
    return 32 * s + 16 * (t // 4) + 4 * q + t % 4


def _wave_sync():
    return ['__builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");', '__builtin_amdgcn_wave_barrier();',
            '__builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");']


def _group_pairs(G, grp):
    """Coupling pairs (k, a, c, [(b, v)]) of the instructions in grp, numbered within the group."""
    out, idx = [], {}
    for (co, a, c, bv) in G.pairs:
        if co['k'] in grp:
            idx[(co['k'], a, c)] = len(out)
            out.append((co, a, c, bv))
    return out, idx


def _row_stride(npp):
    """Coupling-table row stride (floats) with stride = 8 mod 32: the four lane groups' rows (4 apart after the
    slot permutation, i.e. consecutive) then fall on disjoint bank quads."""
    return npp + (8 - npp) % 32


def fwd_source(fs, header=True):
    """HIP source of ``conv_fwdm`` for one fused spec."""
    s = fs.c
    G = _Gen(s)
    S = fs.S
    nk = len(fs.korder)
    coefs = {co['k']: co for co in s.coef}
    pairs, pidx = _group_pairs(G, fs.korder)
    npp = max(4, (len(pairs) + 3) // 4 * 4)
    R = _row_stride(npp)
    oi, no = {}, 0
    for k in fs.korder:
        oi[k] = no
        no += coefs[k]['d3']
    lb = f'NWF * 64, {FWD_WAVES_PER_SIMD}' if FWD_WAVES_PER_SIMD else 'NWF * 64'
    L = [_native.device_header() if header else '',
         f'#define MUL {s.mul}', f'#define NCT {fs.nct}', f'#define X_DIM {s.x_dim}', f'#define Y_DIM {s.y_dim}',
         f'#define OUT_DIM {s.out_dim}', f'#define NWF {NWF}', f'#define RPW {RPW}', '',
         f'extern "C" __global__ __launch_bounds__({lb}) void {fs.kname("conv_fwdm")}(',
         '    const float* __restrict__ x, const float* __restrict__ Y, const unsigned short* __restrict__ hc,',
         '    const float* __restrict__ cutv, const int* __restrict__ rowptr, const int* __restrict__ eids,',
         '    const int* __restrict__ senders, const unsigned short* __restrict__ Wf, float* __restrict__ out,',
         '    int N) {',
         f'  __shared__ __align__(16) unsigned short wl[{nk * S * 3 * 512}];',
         f'  __shared__ __align__(16) float Msf[NWF][{16 * R}];',
         '  __shared__ int le[NWF][MH_WAVE], ls[NWF][MH_WAVE];',
         '  __shared__ float lc[NWF][MH_WAVE];',
         '  const int bid = blockIdx.x, ct = bid % NCT, rg = bid / NCT;',
         '  const int t = threadIdx.x, wave = t >> 6, lane = t & 63, q = lane >> 4, c16 = lane & 15;',
         '  const int u = ct * 16 + c16;                 // this lane\'s channel',
         '  float* __restrict__ ms = Msf[wave];',
         '  int* __restrict__ mye = le[wave];',
         '  int* __restrict__ mys = ls[wave];',
         '  float* __restrict__ myc = lc[wave];',
         f'  {{ const mh_u4* __restrict__ src = reinterpret_cast<const mh_u4*>(Wf) + (size_t)ct * {nk * S * 3 * 64};',
         f'    for (int i = t; i < {nk * S * 3 * 64}; i += NWF * 64) reinterpret_cast<mh_u4*>(wl)[i] = src[i]; }}',
         '  __syncthreads();',
         '  const mh_bf8 zero8 = __builtin_bit_cast(mh_bf8, mh_u4{0u, 0u, 0u, 0u});',
         '  for (int ri = 0; ri < RPW; ++ri) {',
         '    const int r = (rg * RPW + ri) * NWF + wave;',
         '    if (r >= N) break;',
         '    ' + 'float ' + ', '.join(f'acc{o} = 0.0f' for o in range(no)) + ';',
         '    const int p0 = rowptr[r], p1 = rowptr[r + 1];',
         '    for (int pb = p0; pb < p1; pb += MH_WAVE) {',
         '      const int cnt0 = min(MH_WAVE, p1 - pb);',
         '      int my_e = 0;',
         '      float my_c = 0.0f;',
         '      if (lane < cnt0) { my_e = eids[pb + lane]; my_c = cutv[my_e]; }',
         '      const bool keep = my_c != 0.0f;',
         '      const unsigned long long kept = __ballot(keep);',
         '      const int cnt = __popcll(kept);',
         '      if (keep) {',
         '        const int slot = __popcll(kept & ((1ull << lane) - 1ull));',
         '        mye[slot] = my_e; mys[slot] = senders[my_e]; myc[slot] = my_c;',
         '      }']
    L += ['      ' + x for x in _wave_sync()]
    L += ['      for (int tb = 0; tb < cnt; tb += 16) {',
          '        // A operand: c h of edge slot tb + c16 (mlp_hid\'s pre-split parts), zero rows past the list',
          '        const int sa = min(tb + c16, cnt - 1);',
          '        const bool va = tb + c16 < cnt;',
          '        const int ea = mye[sa];',
          f'        mh_bf8 ha[{S}][3];',
          f'        {{ const mh_bf8* __restrict__ hr = reinterpret_cast<const mh_bf8*>(hc) + (size_t)ea * {S * 12} + q;']
    for st in range(S):
        L += [f'          ha[{st}][{p}] = va ? hr[{st * 12 + 4 * p}] : zero8;' for p in range(3)]
    L += ['        }']
    # coupling products of slot tb + c16, stored at row (c16 % 4) * 4 + c16 / 4: a lane group's four slots then sit
    # on consecutive rows
    ys = sorted({co['o2'] + bb for (co, a, c, bv) in pairs for bb, _ in bv})
    L += ['        if (q == 0) {',
          '          const float* __restrict__ yl = Y + (size_t)ea * Y_DIM;',
          f'          float* __restrict__ mrow = ms + ((c16 & 3) * 4 + (c16 >> 2)) * {R};']
    L += [f'          const float y{j} = yl[{j}];' for j in ys]
    for p, (co, a, c, bv) in enumerate(pairs):
        val = _sum([f'{_lit(v)} * y{co["o2"] + bb}' for bb, v in bv])
        L.append(f'          mrow[{p}] = {val};')
    L += ['        }']
    L += ['        ' + x for x in _wave_sync()]

    def wprod(ki, dst):
        P = [f'        mh_f4 {dst} = mh_f4{{0.0f, 0.0f, 0.0f, 0.0f}};']
        for st in range(S):
            P += [f'        {{ const mh_bf8* __restrict__ wb = reinterpret_cast<const mh_bf8*>(wl) + '
                  f'{(ki * S + st) * 3 * 64} + lane;',
                  '          const mh_bf8 bb[3] = {wb[0], wb[64], wb[128]};']
            P += [f'          {dst} = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ha[{st}][{pa}], bb[{pb_}], {dst}, 0, 0, 0);'
                  for pa, pb_ in PAIRS]
            P += ['        }']
        return P

    # the W product of instruction i + 1 is issued before instruction i's arithmetic (the matrix cores run it
    # while the VALU works on the previous result)
    L += wprod(0, 'wn0')
    first = {}
    for ki, k in enumerate(fs.korder):
        first.setdefault(s.ins[k][0], ki)
    for ki, k in enumerate(fs.korder):
        co = coefs[k]
        b = s.ins[k][0]
        l_b, _, off_b = s.in1[b]
        d = 2 * l_b + 1
        if first[b] == ki:
            # x of the lane's four output edges (slots tb + 4 q + rr), channel u of block b
            L += ['        float ' + ', '.join(f'xv{b}_{rr}_{m}' for rr in range(4) for m in range(d)) + ';']
            for rr in range(4):
                L += [f'        {{ const float* __restrict__ xs = x + (size_t)mys[min(tb + 4 * q + {rr}, cnt - 1)] * '
                      f'X_DIM + {off_b} + u * {d};']
                L += [f'          xv{b}_{rr}_{m} = xs[{m}];' for m in range(d)]
                L += ['        }']
        L += ['        asm volatile("" ::: "memory");     // this instruction\'s LDS reads stay here']
        if ki + 1 < nk:
            L += wprod(ki + 1, f'wn{ki + 1}')
        L += ['        {', f'        const mh_f4 w = wn{ki};        // W[slot tb + 4 q + rr][channel u]']
        qs = sorted({pidx[(k, a, c)] // 4 for (co2, a, c, bv) in pairs if co2['k'] == k})
        for rr in range(4):
            L += [f'        {{ const mh_f4* __restrict__ mr = reinterpret_cast<const mh_f4*>(ms + ({rr * 4} + q) * {R});']
            L += [f'          const mh_f4 mq{qq} = mr[{qq}];' for qq in qs]
            for c in range(co['d3']):
                ts = [f'xv{b}_{rr}_{a} * mq{pidx[(k, a, c)] // 4}[{pidx[(k, a, c)] % 4}]' for a in range(co['d1'])
                      if (k, a, c) in pidx]
                if ts:
                    o = oi[k] + c
                    L.append(f'          acc{o} = fmaf(w[{rr}], {_sum(ts)}, acc{o});')
            L += ['        }']
        L += ['        }']
    L += ['        ' + x for x in _wave_sync()]
    L += ['      }', '    }']
    # sum the four lane groups (each saw a quarter of the edges), then q == 0 lanes store
    for o in range(no):
        L += [f'    acc{o} += __shfl_xor(acc{o}, 16, MH_WAVE);', f'    acc{o} += __shfl_xor(acc{o}, 32, MH_WAVE);']
    L += ['    if (q == 0) {', '      float* __restrict__ orow = out + (size_t)r * OUT_DIM;']
    for k in fs.korder:
        co = coefs[k]
        for c in range(co['d3']):
            L.append(f'      orow[{co["o3"] + c} + u * {co["d3"]}] = acc{oi[k] + c};')
    L += ['    }', '  }', '}', '']
    return '\n'.join(L)


NWB = 8                 # waves per backward workgroup


def pack_bwd(fs):
    """Output layer A [HL, NINS·MUL] as the backward's second A operand (dL/d(c h)^T = A gW^T, K = instruction pair
    and channel): per channel tile ct, instruction pair kp (``korder`` positions 2 kp, 2 kp + 1; a missing second
    one is zero), bf16 part p and row tile m (rows j = 16 m .. 16 m + 15) a 64-lane block where lane l = 16 q + i16
    holds A[16 m + i16, k_t·MUL + 16 ct + 4 q + rr] at position 4 t + rr (t = 0, 1; rr = 0..3):
    [ct][kp][p][HL / 16][64][8] uint16."""
    A = np.asarray(fs.m.A[-1], dtype=np.float64)
    parts = bf16_split3(A.astype(np.float32))
    mul, HL = fs.c.mul, fs.HL
    nkp = (len(fs.korder) + 1) // 2
    out = np.zeros((fs.nct, nkp, 3, HL // 16, 64, 8), dtype=np.uint16)
    for ct in range(fs.nct):
        for kp in range(nkp):
            for t in range(2):
                ki = 2 * kp + t
                if ki >= len(fs.korder):
                    continue
                k = fs.korder[ki]
                for m in range(HL // 16):
                    for q in range(4):
                        rows = 16 * m + np.arange(16)
                        cols = k * mul + CT * ct + 4 * q + np.arange(4)
                        for p in range(3):
                            out[ct, kp, p, m, 16 * q:16 * q + 16, 4 * t:4 * t + 4] = parts[p][np.ix_(rows, cols)]
    return out.reshape(-1)


def bwd_source(fs, header=True):
    """HIP source of ``conv_bwdm`` (and ``conv_gysum``) for one fused spec."""
    s = fs.c
    G = _Gen(s)
    S, HL = fs.S, fs.HL
    NT = HL // 16                                      # row tiles of the second product
    nk = len(fs.korder)
    nkp = (nk + 1) // 2
    coefs = {co['k']: co for co in s.coef}
    wf_elems = nk * S * 3 * 512
    wb_elems = nkp * 3 * NT * 512
    L = [_native.device_header() if header else '',
         f'#define MUL {s.mul}', f'#define NCT {fs.nct}', f'#define X_DIM {s.x_dim}', f'#define Y_DIM {s.y_dim}',
         f'#define OUT_DIM {s.out_dim}', f'#define HL {HL}', f'#define NWB {NWB}', '']
    L += [f'extern "C" __global__ __launch_bounds__(NWB * 64) void {fs.kname("conv_bwdm")}(',
          '    const float* __restrict__ x, const float* __restrict__ g, const float* __restrict__ Y,',
          '    const unsigned short* __restrict__ hc, const float* __restrict__ cutv, const int* __restrict__ eids,',
          '    const int* __restrict__ recv, const int* __restrict__ senders, const unsigned short* __restrict__ Wf,',
          '    const unsigned short* __restrict__ Wb, float* __restrict__ gxm, float* __restrict__ gyp,',
          '    float* __restrict__ ghp, int E, int flags, int ngrp) {',
          f'  __shared__ __align__(16) unsigned short wf[{wf_elems}];',
          f'  __shared__ __align__(16) unsigned short wb[{wb_elems}];',
          '  const int bid = blockIdx.x, ct = bid % NCT, gg = bid / NCT;',
          '  const int t = threadIdx.x, wave = t >> 6, lane = t & 63, q = lane >> 4, c16 = lane & 15;',
          '  const bool GX = (flags & 1) != 0;',
          '  const mh_bf8 zero8 = __builtin_bit_cast(mh_bf8, mh_u4{0u, 0u, 0u, 0u});',
          f'  {{ const mh_u4* __restrict__ src = reinterpret_cast<const mh_u4*>(Wf) + (size_t)ct * {nk * S * 3 * 64};',
          f'    for (int i = t; i < {nk * S * 3 * 64}; i += NWB * 64) reinterpret_cast<mh_u4*>(wf)[i] = src[i]; }}',
          f'  {{ const mh_u4* __restrict__ src = reinterpret_cast<const mh_u4*>(Wb) + (size_t)ct * {nkp * 3 * NT * 64};',
          f'    for (int i = t; i < {nkp * 3 * NT * 64}; i += NWB * 64) reinterpret_cast<mh_u4*>(wb)[i] = src[i]; }}',
          '  __syncthreads();',
          '  const int ntiles = (E + 15) >> 4;']

    def g_load(ki):
        co = coefs[fs.korder[ki]]
        d3 = co['d3']
        L = [f'    mh_f4 gk{ki}[{d3}];',
             f'    {{ const mh_f4* __restrict__ gq = reinterpret_cast<const mh_f4*>(gr + {co["o3"]} + '
             f'(16 * ct + 4 * q) * {d3});']
        L += [f'      gk{ki}[{i}] = gq[{i}];' for i in range(d3)]
        return L + ['    }']

    def wprod(ki):
        L = [f'    mh_f4 wn{ki} = mh_f4{{0.0f, 0.0f, 0.0f, 0.0f}};']
        for st in range(S):
            L += [f'    {{ const mh_bf8* __restrict__ wa = reinterpret_cast<const mh_bf8*>(wf) + {(ki * S + st) * 3 * 64} + lane;',
                  '      const mh_bf8 aa[3] = {wa[0], wa[64], wa[128]};']
            L += [f'      wn{ki} = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aa[{pa}], ha[{st}][{pb_}], wn{ki}, 0, 0, 0);'
                  for pa, pb_ in PAIRS]
            L += ['    }']
        return L

    def tile_loop(gxv):
        """The tile loop; gxv: with the dX messages (generated as its own loop, so that no branch on the flag sits
        inside the unrolled instruction blocks, which keeps every message register live across them)."""
        L = ['  for (int ti = gg * NWB + wave; ti < ntiles; ti += ngrp * NWB) {',
             '    const int p = ti * 16 + c16;',
             '    const bool live = p < E;',
             '    const int e = eids[live ? p : E - 1];',
             '    const int r = recv[e], sd = senders[e];']
        # B operand of the W product: c h of this lane's edge (mlp_hid's pre-split parts; zero for dead lanes)
        L += [f'    mh_bf8 ha[{S}][3];',
              f'    {{ const mh_bf8* __restrict__ hr = reinterpret_cast<const mh_bf8*>(hc) + (size_t)e * {S * 12} + q;']
        for st in range(S):
            L += [f'      ha[{st}][{p}] = live ? hr[{st * 12 + 4 * p}] : zero8;' for p in range(3)]
        L += ['    }']
        L += ['    const float* __restrict__ yr = Y + (size_t)e * Y_DIM;']
        xv = lambda b, d, rr, a: f'xb{b}[{(rr * d + a) // 4}][{(rr * d + a) % 4}]'   # noqa: E731
        gmv = lambda b, d, rr, a: f'gm{b}_{rr * d + a}'                              # noqa: E731
        L += ['    ' + 'float ' + ', '.join(f'P{j} = 0.0f' for j in range(s.y_dim)) + ';']
        L += [f'    mh_f4 D2[{NT}];'] + [f'    D2[{m}] = mh_f4{{0.0f, 0.0f, 0.0f, 0.0f}};' for m in range(NT)]
        L += ['    const float* __restrict__ gr = g + (size_t)r * OUT_DIM;',
              '    float gw0_0, gw0_1, gw0_2, gw0_3, gw1_0, gw1_1, gw1_2, gw1_3;     // gW of an instruction pair']
        first = {g[0]: b for b, g in zip(sorted({s.ins[k][0] for k in fs.korder}), fs.groups)}
        last = {g[-1]: b for b, g in zip(sorted({s.ins[k][0] for k in fs.korder}), fs.groups)}
        for ki, k in enumerate(fs.korder):
            co = coefs[k]
            b = s.ins[k][0]
            l1, _, off1 = s.in1[b]
            d1, d3 = co['d1'], co['d3']
            if k in first:
                # x of this group's input block: channels 16 ct + 4 q .. + 3, d1 consecutive floats each; the block's
                # dX messages accumulate over the group and are stored at its end
                L += ['    asm volatile("" ::: "memory");',
                      f'    mh_f4 xb{b}[{d1}];',
                      f'    {{ const mh_f4* __restrict__ xr = reinterpret_cast<const mh_f4*>(x + (size_t)sd * X_DIM + {off1} + '
                      f'(16 * ct + 4 * q) * {d1});']
                L += [f'      xb{b}[{i}] = xr[{i}];' for i in range(d1)]
                L += ['    }']
                if gxv:      # scalars: lane-wise updates of vector registers bloat the live ranges
                    L += ['    float ' + ', '.join(f'gm{b}_{i} = 0.0f' for i in range(4 * d1)) + ';']
            # compiler barrier: keeps each instruction's loads (g rows, LDS fragments) from being hoisted over the
            # earlier ones, which would hold every instruction's operands in registers at once.  The receiver's g rows
            # of this instruction (BWD_PREFETCH_G: of the next one) are loaded right after it
            L += ['    asm volatile("" ::: "memory");']
            if BWD_PREFETCH_G:
                if ki == 0:
                    L += g_load(0)
                if ki + 1 < nk:
                    L += g_load(ki + 1)
            else:
                L += g_load(ki)
            # the W product of the next instruction is issued before this one's arithmetic (the matrix cores run it
            # while the VALU works)
            if ki == 0:
                L += wprod(0)
            if ki + 1 < nk:
                L += wprod(ki + 1)
            L += ['    {',
                  f'      const mh_f4 w = wn{ki};      // W[e][k][16 ct + 4 q + rr], cutoff included']
            gv = lambda rr, c: f'gk{ki}[{(rr * d3 + c) // 4}][{(rr * d3 + c) % 4}]'   # noqa: E731
            # per channel: T[a][b] = sum_c C[a, b, c] g_c, then h_a = sum_b T[a][b] y_b and
            # P_b += w sum_a x_a T[a][b] (the harmonics block of this instruction read from L1)
            L += [f'      const float y{co["o2"] + bb} = yr[{co["o2"] + bb}];' for bb in range(co['d2'])]
            abs_ = {}
            for a_, bb, c, v in co['terms']:
                abs_.setdefault((a_, bb), []).append((c, v))
            for rr in range(4):
                # one channel at a time: without the barrier the scheduler interleaves the four channels' blocks and
                # keeps all their temporaries live
                L.append('      __builtin_amdgcn_sched_barrier(0);')
                L.append('      {')
                for (a_, bb), cv in sorted(abs_.items()):
                    val = _sum([f'{_lit(v)} * {gv(rr, c)}' for c, v in cv])
                    L.append(f'        const float T{a_}_{bb} = {val};')
                hs = []
                for a_ in range(d1):
                    ts = [f'T{a_}_{bb} * y{co["o2"] + bb}' for bb in range(co['d2']) if (a_, bb) in abs_]
                    if not ts:
                        continue
                    L.append(f'        const float h{a_} = {_sum(ts)};')
                    hs.append(a_)
                L.append(f'        gw{ki % 2}_{rr} = {_sum([f"{xv(b, d1, rr, a_)} * h{a_}" for a_ in hs])};')
                if gxv:
                    L += [f'        {gmv(b, d1, rr, a_)} = fmaf(w[{rr}], h{a_}, {gmv(b, d1, rr, a_)});' for a_ in hs]
                for bb in range(co['d2']):
                    ts = [f'{xv(b, d1, rr, a_)} * T{a_}_{bb}' for a_ in range(d1) if (a_, bb) in abs_]
                    if ts:
                        L.append(f'        P{co["o2"] + bb} = fmaf(w[{rr}], {_sum(ts)}, P{co["o2"] + bb});')
                # the accumulators as asm operands: their updates happen here, not sunk to the end of the tile with
                # every input kept live until then
                fence = [f'P{co["o2"] + bb}' for bb in range(co['d2'])] + [f'gw{ki % 2}_{rr}']
                if gxv:
                    fence += [gmv(b, d1, rr, a_) for a_ in hs]
                L.append('        asm volatile("" : ' + ', '.join(f'"+v"({v})' for v in fence) + ');')
                L.append('      }')
            L += ['    }']
            if k in last and gxv:
                L += ['    if (live) {',
                      f'      mh_f4* __restrict__ gq = reinterpret_cast<mh_f4*>(gxm + (size_t)e * X_DIM + {off1} + '
                      f'(16 * ct + 4 * q) * {d1});']
                L += [f'      gq[{i}] = mh_f4{{gm{b}_{4 * i}, gm{b}_{4 * i + 1}, gm{b}_{4 * i + 2}, gm{b}_{4 * i + 3}}};'
                      for i in range(d1)]
                L += ['    }']
            if ki % 2 == 1 or ki == nk - 1:
                kp = ki // 2
                second = [f'gw1_{rr}' for rr in range(4)] if ki % 2 == 1 else ['0.0f'] * 4
                L += ['    asm volatile("" ::: "memory");',
                      '    {',
                      f'      const float v[8] = {{gw0_0, gw0_1, gw0_2, gw0_3, {", ".join(second)}}};',
                      '      mh_bf8 gb[3];',
                      '      mh_split8(v, gb);']
                for m in range(NT):
                    L += [f'      {{ const mh_bf8* __restrict__ wa = reinterpret_cast<const mh_bf8*>(wb) + '
                          f'{(kp * 3 * NT + m) * 64} + lane;',
                          f'        const mh_bf8 a0 = wa[0], a1 = wa[{NT * 64}], a2 = wa[{2 * NT * 64}];',
                          '        const mh_bf8 aa[3] = {a0, a1, a2};']
                    L += [f'        D2[{m}] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aa[{pa}], gb[{pb_}], D2[{m}], 0, 0, 0);'
                          for pa, pb_ in PAIRS]
                    L += ['      }']
                L += ['    }']
        # sum P over the four lane groups (channels), store this tile's partials
        for j in range(s.y_dim):
            L += [f'    P{j} += __shfl_xor(P{j}, 16, MH_WAVE);', f'    P{j} += __shfl_xor(P{j}, 32, MH_WAVE);']
        yp = (s.y_dim + 3) // 4 * 4
        pz = lambda j: f'P{j}' if j < s.y_dim else '0.0f'              # noqa: E731
        L += ['    if (live) {',
              f'      float* __restrict__ gyr = gyp + ((size_t)ct * E + e) * {yp} + 4 * q;',
              '      mh_f4 pv = mh_f4{0.0f, 0.0f, 0.0f, 0.0f};']
        for qq in range(yp // 4):
            L += [f'      if (q == {qq}) pv = mh_f4{{{pz(4 * qq)}, {pz(4 * qq + 1)}, {pz(4 * qq + 2)}, {pz(4 * qq + 3)}}};']
        L += [f'      if (q < {yp // 4}) *reinterpret_cast<mh_f4*>(gyr) = pv;',
              '      float* __restrict__ ghr = ghp + ((size_t)ct * E + e) * HL + 4 * q;']
        L += [f'      *reinterpret_cast<mh_f4*>(ghr + {16 * m}) = D2[{m}];' for m in range(NT)]
        L += ['    }', '  }']
        return L

    yp = (s.y_dim + 3) // 4 * 4
    L += ['  if (GX) {'] + tile_loop(True) + ['  } else {'] + tile_loop(False) + ['  }', '}', '']
    # gY = sum of the channel tiles' partials, in tile order
    L += [f'extern "C" __global__ __launch_bounds__(256) void {fs.kname("conv_gysum")}(const float* __restrict__ gyp,',
          '    float* __restrict__ gY, int E) {',
          '  const long long e = (long long)blockIdx.x * 256 + threadIdx.x;',
          '  if (e >= E) return;',
          '  for (int b = 0; b < Y_DIM; ++b) {',
          f'    float v = gyp[e * {yp} + b];',
          f'    for (int c = 1; c < NCT; ++c) v += gyp[((size_t)c * E + e) * {yp} + b];',
          '    gY[e * Y_DIM + b] = v;',
          '  }',
          '}', '']
    return '\n'.join(L)


def source(fs):
    """The fused module: conv_fwdm, conv_bwdm, conv_gysum and a conv_gxsum for the dX messages."""
    return fwd_source(fs) + '\n' + bwd_source(fs, header=False) + '\n' + '\n'.join(_gx_sum(fs.c))


class FusedConv:
    """The compiled fused kernels of one (convolution, radial MLP) pair and the output layer packed for them."""

    def __init__(self, cspec, mspec, device):
        self.spec = FusedSpec(cspec, mspec)
        fs = self.spec
        self.source = source(fs)
        code = _native.compile_source(self.source)
        with torch.cuda.device(device):
            self.module = _native.Module(code, {
                _native.MH_CONV_FWD_M: (fs.kname('conv_fwdm'), NWF * 64, NWF * RPW, fs.nct),
                _native.MH_CONV_BWD_M: (fs.kname('conv_bwdm'), NWB * 64, NWB, fs.nct),
                _native.MH_CONV_GYSUM: (fs.kname('conv_gysum'), 256, 256),
                _native.MH_CONV_GXSUM: (cspec.kname('conv_gxsum'), gxsum_block(cspec), 1),
            })
        # bf16 parts as int16 bit patterns
        self.Wf = torch.from_numpy(fs.pack_fwd().view(np.int16)).to(device)
        self.Wb = torch.from_numpy(pack_bwd(fs).view(np.int16)).to(device)
        self.yp = (cspec.y_dim + 3) // 4 * 4


class PendingRadial(Pending):
    """The radial MLP's output W0 = MLP(edge_feats) [E, NINS·MUL] not yet formed, for a convolution that forms its
    weights itself: the product with MACE's [E, 1] cutoff column gives a ``FusedWeights``; any other use forms W0
    with the MLP's own kernels (an ordinary autograd-tracked tensor)."""

    def __init__(self, shape, like, ef, mlp):
        self.ef, self.mlp = ef, mlp

    def value(self):
        return _radial_fn().apply(self.ef, self.mlp)

    @classmethod
    def intercept(cls, func, args, kwargs):
        from .conv import _MULS
        if func in _MULS and len(args) == 2 and not kwargs:
            a, b = args
            if isinstance(b, PendingRadial) and not isinstance(a, Pending):
                a, b = b, a
            if (isinstance(a, PendingRadial) and torch.is_tensor(b) and not isinstance(b, Pending)
                    and tuple(b.shape) == (a.shape[0], 1) and b.dtype == torch.float32 and b.device == a.device):
                return FusedWeights(a.shape, a.ef, a.ef, b, a.mlp)
        return NotImplemented


class FusedWeights(Pending):
    """MACE's tp_weights = MLP(edge_feats) * cutoff, not formed: a convolution with the MLP's output layer attached
    (``HipConvTP.attach_mlp``) takes (edge_feats, cutoff) from it; any other use forms the product (W0 by the MLP's
    kernels times the cutoff, handed on unformed as the factored product the plain convolution kernels read)."""

    def __init__(self, shape, like, ef, cut, mlp):
        self.ef, self.cut, self.mlp = ef, cut, mlp

    def value(self):
        from .conv import RadialWeights
        return _radial_fn().apply(self.ef, self.mlp).as_subclass(RadialWeights) * self.cut


def _radial_fn():
    from .radial import _MLPFn
    return _MLPFn


_DOUBLE_BACKWARD = ('mace_hip_kernels: double backward (create_graph=True, e.g. training on forces/stress or an '
                    'autograd Hessian) is not enabled for this HIP module; patch with '
                    'patch_model(model, double_backward=True)')


class ConvMLPFn(torch.autograd.Function):
    """out = conv(x, Y, W) with W = cutoff * MLP(ef) formed inside the kernels.  Inputs (x, Y, ef, cut, edge_index,
    conv op); gradients for x, Y, ef and cut."""

    @staticmethod
    def forward(ctx, x, Y, ef, cut, edge_index, op):
        from . import conv as C
        fc, mlp = op.fused, op.fused_mlp()
        s = op.spec
        if any(t.dtype != torch.float32 for t in (x, Y, ef, cut)):
            raise TypeError('mace_hip_kernels: conv_tp expects float32 inputs')
        if not all(t.is_cuda for t in (x, Y, ef, cut, edge_index)):
            raise RuntimeError('mace_hip_kernels: conv_tp inputs must be on the GPU')
        E, n = Y.shape[0], x.shape[0]
        if x.dim() != 2 or x.shape[1] != s.x_dim or Y.shape != (edge_index.shape[1], s.y_dim):
            raise ValueError(f'node_feats [N, {s.x_dim}] and edge_attrs [E, {s.y_dim}] expected, got '
                             f'{tuple(x.shape)}, {tuple(Y.shape)}')
        if ef.shape[0] != E or cut.numel() != E or n >= 2 ** 31 or E >= 2 ** 31:
            raise ValueError('edge features and cutoff must have one row per edge')
        xc, Yc = x.contiguous(), Y.contiguous()
        efc, cutf = ef.reshape(E, -1).contiguous(), cut.reshape(-1).contiguous()
        gr = C.graph_for(edge_index, n)
        rowptr, eids = gr.by_recv()
        lib, P = _native.load(), _native.ptr
        stream = _native.stream_of(x)
        h = torch.empty(E, fc.spec.S * 3 * 32, device=x.device, dtype=torch.int16)      # c h as bf16 parts
        _native.launch(f'mlp_hid[{mlp.tag}]', lib.mh_mlp_hid, mlp.module.handle, P(efc), P(mlp.WhT), P(cutf), P(h), E,
                       stream)
        out = torch.empty(n, s.out_dim, device=x.device, dtype=torch.float32)
        _native.launch(f'conv_fwd[{op.tag}]', lib.mh_conv_fwd_mlp, fc.module.handle, P(xc), P(Yc), P(h), P(cutf),
                       P(rowptr), P(eids), P(gr.send), P(fc.Wf), P(out), n, stream)
        ctx.save_for_backward(xc, Yc, efc, cutf, h)
        ctx.op, ctx.gr, ctx.shapes = op, gr, (ef.shape, cut.shape)
        return out

    @staticmethod
    def backward(ctx, g):
        from . import conv as C
        if torch.is_grad_enabled():
            raise RuntimeError(_DOUBLE_BACKWARD)
        x, Y, ef, cut, h = ctx.saved_tensors
        op, gr = ctx.op, ctx.gr
        fc, mlp = op.fused, op.fused_mlp()
        s = op.spec
        E, n = Y.shape[0], x.shape[0]
        want_x = C._grad_needed(ctx, 0)
        gc = g.contiguous()
        lib, P = _native.load(), _native.ptr
        stream = _native.stream_of(x)
        dev = x.device
        gx = torch.empty_like(x) if want_x else None
        work = torch.empty(E, s.x_dim, device=dev, dtype=torch.float32) if want_x else None
        gyp = torch.empty(fc.spec.nct, E, fc.yp, device=dev, dtype=torch.float32)
        ghp = torch.empty(fc.spec.nct, E, fc.spec.HL, device=dev, dtype=torch.float32)
        gY = torch.empty_like(Y)
        rowptr_r, eids_r = gr.by_recv()
        rowptr_s, eids_s = gr.by_send() if want_x else (None, None)
        _native.launch(f'conv_bwd[{op.tag}]', lib.mh_conv_bwd_mlp, fc.module.handle, P(x), P(gc), P(Y), P(h), P(cut),
                       P(eids_r), P(gr.recv), P(gr.send), P(rowptr_s), P(eids_s), P(fc.Wf), P(fc.Wb), P(work), P(gx),
                       P(gyp), P(ghp), P(gY), E, n, _native.MH_WANT_GX if want_x else 0, stream)
        gef = torch.empty_like(ef)
        gcut = torch.empty_like(cut)
        _native.launch(f'mlp_bwd[{mlp.tag}]', lib.mh_mlp_hid_bwd, mlp.module.handle, P(ef), P(mlp.Wh), P(ghp),
                       fc.spec.nct, P(cut), P(gef), P(gcut), E, stream)
        ef_shape, cut_shape = ctx.shapes
        return gx, gY, gef.view(ef_shape), gcut.view(cut_shape), None, None


class ConvRadialFn(torch.autograd.Function):
    """out = conv(x, Y, W0 * cut) with W0 = MLP(ef) formed by the radial MLP's own kernels inside this one autograd
    node (``HipConvTP.defer_mlp``).  Inputs (x, Y, ef, cut, edge_index, conv op); gradients for x, Y, ef and cut.

    W0 and dL/dW0 never leave the node, so when the cutoff comes unmodified from the patched radial embedding (an
    edge outside the envelope's support marked -0.0) and the graph has at least ``conv.EDGE_COMPACT_MIN`` edges,
    neither is formed for those edges: the edges inside the support are listed first (``conv.support_rows``), the
    MLP computes and stores W0 rows for them only (the convolution never reads the others: their cutoff is 0), the
    convolution's backward skips the others without writing their dL/dW0 rows (MH_CUT_NOZERO), and the MLP's
    backward reads only the listed rows and writes zero dL/d(edge features) rows for the rest.  Every result equals
    the separate modules' (the MLP's output times a zero cutoff contributes nothing, and its gradient there is
    zero).  With ``conv.PAIR_RADIAL`` the MLP's forward computes one W0 row per edge and its reverse when their
    feature rows are bitwise equal (``conv.support_pairs``; MACE's neighbour lists hold both directions at the same
    length, and the MLP row is a function of the feature row alone), and the convolution reads each edge's row
    through the pairing's row map: the forward's work and W0 stores halve, every value stays bitwise the same, and
    the backward keeps one dL/dW0 row per edge.  With ``conv.PAIR_GRADS``, when the edge features come from the
    patched embedding of the patched geometry's lengths and the shifts need no gradient (``geometry.
    lengths_pair_symmetric``: only the sum of an edge's and its exact reverse's length gradients reaches the
    positions), the pairs are the exact reverses and the MLP's backward projects each shared row once, from the
    pair's summed dL/dW0 rows (``mh_mlp_bwd_pairs``): half the projections; the pair's summed dL/d(edge features),
    and so the forces, are those of the per-edge backward to fp32 rounding, while the split between the two edges
    is not kept (the partner's row is zero).  No double backward: the two-kernel modules take that
    (``patch_model(double_backward=True)``)."""

    @staticmethod
    def forward(ctx, x, Y, ef, cut, edge_index, op):
        from . import conv as C
        from .geometry import lengths_pair_symmetric
        from .radial import mlp_forward
        mlp = op.deferred_mlp()
        s = op.spec
        if any(t.dtype != torch.float32 for t in (x, Y, ef, cut)):
            raise TypeError('mace_hip_kernels: conv_tp expects float32 inputs')
        if not all(t.is_cuda for t in (x, Y, ef, cut, edge_index)):
            raise RuntimeError('mace_hip_kernels: conv_tp inputs must be on the GPU')
        E, n = Y.shape[0], x.shape[0]
        if x.dim() != 2 or x.shape[1] != s.x_dim or Y.shape != (edge_index.shape[1], s.y_dim):
            raise ValueError(f'node_feats [N, {s.x_dim}] and edge_attrs [E, {s.y_dim}] expected, got '
                             f'{tuple(x.shape)}, {tuple(Y.shape)}')
        if ef.shape[-1] != mlp.spec.hs[0] or ef.numel() != E * mlp.spec.hs[0] or cut.numel() != E:
            raise ValueError('edge features and cutoff must have one row per edge')
        if n >= 2 ** 31 or E >= 2 ** 31:
            raise ValueError('graph too large for int32 indices')
        masked = C._support_masked(cut) and op.skip_masked
        xc, Yc = x.contiguous(), Y.contiguous()
        efc, cutf = ef.reshape(E, -1).contiguous(), cut.reshape(-1).contiguous()
        rows = count = wrow = partner = frows = fcount = None
        gr = C.graph_for(edge_index, n)
        if masked and E >= C.EDGE_COMPACT_MIN:
            if C.PAIR_RADIAL:                       # (also lists the support: support_rows is then cached)
                vec = lengths_pair_symmetric(ef) if C.PAIR_GRADS else None
                wrow, frows, fcount, partner = C.support_pairs(efc, cut, gr, vec)
            rows, count = C.support_rows(cut)
            if not C.PAIR_RADIAL:
                frows, fcount = rows, count
            W0 = mlp_forward(mlp, efc, frows, fcount)
        else:
            W0 = mlp_forward(mlp, efc, None, None)
        rowptr, eids = gr.by_recv()
        out = torch.empty(n, s.out_dim, device=x.device, dtype=torch.float32)
        P = _native.ptr
        # edges with cutoff 0 contribute exactly zero and are not read (so the rows the MLP left unset never are);
        # with wrow an edge reads the W0 row of its reverse when their feature rows are equal
        _native.launch(f'conv_fwd[{op.tag}]', _native.load().mh_conv_fwd_cut_rows, op.module.handle, P(xc), P(Yc),
                       P(W0), P(rowptr), P(eids), P(gr.send), P(cutf), P(wrow), P(out), n, _native.stream_of(x))
        ctx.save_for_backward(xc, Yc, efc, cutf)
        ctx.W0, ctx.rows, ctx.count, ctx.masked, ctx.wrow = W0, rows, count, masked, wrow
        ctx.pairs = (frows, fcount, partner) if partner is not None else None
        ctx.op, ctx.gr, ctx.shapes = op, gr, (ef.shape, cut.shape)
        return out

    @staticmethod
    def backward(ctx, g):
        from . import conv as C
        from .radial import _mlp_bwd, _mlp_bwd_pairs
        if torch.is_grad_enabled():
            raise RuntimeError(_DOUBLE_BACKWARD)
        x, Y, ef, cut = ctx.saved_tensors
        op, gr = ctx.op, ctx.gr
        want_x, want_y, want_ef, want_cut = (C._grad_needed(ctx, i) for i in range(4))
        if not (want_x or want_y or want_ef or want_cut):
            return None, None, None, None, None, None
        compact = ctx.rows is not None
        gx, gY, gW0, gcut = C._conv_grads(op, gr, g.contiguous(), x, Y, None, ctx.W0, cut, want_x,
                                          want_y or want_ef or want_cut, masked=ctx.masked, nozero=compact,
                                          wrow=ctx.wrow)
        # every edge inside the support has its own dL/dW0 row, whatever row its W0 came from; with the pairs of
        # exact reverses, one projection per shared row of the pair's summed dL/dW0
        if not want_ef:
            gef = None
        elif ctx.pairs is not None:
            gef = _mlp_bwd_pairs(op.deferred_mlp(), ef, gW0, *ctx.pairs)
        else:
            gef = _mlp_bwd(op.deferred_mlp(), ef, gW0, ctx.rows, ctx.count)
        ef_shape, cut_shape = ctx.shapes
        return (gx, gY if want_y else None, gef.view(ef_shape) if gef is not None else None,
                gcut.view(cut_shape) if want_cut else None, None, None)

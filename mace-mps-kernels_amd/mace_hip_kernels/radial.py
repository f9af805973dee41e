"""
The radial MLP of MACE's interaction blocks on MI355X: a drop-in for ``conv_tp_weights``, e3nn's
``FullyConnectedNet([n_basis] + radial_MLP + [weight_numel], silu)``, which maps the [E, n_basis] edge features to the
[E, weight_numel] per-edge weights of the convolution.

On the GPU the e3nn module is a chain of GEMMs and elementwise launches (a matmul, the normalised SiLU and its
rescale per layer) whose backward adds as many again, every intermediate an [E, 64] tensor, and whose last GEMM
(64 -> weight_numel, e.g. 1280) is most of the arithmetic.  Here each direction is ONE kernel on the matrix
cores, the hidden layers in fp32 (v_mfma_f32_16x16x4f32) and the wide output layer at fp32 accuracy on the bf16
units (v_mfma_f32_16x16x32_bf16, 2.7x the fp32 rate per K):

* a wave owns 16 edges and computes every layer for them with the transposed product out^T = W^T h^T, so that an
  MFMA result tile leaves lane (edge j = lane % 16, q = lane / 16) holding features 16 t + 4 q + r (r = 0..3) of
  its edge — which is exactly the operand layout the next layer's MFMA needs if that layer walks its K index in the
  order k = 16 t + 4 q + r.  Hidden activations never leave registers;
* the hidden layers' weights sit in LDS for the whole workgroup (4 waves, 64 edges); the last layer's weights are
  streamed through LDS 32 output columns at a time, the next PREFETCH chunks in flight in registers while the
  current one is multiplied, and each result tile is stored as one float4 per lane (16 consecutive bytes of an
  edge's row); each wave owns NB_FWD tiles of 16 edges in the forward (every LDS weight fragment feeds NB_FWD
  MFMAs), NB_BWD in the backward (one each: measured fastest, also with two for the 512-output layer-1 MLP alone);
* the output layer splits both fp32 operands exactly into three bf16 parts (v = hi + mid + lo, by truncation; the
  weights once on the host, the activations and dL/dW0 in registers) and sums the six leading partial products
  hi*hi, hi*mid, mid*hi, hi*lo, mid*mid, lo*hi on the bf16 MFMA with fp32 accumulation; the dropped terms are below
  2^-24 of each product, so the result is as accurate as an fp32 dot product;
* the backward recomputes the hidden layers from the edge features (cheaper than storing [E, 64] activations),
  forms dL/dh = dL/dW0 W_last^T over the streamed weight chunks, and walks back through the SiLUs to dL/d(edge
  features).

Weights are read from the module when it is patched and checked against it in float64; there are no weight
gradients (inference, like the other drop-ins).  Behind a double backward the second-order kernels (``mlp_jvp``,
``mlp_bwd2``, ``source_second``) differentiate the backward once more.
"""
import math

import numpy as np
import torch

from . import _native
from . import conv as _conv

BLOCK = 256          # 4 waves
NB_FWD = 1           # 16-edge tiles per wave in the forward (each LDS weight fragment feeds NB_FWD MFMAs)
NB_BWD = 1           # and in the backward
NB_JVP = 1           # and in the forward-mode derivative (twice the hidden registers of the forward)
GW_DIST = 2          # chunks of dL/dW0 in flight ahead of the one being multiplied (backward)
GW_DIST_P = 1        # the same for the paired backward (mlp_bwdp), whose chunks are two rows each
PREFETCH = 2         # output-layer weight chunks in flight ahead of the one being multiplied
HIDDEN_TILES_BWD = 1 # edge tiles whose hidden layers the backward recomputes together (register pressure)
CH_FWD = 32          # output columns of the last layer per LDS chunk, forward (a multiple of 32)
CH_BWD = 32          # and backward (a multiple of 32: one bf16 MFMA K step per 32 columns)
NSPLIT = 3           # bf16 parts per fp32 weight (exact split)
# Store the forward's W0 rows with the non-temporal policy.  The convolution reads them next, partly from the caches:
# measured on config 2's captured E+F call, non-temporal stores made it 42 us slower.
W0_NT = False
# LDS row paddings.  An MFMA operand fragment is read as one 16-byte ds_read_b128 per lane at row (lane % 16), word
# offset 4 (lane / 16) within the row; on gfx950 such reads run at the full LDS rate when the row length is 8 mod 16
# words, and about 17% slower for other lengths that are multiples of 4 (an in-bounds sweep of row lengths 12 .. 84
# words).  Scalar reads of 64 lanes (column c16 + 16 q of a row-major block) want the row length 4 mod 16 instead.
BPAD = 16            # bf16 row padding of a chunk: rows of 64 + 16 (forward) and 32 + 16 (backward) bf16 = 40 / 24 words
PAD = 4              # fp32 row padding of the hidden layers' natural layout (scalar reads, rows of 64 + 4 words)
TPAD = 8             # and of their transposed layout (16-byte reads, rows of 64 + 8 words), from the second layer on
TPAD0 = 4            # the first layer's transposed rows (K = the padded input width, scalar reads: 8 + 4 words)
# Waves per SIMD the forward and backward are compiled for (amdgpu_waves_per_eu; None: the compiler's choice).
# Left to itself the compiler gives mlp_fwd 172 VGPRs + 48 AGPRs (2 waves per SIMD); asked for 3 it fits in 138
# VGPRs without spills, mlp_bwd in 168 (three VGPRs spilled).  mlp_bwd measured (config 2, layer 2 / layer 1, us in
# the E+F call): 2 waves 158.3 / 78.4, 3 waves 144.0 / 72.4, 4 waves (128 VGPRs, no spills) 147.5 / 71.9.
WAVES_FWD = 3
WAVES_BWD = 3
# Waves per workgroup of the first-order backward (16 edges each).  The workgroup streams the whole split output layer
# through LDS, so more waves would amortise that staging over more edges, but every chunk's barrier then waits for
# more waves: config 2, layer 2 / layer 1 in the E+F call, 4 waves 143.6 / 72.6 us, 6 waves 157.6 / 84.2, 8 waves
# 172.1 / 84.0.
WG_WAVES_BWD = 4
# The forward as two kernels (mh_mlp_fwd_ws): the hidden layers of the listed rows into an [E, HL] scratch (mlp_h3),
# then the output layer weight-stationary (mlp_out): a persistent grid whose waves each keep one block of WS_COLS
# output columns of the split output layer in registers and walk the 16-edge tiles of their XCD's share, four waves
# (four blocks) sharing each tile's activations through LDS.  False: the single-kernel forward (mlp_fwd), whose workgroups stream the whole output layer
# through LDS for every 64 edges.
WS_FWD = True
WS_MIN_COLS = 1024   # ... for output layers at least this wide (config 2: layer 2's 1280 columns 84.8 -> 76.5 us in the
                     # E+F call; layer 1's 512 columns 39.5 -> 43.3 us, so the single kernel stays there)
WS_COLS = 64         # output columns per wave of mlp_out (4 MFMA column tiles: 96 VGPRs of split weights)
WS_WAVES = 3         # waves per SIMD mlp_out is compiled for
WS_STAGE_OUT = True  # mlp_out's results through LDS, stored as whole 1 KB row pieces of the column group (output
                     # widths that are a multiple of 256); False: every wave stores its own 16 rows x 64 bytes


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
        if hs[-2] % 32:
            return False, f'last hidden width {hs[-2]} is not a multiple of 32'
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
    """Packing constants shared by the generator and the weight packer (float offsets for the fp32 hidden weights,
    bf16 offsets for the output layer's chunks)."""
    hs = spec.hs
    H0, NW, HL = hs[0], hs[-1], hs[-2]
    K0S = -(-H0 // 4)                                    # MFMA steps of the first layer (K = H0 padded to 4 K0S)
    rows = [4 * K0S] + hs[1:-2]                          # K extent of each hidden layer
    cols = hs[1:-1]                                      # outputs of each hidden layer
    nat, tr, o1, o2 = [], [], 0, 0
    for i, (r, c) in enumerate(zip(rows, cols)):
        nat.append(o1)
        o1 += r * (c + PAD)                              # natural [k][j + PAD]   (backward)
        tr.append(o2)
        o2 += c * (r + _tpad(i))                         # transposed [j][k + TPAD] (forward)
    RSF = HL + BPAD                                      # bf16 row of a forward chunk: one output column, K = HL
    RSB = CH_BWD + BPAD                                  # bf16 row of a backward chunk: one hidden feature, K = CH_BWD
    return dict(H0=H0, NW=NW, HL=HL, K0S=K0S, rows=rows, cols=cols, nat=nat, tr=tr, nat_size=o1, tr_size=o2,
                RSF=RSF, RSB=RSB, chunk_fwd=NSPLIT * CH_FWD * RSF, chunk_bwd=NSPLIT * HL * RSB)


def _tpad(i):
    """Row padding (floats) of hidden layer i's transposed LDS layout."""
    return TPAD0 if i == 0 else TPAD


def _kperm(HL):
    """Forward K order of the output layer: position 32 s + 8 q + 4 t + r holds hidden feature 32 s + 16 t + 4 q + r,
    so the eight bf16 operands of lane group q at step s are one 16-byte read, and they pair with that lane's hidden
    activations h[2 s + t][r] (the fp32 MFMA result layout of the last hidden layer)."""
    perm = np.zeros(HL, dtype=np.int64)
    for s in range(HL // 32):
        for q in range(4):
            for t in range(2):
                for r in range(4):
                    perm[32 * s + 8 * q + 4 * t + r] = 32 * s + 16 * t + 4 * q + r
    return perm


def bf16_split3(a):
    """Exact three-way split of float32 values into bf16 parts (uint16 bit patterns): a = hi + mid + lo exactly
    (truncation at every step leaves at most 16, then 8, significant bits)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    hi = a.view(np.uint32) & np.uint32(0xFFFF0000)
    r1 = (a - hi.view(np.float32)).astype(np.float32)
    mid = r1.view(np.uint32) & np.uint32(0xFFFF0000)
    r2 = (r1 - mid.view(np.float32)).astype(np.float32)
    lo = r2.view(np.uint32)
    assert not np.any(lo & np.uint32(0xFFFF)), 'bf16 split not exact'
    return [(x >> np.uint32(16)).astype(np.uint16) for x in (hi, mid, lo)]


def source(spec):
    """HIP source of ``mlp_fwd`` and ``mlp_bwd`` (and the fused convolution's ``mlp_hid`` / ``mlp_hidb``)."""
    return _source(spec, second=False)


def source_second(spec):
    """HIP source of the second-order kernels behind a double backward (compiled on first use):
    ``mlp_jvp``  the forward on dual numbers, edge features ef + eps v: the eps part of the output, dW0 = J(ef) v
                 (every hidden layer carries a tangent, h' = c silu'(z) z', and the output layer multiplies the last
                 hidden layer's tangent);
    ``mlp_bwd2`` the backward on the same dual numbers with dL/dW0 held real: the eps part of dL/d(edge features),
                 the Hessian-vector product sum_k gW_k d^2 W0_k / def^2 v (walking back, g_z = g_h h'(z) gains the
                 tangent g_h' h'(z) + g_h h''(z) z').
    Both keep the first-order kernels' structure: hidden layers on the fp32 MFMA, the output layer at fp32 accuracy on
    the bf16 MFMA."""
    return _source(spec, second=True)


def _source(spec, second):
    Lo = _layout(spec)
    H0, NW, HL, K0S = Lo['H0'], Lo['NW'], Lo['HL'], Lo['K0S']
    rows, cols = Lo['rows'], Lo['cols']
    RSF, RSB = Lo['RSF'], Lo['RSB']
    nh = len(cols)
    TL = HL // 16
    S = HL // 32                                         # K steps of the forward output layer
    CH = CH_FWD
    NCHK = -(-NW // CH)                                  # the last chunk may hold zero columns past NW
    TAIL = NW % CH != 0
    NO = CH // 16
    lds_fwd = max(Lo['tr_size'], Lo['chunk_fwd'])        # floats; a bf16 chunk of n elements takes n / 2 floats
    lds_bwd = max(Lo['nat_size'], Lo['chunk_bwd'])
    L = [_native.device_header(),
         '// the logistic function 1 / (1 + e^-z) on the hardware exp2 (e^-z = 2^(-z log2 e)) and reciprocal: within',
         '// about 1e-7 of the exact value (z very negative: 1 + inf, whose reciprocal is 0), and about 5 instructions',
         '// where expf and an IEEE division take about 25',
         '__device__ __forceinline__ float mlp_sig(float z) {',
         '  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-1.4426950408889634f * z));',
         '}', '']
    if second:
        # h = c z s(z) (s the logistic function): h' = c s (1 + z (1 - s)), h'' = c s (1 - s) (2 + z (1 - 2 s))
        L += ['__device__ __forceinline__ float mlp_d1(float z) { const float s = mlp_sig(z); '
              'return s * (1.f + z * (1.f - s)); }',
              '__device__ __forceinline__ float mlp_d2(float z) { const float s = mlp_sig(z); '
              'return s * (1.f - s) * (2.f + z * (1.f - 2.f * s)); }', '']

    def head(name, args, lds, nb, waves=BLOCK // 64, indexed=False, wpe=None, extra=''):
        """Kernel prologue: edge slot ej{b} of this lane in tile b (live{b}: a slot < E).  ``indexed``: two more
        arguments, ``rows`` (NULL, or the edge of each slot) and ``count`` (NULL, or the number of slots to compute:
        the rest are not computed, and a backward writes zero gradient rows for their edges); rowc{b} is the edge of
        slot ej{b} (clamped into range) and do{b} whether it is computed."""
        if indexed:
            args += ', const int* __restrict__ rows, const int* __restrict__ count'
        args += extra                                    # parameters after the row list's (mlp_bwdp: partner)
        span = 16 * nb * waves
        occ = f' __attribute__((amdgpu_waves_per_eu({wpe})))' if wpe else ''
        P = [f'extern "C" __global__ __launch_bounds__({64 * waves}){occ} void {name}({args}) {{',
             f'  __shared__ __align__(16) float lds[{lds}];',
             '  unsigned short* __restrict__ ldsb = reinterpret_cast<unsigned short*>(lds);',
             '  const int t = threadIdx.x, wave = t >> 6, lane = t & 63, q = lane >> 4, c16 = lane & 15;',
             '  (void)ldsb; (void)lane;']
        if indexed:
            # the workgroups' worth of computed slots (nact) go to the first nact hardware workgroups, which the
            # dispatcher spreads round-robin over the XCDs, in one contiguous range of slots per XCD (mh_xcd_block
            # over nact); the other workgroups take the remaining slots in order (none computed)
            P += ['  const long long ncount = count ? (long long)count[0] : E;',
                  f'  const int nact = (int)((ncount + {span - 1}) / {span});',
                  '  const long long blk = (int)blockIdx.x < nact ? mh_xcd_block(blockIdx.x, nact) : blockIdx.x;']
        else:
            P += ['  const long long blk = mh_xcd_block(blockIdx.x, gridDim.x);']
        P += [f'  const long long e0 = blk * {span} + wave * {16 * nb};']
        for b in range(nb):      # edge tile b of this wave: this lane's edge as a B column / output row
            P += [f'  const long long ej{b} = e0 + {16 * b} + c16;',
                  f'  const bool live{b} = ej{b} < E;',
                  f'  const long long ejc{b} = live{b} ? ej{b} : E - 1;      // clamped: every load in bounds']
        if indexed:
            P += [f'  const long long rowc{b} = rows ? (long long)rows[ejc{b}] : ejc{b};' for b in range(nb)]
            P += [f'  const bool do{b} = live{b} && ej{b} < ncount;' for b in range(nb)]
        else:
            P += [f'  const long long rowc{b} = ejc{b};' for b in range(nb)]
            P += [f'  const bool do{b} = live{b};' for b in range(nb)]
        return P

    def skip_block(nb, zero_rows, waves=BLOCK // 64):
        """An indexed kernel's workgroup whose slots all lie past ``count`` computes nothing (uniform: before any
        barrier); a backward writes zero dL/d(edge features) rows for the edges of its slots."""
        span = 16 * nb * waves
        P = [f'  const long long slot0 = blk * {span};',
             '  if (slot0 >= ncount) {']
        if zero_rows:
            P += [f'    for (int k = t; k < {span * H0}; k += {64 * waves}) {{',
                  f'      const long long sl = slot0 + k / {H0};',
                  f'      if (sl < E) gef[(rows ? (long long)rows[sl] : sl) * {H0} + k % {H0}] = 0.f;',
                  '    }']
        P += ['    return;', '  }']
        return P

    def stage(src, n, nthreads=BLOCK):
        """Copy n floats to the start of LDS: every thread issues all of its loads before its first LDS write (a
        rolled copy loop waits out one L2 round trip per iteration)."""
        it = -(-(n // 4) // nthreads)
        P = [f'  mh_f4 {", ".join(f"sg{i}" for i in range(it))};']
        P += [f'  sg{i} = reinterpret_cast<const mh_f4*>({src})[min(t + {i * nthreads}, {n // 4 - 1})];' for i in range(it)]
        P += [f'  {"" if (i + 1) * nthreads <= n // 4 else f"if (t + {i * nthreads} < {n // 4}) "}'
              f'reinterpret_cast<mh_f4*>(lds)[t + {i * nthreads}] = sg{i};' for i in range(it)]
        return P

    def xin(tiles, src='ef', name='xin'):
        P = []
        for b in tiles:
            P += [f'  float {name}{b}[{K0S}];']
            P += [f'  {name}{b}[{st}] = {4 * st} + q < {H0} ? {src}[rowc{b} * {H0} + {4 * st} + q] : 0.f;'
                  for st in range(K0S)]
        return P

    def hidden_fwd(transposed, keep, tiles, dual=False, keep_t=False):
        """z_i and h_i = c_i silu(z_i) for every hidden layer on the fp32 MFMA, A operands from LDS (transposed
        layout: one b128 read per 4 MFMAs; natural layout: b32 reads), each A operand used for every edge tile in
        ``tiles``.  ``dual``: also the tangents zt_i (the same A operands applied to the input tangent xv / the
        previous layer's ht) and ht_i = c_i silu'(z_i) zt_i (the last layer's with ``keep_t``)."""
        P = []
        chains = [('z', 'xin', 'h')] + ([('zt', 'xv', 'ht')] if dual else [])
        for i in range(nh):
            T = cols[i] // 16
            for zn, _, _ in chains:
                for b in tiles:
                    P.append(f'  mh_f4 {zn}{i}_{b}[{T}];')
                    P += [f'  {zn}{i}_{b}[{o}] = mh_f4{{0.f, 0.f, 0.f, 0.f}};' for o in range(T)]
            if i == 0:
                for st in range(K0S):
                    for o in range(T):
                        a = (f'lds[{Lo["tr"][0]} + ({16 * o} + c16) * {rows[0] + _tpad(0)} + {4 * st} + q]' if transposed else
                             f'lds[{Lo["nat"][0]} + ({4 * st} + q) * {cols[0] + PAD} + {16 * o} + c16]')
                        P.append(f'  {{ const float a = {a};')
                        P += [f'    {zn}0_{b}[{o}] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, {xn}{b}[{st}], {zn}0_{b}[{o}], '
                              f'0, 0, 0);' for zn, xn, _ in chains for b in tiles]
                        P.append('  }')
            else:
                Tin = cols[i - 1] // 16
                for ti in range(Tin):
                    if transposed:
                        for o in range(T):
                            P.append(f'  const mh_f4 a{i}_{ti}_{o} = *reinterpret_cast<const mh_f4*>(&lds[{Lo["tr"][i]} + '
                                     f'({16 * o} + c16) * {rows[i] + _tpad(i)} + {16 * ti} + 4 * q]);')
                    for r in range(4):
                        for o in range(T):
                            a = (f'a{i}_{ti}_{o}[{r}]' if transposed else
                                 f'lds[{Lo["nat"][i]} + ({16 * ti + r} + 4 * q) * {cols[i] + PAD} + {16 * o} + c16]')
                            P.append(f'  {{ const float a = {a};')
                            P += [f'    {zn}{i}_{b}[{o}] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, {hn}{i - 1}_{b}[{ti}][{r}], '
                                  f'{zn}{i}_{b}[{o}], 0, 0, 0);' for zn, _, hn in chains for b in tiles]
                            P.append('  }')
            if i < nh - 1 or keep:
                for b in tiles:
                    P.append(f'  mh_f4 h{i}_{b}[{T}];')
                    for o in range(T):
                        for r in range(4):
                            P.append(f'  h{i}_{b}[{o}][{r}] = {_lit(spec.c[i])} * z{i}_{b}[{o}][{r}] * '
                                     f'mlp_sig(z{i}_{b}[{o}][{r}]);')
            if dual and (i < nh - 1 or keep_t):
                for b in tiles:
                    P.append(f'  mh_f4 ht{i}_{b}[{T}];')
                    for o in range(T):
                        for r in range(4):
                            P.append(f'  ht{i}_{b}[{o}][{r}] = {_lit(spec.c[i])} * mlp_d1(z{i}_{b}[{o}][{r}]) * '
                                     f'zt{i}_{b}[{o}][{r}];')
        return P

    def chunk_io(src, nx_elems, row_elems, rs, nrows, ind, store_base=None, reg='pre', nthreads=BLOCK):
        """Load (store_base None) or store this thread's 16-byte pieces of a bf16 chunk: piece f is part p, 8-element
        group c8, row rr of a [3][row_elems / 8][nrows][8] block at element offset nx_elems of ``src`` (rows
        innermost, so the eight lanes of one LDS write phase hit eight different rows: conflict-free for any row
        stride that is 4 words mod 8 banks); in LDS the rows are ``rs`` elements apart."""
        per_row = row_elems // 8
        total = NSPLIT * nrows * per_row
        P = []
        for it in range(-(-total // nthreads)):
            exact = (it + 1) * nthreads <= total
            fx = f't + {it * nthreads}' if exact else f'min(t + {it * nthreads}, {total - 1})'
            idx = [f'{ind}{{ const int f = {fx}, p = f / {nrows * per_row}, rem = f - p * {nrows * per_row},',
                   f'{ind}      c8 = rem / {nrows}, rr = rem - c8 * {nrows};']
            if store_base is None:
                P += idx + [f'{ind}  {reg}{it} = *reinterpret_cast<const mh_u4*>({src} + (size_t){nx_elems} + '
                            f'(size_t)f * 8); }}']
            else:
                guard = '' if exact else f'if (t + {it * nthreads} < {total}) '
                P += idx + [f'{ind}  {guard}*reinterpret_cast<mh_u4*>(&ldsb[{store_base} + p * {nrows * rs} + rr * {rs} + '
                            f'8 * c8]) = {reg}{it}; }}']
        return P, -(-total // nthreads)

    PAIRS = [(0, 0), (0, 1), (1, 0), (0, 2), (1, 1), (2, 0)]

    # ------------------------------------------------------------------ forward
    def fwd_kernel(name, tangent):
        """The forward (``tangent``: the JVP: edge features ef + eps ev, the eps part of the output)."""
        # hidden weights transposed [j][k + PAD] in fp32; the output layer as bf16 chunks of CH columns x HL (K in the
        # _kperm order), three parts each, double-buffered in LDS (the hidden weights' space is reused once they are done)
        nb = NB_JVP if tangent else NB_FWD
        ncf = 2 if nb == 1 else 1                            # accumulator chains per result tile
        F = head(name, 'const float* __restrict__ ef, ' + ('const float* __restrict__ ev, ' if tangent else '') +
                 'const float* __restrict__ Wh, const unsigned short* __restrict__ Wl, float* __restrict__ W0, long long E',
                 lds_fwd, nb, indexed=not tangent, wpe=None if tangent else WAVES_FWD)
        if not tangent:
            F += skip_block(nb, zero_rows=False)
        F += stage('Wh', Lo['tr_size']) + ['  __syncthreads();'] + xin(range(nb))
        if tangent:
            F += xin(range(nb), 'ev', 'xv') + hidden_fwd(True, False, range(nb), dual=True, keep_t=True)
        else:
            F += hidden_fwd(True, True, range(nb))
        # the last hidden layer's activations (tangent: their tangents) as bf16 operands: step s, lane group q: features
        # 32 s + 16 t + 4 q + r
        for b in range(nb):
            hl = f'ht{nh - 1}_{b}' if tangent else f'h{nh - 1}_{b}'
            F += [f'  mh_bf8 hb{b}[{S}][3];']
            for st in range(S):
                F += [f'  {{ const float v[8] = {{{", ".join(f"{hl}[{2 * st + tt}][{r}]" for tt in range(2) for r in range(4))}}};',
                      f'    mh_split8(v, hb{b}[{st}]); }}']
        # weight chunks in flight: register set j holds chunk c + PD while chunk c is multiplied (the loop is unrolled PD
        # times so the sets have fixed names; chunks past the last, when PD does not divide the count, are computed from
        # the last chunk's weights and not stored)
        PD = PREFETCH
        NCHP = -(-NCHK // PD) * PD
        npre = -(-(NSPLIT * CH * HL // 8) // BLOCK)
        for j in range(PD):
            F += [f'  mh_u4 {", ".join(f"pre{j}_{i}" for i in range(npre))};']
            F += chunk_io('Wl', f'{min(j, NCHK - 1) * NSPLIT * CH * HL}', HL, RSF, CH, '  ', reg=f'pre{j}_')[0]
        F += ['  __syncthreads();                                // every wave is done with the hidden weights']
        F += chunk_io('Wl', 0, HL, RSF, CH, '  ', store_base='0', reg='pre0_')[0] + ['  __syncthreads();']
        F += [f'  for (int ch = 0; ch < {NCHP}; ch += {PD}) {{']
        for j in range(PD):
            c = f'(ch + {j})' if j else 'ch'
            F += ['  {',
                  f'    const int c = {c}, base = (c & 1) * {Lo["chunk_fwd"]}, nbase = {Lo["chunk_fwd"]} - base;',
                  f'    const size_t nx = (size_t)min(c + {PD}, {NCHK - 1}) * {NSPLIT * CH * HL};']
            F += chunk_io('Wl', 'nx', HL, RSF, CH, '    ', reg=f'pre{j}_')[0]
            F += ['    __builtin_amdgcn_sched_barrier(0);            // the loads go out before the MFMAs']
            for b in range(nb):
                F += [f'    mh_f4 acc{b}[{NO}][{ncf}];']
                F += [f'    acc{b}[{o}][{jj}] = mh_f4{{0.f, 0.f, 0.f, 0.f}};' for o in range(NO) for jj in range(ncf)]
            for st in range(S):
                for o in range(NO):
                    F += [f'    mh_bf8 a{st}_{o}[3];']
                    F += [f'    a{st}_{o}[{p}] = *reinterpret_cast<const mh_bf8*>(&ldsb[base + {p * CH * RSF} + ({16 * o} + c16) '
                          f'* {RSF} + {32 * st} + 8 * q]);' for p in range(3)]
                for k, (pa, pb) in enumerate(PAIRS):
                    for o in range(NO):
                        for b in range(nb):
                            a = f'acc{b}[{o}][{k % ncf}]'
                            F.append(f'    {a} = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a{st}_{o}[{pa}], hb{b}[{st}][{pb}], '
                                     f'{a}, 0, 0, 0);')
            # chunk c + 1 goes to LDS before chunk c's results go out: vmcnt counts loads and stores in issue order, so
            # waiting for the prefetch then never waits for stores (they drain during the next chunk's MFMAs)
            F += chunk_io('Wl', 0, HL, RSF, CH, '    ', store_base='nbase', reg=f'pre{(j + 1) % PD}_')[0]
            F += ['    __builtin_amdgcn_sched_barrier(0);']
            for b in range(nb):
                F.append(f'    if (do{b}{f" && c < {NCHK}" if NCHP > NCHK else ""}) {{')
                for o in range(NO):
                    guard = f'if (c < {NCHK - 1}) ' if TAIL and 16 * (o + 1) > NW % CH else ''
                    val = ' + '.join(f'acc{b}[{o}][{jj}]' for jj in range(ncf))
                    dst = f'reinterpret_cast<mh_f4*>(W0 + rowc{b} * {NW} + c * {CH} + {16 * o} + 4 * q)'
                    F += [f'      {guard}__builtin_nontemporal_store({val}, {dst});' if W0_NT else
                          f'      {guard}*{dst} = {val};']
                F += ['    }']
            F += ['    __syncthreads();', '  }']
        F += ['  }', '}', '']
        return F


    def walk_back(grp, cur, dual=False):
        """Lines walking dL/dh_last (in ``cur``{b}) back through the hidden layers (recomputed z's in scope) to
        dL/d(edge features), stored to gef.  ``dual``: the recomputed layers carry tangents zt (dL/dh_last does not):
        the walk carries the tangent of the gradient too, g_z' = g_h' h'(z) + g_h h''(z) z', and gef receives the
        tangent of dL/d(edge features) instead."""
        B = []
        curt = None
        for i in range(nh - 1, -1, -1):
            T = cols[i] // 16
            if dual:
                nt = f'dht{i}_'
                for b in grp:
                    B.append(f'  mh_f4 {nt}{b}[{T}];')
                    for o in range(T):
                        for r in range(4):
                            prev = f'{curt}{b}[{o}][{r}] * mlp_d1(z) + ' if curt else ''
                            B.append(f'  {{ const float z = z{i}_{b}[{o}][{r}]; {nt}{b}[{o}][{r}] = {_lit(spec.c[i])} * '
                                     f'({prev}{cur}{b}[{o}][{r}] * mlp_d2(z) * zt{i}_{b}[{o}][{r}]); }}')
                curt = nt
            for b in grp:
                for o in range(T):
                    for r in range(4):
                        B += ['  {',
                              f'    const float z = z{i}_{b}[{o}][{r}], s = mlp_sig(z);',
                              f'    {cur}{b}[{o}][{r}] *= {_lit(spec.c[i])} * s * (1.f + z * (1.f - s));',
                              '  }']
            if i > 0:
                Tp = cols[i - 1] // 16
                chains = [(cur, f'dh{i - 1}_')] + ([(curt, f'dhu{i - 1}_')] if dual else [])
                # row j of layer i's natural weights = its input feature j: A[j][k] = W_i[j][k], one b128 per 4 steps
                for _, nxt in chains:
                    for b in grp:
                        B.append(f'  mh_f4 {nxt}{b}[{Tp}];')
                        B += [f'  {nxt}{b}[{o}] = mh_f4{{0.f, 0.f, 0.f, 0.f}};' for o in range(Tp)]
                for ti in range(T):
                    for o in range(Tp):
                        B.append(f'  const mh_f4 b{i}_{ti}_{o} = *reinterpret_cast<const mh_f4*>(&lds[{Lo["nat"][i]} + '
                                 f'({16 * o} + c16) * {cols[i] + PAD} + {16 * ti} + 4 * q]);')
                    for r in range(4):
                        for o in range(Tp):
                            for src, nxt in chains:
                                for b in grp:
                                    B.append(f'  {nxt}{b}[{o}] = __builtin_amdgcn_mfma_f32_16x16x4f32(b{i}_{ti}_{o}[{r}], '
                                             f'{src}{b}[{ti}][{r}], {nxt}{b}[{o}], 0, 0, 0);')
                cur = chains[0][1]
                if dual:
                    curt = chains[1][1]
        if dual:
            cur = curt
        # dL/d(edge features): rows = the H0 inputs (one 16-row tile per 16; rows past the padded K read row 0)
        T0 = cols[0] // 16
        for o in range(-(-H0 // 16)):
            B += ['  {',
                  f'    const int row = {16 * o} + c16 < {rows[0]} ? {16 * o} + c16 : 0;']
            B += [f'    mh_f4 d{b} = mh_f4{{0.f, 0.f, 0.f, 0.f}};' for b in grp]
            for ti in range(T0):
                B.append(f'    const mh_f4 w{ti} = *reinterpret_cast<const mh_f4*>(&lds[{Lo["nat"][0]} + row * '
                         f'{cols[0] + PAD} + {16 * ti} + 4 * q]);')
                for r in range(4):
                    B += [f'    d{b} = __builtin_amdgcn_mfma_f32_16x16x4f32(w{ti}[{r}], {cur}{b}[{ti}][{r}], d{b}, 0, 0, 0);'
                          for b in grp]
            for b in grp:
                for r in range(4):
                    B.append(f'    if (live{b} && {16 * o + r} + 4 * q < {H0}) gef[rowc{b} * {H0} + {16 * o + r} + 4 * q] = '
                             f'do{b} ? d{b}[{r}] : 0.f;')
            B.append('  }')
        return B

    # ------------------------------------------------------------------ backward
    def bwd_kernel(name, dual, paired=False):
        """The backward (``dual``: the Hessian-vector product along ev; ``paired``: ``mlp_bwdp``, the row list's
        slot i < count[0] (edge e = rows[i]) projects the sum of e's dL/dW0 row and that of partner[e] when
        partner[e] >= 0, the edge that reads e's W0 row; the partner's own slot lies past count[0] and gets a zero
        dL/d(edge features) row like every other uncomputed slot)."""
        # dL/dh_last = gW Wl^T first: K = the output columns, one bf16 step of 32 per chunk (lane group q: columns
        # 8 q .. 8 q + 7, two float4 loads of gW split into three bf16 parts); chunks of Wl [HL][CH] as bf16 rows of
        # CH + BPAD.  Then the hidden layers recomputed from the natural-layout fp32 weights and walked back.
        nb = NB_BWD
        ncb = 2 if nb == 1 else 1
        CH = CH_BWD
        KS = CH // 32                                        # bf16 K steps per chunk
        NCHK = -(-NW // CH)
        TAIL = NW % CH != 0
        wg = BLOCK // 64 if dual else WG_WAVES_BWD           # waves per workgroup
        nt = 64 * wg
        dist = GW_DIST_P if paired else GW_DIST
        B = head(name, 'const float* __restrict__ ef, ' + ('const float* __restrict__ ev, ' if dual else '') +
                 'const float* __restrict__ Wh, const unsigned short* __restrict__ Wl, const float* __restrict__ gW, '
                 'float* __restrict__ gef, long long E', lds_bwd, nb, waves=wg, indexed=not dual,
                 wpe=None if dual else WAVES_BWD, extra=', const int* __restrict__ partner' if paired else '')
        if not dual:
            B += skip_block(nb, zero_rows=True, waves=wg)
        if paired:
            # the partner's row when there is one (hp), else the slot's own row again, whose values are then dropped
            for b in range(nb):
                B += [f'  const int prr{b} = partner[rowc{b}];',
                      f'  const bool hp{b} = do{b} && prr{b} >= 0;',
                      f'  const long long prc{b} = hp{b} ? (long long)prr{b} : rowc{b};']
        for b in range(nb):
            B += [f'  mh_f4 dh{b}[{TL}][{ncb}];'] + [f'  dh{b}[{o}][{j}] = mh_f4{{0.f, 0.f, 0.f, 0.f}};'
                                                    for o in range(TL) for j in range(ncb)]
        ld0, npre = chunk_io('Wl', 0, CH, RSB, HL, '  ', nthreads=nt)
        B += [f'  mh_u4 {", ".join(f"pre{i}" for i in range(npre))};'] + ld0
        # columns past NW (the zero-padded tail of the last chunk) read a valid column and are zeroed
        gcol = (lambda c: f'min({c} + 8 * q, {NW - 8})') if TAIL else (lambda c: f'{c} + 8 * q')

        def gload(dst, c, b, decl, row='rowc'):
            """dL/dW0 of edge tile b, columns c + 32 ks + 8 q .. + 7 for each K step ks, into dst_ks_{0,1}"""
            P = []
            for ks in range(KS):
                col = gcol(f'{c} + {32 * ks}')
                P += [f'{decl}{dst}_{ks}_0_{b} = *reinterpret_cast<const mh_f4*>(gW + {row}{b} * {NW} + {col});',
                      f'{decl}{dst}_{ks}_1_{b} = *reinterpret_cast<const mh_f4*>(gW + {row}{b} * {NW} + {col} + 4);']
            return P

        def fold(dst, src, b, decl):
            """dst = src + (the partner's values when there is one), per K step and half"""
            return [f'{decl}{dst}_{ks}_{h}_{b} = {src}_{ks}_{h}_{b} + (hp{b} ? {src}p_{ks}_{h}_{b} : '
                    f'mh_f4{{0.f, 0.f, 0.f, 0.f}});' for ks in range(KS) for h in range(2)]
        # dL/dW0 of chunk ch + d sits in g{d}_* (d = 0 .. dist - 1) while chunk ch is multiplied
        for b in range(nb):
            for d in range(dist):
                if paired:
                    B += gload(f'gi{d}', str(min(d, NCHK - 1) * CH), b, '  mh_f4 ')
                    B += gload(f'gi{d}p', str(min(d, NCHK - 1) * CH), b, '  mh_f4 ', row='prc')
                    B += fold(f'g{d}', f'gi{d}', b, '  mh_f4 ')
                else:
                    B += gload(f'g{d}', str(min(d, NCHK - 1) * CH), b, '  mh_f4 ')
        st0, _ = chunk_io('Wl', 0, CH, RSB, HL, '  ', store_base='0', nthreads=nt)
        B += st0 + ['  __syncthreads();']
        B += [f'  for (int ch = 0; ch < {NCHK}; ++ch) {{',
              f'    const int base = (ch & 1) * {Lo["chunk_bwd"]}, nbase = {Lo["chunk_bwd"]} - base;',
              f'    const int nc = min(ch + 1, {NCHK - 1});',
              f'    const size_t nx = (size_t)nc * {NSPLIT * HL * CH};']
        ldn, _ = chunk_io('Wl', 'nx', CH, RSB, HL, '    ', nthreads=nt)
        B += ldn
        B += [f'    const int gc = min(ch + {dist}, {NCHK - 1}) * {CH};']
        for b in range(nb):
            B += gload('gn', 'gc', b, '    const mh_f4 ')
            if paired:
                B += gload('gnp', 'gc', b, '    const mh_f4 ', row='prc')
        B += ['    __builtin_amdgcn_sched_barrier(0);            // the next chunk\'s loads go out before the MFMAs']
        for ks in range(KS):
            for b in range(nb):
                v = f'g0_{ks}'
                zero = (f' if (ch * {CH} + {32 * ks} + 8 * q >= {NW}) {{ {v}_0_{b} = mh_f4{{0.f, 0.f, 0.f, 0.f}}; '
                        f'{v}_1_{b} = {v}_0_{b}; }}' if TAIL else '')
                B += [f'    mh_bf8 gb{ks}_{b}[3];' + zero,
                      f'    {{ const float v[8] = {{{", ".join(f"{v}_{h}_{b}[{i}]" for h in range(2) for i in range(4))}}}; '
                      f'mh_split8(v, gb{ks}_{b}); }}']
            for o in range(TL):
                B += [f'    mh_bf8 a{ks}_{o}[3];']
                B += [f'    a{ks}_{o}[{p}] = *reinterpret_cast<const mh_bf8*>(&ldsb[base + {p * HL * RSB} + ({16 * o} + c16) * '
                      f'{RSB} + {32 * ks} + 8 * q]);' for p in range(3)]
            for k, (pa, pb) in enumerate(PAIRS):
                for o in range(TL):
                    for b in range(nb):
                        c = f'dh{b}[{o}][{k % ncb}]'
                        B.append(f'    {c} = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a{ks}_{o}[{pa}], gb{ks}_{b}[{pb}], {c}, '
                                 '0, 0, 0);')
        for b in range(nb):
            for ks in range(KS):
                for h in range(2):
                    for d in range(dist - 1):
                        B += [f'    g{d}_{ks}_{h}_{b} = g{d + 1}_{ks}_{h}_{b};']
                    if not paired:
                        B += [f'    g{dist - 1}_{ks}_{h}_{b} = gn_{ks}_{h}_{b};']
            if paired:
                B += fold(f'g{dist - 1}', 'gn', b, '    ')
        stn, _ = chunk_io('Wl', 0, CH, RSB, HL, '    ', store_base='nbase', nthreads=nt)
        B += stn + ['    __syncthreads();', '  }']
        for b in range(nb):
            B += [f'  mh_f4 dhs_{b}[{TL}];'] + [f'  dhs_{b}[{o}] = ' + ' + '.join(f'dh{b}[{o}][{j}]' for j in range(ncb)) + ';'
                                               for o in range(TL)]
        # the hidden layers recomputed and walked back HIDDEN_TILES_BWD edge tiles at a time (each group in a scope of
        # its own, so the registers of its activations are free for the next)
        B += stage('Wh', Lo['nat_size'], nthreads=nt) + ['  __syncthreads();']
        for g0 in range(0, nb, HIDDEN_TILES_BWD):
            grp = range(g0, min(nb, g0 + HIDDEN_TILES_BWD))
            B += ['  {'] + xin(grp)
            if dual:
                B += xin(grp, 'ev', 'xv') + hidden_fwd(False, False, grp, dual=True)
            else:
                B += hidden_fwd(False, False, grp)
            B += walk_back(grp, 'dhs_', dual=dual)
            B += ['  }', '  __builtin_amdgcn_sched_barrier(0);       // one group finished before the next starts']
        B += ['}', '']
        return B

    def hidden_only():
        """mlp_hid / mlp_hidb, the fused convolution's MLP kernels."""

        # ------------------------------------------------------------------ hidden layers only (fused convolution)
        # mlp_hid: cutoff * the last hidden activations, c h, as the fused convolution's MFMA operand: for each K step s
        # of 32 and lane group q, the eight values at K positions 8 q .. 8 q + 7 (features 32 s + 16 t + 4 q + r, the
        # _kperm order, which is this lane's own MFMA result layout) split exactly into three bf16 parts:
        # hc [E][S][3][4][8] uint16.  mlp_hidb: from the sum of the convolution's partial dL/d(c h) (np_ slices
        # [E, HL] in natural feature order, summed in order), dL/dcutoff = sum_j P h and dL/d(edge features) through the
        # hidden layers with dL/dh = c P
        H = head(spec.kname('mlp_hid'), 'const float* __restrict__ ef, const float* __restrict__ Wh, '
                 'const float* __restrict__ cutv, unsigned short* __restrict__ hc, long long E', Lo['tr_size'], NB_FWD)
        H += stage('Wh', Lo['tr_size']) + ['  __syncthreads();'] + xin(range(NB_FWD)) + hidden_fwd(True, True, range(NB_FWD))
        for b in range(NB_FWD):
            hl = f'h{nh - 1}_{b}'
            H += [f'  if (live{b}) {{', f'    const float cb = cutv[ej{b}];']
            for st in range(S):
                H += [f'    {{ const float v[8] = {{{", ".join(f"cb * {hl}[{2 * st + tt}][{r}]" for tt in range(2) for r in range(4))}}};',
                      '      mh_bf8 sp[3];',
                      '      mh_split8(v, sp);',
                      f'      mh_bf8* __restrict__ dst = reinterpret_cast<mh_bf8*>(hc) + (ej{b} * {S} + {st}) * 12 + q;']
                H += [f'      dst[{4 * p}] = sp[{p}];' for p in range(3)]
                H += ['    }']
            H.append('  }')
        L.extend(H + ['}', ''])
        grp = range(NB_BWD)
        H = head(spec.kname('mlp_hidb'), 'const float* __restrict__ ef, const float* __restrict__ Wh, '
                 'const float* __restrict__ gp, int np_, const float* __restrict__ cutv, float* __restrict__ gef, '
                 'float* __restrict__ gcut, long long E', Lo['nat_size'], NB_BWD)
        H += stage('Wh', Lo['nat_size']) + ['  __syncthreads();'] + xin(grp) + hidden_fwd(False, False, grp)
        for b in grp:
            H += [f'  mh_f4 dhs_{b}[{TL}];'] + [f'  dhs_{b}[{o}] = mh_f4{{0.f, 0.f, 0.f, 0.f}};' for o in range(TL)]
            H += ['  for (int pp = 0; pp < np_; ++pp) {',
                  f'    const float* __restrict__ gr = gp + ((size_t)pp * E + ejc{b}) * {HL} + 4 * q;']
            H += [f'    dhs_{b}[{o}] += *reinterpret_cast<const mh_f4*>(gr + {16 * o});' for o in range(TL)]
            H += ['  }', '  {', '    float gc = 0.f;']
            for o in range(TL):
                for r in range(4):
                    H.append(f'    {{ const float z = z{nh - 1}_{b}[{o}][{r}]; '
                             f'gc = fmaf(dhs_{b}[{o}][{r}], {_lit(spec.c[nh - 1])} * z * mlp_sig(z), gc); }}')
            H += ['    gc += __shfl_xor(gc, 16, 64);', '    gc += __shfl_xor(gc, 32, 64);',
                  f'    if (live{b} && q == 0) gcut[ej{b}] = gc;',
                  f'    const float cb = cutv[ejc{b}];']
            H += [f'    dhs_{b}[{o}] *= cb;' for o in range(TL)]
            H += ['  }']
        H += walk_back(grp, 'dhs_')
        L.extend(H + ['}', ''])

    def h3_kernel(name):
        """mlp_h3: slot i < count (edge rows[i]): the last hidden activations, fp32, into h3 [E][HL] at row i with
        the features in the output layer's K order (_kperm: position 32 s + 8 q + 4 t + r holds feature
        32 s + 16 t + 4 q + r, which is what lane group q holds after the last hidden layer: two float4 stores per K
        step of 32)."""
        H = head(name, 'const float* __restrict__ ef, const float* __restrict__ Wh, float* __restrict__ h3, long long E',
                 Lo['tr_size'], 1, indexed=True)
        H += skip_block(1, zero_rows=False)
        H += xin(range(1))                   # the row's features are loaded while the weights are staged
        H += stage('Wh', Lo['tr_size']) + ['  __syncthreads();']
        H += hidden_fwd(True, True, range(1))
        H += ['  if (do0) {']
        H += [f'    *reinterpret_cast<mh_f4*>(h3 + ej0 * {HL} + {32 * st + 4 * tt} + 8 * q) = h{nh - 1}_0[{2 * st + tt}];'
              for st in range(S) for tt in range(2)]
        H += ['  }', '}', '']
        return H

    def out_kernel(name):
        """mlp_out: the output layer over h3, weight-stationary.  A workgroup is 4 waves on 4 consecutive 64-column
        blocks (a column group of 256 columns); each wave keeps its block of the split output layer in registers for
        the whole launch.  The 16-slot tiles are cut into eight contiguous shares, one per XCD (the dispatcher sends
        workgroup b to XCD b % 8), and the XCD's workgroups split its tiles between them: with G workgroups on the XCD
        (the host makes G a multiple of the NCG column groups), workgroup g takes column group g % NCG and tiles
        g / NCG, + G / NCG, ....  Per tile the workgroup loads the 16 rows of h3 once (one float4 per thread, loaded
        a tile ahead), splits them into bf16 parts and writes them to LDS as the MFMA's B operand fragments (two
        buffers, one barrier per tile); every wave reads its six fragments with 16-byte reads and stores its 64
        columns of the 16 rows as one float4 per lane and column tile."""
        CT = WS_COLS // 16
        NCB = -(-NW // WS_COLS)
        NCG = -(-NCB // 4)
        TAILT = (NW % WS_COLS) // 16
        KS = HL // 32
        FR = KS * 3 * 64 * 8                                 # bf16 per tile of operand fragments
        assert HL == 64, 'mlp_out stages one float4 of h3 per thread: HL must be 64'
        SO = WS_STAGE_OUT and NW % (4 * WS_COLS) == 0        # staged stores: whole 256-column groups only
        OS = 4 * WS_COLS + 16                                # floats per staged row: 16 mod 64 banks apart
        F = [f'extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu({WS_WAVES}))) '
             f'void {name}(const float* __restrict__ h3, const unsigned short* __restrict__ Wo, float* __restrict__ W0, '
             'long long E, const int* __restrict__ rows, const int* __restrict__ count) {',
             f'  __shared__ __align__(16) unsigned short frag[2][{FR}];']
        if SO:
            # tile tt's 16 rows x 256 columns, written by the four waves, stored in the next iteration (after its
            # barrier) as one 1 KB row piece per store instruction, wave w taking rows 4 w .. 4 w + 3
            F += [f'  __shared__ __align__(16) float otile[2][16][{OS}];']
        F += [
             '  const int t = threadIdx.x, lane = t & 63, q = lane >> 4, c16 = lane & 15;',
             '  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);',
             '  const long long ncount = count ? (long long)count[0] : E;',
             '  const long long T = (ncount + 15) / 16;',
             '  const int nx8 = gridDim.x < 8 ? (int)gridDim.x : 8;        // XCDs the grid reaches (round-robin)',
             '  const int xcd = (int)blockIdx.x % nx8;',
             '  const int G = ((int)gridDim.x - xcd + nx8 - 1) / nx8;      // workgroups on this XCD',
             '  const int g = (int)blockIdx.x / nx8;',
             '  const long long t0 = T * xcd / nx8, Tx = T * (xcd + 1) / nx8 - t0;   // this XCD\'s tiles',
             '  // G >= NCG: workgroup g keeps column group g % NCG and takes tiles g / NCG, + G / NCG, ... (the workgroups',
             '  // past the last whole set of NCG idle); G < NCG: workgroup g takes column groups g, g + G, ... and every tile',
             f'  const int nsub = G / {NCG};',
             f'  if (nsub > 0 && g >= nsub * {NCG}) return;',
             f'  const int cg0 = nsub > 0 ? g % {NCG} : g, cgs = nsub > 0 ? {NCG} : G;',
             f'  const long long sub = nsub > 0 ? g / {NCG} : 0, step = nsub > 0 ? nsub : 1;',
             '  if (sub >= Tx) return;',
             '  // the staging thread\'s piece of a tile: slot t / 16, K positions 4 u .. 4 u + 3 (u = t % 16), i.e. half',
             '  // u % 2 of lane group (u / 2) % 4\'s fragment at K step u / 8',
             '  const int ps = t >> 4, pu = t & 15, pks = pu >> 3, pq = (pu >> 1) & 3, ph = pu & 1;',
             f'  for (int cg = cg0; cg < {NCG}; cg += cgs) {{',
             '    const int cb = 4 * cg + wave;                              // uniform; a block past NCB computes nothing',
             f'    const bool act = cb < {NCB};',
             f'    mh_bf8 a[{CT}][{KS}][3];',
             '    if (act) {',
             f'      const mh_u4* __restrict__ src = reinterpret_cast<const mh_u4*>(Wo) + (size_t)cb * {CT * KS * 3 * 64} + lane;']
        F += [f'      a[{ct}][{ks}][{p}] = __builtin_bit_cast(mh_bf8, src[{((ct * KS + ks) * 3 + p) * 64}]);'
              for ct in range(CT) for ks in range(KS) for p in range(3)]
        F += ['    } else {']
        F += [f'      a[{ct}][{ks}][{p}] = __builtin_bit_cast(mh_bf8, mh_u4{{0u, 0u, 0u, 0u}});'
              for ct in range(CT) for ks in range(KS) for p in range(3)]
        F += ['    }',
              '    long long tt = sub;',
              '    // a tile\'s staging piece and this lane\'s edge row, loaded a tile ahead (clamped: every load in range)',
              '    auto piece = [&](long long tile) {',
              '      const long long s2 = (t0 + tile) * 16 + ps;',
              f'      return *reinterpret_cast<const mh_f4*>(h3 + (s2 < ncount ? s2 : ncount - 1) * {HL} + 4 * pu);',
              '    };',
              '    auto erow = [&](long long tile) {',
              '      const long long s2 = (t0 + tile) * 16 + c16;',
              '      const long long sc = s2 < ncount ? s2 : ncount - 1;',
              '      return rows ? rows[sc] : (int)sc;',
              '    };',
              '    mh_f4 pc = piece(tt);',
              '    int rc = erow(tt);',
              '    int buf = 0;'] + (['    long long tp = -1;                   // the tile staged in buf ^ 1, stored next',
                                     '    int rp = 0;'] if SO else []) + [
              '    while (true) {',
              '      const long long nx = tt + step;',
              '      const long long tn = nx < Tx ? nx : tt;',
              '      const mh_f4 pn = piece(tn);',
              '      const int rn = erow(tn);',
              '      // tile tt\'s piece, split exactly into three bf16 parts, into its fragments in LDS buffer buf; lane',
              '      // (q, c16) of fragment (ks, p) sits at q * 16 + (c16 ^ (8 ks + 2 q)): each half-wave\'s 8-byte writes',
              '      // then hit 64 different banks, and each wave\'s 16-byte reads of a fragment stay one 1 KB block',
              '      {',
              '        unsigned pk[3][2];',
              '#pragma unroll',
              '        for (int j = 0; j < 4; j += 2) {',
              '          unsigned bb[2][3];',
              '#pragma unroll',
              '          for (int e = 0; e < 2; ++e) {',
              '            const unsigned hbits = __float_as_uint(pc[j + e]) & 0xFFFF0000u;',
              '            const float r1 = pc[j + e] - __uint_as_float(hbits);',
              '            const unsigned mbits = __float_as_uint(r1) & 0xFFFF0000u;',
              '            const float r2 = r1 - __uint_as_float(mbits);',
              '            bb[e][0] = hbits >> 16;',
              '            bb[e][1] = mbits >> 16;',
              '            bb[e][2] = __float_as_uint(r2) >> 16;',
              '          }',
              '#pragma unroll',
              '          for (int p = 0; p < 3; ++p) pk[p][j / 2] = bb[0][p] | (bb[1][p] << 16);',
              '        }',
              '#pragma unroll',
              '        for (int p = 0; p < 3; ++p)',
              '          *reinterpret_cast<uint2*>(&frag[buf][((pks * 3 + p) * 64 + pq * 16 + (ps ^ (8 * pks + 2 * pq))) * 8 + '
              '4 * ph]) = uint2{pk[p][0], pk[p][1]};',
              '      }',
              '      __syncthreads();',
              '      if (act) {',
              f'        mh_bf8 b[{KS}][3];']
        F += [f'        b[{ks}][{p}] = *reinterpret_cast<const mh_bf8*>(&frag[buf][(({ks} * 3 + {p}) * 64 + q * 16 + '
              f'(c16 ^ ({8 * ks} + 2 * q))) * 8]);' for ks in range(KS) for p in range(3)]
        F += [f'        mh_f4 acc[{CT}];'] + [f'        acc[{ct}] = mh_f4{{0.f, 0.f, 0.f, 0.f}};' for ct in range(CT)]
        for ks in range(KS):
            for pa, pb in PAIRS:
                for ct in range(CT):
                    F.append(f'        acc[{ct}] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[{ct}][{ks}][{pa}], b[{ks}][{pb}], '
                             f'acc[{ct}], 0, 0, 0);')
        if SO:
            def store_rows(ind, ob, tile, rcv):
                """Rows 4 wave .. 4 wave + 3 of staged tile ``tile`` (buffer ``ob``, lane edge rows ``rcv``)."""
                R = []
                for i in range(4):
                    R += [f'{ind}{{ const int j = 4 * wave + {i};',
                          f'{ind}  if ((t0 + {tile}) * 16 + j < ncount) {{',
                          f'{ind}    const long long rj = __builtin_amdgcn_readlane({rcv}, j);',
                          f'{ind}    *reinterpret_cast<mh_f4*>(W0 + rj * {NW} + cg * {4 * WS_COLS} + 4 * lane) = '
                          f'*reinterpret_cast<const mh_f4*>(&otile[{ob}][j][4 * lane]);',
                          f'{ind}  }}',
                          f'{ind}}}']
                return R
            F += ['        {',
                  '        if (tp >= 0) {                       // the previous tile, staged before this barrier']
            F += store_rows('          ', 'buf ^ 1', 'tp', 'rp')
            F += ['        }']
            F += [f'        *reinterpret_cast<mh_f4*>(&otile[buf][c16][wave * {WS_COLS} + {16 * ct} + 4 * q]) = acc[{ct}];'
                  for ct in range(CT)]
        else:
            F += ['        if ((t0 + tt) * 16 + c16 < ncount) {',
                  f'          float* __restrict__ dst = W0 + (long long)rc * {NW} + cb * {WS_COLS} + 4 * q;']
            for ct in range(CT):
                guard = f'if (cb < {NCB - 1}) ' if TAILT and ct >= TAILT else ''
                F.append(f'          {guard}*reinterpret_cast<mh_f4*>(dst + {16 * ct}) = acc[{ct}];')
        F += ['        }',
              '      }',
              '      if (nx >= Tx) break;'] + (['      tp = tt;', '      rp = rc;'] if SO else []) + [
              '      tt = nx;',
              '      pc = pn;',
              '      rc = rn;',
              '      buf ^= 1;',
              '    }',
              '    __syncthreads();                     // every wave is done with the buffers before the next group']
        if SO:
            F += store_rows('    ', 'buf', 'tt', 'rc')       # the last tile (its staging complete at the barrier)
        F += ['  }',
              '}', '']
        return F

    if second:
        L += fwd_kernel(spec.kname('mlp_jvp'), True) + bwd_kernel(spec.kname('mlp_bwd2'), True)
    else:
        L += fwd_kernel(spec.kname('mlp_fwd'), False) + bwd_kernel(spec.kname('mlp_bwd'), False)
        L += bwd_kernel(spec.kname('mlp_bwdp'), False, paired=True)
        hidden_only()
        L += h3_kernel(spec.kname('mlp_h3')) + out_kernel(spec.kname('mlp_out'))
    return '\n'.join(L)


def packed_weights(spec):
    """Weight buffers: {'fwd': (hidden transposed fp32, output layer bf16 chunks), 'bwd': (hidden natural fp32,
    output layer bf16 chunks)}.  Hidden layer i is laid out as the kernel's LDS copy: natural [k][j + PAD] (the first
    layer's K padded to a multiple of 4 with zero rows) or transposed [j][k + TPAD] (TPAD0 for the first layer).  The output layer W [HL, NW] is
    split exactly into three bf16 parts (uint16 bit patterns) and cut into chunks of CH_FWD / CH_BWD columns (the last
    zero-padded): forward [chunk][3][HL / 8][CH_FWD][8] with K in the ``_kperm`` order, backward
    [chunk][3][CH_BWD / 8][HL][8] (16-byte groups of a row, rows innermost)."""
    Lo = _layout(spec)
    nat = np.zeros(Lo['nat_size'])
    tr = np.zeros(Lo['tr_size'])
    for i, A in enumerate(spec.A[:-1]):
        r, c = Lo['rows'][i], Lo['cols'][i]
        buf = np.zeros((r, c + PAD))
        buf[:A.shape[0], :c] = A
        nat[Lo['nat'][i]:Lo['nat'][i] + buf.size] = buf.reshape(-1)
        bt = np.zeros((c, r + _tpad(i)))
        bt[:, :A.shape[0]] = A.T
        tr[Lo['tr'][i]:Lo['tr'][i] + bt.size] = bt.reshape(-1)
    HL, NW = spec.A[-1].shape

    def padded(CH):                                          # zero columns up to a whole chunk
        w = np.zeros((HL, -(-NW // CH) * CH), dtype=np.float32)
        w[:, :NW] = spec.A[-1]
        return bf16_split3(w), w.shape[1] // CH
    perm = _kperm(HL)
    parts, n = padded(CH_FWD)
    fwd = np.stack([p.reshape(HL, n, CH_FWD).transpose(1, 2, 0)[:, :, perm] for p in parts], axis=1)
    fwd = fwd.reshape(n, 3, CH_FWD, HL // 8, 8).transpose(0, 1, 3, 2, 4)        # rows innermost (see chunk_io)
    parts, n = padded(CH_BWD)
    bwd = np.stack([p.reshape(HL, n, CH_BWD).transpose(1, 0, 2) for p in parts], axis=1)
    bwd = bwd.reshape(n, 3, HL, CH_BWD // 8, 8).transpose(0, 1, 3, 2, 4)
    # weight-stationary forward: [ncb][ct][ks][part][lane][8], lane = 16 q + c16 holding output column
    # 64 cb + 16 ct + c16 at K positions 32 ks + 8 q .. + 7 (hidden features in the _kperm order)
    ncb, KS = -(-NW // WS_COLS), HL // 32
    w = np.zeros((HL, ncb * WS_COLS), dtype=np.float32)
    w[:, :NW] = spec.A[-1][perm]                             # K position -> hidden feature, as mlp_h3 writes hb
    ws = np.stack([p.reshape(KS, 4, 8, ncb, WS_COLS // 16, 16).transpose(3, 4, 0, 1, 5, 2)
                   .reshape(ncb, WS_COLS // 16, KS, 64, 8) for p in bf16_split3(w)], axis=3)
    return {'fwd': (tr.astype(np.float32), np.ascontiguousarray(fwd).reshape(-1)),
            'bwd': (nat.astype(np.float32), np.ascontiguousarray(bwd).reshape(-1)),
            'ws': np.ascontiguousarray(ws).reshape(-1)}


_DOUBLE_BACKWARD = ('mace_hip_kernels: double backward (create_graph=True, e.g. training on forces/stress or an '
                    'autograd Hessian) is not enabled for this HIP module; patch with '
                    'patch_model(model, double_backward=True)')


def _mlp_bwd(op, ef, g, rows=None, count=None):
    """dL/d(edge features) [E, n_basis] from dL/dW0 (contiguous 2-D operands).  With a row list (``rows``,
    ``count`` from ``conv.support_rows``) only the first count[0] listed edges are computed; the others get zero rows
    and their dL/dW0 rows are not read."""
    gx = torch.empty_like(ef)
    P = _native.ptr
    op.bwd_paired = False
    _native.launch(f'mlp_bwd[{op.tag}]', _native.load().mh_mlp_bwd_rows, op.module.handle, P(ef), P(op.Wh), P(op.Wl),
                   P(g), P(gx), ef.shape[0], P(rows), P(count), _native.stream_of(ef))
    return gx


def _mlp_bwd_pairs(op, ef, g, rows, count, partner):
    """dL/d(edge features) over the rows shared between an edge and its exact reverse (``conv.support_pairs`` with
    the edge vectors): the row of each computed slot's edge e receives J(ef[e])^T (g[e] + g[partner[e]]) and every
    other edge a zero row.  Each pair's two rows add up to what ``_mlp_bwd`` gives them; only that sum reaches the
    positions (the two lengths are equal and their vectors opposite)."""
    gx = torch.empty_like(ef)
    P = _native.ptr
    op.bwd_paired = True
    _native.launch(f'mlp_bwd[{op.tag}]', _native.load().mh_mlp_bwd_pairs, op.module.handle, P(ef), P(op.Wh),
                   P(op.Wl), P(g), P(gx), ef.shape[0], P(rows), P(count), P(partner), _native.stream_of(ef))
    return gx


def mlp_forward(op, ef, rows=None, count=None):
    """W0 = MLP(ef) [E, n_out] (ef contiguous [E, n_basis]); with a row list only the first count[0] listed edges'
    rows are computed and written (the other rows of W0 are left unset)."""
    out = torch.empty(ef.shape[0], op.spec.hs[-1], device=ef.device, dtype=torch.float32)
    P = _native.ptr
    if WS_FWD and op.spec.hs[-1] >= WS_MIN_COLS:
        h3 = torch.empty(ef.shape[0], op.spec.hs[-2], device=ef.device, dtype=torch.float32)
        _native.launch(f'mlp_fwd[{op.tag}]', _native.load().mh_mlp_fwd_ws, op.module.handle, P(ef), P(op.WhT),
                       P(op.Wo), P(h3), P(out), ef.shape[0], P(rows), P(count), op.ncb, _native.stream_of(ef))
    else:
        _native.launch(f'mlp_fwd[{op.tag}]', _native.load().mh_mlp_fwd_rows, op.module.handle, P(ef), P(op.WhT),
                       P(op.WlT), P(out), ef.shape[0], P(rows), P(count), _native.stream_of(ef))
    op.last_rows = count if count is not None else ef.shape[0]     # rows computed: device count or all
    return out


class _MLPFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, ef, op):
        s = op.spec
        if ef.dtype != torch.float32 or not ef.is_cuda:
            raise TypeError('mace_hip_kernels: the radial MLP expects float32 GPU input')
        if ef.shape[-1] != s.hs[0]:
            raise ValueError(f'expected [..., {s.hs[0]}] edge features, got {tuple(ef.shape)}')
        lead = ef.shape[:-1]
        out = mlp_forward(op, ef.reshape(-1, s.hs[0]).contiguous())
        ctx.save_for_backward(ef)            # the input itself: a double backward differentiates through it
        ctx.op, ctx.lead = op, lead
        return out.reshape(*lead, s.hs[-1])

    @staticmethod
    def backward(ctx, g):
        ef, = ctx.saved_tensors
        op = ctx.op
        s = op.spec
        if torch.is_grad_enabled():          # only true under create_graph=True
            if not op.double_backward:
                raise RuntimeError(_DOUBLE_BACKWARD)
            return _MLPAdjFn.apply(g, ef, op), None
        x = ef.reshape(-1, s.hs[0]).contiguous()
        gx = _mlp_bwd(op, x, g.reshape(-1, s.hs[-1]).contiguous())
        return gx.reshape(*ctx.lead, s.hs[0]), None


class _MLPAdjFn(torch.autograd.Function):
    """dL/def = J(ef)^T g as a function of (g, ef), for a double backward: with ggx the gradient arriving for dL/def,
    d<ggx, J^T g>/dg = J(ef) ggx (``mlp_jvp``) and d<ggx, J^T g>/def = sum_k g_k d^2 W0_k/def^2 ggx (``mlp_bwd2``).
    Third derivatives are not provided."""

    @staticmethod
    def forward(ctx, g, ef, op):
        s = op.spec
        ctx.save_for_backward(g, ef)
        ctx.op = op
        x = ef.reshape(-1, s.hs[0]).contiguous()
        return _mlp_bwd(op, x, g.reshape(-1, s.hs[-1]).contiguous()).reshape(ef.shape)

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, ggx):
        g, ef = ctx.saved_tensors
        op = ctx.op
        s = op.spec
        m = op.second_module()
        x = ef.reshape(-1, s.hs[0]).contiguous()
        v = ggx.reshape(-1, s.hs[0]).contiguous()
        E, P, lib, st = x.shape[0], _native.ptr, _native.load(), _native.stream_of(x)
        d_g = d_ef = None
        if ctx.needs_input_grad[0]:
            dW = torch.empty(E, s.hs[-1], device=x.device, dtype=torch.float32)
            _native.launch(f'mlp_jvp[{op.tag}]', lib.mh_mlp_jvp, m.handle, P(x), P(v), P(op.WhT), P(op.WlT), P(dW), E,
                           st)
            d_g = dW.reshape(g.shape)
        if ctx.needs_input_grad[1]:
            gv = torch.empty_like(x)
            _native.launch(f'mlp_bwd2[{op.tag}]', lib.mh_mlp_bwd2, m.handle, P(x), P(v), P(op.Wh), P(op.Wl),
                           P(g.reshape(-1, s.hs[-1]).contiguous()), P(gv), E, st)
            d_ef = gv.reshape(ef.shape)
        return d_g, d_ef, None


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
                _native.MH_MLP_FWD: (self.spec.kname('mlp_fwd'), BLOCK, 64 * NB_FWD),
                _native.MH_MLP_BWD: (self.spec.kname('mlp_bwd'), 64 * WG_WAVES_BWD, 16 * NB_BWD * WG_WAVES_BWD),
                _native.MH_MLP_BWD_P: (self.spec.kname('mlp_bwdp'), 64 * WG_WAVES_BWD, 16 * NB_BWD * WG_WAVES_BWD),
                _native.MH_MLP_HID: (self.spec.kname('mlp_hid'), BLOCK, 64 * NB_FWD),
                _native.MH_MLP_HIDB: (self.spec.kname('mlp_hidb'), BLOCK, 64 * NB_BWD),
                _native.MH_MLP_H3: (self.spec.kname('mlp_h3'), BLOCK, 64),
                _native.MH_MLP_OUT: (self.spec.kname('mlp_out'), BLOCK, 1),
            })
        self.ncb = -(-self.spec.hs[-1] // WS_COLS)
        pw = packed_weights(self.spec)
        for name, arr in (('WhT', pw['fwd'][0]), ('WlT', pw['fwd'][1]), ('Wh', pw['bwd'][0]), ('Wl', pw['bwd'][1]),
                          ('Wo', pw['ws'])):
            # the bf16 parts travel as int16 bit patterns (the kernels read them as raw 16-bit words)
            arr = arr.view(np.int16) if arr.dtype == np.uint16 else arr
            self.register_buffer(name, torch.from_numpy(np.ascontiguousarray(arr)).to(dev), persistent=False)
        self.hs = self.spec.hs
        self.original = [mod]
        self.tag = 'radial_mlp'
        self._device = dev
        # a backward under create_graph=True raises (the reference's behaviour) unless this is set; then the
        # gradient is differentiable once more through the second-order kernels (second_module)
        self.double_backward = False
        self._second = None
        # set by patch_model when the convolution fed by this MLP forms its weights itself (HipConvTP.attach_mlp):
        # the output is then returned unformed
        self.fuse = False

    def second_module(self):
        """The module of the second-order kernels (``mlp_jvp``, ``mlp_bwd2``), compiled on first use."""
        if self._second is None:
            code = _native.compile_source(source_second(self.spec))
            with torch.cuda.device(self._device):
                self._second = _native.Module(code, {
                    _native.MH_MLP_JVP: (self.spec.kname('mlp_jvp'), BLOCK, 64 * NB_JVP),
                    _native.MH_MLP_BWD2: (self.spec.kname('mlp_bwd2'), BLOCK, 64 * NB_BWD)})
        return self._second

    def forward(self, ef):
        if self.fuse and ef.dim() == 2 and ef.shape[1] == self.spec.hs[0]:
            from .conv_mlp import PendingRadial
            return PendingRadial((ef.shape[0], self.spec.hs[-1]), ef, ef, self)
        # the output's product with MACE's cutoff column is handed to the convolution unformed (conv.RadialWeights)
        return _MLPFn.apply(ef, self).as_subclass(_conv.RadialWeights)

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
from .symmetric import element_order
from .pending import Pending, set_slots, slot

KC = 32              # K per chunk: one bf16 MFMA step (input channels u of one attribute v)
CW_BF16 = 64         # output columns per workgroup of the bf16 family (64 or 128)
CW_F32 = 64          # and of the fp32 family (32 or 64).  Config 2's E+F call with 32 (two alternating runs each):
                     # 1.118 -> 1.136-1.138 ms, the 512 -> 512 forward 14 -> 16 us, lin_bwds 17.4 -> 25.5 us
BF16_MIN_OUT = 1024  # outputs (inputs, backward) from which a direction runs on the bf16 family (the config-2 call
                     # measured 2 us slower with the 512-wide maps on it, 4 us with every map)
BLOCK = 256          # 4 waves
WAVES = BLOCK // 64
ROWS = 16            # rows (node, m) of an MFMA row tile
NT = 1               # row tiles per wave, bf16 family: each LDS weight fragment feeds NT MFMAs
WC_BF16 = 1          # column groups of waves, bf16 family: the workgroup's waves form (4 / WC) x WC, each wave
                     # NT * WC row tiles by CT / WC column tiles of the workgroup's tile; 1: every wave takes all
                     # columns.  Config 2's E+F call, all linears per call (two alternating runs): WC 1 240.5 / 246.1
                     # us, 2 249.1 / 246.5 us (a third fewer LDS operand reads, twice the input splits per wave),
                     # 4 287.8 / 288.2 us; results bitwise equal
NT_ATTRS = 1         # the same for skip_tp (attribute terms)
PREFETCH_BF16 = 2    # chunks whose global loads are in flight ahead of the one being multiplied (1, 2 or 4), bf16 family
LIN_XCD = False      # node-group-major, XCD-contiguous workgroup order (see _block_map).  Measured slower: config
                     # 2's call 1.131-1.134 -> 1.191 ms, the 5120 -> 2048 linear 41 -> 55 us, the composed
                     # 2048 -> 2048 26.5 -> 37.5 us.  The weight chunks are the larger stream: in the hardware's
                     # order (blockIdx.x fastest) the workgroups running together share one (block, column group)
                     # slice of weights in L2, while their inputs come from memory once per column group
TILES_MIN_CHUNKS = 8 # fp32 family: K chunks (32 input channels of one attribute) from which a block runs one tile per
                     # wave over the whole K loop instead of splitting K over the workgroup's waves.  Config 2's E+F
                     # call with 4 (the 128-channel maps on one tile per wave; two alternating runs each): the
                     # 512 -> 512 forward 13.8 -> 16.5-21.6 us, lin_bwds 17.4 -> 20.4 us, all linears 242-244 ->
                     # 253-269 us per call; results within the same parity
XPAD = 4             # floats of padding per LDS row of staged inputs
WPAD = 8             # bf16 of padding per LDS row of staged weights


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
        self.suffix = ''
        self._build(_probe(mod, self))

    @classmethod
    def compose(cls, first, second):
        """The spec of ``second`` applied to the output of ``first`` (an attribute-free linear): per input block i,
        output block o and attribute v, W_io = sum_j W1_ij W2_jo[v] over the blocks j between them, formed in
        float64 from the two probed maps (MACE's first interaction block: skip_tp(linear(message)), whose middle
        tensor then never exists)."""
        if first.V or first.out_blocks != second.in_blocks:
            raise ValueError('maps do not compose: the first must be attribute-free with the second\'s input blocks')
        self = cls.__new__(cls)
        self.kind = second.kind
        self.in_blocks, self.Din = first.in_blocks, first.Din
        self.out_blocks, self.Dout = second.out_blocks, second.Dout
        self.V = second.V
        self.suffix = 'c'
        Wio = {}
        for (i, j), w1 in first.Wio.items():
            for (jj, o), w2 in second.Wio.items():
                if jj == j:
                    w = np.einsum('ut,tvw->uvw', w1[:, 0, :], w2)
                    Wio[(i, o)] = Wio[(i, o)] + w if (i, o) in Wio else w
        self._build(Wio)
        return self

    def _build(self, Wio):
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
        # what the kernels stream: exact bf16 splits in chunk order (forward: W_io; backward: its transpose)
        self.pack_fwd = pack(self.out_blocks, self.terms, self.in_blocks, Wio, self.V)
        self.pack_bwd = pack(self.in_blocks, self.bterms, self.out_blocks,
                             {(o, i): np.ascontiguousarray(w.transpose(2, 1, 0)) for (i, o), w in Wio.items()}, self.V)
        # the tiled backward writes the input blocks with the same tiling: their multiplicities must tile too; the
        # others (the node embedding of one-hot element attributes) get a plain one-thread-per-value backward
        self.tiled_bwd = all(m % 16 == 0 for m, *_ in self.in_blocks)

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
        return f'{base}_i{self.Din}_o{self.Dout}' + (f'_v{self.V}' if self.V else '') + self.suffix

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


def _cw(mo, cmax=64):
    """Columns per workgroup: up to cmax (the fp32 family 64, i.e. 4 MFMA column tiles; the bf16 family CW_BF16)
    where the multiplicity allows."""
    for c in (128, 64, 32):
        if c <= cmax and mo % c == 0:
            return c
    return 16


def _grid_y(blocks, cmax=64):
    """(block, column group) pairs of one direction, in blockIdx.y order."""
    return [(o, cg) for o, (mo, *_) in enumerate(blocks) for cg in range(mo // _cw(mo, cmax))]


def _tiles(V):
    """Row tiles per wave of the bf16 family: NT, or NT_ATTRS for attribute terms (skip_tp).  Measured on config 2:
    the 2048 -> 2048 x 4-element skip_tp takes 37.9 us with two tiles per wave and 28.3 us with one (twice the
    workgroups hide the attribute-mask prologue); the captured E+F call is 5 us faster with one tile per wave for
    the attribute-free linears as well."""
    return NT_ATTRS if V else NT


def _group(l, nt=NT):
    """(nodes per row tile, nodes per workgroup) for output irreps of degree l: a tile is 16 // (2l + 1) whole
    nodes (<= 16 rows (node, m)), each wave holds nt tiles."""
    tn = ROWS // (2 * l + 1)
    return tn, WAVES * nt * tn


def _nodes_per_launch_group(blocks, nt=NT):
    """Nodes per workgroup of the launch: the smallest over the output blocks (blocks with more nodes per workgroup
    leave their trailing workgroups idle)."""
    return min(_group(l, nt)[1] for _, l, *_ in blocks)


def pack(blocks, terms, in_blocks, wmats, V):
    """The weights of one direction as the kernel streams them: for output block o, column group cg (CW columns),
    term (input block i), attribute v and chunk uc of 32 input channels, the [32, CW] slice of W_io[u, v, w]
    (rows past mul_i zero) split exactly into three bf16 parts and stored [part][k / 8][column][8] (uint16 bit
    patterns).
    Returns (flat array, {(o, cg): element offset}, {o: [element offset of each term within a column group]})."""
    from .radial import bf16_split3
    VV = max(V, 1)
    out, base, toffs, off = [], {}, {}, 0
    for o, (mo, l, oo, _) in enumerate(blocks):
        CW = _cw(mo, CW_BF16)
        offs, t = [], 0
        for i, _ in terms[o]:
            offs.append(t)
            t += VV * -(-in_blocks[i][0] // KC) * 3 * CW * KC
        toffs[o] = offs
        for cg in range(mo // CW):
            base[(o, cg)] = off
            for i, _ in terms[o]:
                w = wmats[(i, o)]                                   # [mi, VV, mo]
                mi = w.shape[0]
                for v in range(VV):
                    for uc in range(-(-mi // KC)):
                        blk = np.zeros((KC, CW), dtype=np.float32)
                        rows = w[uc * KC:(uc + 1) * KC, v, cg * CW:(cg + 1) * CW]
                        blk[:rows.shape[0]] = rows
                        # [part][k / 8][column][8]: columns innermost, so the eight lanes of an LDS write phase
                        # hit eight different rows of the staged chunk (conflict-free)
                        out += [p.T.reshape(CW, KC // 8, 8).transpose(1, 0, 2).reshape(-1) for p in bf16_split3(blk)]
                        off += 3 * CW * KC
    flat = np.concatenate(out) if out else np.zeros(8, dtype=np.uint16)
    return flat, base, toffs


def _block_map():
    """The kernel's (node group, case) from its workgroup: with LIN_XCD from the dispatch position, node-group major
    and XCD-contiguous (``mh_xcd_block``), so that the cases of one node group, which read the same input rows, run
    one after another on one XCD and find those rows in its L2; else (blockIdx.x, blockIdx.y)."""
    if not LIN_XCD:
        return ['  const int group = blockIdx.x, y = blockIdx.y;']
    return ['  const int P = mh_xcd_block(blockIdx.x + gridDim.x * blockIdx.y, gridDim.x * gridDim.y);',
            '  const int group = P / gridDim.y, y = P - group * gridDim.y;']


def _kernel(name, in_blocks, out_blocks, terms, V, Din, Dout, base, toffs):
    """HIP source of one direction.  blockIdx.y selects (output block o, column group of CW channels), blockIdx.x a
    group of nodes: four waves of NT row tiles, a row tile being 16 // d whole nodes (<= 16 rows (node, m)).

    K is walked in chunks of 32 input channels of one (input block, attribute v) term.  Per chunk the workgroup
    stages, double-buffered in LDS, the chunk's inputs of its nodes (coalesced float4 loads, transposed to rows
    (node, m) x 32 channels) and the chunk's weights (the host's exact three-way bf16 split, [part][column][k]);
    the next chunk's loads are in flight in registers meanwhile.  Each wave splits its rows into bf16 parts (times
    the attribute a[n, v] for skip_tp) and sums the six leading partial products on v_mfma_f32_16x16x32_bf16 (fp32
    accuracy, 2.7x the fp32 matrix rate per K).  Attribute terms v whose a[n, v] is zero on every node of the
    workgroup are skipped (exact: they add 0).  The result tile goes through LDS and out as coalesced float4 rows
    (a node's CW d outputs of a block are contiguous)."""
    fns, cases, lds_max = [], [], 0
    VV = max(V, 1)
    NT = _tiles(V)
    for o, (mo, l, oo, _) in enumerate(out_blocks):
        D = 2 * l + 1
        TN, G = _group(l, NT)
        CW = _cw(mo, CW_BF16)
        CT = CW // 16
        WCo = WC_BF16 if CT % WC_BF16 == 0 and WAVES % WC_BF16 == 0 else 1
        TW, CTW = NT * WCo, CT // WCo                 # row tiles and column tiles per wave
        fn = f'{name}_b{o}'
        L = [f'__device__ __forceinline__ void {fn}(const float* __restrict__ x, const float* __restrict__ attr,',
             '    const unsigned short* __restrict__ W, float* __restrict__ out, int N, int group, int cg,',
             '    float* __restrict__ lds, unsigned* __restrict__ amask, int* __restrict__ vlist, float alpha,',
             '    const int* __restrict__ order, const float* __restrict__ res) {',
             f'  auto nd = [&](int i) {{ return {"order ? order[i] : " if V else ""}i; }};   // node of position i',
             '  (void)alpha; (void)order; (void)res;',
             f'  const int g0 = group * {G};                 // first node of the workgroup',
             '  if (g0 >= N) return;',
             f'  const int ng = min({G}, N - g0);',
             f'  const int t = threadIdx.x, col0 = cg * {CW};']
        if not terms[o]:
            L += [f'  for (int f = t; f < ng * {CW * D}; f += {BLOCK}) {{',
                  f'    const int nl = f / {CW * D}, j = f - nl * {CW * D};',
                  f'    const size_t at = (size_t)nd(g0 + nl) * {Dout} + {oo} + col0 * {D} + j;',
                  '    out[at] = res ? 0.f + res[at] : 0.f;',
                  '  }', '}', '']
            fns += L
            cases.append((o, fn))
            continue
        XS = KC + XPAD                               # floats per staged input row (node, m)
        WS = KC + WPAD                               # bf16 per staged weight row (column)
        XR = G * D                                   # staged input rows
        XB = XR * XS                                 # floats per input buffer
        WB = 3 * CW * WS // 2                        # floats per weight buffer
        # attribute values a[n, v] of each thread's rows for the staged chunk (skip_tp): loaded with the chunk's other
        # operands and passed through LDS, so the MFMA body never waits on a global load
        SOFF = 2 * (XB + WB)
        SB = TW * BLOCK if V else 0                  # floats per attribute buffer
        lds = max(SOFF + 2 * SB, G * CW * D)
        lds_max = max(lds_max, lds)
        NXP = G * KC * D // 4                        # float4 pieces of a chunk's inputs
        NWP = 3 * CW * KC // 8                       # 16-byte pieces of a chunk's weights
        ix, iw = -(-NXP // BLOCK), -(-NWP // BLOCK)
        L += ['  const int wave = t >> 6, lane = t & 63, q = lane >> 4, c16 = lane & 15;',
              f'  const int wr = wave / {WCo}, cb = (wave % {WCo}) * {16 * CTW};   // row group, first column',
              '  (void)lane; (void)cb;']
        if V:
            L += _mask_wave(V, 'g0', 'ng') if V <= 32 else _mask(V, 'g0', 'ng', ordered=True)
        else:
            L += ['  const int nact = 1;']
        # chunk c -> term ti (compile-time boundaries scaled by nact), attribute v, channel chunk uc
        nchs = [-(-in_blocks[i][0] // KC) for i, _ in terms[o]]
        L += [f'  const int nch = nact * {sum(nchs)};',
              f'  const unsigned short* __restrict__ Wg = W + {base[(o, 0)]} + (size_t)cg * '
              f'{toffs[o][-1] + VV * nchs[-1] * 3 * CW * KC};']
        L += ['  auto where = [&](int c, int& oi, int& mi, int& uc, int& v, int& wo) {',
              '    int r = c;']
        for k, ((i, _), nc) in enumerate(zip(terms[o], nchs)):
            mi_, _, oi_, _ = in_blocks[i]
            last = k == len(terms[o]) - 1
            cond = 'true' if last else f'r < nact * {nc}'
            L += [f'    if ({cond}) {{',
                  f'      const int vv = r / {nc};',
                  f'      uc = r - vv * {nc}; oi = {oi_}; mi = {mi_};',
                  f'      v = {("mh_kth_bit(amw, vv)" if V <= 32 else "vlist[1 + vv]") if V else "0"};',
                  f'      wo = {toffs[o][k]} + (v * {nc} + uc) * {3 * CW * KC};',
                  '      return;',
                  '    }']
            if not last:
                L.append(f'    r -= nact * {nc};')
        L += ['  };']
        # staging: thread piece it of the inputs is node nl = f / (8 D), float4 e = f % (8 D) of the node's run of
        # 32 d floats (channel-major, component-minor, as in e3nn's layout)
        # the lane's A rows: row c16 of each of its tiles (rows past the tile's nodes read row 0; never stored)
        for tt in range(TW):
            L += [f'  const int xr{tt} = {(tt) * TN * D} + wr * {TW * TN * D} + (c16 < {TN * D} ? c16 : 0);']
            if V:
                L += [f'  const int an{tt} = nd(min(g0 + xr{tt} / {D}, N - 1));']
        # node of each of the thread's input pieces, once (the chunk loop's loads then depend on no index load;
        # kept out of the loaders, whose order[] loads the compiler cannot hoist past the LDS stores)
        for k in range(ix):
            fx = f't + {k * BLOCK}' if (k + 1) * BLOCK <= NXP else f'min(t + {k * BLOCK}, {NXP - 1})'
            L += [f'  const int xn{k} = nd(min(g0 + ({fx}) / {8 * D}, N - 1));']
        SETS = 'ABCD'[:PREFETCH_BF16] if PREFETCH_BF16 > 1 else ['']
        for S in SETS:
            L += [f'  mh_f4 {", ".join(f"px{S}{k}" for k in range(ix))};',
                  f'  mh_u4 {", ".join(f"pw{S}{k}" for k in range(iw))};']
            if V:
                L += [f'  float {", ".join(f"ps{S}{tt}" for tt in range(TW))};']
            L += [f'  auto load{S} = [&](int c) {{',
                  '    int oi, mi, uc, v, wo;',
                  '    where(c, oi, mi, uc, v, wo);',
                  '    (void)v;']
            if V:
                L += [f'    ps{S}{tt} = attr[(size_t)an{tt} * {V} + v];' for tt in range(TW)]
            # float4 loads where every input block of this output block starts and ends on a 16-byte boundary (a
            # one-hot node embedding with, say, 89 elements does not): else four scalar loads
            vec = Din % 4 == 0 and all(in_blocks[i][2] % 4 == 0 and in_blocks[i][0] * D % 4 == 0 for i, _ in terms[o])
            for k in range(ix):
                fx = f't + {k * BLOCK}' if (k + 1) * BLOCK <= NXP else f'min(t + {k * BLOCK}, {NXP - 1})'
                L += [f'    {{ const int f = {fx}, nl = f / {8 * D}, e = f - nl * {8 * D};',
                      '      (void)nl;',
                      f'      const float* __restrict__ xr = x + (size_t)xn{k} * {Din} + oi;']
                if vec:     # past the block: any valid input (its weights are zero)
                    L += [f'      px{S}{k} = *reinterpret_cast<const mh_f4*>(xr + min(uc * {KC * D} + 4 * e, mi * {D} - 4)); }}']
                else:
                    L += [f'      px{S}{k}[{j}] = xr[min(uc * {KC * D} + 4 * e + {j}, mi * {D} - 1)];' for j in range(4)]
                    L[-1] += ' }'
            for k in range(iw):
                fw = f't + {k * BLOCK}' if (k + 1) * BLOCK <= NWP else f'min(t + {k * BLOCK}, {NWP - 1})'
                L += [f'    pw{S}{k} = *reinterpret_cast<const mh_u4*>(Wg + wo + (size_t)({fw}) * 8);']
            L += ['  };',
                  f'  auto store{S} = [&](int buf) {{',
                  f'    float* __restrict__ xs = lds + buf * {XB};',
                  f'    unsigned short* __restrict__ ws = reinterpret_cast<unsigned short*>(lds + {2 * XB} + buf * {WB});']
            if V:
                L += [f'    lds[{SOFF} + buf * {SB} + {tt * BLOCK} + t] = ps{S}{tt};' for tt in range(TW)]
            for k in range(ix):
                guard = '' if (k + 1) * BLOCK <= NXP else f'if (t + {k * BLOCK} < {NXP}) '
                L += [f'    {guard}{{ const int f = t + {k * BLOCK}, nl = f / {8 * D}, e = f - nl * {8 * D};']
                if D == 1:
                    L += [f'      *reinterpret_cast<mh_f4*>(xs + nl * {XS} + 4 * e) = px{S}{k}; }}']
                else:
                    L += ['#pragma unroll',
                          '      for (int j = 0; j < 4; ++j) {',
                          f'        const int idx = 4 * e + j, u = idx / {D}, m = idx - u * {D};',
                          f'        xs[(nl * {D} + m) * {XS} + u] = px{S}{k}[j];',
                          '      } }']
            for k in range(iw):
                guard = '' if (k + 1) * BLOCK <= NWP else f'if (t + {k * BLOCK} < {NWP}) '
                L += [f'    {guard}{{ const int f = t + {k * BLOCK}, p = f / {CW * KC // 8}, r = f - p * {CW * KC // 8},',
                      f'        k8 = r / {CW}, col = r - k8 * {CW};',
                      f'      *reinterpret_cast<mh_u4*>(ws + (p * {CW} + col) * {WS} + 8 * k8) = pw{S}{k}; }}']
            L += ['  };']
        L += [f'  mh_f4 acc[{TW}][{CTW}];',
              '#pragma unroll',
              f'  for (int a = 0; a < {TW}; ++a)',
              '#pragma unroll',
              f'    for (int b = 0; b < {CTW}; ++b) acc[a][b] = mh_f4{{0.f, 0.f, 0.f, 0.f}};',
]

        def body(cc, buf):
            """The MFMAs of chunk ``cc`` from LDS buffer ``buf`` (xs / ws scoped to it)."""
            B = ['    {',
                 f'    const float* __restrict__ xs = lds + ({buf}) * {XB};',
                 f'    const unsigned short* __restrict__ ws = reinterpret_cast<const unsigned short*>(lds + {2 * XB} + '
                 f'({buf}) * {WB});']
            if V:
                B += [f'    const float* __restrict__ ss = lds + {SOFF} + ({buf}) * {SB};']
            return B + BODY + ['    }']

        BODY = []
        for tt in range(TW):
            BODY += [f'    mh_bf8 a{tt}[3];',
                  '    {',
                  f'      const mh_f4 lo = *reinterpret_cast<const mh_f4*>(xs + xr{tt} * {XS} + 8 * q);',
                  f'      const mh_f4 hi = *reinterpret_cast<const mh_f4*>(xs + xr{tt} * {XS} + 8 * q + 4);']
            if V:
                BODY += [f'      const float s = ss[{tt * BLOCK} + t];',
                      '      const float v8[8] = {lo[0] * s, lo[1] * s, lo[2] * s, lo[3] * s, hi[0] * s, hi[1] * s, '
                      'hi[2] * s, hi[3] * s};']
            else:
                BODY += ['      const float v8[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};']
            BODY += [f'      mh_split8(v8, a{tt});', '    }']
        PAIRS = [(0, 0), (0, 1), (1, 0), (0, 2), (1, 1), (2, 0)]
        for ct in range(CTW):
            BODY += [f'    {{ mh_bf8 b[3];']
            BODY += [f'      b[{p}] = *reinterpret_cast<const mh_bf8*>(ws + ({p * CW + 16 * ct} + cb + c16) * {WS} + 8 * q);'
                  for p in range(3)]
            for pa, pb in PAIRS:
                for tt in range(TW):
                    BODY.append(f'      acc[{tt}][{ct}] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a{tt}[{pa}], b[{pb}], '
                             f'acc[{tt}][{ct}], 0, 0, 0);')
            BODY += ['    }']
        if PREFETCH_BF16 > 1:
            # P register sets (a ring): chunk c's loads go into set c mod P a whole P - 1 chunks before they are stored
            # to LDS buffer c mod 2 (P even, so both indices are compile-time constants in the loop unrolled by P)
            P = PREFETCH_BF16
            L += [f'  load{SETS[k]}(min({k}, nch - 1));' for k in range(P)]
            L += [f'  store{SETS[0]}(0);', '  __syncthreads();',
                  f'  for (int c = 0; c < nch; c += {P}) {{']
            for k in range(P):
                L += [f'    load{SETS[k]}(min(c + {k + P}, nch - 1));',
                      '    __builtin_amdgcn_sched_barrier(0);            // these loads go out before the MFMAs']
                L += body(f'c + {k}', f'{k % 2}')
                L += [f'    store{SETS[(k + 1) % P]}({(k + 1) % 2});',
                      '    __syncthreads();']
                if k < P - 1:
                    L += [f'    if (c + {k + 1} >= nch) break;']
            L += ['  }']
        else:
            L += ['  load(0);', '  store(0);', '  __syncthreads();',
                  '  for (int c = 0; c < nch; ++c) {',
                  '    load(min(c + 1, nch - 1));',
                  '    __builtin_amdgcn_sched_barrier(0);            // the next chunk\'s loads go out before the MFMAs']
            L += body('c', '(c & 1)')
            L += ['    store((c + 1) & 1);',
                  '    __syncthreads();',
                  '  }']
        # epilogue: lane (c16, q) holds rows 4q + r, column 16 ct + c16 of each tile -> LDS [node][column][m] ->
        # coalesced float4 rows of CW d floats per node
        L += ['#pragma unroll',
              f'  for (int tt = 0; tt < {TW}; ++tt)',
              '#pragma unroll',
              '    for (int r = 0; r < 4; ++r) {',
              '      const int row = 4 * q + r;',
              f'      if (row < {TN * D}) {{',
              f'        const int rr = tt * {TN * D} + wr * {TW * TN * D} + row, nl = rr / {D}, m = rr - nl * {D};',
              '#pragma unroll',
              f'        for (int ct = 0; ct < {CTW}; ++ct)',
              f'          lds[(nl * {CW} + cb + 16 * ct + c16) * {D} + m] = alpha * acc[tt][ct][r];',
              '      }',
              '    }',
              '  __syncthreads();',
              f'  for (int f = t; f < ng * {CW * D // 4}; f += {BLOCK}) {{',
              f'    const int nl = f / {CW * D // 4}, j = f - nl * {CW * D // 4};',
              f'    const size_t at = (size_t)nd(g0 + nl) * {Dout} + {oo} + col0 * {D} + 4 * j;',
              f'    mh_f4 v = *reinterpret_cast<const mh_f4*>(lds + nl * {CW * D} + 4 * j);',
              '    if (res) {',
              '      const mh_f4 rv = *reinterpret_cast<const mh_f4*>(res + at);',
              '      v = mh_f4{v[0] + rv[0], v[1] + rv[1], v[2] + rv[2], v[3] + rv[3]};',
              '    }',
              '    *reinterpret_cast<mh_f4*>(out + at) = v;',
              '  }',
              '}', '']
        fns += L
        cases.append((o, fn))
    gy = _grid_y(out_blocks, CW_BF16)
    VW = (V + 31) // 32
    sw = ['  switch (y) {']
    for y, (o, cg) in enumerate(gy):
        fn = dict(cases)[o]
        sw.append(f'    case {y}: {fn}(x, attr, W, out, N, group, {cg}, lds, amask, vlist, alpha, order, res); '
                  'break;')
    sw += ['    default: break;', '  }']
    lds_max = max(lds_max, 4)
    # two workgroups per CU fit the LDS; keep the registers within two waves per SIMD as well (the second prefetch
    # register set would otherwise push the count past 256 and halve the occupancy)
    occ = ' __attribute__((amdgpu_waves_per_eu(2)))' if PREFETCH_BF16 > 1 else ''
    K = [f'extern "C" __global__ __launch_bounds__({BLOCK}){occ} void {name}(const float* __restrict__ x,',
         '    const float* __restrict__ attr, const unsigned short* __restrict__ W, float* __restrict__ out, int N,',
         '    const int* __restrict__ order, float alpha, const float* __restrict__ res) {',
         '  (void)order;',
         f'  __shared__ __align__(16) float lds[{lds_max}];',
         f'  __shared__ unsigned amask[{max(VW, 1)}];',
         f'  __shared__ int vlist[{V + 1}];',
         '  (void)amask; (void)vlist;'] + _block_map() + sw + ['}', '']
    return fns + K


# ---------------------------------------------------------------- the fp32 family (short K, attribute terms)

def _tiles_mode(terms_o, in_blocks, V):
    """One tile per wave with the whole K loop (long K: the pipeline hides the load latency), or one tile per
    workgroup with K split over the waves (short K, or attribute terms: more waves in flight)."""
    return V == 0 and sum(-(-in_blocks[i][0] // KC) for i, _ in terms_o) >= TILES_MIN_CHUNKS


def _nodes_per_group(terms_o, in_blocks, V, l):
    tn = ROWS // (2 * l + 1)
    return WAVES * tn if (terms_o and _tiles_mode(terms_o, in_blocks, V)) else tn


def _loader(fn, i, in_blocks, mi, oi, D, Din, V, woff, mo, CT, NCH, nsum=1):
    """Register loads of chunk c of term i: A (x, times the attribute) and B (weights) in MFMA lane layout.
    With ``nsum`` = 3, A is the sum (x + x2) + x3 of three inputs of x's shape, added as loaded.

    K order inside a chunk: lane group kq takes k = k0 + 8 kq + st at step st, so a lane's 8 values of x are
    consecutive (two float4 loads for scalars); column order inside a group of 16 columns: lane c16 takes the CT
    adjacent columns CT c16 + ct (one vector load of W per step)."""
    VV = max(V, 1)
    vsel = f'vlist[1 + c / {NCH}]' if V else '0'
    vecx = D == 1 and Din % 4 == 0 and oi % 4 == 0 and mi % 8 == 0
    wt = {4: 'float4', 2: 'float2', 1: 'float'}[CT]
    xs3 = 'const float* __restrict__ x2, const float* __restrict__ x3, ' if nsum > 1 else ''
    L = [f'__device__ __forceinline__ void {fn}_ld{i}(const float* __restrict__ x, {xs3}const float* __restrict__ attr,',
         '    const float* __restrict__ W, const int* __restrict__ vlist, const int* __restrict__ order, int n0, int col0,',
         '    int anl, int am,'
         f'    int q, int c16, int c, float (&ra)[{KC // 4}], float (&rb)[{KC // 4}][{CT}]) {{',
         f'  const int v = {vsel}, k0 = (c % {NCH}) * {KC} + 8 * q;',
         '  (void)v; (void)vlist; (void)attr; (void)order;',
         f'  const int nr = {"order ? order[n0 + anl] : " if V else ""}n0 + anl;   // the row\'s node',
         f'  const float* __restrict__ xr = x + (size_t)nr * {Din} + {oi} + am;']
    if V:
        L.append(f'  const float s = attr[(size_t)nr * {V} + v];')
    if vecx:
        # mi % 8 == 0: the lane's 8 channels are all in range or all out of range
        L += [f'  const bool okx = k0 < {mi};',
              f'  const float4* __restrict__ xv = reinterpret_cast<const float4*>(xr + (okx ? k0 : 0));']
        if nsum > 1:
            L += [f'  const size_t xo = (size_t)nr * {Din} + {oi} + am + (okx ? k0 : 0);',
                  '  const float4* __restrict__ xv2 = reinterpret_cast<const float4*>(x2 + xo);',
                  '  const float4* __restrict__ xv3 = reinterpret_cast<const float4*>(x3 + xo);',
                  '  const float4 x0 = (xv[0] + xv2[0]) + xv3[0], x1 = (xv[1] + xv2[1]) + xv3[1];']
        else:
            L += ['  const float4 x0 = xv[0], x1 = xv[1];']
        L += [
              '  const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};']
    L += ['#pragma unroll',
          f'  for (int st = 0; st < {KC // 4}; ++st) {{',
          '    const int k = k0 + st;',
          f'    const bool ok = k < {mi};',
          f'    const int kc = ok ? k : {mi - 1};      // every load in bounds and unconditional']
    if vecx:
        L.append(f'    ra[st] = okx ? xs[st]{" * s" if V else ""} : 0.f;')
    else:
        if nsum > 1:
            L += [f'    const size_t xo = (size_t)nr * {Din} + {oi} + am + (size_t)kc * {D};',
                  f'    const float xa = (xr[kc * {D}] + x2[xo]) + x3[xo];']
        else:
            L += [f'    const float xa = xr[kc * {D}];']
        L += [f'    ra[st] = ok ? xa{" * s" if V else ""} : 0.f;']
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


def _kernel_f32(name, in_blocks, out_blocks, terms, V, Din, Dout, nsum=1):
    """HIP source of one direction on the fp32 matrix cores.  blockIdx.y selects (output block o, column group of CW channels), blockIdx.x a
    group of nodes.  A tile is TN = 16 // d whole nodes, i.e. <= 16 rows (node, m) — one MFMA row tile — and CW
    channels.  Each block runs in one of two modes (``_tiles_mode``):

    * one tile per wave, WAVES tiles per workgroup, each wave running the whole K loop for its tile and storing it
      from the result registers (no LDS, no barrier in the loop);
    * one tile per workgroup, its waves splitting K (chunks dealt round-robin) and the four partial tiles summed
      through LDS, then written node by node (each node's CW * d outputs are contiguous).

    K is walked in chunks c = (active attribute v, 32 input channels); operands are loaded straight into registers
    in the MFMA lane layout (16x16x4: lane (i, kq) = (lane % 16, lane / 16) holds A[i][4s + kq] and B[4s + kq][16 ct
    + i]) with the next chunk in flight.  With ``nsum`` = 3 the input is the sum (x + x2) + x3 of three tensors of
    its shape, added as loaded (``lin_bwds``: a backward over three consumers' gradients)."""
    fns, cases = [], []
    xs3 = 'const float* __restrict__ x2, const float* __restrict__ x3, ' if nsum > 1 else ''
    xa3 = 'x2, x3, ' if nsum > 1 else ''
    for o, (mo, l, oo, _) in enumerate(out_blocks):
        D = 2 * l + 1
        TN = ROWS // D
        CW = _cw(mo, CW_F32)
        CT = CW // 16
        fn = f'{name}_b{o}'
        tiles = bool(terms[o]) and _tiles_mode(terms[o], in_blocks, V)
        G = WAVES * TN if tiles else TN                       # nodes per workgroup
        L = [f'__device__ __forceinline__ void {fn}(const float* __restrict__ x, {xs3}const float* __restrict__ attr,',
             '    const float* __restrict__ W, float* __restrict__ out, int N, int group, int cg, float* __restrict__ red,',
             '    unsigned* __restrict__ amask, int* __restrict__ vlist, const int* __restrict__ order, float alpha,',
             '    const float* __restrict__ res) {',
             '  (void)alpha; (void)res;',
             f'  auto nd = [&](int i) {{ return {"order ? order[i] : " if V else ""}i; }};   // node of position i',
             '  (void)order;',
             f'  const int g0 = group * {G};                 // first node of the workgroup',
             '  if (g0 >= N) return;',
             f'  const int ng = min({G}, N - g0);',
             f'  const int t = threadIdx.x, col0 = cg * {CW};']
        if not terms[o]:
            L += [f'  for (int f = t; f < ng * {CW * D}; f += {BLOCK}) {{',
                  f'    const int nl = f / {CW * D}, j = f - nl * {CW * D};',
                  f'    const size_t at = (size_t)nd(g0 + nl) * {Dout} + {oo} + col0 * {D} + j;',
                  '    out[at] = res ? 0.f + res[at] : 0.f;',
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
            L += _mask(V, 'g0', 'ng', ordered=True)
        for (i, woff) in terms[o]:
            mi, li, oi, _ = in_blocks[i]
            assert li == l
            NCH = -(-mi // KC)
            nchunks = f'nact * {NCH}' if V else f'{NCH}'
            fns += _loader(fn, i, in_blocks, mi, oi, D, Din, V, woff, mo, CT, NCH, nsum)
            ld = f'{fn}_ld{i}(x, {xa3}attr, W, vlist, order, nb, col0, anl, am, q, c16'
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
                L += [f'        const size_t at = (size_t)nd(n0 + row) * {Dout} + {oo} + col0 + 4 * c16;',
                      '        float4 v = make_float4(alpha * acc[0][r], alpha * acc[1][r], alpha * acc[2][r], '
                      'alpha * acc[3][r]);',
                      '        if (res) {',
                      '          const float4 rv = *reinterpret_cast<const float4*>(res + at);',
                      '          v = make_float4(mh_mul_add(alpha, acc[0][r], rv.x), '
                      'mh_mul_add(alpha, acc[1][r], rv.y),',
                      '                          mh_mul_add(alpha, acc[2][r], rv.z), '
                      'mh_mul_add(alpha, acc[3][r], rv.w));',
                      '        }',
                      '        *reinterpret_cast<float4*>(out + at) = v;']
            else:
                L += [f'        const int nl = row / {D}, m = row - nl * {D};',
                      f'        const size_t ob = (size_t)nd(n0 + nl) * {Dout} + {oo} + m;',
                      '        float* __restrict__ o = out + ob;']
                for ct in range(CT):
                    L += [f'        {{ const size_t at = (size_t)(col0 + {CT} * c16 + {ct}) * {D};',
                          f'          o[at] = res ? mh_mul_add(alpha, acc[{ct}][r], res[ob + at]) : '
                          f'alpha * acc[{ct}][r]; }}']
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
                  f'    const float sum = (red[row * {CW} + cc] + red[(16 + row) * {CW} + cc])',
                  f'        + (red[(32 + row) * {CW} + cc] + red[(48 + row) * {CW} + cc]);',
                  f'    const size_t at = (size_t)nd(n0 + nl) * {Dout} + {oo} + col0 * {D} + j;',
                  '    out[at] = res ? mh_mul_add(alpha, sum, res[at]) : alpha * sum;',
                  '  }',
                  '}', '']
        fns += L
        cases.append((o, fn))
    gy = _grid_y(out_blocks, CW_F32)
    cw_max = max(_cw(mo, CW_F32) for mo, *_ in out_blocks)
    VW = (V + 31) // 32
    sw = ['  switch (y) {']
    for y, (o, cg) in enumerate(gy):
        fn = dict(cases)[o]
        sw.append(f'    case {y}: {fn}(x, {xa3}attr, W, out, N, group, {cg}, red, amask, vlist, order, alpha, res); '
                  'break;')
    sw += ['    default: break;', '  }']
    K = [f'extern "C" __global__ __launch_bounds__({BLOCK}) void {name}(const float* __restrict__ x,',
         '    const float* __restrict__ attr, const float* __restrict__ W, float* __restrict__ out, int N,',
         '    const int* __restrict__ order, float alpha, const float* __restrict__ res'
         + (', const float* __restrict__ x2, const float* __restrict__ x3' if nsum > 1 else '') + ') {',
         f'  __shared__ float red[{4 * 16 * cw_max}];',
         f'  __shared__ unsigned amask[{max(VW, 1)}];',
         f'  __shared__ int vlist[{V + 1}];'] + _block_map() + sw + ['}', '']
    return fns + K


def _f32_nodes_per_launch_group(blocks, terms, in_blocks, V):
    """Nodes per workgroup of the launch (its rows per block): the smallest over the output blocks; blocks with more
    nodes per workgroup leave their trailing workgroups idle."""
    return min(_nodes_per_group(terms[o], in_blocks, V, l) for o, (_, l, *_) in enumerate(blocks))


def _mask_wave(V, first, count):
    """The workgroup's attributes that are nonzero somewhere in its nodes (species-ordered positions), as a bit mask
    ``amw`` (V <= 32) that every wave builds by itself: each lane tests a share of the (node, attribute) pairs and
    the wave ORs the lanes' bits together, so there is no LDS, atomic or barrier before the first chunk's loads.
    ``nact`` is the number of live attributes and ``mh_kth_bit(amw, k)`` the k-th of them."""
    return [f'  unsigned amb = 0u;',
            f'  for (int f = lane; f < {count} * {V}; f += 64)',
            f'    if (attr[(size_t)nd({first} + f / {V}) * {V} + f % {V}] != 0.f) amb |= 1u << (f % {V});',
            '#pragma unroll',
            '  for (int b = 1; b < 64; b <<= 1) amb |= (unsigned)__shfl_xor((int)amb, b, 64);',
            '  const unsigned amw = __builtin_amdgcn_readfirstlane(amb);',
            '  const int nact = __popc(amw);']


def _mask(V, first, count, ordered=False):
    """The workgroup's list of attributes that are nonzero somewhere in its nodes (vlist[0] = count); with
    ``ordered`` position i of the workgroup is node nd(i)."""
    VW = (V + 31) // 32
    row = f'(size_t)nd({first} + f / {V}) * {V} + f % {V}' if ordered else f'(size_t){first} * {V} + f'
    return [f'  if (t < {VW}) amask[t] = 0u;',
            '  __syncthreads();',
            f'  for (int f = t; f < {count} * {V}; f += {BLOCK}) {{',
            f'    if (attr[{row}] != 0.f) {{ const int v = f % {V}; '
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


def use_bf16(spec, backward=False):
    """Which kernel family a direction gets: the bf16x6 LDS-staged one for maps with at least 1024 outputs (MACE's
    interaction linears, and the first layer's 2048-wide skip_tp: 40.5 -> 28.3 us per direction on config 2, with
    each chunk's attribute values prefetched alongside its operands and one row tile per wave); the fp32 one with
    per-wave register pipelines otherwise (short K and scalar-only blocks, whose few workgroups and short chunk
    chains favour it)."""
    return (spec.Din if backward else spec.Dout) >= BF16_MIN_OUT


SCALAR_BLOCK = 256


def _scalar_nodes(spec):
    """Nodes per workgroup of the plain backward (one thread per input value)."""
    return max(1, SCALAR_BLOCK // spec.Din)


def _kernel_scalar_bwd(spec):
    """``lin_bwd`` for a module whose input multiplicities do not tile (the node embedding: one input per element):
    one thread per (node, input value), reading the fp32 transposed weights Wt_io [mul_o, V', mul_i] directly,
        gx[n, i, u, m] = alpha sum_o sum_w g[n, o, w, m] (sum_v attrs[n, v]) Wt_io[w, v, u].
    Nothing here is on the energy-and-forces path (the engine never asks for this gradient there); a loss that
    backpropagates into the one-hot attributes, as ``loss.backward()`` does, needs it."""
    NB, VV = _scalar_nodes(spec), max(spec.V, 1)
    L = [f'extern "C" __global__ __launch_bounds__({SCALAR_BLOCK}) void {spec.kname("lin_bwd")}('
         'const float* __restrict__ g,',
         '    const float* __restrict__ attrs, const float* __restrict__ Wt, float* __restrict__ gx, int N,',
         '    const int* __restrict__ order, float alpha, const float* __restrict__ res) {',
         '  (void)order;',
         f'  const int q0 = blockIdx.x * {NB};',
         f'  for (int idx = threadIdx.x; idx < {NB * spec.Din}; idx += {SCALAR_BLOCK}) {{',
         f'    const int n = q0 + idx / {spec.Din}, k = idx % {spec.Din};',
         '    if (n >= N) break;',
         f'    const float* gr = g + (size_t)n * {spec.Dout};',
         '    float acc = 0.0f;']
    for i, (mi, li, oi, _) in enumerate(spec.in_blocks):
        d = 2 * li + 1
        L += [f'    if (k >= {oi} && k < {oi + mi * d}) {{', f'      const int u = (k - {oi}) / {d}, m = (k - {oi}) % {d};']
        for o, woff in spec.bterms[i]:
            mo, lo, oo, _ = spec.out_blocks[o]
            assert lo == li
            if spec.V:
                L += [f'      for (int w = 0; w < {mo}; ++w) {{',
                      f'        const float gv = gr[{oo} + w * {d} + m];',
                      f'        for (int v = 0; v < {spec.V}; ++v)',
                      f'          acc = fmaf(gv * attrs[(size_t)n * {spec.V} + v], Wt[{woff} + (w * {VV} + v) * {mi} + u], '
                      'acc);',
                      '      }']
            else:
                L += [f'      for (int w = 0; w < {mo}; ++w)',
                      f'        acc = fmaf(gr[{oo} + w * {d} + m], Wt[{woff} + w * {mi} + u], acc);']
        L.append('    }')
    L += [f'    const size_t at = (size_t)n * {spec.Din} + k;',
          '    gx[at] = res ? mh_mul_add(alpha, acc, res[at]) : alpha * acc;', '  }', '}', '']
    return L


# alpha * x + r rounded as a separate multiply and add (what adding r to the stored alpha * x gives), never fused
MUL_ADD = r"""
__device__ __forceinline__ float mh_mul_add(float a, float x, float r) {
#pragma clang fp contract(off)
  return a * x + r;
}
"""


def source_sum(spec):
    """HIP source of ``lin_bwds``: ``lin_bwd`` of an fp32-family module over the sum of three gradients (its output
    read by three consumers, each with a gradient slot of its own)."""
    return '\n'.join([_native.device_header(), MUL_ADD, ''] +
                     _kernel_f32(spec.kname('lin_bwds'), spec.out_blocks, spec.in_blocks, spec.bterms, spec.V,
                                 spec.Dout, spec.Din, nsum=3))


def source(spec):
    """HIP source of ``lin_fwd`` and ``lin_bwd`` for one module."""
    L = [_native.device_header(), MUL_ADD, '']
    if use_bf16(spec):
        L += _kernel(spec.kname('lin_fwd'), spec.in_blocks, spec.out_blocks, spec.terms, spec.V, spec.Din, spec.Dout,
                     spec.pack_fwd[1], spec.pack_fwd[2])
    else:
        L += _kernel_f32(spec.kname('lin_fwd'), spec.in_blocks, spec.out_blocks, spec.terms, spec.V, spec.Din,
                         spec.Dout)
    if not spec.tiled_bwd:
        L += _kernel_scalar_bwd(spec)
    else:
        if use_bf16(spec, backward=True):
            L += _kernel(spec.kname('lin_bwd'), spec.out_blocks, spec.in_blocks, spec.bterms, spec.V, spec.Dout,
                         spec.Din, spec.pack_bwd[1], spec.pack_bwd[2])
        else:
            L += _kernel_f32(spec.kname('lin_bwd'), spec.out_blocks, spec.in_blocks, spec.bterms, spec.V, spec.Dout,
                             spec.Din)
    return '\n'.join(L)


_ORDER = [None, None]     # (key, order) of the last attribute tensor seen


def node_order(attrs):
    """int32 permutation of the nodes sorted by species (argmax of the attributes), cached for the attribute tensor
    most recently seen (MACE's one-hot node_attrs are shared by every skip_tp of a call).  The results do not depend
    on it, so a stale cache entry (reused memory with the same shape) costs speed only."""
    key = (attrs.data_ptr(), attrs.shape, attrs._version, attrs.device)
    if _ORDER[0] != key:
        _ORDER[1] = torch.argsort(attrs.argmax(1), stable=True).to(torch.int32)
        _ORDER[0] = key
    return _ORDER[1]


_DOUBLE_BACKWARD = ('mace_hip_kernels: double backward (create_graph=True, e.g. training on forces/stress or an '
                    'autograd Hessian) is not enabled for this HIP module; patch with '
                    'patch_model(model, double_backward=True)')


class _LinFn(torch.autograd.Function):
    """out = scale * L(x, attrs) (+ res: a tensor of the output's shape added in the kernel's store)."""

    @staticmethod
    def forward(ctx, x, attrs, op, scale=1.0, res=None):
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
        order = None
        if a2 is not None and N > 0:
            # MACE's node_attrs is also what the symmetric contraction sorts by element: share that order
            order = element_order(attrs)[1] if attrs.dim() == 2 else node_order(a2)
        r2 = None
        if res is not None:
            if res.shape != (*lead, s.Dout) or res.dtype != torch.float32 or res.device != x.device:
                raise ValueError(f'a residual must be float32 [..., {s.Dout}] like the output, got {tuple(res.shape)}')
            r2 = res.reshape(N, s.Dout).contiguous()
        _native.launch(f'lin_fwd[{op.tag}]', _native.load().mh_lin_fwd_res, op.module.handle, _native.ptr(x2),
                       _native.ptr(a2), _native.ptr(op.W), _native.ptr(out), _native.ptr(order), scale,
                       _native.ptr(r2), N, _native.stream_of(x2))
        if a2 is not None:
            ctx.save_for_backward(a2, order)
        ctx.op, ctx.lead, ctx.N, ctx.scale = op, lead, N, scale
        return out.reshape(*lead, s.Dout)

    @staticmethod
    def backward(ctx, g):
        # node attributes are data (MACE's one-hot element encoding): no gradient flows to them, as in the
        # symmetric contraction; the residual's gradient is g itself
        gres = g if len(ctx.needs_input_grad) > 4 and ctx.needs_input_grad[4] else None
        if not ctx.needs_input_grad[0]:
            return None, None, None, None, gres
        op = ctx.op
        a2, order = ctx.saved_tensors if ctx.saved_tensors else (None, None)
        if torch.is_grad_enabled():          # only true under create_graph=True
            if not op.double_backward:
                raise RuntimeError(_DOUBLE_BACKWARD)
            return _LinAdjFn.apply(g, a2, order, op, ctx.scale, ctx.lead), None, None, None, gres
        return _lin_bwd(op, g, a2, order, ctx.scale, ctx.lead), None, None, None, gres


class _LinSlotsFn(torch.autograd.Function):
    """``_LinFn`` whose output also comes as ``nslot`` aliases (``set_slots``: the same storage, outputs of their
    own), one for each further consumer: the consumers' gradients reach this node separately and, three of them,
    are added by the backward kernel as it loads them (``mh_lin_bwd_sum``: (g + g2) + g3, in slot order) instead of
    by autograd in kernels of their own."""

    @staticmethod
    def forward(ctx, x, attrs, op, nslot):
        out = _LinFn.forward(ctx, x, attrs, op)
        return (out, *[out.detach() for _ in range(nslot)])

    @staticmethod
    def backward(ctx, g, *extra):
        none = (None, None, None, None)
        gs = [t for t in (g, *extra) if t is not None]
        if not ctx.needs_input_grad[0] or not gs:
            return none
        op = ctx.op
        a2, order = ctx.saved_tensors if ctx.saved_tensors else (None, None)
        if torch.is_grad_enabled() or len(gs) != 3:
            total = gs[0]
            for t in gs[1:]:
                total = total + t
            return (_LinFn.backward(ctx, total)[0], None, None, None)
        s = op.spec
        g3 = [t.reshape(-1, s.Dout).contiguous() for t in gs]
        N = g3[0].shape[0]
        gx = torch.empty(N, s.Din, device=g.device, dtype=torch.float32)
        P = _native.ptr
        _native.launch(f'lin_bwd[{op.tag}+sum]', _native.load().mh_lin_bwd_sum, op.sum_module().handle, P(g3[0]),
                       P(g3[1]), P(g3[2]), P(a2), P(op.Wt), P(gx), P(order), ctx.scale, N, _native.stream_of(g3[0]))
        return gx.reshape(*ctx.lead, s.Din), None, None, None


def _lin_bwd(op, g, a2, order, scale, lead):
    """The input gradient L^T g [*lead, Din] of g [*lead, Dout] by the backward kernel."""
    s = op.spec
    g2 = g.reshape(-1, s.Dout).contiguous()
    N = g2.shape[0]
    gx = torch.empty(N, s.Din, device=g.device, dtype=torch.float32)
    _native.launch(f'lin_bwd[{op.tag}]', _native.load().mh_lin_bwd, op.module.handle, _native.ptr(g2),
                   _native.ptr(a2), _native.ptr(op.Wt), _native.ptr(gx), _native.ptr(order), scale, N,
                   _native.stream_of(g2))
    return gx.reshape(*lead, s.Din)


class _LinAdjFn(torch.autograd.Function):
    """gx = L^T g as a function of g, for a double backward.  The map is linear in x, so gx does not depend on x and
    d<ggx, L^T g>/dg = L ggx: the forward map again (through _LinFn, so higher orders follow)."""

    @staticmethod
    def forward(ctx, g, a2, order, op, scale, lead):
        ctx.save_for_backward(a2)
        ctx.op, ctx.scale, ctx.lead = op, scale, lead
        return _lin_bwd(op, g, a2, order, scale, lead)

    @staticmethod
    def backward(ctx, ggx):
        a2, = ctx.saved_tensors
        attrs = a2.reshape(*ctx.lead, a2.shape[-1]) if a2 is not None else None
        return _LinFn.apply(ggx, attrs, ctx.op, ctx.scale), None, None, None, None, None


class HipNodeLinear(torch.nn.Module):
    """Drop-in for an e3nn ``o3.Linear`` (``forward(x)``) or a scalar-attribute ``FullyConnectedTensorProduct``
    (``forward(x, node_attrs)``), at inference (weights read at patch time; no weight gradients)."""

    def __init__(self, mod, device=None, spec=None):
        super().__init__()
        self.spec = LinSpec(mod) if spec is None else spec
        s = self.spec
        self.source = source(s)
        code = _native.compile_source(self.source)
        dev = torch.device(device) if device is not None else torch.device('cuda', torch.cuda.current_device())
        with torch.cuda.device(dev):
            def group(blocks, terms, in_blocks, bf16):
                return (_nodes_per_launch_group(blocks, _tiles(s.V)) if bf16 else
                        _f32_nodes_per_launch_group(blocks, terms, in_blocks, s.V))
            kernels = {_native.MH_LIN_FWD: (s.kname('lin_fwd'), BLOCK,
                                            group(s.out_blocks, s.terms, s.in_blocks, use_bf16(s)),
                                            len(_grid_y(s.out_blocks, CW_BF16 if use_bf16(s) else CW_F32)))}
            if s.tiled_bwd:
                kernels[_native.MH_LIN_BWD] = (s.kname('lin_bwd'), BLOCK,
                                               group(s.in_blocks, s.bterms, s.out_blocks, use_bf16(s, True)),
                                               len(_grid_y(s.in_blocks, CW_BF16 if use_bf16(s, True) else CW_F32)))
            else:
                kernels[_native.MH_LIN_BWD] = (s.kname('lin_bwd'), SCALAR_BLOCK, _scalar_nodes(s))
            self.module = _native.Module(code, kernels)
        # the bf16 family reads its weights as bf16 parts (int16 bit patterns), the fp32 family as float32
        for name, bf16, pk, w in (('W', use_bf16(s), s.pack_fwd[0], s.W),
                                  ('Wt', use_bf16(s, True) and s.tiled_bwd, s.pack_bwd[0], s.Wt)):
            buf = torch.from_numpy(pk.view(np.int16)) if bf16 else torch.tensor(w, dtype=torch.float32)
            self.register_buffer(name, buf.to(dev), persistent=False)
        for k in ('irreps_in', 'irreps_in1', 'irreps_in2', 'irreps_out'):
            if hasattr(mod, k):
                setattr(self, k, getattr(mod, k))
        self.original = [mod]
        self.tag = 'linear'
        # a backward under create_graph=True raises (the reference's behaviour) unless this is set; the map is
        # linear, so its double backward is the forward map again
        self.double_backward = False
        # set by patch_model when the caller divides the output by a constant: forward then returns a PendingLinear
        self.div_hint = None
        # set by patch_model when the output's one consumer runs it in composed form (compose_after) or adds a
        # tensor to it (a residual block's product: linear(node_feats) + sc): forward then returns a PendingLinear
        # (any other use forms the output)
        self.pend_hint = False
        # set by compose_after: the linear whose scaled output this module consumes (its output is then left
        # pending through the division) and the composed map that runs instead of the two
        self.compose_into = None
        self.compose_from = None
        self._composed = []
        # set by patch_model when the output is read by three patched consumers (MACE's product output: the readout
        # and the next block's skip_tp and linear_up): forward then leaves two aliases of the output for them
        # (gradient slots of their own) and the backward adds the three gradients as it loads them (lin_bwds)
        self.slots = 0
        self._sum_module = None

    def sum_module(self):
        """The module of ``lin_bwds`` (the backward over three gradients), compiled on first use; fp32 family with
        a tiled backward only."""
        s = self.spec
        if not s.tiled_bwd or use_bf16(s, True):
            raise RuntimeError('lin_bwds is built for the fp32 family with a tiled backward only')
        if self._sum_module is None:
            code = _native.compile_source(source_sum(s))
            with torch.cuda.device(self.Wt.device):
                self._sum_module = _native.Module(code, {_native.MH_LIN_BWD_SUM: (
                    s.kname('lin_bwds'), BLOCK, _f32_nodes_per_launch_group(s.in_blocks, s.bterms, s.out_blocks, s.V),
                    len(_grid_y(s.in_blocks, CW_F32)))})
        return self._sum_module

    def compose_after(self, first):
        """Consume ``first``'s output in composed form: when this module is called on the pending output of
        ``first`` divided by a constant (MACE's first interaction block: ``skip_tp(linear(message) / avg)``), one
        launch of the composed map (``LinSpec.compose``) on ``first``'s input replaces both launches, in the forward
        and in the backward.  Any other use of ``first``'s output forms it as usual."""
        spec = LinSpec.compose(first.spec, self.spec)
        dev = self.W.device
        op = HipNodeLinear(self.original[0], device=dev, spec=spec)
        op.tag = f'{first.tag}+{self.tag}'
        self._composed = [op]                  # a plain list: not a submodule (unpatch and .modules() skip it)
        # plain attributes, not submodule registrations (nn.Module.__setattr__ would register the other module)
        object.__setattr__(self, 'compose_from', first)
        object.__setattr__(first, 'compose_into', self)

    def forward(self, x, attrs=None):
        if self.spec.V == 0 and attrs is not None:
            raise TypeError('this linear takes no node attributes')
        if (isinstance(x, PendingLinear) and self._composed and x.op is self.compose_from
                and x.attrs is None and x.x.dtype == torch.float32):
            op = self._composed[0]
            op.double_backward = self.double_backward
            return _LinFn.apply(x.x, attrs, op, x.scale)
        if isinstance(x, Pending):
            x = x.value()                      # formed here, under autograd, not inside _LinFn's forward
        x = slot(x)
        if (self.div_hint is not None or self.pend_hint) and x.dtype == torch.float32:
            return PendingLinear(x, attrs, self)
        if self.slots and x.dtype == torch.float32:
            outs = _LinSlotsFn.apply(x, attrs, self, self.slots)
            set_slots(outs[0], outs[1:])
            return outs[0]
        return _LinFn.apply(x, attrs, self)


_DIVS = {torch.Tensor.__truediv__, torch.Tensor.div, torch.div, torch.true_divide}
_ADDS = {torch.Tensor.__add__, torch.Tensor.__radd__, torch.Tensor.add, torch.add}


class PendingLinear(Pending):
    """The output of a node linear whose caller is known to divide it by a constant (MACE's interaction blocks:
    ``self.linear(message) / self.avg_num_neighbors``), times ``scale``, not yet computed.  Dividing it by a Python
    number launches the kernel with the reciprocal folded into its stores (and the backward's), so no division
    kernel runs in either direction; when a patched module consumes the quotient in composed form
    (``HipNodeLinear.compose_after``) the quotient stays pending for it.  Adding a float32 tensor of the same shape
    (MACE's product block: ``self.linear(node_feats) + sc``) launches the kernel with that tensor added in its
    stores.  Any other use computes the plain output first."""

    @staticmethod
    def __new__(cls, x, attrs, op, scale=1.0):
        return Pending.__new__(cls, (*x.shape[:-1], op.spec.Dout), x)

    def __init__(self, x, attrs, op, scale=1.0):
        self.x, self.attrs, self.op, self.scale = x, attrs, op, scale

    def value(self):
        return _LinFn.apply(self.x, self.attrs, self.op, self.scale)

    @classmethod
    def intercept(cls, func, args, kwargs):
        if func in _ADDS and len(args) == 2 and not kwargs:
            a, b = args
            if isinstance(b, PendingLinear) and not isinstance(a, Pending):
                a, b = b, a                    # (a + b and b + a are the same float32 sum)
            if (isinstance(a, PendingLinear) and torch.is_tensor(b) and not isinstance(b, Pending)
                    and tuple(b.shape) == tuple(a.shape) and b.dtype == torch.float32 and b.device == a.device):
                # MACE's product block, linear(node_feats) + sc: the sum in the linear's store
                return _LinFn.apply(a.x, a.attrs, a.op, a.scale, b)
        if (func in _DIVS and len(args) == 2 and not kwargs and isinstance(args[0], PendingLinear)
                and isinstance(args[1], (int, float)) and not isinstance(args[1], bool) and args[1] != 0):
            p = args[0]
            scale = p.scale / float(args[1])
            if p.op.compose_into is not None:
                return PendingLinear(p.x, p.attrs, p.op, scale)
            return _LinFn.apply(p.x, p.attrs, p.op, scale)
        return NotImplemented


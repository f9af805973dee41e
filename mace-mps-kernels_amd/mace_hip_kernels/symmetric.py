"""
MACE ``SymmetricContraction`` as a precomputed symmetrised polynomial, evaluated by one generated HIP kernel per
layer (reference symmetric.py).

At inference the U matrices and product-basis weights are constants, so for element e, channel c and output
component M the contraction is a polynomial in x = X[b, c, :] (n_ell = (l_max+1)^2 components):
    out[b, c, M] = Σ_{i≤j≤k} T3 x_i x_j x_k + Σ_{i≤j} T2 x_i x_j + Σ_i T1 x_i          (correlation 3)
The coefficients T_ν[e, c, M, i…] = Σ_p U_ν[M, i…, p] W_ν[e, p, c] are formed once in float64 on the CPU, summed over
index permutations into sorted monomials, and monomials that vanish for every (element, channel, M) are dropped
(reference symmetric.py:20-75).  Only U and the weights are read, so any correlation order, l_max and CG basis work.

Table layout T[element][monomial × M][channel] (fp32): the 64 lanes of a wave are 64 channels of one node, so every
coefficient row is one coalesced 256-byte load.  Monomials are evaluated in FP32 VALU with shared prefix products.
Backward: ∂/∂x of the polynomial.  A double backward raises unless enabled (``double_backward``); then two more
kernels give the forward-mode derivative and the Hessian-vector product of the same polynomial.
"""
import itertools
import math
import weakref

import numpy as np
import scipy.sparse
import torch

from . import _native, species

WAVE = 64
LOADS_PER_FENCE = 32
GROUP = 4              # nodes per workgroup of the element-grouped kernels


def _poly_coeffs(ct):
    """{ν: {sorted index tuple: coefficient array [n_elem, M, C]}}, M, n_ell (reference symmetric.py:20-39)."""
    corr = ct.correlation
    U = {nu: getattr(ct, f'U_matrix_{nu}').detach().cpu().double().numpy() for nu in range(1, corr + 1)}
    W = {corr: ct.weights_max.detach().cpu().double().numpy()}
    for j, w in enumerate(ct.weights):                  # weights[0] ↔ ν = corr-1, weights[1] ↔ corr-2, …
        W[corr - 1 - j] = w.detach().cpu().double().numpy()
    lead = U[1].ndim - 2                                # 1 if there is an M axis (L > 0), else 0
    M = U[1].shape[0] if lead else 1
    n_ell = U[1].shape[-2]
    res = {}
    for nu in range(1, corr + 1):
        u = U[nu] if lead else U[nu][None]
        u = u.reshape(M, n_ell ** nu, u.shape[-1])                      # [M, ell^ν, p]
        # Sum every index tuple into its sorted representative.  Symmetrisation is linear and U does not depend on
        # the element, so it is applied to U before the (element-dependent) weights are contracted in.
        tuples = list(itertools.product(range(n_ell), repeat=nu))
        keys = sorted(set(tuple(sorted(x)) for x in tuples))
        kid = {k: i for i, k in enumerate(keys)}
        cols = np.array([kid[tuple(sorted(x))] for x in tuples])
        S = scipy.sparse.csr_matrix((np.ones(len(tuples)), (cols, np.arange(len(tuples)))),
                                    shape=(len(keys), len(tuples)))
        u_sym = np.stack([S @ u[m] for m in range(M)])                  # [M, K, p]
        t = np.einsum('mkp,epc->kemc', u_sym, W[nu])                    # [K, e, M, c]
        res[nu] = {k: t[i] for i, k in enumerate(keys)}                 # [e, M, c]
    return res, M, n_ell


def sc_supported(sc):
    """(ok, reason) — duck-type check of a MACE SymmetricContraction (reference symmetric.py:42-49)."""
    try:
        cts = list(sc.contractions)
        for ct in cts:
            _ = ct.correlation, ct.weights_max, ct.U_matrix_1
    except (AttributeError, TypeError) as e:
        return False, f'not a MACE SymmetricContraction ({e})'
    return True, ''


class SCSpec:
    """Term table and coefficient table of one SymmetricContraction (reference symmetric.py:52-75)."""

    def __init__(self, sc, tol=1e-12):
        ok, why = sc_supported(sc)
        if not ok:
            raise ValueError(why)
        self.blocks, rows, out_off = [], [], 0
        self.n_ell = None
        self.C = None
        for ct in sc.contractions:
            coeffs, M, n_ell = _poly_coeffs(ct)
            if self.n_ell not in (None, n_ell):
                raise ValueError('contractions disagree on n_ell')
            self.n_ell = n_ell
            terms = []
            for nu in sorted(coeffs, reverse=True):
                for idx, v in sorted(coeffs[nu].items()):
                    if np.abs(v).max() <= tol:
                        continue
                    terms.append((idx, len(rows)))
                    rows += [v[:, m, :] for m in range(M)]
            C = next(iter(coeffs[1].values())).shape[2]
            if self.C not in (None, C):
                raise ValueError('contractions disagree on the channel count')
            self.C = C
            self.blocks.append(dict(M=M, terms=terms, out_off=out_off))
            out_off += C * M
        self.out_dim, self.nrows = out_off, len(rows)
        self.T = torch.tensor(np.stack(rows, axis=1), dtype=torch.float32)     # [e, rows, c]
        self.n_elem = self.T.shape[0]
        self.n_terms = sum(len(b['terms']) for b in self.blocks)
        self.ncb = (self.C + WAVE - 1) // WAVE
        self.block = self.ncb * WAVE
        # component blocks of x in e3nn's irreps layout (the input before MACE's reshape_irreps): block k of
        # dimension d_k holds channel c's components at C o_k + c d_k + m, o_k = sum of the earlier d
        self.dims = None
        try:
            ir = [(mul, 2 * r.l + 1) for mul, r in sc.irreps_in]
            if all(mul == self.C for mul, _ in ir) and sum(d for _, d in ir) == self.n_ell:
                self.dims = [d for _, d in ir]
        except (AttributeError, TypeError):
            pass

    def kname(self, base):
        """Kernel symbol of this layer (shape-tagged so profiles tell the layers apart)."""
        return f'{base}_c{self.C}_o{self.out_dim}_r{self.nrows}'

    def flops(self):
        """(fwd, bwd) fp32 FLOP per (node, channel) as the generated code evaluates them."""
        fwd = bwd = 0
        for bl in self.blocks:
            M = bl['M']
            for idx, _ in bl['terms']:
                deg = len(idx)
                fwd += (deg - 1) + 2 * M
                bwd += (2 * M - 1) + 2 * len(set(idx)) + (deg - 1)
        return fwd, bwd

    def bytes(self, n_nodes, n_elem_used):
        fwd = 4 * (n_nodes * self.C * self.n_ell + n_nodes * self.out_dim + n_nodes
                   + n_elem_used * self.nrows * self.C)
        bwd = 4 * (2 * n_nodes * self.C * self.n_ell + n_nodes * self.out_dim + n_nodes
                   + n_elem_used * self.nrows * self.C)
        return fwd, bwd


# ------------------------------------------------------------------------------------------------- codegen
def _trie(spec):
    """Prefix trie of every monomial of every contraction block: node = {'terms': [(block, r0, M)], 'kids': {i: node}}.
    Walking it depth first evaluates each prefix product x_i·x_j·… exactly once, right before its last use."""
    root = {'terms': [], 'kids': {}}
    for bi, bl in enumerate(spec.blocks):
        for idx, r0 in bl['terms']:
            node = root
            for i in idx:
                node = node['kids'].setdefault(i, {'terms': [], 'kids': {}})
            node['terms'].append((bi, r0, bl['M']))
    return root


def _fence(L, ind, cnt, M, live, buffered=False):
    """Every LOADS_PER_FENCE coefficient loads, pass the table pointer and the live accumulators through empty asm
    statements.  Work before the fence must finish to produce their inputs and loads after it depend on their output,
    so the coefficient loads (invariant, hence otherwise free to move) cannot all be hoisted to the top of the kernel,
    where they would need hundreds of registers.  Volatile asm statements keep their order, so the operands are split
    into statements of at most 16 and the table pointer (``tb``; the lane offset ``voff`` for buffer loads) goes
    through the last one."""
    cnt[0] += M
    if cnt[0] >= LOADS_PER_FENCE:
        cnt[0] = 0
        chunks = [live[i:i + 16] for i in range(0, len(live), 16)] or [[]]
        for k, ch in enumerate(chunks):
            last = (['"+v"(voff)' if buffered else '"+s"(tb)'] if k == len(chunks) - 1 else [])
            ops = ', '.join([f'"+v"({v})' for v in ch] + last)
            L.append(f'{ind}asm volatile("" : {ops});')
        if not buffered:
            L.append(f'{ind}t = tb + cc;')


def _fwd_walk(spec, node, depth, L, ind, cnt):
    live = [f'a{bi}_{m}' for bi, bl in enumerate(spec.blocks) for m in range(bl['M'])]
    for bi, r0, M in node['terms']:
        _fence(L, ind, cnt, M, live)
        L += [f'{ind}a{bi}_{m} = fmaf(t[{(r0 + m) * spec.C}], p{depth}, a{bi}_{m});' for m in range(M)]
    for i in sorted(node['kids']):
        L.append(f'{ind}{{ const float p{depth + 1} = ' + (f'x{i};' if depth == 0 else f'p{depth} * x{i};'))
        _fwd_walk(spec, node['kids'][i], depth + 1, L, ind + '  ', cnt)
        L.append(f'{ind}}}')


def _bwd_walk(spec, node, depth, L, ind, cnt):
    """Reverse mode along the trie: G{depth} accumulates ∂out/∂p{depth}; a child p' = p·x_i passes G'·p to d_i and
    G'·x_i to G."""
    live = [f'd{i}' for i in range(spec.n_ell)] + [f'G{k}' for k in range(1, depth + 1)]
    for bi, r0, M in node['terms']:
        _fence(L, ind, cnt, M, live)
        s = ' + '.join(f't[{(r0 + m) * spec.C}] * g{bi}_{m}' for m in range(M))
        L.append(f'{ind}G{depth} += {s};')
    for i in sorted(node['kids']):
        kid = node['kids'][i]
        L.append(f'{ind}{{ const float p{depth + 1} = ' + (f'x{i};' if depth == 0 else f'p{depth} * x{i};'))
        L.append(f'{ind}  float G{depth + 1} = 0.0f;')
        _bwd_walk(spec, kid, depth + 1, L, ind + '  ', cnt)
        if depth == 0:
            L.append(f'{ind}  d{i} += G1;')
        else:
            L.append(f'{ind}  d{i} = fmaf(G{depth + 1}, p{depth}, d{i});')
            L.append(f'{ind}  G{depth} = fmaf(G{depth + 1}, x{i}, G{depth});')
        L.append(f'{ind}}}')


def _prefix(depth, i, L, ind):
    """Open the scope of the child x_i: prefix product p and its tangent q along V (p' = p x_i, q' = q x_i + p v_i)."""
    if depth == 0:
        L.append(f'{ind}{{ const float p1 = x{i}; const float q1 = v{i};')
    else:
        L.append(f'{ind}{{ const float p{depth + 1} = p{depth} * x{i}; '
                 f'const float q{depth + 1} = fmaf(q{depth}, x{i}, p{depth} * v{i});')


def _jvp_walk(spec, node, depth, L, ind, cnt):
    """Forward mode along the trie: each term adds coefficient × (tangent of its monomial along V)."""
    live = [f'a{bi}_{m}' for bi, bl in enumerate(spec.blocks) for m in range(bl['M'])]
    if depth > 0:                 # a constant term has no tangent
        for bi, r0, M in node['terms']:
            _fence(L, ind, cnt, M, live)
            L += [f'{ind}a{bi}_{m} = fmaf(t[{(r0 + m) * spec.C}], q{depth}, a{bi}_{m});' for m in range(M)]
    for i in sorted(node['kids']):
        _prefix(depth, i, L, ind)
        _jvp_walk(spec, node['kids'][i], depth + 1, L, ind + '  ', cnt)
        L.append(f'{ind}}}')


def _bwd2_walk(spec, node, depth, L, ind, cnt):
    """The reverse-mode walk of ``_bwd_walk`` with x carried as x + εv: G{depth} is ∂<g,out>/∂p{depth} as before and
    H{depth} its ε part; the ε part of every d_i update goes to h_i, which ends as the directional derivative of the
    gradient along V (terms contribute to G only: coefficients and g do not depend on x)."""
    live = ([f'h{i}' for i in range(spec.n_ell)] + [f'G{k}' for k in range(1, depth + 1)]
            + [f'H{k}' for k in range(1, depth + 1)])
    for bi, r0, M in node['terms']:
        _fence(L, ind, cnt, M, live)
        s = ' + '.join(f't[{(r0 + m) * spec.C}] * g{bi}_{m}' for m in range(M))
        L.append(f'{ind}G{depth} += {s};')
    for i in sorted(node['kids']):
        _prefix(depth, i, L, ind)
        L.append(f'{ind}  float G{depth + 1} = 0.0f; float H{depth + 1} = 0.0f;')
        _bwd2_walk(spec, node['kids'][i], depth + 1, L, ind + '  ', cnt)
        if depth == 0:
            L.append(f'{ind}  h{i} += H1;')
        else:
            L.append(f'{ind}  h{i} = fmaf(H{depth + 1}, p{depth}, fmaf(G{depth + 1}, q{depth}, h{i}));')
            L.append(f'{ind}  G{depth} = fmaf(G{depth + 1}, x{i}, G{depth});')
            L.append(f'{ind}  H{depth} = fmaf(H{depth + 1}, x{i}, fmaf(G{depth + 1}, v{i}, H{depth}));')
        L.append(f'{ind}}}')


def _fwd_walk_g(spec, node, depth, L, ind, cnt, nb):
    """The forward walk for ``nb`` nodes of one element at once: each coefficient load feeds ``nb`` FMAs (node j's
    variables carry the prefix ``j``), in the same order as the one-node walk."""
    live = [f'a{j}_{bi}_{m}' for j in range(nb) for bi, bl in enumerate(spec.blocks) for m in range(bl['M'])]
    for bi, r0, M in node['terms']:
        _fence(L, ind, cnt, M, live, buffered=True)
        for m in range(M):
            L.append(f'{ind}{{ const float tc = TLD({(r0 + m) * spec.C * 4});')
            L += [f'{ind}  a{j}_{bi}_{m} = fmaf(tc, p{j}_{depth}, a{j}_{bi}_{m});' for j in range(nb)]
            L.append(f'{ind}}}')
    for i in sorted(node['kids']):
        decl = ' '.join(f'const float p{j}_{depth + 1} = ' + (f'x{j}_{i};' if depth == 0 else f'p{j}_{depth} * x{j}_{i};')
                        for j in range(nb))
        L.append(f'{ind}{{ {decl}')
        _fwd_walk_g(spec, node['kids'][i], depth + 1, L, ind + '  ', cnt, nb)
        L.append(f'{ind}}}')


def _bwd_walk_g(spec, node, depth, L, ind, cnt, nb):
    """The reverse-mode walk for ``nb`` nodes of one element at once (same expressions as ``_bwd_walk`` per node)."""
    live = [f'd{j}_{i}' for j in range(nb) for i in range(spec.n_ell)] + \
           [f'G{j}_{k}' for j in range(nb) for k in range(1, depth + 1)]
    for bi, r0, M in node['terms']:
        _fence(L, ind, cnt, M, live, buffered=True)
        L.append(f'{ind}{{ ' + ' '.join(f'const float tc{m} = TLD({(r0 + m) * spec.C * 4});' for m in range(M)))
        for j in range(nb):
            s_ = ' + '.join(f'tc{m} * g{j}_{bi}_{m}' for m in range(M))
            L.append(f'{ind}  G{j}_{depth} += {s_};')
        L.append(f'{ind}}}')
    for i in sorted(node['kids']):
        kid = node['kids'][i]
        decl = ' '.join(f'const float p{j}_{depth + 1} = ' + (f'x{j}_{i};' if depth == 0 else f'p{j}_{depth} * x{j}_{i};')
                        for j in range(nb))
        L.append(f'{ind}{{ {decl}')
        L.append(f'{ind}  ' + ' '.join(f'float G{j}_{depth + 1} = 0.0f;' for j in range(nb)))
        _bwd_walk_g(spec, kid, depth + 1, L, ind + '  ', cnt, nb)
        for j in range(nb):
            if depth == 0:
                L.append(f'{ind}  d{j}_{i} += G{j}_1;')
            else:
                L.append(f'{ind}  d{j}_{i} = fmaf(G{j}_{depth + 1}, p{j}_{depth}, d{j}_{i});')
                L.append(f'{ind}  G{j}_{depth} = fmaf(G{j}_{depth + 1}, x{j}_{i}, G{j}_{depth});')
        L.append(f'{ind}}}')


# ------------------------------------------------------------------------------- LDS-staged kernels
STAGE_WAVES = 4        # waves per workgroup of the staged kernels (one channel block, nodes of one element)
STAGE_NPW = 2          # nodes per wave: every coefficient read from LDS feeds STAGE_NPW FMAs
STAGE_ROWS = 64        # coefficient rows per LDS chunk; two chunks resident (double buffer)
STAGE_FENCE = 64       # rows between anti-hoisting fences in the staged walk (0: none; spills)
SLOT_GROUP = STAGE_WAVES * STAGE_NPW     # node slots per workgroup of the staged kernels
# Split staged kernels (opt-in, HipSymmetricContraction.split): STAGE_SPLIT groups of STAGE_WAVES waves per
# workgroup, each walking its own share of the polynomial (a contiguous range of the trie root's children, about equal
# in rows, the first group also the root's own terms) for the same SLOT_GROUP slots, with its own LDS double buffer;
# the groups' partial sums meet in LDS in group order.  Twice the waves for graphs with few nodes, but not faster on
# MI355X at 2,533 nodes (2.5 waves per SIMD unsplit): SC1 forward 24.2 -> 26.4 us, backward 33.0 -> 35.9 us; the
# staged walk is bound by instruction issue per SIMD, not by latency (one node per wave, twice the waves: 29.8 us).
STAGE_SPLIT = 2


def walk_rows(spec):
    """Table rows in the order the trie walk reads them: at every trie node its terms' M rows, then its children in
    index order (the forward and the backward walk read in the same order)."""
    out = []

    def rec(node):
        for _, r0, M in node['terms']:
            out.extend(range(r0, r0 + M))
        for i in sorted(node['kids']):
            rec(node['kids'][i])
    rec(_trie(spec))
    assert sorted(out) == list(range(spec.nrows))
    return out


def _subtree_rows(node):
    return sum(M for _, _, M in node['terms']) + sum(_subtree_rows(k) for k in node['kids'].values())


def split_tries(spec, split):
    """The prefix trie cut into ``split`` pseudo-tries that share no rows: the root's children (in index order) in
    contiguous ranges of about equal row counts, the root's own terms in the first.  Walking each evaluates its
    terms with the same prefix products as the whole trie."""
    root = _trie(spec)
    kids = sorted(root['kids'])
    sizes = [_subtree_rows(root['kids'][i]) for i in kids]
    total = sum(sizes) + sum(M for _, _, M in root['terms'])
    parts, cur, acc = [[] for _ in range(split)], 0, sum(M for _, _, M in root['terms'])
    for i, sz in zip(kids, sizes):
        # move on to the next group once this one holds its share of the rows (never past the last group)
        if cur < split - 1 and parts[cur] and acc + sz / 2 > total * (cur + 1) / split:
            cur += 1
        parts[cur].append(i)
        acc += sz
    return [{'terms': root['terms'] if g == 0 else [], 'kids': {i: root['kids'][i] for i in parts[g]}}
            for g in range(split)]


def _walk_order(node):
    out = []

    def rec(nd):
        for _, r0, M in nd['terms']:
            out.extend(range(r0, r0 + M))
        for i in sorted(nd['kids']):
            rec(nd['kids'][i])
    rec(node)
    return out


def walk_rows_split(spec, split):
    """Per group of the split staged kernels, the table rows in the order its walk reads them."""
    return [_walk_order(t) for t in split_tries(spec, split)]


def stage_chunks(spec, cr=None, split=1):
    """LDS chunks of the staged walk (split > 1: of the longest group's walk, which every group's table is padded
    to)."""
    cr = STAGE_ROWS if cr is None else cr
    if split == 1:
        return -(-spec.nrows // cr)
    return max(-(-len(r) // cr) for r in walk_rows_split(spec, split))


def pack_staged(spec, cr=None):
    """The coefficient table for the staged kernels: rows in walk order, per (element, 64-channel block) a
    contiguous run of chunks of ``cr`` rows; inside a chunk, lane l's four consecutive rows r..r+3 of channel
    64 cb + l are one 16-byte quad: [n_elem][ncb][chunks · cr / 4][64][4] float32 (zero-padded rows and channels).
    A chunk is then one contiguous block that the workgroup copies to LDS as is, and one ds_read_b128 gives a lane
    four rows."""
    cr = STAGE_ROWS if cr is None else cr
    T = spec.T.numpy()                                       # [e, R, C]
    ne, R, C = T.shape
    RP = stage_chunks(spec, cr) * cr
    buf = np.zeros((ne, RP, spec.ncb * WAVE), dtype=np.float32)
    buf[:, :R, :C] = T[:, walk_rows(spec), :]
    buf = buf.reshape(ne, RP // 4, 4, spec.ncb, WAVE)        # [e][quad][row in quad][cb][lane]
    return np.ascontiguousarray(buf.transpose(0, 3, 1, 4, 2))  # [e][cb][quad][lane][row in quad]


def pack_staged_split(spec, split=STAGE_SPLIT, cr=None):
    """The table of the split staged kernels: per (element, 64-channel block) the groups' tables one after the
    other, each in its walk order and zero-padded to the same number of chunks, in pack_staged's chunk layout:
    [n_elem][ncb][split][chunks · cr / 4][64][4]."""
    cr = STAGE_ROWS if cr is None else cr
    T = spec.T.numpy()
    ne, R, C = T.shape
    RP = stage_chunks(spec, cr, split) * cr
    buf = np.zeros((ne, split, RP, spec.ncb * WAVE), dtype=np.float32)
    for g, rows in enumerate(walk_rows_split(spec, split)):
        buf[:, g, :len(rows), :C] = T[:, rows, :]
    buf = buf.reshape(ne, split, RP // 4, 4, spec.ncb, WAVE)  # [e][g][quad][row in quad][cb][lane]
    return np.ascontiguousarray(buf.transpose(0, 4, 1, 2, 5, 3))  # [e][cb][g][quad][lane][row in quad]


class _Stage:
    """Coefficient reads of a staged walk.  Walk position w (row ``walk_rows[w]``) is read from LDS buffer
    (w // cr) % 2; every fourth position loads the lane's next quad.  Entering chunk k >= 1 stores the staged
    registers (chunk k, loaded from global memory during chunk k - 1) into buffer k % 2, whose previous chunk k - 2
    every wave finished before the last barrier, then waits at the workgroup barrier and issues the global loads of
    chunk k + 1."""

    def __init__(self, spec, cr, fence, rows=None, sl='sl'):
        rows = walk_rows(spec) if rows is None else rows
        self.pos = {r: w for w, r in enumerate(rows)}
        self.cr, self.fence, self.nchunk = cr, fence, -(-len(rows) // cr)
        self.nst = cr // 16                   # 16-byte staging registers per thread (256 threads per chunk copy)
        self.sb = cr // 4 * WAVE              # quads per chunk
        self.sl = sl                          # the LDS double buffer's name
        self.next, self.since = 0, 0

    def copy_in(self, k, ind):
        return [f'{ind}sg{v} = src[{k * self.sb} + t + {256 * v}];' for v in range(self.nst)]

    def store(self, k, ind):
        return [f'{ind}{self.sl}[{(k % 2) * self.sb} + t + {256 * v}] = sg{v};' for v in range(self.nst)]

    def prologue(self, ind):
        L = [f'{ind}mh_f4 ' + ', '.join(f'sg{v}' for v in range(self.nst)) + ';', f'{ind}mh_f4 tq;']
        L += self.copy_in(0, ind) + self.store(0, ind)
        if self.nchunk > 1:
            L += self.copy_in(1, ind)
        return L + [f'{ind}__syncthreads();']

    def row(self, r, L, ind, live):
        w = self.pos[r]
        assert w == self.next, (w, self.next)
        self.next += 1
        k = w // self.cr
        if w and w % self.cr == 0:
            L += self.store(k, ind) + [f'{ind}__syncthreads();']
            if k + 1 < self.nchunk:
                L += self.copy_in(k + 1, ind)
        if w % 4 == 0:
            self.since += 4
            if self.fence and self.since >= self.fence:
                self.since = 0
                chunks = [live[i:i + 16] for i in range(0, len(live), 16)] or [[]]
                for ci, ch in enumerate(chunks):
                    ops = ', '.join([f'"+v"({v})' for v in ch] + (['"+v"(lo)'] if ci == len(chunks) - 1 else []))
                    L.append(f'{ind}asm volatile("" : {ops});')
            L.append(f'{ind}tq = {self.sl}[{(k % 2) * self.sb + (w % self.cr) // 4 * WAVE} + lo];')
        return f'tq[{w % 4}]'


def _fwd_walk_s(spec, node, depth, L, ind, st, nb):
    """The forward walk for ``nb`` nodes of one element with coefficients from LDS (same expressions per node as
    ``_fwd_walk``)."""
    live = [f'a{j}_{bi}_{m}' for j in range(nb) for bi, bl in enumerate(spec.blocks) for m in range(bl['M'])]
    for bi, r0, M in node['terms']:
        for m in range(M):
            e = st.row(r0 + m, L, ind, live)
            L.append(f'{ind}{{ const float tc = {e};')
            L += [f'{ind}  a{j}_{bi}_{m} = fmaf(tc, p{j}_{depth}, a{j}_{bi}_{m});' for j in range(nb)]
            L.append(f'{ind}}}')
    for i in sorted(node['kids']):
        decl = ' '.join(f'const float p{j}_{depth + 1} = ' + (f'x{j}_{i};' if depth == 0 else f'p{j}_{depth} * x{j}_{i};')
                        for j in range(nb))
        L.append(f'{ind}{{ {decl}')
        _fwd_walk_s(spec, node['kids'][i], depth + 1, L, ind + '  ', st, nb)
        L.append(f'{ind}}}')


def _bwd_walk_s(spec, node, depth, L, ind, st, nb):
    """The reverse-mode walk for ``nb`` nodes of one element with coefficients from LDS (same expressions per node
    as ``_bwd_walk``)."""
    live = [f'd{j}_{i}' for j in range(nb) for i in range(spec.n_ell)] + \
           [f'G{j}_{k}' for j in range(nb) for k in range(1, depth + 1)]
    for bi, r0, M in node['terms']:
        L.append(f'{ind}{{')
        for m in range(M):
            e = st.row(r0 + m, L, ind + '  ', live)
            L.append(f'{ind}  const float tc{m} = {e};')
        for j in range(nb):
            s_ = ' + '.join(f'tc{m} * g{j}_{bi}_{m}' for m in range(M))
            L.append(f'{ind}  G{j}_{depth} += {s_};')
        L.append(f'{ind}}}')
    for i in sorted(node['kids']):
        kid = node['kids'][i]
        decl = ' '.join(f'const float p{j}_{depth + 1} = ' + (f'x{j}_{i};' if depth == 0 else f'p{j}_{depth} * x{j}_{i};')
                        for j in range(nb))
        L.append(f'{ind}{{ {decl}')
        L.append(f'{ind}  ' + ' '.join(f'float G{j}_{depth + 1} = 0.0f;' for j in range(nb)))
        _bwd_walk_s(spec, kid, depth + 1, L, ind + '  ', st, nb)
        for j in range(nb):
            if depth == 0:
                L.append(f'{ind}  d{j}_{i} += G{j}_1;')
            else:
                L.append(f'{ind}  d{j}_{i} = fmaf(G{j}_{depth + 1}, p{j}_{depth}, d{j}_{i});')
                L.append(f'{ind}  G{j}_{depth} = fmaf(G{j}_{depth + 1}, x{j}_{i}, G{j}_{depth});')
        L.append(f'{ind}}}')


def _source_staged(spec, irreps=False, npw=None, cr=None, fence=None):
    """HIP source of the LDS-staged kernels ``sc_fwds`` / ``sc_bwds`` (``i`` suffix: x and its gradient in e3nn's
    irreps layout).  Workgroup = STAGE_WAVES waves on one 64-channel block (blockIdx.y) and SLOT_GROUP consecutive
    slots of the element-grouped node list (``group_slots``: every group holds nodes of one element; -1 marks an
    empty slot).  The element's coefficient rows stream through LDS in chunks of ``cr`` rows, copied once per
    workgroup, so each row read from L2 serves every node of the workgroup and each LDS read npw nodes of a wave.
    Per node the arithmetic is the one-node kernels' sequence."""
    npw = STAGE_NPW if npw is None else npw
    cr = STAGE_ROWS if cr is None else cr
    fence = STAGE_FENCE if fence is None else fence
    assert cr % 16 == 0
    C, n = spec.C, spec.n_ell
    sfx = 'i' if irreps else ''
    slots = STAGE_WAVES * npw
    comp = []
    if irreps:
        o = 0
        for d in spec.dims:
            comp += [(o, d, m) for m in range(d)]
            o += d

    def xidx(node, i, ch):
        if not irreps:
            return f'((size_t)({node}) * C + {ch}) * N_ELL + {i}'
        ok, d, m = comp[i]
        return f'(size_t)({node}) * (C * N_ELL) + {C * ok} + {ch} * {d} + {m}'
    nchunk = stage_chunks(spec, cr)
    sb = cr // 4 * WAVE
    L = [_native.device_header(),
         f'#define C {C}', f'#define NCB {spec.ncb}', f'#define N_ELL {n}', f'#define OUT_DIM {spec.out_dim}',
         f'#define SLOTS {slots}', f'#define CHUNK_QUADS {sb}', f'#define NCHUNK {nchunk}']

    def head(name, extra_args):
        H = [f'extern "C" __global__ __launch_bounds__({STAGE_WAVES * WAVE}) void {spec.kname(name + sfx)}('
             'const float* __restrict__ X,',
             '    const int* __restrict__ slots, const int* __restrict__ elem, const float* __restrict__ TS,',
             f'    {extra_args}, int N) {{',
             '  __shared__ mh_f4 sl[2 * CHUNK_QUADS];',
             '  const int t = threadIdx.x, wv = t >> 6;',
             '  int lo = t & 63;',
             '  const int q0 = blockIdx.x * SLOTS;',
             '  const int s0 = slots[q0];',
             '  if (s0 < 0) return;                       // past the last group (uniform over the workgroup)',
             '  const int c = blockIdx.y * 64 + lo;',
             '  const bool active = c < C;',
             '  const int cc = active ? c : C - 1;',
             '  const mh_f4* __restrict__ src = reinterpret_cast<const mh_f4*>(TS) +',
             '      (size_t)(elem[s0] * NCB + blockIdx.y) * (NCHUNK * CHUNK_QUADS);']
        for j in range(npw):
            H += [f'  const int m{j} = slots[q0 + wv * {npw} + {j}];',
                  f'  const int n{j} = m{j} >= 0 ? m{j} : s0;             // empty slot: compute on s0, store nothing']
            H += [f'  const float x{j}_{i} = X[{xidx(f"n{j}", i, "cc")}];' for i in range(n)]
        return H

    # forward
    st = _Stage(spec, cr, fence)
    L += head('sc_fwds', 'float* __restrict__ out')
    L += st.prologue('  ')
    L += [f'  float a{j}_{bi}_{m} = 0.0f;' for j in range(npw) for bi, bl in enumerate(spec.blocks)
          for m in range(bl['M'])]
    _fwd_walk_s(spec, _trie(spec), 0, L, '  ', st, npw)
    for j in range(npw):
        L.append(f'  if (active && m{j} >= 0) {{')
        for bi, bl in enumerate(spec.blocks):
            M = bl['M']
            L += [f'    out[(size_t)n{j} * OUT_DIM + {bl["out_off"]} + c * {M} + {m}] = a{j}_{bi}_{m};'
                  for m in range(M)]
        L.append('  }')
    L += ['}', '']
    # backward
    st = _Stage(spec, cr, fence)
    L += head('sc_bwds', 'const float* __restrict__ G, float* __restrict__ GX')
    for j in range(npw):
        L += [f'  float d{j}_{i} = 0.0f;' for i in range(n)]
        for bi, bl in enumerate(spec.blocks):
            M = bl['M']
            L += [f'  const float g{j}_{bi}_{m} = G[(size_t)n{j} * OUT_DIM + {bl["out_off"]} + cc * {M} + {m}];'
                  for m in range(M)]
    L += st.prologue('  ')
    L.append('  ' + ' '.join(f'float G{j}_0 = 0.0f;' for j in range(npw)))
    _bwd_walk_s(spec, _trie(spec), 0, L, '  ', st, npw)
    L.append('  ' + ' '.join(f'(void)G{j}_0;' for j in range(npw)))
    for j in range(npw):
        L.append(f'  if (active && m{j} >= 0) {{')
        L += [f'    GX[{xidx(f"n{j}", i, "c")}] = d{j}_{i};' for i in range(n)]
        L.append('  }')
    L += ['}', '']
    return '\n'.join(L)


def split_fits(spec, split=STAGE_SPLIT, npw=None, cr=None):
    """Whether the split staged kernels can exchange their partial sums through one group's LDS double buffer (the
    backward's n_ell and the forward's output components per node, per wave)."""
    npw = STAGE_NPW if npw is None else npw
    cr = STAGE_ROWS if cr is None else cr
    nout = sum(bl['M'] for bl in spec.blocks)
    return split > 1 and STAGE_WAVES * npw * max(spec.n_ell, nout) * WAVE <= 2 * (cr // 4 * WAVE) * 4


def _source_staged_split(spec, irreps=False, split=STAGE_SPLIT, npw=None, cr=None, fence=None):
    """HIP source of the split staged kernels ``sc_fwds2`` / ``sc_bwds2`` (``i`` suffix: e3nn's irreps layout).
    Workgroup = ``split`` groups of STAGE_WAVES waves on the same SLOT_GROUP slots and 64-channel block; group g walks
    its part of the polynomial (``split_tries``) with its coefficient rows streamed through its own LDS double
    buffer, exactly as the unsplit kernel walks the whole (the same staging, fences and per-node expressions).  All
    groups pass the same number of barriers (a group with fewer chunks waits at the rest); after one more, which
    every wave reaches only when its walk is done, the groups past the first leave their partial sums (outputs, or
    x-gradients) in their LDS buffer, and after another the first group adds them in group order and stores.
    ``grp`` is read as a scalar, so every branch on it is uniform per wave."""
    npw = STAGE_NPW if npw is None else npw
    cr = STAGE_ROWS if cr is None else cr
    fence = STAGE_FENCE if fence is None else fence
    assert cr % 16 == 0 and split_fits(spec, split, npw, cr)
    C, n = spec.C, spec.n_ell
    sfx = 'i' if irreps else ''
    slots = STAGE_WAVES * npw
    comp = []
    if irreps:
        o = 0
        for d in spec.dims:
            comp += [(o, d, m) for m in range(d)]
            o += d

    def xidx(node, i, ch):
        if not irreps:
            return f'((size_t)({node}) * C + {ch}) * N_ELL + {i}'
        ok, d, m = comp[i]
        return f'(size_t)({node}) * (C * N_ELL) + {C * ok} + {ch} * {d} + {m}'
    tries = split_tries(spec, split)
    rows = [_walk_order(t) for t in tries]
    nchunk = stage_chunks(spec, cr, split)
    sb = cr // 4 * WAVE
    outs = [(bi, m) for bi, bl in enumerate(spec.blocks) for m in range(bl['M'])]
    L = [_native.device_header(),
         f'#define C {C}', f'#define NCB {spec.ncb}', f'#define N_ELL {n}', f'#define OUT_DIM {spec.out_dim}',
         f'#define SLOTS {slots}', f'#define CHUNK_QUADS {sb}', f'#define NCHUNK {nchunk}', f'#define SPLIT {split}']

    def head(name, extra_args):
        H = [f'extern "C" __global__ __launch_bounds__({split * STAGE_WAVES * WAVE}) void {spec.kname(name + sfx)}('
             'const float* __restrict__ X,',
             '    const int* __restrict__ slots, const int* __restrict__ elem, const float* __restrict__ TS,',
             f'    {extra_args}, int N) {{',
             '  __shared__ mh_f4 sl[SPLIT * 2 * CHUNK_QUADS];',
             f'  const int grp = __builtin_amdgcn_readfirstlane((int)threadIdx.x / {STAGE_WAVES * WAVE});',
             f'  const int t = (int)threadIdx.x & {STAGE_WAVES * WAVE - 1}, wv = t >> 6;   // thread, wave in the group',
             '  int lo = t & 63;',
             '  const int q0 = blockIdx.x * SLOTS;',
             '  const int s0 = slots[q0];',
             '  if (s0 < 0) return;                       // past the last group (uniform over the workgroup)',
             '  const int c = blockIdx.y * 64 + lo;',
             '  const bool active = c < C;',
             '  const int cc = active ? c : C - 1;',
             '  mh_f4* __restrict__ slg = sl + grp * (2 * CHUNK_QUADS);',
             '  const mh_f4* __restrict__ src = reinterpret_cast<const mh_f4*>(TS) +',
             '      ((size_t)(elem[s0] * NCB + blockIdx.y) * SPLIT + grp) * (NCHUNK * CHUNK_QUADS);']
        for j in range(npw):
            H += [f'  const int m{j} = slots[q0 + wv * {npw} + {j}];',
                  f'  const int n{j} = m{j} >= 0 ? m{j} : s0;             // empty slot: compute on s0, store nothing']
            H += [f'  const float x{j}_{i} = X[{xidx(f"n{j}", i, "cc")}];' for i in range(n)]
        return H

    def groups(walk, acc_names):
        """Each group's staged walk in a uniform branch, padded to NCHUNK barriers; then the partials of the groups
        past the first into their LDS buffers (acc_names: the per-node accumulators, lane-contiguous rows)."""
        G = []
        for g in range(split):
            st = _Stage(spec, cr, fence, rows=rows[g], sl='slg')
            G.append(f'  {"if" if g == 0 else "else if"} (grp == {g}) {{')
            G += st.prologue('    ')
            walk(tries[g], G, '    ', st)
            G += ['    __syncthreads();                      // (the longest group\'s remaining chunk boundaries)'] * \
                (nchunk - st.nchunk)
            G.append('  }')
        G += ['  __syncthreads();                          // every wave done with its group\'s chunks',
              '  if (grp > 0) {',
              '    float* __restrict__ pp = reinterpret_cast<float*>(slg);']
        G += [f'    pp[{k * WAVE} + (wv * {len(acc_names)}) * {WAVE} + lo] = {a};' for k, a in enumerate(acc_names)]
        G += ['  }', '  __syncthreads();', '  if (grp != 0) return;']
        for g in range(1, split):
            G.append(f'  {{ const float* __restrict__ pp = reinterpret_cast<const float*>(sl + {g} * 2 * CHUNK_QUADS);')
            G += [f'    {a} += pp[{k * WAVE} + (wv * {len(acc_names)}) * {WAVE} + lo];' for k, a in enumerate(acc_names)]
            G.append('  }')
        return G

    # forward
    L += head('sc_fwds2', 'float* __restrict__ out')
    accs = [f'a{j}_{bi}_{m}' for j in range(npw) for bi, m in outs]
    L += [f'  float {a} = 0.0f;' for a in accs]
    L += groups(lambda node, G, ind, st: _fwd_walk_s(spec, node, 0, G, ind, st, npw), accs)
    for j in range(npw):
        L.append(f'  if (active && m{j} >= 0) {{')
        for bi, bl in enumerate(spec.blocks):
            M = bl['M']
            L += [f'    out[(size_t)n{j} * OUT_DIM + {bl["out_off"]} + c * {M} + {m}] = a{j}_{bi}_{m};'
                  for m in range(M)]
        L.append('  }')
    L += ['}', '']
    # backward
    L += head('sc_bwds2', 'const float* __restrict__ G, float* __restrict__ GX')
    for j in range(npw):
        L += [f'  float d{j}_{i} = 0.0f;' for i in range(n)]
        for bi, bl in enumerate(spec.blocks):
            M = bl['M']
            L += [f'  const float g{j}_{bi}_{m} = G[(size_t)n{j} * OUT_DIM + {bl["out_off"]} + cc * {M} + {m}];'
                  for m in range(M)]

    def bwd_walk(node, G_, ind, st):
        G_.append(f'{ind}' + ' '.join(f'float G{j}_0 = 0.0f;' for j in range(npw)))
        _bwd_walk_s(spec, node, 0, G_, ind, st, npw)
        G_.append(f'{ind}' + ' '.join(f'(void)G{j}_0;' for j in range(npw)))
    L += groups(bwd_walk, [f'd{j}_{i}' for j in range(npw) for i in range(n)])
    for j in range(npw):
        L.append(f'  if (active && m{j} >= 0) {{')
        L += [f'    GX[{xidx(f"n{j}", i, "c")}] = d{j}_{i};' for i in range(n)]
        L.append('  }')
    L += ['}', '']
    return '\n'.join(L)


def split_usable(spec, split=STAGE_SPLIT):
    """Whether the split staged kernels serve this contraction: the partial sums fit the LDS buffers and every
    group has rows to walk."""
    return split_fits(spec, split, STAGE_NPW, STAGE_ROWS) and all(walk_rows_split(spec, split))


def source_split(spec, split=STAGE_SPLIT):
    """HIP source of the module of the split staged kernels (both layouts when the input irreps are known)."""
    src = _source_staged_split(spec, split=split)
    if spec.dims is not None:
        alt = _source_staged_split(spec, irreps=True, split=split)
        src += '\n' + alt[alt.index('#define SLOTS'):]
    return src


def _source_layout(spec, group=None, irreps=False, second=False):
    """HIP source of the per-node kernels ``sc_fwd`` / ``sc_bwd`` (one workgroup per node, the reference's launch
    shape) and the element-grouped kernels ``sc_fwdg`` / ``sc_bwdg``: one workgroup per GROUP consecutive nodes of an
    element-sorted order.  When the group's nodes share an element (every group but those straddling an element
    boundary) every coefficient load feeds GROUP FMAs instead of one; other groups run the one-node body per node.
    Per node the arithmetic is the same sequence either way.  With ``irreps`` the same four kernels (names ending
    in ``i``) read x and write its gradient in e3nn's irreps layout [N, sum C (2l+1)] (MACE's reshape_irreps input),
    so that permutation never runs.  With ``second`` the module holds instead the two second-order kernels
    ``sc_jvp`` / ``sc_bwd2`` (one node per workgroup) behind a double backward."""
    group = GROUP if group is None else group
    C, R, n = spec.C, spec.nrows, spec.n_ell
    sfx = 'i' if irreps else ''
    if irreps:
        comp, o = [], 0
        for d in spec.dims:
            comp += [(o, d, m) for m in range(d)]
            o += d

    def xidx(node, i, ch):
        """Index of component i of channel ch of node `node` in X (and GX)."""
        if not irreps:
            return f'((size_t)({node}) * C + {ch}) * N_ELL + {i}'
        ok, d, m = comp[i]
        return f'(size_t)({node}) * (C * N_ELL) + {C * ok} + {ch} * {d} + {m}'
    L = [_native.device_header(),
         f'#define C {C}', f'#define NCB {spec.ncb}', f'#define BLOCK {spec.block}', f'#define N_ELL {n}',
         f'#define R {R}', f'#define OUT_DIM {spec.out_dim}', f'#define GROUP {group}',
         f'#define TBYTES {spec.n_elem * R * C * 4}',
         # coefficient row loads: raw buffer loads over T at lane offset voff (VGPR) + row offset, the row offset split
         # into a 4 KiB-aligned part (SGPR, shared by 8 consecutive rows) and the instruction's 12-bit immediate
         '#define TLD(off) __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, voff + ((off) & 4095), '
         '(off) & ~4095, 0))']
    assert spec.n_elem * R * C * 4 < 2 ** 31, 'coefficient table too large for 32-bit buffer offsets'
    trie = _trie(spec)
    lane = ['  const int c = threadIdx.x;', '  const bool active = c < C;', '  const int cc = active ? c : C - 1;',
            '  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)T, (short)0, TBYTES, 0x00020000);']

    def node_head(ind, bexpr):
        return ([f'{ind}const int b = {bexpr};'] +
                [f'{ind}const float x{i} = X[{xidx("b", i, "cc")}];' for i in range(n)] +
                [f'{ind}const float* tb = T + (size_t)elem[b] * ((size_t)R * C);', f'{ind}const float* t = tb + cc;'])

    def fwd_one(ind):
        B = [f'{ind}float a{bi}_{m} = 0.0f;' for bi, bl in enumerate(spec.blocks) for m in range(bl['M'])]
        _fwd_walk(spec, trie, 0, B, ind, [0])
        B.append(f'{ind}if (active) {{')
        for bi, bl in enumerate(spec.blocks):
            M = bl['M']
            B += [f'{ind}  out[(size_t)b * OUT_DIM + {bl["out_off"]} + c * {M} + {m}] = a{bi}_{m};' for m in range(M)]
        return B + [f'{ind}}}']

    def bwd_one(ind):
        B = [f'{ind}float d{i} = 0.0f;' for i in range(n)]
        for bi, bl in enumerate(spec.blocks):
            M = bl['M']
            B += [f'{ind}const float g{bi}_{m} = G[(size_t)b * OUT_DIM + {bl["out_off"]} + cc * {M} + {m}];'
                  for m in range(M)]
        B.append(f'{ind}float G0 = 0.0f;')
        _bwd_walk(spec, trie, 0, B, ind, [0])
        B += [f'{ind}(void)G0;', f'{ind}if (active) {{']
        B += [f'{ind}  GX[{xidx("b", i, "c")}] = d{i};' for i in range(n)]
        return B + [f'{ind}}}']

    def group_head():
        H = ['  const int q0 = mh_xcd_block(blockIdx.x, gridDim.x) * GROUP;', '  if (q0 >= N) return;'] + lane
        H.append('  const int qn = min(GROUP, N - q0);')
        # nodes past the end repeat the last one (loaded, never stored), so every index stays in range
        H += [f'  const int n{j} = order[q0 + min({j}, qn - 1)];' for j in range(group)]
        H += [f'  const int e{j} = elem[n{j}];' for j in range(group)]
        same = ' && '.join(f'e0 == e{j}' for j in range(1, group)) or 'true'
        H += [f'  if ({same}) {{', '    int voff = (e0 * (R * C) + cc) * 4;']
        for j in range(group):
            H += [f'    const float x{j}_{i} = X[{xidx(f"n{j}", i, "cc")}];' for i in range(n)]
        return H

    def guarded(j, lines):
        return lines if j == 0 else [f'      if ({j} < qn) {{'] + ['  ' + x for x in lines] + ['      }']

    if second:
        vload = lambda ind: [f'{ind}const float v{i} = V[{xidx("b", i, "cc")}];' for i in range(n)]  # noqa: E731
        # forward-mode derivative: out = d/dε P(X + εV)
        L += [f'extern "C" __global__ __launch_bounds__(BLOCK) void {spec.kname("sc_jvp" + sfx)}(const float* __restrict__ X,',
              '    const float* __restrict__ V, const int* __restrict__ elem, const float* __restrict__ T,',
              '    float* __restrict__ out, int N) {',
              '  const int bq = mh_xcd_block(blockIdx.x, gridDim.x);', '  if (bq >= N) return;'] + lane
        L += node_head('  ', 'bq') + vload('  ')
        L += [f'  float a{bi}_{m} = 0.0f;' for bi, bl in enumerate(spec.blocks) for m in range(bl['M'])]
        _jvp_walk(spec, trie, 0, L, '  ', [0])
        L.append('  if (active) {')
        for bi, bl in enumerate(spec.blocks):
            M = bl['M']
            L += [f'    out[(size_t)b * OUT_DIM + {bl["out_off"]} + c * {M} + {m}] = a{bi}_{m};' for m in range(M)]
        L += ['  }', '}', '']
        # directional derivative of the gradient: GX = d/dε ∂<G, P>/∂X at X + εV
        L += [f'extern "C" __global__ __launch_bounds__(BLOCK) void {spec.kname("sc_bwd2" + sfx)}(const float* __restrict__ X,',
              '    const float* __restrict__ V, const int* __restrict__ elem, const float* __restrict__ T,',
              '    const float* __restrict__ G, float* __restrict__ GX, int N) {',
              '  const int bq = mh_xcd_block(blockIdx.x, gridDim.x);', '  if (bq >= N) return;'] + lane
        L += node_head('  ', 'bq') + vload('  ')
        L += [f'  float h{i} = 0.0f;' for i in range(n)]
        for bi, bl in enumerate(spec.blocks):
            M = bl['M']
            L += [f'  const float g{bi}_{m} = G[(size_t)b * OUT_DIM + {bl["out_off"]} + cc * {M} + {m}];'
                  for m in range(M)]
        L.append('  float G0 = 0.0f;')
        _bwd2_walk(spec, trie, 0, L, '  ', [0])
        L += ['  (void)G0;', '  if (active) {']
        L += [f'    GX[{xidx("b", i, "c")}] = h{i};' for i in range(n)]
        L += ['  }', '}', '']
        return '\n'.join(L)
    # ------------------------------------------------------------------------------- per-node forward
    L += [f'extern "C" __global__ __launch_bounds__(BLOCK) void {spec.kname("sc_fwd" + sfx)}(const float* __restrict__ X,',
          '    const int* __restrict__ elem, const float* __restrict__ T, float* __restrict__ out, int N) {',
          '  const int bq = mh_xcd_block(blockIdx.x, gridDim.x);', '  if (bq >= N) return;'] + lane
    L += node_head('  ', 'bq') + fwd_one('  ') + ['}', '']
    # ------------------------------------------------------------------------------ per-node backward
    L += [f'extern "C" __global__ __launch_bounds__(BLOCK) void {spec.kname("sc_bwd" + sfx)}(const float* __restrict__ X,',
          '    const int* __restrict__ elem, const float* __restrict__ T, const float* __restrict__ G,',
          '    float* __restrict__ GX, int N) {',
          '  const int bq = mh_xcd_block(blockIdx.x, gridDim.x);', '  if (bq >= N) return;'] + lane
    L += node_head('  ', 'bq') + bwd_one('  ') + ['}', '']
    # -------------------------------------------------------------------------------- grouped forward
    L += [f'extern "C" __global__ __launch_bounds__(BLOCK) void {spec.kname("sc_fwdg" + sfx)}(const float* __restrict__ X,',
          '    const int* __restrict__ elem, const int* __restrict__ order, const float* __restrict__ T,',
          '    float* __restrict__ out, int N) {']
    L += group_head()
    L += [f'    float a{j}_{bi}_{m} = 0.0f;' for j in range(group) for bi, bl in enumerate(spec.blocks)
          for m in range(bl['M'])]
    _fwd_walk_g(spec, trie, 0, L, '    ', [0], group)
    L.append('    if (active) {')
    for j in range(group):
        st = []
        for bi, bl in enumerate(spec.blocks):
            M = bl['M']
            st += [f'      out[(size_t)n{j} * OUT_DIM + {bl["out_off"]} + c * {M} + {m}] = a{j}_{bi}_{m};'
                   for m in range(M)]
        L += guarded(j, st)
    L += ['    }', '  } else {', '    for (int j = 0; j < qn; ++j) {']
    L += ['  ' + x for x in node_head('    ', 'order[q0 + j]') + fwd_one('    ')]
    L += ['    }', '  }', '}', '']
    # ------------------------------------------------------------------------------- grouped backward
    L += [f'extern "C" __global__ __launch_bounds__(BLOCK) void {spec.kname("sc_bwdg" + sfx)}(const float* __restrict__ X,',
          '    const int* __restrict__ elem, const int* __restrict__ order, const float* __restrict__ T,',
          '    const float* __restrict__ G, float* __restrict__ GX, int N) {']
    L += group_head()
    for j in range(group):
        L += [f'    float d{j}_{i} = 0.0f;' for i in range(n)]
        for bi, bl in enumerate(spec.blocks):
            M = bl['M']
            L += [f'    const float g{j}_{bi}_{m} = G[(size_t)n{j} * OUT_DIM + {bl["out_off"]} + cc * {M} + {m}];'
                  for m in range(M)]
    L.append('    ' + ' '.join(f'float G{j}_0 = 0.0f;' for j in range(group)))
    _bwd_walk_g(spec, trie, 0, L, '    ', [0], group)
    L.append('    ' + ' '.join(f'(void)G{j}_0;' for j in range(group)))
    L.append('    if (active) {')
    for j in range(group):
        st = [f'      GX[{xidx(f"n{j}", i, "c")}] = d{j}_{i};' for i in range(n)]
        L += guarded(j, st)
    L += ['    }', '  } else {', '    for (int j = 0; j < qn; ++j) {']
    L += ['  ' + x for x in node_head('    ', 'order[q0 + j]') + bwd_one('    ')]
    L += ['    }', '  }', '}', '']
    return '\n'.join(L)


def source_second(spec):
    """HIP source of the second-order module: ``sc_jvp`` / ``sc_bwd2`` on the [N, C, n_ell] layout and, when the
    input irreps are known, on e3nn's irreps layout (``sc_jvpi`` / ``sc_bwd2i``).  Compiled only for a double
    backward."""
    src = _source_layout(spec, second=True)
    if spec.dims is not None:
        alt = _source_layout(spec, irreps=True, second=True)
        src += '\n' + alt[alt.index('extern "C"'):]
    return src


def source(spec, group=None):
    """HIP source of one layer's module: the six kernels on the [N, C, n_ell] layout (per node, element-grouped,
    LDS-staged; forward and backward) and, when the input irreps are known, the same six on e3nn's irreps layout
    (one shared header)."""
    src = _source_layout(spec, group)
    for irreps in ((False, True) if spec.dims is not None else (False,)):
        if irreps:
            alt = _source_layout(spec, group, irreps=True)
            src += '\n' + alt[alt.index('extern "C"'):]
        st = _source_staged(spec, irreps=irreps)
        src += '\n' + st[st.index('#define SLOTS'):]
    return src


# ------------------------------------------------------------------------------------------------ autograd
_DOUBLE_BACKWARD = ('mace_hip_kernels: double backward (create_graph=True, e.g. training on forces/stress or an '
                    'autograd Hessian) is not enabled for this HIP module; patch with '
                    'patch_model(model, double_backward=True)')

_elem_cache = []          # [(weakref(node_attrs), version, (elem, order, slots) int32)], most recent first
_SIMDS = {}               # device index -> SIMD count (4 per compute unit)


def _species(node_attrs):
    """(elem, order, slots) of a node_attrs tensor (``species.species_order``, one launch), cached per tensor."""
    ver = node_attrs._version
    for ref, v, eos in _elem_cache:
        if ref() is node_attrs and v == ver:
            return _native.hold_for_capture(eos)
    eos = species.species_order(node_attrs, SLOT_GROUP)
    if _native.capturing():
        return eos             # recomputed by every replay; its memory only holds values once the graph runs
    _elem_cache.insert(0, (weakref.ref(node_attrs), ver, eos))
    del _elem_cache[4:]
    return eos


def element_order(node_attrs):
    """(elem, order): the argmax of the one-hot node attributes as int32 (reference symmetric.py:169) and the node
    indices stably sorted by element, which the grouped kernels walk.  Cached per node_attrs tensor."""
    elem, order, _ = _species(node_attrs)
    return elem, order


def group_slots(node_attrs):
    """Node slots of the staged kernels: the element-sorted node order with every element's run padded with -1 to a
    multiple of SLOT_GROUP, so that each workgroup's SLOT_GROUP slots hold nodes of one element, and -1 up to the
    fixed length ceil(N / SLOT_GROUP) SLOT_GROUP + n_elem SLOT_GROUP (an upper bound for any element mix, so the
    launch size needs no device-to-host copy).  Cached per node_attrs tensor, computed with element_order."""
    return _species(node_attrs)[2]


def element_index(node_attrs):
    """argmax of the one-hot node attributes as int32 (reference symmetric.py:169)."""
    return element_order(node_attrs)[0]


def _sc_fwd(op, layout, kind, x, elem, order, slots):
    """Launch the contraction on contiguous x in ``layout`` ('mace' [N, C, n_ell] or 'irreps' [N, C n_ell]) with
    the kernel family ``kind`` ('node', 'grouped', 'staged' or 'staged2')."""
    N = x.shape[0]
    out = torch.empty(N, op.spec.out_dim, device=x.device, dtype=torch.float32)
    lib, P = _native.load(), _native.ptr
    st = _native.stream_of(x)
    if kind in ('staged', 'staged2'):
        m, ts = op.split_module() if kind == 'staged2' else (op.module, op.TS)
        _native.launch(f'sc_fwd[{op.tag}]', lib.mh_sc_fwd_staged, m.handle, P(x), P(slots), slots.numel(),
                       P(elem), P(ts), P(out), N, int(layout == 'irreps'), st)
    elif layout == 'irreps':
        _native.launch(f'sc_fwd[{op.tag}]', lib.mh_sc_fwd_irreps, op.module.handle, P(x), P(elem),
                       P(order) if kind == 'grouped' else None, P(op.T), P(out), N, st)
    elif kind == 'grouped':
        _native.launch(f'sc_fwd[{op.tag}]', lib.mh_sc_fwd_sorted, op.module.handle, P(x), P(elem), P(order),
                       P(op.T), P(out), N, st)
    else:
        _native.launch(f'sc_fwd[{op.tag}]', lib.mh_sc_fwd, op.module.handle, P(x), P(elem), P(op.T), P(out), N, st)
    return out


def _sc_bwd(op, layout, kind, x, elem, order, slots, g):
    """Launch the contraction's x-gradient for contiguous x and g; the gradient has x's layout."""
    gx = torch.empty_like(x)
    lib, P = _native.load(), _native.ptr
    st, N = _native.stream_of(x), x.shape[0]
    if kind in ('staged', 'staged2'):
        m, ts = op.split_module() if kind == 'staged2' else (op.module, op.TS)
        _native.launch(f'sc_bwd[{op.tag}]', lib.mh_sc_bwd_staged, m.handle, P(x), P(slots), slots.numel(),
                       P(elem), P(ts), P(g), P(gx), N, int(layout == 'irreps'), st)
    elif layout == 'irreps':
        _native.launch(f'sc_bwd[{op.tag}]', lib.mh_sc_bwd_irreps, op.module.handle, P(x), P(elem),
                       P(order) if kind == 'grouped' else None, P(op.T), P(g), P(gx), N, st)
    elif kind == 'grouped':
        _native.launch(f'sc_bwd[{op.tag}]', lib.mh_sc_bwd_sorted, op.module.handle, P(x), P(elem), P(order),
                       P(op.T), P(g), P(gx), N, st)
    else:
        _native.launch(f'sc_bwd[{op.tag}]', lib.mh_sc_bwd, op.module.handle, P(x), P(elem), P(op.T), P(g), P(gx), N,
                       st)
    return gx


def _sc_backward(ctx, g):
    """Shared backward of the two layouts' functions: the first-order kernel, or under create_graph (only then is
    grad mode on here) the same gradient as a differentiable function of (g, x) when the module allows it."""
    x, elem, order, slots = ctx.saved_tensors
    op = ctx.op
    if torch.is_grad_enabled():
        if not op.double_backward:
            raise RuntimeError(_DOUBLE_BACKWARD)
        return _SCAdjFn.apply(g, x, elem, order, slots, op, ctx.layout, ctx.kind), None, None, None, None
    return (_sc_bwd(op, ctx.layout, ctx.kind, x.contiguous(), elem, order, slots, g.contiguous()),
            None, None, None, None)


class _SCFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, elem, order, slots, op):
        s = op.spec
        if x.dtype != torch.float32 or not x.is_cuda:
            raise TypeError('mace_hip_kernels: symmetric contraction expects float32 GPU input')
        if x.dim() != 3 or x.shape[1] != s.C or x.shape[2] != s.n_ell:
            raise ValueError(f'node_feats must be [N, {s.C}, {s.n_ell}], got {tuple(x.shape)}')
        kind = op.kernel_family(x.shape[0], x.device)
        out = _sc_fwd(op, 'mace', kind, x.contiguous(), elem, order, slots)
        ctx.save_for_backward(x, elem, order, slots)     # the input itself: a double backward differentiates it
        ctx.kind, ctx.op, ctx.layout = kind, op, 'mace'
        return out

    backward = staticmethod(_sc_backward)


class _SCIrrepsFn(torch.autograd.Function):
    """The contraction on x in e3nn's irreps layout [N, C n_ell] (the kernels with the ``i`` suffix); the gradient
    comes back in that layout."""

    @staticmethod
    def forward(ctx, x, elem, order, slots, op):
        s = op.spec
        if x.dtype != torch.float32 or not x.is_cuda or x.dim() != 2 or x.shape[1] != s.C * s.n_ell:
            raise ValueError(f'expected float32 GPU input [N, {s.C * s.n_ell}], got {tuple(x.shape)}')
        kind = op.kernel_family(x.shape[0], x.device)
        out = _sc_fwd(op, 'irreps', kind, x.contiguous(), elem, order, slots)
        ctx.save_for_backward(x, elem, order, slots)
        ctx.kind, ctx.op, ctx.layout = kind, op, 'irreps'
        return out

    backward = staticmethod(_sc_backward)


class _SCAdjFn(torch.autograd.Function):
    """gx = (∂P/∂x)^T g as a function of (g, x), which a double backward differentiates: with ggx the incoming
    gradient, d<ggx, gx>/dg is the forward-mode derivative of P along ggx (``mh_sc_jvp``) and d<ggx, gx>/dx the
    Hessian-vector product of <g, P> (``mh_sc_bwd2``).  Third derivatives are not provided."""

    @staticmethod
    def forward(ctx, g, x, elem, order, slots, op, layout, kind):
        gx = _sc_bwd(op, layout, kind, x.contiguous(), elem, order, slots, g.contiguous())
        ctx.save_for_backward(g, x, elem)
        ctx.op, ctx.layout = op, layout
        return gx

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, ggx):
        g, x, elem = ctx.saved_tensors
        op = ctx.op
        m = op.second_module()
        lay = 1 if ctx.layout == 'irreps' else 0
        x, v, g = x.contiguous(), ggx.contiguous(), g.contiguous()
        lib, P, N = _native.load(), _native.ptr, x.shape[0]
        gg = gx = None
        if ctx.needs_input_grad[0]:
            gg = torch.empty(N, op.spec.out_dim, device=x.device, dtype=torch.float32)
            _native.launch(f'sc_jvp[{op.tag}]', lib.mh_sc_jvp, m.handle, P(x), P(v), P(elem), P(op.T), P(gg), N,
                           lay, _native.stream_of(x))
        if ctx.needs_input_grad[1]:
            gx = torch.empty_like(x)
            _native.launch(f'sc_bwd2[{op.tag}]', lib.mh_sc_bwd2, m.handle, P(x), P(v), P(elem), P(op.T), P(g),
                           P(gx), N, lay, _native.stream_of(x))
        return gg, gx, None, None, None, None, None, None


class HipSymmetricContraction(torch.nn.Module):
    """Drop-in for mace ``SymmetricContraction`` at inference: ``forward(x[N, C, n_ell], node_attrs[N, n_elem])``
    (reference symmetric.py:158-170)."""

    def __init__(self, sc, device=None):
        super().__init__()
        self.spec = SCSpec(sc)
        dev = torch.device(device) if device is not None else torch.device('cuda', torch.cuda.current_device())
        self.register_buffer('T', self.spec.T.to(dev).contiguous())
        self.register_buffer('TS', torch.from_numpy(pack_staged(self.spec)).to(dev))
        self.source = source(self.spec)
        code = _native.compile_source(self.source)
        with torch.cuda.device(dev):
            sw, ncb = STAGE_WAVES * WAVE, self.spec.ncb
            kinds = {
                _native.MH_SC_FWD: (self.spec.kname('sc_fwd'), self.spec.block, 1),
                _native.MH_SC_BWD: (self.spec.kname('sc_bwd'), self.spec.block, 1),
                _native.MH_SC_FWD_G: (self.spec.kname('sc_fwdg'), self.spec.block, GROUP),
                _native.MH_SC_BWD_G: (self.spec.kname('sc_bwdg'), self.spec.block, GROUP),
                _native.MH_SC_FWD_S: (self.spec.kname('sc_fwds'), sw, SLOT_GROUP, ncb),
                _native.MH_SC_BWD_S: (self.spec.kname('sc_bwds'), sw, SLOT_GROUP, ncb),
            }
            if self.spec.dims is not None:
                kinds.update({
                    _native.MH_SC_FWD_I: (self.spec.kname('sc_fwdi'), self.spec.block, 1),
                    _native.MH_SC_BWD_I: (self.spec.kname('sc_bwdi'), self.spec.block, 1),
                    _native.MH_SC_FWD_GI: (self.spec.kname('sc_fwdgi'), self.spec.block, GROUP),
                    _native.MH_SC_BWD_GI: (self.spec.kname('sc_bwdgi'), self.spec.block, GROUP),
                    _native.MH_SC_FWD_SI: (self.spec.kname('sc_fwdsi'), sw, SLOT_GROUP, ncb),
                    _native.MH_SC_BWD_SI: (self.spec.kname('sc_bwdsi'), sw, SLOT_GROUP, ncb),
                })
            self.module = _native.Module(code, kinds)
        self.register_buffer('TS2', None)        # the split kernels' table (split_module)
        self._split = None
        self.irreps_in, self.irreps_out = sc.irreps_in, sc.irreps_out
        self.original = [sc]
        self.tag = 'sc'               # name used in launch timings (patch_model sets the module path)
        self.grouped = None           # True / False: force the grouped / per-node global-memory kernels
        self.staged = None            # None: by size (kernel_family); True: force the LDS-staged kernels
        self.split = None             # True: the split staged kernels (split_module) in place of the staged ones
        self.last_layout = None       # input layout of the last call: 'mace' [N, C, n_ell] or 'irreps'
        # a backward under create_graph=True: raise (the reference's behaviour) unless this is set, in which case
        # the gradient is differentiable once more through the second-order kernels (second_module)
        self.double_backward = False
        self._second = None

    def split_module(self):
        """The module of the split staged kernels (the same entry points and kinds as the staged ones, bound to
        ``sc_fwds2`` / ``sc_bwds2``) and its table, compiled and packed on first use."""
        if self._split is None:
            s = self.spec
            if not split_usable(s):
                raise ValueError('mace_hip_kernels: the split staged kernels do not serve this contraction')
            self.TS2 = torch.from_numpy(pack_staged_split(s)).to(self.T.device)
            code = _native.compile_source(source_split(s))
            sw, ncb = STAGE_SPLIT * STAGE_WAVES * WAVE, s.ncb
            kinds = {_native.MH_SC_FWD_S: (s.kname('sc_fwds2'), sw, SLOT_GROUP, ncb),
                     _native.MH_SC_BWD_S: (s.kname('sc_bwds2'), sw, SLOT_GROUP, ncb)}
            if s.dims is not None:
                kinds.update({_native.MH_SC_FWD_SI: (s.kname('sc_fwds2i'), sw, SLOT_GROUP, ncb),
                              _native.MH_SC_BWD_SI: (s.kname('sc_bwds2i'), sw, SLOT_GROUP, ncb)})
            with torch.cuda.device(self.T.device):
                self._split = _native.Module(code, kinds)
        return self._split, self.TS2

    def second_module(self):
        """The module of the second-order kernels (``sc_jvp``, ``sc_bwd2``), compiled on first use."""
        if self._second is None:
            s = self.spec
            code = _native.compile_source(source_second(s))
            kinds = {_native.MH_SC_JVP: (s.kname('sc_jvp'), s.block, 1),
                     _native.MH_SC_BWD2: (s.kname('sc_bwd2'), s.block, 1)}
            if s.dims is not None:
                kinds.update({_native.MH_SC_JVP_I: (s.kname('sc_jvpi'), s.block, 1),
                              _native.MH_SC_BWD2_I: (s.kname('sc_bwd2i'), s.block, 1)})
            with torch.cuda.device(self.T.device):
                self._second = _native.Module(code, kinds)
        return self._second

    def use_grouped(self, n_nodes, device):
        """The element-grouped kernels serve GROUP nodes per workgroup, so they need GROUP times more nodes to keep
        the GPU busy: use them when they still give at least 4 waves per SIMD (config 4's 20,000 atoms: 1.7-1.9x
        faster than one node per workgroup; config 2's 2,533 atoms: slower)."""
        if self.grouped is not None:
            return bool(self.grouped)
        key = device.index if device.index is not None else torch.cuda.current_device()
        if key not in _SIMDS:
            _SIMDS[key] = 4 * torch.cuda.get_device_properties(key).multi_processor_count
        waves = -(-n_nodes // GROUP) * self.spec.ncb
        return waves >= 4 * _SIMDS[key]

    def kernel_family(self, n_nodes, device):
        """'staged' (coefficient rows through LDS, SLOT_GROUP nodes of one element per workgroup), 'staged2' (the
        same split over two groups of waves), 'grouped' or 'node' (coefficients from global memory): ``split`` /
        ``staged`` / ``grouped`` force a family (``staged`` False: the global-memory family that ``use_grouped``
        picks), else the staged kernels."""
        if self.split:
            return 'staged2'
        if self.staged:
            return 'staged'
        if self.grouped is not None:
            return 'grouped' if self.grouped else 'node'
        if self.staged is False:
            return 'grouped' if self.use_grouped(n_nodes, device) else 'node'
        return 'staged'

    def forward(self, x, y):
        if y.shape != (x.shape[0], self.spec.n_elem):
            raise ValueError(f'node_attrs must be [{x.shape[0]}, {self.spec.n_elem}], got {tuple(y.shape)}')
        elem, order = element_order(y)
        slots = group_slots(y) if self.kernel_family(x.shape[0], x.device) in ('staged', 'staged2') else None
        src = getattr(x, 'irreps_source', None)
        if src is not None and self.spec.dims is not None and src(self.spec.dims) is not None:
            # x is MACE's reshape_irreps of a tensor in e3nn's layout, not yet formed: read that tensor directly
            self.last_layout = 'irreps'
            return _SCIrrepsFn.apply(src(self.spec.dims), elem, order, slots, self)
        self.last_layout = 'mace'
        return _SCFn.apply(x, elem, order, slots, self)

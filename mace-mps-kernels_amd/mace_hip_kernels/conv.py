"""
Fused MACE interaction convolution on MI355X: gather → channel-wise ('uvu') tensor product → scatter-sum, one
generated HIP module per e3nn ``TensorProduct`` (reference conv.py).

Coefficients.  The effective coefficient of every path (Clebsch-Gordan × e3nn normalisation × path weight) is
probed from the TensorProduct itself with unit inputs (reference conv.py:57-88) — here on a float64 CPU copy, so the
literals baked into the kernel are exact to fp32 rounding rather than fp32-probed.

Kernels (all deterministic, no atomics; one lane per channel, 64-lane wavefronts, ceil(MUL/64) waves per row):
  * ``conv_fwd``  one workgroup per receiver n walks the receiver-sorted CSR; per edge the wave loads its W row
    slice (coalesced), the sender's x slice, and Y[e] as wave-uniform scalars; accumulators stay in registers and
    the [N, OUT_DIM] output is written once (reference conv.py:109-141).
  * ``conv_bwd``  one workgroup per sender s walks the sender-sorted CSR and produces, in one pass, gx[s]
    (reference conv.py:144-176) and gW[e], gY[e] (reference conv.py:179-222): W and g[receiver] are read once
    instead of twice, x[s] is loaded once per sender.  gY[e, j] = Σ_u (…) is reduced over the wave by a transpose
    reduction and over the workgroup's waves through LDS, in a fixed order.
  * ``conv_bwd_wy`` the per-edge d/dW, d/dY kernel of the reference's C ABI (no CSR): 64 consecutive edges per
    workgroup.

Layouts are the reference's (conv.py:9-14): x [N, X_DIM] mul_ir, Y [E, Y_DIM], W [E, NINS*MUL] (instruction k,
channel u at k*MUL+u), out [N, OUT_DIM].  ``edge_index = [sender, receiver]``.
"""
import copy
import math
import warnings
import weakref

import numpy as np
import torch

from . import _native, neighbours
from .pending import stash_owner
from .conv_codegen import gxsum_block, source

WAVE = 64


def _blocks(irreps):
    res, off = [], 0
    for mul, ir in irreps:
        res.append((ir.l, mul, off))
        off += mul * (2 * ir.l + 1)
    return res, off


def conv_supported(tp):
    """(ok, reason) — whether an e3nn TensorProduct can be replaced by the fused convolution (reference conv.py:31-51).
    """
    try:
        ins = tp.instructions
        if any(i.connection_mode != 'uvu' or not i.has_weight for i in ins):
            return False, 'only weighted uvu instructions are supported'
        if getattr(tp, 'shared_weights', True) or getattr(tp, 'internal_weights', True):
            return False, 'per-edge (external, unshared) weights required'
        muls = {m for m, _ in tp.irreps_in1} | {m for m, _ in tp.irreps_out}
        if len(muls) != 1:
            return False, 'all node/out blocks must have the same multiplicity'
        mul = muls.pop()
        if mul % 32:
            return False, f'multiplicity {mul} is not a multiple of 32'
        if any(m != 1 for m, _ in tp.irreps_in2):
            return False, 'edge attributes must have multiplicity 1 per l'
        if tp.weight_numel != len(ins) * mul:
            return False, 'unexpected weight layout'
        if tp.irreps_in2.dim > WAVE:
            return False, f'edge attribute dimension {tp.irreps_in2.dim} > {WAVE}'
        if len({i.i_out for i in ins}) != len(ins):
            return False, 'each output block must come from exactly one instruction'
    except AttributeError as e:
        return False, f'not an e3nn TensorProduct ({e})'
    return True, ''


def _probe_tp(tp):
    """(callable, device, dtype) used for probing: a float64 CPU copy when the TP can be copied, else the TP itself."""
    try:
        cp = copy.deepcopy(tp).to(device='cpu', dtype=torch.float64)
        return cp, torch.device('cpu'), torch.float64
    except Exception as e:  # noqa: BLE001  (a TP that cannot be copied: probe it where it lives, like the reference)
        warnings.warn(f'mace_hip_kernels: probing {type(tp).__name__} in its own dtype/device ({e}); path '
                      'coefficients carry that precision')
        dev = next(iter(tp.buffers()), torch.zeros(1)).device
        return tp, dev, torch.get_default_dtype()


class ConvSpec:
    """Instruction table and effective path coefficients of one 'uvu' TensorProduct (reference conv.py:54-102)."""

    def __init__(self, tp, tol=1e-10):
        ok, why = conv_supported(tp)
        if not ok:
            raise ValueError(why)
        self.in1, self.x_dim = _blocks(tp.irreps_in1)
        self.in2, self.y_dim = _blocks(tp.irreps_in2)
        self.outb, self.out_dim = _blocks(tp.irreps_out)
        self.mul = self.in1[0][1]
        self.ins = [(i.i_in1, i.i_in2, i.i_out) for i in tp.instructions]
        self.nins = len(self.ins)
        probe, dev, dt = _probe_tp(tp)
        self.coef = []
        for k, (i1, i2, io) in enumerate(self.ins):
            l1, _, o1 = self.in1[i1]
            l2, _, o2 = self.in2[i2]
            l3, _, o3 = self.outb[io]
            d1, d2, d3 = 2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1
            x1 = torch.zeros(d1 * d2, self.x_dim, device=dev, dtype=dt)
            x2 = torch.zeros(d1 * d2, self.y_dim, device=dev, dtype=dt)
            w = torch.zeros(d1 * d2, tp.weight_numel, device=dev, dtype=dt)
            for a in range(d1):
                for b in range(d2):
                    r = a * d2 + b
                    x1[r, o1 + a] = 1.0          # channel u = 0
                    x2[r, o2 + b] = 1.0
                    w[r, k * self.mul] = 1.0
            with torch.no_grad():
                y = probe(x1, x2, w)[:, o3:o3 + d3].double().cpu().reshape(d1, d2, d3)
            terms = [(a, b, c, float(y[a, b, c])) for a in range(d1) for b in range(d2) for c in range(d3)
                     if abs(float(y[a, b, c])) > tol]
            self.coef.append(dict(k=k, l1=l1, l2=l2, l3=l3, o1=o1, o2=o2, o3=o3, d1=d1, d2=d2, d3=d3, terms=terms))
        self.nnz = sum(len(c['terms']) for c in self.coef)
        self.ncb = (self.mul + WAVE - 1) // WAVE
        self.block = self.ncb * WAVE
        self.y_pad = 1 << max(0, (self.y_dim - 1).bit_length())

    def kname(self, base):
        """Kernel symbol of this layer (shape-tagged so profiles tell the layers apart)."""
        return f'{base}_x{self.x_dim}_o{self.out_dim}'

    def xreg(self):
        r, idx = 0, {}
        for b, (l, _, _) in enumerate(self.in1):
            idx[b] = r
            r += 2 * l + 1
        return idx, r

    def oreg(self):
        r, idx = 0, {}
        for c in self.coef:
            idx[c['k']] = r
            r += 2 * c['l3'] + 1
        return idx, r

    # ---------------------------------------------------------------------------------------- cost model
    def flops(self):
        """(fwd, bwd) fp32 FLOP per real edge per channel as the generated code evaluates them."""
        nnz = self.nnz
        pairs = sum(len({(a, c) for a, _, c, _ in co['terms']}) for co in self.coef)
        d3 = sum(co['d3'] for co in self.coef)
        d1 = sum(co['d1'] for co in self.coef)
        fwd = 2 * nnz + 2 * pairs + 2 * d3
        bwd = (2 * nnz + 2 * d1) + (2 * d1) + (4 * nnz + 2 * self.y_dim)   # h (gx), gW, gY partials
        return fwd, bwd

    def bytes(self, n_nodes, n_edges):
        """Algorithmic HBM bytes (fwd, bwd) of one call: every tensor read or written once, 4 B per element."""
        nw = self.nins * self.mul
        fwd = 4 * (n_edges * (nw + self.y_dim + 2) + n_nodes * (self.x_dim + self.out_dim) + (n_nodes + 1))
        bwd = 4 * (n_edges * (2 * nw + 2 * self.y_dim + 4) + n_nodes * (2 * self.x_dim + self.out_dim)
                   + 2 * (n_nodes + 1))
        return fwd, bwd


# ------------------------------------------------------------------------------------------- graph cache
def graph_source():
    """HIP source of the graph-build kernels behind ``mh_graph_build`` (both CSRs of an edge list, device work only).
    Each kernel handles one index row per grid row (blockIdx.y: 0 senders, 1 receivers).  Segments are filled in
    whatever order the atomics land and then ordered by edge id, so the result is what a stable sort by the index
    gives (reference conv.py:229-235) and never depends on timing.  A segment of at most RANK_MAX edges is ordered by
    counting (each edge counts the smaller ids in its segment, L reads per edge: ~40 for MACE graphs); a longer one
    (a hub node, or padding edges all sent to one node) is sorted in place by one workgroup (``csr_sort_long``: a
    bitonic network of ascending comparators, so comparators that reach past the segment's end are simply skipped,
    O(L log^2 L) work, in LDS up to SORT_LDS edges) and then copied."""
    return _native.device_header() + (f"#define RANK_MAX {RANK_MAX}\n#define SORT_LDS {SORT_LDS}\n"
                                      f"#define PAIR_DEG_MAX {PAIR_DEG_MAX}\n") + r"""
extern "C" __global__ __launch_bounds__(256) void csr_fill(int* __restrict__ cnt, int* __restrict__ bad, int n) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i <= n) cnt[(long long)blockIdx.y * (n + 1) + i] = 0;
  if (i == 0 && blockIdx.y == 0) bad[0] = 0;
}

extern "C" __global__ __launch_bounds__(256) void csr_count(const long long* __restrict__ index, int* __restrict__ keys,
    int* __restrict__ cnt, int* __restrict__ bad, long long E, int n) {
  const long long e = (long long)blockIdx.x * 256 + threadIdx.x;
  if (e >= E) return;
  const long long r = blockIdx.y;
  long long k = index[r * E + e];
  if (k < 0 || k >= n) {                  // flagged for the caller; clamped so that nothing reads out of range
    atomicOr(bad, 1);
    k = k < 0 ? 0 : n - 1;
  }
  keys[r * E + e] = (int)k;
  atomicAdd(&cnt[r * (n + 1) + k], 1);
}

extern "C" __global__ __launch_bounds__(1024) void csr_scan(const int* __restrict__ cnt, int* __restrict__ rowptr,
    int* __restrict__ cursor, int n) {
  const long long r = blockIdx.y;
  __shared__ int wsum[16];
  int carry = 0;
  for (long long base = 0; base <= n; base += 1024) {
    const long long i = base + threadIdx.x;
    const int v = i < n ? cnt[r * (n + 1) + i] : 0;
    int total;
    const int excl = carry + mh_block_excl_scan<int, 16>(v, total, wsum);
    if (i <= n) {
      rowptr[r * (n + 1) + i] = excl;
      cursor[r * (n + 1) + i] = excl;
    }
    carry += total;
  }
}

extern "C" __global__ __launch_bounds__(256) void csr_scatter(const int* __restrict__ keys, int* __restrict__ cursor,
    int* __restrict__ tmp, long long E, int n) {
  const long long e = (long long)blockIdx.x * 256 + threadIdx.x;
  if (e >= E) return;
  const long long r = blockIdx.y;
  const int pos = atomicAdd(&cursor[r * (n + 1) + keys[r * E + e]], 1);
  tmp[r * E + pos] = (int)e;
}

extern "C" __global__ __launch_bounds__(256) void csr_rank(const int* __restrict__ keys, const int* __restrict__ rowptr,
    const int* __restrict__ tmp, int* __restrict__ eids, long long E, int n) {
  const long long p = (long long)blockIdx.x * 256 + threadIdx.x;
  if (p >= E) return;
  const long long r = blockIdx.y;
  const int e = tmp[r * E + p];
  const int k = keys[r * E + e];
  const int b = rowptr[r * (n + 1) + k], t = rowptr[r * (n + 1) + k + 1];
  if (t - b > RANK_MAX) {                 // sorted in place by csr_sort_long
    eids[r * E + p] = e;
    return;
  }
  int rank = 0;
  for (int q = b; q < t; ++q) rank += tmp[r * E + q] < e;
  eids[r * E + b + rank] = e;
}

// Comparator c of step (k, j) of an ascending-only bitonic network over P = 2^m slots: lo has bit j clear; the first
// step of stage k pairs lo with its mirror image lo ^ (k - 1), the others with lo | j.  Every comparator puts the
// smaller value at the lower index, so slots past the segment's end behave as +infinity and their comparators are
// skipped.
__device__ __forceinline__ void csr_cmp_pair(int c, int k, int j, int& lo, int& hi) {
  lo = ((c & ~(j - 1)) << 1) | (c & (j - 1));
  hi = j == (k >> 1) ? (lo ^ (k - 1)) : (lo | j);
}

extern "C" __global__ __launch_bounds__(256) void csr_sort_long(const int* __restrict__ rowptr,
    int* __restrict__ tmp, long long E, int n) {
  const int node = blockIdx.x;
  if (node >= n) return;
  const long long r = blockIdx.y;
  const int b = rowptr[r * (n + 1) + node], L = rowptr[r * (n + 1) + node + 1] - b;
  if (L <= RANK_MAX) return;
  int P = 1;
  while (P < L) P <<= 1;
  int* __restrict__ seg = tmp + r * E + b;
  __shared__ int s[SORT_LDS];
  const bool in_lds = P <= SORT_LDS;
  int* a = in_lds ? s : seg;
  if (in_lds) {
    for (int i = threadIdx.x; i < L; i += 256) s[i] = seg[i];
    __syncthreads();
  }
  for (int k = 2; k <= P; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int c = threadIdx.x; c < (P >> 1); c += 256) {
        int lo, hi;
        csr_cmp_pair(c, k, j, lo, hi);
        if (hi < L) {
          const int x = a[lo], y = a[hi];
          if (x > y) { a[lo] = y; a[hi] = x; }
        }
      }
      __syncthreads();
    }
  }
  if (in_lds)
    for (int i = threadIdx.x; i < L; i += 256) seg[i] = s[i];
}

// Edge rows of a masked cutoff (mh_edge_compact): the edges whose cutoff is not -0.0 (inside the cutoff envelope's
// support) in increasing order from the front, the others from the back, and their number.  Workgroups of
// EC_EDGES edges (1024 threads x 4): edge_count writes each workgroup's count of kept edges, edge_place adds the
// counts of the workgroups before its own and places its edges by a block scan.  No atomics: the order is fixed.
// With a flag array kv (mh_edge_pairs) a second list is built in the same pass: rows2 / count2 hold the edges whose
// flag is set, in the same arrangement (per-workgroup counts of both lists in bc[0 .. nb) and bc[nb .. 2 nb)).
#define EC_EDGES 4096
__device__ __forceinline__ int ec_keep(const float* __restrict__ cut, long long e, long long E) {
  return e < E && __float_as_uint(cut[e]) != 0x80000000u ? 1 : 0;
}
__device__ __forceinline__ int ec_flag(const int* __restrict__ kv, long long e, long long E) {
  return e < E && kv[e] != 0 ? 1 : 0;
}

extern "C" __global__ __launch_bounds__(1024) void edge_count(const float* __restrict__ cut, long long E,
    int* __restrict__ bc, const int* __restrict__ kv) {
  __shared__ int wsum[16];
  const long long e0 = (long long)blockIdx.x * EC_EDGES + 4 * threadIdx.x;
  int c = 0, c2 = 0;
  for (int k = 0; k < 4; ++k) c += ec_keep(cut, e0 + k, E);
  if (kv)
    for (int k = 0; k < 4; ++k) c2 += ec_flag(kv, e0 + k, E);
  int total;
  mh_block_excl_scan<int, 16>(c, total, wsum);
  if (threadIdx.x == 0) bc[blockIdx.x] = total;
  if (kv) {                               // (uniform: the same pointer for every thread)
    __syncthreads();                      // wsum reused
    mh_block_excl_scan<int, 16>(c2, total, wsum);
    if (threadIdx.x == 0) bc[gridDim.x + blockIdx.x] = total;
  }
}

// Place one list: kept edges in increasing order from the front, the others from the back.
__device__ __forceinline__ void ec_place(const int (&kk)[4], long long e0, long long E, const int* __restrict__ bcl,
    int nb, int* __restrict__ rows, int* __restrict__ count, int* wsum) {
  const int b = blockIdx.x;
  int part = 0;                           // kept edges of the workgroups before this one
  for (int j = threadIdx.x; j < b; j += 1024) part += bcl[j];
  int off;
  mh_block_excl_scan<int, 16>(part, off, wsum);
  __syncthreads();                        // wsum reused
  const int c = kk[0] + kk[1] + kk[2] + kk[3];
  int mine;
  long long p = off + mh_block_excl_scan<int, 16>(c, mine, wsum);    // kept edges before e0
  for (int k = 0; k < 4; ++k) {
    const long long e = e0 + k;
    if (e >= E) break;
    if (kk[k]) rows[p++] = (int)e;
    else rows[E - 1 - (e - p)] = (int)e;  // e - p dropped edges come before e
  }
  if (b == nb - 1 && threadIdx.x == 0) count[0] = off + mine;
}

extern "C" __global__ __launch_bounds__(1024) void edge_place(const float* __restrict__ cut, long long E,
    const int* __restrict__ bc, int nb, int* __restrict__ rows, int* __restrict__ count, const int* __restrict__ kv,
    int* __restrict__ rows2, int* __restrict__ count2) {
  __shared__ int wsum[16];
  const long long e0 = (long long)blockIdx.x * EC_EDGES + 4 * threadIdx.x;
  int kk[4];
  for (int k = 0; k < 4; ++k) kk[k] = ec_keep(cut, e0 + k, E);
  ec_place(kk, e0, E, bc, nb, rows, count, wsum);
  if (kv) {
    __syncthreads();
    for (int k = 0; k < 4; ++k) kk[k] = ec_flag(kv, e0 + k, E);
    ec_place(kk, e0, E, bc + nb, nb, rows2, count2, wsum);
  }
}

// Shared radial-MLP rows between an edge and its reverse (mh_edge_pairs).  The MLP's output row is a function of
// the edge's feature row alone, so two edges whose feature rows are bitwise equal have bitwise-equal W0 rows.  For
// an edge e = (s -> r) inside the cutoff's support with r < s, the edges r -> s into s (MACE's neighbour lists hold
// the reverse of every edge, at the same length) are searched for one inside the support whose feature row equals
// e's bit for bit; the first in CSR order becomes e's W0 row (wrow[e]) and e needs no row of its own (keep[e] = 0).
// Every other edge inside the support keeps its own row.  A partner always keeps its own row (its sender is the
// smaller endpoint), so every row read through wrow is computed.  One wave per node s: the edges out of s one per
// lane, the edges into s 64 at a time in registers, scanned by readlane.  Deterministic; no atomics.
//
// With vec (the edge vectors, [E][3]) and partner: a candidate must also be e's exact reverse, vec[e2] == -vec[e]
// component by component, and each candidate is taken by one edge at most, so that partner[e2] = e names the one
// edge that reads e2's row (-1: none).  Every such claim on an edge into s is made by s's own wave: the claims are
// recorded in an LDS bitmap of s's incoming CSR positions (lanes of one round that want the same candidate: the
// lowest lane takes it, the others search on), partner[] is written for the claims as they are made and with -1 for
// every other edge into s at the end, each entry once.  A node with more than PAIR_DEG_MAX incoming edges makes no
// claims (its edges keep their own rows).
extern "C" __global__ __launch_bounds__(256) void edge_pair(const float* __restrict__ ef, int nf,
    const float* __restrict__ cut, const int* __restrict__ rowptr_r, const int* __restrict__ eids_r,
    const int* __restrict__ rowptr_s, const int* __restrict__ eids_s, const int* __restrict__ senders,
    const int* __restrict__ receivers, int N, int* __restrict__ wrow, int* __restrict__ keep,
    const float* __restrict__ vec, int* __restrict__ partner) {
  __shared__ unsigned claimed[4][PAIR_DEG_MAX / 32];
  // node, ranges and loop bounds wave-uniform (readfirstlane: scalar registers and scalar branches)
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int s = blockIdx.x * 4 + wv;
  if (s >= N) return;
  const int a0 = __builtin_amdgcn_readfirstlane(rowptr_r[s]), a1 = __builtin_amdgcn_readfirstlane(rowptr_r[s + 1]);
  const int b0 = __builtin_amdgcn_readfirstlane(rowptr_s[s]), b1 = __builtin_amdgcn_readfirstlane(rowptr_s[s + 1]);
  const bool rev = partner != nullptr;                    // unique exact-reverse partners (wave-uniform)
  const bool can = !rev || a1 - a0 <= PAIR_DEG_MAX;      // (wave-uniform)
  if (rev)
    for (int w = lane; w < PAIR_DEG_MAX / 32; w += 64) claimed[wv][w] = 0u;
  // the first 64 edges into s (all of them for most nodes): edge ids and senders held in registers; their index
  // loads go out together with those of the first 64 edges out of s (positions clamped into the ranges, the
  // conditions wave-uniform), so the two chains share their round trips
  // (one basic block for the common case: a wait-count pass merges branches conservatively)
  int eid0 = 0, is0 = -1, eo0 = 0;
  if (a1 > a0 && b1 > b0) {
    eid0 = eids_r[min(a0 + lane, a1 - 1)];
    eo0 = eids_s[min(b0 + lane, b1 - 1)];
  } else if (a1 > a0) {
    eid0 = eids_r[min(a0 + lane, a1 - 1)];
  }
  for (int pb = b0; pb < b1; pb += 64) {
    const int p = pb + lane;
    int e = 0, r = 0, w = 0, kp = 0;
    bool look = false;
    float vx = 0.f, vy = 0.f, vz = 0.f;
    unsigned ce = 0x80000000u;
    if (p < b1) {
      e = pb == b0 ? eo0 : eids_s[p];
      r = receivers[e];
      ce = __float_as_uint(cut[e]);
      if (rev) { vx = vec[3 * (size_t)e]; vy = vec[3 * (size_t)e + 1]; vz = vec[3 * (size_t)e + 2]; }
    }
    if (pb == b0 && a1 > a0) is0 = senders[eid0];       // in flight with the loads above
    if (p < b1) {                                        // (the loaded values used only after every load is out)
      w = e;
      kp = ce != 0x80000000u ? 1 : 0;
      look = kp && r < s && can;
    }
    // Each round finds, per looking lane, the first edge from r into s at CSR position >= from (registers and
    // readlane only), then checks that candidate's cutoff, feature row and vector with one round of loads (all
    // issued before any is used: indices clamped in range instead of branches); a lane whose candidate differs (or,
    // with partners, is taken) resumes after it (another image of the same pair), one with none stops.
    int from = a0;
    while (__any(look)) {
      int cand = -1;
      for (int qb = a0; qb < a1; qb += 64) {
        int is = is0;
        if (qb != a0) {
          is = -1;
          if (qb + lane < a1) is = senders[eids_r[qb + lane]];
        }
        const int nq = min(64, a1 - qb);
        for (int q = 0; q < nq; ++q) {
          const int s2 = __builtin_amdgcn_readlane(is, q);
          if (look && cand < 0 && s2 == r && qb + q >= from) cand = qb + q;
          if ((q & 7) == 7 && !__any(look && cand < 0)) break;     // every lane has its candidate
        }
        if (!__any(look && cand < 0)) break;
      }
      const int e2r = __shfl(eid0, (cand - a0) & 63);    // the candidate's edge id when among the first 64
      bool same = false;
      int e2 = 0;
      if (look && cand >= 0) {
        e2 = cand < a0 + 64 ? e2r : eids_r[cand];
        const unsigned c2 = __float_as_uint(cut[e2]);
        const float* __restrict__ vb = rev ? vec : cut;  // without vectors: any valid address, result unused
        const size_t vo = rev ? 3 * (size_t)e2 : 0;
        const int vs = rev ? 1 : 0;
        const float w0 = vb[vo], w1 = vb[vo + vs], w2 = vb[vo + 2 * vs];
        unsigned d = 0u;                                  // bitwise difference of the two feature rows
        for (int f0 = 0; f0 < nf; f0 += 8) {
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int f = min(f0 + j, nf - 1);
            d |= __float_as_uint(ef[(size_t)e * nf + f]) ^ __float_as_uint(ef[(size_t)e2 * nf + f]);
          }
        }
        same = c2 != 0x80000000u && d == 0u && (!rev || (w0 == -vx && w1 == -vy && w2 == -vz));
      }
      if (rev) {
        // one claim per candidate: not taken in an earlier round, and no lower lane of this round wants it
        const int want = same ? cand - a0 : -1;
        bool take = same && !(claimed[wv][want >> 5 & (PAIR_DEG_MAX / 32 - 1)] >> (want & 31) & 1u);
        const int nj = min(64, b1 - pb);                  // lanes holding an edge of this batch
        for (int j = 0; j < nj; ++j) {
          const int wj = __builtin_amdgcn_readlane(want, j);
          if (j < lane && wj == want) take = false;
        }
        if (take) {
          atomicOr(&claimed[wv][want >> 5], 1u << (want & 31));
          partner[e2] = e;
        }
        same = take;
      }
      if (look) {
        if (cand < 0) {
          look = false;
        } else if (same) {
          w = e2; kp = 0; look = false;
        } else {
          from = cand + 1;
        }
      }
    }
    if (p < b1) { wrow[e] = w; keep[e] = kp; }
  }
  if (rev) {
    __builtin_amdgcn_wave_barrier();
    for (int q = a0 + lane; q < a1; q += 64)
      if (!can || !(claimed[wv][((q - a0) >> 5) & (PAIR_DEG_MAX / 32 - 1)] >> ((q - a0) & 31) & 1u))
        partner[q < a0 + 64 ? eid0 : eids_r[q]] = -1;
  }
}
"""


RANK_MAX = 128             # longest segment ordered by counting in csr_rank; longer ones by csr_sort_long
EC_EDGES = 4096            # edges per workgroup of mh_edge_compact's kernels (fixed in graph_source)
SORT_LDS = 8192            # longest segment csr_sort_long sorts in LDS (longer: in place in global memory)
PAIR_DEG_MAX = 2048        # incoming edges of a node up to which edge_pair records unique partners (a power of 2)
_GRAPH_MODULES = {}        # device index -> module of the graph-build kernels


def _graph_module(device):
    idx = device.index if device.index is not None else torch.cuda.current_device()
    m = _GRAPH_MODULES.get(idx)
    if m is None:
        code = _native.compile_source(graph_source())
        with torch.cuda.device(idx):
            m = _native.Module(code, {_native.MH_CSR_FILL: ('csr_fill', 256, 256, 2),
                                      _native.MH_CSR_COUNT: ('csr_count', 256, 256, 2),
                                      _native.MH_CSR_SCAN: ('csr_scan', 1024, 1, 2),
                                      _native.MH_CSR_SCATTER: ('csr_scatter', 256, 256, 2),
                                      _native.MH_CSR_RANK: ('csr_rank', 256, 256, 2),
                                      _native.MH_CSR_SORT: ('csr_sort_long', 256, 1, 2),
                                      _native.MH_EDGE_COUNT: ('edge_count', 1024, EC_EDGES),
                                      _native.MH_EDGE_PLACE: ('edge_place', 1024, EC_EDGES),
                                      _native.MH_EDGE_PAIR: ('edge_pair', 256, 4)})
        _GRAPH_MODULES[idx] = m
    return m


def build_graph(edge_index, n):
    """(keys [2, E], rowptr [2, n + 1], eids [2, E], bad [1]) of an edge list on the GPU (``mh_graph_build``): the
    int32 senders and receivers clamped into [0, n), both CSRs, and a flag set when an index was out of range."""
    ei = edge_index if edge_index.dtype == torch.int64 else edge_index.to(torch.int64)
    ei = ei.contiguous()
    E = ei.shape[1]
    if E > 0 and n == 0:
        raise ValueError('edge_index has edges but there are no nodes')
    if E >= 2 ** 31 or n >= 2 ** 31 - 1:
        raise ValueError('graph too large for int32 indices')
    dev = ei.device
    keys = torch.empty(2, E, device=dev, dtype=torch.int32)
    rowptr = torch.empty(2, n + 1, device=dev, dtype=torch.int32)
    eids = torch.empty(2, E, device=dev, dtype=torch.int32)
    work = torch.empty(4 * (n + 1) + 2 * E, device=dev, dtype=torch.int32)
    bad = torch.empty(1, device=dev, dtype=torch.int32)
    P = _native.ptr
    _native.launch('graph_build', _native.load().mh_graph_build, _graph_module(dev).handle, P(ei), E, n, P(keys),
                   P(rowptr), P(eids), P(work), P(bad), _native.stream_of(ei))
    return keys, rowptr, eids, bad


# How a new edge_index is checked for nodes outside [0, n).  The graph build clamps such indices (so no kernel ever
# reads out of range) and sets a device flag.  'deferred': the flag is copied to pinned host memory behind the build
# and read when that copy has landed, at the next graph lookup or at check_graphs(); no host synchronisation.
# 'sync': the flag is read at once (one device-to-host synchronisation per new edge_index).  Edge lists made by
# mace_hip_kernels.neighbours are in range by construction and are not checked.
GRAPH_CHECK = 'deferred'
_pending_checks = []       # [(pinned int32 [1], event, shape, n)] of edge lists whose flag has not been read


def check_graphs(block=True):
    """Read the out-of-range flags of the edge lists built since the last check (``block``: wait for them; else
    only those already available) and raise ValueError if any edge_index held a node outside [0, n)."""
    keep, bad = [], None
    for item in _pending_checks:
        flag, ev, shape, n = item
        if not block and not ev.query():
            keep.append(item)
            continue
        ev.synchronize()
        if int(flag[0]) and bad is None:
            bad = (shape, n)
    _pending_checks[:] = keep
    if bad is not None:
        raise ValueError(f'an edge_index of shape {bad[0]} given to a patched convolution held nodes outside '
                         f'[0, {bad[1]}); that call clamped them (its results are wrong)')


class _Graph:
    """int32 senders/receivers and both CSRs of one edge_index (``build_graph``), shared by every layer of a call.

    Out-of-range indices are clamped into [0, n), so a bad edge list gives wrong numbers, never an out-of-range
    access; ``validate`` reports them (see GRAPH_CHECK).  ``validate=False`` (a graph first met inside a HIP graph
    capture, which can neither synchronise nor record the check): no report."""

    def __init__(self, edge_index, n, validate=True):
        if edge_index.dim() != 2 or edge_index.shape[0] != 2:
            raise ValueError(f'edge_index must be [2, E], got {tuple(edge_index.shape)}')
        self.n = n
        keys, rowptr, eids, bad = build_graph(edge_index, n)
        if validate and edge_index.shape[1] and not neighbours.built_here(edge_index, n):
            if GRAPH_CHECK == 'sync':
                if int(bad.item()):
                    # the kernels index x, g and the CSRs with these values: out-of-range nodes are an error
                    lo, hi = (int(v) for v in torch.aminmax(edge_index))
                    raise ValueError(f'edge_index holds node {lo if lo < 0 else hi} outside [0, {n})')
            else:
                flag = torch.empty(1, dtype=torch.int32, pin_memory=True)
                flag.copy_(bad, non_blocking=True)
                ev = torch.cuda.Event()
                ev.record()
                _pending_checks.append((flag, ev, tuple(edge_index.shape), n))
        self.send, self.recv = keys[0], keys[1]
        self._by_send = (rowptr[0], eids[0])
        self._by_recv = (rowptr[1], eids[1])
        self._keep = (keys, rowptr, eids)

    def by_recv(self):
        return self._by_recv

    def by_send(self):
        return self._by_send


_graph_cache = []          # [(weakref(edge_index), version, n, _Graph)], most recent first
_GRAPH_CACHE_SIZE = 4
# Set by graphs.capture(rebuild_graph=True): a capture builds the graph of an edge_index it meets (clamped, no host
# validation) instead of reusing the eager cache, so every replay rebuilds the CSRs from the tensor's contents.
_capture_rebuild = False
_capture_graphs = {}       # graphs built inside the current capture, by (id(edge_index), n); cleared after capture


def graph_for(edge_index, n):
    """Cached ``_Graph`` for this edge_index tensor object (invalidated by in-place modification or deletion)."""
    if _pending_checks and not _native.capturing():
        check_graphs(block=False)
    if _native.capturing() and _capture_rebuild:
        gr = _capture_graphs.get((id(edge_index), n))
        if gr is None or gr.src is not edge_index:
            gr = _Graph(edge_index, n, validate=False)
            gr.src = edge_index
            _capture_graphs[(id(edge_index), n)] = gr
        return _native.hold_for_capture(gr)
    ver = edge_index._version
    for i, (ref, v, nn_, gr) in enumerate(_graph_cache):
        if ref() is edge_index and v == ver and nn_ == n:
            if i:
                _graph_cache.insert(0, _graph_cache.pop(i))
            return _native.hold_for_capture(gr)
    if _native.capturing():
        # building a graph validates it on the host (a synchronisation), which a capture cannot contain
        raise RuntimeError('mace_hip_kernels: this edge_index is new inside a HIP graph capture; run the model once '
                           'eagerly on the same tensors before capturing (mace_hip_kernels.graphs.capture does), or '
                           'capture with rebuild_graph=True')
    gr = _Graph(edge_index, n)
    _graph_cache.insert(0, (weakref.ref(edge_index), ver, n, gr))
    del _graph_cache[_GRAPH_CACHE_SIZE:]
    return gr


def clear_graph_cache():
    _graph_cache.clear()


# ------------------------------------------------------------------------------------------------ autograd
_DOUBLE_BACKWARD = ('mace_hip_kernels: double backward (create_graph=True, e.g. training on forces/stress or an '
                    'autograd Hessian) is not enabled for this HIP module; patch with '
                    'patch_model(model, double_backward=True)')


def _check_inputs(op, x, Y, W, edge_index):
    s = op.spec
    if x.dtype != torch.float32 or Y.dtype != torch.float32 or W.dtype != torch.float32:
        raise TypeError('mace_hip_kernels: conv_tp expects float32 inputs')
    if not (x.is_cuda and Y.is_cuda and W.is_cuda and edge_index.is_cuda):
        raise RuntimeError('mace_hip_kernels: conv_tp inputs must be on the GPU')
    E = edge_index.shape[1]
    if x.dim() != 2 or x.shape[1] != s.x_dim:
        raise ValueError(f'node_feats must be [N, {s.x_dim}], got {tuple(x.shape)}')
    if Y.shape != (E, s.y_dim):
        raise ValueError(f'edge_attrs must be [{E}, {s.y_dim}], got {tuple(Y.shape)}')
    if W.shape != (E, s.nins * s.mul):
        raise ValueError(f'tp_weights must be [{E}, {s.nins * s.mul}], got {tuple(W.shape)}')
    if x.shape[0] >= 2 ** 31 or E >= 2 ** 31:
        raise ValueError('graph too large for int32 indices')


def _grad_needed(ctx, i):
    """Whether this backward pass uses the gradient of input i.  ``needs_input_grad`` is fixed at forward time; the
    engine knows more: under ``autograd.grad(E, positions)`` the branch from the first layer's node features to
    ``node_attrs`` is never executed, so that gradient would be computed and dropped.  e3nn's own backward ops skip
    such outputs through the engine's output mask; here the engine is asked whether the node that receives the
    gradient will run.  Anything it cannot answer (a leaf that is itself a requested input) counts as needed."""
    if not ctx.needs_input_grad[i]:
        return False
    node = ctx.next_functions[i][0]
    if node is None:
        return True
    try:
        return bool(torch._C._will_engine_execute_node(node))
    except (RuntimeError, AttributeError):
        return True


def _factored_weights(W):
    """(W0, cutoff) when ``W`` is the product ``W0 * cutoff`` that MACE forms right before the convolution
    (``tp_weights = self.conv_tp_weights(edge_feats) * cutoff``, W0 [E, NW], cutoff [E, 1]), read from the product's
    autograd node; otherwise None.  The backward then takes the gradients of W0 and cutoff from the kernel directly
    and the product's own backward (a pass over [E, NW] for each factor) never runs; any other use of the product
    still gets its gradient through that node.  Anything unexpected (no graph, other op, other shapes, a factor that
    needs no gradient, a factor modified in place) keeps the plain path."""
    gf = W.grad_fn
    if gf is None or type(gf).__name__ != 'MulBackward0' or W.dim() != 2:
        return None
    try:
        a, b = gf._saved_self, gf._saved_other
    except (RuntimeError, AttributeError):
        return None
    if a is None or b is None:
        return None
    E, nw = W.shape
    for w0, c in ((a, b), (b, a)):
        if (isinstance(w0, torch.Tensor) and isinstance(c, torch.Tensor) and tuple(w0.shape) == (E, nw)
                and tuple(c.shape) in ((E, 1), (E,)) and w0.dtype == torch.float32 and c.dtype == torch.float32
                and w0.device == W.device and c.device == W.device):
            return w0, c
    return None


class CutoffProduct(torch.Tensor):
    """The product W0 * cutoff ([E, NW] * [E, 1]) that MACE forms from the radial MLP's output right before the
    convolution, kept as its two factors: a tensor of the product's shape and dtype without storage of its own.
    The convolution reads the factors (its kernels scale W0 by the cutoff in registers), so the product is never
    written to or read from memory; any other operation on it computes the product first and runs on that, so
    every other consumer sees an ordinary tensor.  Its autograd node is the product rule (``_CutoffMul``)."""

    @staticmethod
    def __new__(cls, w0, cut):
        return torch.Tensor._make_wrapper_subclass(cls, w0.shape, dtype=w0.dtype, device=w0.device,
                                                   requires_grad=False)

    def __init__(self, w0, cut):
        self.w0, self.cut = w0, cut

    __torch_function__ = torch._C._disabled_torch_function_impl

    @classmethod
    def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
        def real(t):
            return t.w0 * t.cut if isinstance(t, CutoffProduct) else t
        args = torch.utils._pytree.tree_map(real, args)
        kwargs = torch.utils._pytree.tree_map(real, kwargs or {})
        return func(*args, **kwargs)


class _CutoffMul(torch.autograd.Function):
    @staticmethod
    def forward(ctx, w0, cut):
        ctx.save_for_backward(w0, cut)
        return CutoffProduct(w0, cut)

    @staticmethod
    def backward(ctx, g):
        w0, cut = ctx.saved_tensors
        gw0 = g * cut if ctx.needs_input_grad[0] else None
        gc = (g * w0).sum(-1, keepdim=True).reshape(cut.shape) if ctx.needs_input_grad[1] else None
        return gw0, gc


class RadialWeights(torch.Tensor):
    """A radial MLP's output W0 [E, NW] (an ordinary tensor of this subclass) whose product with a per-edge column
    ``W0 * cutoff`` ([E, 1], same device and dtype) is returned as a ``CutoffProduct`` instead of being computed.
    Every other operation behaves as on a plain tensor and returns plain tensors."""

    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        if func in _MULS and len(args) == 2 and not kwargs:
            a, b = args
            if isinstance(b, RadialWeights) and not isinstance(a, RadialWeights):
                a, b = b, a
            if (isinstance(a, RadialWeights) and torch.is_tensor(b) and not isinstance(b, RadialWeights)
                    and a.dim() == 2 and tuple(b.shape) == (a.shape[0], 1) and b.dtype == a.dtype
                    and b.device == a.device and a.dtype == torch.float32):
                return _CutoffMul.apply(a.as_subclass(torch.Tensor), b)
        with torch._C.DisableTorchFunctionSubclass():
            return func(*args, **kwargs)


_MULS = {torch.Tensor.__mul__, torch.Tensor.__rmul__, torch.Tensor.mul, torch.mul}


EDGE_COMPACT_MIN = 16384   # fewer edges: the radial MLP walks every edge (compacting costs two launches)
# patch_model runs each patched convolution's patched radial MLP inside the convolution's autograd node
# (HipConvTP.defer_mlp, conv_mlp.ConvRadialFn) unless double_backward or fuse_radial asks otherwise
DEFER_RADIAL = True


def support_rows(cut):
    """(rows int32 [E], count int32 [1]) of a cutoff column (``mh_edge_compact``): the edges inside the cutoff's
    support (cutoff not -0.0) in increasing order, then the others; count[0] = how many are inside.  Cached on the
    tensor for its current version, so the interaction layers sharing MACE's cutoff compact it once per call."""
    owner = stash_owner(cut)
    c = getattr(owner, '_mh_rows', None)
    if c is not None and c[0] == cut._version:
        return c[1], c[2]
    flat = cut.reshape(-1).contiguous()
    E = flat.shape[0]
    lib, P = _native.load(), _native.ptr
    rows = torch.empty(E, dtype=torch.int32, device=cut.device)
    count = torch.empty(1, dtype=torch.int32, device=cut.device)
    work = torch.empty(-(-lib.mh_edge_compact_work_size(E) // 4), dtype=torch.int32, device=cut.device)
    _native.launch('edge_compact', lib.mh_edge_compact, _graph_module(cut.device).handle, P(flat), E, P(rows),
                   P(count), P(work), _native.stream_of(flat))
    owner._mh_rows = (cut._version, rows, count)
    return rows, count


# the deferred radial MLP computes one W0 row per pair of an edge and its reverse when their feature rows are equal
# (support_pairs); off, one row per edge inside the cutoff's support
PAIR_RADIAL = True
# ... and, when only the sum of an edge's and its exact reverse's length gradients reaches the positions (features of
# the patched geometry's lengths, shifts without gradient), the MLP's backward projects each shared row once from the
# pair's summed dL/dW0 (conv_mlp.ConvRadialFn, mh_mlp_bwd_pairs)
PAIR_GRADS = True


def support_pairs(ef, cut, gr, vec=None):
    """(wrow int32 [E], rows int32 [E], count int32 [1], partner int32 [E] or None) of ``mh_edge_pairs`` for the MLP
    input rows ``ef`` [E, nf], the cutoff column ``cut`` and the graph ``gr`` (both CSRs): edge e reads its W0 row at
    wrow[e], and rows[:count] lists the edges whose rows the MLP computes (inside the cutoff's support, not mapped to
    a reverse edge with an equal feature row).  With the edge vectors ``vec`` [E, 3] a partner must also be the exact
    reverse (negated vector), each row is shared by one other edge at most, and ``partner[e]`` names it (-1: none):
    the map of the paired MLP backward.  Cached on the cutoff tensor for its version, the features' and vectors'
    storage and version and the graph, so both interaction layers (which share MACE's edge features and cutoff) pair
    the edges once per call; the same launch also fills ``support_rows``'s cache for the cutoff."""
    vkey = None if vec is None else (vec.data_ptr(), vec._version)
    key = (cut._version, ef.data_ptr(), ef._version, gr, vkey)
    owner = stash_owner(cut)
    c = getattr(owner, '_mh_pairs', None)
    if c is not None and c[0] == key:
        return c[1], c[2], c[3], c[4]
    E = cut.numel()
    efc = ef.reshape(E, -1).contiguous()
    cutf = cut.reshape(-1).contiguous()
    dev = cut.device
    lib, P = _native.load(), _native.ptr
    wrow = torch.empty(E, dtype=torch.int32, device=dev)
    rows = torch.empty(E, dtype=torch.int32, device=dev)
    count = torch.empty(1, dtype=torch.int32, device=dev)
    srows = torch.empty(E, dtype=torch.int32, device=dev)
    scount = torch.empty(1, dtype=torch.int32, device=dev)
    vc = None if vec is None else vec.reshape(E, 3).contiguous()
    partner = None if vec is None else torch.empty(E, dtype=torch.int32, device=dev)
    work = torch.empty(-(-lib.mh_edge_pairs_work_size(E) // 4), dtype=torch.int32, device=dev)
    (rowptr_r, eids_r), (rowptr_s, eids_s) = gr.by_recv(), gr.by_send()
    _native.launch('edge_pairs', lib.mh_edge_pairs, _graph_module(dev).handle, P(efc), efc.shape[1], P(cutf),
                   P(rowptr_r), P(eids_r), P(rowptr_s), P(eids_s), P(gr.send), P(gr.recv), gr.n, E, P(vc), P(wrow),
                   P(partner), P(rows), P(count), P(srows), P(scount), P(work), _native.stream_of(cutf))
    owner._mh_pairs = (key, wrow, rows, count, partner, efc, vc)   # (efc, vc keep the keyed storage alive)
    owner._mh_rows = (cut._version, srows, scount)            # the support list came from the same pass
    return wrow, rows, count, partner


def _support_masked(cut):
    """Whether ``cut`` is a patched radial embedding's cutoff, unmodified since: -0.0 then marks exactly the edges
    outside the envelope's support, where the envelope's derivative is zero."""
    return getattr(stash_owner(cut), '_mh_support_mask', None) == cut._version


def _conv_grads(op, gr, g, x, Y, W, W0, cut, want_x, want_wy, masked=False, nozero=False, wrow=None):
    """First-order gradients (gx, gY, gW or gW0, gcut) of <g, conv(x, Y, W)> for contiguous operands, by the
    kernels; W = W0 * cut (cut flat [E]) when W is None.  Entries not wanted are None.  ``masked`` (factored only):
    edges with cut == -0.0 lie outside the cutoff envelope's support, and their gradients, gcut included, are zero
    (the envelope's derivative there is zero, so gcut's true value there never matters to its producer).
    ``nozero`` (with ``masked``): those edges' gW0 rows are left unset, for a consumer that skips them.  ``wrow``
    (factored only): edge e's W0 row is row wrow[e] (support_pairs); gW0 stays one row per edge."""
    factored = W is None
    E = Y.shape[0]
    gx = torch.empty_like(x) if want_x else None
    gY = torch.empty_like(Y) if want_wy else None
    gW = torch.empty_like(W0 if factored else W) if want_wy else None
    gcut = torch.empty_like(cut) if want_wy and factored else None
    # with no edges gW and gY are empty (NULL data pointers): nothing to compute for them
    flags = (_native.MH_WANT_GX if want_x else 0) | (_native.MH_WANT_GWY if want_wy and E > 0 else 0)
    if masked and factored and flags & _native.MH_WANT_GWY:
        flags |= _native.MH_CUT_MASKED | (_native.MH_CUT_NOZERO if nozero else 0)
    lib = _native.load()
    P = _native.ptr
    if flags & _native.MH_WANT_GWY and (op.bwd_recv or factored):
        # receiver order: g rows read once per receiver; dX goes through per-edge messages in `work`
        rowptr_r, eids_r = gr.by_recv()
        rowptr_s, eids_s = gr.by_send() if want_x else (None, None)
        work = torch.empty(E, op.spec.x_dim, device=x.device, dtype=torch.float32) if want_x else None
        _native.launch(f'conv_bwd[{op.tag}]', lib.mh_conv_bwd_recv_rows, op.module.handle, P(x), P(g), P(Y),
                       P(W0 if factored else W), P(rowptr_r), P(eids_r), P(gr.send), P(rowptr_s), P(eids_s),
                       P(work), P(gx), P(gW), P(gY), P(cut), P(gcut), P(wrow), x.shape[0], flags,
                       _native.stream_of(x))
    elif flags:
        if factored:                     # dX only: the sender-ordered kernel needs the product
            # rows of edges with a zero cutoff may be unset (a row-listed MLP skips them): exact zeros there
            c = cut[:, None]
            W = torch.where(c == 0, torch.zeros((), device=c.device), (W0 if wrow is None else W0[wrow.long()]) * c)
        rowptr_s, eids_s = gr.by_send()
        _native.launch(f'conv_bwd[{op.tag}]', lib.mh_conv_bwd, op.module.handle, P(x), P(g), P(Y), P(W),
                       P(rowptr_s), P(eids_s), P(gr.recv), P(gx), P(gW), P(gY), x.shape[0], flags,
                       _native.stream_of(x))
    return gx, gY, gW, gcut


class _ConvFn(torch.autograd.Function):
    """Inputs (x, Y, W, W0, cut, edge_index, op).  Plain: W is the weight tensor, W0 = cut = None.  Factored:
    W is None, W0 and cut are the differentiable inputs and the kernels form W0 * cut per edge in registers."""

    @staticmethod
    def forward(ctx, x, Y, W, W0, cut, edge_index, op):
        _check_inputs(op, x, Y, W if W is not None else W0, edge_index)
        xc, Yc = x.contiguous(), Y.contiguous()
        n = x.shape[0]
        gr = graph_for(edge_index, n)
        rowptr, eids = gr.by_recv()
        out = torch.empty(n, op.spec.out_dim, device=x.device, dtype=torch.float32)
        lib = _native.load()
        ctx.factored = W0 is not None
        P = _native.ptr
        # the inputs themselves are saved (contiguous copies are made again in backward if needed): a double
        # backward differentiates through them
        if ctx.factored:
            cutf = cut.reshape(-1).contiguous()
            # edges with cutoff 0 (padding, or beyond r_max in a skinned neighbour list) contribute exactly zero
            _native.launch(f'conv_fwd[{op.tag}]', lib.mh_conv_fwd_cut, op.module.handle, P(xc), P(Yc),
                           P(W0.contiguous()), P(rowptr), P(eids), P(gr.send), P(cutf), P(out), n,
                           _native.stream_of(x))
            ctx.cut_shape = cut.shape
            ctx.masked = _support_masked(cut)
            ctx.save_for_backward(x, Y, W0, cut, edge_index)
        else:
            _native.launch(f'conv_fwd[{op.tag}]', lib.mh_conv_fwd, op.module.handle, P(xc), P(Yc), P(W.contiguous()),
                           P(rowptr), P(eids), P(gr.send), P(out), n, _native.stream_of(x))
            ctx.save_for_backward(x, Y, W, edge_index)
        ctx.op, ctx.gr = op, gr
        return out

    @staticmethod
    def backward(ctx, g):
        op, gr = ctx.op, ctx.gr
        if ctx.factored:
            x, Y, W0, cut, edge_index = ctx.saved_tensors
            want_w0, want_cut = _grad_needed(ctx, 3), _grad_needed(ctx, 4)
            want_w = want_w0 or want_cut
        else:
            x, Y, W, edge_index = ctx.saved_tensors
            want_w = _grad_needed(ctx, 2)
        want_x, want_y = _grad_needed(ctx, 0), _grad_needed(ctx, 1)
        if torch.is_grad_enabled():          # only true under create_graph=True
            if not op.double_backward:
                raise RuntimeError(_DOUBLE_BACKWARD)
            # the gradients as a differentiable function of (g, x, Y, W or W0 and cut)
            if ctx.factored:
                gx, gY, gW0, gc = _ConvAdjFn.apply(g, x, Y, None, W0, cut, edge_index, op, gr,
                                                   (want_x, want_y, want_w0, want_cut))
                return gx, gY, None, gW0, gc, None, None
            gx, gY, gW, _ = _ConvAdjFn.apply(g, x, Y, W, None, None, edge_index, op, gr,
                                             (want_x, want_y, want_w, False))
            return gx, gY, gW, None, None, None, None
        xc, Yc, gc_ = x.contiguous(), Y.contiguous(), g.contiguous()
        if ctx.factored:
            gx, gY, gW, gcut = _conv_grads(op, gr, gc_, xc, Yc, None, W0.contiguous(), cut.reshape(-1).contiguous(),
                                           want_x, want_y or want_w, masked=ctx.masked and op.skip_masked)
            return gx, gY, None, gW, gcut.view(ctx.cut_shape) if gcut is not None else None, None, None
        gx, gY, gW, _ = _conv_grads(op, gr, gc_, xc, Yc, W.contiguous(), None, None, want_x, want_y or want_w)
        return gx, gY, gW, None, None, None, None


class _ConvAdjFn(torch.autograd.Function):
    """The first-order gradients of <g, conv(x, Y, W)> as a differentiable function of (g, x, Y, W), for a double
    backward; with factored weights W = W0 * cut the inputs are (g, x, Y, W0, cut) and the outputs (gx, gY, gW0,
    gcut).  The convolution is linear in each of x, Y and W (in each of x, Y, W0 and cut), so each second
    derivative is a first-order quantity with one argument replaced by the direction arriving for it: with
    (ggx, ggY, ggW) the gradients arriving for (gx, gY, gW),
        d/dg = conv(ggx, Y, W) + conv(x, ggY, W) + conv(x, Y, ggW),
        d/dx = gx(g; ggY, W) + gx(g; Y, ggW),  d/dY = gY(g; ggx, W) + gY(g; x, ggW),  d/dW = gW(g; ggx, Y) + gW(g; x, ggY),
    and likewise over four arguments when factored (e.g. d/dW0 gains gW(g; x, Y) * ggcut, the gradient of
    <ggcut, gcut>).  Every term is one call of the same kernels (through this function and _ConvFn again, so higher
    orders follow); factored, W0 * cut is never formed.  ``want`` (x, Y, W or W0, cut) says which gradients to
    form; the others are returned as None."""

    @staticmethod
    def forward(ctx, g, x, Y, W, W0, cut, edge_index, op, gr, want):
        wx, wy, ww, wc = want
        factored = W is None
        gx, gY, gW, gc = _conv_grads(op, gr, g.contiguous(), x.contiguous(), Y.contiguous(),
                                     None if factored else W.contiguous(), W0.contiguous() if factored else None,
                                     cut.reshape(-1).contiguous() if factored else None, wx, wy or ww or wc)
        ctx.save_for_backward(g, x, Y, W, W0, cut, edge_index)
        ctx.factored, ctx.op, ctx.gr = factored, op, gr
        return (gx if wx else None, gY if wy else None, gW if ww else None,
                gc.view(cut.shape) if wc and gc is not None else None)

    @staticmethod
    def backward(ctx, ggx, ggY, ggW, ggc):
        g, x, Y, W, W0, cut, edge_index = ctx.saved_tensors
        op, gr = ctx.op, ctx.gr
        need = [_grad_needed(ctx, i) for i in range(6)]          # g, x, Y, W, W0, cut
        if ctx.factored:
            args, dirs, slot = [x, Y, W0, cut], [ggx, ggY, ggW, ggc], [1, 2, 4, 5]
        else:
            args, dirs, slot = [x, Y, W], [ggx, ggY, ggW], [1, 2, 3]
        acc = [None] * 6

        def add(i, t):
            if t is not None:
                acc[i] = t if acc[i] is None else acc[i] + t

        def split(a):                        # argument list -> (x, Y, W, W0, cut)
            return (a[0], a[1], None, a[2], a[3]) if ctx.factored else (a[0], a[1], a[2], None, None)

        for j, d in enumerate(dirs):
            if d is None:
                continue
            a = list(args)
            a[j] = d
            if need[0]:
                add(0, _ConvFn.apply(*split(a), edge_index, op))
            want = [need[slot[k]] and k != j for k in range(len(args))]
            if any(want):
                res = _ConvAdjFn.apply(g, *split(a), edge_index, op, gr, tuple(want + [False] * (4 - len(want))))
                for k in range(len(args)):
                    if k != j:
                        add(slot[k], res[k])
        return acc[0], acc[1], acc[2], acc[3], acc[4], acc[5], None, None, None, None


class HipConvTP(torch.nn.Module):
    """Replacement for an interaction block's ``conv_tp`` under MACE's ``conv_fusion`` path:
    ``forward(node_feats, edge_attrs, tp_weights, edge_index) → summed messages [N, OUT_DIM]``
    (reference conv.py:273-285)."""

    def __init__(self, tp, device=None):
        super().__init__()
        self.spec = ConvSpec(tp)
        self.source = source(self.spec)
        code = _native.compile_source(self.source)
        dev = torch.device(device) if device is not None else torch.device('cuda', torch.cuda.current_device())
        with torch.cuda.device(dev):
            self.module = _native.Module(code, {
                _native.MH_CONV_FWD: (self.spec.kname('conv_fwd'), self.spec.block, 1),
                _native.MH_CONV_BWD: (self.spec.kname('conv_bwd'), self.spec.block, 1),
                _native.MH_CONV_BWD_WY: (self.spec.kname('conv_bwd_wy'), self.spec.block, WAVE),
                _native.MH_CONV_BWD_R: (self.spec.kname('conv_bwdr'), self.spec.block, 1),
                _native.MH_CONV_BWD_RC: (self.spec.kname('conv_bwdrc'), self.spec.block, 1),
                _native.MH_CONV_FWD_C: (self.spec.kname('conv_fwdc'), self.spec.block, 1),
                _native.MH_CONV_FWD_CR: (self.spec.kname('conv_fwdcr'), self.spec.block, 1),
                _native.MH_CONV_GXSUM: (self.spec.kname('conv_gxsum'), gxsum_block(self.spec), 1),
            })
        self.irreps_in1, self.irreps_in2, self.irreps_out = tp.irreps_in1, tp.irreps_in2, tp.irreps_out
        self.instructions = tp.instructions
        self.weight_numel = tp.weight_numel
        self.original = [tp]          # kept (outside the module tree) so the patch can be undone
        self.tag = 'conv'             # name used in launch timings (patch_model sets the module path)
        # backward walks the receiver CSR when gW/gY are wanted (False: the sender-ordered fused kernel)
        self.bwd_recv = True
        # differentiate MACE's tp_weights = W0 * cutoff inside the backward kernel (see _factored_weights)
        self.fuse_cutoff = True
        # first-order backward: skip edges outside the cutoff's support when the cutoff comes unmodified from a
        # patched radial embedding (MH_CUT_MASKED)
        self.skip_masked = True
        # a backward under create_graph=True: raise (the reference's behaviour) unless this is set, in which case
        # the gradients are differentiable again (_ConvAdjFn)
        self.double_backward = False
        # the radial MLP whose output layer the fused kernels carry (attach_mlp), and those kernels
        self.fused = None
        self._fused_mlp = []
        # the radial MLP run inside this convolution's autograd node (defer_mlp: conv_mlp.ConvRadialFn)
        self._deferred_mlp = []

    def attach_mlp(self, mlp):
        """Form this convolution's weights inside its kernels from ``mlp``'s (a HipRadialMLP) last hidden
        activations: compiles the fused kernels and packs the MLP's output layer for them.  (ok, reason)."""
        from .conv_mlp import FusedConv, fused_supported
        ok, why = fused_supported(self.spec, mlp.spec)
        if not ok:
            return False, why
        self.fused = FusedConv(self.spec, mlp.spec, mlp.WhT.device)
        self._fused_mlp = [mlp]                 # a plain list: the MLP stays a module of its own block only
        return True, ''

    def detach_mlp(self):
        self.fused, self._fused_mlp = None, []

    def defer_mlp(self, mlp):
        """Run ``mlp`` (the HipRadialMLP producing this convolution's weights, its output handed over unformed) in
        this convolution's autograd node, so that W0 and dL/dW0 stay inside it and the edges outside the cutoff's
        support are skipped by both modules' kernels (``conv_mlp.ConvRadialFn``).  None detaches it."""
        self._deferred_mlp = [mlp] if mlp is not None else []

    def deferred_mlp(self):
        return self._deferred_mlp[0] if self._deferred_mlp else None

    def fused_mlp(self):
        return self._fused_mlp[0] if self._fused_mlp else None

    def forward(self, node_feats, edge_attrs, tp_weights, edge_index):
        from .conv_mlp import ConvMLPFn, ConvRadialFn, FusedWeights
        from .edgefeat import slot
        # the patched edge pass's outputs shared by several convolutions: this one reads aliases with gradient slots
        # of their own where the pass left them (their gradients then need no separate sum)
        edge_attrs = slot(edge_attrs)
        if isinstance(tp_weights, FusedWeights):
            if self.fused is not None and tp_weights.mlp is self.fused_mlp():
                # W = cutoff * MLP(edge_feats) formed inside the kernels: neither W nor its gradient is stored
                return ConvMLPFn.apply(node_feats, edge_attrs, slot(tp_weights.ef), slot(tp_weights.cut), edge_index,
                                       self)
            if tp_weights.mlp is self.deferred_mlp():
                # the MLP's kernels and this convolution's in one node: rows outside the cutoff's support skipped
                return ConvRadialFn.apply(node_feats, edge_attrs, slot(tp_weights.ef), slot(tp_weights.cut),
                                          edge_index, self)
            tp_weights = tp_weights.value()
        if isinstance(tp_weights, CutoffProduct):
            # the radial MLP's output times the cutoff, never formed: the kernels take the two factors
            return _ConvFn.apply(node_feats, edge_attrs, None, tp_weights.w0, tp_weights.cut, edge_index, self)
        fac = _factored_weights(tp_weights) if self.fuse_cutoff and torch.is_grad_enabled() else None
        if fac is not None:
            W0, cut = fac
            return _ConvFn.apply(node_feats, edge_attrs, None, W0, cut, edge_index, self)
        return _ConvFn.apply(node_feats, edge_attrs, tp_weights, None, None, edge_index, self)

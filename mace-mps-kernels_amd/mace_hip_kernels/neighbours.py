"""
Periodic neighbour lists of a batch of structures on the GPU, in MACE's edge convention and with the fixed-size
padded layout the reference recommends for long runs (reference README.md:77-78: "long runs should use fixed-size
(padded) graphs").

An edge (sender i, receiver j, unit shift o) exists when |pos[j] + o @ cell - pos[i]| < r_max and (i, i, 0) is
excluded.  The search covers the lattice translations reps_k = max(ceil(r_max / h_k), floor(r_max / h_k + span_k))
deep along each periodic direction k (h_k the distance between lattice planes, span_k the range of the structure's
fractional coordinates along k), which holds every such edge also for atoms outside the cell (unwrapped MD
coordinates); more than 64 translations are not searched, and the structure is reported (``n_edges`` -1).
Edges are ordered by (sender, receiver, image), the image index enumerating o lexicographically; with ``pad_edges_to = P`` structure b owns edges [b P, (b + 1) P) and every sender's
real edges are followed by its share of padding edges (self-loops shifted (0, 0, kz) cells, kz = ceil((r_max + 1) /
|c_2|), so the cutoff is exactly zero on them), the padding edges spread round-robin over the structure's atoms.
That is exactly the host builder ``mace_lite.data.neighbour_list`` + ``batch_graphs(pad_edges_to=P)`` (scipy cKDTree
there), which the GPU tests compare against element by element.

The build is one C-ABI call (``mh_neighbour_list``), device work only:
  nl_setup    one workgroup per structure: bounding box of its atoms, periodic image depth, a cell grid of bins at
              least r_max wide (at most n + 1 bins);
  nl_zero, nl_bins, nl_scan, nl_place
              atoms counted into bins, bin offsets by a one-workgroup scan, atoms placed (a counting sort) as
              (x, y, z, index) quads in bin order;
  nl_count    one wave per sender: for each image, the bins within r_max of the sender's image-shifted position are
              walked 64 candidates at a time (the bins of one grid column are contiguous, so each column is one
              range); the distance test is in float64 with no fused multiply-add, as the host computes it;
  nl_offsets  one workgroup per structure: its edge count (``n_edges``), padding shares, and each sender's segment
              start within the structure; nl_bases: each structure's first slot (b P padded, a prefix of the edge
              counts exact);
  nl_fill     one wave per sender: the same walk writes each hit's key (receiver, image) into the sender's segment,
              the segment is ordered by key (each key's rank = the number of smaller keys, counted in LDS), and the
              edges and their padding are written.
No host synchronisation and no allocation inside the call, so a padded build can be captured in a HIP graph.  A
structure with more than ``pad_edges_to`` real edges fills its slots with a subset of its edges (in range, ordered)
and reports its true count in ``n_edges`` (``NeighbourList.check()`` raises on it).  Without padding the edge count
is read back once (a count call, one synchronisation, then the build).
"""
import weakref

import torch

from . import _native

WAVE = 64
SENDERS_PER_BLOCK = 4          # waves per workgroup of nl_count / nl_fill, one sender each
NL_EPS = 1e-6                  # Å of slack in the bin ranges (bins only prune; the distance test is exact)
LDS_KEYS = 256                 # a sender's keys ranked from LDS up to this many (longer segments from L2)


def source():
    """HIP source of the neighbour-list kernels (float64 geometry, int64 keys)."""
    return _native.device_header() + f"""
#define NL_SPB {SENDERS_PER_BLOCK}
#define NL_EPS {NL_EPS!r}
#define NL_LDS_KEYS {LDS_KEYS}
""" + r"""
#pragma clang fp contract(off)
// per-structure parameters: prmd [B][16] doubles (lo[3], bs[3], cell rows c[9]); prmi [B][16] ints (nb[3], reps[3],
// n0, n, nimg, bin0, kz, cut)
#define NL_PD 16
#define NL_PI 16

__device__ __forceinline__ int nl_struct_of(const long long* __restrict__ ptr, int B, long long i) {
  int lo = 0, hi = B;                       // the last b with ptr[b] <= i (ptr[B] = N > i)
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (ptr[mid] <= i) lo = mid; else hi = mid;
  }
  return lo;
}

extern "C" __global__ __launch_bounds__(256) void nl_setup(const double* __restrict__ pos,
    const double* __restrict__ cell, const int* __restrict__ pbc, const long long* __restrict__ ptr, int B,
    double r_max, double* __restrict__ prmd, int* __restrict__ prmi) {
  const int b = blockIdx.x;
  if (b >= B) return;
  const long long n0 = ptr[b], n1 = ptr[b + 1];
  const double* c = cell + 9 * (long long)b;
  // g_k = c_{k+1} x c_{k+2}: the fractional coordinate of x along lattice vector k is (x . g_k) / det
  double g[3][3];
  for (int k = 0; k < 3; ++k) {
    const double* a = c + 3 * ((k + 1) % 3);
    const double* d = c + 3 * ((k + 2) % 3);
    g[k][0] = a[1] * d[2] - a[2] * d[1];
    g[k][1] = a[2] * d[0] - a[0] * d[2];
    g[k][2] = a[0] * d[1] - a[1] * d[0];
  }
  const double det = c[0] * g[0][0] + c[1] * g[0][1] + c[2] * g[0][2];
  const double vol = fabs(det);
  // per thread, over its atoms: minima (red rows 0-5: x, y, z, then the three fractional coordinates), maxima (6-11)
  __shared__ double red[12][256];
  double lo[6], hi[6];
  for (int k = 0; k < 6; ++k) { lo[k] = 1e300; hi[k] = -1e300; }
  for (long long i = n0 + threadIdx.x; i < n1; i += 256) {
    const double x[3] = {pos[3 * i], pos[3 * i + 1], pos[3 * i + 2]};
    for (int k = 0; k < 3; ++k) {
      const double f = (x[0] * g[k][0] + x[1] * g[k][1] + x[2] * g[k][2]) / det;
      lo[k] = fmin(lo[k], x[k]); hi[k] = fmax(hi[k], x[k]);
      lo[3 + k] = fmin(lo[3 + k], f); hi[3 + k] = fmax(hi[3 + k], f);
    }
  }
  const int t = threadIdx.x;
  for (int k = 0; k < 6; ++k) { red[k][t] = lo[k]; red[6 + k][t] = hi[k]; }
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (t < s) {
      for (int k = 0; k < 6; ++k) {
        red[k][t] = fmin(red[k][t], red[k][t + s]);
        red[6 + k][t] = fmax(red[6 + k][t], red[6 + k][t + s]);
      }
    }
    __syncthreads();
  }
  if (t != 0) return;
  const long long n = n1 - n0;
  double blo[3], ext[3];
  for (int k = 0; k < 3; ++k) {
    blo[k] = n > 0 && red[k][0] <= red[6 + k][0] ? red[k][0] : 0.0;
    ext[k] = n > 0 && red[k][0] <= red[6 + k][0] ? red[6 + k][0] - red[k][0] : 0.0;
  }
  // images along periodic k: an edge needs |o_k + f_j,k - f_i,k| < r_max / h_k (h_k = |det| / |g_k|, the spacing of
  // lattice planes k), so |o_k| <= floor(r_max / h_k + span_k), span_k the range of the structure's fractional
  // coordinates along k.  For atoms inside the cell (span_k < 1) that is at most ceil(r_max / h_k), which is used
  // then; atoms further apart (unwrapped coordinates) widen the search.  Beyond 64 translations the search is cut
  // and the structure is flagged (prmi[11]; n_edges -1).
  int reps[3], cut = 0;
  long long nimg = 1;
  for (int k = 0; k < 3; ++k) {
    const double h = vol / sqrt(g[k][0] * g[k][0] + g[k][1] * g[k][1] + g[k][2] * g[k][2]);
    const double span = n > 0 && red[3 + k][0] <= red[9 + k][0] ? red[9 + k][0] - red[3 + k][0] : 0.0;
    double rk = pbc[3 * b + k] ? fmax(ceil(r_max / h), floor(r_max / h + span + 1e-9)) : 0.0;
    if (!(rk >= 0.0)) rk = 0.0;               // a degenerate (zero-volume) cell has no lattice translations
    if (rk > 64.0) { rk = 64.0; cut = 1; }
    reps[k] = (int)rk;
    nimg *= 2 * reps[k] + 1;
  }
  // bins at least r_max + NL_EPS wide, at most n + 1 of them
  const double cw = r_max + NL_EPS;
  long long nb[3];
  for (int k = 0; k < 3; ++k) {
    const double q = floor(ext[k] / cw);
    nb[k] = q >= 1.0 ? (q < 4096.0 ? (long long)q : 4096) : 1;
  }
  while (nb[0] * nb[1] * nb[2] > n + 1) {
    const int k = nb[0] >= nb[1] && nb[0] >= nb[2] ? 0 : (nb[1] >= nb[2] ? 1 : 2);
    nb[k] = nb[k] / 2 > 1 ? nb[k] / 2 : 1;
  }
  double* P = prmd + NL_PD * (long long)b;
  int* I = prmi + NL_PI * (long long)b;
  for (int k = 0; k < 3; ++k) {
    P[k] = blo[k];
    P[3 + k] = fmax(ext[k] / (double)nb[k], cw);
    I[k] = (int)nb[k];
    I[3 + k] = reps[k];
  }
  for (int k = 0; k < 9; ++k) P[6 + k] = c[k];
  const double c2 = sqrt(c[6] * c[6] + c[7] * c[7] + c[8] * c[8]);
  I[6] = (int)n0;
  I[7] = (int)n;
  I[8] = (int)nimg;
  I[9] = (int)(n0 + b);                      // this structure's bins: [n0 + b, n0 + b + n + 1)
  const double kz = ceil((r_max + 1.0) / c2);
  I[10] = kz >= 1.0 && kz < 1e9 ? (int)kz : 0;   // padding shift; 0: none exists (c_2 zero), flagged if needed
  I[11] = cut;                                    // 1: the image search was cut at 64 translations
}

extern "C" __global__ __launch_bounds__(256) void nl_zero(int* __restrict__ a, long long n) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i < n) a[i] = 0;
}

__device__ __forceinline__ int nl_axis_bin(double v, double lo, double bs, int nb) {
  const double t = (v - lo) / bs;
  if (!(t >= 0.0)) return 0;                 // also NaN
  return t < (double)nb ? (int)floor(t) : nb - 1;
}

extern "C" __global__ __launch_bounds__(256) void nl_bins(const double* __restrict__ pos,
    const long long* __restrict__ ptr, int B, int N, const double* __restrict__ prmd, const int* __restrict__ prmi,
    int* __restrict__ abin, int* __restrict__ bcnt) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= N) return;
  const int b = nl_struct_of(ptr, B, i);
  const double* P = prmd + NL_PD * (long long)b;
  const int* I = prmi + NL_PI * (long long)b;
  const int bx = nl_axis_bin(pos[3 * i], P[0], P[3], I[0]);
  const int by = nl_axis_bin(pos[3 * i + 1], P[1], P[4], I[1]);
  const int bz = nl_axis_bin(pos[3 * i + 2], P[2], P[5], I[2]);
  const int bin = I[9] + (bx * I[1] + by) * I[2] + bz;
  abin[i] = bin;
  atomicAdd(&bcnt[bin], 1);
}

extern "C" __global__ __launch_bounds__(1024) void nl_scan(const int* __restrict__ cnt, int* __restrict__ start,
    int* __restrict__ cursor, int n) {
  __shared__ int wsum[16];
  int carry = 0;
  for (long long base = 0; base <= n; base += 1024) {
    const long long i = base + threadIdx.x;
    const int v = i < n ? cnt[i] : 0;
    int total;
    const int ex = mh_block_excl_scan<int, 16>(v, total, wsum);
    if (i <= n) {
      start[i] = carry + ex;
      cursor[i] = carry + ex;
    }
    carry += total;
  }
}

// Each atom into its bin: slot p of the bin order gets (x, y, z, atom index) as four doubles, so a candidate walk
// reads one 32-byte quad per candidate with no dependent index load.
extern "C" __global__ __launch_bounds__(256) void nl_place(const double* __restrict__ pos,
    const int* __restrict__ abin, int* __restrict__ cursor, double* __restrict__ pbin, int N) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= N) return;
  const long long p = atomicAdd(&cursor[abin[i]], 1);
  pbin[4 * p] = pos[3 * i];
  pbin[4 * p + 1] = pos[3 * i + 1];
  pbin[4 * p + 2] = pos[3 * i + 2];
  pbin[4 * p + 3] = (double)i;
}

// Walk sender i's candidates (one wave; every lane returns the same count).  FILL: write the key
// (receiver - n0) * nimg + image of each hit at keys[kpos + k] for k in hit order, where kpos + k < klim.
template <bool FILL>
__device__ long long nl_walk(long long i, int b, const double* __restrict__ pos, const double* __restrict__ prmd,
    const int* __restrict__ prmi, const int* __restrict__ bstart, const double* __restrict__ pbin, double r_max,
    long long* keys, long long kpos, long long klim) {
  const int lane = threadIdx.x & (MH_WAVE - 1);
  const double* P = prmd + NL_PD * (long long)b;
  const int* I = prmi + NL_PI * (long long)b;
  const double cw = r_max + NL_EPS;
  const int nb0 = I[0], nb1 = I[1], nb2 = I[2], r0 = I[3], r1 = I[4], r2 = I[5];
  const long long n0 = I[6];
  const int nimg = I[8], bin0 = I[9];
  const int ny = 2 * r1 + 1, nz = 2 * r2 + 1;
  const int ozero = (r0 * ny + r1) * nz + r2;
  const double pix = pos[3 * i], piy = pos[3 * i + 1], piz = pos[3 * i + 2];
  long long hits = 0;
  for (int o = 0; o < nimg; ++o) {
    const double oi = (double)(o / (ny * nz) - r0), oj = (double)((o / nz) % ny - r1), ok = (double)(o % nz - r2);
    const double sx = (oi * P[6] + oj * P[9]) + ok * P[12];
    const double sy = (oi * P[7] + oj * P[10]) + ok * P[13];
    const double sz = (oi * P[8] + oj * P[11]) + ok * P[14];
    const double q[3] = {pix - sx, piy - sy, piz - sz};
    int blo[3], bhi[3];
    const int nbk[3] = {nb0, nb1, nb2};
    bool empty = false;
    for (int k = 0; k < 3; ++k) {
      const double t0 = (q[k] - cw - P[k]) / P[3 + k], t1 = (q[k] + cw - P[k]) / P[3 + k];
      if (!(t1 >= 0.0) || !(t0 < (double)nbk[k])) { empty = true; break; }   // also NaN
      blo[k] = t0 < 0.0 ? 0 : (int)floor(t0);
      bhi[k] = t1 >= (double)nbk[k] ? nbk[k] - 1 : (int)floor(t1);
    }
    if (empty) continue;
    for (int bx = blo[0]; bx <= bhi[0]; ++bx) {
      for (int by = blo[1]; by <= bhi[1]; ++by) {
        const int col = bin0 + (bx * nb1 + by) * nb2;
        const int t_first = bstart[col + blo[2]], t_last = bstart[col + bhi[2] + 1];
        for (int tb = t_first; tb < t_last; tb += MH_WAVE) {
          const int t = tb + lane;
          bool hit = false;
          int j = 0;
          if (t < t_last) {
            const double2 a = reinterpret_cast<const double2*>(pbin)[2 * (long long)t];
            const double2 c = reinterpret_cast<const double2*>(pbin)[2 * (long long)t + 1];
            j = (int)c.y;
            const double dx = (a.x + sx) - pix;
            const double dy = (a.y + sy) - piy;
            const double dz = (c.x + sz) - piz;
            const double d2 = (dx * dx + dy * dy) + dz * dz;
            hit = sqrt(d2) < r_max && !(j == i && o == ozero);
          }
          const unsigned long long m = __ballot(hit);
          if (FILL && hit) {
            const long long kq = kpos + hits + __popcll(m & ((1ull << lane) - 1ull));
            if (kq < klim) keys[kq] = ((long long)j - n0) * nimg + o;
          }
          hits += __popcll(m);
        }
      }
    }
  }
  return hits;
}

extern "C" __global__ __launch_bounds__(MH_WAVE * NL_SPB) void nl_count(const double* __restrict__ pos,
    const long long* __restrict__ ptr, int B, int N, const double* __restrict__ prmd, const int* __restrict__ prmi,
    const int* __restrict__ bstart, const double* __restrict__ pbin, double r_max, long long* __restrict__ cnt) {
  const long long i = (long long)blockIdx.x * NL_SPB + (threadIdx.x >> 6);
  if (i >= N) return;                        // whole waves
  const int b = nl_struct_of(ptr, B, i);
  const long long h = nl_walk<false>(i, b, pos, prmd, prmi, bstart, pbin, r_max, nullptr, 0, 0);
  if ((threadIdx.x & (MH_WAVE - 1)) == 0) cnt[i] = h;
}

// One workgroup per structure b: its edge count n_edges[b] (its real edges, even past e_pad) and each sender's
// segment start relative to the structure's first slot: the exclusive prefix of (hits + padding share) over the
// structure's senders.  A structure that needs padding but cannot have any (no atoms, or a zero third lattice vector),
// or whose image search was cut (more than 64 translations along a lattice direction), gets n_edges[b] = -1; an
// atomless one's slots are filled with zero-length self-loops of a neighbouring atom (their length makes the model's
// result NaN, never an index fault).
extern "C" __global__ __launch_bounds__(1024) void nl_offsets(const long long* __restrict__ ptr, int B, int N,
    const int* __restrict__ prmi, const long long* __restrict__ cnt, long long e_pad, long long e_total,
    long long* __restrict__ start, long long* __restrict__ tot, int* __restrict__ n_edges,
    long long* __restrict__ edge_index, void* __restrict__ ushift, void* __restrict__ shift, int f64) {
  __shared__ long long wsum[16];
  const int t = threadIdx.x, b = blockIdx.x;
  if (b >= B) return;
  const long long n0 = ptr[b], n1 = ptr[b + 1], n = n1 - n0;
  long long part = 0;
  for (long long i = n0 + t; i < n1; i += 1024) part += cnt[i];
  long long total;
  mh_block_excl_scan<long long, 16>(part, total, wsum);
  const long long extra = e_pad > 0 && total < e_pad ? e_pad - total : 0;
  const bool unpaddable = extra > 0 && (n == 0 || prmi[NL_PI * (long long)b + 10] == 0);
  const bool cut = prmi[NL_PI * (long long)b + 11] != 0;
  if (t == 0) {
    tot[b] = total;
    n_edges[b] = unpaddable || cut ? -1 : (total < 0x7fffffffLL ? (int)total : 0x7fffffff);
  }
  if (n == 0 && extra > 0 && edge_index && N > 0) {
    const long long a = n0 < N ? n0 : N - 1;
    for (long long p = t; p < e_pad; p += 1024) {
      const long long e = (long long)b * e_pad + p;
      edge_index[e] = a;
      edge_index[e_total + e] = a;
      for (int k = 0; k < 3; ++k) {
        if (f64) { ((double*)ushift)[3 * e + k] = 0.0; ((double*)shift)[3 * e + k] = 0.0; }
        else { ((float*)ushift)[3 * e + k] = 0.0f; ((float*)shift)[3 * e + k] = 0.0f; }
      }
    }
  }
  long long carry = 0;
  for (long long base = n0; base < n1; base += 1024) {
    const long long i = base + t;
    long long v = 0;
    if (i < n1) {
      const long long il = i - n0;
      v = cnt[i] + (extra > 0 ? extra / n + (il < extra % n ? 1 : 0) : 0);
    }
    long long chunk;
    const long long ex = mh_block_excl_scan<long long, 16>(v, chunk, wsum);
    if (i < n1) start[i] = carry + ex;
    carry += chunk;
  }
}

// The first slot of each structure: b * e_pad (padded layout) or the running total of the edge counts of the
// structures before b (exact layout), one workgroup.
extern "C" __global__ __launch_bounds__(1024) void nl_bases(const long long* __restrict__ tot, int B, long long e_pad,
    long long* __restrict__ sbase) {
  __shared__ long long wsum[16];
  long long carry = 0;
  for (long long b0 = 0; b0 < B; b0 += 1024) {
    const long long b = b0 + threadIdx.x;
    const long long v = b < B ? tot[b] : 0;
    long long chunk;
    const long long ex = mh_block_excl_scan<long long, 16>(v, chunk, wsum);
    if (b < B) sbase[b] = e_pad > 0 ? b * e_pad : carry + ex;
    carry += chunk;
  }
}

extern "C" __global__ __launch_bounds__(MH_WAVE * NL_SPB) void nl_fill(const double* __restrict__ pos,
    const long long* __restrict__ ptr, int B, int N, const double* __restrict__ prmd, const int* __restrict__ prmi,
    const int* __restrict__ bstart, const double* __restrict__ pbin, double r_max, const long long* __restrict__ cnt,
    const long long* __restrict__ start, const long long* __restrict__ tot, const long long* __restrict__ sbase,
    long long e_pad, long long e_total, long long* __restrict__ keys, long long* __restrict__ edge_index,
    void* __restrict__ ushift,
    void* __restrict__ shift, int f64) {
  const long long i = (long long)blockIdx.x * NL_SPB + (threadIdx.x >> 6);
  if (i >= N) return;                        // whole waves
  const int lane = threadIdx.x & (MH_WAVE - 1);
  const int b = nl_struct_of(ptr, B, i);
  const long long kpos = sbase[b] + start[i];
  const long long klim = e_pad > 0 ? (long long)b * e_pad + e_pad : e_total;
  const long long h = cnt[i];
  const long long L = kpos >= klim ? 0 : (h < klim - kpos ? h : klim - kpos);
  // the walk writes the keys of a segment of up to NL_LDS_KEYS edges into this wave's LDS region (h is known from
  // the count pass), a longer segment's into global memory; the ranking below reads them back from there
  __shared__ long long skeys[NL_SPB][NL_LDS_KEYS];
  const bool in_lds = L <= NL_LDS_KEYS;
  long long* sk = skeys[threadIdx.x >> 6];
  if (in_lds) {
    nl_walk<true>(i, b, pos, prmd, prmi, bstart, pbin, r_max, sk, 0, L);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
  } else {
    nl_walk<true>(i, b, pos, prmd, prmi, bstart, pbin, r_max, keys, kpos, klim);
    __threadfence();                         // this wave's key stores before its loads below
  }
  const long long* kk = in_lds ? sk : keys + kpos;
  const double* P = prmd + NL_PD * (long long)b;
  const int* I = prmi + NL_PI * (long long)b;
  const long long n0 = I[6], n = I[7];
  const int nimg = I[8], r0 = I[3], r1 = I[4], r2 = I[5], kz = I[10];
  const int ny = 2 * r1 + 1, nz = 2 * r2 + 1;
  for (long long p = lane; p < L; p += MH_WAVE) {
    const long long kp = kk[p];
    long long rank = 0;
    for (long long q = 0; q < L; ++q) rank += kk[q] < kp;
    const long long e = kpos + rank;
    const int o = (int)(kp % nimg);
    const double oi = (double)(o / (ny * nz) - r0), oj = (double)((o / nz) % ny - r1), ok = (double)(o % nz - r2);
    edge_index[e] = i;
    edge_index[e_total + e] = n0 + kp / nimg;
    const double u[3] = {oi, oj, ok};
    const double sv[3] = {(oi * P[6] + oj * P[9]) + ok * P[12], (oi * P[7] + oj * P[10]) + ok * P[13],
                          (oi * P[8] + oj * P[11]) + ok * P[14]};
    for (int k = 0; k < 3; ++k) {
      if (f64) { ((double*)ushift)[3 * e + k] = u[k]; ((double*)shift)[3 * e + k] = sv[k]; }
      else { ((float*)ushift)[3 * e + k] = (float)u[k]; ((float*)shift)[3 * e + k] = (float)sv[k]; }
    }
  }
  if (e_pad <= 0 || n <= 0) return;
  const long long total = tot[b];
  if (total >= e_pad) return;
  const long long extra = e_pad - total, il = i - n0;
  const long long np = extra / n + (il < extra % n ? 1 : 0);
  const double sv[3] = {(double)kz * P[12], (double)kz * P[13], (double)kz * P[14]};
  for (long long p = lane; p < np; p += MH_WAVE) {
    const long long e = kpos + h + p;         // < b * e_pad + e_pad: the shares add up to the padding exactly
    edge_index[e] = i;
    edge_index[e_total + e] = i;
    const double u[3] = {0.0, 0.0, (double)kz};
    for (int k = 0; k < 3; ++k) {
      if (f64) { ((double*)ushift)[3 * e + k] = u[k]; ((double*)shift)[3 * e + k] = sv[k]; }
      else { ((float*)ushift)[3 * e + k] = (float)u[k]; ((float*)shift)[3 * e + k] = (float)sv[k]; }
    }
  }
}
"""


_MODULES = {}              # device index -> module of the neighbour-list kernels


def _module(device):
    idx = device.index if device.index is not None else torch.cuda.current_device()
    m = _MODULES.get(idx)
    if m is None:
        code = _native.compile_source(source())
        with torch.cuda.device(idx):
            m = _native.Module(code, {_native.MH_NL_SETUP: ('nl_setup', 256, 1),
                                      _native.MH_NL_BASES: ('nl_bases', 1024, 1),
                                      _native.MH_NL_ZERO: ('nl_zero', 256, 256),
                                      _native.MH_NL_BINS: ('nl_bins', 256, 256),
                                      _native.MH_NL_SCAN: ('nl_scan', 1024, 1),
                                      _native.MH_NL_PLACE: ('nl_place', 256, 256),
                                      _native.MH_NL_COUNT: ('nl_count', WAVE * SENDERS_PER_BLOCK, SENDERS_PER_BLOCK),
                                      _native.MH_NL_OFFSETS: ('nl_offsets', 1024, 1),  # one workgroup per structure
                                      _native.MH_NL_FILL: ('nl_fill', WAVE * SENDERS_PER_BLOCK, SENDERS_PER_BLOCK)})
        _MODULES[idx] = m
    return m


# Edge lists this module built (weak references with the tensor version at build time): their indices lie in
# [0, N) by construction, so the convolution's graph build need not check them.
_built = []


def built_here(edge_index, n):
    """Whether ``edge_index`` is an unmodified output of ``neighbour_list`` over ``n`` atoms."""
    for ref, ver, nn in _built:
        if ref() is edge_index and ver == edge_index._version and nn == n:
            return True
    return False


def _register(edge_index, n):
    _built[:] = [r for r in _built if r[0]() is not None][-15:]
    _built.append((weakref.ref(edge_index), edge_index._version, n))


class NeighbourList:
    """Result of ``neighbour_list``: ``edge_index`` [2, E] int64 (sender, receiver), ``shifts`` [E, 3] (unit_shifts @
    cell), ``unit_shifts`` [E, 3], ``n_edges`` [B] int32 on the device (real edges per structure, also past the
    padding), ``pad_edges_to`` (None: exact layout)."""

    def __init__(self, edge_index, shifts, unit_shifts, n_edges, pad_edges_to):
        self.edge_index, self.shifts, self.unit_shifts = edge_index, shifts, unit_shifts
        self.n_edges, self.pad_edges_to = n_edges, pad_edges_to

    def overflowed(self):
        """Structures whose graph is incomplete (synchronises): more real edges than ``pad_edges_to``, or n_edges -1:
        padding needed where none can be placed (no atoms, or a zero third lattice vector), or an image search cut
        at 64 lattice translations (atoms spread over about that many cells)."""
        return incomplete(self.n_edges.cpu(), self.pad_edges_to)

    def check(self):
        raise_incomplete(self.n_edges.cpu(), self.pad_edges_to)
        return self


def incomplete(counts, pad_edges_to):
    """Indices of the structures whose host-side edge ``counts`` (``NeighbourList.n_edges`` copied to the host) show
    an incomplete graph: -1, or more real edges than ``pad_edges_to``."""
    bad = counts < 0
    if pad_edges_to is not None:
        bad = bad | (counts > pad_edges_to)
    return torch.nonzero(bad).reshape(-1).tolist()


def raise_incomplete(counts, pad_edges_to):
    """ValueError naming the incomplete structures of ``counts`` (see ``incomplete``), if any."""
    bad = incomplete(counts, pad_edges_to)
    if bad:
        raise ValueError(f'neighbour list: structures {bad} do not fit pad_edges_to={pad_edges_to} or are incomplete '
                         f'(real edges {counts[bad].tolist()}; -1: no atoms or no third lattice vector to '
                         f'shift padding along, or atoms spread over more than 64 cells); rebuild with a larger '
                         f'padding or wrapped positions')


def _work_bytes(B, N, e_total):
    return int(_native.load().mh_neighbour_list_work_size(B, N, e_total))


def neighbour_list(positions, cell, ptr, r_max, pbc=(True, True, True), pad_edges_to=None, dtype=None):
    """Neighbour list of the structures ``ptr`` delimits (positions [N, 3], cell [B, 3, 3] or MACE's stacked
    [3 B, 3], ptr [B + 1] int64) on the GPU.  ``pbc``: three booleans for every structure, or a [B, 3] tensor.
    ``pad_edges_to``: edges per structure in the fixed-size layout (no host synchronisation); None: exactly the real
    edges (one synchronisation to size the output).  ``dtype`` of the shifts: the positions' (float32 or float64)
    by default.  The geometry is evaluated in float64 either way."""
    if not positions.is_cuda:
        raise RuntimeError('mace_hip_kernels: neighbour_list needs GPU tensors')
    dev = positions.device
    N = positions.shape[0]
    if positions.dim() != 2 or positions.shape[1] != 3:
        raise ValueError(f'positions must be [N, 3], got {tuple(positions.shape)}')
    B = ptr.numel() - 1
    if B < 1:
        raise ValueError('ptr must hold at least one structure')
    cell = cell.reshape(B, 3, 3)
    if not (r_max > 0 and r_max < float('inf')):
        raise ValueError(f'r_max must be positive and finite, got {r_max}')
    if N >= 2 ** 31 - B - 1:
        raise ValueError('too many atoms for int32 bins')
    dtype = dtype or (positions.dtype if positions.dtype in (torch.float32, torch.float64) else torch.float32)
    pos = positions.detach().to(torch.float64).contiguous()
    cl = cell.detach().to(dev, torch.float64).contiguous()
    if torch.is_tensor(pbc):
        pb = pbc.to(dev, torch.int32).reshape(B, 3).contiguous()
    else:
        pb = torch.tensor([[int(bool(v)) for v in pbc]] * B, dtype=torch.int32, device=dev)
    pt = ptr.to(dev, torch.int64).contiguous()
    n_edges = torch.empty(B, dtype=torch.int32, device=dev)
    m, lib, P = _module(dev), _native.load(), _native.ptr
    st = _native.stream_of(pos)
    f64 = int(dtype == torch.float64)
    if pad_edges_to is None:
        work = torch.empty(_work_bytes(B, N, 0), dtype=torch.uint8, device=dev)
        _native.launch('neighbour_list', lib.mh_neighbour_list, m.handle, P(pos), P(cl), P(pb), P(pt), B, N,
                       float(r_max), 0, 0, None, None, None, f64, P(n_edges), P(work), st)
        counts = n_edges.cpu()                                               # the one synchronisation
        if bool((counts < 0).any()):
            raise ValueError(f'neighbour list: structures {torch.nonzero(counts < 0).reshape(-1).tolist()} need more '
                             f'than 64 lattice translations along a periodic direction (atoms spread over that many '
                             f'cells); wrap the positions into the cell')
        e_total = int(counts.to(torch.int64).sum())
        e_pad = 0
    else:
        e_pad = int(pad_edges_to)
        if e_pad < 1:
            raise ValueError('pad_edges_to must be positive')
        e_total = B * e_pad
    edge_index = torch.empty(2, e_total, dtype=torch.int64, device=dev)
    ush = torch.empty(e_total, 3, dtype=dtype, device=dev)
    sh = torch.empty(e_total, 3, dtype=dtype, device=dev)
    work = torch.empty(_work_bytes(B, N, e_total), dtype=torch.uint8, device=dev)
    _native.launch('neighbour_list', lib.mh_neighbour_list, m.handle, P(pos), P(cl), P(pb), P(pt), B, N,
                   float(r_max), e_pad, e_total, P(edge_index), P(ush), P(sh), f64, P(n_edges), P(work), st)
    _register(edge_index, N)
    return NeighbourList(edge_index, sh, ush, n_edges, pad_edges_to)


def update_batch(batch, r_max, pbc=(True, True, True), pad_edges_to=None):
    """Rebuild a MACE batch dict's graph (edge_index, shifts, unit_shifts) on the GPU from its positions, cell and
    ptr, in place; returns the ``NeighbourList``."""
    nl = neighbour_list(batch['positions'], batch['cell'], batch['ptr'], r_max, pbc=pbc, pad_edges_to=pad_edges_to,
                        dtype=batch['positions'].dtype)
    batch['edge_index'], batch['shifts'], batch['unit_shifts'] = nl.edge_index, nl.shifts, nl.unit_shifts
    return nl

"""
Edge geometry of MACE on MI355X: vectors[e] = positions[receiver[e]] - positions[sender[e]] + shifts[e] and
lengths[e] = |vectors[e]| (MACE's ``get_edge_vectors_and_lengths``), with the backward that forces and stress run
through: dL/dpositions[n] = sum over edges into n of dL/dv - sum over edges out of n of dL/dv, where
dL/dv = g_vectors + g_lengths v / |v|, and dL/dshifts = dL/dv.

In PyTorch the backward of the two row gathers is an index_put with accumulation per gather (a sort of the edge
list and a segmented sum each call).  Here the forward is one thread per edge, and the backward one wave per atom
summing dL/dv over the receiver-sorted and sender-sorted edge lists (CSRs) that the convolution already keeps for
the same edge_index: deterministic, no atomics, no sort.

With stress or virials, MACE first strains each structure (``get_symmetric_displacement``): positions + positions
@ sym[batch] and shifts = unit_shifts @ cell[batch[sender]].  The backward of those two per-structure gathers is, in
PyTorch, an index_put with accumulation whose runs of equal indices are summed serially: on one structure every
atom and edge carries the same index and the two take ~1.9 ms of a 2.6 ms E+F+stress call.  Here the gathers stay
and their backward is a segmented sum per structure (``geom_segsum``; atoms by the batch's ptr, edges by the sender
CSR), one workgroup per structure in a fixed order.

MACE's per-structure energy sums (``scatter_sum`` of the node energies by the batch vector) are an index_add with
float atomics in PyTorch (~9 us each on config 2's 16 structures, and the summation order varies from run to run);
here they are a segmented sum over the batch's ptr (``geom_segsum1``), deterministic, taken when the index is the
batch vector of the running forward itself.

These computations are module-level functions of MACE, not modules, so ``patch_model`` routes them here through the
model's own module namespace: the functions there are wrapped once, and the wrappers only take this path while a
patched model's forward is running (a context variable set by that model's forward, which also carries the batch's
batch vector and ptr); every other caller, unpatched models included, keeps the original functions.
"""
import contextvars
import functools
import inspect
import sys
import types

import torch

from . import _native
from . import conv as _conv

BLOCK = 256
_ACTIVE = contextvars.ContextVar('mace_hip_kernels_geometry', default=False)
_PTR = contextvars.ContextVar('mace_hip_kernels_geometry_ptr', default=None)   # the batch's ptr during a forward
_BATCH = contextvars.ContextVar('mace_hip_kernels_geometry_batch', default=None)  # the batch vector, likewise
# (harmonics, embedding) drop-ins of the running forward whose outputs the geometry's forward makes too (edgefeat)
_EDGE = contextvars.ContextVar('mace_hip_kernels_geometry_edge', default=None)
FUNCTION = 'get_edge_vectors_and_lengths'
DISPLACEMENT = 'get_symmetric_displacement'
SCATTER = 'scatter_sum'

_SOURCE = r'''
#define BLOCK 256
extern "C" __global__ __launch_bounds__(BLOCK) void geom_fwd(const float* __restrict__ pos,
    const int* __restrict__ send, const int* __restrict__ recv, const float* __restrict__ shifts,
    float* __restrict__ vec, float* __restrict__ len, long long E) {
  const long long e = (long long)mh_xcd_block(blockIdx.x, gridDim.x) * BLOCK + threadIdx.x;
  if (e >= E) return;
  const long long s = send[e], r = recv[e];
  const float vx = (pos[3 * r] - pos[3 * s]) + shifts[3 * e];
  const float vy = (pos[3 * r + 1] - pos[3 * s + 1]) + shifts[3 * e + 1];
  const float vz = (pos[3 * r + 2] - pos[3 * s + 2]) + shifts[3 * e + 2];
  vec[3 * e] = vx; vec[3 * e + 1] = vy; vec[3 * e + 2] = vz;
  len[e] = sqrtf(vx * vx + vy * vy + vz * vz);
}

// dL/dv of edge e: g_vec + g_len * v / |v| (the norm's gradient is 0 at |v| = 0, as PyTorch's)
__device__ __forceinline__ void geom_gv(const float* __restrict__ vec, const float* __restrict__ len,
    const float* __restrict__ gvec, const float* __restrict__ glen, int e, float& gx, float& gy, float& gz) {
  gx = gvec ? gvec[3 * e] : 0.f;
  gy = gvec ? gvec[3 * e + 1] : 0.f;
  gz = gvec ? gvec[3 * e + 2] : 0.f;
  if (glen) {
    const float l = len[e];
    const float c = l != 0.f ? glen[e] / l : 0.f;
    gx += c * vec[3 * e]; gy += c * vec[3 * e + 1]; gz += c * vec[3 * e + 2];
  }
}

__device__ __forceinline__ float geom_wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// one wave per atom: the edges into it (receiver CSR) minus the edges out of it (sender CSR)
extern "C" __global__ __launch_bounds__(BLOCK) void geom_bwd(const float* __restrict__ vec,
    const float* __restrict__ len, const float* __restrict__ gvec, const float* __restrict__ glen,
    const int* __restrict__ rowptr_r, const int* __restrict__ eids_r, const int* __restrict__ rowptr_s,
    const int* __restrict__ eids_s, float* __restrict__ gpos, float* __restrict__ gshifts, int N) {
  const int n = mh_xcd_block(blockIdx.x, gridDim.x) * (BLOCK / 64) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (n >= N) return;
  float sx = 0.f, sy = 0.f, sz = 0.f;
  for (int k = rowptr_r[n] + lane; k < rowptr_r[n + 1]; k += 64) {
    const int e = eids_r[k];
    float gx, gy, gz;
    geom_gv(vec, len, gvec, glen, e, gx, gy, gz);
    sx += gx; sy += gy; sz += gz;
    if (gshifts) { gshifts[3 * e] = gx; gshifts[3 * e + 1] = gy; gshifts[3 * e + 2] = gz; }
  }
  for (int k = rowptr_s[n] + lane; k < rowptr_s[n + 1]; k += 64) {
    float gx, gy, gz;
    geom_gv(vec, len, gvec, glen, eids_s[k], gx, gy, gz);
    sx -= gx; sy -= gy; sz -= gz;
  }
  sx = geom_wave_sum(sx); sy = geom_wave_sum(sy); sz = geom_wave_sum(sz);
  if (lane == 0) { gpos[3 * n] = sx; gpos[3 * n + 1] = sy; gpos[3 * n + 2] = sz; }
}

// Second derivatives behind a double backward.  With d = ggpos[r] - ggpos[s] + ggshifts[e] the direction that the
// incoming gradients give edge e's vector and u = v / |v|: d/dg_vec = d, d/dg_len = u.d, and the part that goes
// back through v (and from there to the atoms, through geom_bwd) h = g_len (d - u (u.d)) / |v| (0 at |v| = 0).
extern "C" __global__ __launch_bounds__(BLOCK) void geom_jvp(const float* __restrict__ vec,
    const float* __restrict__ len, const float* __restrict__ ggpos, const float* __restrict__ ggshifts,
    const int* __restrict__ send, const int* __restrict__ recv, const float* __restrict__ glen,
    float* __restrict__ dgvec, float* __restrict__ dglen, float* __restrict__ h, long long E) {
  const long long e = (long long)mh_xcd_block(blockIdx.x, gridDim.x) * BLOCK + threadIdx.x;
  if (e >= E) return;
  float dx = 0.f, dy = 0.f, dz = 0.f;
  if (ggpos) {
    const long long s = send[e], r = recv[e];
    dx = ggpos[3 * r] - ggpos[3 * s]; dy = ggpos[3 * r + 1] - ggpos[3 * s + 1]; dz = ggpos[3 * r + 2] - ggpos[3 * s + 2];
  }
  if (ggshifts) { dx += ggshifts[3 * e]; dy += ggshifts[3 * e + 1]; dz += ggshifts[3 * e + 2]; }
  dgvec[3 * e] = dx; dgvec[3 * e + 1] = dy; dgvec[3 * e + 2] = dz;
  const float l = len[e];
  const float il = l != 0.f ? 1.f / l : 0.f;
  const float ux = vec[3 * e] * il, uy = vec[3 * e + 1] * il, uz = vec[3 * e + 2] * il;
  const float ud = ux * dx + uy * dy + uz * dz;
  dglen[e] = ud;
  const float c = glen ? glen[e] * il : 0.f;
  h[3 * e] = c * (dx - ux * ud); h[3 * e + 1] = c * (dy - uy * ud); h[3 * e + 2] = c * (dz - uz * ud);
}

// Segmented sums of K-wide rows (the backward of gathering a per-structure table by structure index): out[b, k] =
// sum over the rows of segment b (rows perm[seg[b]] .. perm[seg[b + 1] - 1], or seg[b] .. seg[b + 1] - 1 without
// perm) of g[row, k].  One workgroup per segment; every thread sums a fixed stride of rows, then a fixed-order tree
// over the workgroup: deterministic, no atomics.
#define SEG_K 9
extern "C" __global__ __launch_bounds__(BLOCK) void geom_segsum(const float* __restrict__ g,
    const int* __restrict__ perm, const long long* __restrict__ seg, float* __restrict__ out, int B) {
  const int b = blockIdx.x;
  if (b >= B) return;
  const long long lo = seg[b], hi = seg[b + 1];
  float acc[SEG_K];
  for (int k = 0; k < SEG_K; ++k) acc[k] = 0.f;
  for (long long r = lo + threadIdx.x; r < hi; r += BLOCK) {
    const long long row = perm ? (long long)perm[r] : r;
    for (int k = 0; k < SEG_K; ++k) acc[k] += g[row * SEG_K + k];
  }
  __shared__ float red[SEG_K][BLOCK];
  for (int k = 0; k < SEG_K; ++k) red[k][threadIdx.x] = acc[k];
  __syncthreads();
  for (int w = BLOCK / 2; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w)
      for (int k = 0; k < SEG_K; ++k) red[k][threadIdx.x] += red[k][threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x < SEG_K) out[(long long)b * SEG_K + threadIdx.x] = red[threadIdx.x][0];
}

// The same for one column (MACE's per-structure energy sums): out[b] = sum of g[seg[b]] .. g[seg[b + 1] - 1].
extern "C" __global__ __launch_bounds__(BLOCK) void geom_segsum1(const float* __restrict__ g,
    const long long* __restrict__ seg, float* __restrict__ out, int B) {
  const int b = blockIdx.x;
  if (b >= B) return;
  const long long lo = seg[b], hi = seg[b + 1];
  float acc = 0.f;
  for (long long r = lo + threadIdx.x; r < hi; r += BLOCK) acc += g[r];
  __shared__ float red[BLOCK];
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int w = BLOCK / 2; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[b] = red[0];
}
'''

_modules = {}


def _module(device):
    """The geometry kernels, loaded once per device."""
    key = torch.device(device).index
    if key not in _modules:
        code = _native.compile_source(_native.device_header() + _SOURCE)
        with torch.cuda.device(device):
            _modules[key] = _native.Module(code, {_native.MH_GEOM_FWD: ('geom_fwd', BLOCK, BLOCK),
                                                  _native.MH_GEOM_BWD: ('geom_bwd', BLOCK, BLOCK // 64),
                                                  _native.MH_GEOM_JVP: ('geom_jvp', BLOCK, BLOCK),
                                                  _native.MH_GEOM_SEGSUM: ('geom_segsum', BLOCK, 1),
                                                  _native.MH_GEOM_SEGSUM1: ('geom_segsum1', BLOCK, 1)})
    return _modules[key]


def source():
    return _native.device_header() + _SOURCE


_DOUBLE_BACKWARD = ('mace_hip_kernels: double backward (create_graph=True, e.g. training on forces/stress or an '
                    'autograd Hessian) is not enabled for the edge geometry; patch with '
                    'patch_model(model, double_backward=True)')


def _geom_bwd(vec, ln, gv, gl, gr, N, want_shifts):
    rp_r, ei_r = gr.by_recv()
    rp_s, ei_s = gr.by_send()
    gpos = torch.empty(N, 3, device=vec.device, dtype=torch.float32)
    gsh = torch.empty_like(vec) if want_shifts else None
    gv = None if gv is None else gv.contiguous()
    gl = None if gl is None else gl.contiguous()
    mod = _module(vec.device)
    _native.launch('geom_bwd', _native.load().mh_geom_bwd, mod.handle, _native.ptr(vec), _native.ptr(ln),
                   _native.ptr(gv), _native.ptr(gl), _native.ptr(rp_r), _native.ptr(ei_r), _native.ptr(rp_s),
                   _native.ptr(ei_s), _native.ptr(gpos), _native.ptr(gsh), N, _native.stream_of(vec))
    return gpos, gsh


class _GeomFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, positions, shifts, edge_index, double_backward=False, edge_ops=None):
        N, E = positions.shape[0], edge_index.shape[1]
        gr = _conv.graph_for(edge_index, N)
        p = positions.contiguous()
        sh = shifts.contiguous()
        vec = torch.empty(E, 3, device=p.device, dtype=torch.float32)
        ln = torch.empty(E, 1, device=p.device, dtype=torch.float32)
        if edge_ops is not None:
            # the harmonics and the embedding of the same edges in the same pass, left on vec for those modules
            from . import edgefeat
            edgefeat.forward_all(p, gr, sh, vec, ln, edge_ops)
        else:
            mod = _module(p.device)
            _native.launch('geom_fwd', _native.load().mh_geom_fwd, mod.handle, _native.ptr(p), _native.ptr(gr.send),
                           _native.ptr(gr.recv), _native.ptr(sh), _native.ptr(vec), _native.ptr(ln), E,
                           _native.stream_of(p))
        ctx.save_for_backward(positions, shifts, vec, ln)
        ctx.gr, ctx.N, ctx.double_backward = gr, N, double_backward
        return vec, ln

    @staticmethod
    def backward(ctx, gv, gl):
        positions, shifts, vec, ln = ctx.saved_tensors
        if torch.is_grad_enabled():          # only true under create_graph=True
            if not ctx.double_backward:
                raise RuntimeError(_DOUBLE_BACKWARD)
            gpos, gsh = _GeomAdjFn.apply(gv, gl, positions, shifts, vec.detach(), ln.detach(), ctx.gr, ctx.N,
                                         ctx.needs_input_grad[1])
        else:
            gpos, gsh = _geom_bwd(vec, ln, gv, gl, ctx.gr, ctx.N, ctx.needs_input_grad[1])
        return (gpos if ctx.needs_input_grad[0] else None), gsh, None, None, None


class _GeomAdjFn(torch.autograd.Function):
    """(dL/dpositions, dL/dshifts) as a function of (g_vec, g_len, positions, shifts), for a double backward (see
    ``geom_jvp``): the incoming gradients become a direction d per edge; d/dg_vec = d, d/dg_len = u.d, and the
    curvature of |v| gives h per edge, summed onto the atoms (and the shifts) by the first-order kernel.  Third
    derivatives are not provided."""

    @staticmethod
    def forward(ctx, gv, gl, positions, shifts, vec, ln, gr, N, want_shifts):
        ctx.save_for_backward(gl, vec, ln)
        ctx.gr, ctx.N = gr, N
        return _geom_bwd(vec, ln, gv, gl, gr, N, want_shifts)

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, ggpos, ggsh):
        gl, vec, ln = ctx.saved_tensors
        gr, N, E = ctx.gr, ctx.N, vec.shape[0]
        P = _native.ptr
        ggpos = None if ggpos is None else ggpos.contiguous()
        ggsh = None if ggsh is None else ggsh.contiguous()
        glc = None if gl is None else gl.contiguous()
        dgv = torch.empty(E, 3, device=vec.device, dtype=torch.float32)
        dgl = torch.empty(E, 1, device=vec.device, dtype=torch.float32)
        h = torch.empty(E, 3, device=vec.device, dtype=torch.float32)
        _native.launch('geom_jvp', _native.load().mh_geom_jvp, _module(vec.device).handle, P(vec), P(ln), P(ggpos),
                       P(ggsh), P(gr.send), P(gr.recv), P(glc), P(dgv), P(dgl), P(h), E, _native.stream_of(vec))
        need = ctx.needs_input_grad
        gpos = gsh = None
        if need[2] or need[3]:
            gpos, gsh = _geom_bwd(vec, ln, h, None, gr, N, need[3])
        return (dgv if need[0] else None, dgl if need[1] else None, gpos if need[2] else None, gsh,
                None, None, None, None, None)


def edge_vectors_and_lengths(positions, edge_index, shifts):
    """(vectors [E, 3], lengths [E, 1]) on the GPU kernels, differentiable in positions and shifts."""
    if positions.dtype != torch.float32 or shifts.dtype != torch.float32 or not positions.is_cuda:
        raise TypeError('mace_hip_kernels: edge geometry expects float32 GPU positions and shifts')
    if positions.shape[-1] != 3 or shifts.shape != (edge_index.shape[1], 3):
        raise ValueError(f'positions [N, 3] and shifts [E, 3] expected, got {tuple(positions.shape)}, '
                         f'{tuple(shifts.shape)}')
    vec, ln = _GeomFn.apply(positions, shifts, edge_index, _ACTIVE.get() == 'double_backward', _EDGE.get())
    if not shifts.requires_grad:
        # The lengths' one differentiable input is then the positions, through pos[recv] - pos[send] + shift: an edge
        # and its exact reverse (negated vector) have equal lengths whose gradients reach the two end atoms along the
        # same axis with opposite signs, so only the sum of the pair's length gradients reaches the positions.  A
        # patched radial embedding passes this on to its features (lengths_pair_symmetric).
        ln._mh_vec = (ln._version, vec, vec._version)
    return vec, ln


def lengths_pair_symmetric(t):
    """The edge vectors behind ``t`` (edge lengths from ``edge_vectors_and_lengths``, or a patched radial
    embedding's features of them) when only the sum of an edge's and its exact reverse's gradients in ``t`` reaches
    any input (the shifts need no gradient), and ``t`` and the vectors are unmodified since; else None."""
    from .pending import stash_owner
    m = getattr(stash_owner(t), '_mh_vec', None)
    if m is None or m[0] != t._version or m[1]._version != m[2]:
        return None
    return m[1]


def _segsum(g, perm, seg, B):
    """[B, 3, 3] per-segment sums of g [M, 3, 3] (rows of segment b: perm[seg[b]:seg[b + 1]], or seg[b]:seg[b + 1])."""
    out = torch.empty(B, 3, 3, device=g.device, dtype=torch.float32)
    gc = g.reshape(-1, 9).contiguous()
    _native.launch('geom_segsum', _native.load().mh_geom_segsum, _module(g.device).handle, _native.ptr(gc),
                   _native.ptr(perm), _native.ptr(seg), _native.ptr(out), B, _native.stream_of(gc))
    return out


class _GraphGather(torch.autograd.Function):
    """table[index] for a per-structure table [B, 3, 3] and the structure index of each row, with the backward a
    segmented sum over each structure's rows (``geom_segsum``; segments perm[seg[b]:seg[b + 1]]) instead of
    PyTorch's index_put with accumulation, which sorts the index and sums each run of equal entries serially:
    ~0.9 ms per call on one 160-atom structure, where every edge carries the same index."""

    @staticmethod
    def forward(ctx, table, index, perm, seg):
        ctx.save_for_backward(index, perm, seg)
        ctx.B = table.shape[0]
        return table[index]

    @staticmethod
    def backward(ctx, g):
        index, perm, seg = ctx.saved_tensors
        return _GraphSegSum.apply(g, index, perm, seg, ctx.B), None, None, None


class _GraphSegSum(torch.autograd.Function):
    """The adjoint of _GraphGather (a segmented sum); its own backward is the gather again, so higher orders follow."""

    @staticmethod
    def forward(ctx, g, index, perm, seg, B):
        ctx.save_for_backward(index, perm, seg)
        return _segsum(g, perm, seg, B)

    @staticmethod
    def backward(ctx, gg):
        index, perm, seg = ctx.saved_tensors
        return _GraphGather.apply(gg, index, perm, seg), None, None, None, None


def _segsum1(src, seg, B):
    out = torch.empty(B, device=src.device, dtype=torch.float32)
    _native.launch('geom_segsum1', _native.load().mh_geom_segsum1, _module(src.device).handle, _native.ptr(src),
                   _native.ptr(seg), _native.ptr(out), B, _native.stream_of(src))
    return out


class _StructureSum(torch.autograd.Function):
    """out[b] = sum of src over structure b's atoms (rows ptr[b] .. ptr[b + 1] - 1 of the sorted batch); the backward
    is the gather g[batch] (_StructureGather), whose own backward is this sum again, so higher orders follow."""

    @staticmethod
    def forward(ctx, src, batch, seg):
        ctx.save_for_backward(batch, seg)
        return _segsum1(src.contiguous(), seg, seg.shape[0] - 1)

    @staticmethod
    def backward(ctx, g):
        batch, seg = ctx.saved_tensors
        return _StructureGather.apply(g, batch, seg), None, None


class _StructureGather(torch.autograd.Function):
    @staticmethod
    def forward(ctx, g, batch, seg):
        ctx.save_for_backward(batch, seg)
        return g.index_select(0, batch)

    @staticmethod
    def backward(ctx, gg):
        batch, seg = ctx.saved_tensors
        return _StructureSum.apply(gg, batch, seg), None, None


def structure_sum(src, batch, ptr):
    """Per-structure sums [B] of per-atom values src [N] (float32, GPU) for a sorted batch vector with offsets ptr
    [B + 1]: MACE's ``scatter_sum(src, batch, dim=0, dim_size=B)``, as segmented sums in a fixed order."""
    return _StructureSum.apply(src, batch, ptr.to(torch.int64).contiguous())


def symmetric_displacement(positions, unit_shifts, cell, edge_index, num_graphs, batch, ptr):
    """MACE's ``get_symmetric_displacement`` (positions and shifts under a symmetric strain of each structure's cell,
    for the virials and the stress) with its two per-structure gathers, sym[batch] over the atoms and
    cell[batch[sender]] over the edges, differentiated by segmented sums: atoms by ``ptr`` (structure b owns atoms
    ptr[b] .. ptr[b + 1] - 1), edges through the sender CSR the convolution keeps for this edge_index (structure b's
    edges are the sender segments of its atoms)."""
    sender = edge_index[0]
    n = positions.shape[0]
    displacement = torch.zeros((num_graphs, 3, 3), dtype=positions.dtype, device=positions.device)
    displacement.requires_grad_(True)
    sym = 0.5 * (displacement + displacement.transpose(-1, -2))
    seg_atoms = ptr.to(torch.int64).contiguous()
    # row vector times a 3x3 matrix per row, as a broadcast product and a sum over three terms: the einsum / matmul
    # of MACE's expression become batched GEMMs of 3x3 blocks on the GPU (hipBLASLt launches of tens of us each)
    positions = positions + (positions.unsqueeze(-1) * _GraphGather.apply(sym, batch, None, seg_atoms)).sum(-2)
    cell = cell.view(-1, 3, 3)
    cell = cell + (cell.unsqueeze(-1) * sym.unsqueeze(-3)).sum(-2)
    rp_s, ei_s = _conv.graph_for(edge_index, n).by_send()
    seg_edges = rp_s.to(torch.int64)[seg_atoms].contiguous()
    cells = _GraphGather.apply(cell, batch[sender], ei_s, seg_edges)
    shifts = (unit_shifts.unsqueeze(-1) * cells).sum(-2)
    return positions, shifts, displacement


def _supported_displacement(positions, unit_shifts, cell, edge_index, num_graphs, batch, ptr):
    return (_supported_call(positions, edge_index, unit_shifts) and torch.is_tensor(cell) and cell.is_cuda
            and cell.dtype == torch.float32 and cell.numel() == 9 * num_graphs and torch.is_tensor(batch)
            and batch.is_cuda and batch.shape == (positions.shape[0],) and torch.is_tensor(ptr) and ptr.is_cuda
            and ptr.shape == (num_graphs + 1,))


def _supported_call(positions, edge_index, shifts):
    return (torch.is_tensor(positions) and positions.is_cuda and positions.dtype == torch.float32
            and positions.dim() == 2 and torch.is_tensor(shifts) and shifts.dtype == torch.float32
            and torch.is_tensor(edge_index) and edge_index.is_cuda and edge_index.dim() == 2 and edge_index.shape[0] == 2
            and shifts.shape == (edge_index.shape[1], 3))


def _wrap(orig):
    @functools.wraps(orig)
    def get_edge_vectors_and_lengths(positions, edge_index, shifts, normalize=False, eps=1e-9):
        if _ACTIVE.get() and _supported_call(positions, edge_index, shifts):
            vectors, lengths = edge_vectors_and_lengths(positions, edge_index, shifts)
            if normalize:
                vectors = vectors / (lengths + eps)
            return vectors, lengths
        return orig(positions, edge_index, shifts, normalize=normalize, eps=eps) if normalize else \
            orig(positions, edge_index, shifts)
    get_edge_vectors_and_lengths._mh_original = orig
    return get_edge_vectors_and_lengths


def _wrap_displacement(orig):
    @functools.wraps(orig)
    def get_symmetric_displacement(positions, unit_shifts, cell, edge_index, num_graphs, batch):
        ptr = _PTR.get()
        if _ACTIVE.get() and _supported_displacement(positions, unit_shifts, cell, edge_index, num_graphs, batch,
                                                     ptr):
            return symmetric_displacement(positions, unit_shifts, cell, edge_index, num_graphs, batch, ptr)
        return orig(positions, unit_shifts, cell, edge_index, num_graphs, batch)
    get_symmetric_displacement._mh_original = orig
    return get_symmetric_displacement


def _wrap_scatter(orig):
    try:
        sig = inspect.signature(orig)
    except (TypeError, ValueError):
        sig = None

    @functools.wraps(orig)
    def scatter_sum(src, index, *args, **kwargs):
        bp = _BATCH.get()
        if _ACTIVE.get() and bp is not None and sig is not None and index is bp[0]:
            try:
                ba = sig.bind(src, index, *args, **kwargs)
            except TypeError:
                ba = None
            if ba is not None:
                ba.apply_defaults()
                a = ba.arguments
                batch, ptr = bp
                if (a.get('out') is None and a.get('dim') in (0, -1) and torch.is_tensor(src) and src.dim() == 1
                        and src.is_cuda and src.dtype == torch.float32 and src.shape[0] == batch.shape[0]
                        and torch.is_tensor(ptr) and ptr.is_cuda and ptr.dim() == 1
                        and a.get('dim_size') == ptr.shape[0] - 1 and a.get('reduce', 'sum') == 'sum'):
                    return structure_sum(src, batch, ptr)
        return orig(src, index, *args, **kwargs)
    scatter_sum._mh_original = orig
    return scatter_sum


def _edge_ops(model):
    """(harmonics, embedding) of ``model`` when both are drop-ins and the fused edge pass is on, else None."""
    from . import edgefeat
    from .edge import HipSphericalHarmonics
    from .embedding import HipRadialEmbedding
    sh, emb = getattr(model, 'spherical_harmonics', None), getattr(model, 'radial_embedding', None)
    if edgefeat.FUSE and isinstance(sh, HipSphericalHarmonics) and isinstance(emb, HipRadialEmbedding):
        return sh, emb
    return None


def _forward_with_geometry(self, *args, **kwargs):
    token = _ACTIVE.set('double_backward' if getattr(self, '_mh_geometry_double_backward', False) else True)
    token_edge = _EDGE.set(_edge_ops(self))
    data = args[0] if args else kwargs.get('data')
    token_ptr = _PTR.set(data.get('ptr') if isinstance(data, dict) else None)
    b = data.get('batch') if isinstance(data, dict) else None
    token_batch = _BATCH.set((b, data.get('ptr')) if torch.is_tensor(b) and b.dim() == 1 else None)
    try:
        return type(self).forward(self, *args, **kwargs)
    finally:
        _BATCH.reset(token_batch)
        _PTR.reset(token_ptr)
        _EDGE.reset(token_edge)
        _ACTIVE.reset(token)


def install(model):
    """Route the model's edge geometry through the kernels; False (nothing changed) if its module has no such
    function."""
    mod = sys.modules.get(type(model).__module__)
    fn = getattr(mod, FUNCTION, None) if mod is not None else None
    if fn is None or not callable(fn):
        return False
    if not hasattr(fn, '_mh_original'):
        setattr(mod, FUNCTION, _wrap(fn))
    disp = getattr(mod, DISPLACEMENT, None)
    if callable(disp) and not hasattr(disp, '_mh_original'):
        setattr(mod, DISPLACEMENT, _wrap_displacement(disp))
    sc = getattr(mod, SCATTER, None)
    if callable(sc) and not hasattr(sc, '_mh_original'):
        setattr(mod, SCATTER, _wrap_scatter(sc))
    model.forward = types.MethodType(_forward_with_geometry, model)
    return True


def installed(model):
    f = model.__dict__.get('forward')
    return isinstance(f, types.MethodType) and f.__func__ is _forward_with_geometry


def uninstall(model):
    model.__dict__.pop('_mh_geometry_double_backward', None)
    if installed(model):
        del model.forward
        return True
    return False

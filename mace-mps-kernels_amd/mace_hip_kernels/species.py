"""
The species order of a batch's nodes in one launch (``mh_species_order``): from MACE's one-hot node attributes
[N, n_elem], the element index elem = argmax (the first maximum, as torch.argmax; reference symmetric.py:169), the
node indices stably sorted by element (``order``: what torch.argsort(elem, stable=True) gives), and the
symmetric contraction's node slots (``slots``: that order with every element's run padded with -1 to a multiple of
``group``, then -1 up to a fixed length).  One workgroup: the element histogram, its prefix sums, then the nodes in
chunks of 1024, each placed at its element's running count plus the number of earlier same-element nodes in its
chunk (ballots within a wave, per-wave counts in LDS across waves).  No atomics on global memory and no host
synchronisation; the result does not depend on scheduling.
"""
import torch

from . import _native

MAX_ELEM = 128             # elements the kernel handles (LDS tables); larger tables take the torch expressions


def source():
    return _native.device_header() + f'#define SP_MAX_ELEM {MAX_ELEM}\n' + r"""
extern "C" __global__ __launch_bounds__(1024) void species_order(const float* __restrict__ attrs, int N, int ne,
    int* __restrict__ elem, int* __restrict__ order, int* __restrict__ slots, int nslots, int group) {
  __shared__ int hist[SP_MAX_ELEM], start[SP_MAX_ELEM], pstart[SP_MAX_ELEM], run[SP_MAX_ELEM];
  __shared__ int wcnt[16][SP_MAX_ELEM];
  const int t = threadIdx.x, lane = t & (MH_WAVE - 1), wave = t >> 6;
  for (int k = t; k < SP_MAX_ELEM; k += 1024) { hist[k] = 0; run[k] = 0; }
  for (int k = t; k < 16 * SP_MAX_ELEM; k += 1024) (&wcnt[0][0])[k] = 0;
  for (int k = t; k < nslots; k += 1024) slots[k] = -1;
  __syncthreads();
  for (int i = t; i < N; i += 1024) {                 // element = first maximum of the row
    const float* __restrict__ row = attrs + (size_t)i * ne;
    float best = row[0];
    int e = 0;
    for (int k = 1; k < ne; ++k) {
      const float v = row[k];
      if (v > best) { best = v; e = k; }
    }
    elem[i] = e;
    atomicAdd(&hist[e], 1);
  }
  __syncthreads();
  if (t == 0) {
    int s = 0, ps = 0;
    for (int k = 0; k < ne; ++k) {
      start[k] = s;
      pstart[k] = ps;
      s += hist[k];
      ps += (hist[k] + group - 1) / group * group;
    }
  }
  __syncthreads();
  for (int base = 0; base < N; base += 1024) {
    const int i = base + t;
    const bool live = i < N;
    const int e = live ? elem[i] : -1;
    int before = 0;                                   // earlier lanes of this wave with the same element
    for (int l = 0; l < MH_WAVE; ++l) {
      const int el = __shfl(e, l, MH_WAVE);
      before += (l < lane && el == e) ? 1 : 0;
    }
    if (live) atomicAdd(&wcnt[wave][e], 1);
    __syncthreads();
    if (live) {
      int pos = run[e] + before;
      for (int w = 0; w < wave; ++w) pos += wcnt[w][e];
      order[start[e] + pos] = i;
      slots[pstart[e] + pos] = i;
    }
    __syncthreads();
    for (int k = t; k < ne; k += 1024) {
      int c = 0;
      for (int w = 0; w < 16; ++w) { c += wcnt[w][k]; wcnt[w][k] = 0; }
      run[k] += c;
    }
    __syncthreads();
  }
}
"""


_MODULES = {}


def _module(device):
    idx = device.index if device.index is not None else torch.cuda.current_device()
    m = _MODULES.get(idx)
    if m is None:
        code = _native.compile_source(source())
        with torch.cuda.device(idx):
            m = _native.Module(code, {_native.MH_SPECIES_ORDER: ('species_order', 1024, 1)})
        _MODULES[idx] = m
    return m


def slot_count(n, n_elem, group):
    """Length of the slot array: ceil(n / group) group + n_elem group, an upper bound for any element mix, so the
    launch size of the kernels that walk it needs no device-to-host copy."""
    return -(-n // group) * group + n_elem * group


def species_order(node_attrs, group):
    """(elem int32 [N], order int32 [N], slots int32 [slot_count]) of one-hot node attributes [N, n_elem]: one launch
    of ``species_order`` for a GPU tensor; the same results from torch expressions when n_elem > MAX_ELEM or for a
    host tensor (the patched model itself runs on the GPU only)."""
    if node_attrs.dim() != 2:
        raise ValueError(f'node_attrs must be [N, n_elem], got {tuple(node_attrs.shape)}')
    n, ne = node_attrs.shape
    dev = node_attrs.device
    ns = slot_count(n, ne, group)
    if ne > MAX_ELEM or ne == 0 or node_attrs.dtype != torch.float32 or not node_attrs.is_cuda:
        elem = torch.argmax(node_attrs, dim=1).to(torch.int32).contiguous()
        order = torch.argsort(elem, stable=True).to(torch.int32).contiguous()
        el = elem.long()
        cnt = torch.zeros(ne, dtype=torch.int64, device=dev).scatter_add_(0, el, torch.ones_like(el))
        run = (cnt + group - 1) // group * group
        start, pstart = torch.cumsum(cnt, 0) - cnt, torch.cumsum(run, 0) - run
        es = el[order.long()]
        pos = pstart[es] + torch.arange(n, device=dev) - start[es]
        slots = torch.full((ns,), -1, dtype=torch.int32, device=dev)
        slots.scatter_(0, pos, order)
        return elem, order, slots
    attrs = node_attrs.detach().contiguous()
    elem = torch.empty(n, dtype=torch.int32, device=dev)
    order = torch.empty(n, dtype=torch.int32, device=dev)
    slots = torch.empty(ns, dtype=torch.int32, device=dev)
    P = _native.ptr
    _native.launch('species_order', _native.load().mh_species_order, _module(dev).handle, P(attrs), n, ne, P(elem),
                   P(order), P(slots), ns, group, _native.stream_of(attrs))
    return elem, order, slots

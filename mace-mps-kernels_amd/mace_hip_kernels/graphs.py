"""
One patched model call captured as a HIP graph.

An energy+forces call of the patched MACE model still issues about 150 launches from Python (the HIP kernels plus
PyTorch's scatter, sums and autograd bookkeeping); unpatched it issues about a thousand, and at the sizes of a batch
of ~160-atom structures such a call is bound by host launch cost, not by the GPU.  For a fixed graph (fixed atoms and edge list, as with padded batches or an MD neighbour list with a
skin) the whole call — forward, ``autograd.grad`` and the HIP kernels — can be captured once and replayed:

    from mace_hip_kernels import patch_model
    from mace_hip_kernels.graphs import capture
    patch_model(model)
    call = capture(model, batch, compute_force=True)     # warms up eagerly, then captures one call
    with torch.no_grad():                                 # the batch tensors are the graph's inputs: update in place
        batch['positions'].copy_(new_positions)
    out = call.replay()                                   # every kernel runs again; out['forces'] is overwritten

What is frozen: the tensors of ``batch`` (their addresses and shapes).  By default the edge list's content is frozen
too — the CSRs the convolution kernels read are built by the eager warm-up and reused; after a neighbour-list
rebuild, capture again.  With ``rebuild_graph=True`` the captured call also rebuilds the CSRs (``mh_graph_build``: a
counting sort per direction) from the current contents of ``batch['edge_index']``, so a neighbour list of the same size (padded)
can be copied in before each replay.  Those rebuilt graphs cannot be validated on the host inside the graph: node
indices are clamped into range instead (a bad edge list gives wrong numbers, never a bad memory access).  The caller
must not resize or reallocate the batch tensors while the capture is in use.

A molecular-dynamics step can be captured whole: with ``neighbours=dict(r_max=..., pbc=<[B, 3] bool GPU tensor>,
pad_edges_to=...)`` every replay first rebuilds the neighbour list on the GPU from the current positions
(``mace_hip_kernels.neighbours``, the fixed-size padded layout), then the graph's CSRs, then runs the call:

    step = capture(model, batch, neighbours=dict(r_max=5.0, pbc=pbc, pad_edges_to=6000), compute_force=True)
    batch['positions'].copy_(new_positions)
    out = step.replay()                                   # neighbour list, CSRs, energy and forces
    step.check()                                          # (synchronises) every structure fitted its padding

Each replay of such a step copies the per-structure edge counts to pinned host memory behind an event; the next
replay reads the copies that have landed, without waiting, and raises ValueError for a structure that outgrew
``pad_edges_to`` (its graph then held only a subset of its edges) or could not be padded or searched (n_edges -1).
``check()`` waits for every copy.  So a bad step is reported one replay late at the latest, and no replay
synchronises.
"""
import collections

import torch

from . import _native
from . import conv as _conv
from .neighbours import raise_incomplete, update_batch

PENDING_COUNTS = 4         # edge-count copies in flight before a replay waits for the oldest

__all__ = ['capture', 'CapturedCall']


class CapturedCall:
    """A captured model call: ``replay()`` re-runs it on the current contents of ``batch`` and returns the outputs
    (the same tensors every time, overwritten by each replay)."""

    def __init__(self, model, batch, warmup=2, rebuild_graph=False, neighbours=None, **kwargs):
        if not torch.cuda.is_available():
            raise RuntimeError('HIP graph capture needs a GPU')
        self.model, self.batch, self.kwargs = model, batch, kwargs
        self.neighbour_list = None
        self._pad = neighbours.get('pad_edges_to') if neighbours is not None else None
        self._counts = collections.deque()           # (pinned int32 [B], event) of replays not yet checked
        self._free = []                              # pinned buffers whose counts were checked
        if neighbours is not None:
            pbc = neighbours.get('pbc')
            if not (torch.is_tensor(pbc) and pbc.is_cuda):
                raise ValueError('neighbours: pbc must be a [B, 3] GPU tensor (a host copy cannot be captured)')
            if neighbours.get('pad_edges_to') is None:
                raise ValueError('neighbours: pad_edges_to is required (the layout must not depend on the positions)')
            rebuild_graph = True

        def call():
            if neighbours is not None:
                self.neighbour_list = update_batch(batch, neighbours['r_max'], pbc=neighbours['pbc'],
                                                   pad_edges_to=neighbours['pad_edges_to'])
            return model(batch, **kwargs)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            # builds and caches the CSRs and element indices the capture will read; the caching allocator also
            # settles its pools off the capture stream
            for _ in range(max(1, warmup)):
                call()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        if self.neighbour_list is not None:
            self.neighbour_list.check()              # the warm-up's graph (synchronised above)
        _native.take_capture_holds()
        self.graph = torch.cuda.CUDAGraph()
        _conv._capture_rebuild = bool(rebuild_graph)
        try:
            with torch.cuda.graph(self.graph):
                self.out = call()
        finally:
            _conv._capture_rebuild = False
            _conv._capture_graphs.clear()
            self._held = _native.take_capture_holds()     # cached device memory the graph reads

    def replay(self):
        self._check_counts(block=len(self._counts) >= PENDING_COUNTS)
        self.graph.replay()
        if self.neighbour_list is not None:
            n = self.neighbour_list.n_edges
            buf = self._free.pop() if self._free else torch.empty(n.shape, dtype=n.dtype, pin_memory=True)
            buf.copy_(n, non_blocking=True)
            ev = torch.cuda.Event()
            ev.record()
            self._counts.append((buf, ev))
        return self.out

    def _check_counts(self, block):
        """Read the edge counts of earlier replays whose copies have landed (``block``: wait for the oldest first)
        and raise for an incomplete graph."""
        while self._counts and (block or self._counts[0][1].query()):
            buf, ev = self._counts.popleft()
            ev.synchronize()
            block = False
            self._free.append(buf)
            raise_incomplete(buf, self._pad)

    def check(self):
        """Wait for the edge counts of every replay so far and raise ValueError if a structure's neighbour list was
        incomplete (a no-op without ``neighbours``)."""
        while self._counts:
            self._check_counts(block=True)
        return self


def capture(model, batch, warmup=2, rebuild_graph=False, neighbours=None, **kwargs):
    """Capture ``model(batch, **kwargs)`` (energy, forces, ...) as a HIP graph, with ``neighbours`` preceded by a GPU
    neighbour-list rebuild into ``batch``; see the module docstring."""
    return CapturedCall(model, batch, warmup=warmup, rebuild_graph=rebuild_graph, neighbours=neighbours, **kwargs)

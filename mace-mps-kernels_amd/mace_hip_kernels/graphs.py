"""
One patched model call captured as a HIP graph.

An energy+forces call of MACE issues about a thousand small launches from Python (linears, radial MLP, spherical
harmonics, scatter, autograd), so at the sizes of a batch of ~160-atom structures it is bound by host launch cost,
not by the GPU.  For a fixed graph (fixed atoms and edge list, as with padded batches or an MD neighbour list with a
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
rebuild, capture again.  With ``rebuild_graph=True`` the captured call also rebuilds the CSRs (a stable device sort
per direction) from the current contents of ``batch['edge_index']``, so a neighbour list of the same size (padded)
can be copied in before each replay.  Those rebuilt graphs cannot be validated on the host inside the graph: node
indices are clamped into range instead (a bad edge list gives wrong numbers, never a bad memory access).  The caller
must not resize or reallocate the batch tensors while the capture is in use.
"""
import torch

from . import _native
from . import conv as _conv

__all__ = ['capture', 'CapturedCall']


class CapturedCall:
    """A captured model call: ``replay()`` re-runs it on the current contents of ``batch`` and returns the outputs
    (the same tensors every time, overwritten by each replay)."""

    def __init__(self, model, batch, warmup=2, rebuild_graph=False, **kwargs):
        if not torch.cuda.is_available():
            raise RuntimeError('HIP graph capture needs a GPU')
        self.model, self.batch, self.kwargs = model, batch, kwargs
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            # builds and caches the CSRs and element indices the capture will read; the caching allocator also
            # settles its pools off the capture stream
            for _ in range(max(1, warmup)):
                model(batch, **kwargs)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        _native.take_capture_holds()
        self.graph = torch.cuda.CUDAGraph()
        _conv._capture_rebuild = bool(rebuild_graph)
        try:
            with torch.cuda.graph(self.graph):
                self.out = model(batch, **kwargs)
        finally:
            _conv._capture_rebuild = False
            _conv._capture_graphs.clear()
            self._held = _native.take_capture_holds()     # cached device memory the graph reads

    def replay(self):
        self.graph.replay()
        return self.out


def capture(model, batch, warmup=2, rebuild_graph=False, **kwargs):
    """Capture ``model(batch, **kwargs)`` (energy, forces, ...) as a HIP graph; see the module docstring."""
    return CapturedCall(model, batch, warmup=warmup, rebuild_graph=rebuild_graph, **kwargs)

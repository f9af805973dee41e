"""
Storage-less stand-ins for outputs that the next patched op can consume in a cheaper form than the plain tensor
(an interaction linear's output that MACE divides by a constant; a reshape_irreps that a symmetric contraction can
read in the irreps layout).  A ``Pending`` tensor has the plain output's shape, dtype and device, answers metadata
queries (shape, size, dim, dtype, device, ...) from them, and forms the plain output (``value()``, an ordinary
autograd-tracked computation) the moment anything else uses it, so every other consumer sees an ordinary tensor.
"""
import torch

# metadata queries answered from the stand-in itself, without forming the output
_META = {torch.Tensor.shape.__get__, torch.Tensor.dtype.__get__, torch.Tensor.device.__get__,
         torch.Tensor.ndim.__get__, torch.Tensor.is_cuda.__get__, torch.Tensor.requires_grad.__get__,
         torch.Tensor.layout.__get__, torch.Tensor.dim, torch.Tensor.size, torch.Tensor.numel,
         torch.Tensor.__len__, torch.Tensor.get_device}


class Pending(torch.Tensor):
    """Base class: subclasses set up their fields in ``__init__`` and implement ``value()``."""

    @staticmethod
    def __new__(cls, shape, like, *args):
        return torch.Tensor._make_wrapper_subclass(cls, tuple(shape), dtype=like.dtype, device=like.device,
                                                   requires_grad=False)

    def value(self):
        raise NotImplementedError

    @classmethod
    def intercept(cls, func, args, kwargs):
        """A subclass's shortcut for ``func`` (returns NotImplemented when there is none)."""
        return NotImplemented

    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        if func in _META:
            with torch._C.DisableTorchFunctionSubclass():
                return func(*args, **kwargs)
        got = cls.intercept(func, args, kwargs)
        if got is not NotImplemented:
            return got
        real = lambda t: t.value() if isinstance(t, Pending) else t   # noqa: E731
        args = torch.utils._pytree.tree_map(real, args)
        kwargs = torch.utils._pytree.tree_map(real, kwargs)
        with torch._C.DisableTorchFunctionSubclass():
            return func(*args, **kwargs)

    @classmethod
    def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
        # reached only by code that bypasses __torch_function__: form the output and run on it
        real = lambda t: t.value() if isinstance(t, Pending) else t   # noqa: E731
        args = torch.utils._pytree.tree_map(real, args)
        kwargs = torch.utils._pytree.tree_map(real, kwargs or {})
        return func(*args, **kwargs)


def stash_owner(t):
    """The tensor whose attributes hold the per-call caches of ``t``: ``t`` itself or, for an alias that gives
    another consumer a gradient slot of its own (``edgefeat.slot``), the tensor it aliases (held weakly)."""
    ref = getattr(t, '_mh_base', None)
    base = ref() if ref is not None else None
    return t if base is None else base


def set_slots(t, aliases):
    """Leave ``aliases`` of ``t`` (outputs of the same autograd node, each a gradient slot of its own) for the next
    consumers that call ``slot(t)``."""
    import weakref
    for a in aliases:
        a._mh_base = weakref.ref(t)            # (weak: no reference cycle through t's own stash)
    t._mh_slots = (t._version, list(aliases))


def slot(t):
    """``t``, or the next alias of it left by ``set_slots`` (same storage and version counter, an output of its own
    node, so that this consumer's gradient reaches the node separately); ``t`` itself once none is left."""
    s = getattr(t, '_mh_slots', None)
    if s is None or s[0] != t._version or not s[1]:
        return t
    return s[1].pop(0)

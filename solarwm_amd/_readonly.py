"""Read-only tensors for the slot cache's reference dict surface.

The reference mutates its cache through the dict it hands out: ``.fill_`` on the index tensors
(causal_model.py:2916-2921), slice assignment into ``k``/``v`` (:2881-2914, :1428-1451), ``.copy_``
of the camera metadata (:2068-2075).  The slot cache keeps that state elsewhere (host integers,
frame slots, a per-slot camera store), so a tensor handed out through the dict is a snapshot: a
write into it would be lost.  These tensors make every such write raise ``CacheWriteError``
instead, naming the calls that do update the cache.  Reads, arithmetic and copies work as usual;
results are plain tensors unless they alias the snapshot's storage (views stay read-only).
"""

from __future__ import annotations

import torch

_INPLACE_DUNDERS = frozenset({
    "__setitem__", "__iadd__", "__isub__", "__imul__", "__itruediv__", "__ifloordiv__",
    "__imod__", "__ipow__", "__iand__", "__ior__", "__ixor__", "__ilshift__", "__irshift__",
    "__imatmul__",
})
# trailing-underscore methods that change no element
_HARMLESS = frozenset({"requires_grad_", "share_memory_", "retain_grad"})

WRITE_HINT = (
    "the slot cache's dict entries are read-only snapshots; update the cache with "
    "solarwm_amd.attend_cached + apply_cache_updates (K/V and indices), "
    "prope.stage_camera_cache (cameras) or drop_camera_cache"
)


class CacheWriteError(RuntimeError):
    """A write through the slot cache's dict surface, which the cache would not see."""


def _mutates(name: str) -> bool:
    if name in _INPLACE_DUNDERS:
        return True
    return name.endswith("_") and not name.startswith("__") and name not in _HARMLESS


def _storage_ptr(t: torch.Tensor) -> int:
    try:
        return t.untyped_storage().data_ptr()
    except (RuntimeError, NotImplementedError):
        return -1


class ReadOnlyCacheTensor(torch.Tensor):
    """A tensor whose in-place operations (and ``out=`` writes into it) raise CacheWriteError."""

    label = "cache entry"

    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        name = getattr(func, "__name__", "")
        if args and isinstance(args[0], ReadOnlyCacheTensor) and _mutates(name):
            raise CacheWriteError(f"{name} on {args[0].label}: {WRITE_HINT}")
        outs = kwargs.get("out")
        if outs is not None:
            for o in outs if isinstance(outs, (tuple, list)) else (outs,):
                if isinstance(o, ReadOnlyCacheTensor):
                    raise CacheWriteError(f"out= {o.label} in {name}: {WRITE_HINT}")
        with torch._C.DisableTorchFunctionSubclass():
            ret = func(*args, **kwargs)
        protected = {_storage_ptr(a): a.label for a in args if isinstance(a, ReadOnlyCacheTensor)}
        return _rewrap(ret, protected)


def _rewrap(ret, protected: dict[int, str]):
    if isinstance(ret, torch.Tensor):
        if isinstance(ret, ReadOnlyCacheTensor):
            ret = ret.as_subclass(torch.Tensor)
        ptr = _storage_ptr(ret)
        if ptr in protected and ptr != -1:
            return readonly(ret, protected[ptr])
        return ret
    if isinstance(ret, (tuple, list)):
        vals = [_rewrap(r, protected) for r in ret]
        if isinstance(ret, list):
            return vals
        try:
            return type(ret)(vals)
        except TypeError:
            return tuple(vals)
    return ret


def readonly(t: torch.Tensor, label: str) -> ReadOnlyCacheTensor:
    """``t`` as a read-only snapshot named ``label`` in error messages."""
    out = t.as_subclass(ReadOnlyCacheTensor)
    out.label = label
    return out

"""``EnvMemoryView``: emulated memory as the reference's env-major ``[N, 65536]``
uint8 tensor, over the 64-env interleaved device image.

The reference's ``memory_torch()`` (``backends/warp_vec.py:799-810``) is a
plain ``uint8 [N, 65536]`` view of env-major memory, and its RL code indexes
it directly: ``mem[:, ADDR]``, ``mem[:, lo:hi]`` and ``mem[env, lo:hi]``
(``rl/pokered_packed_parcel_env.py:274-291, 387-391, 511``), after type,
dtype and rank checks (``rl/pokered_parcel_detectors.py:101-132``).  Here
memory is interleaved in blocks of 64 envs, and no strided view of that shape
exists over it.  ``EnvMemoryView`` is a ``torch.Tensor`` of that shape,
dtype and device without storage of its own:

* indexing reads the rectangle of envs x addresses the index covers with one
  ``gbx_read_mem`` launch into a new env-major tensor and applies the index to
  that, so results have the shapes and values the reference's view gives.
  They are copies: writing into a result does not reach emulator memory;
* assignment (``mem[:, 0xFF40] |= 0x80``, ``mem[e, lo:hi] = x``) writes the
  rectangle back with one ``gbx_write_mem`` launch (a read-modify-write when
  the index is strided or a list of positions);
* every other operation runs on an env-major copy of all memory (in-place
  operations write it back): correct, but it moves N x 64 KiB each time.
  Above 1 GiB (16,384 envs) the view warns once (``FullCopyWarning``) and
  names the indexed forms and ``memory_blocks_torch()``.

All launches go to torch's current stream, in program order.
"""

from __future__ import annotations

import warnings
from typing import Any, Callable

import numpy as np
import torch
from torch.utils._pytree import tree_map

from .abi import MEM_SIZE

ReadRect = Callable[[int, int, int, int], torch.Tensor]
WriteRect = Callable[[int, int, int, int, torch.Tensor], None]

# Tensor methods and properties that only read the view's metadata.
_META_METHODS = frozenset(
    ("size", "dim", "numel", "nelement", "element_size", "is_contiguous", "stride",
     "get_device", "is_floating_point", "is_complex", "is_signed", "__len__", "ndimension",
     "type")
)  # fmt: skip
_META_PROPS = frozenset(
    ("shape", "dtype", "device", "ndim", "is_cuda", "layout", "requires_grad", "is_leaf",
     "grad", "grad_fn", "is_sparse", "is_quantized", "is_meta", "is_nested", "itemsize", "nbytes")
)  # fmt: skip
_INPLACE_DUNDER = frozenset(
    ("__iadd__", "__isub__", "__imul__", "__iand__", "__ior__", "__ixor__", "__ilshift__",
     "__irshift__", "__itruediv__", "__ifloordiv__", "__imod__")
)  # fmt: skip


# A full env-major copy larger than this warns once per view.
FULL_COPY_WARN_BYTES = 1 << 30


class FullCopyWarning(UserWarning):
    """An operation on an ``EnvMemoryView`` copied all of emulated memory."""


def _is_inplace(name: str) -> bool:
    return name in _INPLACE_DUNDER or (name.endswith("_") and not name.startswith("_"))


def _axis(sel: Any, size: int) -> tuple[int, int, Any] | None:
    """``(lo, hi, sub)`` such that ``x[sel]`` along this axis equals
    ``x[lo:hi][sub]``; ``None`` for selections handled on a full copy."""
    if isinstance(sel, bool) or sel is None:
        return None
    if isinstance(sel, (int, np.integer)) or (
        isinstance(sel, torch.Tensor) and sel.ndim == 0 and sel.dtype not in (torch.bool, torch.uint8)
        and not sel.is_floating_point()
    ):  # fmt: skip
        i = int(sel)
        if i < -size or i >= size:
            raise IndexError(f"index {i} is out of bounds for dimension with size {size}")
        i = i + size if i < 0 else i
        return i, i + 1, 0
    if isinstance(sel, slice):
        start, stop, step = sel.indices(size)
        if step <= 0:
            raise ValueError("step must be greater than zero")
        r = range(start, stop, step)
        if len(r) == 0:
            return start, start, slice(0, 0)
        lo, hi = r[0], r[-1] + 1
        return lo, hi, (slice(None) if step == 1 else slice(0, hi - lo, step))
    idx = sel if isinstance(sel, torch.Tensor) else torch.as_tensor(np.asarray(sel))
    if idx.is_floating_point():
        raise IndexError("tensors used as indices must be long, int, byte or bool tensors")
    if idx.dtype in (torch.bool, torch.uint8):
        if idx.ndim != 1 or int(idx.shape[0]) != size:
            return None
        idx = idx.bool().nonzero().squeeze(1)
    idx = idx.to(torch.int64)
    if idx.numel() == 0:
        return 0, 0, idx
    lo_i, hi_i = int(idx.min()), int(idx.max())
    if lo_i < -size or hi_i >= size:
        bad = hi_i if hi_i >= size else lo_i
        raise IndexError(f"index {bad} is out of bounds for dimension with size {size}")
    idx = torch.where(idx < 0, idx + size, idx)
    lo, hi = int(idx.min()), int(idx.max()) + 1
    return lo, hi, idx - lo


def _split_key(key: Any) -> tuple[Any, Any] | None:
    """The (env, address) selections of an index into a 2-D tensor."""
    if not isinstance(key, tuple):
        key = (key,)
    if sum(k is Ellipsis for k in key) > 1:
        raise IndexError("an index can only have a single ellipsis ('...')")
    if any(k is Ellipsis for k in key):
        i = next(j for j, k in enumerate(key) if k is Ellipsis)
        key = key[:i] + (slice(None),) * (3 - len(key)) + key[i + 1 :]
    if any(k is None for k in key):
        return None
    if len(key) > 2:
        raise IndexError(f"too many indices for tensor of dimension 2 (got {len(key)})")
    key = key + (slice(None),) * (2 - len(key))
    return key[0], key[1]


class EnvMemoryView(torch.Tensor):
    """``uint8 [num_envs, 65536]`` emulated memory, indexed like the
    reference's env-major ``memory_torch()`` view."""

    _read_rect: ReadRect
    _write_rect: WriteRect

    @staticmethod
    def __new__(cls, num_envs: int, device: torch.device, read_rect: ReadRect, write_rect: WriteRect):
        t = torch.Tensor._make_wrapper_subclass(cls, (int(num_envs), MEM_SIZE), dtype=torch.uint8, device=device)
        t._read_rect = read_rect
        t._write_rect = write_rect
        return t

    def __init__(self, *args: Any, **kwargs: Any) -> None:
        pass

    @property
    def num_envs(self) -> int:
        with torch._C.DisableTorchFunctionSubclass():
            return int(self.shape[0])

    # -- the three access paths ------------------------------------------------
    def _dense(self) -> torch.Tensor:
        """Env-major copy of all memory, ``[num_envs, 65536]``."""
        nbytes = self.num_envs * MEM_SIZE
        if nbytes > FULL_COPY_WARN_BYTES and not getattr(self, "_warned", False):
            self._warned = True
            warnings.warn(
                f"an operation on memory_torch() copied all emulated memory ({nbytes / 2**30:.1f} GiB, "
                "and writes it back if in place); index the view (mem[:, ADDR], mem[:, lo:hi], "
                "mem[env, lo:hi]) or use ram_senses_torch() / memory_blocks_torch() to avoid it",
                FullCopyWarning,
                stacklevel=4,
            )
        return self._read_rect(0, self.num_envs, 0, MEM_SIZE)

    def _getitem(self, key: Any) -> torch.Tensor:
        parts = _split_key(key)
        ke = ka = None
        if parts is not None:
            ke, ka = _axis(parts[0], self.num_envs), _axis(parts[1], MEM_SIZE)
        if ke is None or ka is None:
            return self._dense()[key]
        sub = self._read_rect(ke[0], ke[1], ka[0], ka[1])
        return sub[ke[2], ka[2]]

    def _setitem(self, key: Any, value: Any) -> None:
        parts = _split_key(key)
        ke = ka = None
        if parts is not None:
            ke, ka = _axis(parts[0], self.num_envs), _axis(parts[1], MEM_SIZE)
        if ke is None or ka is None:
            full = self._dense()
            full[key] = value
            self._write_rect(0, self.num_envs, 0, MEM_SIZE, full)
            return
        (e0, e1, se), (a0, a1, sa) = ke, ka
        if e1 == e0 or a1 == a0:
            return
        covers = all(isinstance(s, int) or (isinstance(s, slice) and s == slice(None)) for s in (se, sa))
        if covers:  # the index selects the whole rectangle: no read needed
            sub = torch.empty((e1 - e0, a1 - a0), dtype=torch.uint8, device=self.device)
        else:
            sub = self._read_rect(e0, e1, a0, a1)
        sub[se, sa] = value
        self._write_rect(e0, e1, a0, a1, sub)

    # -- torch protocol ----------------------------------------------------------
    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):  # type: ignore[override]
        kwargs = kwargs or {}
        if func is torch.Tensor.__getitem__:
            return args[0]._getitem(args[1])
        if func is torch.Tensor.__setitem__:
            args[0]._setitem(args[1], args[2])
            return None
        name = getattr(func, "__name__", "")
        if name == "__get__":
            prop = getattr(getattr(func, "__self__", None), "__name__", "")
            if prop in _META_PROPS:
                with torch._C.DisableTorchFunctionSubclass():
                    return func(*args, **kwargs)
        elif name in _META_METHODS:
            with torch._C.DisableTorchFunctionSubclass():
                return func(*args, **kwargs)
        # everything else on env-major copies
        conv = lambda a: a._dense() if isinstance(a, EnvMemoryView) else a  # noqa: E731
        dargs, dkwargs = tree_map(conv, args), tree_map(conv, kwargs)
        with torch._C.DisableTorchFunctionSubclass():
            out = func(*dargs, **dkwargs)
        if _is_inplace(name) and args and isinstance(args[0], EnvMemoryView):
            view = args[0]
            view._write_rect(0, view.num_envs, 0, MEM_SIZE, dargs[0])
            return view
        return out

    @classmethod
    def __torch_dispatch__(cls, func, types, args=(), kwargs=None):  # type: ignore[override]
        raise TypeError(
            f"EnvMemoryView has no storage of its own ({func}); index it (mem[:, lo:hi]) "
            "or take a copy with mem.clone()"
        )

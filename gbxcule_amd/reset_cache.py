"""``ResetCache``: snapshot one env, restore it into any masked subset.

Mirrors ``src/gbxcule/core/reset_cache.py:23-411``.  The snapshot lives in the
backend's device context (one slot per backend); ``apply_mask_torch`` runs the
masked restore as two kernels on torch's current stream instead of the
reference's 37 per-array launches.  Restored: memory, cart RAM, cart state,
serial buffer, unpacked pixels (when the backend renders them), registers,
counters, timer/PPU/IRQ state and the action slot; not restored: packed pixels
and the env-0 scanline latches (as in the reference).
"""

from __future__ import annotations

import ctypes
from typing import Any

import numpy as np

from .backend import HipVecBackend, _cur_stream, _torch


class ResetCache:
    def __init__(self, backend: HipVecBackend, env_idx: int, generation: int):
        self.backend = backend
        self.num_envs = backend.num_envs
        self.env_idx = env_idx
        self._generation = generation

    @classmethod
    def from_backend(cls, backend: HipVecBackend, *, env_idx: int = 0) -> ResetCache:
        """Capture env ``env_idx`` (reference core/reset_cache.py:68-190)."""
        if not backend._initialized:
            raise RuntimeError("Backend not initialized")
        if env_idx < 0 or env_idx >= backend.num_envs:
            raise ValueError(f"env_idx {env_idx} out of range")
        with_pix = 1 if backend._render_pixels else 0
        backend._call(
            "gbx_snapshot", backend.ctx, env_idx, with_pix, ctypes.c_void_p(_cur_stream())
        )
        _torch().cuda.synchronize()
        backend._snapshot_gen += 1
        return cls(backend, env_idx, backend._snapshot_gen)

    def _check_live(self) -> None:
        if self._generation != self.backend._snapshot_gen:
            raise RuntimeError(
                "this ResetCache was superseded by a newer snapshot of the same backend"
            )

    def apply_mask_torch(self, mask: Any) -> None:
        """Restore envs where ``mask`` is non-zero (reference :381-411)."""
        self._check_live()
        torch = _torch()
        if not isinstance(mask, torch.Tensor):
            raise TypeError("mask must be a torch.Tensor")
        if mask.device.type != "cuda":
            raise ValueError("mask must be a CUDA tensor")
        if mask.ndim != 1 or int(mask.shape[0]) != self.num_envs:
            raise ValueError(f"mask must have shape ({self.num_envs},)")
        if mask.dtype is torch.bool:
            mask_u8 = mask.to(torch.uint8)
        elif mask.dtype is torch.uint8:
            mask_u8 = mask
        else:
            raise ValueError("mask must be bool or uint8")
        mask_u8 = mask_u8.contiguous()
        self.backend._call(
            "gbx_masked_reset",
            self.backend.ctx,
            ctypes.c_void_p(mask_u8.data_ptr()),
            ctypes.c_void_p(_cur_stream()),
        )

    def apply_mask_np(self, mask: np.ndarray) -> None:
        """Host-mask convenience: uploads ``mask`` then runs the same restore.
        (The reference accepts numpy masks only on its CPU device.)"""
        self._check_live()
        mask = np.asarray(mask)
        if mask.shape != (self.num_envs,):
            raise ValueError("mask must have shape (num_envs,)")
        torch = _torch()
        t = torch.from_numpy(mask.astype(np.uint8, copy=False)).to("cuda")
        self.apply_mask_torch(t)
        torch.cuda.synchronize()

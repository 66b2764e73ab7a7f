"""2-bit packed pixel helpers (reference ``src/gbxcule/rl/packed_pixels.py``
and ``packed_metrics.py``).  A packed byte holds four horizontally adjacent
shades, the leftmost in bits 0-1."""

from __future__ import annotations

from typing import Any

_LUTS: dict[tuple[str, str], Any] = {}


def _torch():
    import torch

    return torch


def get_unpack_lut(device=None, dtype=None):
    """``[256, 4]``: the four shades of every byte value."""
    torch = _torch()
    dtype = torch.uint8 if dtype is None else dtype
    key = ("unpack", f"{device}:{dtype}")
    lut = _LUTS.get(key)
    if lut is None:
        v = torch.arange(256, dtype=torch.int32)
        lut = torch.stack([(v >> (2 * k)) & 3 for k in range(4)], dim=1).to(dtype)
        if device is not None:
            lut = lut.to(device)
        _LUTS[key] = lut
    return lut


def pack_2bpp_u8(unpacked_u8):
    """Shades 0-3 along the last dimension -> packed bytes (width / 4)."""
    torch = _torch()
    if unpacked_u8.dtype is not torch.uint8:
        raise ValueError("unpacked_u8 must be uint8")
    w = int(unpacked_u8.shape[-1])
    if w % 4:
        raise ValueError("last dimension must be divisible by 4")
    q = unpacked_u8.reshape(*unpacked_u8.shape[:-1], w // 4, 4)
    return q[..., 0] | (q[..., 1] << 2) | (q[..., 2] << 4) | (q[..., 3] << 6)


def unpack_2bpp_u8(packed_u8, lut=None):
    """Packed bytes -> shades 0-3 along the last dimension (width * 4)."""
    torch = _torch()
    if packed_u8.dtype is not torch.uint8:
        raise ValueError("packed_u8 must be uint8")
    if lut is not None:
        out = lut[packed_u8.to(torch.int64)]
    else:
        out = torch.stack([(packed_u8 >> (2 * k)) & 3 for k in range(4)], dim=-1)
    return out.reshape(*packed_u8.shape[:-1], packed_u8.shape[-1] * 4)


def get_diff_lut(device=None):
    """``[256, 256]`` uint8: L1 distance between the four shades of two bytes."""
    torch = _torch()
    key = ("diff", str(device))
    lut = _LUTS.get(key)
    if lut is None:
        u = get_unpack_lut(dtype=torch.int16)
        lut = (u[:, None, :] - u[None, :, :]).abs().sum(dim=-1).to(torch.uint8)
        if device is not None:
            lut = lut.to(device)
        _LUTS[key] = lut
    return lut


def packed_l1_distance(packed_obs, packed_goal):
    """Mean per-pixel shade distance to a goal, in [0, 1]: sum |obs - goal| over
    the 4 x H x W_bytes pixels of each env, divided by 3 x pixels
    (reference packed_metrics.py:16-41).  Computed with shifts on the packed
    bytes, no table gather; the sums are small integers, exact in float32."""
    torch = _torch()
    for name, t in (("packed_obs", packed_obs), ("packed_goal", packed_goal)):
        if t.dtype is not torch.uint8:
            raise ValueError(f"{name}: expected uint8 packed frames, got {t.dtype}")
    if packed_obs.ndim != 4:
        raise ValueError(f"packed_obs: expected [N, 1, H, W_bytes], got {tuple(packed_obs.shape)}")
    # one goal for every env ([1, H, W_bytes] or [1, 1, H, W_bytes]) or one
    # per env ([N, 1, H, W_bytes]), as the reference accepts them
    goal = packed_goal.unsqueeze(0) if packed_goal.ndim == 3 else packed_goal
    if goal.ndim != 4:
        raise ValueError(
            f"packed_goal: expected [1, 1, H, W_bytes], [N, 1, H, W_bytes] or [1, H, W_bytes], "
            f"got {tuple(packed_goal.shape)}"
        )
    if goal.shape[1] != 1:
        raise ValueError(f"packed_goal: expected channel dim 1, got {tuple(packed_goal.shape)}")
    if goal.shape[2:] != packed_obs.shape[2:]:
        raise ValueError(
            f"packed_goal: spatial shape {tuple(goal.shape[2:])} differs from the observations' "
            f"{tuple(packed_obs.shape[2:])}"
        )
    if goal.shape[0] not in (1, packed_obs.shape[0]):
        raise ValueError(
            f"packed_goal: {goal.shape[0]} goals for {packed_obs.shape[0]} observations (expected 1 or N)"
        )
    packed_goal = goal
    o = packed_obs.to(torch.int16)
    g = packed_goal.to(torch.int16)
    d = torch.zeros_like(o)
    for k in range(4):
        d += (((o >> (2 * k)) & 3) - ((g >> (2 * k)) & 3)).abs()
    total = d.sum(dim=(1, 2, 3), dtype=torch.int32).to(torch.float32)
    pixels = int(packed_obs.shape[2] * packed_obs.shape[3] * 4)
    return total / float(pixels * 3)

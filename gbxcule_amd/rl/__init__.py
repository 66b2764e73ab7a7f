"""RL-side plumbing around the HIP backend: the zero-copy rollout pattern of
the reference's RL engines (``src/gbxcule/rl/``) -- preallocated rollout
buffers, double-buffer stream coordination, packed-pixel helpers and a
game-agnostic packed-pixel env that chains step -> render into a rollout slot
-> RAM senses -> masked reset on torch's current stream with no host sync."""

from .async_buffers import AsyncPPOBufferManager, AsyncPPOBufferState
from .env import PackedPixelEnv, collect_rollout
from .packed import (
    get_diff_lut,
    get_unpack_lut,
    pack_2bpp_u8,
    packed_l1_distance,
    unpack_2bpp_u8,
)
from .rollout import RolloutBuffer

__all__ = [
    "AsyncPPOBufferManager",
    "AsyncPPOBufferState",
    "PackedPixelEnv",
    "RolloutBuffer",
    "collect_rollout",
    "get_diff_lut",
    "get_unpack_lut",
    "pack_2bpp_u8",
    "packed_l1_distance",
    "unpack_2bpp_u8",
]

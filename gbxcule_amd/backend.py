"""``HipVecBackend``: gbxcule's vectorized backend API over the HIP core.

Mirrors ``WarpVecCudaBackend`` (reference ``src/gbxcule/backends/warp_vec.py``
:89-1476) and the ``VecBackend`` protocol (``backends/common.py:175-242``):
same constructor keywords, method names, shapes, dtypes and exception types.
Every launch goes through the C ABI of ``libgbx_hip.so`` on torch's current
HIP stream; there is no CPU fallback.

Emulated memory is interleaved in blocks of 64 envs on the device.
``memory_torch()`` still answers as the reference's env-major ``[N, 65536]``
uint8 tensor (``EnvMemoryView``: indexing reads and writes the selected
rectangle in one launch); ``memory_blocks_torch()`` is the native zero-copy
``[blocks, 65536, 64]`` view, and ``ram_senses_torch`` gathers fixed RAM bytes
of every env in one launch.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Any

import numpy as np

from . import _lib
from .abi import (
    ACTION_CODEC_ID,
    ACTION_NAMES,
    BOOTROM_SIZE,
    CART_STATE_FIELDS,
    CART_STATE_STRIDE,
    DOWNSAMPLE_H,
    DOWNSAMPLE_W,
    DOWNSAMPLE_W_BYTES,
    ENV_BLOCK,
    MEM_SIZE,
    NUM_ACTIONS,
    OBS_DIM_DEFAULT,
    ROM_LIMIT,
    SERIAL_MAX,
    STAGE_ID,
    parse_cartridge_header,
)
from .carts.bootstub import build_bootstub


class ArraySpec(dict):
    """Shape/dtype/meaning record (reference backends/common.py:44-70)."""

    def __init__(self, shape: tuple[int, ...], dtype: str, meaning: str):
        super().__init__(shape=shape, dtype=dtype, meaning=meaning)
        self.shape, self.dtype, self.meaning = shape, dtype, meaning


def flags_from_f(f: int) -> dict[str, int]:
    """Z/N/H/C bits of F (reference backends/common.py:317-337)."""
    return {"z": (f >> 7) & 1, "n": (f >> 6) & 1, "h": (f >> 5) & 1, "c": (f >> 4) & 1}


class _DevArray:
    """Exposes a device pointer through ``__cuda_array_interface__``."""

    def __init__(self, ptr: int, shape: tuple[int, ...], typestr: str):
        self.__cuda_array_interface__ = {
            "shape": tuple(int(s) for s in shape),
            "typestr": typestr,
            "data": (int(ptr), False),
            "version": 3,
            "strides": None,
        }


_TYPESTR = {"uint8": "|u1", "int32": "<i4", "float32": "<f4", "int64": "<i8", "uint64": "<u8"}


def _torch():
    import torch

    return torch


def _cur_stream() -> int:
    torch = _torch()
    return int(torch.cuda.current_stream().cuda_stream)


def _read_bytes(src: str | os.PathLike | bytes | bytearray | None, default: bytes | None) -> bytes:
    if src is None:
        if default is None:
            raise ValueError("no data given")
        return default
    if isinstance(src, (bytes, bytearray)):
        return bytes(src)
    p = Path(src)
    if not p.exists():
        raise FileNotFoundError(f"ROM file not found: {p}")
    return p.read_bytes()


class HipVecBackend:
    """N Game Boys on one MI355X behind the gbxcule backend API."""

    name: str = "hip_vec"

    def __init__(
        self,
        rom_path: str | os.PathLike | bytes,
        *,
        num_envs: int = 1,
        frames_per_step: int = 24,
        release_after_frames: int = 8,
        obs_dim: int = OBS_DIM_DEFAULT,
        base_seed: int | None = None,
        action_codec: str = ACTION_CODEC_ID,
        stage: str = "obs_only",
        render_bg: bool = False,
        render_pixels: bool = False,
        render_pixels_packed: bool = False,
        render_on_step: bool = True,
        force_lcdc_on_render: bool = False,
        bootrom: str | os.PathLike | bytes | None = None,
    ) -> None:
        if obs_dim != OBS_DIM_DEFAULT:
            raise ValueError(f"obs_dim {obs_dim} unsupported; expected {OBS_DIM_DEFAULT}")
        if action_codec != ACTION_CODEC_ID:
            raise ValueError(f"Unknown action codec: {action_codec}")
        if stage not in STAGE_ID:
            raise ValueError(f"unknown stage {stage!r}")
        if num_envs <= 0:
            raise ValueError("num_envs must be > 0")
        _lib.load()
        self.num_envs = int(num_envs)
        self.device = "cuda"
        self._rom_src = rom_path
        self._boot_src = bootrom
        self._obs_dim = obs_dim
        self._frames_per_step = int(frames_per_step)
        self._release_after_frames = int(release_after_frames)
        self._base_seed = base_seed
        self._stage = stage
        self._render_bg = bool(render_bg)
        self._render_pixels = bool(render_pixels)
        self._render_pixels_packed = bool(render_pixels_packed)
        self._render_on_step = bool(render_on_step)
        self._force_lcdc_on_render = bool(force_lcdc_on_render)
        self.num_actions = NUM_ACTIONS
        self.action_codec = {"id": ACTION_CODEC_ID, "action_names": ACTION_NAMES}
        self.action_spec = ArraySpec(
            (num_envs,), "int32", f"action index [0, {self.num_actions})"
        )
        self.obs_spec = ArraySpec(
            (num_envs, obs_dim), "float32", "Observation vector per environment"
        )
        self._ctx: ctypes.c_void_p | None = None
        self._initialized = False
        self._rom_bytes: bytes | None = None
        self._boot_bytes: bytes | None = None
        self._views: dict[str, Any] = {}
        self._snapshot_gen = 0

    # -- context -------------------------------------------------------------
    @property
    def ctx(self) -> ctypes.c_void_p:
        if self._ctx is None or not self._initialized:
            raise RuntimeError("Backend not initialized. Call reset() first.")
        return self._ctx

    def _call(self, fn: str, *args: Any) -> None:
        _lib.check(getattr(_lib.load(), fn)(*args))

    def _buffer(self, which: int) -> tuple[int, int]:
        ptr = ctypes.c_void_p()
        nbytes = ctypes.c_int64()
        self._call("gbx_buffer", self.ctx, which, ctypes.byref(ptr), ctypes.byref(nbytes))
        return int(ptr.value or 0), int(nbytes.value)

    @property
    def step_lanes(self) -> int:
        """Envs per wavefront of the step kernel (64, 32, 16 or 8)."""
        return self._info(_lib.INFO_STEP_LANES)

    def _info(self, key: int) -> int:
        out = ctypes.c_int64()
        self._call("gbx_info", self.ctx, key, ctypes.byref(out))
        return int(out.value)

    def _view(self, which: int, shape: tuple[int, ...], dtype: str):
        key = f"{which}:{shape}:{dtype}"
        v = self._views.get(key)
        if v is None:
            torch = _torch()
            ptr, nbytes = self._buffer(which)
            need = int(np.prod(shape)) * np.dtype(dtype).itemsize
            if need > nbytes:
                raise RuntimeError("device buffer smaller than the requested view")
            v = torch.as_tensor(_DevArray(ptr, shape, _TYPESTR[dtype]), device="cuda")
            self._views[key] = v
        return v

    # -- VecBackend protocol --------------------------------------------------
    def reset(self, seed: int | None = None) -> tuple[np.ndarray, dict[str, Any]]:
        """Power-on state for every env (reference warp_vec.py:249-513)."""
        rom = _read_bytes(self._rom_src, None)
        boot = _read_bytes(self._boot_src, build_bootstub())
        if len(boot) != BOOTROM_SIZE:
            raise ValueError(f"Boot ROM must be 256 bytes, got {len(boot)}")
        spec = parse_cartridge_header(rom)
        if len(rom) < spec.rom_byte_length:
            raise ValueError(
                f"ROM smaller than header advertises: {len(rom)} < {spec.rom_byte_length}"
            )
        rom = rom[: spec.rom_byte_length]
        if self._ctx is not None and rom == self._rom_bytes and boot == self._boot_bytes:
            self._call("gbx_reset", self._ctx, ctypes.c_void_p(_cur_stream()))
        else:
            self.close()
            self._rom_bytes, self._boot_bytes = rom, boot
            rom_buf = (ctypes.c_uint8 * len(rom)).from_buffer_copy(rom)
            boot_buf = (ctypes.c_uint8 * len(boot)).from_buffer_copy(boot)
            h = ctypes.c_void_p()
            self._call(
                "gbx_create",
                self.num_envs,
                rom_buf,
                len(rom),
                boot_buf,
                len(boot),
                self._obs_dim,
                ctypes.byref(h),
            )
            self._ctx = h
        self._initialized = True
        self.spec = spec
        obs = np.zeros((self.num_envs, self._obs_dim), dtype=np.float32)
        if self._stage in ("obs_only", "full_step"):
            self._launch_step(None, frames_to_run=0, release_after_frames=0, render=False)
            obs = self._read_obs()
        return obs, {"seed": seed}

    def step(self, actions: np.ndarray):
        """Host actions -> one launch; returns (obs, reward, done, trunc, info)
        like the reference (warp_vec.py:515-563, reward/done/trunc are zeros)."""
        if not self._initialized:
            raise RuntimeError("Backend not initialized. Call reset() first.")
        actions = np.asarray(actions)
        if actions.ndim != 1:
            raise ValueError(f"Actions must be 1D, got ndim={actions.ndim}, shape={actions.shape}")
        if len(actions) != self.num_envs:
            raise ValueError(f"Actions length {len(actions)} != num_envs {self.num_envs}")
        if not np.issubdtype(actions.dtype, np.integer):
            raise ValueError(f"Actions dtype must be integer, got {actions.dtype}")
        actions = np.ascontiguousarray(actions, dtype=np.int32)
        bad = (actions < 0) | (actions >= self.num_actions)
        if np.any(bad):
            raise ValueError(f"Action {int(actions[bad][0])} out of range [0, {self.num_actions})")
        stream = ctypes.c_void_p(_cur_stream())
        self._call("gbx_upload_actions", self.ctx, actions.ctypes.data_as(ctypes.c_void_p), stream)
        self._launch_step(None)
        if self._stage in ("obs_only", "full_step"):
            obs = self._read_obs()
        else:
            obs = np.zeros((self.num_envs, self._obs_dim), dtype=np.float32)
        z = np.zeros((self.num_envs,), dtype=np.float32)
        done = np.zeros((self.num_envs,), dtype=np.bool_)
        return obs, z, done, done.copy(), {}

    def step_torch(self, actions) -> None:
        """Device actions, no host staging (reference warp_vec.py:1234-1269)."""
        if not self._initialized:
            raise RuntimeError("Backend not initialized. Call reset() first.")
        torch = _torch()
        if not isinstance(actions, torch.Tensor):
            raise TypeError("actions must be a torch.Tensor")
        if actions.device.type != "cuda":
            raise ValueError("actions must be a CUDA tensor")
        if actions.ndim != 1 or int(actions.shape[0]) != self.num_envs:
            raise ValueError(f"actions must have shape ({self.num_envs},)")
        if actions.dtype is not torch.int32:
            raise ValueError("actions must have dtype torch.int32 (no implicit cast)")
        if not actions.is_contiguous():
            raise ValueError("actions must be contiguous")
        if os.environ.get("GBXCULE_VALIDATE_ACTIONS") == "1":
            invalid = (actions < 0) | (actions >= self.num_actions)
            if torch.any(invalid).item():
                raise ValueError("actions contain out-of-range values")
        self._launch_step(actions.data_ptr())

    def _launch_step(
        self,
        actions_ptr: int | None,
        *,
        frames_to_run: int | None = None,
        release_after_frames: int | None = None,
        render: bool = True,
    ) -> None:
        frames = self._frames_per_step if frames_to_run is None else frames_to_run
        release = self._release_after_frames if release_after_frames is None else release_after_frames
        stream = ctypes.c_void_p(_cur_stream())
        self._call(
            "gbx_step",
            self.ctx,
            ctypes.c_void_p(actions_ptr) if actions_ptr else None,
            int(frames),
            int(release),
            STAGE_ID[self._stage],
            stream,
        )
        if render and self._render_bg:
            self._call("gbx_render_bg_env0", self.ctx, None, stream)
        if render and self._render_on_step:
            self._launch_render_pixels()

    def _read_obs(self) -> np.ndarray:
        obs = self._view(_lib.BUF_OBS, (self.num_envs, self._obs_dim), "float32")
        return obs.cpu().numpy().copy()

    def reward_torch(self):
        """Device view of reward_v0 written by reward_only/full_step launches."""
        return self._view(_lib.BUF_REWARD, (self.num_envs,), "float32")

    def obs_torch(self):
        """Device view of obs_v0 written by obs_only/full_step launches."""
        return self._view(_lib.BUF_OBS, (self.num_envs, self._obs_dim), "float32")

    # -- rendering -----------------------------------------------------------
    def _launch_render_pixels(self) -> None:
        if not (self._render_pixels or self._render_pixels_packed):
            return
        if self._force_lcdc_on_render:
            self._apply_lcdc_override()
        stream = ctypes.c_void_p(_cur_stream())
        if self._render_pixels:
            self._call("gbx_render", self.ctx, None, 0, 0, stream)
        if self._render_pixels_packed:
            self._call("gbx_render", self.ctx, None, 0, 1, stream)

    def _apply_lcdc_override(self) -> None:
        """Set LCDC bit 7 where it is clear, keeping the other bits
        (reference warp_vec.py:734-757): one read and one write launch of
        row 0xFF40."""
        mem = self.memory_torch()
        mem[:, 0xFF40] |= 0x80

    def render_pixels_snapshot(self) -> None:
        if not self._initialized:
            raise RuntimeError("Backend not initialized. Call reset() first.")
        self._launch_render_pixels()

    def render_pixels_snapshot_torch(self) -> None:
        self.render_pixels_snapshot()

    def render_pixels_snapshot_packed_to_torch(self, out, base_offset_bytes: int = 0) -> None:
        """Packed render into a caller tensor (reference warp_vec.py:1293-1352)."""
        if not self._initialized:
            raise RuntimeError("Backend not initialized. Call reset() first.")
        torch = _torch()
        if not isinstance(out, torch.Tensor):
            raise TypeError("out must be a torch.Tensor")
        if out.device.type != "cuda":
            raise ValueError("out must be a CUDA tensor")
        if out.dtype is not torch.uint8:
            raise ValueError("out must have dtype torch.uint8")
        if not out.is_contiguous():
            raise ValueError("out must be contiguous")
        if base_offset_bytes < 0:
            raise ValueError("base_offset_bytes must be >= 0")
        frame_bytes = self.num_envs * DOWNSAMPLE_W_BYTES * DOWNSAMPLE_H
        if base_offset_bytes + frame_bytes > int(out.numel()):
            raise ValueError("out does not have enough capacity for packed frame")
        if self._force_lcdc_on_render:
            self._apply_lcdc_override()
        self._call(
            "gbx_render",
            self.ctx,
            ctypes.c_void_p(out.data_ptr()),
            int(base_offset_bytes),
            1,
            ctypes.c_void_p(_cur_stream()),
        )

    def render_pixels_snapshot_to_torch(self, out, base_offset_bytes: int = 0) -> None:
        """Unpacked counterpart of render_pixels_snapshot_packed_to_torch."""
        torch = _torch()
        if not isinstance(out, torch.Tensor) or out.dtype is not torch.uint8:
            raise TypeError("out must be a torch.uint8 tensor")
        if out.device.type != "cuda" or not out.is_contiguous():
            raise ValueError("out must be a contiguous CUDA tensor")
        frame_bytes = self.num_envs * DOWNSAMPLE_W * DOWNSAMPLE_H
        if base_offset_bytes < 0 or base_offset_bytes + frame_bytes > int(out.numel()):
            raise ValueError("out does not have enough capacity for the frame")
        self._call(
            "gbx_render",
            self.ctx,
            ctypes.c_void_p(out.data_ptr()),
            int(base_offset_bytes),
            0,
            ctypes.c_void_p(_cur_stream()),
        )

    def read_frame_bg_shade_env0(self) -> bytes:
        """Env 0's 160x144 frame of shades 0-3, rendered after each step when
        ``render_bg`` is set (reference warp_vec.py:852-857, 1389-1407)."""
        if not self._initialized:
            raise RuntimeError("Backend not initialized. Call reset() first.")
        return self.frame_bg_torch().cpu().numpy().tobytes()

    def frame_bg_torch(self):
        """Device view ``[144, 160]`` uint8 of env 0's latched full frame."""
        return self._view(_lib.BUF_FRAME_BG, (144, 160), "uint8")

    def render_bg_env0(self) -> None:
        """Render env 0's full frame now, from the latches of its last step."""
        self._call("gbx_render_bg_env0", self.ctx, None, ctypes.c_void_p(_cur_stream()))

    def pixels_torch(self):
        if not self._initialized or not self._render_pixels:
            raise RuntimeError("Pixel buffer not initialized. Call reset() first.")
        return self._view(_lib.BUF_PIX, (self.num_envs, DOWNSAMPLE_H, DOWNSAMPLE_W), "uint8")

    def pixels_packed_torch(self):
        if not self._initialized or not self._render_pixels_packed:
            raise RuntimeError("Packed pixel buffer not initialized. Call reset() first.")
        return self._view(
            _lib.BUF_PIX_PACKED, (self.num_envs, DOWNSAMPLE_H, DOWNSAMPLE_W_BYTES), "uint8"
        )

    # -- memory ----------------------------------------------------------------
    def memory_torch(self):
        """``uint8 [N, 65536]`` emulated memory as the reference's env-major view
        (warp_vec.py:799-810).  Indexing it (``mem[:, addr]``, ``mem[:, lo:hi]``,
        ``mem[env, lo:hi]``) returns new tensors of the reference's shapes from
        one ``gbx_read_mem`` launch; assigning through it writes memory with one
        ``gbx_write_mem`` launch (see ``gbxcule_amd.memview``)."""
        if not self._initialized:
            raise RuntimeError("Backend not initialized. Call reset() first.")
        v = self._views.get("env_memory")
        if v is None:
            from .memview import EnvMemoryView

            torch = _torch()
            dev = torch.device("cuda", torch.cuda.current_device())
            v = EnvMemoryView(self.num_envs, dev, self._read_mem_rect, self._write_mem_rect)
            self._views["env_memory"] = v
        return v

    def _read_mem_rect(self, env_lo: int, env_hi: int, lo: int, hi: int):
        torch = _torch()
        out = torch.empty((env_hi - env_lo, hi - lo), dtype=torch.uint8, device="cuda")
        if out.numel():
            self._call(
                "gbx_read_mem", self.ctx, env_lo, env_hi, lo, hi,
                ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(_cur_stream()),
            )  # fmt: skip
        return out

    def _write_mem_rect(self, env_lo: int, env_hi: int, lo: int, hi: int, src) -> None:
        torch = _torch()
        src = src.to(device="cuda", dtype=torch.uint8).contiguous()
        if tuple(src.shape) != (env_hi - env_lo, hi - lo):
            raise ValueError("source does not match the memory rectangle")
        if src.numel():
            self._call(
                "gbx_write_mem", self.ctx, env_lo, env_hi, lo, hi,
                ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(_cur_stream()),
            )  # fmt: skip

    def memory_blocks_torch(self):
        """Native zero-copy ``uint8 [ceil(N/64), 65536, 64]`` view: env ``e`` is
        ``[e // 64, :, e % 64]``.  Once it has been handed out, masked resets
        also restore the rows the step never writes (below 0x8000, A000-BFFF,
        E000-FDFF), since the view can write them."""
        npad = self._info(_lib.INFO_PADDED_ENVS)
        return self._view(_lib.BUF_MEM, (npad // ENV_BLOCK, MEM_SIZE, ENV_BLOCK), "uint8")

    def read_memory_torch(self, env_idx: int, lo: int, hi: int):
        """RAM/IO bytes [lo, hi) (lo >= 0x8000) of one env: ``memory_torch()[env_idx,
        lo:hi]`` as the reference takes it (warp_vec.py:812-822)."""
        if env_idx < 0 or env_idx >= self.num_envs:
            raise ValueError(f"env_idx {env_idx} out of range [0, {self.num_envs})")
        if lo < 0 or hi < 0 or lo > MEM_SIZE or hi > MEM_SIZE or lo > hi:
            raise ValueError(f"Invalid memory range: lo={lo} hi={hi}")
        if lo < ROM_LIMIT:
            raise ValueError("read_memory_torch only supports RAM/IO ranges >= 0x8000")
        return self.memory_torch()[env_idx, lo:hi]

    def ram_senses_torch(self, addrs, out=None):
        """``out[e, j] = mem[e][addrs[j]]`` for all envs in one launch.  Host
        address lists are uploaded once and reused while the same list comes
        back (an RL loop passes one fixed list every step)."""
        torch = _torch()
        if isinstance(addrs, torch.Tensor):
            a = addrs.to(torch.int32).to(torch.int16).to(device="cuda").contiguous()
        else:
            key = np.asarray(addrs, dtype=np.int64).tobytes()
            cached = getattr(self, "_senses_addrs", None)
            if cached is not None and cached[0] == key:
                a = cached[1]
            else:
                a = torch.as_tensor(addrs, dtype=torch.int32).to(torch.int16).to(device="cuda").contiguous()
                self._senses_addrs = (key, a)
        k = int(a.numel())
        if out is None:
            out = torch.empty((self.num_envs, k), dtype=torch.uint8, device="cuda")
        if out.dtype is not torch.uint8 or not out.is_contiguous() or out.numel() < self.num_envs * k:
            raise ValueError("out must be a contiguous uint8 tensor of N*k bytes")
        self._call(
            "gbx_gather_mem",
            self.ctx,
            ctypes.c_void_p(a.data_ptr()),
            k,
            ctypes.c_void_p(out.data_ptr()),
            ctypes.c_void_p(_cur_stream()),
        )
        return out

    def state_hash_torch(self):
        """Per-env uint64 hash of memory + registers (see gbx_state_hash)."""
        torch = _torch()
        out = torch.empty((self.num_envs,), dtype=torch.int64, device="cuda")
        self._call(
            "gbx_state_hash", self.ctx, ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(_cur_stream())
        )
        return out

    def export_memory(self, env_lo: int = 0, env_hi: int | None = None, lo: int = 0, hi: int = MEM_SIZE) -> np.ndarray:
        """Raw memory of envs [env_lo, env_hi) as an env-major uint8 array."""
        env_hi = self.num_envs if env_hi is None else env_hi
        out = np.empty((max(env_hi - env_lo, 0), max(hi - lo, 0)), dtype=np.uint8)
        self._call(
            "gbx_export_mem", self.ctx, env_lo, env_hi, lo, hi, out.ctypes.data_as(ctypes.c_void_p)
        )
        return out

    def read_memory(self, env_idx: int, lo: int, hi: int) -> bytes:
        """Bytes [lo, hi); below 0x8000 the boot image and linear ROM bytes are
        substituted as in the reference (warp_vec.py:766-797)."""
        if not self._initialized:
            raise RuntimeError("Backend not initialized. Call reset() first.")
        if env_idx < 0 or env_idx >= self.num_envs:
            raise ValueError(f"env_idx {env_idx} out of range [0, {self.num_envs})")
        if lo < 0 or hi < 0 or lo > MEM_SIZE or hi > MEM_SIZE or lo > hi:
            raise ValueError(f"Invalid memory range: lo={lo} hi={hi}")
        parts = []
        if lo < ROM_LIMIT:
            top = min(hi, ROM_LIMIT)
            rom, boot = self._rom_bytes or b"", self._boot_bytes or b""
            parts.append(
                bytes(
                    boot[a] if a < BOOTROM_SIZE else (rom[a] if a < len(rom) else 0xFF)
                    for a in range(lo, top)
                )
            )
        if hi > ROM_LIMIT:
            start = max(lo, ROM_LIMIT)
            parts.append(self.export_memory(env_idx, env_idx + 1, start, hi)[0].tobytes())
        return b"".join(parts)

    def write_memory(self, env_idx: int, addr: int, data: bytes) -> None:
        """Raw write into one env's memory image (debug helper)."""
        if not self._initialized:
            raise RuntimeError("Backend not initialized. Call reset() first.")
        if env_idx < 0 or env_idx >= self.num_envs:
            raise ValueError(f"env_idx {env_idx} out of range [0, {self.num_envs})")
        if addr < 0 or addr + len(data) > MEM_SIZE:
            raise ValueError(f"Write out of range: addr={addr} len={len(data)}")
        buf = (ctypes.c_uint8 * max(len(data), 1)).from_buffer_copy(bytes(data) or b"\0")
        self._call("gbx_import_mem", self.ctx, env_idx, addr, buf, len(data))

    # -- state readback --------------------------------------------------------
    def export_field(self, name: str) -> np.ndarray:
        out = np.empty((self.num_envs,), dtype=np.int64)
        self._call(
            "gbx_export_scalar", self.ctx, _lib.FIELD_ID[name], out.ctypes.data_as(ctypes.c_void_p)
        )
        return out

    def import_field(self, name: str, values: np.ndarray) -> None:
        v = np.ascontiguousarray(values, dtype=np.int64)
        if v.shape != (self.num_envs,):
            raise ValueError("values must have shape (num_envs,)")
        self._call(
            "gbx_import_scalar", self.ctx, _lib.FIELD_ID[name], v.ctypes.data_as(ctypes.c_void_p)
        )

    def export_cart_state(self) -> np.ndarray:
        out = np.empty((self.num_envs, CART_STATE_STRIDE), dtype=np.int32)
        self._call("gbx_export_cart_state", self.ctx, out.ctypes.data_as(ctypes.c_void_p))
        return out

    def import_cart_state(self, values: np.ndarray) -> None:
        v = np.ascontiguousarray(values, dtype=np.int32)
        if v.shape != (self.num_envs, CART_STATE_STRIDE):
            raise ValueError("cart state must have shape (num_envs, 20)")
        self._call("gbx_import_cart_state", self.ctx, v.ctypes.data_as(ctypes.c_void_p))

    def export_cart_ram(self, env_lo: int = 0, env_hi: int | None = None) -> np.ndarray:
        env_hi = self.num_envs if env_hi is None else env_hi
        stride = self._info(_lib.INFO_CART_RAM_STRIDE)
        out = np.empty((env_hi - env_lo, stride), dtype=np.uint8)
        self._call("gbx_export_cart_ram", self.ctx, env_lo, env_hi, out.ctypes.data_as(ctypes.c_void_p))
        return out

    def export_serial(self) -> np.ndarray:
        out = np.empty((self.num_envs, SERIAL_MAX), dtype=np.uint8)
        self._call("gbx_export_serial", self.ctx, out.ctypes.data_as(ctypes.c_void_p))
        return out

    def export_latches(self) -> np.ndarray:
        out = np.empty((9, 144), dtype=np.uint8)
        self._call("gbx_export_latches", self.ctx, out.ctypes.data_as(ctypes.c_void_p))
        return out

    def get_pc_snapshot(self) -> np.ndarray:
        return self.export_field("pc").astype(np.int32)

    def get_cpu_state(self, env_idx: int) -> dict[str, Any]:
        """Registers and counters of one env (reference warp_vec.py:947-1009)."""
        if env_idx < 0 or env_idx >= self.num_envs:
            raise ValueError(f"env_idx {env_idx} out of range [0, {self.num_envs})")
        if not self._initialized:
            raise RuntimeError("Backend not initialized. Call reset() first.")
        names = ("pc", "sp", "a", "f", "b", "c", "d", "e", "h", "l", "instr_count",
                 "cycle_count", "trap_flag", "trap_pc", "trap_opcode", "trap_kind")  # fmt: skip
        st = {n: int(self.export_field(n)[env_idx]) for n in names}
        st["pc"] &= 0xFFFF
        st["sp"] &= 0xFFFF
        for r in "abcdehl":
            st[r] &= 0xFF
        st["f"] &= 0xF0
        st["trap_pc"] &= 0xFFFF
        st["trap_opcode"] &= 0xFF
        st["flags"] = flags_from_f(st["f"])
        return st

    def get_cart_state(self, env_idx: int) -> dict[str, int]:
        if env_idx < 0 or env_idx >= self.num_envs:
            raise ValueError(f"env_idx {env_idx} out of range [0, {self.num_envs})")
        row = self.export_cart_state()[env_idx]
        return {name: int(row[i]) for i, name in enumerate(CART_STATE_FIELDS)}

    def read_serial(self, env_idx: int) -> bytes:
        if env_idx < 0 or env_idx >= self.num_envs:
            raise ValueError(f"env_idx {env_idx} out of range [0, {self.num_envs})")
        n = min(int(self.export_field("serial_len")[env_idx]), SERIAL_MAX)
        if n <= 0:
            return b""
        return self.export_serial()[env_idx, :n].tobytes()

    def drain_serial(self, env_idx: int) -> bytes:
        data = self.read_serial(env_idx)
        for name in ("serial_len", "serial_overflow"):
            v = self.export_field(name)
            v[env_idx] = 0
            self.import_field(name, v)
        return data

    def set_debug_traps(self, rst38: bool = False, trap_pc: int = 0, max_instr: int = 0, watch_addr: int = 0) -> None:
        """Runtime form of the reference's GBXCULE_TRAP_* kernel switches."""
        self._call("gbx_set_debug", self.ctx, int(bool(rst38)), trap_pc, max_instr, watch_addr)

    # -- savestates (reference warp_vec.py:1024-1074) ---------------------------
    def _check_env(self, env_idx: int) -> None:
        if not self._initialized:
            raise RuntimeError("Backend not initialized. Call reset() first.")
        if env_idx < 0 or env_idx >= self.num_envs:
            raise ValueError(f"env_idx {env_idx} out of range [0, {self.num_envs})")

    def export_env(self, env_idx: int):
        """One env's scalars, cart state, memory and cart RAM (one device call)."""
        from .state_io import EnvImage

        self._check_env(env_idx)
        img = EnvImage(
            scalars=np.zeros(len(_lib.FIELDS), dtype=np.int64),
            cart_state=np.zeros(CART_STATE_STRIDE, dtype=np.int32),
            mem=np.zeros(MEM_SIZE, dtype=np.uint8),
            cart_ram=np.zeros(self._info(_lib.INFO_RAM_BYTES), dtype=np.uint8),
        )
        p = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
        self._call(
            "gbx_export_env", self.ctx, env_idx, p(img.scalars), p(img.cart_state), p(img.mem),
            p(img.cart_ram) if img.cart_ram.size else None,
        )  # fmt: skip
        return img

    def import_env(self, env_idx: int, img) -> None:
        """Write an ``EnvImage`` back into env ``env_idx`` (cart RAM and the
        env-0 latches only when the image carries them)."""
        self._check_env(env_idx)
        sc = np.ascontiguousarray(img.scalars, dtype=np.int64)
        cs = np.ascontiguousarray(img.cart_state, dtype=np.int32)
        mem = np.ascontiguousarray(img.mem, dtype=np.uint8)
        if sc.shape != (len(_lib.FIELDS),) or cs.shape != (CART_STATE_STRIDE,) or mem.shape != (MEM_SIZE,):
            raise ValueError("env image has the wrong shape")
        cram = np.ascontiguousarray(img.cart_ram, dtype=np.uint8)
        if cram.size and cram.size != self._info(_lib.INFO_RAM_BYTES):
            raise ValueError("cart RAM image has the wrong size")
        lat = None if img.latches is None else np.ascontiguousarray(img.latches, dtype=np.uint8)
        if lat is not None and lat.shape != (9, 144):
            raise ValueError("latches must have shape (9, 144)")
        p = lambda a: None if a is None or a.size == 0 else a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
        self._call("gbx_import_env", self.ctx, env_idx, p(sc), p(cs), p(mem), p(cram), p(lat))

    def save_state(self, env_idx: int = 0):
        """Env ``env_idx`` as a ``PyBoyState``."""
        from .state_io import state_from_warp_backend

        return state_from_warp_backend(self, env_idx)

    def save_state_file(self, path: str, env_idx: int = 0) -> None:
        """Write env ``env_idx`` to a PyBoy version-9 savestate file."""
        from .state_io import save_pyboy_state, state_from_warp_backend

        save_pyboy_state(state_from_warp_backend(self, env_idx), path)

    def load_state(self, state, env_idx: int = 0) -> None:
        """Load a ``PyBoyState`` into env ``env_idx``."""
        from .state_io import apply_state_to_warp_backend

        apply_state_to_warp_backend(state, self, env_idx)

    def load_state_file(self, path: str, env_idx: int = 0) -> None:
        """Load a PyBoy savestate file (versions 9-15) into env ``env_idx``."""
        from .state_io import apply_state_to_warp_backend, load_pyboy_state

        expected = 0
        if self._rom_bytes is not None:
            expected = int(parse_cartridge_header(self._rom_bytes).ram_byte_length)
        state = load_pyboy_state(path, expected_cart_ram_size=expected)
        apply_state_to_warp_backend(state, self, env_idx)

    def close(self) -> None:
        self._views.clear()
        if self._ctx is not None:
            try:
                self._call("gbx_destroy", self._ctx)
            finally:
                self._ctx = None
        self._initialized = False

    def __del__(self) -> None:  # pragma: no cover - best effort
        try:
            self.close()
        except Exception:
            pass


# Drop-in names used by gbxcule callers (backends/warp_vec.py:1185, 1479).
WarpVecCudaBackend = HipVecBackend

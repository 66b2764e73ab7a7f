"""Game-agnostic packed-pixel RL env over ``HipVecBackend`` and the rollout
actor loop (the pattern of the reference's ``rl/pokered_packed_parcel_env.py``
:160-520 and ``rl/async_ppo_engine.py``:740-780, without the game-specific
detectors and rewards).

One env step, all on torch's current stream, no host synchronisation:

1. ``step_torch(actions)``: one step-kernel launch;
2. packed render straight into the caller's tensor (a rollout slot);
3. RAM senses: one gather launch into a preallocated ``[N, k]`` tensor;
4. reward / termination from caller hooks (torch ops on device tensors);
5. ``reset_mask``: masked restore of the start snapshot, counters cleared and
   the start frame put back into the pixels of the restored envs with
   ``torch.where`` (no boolean indexing, so no device-to-host sync).
"""

from __future__ import annotations

from collections.abc import Callable, Sequence
from pathlib import Path
from typing import Any

from ..abi import DOWNSAMPLE_H, DOWNSAMPLE_W_BYTES
from ..backend import HipVecBackend
from ..reset_cache import ResetCache

RewardFn = Callable[["PackedPixelEnv", Any, Any], tuple[Any, Any]]


class PackedPixelEnv:
    """Dict observations ``{"pixels": uint8[N, 1, 72, 20], "senses": uint8[N, k]}``
    on the GPU; ``senses`` are the raw bytes at ``sense_addrs``."""

    def __init__(
        self,
        rom_path: str | bytes,
        *,
        state_path: str | None = None,
        num_envs: int = 1,
        frames_per_step: int = 24,
        release_after_frames: int = 8,
        max_steps: int = 2048,
        sense_addrs: Sequence[int] = (),
        force_lcdc_on_render: bool = True,
        skip_reset_if_empty: bool = False,
        reward_fn: RewardFn | None = None,
        stage: str = "emulate_only",
        bootrom: str | bytes | None = None,
    ) -> None:
        import torch

        if num_envs < 1:
            raise ValueError(f"num_envs must be >= 1, got {num_envs}")
        if max_steps < 1:
            raise ValueError(f"max_steps must be >= 1, got {max_steps}")
        if not torch.cuda.is_available():
            raise RuntimeError("a HIP device is required for PackedPixelEnv")
        self._torch = torch
        self.backend = HipVecBackend(
            rom_path,
            num_envs=num_envs,
            frames_per_step=frames_per_step,
            release_after_frames=release_after_frames,
            stage=stage,
            render_pixels=False,
            render_pixels_packed=True,
            render_on_step=False,
            force_lcdc_on_render=force_lcdc_on_render,
            bootrom=bootrom,
        )
        self.num_envs = int(num_envs)
        self.num_actions = int(self.backend.num_actions)
        self.max_steps = int(max_steps)
        self._state_path = None if state_path is None else str(Path(state_path))
        self._skip_reset_if_empty = bool(skip_reset_if_empty)
        self._reward_fn = reward_fn
        self._sense_addrs = [int(a) for a in sense_addrs]
        for a in self._sense_addrs:
            if not 0 <= a <= 0xFFFF:
                raise ValueError(f"sense address {a:#x} out of range")
        self._addrs_dev = None
        self._pixels = None
        self._senses = None
        self._start_pixels = None
        self._episode_step = None
        self._reset_cache: ResetCache | None = None
        self._obs: dict[str, Any] | None = None

    @property
    def obs(self) -> dict[str, Any]:
        if self._obs is None:
            raise RuntimeError("Call reset() before accessing obs.")
        return self._obs

    @property
    def start_pixels(self):
        """The start frame ``[1, 72, 20]`` every restored env shows."""
        if self._start_pixels is None:
            raise RuntimeError("Call reset() first.")
        return self._start_pixels

    def _gather_senses(self) -> None:
        if self._sense_addrs:
            self.backend.ram_senses_torch(self._addrs_dev, out=self._senses)

    def reset(self, seed: int | None = None) -> dict[str, Any]:
        """Power on, optionally load a savestate into env 0, snapshot env 0 and
        restore it into every env (reference pokered_packed_parcel_env.py
        :168-265)."""
        torch = self._torch
        self.backend.reset(seed=seed)
        if self._state_path is not None:
            self.backend.load_state_file(self._state_path, env_idx=0)
        n = self.num_envs
        if self._pixels is None:
            self._pixels = torch.empty((n, 1, DOWNSAMPLE_H, DOWNSAMPLE_W_BYTES),
                                       dtype=torch.uint8, device="cuda")  # fmt: skip
            self._senses = torch.zeros((n, len(self._sense_addrs)), dtype=torch.uint8, device="cuda")
            # uint16 addresses carried in int16 storage (the gather reads them unsigned)
            a = torch.tensor(self._sense_addrs, dtype=torch.int32).to(torch.int16)
            self._addrs_dev = a.to("cuda")
            self._episode_step = torch.zeros((n,), dtype=torch.int32, device="cuda")
        self.backend.render_pixels_snapshot_packed_to_torch(self._pixels, 0)
        self._reset_cache = ResetCache.from_backend(self.backend, env_idx=0)
        self._reset_cache.apply_mask_torch(torch.ones((n,), dtype=torch.uint8, device="cuda"))
        self._start_pixels = self._pixels[0].clone()
        self._pixels.copy_(self._start_pixels.expand_as(self._pixels))
        self._episode_step.zero_()
        self._gather_senses()
        self._obs = {"pixels": self._pixels, "senses": self._senses}
        return self._obs

    def render_into(self, out) -> None:
        """Packed render of every env into ``out`` (``[N, 1, 72, 20]`` uint8)."""
        self.backend.render_pixels_snapshot_packed_to_torch(out, 0)

    def step(self, actions, pixels_out=None):
        """One step.  ``pixels_out`` (``[N, 1, 72, 20]`` uint8, e.g. a rollout
        slot) receives the new frame instead of the env's own pixel buffer.
        Returns ``(obs, reward, terminated, truncated, info)``."""
        torch = self._torch
        if self._obs is None or self._reset_cache is None:
            raise RuntimeError("Call reset() before step().")
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
        pixels = self._pixels if pixels_out is None else pixels_out
        self.backend.step_torch(actions)
        self.backend.render_pixels_snapshot_packed_to_torch(pixels, 0)
        self._gather_senses()
        self._episode_step.add_(1)
        truncated = self._episode_step >= self.max_steps
        if self._reward_fn is not None:
            reward, terminated = self._reward_fn(self, pixels, self._senses)
        else:
            reward = torch.zeros((self.num_envs,), dtype=torch.float32, device="cuda")
            terminated = torch.zeros((self.num_envs,), dtype=torch.bool, device="cuda")
        obs = self._obs if pixels_out is None else {"pixels": pixels, "senses": self._senses}
        return obs, reward, terminated, truncated, {"reset_mask": terminated | truncated}

    def reset_mask(self, mask, pixels=None) -> None:
        """Restore the start snapshot where ``mask`` is set; ``pixels`` (default:
        the env's own buffer) gets the start frame for those envs."""
        torch = self._torch
        if self._reset_cache is None:
            raise RuntimeError("Reset cache not initialized. Call reset() first.")
        if not isinstance(mask, torch.Tensor):
            raise TypeError("mask must be a torch.Tensor")
        if mask.device.type != "cuda":
            raise ValueError("mask must be a CUDA tensor")
        if mask.ndim != 1 or int(mask.shape[0]) != self.num_envs:
            raise ValueError(f"mask must have shape ({self.num_envs},)")
        m = mask.to(torch.bool)
        if self._skip_reset_if_empty and not bool(m.any()):
            return
        self._reset_cache.apply_mask_torch(m.to(torch.uint8))
        self._episode_step.copy_(torch.where(m, torch.zeros_like(self._episode_step), self._episode_step))
        px = self._pixels if pixels is None else pixels
        px.copy_(torch.where(m[:, None, None, None], self._start_pixels.unsqueeze(0), px))
        self._gather_senses()

    def close(self) -> None:
        self.backend.close()
        self._obs = None
        self._pixels = None
        self._senses = None
        self._start_pixels = None
        self._reset_cache = None


def collect_rollout(env: PackedPixelEnv, policy: Callable[[Any], tuple[Any, Any, Any]], rollout) -> Any:
    """Fill ``rollout`` (a ``RolloutBuffer`` with ``obs_format="packed2"``,
    ``stack_k=1`` and ``obs_steps >= steps + 1``) with one rollout, the actor
    loop of the reference's async PPO engine (async_ppo_engine.py:740-780):
    frames are rendered straight into ``rollout.obs_slot(t + 1)``, ended
    episodes are restored in place and their start frame written into that
    slot.  ``policy(obs)`` returns ``(actions int32, values, logprobs)`` device
    tensors.  Runs on torch's current stream; returns the last observation."""
    if rollout.obs_steps < rollout.steps + 1:
        raise ValueError("rollout.obs_steps must be >= steps + 1")
    if rollout.obs_format != "packed2" or rollout.stack_k != 1:
        raise ValueError("rollout must hold packed2 frames with stack_k = 1")
    rollout.reset()
    obs = rollout.obs_slot(0)
    env.render_into(obs)
    for t in range(rollout.steps):
        actions, values, logprobs = policy(obs)
        nxt = rollout.obs_slot(t + 1)
        _, reward, terminated, truncated, _ = env.step(actions, pixels_out=nxt)
        done = terminated | truncated
        rollout.set_step_fields(t, actions, reward, done, values, logprobs)
        env.reset_mask(done, pixels=nxt)
        obs = nxt
    return obs

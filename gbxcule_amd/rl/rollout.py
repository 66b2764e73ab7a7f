"""Preallocated rollout storage (reference ``src/gbxcule/rl/rollout.py``).

Observations live in ``obs_u8[obs_steps, N, stack_k, H, W]``; ``obs_slot(t)``
is a contiguous view a renderer writes into directly, so a step's pixels are
never copied.  Same constructor, properties, methods and errors as the
reference's ``RolloutBuffer``.
"""

from __future__ import annotations

from ..abi import DOWNSAMPLE_H, DOWNSAMPLE_W, DOWNSAMPLE_W_BYTES

# per-step fields: name -> torch dtype attribute
_FIELDS = (("actions", "int32"), ("rewards", "float32"), ("dones", "bool"),
           ("values", "float32"), ("logprobs", "float32"))  # fmt: skip


class RolloutBuffer:
    def __init__(
        self,
        *,
        steps: int,
        num_envs: int,
        stack_k: int,
        obs_format: str = "u8",
        obs_steps: int | None = None,
        height: int = DOWNSAMPLE_H,
        width: int = DOWNSAMPLE_W,
        device: str = "cuda",
    ) -> None:
        import torch

        if steps < 1:
            raise ValueError("steps must be >= 1")
        if num_envs < 1:
            raise ValueError("num_envs must be >= 1")
        if stack_k < 1:
            raise ValueError("stack_k must be >= 1")
        if height < 1 or width < 1:
            raise ValueError("height/width must be >= 1")
        if obs_format not in ("u8", "packed2"):
            raise ValueError("obs_format must be 'u8' or 'packed2'")
        if obs_format == "packed2":
            width = DOWNSAMPLE_W_BYTES if width == DOWNSAMPLE_W else width
            if width != DOWNSAMPLE_W_BYTES:
                raise ValueError("packed2 width must equal DOWNSAMPLE_W_BYTES")
        self._torch = torch
        self.steps = int(steps)
        self.obs_steps = int(steps if obs_steps is None else obs_steps)
        if self.obs_steps < self.steps:
            raise ValueError("obs_steps must be >= steps")
        self.num_envs = int(num_envs)
        self.stack_k = int(stack_k)
        self.obs_format = obs_format
        self.height = int(height)
        self.width = int(width)
        self.device = torch.device(device)
        self.obs_u8 = torch.empty(
            (self.obs_steps, self.num_envs, self.stack_k, self.height, self.width),
            dtype=torch.uint8,
            device=self.device,
        )
        for name, dt in _FIELDS:
            setattr(self, name, torch.empty((self.steps, self.num_envs),
                                            dtype=getattr(torch, dt), device=self.device))  # fmt: skip
        self._step = 0

    @property
    def step(self) -> int:
        return self._step

    @property
    def obs(self):
        return self.obs_u8

    def reset(self) -> None:
        self._step = 0

    def _check_fields(self, values: dict) -> None:
        torch = self._torch
        for name, dt in _FIELDS:
            v = values[name]
            if v.shape != (self.num_envs,):
                raise ValueError(f"{name} shape mismatch")
            if v.dtype is not getattr(torch, dt):
                raise ValueError(f"{name} must be {dt}")

    def add(self, obs_u8, actions, rewards, dones, values, logprobs) -> None:
        if self._step >= self.steps:
            raise RuntimeError("rollout buffer is full")
        if obs_u8.shape != (self.num_envs, self.stack_k, self.height, self.width):
            raise ValueError("obs_u8 shape mismatch")
        if obs_u8.dtype is not self._torch.uint8:
            raise ValueError("obs_u8 must be uint8")
        fields = dict(actions=actions, rewards=rewards, dones=dones, values=values, logprobs=logprobs)
        self._check_fields(fields)
        self.obs_u8[self._step].copy_(obs_u8)
        for name, v in fields.items():
            getattr(self, name)[self._step].copy_(v)
        self._step += 1

    def obs_slot(self, step_idx: int):
        if step_idx < 0 or step_idx >= self.obs_steps:
            raise ValueError("step_idx out of range")
        return self.obs_u8[step_idx]

    def set_step_fields(self, step_idx: int, actions, rewards, dones, values, logprobs) -> None:
        if step_idx < 0 or step_idx >= self.steps:
            raise ValueError("step_idx out of range")
        fields = dict(actions=actions, rewards=rewards, dones=dones, values=values, logprobs=logprobs)
        self._check_fields(fields)
        for name, v in fields.items():
            getattr(self, name)[step_idx].copy_(v)
        if step_idx == self._step:
            self._step += 1

    def as_batch(self, *, flatten_obs: bool = True):
        if self._step != self.steps:
            raise RuntimeError("rollout buffer is not full")
        b = self.steps * self.num_envs
        obs = self.obs_u8[: self.steps]
        if flatten_obs:
            obs = obs.reshape(b, self.stack_k, self.height, self.width)
        out = {"obs_u8": obs}
        for name, _ in _FIELDS:
            out[name] = getattr(self, name).reshape(b)
        return out

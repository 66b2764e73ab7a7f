"""Device storage for one rollout, written in place by the emulator.

A rollout is a stack of frames plus one row per step of typed columns:

* frames ``[obs_steps, N, stack_k, H, W]`` uint8 (unpacked shades, or packed
  2-bit bytes with W = 20).  ``obs_slot(t)`` is a contiguous view of one
  step's frames, so the renderer writes a step's pixels straight into the
  rollout and nothing is copied;
* columns ``[steps, N]``: the schema ``COLUMNS`` fixes each column's dtype,
  and every write is checked against it.

``steps`` counts the rows written so far.  ``obs_steps`` may exceed ``steps``
so that the frame after the last action (the bootstrap observation) has a
slot of its own.  The class keeps the name, keyword arguments, attributes and
methods of the reference's ``RolloutBuffer`` (``src/gbxcule/rl/rollout.py``),
which the reference's RL engines call.
"""

from __future__ import annotations

from typing import Any

from ..abi import DOWNSAMPLE_H, DOWNSAMPLE_W, DOWNSAMPLE_W_BYTES

# per-step columns and their torch dtypes (resolved by name)
COLUMNS: dict[str, str] = {
    "actions": "int32",
    "rewards": "float32",
    "dones": "bool",
    "values": "float32",
    "logprobs": "float32",
}
FRAME_FORMATS = ("u8", "packed2")


def _positive(**dims: int) -> dict[str, int]:
    out = {}
    for name, v in dims.items():
        if int(v) < 1:
            raise ValueError(f"{name} has to be at least 1 (got {v})")
        out[name] = int(v)
    return out


def _frame_shape(obs_format: str, height: int, width: int) -> tuple[int, int]:
    """(H, W) of one stored frame.  Packed frames hold 4 shades per byte: the
    unpacked width 80 names the same frame as the packed width 20."""
    if obs_format not in FRAME_FORMATS:
        raise ValueError(f"obs_format {obs_format!r} is not one of {FRAME_FORMATS}")
    h, w = _positive(height=height, width=width).values()
    if obs_format == "packed2":
        if w == DOWNSAMPLE_W:
            w = DOWNSAMPLE_W_BYTES
        if w != DOWNSAMPLE_W_BYTES:
            raise ValueError(f"packed2 frames are {DOWNSAMPLE_W_BYTES} bytes wide (got width {width})")
    return h, w


class RolloutBuffer:
    """Frames and per-step columns of one rollout, preallocated on ``device``."""

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

        dims = _positive(steps=steps, num_envs=num_envs, stack_k=stack_k)
        self.steps, self.num_envs, self.stack_k = dims["steps"], dims["num_envs"], dims["stack_k"]
        self.obs_steps = self.steps if obs_steps is None else int(obs_steps)
        if self.obs_steps < self.steps:
            raise ValueError(f"obs_steps ({self.obs_steps}) leaves no frame slot for some of the {self.steps} steps")
        self.obs_format = obs_format
        self.height, self.width = _frame_shape(obs_format, height, width)
        self.device = torch.device(device)
        self._torch = torch
        self._frame = (self.num_envs, self.stack_k, self.height, self.width)
        self.obs_u8 = torch.empty((self.obs_steps, *self._frame), dtype=torch.uint8, device=self.device)
        self._dtypes = {name: getattr(torch, dt) for name, dt in COLUMNS.items()}
        self._columns = {
            name: torch.empty((self.steps, self.num_envs), dtype=dt, device=self.device)
            for name, dt in self._dtypes.items()
        }
        self._written = 0

    # columns read as attributes (buffer.actions, buffer.rewards, ...)
    def __getattr__(self, name: str) -> Any:
        cols = self.__dict__.get("_columns")
        if cols is not None and name in cols:
            return cols[name]
        raise AttributeError(name)

    @property
    def step(self) -> int:
        """Rows written since the last ``reset``."""
        return self._written

    @property
    def obs(self):
        return self.obs_u8

    def reset(self) -> None:
        self._written = 0

    def _check(self, name: str, t, shape: tuple[int, ...], dtype) -> None:
        if tuple(t.shape) != shape:
            raise ValueError(f"{name}: expected shape {shape}, got {tuple(t.shape)}")
        if t.dtype is not dtype:
            raise ValueError(f"{name}: expected dtype {dtype}, got {t.dtype}")

    def _row(self, t: int, values: dict[str, Any]) -> None:
        """Validate every column first, then write row ``t``."""
        missing = set(COLUMNS) - set(values)
        if missing:
            raise ValueError(f"missing columns {sorted(missing)}")
        for name, v in values.items():
            self._check(name, v, (self.num_envs,), self._dtypes[name])
        for name, v in values.items():
            self._columns[name][t].copy_(v)

    def obs_slot(self, step_idx: int):
        """Contiguous ``[N, stack_k, H, W]`` view of the frames of step ``step_idx``."""
        if not 0 <= step_idx < self.obs_steps:
            raise ValueError(f"step_idx {step_idx} is outside the {self.obs_steps} frame slots")
        return self.obs_u8[step_idx]

    def set_step_fields(self, step_idx: int, actions, rewards, dones, values, logprobs) -> None:
        """Write the columns of step ``step_idx`` (its frame is written in place
        through ``obs_slot``); writing the next unwritten row advances ``step``."""
        if not 0 <= step_idx < self.steps:
            raise ValueError(f"step_idx {step_idx} is outside the {self.steps} rows")
        self._row(step_idx, dict(actions=actions, rewards=rewards, dones=dones, values=values, logprobs=logprobs))
        if step_idx == self._written:
            self._written += 1

    def add(self, obs_u8, actions, rewards, dones, values, logprobs) -> None:
        """Append one step: copy its frames into the next slot and its columns
        into the next row."""
        if self._written == self.steps:
            raise RuntimeError(f"rollout buffer is full ({self.steps} steps written)")
        self._check("obs_u8", obs_u8, self._frame, self._torch.uint8)
        self._row(self._written, dict(actions=actions, rewards=rewards, dones=dones, values=values, logprobs=logprobs))
        self.obs_u8[self._written].copy_(obs_u8)
        self._written += 1

    def as_batch(self, *, flatten_obs: bool = True) -> dict[str, Any]:
        """The full rollout as a batch: steps x envs rows (views, no copies)."""
        if self._written != self.steps:
            raise RuntimeError(f"rollout buffer is not full ({self._written} of {self.steps} steps written)")
        frames = self.obs_u8[: self.steps]
        if flatten_obs:
            frames = frames.reshape(self.steps * self.num_envs, *self._frame[1:])
        batch = {"obs_u8": frames}
        batch.update({name: col.reshape(-1) for name, col in self._columns.items()})
        return batch

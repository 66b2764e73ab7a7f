"""Rollout buffers passed between an actor stream and a learner stream.

Each buffer carries two batons, HIP events that one stream records and the
other waits on: ``ready`` goes from the actor (the buffer is filled) to the
learner, ``free`` from the learner (the buffer is consumed) back to the
actor.  Every buffer starts free.  No call synchronises the host, and all
streams keep the default priority.

``AsyncPPOBufferManager`` keeps the method names of the reference's async PPO
module (``src/gbxcule/rl/async_ppo.py``), which its engine calls;
``filling`` and ``reading`` wrap a hand-off as a ``with`` block.
"""

from __future__ import annotations

from contextlib import contextmanager
from typing import Any, Iterator


class _Baton:
    """An event recorded by the stream that hands over and waited on by the
    stream that takes over."""

    __slots__ = ("event",)

    def __init__(self) -> None:
        import torch

        self.event = torch.cuda.Event()

    def hand_over(self, stream) -> None:
        self.event.record(stream)

    def take(self, stream) -> None:
        stream.wait_event(self.event)


class AsyncPPOBufferState:
    """The batons of one buffer and the policy version that last filled it."""

    __slots__ = ("ready", "free", "policy_version")

    def __init__(self) -> None:
        self.ready, self.free = _Baton(), _Baton()
        self.policy_version = 0

    @property
    def ready_event(self):
        return self.ready.event

    @property
    def free_event(self):
        return self.free.event


class AsyncPPOBufferManager:
    """``num_buffers`` buffers cycling actor -> learner -> actor."""

    def __init__(self, num_buffers: int = 2) -> None:
        import torch

        if int(num_buffers) < 1:
            raise ValueError(f"need at least one buffer (got {num_buffers})")
        self._state = [AsyncPPOBufferState() for _ in range(int(num_buffers))]
        start = torch.cuda.current_stream()
        for st in self._state:  # nothing has filled a buffer yet: all free
            st.free.hand_over(start)

    def _at(self, buf_idx: int) -> AsyncPPOBufferState:
        if not 0 <= buf_idx < len(self._state):
            raise IndexError(f"buffer {buf_idx} of {len(self._state)}")
        return self._state[buf_idx]

    @property
    def num_buffers(self) -> int:
        return len(self._state)

    def wait_free(self, buf_idx: int, stream) -> None:
        """``stream`` (the actor) may overwrite buffer ``buf_idx`` from here on."""
        self._at(buf_idx).free.take(stream)

    def mark_ready(self, buf_idx: int, stream, policy_version: int) -> None:
        """``stream`` has filled the buffer with rollouts of ``policy_version``."""
        st = self._at(buf_idx)
        st.policy_version = int(policy_version)
        st.ready.hand_over(stream)

    def wait_ready(self, buf_idx: int, stream) -> None:
        """``stream`` (the learner) may read buffer ``buf_idx`` from here on."""
        self._at(buf_idx).ready.take(stream)

    def mark_free(self, buf_idx: int, stream) -> None:
        """``stream`` no longer reads the buffer."""
        self._at(buf_idx).free.hand_over(stream)

    def policy_version(self, buf_idx: int) -> int:
        return self._at(buf_idx).policy_version

    @contextmanager
    def filling(self, buf_idx: int, stream, policy_version: int) -> Iterator[Any]:
        """Actor side: wait until the buffer is free, then mark it ready on exit."""
        self.wait_free(buf_idx, stream)
        yield stream
        self.mark_ready(buf_idx, stream, policy_version)

    @contextmanager
    def reading(self, buf_idx: int, stream) -> Iterator[Any]:
        """Learner side: wait until the buffer is ready, then free it on exit."""
        self.wait_ready(buf_idx, stream)
        yield stream
        self.mark_free(buf_idx, stream)

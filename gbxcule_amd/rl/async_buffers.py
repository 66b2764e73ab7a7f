"""Double-buffered actor/learner coordination with HIP events
(reference ``src/gbxcule/rl/async_ppo.py``): the actor stream fills buffer i
while the learner stream consumes buffer i - 1; events order the hand-offs
without host synchronisation.  Streams keep the default priority."""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any


@dataclass
class AsyncPPOBufferState:
    ready_event: Any
    free_event: Any
    policy_version: int = 0


class AsyncPPOBufferManager:
    def __init__(self, num_buffers: int = 2) -> None:
        import torch

        if num_buffers < 1:
            raise ValueError("num_buffers must be >= 1")
        self._buffers = [
            AsyncPPOBufferState(torch.cuda.Event(), torch.cuda.Event()) for _ in range(num_buffers)
        ]
        cur = torch.cuda.current_stream()
        for b in self._buffers:
            b.free_event.record(cur)  # every buffer starts free

    @property
    def num_buffers(self) -> int:
        return len(self._buffers)

    def wait_free(self, buf_idx: int, stream) -> None:
        stream.wait_event(self._buffers[buf_idx].free_event)

    def wait_ready(self, buf_idx: int, stream) -> None:
        stream.wait_event(self._buffers[buf_idx].ready_event)

    def mark_ready(self, buf_idx: int, stream, policy_version: int) -> None:
        b = self._buffers[buf_idx]
        b.policy_version = int(policy_version)
        b.ready_event.record(stream)

    def mark_free(self, buf_idx: int, stream) -> None:
        self._buffers[buf_idx].free_event.record(stream)

    def policy_version(self, buf_idx: int) -> int:
        return int(self._buffers[buf_idx].policy_version)

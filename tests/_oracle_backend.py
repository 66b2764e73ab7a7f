"""The oracle behind the gbxcule ``VecBackend`` surface, for harness tests
(reference backend side of a lockstep verify).  ``plant`` injects a known
fault into the oracle -- a register flipped after a given step -- so the
verify path's mismatch handling can be tested on the CPU."""

from __future__ import annotations

from pathlib import Path

import numpy as np

from gbxcule_amd.abi import CART_STATE_FIELDS, NUM_ACTIONS
from gbxcule_amd.carts.bootstub import build_bootstub
from oracle.ref import RefMachine


class OracleBackend:
    name = "oracle"
    device = "cpu"

    def __init__(self, rom_path, *, num_envs=1, frames_per_step=24, release_after_frames=8,
                 stage="emulate_only", render_bg=False, plant=None, **_):  # fmt: skip
        self.rom = Path(rom_path).read_bytes() if not isinstance(rom_path, bytes) else rom_path
        self.boot = build_bootstub()
        self.num_envs = num_envs
        self.num_actions = NUM_ACTIONS
        self.fs, self.release, self.stage = frames_per_step, release_after_frames, stage
        self.plant = plant  # (step index, register name)
        self.m = RefMachine(num_envs, self.rom, self.boot)
        self.steps = 0

    def reset(self, seed=None):
        self.m.reset()
        self.steps = 0
        return np.zeros((self.num_envs, 32), np.float32), {"seed": seed}

    def step(self, actions):
        self.m.step(np.asarray(actions, np.int32), self.fs, self.release, self.stage)
        if self.plant is not None and self.steps == self.plant[0]:
            self.m.field(self.plant[1])[0] ^= 1
        self.steps += 1

    def get_cpu_state(self, i):
        st = {k: int(self.m.field(k)[i]) for k in ("pc", "sp", "a", "f", "b", "c", "d", "e", "h", "l",
                                                    "instr_count", "cycle_count", "trap_flag",
                                                    "trap_pc", "trap_opcode", "trap_kind")}  # fmt: skip
        f = st["f"]
        st["flags"] = {"z": (f >> 7) & 1, "n": (f >> 6) & 1, "h": (f >> 5) & 1, "c": (f >> 4) & 1}
        return st

    def read_memory(self, i, lo, hi):
        out = bytearray()
        for a in range(lo, hi):
            if a < 0x100:
                out.append(self.boot[a])
            elif a < 0x8000:
                out.append(self.rom[a] if a < len(self.rom) else 0xFF)
            else:
                out.append(int(self.m.mem[i, a]))
        return bytes(out)

    def get_cart_state(self, i):
        return {n: int(v) for n, v in zip(CART_STATE_FIELDS, self.m.cart_state[i])}

    def read_frame_bg_shade_env0(self):
        return self.m.render_bg_env0().tobytes()

    def get_pc_snapshot(self):
        return self.m.field("pc").astype(np.int32)

    def close(self):
        self.m.close()

"""Env 0's full-frame renderer (``render_bg``) on the device against the
oracle: after real steps (latches captured by the step kernel) and from
random VRAM/OAM with random per-line latches.
"""

from __future__ import annotations

import numpy as np
import pytest

from gbxcule_amd.carts.synth import seeded_actions
from oracle.ref import RefMachine

from .conftest import require_gpu

pytestmark = pytest.mark.gpu


def _backend(rom, boot, n, **kw):
    from gbxcule_amd.backend import HipVecBackend

    return HipVecBackend(rom, num_envs=n, frames_per_step=kw.pop("fs", 24), release_after_frames=8,
                         stage="emulate_only", bootrom=boot, **kw)  # fmt: skip


@pytest.mark.parametrize("cart,fs", [("c3", 24), ("c3", 1), ("c5", 24)])
def test_frame_after_steps(carts, bootstub, cart, fs):
    require_gpu()
    n = 64
    rom = carts[cart]
    dut = _backend(rom, bootstub, n, fs=fs, render_bg=True)
    ref = RefMachine(n, rom, bootstub)
    try:
        dut.reset(seed=0)
        frames = []
        for k in range(4):
            act = seeded_actions(k + 1, k, n)
            dut.step(act)
            ref.step(act, fs, 8, "emulate_only", threads=8)
            np.testing.assert_array_equal(dut.export_latches(), ref.latches, err_msg=f"latches {k}")
            got = np.frombuffer(dut.read_frame_bg_shade_env0(), np.uint8).reshape(144, 160)
            want = ref.render_bg_env0()
            np.testing.assert_array_equal(got, want, err_msg=f"{cart} fs {fs} step {k}")
            frames.append(got)
        assert len({f.tobytes() for f in frames}) > 1 or fs == 1  # the scene moves
        assert np.unique(frames[-1]).size >= 2
    finally:
        dut.close()
        ref.close()


def test_frame_random_scenes(carts, bootstub):
    """Random VRAM, OAM and latches written into env 0 through the env image
    call; the frame must equal the oracle's for the same bytes."""
    require_gpu()
    rom = carts["c1"]
    dut = _backend(rom, bootstub, 3)
    ref = RefMachine(1, rom, bootstub)
    rng = np.random.default_rng(31)
    try:
        dut.reset(seed=0)
        for trial in range(6):
            img = dut.export_env(0)
            img.mem[0x8000:0xA000] = rng.integers(0, 256, 0x2000, dtype=np.uint8)
            oam = rng.integers(0, 256, 160, dtype=np.uint8)
            oam[0::4] = rng.integers(0, 176, 40)
            oam[1::4] = rng.integers(0, 176, 40)
            img.mem[0xFE00:0xFEA0] = oam
            lat = rng.integers(0, 256, (9, 144), dtype=np.uint8)
            lat[4] = rng.integers(0, 175, 144)
            lat[5] = rng.integers(0, 160, 144)
            if trial % 2:
                lat[0] = rng.integers(0, 256)
            img.latches = lat
            dut.import_env(0, img)
            dut.render_bg_env0()
            got = dut.frame_bg_torch().cpu().numpy()
            ref.mem[0] = img.mem
            ref.latches[:] = lat
            np.testing.assert_array_equal(got, ref.render_bg_env0(), err_msg=f"trial {trial}")
    finally:
        dut.close()
        ref.close()

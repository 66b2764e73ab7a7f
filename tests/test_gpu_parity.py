"""Bit-exact parity of the HIP step/render/reset kernels against the oracle.

Every config runs the same cartridge, boot image and seeded action trace on
the HIP backend and on the oracle, and compares after every step: all 32
per-env scalars (registers, flags, IME/HALT, timer, PPU, counters, traps), the
cart state, cart RAM, serial bytes, the full 64 KiB memory image per env, the
obs_v0/reward_v0 floats (bitwise) and the rendered pixels.
"""

from __future__ import annotations

import numpy as np
import pytest

from gbxcule_amd.carts.synth import seeded_actions
from oracle.ref import RefMachine

from ._parity import assert_same_state
from .conftest import require_gpu

pytestmark = pytest.mark.gpu

CASES = [
    # cart, envs, frameskip, steps, action seed, render
    ("c1", 64, 4, 24, 0, None),
    ("c2", 128, 24, 4, 1, None),
    ("c3", 96, 24, 4, 2, "packed"),
    ("c3", 64, 24, 3, 9, "unpacked"),
    ("c4", 64, 24, 4, 3, None),
    ("c4m3", 64, 24, 4, 4, None),
]


def _backend(rom, boot, n, fs, render):
    from gbxcule_amd.backend import HipVecBackend

    return HipVecBackend(
        rom,
        num_envs=n,
        frames_per_step=fs,
        release_after_frames=8,
        stage="full_step",
        render_pixels=render == "unpacked",
        render_pixels_packed=render == "packed",
        bootrom=boot,
    )


@pytest.mark.parametrize("cart,n,fs,steps,seed,render", CASES)
def test_step_parity(carts, bootstub, cart, n, fs, steps, seed, render):
    require_gpu()
    rom = carts[cart]
    dut = _backend(rom, bootstub, n, fs, render)
    ref = RefMachine(n, rom, bootstub)
    try:
        obs0, _ = dut.reset(seed=seed)
        ref.step(None, 0, 0, "full_step")  # the reset's 0-frame launch
        np.testing.assert_array_equal(obs0.view(np.uint32), ref.obs.view(np.uint32))
        assert_same_state(dut, ref, step=-1, tag=cart)
        for k in range(steps):
            act = seeded_actions(seed, k, n)
            obs, *_ = dut.step(act)
            ref.step(act, fs, 8, "full_step", threads=8)
            tag = f"{cart}/{render}"
            assert_same_state(dut, ref, step=k, tag=tag)
            np.testing.assert_array_equal(
                obs.view(np.uint32), ref.obs.view(np.uint32), err_msg=f"{tag} obs step {k}"
            )
            rew = dut.reward_torch().cpu().numpy()
            np.testing.assert_array_equal(rew.view(np.uint32), ref.reward.view(np.uint32))
            np.testing.assert_array_equal(dut.export_latches(), ref.latches)
            if render == "packed":
                ref.render(packed=True, threads=8)
                got = dut.pixels_packed_torch().cpu().numpy()
                np.testing.assert_array_equal(got, ref.pix_packed, err_msg=f"{tag} px {k}")
            elif render == "unpacked":
                ref.render(packed=False, threads=8)
                got = dut.pixels_torch().cpu().numpy()
                np.testing.assert_array_equal(got, ref.pix, err_msg=f"{tag} px {k}")
        # the trace must actually exercise the machine
        assert int(ref.field("instr_count").min()) > 0
        assert int(ref.field("trap_flag").sum()) == 0
    finally:
        dut.close()
        ref.close()


@pytest.mark.parametrize("cart,n", [("c5", 128), ("c4m3", 200)])
def test_masked_reset_and_senses_parity(carts, bootstub, cart, n):
    """C5 shape in miniature: snapshot at step 0, ~10% masked restores per
    step, unpacked pixels and a 32-byte RAM-sense gather every step (the
    MBC3 cart also restores its 32 KiB of cart RAM per env)."""
    require_gpu()
    import torch

    from gbxcule_amd.reset_cache import ResetCache

    rom = carts[cart]
    fs = 24
    dut = _backend(rom, bootstub, n, fs, "unpacked")
    ref = RefMachine(n, rom, bootstub)
    rng = np.random.default_rng(5)
    addrs = np.sort(rng.choice(np.arange(0xC000, 0xE000), 32, replace=False)).astype(np.int32)
    addrs[:4] = (0xFF40, 0xFF44, 0xFF0F, 0xFFFF)
    try:
        dut.reset(seed=0)
        ref.step(None, 0, 0, "full_step")
        dut.step(seeded_actions(5, 0, n))
        ref.step(seeded_actions(5, 0, n), fs, 8, "full_step", threads=8)
        ref.render(packed=False)
        cache = ResetCache.from_backend(dut, env_idx=0)
        ref.snapshot(0, with_pix=True)
        for k in range(1, 5):
            mask = (rng.random(n) < 0.1).astype(np.uint8)
            cache.apply_mask_torch(torch.from_numpy(mask).cuda().bool())
            ref.masked_reset(mask)
            assert_same_state(dut, ref, step=k, tag="c5-reset")
            np.testing.assert_array_equal(dut.pixels_torch().cpu().numpy(), ref.pix)
            act = seeded_actions(5, k, n)
            dut.step(act)
            ref.step(act, fs, 8, "full_step", threads=8)
            ref.render(packed=False)
            assert_same_state(dut, ref, step=k, tag="c5-step")
            np.testing.assert_array_equal(dut.pixels_torch().cpu().numpy(), ref.pix)
            senses = dut.ram_senses_torch(addrs).cpu().numpy()
            np.testing.assert_array_equal(senses, ref.mem[:, addrs])
    finally:
        dut.close()
        ref.close()


@pytest.mark.parametrize("route", ["write_memory", "memory_torch"])
def test_masked_reset_restores_rows_below_0x8000(carts, bootstub, route):
    """Rows below 0x8000 are skipped by the restore only while nothing but the
    power-on fill has written them; a write there (an import, or through the
    raw memory view) must make the next restore put them back."""
    require_gpu()
    import torch

    from gbxcule_amd.reset_cache import ResetCache

    n = 64
    dut = _backend(carts["c3"], bootstub, n, 4, None)
    try:
        dut.reset(seed=0)
        dut.step(seeded_actions(0, 0, n))
        cache = ResetCache.from_backend(dut, env_idx=0)
        want = dut.export_memory(0, 1)[0]
        if route == "write_memory":
            dut.write_memory(5, 0x1234, b"\xab\xcd")
        else:
            dut.memory_blocks_torch()[0, 0x1234, 5] = 0xAB
            torch.cuda.synchronize()
        assert dut.export_memory(5, 6, 0x1234, 0x1235)[0, 0] == 0xAB
        mask = np.zeros(n, dtype=np.uint8)
        mask[5] = 1
        cache.apply_mask_torch(torch.from_numpy(mask).cuda().bool())
        torch.cuda.synchronize()
        np.testing.assert_array_equal(dut.export_memory(5, 6)[0], want)
    finally:
        dut.close()

"""The 72x80 snapshot renderer on random scenes against the oracle.

Every env gets its own random VRAM, OAM and LCDC/scroll/window/palette
registers (8x8 and 8x16 sprites, both tile-data and tile-map selects, window
on and off, BG and sprites each enabled or not), with sprites crowded onto a
few lines so the 10-per-line limit, x-priority ties and BG-over-OBJ all come
up; the packed and unpacked outputs must equal the oracle's bytes.  The
larger env counts are rendered by workgroups that each take several groups
of envs in turn (one workgroup per CU), 4,056 with padding envs in its last
block.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle.ref import RefMachine

from .conftest import require_gpu

pytestmark = pytest.mark.gpu


def _scene(rng: np.random.Generator) -> dict[int, bytes]:
    vram = rng.integers(0, 256, 0x2000, dtype=np.uint8)
    oam = rng.integers(0, 256, 160, dtype=np.uint8)
    crowd = rng.random() < 0.5
    oam[0::4] = rng.integers(14, 40, 40) if crowd else rng.integers(0, 176, 40)
    xs = rng.integers(0, 176, 40)
    if crowd:  # equal x for some pairs: OAM order breaks the tie
        xs[1::5] = xs[0::5]
    oam[1::4] = xs
    io = rng.integers(0, 256, 12, dtype=np.uint8)  # FF40-FF4B
    io[0xA] = rng.integers(0, 150)  # WY
    io[0xB] = rng.integers(0, 175)  # WX
    return {0x8000: vram.tobytes(), 0xFE00: oam.tobytes(), 0xFF40: io.tobytes()}


@pytest.mark.parametrize("n,seed", [(200, 5), (64, 6), (256, 7), (4056, 8), (8192, 9)])
def test_snapshot_render_random_scenes(carts, bootstub, n, seed):
    require_gpu()
    import torch

    from gbxcule_amd.backend import HipVecBackend

    rom = carts["c1"]
    dut = HipVecBackend(rom, num_envs=n, frames_per_step=1, release_after_frames=1,
                        render_pixels=True, render_pixels_packed=True, render_on_step=False,
                        bootrom=bootstub)  # fmt: skip
    ref = RefMachine(n, rom, bootstub)
    rng = np.random.default_rng(seed)
    try:
        dut.reset(seed=0)
        ref.step(None, 0, 0, "full_step")
        for e in range(n):
            for addr, data in _scene(rng).items():
                dut.write_memory(e, addr, data)
                ref.mem[e, addr : addr + len(data)] = np.frombuffer(data, np.uint8)
        dut.render_pixels_snapshot()
        ref.render(packed=False, threads=8)
        np.testing.assert_array_equal(dut.pixels_torch().cpu().numpy(), ref.pix)
        ref.render(packed=True, threads=8)
        for off in (3, 4, 16):  # rows at byte, word and 16-byte alignment
            out = torch.zeros(n * 72 * 20 + off, dtype=torch.uint8, device="cuda")
            dut.render_pixels_snapshot_packed_to_torch(out, off)
            got = out[off:].cpu().numpy().reshape(n, 72, 20)
            np.testing.assert_array_equal(got, ref.pix_packed)
        assert np.unique(ref.pix).size == 4
    finally:
        dut.close()
        ref.close()


# LCDC per group of 8 envs (the envs a render workgroup takes together):
# BG through 9800 or 9C00 with 8000 tiles, BG and window on different maps,
# the signed 9000 tile data, BG off (sprites only), and groups mixing two
# settings.
LCDC_GROUPS = [
    (0x91,), (0x99,), (0xF3,), (0xB1,), (0xE3,), (0x83,), (0x90,), (0x02,),
    (0x91, 0x99), (0x93, 0x83), (0xF1, 0x90),
]


@pytest.mark.parametrize("n,seed", [(256, 11), (8192, 12)])
def test_snapshot_render_group_lcdc(carts, bootstub, n, seed):
    """Every group of 8 envs shares one LCDC pattern (random scenes give a
    group eight independent ones); VRAM everywhere is random."""
    require_gpu()
    from gbxcule_amd.backend import HipVecBackend

    rom = carts["c1"]
    dut = HipVecBackend(rom, num_envs=n, frames_per_step=1, release_after_frames=1,
                        render_pixels=True, render_pixels_packed=False, render_on_step=False,
                        bootrom=bootstub)  # fmt: skip
    ref = RefMachine(n, rom, bootstub)
    rng = np.random.default_rng(seed)
    try:
        dut.reset(seed=0)
        ref.step(None, 0, 0, "full_step")
        for e in range(n):
            scene = _scene(rng)
            pat = LCDC_GROUPS[(e // 8) % len(LCDC_GROUPS)]
            io = bytearray(scene[0xFF40])
            io[0] = pat[e % len(pat)]
            scene[0xFF40] = bytes(io)
            for addr, data in scene.items():
                dut.write_memory(e, addr, data)
                ref.mem[e, addr : addr + len(data)] = np.frombuffer(data, np.uint8)
        dut.render_pixels_snapshot()
        ref.render(packed=False, threads=8)
        np.testing.assert_array_equal(dut.pixels_torch().cpu().numpy(), ref.pix)
    finally:
        dut.close()
        ref.close()

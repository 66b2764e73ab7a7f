"""Memory access through ``memory_torch()`` and the rows-below-0x8000 rule of
the masked restore, on the GPU.

``memory_torch()`` must answer the reference's env-major indexing
(``backends/warp_vec.py:799-810``; the expressions below are those of
``rl/pokered_packed_parcel_env.py:277-291, 387-391``) with the shapes and
bytes that ``export_memory`` reads back, and writes through it must land in
the interleaved image.  The masked restore skips rows below 0x8000 while
every such row still holds the power-on fill; savestate loads that leave them
so must keep the skip, and anything that changes them must end it.  OAM DMA
from a page below 0x80 reads those rows, so the oracle comparison after a
restore and a DMA sees any row the restore should have put back.
"""

from __future__ import annotations

import numpy as np
import pytest

from gbxcule_amd.carts.asm import Asm
from gbxcule_amd.carts.synth import PROGRAM_ORIGIN, _vectors, finalize_rom, seeded_actions
from oracle.ref import RefMachine

from ._parity import assert_same_state, ref_export_env, ref_import_env
from .conftest import require_gpu

pytestmark = pytest.mark.gpu

EVENTS_START, EVENTS_LENGTH = 0xD747, 320
MAP_ID_ADDR, PLAYER_X_ADDR, PLAYER_Y_ADDR = 0xD35E, 0xD362, 0xD361


def _backend(rom, boot, n, fs=4, render=None):
    from gbxcule_amd.backend import HipVecBackend

    return HipVecBackend(
        rom, num_envs=n, frames_per_step=fs, release_after_frames=8, stage="full_step",
        render_pixels=render == "unpacked", bootrom=boot,
    )  # fmt: skip


def test_reference_indexing_matches_export(carts, bootstub):
    require_gpu()
    import torch

    n = 100  # two memory blocks, the second partly padding
    dut = _backend(carts["c3"], bootstub, n)
    try:
        dut.reset(seed=0)
        for k in range(2):
            dut.step(seeded_actions(2, k, n))
        want = dut.export_memory()
        mem = dut.memory_torch()
        assert isinstance(mem, torch.Tensor) and mem.dtype is torch.uint8
        assert tuple(mem.shape) == (n, 65536) and mem.ndim == 2 and mem.is_cuda
        events = mem[:, EVENTS_START : EVENTS_START + EVENTS_LENGTH]
        map_id, x, y = mem[:, MAP_ID_ADDR], mem[:, PLAYER_X_ADDR], mem[:, PLAYER_Y_ADDR]
        assert events.shape == (n, EVENTS_LENGTH) and map_id.shape == (n,)
        np.testing.assert_array_equal(events.cpu().numpy(), want[:, EVENTS_START : EVENTS_START + EVENTS_LENGTH])
        for t, a in ((map_id, MAP_ID_ADDR), (x, PLAYER_X_ADDR), (y, PLAYER_Y_ADDR)):
            np.testing.assert_array_equal(t.cpu().numpy(), want[:, a])
        np.testing.assert_array_equal(mem[:, MAP_ID_ADDR].float().cpu().numpy(), want[:, MAP_ID_ADDR].astype(np.float32))
        assert int(mem[0, MAP_ID_ADDR].item()) == int(want[0, MAP_ID_ADDR])
        np.testing.assert_array_equal(mem[73, 0x8000:0x9800].cpu().numpy(), want[73, 0x8000:0x9800])
        np.testing.assert_array_equal(mem[70:90, 0xFF00:].cpu().numpy(), want[70:90, 0xFF00:])
        np.testing.assert_array_equal(mem.clone().cpu().numpy(), want)  # whole image, env-major
        np.testing.assert_array_equal(dut.read_memory_torch(99, 0xC000, 0xC100).cpu().numpy(), want[99, 0xC000:0xC100])
        # writes: the LCDC override expression, a block of one env, a column
        mem[:, 0xFF40] |= 0x80
        want[:, 0xFF40] |= 0x80
        blob = np.random.default_rng(0).integers(0, 256, (n, 16), dtype=np.uint8)
        mem[:, 0xC100:0xC110] = torch.from_numpy(blob).cuda()
        want[:, 0xC100:0xC110] = blob
        mem[65, 0xDF00:0xDF08] = 0x5A
        want[65, 0xDF00:0xDF08] = 0x5A
        torch.cuda.synchronize()
        np.testing.assert_array_equal(dut.export_memory(), want)
    finally:
        dut.close()


def dma_cart() -> bytes:
    """ROM-only cart that, every frame, runs OAM DMA from page 0x00 (the boot
    image rows of memory), page 0x01, page 0xA0 (cartridge-RAM rows, which a
    cart without RAM never writes) and page 0xE1 (echo rows, whose writes fold
    to work RAM), and copies OAM bytes to WRAM."""
    a = Asm(origin=PROGRAM_ORIGIN)
    a.ld_rr_d16("SP", 0xDFF0)
    a.ld_r_d8("A", 0x91)
    a.ldh_a8_a(0x40)
    a.label("loop")
    a.label("w1")
    a.ldh_a_a8(0x44)
    a.alu_d8("CP", 144)
    a.jr("w1", "NZ")
    for i, page in enumerate((0x00, 0x01, 0xA0, 0xE1)):
        a.ld_r_d8("A", page)
        a.ldh_a8_a(0x46)
        a.ld_r_d8("A", 0xFF)  # a few cycles between transfers
        a.label(f"w{i + 2}")
        a.ldh_a_a8(0x44)
        a.alu_d8("CP", 145 + i)
        a.jr(f"w{i + 2}", "NZ")
        a.ld_a_a16(0xFE00 + 3 * i)
        a.ld_a16_a(0xC000 + i)
    a.jp("loop")
    rom = bytearray(0x8000)
    _vectors(rom)
    code = a.resolve()
    rom[PROGRAM_ORIGIN : PROGRAM_ORIGIN + len(code)] = code
    return finalize_rom(rom, "DMALOW", 0x00, 0x00, 0x00)


@pytest.mark.parametrize(
    "route",
    [
        "load_state",
        "load_state_low_rows",
        "load_state_cart_ram_rows",
        "load_state_echo_rows",
        "memory_torch",
        "memory_torch_cart_ram_rows",
        "memory_torch_echo_rows",
        "memory_blocks_torch",
    ],
)
def test_dead_rows_restored_exactly_when_changed(bootstub, route):
    """Rows the step never writes (below 0x8000, A000-BFFF, E000-FDFF) are
    skipped by masked resets until a route may have changed them; every route
    that can must make the restore cover them again."""
    require_gpu()
    import torch

    from gbxcule_amd.reset_cache import ResetCache

    n, fs = 64, 2
    rom = dma_cart()
    dut = _backend(rom, bootstub, n, fs)
    ref = RefMachine(n, rom, bootstub)
    try:
        dut.reset(seed=0)
        ref.step(None, 0, 0, "full_step")
        for k in range(2):
            act = seeded_actions(7, k, n)
            dut.step(act)
            ref.step(act, fs, 8, "full_step")
        cache = ResetCache.from_backend(dut, env_idx=0)
        ref.snapshot(0)
        # change env 5 by the route under test, on both machines
        if route.startswith("load_state"):
            img = dut.export_env(9)
            np.testing.assert_array_equal(img.mem, ref_export_env(ref, 9).mem)
            if route == "load_state_low_rows":
                img.mem[0x00:0x40] ^= 0xA5  # boot-image rows, read by the page-0 DMA
            elif route == "load_state_cart_ram_rows":
                img.mem[0xA000:0xA040] ^= 0x5A  # read by the page-0xA0 DMA
            elif route == "load_state_echo_rows":
                img.mem[0xE100:0xE140] ^= 0x3C  # read by the page-0xE1 DMA
            dut.import_env(5, img)
            ref_import_env(ref, 5, img)
        elif route.startswith("memory_torch"):
            lo = {"memory_torch": 0x0010, "memory_torch_cart_ram_rows": 0xA010, "memory_torch_echo_rows": 0xE110}[route]
            dut.memory_torch()[5, lo : lo + 0x10] = 0x77
            ref.mem[5, lo : lo + 0x10] = 0x77
        else:
            blocks = dut.memory_blocks_torch()
            blocks[0, 0x0030, 5] = 0x66
            ref.mem[5, 0x0030] = 0x66
        torch.cuda.synchronize()
        assert_same_state(dut, ref, step=2, tag=route)
        mask = np.zeros(n, dtype=np.uint8)
        mask[[3, 5, 40]] = 1
        cache.apply_mask_torch(torch.from_numpy(mask).cuda().bool())
        ref.masked_reset(mask)
        assert_same_state(dut, ref, step=3, tag=f"{route} restore")
        for k in range(3, 6):  # the DMAs read rows 0x0000-0x019F, 0xA000-0xA09F, 0xE100-0xE19F
            act = seeded_actions(7, k, n)
            dut.step(act)
            ref.step(act, fs, 8, "full_step")
            assert_same_state(dut, ref, step=k, tag=f"{route} dma")
    finally:
        dut.close()
        ref.close()


def test_ram_senses_address_lists(carts, bootstub):
    """``ram_senses_torch`` keeps the last host address list on the device;
    a changed list, a list changed in place, a repeated one and a device
    tensor must each read the bytes ``export_memory`` returns, and a 16-byte
    multiple of senses (the 16-byte store path) and an odd count (the byte
    path) both."""
    require_gpu()
    import torch

    n = 130  # three memory blocks, the last partly padding
    dut = _backend(carts["c3"], bootstub, n)
    try:
        dut.reset(seed=0)
        for k in range(2):
            dut.step(seeded_actions(3, k, n))
        mem = dut.export_memory()
        rng = np.random.default_rng(5)
        a = np.sort(rng.choice(np.arange(0x8000, 0x10000), 32, replace=False))
        b = np.sort(rng.choice(np.arange(0xC000, 0xE000), 7, replace=False))
        c = a.copy()
        for addrs in (a, b, a, c, torch.as_tensor(b.astype(np.int32), device="cuda")):
            got = dut.ram_senses_torch(addrs).cpu().numpy()
            want = mem[:, np.asarray(addrs.cpu() if isinstance(addrs, torch.Tensor) else addrs)]
            np.testing.assert_array_equal(got, want)
        c[3] ^= 0x0100  # the same array object, changed in place
        np.testing.assert_array_equal(dut.ram_senses_torch(c).cpu().numpy(), mem[:, c])
    finally:
        dut.close()

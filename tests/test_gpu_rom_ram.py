"""A ROM-only cart (type 0x00) whose header declares 8 KiB of RAM, against
the oracle.

Such a cart has no MBC to enable its RAM, so only an imported cart state
(RAM enable set) reaches it; the reference then reads and writes cartridge
RAM bank 0 at A000-BFFF (core/cartridge.py's read8/write8 path for cart RAM,
restated in oracle/gbx_ref.cpp).  Half the envs get RAM enabled and half not
(reads 0xFF, writes dropped).  The program reads, increments and writes back
random cart-RAM bytes, also through LD A,(a16) and 16-bit POPs, and copies
what it read into work RAM; state, cart RAM included, is compared in full
after every step.
"""

from __future__ import annotations

import numpy as np
import pytest

from gbxcule_amd.abi import CART_STATE_INDEX
from gbxcule_amd.carts.asm import Asm
from gbxcule_amd.carts.synth import PROGRAM_ORIGIN, _vectors, finalize_rom, seeded_actions
from oracle.ref import RefMachine

from ._isa import CS_BOOT
from ._parity import assert_same_state
from .conftest import require_gpu

pytestmark = pytest.mark.gpu


def rom_ram_cart(seed: int) -> bytes:
    rng = np.random.default_rng(seed)
    rom = bytearray(0x8000)
    _vectors(rom)
    a = Asm(origin=PROGRAM_ORIGIN)
    a.ld_rr_d16("SP", 0xDFF0)
    a.label("loop")
    for i in range(10):
        addr = 0xBFFF if i == 0 else int(rng.integers(0xA000, 0xC000))
        a.ld_rr_d16("HL", addr)
        a.emit(0x7E)  # LD A,(HL)
        a.alu_d8("ADD", int(rng.integers(1, 256)))
        a.emit(0x77)  # LD (HL),A
        a.ld_a_a16(addr)  # read back through LD A,(a16)
        a.ld_a16_a(0xC000 + i)
    # a 16-bit read from cart RAM through the stack
    a.ld_rr_d16("HL", 0)
    a.add_hl_rr("SP")
    a.ld_rr_d16("SP", int(rng.integers(0xA000, 0xBFFE)))
    a.pop("BC")
    a.ld_sp_hl()
    a.ld_r_r("A", "B")
    a.ld_a16_a(0xC010)
    a.ld_r_r("A", "C")
    a.ld_a16_a(0xC011)
    a.jp("loop")
    code = a.resolve()
    rom[PROGRAM_ORIGIN : PROGRAM_ORIGIN + len(code)] = code
    return finalize_rom(rom, "GBXAMD ROMRAM", 0x00, 0x00, 0x02)


def test_rom_only_cart_ram_parity(bootstub):
    require_gpu()
    from gbxcule_amd.backend import HipVecBackend

    rom = rom_ram_cart(31)
    n, fs, steps = 128, 2, 4
    dut = HipVecBackend(rom, num_envs=n, frames_per_step=fs, release_after_frames=1,
                        stage="emulate_only", bootrom=bootstub)  # fmt: skip
    ref = RefMachine(n, rom, bootstub)
    try:
        dut.reset(seed=0)
        ref.step(None, 0, 0, "emulate_only")
        # boot overlay off, PC at the program, RAM enabled in every other env
        cs = dut.export_cart_state()
        cs[:, CS_BOOT] = 0
        cs[::2, CART_STATE_INDEX["ram_enable"]] = 1
        dut.import_cart_state(cs)
        ref.cart_state[:] = cs
        pc = np.full(n, PROGRAM_ORIGIN, np.int64)
        dut.import_field("pc", pc)
        ref.field("pc")[:] = pc
        assert_same_state(dut, ref, step=-1, tag="romram")
        for k in range(steps):
            act = seeded_actions(31, k, n)
            dut.step(act)
            ref.step(act, fs, 1, "emulate_only", threads=8)
            assert_same_state(dut, ref, step=k, tag="romram")
        cr = ref.cart_ram.reshape(n, -1)
        assert cr[0].any() and not cr[1].any()  # enabled envs wrote, disabled ones did not
        assert int(ref.field("trap_flag").sum()) == 0
    finally:
        dut.close()
        ref.close()

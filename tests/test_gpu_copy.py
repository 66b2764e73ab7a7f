"""Block-copy loops (LD A,(HL+); LD (DE),A; INC DE; DEC BC; LD A,B; OR C;
JR NZ) against the oracle.

The step kernel runs whole passes of such a loop as one step, up to the next
scanline (or STAT mode boundary with the HBlank source on), TIMA overflow,
frame end or interrupt service, and only while source and destination stay
inside one ROM bank window, video RAM or work RAM.  These carts copy from
both ROM windows (MBC1 banks switched by the joypad), video and work RAM,
with overlapping ranges in both directions, ranges that run out of their
window, destinations that are never batched (HRAM, OAM), joypad-dependent
lengths, interrupts with IME on and off, and the LCD switched off; state is
compared in full after every step.
"""

from __future__ import annotations

import numpy as np
import pytest

from gbxcule_amd.carts.asm import Asm
from gbxcule_amd.carts.synth import PROGRAM_ORIGIN, _vectors, finalize_rom, seeded_actions
from oracle.ref import RefMachine

from ._isa import CS_BOOT
from ._parity import assert_same_state
from .conftest import require_gpu

pytestmark = pytest.mark.gpu


def _copy(a: Asm, src: int, dst: int, count: int | None, tag: str, c_first: bool = False) -> None:
    """HL=src, DE=dst, BC=count (None: BC already set); the copy loop."""
    a.ld_rr_d16("HL", src)
    a.ld_rr_d16("DE", dst)
    if count is not None:
        a.ld_rr_d16("BC", count)
    a.label(tag)
    a.ld_a_hli()
    a.ld_de_a()
    a.inc_rr("DE")
    a.dec_rr("BC")
    if c_first:
        a.ld_r_r("A", "C")
        a.alu_r("OR", "B")
    else:
        a.ld_r_r("A", "B")
        a.alu_r("OR", "C")
    a.jr(tag, "NZ")


def copy_cart(seed: int, ime: bool, ie: int, tac: int, stat: int, lcd_off: bool, mbc1: bool) -> bytes:
    """A ROM-only (32 KiB) or MBC1 (64 KiB) cart whose main loop copies
    between every window kind."""
    rng = np.random.default_rng(seed)
    size = 0x10000 if mbc1 else 0x8000
    rom = bytearray(size)
    rom[0x1000:0x4000] = rng.integers(0, 256, 0x3000, dtype=np.uint8).tobytes()
    rom[0x4000:size] = rng.integers(0, 256, size - 0x4000, dtype=np.uint8).tobytes()
    h = Asm(origin=0x0068)
    for name, counter in (("vbl", 0xDF00), ("stat", 0xDF01), ("timer", 0xDF02)):
        h.label(name)
        h.push("AF")
        h.push("HL")
        h.ld_rr_d16("HL", counter)
        h.emit(0x34)  # INC (HL)
        h.pop("HL")
        h.pop("AF")
        h.reti()
    code = h.resolve()
    rom[0x68 : 0x68 + len(code)] = code
    _vectors(rom, {0x40: h.labels["vbl"], 0x48: h.labels["stat"], 0x50: h.labels["timer"]})

    r = lambda lo, hi: int(rng.integers(lo, hi))  # noqa: E731
    a = Asm(origin=PROGRAM_ORIGIN)
    a.ld_rr_d16("SP", 0xDFF0)
    a.ld_r_d8("A", r(0, 256))
    a.ldh_a8_a(0x06)  # TMA
    a.ld_r_d8("A", tac)
    a.ldh_a8_a(0x07)  # TAC
    a.ld_r_d8("A", r(0, 154))
    a.ldh_a8_a(0x45)  # LYC
    a.ld_r_d8("A", stat)
    a.ldh_a8_a(0x41)  # STAT interrupt sources
    a.ld_r_d8("A", ie)
    a.ldh_a8_a(0xFF)
    a.ld_r_d8("A", 0x00)
    a.ldh_a8_a(0x0F)
    if ime:
        a.ei()
    a.ld_r_d8("A", 0x91)
    a.ldh_a8_a(0x40)  # LCD on
    a.label("loop")
    # joypad nibble: the ROM bank (MBC1) and the first copy's length
    a.ld_r_d8("A", 0x10)
    a.ldh_a8_a(0x00)
    a.ldh_a_a8(0x00)
    a.alu_d8("AND", 0x0F)
    if mbc1:
        a.ld_a16_a(0x2000)  # bank 1-3 (0 selects 1), from the low bits
    a.alu_d8("ADD", 16)
    a.ld_r_r("C", "A")
    a.ld_r_d8("B", 0)
    _copy(a, 0x4000 + r(0, 0x3000), 0x8000 + r(0, 0x1000), None, "c_romx_vram")
    _copy(a, 0x1000 + r(0, 0x2000), 0xC000 + r(0x1000, 0x1800), r(50, 300), "c_rom0_wram", c_first=True)
    _copy(a, 0xC000, 0xC003, 200, "c_fwd_overlap")
    _copy(a, 0xC400, 0xC3FD, 200, "c_back_overlap")
    _copy(a, 0xC500, 0xC500, 64, "c_same")
    _copy(a, 0x8100, 0xD000, 300, "c_vram_wram", c_first=True)
    _copy(a, 0x3FF0, 0xD800, 64, "c_rom0_edge")  # source runs into the bank window
    _copy(a, 0xC800, 0x9FF0, 40, "c_vram_edge")  # destination runs into cart RAM
    _copy(a, 0x9FF8, 0xD400, 24, "c_src_edge")  # source runs into cart RAM (reads 0xFF)
    _copy(a, 0xC900, 0xFF80, 16, "c_hram")  # HRAM: never batched
    _copy(a, 0xC900, 0xFE00, 32, "c_oam")  # OAM: never batched
    _copy(a, 0xDE00, 0xDE01, 1, "c_one")  # one pass: nothing to batch
    a.ld_a_a16(0xDE80)
    a.inc_r("A")
    a.ld_a16_a(0xDE80)
    if lcd_off:
        a.alu_d8("AND", 0x03)
        a.jr("loop_end", "NZ")
        a.ld_r_d8("A", 0x11)
        a.ldh_a8_a(0x40)  # LCD off: no scanline bounds the batches
        _copy(a, 0x4000, 0x8000, 0x1800, "c_lcd_off")
        a.ld_r_d8("A", 0x91)
        a.ldh_a8_a(0x40)
        a.label("loop_end")
    a.jp("loop")
    code = a.resolve()
    rom[PROGRAM_ORIGIN : PROGRAM_ORIGIN + len(code)] = code
    assert PROGRAM_ORIGIN + len(code) < 0x1000
    return finalize_rom(rom, "GBXAMD COPY", 0x01 if mbc1 else 0x00, 0x01 if mbc1 else 0x00, 0x00)


CASES = [
    # seed, IME, IE, TAC, STAT sources, LCD-off phases, MBC1
    (1, True, 0x04, 0x05, 0x40, False, False),
    (2, True, 0x03, 0x04, 0x40, True, False),
    (3, False, 0x07, 0x06, 0x08, False, True),
    (4, True, 0x02, 0x00, 0x08, False, False),
    (5, True, 0x05, 0x07, 0x10, True, True),
    (6, False, 0x00, 0x05, 0x00, True, False),
]


@pytest.mark.parametrize("seed,ime,ie,tac,stat,lcd_off,mbc1", CASES)
def test_copy_loop_parity(bootstub, seed, ime, ie, tac, stat, lcd_off, mbc1):
    require_gpu()
    from gbxcule_amd.backend import HipVecBackend

    rom = copy_cart(seed, ime, ie, tac, stat, lcd_off, mbc1)
    n, fs, steps = 64, 24, 4
    dut = HipVecBackend(rom, num_envs=n, frames_per_step=fs, release_after_frames=8,
                        stage="emulate_only", bootrom=bootstub)  # fmt: skip
    ref = RefMachine(n, rom, bootstub)
    try:
        dut.reset(seed=seed)
        ref.step(None, 0, 0, "emulate_only")
        assert_same_state(dut, ref, step=-1, tag=f"copy{seed}")
        for k in range(steps):
            act = seeded_actions(seed, k, n)
            dut.step(act)
            ref.step(act, fs, 8, "emulate_only", threads=8)
            assert_same_state(dut, ref, step=k, tag=f"copy{seed}")
        mem = ref.mem
        assert int(mem[0, 0xDE80]) > 0  # the loop completed
        if ime and ie & 4 and tac & 4:
            assert int(mem[0, 0xDF02]) > 0  # timer interrupts were serviced
        if ime and ie & 2 and stat & 0x08:
            assert int(mem[0, 0xDF01]) > 0  # HBlank STAT interrupts were serviced
        assert int(ref.field("trap_flag").sum()) == 0
    finally:
        dut.close()
        ref.close()


def test_copy_loop_under_boot_overlay():
    """A boot image that hands over without unmapping itself: the cart's
    copy loops read 0x0000-0x0107 through the overlay (the boot image, then
    the cart past 0x00FF), which is never batched, and then unmap it."""
    require_gpu()
    from gbxcule_amd.backend import HipVecBackend

    boot_asm = Asm(origin=0x0000)
    boot_asm.ld_rr_d16("SP", 0xFFFE)
    boot_asm.jp(0x0100)
    boot = bytearray(boot_asm.resolve())
    boot.extend(bytes((0x40 + i) & 0xFF for i in range(0x100 - len(boot))))  # read through the overlay
    rng = np.random.default_rng(11)
    rom = bytearray(0x8000)
    rom[0x0000:0x0100] = rng.integers(0, 256, 0x100, dtype=np.uint8).tobytes()  # hidden while mapped
    rom[0x1000:0x4000] = rng.integers(0, 256, 0x3000, dtype=np.uint8).tobytes()
    a = Asm(origin=PROGRAM_ORIGIN)
    a.ld_rr_d16("SP", 0xDFF0)
    a.label("loop")
    _copy(a, 0x0000, 0xC000, 0x108, "c_boot")  # boot image, then cart bytes
    _copy(a, 0x00F0, 0xC200, 0x40, "c_edge")
    _copy(a, 0x1000, 0xC400, 0x200, "c_rom")
    a.ld_a_a16(0xDE80)
    a.inc_r("A")
    a.ld_a16_a(0xDE80)
    a.alu_d8("AND", 0x07)
    a.jr("loop", "NZ")
    a.ld_r_d8("A", 0x01)
    a.ldh_a8_a(0x50)  # unmap the boot image; later passes read the cart
    a.jp("loop")
    code = a.resolve()
    rom[PROGRAM_ORIGIN : PROGRAM_ORIGIN + len(code)] = code
    rom = finalize_rom(rom, "GBXAMD BOOTCP", 0x00, 0x00, 0x00)
    n, fs = 64, 24
    dut = HipVecBackend(rom, num_envs=n, frames_per_step=fs, release_after_frames=8,
                        stage="emulate_only", bootrom=bytes(boot))  # fmt: skip
    ref = RefMachine(n, rom, bytes(boot))
    try:
        dut.reset(seed=11)
        ref.step(None, 0, 0, "emulate_only")
        for k in range(3):
            act = seeded_actions(11, k, n)
            dut.step(act)
            ref.step(act, fs, 8, "emulate_only", threads=8)
            assert_same_state(dut, ref, step=k, tag="bootcopy")
        assert int(ref.mem[0, 0xDE80]) > 8  # ran before and after the unmap
        assert int(ref.cart_state[0, CS_BOOT]) == 0
    finally:
        dut.close()
        ref.close()

"""Known answers for the STAT interrupt sources and for the frame accounting
of LCD switches.

STAT (``kernels/cpu_step_builder.py:435-492`` with the line-change block
``1406-1500``).  The reference evaluates STAT request edges only at scanline
changes, where the current bits are mode 0 (LY < 144) or mode 1 (LY >= 144)
plus LY == LYC, against the bits left by the end of the previous instruction.
Every instruction is at most 24 cycles, so the last instruction of a line
ends at scanline cycle >= 432, in mode 0 for lines 0-143 and mode 1 for lines
144-153.  That fixes the steady state in closed form, per source:

* VBlank (STAT bit 4): the change into line 144, once a frame;
* LYC (bit 6): the change into line LYC when LYC < 154, once a frame;
* HBlank (bit 3): only the change 153 -> 0, where mode 1 becomes mode 0;
* OAM (bit 5): never (mode 2 is never current at a change);
* sources that fire at the same change raise one request.

So requests per frame = |{144 if VBlank} U {LYC if LYC and LYC < 154} U
{0 if HBlank}|.  A STAT handler counts them in work RAM for every one of the
16 source masks and several LYC values.

LCD switches (``cpu_step_builder.py:1283-1300, 1706-1758``): switching the
LCD off counts a frame and restarts the frame count at the switching step's
cycles (interrupt service included), minus 4 when the step was
``LDH (40),A``; a halted CPU whose interrupt push switches it off restarts it
at 0; switching it on counts a frame, restarts the count at 0 and puts the
PPU at line 0, cycle 0, mode 2.  The cases below compute the expected
counters by hand from those rules and the public cycle table.
"""

from __future__ import annotations

import numpy as np
import pytest

from ._isa import flat_rom, oracle, set_regs

STAT_MASKS = list(range(16))  # bit 0 HBlank, 1 VBlank, 2 OAM, 3 LYC -> STAT bits 3-6
LYCS = [0, 1, 77, 143, 144, 145, 153, 154, 255]


def requests_per_frame(mask: int, lyc: int) -> int:
    lines = set()
    if mask & 2:
        lines.add(144)
    if mask & 8 and lyc < 154:
        lines.add(lyc)
    if mask & 1:
        lines.add(0)
    return len(lines)


def _stat_rom() -> bytes:
    main = bytes([
        0x00,              # NOP            4
        0x06, 0x12,        # LD B,0x12      8
        0x11, 0x34, 0x12,  # LD DE,0x1234  12
        0xFA, 0x00, 0xD0,  # LD A,(D000)   16
        0xC5,              # PUSH BC       16
        0xC1,              # POP BC        12
        0x18, 0xF4,        # JR -12 (to the NOP)
    ])  # fmt: skip
    return flat_rom({0x48: bytes([0x34, 0xD9]), 0x150: main})  # INC (HL); RETI


def test_stat_requests_per_frame_closed_form():
    cases = [(m, lyc) for m in STAT_MASKS for lyc in LYCS]
    n = len(cases)
    m = oracle(_stat_rom(), n, pc=0x150)
    try:
        set_regs(m, h=0xC0, l=0x00, sp=0xDFF0, ime=1)
        m.mem[:, 0xFF40] = 0x91
        m.mem[:, 0xFF41] = [(mask << 3) for mask, _ in cases]
        m.mem[:, 0xFF45] = [lyc for _, lyc in cases]
        m.mem[:, 0xFFFF] = 0x02
        m.mem[:, 0xFF0F] = 0x00
        m.step(None, frames=2)  # settle
        c0 = m.mem[:, 0xC000].astype(int)
        frames = 4
        m.step(None, frames=frames)
        got = (m.mem[:, 0xC000].astype(int) - c0) % 256
        want = np.array([frames * requests_per_frame(mask, lyc) for mask, lyc in cases])
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, [(cases[i], int(got[i]), int(want[i])) for i in bad[:6]]
        assert int(m.field("trap_flag").sum()) == 0
    finally:
        m.close()


def _lcd_case(code: bytes, *, lcdc: int, ly: int = 0, scan: int = 0, cframe: int = 0, **regs):
    """One env at 0x150 running ``code``; returns the machine after a one-frame
    launch (which the LCD switch ends)."""
    rom = flat_rom({0x150: code, 0x50: bytes([0xD9])})
    m = oracle(rom, 1, pc=0x150)
    m.mem[0, 0xFF40] = lcdc
    m.mem[0, 0xFF44] = ly
    set_regs(m, ppu_ly=ly, ppu_scanline_cycle=scan, cycle_in_frame=cframe, sp=0xDFF0, **regs)
    m.step(None, frames=1)
    return m


@pytest.mark.parametrize(
    "code,tail,cycles",
    [
        (bytes([0x3E, 0x11, 0xE0, 0x40]), 12 - 4, 8 + 12),        # LD A,11; LDH (40),A
        (bytes([0x3E, 0x11, 0xEA, 0x40, 0xFF]), 16, 8 + 16),      # LD A,11; LD (FF40),A
        (bytes([0x3E, 0x11, 0x77]), 8, 8 + 8),                    # LD A,11; LD (HL),A, HL=FF40
        (bytes([0x3E, 0x11, 0xE2]), 8, 8 + 8),                    # LD A,11; LD (C),A, C=40
    ],
)  # fmt: skip
def test_lcd_off_counts_a_frame_and_restarts_at_the_step_tail(code, tail, cycles):
    m = _lcd_case(code, lcdc=0x91, ly=2, scan=88, cframe=2 * 456 + 88, h=0xFF, l=0x40, c=0x40)
    try:
        st = m.scalars()
        assert int(st["cycle_count"][0]) == cycles  # the launch ended at the switch
        assert int(st["instr_count"][0]) == 2
        assert int(st["cycle_in_frame"][0]) == tail
        assert int(st["pc"][0]) == 0x150 + len(code)
        assert (int(st["ppu_ly"][0]), int(st["ppu_scanline_cycle"][0])) == (0, 0)
        assert int(m.mem[0, 0xFF44]) == 0
    finally:
        m.close()


def test_lcd_off_by_ldh_with_interrupt_service_in_the_same_step():
    """TIMA (TAC 0x05: DIV bit 3, 16-cycle period) overflows 4 cycles into the
    LDH and reloads 4 cycles later, so the timer interrupt is serviced in the
    step that switches the LCD off: 12 + 20 cycles, tail 32 - 4 = 28.  The
    service's 20 cycles take DIV from 24 to 44, one more TIMA edge (at 32)."""
    code = bytes([0x3E, 0x11, 0xE0, 0x40])
    rom = flat_rom({0x150: code, 0x50: bytes([0xD9])})
    m = oracle(rom, 1, pc=0x150)
    try:
        m.mem[0, 0xFF40] = 0x91
        m.mem[0, 0xFF05], m.mem[0, 0xFF06], m.mem[0, 0xFF07] = 0xFF, 0x42, 0x05
        m.mem[0, 0xFFFF] = 0x04
        set_regs(m, ppu_ly=2, ppu_scanline_cycle=88, cycle_in_frame=2 * 456 + 88, sp=0xDFF0, ime=1,
                 div_counter=4)  # fmt: skip
        m.step(None, frames=1)
        st = m.scalars()
        assert int(st["pc"][0]) == 0x50 and int(st["sp"][0]) == 0xDFEE
        assert (int(m.mem[0, 0xDFEF]), int(m.mem[0, 0xDFEE])) == (0x01, 0x54)
        assert int(st["cycle_in_frame"][0]) == 28
        assert int(st["cycle_count"][0]) == 8 + 12 + 20
        assert int(st["div_counter"][0]) == 44
        assert int(m.mem[0, 0xFF05]) == 0x43
        assert int(m.mem[0, 0xFF0F]) & 0x04 == 0 and int(st["ime"][0]) == 0
    finally:
        m.close()


def test_halted_push_switching_lcd_off_restarts_frame_at_zero():
    """A halted CPU wakes on a pending VBlank request with IME set; the push
    of PC = 0x0123 with SP = 0xFF42 writes 0x01 to STAT and 0x23 to LCDC,
    switching the LCD off inside the halted step (4 cycles + 20 service)."""
    rom = flat_rom({0x40: bytes([0xD9])})
    m = oracle(rom, 1, pc=0x0123)
    try:
        m.mem[0, 0xFF40] = 0x91
        m.mem[0, 0xFFFF] = 0x01
        m.mem[0, 0xFF0F] = 0x01
        set_regs(m, halted=1, ime=1, sp=0xFF42, ppu_ly=50, ppu_scanline_cycle=100,
                 cycle_in_frame=50 * 456 + 100)  # fmt: skip
        m.step(None, frames=1)
        st = m.scalars()
        assert int(st["cycle_in_frame"][0]) == 0
        assert int(st["cycle_count"][0]) == 4 + 20
        assert int(st["instr_count"][0]) == 0
        assert (int(st["pc"][0]), int(st["sp"][0])) == (0x40, 0xFF40)
        assert int(m.mem[0, 0xFF40]) == 0x23
        assert (int(st["halted"][0]), int(st["ime"][0])) == (0, 0)
        assert int(m.mem[0, 0xFF0F]) & 0x01 == 0
    finally:
        m.close()


@pytest.mark.parametrize("lyc", [0, 7])
def test_lcd_on_counts_a_frame_and_starts_line_0_mode_2(lyc):
    rom = flat_rom({0x150: bytes([0x3E, 0x91, 0xE0, 0x40])})
    m = oracle(rom, 1, pc=0x150)
    try:
        m.mem[0, 0xFF40] = 0x11
        m.mem[0, 0xFF45] = lyc
        set_regs(m, cycle_in_frame=5000, sp=0xDFF0)
        m.step(None, frames=1)
        st = m.scalars()
        assert int(st["cycle_in_frame"][0]) == 0
        assert int(st["cycle_count"][0]) == 8 + 12
        assert int(st["pc"][0]) == 0x154
        assert (int(st["ppu_ly"][0]), int(st["ppu_scanline_cycle"][0])) == (0, 0)
        coin = 1 if lyc == 0 else 0
        assert int(st["ppu_stat_prev"][0]) == 0x04 | (coin << 3)
        assert int(m.mem[0, 0xFF41]) & 0x07 == 2 | (coin << 2)
    finally:
        m.close()


def test_obs_mix_slots_28_to_31_known_values():
    """obs_v0 slots 26-31 (``cpu_templates/post_step.py:92-102``): byte mixes
    of C000-C007 with A, B, C, D, each wrapped to 8 bits and divided by 255."""
    rom = flat_rom({0x150: bytes([0x00])})
    m = oracle(rom, 3, pc=0x150)
    try:
        mem = np.array([
            [0x0F, 0xF0, 0x10, 0x20, 0x0F, 0xF0, 0xAA, 0x80],
            [0x00, 0x00, 0xFF, 0xFF, 0xFF, 0x01, 0x55, 0xFF],
            [0x12, 0x34, 0x56, 0x78, 0x9A, 0xBC, 0xDE, 0xF0],
        ], dtype=np.uint8)  # fmt: skip
        m.mem[:, 0xC000:0xC008] = mem
        set_regs(m, a=[0xF0, 0x0F, 0x00], b=[0x10, 0xFF, 0x44], c=[0x55, 0x55, 0xDE], d=[0x80, 0x01, 0x10])
        m.step(None, frames=0, stage="obs_only")
        want = np.array([
            # 26: m0^m1, 27: m2+5*m3, 28: m4^A, 29: m5+B, 30: m6^C, 31: m7+D (mod 256)
            [0xFF, 0xB0, 0xFF, 0x00, 0xFF, 0x00],
            [0x00, 0xFA, 0xF0, 0x00, 0x00, 0x00],
            [0x26, 0xAE, 0x9A, 0x00, 0x00, 0x00],
        ], dtype=np.float32) / np.float32(255.0)  # fmt: skip
        np.testing.assert_array_equal(m.obs[:, 26:32].view(np.uint32), want.view(np.uint32))
    finally:
        m.close()

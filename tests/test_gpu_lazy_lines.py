"""Scanline changes that raise no request and TIMA edges short of an
overflow, run through by the fast path, against the oracle.

Between the steps that can raise a request (the change into line 144, into
line LYC with the LYC STAT source on, every change with the HBlank source
on, the TIMA overflow), the step kernel lets plain instructions run through
scanline changes and TIMA edges without applying them, and LY, STAT, TIMA
and DIV reads derive their values.  These carts spend their time in delay
loops of seeded, joypad-dependent lengths and read LY, STAT, TIMA and DIV
through LDH, LD A,(C) and LD A,(HL) at whatever position the loop ends,
folding each byte into work RAM.  Interrupt handlers read LY and STAT too
and move LYC; the window is on in some carts (its line counter is part of
the compared state), some carts write LY, DIV, TIMA and TAC or switch the
LCD off and on, the timer runs at every rate, and env 0 (which applies every scanline change) shares a
wavefront with envs that defer.  State is compared in full after every step.
"""

from __future__ import annotations

import numpy as np
import pytest

from gbxcule_amd.carts.asm import Asm
from gbxcule_amd.carts.synth import PROGRAM_ORIGIN, _vectors, finalize_rom, seeded_actions
from oracle.ref import RefMachine

from ._parity import assert_same_state
from .conftest import require_gpu

pytestmark = pytest.mark.gpu


def lazy_cart(seed: int, ime: bool, ie: int, tac: int, stat: int, window: bool, ly_write: bool,
              timer_writes: bool = False, lcd_toggle: bool = False) -> bytes:
    rng = np.random.default_rng(seed)
    rom = bytearray(0x8000)
    h = Asm(origin=0x0068)
    for name, counter in (("vbl", 0xDF00), ("stat", 0xDF01), ("timer", 0xDF02)):
        h.label(name)
        h.push("AF")
        h.push("HL")
        h.ld_rr_d16("HL", counter)
        h.emit(0x34)  # INC (HL)
        h.ldh_a_a8(0x44)
        h.ld_rr_d16("HL", counter + 0x10)
        h.alu_r("ADD", "(HL)")
        h.emit(0x77)  # LD (HL),A
        h.ldh_a_a8(0x41)
        h.ld_rr_d16("HL", counter + 0x20)
        h.alu_r("XOR", "(HL)")
        h.emit(0x77)
        if name == "stat":  # move LYC on
            h.ldh_a_a8(0x45)
            h.alu_d8("ADD", int(rng.integers(3, 60)))
            h.alu_d8("CP", 154)
            h.jr("lyc_ok", "C")
            h.alu_d8("SUB", 154)
            h.label("lyc_ok")
            h.ldh_a8_a(0x45)
        h.pop("HL")
        h.pop("AF")
        h.reti()
    code = h.resolve()
    rom[0x68 : 0x68 + len(code)] = code
    _vectors(rom, {0x40: h.labels["vbl"], 0x48: h.labels["stat"], 0x50: h.labels["timer"]})

    a = Asm(origin=PROGRAM_ORIGIN)
    a.ld_rr_d16("SP", 0xDFF0)
    a.ld_r_d8("A", int(rng.integers(0, 256)))
    a.ldh_a8_a(0x06)  # TMA
    a.ld_r_d8("A", tac)
    a.ldh_a8_a(0x07)  # TAC
    a.ld_r_d8("A", int(rng.integers(0, 154)))
    a.ldh_a8_a(0x45)  # LYC
    a.ld_r_d8("A", int(rng.integers(0, 144)))
    a.ldh_a8_a(0x4A)  # WY
    a.ld_r_d8("A", stat)
    a.ldh_a8_a(0x41)  # STAT interrupt sources
    a.ld_r_d8("A", ie)
    a.ldh_a8_a(0xFF)
    a.ld_r_d8("A", 0x00)
    a.ldh_a8_a(0x0F)
    if ime:
        a.ei()
    a.ld_r_d8("A", 0xB1 if window else 0x91)
    a.ldh_a8_a(0x40)  # LCD on
    a.label("loop")
    for i in range(12):
        # a joypad-dependent delay: lanes end it at different positions
        a.ld_r_d8("A", 0x20 if i % 2 else 0x10)
        a.ldh_a8_a(0x00)
        a.ldh_a_a8(0x00)
        a.alu_d8("AND", 0x0F)
        a.alu_d8("ADD", int(rng.integers(1, 200)))
        a.ld_r_r("B", "A")
        a.label(f"d{i}")
        a.dec_r("B")
        a.jr(f"d{i}", "NZ")
        kind = i % 6
        if kind == 0:
            a.ldh_a_a8(0x44)
        elif kind == 1:
            a.ldh_a_a8(0x41)
        elif kind == 2:
            a.ld_r_d8("C", (0x44, 0x05)[i // 6] if i < 12 else 0x41)
            a.emit(0xF2)  # LD A,(C)
        elif kind == 3:
            a.ld_rr_d16("HL", (0xFF41, 0xFF04)[i // 6])
            a.emit(0x7E)  # LD A,(HL)
        elif kind == 4:
            a.ldh_a_a8(0x05)  # TIMA
        else:
            a.ldh_a_a8(0x04)  # DIV
        a.ld_rr_d16("HL", 0xC000 + i)
        a.alu_r("ADD", "(HL)")
        a.emit(0x77)  # LD (HL),A
        if ly_write and i == 5:
            a.ld_r_d8("A", int(rng.integers(0, 154)))
            a.ldh_a8_a(0x44)  # the next change overwrites it
            a.ldh_a_a8(0x44)
            a.ld_a16_a(0xC010)
        if lcd_toggle and i == 8:  # LCD off and on again after a delay-loop's deferred lines
            a.ld_r_d8("A", 0x11)
            a.ldh_a8_a(0x40)
            a.ldh_a_a8(0x44)
            a.ld_a16_a(0xC01E)
            a.ld_r_d8("A", 0xB1 if window else 0x91)
            a.ldh_a8_a(0x40)
        if timer_writes and i in (3, 7, 10):
            if i == 3:
                a.ldh_a8_a(0x04)  # DIV reset
            elif i == 7:
                a.ld_r_d8("A", int(rng.integers(0, 256)))
                a.ldh_a8_a(0x05)  # TIMA
            else:
                a.ldh_a_a8(0x07)
                a.alu_d8("XOR", 0x01)  # another rate
                a.ldh_a8_a(0x07)
            a.ldh_a_a8(0x05)
            a.ld_a16_a(0xC011 + i)
    a.jp("loop")
    code = a.resolve()
    rom[PROGRAM_ORIGIN : PROGRAM_ORIGIN + len(code)] = code
    return finalize_rom(rom, "GBXAMD LAZY", 0x00, 0x00, 0x00)


CASES = [
    # seed, IME, IE, TAC, STAT sources (HBlank 0x08, VBlank 0x10, OAM 0x20, LYC 0x40), window, LY write,
    # DIV/TIMA/TAC writes[, LCD switched off and on]
    (1, True, 0x03, 0x00, 0x40, True, False, False),
    (2, True, 0x01, 0x05, 0x10, False, False, False),
    (3, False, 0x00, 0x00, 0x00, True, False, False),
    (4, True, 0x02, 0x00, 0x08, False, False, False),
    (5, True, 0x07, 0x04, 0x60, True, False, False),
    (6, False, 0x02, 0x06, 0x50, False, True, False),
    (7, True, 0x06, 0x07, 0x20, True, True, False),
    (8, True, 0x04, 0x05, 0x00, False, False, True),
    (9, False, 0x04, 0x06, 0x40, True, False, True),
    (10, True, 0x05, 0x07, 0x10, False, True, True),
    (11, True, 0x07, 0x04, 0x08, True, False, True),
    (12, True, 0x03, 0x05, 0x40, True, False, False, True),
    (13, False, 0x01, 0x00, 0x10, False, True, True, True),
]


@pytest.mark.parametrize("case", CASES, ids=[str(c[0]) for c in CASES])
def test_lazy_scanline_parity(bootstub, case):
    require_gpu()
    from gbxcule_amd.backend import HipVecBackend

    seed, ime, ie, tac, stat = case[:5]
    rom = lazy_cart(*case)
    n, fs, steps = 128, 6, 4
    dut = HipVecBackend(rom, num_envs=n, frames_per_step=fs, release_after_frames=3,
                        stage="emulate_only", bootrom=bootstub)  # fmt: skip
    ref = RefMachine(n, rom, bootstub)
    try:
        dut.reset(seed=seed)
        ref.step(None, 0, 0, "emulate_only")
        assert_same_state(dut, ref, step=-1, tag=f"lazy{seed}")
        for k in range(steps):
            act = seeded_actions(seed, k, n)
            dut.step(act)
            ref.step(act, fs, 3, "emulate_only", threads=8)
            assert_same_state(dut, ref, step=k, tag=f"lazy{seed}")
        np.testing.assert_array_equal(dut.export_latches(), ref.latches)
        mem = ref.mem
        # the reads saw different positions in different envs
        assert len({bytes(mem[e, 0xC000:0xC00C]) for e in range(n)}) > 1
        lcd_toggle = len(case) > 8 and case[8]
        # (switching the LCD off each pass never reaches line 144 or, here, LYC)
        if ime and ie & 1 and not lcd_toggle:
            assert int(mem[1, 0xDF00]) > 0  # VBlank interrupts were serviced
        if ime and ie & 2 and stat & 0x48 and not lcd_toggle:
            assert int(mem[1, 0xDF01]) > 0  # STAT interrupts were serviced
        if ime and ie & 4 and tac & 4:
            assert int(mem[1, 0xDF02]) > 0  # timer interrupts were serviced
        assert int(ref.field("trap_flag").sum()) == 0
    finally:
        dut.close()
        ref.close()

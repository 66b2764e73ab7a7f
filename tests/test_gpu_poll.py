"""LY poll loops (LDH A,(44) or LD A,(FF44); CP d8; JR cc or JP cc back to
the load) against the oracle.

The step kernel advances whole passes of such a loop in one step up to the
next scanline, TIMA overflow, frame end or interrupt service.  Besides the
LDH/JR form the carts poll with LD A,(FF44) and with JP (passes of 36 and 40
cycles), and with a pair of JP loops that jump to each other, which the
kernel must run one instruction at a time.  STAT mode waits (LDH A,(41) or
LD A,(FF41); AND m or BIT b,A; JR NZ or JR Z) run one instruction at a time
and check that each read of STAT returns the mode of the exact cycle it
falls on, between LY polls that are batched.  These carts
poll with every jump condition while timer, VBlank and STAT interrupts (LYC,
HBlank and VBlank sources) fire with IME on or off, the LCD is switched off
and on, and TIMA runs at every rate; state is compared in full after every
step.
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


FORMS = ("ldh_jr", "ld_jr", "ldh_jp", "ld_jp")


def _poll(a: Asm, label: str, d8: int, cond: str, form: str) -> None:
    """One LY poll loop in the given form: the load, CP d8, the jump back."""
    a.label(label)
    if form.startswith("ldh"):
        a.ldh_a_a8(0x44)
    else:
        a.ld_a_a16(0xFF44)
    a.alu_d8("CP", d8)
    if form.endswith("jr"):
        a.jr(label, cond)
    else:
        a.jp(label, cond)


def poll_cart(seed: int, ime: bool, ie: int, tac: int, lcd_off_frames: bool, stat: int = 0x40,
              halt: bool = False, forms: tuple[str, ...] = ("ldh_jr",), pair: bool = False) -> bytes:
    """A 32 KiB ROM-only cart whose main loop waits on LY four ways (and, with
    ``halt``, in HALT until an interrupt request); loop k is written in form
    ``forms[k % len(forms)]``; with ``pair``, also two JP loops that jump to
    each other."""
    rng = np.random.default_rng(seed)
    rom = bytearray(0x8000)
    h = Asm(origin=0x0068)
    for name, counter in (("vbl", 0xDF00), ("stat", 0xDF01), ("timer", 0xDF02)):
        h.label(name)
        h.push("AF")
        h.push("HL")
        h.ld_rr_d16("HL", counter)
        h.emit(0x34)  # INC (HL)
        if name == "stat":  # move LYC on
            h.ldh_a_a8(0x45)
            h.alu_d8("ADD", int(rng.integers(5, 40)))
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
    lines = [int(x) for x in rng.integers(1, 153, 3)]
    f = lambda k: forms[k % len(forms)]  # noqa: E731
    _poll(a, "w1", 144, "NZ", f(0))  # until LY == 144
    _poll(a, "w2", 144, "Z", f(1))  # while LY == 144
    _poll(a, "w3", lines[0], "C", f(2))  # while LY < n
    _poll(a, "w4", lines[1], "NC", f(3))  # until LY < n (wraps through VBlank)
    if pair:  # until LY == n, alternating between two loads
        a.label("pa")
        a.ldh_a_a8(0x44)
        a.alu_d8("CP", lines[2])
        a.jp("pb", "NZ")
        a.jp("pdone")
        a.label("pb")
        a.ld_a_a16(0xFF44)
        a.alu_d8("CP", lines[2])
        a.jp("pa", "NZ")
        a.label("pdone")
    if halt:
        a.halt()
        a.nop()  # an IME=0 wake skips this byte
    a.ld_a_a16(0xC000)
    a.inc_r("A")
    a.ld_a16_a(0xC000)
    if lcd_off_frames:
        a.alu_d8("AND", 0x03)
        a.jr("loop", "NZ")
        a.ld_r_d8("A", 0x11)
        a.ldh_a8_a(0x40)  # LCD off: LY reads 0
        _poll(a, "w5", lines[2], "NZ", f(4))  # until LY == n: never, while the LCD is off
    a.jp("loop")
    code = a.resolve()
    rom[PROGRAM_ORIGIN : PROGRAM_ORIGIN + len(code)] = code
    return finalize_rom(rom, "GBXAMD POLL", 0x00, 0x00, 0x00)


CASES = [
    # seed, IME, IE, TAC, LCD-off frames, STAT sources (LYC 0x40, HBlank 0x08, VBlank 0x10)
    (1, True, 0x07, 0x05, False, 0x40),
    (2, True, 0x05, 0x04, False, 0x40),
    (3, False, 0x07, 0x07, False, 0x40),
    (4, True, 0x03, 0x00, True, 0x40),
    (5, True, 0x04, 0x06, True, 0x40),
    (6, True, 0x02, 0x00, False, 0x08),
    (7, True, 0x03, 0x05, False, 0x58),
    (8, False, 0x02, 0x00, True, 0x18),
]
# HALT waits between the polls.  A halted CPU runs to the first event that
# can wake it: with the HBlank source off, only the scanline changes into
# line 144 (VBlank, STAT mode-1 source) and into LYC (STAT LYC source) count
# when IE enables them; the mode-2 source never fires at a change.
HALT_CASES = [
    (9, True, 0x02, 0x00, False, 0x08),
    (10, True, 0x07, 0x05, False, 0x48),
    (11, False, 0x06, 0x04, False, 0x08),
    (12, True, 0x01, 0x06, True, 0x10),
    (13, True, 0x02, 0x00, False, 0x40),
    (14, True, 0x06, 0x05, False, 0x10),
    (15, False, 0x04, 0x07, False, 0x20),
    (16, True, 0x03, 0x04, True, 0x40),
    (17, True, 0x05, 0x06, False, 0x60),
]


# The same waits written as LD A,(FF44) and JP loops (36- and 40-cycle
# passes), mixed with the LDH/JR form, and the pair of JP loops that jump to
# each other.
FORM_CASES = [
    (31, True, 0x07, 0x05, False, 0x40, False),
    (32, False, 0x07, 0x07, True, 0x40, False),
    (33, True, 0x02, 0x00, False, 0x08, False),
    (34, True, 0x03, 0x05, False, 0x58, False),
    (35, True, 0x06, 0x05, False, 0x10, True),
    (36, True, 0x03, 0x04, True, 0x40, True),
]


@pytest.mark.parametrize("seed,ime,ie,tac,lcd_off,stat,halt,forms,pair",
                         [c + (False, ("ldh_jr",), False) for c in CASES]
                         + [c + (True, ("ldh_jr",), False) for c in HALT_CASES]
                         + [c + (("ld_jr", "ldh_jp", "ld_jp", "ldh_jr", "ld_jp"), True) for c in FORM_CASES])  # fmt: skip
def test_poll_loop_parity(bootstub, seed, ime, ie, tac, lcd_off, stat, halt, forms, pair):
    require_gpu()
    from gbxcule_amd.backend import HipVecBackend

    rom = poll_cart(seed, ime, ie, tac, lcd_off, stat, halt, forms, pair)
    n, fs, steps = 64, 24, 4
    dut = HipVecBackend(rom, num_envs=n, frames_per_step=fs, release_after_frames=8,
                        stage="emulate_only", bootrom=bootstub)  # fmt: skip
    ref = RefMachine(n, rom, bootstub)
    try:
        dut.reset(seed=seed)
        ref.step(None, 0, 0, "emulate_only")
        assert_same_state(dut, ref, step=-1, tag=f"poll{seed}")
        for k in range(steps):
            act = seeded_actions(seed, k, n)
            dut.step(act)
            ref.step(act, fs, 8, "emulate_only", threads=8)
            assert_same_state(dut, ref, step=k, tag=f"poll{seed}")
        mem = ref.mem
        assert int(mem[0, 0xC000]) > 0  # the loops completed passes
        if ime and ie & 4 and tac & 4:
            assert int(mem[0, 0xDF02]) > 0  # timer interrupts were serviced
        if ime and ie & 2 and stat & 0x08:
            assert int(mem[0, 0xDF01]) > 0  # HBlank STAT interrupts were serviced
        assert int(ref.field("trap_flag").sum()) == 0
    finally:
        dut.close()
        ref.close()


STAT_WAITS = (
    # (load, op, operand, jump): AND m / BIT b,A, then JR NZ or JR Z back
    ("ldh", "and", 3, "NZ"),  # until mode 0 (HBlank)
    ("ldh", "and", 2, "NZ"),  # until mode 0 or 1
    ("ld", "bit", 1, "NZ"),  # until mode 0 or 1, A keeps all of STAT
    ("ldh", "and", 3, "Z"),  # while mode 0
    ("ld", "and", 1, "NZ"),  # until mode 0 or 2
    ("ldh", "bit", 0, "Z"),  # while mode 0 or 2
    ("ld", "and", 2, "Z"),  # while mode 0 or 1 (through VBlank)
)


def _stat_wait(a: Asm, label: str, load: str, op: str, v: int, cond: str) -> None:
    a.label(label)
    if load == "ldh":
        a.ldh_a_a8(0x41)
    else:
        a.ld_a_a16(0xFF41)
    if op == "and":
        a.alu_d8("AND", v)
    else:
        a.cb(0x47 | (v << 3))  # BIT v,A
    a.jr(label, cond)


def stat_cart(seed: int, ime: bool, ie: int, tac: int, stat: int, lcd_off_frames: bool) -> bytes:
    """A 32 KiB ROM-only cart whose main loop runs every STAT mode wait of
    STAT_WAITS, each after a joypad-dependent delay and between LY polls, with
    timer, VBlank and STAT interrupts (handlers move LYC on)."""
    rng = np.random.default_rng(seed)
    rom = bytearray(0x8000)
    h = Asm(origin=0x0068)
    for name, counter in (("vbl", 0xDF00), ("stat", 0xDF01), ("timer", 0xDF02)):
        h.label(name)
        h.push("AF")
        h.push("HL")
        h.ld_rr_d16("HL", counter)
        h.emit(0x34)  # INC (HL)
        if name == "stat":
            h.ldh_a_a8(0x45)
            h.alu_d8("ADD", int(rng.integers(5, 40)))
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
    for reg, val in ((0x06, int(rng.integers(0, 256))), (0x07, tac), (0x45, int(rng.integers(0, 154))),
                     (0x41, stat), (0xFF, ie), (0x0F, 0)):  # fmt: skip
        a.ld_r_d8("A", val)
        a.ldh_a8_a(reg)
    if ime:
        a.ei()
    a.ld_r_d8("A", 0x91)
    a.ldh_a8_a(0x40)  # LCD on
    a.label("loop")
    for k, (load, op, v, cond) in enumerate(STAT_WAITS):
        # a joypad-dependent delay, so that lanes reach the wait at
        # different scanline positions
        a.ld_r_d8("A", 0x10)
        a.ldh_a8_a(0x00)
        a.ldh_a_a8(0x00)
        a.alu_d8("AND", 0x0F)
        a.alu_d8("ADD", int(rng.integers(1, 30)))
        a.ld_r_r("B", "A")
        a.label(f"d{k}")
        a.dec_r("B")
        a.jr(f"d{k}", "NZ")
        _stat_wait(a, f"s{k}", load, op, v, cond)
        if k == 3:
            _poll(a, "ly1", int(rng.integers(1, 153)), "NZ", "ldh_jr")
    a.ld_a_a16(0xC000)
    a.inc_r("A")
    a.ld_a16_a(0xC000)
    if lcd_off_frames:
        a.alu_d8("AND", 0x03)
        a.jp("loop", "NZ")
        a.ld_r_d8("A", 0x11)
        a.ldh_a8_a(0x40)  # LCD off: every mode reads 0
        _stat_wait(a, "off1", "ldh", "and", 3, "NZ")  # exits at once
        a.ld_r_d8("A", 0x91)
        a.ldh_a8_a(0x40)  # LCD on again
    a.jp("loop")
    code = a.resolve()
    rom[PROGRAM_ORIGIN : PROGRAM_ORIGIN + len(code)] = code
    return finalize_rom(rom, "GBXAMD STAT", 0x00, 0x00, 0x00)


STAT_CASES = [
    # seed, IME, IE, TAC, STAT sources, LCD-off frames
    (41, True, 0x07, 0x05, 0x40, False),
    (42, False, 0x07, 0x06, 0x40, True),
    (43, True, 0x02, 0x00, 0x08, False),  # HBlank STAT interrupts
    (44, True, 0x03, 0x04, 0x50, True),
    (45, True, 0x06, 0x07, 0x20, False),  # OAM source: never fires at a change
    (46, False, 0x00, 0x00, 0x00, False),
]


@pytest.mark.parametrize("seed,ime,ie,tac,stat,lcd_off", STAT_CASES)
def test_stat_wait_parity(bootstub, seed, ime, ie, tac, stat, lcd_off):
    """STAT mode waits (every form of STAT_WAITS) against the oracle, full
    state after every step."""
    require_gpu()
    from gbxcule_amd.backend import HipVecBackend

    rom = stat_cart(seed, ime, ie, tac, stat, lcd_off)
    n, fs, steps = 64, 12, 5
    dut = HipVecBackend(rom, num_envs=n, frames_per_step=fs, release_after_frames=8,
                        stage="emulate_only", bootrom=bootstub)  # fmt: skip
    ref = RefMachine(n, rom, bootstub)
    try:
        dut.reset(seed=seed)
        ref.step(None, 0, 0, "emulate_only")
        for k in range(steps):
            act = seeded_actions(seed, k, n)
            dut.step(act)
            ref.step(act, fs, 8, "emulate_only", threads=8)
            assert_same_state(dut, ref, step=k, tag=f"stat{seed}")
        assert int(ref.mem[:, 0xC000].min()) > 0  # the waits completed
        assert int(ref.field("trap_flag").sum()) == 0
    finally:
        dut.close()
        ref.close()


def ly_write_cart(seed: int) -> bytes:
    """IME off; waits for line 153, writes FF44 (LY) with a smaller value and
    polls with JR C until LY >= 153, then writes a value >= d8 and polls with
    JR NC until LY < d8.  The written value is what the first pass reads; the
    next scanline change overwrites it."""
    rng = np.random.default_rng(seed)
    rom = bytearray(0x8000)
    _vectors(rom)
    a = Asm(origin=PROGRAM_ORIGIN)
    a.ld_rr_d16("SP", 0xDFF0)
    a.ld_r_d8("A", 0x91)
    a.ldh_a8_a(0x40)
    a.label("loop")
    a.label("w1")
    a.ldh_a_a8(0x44)
    a.alu_d8("CP", 153)
    a.jr("w1", "NZ")
    a.ld_r_d8("B", 20)  # about 330 cycles further into line 153
    a.label("dl")
    a.dec_r("B")
    a.jr("dl", "NZ")
    a.ld_r_d8("A", int(rng.integers(0, 153)))
    a.ldh_a8_a(0x44)
    a.label("w2")  # while LY < 153: from line 153, once around the frame
    a.ldh_a_a8(0x44)
    a.alu_d8("CP", 153)
    a.jr("w2", "C")
    d8 = int(rng.integers(1, 150))
    a.ld_r_d8("A", int(rng.integers(d8, 256)))
    a.ldh_a8_a(0x44)
    a.label("w3")  # while LY >= d8
    a.ldh_a_a8(0x44)
    a.alu_d8("CP", d8)
    a.jr("w3", "NC")
    a.ld_a_a16(0xC000)
    a.inc_r("A")
    a.ld_a16_a(0xC000)
    a.jp("loop")
    code = a.resolve()
    rom[PROGRAM_ORIGIN : PROGRAM_ORIGIN + len(code)] = code
    return finalize_rom(rom, "GBXAMD LYW", 0x00, 0x00, 0x00)


@pytest.mark.parametrize("seed", [21, 22])
def test_poll_after_ly_write_with_frame_offset(bootstub, seed):
    """A poll that starts on line 153 after the program wrote FF44 runs once
    around the frame (154 scanline changes).  With the frame count out of
    step with the scanlines (each env gets a random cycle_in_frame, as a
    loaded savestate can carry), the frame end does not bound that run, so the
    loop's own end must.  Half the envs get a frame end just past the change
    into line 153 (cycle_in_frame ahead of the scanline position by a line
    less 40-300 cycles): the window where a bound taken from the frame end
    alone would batch passes that read LY = 153."""
    require_gpu()
    from gbxcule_amd.backend import HipVecBackend

    rom = ly_write_cart(seed)
    n, fs, steps = 128, 6, 5
    dut = HipVecBackend(rom, num_envs=n, frames_per_step=fs, release_after_frames=8,
                        stage="emulate_only", bootrom=bootstub)  # fmt: skip
    ref = RefMachine(n, rom, bootstub)
    try:
        dut.reset(seed=seed)
        ref.step(None, 0, 0, "emulate_only")
        act = seeded_actions(seed, 0, n)
        dut.step(act)
        ref.step(act, fs, 8, "emulate_only", threads=8)
        rng = np.random.default_rng(seed)
        off = rng.integers(0, 70224, n)
        pos = ref.field("ppu_ly").astype(np.int64) * 456 + ref.field("ppu_scanline_cycle")
        near = (pos + 456 - rng.integers(40, 300, n)) % 70224
        off[::2] = near[::2]
        ref.field("cycle_in_frame")[:] = off
        dut.import_field("cycle_in_frame", off)
        for k in range(1, steps):
            act = seeded_actions(seed, k, n)
            dut.step(act)
            ref.step(act, fs, 8, "emulate_only", threads=8)
            assert_same_state(dut, ref, step=k, tag=f"lyw{seed}")
        assert int(ref.mem[:, 0xC000].min()) > 0  # every env finished loop passes
        assert int(ref.field("trap_flag").sum()) == 0
    finally:
        dut.close()
        ref.close()

"""Bank switches made from the switched window, and interrupt requests left
pending while IME is clear, against the oracle.

The fast path lets a running CPU with IME clear go on while requests pend
(the step's interrupt check does nothing then), and an MBC bank write drops
the instruction record already fetched for the next pc instead of taking the
full sequence.  These carts make both matter:

* bank hop (MBC1 and MBC3, 8 banks): every bank holds the same ring of
  segments at the same addresses; each segment writes the next bank number
  (from an accumulator that the joypad feeds and a constant of the bank and
  segment) to 2000-3FFF from inside the 4000-7FFF window, and
  the instruction right after the write (an ALU op with a bank-specific
  opcode and constant, folded into the accumulator) must come from the new
  bank;
* pending requests (ROM-only): with IME clear, timer, VBlank and STAT LYC
  requests pend through a joypad-dependent delay, IF is read, then EI, HALT,
  RETI through a pushed address, or EI + HALT re-enables them (or IF is
  cleared first); the handlers read IF too.

State is compared in full after every step (reference: cpu_step_builder.py's
interrupt check after every instruction and the MBC write path of
core/cartridge.py, restated in oracle/gbx_ref.cpp).
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

BANK = 0x4000
NBANKS = 8
SEGS = 40


def bank_hop_cart(seed: int, mbc: int) -> bytes:
    rng = np.random.default_rng(seed)
    rom = bytearray(NBANKS * BANK)
    _vectors(rom)
    a = Asm(origin=PROGRAM_ORIGIN)
    a.ld_rr_d16("SP", 0xDFF0)
    a.ld_r_d8("B", 0)
    a.ld_r_d8("C", 0)
    a.label("loop")
    # C takes in both joypad groups; the start bank follows from C
    a.ld_r_d8("A", 0x10)
    a.ldh_a8_a(0x00)
    a.ldh_a_a8(0x00)
    a.ld_r_r("D", "A")
    a.ld_r_d8("A", 0x20)
    a.ldh_a8_a(0x00)
    a.ldh_a_a8(0x00)
    a.alu_r("XOR", "D")
    a.alu_r("ADD", "C")
    a.ld_r_r("C", "A")
    a.alu_d8("AND", 0x07)
    a.alu_d8("OR", 0x01)  # start bank 1..7
    a.ld_a16_a(0x2000)
    a.ld_r_r("A", "C")
    a.ld_a16_a(0xC000)
    a.ld_r_r("A", "B")
    a.ld_a16_a(0xC001)
    a.jp(BANK)
    code = a.resolve()
    rom[PROGRAM_ORIGIN : PROGRAM_ORIGIN + len(code)] = code
    loop = a.labels["loop"]
    # one write form per segment, the same in every bank so the offsets agree
    forms = rng.integers(0, 2, SEGS)
    for k in range(1, NBANKS):
        b = Asm(origin=BANK)
        for s in range(SEGS):
            # the next bank from C and a constant of this bank and segment
            if forms[s] == 1:
                b.ld_rr_d16("HL", 0x2000 + int(rng.integers(0, 0x2000)))
            b.ld_r_r("A", "C")
            b.alu_d8("XOR", int(rng.integers(0, 256)))
            b.alu_d8("AND", 0x07)
            b.alu_d8("OR", 0x01)
            if forms[s] == 0:
                b.ld_a16_a(0x2000 + int(rng.integers(0, 0x2000)))  # LD (a16),A
            else:
                b.emit(0x77)  # LD (HL),A
            # runs from the new bank: a bank-specific opcode and constant
            b.alu_d8(str(rng.choice(["ADD", "XOR", "SUB", "ADC", "OR"])), int(rng.integers(0, 256)))
            b.alu_r("ADD", "C")
            b.ld_r_r("C", "A")
            b.inc_r("B")
        b.jp(loop)
        bcode = b.resolve()
        rom[k * BANK : k * BANK + len(bcode)] = bcode
    cart_type = 0x01 if mbc == 1 else 0x11
    return finalize_rom(rom, "GBXAMD HOP", cart_type, 0x02, 0x00)


def pending_irq_cart(seed: int) -> bytes:
    rng = np.random.default_rng(seed)
    rom = bytearray(0x8000)
    h = Asm(origin=0x0068)
    for name, counter in (("vbl", 0xDF00), ("stat", 0xDF01), ("timer", 0xDF02)):
        h.label(name)
        h.push("AF")
        h.push("HL")
        h.ld_rr_d16("HL", counter)
        h.emit(0x34)  # INC (HL)
        h.ldh_a_a8(0x0F)  # IF as the handler sees it
        h.ld_rr_d16("HL", counter + 0x10)
        h.alu_r("ADD", "(HL)")
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
    a.ld_r_d8("A", int(rng.integers(4, 8)))
    a.ldh_a8_a(0x07)  # TAC on
    a.ld_r_d8("A", int(rng.integers(0, 154)))
    a.ldh_a8_a(0x45)  # LYC
    a.ld_r_d8("A", 0x40)
    a.ldh_a8_a(0x41)  # STAT: LYC source
    a.ld_r_d8("A", 0x07)
    a.ldh_a8_a(0xFF)  # IE = VBlank | STAT | Timer
    a.ld_r_d8("A", 0x00)
    a.ldh_a8_a(0x0F)
    a.ld_r_d8("A", 0x91)
    a.ldh_a8_a(0x40)  # LCD on
    a.label("loop")
    for i in range(6):
        a.di()
        # a joypad-dependent delay while requests pend
        a.ld_r_d8("A", 0x10 if i % 2 else 0x20)
        a.ldh_a8_a(0x00)
        a.ldh_a_a8(0x00)
        a.alu_d8("AND", 0x0F)
        a.alu_d8("ADD", int(rng.integers(1, 250)))
        a.ld_r_r("B", "A")
        a.label(f"d{i}")
        a.dec_r("B")
        a.jr(f"d{i}", "NZ")
        a.ldh_a_a8(0x0F)
        a.ld_rr_d16("HL", 0xC000 + i)
        a.alu_r("ADD", "(HL)")
        a.emit(0x77)
        # the way IME comes back, from the joypad
        a.ld_r_d8("A", 0x20 if i % 2 else 0x10)
        a.ldh_a8_a(0x00)
        a.ldh_a_a8(0x00)
        a.alu_d8("AND", 0x03)
        a.jr(f"p0_{i}", "Z")
        a.alu_d8("CP", 1)
        a.jr(f"p1_{i}", "Z")
        a.alu_d8("CP", 2)
        a.jr(f"p2_{i}", "Z")
        a.ei()  # 3: EI, then HALT
        a.halt()
        a.nop()
        a.jr(f"end_{i}")
        a.label(f"p0_{i}")  # 0: EI
        a.ei()
        a.nop()
        a.jr(f"end_{i}")
        a.label(f"p1_{i}")  # 1: HALT with IME clear (IF cleared first in some)
        if i % 3 == 1:
            a.ld_r_d8("A", 0x00)
            a.ldh_a8_a(0x0F)
        a.halt()
        a.nop()
        a.ei()
        a.jr(f"end_{i}")
        a.label(f"p2_{i}")  # 2: RETI to a pushed address
        a.ld_rr_d16("HL", f"end_{i}")
        a.push("HL")
        a.reti()
        a.label(f"end_{i}")
        a.ld_a_a16(0xC010 + i)
        a.inc_r("A")
        a.ld_a16_a(0xC010 + i)
    a.jp("loop")
    code = a.resolve()
    rom[PROGRAM_ORIGIN : PROGRAM_ORIGIN + len(code)] = code
    return finalize_rom(rom, "GBXAMD PEND", 0x00, 0x00, 0x00)


CASES = [("hop_mbc1", 1), ("hop_mbc3", 3), ("pending", 0)]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("seed", [1, 2])
def test_irq_and_bank_parity(bootstub, case, seed):
    require_gpu()
    from gbxcule_amd.backend import HipVecBackend

    name, mbc = case
    rom = bank_hop_cart(seed, mbc) if name.startswith("hop") else pending_irq_cart(seed)
    n, fs, steps = 128, 4, 4
    dut = HipVecBackend(rom, num_envs=n, frames_per_step=fs, release_after_frames=2,
                        stage="emulate_only", bootrom=bootstub)  # fmt: skip
    ref = RefMachine(n, rom, bootstub)
    try:
        dut.reset(seed=seed)
        ref.step(None, 0, 0, "emulate_only")
        assert_same_state(dut, ref, step=-1, tag=f"{name}{seed}")
        for k in range(steps):
            act = seeded_actions(seed, k, n)
            dut.step(act)
            ref.step(act, fs, 2, "emulate_only", threads=8)
            assert_same_state(dut, ref, step=k, tag=f"{name}{seed}")
        mem = ref.mem
        assert int(ref.field("trap_flag").sum()) == 0
        if name.startswith("hop"):
            # the rings ran and took different paths in different envs
            assert len({bytes(mem[e, 0xC000:0xC002]) for e in range(n)}) > 1
        else:
            assert int(mem[:, 0xDF00:0xDF03].astype(np.int64).sum()) > 0  # requests were serviced
            assert len({bytes(mem[e, 0xC010:0xC016]) for e in range(n)}) > 1
    finally:
        dut.close()
        ref.close()

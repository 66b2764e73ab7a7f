"""Randomized carts that mix everything the step kernel batches or shortcuts
with random code, against the oracle.

Each seed builds a cart whose main loop runs a block of random legal code
(CB included, joypad-keyed branches, stores into work RAM), an LY poll loop
with a random condition and line, a block-copy loop between random windows
with a random length (overlaps and window edges included), and optionally a
HALT wait, under a random timer rate, STAT source set, IE mask and IME, on
ROM-only, MBC1 and MBC3 (cart RAM, RTC) carts whose loops also switch banks.
The random code itself may write IO registers (and MBC3 cart RAM).  State
is compared in full after every step.
"""

from __future__ import annotations

import numpy as np
import pytest

from gbxcule_amd.carts.asm import Asm
from gbxcule_amd.carts.synth import (
    LEGAL_NON_CB,
    PROGRAM_ORIGIN,
    CodeGen,
    _cb_pool,
    _emit_random_program,
    _vectors,
    finalize_rom,
    seeded_actions,
)
from oracle.ref import RefMachine

from ._parity import assert_same_state
from .conftest import require_gpu

pytestmark = pytest.mark.gpu

# copy windows: (lo, hi) of the source or destination start address
_SRC = [(0x0100, 0x3F00), (0x3F80, 0x4000), (0x4000, 0x7F00), (0x8000, 0x9F00), (0x9F80, 0xA000),
        (0xC000, 0xDC00)]  # fmt: skip
_DST = [(0x8000, 0x9F00), (0x9FC0, 0xA000), (0xC000, 0xDC00), (0xFE00, 0xFE80)]


def fuzz_cart(seed: int, mbc: int = 0) -> bytes:
    """ROM-only (mbc 0), MBC1 with 4 banks (1) or MBC3 with 4 banks and
    32 KiB of cart RAM (3)."""
    rng = np.random.default_rng(seed)
    r = lambda lo, hi: int(rng.integers(lo, hi))  # noqa: E731
    size = 0x8000 if mbc == 0 else 0x10000
    rom = bytearray(size)
    rom[0x1000:size] = rng.integers(0, 256, size - 0x1000, dtype=np.uint8).tobytes()
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

    a = Asm(origin=PROGRAM_ORIGIN)
    a.ld_rr_d16("SP", 0xDFF0)
    if mbc == 3:
        a.ld_r_d8("A", 0x0A)
        a.ld_a16_a(0x0000)  # cart RAM and RTC on
    for reg, val in ((0x06, r(0, 256)), (0x07, r(0, 8)), (0x45, r(0, 154)),
                     (0x41, int(rng.choice([0x00, 0x08, 0x10, 0x20, 0x40, 0x48, 0x50, 0x78]))),
                     (0xFF, r(0, 32)), (0x0F, 0x00)):  # fmt: skip
        a.ld_r_d8("A", val)
        a.ldh_a8_a(reg)
    if rng.random() < 0.6:
        a.ei()
    a.ld_r_d8("A", 0x91)
    a.ldh_a8_a(0x40)
    a.label("loop")
    for part in rng.permutation(5):
        if part == 4:  # the ROM bank from the joypad; an MBC3 RAM bank or RTC register
            if mbc:
                a.ld_r_d8("A", 0x10)
                a.ldh_a8_a(0x00)
                a.ldh_a_a8(0x00)
                a.alu_d8("AND", 0x03)
                a.ld_a16_a(0x2000)
            if mbc == 3:
                a.ld_r_d8("A", int(rng.choice([0, 1, 2, 3, 8, 9, 0xC])))
                a.ld_a16_a(0x4000)
                a.ld_r_d8("A", 0x00)
                a.ld_a16_a(0x6000)
                a.ld_r_d8("A", 0x01)
                a.ld_a16_a(0x6000)  # latch the RTC
        elif part == 0:  # random code
            gen = CodeGen(rng, a, stack="reseed", joypad_conditions=True, store_lo=0xC000,
                          store_hi=0xDDFF, cart_ram=mbc == 3)  # fmt: skip
            _emit_random_program(gen, r(24, 96), LEGAL_NON_CB + _cb_pool())
            end = a.pc
            gen.resolve(end)
        elif part == 1:  # LY poll
            a.label("poll")
            a.ldh_a_a8(0x44)
            a.alu_d8("CP", r(0, 154))
            a.jr("poll", str(rng.choice(["NZ", "Z", "NC", "C"])))
        elif part == 2:  # block copy
            lo, hi = _SRC[r(0, len(_SRC))]
            src = r(lo, hi)
            if rng.random() < 0.3:  # overlap with the source
                dst = max(0xC000, min(0xDC00, src + r(-8, 9))) if src >= 0xC000 else r(0xC000, 0xDC00)
            else:
                lo, hi = _DST[r(0, len(_DST))]
                dst = r(lo, hi)
            a.ld_rr_d16("HL", src)
            a.ld_rr_d16("DE", dst)
            a.ld_rr_d16("BC", r(1, 600))
            a.label("copy")
            a.ld_a_hli()
            a.ld_de_a()
            a.inc_rr("DE")
            a.dec_rr("BC")
            if rng.random() < 0.5:
                a.ld_r_r("A", "B")
                a.alu_r("OR", "C")
            else:
                a.ld_r_r("A", "C")
                a.alu_r("OR", "B")
            a.jr("copy", "NZ")
        elif rng.random() < 0.5:  # HALT wait
            a.halt()
            a.nop()
    a.ld_rr_d16("SP", 0xDFF0)
    a.ld_a_a16(0xDE80)
    a.inc_r("A")
    a.ld_a16_a(0xDE80)
    a.jp("loop")
    code = a.resolve()
    assert PROGRAM_ORIGIN + len(code) < 0x1000
    rom[PROGRAM_ORIGIN : PROGRAM_ORIGIN + len(code)] = code
    kind = {0: (0x00, 0x00, 0x00), 1: (0x01, 0x01, 0x00), 3: (0x10, 0x01, 0x03)}[mbc]
    return finalize_rom(rom, "GBXAMD FUZZ", *kind)


@pytest.mark.parametrize("seed,mbc", [(s, 0) for s in range(100, 112)] + [(s, 1) for s in range(120, 124)]
                         + [(s, 3) for s in range(130, 134)])  # fmt: skip
def test_fuzz_parity(bootstub, seed, mbc):
    require_gpu()
    from gbxcule_amd.backend import HipVecBackend

    rom = fuzz_cart(seed, mbc)
    n, fs, steps = 64, 24, 3
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
            assert_same_state(dut, ref, step=k, tag=f"fuzz{seed}")
    finally:
        dut.close()
        ref.close()

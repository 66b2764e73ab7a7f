"""Instruction fetch outside the pre-decoded ROM images, against the oracle.

The step kernel decodes an instruction from a pre-built record when its bytes
lie inside one 16 KiB ROM window of a mapped bank or inside the boot image;
everything else is fetched byte by byte through the bus (the reference's
read8 for the opcode and each operand, ``kernels/cpu_step_builder.py:
538-657``).  These carts run that path the way games do:

* bank edges: an instruction at 0x3FFE whose last operand byte is 0x4000 of
  the switched bank, code continuing at 0x4001 of that bank, an instruction
  at 0x7FFF whose operands are the first two bytes of video RAM, and code
  continuing in video RAM; MBC1 and MBC3 banks switched from the joypad
  every frame;
* code in RAM: an OAM DMA routine copied to high RAM and called every frame,
  a routine in work RAM whose immediate operand the main loop rewrites before
  every call, and an instruction at 0xDFFE whose operand byte 0xE000 is echo
  RAM (work RAM 0xC000), with execution continuing in echo RAM;
* the boot overlay edge: boot images whose last instruction ends at 0x00FE
  (overlay off, next fetch from the cartridge at 0x00FF) or starts at 0x00FF
  with its operand at 0x0100 read from the cartridge while the overlay is on.

Every step compares the full state of every env.
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


def _run(rom: bytes, boot: bytes, n: int = 64, fs: int = 2, steps: int = 6, seed: int = 3) -> None:
    from gbxcule_amd.backend import HipVecBackend

    dut = HipVecBackend(rom, num_envs=n, frames_per_step=fs, release_after_frames=8,
                        stage="full_step", bootrom=boot)  # fmt: skip
    ref = RefMachine(n, rom, boot)
    try:
        dut.reset(seed=seed)
        ref.step(None, 0, 0, "full_step")
        assert_same_state(dut, ref, step=-1, tag="fetch")
        for k in range(steps):
            act = seeded_actions(seed, k, n)
            obs, *_ = dut.step(act)
            ref.step(act, fs, 8, "full_step", threads=8)
            assert_same_state(dut, ref, step=k, tag="fetch")
            np.testing.assert_array_equal(obs.view(np.uint32), ref.obs.view(np.uint32))
        assert int(ref.field("trap_flag").sum()) == 0
        assert int(ref.field("instr_count").min()) > 0
    finally:
        dut.close()
        ref.close()


def _emit_bytes(a: Asm, addr: int, data: bytes) -> None:
    """Store ``data`` at ``addr`` from code (LD HL,addr; LD A,b; LD (HL+),A ...)."""
    a.ld_rr_d16("HL", addr)
    for b in data:
        a.ld_r_d8("A", b)
        a.ld_hli_a()


def _wait_frame(a: Asm, tag: str) -> None:
    a.label(f"{tag}1")
    a.ldh_a_a8(0x44)
    a.alu_d8("CP", 144)
    a.jr(f"{tag}1", "NZ")
    a.label(f"{tag}2")
    a.ldh_a_a8(0x44)
    a.alu_d8("CP", 145)
    a.jr(f"{tag}2", "NZ")


def bank_edge_cart(mbc3: bool) -> bytes:
    banks = 8
    rom = bytearray(0x4000 * banks)
    _vectors(rom)
    a = Asm(origin=PROGRAM_ORIGIN)
    a.ld_rr_d16("SP", 0xDFF0)
    # video RAM 0x8002: LD A,H; LD (C020),A; LD A,L; LD (C021),A; RET
    _emit_bytes(a, 0x8002, bytes([0x7C, 0xEA, 0x20, 0xC0, 0x7D, 0xEA, 0x21, 0xC0, 0xC9]))
    a.label("loop")
    a.ld_r_d8("A", 0x20)
    a.ldh_a8_a(0x00)
    a.ldh_a_a8(0x00)  # d-pad bits, low nibble
    a.alu_d8("AND", 0x07)
    a.ld_r_r("B", "A")
    a.ld_a16_a(0x2000)  # ROM bank (0 selects 1)
    a.ld_r_r("A", "B")
    a.ld_a16_a(0x8000)  # operand bytes of the instruction at 0x7FFF
    a.alu_d8("XOR", 0x5A)
    a.ld_a16_a(0x8001)
    a.call(0x3FFE)
    _wait_frame(a, "wf")
    a.jp("loop")
    code = a.resolve()
    rom[PROGRAM_ORIGIN : PROGRAM_ORIGIN + len(code)] = code
    rom[0x3FFE:0x4000] = bytes([0x21, 0x34])  # LD HL,(0x4000)<<8 | 0x34
    for b in range(1, banks):
        base = 0x4000 * b
        rom[base] = 0x11 * b  # H of the LD HL at 0x3FFE
        # 0x4001: LD A,H; LD (C000+b),A; CALL 7FFE; RET
        rom[base + 1 : base + 8] = bytes([0x7C, 0xEA, b, 0xC0, 0xCD, 0xFE, 0x7F])
        rom[base + 8] = 0xC9
        rom[base + 0x3FFE : base + 0x4000] = bytes([0x00, 0x21])  # NOP; LD HL,(8000)
    if mbc3:
        return finalize_rom(rom, "GBXAMD EDGE3", 0x13, 0x02, 0x03)
    return finalize_rom(rom, "GBXAMD EDGE1", 0x01, 0x02, 0x00)


def ram_code_cart() -> bytes:
    rom = bytearray(0x8000)
    _vectors(rom)
    # high RAM routine (the usual OAM DMA wait): LD A,C2; LDH (46),A; LD A,28;
    # w: DEC A; JR NZ,w; RET
    hram = bytes([0x3E, 0xC2, 0xE0, 0x46, 0x3E, 0x28, 0x3D, 0x20, 0xFD, 0xC9])
    # work RAM routine at C100: LD A,d8 (patched); LD (C300),A; LD HL,C301; INC (HL); RET
    wram = bytes([0x3E, 0x00, 0xEA, 0x00, 0xC3, 0x21, 0x01, 0xC3, 0x34, 0xC9])
    a = Asm(origin=PROGRAM_ORIGIN)
    a.ld_rr_d16("SP", 0xD000)
    _emit_bytes(a, 0xFF80, hram)
    _emit_bytes(a, 0xC100, wram)
    # 0xDFFE: LD HL,(E000)<<8 | 0x77 -> C000 byte; continues at E001 = C001: RET
    _emit_bytes(a, 0xDFFE, bytes([0x21, 0x77]))
    _emit_bytes(a, 0xC000, bytes([0x55, 0xC9]))
    a.label("loop")
    a.ld_r_d8("A", 0x10)
    a.ldh_a8_a(0x00)
    a.ldh_a_a8(0x00)  # buttons
    a.ld_r_r("B", "A")
    a.ld_a_a16(0xC200)
    a.alu_r("ADD", "B")
    a.ld_a16_a(0xC200)  # also the first byte OAM DMA copies
    a.ld_a16_a(0xC101)  # patch the immediate of the routine at C100
    a.call(0xFF80)
    a.call(0xC100)
    a.call(0xDFFE)
    a.ld_r_r("A", "H")
    a.ld_a16_a(0xC010)
    _wait_frame(a, "wf")
    a.jp("loop")
    code = a.resolve()
    rom[PROGRAM_ORIGIN : PROGRAM_ORIGIN + len(code)] = code
    return finalize_rom(rom, "GBXAMD RAMCODE", 0x00, 0x00, 0x00)


def boot_edge_image(variant: str) -> bytes:
    """Boot image ending across the overlay edge.  ``off_at_fd``: LDH (50),A
    at 0x00FD, so the fetch at 0x00FF comes from the cartridge (the boot
    image holds HALT there, which must not run).  ``operand_from_cart``:
    LD A,d8 at 0x00FF with the overlay still on, whose operand at 0x0100 is
    the cartridge's; the cartridge then switches the overlay off itself."""
    a = Asm(origin=0x0000)
    a.ld_rr_d16("SP", 0xFFFE)
    a.ld_r_d8("A", 0x91)
    a.ldh_a8_a(0x40)
    a.ld_r_d8("A", 0x01)
    end = {"off_at_fd": 0xFD, "operand_from_cart": 0xFF}[variant]
    a.jp(end)
    code = bytearray(a.resolve())
    code.extend(b"\x00" * (0x100 - len(code)))
    if variant == "off_at_fd":
        code[0xFD:0xFF] = bytes([0xE0, 0x50])
        code[0xFF] = 0x76
    else:
        code[0xFF] = 0x3E
    return bytes(code)


def boot_edge_cart() -> bytes:
    rom = bytearray(0x8000)
    _vectors(rom)
    rom[0xFF] = 0x00  # NOP, fetched after an overlay switched off at 0x00FD
    a = Asm(origin=PROGRAM_ORIGIN)
    a.ld_rr_d16("SP", 0xDFF0)
    a.ld_a16_a(0xC000)  # A as the boot image's last instruction left it
    a.ld_r_d8("A", 0x01)
    a.ldh_a8_a(0x50)  # overlay off (a no-op if already off)
    a.label("loop")
    a.ld_a_a16(0xC001)
    a.inc_r("A")
    a.ld_a16_a(0xC001)
    _wait_frame(a, "wf")
    a.jp("loop")
    code = a.resolve()
    rom[PROGRAM_ORIGIN : PROGRAM_ORIGIN + len(code)] = code
    return finalize_rom(rom, "GBXAMD BOOTEDGE", 0x00, 0x00, 0x00)


@pytest.mark.parametrize("mbc3", [False, True])
def test_bank_edges_and_video_ram_code(bootstub, mbc3):
    require_gpu()
    _run(bank_edge_cart(mbc3), bootstub)


def test_routines_in_high_work_and_echo_ram(bootstub):
    require_gpu()
    _run(ram_code_cart(), bootstub)


@pytest.mark.parametrize("variant", ["off_at_fd", "operand_from_cart"])
def test_boot_overlay_edge(variant):
    require_gpu()
    _run(boot_edge_cart(), boot_edge_image(variant), steps=3)

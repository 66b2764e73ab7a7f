"""A 256-byte DMG boot stub authored for this project.

It reproduces the documented post-boot CPU/IO state (Pan Docs "Power Up
Sequence": SP=FFFE, AF=01B0, BC=0013, DE=00D8, HL=014D, LCDC=91, BGP=FC) and
hands over to the cartridge by writing FF50 from address 0x00FE, so that the
fetch at 0x0100 already comes from the cartridge.  No Nintendo boot ROM bytes
are used; the emulator treats whatever 256 bytes it is given as opaque input.
"""

from __future__ import annotations

from .asm import Asm

BOOTSTUB_SIZE = 0x100


def build_bootstub() -> bytes:
    a = Asm(origin=0x0000)
    a.ld_rr_d16("SP", 0xFFFE)
    a.ld_r_d8("A", 0x91)
    a.ldh_a8_a(0x40)  # LCDC
    a.ld_r_d8("A", 0xFC)
    a.ldh_a8_a(0x47)  # BGP
    a.ld_rr_d16("BC", 0x01B0)
    a.push("BC")
    a.pop("AF")  # A=01, F=B0
    a.ld_rr_d16("BC", 0x0013)
    a.ld_rr_d16("DE", 0x00D8)
    a.ld_rr_d16("HL", 0x014D)
    a.jp(0x00FE)
    code = bytearray(a.resolve())
    code.extend(b"\x00" * (0xFE - len(code)))
    code.extend(bytes([0xE0, 0x50]))  # LDH (50),A with A=01: boot ROM off
    assert len(code) == BOOTSTUB_SIZE
    return bytes(code)

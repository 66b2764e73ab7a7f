"""Helpers to run hand-placed SM83 code on the oracle (and the HIP backend)
from a chosen register state, skipping the boot stub."""

from __future__ import annotations

import numpy as np

from gbxcule_amd.carts.bootstub import build_bootstub
from gbxcule_amd.carts.synth import finalize_rom

CS_BOOT = 6  # cart_state slot BOOTROM_ENABLED


def flat_rom(
    blocks: dict[int, bytes],
    *,
    cart_type: int = 0x00,
    rom_code: int = 0x00,
    ram_code: int = 0x00,
    fill: int = 0x00,
) -> bytes:
    """A cart whose bytes at each address in ``blocks`` are the given code.
    Addresses >= 0x4000 are physical offsets (bank * 0x4000 + offset)."""
    rom = bytearray([fill]) * ((32 * 1024) << rom_code)
    for addr, code in blocks.items():
        rom[addr : addr + len(code)] = code
    return finalize_rom(rom, "GBXAMD TEST", cart_type, rom_code, ram_code)


def oracle(rom: bytes, n: int, pc: int | np.ndarray = 0x150):
    """Oracle machine with the boot overlay off and PC at ``pc``; all other
    state is power-on (registers 0, LCD off)."""
    from oracle.ref import RefMachine

    m = RefMachine(n, rom, build_bootstub())
    m.cart_state[:, CS_BOOT] = 0
    m.field("pc")[:] = pc
    return m


def set_regs(m, **regs: np.ndarray | int) -> None:
    for name, v in regs.items():
        m.field(name)[:] = v


def run_instructions(m, k: int, *, actions=None, release: int = 8) -> None:
    """Execute exactly ``k`` instructions per env (debug max-instruction trap),
    then clear the trap so the machine can continue."""
    m.set_debug(max_instr=k)
    m.step(actions, frames=1, release=release)
    m.set_debug(max_instr=0)
    for f in ("trap_flag", "trap_pc", "trap_opcode", "trap_kind"):
        m.field(f)[:] = 0


def run_frames(m, frames: int, *, actions=None, release: int = 8) -> None:
    m.step(actions, frames=frames, release=release)

"""Differential test of the HIP kernel against the oracle from random machine
states, one env per opcode x random state: every unprefixed and CB opcode,
random registers, SP, IME/IE/IF, timer, LCD/STAT/LYC registers and WRAM/HRAM
contents, on ROM-only, MBC1 and MBC3+RAM carts.  Address registers point
anywhere, so reads and writes also hit IO, MBC and cart-RAM side effects.

After 1, 2 and 6 instructions (debug max-instruction trap) and after one full
frame of continued execution of the random ROM, the whole state must match.
Seed 2 (compared after every one of 8 frames) always runs: on the MBC3 cart
it halts with SP inside the RTC registers and an interrupt's push sets the
RTC halt bit at the end of a halt the kernel runs as one step, where the RTC
must have counted every 4-cycle halted step before the push.
GBX_ISA_SEEDS=k adds k more random states per cart, each compared after every
one of 8 frames (about 2 s per seed and cart).
"""

from __future__ import annotations

import os

import numpy as np
import pytest

from gbxcule_amd.carts.asm import ILLEGAL

from ._isa import CS_BOOT, flat_rom
from ._parity import assert_same_state
from .conftest import require_gpu

pytestmark = pytest.mark.gpu

OPS = [op for op in range(256) if op != 0xCB] + [0x100 | cb for cb in range(256)]
CARTS = [(0x00, 0x00, 0x00), (0x01, 0x02, 0x00), (0x13, 0x02, 0x03)]
SEEDS = [0, 2] + [k for k in range(1, 1 + int(os.environ.get("GBX_ISA_SEEDS", "0"))) if k != 2]


def _rom(rng, cart_type, rom_code, ram_code, pcs, ops):
    size = (32 * 1024) << rom_code
    body = rng.integers(0, 256, size, dtype=np.uint8)
    # keep the random code mostly legal so envs run past their first opcode
    bad = np.isin(body, np.array(sorted(ILLEGAL | {0x10}), dtype=np.uint8))
    body[bad] = 0x00
    blocks = {0: bytes(body[:0x100]), 0x150: bytes(body[0x150:])}
    for pc, op in zip(pcs, ops):
        blocks[int(pc)] = bytes([0xCB, op & 0xFF]) if op & 0x100 else bytes([op])
    return flat_rom(blocks, cart_type=cart_type, rom_code=rom_code, ram_code=ram_code)


def _randomize(rng, n, ref, dut, pcs):
    import torch

    regs = {r: rng.integers(0, 256, n) for r in "abcdehl"}
    regs["f"] = rng.integers(0, 16, n) << 4
    regs["sp"] = rng.integers(0, 0x10000, n)
    regs["pc"] = pcs
    regs["ime"] = rng.integers(0, 2, n)
    regs["div_counter"] = rng.integers(0, 0x10000, n)
    io = {
        0xFF04: regs["div_counter"] >> 8,
        0xFF05: rng.integers(0, 256, n),
        0xFF06: rng.integers(0, 256, n),
        0xFF07: rng.integers(0, 8, n),
        0xFF0F: rng.integers(0, 32, n),
        0xFFFF: rng.integers(0, 32, n),
        0xFF40: rng.choice([0x00, 0x91, 0xE3, 0x83], n),
        0xFF41: rng.integers(0, 256, n) & 0x78,
        0xFF45: rng.integers(0, 154, n),
        0xFF4A: rng.integers(0, 150, n),
    }
    wram = rng.integers(0, 256, (n, 0x2000), dtype=np.uint8)
    hram = rng.integers(0, 256, (n, 0x7F), dtype=np.uint8)
    # oracle
    for k, v in regs.items():
        ref.field(k)[:] = v
    for a, v in io.items():
        ref.mem[:, a] = v
    ref.mem[:, 0xC000:0xE000] = wram
    ref.mem[:, 0xFF80:0xFFFF] = hram
    ref.cart_state[:, CS_BOOT] = 0
    # device
    for k, v in regs.items():
        dut.import_field(k, np.asarray(v, np.int64))
    cs = dut.export_cart_state()
    cs[:, CS_BOOT] = 0
    dut.import_cart_state(cs)
    # through the env-major memory_torch() view, as the reference's callers write
    mem = dut.memory_torch()
    for a, v in io.items():
        mem[:, a] = torch.from_numpy(np.asarray(v, np.uint8)).cuda()
    mem[:, 0xC000:0xE000] = torch.from_numpy(wram).cuda()
    mem[:, 0xFF80:0xFFFF] = torch.from_numpy(hram).cuda()
    torch.cuda.synchronize()


def _clear_traps(ref, dut):
    for f in ("trap_flag", "trap_pc", "trap_opcode", "trap_kind"):
        ref.field(f)[:] = 0
        dut.import_field(f, np.zeros(dut.num_envs, np.int64))


@pytest.mark.parametrize("seed", SEEDS)
@pytest.mark.parametrize("cart", CARTS, ids=["rom_only", "mbc1", "mbc3_ram"])
def test_every_opcode_from_random_states(bootstub, cart, seed):
    require_gpu()
    from gbxcule_amd.backend import HipVecBackend
    from oracle.ref import RefMachine

    rng = np.random.default_rng(1234 + cart[0] if seed == 0 else seed * 7919 + cart[0])
    frames = 1 if seed == 0 else 8
    reps = 2
    ops = np.array(OPS * reps)
    n = ops.size
    pcs = 0x200 + 4 * (np.arange(n) % 4000)
    rom = _rom(rng, *cart, pcs, ops)
    dut = HipVecBackend(rom, num_envs=n, frames_per_step=1, stage="full_step", bootrom=bootstub)
    ref = RefMachine(n, rom, bootstub)
    try:
        dut.reset()
        _randomize(rng, n, ref, dut, pcs)
        acts = rng.integers(0, 8, n).astype(np.int32)
        assert_same_state(dut, ref, step=-1, tag=f"{cart} setup")
        for k, tag in ((1, "1 instr"), (1, "2 instr"), (4, "6 instr")):
            ref.set_debug(max_instr=k)
            dut.set_debug_traps(max_instr=k)
            ref.step(acts, 1, 8, "full_step", threads=8)
            dut.step(acts)
            assert_same_state(dut, ref, step=k, tag=f"{cart} {tag}")
            _clear_traps(ref, dut)
        ref.set_debug()
        dut.set_debug_traps()
        for f in range(frames):
            ref.step(acts, 1, 8, "full_step", threads=8)
            dut.step(acts)
            assert_same_state(dut, ref, step=99 + f, tag=f"{cart} seed {seed} frame {f}")
        np.testing.assert_array_equal(dut.export_latches(), ref.latches)
    finally:
        dut.close()
        ref.close()


# stack pointers and LD (a16),SP targets whose two written bytes straddle
# FF00 (JOYP), IE, IO registers with side effects, MBC registers, cart RAM,
# echo RAM, OAM and HRAM
EDGE_SP = [0xFF01, 0xFF02, 0x0001, 0x0000, 0xA001, 0xFF81, 0xE001, 0xFEA1, 0xFF10, 0x8001,
           0xC001, 0xFF06, 0xFF46, 0xFF51, 0x2001, 0x4001]  # fmt: skip
EDGE_A16 = [0xFEFF, 0xFFFF, 0xFF00, 0x7FFF, 0x9FFF, 0xBFFF, 0xDFFF, 0xFF0E, 0xFF45, 0xFF04,
            0x1FFF, 0x3FFF, 0x5FFF, 0xFDFF, 0xFF7F]  # fmt: skip


@pytest.mark.parametrize("cart", CARTS, ids=["rom_only", "mbc1", "mbc3_ram"])
def test_two_byte_writes_at_region_edges(bootstub, cart):
    """PUSH, CALL, RST and LD (a16),SP whose two bytes land on two different
    kinds of address (one of them often FF00, whose stored value is the
    joypad read for the written select bits)."""
    require_gpu()
    from gbxcule_amd.backend import HipVecBackend
    from oracle.ref import RefMachine

    from ._isa import flat_rom

    rng = np.random.default_rng(77 + cart[0])
    size = (32 * 1024) << cart[1]
    body = rng.integers(0, 256, size, dtype=np.uint8)
    body[np.isin(body, np.array(sorted(ILLEGAL | {0x10}), dtype=np.uint8))] = 0x00
    blocks = {0: bytes(body[:0x100]), 0x150: bytes(body[0x150:])}
    envs = []  # (pc, bytes, sp)
    for sp in EDGE_SP:
        for op in (0xC5, 0xD5, 0xE5, 0xF5, 0xCD, 0xFF, 0xC7):
            tgt = int(rng.integers(0x200, 0x3000))
            envs.append((op, tgt, sp))
    for a16 in EDGE_A16:
        for _ in range(3):
            envs.append((0x08, a16, int(rng.integers(0, 0x10000))))
    n = len(envs)
    pcs = 0x4000 - 4 * n + 4 * np.arange(n)
    for pc, (op, k16, _) in zip(pcs, envs):
        blocks[int(pc)] = bytes([op, k16 & 0xFF, k16 >> 8])
    rom = flat_rom(blocks, cart_type=cart[0], rom_code=cart[1], ram_code=cart[2])
    dut = HipVecBackend(rom, num_envs=n, frames_per_step=1, stage="full_step", bootrom=bootstub)
    ref = RefMachine(n, rom, bootstub)
    try:
        dut.reset()
        _randomize(rng, n, ref, dut, pcs)
        sps = np.array([sp for _, _, sp in envs], np.int64)
        ref.field("sp")[:] = sps
        dut.import_field("sp", sps)
        acts = rng.integers(0, 8, n).astype(np.int32)
        assert_same_state(dut, ref, step=-1, tag=f"{cart} setup")
        for k, tag in ((1, "1 instr"), (1, "2 instr"), (4, "6 instr")):
            ref.set_debug(max_instr=k)
            dut.set_debug_traps(max_instr=k)
            ref.step(acts, 1, 8, "full_step", threads=8)
            dut.step(acts)
            assert_same_state(dut, ref, step=k, tag=f"{cart} {tag}")
            _clear_traps(ref, dut)
        ref.set_debug()
        dut.set_debug_traps()
        ref.step(acts, 1, 8, "full_step", threads=8)
        dut.step(acts)
        assert_same_state(dut, ref, step=99, tag=f"{cart} frame")
    finally:
        dut.close()
        ref.close()

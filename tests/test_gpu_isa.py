"""Differential test of the HIP kernel against the oracle from random machine
states, one env per opcode x random state: every unprefixed and CB opcode,
random registers, SP, IME/IE/IF, timer, LCD/STAT/LYC registers and WRAM/HRAM
contents, on ROM-only, MBC1 and MBC3+RAM carts.  Address registers point
anywhere, so reads and writes also hit IO, MBC and cart-RAM side effects.

After 1, 2 and 6 instructions (debug max-instruction trap) and after one full
frame of continued execution of the random ROM, the whole state must match.
"""

from __future__ import annotations

import numpy as np
import pytest

from gbxcule_amd.carts.asm import ILLEGAL

from ._isa import CS_BOOT, flat_rom
from ._parity import assert_same_state
from .conftest import require_gpu

pytestmark = pytest.mark.gpu

OPS = [op for op in range(256) if op != 0xCB] + [0x100 | cb for cb in range(256)]
CARTS = [(0x00, 0x00, 0x00), (0x01, 0x02, 0x00), (0x13, 0x02, 0x03)]


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
    mem = dut.memory_torch()
    npad = mem.shape[0] * 64

    def col(v):
        x = np.zeros(npad, np.uint8)
        x[:n] = v
        return torch.from_numpy(x.reshape(-1, 64)).cuda()

    for a, v in io.items():
        mem[:, a, :] = col(v)
    w = np.zeros((npad, 0x2000), np.uint8)
    w[:n] = wram
    mem[:, 0xC000:0xE000, :] = torch.from_numpy(w.reshape(-1, 64, 0x2000).transpose(0, 2, 1).copy()).cuda()
    h = np.zeros((npad, 0x7F), np.uint8)
    h[:n] = hram
    mem[:, 0xFF80:0xFFFF, :] = torch.from_numpy(h.reshape(-1, 64, 0x7F).transpose(0, 2, 1).copy()).cuda()
    torch.cuda.synchronize()


def _clear_traps(ref, dut):
    for f in ("trap_flag", "trap_pc", "trap_opcode", "trap_kind"):
        ref.field(f)[:] = 0
        dut.import_field(f, np.zeros(dut.num_envs, np.int64))


@pytest.mark.parametrize("cart", CARTS, ids=["rom_only", "mbc1", "mbc3_ram"])
def test_every_opcode_from_random_states(bootstub, cart):
    require_gpu()
    from gbxcule_amd.backend import HipVecBackend
    from oracle.ref import RefMachine

    rng = np.random.default_rng(1234 + cart[0])
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
        ref.step(acts, 1, 8, "full_step", threads=8)
        dut.step(acts)
        assert_same_state(dut, ref, step=99, tag=f"{cart} frame")
        np.testing.assert_array_equal(dut.export_latches(), ref.latches)
    finally:
        dut.close()
        ref.close()

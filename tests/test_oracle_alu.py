"""Pins the oracle's 8-bit/16-bit ALU and CB semantics against closed forms.

The expected values are written from the published SM83 definitions with a
different formulation than the oracle's (carries from bit arithmetic on the
full-width result, half-carries from ``a ^ b ^ result``), so a dropped term,
swapped operand or wrong flag bit fails here.  Each case executes exactly one
instruction in a separate env.
"""

from __future__ import annotations

import numpy as np
import pytest

from ._isa import flat_rom, oracle, run_instructions, set_regs

ALU = ("ADD", "ADC", "SUB", "SBC", "AND", "XOR", "OR", "CP")


def _flags(z, n, h, c):
    return (z.astype(np.int64) << 7) | (n << 6) | (h.astype(np.int64) << 5) | (c.astype(np.int64) << 4)


def expected_alu(kind: int, a: np.ndarray, v: np.ndarray, cin: np.ndarray):
    """(A', F') for ALU op ``kind`` from the textbook definitions."""
    if kind in (0, 1):  # ADD / ADC
        c = cin if kind == 1 else 0
        full = a + v + c
        res = full & 0xFF
        h = ((a ^ v ^ full) & 0x10) != 0
        return res, _flags(res == 0, 0, h, full > 0xFF)
    if kind in (2, 3, 7):  # SUB / SBC / CP
        c = cin if kind == 3 else 0
        full = a - v - c
        res = full & 0xFF
        h = ((a ^ v ^ full) & 0x10) != 0
        newa = a if kind == 7 else res
        return newa, _flags(res == 0, 1, h, full < 0)
    if kind == 4:
        res = a & v
        return res, _flags(res == 0, 0, np.ones_like(a, bool), np.zeros_like(a, bool))
    res = (a ^ v) if kind == 5 else (a | v)
    return res, _flags(res == 0, 0, np.zeros_like(a, bool), np.zeros_like(a, bool))


@pytest.mark.parametrize("kind", range(8), ids=ALU)
def test_alu_register_operand_exhaustive(kind):
    """ALU A,B over all A, B and carry-in values."""
    op = 0x80 | (kind << 3) | 0  # ALU A,B
    rom = flat_rom({0x150: bytes([op])})
    a_all, v_all, c_all = np.meshgrid(np.arange(256), np.arange(256), np.arange(2), indexing="ij")
    a_all, v_all, c_all = a_all.ravel(), v_all.ravel(), c_all.ravel()
    n = 8192
    m = oracle(rom, n)
    try:
        for lo in range(0, a_all.size, n):
            a, v, c = a_all[lo : lo + n], v_all[lo : lo + n], c_all[lo : lo + n]
            set_regs(m, pc=0x150, a=a, b=v, f=c << 4)
            run_instructions(m, 1)
            ea, ef = expected_alu(kind, a, v, c)
            np.testing.assert_array_equal(m.field("a"), ea)
            np.testing.assert_array_equal(m.field("f"), ef)
            np.testing.assert_array_equal(m.field("pc"), 0x151)
    finally:
        m.close()


@pytest.mark.parametrize("kind", range(8), ids=ALU)
def test_alu_immediate_and_memory_operands(kind):
    """ALU A,d8 and ALU A,(HL) read their operand from the immediate byte and
    from WRAM; results must equal the register form's closed form."""
    rng = np.random.default_rng(kind)
    n = 2048
    imm_rom = {0x150 + 2 * v: bytes([0xC6 | (kind << 3), v]) for v in range(256)}
    imm_rom[0x400] = bytes([0x80 | (kind << 3) | 6])  # ALU A,(HL)
    rom = flat_rom(imm_rom)
    m = oracle(rom, n)
    try:
        a = rng.integers(0, 256, n)
        v = rng.integers(0, 256, n)
        c = rng.integers(0, 2, n)
        set_regs(m, pc=0x150 + 2 * v, a=a, f=c << 4)
        run_instructions(m, 1)
        ea, ef = expected_alu(kind, a, v, c)
        np.testing.assert_array_equal(m.field("a"), ea)
        np.testing.assert_array_equal(m.field("f"), ef)
        np.testing.assert_array_equal(m.field("pc"), 0x150 + 2 * v + 2)
        # (HL) form: operand in WRAM at a random address
        hl = rng.integers(0xC000, 0xE000, n)
        m.mem[np.arange(n), hl] = v
        set_regs(m, pc=0x400, a=a, f=c << 4, h=hl >> 8, l=hl & 0xFF)
        run_instructions(m, 1)
        np.testing.assert_array_equal(m.field("a"), ea)
        np.testing.assert_array_equal(m.field("f"), ef)
    finally:
        m.close()


def test_inc_dec_r8_exhaustive():
    """INC B / DEC B: Z, N, H from the nibble borrow/carry, C preserved."""
    rom = flat_rom({0x150: bytes([0x04]), 0x151: bytes([0x05])})
    v = np.repeat(np.arange(256), 2)
    c = np.tile(np.arange(2), 256)
    m = oracle(rom, v.size)
    try:
        for op_pc, delta in ((0x150, 1), (0x151, -1)):
            set_regs(m, pc=op_pc, b=v, f=c << 4)
            run_instructions(m, 1)
            res = (v + delta) & 0xFF
            h = ((v ^ 1 ^ ((v + delta) & 0x1FF)) & 0x10) != 0
            ef = _flags(res == 0, 1 if delta < 0 else 0, h, c.astype(bool))
            np.testing.assert_array_equal(m.field("b"), res)
            np.testing.assert_array_equal(m.field("f"), ef)
    finally:
        m.close()


def _bcd(x):
    return ((x // 10) << 4) | (x % 10)


def test_daa_gives_bcd_sum_and_difference():
    """ADD/SUB of two packed-BCD bytes followed by DAA yields the decimal sum
    (difference) mod 100 with carry (borrow) -- what DAA exists to do."""
    p, q = np.meshgrid(np.arange(100), np.arange(100), indexing="ij")
    p, q = p.ravel(), q.ravel()
    rom = flat_rom({0x150: bytes([0x80, 0x27]), 0x160: bytes([0x90, 0x27])})
    m = oracle(rom, p.size)
    try:
        set_regs(m, pc=0x150, a=_bcd(p), b=_bcd(q), f=0)
        run_instructions(m, 2)
        s = p + q
        np.testing.assert_array_equal(m.field("a"), _bcd(s % 100))
        np.testing.assert_array_equal((m.field("f") >> 4) & 1, (s >= 100).astype(int))
        np.testing.assert_array_equal((m.field("f") >> 7) & 1, (s % 100 == 0).astype(int))
        set_regs(m, pc=0x160, a=_bcd(p), b=_bcd(q), f=0)
        run_instructions(m, 2)
        d = p - q
        np.testing.assert_array_equal(m.field("a"), _bcd(d % 100))
        np.testing.assert_array_equal((m.field("f") >> 4) & 1, (d < 0).astype(int))
    finally:
        m.close()


def _rot(kind, v, cin):
    """CB rotate/shift group 0 from bit-level definitions -> (result, carry)."""
    b7, b0 = (v >> 7) & 1, v & 1
    if kind == 0:  # RLC
        return ((v << 1) | b7) & 0xFF, b7
    if kind == 1:  # RRC
        return (v >> 1) | (b0 << 7), b0
    if kind == 2:  # RL
        return ((v << 1) | cin) & 0xFF, b7
    if kind == 3:  # RR
        return (v >> 1) | (cin << 7), b0
    if kind == 4:  # SLA
        return (v << 1) & 0xFF, b7
    if kind == 5:  # SRA keeps bit 7
        return (v >> 1) | (v & 0x80), b0
    if kind == 6:  # SWAP
        return ((v << 4) | (v >> 4)) & 0xFF, np.zeros_like(v)
    return v >> 1, b0  # SRL


def test_cb_all_opcodes_on_register_and_memory():
    """Every CB opcode on every operand value (register forms) and on random
    (HL) operands, against bit-level definitions."""
    code = {0x200 + 2 * cb: bytes([0xCB, cb]) for cb in range(256)}
    rom = flat_rom(code)
    cbs = np.repeat(np.arange(256), 512)
    v = np.tile(np.repeat(np.arange(256), 2), 256)
    cin = np.tile(np.arange(2), 256 * 256)
    n = 16384
    for lo in range(0, cbs.size, n):
        cb, val, c = cbs[lo : lo + n], v[lo : lo + n], cin[lo : lo + n]
        m = oracle(rom, cb.size)
        try:
            reg = cb & 7
            hl = 0xC000 + (np.arange(cb.size) % 0x1000)
            regs = {r: np.zeros(cb.size, np.int64) for r in "bcdehla"}
            names = "bcdehl?a"
            for i, r in enumerate(names):
                if r != "?":
                    regs[r] = np.where(reg == i, val, (i * 37 + 11) & 0xFF)
            regs["h"] = np.where(reg == 6, hl >> 8, regs["h"])
            regs["l"] = np.where(reg == 6, hl & 0xFF, regs["l"])
            set_regs(m, pc=0x200 + 2 * cb, f=c << 4, **regs)
            m.mem[np.arange(cb.size), hl] = np.where(reg == 6, val, 0)
            run_instructions(m, 1)
            grp, sub = cb >> 6, (cb >> 3) & 7
            out_reg = np.zeros(cb.size, np.int64)
            for i, r in enumerate(names):
                if r == "?":
                    out_reg = np.where(reg == 6, m.mem[np.arange(cb.size), hl], out_reg)
                else:
                    out_reg = np.where(reg == i, m.field(r), out_reg)
            f = m.field("f")
            exp = val.copy()
            ef = f.copy()
            for k in range(8):
                r_, c_ = _rot(k, val, c)
                sel = (grp == 0) & (sub == k)
                exp = np.where(sel, r_, exp)
                ef = np.where(sel, _flags(r_ == 0, 0, np.zeros_like(sel), c_.astype(bool)), ef)
            bit = (val >> sub) & 1
            ef = np.where(grp == 1, _flags(bit == 0, 0, np.ones_like(bit, bool), c.astype(bool)), ef)
            exp = np.where(grp == 2, val & ~(1 << sub) & 0xFF, exp)
            exp = np.where(grp == 3, val | (1 << sub), exp)
            np.testing.assert_array_equal(out_reg, exp)
            np.testing.assert_array_equal(f, ef)
            np.testing.assert_array_equal(m.field("pc"), 0x200 + 2 * cb + 2)
        finally:
            m.close()


def test_add_hl_rr_and_sp_offset_flags():
    """ADD HL,DE: H from bit 11, C from bit 15, Z kept.  ADD SP,e8 and
    LD HL,SP+e8: H and C from the low nibble/byte of SP + unsigned e8."""
    rng = np.random.default_rng(7)
    n = 8192
    rom = flat_rom({0x150: bytes([0x19])} | {0x200 + 2 * e: bytes([0xE8, e]) for e in range(256)}
                   | {0x400 + 2 * e: bytes([0xF8, e]) for e in range(256)})
    m = oracle(rom, n)
    try:
        hl = rng.integers(0, 0x10000, n)
        de = rng.integers(0, 0x10000, n)
        z = rng.integers(0, 2, n)
        set_regs(m, pc=0x150, h=hl >> 8, l=hl & 0xFF, d=de >> 8, e=de & 0xFF, f=z << 7)
        run_instructions(m, 1)
        s = hl + de
        got = (m.field("h") << 8) | m.field("l")
        np.testing.assert_array_equal(got, s & 0xFFFF)
        hf = ((hl ^ de ^ s) & 0x1000) != 0
        np.testing.assert_array_equal(m.field("f"), _flags(z.astype(bool), 0, hf, s > 0xFFFF))
        sp = rng.integers(0, 0x10000, n)
        e8 = rng.integers(0, 256, n)
        signed = np.where(e8 >= 128, e8 - 256, e8)
        hf = ((sp & 0xF) + (e8 & 0xF)) > 0xF
        cf = ((sp & 0xFF) + e8) > 0xFF
        for base, target in ((0x200, "sp"), (0x400, "hl")):
            set_regs(m, pc=base + 2 * e8, sp=sp, f=0xF0)
            run_instructions(m, 1)
            got = m.field("sp") if target == "sp" else (m.field("h") << 8) | m.field("l")
            np.testing.assert_array_equal(got, (sp + signed) & 0xFFFF)
            np.testing.assert_array_equal(m.field("f"), _flags(np.zeros(n, bool), 0, hf, cf))
    finally:
        m.close()

"""Known answers for every unprefixed opcode outside the 8-bit ALU block.

The expected machine state after one instruction comes from ``sm83_effect``
below, a model written from the published SM83 instruction definitions (Pan
Docs: loads, 16-bit increments, stack, jumps/calls/returns, rotates of A,
CPL/SCF/CCF, DI/EI/RETI) plus the two rules the reference states for them:
EI sets IME at once (``cpu_templates/misc.py:13-34``) and POP AF keeps only
the high nibble of F (``cpu_step_builder.py:1375``).  It shares no code with
the oracle: the model names registers, computes effective addresses and
stack transfers as the instruction set describes them, and the test runs the
oracle one instruction from random register, flag and memory states with
``max_instr`` and compares registers, F, SP, PC, IME, HALT and every byte of
work RAM and high RAM.  Reference templates covered:
``cpu_templates/loads.py:14-893``, ``stack.py:9-1582``,
``jumps.py:13-371``, ``bitops.py:13-48``, ``alu.py:925-950`` and
``misc.py:7-73``.
"""

from __future__ import annotations

import numpy as np
import pytest

from gbxcule_amd.carts.asm import ILLEGAL

from ._isa import flat_rom, oracle, run_instructions, set_regs

R8 = ("b", "c", "d", "e", "h", "l", None, "a")  # operand code 6 is (HL)
PAIRS = {"bc": ("b", "c"), "de": ("d", "e"), "hl": ("h", "l"), "af": ("a", "f")}
COND = ("nz", "z", "nc", "c")


def _pair(st: dict, name: str) -> int:
    if name == "sp":
        return st["sp"]
    hi, lo = PAIRS[name]
    return (st[hi] << 8) | st[lo]


def _set_pair(st: dict, name: str, v: int) -> None:
    v &= 0xFFFF
    if name == "sp":
        st["sp"] = v
        return
    hi, lo = PAIRS[name]
    st[hi], st[lo] = v >> 8, v & 0xFF
    if name == "af":
        st["f"] &= 0xF0


def _cond(st: dict, c: str) -> bool:
    z, cy = bool(st["f"] & 0x80), bool(st["f"] & 0x10)
    return {"nz": not z, "z": z, "nc": not cy, "c": cy}[c]


def sm83_effect(op: int, b1: int, b2: int, st: dict, mem: np.ndarray) -> tuple[dict, dict[int, int]]:
    """New register state and the bytes written, for one instruction at
    ``st['pc']`` whose bytes are ``op, b1, b2``; ``mem`` is read-only."""
    st = dict(st)
    pc = st["pc"]
    imm16 = b1 | (b2 << 8)
    e8 = b1 - 256 if b1 & 0x80 else b1
    writes: dict[int, int] = {}

    def rd(addr: int) -> int:
        addr &= 0xFFFF
        return writes.get(addr, int(mem[addr]))

    def wr(addr: int, v: int) -> None:
        writes[addr & 0xFFFF] = v & 0xFF

    def push16(v: int) -> None:
        st["sp"] = (st["sp"] - 1) & 0xFFFF
        wr(st["sp"], v >> 8)
        st["sp"] = (st["sp"] - 1) & 0xFFFF
        wr(st["sp"], v & 0xFF)

    def pop16() -> int:
        lo = rd(st["sp"])
        hi = rd(st["sp"] + 1)
        st["sp"] = (st["sp"] + 2) & 0xFFFF
        return lo | (hi << 8)

    nxt = pc + 1
    x, y, z = op >> 6, (op >> 3) & 7, op & 7
    rp = ("bc", "de", "hl", "sp")[y >> 1]
    if op == 0x00:
        pass
    elif x == 1:  # LD r,r'
        src = rd(_pair(st, "hl")) if R8[z] is None else st[R8[z]]
        if R8[y] is None:
            wr(_pair(st, "hl"), src)
        else:
            st[R8[y]] = src
    elif x == 0 and z == 6:  # LD r,d8
        nxt = pc + 2
        if R8[y] is None:
            wr(_pair(st, "hl"), b1)
        else:
            st[R8[y]] = b1
    elif x == 0 and z == 1 and not y & 1:  # LD rr,d16
        nxt = pc + 3
        _set_pair(st, rp, imm16)
    elif x == 0 and z == 3:  # INC rr / DEC rr
        _set_pair(st, rp, _pair(st, rp) + (1 if not y & 1 else -1))
    elif x == 0 and z == 2:  # LD (BC)/(DE)/(HL+)/(HL-) with A, both ways
        ptr = ("bc", "de", "hl", "hl")[y >> 1]
        addr = _pair(st, ptr)
        if y & 1:
            st["a"] = rd(addr)
        else:
            wr(addr, st["a"])
        if y >> 1 == 2:
            _set_pair(st, "hl", addr + 1)
        elif y >> 1 == 3:
            _set_pair(st, "hl", addr - 1)
    elif op == 0x08:  # LD (a16),SP: low byte first
        nxt = pc + 3
        wr(imm16, st["sp"] & 0xFF)
        wr(imm16 + 1, st["sp"] >> 8)
    elif op in (0x07, 0x0F, 0x17, 0x1F):  # rotates of A: Z, N, H cleared
        a, cin = st["a"], (st["f"] >> 4) & 1
        if op == 0x07:
            out = a >> 7
            a = ((a << 1) | out) & 0xFF
        elif op == 0x0F:
            out = a & 1
            a = (a >> 1) | (out << 7)
        elif op == 0x17:
            out = a >> 7
            a = ((a << 1) | cin) & 0xFF
        else:
            out = a & 1
            a = (a >> 1) | (cin << 7)
        st["a"], st["f"] = a, out << 4
    elif op == 0x2F:  # CPL: N and H set
        st["a"] ^= 0xFF
        st["f"] = (st["f"] & 0x90) | 0x60
    elif op == 0x37:  # SCF
        st["f"] = (st["f"] & 0x80) | 0x10
    elif op == 0x3F:  # CCF
        st["f"] = (st["f"] & 0x80) | (0x10 ^ (st["f"] & 0x10))
    elif x == 0 and z == 1 and y & 1:  # ADD HL,rr: Z kept, N clear, H bit 11, C bit 15
        hl, v = _pair(st, "hl"), _pair(st, rp)
        h = int((hl & 0xFFF) + (v & 0xFFF) > 0xFFF)
        c = int(hl + v > 0xFFFF)
        _set_pair(st, "hl", hl + v)
        st["f"] = (st["f"] & 0x80) | (h << 5) | (c << 4)
    elif op == 0x18 or op in (0x20, 0x28, 0x30, 0x38):  # JR [cc],e8
        nxt = pc + 2
        if op == 0x18 or _cond(st, COND[y - 4]):
            nxt = pc + 2 + e8
    elif op in (0xC3, 0xC2, 0xCA, 0xD2, 0xDA):  # JP [cc],a16
        nxt = pc + 3
        if op == 0xC3 or _cond(st, COND[y]):
            nxt = imm16
    elif op == 0xE9:  # JP (HL)
        nxt = _pair(st, "hl")
    elif op in (0xCD, 0xC4, 0xCC, 0xD4, 0xDC):  # CALL [cc],a16
        nxt = pc + 3
        if op == 0xCD or _cond(st, COND[y]):
            push16(pc + 3)
            nxt = imm16
    elif op in (0xC9, 0xD9, 0xC0, 0xC8, 0xD0, 0xD8):  # RET [cc], RETI
        if op in (0xC9, 0xD9) or _cond(st, COND[y]):
            nxt = pop16()
        if op == 0xD9:
            st["ime"] = 1
    elif x == 3 and z == 7:  # RST n: pushes the address after it
        push16(pc + 1)
        nxt = y * 8
    elif x == 3 and z == 5 and not y & 1:  # PUSH rr
        push16(_pair(st, ("bc", "de", "hl", "af")[y >> 1]))
    elif x == 3 and z == 1 and not y & 1:  # POP rr
        _set_pair(st, ("bc", "de", "hl", "af")[y >> 1], pop16())
    elif op == 0xE0:
        nxt = pc + 2
        wr(0xFF00 + b1, st["a"])
    elif op == 0xF0:
        nxt = pc + 2
        st["a"] = rd(0xFF00 + b1)
    elif op == 0xE2:
        wr(0xFF00 + st["c"], st["a"])
    elif op == 0xF2:
        st["a"] = rd(0xFF00 + st["c"])
    elif op == 0xEA:
        nxt = pc + 3
        wr(imm16, st["a"])
    elif op == 0xFA:
        nxt = pc + 3
        st["a"] = rd(imm16)
    elif op == 0xF9:
        st["sp"] = _pair(st, "hl")
    elif op in (0xE8, 0xF8):  # ADD SP,e8 / LD HL,SP+e8: carries from the low byte
        nxt = pc + 2
        sp = st["sp"]
        h = int((sp & 0xF) + (b1 & 0xF) > 0xF)
        c = int((sp & 0xFF) + b1 > 0xFF)
        st["f"] = (h << 5) | (c << 4)
        _set_pair(st, "sp" if op == 0xE8 else "hl", sp + e8)
    elif op == 0xF3:
        st["ime"] = 0
    elif op == 0xFB:
        st["ime"] = 1
    else:
        raise KeyError(f"opcode {op:#04x} is not in this model")
    st["pc"] = nxt & 0xFFFF
    return st, writes


ALU_BLOCK = set(range(0x80, 0xC0)) | {0xC6, 0xCE, 0xD6, 0xDE, 0xE6, 0xEE, 0xF6, 0xFE}
INC_DEC_8 = {op for op in range(0x40) if op & 7 in (4, 5)} | {0x27}  # INC/DEC r, DAA
OPCODES = [
    op for op in range(256)
    if op not in ILLEGAL and op not in ALU_BLOCK and op not in INC_DEC_8
    and op not in (0x10, 0x76, 0xCB)
]  # fmt: skip
STATES = 12  # random states per opcode
REGS = ("a", "f", "b", "c", "d", "e", "h", "l", "sp", "pc", "ime")


def _operands(op: int, rng) -> tuple[int, int]:
    """Immediate bytes keeping memory operands in work RAM / high RAM."""
    b1, b2 = int(rng.integers(0, 256)), int(rng.integers(0, 256))
    if op in (0xEA, 0xFA, 0x08):
        a = int(rng.integers(0xC000, 0xDFFF))
        b1, b2 = a & 0xFF, a >> 8
    if op in (0xE0, 0xF0):
        b1 = int(rng.integers(0x80, 0xFF))
    return b1, b2


@pytest.fixture(scope="module")
def oracle_run():
    """The oracle after one instruction from random states: every opcode of
    OPCODES from STATES states, one env each."""
    rng = np.random.default_rng(1234)
    ops = np.repeat(np.array(OPCODES), STATES)
    n = ops.size
    pcs = 0x0200 + 4 * np.arange(n)
    assert pcs[-1] + 3 < 0x4000
    imm = [_operands(int(op), rng) for op in ops]
    blocks = {int(pc): bytes([int(op), b1, b2]) for pc, op, (b1, b2) in zip(pcs, ops, imm)}
    rom = flat_rom(blocks)
    m = oracle(rom, n, pc=pcs)
    try:
        regs = {r: rng.integers(0, 256, n) for r in "abcdehl"}
        regs["f"] = rng.integers(0, 16, n) << 4
        # pointers into work RAM or high RAM (no IO side effects), stack inside work RAM
        hl = np.where(rng.random(n) < 0.8, rng.integers(0xC000, 0xE000, n), rng.integers(0xFF80, 0xFFFF, n))
        bc = rng.integers(0xC000, 0xE000, n)
        de = rng.integers(0xC000, 0xE000, n)
        regs["h"], regs["l"] = hl >> 8, hl & 0xFF
        regs["b"], regs["c"] = bc >> 8, bc & 0xFF
        regs["d"], regs["e"] = de >> 8, de & 0xFF
        # LD (C),A / LD A,(C) address FF00+C: keep C in high RAM for them
        is_c_io = np.isin(ops, [0xE2, 0xF2])
        regs["c"] = np.where(is_c_io, rng.integers(0x80, 0xFF, n), regs["c"])
        regs["sp"] = rng.integers(0xC002, 0xDFFE, n)
        regs["ime"] = rng.integers(0, 2, n)
        set_regs(m, **regs)
        m.mem[:, 0xC000:0xE000] = rng.integers(0, 256, (n, 0x2000), dtype=np.uint8)
        m.mem[:, 0xFF80:0xFFFF] = rng.integers(0, 256, (n, 0x7F), dtype=np.uint8)
        before = m.mem.copy()
        st0 = {r: m.field(r).astype(np.int64).copy() for r in REGS}
        run_instructions(m, 1)
        after_regs = {r: m.field(r).astype(np.int64).copy() for r in REGS + ("halted",)}
        yield ops, imm, st0, before, after_regs, m.mem.copy()
    finally:
        m.close()


REGION = np.r_[0xC000:0xE000, 0xFF80:0xFFFF]


def _mismatches(run, model) -> list[str]:
    ops, imm, st0, before, after_regs, after = run
    bad = []
    for i in range(ops.size):
        op, (b1, b2) = int(ops[i]), imm[i]
        st = {r: int(st0[r][i]) for r in REGS}
        want, writes = model(op, b1, b2, st, before[i])
        got = {r: int(after_regs[r][i]) for r in REGS}
        exp = before[i].copy()
        for a, v in writes.items():
            exp[a] = v
        if got != want:
            bad.append(f"op {op:#04x} env {i}: registers {got} != {want}")
        elif not np.array_equal(after[i, REGION], exp[REGION]):
            diff = REGION[np.nonzero(after[i, REGION] != exp[REGION])[0]]
            bad.append(f"op {op:#04x} env {i}: memory differs at {[hex(a) for a in diff[:4]]}")
        elif after_regs["halted"][i] != 0:
            bad.append(f"op {op:#04x} env {i}: halted")
    return bad


def test_unprefixed_non_alu_opcodes_from_random_states(oracle_run):
    bad = _mismatches(oracle_run, sm83_effect)
    assert not bad, f"{len(bad)} mismatches, first: {bad[:3]}"


def _mutant(kind: str):
    """The model with one plausible mistake planted."""

    def model(op, b1, b2, st, mem):
        if kind == "push_order" and op in (0xC5, 0xD5, 0xE5, 0xF5):
            want, w = sm83_effect(op, b1, b2, st, mem)
            sp = want["sp"]
            return want, {sp: w[(sp + 1) & 0xFFFF], (sp + 1) & 0xFFFF: w[sp]}
        if kind == "sp_store_big_endian" and op == 0x08:
            want, w = sm83_effect(op, b1, b2, st, mem)
            a = b1 | (b2 << 8)
            return want, {a: st["sp"] >> 8, (a + 1) & 0xFFFF: st["sp"] & 0xFF}
        if kind == "jr_unsigned" and op == 0x18:
            want, w = sm83_effect(op, b1, b2, st, mem)
            want["pc"] = (st["pc"] + 2 + b1) & 0xFFFF
            return want, w
        if kind == "rlca_keeps_z" and op == 0x07:
            want, w = sm83_effect(op, b1, b2, st, mem)
            want["f"] |= st["f"] & 0x80
            return want, w
        if kind == "call_pushes_pc" and op == 0xCD:
            st2 = dict(st)
            st2["pc"] = (st["pc"] - 3) & 0xFFFF  # pushes the CALL's own address
            want, w = sm83_effect(op, b1, b2, st2, mem)
            return want, w
        if kind == "hl_minus_is_plus" and op == 0x3A:
            want, w = sm83_effect(0x2A, b1, b2, st, mem)
            return want, w
        if kind == "reti_keeps_ime" and op == 0xD9:
            want, w = sm83_effect(op, b1, b2, st, mem)
            want["ime"] = st["ime"]
            return want, w
        if kind == "cpl_clears_h" and op == 0x2F:
            want, w = sm83_effect(op, b1, b2, st, mem)
            want["f"] &= ~0x20
            return want, w
        return sm83_effect(op, b1, b2, st, mem)

    return model


@pytest.mark.parametrize(
    "kind",
    ["push_order", "sp_store_big_endian", "jr_unsigned", "rlca_keeps_z", "call_pushes_pc",
     "hl_minus_is_plus", "reti_keeps_ime", "cpl_clears_h"],
)  # fmt: skip
def test_planted_model_mistakes_are_caught(oracle_run, kind):
    """The comparison discriminates: each planted mistake disagrees with the
    oracle on at least one of the random states."""
    assert _mismatches(oracle_run, _mutant(kind))


@pytest.mark.parametrize(
    "op,regs,want",
    [
        # 16-bit INC/DEC wrap, flags untouched
        (0x03, dict(b=0xFF, c=0xFF, f=0xB0), dict(b=0x00, c=0x00, f=0xB0)),
        (0x1B, dict(d=0x00, e=0x00, f=0x50), dict(d=0xFF, e=0xFF, f=0x50)),
        (0x33, dict(sp=0xFFFF), dict(sp=0x0000)),
        (0x2B, dict(h=0x01, l=0x00), dict(h=0x00, l=0xFF)),
        # rotates of A always clear Z (A = 0 after RLCA of 0)
        (0x07, dict(a=0x00, f=0x80), dict(a=0x00, f=0x00)),
        (0x17, dict(a=0x80, f=0x00), dict(a=0x00, f=0x10)),
        (0x1F, dict(a=0x01, f=0x10), dict(a=0x80, f=0x10)),
        (0x0F, dict(a=0x01, f=0x00), dict(a=0x80, f=0x10)),
        # CPL / SCF / CCF keep Z
        (0x2F, dict(a=0x35, f=0x90), dict(a=0xCA, f=0xF0)),
        (0x37, dict(f=0xE0), dict(f=0x90)),
        (0x3F, dict(f=0x90), dict(f=0x80)),
        (0x3F, dict(f=0x00), dict(f=0x10)),
    ],
)
def test_single_opcode_known_values(op, regs, want):
    rom = flat_rom({0x200: bytes([op, 0, 0])})
    m = oracle(rom, 1, pc=0x200)
    try:
        set_regs(m, **regs)
        run_instructions(m, 1)
        for k, v in want.items():
            assert int(m.field(k)[0]) == v, (hex(op), k, int(m.field(k)[0]), v)
    finally:
        m.close()


def test_stack_byte_order_known_values():
    """LD (a16),SP stores low then high; PUSH BC stores B at SP-1 and C at
    SP-2; CALL pushes the address after it high byte first; POP AF drops
    F's low nibble."""
    code = bytes([0x08, 0x00, 0xC1, 0xC5, 0xCD, 0x34, 0x12])
    rom = flat_rom({0x200: code, 0x1234: bytes([0xF1])})
    m = oracle(rom, 1, pc=0x200)
    try:
        set_regs(m, sp=0xD00E, b=0xAB, c=0xCD)
        run_instructions(m, 1)  # LD (C100),SP
        assert (int(m.mem[0, 0xC100]), int(m.mem[0, 0xC101])) == (0x0E, 0xD0)
        run_instructions(m, 1)  # PUSH BC
        assert int(m.field("sp")[0]) == 0xD00C
        assert (int(m.mem[0, 0xD00D]), int(m.mem[0, 0xD00C])) == (0xAB, 0xCD)
        run_instructions(m, 1)  # CALL 1234: pushes 0x0207
        assert int(m.field("pc")[0]) == 0x1234 and int(m.field("sp")[0]) == 0xD00A
        assert (int(m.mem[0, 0xD00B]), int(m.mem[0, 0xD00A])) == (0x02, 0x07)
        run_instructions(m, 1)  # POP AF: A = 0x02, F = 0x07 & 0xF0
        assert (int(m.field("a")[0]), int(m.field("f")[0])) == (0x02, 0x00)
        assert int(m.field("sp")[0]) == 0xD00C
    finally:
        m.close()

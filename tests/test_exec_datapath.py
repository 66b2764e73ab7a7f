"""The step kernel's instruction decode (gbx_decode.h) and straight-line
datapath (gbx_exec.h), built for the host, against the oracle: every
unprefixed and CB opcode from random register, flag and memory states.

Bus operands are steered into WRAM/HRAM (address registers, SP, a8/a16
immediates), so the bytes the datapath reads and writes are plain memory
and the expected values come from the oracle's memory image.  The oracle
runs exactly one instruction per env (debug max-instruction trap); the
registers, F, SP, next pc, IME/HALT/trap and every byte of memory must then
equal what the datapath produced.  The datapath's cycle count must match
the public opcode table, taken or not taken as F decides.
"""

from __future__ import annotations

import ctypes
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

from gbxcule_amd.carts.asm import ILLEGAL

from ._isa import flat_rom, oracle, set_regs

ROOT = Path(__file__).resolve().parent
OPS = [op for op in range(256) if op != 0xCB] + [0x100 | cb for cb in range(256)]


@pytest.fixture(scope="module")
def harness(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    out = tmp_path_factory.mktemp("exec") / "exec_harness.so"
    subprocess.run(
        [gxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-o", str(out),
         str(ROOT / "native" / "exec_harness.cpp")],
        check=True,
    )  # fmt: skip
    lib = ctypes.CDLL(str(out))
    u32p = ctypes.POINTER(ctypes.c_uint32)
    lib.harness_decode.argtypes = [ctypes.c_uint32] * 3 + [u32p]
    lib.harness_exec.argtypes = [u32p, u32p]
    lib.harness_poll.argtypes = [ctypes.c_char_p, ctypes.c_uint32, u32p]
    lib.harness_copy.argtypes = [ctypes.c_char_p, u32p]
    return lib


def _arr(n):
    return (ctypes.c_uint32 * n)()


def _states(rng, n):
    """Registers with every address register, SP and C pointing into RAM."""
    r = {
        "a": rng.integers(0, 256, n),
        "b": rng.integers(0xC0, 0xE0, n),
        "c": rng.integers(0x80, 0xFE, n),
        "d": rng.integers(0xC0, 0xE0, n),
        "e": rng.integers(0, 256, n),
        "h": rng.integers(0xC0, 0xE0, n),
        "l": rng.integers(0, 256, n),
        "f": rng.integers(0, 16, n) << 4,
        "sp": rng.integers(0xC004, 0xDFFC, n),
        "ime": rng.integers(0, 2, n),
    }
    # HL, BC, DE + 1 must stay below E000 (echo RAM) for two-byte accesses
    for hi, lo in (("h", "l"), ("b", "c"), ("d", "e")):
        v = (r[hi] << 8) | r[lo]
        r[lo] = np.where(v >= 0xDFFE, r[lo] & 0x7F, r[lo])
    return r


def _expected_cycles(op: int, f: int) -> int:
    """Opcode-table cycles of op (0x100 | cb for CB) with flags f; 0 for a trap."""
    from .test_oracle_programs import LEGAL, table_cycles

    if op & 0x100:
        cb = op & 0xFF
        return 8 if cb & 7 != 6 else 12 if cb >> 6 == 1 else 16
    if op == 0x76:  # HALT
        return 4
    if op not in LEGAL:  # STOP and the unused opcodes trap
        return 0
    taken, not_taken = table_cycles(op)
    if op in (0x20, 0x28, 0x30, 0x38, 0xC0, 0xC8, 0xD0, 0xD8, 0xC2, 0xCA, 0xD2, 0xDA,
              0xC4, 0xCC, 0xD4, 0xDC):  # fmt: skip
        cc = (op >> 3) & 3  # NZ Z NC C
        flag = (f >> 7) & 1 if cc < 2 else (f >> 4) & 1
        return taken if flag == (cc & 1) else not_taken
    return taken


@pytest.mark.parametrize("seed", [11, 12])
def test_datapath_matches_oracle(harness, seed):
    rng = np.random.default_rng(seed)
    ops = np.array(OPS * 3)
    n = ops.size
    pcs = 0x200 + 4 * np.arange(n)
    b1 = rng.integers(0, 256, n)
    b2 = rng.integers(0, 256, n)
    for i, op in enumerate(ops):
        if op in (0xEA, 0xFA, 0x08):  # a16 operand in WRAM
            b2[i] = rng.integers(0xC0, 0xE0)
            b1[i] = rng.integers(0, 0xFE)
        elif op in (0xE0, 0xF0):  # a8 operand in HRAM
            b1[i] = rng.integers(0x80, 0xFE)
    blocks = {}
    for i, op in enumerate(ops):
        code = [0xCB, op & 0xFF, b2[i]] if op & 0x100 else [op, b1[i], b2[i]]
        blocks[int(pcs[i])] = bytes(int(x) for x in code)
    # CB opcodes: byte 1 is the CB sub-opcode, byte 2 the next byte
    b1 = np.where(ops & 0x100, ops & 0xFF, b1)
    rom = flat_rom(blocks)
    m = oracle(rom, n, pcs)
    regs = _states(rng, n)
    set_regs(m, **regs)
    m.mem[:, 0xC000:0xE000] = rng.integers(0, 256, (n, 0x2000), dtype=np.uint8)
    m.mem[:, 0xFF80:0xFFFF] = rng.integers(0, 256, (n, 0x7F), dtype=np.uint8)
    mem0 = m.mem.copy()
    m.set_debug(max_instr=1)
    m.step(None, frames=1, release=8)

    rec, inp, out = _arr(16), _arr(22), _arr(12)
    bad = []
    for i, op in enumerate(ops):
        opb = 0xCB if op & 0x100 else int(op)
        harness.harness_decode(opb, int(b1[i]), int(b2[i]), rec)
        w0 = (int(regs["b"][i]) << 24) | (int(regs["c"][i]) << 16) | (int(regs["d"][i]) << 8)
        w0 |= int(regs["e"][i])
        w1 = (int(regs["h"][i]) << 24) | (int(regs["l"][i]) << 16) | (int(regs["f"][i]) << 8)
        w1 |= int(regs["a"][i])
        sp = int(regs["sp"][i])
        # operand address as the datapath computes it; the bytes there
        for k in range(16):
            inp[k] = rec[k]
        inp[16], inp[17], inp[18], inp[19] = w0, w1, sp, int(pcs[i])
        inp[20] = inp[21] = 0
        harness.harness_exec(inp, out)
        ra = out[0]
        inp[20] = int(mem0[i, ra & 0xFFFF])
        inp[21] = int(mem0[i, (ra + 1) & 0xFFFF])
        harness.harness_exec(inp, out)
        o = list(out)
        misc = o[11]
        want = {
            "a": o[2] & 0xFF, "b": o[1] >> 24, "c": (o[1] >> 16) & 0xFF, "d": (o[1] >> 8) & 0xFF,
            "e": o[1] & 0xFF, "h": o[2] >> 24, "l": (o[2] >> 16) & 0xFF, "f": (o[2] >> 8) & 0xFF,
            "sp": o[3], "pc": o[4],
        }  # fmt: skip
        want["ime"] = (misc >> 1) & 1 if misc & 1 else int(regs["ime"][i])
        want["halted"] = (misc >> 2) & 1
        cyc = _expected_cycles(int(op), int(regs["f"][i]))
        if o[5] != cyc:
            bad.append(f"op {op:#05x}: cycles datapath={o[5]} table={cyc}")
        for name, v in want.items():
            got = int(m.field(name)[i])
            if got != v:
                bad.append(f"op {op:#05x}: {name} datapath={v:#x} oracle={got:#x}")
        exp = mem0[i].copy()
        if o[6] > 2 or any(x > 0xFF for x in (o[8], o[10])):
            bad.append(f"op {op:#05x}: bad write list {o[6:11]}")
            continue
        for k in range(o[6]):
            a, v = (o[7], o[8]) if k == 0 else (o[9], o[10])
            exp[a & 0xFFFF] = v
        if not np.array_equal(exp, m.mem[i]):
            d = np.nonzero(exp != m.mem[i])[0]
            bad.append(f"op {op:#05x}: memory differs at {[hex(x) for x in d[:4]]}")
        trapped = int(m.field("trap_kind")[i]) == 1
        if bool((misc >> 3) & 1) != trapped or (trapped and op not in ILLEGAL | {0x10}):
            bad.append(f"op {op:#05x}: trap datapath={misc >> 3} oracle kind={m.field('trap_kind')[i]}")
    assert not bad, f"{len(bad)} mismatches:\n" + "\n".join(bad[:30])


LEN3 = {0x01, 0x11, 0x21, 0x31, 0x08, 0xC2, 0xC3, 0xC4, 0xCA, 0xCC, 0xCD, 0xD2, 0xD4, 0xDA,
        0xDC, 0xEA, 0xFA}  # fmt: skip
LEN2 = {0x06, 0x0E, 0x16, 0x1E, 0x26, 0x2E, 0x36, 0x3E, 0x18, 0x20, 0x28, 0x30, 0x38, 0xC6,
        0xCE, 0xD6, 0xDE, 0xE6, 0xEE, 0xF6, 0xFE, 0xE0, 0xF0, 0xE8, 0xF8}  # fmt: skip


def test_record_cycles_and_lengths_match_opcode_table(harness):
    """Length and both cycle counts of every record against the public SM83
    opcode table (the same table the oracle's cycle-count test uses)."""
    from .test_oracle_programs import LEGAL, table_cycles

    rec = _arr(16)
    for op in LEGAL:
        harness.harness_decode(op, 0, 0, rec)
        taken, not_taken = ((rec[0] >> 26) & 7) * 4, (rec[0] >> 29) * 4
        assert (taken, not_taken) == table_cycles(op), f"op {op:#04x}"
        exp_len = 3 if op in LEN3 else 2 if op in LEN2 else 1
        assert (rec[0] >> 24) & 3 == exp_len, f"op {op:#04x} length"
    for cb in range(256):
        harness.harness_decode(0xCB, cb, 0, rec)
        exp = 8 if cb & 7 != 6 else 12 if cb >> 6 == 1 else 16
        assert ((rec[0] >> 26) & 7) * 4 == exp, f"cb {cb:#04x}"
        assert (rec[0] >> 24) & 3 == 2


def test_poll_loop_marking(harness):
    """The record builder marks exactly a load of LY into A (LDH A,(44) or
    LD A,(FF44)), CP d8 and a conditional jump back (JR cc onto the load, or
    JP cc,a16 below 0x8000, whose target the kernel checks against the pc),
    and stores the compare constant, the condition, the pass cycles and the
    JP target."""
    out = _arr(3)

    def mark(code: bytes):
        harness.harness_poll(code + bytes(8 - len(code)), len(code), out)
        return int(out[0]), int(out[1]), int(out[2])

    for load, ncyc in ((bytes([0xF0, 0x44]), 12), (bytes([0xFA, 0x44, 0xFF]), 16)):
        n = len(load)
        for cc in range(4):
            jr = bytes([0x20 + 8 * cc, (0x100 - (n + 4)) & 0xFF])
            ln, fl, dw = mark(load + bytes([0xFE, 0x90]) + jr)
            assert ln == n + 4 and fl & (1 << 28)
            assert dw == 0x90 | (cc << 8) | ((ncyc + 8 + 12) // 4 << 10)
            # the load itself still decodes and executes as a load
            assert (fl & ~(1 << 28)) & (0x7F << 24) == 0
            jp = bytes([0xC2 + 8 * cc, 0x34, 0x12])
            ln, fl, dw = mark(load + bytes([0xFE, 0x90]) + jp)
            assert ln == n + 5 and fl & (1 << 28)
            assert dw == 0x90 | (cc << 8) | ((ncyc + 8 + 16) // 4 << 10) | (1 << 14) | (0x1234 << 16)
    for bad in (
        [0xF0, 0x45, 0xFE, 0x90, 0x20, 0xFA],  # not LY
        [0xF0, 0x44, 0xE6, 0x90, 0x20, 0xFA],  # AND, not CP
        [0xF0, 0x44, 0xFE, 0x90, 0x18, 0xFA],  # unconditional JR
        [0xF0, 0x44, 0xFE, 0x90, 0x20, 0xFB],  # jumps elsewhere
        [0xFA, 0x44, 0xFF, 0xFE, 0x90, 0x20, 0xFA],  # LD A,(FF44) with the LDH's displacement
        [0xFA, 0x45, 0xFF, 0xFE, 0x90, 0x20, 0xF9],  # LD A,(FF45)
        [0xFA, 0x44, 0xFE, 0xFE, 0x90, 0x20, 0xF9],  # LD A,(FE44)
        [0xF0, 0x44, 0xFE, 0x90, 0xC3, 0x50, 0x01],  # unconditional JP
        [0xF0, 0x44, 0xFE, 0x90, 0xC2, 0x00, 0xC0],  # JP into RAM
        [0xF0, 0x44, 0xFE, 0x90, 0xC4, 0x50, 0x01],  # CALL
        [0xF0, 0x44, 0xFE],  # truncated
    ):
        ln, fl, _ = mark(bytes(bad))
        assert ln == 0 and not fl & (1 << 28), bad


def test_poll_loops_in_carts_are_marked(harness):
    """Every LY poll loop of the poll parity carts, in each of its forms, is
    marked, so those tests run the batched passes; the two loads of the JP
    pair are marked as well (their targets are only checked at run time)."""
    from tests.test_gpu_poll import CASES, FORM_CASES, poll_cart

    out = _arr(3)

    def marked(rom: bytes) -> int:
        return sum(1 for i in range(0x150, 0x8000 - 8)
                   if (harness.harness_poll(rom[i : i + 8], 8, out), out[0])[1] != 0)  # fmt: skip

    for case in CASES[:3]:
        assert marked(poll_cart(*case)) == 4 + (1 if case[4] else 0)
    forms = ("ld_jr", "ldh_jp", "ld_jp", "ldh_jr", "ld_jp")
    for case in FORM_CASES:
        seed, ime, ie, tac, lcd_off, stat, halt = case
        rom = poll_cart(seed, ime, ie, tac, lcd_off, stat, halt, forms, True)
        assert marked(rom) == 4 + (1 if lcd_off else 0) + 2


def test_copy_loop_marking(harness):
    """The record builder marks exactly LD A,(HL+); LD (DE),A; INC DE; DEC BC;
    LD A,B; OR C (or LD A,C; OR B); JR NZ back to the LD (displacement -8),
    and the marked LD A,(HL+)
    still decodes as itself (one read, no writes, 8 cycles)."""
    out = _arr(3)
    plain = _arr(16)
    harness.harness_decode(0x2A, 0x12, 0x13, plain)
    for tail in ([0x78, 0xB1], [0x79, 0xB0]):
        harness.harness_copy(bytes([0x2A, 0x12, 0x13, 0x0B] + tail + [0x20, 0xF8]), out)
        assert out[0] == 1 and out[1] == plain[10] | (1 << 28) and out[2] == 1 << 31
        assert plain[15] == 0 and (plain[7] >> 8) & 3 == 1 and (plain[11] >> 5) & 3 == 0
    for bad in (
        [0x2A, 0x12, 0x13, 0x0B, 0x78, 0xB1, 0x20, 0xF9],  # jumps into the loop
        [0x2A, 0x12, 0x13, 0x0B, 0x78, 0xB1, 0x28, 0xF8],  # JR Z
        [0x2A, 0x12, 0x13, 0x0B, 0x78, 0xB0, 0x20, 0xF8],  # LD A,B; OR B
        [0x3A, 0x12, 0x13, 0x0B, 0x78, 0xB1, 0x20, 0xF8],  # LD A,(HL-)
        [0x2A, 0x12, 0x1B, 0x0B, 0x78, 0xB1, 0x20, 0xF8],  # DEC DE
        [0x2A, 0x22, 0x13, 0x0B, 0x78, 0xB1, 0x20, 0xF8],  # LD (HL+),A
    ):
        harness.harness_copy(bytes(bad), out)
        assert out[0] == 0 and not out[1] & (1 << 28)


def test_copy_loops_in_carts_are_marked(harness):
    """Every copy loop of the C3 cart and of the copy-loop parity carts
    matches the marked pattern, so those tests run the batched passes."""
    from gbxcule_amd.carts.synth import cart_c3
    from tests.test_gpu_copy import CASES, copy_cart

    out = _arr(3)

    def marked(rom: bytes) -> int:
        return sum(1 for i in range(len(rom) - 8) if rom[i] == 0x2A and
                   (harness.harness_copy(rom[i : i + 8], out), out[0])[1] == 1)  # fmt: skip

    assert marked(cart_c3(2)) == 4
    for case in CASES:
        assert marked(copy_cart(*case)) == (13 if case[5] else 12)

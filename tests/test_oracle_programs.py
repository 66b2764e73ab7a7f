"""Known-answer programs that pin the oracle beyond single ALU ops.

Each expected value follows from the published SM83/DMG behaviour as the
reference defines it (including the reference's documented quirks), not from
the oracle's code: cycle counts from the public opcode table, post-boot
registers, JOYP bit layout, timer edges and PPU lines from cycle-by-cycle
brute force, interrupt vectors, MBC bank arithmetic, DMA, serial.
"""

from __future__ import annotations

import numpy as np
import pytest

from gbxcule_amd.carts.asm import Asm, ILLEGAL

from ._isa import flat_rom, oracle, run_frames, run_instructions, set_regs

# ---------------------------------------------------------------------------
# Cycle table (T-states) from the public SM83 opcode table; (taken, not taken)
# ---------------------------------------------------------------------------


def table_cycles(op: int) -> tuple[int, int]:
    hi, lo = op >> 4, op & 0xF
    if 0x40 <= op < 0x80:
        return (8, 8) if (op & 7) == 6 or (op >> 3) & 7 == 6 else (4, 4)
    if 0x80 <= op < 0xC0:
        return (8, 8) if (op & 7) == 6 else (4, 4)
    fixed = {
        0x00: 4, 0x01: 12, 0x02: 8, 0x03: 8, 0x07: 4, 0x08: 20, 0x09: 8, 0x0A: 8,
        0x0B: 8, 0x0F: 4, 0x11: 12, 0x12: 8, 0x13: 8, 0x17: 4, 0x18: 12, 0x19: 8,
        0x1A: 8, 0x1B: 8, 0x1F: 4, 0x21: 12, 0x22: 8, 0x23: 8, 0x27: 4, 0x29: 8,
        0x2A: 8, 0x2B: 8, 0x2F: 4, 0x31: 12, 0x32: 8, 0x33: 8, 0x34: 12, 0x35: 12,
        0x36: 12, 0x37: 4, 0x39: 8, 0x3A: 8, 0x3B: 8, 0x3F: 4, 0xC3: 16, 0xC9: 16,
        0xCD: 24, 0xD9: 16, 0xE0: 12, 0xE2: 8, 0xE8: 16, 0xE9: 4, 0xEA: 16,
        0xF0: 12, 0xF2: 8, 0xF3: 4, 0xF8: 12, 0xF9: 8, 0xFA: 16, 0xFB: 4,
    }  # fmt: skip
    if op in fixed:
        return fixed[op], fixed[op]
    if hi < 4 and lo in (0x4, 0x5, 0xC, 0xD):
        return 4, 4  # INC/DEC r
    if hi < 4 and lo in (0x6, 0xE):
        return 8, 8  # LD r,d8
    if op in (0x20, 0x28, 0x30, 0x38):
        return 12, 8
    if op in (0xC0, 0xC8, 0xD0, 0xD8):
        return 20, 8
    if op in (0xC2, 0xCA, 0xD2, 0xDA):
        return 16, 12
    if op in (0xC4, 0xCC, 0xD4, 0xDC):
        return 24, 12
    if op in (0xC1, 0xD1, 0xE1, 0xF1):
        return 12, 12
    if op in (0xC5, 0xD5, 0xE5, 0xF5):
        return 16, 16
    if op in (0xC6, 0xCE, 0xD6, 0xDE, 0xE6, 0xEE, 0xF6, 0xFE):
        return 8, 8
    if op & 0xC7 == 0xC7:
        return 16, 16  # RST
    raise KeyError(hex(op))


LEGAL = [op for op in range(256) if op not in ILLEGAL and op not in (0xCB, 0x10, 0x76)]


def test_cycle_counts_match_opcode_table():
    """cycle_count after one instruction equals the table value, for every
    legal opcode with conditions both true and false, and every CB opcode."""
    ops = np.array(LEGAL + [0x100 | cb for cb in range(256)])
    envs = np.repeat(ops, 2)
    cond = np.tile(np.arange(2), ops.size)
    blocks = {}
    for k, op in enumerate(ops):
        addr = 0x200 + 4 * k
        blocks[addr] = bytes([0xCB, op & 0xFF, 0, 0]) if op & 0x100 else bytes([op, 0x00, 0xC1, 0])
    rom = flat_rom(blocks)
    idx = np.repeat(np.arange(ops.size), 2)
    m = oracle(rom, envs.size, pc=0x200 + 4 * idx)
    try:
        # flags: env pair (0, 1) = (all clear, all set) so every condition is
        # both taken and not taken once
        set_regs(m, f=np.where(cond == 1, 0xF0, 0x00), sp=0xDFF0, h=0xC1, l=0x23)
        run_instructions(m, 2)  # the second instruction traps before counting
        got = m.field("cycle_count")
        for i, op in enumerate(envs):
            if op & 0x100:
                cb = op & 0xFF
                want = 8 if cb & 7 != 6 else (12 if 0x40 <= cb < 0x80 else 16)
            else:
                taken, not_taken = table_cycles(int(op))
                c = cond[i]
                z, cf = c, c
                cc = {0x20: not z, 0x28: z, 0x30: not cf, 0x38: cf}
                ccs = {0: not z, 1: z, 2: not cf, 3: cf}
                if op in cc:
                    want = taken if cc[op] else not_taken
                elif op in (0xC0, 0xC8, 0xD0, 0xD8, 0xC2, 0xCA, 0xD2, 0xDA, 0xC4, 0xCC, 0xD4, 0xDC):
                    want = taken if ccs[(op >> 3) & 3] else not_taken
                else:
                    want = taken
            assert got[i] == want, f"op {op:#x} cond {cond[i]}: {got[i]} != {want}"
    finally:
        m.close()


def test_illegal_opcodes_trap_with_pc_and_opcode():
    """STOP and the 11 holes freeze the env: trap kind 1 at the opcode's PC."""
    ops = [0x10] + sorted(ILLEGAL)
    rom = flat_rom({0x300 + k: bytes([op]) for k, op in enumerate(ops)})
    m = oracle(rom, len(ops), pc=0x300 + np.arange(len(ops)))
    try:
        run_frames(m, 1)
        np.testing.assert_array_equal(m.field("trap_flag"), 1)
        np.testing.assert_array_equal(m.field("trap_kind"), 1)
        np.testing.assert_array_equal(m.field("trap_pc"), 0x300 + np.arange(len(ops)))
        np.testing.assert_array_equal(m.field("trap_opcode"), ops)
        np.testing.assert_array_equal(m.field("instr_count"), 0)
    finally:
        m.close()


def test_boot_stub_hands_over_documented_post_boot_state(bootstub):
    """From power-on, the boot image runs with the overlay on and reaches
    0x0100 with the documented DMG post-boot registers and the overlay off."""
    from oracle.ref import RefMachine

    rom = flat_rom({0x100: bytes([0x00, 0xC3, 0x00, 0x01])})
    m = RefMachine(4, rom, bootstub)
    try:
        m.set_debug(trap_pc=0x100)
        m.step(None, frames=4)
        st = m.scalars()
        assert (st["trap_kind"] == 5).all() and (st["pc"] == 0x100).all()
        want = dict(a=0x01, f=0xB0, b=0x00, c=0x13, d=0x00, e=0xD8, h=0x01, l=0x4D, sp=0xFFFE)
        for k, v in want.items():
            assert (st[k] == v).all(), k
        assert (m.mem[:, 0xFF40] == 0x91).all() and (m.mem[:, 0xFF47] == 0xFC).all()
        assert (m.cart_state[:, 6] == 0).all()  # boot overlay disabled by FF50
    finally:
        m.close()


def test_sum_loop_value_and_cycles():
    a = Asm(0x150)
    a.ld_r_d8("A", 0)
    a.ld_r_d8("B", 10)
    a.label("loop")
    a.alu_r("ADD", "B")
    a.dec_r("B")
    a.jr("loop", "NZ")
    a.label("end")
    a.jr("end")
    rom = flat_rom({0x150: a.resolve()})
    m = oracle(rom, 1)
    try:
        run_instructions(m, 2 + 30 + 1)
        assert m.field("a")[0] == 55
        assert m.field("b")[0] == 0
        # 8 + 8 + 10*(4 + 4) + 9*12 + 8
        assert m.field("cycle_count")[0] == 8 + 8 + 80 + 108 + 8
    finally:
        m.close()


def test_stack_call_ret_and_push_pop_af():
    a = Asm(0x150)
    a.ld_rr_d16("SP", 0xDFF0)
    a.ld_rr_d16("BC", 0x1234)
    a.push("BC")
    a.pop("DE")
    a.ld_rr_d16("BC", 0x12FF)
    a.push("BC")
    a.pop("AF")
    a.call("sub")
    a.label("after_call")
    a.ld_r_r("H", "A")
    a.label("end")
    a.jr("end")
    a.label("sub")
    a.ld_r_d8("A", 0x42)
    a.ret()
    rom = flat_rom({0x150: a.resolve()})
    m = oracle(rom, 1)
    try:
        run_instructions(m, 11)
        assert (m.field("d")[0], m.field("e")[0]) == (0x12, 0x34)
        assert m.field("f")[0] == 0xF0  # POP AF drops the low nibble
        assert m.field("h")[0] == 0x42
        assert m.field("sp")[0] == 0xDFF0
        ret = a.labels["after_call"]
        assert (m.mem[0, 0xDFEF], m.mem[0, 0xDFEE]) == (ret >> 8, ret & 0xFF)
    finally:
        m.close()


# JOYP: bit 0 Right/A, 1 Left/B, 2 Up/Select, 3 Down/Start (active low)
ACTION_BITS = {1: ("btn", 0), 2: ("btn", 1), 3: ("btn", 3), 4: ("dpad", 2), 5: ("dpad", 3),
               6: ("dpad", 1), 7: ("dpad", 0)}  # fmt: skip


@pytest.mark.parametrize("release", [8, 0])
def test_joypad_matrix(release):
    """JOYP value for every action x select value, pressed and released."""
    sels = [0x00, 0x10, 0x20, 0x30]
    a = Asm(0x150)
    a.ldh_a8_a(0x00)  # A holds the select value
    a.label("loop")
    a.ldh_a_a8(0x00)
    a.jr("loop")
    rom = flat_rom({0x150: a.resolve()})
    act = np.repeat(np.arange(8), 4)
    sel = np.tile(sels, 8)
    m = oracle(rom, act.size)
    try:
        set_regs(m, a=sel)
        run_instructions(m, 2, actions=act.astype(np.int32), release=release)
        want = np.full(act.size, 0xCF)
        for i, (ac, s) in enumerate(zip(act, sel)):
            if release > 0 and ac in ACTION_BITS:
                group, bit = ACTION_BITS[int(ac)]
                if (s == 0x20 and group == "dpad") or (s == 0x10 and group == "btn"):
                    want[i] = 0xC0 | (0x0F & ~(1 << bit))
        np.testing.assert_array_equal(m.field("a"), want)
        np.testing.assert_array_equal(m.field("joyp_select"), sel & 0x30)
    finally:
        m.close()


def _loop_rom():
    return flat_rom({0x150: bytes([0x18, 0xFE])})  # JR -2 (12 cycles)


def brute_force_timer(div, tima, tma, tac, cycles):
    """Cycle-by-cycle DIV/TIMA: TIMA counts falling edges of DIV bit
    {9,3,5,7}[TAC&3] while TAC bit 2 is set; an overflow reloads TMA and
    raises IF bit 2 four cycles later."""
    bit = {0: 9, 1: 3, 2: 5, 3: 7}[tac & 3]
    reload_at, if2 = None, 0
    for t in range(1, cycles + 1):
        old = div
        div = (div + 1) & 0xFFFF
        if tac & 4 and (old >> bit) & 1 and not (div >> bit) & 1:
            tima = (tima + 1) & 0xFF
            if tima == 0:
                reload_at = t + 4
        if reload_at == t:
            tima, if2, reload_at = tma, 1, None
    return div, tima, if2


@pytest.mark.parametrize("tac", [0x04, 0x05, 0x06, 0x07, 0x01])
def test_timer_against_cycle_brute_force(tac):
    rng = np.random.default_rng(tac)
    n = 16
    m = oracle(_loop_rom(), n)
    try:
        div0 = rng.integers(0, 0x10000, n)
        tima0 = rng.integers(0xF0, 0x100, n)
        tma0 = rng.integers(0, 256, n)
        set_regs(m, div_counter=div0)
        m.mem[:, 0xFF04] = div0 >> 8
        m.mem[:, 0xFF05] = tima0
        m.mem[:, 0xFF06] = tma0
        m.mem[:, 0xFF07] = tac
        run_frames(m, 1)
        cyc = m.field("cycle_count")
        for i in range(n):
            d, t, if2 = brute_force_timer(int(div0[i]), int(tima0[i]), int(tma0[i]), tac, int(cyc[i]))
            assert m.field("div_counter")[i] == d
            assert m.mem[i, 0xFF04] == d >> 8
            assert m.mem[i, 0xFF05] == t, (i, tac)
            assert (m.mem[i, 0xFF0F] >> 2) & 1 == if2
    finally:
        m.close()


def test_ppu_lines_modes_and_vblank_against_brute_force():
    """LCD on from a line start: after C cycles LY = (C // 456) % 154, the
    scanline cycle is C % 456, STAT holds the mode of that position, IF bit 0
    is raised by the 143->144 transition."""
    m = oracle(_loop_rom(), 3)
    try:
        m.mem[:, 0xFF40] = 0x91
        m.mem[:, 0xFF45] = (0, 10, 153)
        set_regs(m, ppu_stat_prev=0)
        for _ in range(3):
            run_instructions(m, 5000)
            cyc = m.field("cycle_count")
            ly = (cyc // 456) % 154
            scan = cyc % 456
            np.testing.assert_array_equal(m.field("ppu_ly"), ly)
            np.testing.assert_array_equal(m.mem[:, 0xFF44], ly)
            np.testing.assert_array_equal(m.field("ppu_scanline_cycle"), scan)
            mode = np.where(ly >= 144, 1, np.where(scan < 80, 2, np.where(scan < 250, 3, 0)))
            coin = (ly == m.mem[:, 0xFF45]).astype(int)
            np.testing.assert_array_equal(m.mem[:, 0xFF41] & 7, mode | (coin << 2))
            np.testing.assert_array_equal(m.mem[:, 0xFF0F] & 1, (cyc >= 144 * 456).astype(int))
    finally:
        m.close()


def _irq_rom(handler_addr: int, main: Asm) -> bytes:
    h = Asm(handler_addr)
    h.push("AF")
    h.ld_a_a16(0xC000)
    h.inc_r("A")
    h.ld_a16_a(0xC000)
    h.pop("AF")
    h.reti()
    return flat_rom({0x150: main.resolve(), handler_addr: h.resolve()})


def test_vblank_interrupt_once_per_frame():
    a = Asm(0x150)
    a.ld_rr_d16("SP", 0xDFF0)
    a.ld_r_d8("A", 0x01)
    a.ldh_a8_a(0xFF)  # IE = VBlank
    a.ld_r_d8("A", 0x91)
    a.ldh_a8_a(0x40)  # LCD on
    a.ei()
    a.label("loop")
    a.jr("loop")
    rom = _irq_rom(0x40, a)
    m = oracle(rom, 2)
    try:
        run_frames(m, 10)
        # the LCD-on write counts as a frame; 9 full frames follow, each with
        # exactly one 143 -> 144 transition
        assert (m.mem[:, 0xC000] == 9).all()
        assert (m.field("ime") == 1).all()
    finally:
        m.close()


def test_stat_lyc_interrupt_once_per_frame():
    a = Asm(0x150)
    a.ld_rr_d16("SP", 0xDFF0)
    a.ld_r_d8("A", 77)
    a.ldh_a8_a(0x45)  # LYC
    a.ld_r_d8("A", 0x40)
    a.ldh_a8_a(0x41)  # STAT: LYC source
    a.ld_r_d8("A", 0x02)
    a.ldh_a8_a(0xFF)  # IE = STAT
    a.ld_r_d8("A", 0x91)
    a.ldh_a8_a(0x40)
    a.ei()
    a.label("loop")
    a.jr("loop")
    rom = _irq_rom(0x48, a)
    m = oracle(rom, 1)
    try:
        run_frames(m, 7)
        assert m.mem[0, 0xC000] == 6
    finally:
        m.close()


def test_halt_wake_with_ime_off_skips_one_byte():
    """The reference's HALT: with IME=0 a pending interrupt clears HALT and
    advances PC past the next byte (cpu_step_builder.py:1181-1183)."""
    a = Asm(0x150)
    a.di()
    a.ld_r_d8("A", 0x04)
    a.ldh_a8_a(0xFF)  # IE = timer
    a.ld_r_d8("A", 0x05)
    a.ldh_a8_a(0x07)  # TAC on, 16-cycle period
    a.halt()
    a.inc_r("B")  # skipped
    a.inc_r("C")
    a.label("end")
    a.jr("end")
    rom = flat_rom({0x150: a.resolve()})
    m = oracle(rom, 1)
    try:
        run_frames(m, 1)
        assert m.field("b")[0] == 0 and m.field("c")[0] == 1
        assert m.field("halted")[0] == 0
    finally:
        m.close()


def test_ei_takes_effect_immediately():
    """EI sets IME at once, so an already pending interrupt is serviced right
    after the EI instruction (misc.py:21-26)."""
    a = Asm(0x150)
    a.ld_rr_d16("SP", 0xDFF0)
    a.ld_r_d8("A", 0x04)
    a.ldh_a8_a(0xFF)
    a.ldh_a8_a(0x0F)  # IF = timer pending
    a.ei()
    a.inc_r("B")
    a.label("end")
    a.jr("end")
    rom = flat_rom({0x150: a.resolve(), 0x50: bytes([0x3E, 0x77, 0xD9])})  # LD A,77; RETI
    m = oracle(rom, 1)
    try:
        run_instructions(m, 6)  # 5 instructions + the handler's first
        assert m.field("a")[0] == 0x77
        assert m.field("b")[0] == 0  # INC B not reached before the handler
        assert m.mem[0, 0xDFEF] == (a.labels["end"] - 1) >> 8
    finally:
        m.close()


def _banked_rom(cart_type, rom_code, ram_code):
    blocks = {0x150: b""}
    nbanks = (32 << rom_code) // 16
    for b in range(1, nbanks):
        blocks[b * 0x4000] = bytes([b & 0xFF])
    return blocks, nbanks


@pytest.mark.parametrize("cart_type,ram_code", [(0x01, 0x00), (0x13, 0x03)])
def test_mbc_rom_bank_select(cart_type, ram_code):
    """Writing N to 2000-3FFF maps bank N (0 -> 1) at 4000; MBC1 keeps 5 bits,
    MBC3 7 bits, both masked by the bank count (32 banks here)."""
    code = Asm(0x150)
    code.ld_a16_a(0x2000)
    code.ld_a_a16(0x4000)
    code.label("end")
    code.jr("end")
    blocks, nbanks = _banked_rom(cart_type, 0x04, ram_code)
    blocks[0x150] = code.resolve()
    rom = flat_rom(blocks, cart_type=cart_type, rom_code=0x04, ram_code=ram_code)
    vals = np.arange(256)
    m = oracle(rom, 256)
    try:
        set_regs(m, a=vals)
        run_instructions(m, 3)
        bits = 0x1F if cart_type == 0x01 else 0x7F
        bank = vals & bits
        bank = np.where(bank == 0, 1, bank) & (nbanks - 1)
        np.testing.assert_array_equal(m.field("a"), bank)
    finally:
        m.close()


def test_mbc3_ram_banks_and_rtc_seconds():
    code = Asm(0x150)
    code.ld_r_d8("A", 0x0A)
    code.ld_a16_a(0x0000)  # RAM enable
    for bank in range(4):
        code.ld_r_d8("A", bank)
        code.ld_a16_a(0x4000)
        code.ld_r_d8("A", 0x10 + bank)
        code.ld_a16_a(0xA123)
    code.ld_r_d8("A", 0x02)
    code.ld_a16_a(0x4000)
    code.ld_a_a16(0xA123)
    code.ld_r_r("B", "A")
    code.label("end")
    code.jr("end")
    rom = flat_rom({0x150: code.resolve()}, cart_type=0x10, rom_code=0x01, ram_code=0x03)
    m = oracle(rom, 1)
    try:
        run_frames(m, 61)
        assert m.field("b")[0] == 0x12
        ram = m.cart_ram[0]
        assert [ram[b * 0x2000 + 0x123] for b in range(4)] == [0x10, 0x11, 0x12, 0x13]
        cyc = int(m.field("cycle_count")[0])
        assert m.cart_state[0, 9] == cyc // 4194304  # RTC seconds
        assert m.cart_state[0, 14] == cyc % 4194304  # sub-second cycles
    finally:
        m.close()


def test_echo_dma_masks_and_serial():
    code = Asm(0x150)
    code.ld_r_d8("A", 0x5A)
    code.ld_a16_a(0xE1F0)  # echo of C1F0
    code.ld_rr_d16("HL", 0xC100)
    code.ld_r_d8("B", 160)
    code.label("fill")
    code.ld_r_r("A", "B")
    code.ld_hli_a()
    code.dec_r("B")
    code.jr("fill", "NZ")
    code.ld_r_d8("A", 0xC1)
    code.ldh_a8_a(0x46)  # DMA C100 -> FE00
    code.ld_r_d8("A", 0xFF)
    code.ldh_a8_a(0x0F)
    code.ldh_a8_a(0xFF)
    code.ld_r_d8("A", 0x41)
    code.ldh_a8_a(0x01)
    code.ld_r_d8("A", 0x81)
    code.ldh_a8_a(0x02)  # serial transfer
    code.ld_a_a16(0xE1F0)
    code.label("end")
    code.jr("end")
    rom = flat_rom({0x150: code.resolve()})
    m = oracle(rom, 1)
    try:
        run_frames(m, 1)
        assert m.mem[0, 0xC1F0] == 0x5A and m.mem[0, 0xE1F0] == 0
        assert m.field("a")[0] == 0x5A
        np.testing.assert_array_equal(m.mem[0, 0xFE00:0xFEA0], np.arange(160, 0, -1))
        assert m.mem[0, 0xFFFF] == 0x1F
        assert m.mem[0, 0xFF0F] == 0x1F  # 0xFF masked, serial IF bit already in
        assert m.field("serial_len")[0] == 1 and m.serial_buf[0, 0] == 0x41
        assert m.mem[0, 0xFF02] == 0x01
    finally:
        m.close()

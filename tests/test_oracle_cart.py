"""Known answers for the cartridge side of the oracle.

Covers the MBC3 real-time clock (carry chain into minutes, hours, days and
the day-overflow bit, the halt bit, the latch, register access through
A000-BFFF), MBC1 banking mode 1 and RAM enable, cartridge RAM that is
disabled or absent, and the serial buffer's overflow.

The expected values come from closed forms written from the reference's text
(``kernels/cpu_step_builder.py:374-419`` for the clock, ``:555-657`` for bus
reads, ``:710-723`` for serial, ``:777-872`` for cartridge writes), not from
the oracle's code: the clock is a count of whole seconds taken apart with
integer division, the banks are bit arithmetic on the written values.  Each
closed form is shown to discriminate: a model with one plausible mistake
planted must disagree with the oracle on the same states.
"""

from __future__ import annotations

import numpy as np
import pytest

from gbxcule_amd.abi import CART_STATE_INDEX as CS
from gbxcule_amd.carts.asm import Asm

from ._isa import flat_rom, oracle, run_frames, run_instructions, set_regs

RTC_HZ = 4_194_304  # emulated cycles per RTC second
RTC_SLOTS = ("rtc_seconds", "rtc_minutes", "rtc_hours", "rtc_days_low", "rtc_days_high")


def _mbc3_rom(code: bytes, ram_code: int = 0x03) -> bytes:
    return flat_rom({0x150: code}, cart_type=0x10, rom_code=0x01, ram_code=ram_code)


def _idle() -> bytes:
    a = Asm(0x150)
    a.label("end")
    a.jr("end")
    return a.resolve()


# ---------------------------------------------------------------------------
# RTC carry chain
# ---------------------------------------------------------------------------


def rtc_model(state: dict, cycles: int, mistake: str | None = None) -> dict:
    """The clock after ``cycles`` emulated cycles from in-range registers.

    A halted clock (days-high bit 6) keeps every register and the sub-second
    count.  Otherwise the sub-second count (negative counts as 0) gains the
    cycles; the whole seconds it reaches are added to the time as one count
    of seconds since day 0, 00:00:00, and taken apart again; a day count
    past 511 wraps and sets the day-overflow bit 7, which then stays set.
    Days-high keeps bits 6-7 and holds bit 8 of the day in bit 0; its other
    bits read back as 0 after a tick.
    """
    dh = state["rtc_days_high"]
    if dh & 0x40 and mistake != "halt_ignored":
        return dict(state)
    sub = max(state["rtc_last_cycle"], 0) if mistake != "negative_sub_kept" else state["rtc_last_cycle"]
    sub += cycles
    n, sub = divmod(sub, RTC_HZ)
    if mistake == "sub_dropped" and n:
        sub = 0
    day = ((dh & 1) << 8) | state["rtc_days_low"]
    if mistake == "day_8bit":
        day = state["rtc_days_low"]
    t = ((day * 24 + state["rtc_hours"]) * 60 + state["rtc_minutes"]) * 60 + state["rtc_seconds"] + n
    days = t // 86400
    limit = 256 if mistake == "day_8bit" else 512
    over = days >= limit and mistake != "no_day_carry"
    days %= limit
    keep = 0xFE if mistake == "stray_bits_kept" else 0xC0
    out = dict(state)
    out.update(
        rtc_seconds=t % 60,
        rtc_minutes=t // 60 % 60,
        rtc_hours=t // 3600 % (32 if mistake == "hours_roll_at_32" else 24),
        rtc_days_low=days & 0xFF,
        rtc_days_high=(dh & keep) | (0x80 if over else 0) | (days >> 8),
        rtc_last_cycle=sub,
    )
    return out


def _rtc_states() -> list[dict]:
    """Boundary cases first, then random in-range clocks."""

    def st(sec, mn, hr, day, dh_extra=0, sub=0):
        return dict(
            rtc_seconds=sec,
            rtc_minutes=mn,
            rtc_hours=hr,
            rtc_days_low=day & 0xFF,
            rtc_days_high=((day >> 8) & 1) | dh_extra,
            rtc_last_cycle=sub,
        )

    edge = RTC_HZ - 1000
    cases = [
        st(0, 0, 0, 0),
        st(59, 0, 0, 0, sub=edge),  # second -> minute
        st(58, 59, 0, 0, sub=edge),  # minute -> hour
        st(59, 59, 23, 0, sub=edge),  # hour -> day
        st(59, 59, 23, 255, sub=edge),  # days-low -> day bit 8
        st(59, 59, 23, 511, sub=edge),  # day 511 -> 0, overflow bit
        st(59, 59, 23, 511, 0x80, sub=edge),  # overflow already set
        st(58, 59, 23, 300, 0x80, sub=12345),
        st(59, 59, 23, 511, 0x3E, sub=edge),  # stray days-high bits
        st(59, 59, 23, 1, sub=-5),  # negative sub-second count
        st(59, 59, 23, 511, 0x40, sub=edge),  # halted
        st(59, 59, 23, 511, 0xC0, sub=edge),  # halted with overflow set
        st(10, 20, 5, 7, 0x40, sub=-9),  # halted, negative count kept
    ]
    rng = np.random.default_rng(7)
    for _ in range(35):
        cases.append(
            st(
                int(rng.integers(0, 60)),
                int(rng.integers(0, 60)),
                int(rng.integers(0, 24)),
                int(rng.integers(0, 512)),
                int(rng.choice([0, 0x80])),
                int(rng.integers(0, RTC_HZ)),
            )
        )
    return cases


@pytest.fixture(scope="module")
def rtc_run():
    """Each state run for 130 frames (about 2.2 emulated seconds)."""
    states = _rtc_states()
    m = oracle(_mbc3_rom(_idle()), len(states))
    try:
        for k, s in enumerate(states):
            for name, v in s.items():
                m.cart_state[k, CS[name]] = v
            m.cart_state[k, CS["rtc_latched_seconds"] : CS["rtc_latched_days_high"] + 1] = 0x77
        c0 = m.field("cycle_count").copy()
        run_frames(m, 130)
        cycles = (m.field("cycle_count") - c0).astype(np.int64)
        got = [{name: int(m.cart_state[k, CS[name]]) for name in states[0]} for k in range(len(states))]
        latched = m.cart_state[:, CS["rtc_latched_seconds"] : CS["rtc_latched_days_high"] + 1].copy()
    finally:
        m.close()
    return states, cycles, got, latched


def _rtc_mismatches(rtc_run, mistake=None):
    states, cycles, got, _ = rtc_run
    return [k for k, s in enumerate(states) if rtc_model(s, int(cycles[k]), mistake) != got[k]]


def test_rtc_carry_chain_closed_form(rtc_run):
    """Seconds, minutes, hours, the 9-bit day and the overflow bit after
    about 2.2 s, from boundary and random clocks; the halt bit freezes all."""
    states, cycles, got, latched = rtc_run
    assert cycles.min() > 2 * RTC_HZ  # every running clock crossed two seconds
    assert _rtc_mismatches(rtc_run) == []
    # spot checks written out by hand
    assert got[5]["rtc_days_high"] == 0x80 and got[5]["rtc_days_low"] == 0  # 511 -> 0
    assert got[4]["rtc_days_high"] == 0x01 and got[4]["rtc_days_low"] == 0  # 255 -> 256
    assert got[8]["rtc_days_high"] == 0x80  # stray bits 1-5 dropped
    assert got[10] == states[10] and got[12] == states[12]  # halted
    assert (latched == 0x77).all()  # ticking never touches the latched copy


@pytest.mark.parametrize(
    "mistake",
    ["halt_ignored", "negative_sub_kept", "sub_dropped", "day_8bit", "no_day_carry",
     "stray_bits_kept", "hours_roll_at_32"],
)  # fmt: skip
def test_rtc_planted_mistakes_are_caught(rtc_run, mistake):
    assert _rtc_mismatches(rtc_run, mistake)


# ---------------------------------------------------------------------------
# RTC registers through A000-BFFF and the MBC3 select
# ---------------------------------------------------------------------------

_RTC_LIVE = dict(rtc_seconds=11, rtc_minutes=22, rtc_hours=3, rtc_days_low=44)


def rtc_access_model(sel: int, val: int, halted: bool, mistake: str | None = None):
    """(byte read before the write, byte read after it, RTC slot written or
    None, cart RAM bank written or None) for select ``sel`` and value
    ``val``, with RAM bank 2 selected before and the clock halted or not.

    Selects 0-3 also pick the RAM bank; 4-7 and 0D-0F leave bank 2 mapped.
    Selects 08-0C map a clock register, which a write sets to the whole
    byte; the tick at the end of the writing instruction then masks it to
    the register's width (seconds and days-low 8 bits, minutes 6, hours 5,
    days-high bits 7, 6 and 0), unless the clock is halted, days-high bit 6
    included as just written.
    """
    if 8 <= sel <= 12 and not (mistake == "rtc_select_0d" and sel == 12):
        field = RTC_SLOTS[sel - 8]
        before = {**_RTC_LIVE, "rtc_days_high": 0x40 if halted else 0}[field]
        widths = {"rtc_seconds": 0xFF, "rtc_minutes": 0x3F, "rtc_hours": 0x1F, "rtc_days_low": 0xFF,
                  "rtc_days_high": 0xC1}  # fmt: skip
        if mistake == "minutes_7bit":
            widths["rtc_minutes"] = 0x7F
        stopped = (val & 0x40) if sel == 12 else halted
        if mistake == "mask_ignores_halt":
            stopped = False
        after = val if (stopped or mistake == "no_tick_mask") else val & widths[field]
        return before, after, field, None
    bank = sel if sel <= 3 else 2
    if mistake == "select_low_bits" and 4 <= sel <= 7:
        bank = sel & 3
    return 0xB0 | bank, val, None, bank


_ACCESS_VALS = (0x00, 0x3B, 0x7F, 0xC1, 0xFF, 0x5A, 0x41, 0x80)


@pytest.fixture(scope="module")
def rtc_access_run():
    cases = [(sel, val, h) for sel in range(16) for val in _ACCESS_VALS for h in (False, True)]
    a = Asm(0x150)
    a.ld_r_d8("A", 0x0A)
    a.ld_a16_a(0x0000)  # RAM and RTC enable
    a.ld_r_r("A", "B")
    a.ld_a16_a(0x4000)  # select
    a.ld_a_a16(0xA123)
    a.ld_r_r("E", "A")  # read before the write
    a.ld_r_r("A", "C")
    a.ld_a16_a(0xA123)  # write
    a.ld_a_a16(0xA123)
    a.ld_r_r("D", "A")  # read after
    a.label("end")
    a.jr("end")
    m = oracle(_mbc3_rom(a.resolve()), len(cases))
    try:
        for k, (sel, val, h) in enumerate(cases):
            for name, v in _RTC_LIVE.items():
                m.cart_state[k, CS[name]] = v
            m.cart_state[k, CS["rtc_days_high"]] = 0x40 if h else 0
            m.cart_state[k, CS["ram_bank"]] = 2
            for b in range(4):
                m.cart_ram[k, b * 0x2000 + 0x123] = 0xB0 | b
        set_regs(m, b=np.array([c[0] for c in cases]), c=np.array([c[1] for c in cases]))
        run_instructions(m, 10)
        out = dict(
            e=m.field("e").copy(),
            d=m.field("d").copy(),
            cs=m.cart_state.copy(),
            ram=m.cart_ram[:, [b * 0x2000 + 0x123 for b in range(4)]].copy(),
        )
    finally:
        m.close()
    return cases, out


def _access_mismatches(rtc_access_run, mistake=None):
    cases, out = rtc_access_run
    bad = []
    for k, (sel, val, h) in enumerate(cases):
        before, after, field, bank = rtc_access_model(sel, val, h, mistake)
        ok = out["e"][k] == before and out["d"][k] == after
        ram = [0xB0 | b for b in range(4)]
        if bank is not None:
            ram[bank] = val
        ok &= list(out["ram"][k]) == ram
        if field is not None:
            ok &= out["cs"][k, CS[field]] == after
        ok &= out["cs"][k, CS["rtc_select"]] == sel
        ok &= out["cs"][k, CS["ram_bank"]] == (sel if sel <= 3 else 2)
        if not ok:
            bad.append(k)
    return bad


def test_rtc_registers_through_a000(rtc_access_run):
    """Every select value 00-0F: RAM banks 0-3, bank left as is for 04-07
    and 0D-0F, clock registers 08-0C read and written with the tick's
    masking and the halt bit's exception."""
    assert _access_mismatches(rtc_access_run) == []


@pytest.mark.parametrize(
    "mistake", ["no_tick_mask", "mask_ignores_halt", "minutes_7bit", "select_low_bits", "rtc_select_0d"]
)
def test_rtc_access_planted_mistakes_are_caught(rtc_access_run, mistake):
    assert _access_mismatches(rtc_access_run, mistake)


# ---------------------------------------------------------------------------
# RTC latch
# ---------------------------------------------------------------------------


def _read_rtc_into(a: Asm, dst: int) -> None:
    """Read the five clock registers through A000 into dst..dst+4."""
    for j, sel in enumerate(range(8, 13)):
        a.ld_r_d8("A", sel)
        a.ld_a16_a(0x4000)
        a.ld_a_a16(0xA000)
        a.ld_a16_a(dst + j)


def _latch_program():
    blocks, entry = {}, {}
    a = Asm(0x150)  # enable, then latch: write 0 then 1
    a.ld_r_d8("A", 0x0A)
    a.ld_a16_a(0x0000)
    a.alu_r("XOR", "A")
    a.ld_a16_a(0x6000)
    a.inc_r("A")
    a.ld_a16_a(0x6000)
    a.label("end")
    a.jr("end")
    blocks[0x150], entry["latch"] = a.resolve(), (0x150, 6)
    a = Asm(0x200)  # read the latched registers
    _read_rtc_into(a, 0xC000)
    a.label("end")
    a.jr("end")
    blocks[0x200], entry["read"] = a.resolve(), (0x200, 20)
    a = Asm(0x280)  # write 2, then 1: neither clears nor re-copies
    a.ld_r_d8("A", 2)
    a.ld_a16_a(0x6000)
    a.ld_r_d8("A", 1)
    a.ld_a16_a(0x6000)
    _read_rtc_into(a, 0xC010)
    a.label("end")
    a.jr("end")
    blocks[0x280], entry["again"] = a.resolve(), (0x280, 24)
    a = Asm(0x300)  # write 0: reads show the live registers
    a.alu_r("XOR", "A")
    a.ld_a16_a(0x6000)
    _read_rtc_into(a, 0xC020)
    a.label("end")
    a.jr("end")
    blocks[0x300], entry["clear"] = a.resolve(), (0x300, 22)
    return flat_rom(blocks, cart_type=0x10, rom_code=0x01, ram_code=0x03), entry


def _run_phase(m, entry, name):
    pc, k = entry[name]
    m.field("pc")[:] = pc
    run_instructions(m, k)


def latch_model(initial: dict, live_late: dict, mistake: str | None = None):
    """(latched read, read after writing 2 then 1, read after writing 0).
    The 0 -> 1 write copies the live registers; while the latch is set reads
    return the copy; writing 1 again or any value other than 0 changes
    nothing; writing 0 clears the latch and reads show the live registers."""
    first = [initial[f] for f in RTC_SLOTS]
    late = [live_late[f] for f in RTC_SLOTS]
    if mistake == "reads_live":
        return late, late, late
    if mistake in ("recopy_on_1", "clear_on_non_1"):
        return first, late, late
    if mistake == "zero_keeps_latch":
        return first, first, first
    return first, first, late


@pytest.fixture(scope="module")
def latch_run():
    rom, entry = _latch_program()
    rng = np.random.default_rng(11)
    states = [
        dict(rtc_seconds=int(rng.integers(0, 60)), rtc_minutes=int(rng.integers(0, 60)),
             rtc_hours=int(rng.integers(0, 24)), rtc_days_low=int(rng.integers(0, 256)),
             rtc_days_high=int(rng.choice([0, 1, 0x80, 0x81])))
        for _ in range(16)
    ]  # fmt: skip
    m = oracle(rom, len(states))
    try:
        for k, s in enumerate(states):
            for name, v in s.items():
                m.cart_state[k, CS[name]] = v
            m.cart_state[k, CS["rtc_last_cycle"]] = 0
        _run_phase(m, entry, "latch")
        latched_slots = m.cart_state[:, CS["rtc_latched_seconds"] : CS["rtc_latched_days_high"] + 1].copy()
        run_frames(m, 130)  # about 2.2 s: the live clock moves on
        live_late = [{f: int(m.cart_state[k, CS[f]]) for f in RTC_SLOTS} for k in range(len(states))]
        for name in ("read", "again", "clear"):
            _run_phase(m, entry, name)
        reads = m.mem[:, 0xC000:0xC030].copy()
        latch_flag = m.cart_state[:, CS["rtc_latch"]].copy()
    finally:
        m.close()
    return states, latched_slots, live_late, reads, latch_flag


def _latch_mismatches(latch_run, mistake=None):
    states, _, live_late, reads, _ = latch_run
    bad = []
    for k, s in enumerate(states):
        want = latch_model(s, live_late[k], mistake)
        got = [list(reads[k, o : o + 5]) for o in (0x00, 0x10, 0x20)]
        if got != [list(w) for w in want]:
            bad.append(k)
    return bad


def test_rtc_latch_holds_while_live_clock_runs(latch_run):
    states, latched_slots, live_late, _, latch_flag = latch_run
    for k, s in enumerate(states):
        assert list(latched_slots[k]) == [s[f] for f in RTC_SLOTS]
        assert live_late[k] != s  # the live clock advanced
    assert _latch_mismatches(latch_run) == []
    assert (latch_flag == 0).all()


@pytest.mark.parametrize("mistake", ["reads_live", "recopy_on_1", "clear_on_non_1", "zero_keeps_latch"])
def test_rtc_latch_planted_mistakes_are_caught(latch_run, mistake):
    assert _latch_mismatches(latch_run, mistake)


# ---------------------------------------------------------------------------
# MBC1 banking modes, RAM enable, disabled and absent cart RAM
# ---------------------------------------------------------------------------


def mbc1_model(en: int, hi: int, mode: int, lo: int, nbanks: int, ram_banks: int, mistake=None):
    """(byte at 0200 = bank of the 0000 window, byte at 4200 = bank of the
    4000 window, byte read at A123, RAM bank the write to A124 lands in or
    None).  RAM is enabled iff the low nibble written to 0000-1FFF is 0xA;
    2000-3FFF keeps 5 bits with 0 read as 1; 4000-5FFF 2 bits, used as ROM
    bank bits 5-6 in the 4000 window always, and in mode 1 also as the
    0000 window's bank and as the RAM bank (mode 0: RAM bank 0).  Banks wrap
    at the ROM's bank count; without RAM, or with it disabled, reads are
    0xFF and writes are dropped."""
    enabled = (en & 0x0F) == 0x0A
    if mistake == "enable_full_byte":
        enabled = en == 0x0A
    lo5 = lo & 0x1F
    if lo5 == 0 and mistake != "lo_zero_kept":
        lo5 = 1
    hi2 = hi & 3
    m1 = mode & 1
    b0 = (hi2 << 5) if m1 and mistake != "mode1_rom0_ignored" else 0
    b1 = lo5 if mistake == "hi_not_in_4000" else (hi2 << 5) | lo5
    rb = hi2 if (m1 or mistake == "ram_bank_mode0") else 0
    b0 &= nbanks - 1
    b1 &= nbanks - 1
    if ram_banks == 0 or not enabled:
        return b0, b1, 0xFF, None
    rb %= ram_banks
    return b0, b1, 0xA0 | rb, rb


_EN = (0x0A, 0x1A, 0xFA, 0x0B, 0x00)
_HI = (0, 1, 2, 3, 0xFE)
_MODE = (0, 1, 0xFF, 2)
_LO = (0, 1, 0x1F, 0x20, 0x35)


@pytest.fixture(scope="module", params=[(0x06, 0x03), (0x04, 0x03), (0x06, 0x02), (0x05, 0x00)],
                ids=["2MiB_ram32K", "512K_ram32K", "2MiB_ram8K", "1MiB_noram"])  # fmt: skip
def mbc1_run(request):
    rom_code, ram_code = request.param
    nbanks = (32 << rom_code) // 16
    ram_banks = {0x00: 0, 0x02: 1, 0x03: 4}[ram_code]
    a = Asm(0x150)
    for reg, addr in (("B", 0x0000), ("C", 0x4000), ("D", 0x6000), ("E", 0x2000)):
        a.ld_r_r("A", reg)
        a.ld_a16_a(addr)
    for src, dst in ((0x0200, 0xC000), (0x4200, 0xC001), (0xA123, 0xC002)):
        a.ld_a_a16(src)
        a.ld_a16_a(dst)
    a.ld_r_d8("A", 0x77)
    a.ld_a16_a(0xA124)
    a.label("end")
    a.jr("end")
    code = a.resolve()
    blocks = {}
    for b in range(nbanks):
        if b % 32 == 0:  # mode 1 maps bank 32 * (bits 5-6) at 0000: the code runs on there
            blocks[b * 0x4000 + 0x150] = code
        blocks[b * 0x4000 + 0x200] = bytes([b])
    rom = flat_rom(blocks, cart_type=0x03 if ram_banks else 0x01, rom_code=rom_code, ram_code=ram_code)
    cases = [(en, hi, mo, lo) for en in _EN for hi in _HI for mo in _MODE for lo in _LO]
    m = oracle(rom, len(cases))
    try:
        if ram_banks:
            for b in range(ram_banks):
                m.cart_ram[:, b * 0x2000 + 0x123] = 0xA0 | b
        cols = np.array(cases)
        set_regs(m, b=cols[:, 0], c=cols[:, 1], d=cols[:, 2], e=cols[:, 3])
        run_instructions(m, 18)
        out = dict(
            reads=m.mem[:, 0xC000:0xC003].copy(),
            ram=m.cart_ram[:, [b * 0x2000 + 0x124 for b in range(ram_banks)]].copy() if ram_banks else None,
            cs=m.cart_state.copy(),
            a124=m.mem[:, 0xA124].copy(),
        )
    finally:
        m.close()
    return cases, out, nbanks, ram_banks


def _mbc1_mismatches(mbc1_run, mistake=None):
    cases, out, nbanks, ram_banks = mbc1_run
    bad = []
    for k, (en, hi, mo, lo) in enumerate(cases):
        b0, b1, rd, wb = mbc1_model(en, hi, mo, lo, nbanks, ram_banks, mistake)
        ok = list(out["reads"][k]) == [b0, b1, rd]
        if ram_banks:
            want = [0x77 if b == wb else 0 for b in range(ram_banks)]
            ok &= list(out["ram"][k]) == want
        ok &= out["a124"][k] == 0  # cart RAM writes never reach the memory image
        ok &= out["cs"][k, CS["rom_bank_hi"]] == hi & 3 and out["cs"][k, CS["ram_bank"]] == hi & 3
        ok &= out["cs"][k, CS["bank_mode"]] == mo & 1
        ok &= out["cs"][k, CS["ram_enable"]] == int((en & 0x0F) == 0x0A)
        if not ok:
            bad.append(k)
    return bad


def test_mbc1_banking_modes_and_ram_enable(mbc1_run):
    """Both windows and the RAM bank for every combination of enable value,
    4000-5FFF bits, mode and 2000-3FFF value, on 2 MiB (128 banks), 1 MiB
    without RAM and 512 KiB (32 banks, where bits 5-6 wrap away) carts."""
    assert _mbc1_mismatches(mbc1_run) == []


@pytest.mark.parametrize(
    "mistake",
    ["enable_full_byte", "lo_zero_kept", "mode1_rom0_ignored", "hi_not_in_4000", "ram_bank_mode0"],
)
def test_mbc1_planted_mistakes_are_caught(mbc1_run, mistake):
    cases, out, nbanks, ram_banks = mbc1_run
    if mistake in ("mode1_rom0_ignored", "hi_not_in_4000") and nbanks <= 32:
        pytest.skip("bits 5-6 wrap away on a 32-bank cart")
    if mistake == "ram_bank_mode0" and ram_banks <= 1:
        pytest.skip("one RAM bank: every bank number maps to it")
    if mistake == "enable_full_byte" and ram_banks == 0:
        pytest.skip("no RAM: enabling changes nothing the bus shows")
    assert _mbc1_mismatches(mbc1_run, mistake)


def test_rom_only_cart_ram_reads_ff_and_drops_writes():
    """A cart without RAM: A000-BFFF reads 0xFF and writes change nothing,
    even with the enable slot set."""
    a = Asm(0x150)
    a.ld_r_d8("A", 0x12)
    a.ld_a16_a(0xA000)
    a.ld_a16_a(0xBFFF)
    a.ld_a_a16(0xA000)
    a.ld_r_r("B", "A")
    a.ld_a_a16(0xBFFF)
    a.ld_r_r("C", "A")
    a.label("end")
    a.jr("end")
    m = oracle(flat_rom({0x150: a.resolve()}), 2)
    try:
        m.cart_state[1, CS["ram_enable"]] = 1
        run_instructions(m, 7)
        assert list(m.field("b")) == [0xFF, 0xFF] and list(m.field("c")) == [0xFF, 0xFF]
        assert (m.mem[:, 0xA000] == 0).all() and (m.mem[:, 0xBFFF] == 0).all()
    finally:
        m.close()


# ---------------------------------------------------------------------------
# Serial buffer overflow
# ---------------------------------------------------------------------------

SERIAL_MAX = 1024


def serial_model(count: int, mistake: str | None = None):
    """(bytes kept, overflow flag, FF02 after a final 0x80 write).  Each
    internal-clock transfer (FF02 written with bits 7 and 0) appends FF01 to
    the 1,024-byte buffer while there is room, else sets the overflow flag;
    it stores FF02 with bit 7 clear and raises IF bit 3.  A write without
    bit 0 is stored as is and transfers nothing."""
    sent = [(count - j) & 0xFF for j in range(count)]
    cap = SERIAL_MAX - 1 if mistake == "overflow_at_1023" else SERIAL_MAX
    kept = sent[:cap] if mistake != "ring" else (sent[-cap:] if count > cap else sent)
    if mistake == "external_clock_sends" and len(kept) < cap:
        kept = kept + [0]
    over = 1 if count > cap else 0
    return kept, over, 0x00 if mistake == "ff02_bit7_cleared_always" else 0x80


_SERIAL_COUNTS = (1, 2, 1023, 1024, 1025, 1100)


@pytest.fixture(scope="module")
def serial_run():
    a = Asm(0x150)
    a.label("loop")
    a.ld_r_r("A", "L")
    a.ldh_a8_a(0x01)
    a.ld_r_d8("A", 0x81)
    a.ldh_a8_a(0x02)
    a.dec_rr("HL")
    a.ld_r_r("A", "H")
    a.alu_r("OR", "L")
    a.jr("loop", "NZ")
    a.ld_r_d8("A", 0x00)
    a.ldh_a8_a(0x01)
    a.ld_r_d8("A", 0x80)  # external clock: no transfer
    a.ldh_a8_a(0x02)
    a.label("end")
    a.jr("end")
    counts = np.array(_SERIAL_COUNTS)
    m = oracle(flat_rom({0x150: a.resolve()}), counts.size)
    try:
        set_regs(m, h=counts >> 8, l=counts & 0xFF)
        run_frames(m, 2)  # 64 cycles per byte: 1,100 bytes take more than a frame
        out = dict(
            n=m.field("serial_len").copy(),
            over=m.field("serial_overflow").copy(),
            buf=m.serial_buf.copy(),
            ff02=m.mem[:, 0xFF02].copy(),
            iff=m.mem[:, 0xFF0F].copy(),
            pc=m.field("pc").copy(),
        )
    finally:
        m.close()
    return counts, out


def _serial_mismatches(serial_run, mistake=None):
    counts, out = serial_run
    bad = []
    for k, c in enumerate(counts):
        kept, over, ff02 = serial_model(int(c), mistake)
        ok = out["n"][k] == len(kept) and list(out["buf"][k, : len(kept)]) == kept
        ok &= out["over"][k] == over and out["ff02"][k] == ff02 and (out["iff"][k] & 0x08) != 0
        if not ok:
            bad.append(k)
    return bad


def test_serial_buffer_overflow(serial_run):
    counts, out = serial_run
    assert (out["pc"] == out["pc"][0]).all()  # every env reached the idle loop
    assert _serial_mismatches(serial_run) == []


@pytest.mark.parametrize(
    "mistake", ["overflow_at_1023", "ring", "external_clock_sends", "ff02_bit7_cleared_always"]
)
def test_serial_planted_mistakes_are_caught(serial_run, mistake):
    assert _serial_mismatches(serial_run, mistake)

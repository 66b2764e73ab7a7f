"""PyBoy savestate I/O on the host: file layout, versions 9-15, errors, and the
mapping between a savestate and one env's image.

The layout checks build files at the absolute offsets of the reference's
format document (``docs/pyboy_state_format.md``: CPU at 5, LCD at 23, sound
at 9125, renderer at 9263, RAM at 124463, timer at 133006, cart at 133014,
133021 bytes without cart RAM) with distinct sentinel bytes in every field,
so a section read at the wrong place or with the wrong length shows up as a
wrong value.  The timer field order is the reference parser's
(``core/state_io.py:467-473``: DIV, TIMA, DIV counter, TIMA counter, TMA,
TAC), which is what PyBoy writes; the document's table lists it differently.
Mapping checks are known answers from the reference's
``state_from_warp_backend`` / ``apply_state_to_warp_backend`` text
(``core/state_io.py:662-1154``) and its tests (``tests/test_state_io.py``).
"""

from __future__ import annotations

import struct

import numpy as np
import pytest

from gbxcule_amd import state_io as sio
from gbxcule_amd.abi import CART_STATE_FIELDS

CS = {n: i for i, n in enumerate(CART_STATE_FIELDS)}
RNG = np.random.default_rng(2024)


def _rand(n: int) -> bytes:
    return RNG.integers(0, 256, n, dtype=np.uint8).tobytes()


class Spec:
    """Sentinel values for every field a savestate carries."""

    def __init__(self, cart_ram: bytes = b""):
        self.bootrom = 1
        self.regs = (0x11, 0xB0, 0x22, 0x33, 0x44, 0x55)  # A F B C D E
        self.hl, self.sp, self.pc = 0xC0DE, 0xDFF0, 0x1234
        self.cpu_flags = (1, 0, 0, 0x1F, 0, 0x05)  # IME HALT STOP IE queued IF
        self.vram, self.oam = _rand(8192), _rand(160)
        self.lcd = (0x91, 0xE4, 0xD0, 0xE0, 0x85, 0x42, 0x43, 0x10, 0x20, 0x30, 0x47)
        self.clock, self.target, self.mode = 70000, 70224, 2
        self.scan = _rand(720)
        self.wram, self.non_io0, self.io = _rand(8192), _rand(96), _rand(76)
        self.hram, self.non_io1 = _rand(127), _rand(52)
        self.timer = (0xAB, 0x17, 0x3456, 0x0789, 0x80, 0x05)  # DIV TIMA DIVc TIMAc TMA TAC
        self.cart = (0x1A5, 2, 1, 1)
        self.cart_ram = cart_ram
        self.joy = (0x0E, 0x07)
        self.cpu_cycles = 0x0102030405060708
        self.serial = (0x5A, 0x81)


def _v9_at_documented_offsets(sp: Spec) -> bytes:
    buf = bytearray(133021)
    buf[0], buf[1] = 9, sp.bootrom
    buf[5:11] = bytes(sp.regs)
    buf[11:17] = struct.pack("<HHH", sp.hl, sp.sp, sp.pc)
    buf[17:23] = bytes(sp.cpu_flags)
    buf[23:8215] = sp.vram
    buf[8215:8375] = sp.oam
    buf[8375:8386] = bytes(sp.lcd)  # LCDC BGP OBP0 OBP1 STAT LY LYC SCY SCX WY WX
    buf[8388:8405] = struct.pack("<QQB", sp.clock, sp.target, sp.mode)
    buf[8405:9125] = sp.scan
    # 9125: sound (138), 9263: renderer (115200), zero-filled
    buf[124463:132655] = sp.wram
    buf[132655:132751] = sp.non_io0
    buf[132751:132827] = sp.io
    buf[132827:132954] = sp.hram
    buf[132954:133006] = sp.non_io1
    buf[133006:133014] = struct.pack("<BBHHBB", *sp.timer)
    buf[133014:133019] = struct.pack("<HBBB", *sp.cart)
    buf[133019:133021] = bytes(sp.joy)
    return bytes(buf[:133019]) + sp.cart_ram + bytes(buf[133019:])


def _check(st: sio.PyBoyState, sp: Spec, version: int) -> None:
    assert st.version == version
    assert st.bootrom_enabled == sp.bootrom
    assert (st.a, st.f, st.b, st.c, st.d, st.e) == sp.regs
    assert (st.h, st.l_reg, st.sp, st.pc) == (sp.hl >> 8, sp.hl & 0xFF, sp.sp, sp.pc)
    assert (st.ime, st.halted, st.stopped, st.ie, st.interrupt_queued, st.if_reg) == sp.cpu_flags
    assert st.vram == sp.vram and st.oam == sp.oam
    lcd = (st.lcdc, st.bgp, st.obp0, st.obp1, st.stat, st.ly, st.lyc, st.scy, st.scx, st.wy, st.wx)
    assert lcd == sp.lcd
    assert (st.lcd_clock, st.lcd_clock_target, st.next_stat_mode) == (sp.clock, sp.target, sp.mode)
    assert st.scanline_params == sp.scan
    assert st.wram == sp.wram and st.non_io_ram0 == sp.non_io0 and st.io_ports == sp.io
    assert st.hram == sp.hram and st.non_io_ram1 == sp.non_io1
    assert (st.div, st.tima, st.div_counter, st.tima_counter, st.tma, st.tac) == sp.timer
    assert (st.rombank, st.rambank, st.rambank_enabled, st.memorymodel) == sp.cart
    assert st.cart_ram == sp.cart_ram
    assert (st.joypad_directional, st.joypad_standard) == sp.joy
    if version >= 12:
        assert st.cpu_cycles == sp.cpu_cycles
    else:
        assert st.cpu_cycles == 0
    if version >= 15:
        assert (st.serial_sb, st.serial_sc) == sp.serial
    else:
        assert (st.serial_sb, st.serial_sc) == (sp.io[1], sp.io[2])


@pytest.mark.parametrize("cart_ram", [0, 8192, 32768])
def test_v9_documented_offsets(cart_ram):
    sp = Spec(_rand(cart_ram))
    data = _v9_at_documented_offsets(sp)
    assert len(data) == 133021 + cart_ram
    st = sio.parse_pyboy_state(data)
    _check(st, sp, 9)
    # the writer produces the same bytes (zero sound and renderer sections)
    assert sio.pack_pyboy_state(st) == data


def test_v9_old_renderer_size_keeps_hram():
    """v9-v12 files from older PyBoy carry a 92,022-byte renderer; the HRAM
    (OAM DMA routine) must still be read from the right place (the
    reference's HRAM regression test)."""
    sp = Spec()
    sp.hram = bytes([0x3E, 0xC3, 0xE0, 0x46, 0xC9]) + sp.hram[5:]
    new = _v9_at_documented_offsets(sp)
    old = new[:9263] + bytes(92022) + new[9263 + 115200 :]
    _check(sio.parse_pyboy_state(old), sp, 9)
    _check(sio.parse_pyboy_state(new), sp, 9)


def _sound(version: int, spf: int = 3) -> bytes:
    """Sound section as the reference parser walks it: v13 fixed fields,
    v14+ with an audio buffer of (samples_per_frame + 1) * 2 bytes."""
    tone = 2 + 3 + 2 + 1 + 1 + 6 * 8
    channels = (tone + 3 + 8 + 1 + 8) + tone + (16 + 1 + 1 + 1 + 2 + 1 + 1 + 5 * 8) + (8 + 1 + 7 * 8)
    if version <= 12:
        return _rand(138)
    if version == 13:
        return _rand(16 + channels)
    head = _rand(8) + struct.pack("<Q", spf) + _rand(8) + _rand((spf + 1) * 2)
    return head + _rand(1 + 7 * 8 + 1 + 1 + 8 + channels)


def _build(version: int, sp: Spec, *, sound: bytes, renderer: int = 115200) -> bytes:
    """Section by section, with each version's additions."""
    out = [bytes([version, sp.bootrom, 0, 0, 0]), bytes(sp.regs),
           struct.pack("<HHH", sp.hl, sp.sp, sp.pc), bytes(sp.cpu_flags)]  # fmt: skip
    if version >= 12:
        out.append(struct.pack("<Q", sp.cpu_cycles))
    out += [sp.vram, sp.oam, bytes(sp.lcd), bytes(2)]
    if version >= 13:
        out.append(_rand(8))  # LCD last_cycles
    out += [struct.pack("<QQB", sp.clock, sp.target, sp.mode), sp.scan, sound, _rand(renderer)]
    out += [sp.wram, sp.non_io0, sp.io, sp.hram, sp.non_io1, struct.pack("<BBHHBB", *sp.timer)]
    if version >= 12:
        out.append(_rand(8))  # timer last_cycles
    if version >= 13:
        out.append(_rand(8))  # timer cycles_to_interrupt
    out += [struct.pack("<HBBB", *sp.cart), sp.cart_ram, bytes(sp.joy)]
    if version >= 15:
        out.append(bytes(sp.serial) + _rand(2 + 32))
    return b"".join(out)


@pytest.mark.parametrize("version", [10, 11, 12, 13, 14, 15])
@pytest.mark.parametrize("cart_ram", [0, 8192])
def test_versions_10_to_15(version, cart_ram):
    sp = Spec(_rand(cart_ram))
    renderer = 92022 if version <= 12 else 115200
    data = _build(version, sp, sound=_sound(version), renderer=renderer)
    _check(sio.parse_pyboy_state(data), sp, version)
    if version <= 12:  # the newer renderer size is recognised too
        data = _build(version, sp, sound=_sound(version), renderer=115200)
        _check(sio.parse_pyboy_state(data), sp, version)


@pytest.mark.parametrize("version", [14, 15])
def test_sound_size_from_expected_cart_ram(version):
    """With the cart RAM size known, the v14+ sound section is what lies
    between the scanline parameters and the sections after it.  For v15 the
    reference takes one byte more than that arithmetic (state_io.py:349-373),
    so a v15 file whose later sections total one byte less than the stated
    cart RAM implies (here: 8,191 bytes of cart RAM for an 8 KiB header)
    parses cleanly."""
    cram = 8192 if version == 14 else 8191
    sp = Spec(_rand(cram))
    data = _build(version, sp, sound=_sound(version, spf=700))
    _check(sio.parse_pyboy_state(data, expected_cart_ram_size=8192), sp, version)
    # too small a file for the stated cart RAM
    with pytest.raises(ValueError, match="sound section"):
        sio.parse_pyboy_state(data[:130000], expected_cart_ram_size=8192)


def test_errors():
    sp = Spec()
    data = bytearray(_v9_at_documented_offsets(sp))
    for v in (8, 16):
        data[0] = v
        with pytest.raises(ValueError, match="Unsupported state version"):
            sio.parse_pyboy_state(bytes(data))
    data[0] = 9
    data[4] = 1
    with pytest.raises(ValueError, match="CGB"):
        sio.parse_pyboy_state(bytes(data))
    data[4] = 0
    with pytest.raises(EOFError):
        sio.parse_pyboy_state(bytes(data[:20]))
    with pytest.raises(EOFError):  # ends inside the renderer section
        sio.parse_pyboy_state(bytes(data[:9300]))
    # fewer than 2 bytes after the cart header: no room for the joypad bytes
    v15 = _build(15, sp, sound=_sound(15))
    with pytest.raises(ValueError, match="cart RAM"):
        sio.parse_pyboy_state(v15[:-37])


def test_file_roundtrip(tmp_path):
    sp = Spec(_rand(32768))
    st = sio.parse_pyboy_state(_v9_at_documented_offsets(sp))
    path = tmp_path / "x.state"
    sio.save_pyboy_state(st, path)
    assert path.stat().st_size == 133021 + 32768
    assert sio.load_pyboy_state(path) == st


def _image(ram: int = 0) -> sio.EnvImage:
    return sio.EnvImage(
        scalars=RNG.integers(0, 1 << 20, 32).astype(np.int64),
        cart_state=RNG.integers(0, 200, 20).astype(np.int32),
        mem=RNG.integers(0, 256, 65536, dtype=np.uint8),
        cart_ram=RNG.integers(0, 256, ram, dtype=np.uint8),
    )


def test_apply_known_answers():
    sp = Spec(b"\x42" * 2048)  # a 2 KiB cart RAM image for an 8 KiB cart: zero-padded
    st = sio.parse_pyboy_state(_v9_at_documented_offsets(sp))
    img = _image(ram=8192)
    before = img.mem.copy()
    keep = {n: img.get(n) for n in ("instr_count", "trap_flag", "actions", "serial_len")}
    mbc = int(img.cart_state[CS["mbc_kind"]])
    sio.apply_state_to_image(st, img)
    m = img.mem
    # registers and CPU flags
    assert [img.get(n) for n in "abcdefhl"] == [0x11, 0x22, 0x33, 0x44, 0x55, 0xB0, 0xC0, 0xDE]
    assert (img.get("sp"), img.get("pc"), img.get("ime"), img.get("halted")) == (0xDFF0, 0x1234, 1, 0)
    assert img.get("ime_delay") == 0
    # memory regions and the registers written after the IO dump
    assert m[0x8000:0xA000].tobytes() == sp.vram and m[0xC000:0xE000].tobytes() == sp.wram
    assert m[0xFE00:0xFEA0].tobytes() == sp.oam and m[0xFEA0:0xFF00].tobytes() == sp.non_io0
    assert m[0xFF80:0xFFFF].tobytes() == sp.hram and m[0xFF4C:0xFF80].tobytes() == sp.non_io1
    assert m[0xFF00] == 0xCF and m[0xFFFF] == 0x1F and m[0xFF0F] == 0x05
    assert m[0xFF01] == sp.io[1] and m[0xFF02] == sp.io[2]
    assert list(m[0xFF04:0xFF08]) == [0xAB, 0x17, 0x80, 0x05]
    assert list(m[0xFF40:0xFF46]) == [0x91, 0x85, 0x10, 0x20, 0x42, 0x43]
    assert list(m[0xFF47:0xFF4C]) == [0xE4, 0xD0, 0xE0, 0x30, 0x47]
    assert m[0xFF03] == sp.io[3] and m[0xFF46] == sp.io[0x46]  # straight from the IO dump
    # outside the savestate: ROM area, cart RAM window, echo RAM untouched
    for lo, hi in ((0, 0x8000), (0xA000, 0xC000), (0xE000, 0xFE00)):
        assert np.array_equal(m[lo:hi], before[lo:hi])
    # timer: DIV counter = DIV << 8 | low byte; TAC 5 selects bit 3
    assert img.get("div_counter") == 0xAB56
    assert img.get("timer_prev_in") == (0xAB56 >> 3) & 1 == 0
    assert img.get("tima_reload_pending") == 0 and img.get("tima_reload_delay") == 0
    assert img.get("joyp_select") == 0x30
    # PPU: LY, position in the line, window line, STAT edge memory
    assert img.get("ppu_ly") == 0x42 and img.get("ppu_scanline_cycle") == 70000 % 456
    assert img.get("ppu_window_line") == 0x42 - 0x30
    assert img.get("ppu_stat_prev") == 0b0010  # STAT mode 1 (0x85 & 3) is bit 1; LY != LYC
    assert img.get("cycle_count") == 70000 and img.get("cycle_in_frame") == 0
    # cart: PyBoy's 9-bit bank number kept whole across the two slots
    cs = img.cart_state
    assert (cs[CS["rom_bank_lo"]], cs[CS["rom_bank_hi"]]) == (0xA5, 1)
    assert (cs[CS["ram_bank"]], cs[CS["ram_enable"]], cs[CS["bank_mode"]]) == (2, 1, 1)
    assert cs[CS["bootrom_enabled"]] == 1 and cs[CS["mbc_kind"]] == mbc
    assert img.cart_ram[:2048].tolist() == [0x42] * 2048 and not img.cart_ram[2048:].any()
    # untouched scalars
    assert {n: img.get(n) for n in keep} == keep
    # env-0 latches from the per-line scroll/window parameters
    lat, scan = img.latches, sp.scan
    for y in (0, 47, 48, 143):
        scx, scy, wx, wy = scan[5 * y : 5 * y + 4]
        want = [0x91, scx, scy, 0xE4, wx, wy, (y - wy) & 0xFF if y >= wy else 0, 0xD0, 0xE0]
        assert lat[:, y].tolist() == want


@pytest.mark.parametrize(
    "tac,want_bit", [(0, None), (3, None), (4, 9), (5, 3), (6, 5), (7, 7)]
)
def test_apply_timer_edge_input(tac, want_bit):
    st = sio.parse_pyboy_state(_v9_at_documented_offsets(Spec()))
    for div, low in ((0x02, 0x00), (0x00, 0x08), (0x00, 0x20), (0x00, 0x80), (0xFF, 0xFF)):
        st.tac, st.div, st.div_counter = tac, div, low
        img = _image()
        sio.apply_state_to_image(st, img)
        full = (div << 8) | low
        exp = 0 if want_bit is None else (full >> want_bit) & 1
        assert img.get("timer_prev_in") == exp


def test_apply_stat_window_and_cycles():
    st = sio.parse_pyboy_state(_v9_at_documented_offsets(Spec()))
    for stat, ly, lyc, want in ((0x80, 3, 3, 0b1001), (0x81, 150, 0, 0b0010), (0x82, 7, 8, 0b0100),
                                (0x83, 9, 9, 0b1000)):  # fmt: skip
        st.stat, st.ly, st.lyc = stat, ly, lyc
        img = _image()
        sio.apply_state_to_image(st, img)
        assert img.get("ppu_stat_prev") == want
    st.ly, st.wy = 10, 20
    img = _image()
    sio.apply_state_to_image(st, img)
    assert img.get("ppu_window_line") == 0
    st.cpu_cycles, st.lcd_clock = 123456789, 5
    sio.apply_state_to_image(st, img)
    assert img.get("cycle_count") == 123456789
    st.cpu_cycles, st.lcd_clock = 0, 2**64 - 1
    sio.apply_state_to_image(st, img)
    assert img.get("cycle_count") == 2**63 - 1


def test_state_from_image_known_answers():
    img = _image(ram=2048)
    m, cs = img.mem, img.cart_state
    img.set("ppu_ly", 0x142)  # masked to 8 bits
    for scan, ly, mode in ((79, 10, 2), (80, 10, 3), (251, 10, 3), (252, 10, 0), (5, 144, 1)):
        img.set("ppu_scanline_cycle", scan)
        img.set("ppu_ly", ly)
        st = sio.state_from_image(img)
        assert st.next_stat_mode == mode
        assert st.lcd_clock == ly * 456 + scan and st.lcd_clock_target == st.lcd_clock + 456
    img.set("div_counter", 0x1ABCD)
    img.set("f", 0x1FF)
    cs[CS["rom_bank_lo"]], cs[CS["rom_bank_hi"]] = 0xFF, 0x07
    st = sio.state_from_image(img)
    assert (st.div, st.div_counter) == (0xAB, 0xCD)
    assert st.f == 0xF0
    assert st.rombank == (3 << 5) | 0x7F
    assert st.ie == m[0xFFFF] and st.if_reg == m[0xFF0F] and st.stat == m[0xFF41]
    assert st.scanline_params == bytes((m[0xFF43], m[0xFF42], m[0xFF4B], m[0xFF4A], 0)) * 144
    assert (st.joypad_directional, st.joypad_standard, st.tima_counter) == (0x0F, 0x0F, 0)
    assert st.cart_ram == img.cart_ram.tobytes() and len(st.cart_ram) == 2048
    assert st.version == 9 and st.stopped == 0 and st.interrupt_queued == 0


def test_image_roundtrip_through_file(tmp_path):
    """image -> state -> file -> state -> fresh image -> state is stable."""
    img = _image(ram=8192)
    img.set("ppu_ly", 100)
    img.set("ppu_scanline_cycle", 300)
    img.set("halted", 1)
    st = sio.state_from_image(img)
    path = tmp_path / "rt.state"
    sio.save_pyboy_state(st, path)
    st2 = sio.load_pyboy_state(path, expected_cart_ram_size=8192)
    # version 9 has no CPU cycle field: the count does not survive a file
    assert st2.cpu_cycles == 0
    st2.cpu_cycles = st.cpu_cycles
    assert st2 == st
    st2.cpu_cycles = 0
    img2 = _image(ram=8192)
    sio.apply_state_to_image(st2, img2)
    assert img2.get("cycle_count") == 100 * 456 + 300  # falls back to the LCD clock
    st3 = sio.state_from_image(img2)
    for k, v in st.__dict__.items():
        if k not in ("cpu_cycles", "io_ports"):
            assert getattr(st3, k) == v, k

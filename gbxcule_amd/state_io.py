"""PyBoy ``.state`` savestates for the HIP backend.

The file format is host work: a ~133 KB little-endian record parsed and
written here in Python.  Moving one env's state between the device and that
record is one synchronous call each way through the C ABI
(``gbx_export_env`` / ``gbx_import_env``), in place of the reference's one
Warp copy per field.

Behaviour follows the reference's ``src/gbxcule/core/state_io.py``:

* ``load_pyboy_state`` reads versions 9-15 (``state_io.py:253-551``),
  including the size-derived sound section of v14+ and the renderer-size
  detection of v9-12 files;
* ``save_pyboy_state`` writes version 9 (``state_io.py:553-659``);
* ``state_from_warp_backend`` / ``apply_state_to_warp_backend`` map a state
  to and from one env (``state_io.py:662-837`` / ``839-1154``).  The mapping
  itself is ``state_from_image`` / ``apply_state_to_image`` on a host
  ``EnvImage``, so it is testable without a GPU.

The byte layout is documented in the reference's
``docs/pyboy_state_format.md``.
"""

from __future__ import annotations

import struct
from dataclasses import dataclass
from pathlib import Path
from typing import TYPE_CHECKING, BinaryIO

import numpy as np

from .abi import CART_STATE_FIELDS, CART_STATE_STRIDE, MEM_SIZE

if TYPE_CHECKING:  # pragma: no cover
    from .backend import HipVecBackend

PYBOY_STATE_VERSION_MIN = 9
PYBOY_STATE_VERSION_MAX = 15
PYBOY_STATE_VERSION_SAVE = 9

VRAM_SIZE = 8192
OAM_SIZE = 160
WRAM_SIZE = 8192
HRAM_SIZE = 127
IO_PORTS_SIZE = 76
NON_IO_RAM0_SIZE = 96
NON_IO_RAM1_SIZE = 52
SCANLINE_PARAMS_SIZE = 720
SOUND_SIZE_V9 = 138
RENDERER_SIZE_V9_12 = 144 * 160 * 4 - 138  # 92,022 bytes in older v9-v12 files
RENDERER_SIZE = 144 * 160 * 5  # 115,200 bytes
SERIAL_STATE_SIZE = 36  # v15+
CART_RAM_SIZES = (0, 2048, 8192, 32768, 131072)

CYCLES_PER_SCANLINE = 456
SCREEN_H = 144
_RAM_BLOCK = WRAM_SIZE + NON_IO_RAM0_SIZE + IO_PORTS_SIZE + HRAM_SIZE + NON_IO_RAM1_SIZE

# per-env scalar ids of the C ABI (GBX_FIELD_*)
FIELDS = (
    "pc", "sp", "a", "b", "c", "d", "e", "h", "l", "f",
    "instr_count", "cycle_count", "cycle_in_frame", "trap_flag", "trap_pc",
    "trap_opcode", "trap_kind", "actions", "joyp_select", "serial_len",
    "serial_overflow", "ime", "ime_delay", "halted", "div_counter",
    "timer_prev_in", "tima_reload_pending", "tima_reload_delay",
    "ppu_scanline_cycle", "ppu_ly", "ppu_window_line", "ppu_stat_prev",
)  # fmt: skip
_F = {name: i for i, name in enumerate(FIELDS)}
_CS = {name: i for i, name in enumerate(CART_STATE_FIELDS)}
# env-0 scanline latch rows (order of the reference's latch arrays,
# kernels/cpu_step_builder.py:494-524)
LATCH_ROWS = ("lcdc", "scx", "scy", "bgp", "wx", "wy", "win_line", "obp0", "obp1")


@dataclass
class PyBoyState:
    """One DMG machine as a PyBoy savestate holds it (field names of the
    reference's ``PyBoyState``, ``state_io.py:54-126``)."""

    version: int
    bootrom_enabled: int
    a: int
    f: int
    b: int
    c: int
    d: int
    e: int
    h: int
    l_reg: int
    sp: int
    pc: int
    ime: int
    halted: int
    stopped: int
    ie: int
    interrupt_queued: int
    if_reg: int
    cpu_cycles: int
    vram: bytes
    oam: bytes
    lcdc: int
    stat: int
    ly: int
    lyc: int
    scy: int
    scx: int
    wy: int
    wx: int
    bgp: int
    obp0: int
    obp1: int
    lcd_clock: int
    lcd_clock_target: int
    next_stat_mode: int
    scanline_params: bytes
    wram: bytes
    hram: bytes
    io_ports: bytes
    non_io_ram0: bytes
    non_io_ram1: bytes
    div: int
    tima: int
    tma: int
    tac: int
    div_counter: int
    tima_counter: int
    rombank: int
    rambank: int
    rambank_enabled: int
    memorymodel: int
    cart_ram: bytes
    joypad_directional: int
    joypad_standard: int
    serial_sb: int
    serial_sc: int


# -- reading -----------------------------------------------------------------
class _Cursor:
    """Read position over a whole file held in memory.  Integer reads raise
    ``EOFError`` when the file ends early; blob reads return what is left,
    as a file object's ``read`` does."""

    def __init__(self, data: bytes) -> None:
        self.data = data
        self.pos = 0

    def blob(self, n: int) -> bytes:
        out = self.data[self.pos : self.pos + n]
        self.pos = min(self.pos + n, len(self.data))
        return out

    def skip(self, n: int) -> None:
        self.pos = min(self.pos + n, len(self.data))

    def _int(self, n: int, fmt: str) -> int:
        raw = self.blob(n)
        if len(raw) != n:
            raise EOFError("Unexpected end of file")
        return struct.unpack(fmt, raw)[0]

    def u8(self) -> int:
        return self._int(1, "<B")

    def u16(self) -> int:
        return self._int(2, "<H")

    def u64(self) -> int:
        return self._int(8, "<Q")

    @property
    def left(self) -> int:
        return len(self.data) - self.pos


def _timer_block_size(version: int) -> int:
    return 8 + (8 if version >= 12 else 0) + (8 if version >= 13 else 0)


def _tail_size(version: int) -> int:
    """Joypad bytes plus the v15+ serial block at the end of the file."""
    return 2 + (SERIAL_STATE_SIZE if version >= 15 else 0)


# Sound channel records of PyBoy v13+ (state_io.py:218-250): fixed sizes.
_TONE = 2 + 3 + 2 + 1 + 1 + 8 * 6
_SWEEP = _TONE + 3 + 8 + 1 + 8
_WAVE = 16 + 1 + 1 + 1 + 2 + 1 + 1 + 8 * 5
_NOISE = 8 + 1 + 8 * 7
_CHANNELS = _SWEEP + _TONE + _WAVE + _NOISE


def _skip_sound(cur: _Cursor, version: int, max_sound_size: int | None) -> None:
    """Sound section (state_io.py:162-215)."""
    if version == 13:
        cur.skip(16 + _CHANNELS)  # last_cycles, cycles, four channels
    elif version >= 14:
        if max_sound_size is not None:
            if max_sound_size < 0:
                raise ValueError(
                    f"State file too small for sound section: {max_sound_size} bytes"
                )
            cur.skip(max_sound_size)
            return
        cur.skip(8)  # audiobuffer head
        samples_per_frame = cur.u64()
        cur.skip(8)  # cycles per sample
        cur.skip((samples_per_frame + 1) * 2)  # audio buffer
        cur.skip(1 + 8 * 7 + 1 + 1 + 8)  # speed shift .. channel enable bits
        cur.skip(_CHANNELS)
    else:
        cur.skip(SOUND_SIZE_V9)


def _renderer_size(cur: _Cursor, version: int) -> int:
    """v9-v12 files come with either renderer size; take the one that leaves a
    valid cart RAM size behind, preferring the older (state_io.py:407-459)."""
    if version > 12:
        return RENDERER_SIZE
    after = _RAM_BLOCK + _timer_block_size(version) + 5 + _tail_size(version)
    old_left = cur.left - RENDERER_SIZE_V9_12 - after
    new_left = cur.left - RENDERER_SIZE - after
    old_ok, new_ok = old_left in CART_RAM_SIZES, new_left in CART_RAM_SIZES
    if new_ok and not old_ok:
        return RENDERER_SIZE
    if old_ok or old_left >= 0:
        return RENDERER_SIZE_V9_12
    return RENDERER_SIZE


def parse_pyboy_state(data: bytes, *, expected_cart_ram_size: int | None = None) -> PyBoyState:
    """Parse the bytes of a v9-v15 DMG savestate (state_io.py:275-551)."""
    cur = _Cursor(bytes(data))
    version = cur.u8()
    if not PYBOY_STATE_VERSION_MIN <= version <= PYBOY_STATE_VERSION_MAX:
        raise ValueError(
            f"Unsupported state version {version}, "
            f"expected {PYBOY_STATE_VERSION_MIN}-{PYBOY_STATE_VERSION_MAX}"
        )
    bootrom_enabled = cur.u8()
    cur.u8()  # key1
    cur.u8()  # double speed
    if cur.u8() != 0:
        raise ValueError("CGB mode not supported, only DMG")

    a, f, b, c, d, e = (cur.u8() for _ in range(6))
    hl, sp, pc = cur.u16(), cur.u16(), cur.u16()
    ime, halted, stopped, ie, queued, if_reg = (cur.u8() for _ in range(6))
    cpu_cycles = cur.u64() if version >= 12 else 0

    vram = cur.blob(VRAM_SIZE)
    oam = cur.blob(OAM_SIZE)
    lcdc, bgp, obp0, obp1, stat, ly, lyc, scy, scx, wy, wx = (cur.u8() for _ in range(11))
    cur.u8()  # LCD cgb flag
    cur.u8()  # LCD speed shift
    if version >= 13:
        cur.u64()  # LCD last_cycles
    lcd_clock = cur.u64()
    lcd_clock_target = cur.u64()
    next_stat_mode = cur.u8()
    scanline_params = cur.blob(SCANLINE_PARAMS_SIZE)

    max_sound = None
    if expected_cart_ram_size is not None and version >= 14:
        after = (
            RENDERER_SIZE
            + _RAM_BLOCK
            + _timer_block_size(version)
            + 5
            + expected_cart_ram_size
            + _tail_size(version)
        )
        max_sound = cur.left - after + (1 if version >= 15 else 0)
    _skip_sound(cur, version, max_sound)
    cur.skip(_renderer_size(cur, version))

    wram = cur.blob(WRAM_SIZE)
    non_io_ram0 = cur.blob(NON_IO_RAM0_SIZE)
    io_ports = cur.blob(IO_PORTS_SIZE)
    hram = cur.blob(HRAM_SIZE)
    non_io_ram1 = cur.blob(NON_IO_RAM1_SIZE)

    div, tima = cur.u8(), cur.u8()
    div_counter, tima_counter = cur.u16(), cur.u16()
    tma, tac = cur.u8(), cur.u8()
    if version >= 12:
        cur.u64()  # timer last_cycles
    if version >= 13:
        cur.u64()  # timer cycles_to_interrupt

    rombank = cur.u16()
    rambank, rambank_enabled, memorymodel = cur.u8(), cur.u8(), cur.u8()
    cart_ram_size = cur.left - _tail_size(version)
    if cart_ram_size < 0:
        raise ValueError(f"State file too small for cart RAM: {cart_ram_size} bytes remaining")
    cart_ram = cur.blob(cart_ram_size)
    if len(cart_ram) != cart_ram_size:  # pragma: no cover - cannot happen on bytes
        raise EOFError("Unexpected end of file while reading cart RAM")
    joypad_directional, joypad_standard = cur.u8(), cur.u8()
    if version >= 15:
        serial_sb, serial_sc = cur.u8(), cur.u8()
    else:
        serial_sb, serial_sc = io_ports[0x01], io_ports[0x02]

    return PyBoyState(
        version=version, bootrom_enabled=bootrom_enabled,
        a=a, f=f, b=b, c=c, d=d, e=e, h=(hl >> 8) & 0xFF, l_reg=hl & 0xFF,
        sp=sp, pc=pc, ime=ime, halted=halted, stopped=stopped, ie=ie,
        interrupt_queued=queued, if_reg=if_reg, cpu_cycles=cpu_cycles,
        vram=vram, oam=oam, lcdc=lcdc, stat=stat, ly=ly, lyc=lyc, scy=scy, scx=scx,
        wy=wy, wx=wx, bgp=bgp, obp0=obp0, obp1=obp1, lcd_clock=lcd_clock,
        lcd_clock_target=lcd_clock_target, next_stat_mode=next_stat_mode,
        scanline_params=scanline_params, wram=wram, hram=hram, io_ports=io_ports,
        non_io_ram0=non_io_ram0, non_io_ram1=non_io_ram1, div=div, tima=tima, tma=tma,
        tac=tac, div_counter=div_counter, tima_counter=tima_counter, rombank=rombank,
        rambank=rambank, rambank_enabled=rambank_enabled, memorymodel=memorymodel,
        cart_ram=cart_ram, joypad_directional=joypad_directional,
        joypad_standard=joypad_standard, serial_sb=serial_sb, serial_sc=serial_sc,
    )  # fmt: skip


def load_pyboy_state(
    path: str | Path, *, expected_cart_ram_size: int | None = None
) -> PyBoyState:
    """Read a PyBoy savestate file (versions 9-15, DMG only)."""
    return parse_pyboy_state(Path(path).read_bytes(), expected_cart_ram_size=expected_cart_ram_size)


# -- writing -----------------------------------------------------------------
def pack_pyboy_state(state: PyBoyState) -> bytes:
    """The version-9 record of ``state`` (state_io.py:565-659): sound and
    renderer sections are zero-filled, the renderer at 115,200 bytes."""
    blobs = (
        ("vram", VRAM_SIZE), ("oam", OAM_SIZE), ("scanline_params", SCANLINE_PARAMS_SIZE),
        ("wram", WRAM_SIZE), ("non_io_ram0", NON_IO_RAM0_SIZE), ("io_ports", IO_PORTS_SIZE),
        ("hram", HRAM_SIZE), ("non_io_ram1", NON_IO_RAM1_SIZE),
    )  # fmt: skip
    for name, size in blobs:
        assert len(getattr(state, name)) == size, f"{name} must be {size} bytes"
    s = state
    u8 = lambda *v: bytes(x & 0xFF for x in v)  # noqa: E731
    u16 = lambda v: struct.pack("<H", v & 0xFFFF)  # noqa: E731
    u64 = lambda v: struct.pack("<Q", v & 0xFFFFFFFFFFFFFFFF)  # noqa: E731
    out = [
        u8(PYBOY_STATE_VERSION_SAVE, s.bootrom_enabled & 1, 0, 0, 0),
        u8(s.a, s.f, s.b, s.c, s.d, s.e),
        u16((s.h << 8) | s.l_reg), u16(s.sp), u16(s.pc),
        u8(s.ime, s.halted, s.stopped, s.ie, s.interrupt_queued, s.if_reg),
        bytes(s.vram), bytes(s.oam),
        u8(s.lcdc, s.bgp, s.obp0, s.obp1, s.stat, s.ly, s.lyc, s.scy, s.scx, s.wy, s.wx),
        u8(0, 0), u64(s.lcd_clock), u64(s.lcd_clock_target), u8(s.next_stat_mode),
        bytes(s.scanline_params),
        bytes(SOUND_SIZE_V9), bytes(RENDERER_SIZE),
        bytes(s.wram), bytes(s.non_io_ram0), bytes(s.io_ports), bytes(s.hram),
        bytes(s.non_io_ram1),
        u8(s.div, s.tima), u16(s.div_counter), u16(s.tima_counter), u8(s.tma, s.tac),
        u16(s.rombank), u8(s.rambank, s.rambank_enabled, s.memorymodel),
        bytes(s.cart_ram or b""),
        u8(s.joypad_directional, s.joypad_standard),
    ]  # fmt: skip
    return b"".join(out)


def save_pyboy_state(state: PyBoyState, path: str | Path) -> None:
    """Write ``state`` as a version-9 savestate file."""
    Path(path).write_bytes(pack_pyboy_state(state))


def _write_to(f: BinaryIO, state: PyBoyState) -> None:  # pragma: no cover - helper
    f.write(pack_pyboy_state(state))


# -- one env <-> state ---------------------------------------------------------
@dataclass
class EnvImage:
    """One env's device state on the host, as ``gbx_export_env`` returns it."""

    scalars: np.ndarray  # int64[32], FIELDS order
    cart_state: np.ndarray  # int32[20], CART_STATE_FIELDS order
    mem: np.ndarray  # uint8[65536]
    cart_ram: np.ndarray  # uint8[cart RAM bytes], empty when the cart has none
    latches: np.ndarray | None = None  # uint8[9, 144] env-0 latches to write

    def get(self, name: str) -> int:
        return int(self.scalars[_F[name]])

    def set(self, name: str, value: int) -> None:
        self.scalars[_F[name]] = int(value)


def state_from_image(img: EnvImage) -> PyBoyState:
    """PyBoyState of one env (state_from_warp_backend, state_io.py:662-837)."""
    mem, cs = img.mem, img.cart_state

    def region(lo: int, size: int) -> bytes:
        return bytes(mem[lo : lo + size])

    def m(addr: int) -> int:
        return int(mem[addr])

    ly = img.get("ppu_ly") & 0xFF
    scan = img.get("ppu_scanline_cycle")
    div_full = img.get("div_counter") & 0xFFFF
    lcd_clock = ly * CYCLES_PER_SCANLINE + scan
    if ly >= 144:
        mode = 1
    elif scan < 80:
        mode = 2
    elif scan < 252:
        mode = 3
    else:
        mode = 0
    line = bytes((m(0xFF43), m(0xFF42), m(0xFF4B), m(0xFF4A), 0))
    return PyBoyState(
        version=PYBOY_STATE_VERSION_SAVE,
        bootrom_enabled=int(cs[_CS["bootrom_enabled"]]) & 0x01,
        a=img.get("a") & 0xFF, f=img.get("f") & 0xF0, b=img.get("b") & 0xFF,
        c=img.get("c") & 0xFF, d=img.get("d") & 0xFF, e=img.get("e") & 0xFF,
        h=img.get("h") & 0xFF, l_reg=img.get("l") & 0xFF, sp=img.get("sp") & 0xFFFF,
        pc=img.get("pc") & 0xFFFF, ime=img.get("ime") & 0x01,
        halted=img.get("halted") & 0x01, stopped=0, ie=m(0xFFFF), interrupt_queued=0,
        if_reg=m(0xFF0F), cpu_cycles=img.get("cycle_count"),
        vram=region(0x8000, VRAM_SIZE), oam=region(0xFE00, OAM_SIZE),
        lcdc=m(0xFF40), stat=m(0xFF41), ly=ly, lyc=m(0xFF45), scy=m(0xFF42), scx=m(0xFF43),
        wy=m(0xFF4A), wx=m(0xFF4B), bgp=m(0xFF47), obp0=m(0xFF48), obp1=m(0xFF49),
        lcd_clock=lcd_clock, lcd_clock_target=lcd_clock + CYCLES_PER_SCANLINE,
        next_stat_mode=mode, scanline_params=line * SCREEN_H,
        wram=region(0xC000, WRAM_SIZE), hram=region(0xFF80, HRAM_SIZE),
        io_ports=region(0xFF00, IO_PORTS_SIZE), non_io_ram0=region(0xFEA0, NON_IO_RAM0_SIZE),
        non_io_ram1=region(0xFF4C, NON_IO_RAM1_SIZE),
        div=(div_full >> 8) & 0xFF, tima=m(0xFF05), tma=m(0xFF06), tac=m(0xFF07),
        div_counter=div_full & 0xFF, tima_counter=0,
        rombank=((int(cs[_CS["rom_bank_hi"]]) & 0x03) << 5)
        | (int(cs[_CS["rom_bank_lo"]]) & 0x7F),
        rambank=int(cs[_CS["ram_bank"]]) & 0xFF,
        rambank_enabled=int(cs[_CS["ram_enable"]]) & 0x01,
        memorymodel=int(cs[_CS["bank_mode"]]) & 0x01,
        cart_ram=bytes(img.cart_ram), joypad_directional=0x0F, joypad_standard=0x0F,
        serial_sb=m(0xFF01), serial_sc=m(0xFF02),
    )  # fmt: skip


_TIMER_BIT = (9, 3, 5, 7)  # TAC clock select -> DIV counter bit


def apply_state_to_image(state: PyBoyState, img: EnvImage) -> None:
    """Overlay ``state`` on one env's image (apply_state_to_warp_backend,
    state_io.py:839-1154).  Memory outside the regions a savestate carries
    (ROM area, cart RAM window, echo RAM) and the counters, trap fields,
    action and serial length keep their values.  ``img.latches`` is set from
    the scanline parameters: like the reference, loading into any env
    rewrites the env-0 latch rows."""
    st, mem, cs = state, img.mem, img.cart_state
    for name, value in (
        ("a", st.a), ("f", st.f), ("b", st.b), ("c", st.c), ("d", st.d), ("e", st.e),
        ("h", st.h), ("l", st.l_reg), ("sp", st.sp), ("pc", st.pc), ("ime", st.ime),
        ("ime_delay", 0), ("halted", st.halted),
    ):  # fmt: skip
        img.set(name, value)

    cs[_CS["bootrom_enabled"]] = 1 if st.bootrom_enabled != 0 else 0
    cs[_CS["rom_bank_lo"]] = st.rombank & 0xFF  # all 9 bits of PyBoy's bank number
    cs[_CS["rom_bank_hi"]] = (st.rombank >> 8) & 0xFF
    cs[_CS["ram_bank"]] = st.rambank & 0xFF
    cs[_CS["ram_enable"]] = st.rambank_enabled & 0x01
    cs[_CS["bank_mode"]] = st.memorymodel & 0x01
    if img.cart_ram.size > 0 and st.cart_ram:
        src = np.frombuffer(st.cart_ram, dtype=np.uint8)[: img.cart_ram.size]
        img.cart_ram[:] = 0
        img.cart_ram[: src.size] = src

    def put(lo: int, data: bytes) -> None:
        mem[lo : lo + len(data)] = np.frombuffer(data, dtype=np.uint8)

    put(0x8000, st.vram)
    put(0xFE00, st.oam)
    put(0xC000, st.wram)
    put(0xFF80, st.hram)
    put(0xFF00, st.io_ports)
    put(0xFEA0, st.non_io_ram0)
    put(0xFF4C, st.non_io_ram1)
    # registers the savestate keeps outside the IO-port dump
    for addr, value in (
        (0xFF40, st.lcdc), (0xFF41, st.stat), (0xFF42, st.scy), (0xFF43, st.scx),
        (0xFF44, st.ly), (0xFF45, st.lyc), (0xFF47, st.bgp), (0xFF48, st.obp0),
        (0xFF49, st.obp1), (0xFF4A, st.wy), (0xFF4B, st.wx), (0xFF0F, st.if_reg),
        (0xFFFF, st.ie), (0xFF01, st.serial_sb & 0xFF), (0xFF02, st.serial_sc & 0xFF),
        (0xFF00, 0xCF), (0xFF04, st.div), (0xFF05, st.tima), (0xFF06, st.tma),
        (0xFF07, st.tac),
    ):  # fmt: skip
        mem[addr] = value & 0xFF

    scan = st.scanline_params
    if len(scan) >= SCREEN_H * 5:
        lat = np.zeros((len(LATCH_ROWS), SCREEN_H), dtype=np.uint8)
        for y in range(SCREEN_H):
            scx, scy, wx, wy = scan[5 * y : 5 * y + 4]
            lat[:, y] = (
                st.lcdc & 0xFF, scx, scy, st.bgp & 0xFF, wx, wy,
                (y - wy) & 0xFF if y >= wy else 0, st.obp0 & 0xFF, st.obp1 & 0xFF,
            )  # fmt: skip
        img.latches = lat

    div_full = ((st.div & 0xFF) << 8) | (st.div_counter & 0xFF)
    img.set("div_counter", div_full)
    tac = st.tac
    img.set("timer_prev_in", (div_full >> _TIMER_BIT[tac & 3]) & 1 if tac & 0x04 else 0)
    img.set("tima_reload_pending", 0)
    img.set("tima_reload_delay", 0)
    img.set("joyp_select", 0x30)
    img.set("ppu_ly", st.ly)
    img.set("ppu_scanline_cycle", st.lcd_clock % CYCLES_PER_SCANLINE)
    cycles = st.cpu_cycles if st.cpu_cycles != 0 else st.lcd_clock
    img.set("cycle_count", min(max(cycles, -(2**63)), 2**63 - 1))
    img.set("cycle_in_frame", 0)
    img.set("ppu_window_line", st.ly - st.wy if st.ly >= st.wy else 0)
    mode = st.stat & 0x03
    stat_prev = (
        int(mode == 0) | (int(mode == 1) << 1) | (int(mode == 2) << 2) | (int(st.ly == st.lyc) << 3)
    )
    img.set("ppu_stat_prev", stat_prev)


def state_from_warp_backend(backend: HipVecBackend, env_idx: int = 0) -> PyBoyState:
    """PyBoyState of env ``env_idx`` (reference name kept for callers)."""
    if not backend._initialized:
        raise RuntimeError("Backend not initialized")
    return state_from_image(backend.export_env(env_idx))


def apply_state_to_warp_backend(state: PyBoyState, backend: HipVecBackend, env_idx: int = 0) -> None:
    """Load ``state`` into env ``env_idx`` (reference name kept for callers)."""
    if not backend._initialized:
        raise RuntimeError("Backend not initialized")
    img = backend.export_env(env_idx)
    apply_state_to_image(state, img)
    backend.import_env(env_idx, img)


state_from_backend = state_from_warp_backend
apply_state_to_backend = apply_state_to_warp_backend

__all__ = [
    "CART_STATE_STRIDE",
    "EnvImage",
    "FIELDS",
    "MEM_SIZE",
    "PyBoyState",
    "apply_state_to_backend",
    "apply_state_to_image",
    "apply_state_to_warp_backend",
    "load_pyboy_state",
    "pack_pyboy_state",
    "parse_pyboy_state",
    "save_pyboy_state",
    "state_from_backend",
    "state_from_image",
    "state_from_warp_backend",
]

"""Seeded synthetic cartridges for the five benchmark/parity workloads.

Every cart carries a valid header (entry ``NOP; JP 0150``, type/size codes,
header and global checksums) like the reference's micro-ROM builder
(``bench/roms/build_micro_rom.py:33-144``); the 48-byte logo area is left zero
because nothing on this path checks it.

Programs are random but structured so that every environment keeps running
legal code: jump/call/return targets are instruction boundaries inside the
program, stores that go through address registers are re-seeded into WRAM
first, and the stack pointer is kept inside WRAM.

* ``cart_c1``: 32 KiB ROM-only, 4 KiB loop of uniformly drawn legal non-CB
  opcodes (no HALT/STOP), LCD switched off, stores in C000-DFFF (LDH/LD (C)
  stores land in HRAM FF80-FFFE, the only place those opcodes can store to
  without touching IO).
* ``cart_c2``: 32 KiB ROM-only, 8 KiB of all legal opcodes including CB;
  every conditional branch is keyed on a JOYP read after a select write, so
  lanes diverge with their actions.  LCD stays on (boot value 0x91), BG blank.
* ``cart_c3``: PPU cart: 384 random tiles, random BG and window maps, window
  on at random WX/WY, 40 random 8x8 sprites written through OAM DMA, SCX/SCY
  walked once per frame from a seeded table (plus the button nibble on SCX).
* ``cart_c4``: 512 KiB MBC1 (or MBC3 + 32 KiB RAM) with a seeded program in
  each of banks 1..31, bank selected from the joypad each pass, timer IRQ at a
  random TAC rate, STAT LYC IRQ, VBlank IRQ, and EI/DI + HALT wake loops.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .asm import ILLEGAL, Asm, opcode_length

ROM_BANK = 0x4000
PROGRAM_ORIGIN = 0x0150


# ---------------------------------------------------------------------------
# Header
# ---------------------------------------------------------------------------
def header_checksum(rom: bytes | bytearray) -> int:
    x = 0
    for i in range(0x0134, 0x014D):
        x = (x - rom[i] - 1) & 0xFF
    return x


def global_checksum(rom: bytes | bytearray) -> int:
    arr = np.frombuffer(bytes(rom), dtype=np.uint8).astype(np.uint64)
    total = int(arr.sum()) - int(rom[0x014E]) - int(rom[0x014F])
    return total & 0xFFFF


def finalize_rom(
    rom: bytearray, title: str, cart_type: int, rom_code: int, ram_code: int
) -> bytes:
    rom[0x0100:0x0104] = bytes([0x00, 0xC3, 0x50, 0x01])
    t = title.upper().encode("ascii")[:11]
    rom[0x0134 : 0x0134 + len(t)] = t
    rom[0x0147] = cart_type
    rom[0x0148] = rom_code
    rom[0x0149] = ram_code
    rom[0x014A] = 0x01
    rom[0x014D] = header_checksum(rom)
    g = global_checksum(rom)
    rom[0x014E] = (g >> 8) & 0xFF
    rom[0x014F] = g & 0xFF
    return bytes(rom)


def _vectors(rom: bytearray, irq_targets: dict[int, int] | None = None) -> None:
    """RST vectors return immediately; IRQ vectors RETI unless redirected."""
    for v in range(0x00, 0x40, 8):
        rom[v] = 0xC9  # RET
    for v in range(0x40, 0x68, 8):
        rom[v] = 0xD9  # RETI
    for v, target in (irq_targets or {}).items():
        rom[v : v + 3] = bytes([0xC3, target & 0xFF, target >> 8])


# ---------------------------------------------------------------------------
# Random code generator
# ---------------------------------------------------------------------------
STORE_HL = {0x70, 0x71, 0x72, 0x73, 0x74, 0x75, 0x77, 0x36, 0x22, 0x32, 0x34, 0x35}
PUSH_OPS = {0xC5, 0xD5, 0xE5, 0xF5}
POP_OPS = {0xC1, 0xD1, 0xE1, 0xF1}
RST_OPS = {0xC7, 0xCF, 0xD7, 0xDF, 0xE7, 0xEF, 0xF7, 0xFF}
CALL_CC = {0xC4, 0xCC, 0xD4, 0xDC}
RET_CC = {0xC0, 0xC8, 0xD0, 0xD8}
JP_CC = {0xC2, 0xCA, 0xD2, 0xDA}
JR_CC = {0x20, 0x28, 0x30, 0x38}
SP_MOD = {0x31, 0xF9, 0x33, 0x3B, 0xE8}
CONDITIONAL = CALL_CC | RET_CC | JP_CC | JR_CC

LEGAL_NON_CB = [
    op for op in range(256) if op not in ILLEGAL and op not in (0xCB, 0x10, 0x76)
]


@dataclass
class _Jump:
    pos: int  # offset of the operand in the buffer
    kind: str  # "rel8" | "abs16"
    forward_only: bool
    block: int  # index of the block holding the jump


class CodeGen:
    """Emits random legal blocks into ``asm`` and resolves jump targets.

    ``stack`` selects the stack discipline: ``"reseed"`` reloads SP with a WRAM
    address before every stack instruction (used for looping programs), and
    ``"balanced"`` keeps SP balanced so the program can ``RET`` to its caller
    and interrupts can nest anywhere (used for banked subprograms).
    """

    def __init__(
        self,
        rng: np.random.Generator,
        asm: Asm,
        *,
        stack: str,
        joypad_conditions: bool,
        store_lo: int = 0xC000,
        store_hi: int = 0xDFFF,
        cart_ram: bool = False,
        backward_prob: float = 0.3,
    ) -> None:
        self.rng = rng
        self.a = asm
        self.stack = stack
        self.joy = joypad_conditions
        self.store_lo = store_lo
        self.store_hi = store_hi
        self.cart_ram = cart_ram
        self.backward_prob = backward_prob
        self.block_starts: list[int] = []
        self.jumps: list[_Jump] = []
        self.leaf_labels: list[int] = []

    # -- helpers -------------------------------------------------------------
    def r8(self) -> int:
        return int(self.rng.integers(0, 256))

    def store_addr(self, span: int = 1) -> int:
        if self.cart_ram and self.rng.random() < 0.3:
            return int(self.rng.integers(0xA000, 0xC000 - span + 1))
        return int(self.rng.integers(self.store_lo, self.store_hi - span + 2))

    def sp_value(self) -> int:
        return int(self.rng.integers(0xC100, 0xDE00)) & 0xFFFE

    def _jump(self, kind: str, forward_only: bool) -> None:
        self.jumps.append(
            _Jump(len(self.a.buf), kind, forward_only, len(self.block_starts) - 1)
        )
        self.a.emit(0) if kind == "rel8" else self.a.emit16(0)

    def joy_test(self) -> None:
        """Set Z and C from the JOYP low nibble (dpad or buttons)."""
        a = self.a
        a.ld_r_d8("A", 0x20 if self.rng.random() < 0.5 else 0x10)
        a.ldh_a8_a(0x00)
        a.ldh_a_a8(0x00)
        a.alu_d8("AND", 0x0F)
        a.alu_d8("CP", int(self.rng.integers(0, 16)))

    def raw(self, op: int) -> None:
        n = opcode_length(op)
        if op == 0xCB:
            cb = self.r8()
            if (cb & 7) == 6 and not (0x40 <= cb < 0x80):  # RMW on (HL)
                self.a.ld_rr_d16("HL", self.store_addr())
            self.a.emit(0xCB, cb)
            return
        self.a.emit(op)
        for _ in range(n - 1):
            self.a.emit(self.r8())

    # -- one block -------------------------------------------------------------
    def block(self, op: int) -> None:
        a = self.a
        self.block_starts.append(a.pc)
        reseed = self.stack == "reseed"
        if op in STORE_HL:
            a.ld_rr_d16("HL", self.store_addr())
            a.emit(op)
            if op == 0x36:
                a.emit(self.r8())
        elif op == 0x02:
            a.ld_rr_d16("BC", self.store_addr())
            a.emit(op)
        elif op == 0x12:
            a.ld_rr_d16("DE", self.store_addr())
            a.emit(op)
        elif op == 0xEA:
            a.emit(op)
            a.emit16(self.store_addr())
        elif op == 0x08:
            a.emit(op)
            a.emit16(self.store_addr(2))
        elif op == 0xE0:
            a.emit(op, int(self.rng.integers(0x80, 0xFF)))
        elif op == 0xE2:
            a.ld_r_d8("C", int(self.rng.integers(0x80, 0xFF)))
            a.emit(op)
        elif op in PUSH_OPS:
            if reseed:
                a.ld_rr_d16("SP", self.sp_value())
                a.emit(op)
            else:
                a.emit(op)
                for _ in range(int(self.rng.integers(0, 3))):
                    self.raw(self._plain_op())
                a.emit(0xC1 | (int(self.rng.integers(0, 4)) << 4))
        elif op in POP_OPS:
            if reseed:
                a.ld_rr_d16("SP", self.sp_value())
                a.emit(op)
            else:
                a.emit(0xC5 | (int(self.rng.integers(0, 4)) << 4))
                a.emit(op)
        elif op in RST_OPS:
            if reseed:
                a.ld_rr_d16("SP", self.sp_value())
            a.emit(op)
        elif op in SP_MOD:
            if reseed:
                if op == 0x31:
                    a.emit(op)
                    a.emit16(self.sp_value())
                elif op == 0xF9:
                    a.ld_rr_d16("HL", self.sp_value())
                    a.emit(op)
                else:
                    a.ld_rr_d16("SP", self.sp_value())
                    a.emit(op)
                    if op == 0xE8:
                        a.emit(self.r8())
            else:  # balanced pairs
                if op == 0x33:
                    a.emit(0x33, 0x3B)
                elif op == 0x3B:
                    a.emit(0x3B, 0x33)
                elif op == 0xE8:
                    k = int(self.rng.integers(-64, 64))
                    a.emit(0xE8, k & 0xFF, 0xE8, (-k) & 0xFF)
                else:  # LD SP,d16 / LD SP,HL would unbalance: read SP instead
                    a.emit(0xF8, self.r8())
        elif op in (0xC3, 0x18):
            a.emit(op)
            self._jump("abs16" if op == 0xC3 else "rel8", True)
        elif op in JP_CC or op in JR_CC:
            if self.joy:
                self.joy_test()
            a.emit(op)
            back = self.rng.random() < self.backward_prob
            self._jump("abs16" if op in JP_CC else "rel8", not back)
        elif op == 0xE9:  # JP (HL)
            a.emit(0x21)
            self._jump("abs16", True)
            a.emit(0xE9)
        elif op == 0xCD or op in CALL_CC:
            if reseed:
                a.ld_rr_d16("SP", self.sp_value())
            if op in CALL_CC and self.joy:
                self.joy_test()
            a.emit(op)
            if reseed:
                self._jump("abs16", True)
            else:
                self.jumps.append(_Jump(len(a.buf), "leaf", True, 0))
                a.emit16(0)
        elif op in (0xC9, 0xD9) or op in RET_CC:
            if reseed:
                a.ld_rr_d16("SP", self.sp_value())
            a.emit(0x21)  # LD HL,target ; PUSH HL ; RET
            self._jump("abs16", True)
            a.emit(0xE5)
            if op in RET_CC and self.joy:
                self.joy_test()
            a.emit(op)
            if op in RET_CC and not reseed:
                a.emit(0xE1)  # not taken: drop the pushed target
        else:
            self.raw(op)

    def _plain_op(self) -> int:
        """An opcode with no control flow, stack or store side effects."""
        while True:
            op = int(self.rng.choice(LEGAL_NON_CB))
            if (
                op in STORE_HL
                or op in PUSH_OPS
                or op in POP_OPS
                or op in RST_OPS
                or op in SP_MOD
                or op in CONDITIONAL
                or op in (0x02, 0x12, 0xEA, 0x08, 0xE0, 0xE2, 0xC3, 0x18, 0xE9)
                or op in (0xCD, 0xC9, 0xD9, 0xF3, 0xFB)
            ):
                continue
            return op

    def leaf(self) -> None:
        """A CALL target for balanced programs: a few plain ops then RET."""
        self.leaf_labels.append(self.a.pc)
        for _ in range(int(self.rng.integers(1, 6))):
            self.raw(self._plain_op())
        self.a.ret()

    # -- target resolution -------------------------------------------------------
    def resolve(self, end_block_addr: int) -> None:
        starts = np.array(self.block_starts + [end_block_addr], dtype=np.int64)
        buf = self.a.buf
        for j in self.jumps:
            if j.kind == "leaf":
                t = int(self.rng.choice(self.leaf_labels))
                buf[j.pos] = t & 0xFF
                buf[j.pos + 1] = t >> 8
                continue
            here = self.a.origin + j.pos + (1 if j.kind == "rel8" else 2)
            if j.forward_only:
                cand = starts[starts >= here]
            else:
                cand = starts
            if j.kind == "rel8":
                cand = cand[(cand - (here) >= -128) & (cand - here <= 127)]
            if cand.size == 0:
                cand = np.array([here])  # next instruction
            t = int(self.rng.choice(cand))
            if j.kind == "rel8":
                buf[j.pos] = (t - here) & 0xFF
            else:
                buf[j.pos] = t & 0xFF
                buf[j.pos + 1] = t >> 8


def _cb_pool() -> list[int]:
    return [0x100 | cb for cb in range(256)]


def _emit_random_program(gen: CodeGen, size: int, pool: list[int]) -> None:
    a = gen.a
    start = len(a.buf)
    while len(a.buf) - start < size:
        choice = int(gen.rng.choice(pool))
        if choice & 0x100:
            gen.block_starts.append(a.pc)
            cb = choice & 0xFF
            if (cb & 7) == 6 and not (0x40 <= cb < 0x80):
                a.ld_rr_d16("HL", gen.store_addr())
            a.emit(0xCB, cb)
        else:
            gen.block(choice)


# ---------------------------------------------------------------------------
# Configs
# ---------------------------------------------------------------------------
def cart_c1(seed: int = 0) -> bytes:
    """32 KiB ROM-only loop of legal non-CB opcodes with the LCD off."""
    rng = np.random.default_rng(seed)
    rom = bytearray(0x8000)
    _vectors(rom)
    a = Asm(origin=PROGRAM_ORIGIN)
    a.ld_rr_d16("SP", 0xDFF0)
    a.ld_r_d8("A", 0x00)
    a.ldh_a8_a(0x40)  # LCDC = 0 (LCD off)
    loop = a.pc
    gen = CodeGen(rng, a, stack="reseed", joypad_conditions=False)
    _emit_random_program(gen, 4096, LEGAL_NON_CB)
    end = a.pc
    a.jp(loop)
    gen.resolve(end)
    code = a.resolve()
    rom[PROGRAM_ORIGIN : PROGRAM_ORIGIN + len(code)] = code
    return finalize_rom(rom, "GBXAMD C1", 0x00, 0x00, 0x00)


def cart_c2(seed: int = 1) -> bytes:
    """32 KiB ROM-only, all legal opcodes incl. CB, joypad-keyed branches."""
    rng = np.random.default_rng(seed)
    rom = bytearray(0x8000)
    _vectors(rom)
    a = Asm(origin=PROGRAM_ORIGIN)
    a.ld_rr_d16("SP", 0xDFF0)
    loop = a.pc
    gen = CodeGen(rng, a, stack="reseed", joypad_conditions=True)
    _emit_random_program(gen, 8192, LEGAL_NON_CB + _cb_pool())
    end = a.pc
    a.jp(loop)
    gen.resolve(end)
    code = a.resolve()
    rom[PROGRAM_ORIGIN : PROGRAM_ORIGIN + len(code)] = code
    return finalize_rom(rom, "GBXAMD C2", 0x00, 0x00, 0x00)


# ROM data placement for the PPU cart (ROM-only: bank 1 is fixed at 0x4000).
_C3_TILES = 0x4000  # 384 * 16 = 6144 bytes
_C3_BGMAP = 0x5800  # 1024
_C3_WINMAP = 0x5C00  # 1024
_C3_OAM = 0x6000  # 160
_C3_WALK_X = 0x7000  # 256
_C3_WALK_Y = 0x7100  # 256


def _copy_loop(a: Asm, src: int, dst: int, count: int, tag: str) -> None:
    """HL=src, DE=dst, BC=count; copy bytes with LD A,(HL+) / LD (DE),A."""
    a.ld_rr_d16("HL", src)
    a.ld_rr_d16("DE", dst)
    a.ld_rr_d16("BC", count)
    a.label(tag)
    a.ld_a_hli()
    a.ld_de_a()
    a.inc_rr("DE")
    a.dec_rr("BC")
    a.ld_r_r("A", "B")
    a.alu_r("OR", "C")
    a.jr(tag, "NZ")


def cart_c3(seed: int = 2) -> bytes:
    """PPU cart: random VRAM/OAM, window on, SCX/SCY walked each frame."""
    rng = np.random.default_rng(seed)
    rom = bytearray(0x8000)
    _vectors(rom)
    rom[_C3_TILES : _C3_TILES + 6144] = rng.integers(0, 256, 6144, dtype=np.uint8).tobytes()
    rom[_C3_BGMAP : _C3_BGMAP + 1024] = rng.integers(0, 256, 1024, dtype=np.uint8).tobytes()
    rom[_C3_WINMAP : _C3_WINMAP + 1024] = rng.integers(0, 256, 1024, dtype=np.uint8).tobytes()
    oam = bytearray()
    for _ in range(40):
        y = int(rng.integers(0, 176))
        x = int(rng.integers(0, 176))
        tile = int(rng.integers(0, 256))
        attr = int(rng.integers(0, 256)) & 0xF0  # priority, flips, palette
        oam.extend((y, x, tile, attr))
    rom[_C3_OAM : _C3_OAM + 160] = bytes(oam)
    walk_x = np.cumsum(rng.integers(-2, 3, 256)) & 0xFF
    walk_y = np.cumsum(rng.integers(-2, 3, 256)) & 0xFF
    rom[_C3_WALK_X : _C3_WALK_X + 256] = walk_x.astype(np.uint8).tobytes()
    rom[_C3_WALK_Y : _C3_WALK_Y + 256] = walk_y.astype(np.uint8).tobytes()

    a = Asm(origin=PROGRAM_ORIGIN)
    a.ld_rr_d16("SP", 0xDFF0)
    _copy_loop(a, _C3_TILES, 0x8000, 6144, "cp_tiles")
    _copy_loop(a, _C3_BGMAP, 0x9800, 1024, "cp_bg")
    _copy_loop(a, _C3_WINMAP, 0x9C00, 1024, "cp_win")
    _copy_loop(a, _C3_OAM, 0xC100, 160, "cp_oam")
    a.ld_r_d8("A", 0xC1)
    a.ldh_a8_a(0x46)  # OAM DMA from C100
    for reg, val in (
        (0x47, int(rng.integers(0, 256))),  # BGP
        (0x48, int(rng.integers(0, 256))),  # OBP0
        (0x49, int(rng.integers(0, 256))),  # OBP1
        (0x4A, int(rng.integers(0, 144))),  # WY
        (0x4B, int(rng.integers(7, 167))),  # WX
    ):
        a.ld_r_d8("A", val)
        a.ldh_a8_a(reg)
    lcdc = 0x80 | 0x40 | 0x20 | 0x02 | 0x01 | (0x10 if rng.random() < 0.5 else 0)
    a.ld_r_d8("A", lcdc)
    a.ldh_a8_a(0x40)
    a.ld_r_d8("A", 0x00)
    a.ld_a16_a(0xC000)  # frame counter
    a.label("frame")
    a.label("wait_vbl")
    a.ldh_a_a8(0x44)
    a.alu_d8("CP", 144)
    a.jr("wait_vbl", "NZ")
    # frame counter -> walk table index
    a.ld_a_a16(0xC000)
    a.inc_r("A")
    a.ld_a16_a(0xC000)
    a.ld_r_r("L", "A")
    a.ld_r_d8("H", _C3_WALK_X >> 8)
    a.ld_r_r("B", "(HL)")
    a.ld_r_d8("H", _C3_WALK_Y >> 8)
    a.ld_r_r("A", "(HL)")
    a.ldh_a8_a(0x42)  # SCY
    a.ld_r_d8("A", 0x10)  # select buttons
    a.ldh_a8_a(0x00)
    a.ldh_a_a8(0x00)
    a.alu_d8("AND", 0x0F)
    a.alu_r("ADD", "B")
    a.ldh_a8_a(0x43)  # SCX = walk + button nibble
    a.label("wait_end")
    a.ldh_a_a8(0x44)
    a.alu_d8("CP", 144)
    a.jr("wait_end", "Z")
    a.jp("frame")
    code = a.resolve()
    rom[PROGRAM_ORIGIN : PROGRAM_ORIGIN + len(code)] = code
    return finalize_rom(rom, "GBXAMD C3", 0x00, 0x00, 0x00)


def cart_c4(seed: int = 3, mbc: int = 1) -> bytes:
    """512 KiB banked cart (MBC1, or MBC3 with 32 KiB RAM when ``mbc == 3``)."""
    rng = np.random.default_rng(seed)
    nbanks = 32
    rom = bytearray(nbanks * ROM_BANK)
    mbc3 = mbc == 3
    cart_type, ram_code = (0x13, 0x03) if mbc3 else (0x01, 0x00)

    # ---- bank 0: IRQ handlers + dispatcher --------------------------------
    h = Asm(origin=0x0068)  # handlers right after the vector table
    h.label("vbl")
    h.push("AF")
    h.push("HL")
    h.ld_rr_d16("HL", 0xDF00)
    h.emit(0x34)  # INC (HL)
    h.pop("HL")
    h.pop("AF")
    h.reti()
    h.label("stat")
    h.push("AF")
    h.ldh_a_a8(0x45)
    h.alu_d8("ADD", int(rng.integers(3, 40)))
    h.alu_d8("CP", 154)
    h.jr("stat_ok", "C")
    h.alu_d8("SUB", 154)
    h.label("stat_ok")
    h.ldh_a8_a(0x45)  # move LYC
    h.pop("AF")
    h.reti()
    h.label("timer")
    h.push("AF")
    h.push("HL")
    h.ld_rr_d16("HL", 0xDF01)
    h.emit(0x34)
    h.pop("HL")
    h.pop("AF")
    h.reti()
    hcode = h.resolve()
    assert 0x68 + len(hcode) <= 0x100
    rom[0x68 : 0x68 + len(hcode)] = hcode
    _vectors(rom, {0x40: h.labels["vbl"], 0x48: h.labels["stat"], 0x50: h.labels["timer"]})

    a = Asm(origin=PROGRAM_ORIGIN)
    a.ld_rr_d16("SP", 0xDFF0)
    if mbc3:
        a.ld_r_d8("A", 0x0A)
        a.ld_a16_a(0x0000)  # RAM enable
    a.ld_r_d8("A", int(rng.integers(0, 256)))
    a.ldh_a8_a(0x06)  # TMA
    a.ld_r_d8("A", 0x04 | int(rng.integers(0, 4)))
    a.ldh_a8_a(0x07)  # TAC on
    a.ld_r_d8("A", int(rng.integers(0, 154)))
    a.ldh_a8_a(0x45)  # LYC
    a.ld_r_d8("A", 0x40)
    a.ldh_a8_a(0x41)  # STAT: LYC interrupt source
    a.ld_r_d8("A", 0x07)
    a.ldh_a8_a(0xFF)  # IE = VBlank | STAT | Timer
    a.ld_r_d8("A", 0x00)
    a.ldh_a8_a(0x0F)
    a.ei()
    a.label("loop")
    a.ld_r_d8("A", 0x20)
    a.ldh_a8_a(0x00)
    a.ldh_a_a8(0x00)
    a.alu_d8("AND", 0x0F)
    a.ld_r_r("B", "A")
    a.ld_r_d8("A", 0x10)
    a.ldh_a8_a(0x00)
    a.ldh_a_a8(0x00)
    a.cb(0x37)  # SWAP A
    a.alu_r("XOR", "B")
    a.ld_a16_a(0xDF02)
    a.alu_d8("AND", 0x1F)
    a.ld_a16_a(0x2000)  # ROM bank (0 -> 1 in the MBC)
    if mbc3:
        a.ld_a_a16(0xDF02)
        a.alu_d8("AND", 0x03)
        a.ld_a16_a(0x4000)  # RAM bank
        a.ld_r_d8("A", 0x00)
        a.ld_a16_a(0x6000)
        a.ld_r_d8("A", 0x01)
        a.ld_a16_a(0x6000)  # latch RTC
        a.ld_r_d8("A", 0x08)
        a.ld_a16_a(0x4000)  # select RTC seconds
        a.ld_a_a16(0xA000)
        a.ld_a16_a(0xDF03)
        a.ld_a_a16(0xDF02)
        a.alu_d8("AND", 0x03)
        a.ld_a16_a(0x4000)  # back to the RAM bank
    a.call(0x4000)
    a.ld_a_a16(0xDF02)
    a.bit(4, "A")
    a.jr("ime_off", "NZ")
    a.ei()
    a.halt()
    a.nop()
    a.jp("loop")
    a.label("ime_off")
    a.di()
    a.halt()
    a.nop()  # IME=0 wake skips this byte
    a.ei()
    a.jp("loop")
    code = a.resolve()
    rom[PROGRAM_ORIGIN : PROGRAM_ORIGIN + len(code)] = code

    # ---- banks 1..31: balanced random subprograms ending in RET ------------
    for bank in range(1, nbanks):
        b = Asm(origin=0x4000)
        gen = CodeGen(
            rng,
            b,
            stack="balanced",
            joypad_conditions=False,
            store_lo=0xC000,
            store_hi=0xDDFF,
            cart_ram=mbc3,
            backward_prob=0.0,
        )
        size = int(rng.integers(1024, 4096))
        pool = LEGAL_NON_CB + _cb_pool()
        _emit_random_program(gen, size, pool)
        end = b.pc
        b.ret()
        for _ in range(8):
            gen.leaf()
        gen.resolve(end)
        bcode = b.resolve()
        assert len(bcode) <= ROM_BANK
        rom[bank * ROM_BANK : bank * ROM_BANK + len(bcode)] = bcode
    title = "GBXAMD C4M3" if mbc3 else "GBXAMD C4"
    return finalize_rom(rom, title, cart_type, 0x04, ram_code)


CARTS = {
    "c1": cart_c1,
    "c2": cart_c2,
    "c3": cart_c3,
    "c4": lambda seed=3: cart_c4(seed, mbc=1),
    "c4m3": lambda seed=4: cart_c4(seed, mbc=3),
    "c5": cart_c3,
}


@dataclass(frozen=True)
class Workload:
    """One benchmark/parity configuration (num envs, frameskip, steps ...)."""

    name: str
    cart: str
    cart_seed: int
    num_envs: int
    frames_per_step: int
    steps: int
    actions_seed: int
    release_after_frames: int = 8
    stage: str = "emulate_only"
    render: str | None = None  # None | "packed" | "unpacked"
    reset_prob: float = 0.0
    senses: int = 0

    def rom(self) -> bytes:
        return CARTS[self.cart](self.cart_seed)


WORKLOADS = {
    "c1": Workload("c1_cpu_parity_smoke", "c1", 0, 64, 4, 256, 0),
    "c2": Workload("c2_cpu_step_16k", "c2", 1, 16_384, 24, 1000, 1),
    "c3": Workload("c3_ppu_packed_16k", "c3", 2, 16_384, 24, 1000, 2, render="packed"),
    "c4": Workload("c4_mbc1_irq_64k", "c4", 3, 65_536, 24, 200, 3),
    "c4m3": Workload("c4_mbc3_ram_irq_64k", "c4m3", 4, 65_536, 24, 200, 4),
    "c5": Workload(
        "c5_rl_rollout_128k",
        "c5",
        2,
        131_072,
        24,
        2000,
        5,
        render="unpacked",
        reset_prob=0.01,
        senses=32,
    ),
}


def seeded_actions(seed: int, step_idx: int, num_envs: int, num_actions: int = 8) -> np.ndarray:
    """The harness's ``seeded_random`` generator (bench/harness.py:236-243)."""
    rng = np.random.default_rng(seed + step_idx)
    return rng.integers(0, num_actions, size=(num_envs,), dtype=np.int32)

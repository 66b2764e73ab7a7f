"""A small SM83 (Game Boy CPU) assembler used to author the boot stub and the
synthetic cartridges.

Encodings follow the public SM83 opcode map (Pan Docs).  Only what the cart
generators need is provided: byte emitters per instruction family, labels with
8-bit relative and 16-bit absolute fix-ups, and per-opcode metadata (length,
operand kind) used to draw random legal instructions.
"""

from __future__ import annotations

from dataclasses import dataclass, field

R8 = ("B", "C", "D", "E", "H", "L", "(HL)", "A")
R8_INDEX = {name: i for i, name in enumerate(R8)}
R16 = ("BC", "DE", "HL", "SP")
R16_STACK = ("BC", "DE", "HL", "AF")
ALU_OPS = ("ADD", "ADC", "SUB", "SBC", "AND", "XOR", "OR", "CP")
COND = ("NZ", "Z", "NC", "C")

# Unprefixed opcodes with no SM83 instruction.
ILLEGAL = frozenset({0xD3, 0xDB, 0xDD, 0xE3, 0xE4, 0xEB, 0xEC, 0xED, 0xF4, 0xFC, 0xFD})


def opcode_length(op: int) -> int:
    """Encoded length in bytes of an unprefixed opcode (CB counts as 2)."""
    if op in (0x01, 0x11, 0x21, 0x31, 0x08, 0xEA, 0xFA):
        return 3
    if op in (0xC2, 0xC3, 0xCA, 0xD2, 0xDA, 0xC4, 0xCC, 0xCD, 0xD4, 0xDC):
        return 3
    if op in (0x06, 0x0E, 0x16, 0x1E, 0x26, 0x2E, 0x36, 0x3E):
        return 2
    if op in (0x18, 0x20, 0x28, 0x30, 0x38, 0xE0, 0xF0, 0xE8, 0xF8, 0xCB, 0x10):
        return 2
    if op in (0xC6, 0xCE, 0xD6, 0xDE, 0xE6, 0xEE, 0xF6, 0xFE):
        return 2
    return 1


@dataclass
class Fixup:
    pos: int  # byte offset in the buffer to patch
    label: str
    kind: str  # "rel8" or "abs16"


@dataclass
class Asm:
    """Byte buffer with labels; ``origin`` is the CPU address of byte 0."""

    origin: int
    buf: bytearray = field(default_factory=bytearray)
    labels: dict[str, int] = field(default_factory=dict)
    fixups: list[Fixup] = field(default_factory=list)

    # -- bookkeeping -------------------------------------------------------
    @property
    def pc(self) -> int:
        return self.origin + len(self.buf)

    def label(self, name: str) -> None:
        if name in self.labels:
            raise ValueError(f"duplicate label {name}")
        self.labels[name] = self.pc

    def emit(self, *data: int) -> None:
        for b in data:
            if not 0 <= b <= 0xFF:
                raise ValueError(f"byte out of range: {b}")
        self.buf.extend(data)

    def emit16(self, value: int) -> None:
        self.emit(value & 0xFF, (value >> 8) & 0xFF)

    def _target16(self, target: int | str) -> None:
        if isinstance(target, str):
            self.fixups.append(Fixup(len(self.buf), target, "abs16"))
            self.emit16(0)
        else:
            self.emit16(target)

    def _target_rel(self, target: int | str) -> None:
        if isinstance(target, str):
            self.fixups.append(Fixup(len(self.buf), target, "rel8"))
            self.emit(0)
        else:
            off = target - (self.pc + 1)
            if not -128 <= off <= 127:
                raise ValueError(f"JR target out of range: {off}")
            self.emit(off & 0xFF)

    def resolve(self, extra: dict[str, int] | None = None) -> bytes:
        table = dict(self.labels)
        if extra:
            table.update(extra)
        for fx in self.fixups:
            addr = table[fx.label]
            if fx.kind == "abs16":
                self.buf[fx.pos] = addr & 0xFF
                self.buf[fx.pos + 1] = (addr >> 8) & 0xFF
            else:
                off = addr - (self.origin + fx.pos + 1)
                if not -128 <= off <= 127:
                    raise ValueError(f"JR to {fx.label} out of range ({off})")
                self.buf[fx.pos] = off & 0xFF
        self.fixups.clear()
        return bytes(self.buf)

    # -- loads ---------------------------------------------------------------
    def ld_r_r(self, dst: str, src: str) -> None:
        op = 0x40 | (R8_INDEX[dst] << 3) | R8_INDEX[src]
        if op == 0x76:
            raise ValueError("LD (HL),(HL) is HALT")
        self.emit(op)

    def ld_r_d8(self, dst: str, value: int) -> None:
        self.emit(0x06 | (R8_INDEX[dst] << 3), value & 0xFF)

    def ld_rr_d16(self, rr: str, value: int | str) -> None:
        self.emit(0x01 | (R16.index(rr) << 4))
        self._target16(value)

    def ld_a16_a(self, addr: int) -> None:
        self.emit(0xEA)
        self.emit16(addr)

    def ld_a_a16(self, addr: int) -> None:
        self.emit(0xFA)
        self.emit16(addr)

    def ldh_a8_a(self, a8: int) -> None:
        self.emit(0xE0, a8 & 0xFF)

    def ldh_a_a8(self, a8: int) -> None:
        self.emit(0xF0, a8 & 0xFF)

    def ld_hli_a(self) -> None:
        self.emit(0x22)

    def ld_a_hli(self) -> None:
        self.emit(0x2A)

    def ld_de_a(self) -> None:
        self.emit(0x12)

    def ld_a_de(self) -> None:
        self.emit(0x1A)

    def ld_sp_hl(self) -> None:
        self.emit(0xF9)

    # -- ALU -----------------------------------------------------------------
    def alu_r(self, op: str, src: str) -> None:
        self.emit(0x80 | (ALU_OPS.index(op) << 3) | R8_INDEX[src])

    def alu_d8(self, op: str, value: int) -> None:
        self.emit(0xC6 | (ALU_OPS.index(op) << 3), value & 0xFF)

    def inc_r(self, r: str) -> None:
        self.emit(0x04 | (R8_INDEX[r] << 3))

    def dec_r(self, r: str) -> None:
        self.emit(0x05 | (R8_INDEX[r] << 3))

    def inc_rr(self, rr: str) -> None:
        self.emit(0x03 | (R16.index(rr) << 4))

    def dec_rr(self, rr: str) -> None:
        self.emit(0x0B | (R16.index(rr) << 4))

    def add_hl_rr(self, rr: str) -> None:
        self.emit(0x09 | (R16.index(rr) << 4))

    # -- stack ---------------------------------------------------------------
    def push(self, rr: str) -> None:
        self.emit(0xC5 | (R16_STACK.index(rr) << 4))

    def pop(self, rr: str) -> None:
        self.emit(0xC1 | (R16_STACK.index(rr) << 4))

    # -- control flow ----------------------------------------------------------
    def jp(self, target: int | str, cond: str | None = None) -> None:
        self.emit(0xC3 if cond is None else 0xC2 | (COND.index(cond) << 3))
        self._target16(target)

    def jr(self, target: int | str, cond: str | None = None) -> None:
        self.emit(0x18 if cond is None else 0x20 | (COND.index(cond) << 3))
        self._target_rel(target)

    def call(self, target: int | str, cond: str | None = None) -> None:
        self.emit(0xCD if cond is None else 0xC4 | (COND.index(cond) << 3))
        self._target16(target)

    def ret(self, cond: str | None = None) -> None:
        self.emit(0xC9 if cond is None else 0xC0 | (COND.index(cond) << 3))

    def reti(self) -> None:
        self.emit(0xD9)

    def nop(self) -> None:
        self.emit(0x00)

    def di(self) -> None:
        self.emit(0xF3)

    def ei(self) -> None:
        self.emit(0xFB)

    def halt(self) -> None:
        self.emit(0x76)

    def cb(self, cb_op: int) -> None:
        self.emit(0xCB, cb_op & 0xFF)

    def bit(self, b: int, r: str) -> None:
        self.cb(0x40 | (b << 3) | R8_INDEX[r])

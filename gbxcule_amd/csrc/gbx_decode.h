// gbx_decode.h -- SM83 instruction decode into a 128-bit micro-op record.
//
// Every instruction (unprefixed opcode, or CB prefix + second byte) maps to
// one record of four 32-bit words whose fields drive the step kernel's
// straight-line datapath.  Cycle counts, lengths and operand roles follow
// the reference opcode table (src/gbxcule/core/isa_sm83.py) and the opcode
// templates under src/gbxcule/kernels/cpu_templates/ (loads.py, alu.py,
// bitops.py, jumps.py, stack.py, misc.py).
//
// Register file.  The eight 8-bit registers live in two dwords read and
// written with byte permutes: w0 = B C D E (B in bits 31-24), w1 = H L - A
// (A in bits 7-0).  "Byte index" below numbers the 8 bytes of {w1:w0} as the
// permute does: 0 E, 1 D, 2 C, 3 B, 4 A, 5 unused, 6 L, 7 H; 12 reads zero.
//
// w0  [0:7] opcode  [8:15] byte 1  [16:23] byte 2  [24:25] length
//     [26:28] cycles/4 (branch taken or unconditional)  [29:31] cycles/4 not taken
// w1  8-bit datapath
//     [0:3]   xi     byte index of the first ALU operand
//     [4]     xmem   first operand is the bus byte rd0
//     [5:8]   yi     byte index of the second operand (ysrc 0)
//     [9:11]  ysrc   second operand: 0 register yi, 1 rd0, 2 const8, 3 byte 1, 4 rd1
//     [12:13] unit   0 none, 1 adder, 2 logic, 3 shifter
//     [14]    sub    adder subtracts (second operand complemented, carry inverted)
//     [15]    usec   adder adds the carry flag (ADC, SBC)
//     [16]    mA     logic result includes x AND y
//     [17]    mX     logic result includes x XOR y (both: OR; neither: 0)
//     [18:21] ib     shifter in-bit: bit ib of (C flag << 9 | x): 7, 0, 9 or 10 (zero)
//     [22:24] shamt  shifter right shift of the 16-bit funnel: 7 left, 1 right, 4 swap
//     [25:28] cbit   shifter carry-out: bit cbit of x (8 = zero, for SWAP)
//     [29]    hi_in  funnel high byte is the in-bit (right shifts), else x
//     [30]    lo_in  funnel low byte is in-bit << 7 (left shifts), else x
//     [31]    daa    decimal adjust
// w2  [0:7]   const8 constant second operand (1, bit masks, 0xFF) or a 16-bit
//                    addend sign-extended (INC/DEC rr: 1, -1; LD SP,HL: 0)
//     [8:10]  am     bus address mode of the read/write operand (Am)
//     [12:15] K      flags kept from F (Z N H C = bits 15..12)
//     [16:17] nr     bus reads (0, 1, or 2 for POP/RET)
//     [18:19] hlinc  HL post-update: 0 none, 1 HL+1, 2 HL-1
//     [20:23] S      flags set to 1
//     [24:27] X      flags inverted after the keep mask (CCF)
//     [28:31] E      flags taken from the computed Z/H/C of the active unit
// w3  register writeback byte masks at bits 2, 10, 18, 26 (w0 bytes 0..3) and
//     3, 11, 19, 27 (w1 bytes 0..3), interleaved with:
//     [0]     wmem   the 8-bit result is written to the bus at the operand address
//     [1]     hlw    w1 takes (HL value << 16 | result), else the result in every byte
//     [4:7]   op16   stack / control micro-op (Op16)
//     [8:9]   a16    16-bit adder first operand: 0 zero, 1 source pair, 2 HL, 3 SP
//     [12:14] b16    second operand: 0 imm16, 1 sext(const8), 2 source pair, 3 sext(byte 1), 4 rd1:rd0
//     [15]    spw    SP takes the 16-bit result
//     [16]    w0p    w0 takes the 16-bit result in both halves, else the 8-bit result
//     [17]    f16    H/C come from the 16-bit adder (ADD HL,rr; SP+e8)
//     [20:21] rr     source pair: 0 BC, 1 DE, 2 HL, 3 SP (AF with af)
//     [22]    af     source pair is AF (PUSH AF)
//     [23]    spadd  16-bit flags use the SP+e8 rule (low nibble / low byte)
//     [24]    popaf  F takes rd0 & 0xF0 (POP AF)
//     [28:30] cc     branch condition: 0 always, 1 NZ, 2 Z, 3 NC, 4 C
#pragma once
#include <stdint.h>

namespace gbx {

enum Op16 : uint32_t {
  O_NONE = 0, O_PUSH, O_POP, O_STSP, O_JR, O_JP, O_JPHL, O_CALL, O_RET, O_RETI, O_RST,
  O_DI, O_EI, O_HALT, O_TRAP
};
enum Am : uint32_t { AM_NONE = 0, AM_HL, AM_BC, AM_DE, AM_A16, AM_A8, AM_C, AM_SP };
enum Unit : uint32_t { U_NONE = 0, U_ADD, U_LOGIC, U_SHIFT };
enum YSrc : uint32_t { Y_REG = 0, Y_RD0, Y_CONST, Y_IMM, Y_RD1 };
// flag bits inside a nibble: Z N H C
constexpr uint32_t FZ = 8, FN = 4, FH = 2, FC = 1, FALL = 15;
constexpr uint32_t kZeroByte = 12;  // permute selector that reads 0

struct Rec {
  uint32_t w0, w1, w2, w3;
};

// byte index of 8-bit register r in B C D E H L (HL) A order
__host__ __device__ constexpr uint32_t reg_byte(uint32_t r) {
  return r == 0 ? 3 : r == 1 ? 2 : r == 2 ? 1 : r == 3 ? 0 : r == 4 ? 7 : r == 5 ? 6 : 4;
}
// writeback mask bits in w3 for the byte index of a register
__host__ __device__ constexpr uint32_t wb_bit(uint32_t byte) {
  return byte < 4 ? 1u << (2 + 8 * byte) : 1u << (3 + 8 * (byte - 4));
}
__host__ __device__ constexpr uint32_t wb_pair(uint32_t rr) {  // BC DE HL
  return rr == 0 ? wb_bit(2) | wb_bit(3) : rr == 1 ? wb_bit(0) | wb_bit(1) : wb_bit(6) | wb_bit(7);
}

struct Dec {
  uint32_t len = 1, cyc4 = 1, cycnt4 = 0;
  uint32_t xi = kZeroByte, xmem = 0, yi = kZeroByte, ysrc = Y_REG, unit = U_NONE, sub = 0, usec = 0,
           mA = 0, mX = 0, ib = 10, shamt = 0, cbit = 8, hi_in = 0, lo_in = 0, daa = 0;
  uint32_t const8 = 0, am = AM_NONE, K = FALL, nr = 0, hlinc = 0, S = 0, X = 0, E = 0;
  uint32_t wb = 0, wmem = 0, hlw = 0, op16 = O_NONE, a16 = 0, b16 = 0, spw = 0, w0p = 0, f16 = 0,
           rr = 0, af = 0, spadd = 0, popaf = 0, cc = 0;
};

__host__ __device__ constexpr Rec pack(Dec d) {
  if (d.cycnt4 == 0) d.cycnt4 = d.cyc4;
  Rec r{};
  r.w0 = (d.len << 24) | (d.cyc4 << 26) | (d.cycnt4 << 29);
  r.w1 = d.xi | (d.xmem << 4) | (d.yi << 5) | (d.ysrc << 9) | (d.unit << 12) | (d.sub << 14) |
         (d.usec << 15) | (d.mA << 16) | (d.mX << 17) | (d.ib << 18) | (d.shamt << 22) |
         (d.cbit << 25) | (d.hi_in << 29) | (d.lo_in << 30) | (d.daa << 31);
  r.w2 = (d.const8 & 0xFFu) | (d.am << 8) | (d.K << 12) | (d.nr << 16) | (d.hlinc << 18) |
         (d.S << 20) | (d.X << 24) | (d.E << 28);
  r.w3 = d.wb | d.wmem | (d.hlw << 1) | (d.op16 << 4) | (d.a16 << 8) | (d.b16 << 12) |
         (d.spw << 15) | (d.w0p << 16) | (d.f16 << 17) | (d.rr << 20) | (d.af << 22) |
         (d.spadd << 23) | (d.popaf << 24) | (d.cc << 28);
  return r;
}

// 8-bit destination: register r (writeback mask) or the bus operand (r = 6)
__host__ __device__ constexpr void set_dst(Dec& d, uint32_t r) {
  if (r == 6) d.wmem = 1;
  else d.wb = wb_bit(reg_byte(r));
}
// second operand from register r, the bus (r = 6) or the immediate byte (r = 8)
__host__ __device__ constexpr void set_y(Dec& d, uint32_t r) {
  if (r == 6) d.ysrc = Y_RD0;
  else if (r == 8) d.ysrc = Y_IMM;
  else d.yi = reg_byte(r);
}
// first operand from register r or the bus (r = 6)
__host__ __device__ constexpr void set_x(Dec& d, uint32_t r) {
  if (r == 6) d.xmem = 1;
  else d.xi = reg_byte(r);
}

// 8-bit ALU op of opcode bits 5-3 in 0x80-0xBF / 0xC6-0xFE: ADD ADC SUB SBC AND XOR OR CP
__host__ __device__ constexpr void set_alu(Dec& d, uint32_t y) {
  d.xi = reg_byte(7);
  d.K = 0;
  if (y <= 3 || y == 7) {
    d.unit = U_ADD;
    d.sub = (y == 2 || y == 3 || y == 7) ? 1 : 0;
    d.usec = (y == 1 || y == 3) ? 1 : 0;
    d.S = d.sub ? FN : 0;
    d.E = FZ | FH | FC;
  } else {
    d.unit = U_LOGIC;
    d.mA = (y == 4 || y == 6) ? 1 : 0;
    d.mX = (y == 5 || y == 6) ? 1 : 0;
    d.S = y == 4 ? FH : 0;
    d.E = FZ;
  }
  if (y != 7) d.wb = wb_bit(reg_byte(7));
}
// shifter op sub (CB order RLC RRC RL RR SLA SRA SWAP SRL)
__host__ __device__ constexpr void set_shift(Dec& d, uint32_t sub) {
  d.unit = U_SHIFT;
  const bool left = sub == 0 || sub == 2 || sub == 4;
  if (sub == 6) {
    d.shamt = 4;
    d.cbit = 8;
  } else if (left) {
    d.shamt = 7;
    d.lo_in = 1;
    d.cbit = 7;
    d.ib = sub == 0 ? 7 : sub == 2 ? 9 : 10;
  } else {
    d.shamt = 1;
    d.hi_in = 1;
    d.cbit = 0;
    d.ib = sub == 1 ? 0 : sub == 3 ? 9 : sub == 5 ? 7 : 10;
  }
  d.K = 0;
  d.E = FZ | FC;
}

// CB-prefixed instruction (second byte cb).  bitops.py: rotates/shifts,
// BIT (flags only), RES, SET; (HL) forms read and write back the bus.
__host__ __device__ constexpr Rec decode_cb(uint32_t cb) {
  Dec d;
  const uint32_t idx = cb & 7u, grp = cb >> 6, sub = (cb >> 3) & 7u;
  d.len = 2;
  set_x(d, idx);
  if (idx == 6) {
    d.am = AM_HL;
    d.nr = 1;
    d.cyc4 = grp == 1 ? 3 : 4;
  } else {
    d.cyc4 = 2;
  }
  if (grp == 0) {
    set_shift(d, sub);
    set_dst(d, idx);
  } else {
    d.unit = U_LOGIC;
    d.ysrc = Y_CONST;
    d.mA = 1;
    if (grp == 1) {  // BIT: Z = bit clear, H = 1, C kept
      d.const8 = 1u << sub;
      d.K = FC;
      d.S = FH;
      d.E = FZ;
    } else {
      if (grp == 2) {  // RES: x AND ~bit
        d.const8 = ~(1u << sub) & 0xFFu;
      } else {  // SET: x OR bit
        d.mX = 1;
        d.const8 = 1u << sub;
      }
      set_dst(d, idx);
    }
  }
  return pack(d);
}

__host__ __device__ constexpr Rec decode_op(uint32_t op) {
  Dec d;
  const uint32_t y = (op >> 3) & 7u, z = op & 7u, p = (op >> 4) & 3u;
  if (op == 0x76u) {  // HALT
    d.op16 = O_HALT;
    return pack(d);
  }
  if (op >= 0x40u && op < 0x80u) {  // LD r,r' / LD r,(HL) / LD (HL),r
    d.unit = U_LOGIC;
    d.mX = 1;  // 0 ^ y
    set_y(d, z);
    set_dst(d, y);
    if (y == 6 || z == 6) {
      d.am = AM_HL;
      d.cyc4 = 2;
      d.nr = z == 6 ? 1 : 0;
    }
    return pack(d);
  }
  if (op >= 0x80u && op < 0xC0u) {  // ALU A,r / ALU A,(HL)
    set_alu(d, y);
    set_y(d, z);
    if (z == 6) {
      d.am = AM_HL;
      d.nr = 1;
      d.cyc4 = 2;
    }
    return pack(d);
  }
  switch (op) {
    case 0x00: return pack(d);  // NOP
    case 0xF3: d.op16 = O_DI; return pack(d);
    case 0xFB: d.op16 = O_EI; return pack(d);
    case 0x01: case 0x11: case 0x21: case 0x31:  // LD rr,d16
      d.len = 3; d.cyc4 = 3; d.a16 = 0; d.b16 = 0;
      if (p == 3) d.spw = 1;
      else if (p == 2) { d.hlw = 1; d.wb = wb_pair(2); }
      else { d.w0p = 1; d.wb = wb_pair(p); }
      return pack(d);
    case 0x03: case 0x13: case 0x23: case 0x33:  // INC rr
    case 0x0B: case 0x1B: case 0x2B: case 0x3B:  // DEC rr
      d.cyc4 = 2; d.rr = p; d.a16 = 1; d.b16 = 1; d.const8 = (op & 8u) ? 0xFFu : 1u;
      if (p == 3) d.spw = 1;
      else if (p == 2) { d.hlw = 1; d.wb = wb_pair(2); }
      else { d.w0p = 1; d.wb = wb_pair(p); }
      return pack(d);
    case 0x09: case 0x19: case 0x29: case 0x39:  // ADD HL,rr (alu.py:72-111)
      d.cyc4 = 2; d.rr = p; d.a16 = 2; d.b16 = 2; d.hlw = 1; d.wb = wb_pair(2);
      d.f16 = 1; d.K = FZ; d.E = FH | FC;
      return pack(d);
    case 0xF9:  // LD SP,HL
      d.cyc4 = 2; d.a16 = 2; d.b16 = 1; d.const8 = 0; d.spw = 1;
      return pack(d);
    case 0x02: case 0x12: case 0x22: case 0x32:  // LD (BC)/(DE)/(HL+)/(HL-),A
      d.cyc4 = 2; d.unit = U_LOGIC; d.mX = 1; set_y(d, 7); d.wmem = 1;
      d.am = op == 0x02 ? AM_BC : op == 0x12 ? AM_DE : AM_HL;
      if (op == 0x22 || op == 0x32) {
        d.hlinc = op == 0x22 ? 1 : 2; d.hlw = 1; d.wb = wb_pair(2);
      }
      return pack(d);
    case 0x0A: case 0x1A: case 0x2A: case 0x3A:  // LD A,(BC)/(DE)/(HL+)/(HL-)
      d.cyc4 = 2; d.unit = U_LOGIC; d.mX = 1; d.ysrc = Y_RD0; d.nr = 1;
      d.wb = wb_bit(reg_byte(7));
      d.am = op == 0x0A ? AM_BC : op == 0x1A ? AM_DE : AM_HL;
      if (op == 0x2A || op == 0x3A) {
        d.hlinc = op == 0x2A ? 1 : 2; d.hlw = 1; d.wb |= wb_pair(2);
      }
      return pack(d);
    case 0xEA: case 0xE0: case 0xE2:  // LD (a16),A / LDH (a8),A / LD (C),A
      d.len = op == 0xEA ? 3 : op == 0xE0 ? 2 : 1;
      d.cyc4 = op == 0xEA ? 4 : op == 0xE0 ? 3 : 2;
      d.am = op == 0xEA ? AM_A16 : op == 0xE0 ? AM_A8 : AM_C;
      d.unit = U_LOGIC; d.mX = 1; set_y(d, 7); d.wmem = 1;
      return pack(d);
    case 0xFA: case 0xF0: case 0xF2:  // LD A,(a16) / LDH A,(a8) / LD A,(C)
      d.len = op == 0xFA ? 3 : op == 0xF0 ? 2 : 1;
      d.cyc4 = op == 0xFA ? 4 : op == 0xF0 ? 3 : 2;
      d.am = op == 0xFA ? AM_A16 : op == 0xF0 ? AM_A8 : AM_C;
      d.unit = U_LOGIC; d.mX = 1; d.ysrc = Y_RD0; d.nr = 1; d.wb = wb_bit(reg_byte(7));
      return pack(d);
    case 0x36:  // LD (HL),d8
      d.len = 2; d.cyc4 = 3; d.am = AM_HL; d.unit = U_LOGIC; d.mX = 1; d.ysrc = Y_IMM; d.wmem = 1;
      return pack(d);
    case 0x06: case 0x0E: case 0x16: case 0x1E: case 0x26: case 0x2E: case 0x3E:  // LD r,d8
      d.len = 2; d.cyc4 = 2; d.unit = U_LOGIC; d.mX = 1; d.ysrc = Y_IMM; set_dst(d, y);
      return pack(d);
    case 0x04: case 0x0C: case 0x14: case 0x1C: case 0x24: case 0x2C: case 0x3C:
    case 0x05: case 0x0D: case 0x15: case 0x1D: case 0x25: case 0x2D: case 0x3D:
    case 0x34: case 0x35:  // INC/DEC r, (HL): alu.py:13-22, 208-217, 913-946
      d.unit = U_ADD; d.sub = op & 1u; d.ysrc = Y_CONST; d.const8 = 1;
      set_x(d, y); set_dst(d, y);
      d.K = FC; d.S = d.sub ? FN : 0; d.E = FZ | FH;
      if (y == 6) { d.am = AM_HL; d.nr = 1; d.cyc4 = 3; }
      return pack(d);
    case 0x07: case 0x0F: case 0x17: case 0x1F:  // RLCA RRCA RLA RRA (Z cleared)
      set_shift(d, y); set_x(d, 7); set_dst(d, 7); d.E = FC;
      return pack(d);
    case 0x27:  // DAA (alu.py:897-950): N kept, H cleared, Z and C computed
      set_x(d, 7); set_dst(d, 7); d.daa = 1; d.K = FN; d.E = FZ | FC;
      return pack(d);
    case 0x2F:  // CPL
      set_x(d, 7); set_dst(d, 7); d.unit = U_LOGIC; d.mX = 1; d.ysrc = Y_CONST; d.const8 = 0xFF;
      d.K = FZ | FC; d.S = FN | FH;
      return pack(d);
    case 0x37: d.K = FZ; d.S = FC; return pack(d);               // SCF
    case 0x3F: d.K = FZ | FC; d.X = FC; return pack(d);          // CCF
    case 0xC6: case 0xCE: case 0xD6: case 0xDE: case 0xE6: case 0xEE: case 0xF6: case 0xFE:
      d.len = 2; d.cyc4 = 2; set_alu(d, y); d.ysrc = Y_IMM;
      return pack(d);
    // control flow
    case 0x18: d.len = 2; d.cyc4 = 3; d.op16 = O_JR; return pack(d);
    case 0x20: case 0x28: case 0x30: case 0x38:
      d.len = 2; d.cyc4 = 3; d.cycnt4 = 2; d.op16 = O_JR; d.cc = (y & 3u) + 1u;
      return pack(d);
    case 0xC3: d.len = 3; d.cyc4 = 4; d.op16 = O_JP; return pack(d);
    case 0xC2: case 0xCA: case 0xD2: case 0xDA:
      d.len = 3; d.cyc4 = 4; d.cycnt4 = 3; d.op16 = O_JP; d.cc = (y & 3u) + 1u;
      return pack(d);
    case 0xE9: d.op16 = O_JPHL; return pack(d);
    case 0xCD: d.len = 3; d.cyc4 = 6; d.op16 = O_CALL; return pack(d);
    case 0xC4: case 0xCC: case 0xD4: case 0xDC:
      d.len = 3; d.cyc4 = 6; d.cycnt4 = 3; d.op16 = O_CALL; d.cc = (y & 3u) + 1u;
      return pack(d);
    case 0xC9: case 0xD9:
      d.cyc4 = 4; d.op16 = op == 0xC9 ? O_RET : O_RETI; d.am = AM_SP; d.nr = 2;
      return pack(d);
    case 0xC0: case 0xC8: case 0xD0: case 0xD8:
      d.cyc4 = 5; d.cycnt4 = 2; d.op16 = O_RET; d.am = AM_SP; d.nr = 2; d.cc = (y & 3u) + 1u;
      return pack(d);
    case 0xC7: case 0xCF: case 0xD7: case 0xDF: case 0xE7: case 0xEF: case 0xF7: case 0xFF:
      d.cyc4 = 4; d.op16 = O_RST; return pack(d);
    case 0xC5: case 0xD5: case 0xE5: case 0xF5:  // PUSH rr
      d.cyc4 = 4; d.op16 = O_PUSH; d.rr = p; d.af = p == 3 ? 1 : 0;
      return pack(d);
    case 0xC1: case 0xD1: case 0xE1: case 0xF1:  // POP rr
      d.cyc4 = 3; d.op16 = O_POP; d.am = AM_SP; d.nr = 2;
      if (p == 3) {  // POP AF: A = rd1, F = rd0 & 0xF0
        d.unit = U_LOGIC; d.mX = 1; d.ysrc = Y_RD1; d.wb = wb_bit(reg_byte(7)); d.popaf = 1;
      } else {
        d.a16 = 0; d.b16 = 4;
        if (p == 2) { d.hlw = 1; d.wb = wb_pair(2); }
        else { d.w0p = 1; d.wb = wb_pair(p); }
      }
      return pack(d);
    case 0xE8: case 0xF8:  // ADD SP,e8 / LD HL,SP+e8 (alu.py:114-177)
      d.len = 2; d.cyc4 = op == 0xE8 ? 4 : 3; d.a16 = 3; d.b16 = 3;
      if (op == 0xE8) d.spw = 1;
      else { d.hlw = 1; d.wb = wb_pair(2); }
      d.f16 = 1; d.spadd = 1; d.K = 0; d.E = FH | FC;
      return pack(d);
    case 0x08: d.len = 3; d.cyc4 = 5; d.op16 = O_STSP; return pack(d);
    case 0xCB: return Rec{};  // resolved with the second byte (decode_cb)
    default:  // STOP and the 11 unused opcodes: trap, pc frozen (misc.py:42-56)
      d.cyc4 = 0;
      d.op16 = O_TRAP;
      return pack(d);
  }
}

// Decode of the instruction whose first three bytes are op, b1, b2, with
// the instruction bytes placed in w0.
__host__ __device__ constexpr Rec decode_insn(uint32_t op, uint32_t b1, uint32_t b2) {
  Rec r = op == 0xCBu ? decode_cb(b1) : decode_op(op);
  r.w0 |= op | (b1 << 8) | (b2 << 16);
  return r;
}

}  // namespace gbx

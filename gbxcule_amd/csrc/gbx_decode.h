// gbx_decode.h -- SM83 instruction decode into a 512-bit micro-op record.
//
// Every instruction (unprefixed opcode, or CB prefix + second byte) maps to
// one record of sixteen 32-bit words that drive the step kernel's
// straight-line datapath (gbx_exec.h).  Cycle counts, lengths and operand
// roles follow the reference opcode table (src/gbxcule/core/isa_sm83.py)
// and the opcode templates under src/gbxcule/kernels/cpu_templates/
// (loads.py, alu.py, bitops.py, jumps.py, stack.py, misc.py).
//
// Nearly every word is an operand of one datapath instruction as it stands:
// a byte-permute selector, a bit-field offset, an AND/XOR mask or a pair of
// 16-bit address deltas.  Values that depend on the instruction's immediate
// bytes (imm16, 0xFF00 | a8, sign-extended e8, the JR displacement) are
// bound into the record when it is built (bind_bytes), so the datapath does
// no per-opcode selection at all.
//
// Byte permutes (V_PERM_B32): result byte k is byte sel_k of the 8-byte value
// {S0:S1} (S1 = bytes 0-3); selectors 8..11 replicate the sign bit of byte
// 1, 3, 5, 7; 12 reads 0x00; 13 reads 0xFF.  The operand spaces:
//   registers  {W1:W0}   W0 = B C D E, W1 = H L F A  (0 E, 1 D, 2 C, 3 B, 4 A, 5 F, 6 L, 7 H)
//   bus        {X1:X0}   X0 = rd0 rd1 Klo Khi, X1 = PC, SP  (0 rd0, 1 rd1, 2/3 K, 4/5 PC, 6/7 SP)
//   writeback  {U:W}     U = result, new F, v16 lo, v16 hi  (0-3 keep W byte, 4 res, 5 F, 6/7 v16)
//   write data {U:SEQ}   SEQ = pc + length  (0/1 SEQ lo/hi, 4-7 U)
//   shifter    {CW:XW}   XW = x x 0 0, CW = W1 << 19 (C flag in bit 31)
//   flag src   {T16:XW}  T16 = carry vector of the 16-bit adder
//
// w0  [0:7] opcode  [8:15] byte 1  [16:23] byte 2  [24:25] length
//     [26:28] cycles/4 (branch taken or unconditional)  [29:31] cycles/4 not taken
// w1  RAP   bus address from the registers        (operand address = RAP | RAQ result)
// w2  RAQ   bus address from {X1:K}
// w3  XYP   ALU operands x (byte 0) and y (byte 1) from the registers
// w4  XYQ   ALU operands from the bus space
// w5  ABP   16-bit adder operands A (bytes 0-1) and B (bytes 2-3) from the registers
// w6  ABQ   16-bit adder operands from the bus space
// w7  KW    [0:7] F source for kept flags (1 F, 4 rd0)  [8:9] bus reads  [12:14] immediate
//           binding (KMode)  [16:31] K, the record's 16-bit constant
// w8  SW0   writeback selector of W0
// w9  SW1   writeback selector of W1 (F always takes the new flags)
// w10 FL    [0:7] flags taken from the computed Z/H/C  [8:15] flags not forced to 0
//           [16:23] flags inverted last  [24] IME write  [25] IME value  [26] HALT
//           [27] trap  [28] LY poll or block-copy loop starts here (set by the
//           record builder)
//           [29] SP takes the 16-bit sum  [30] DAA
// w11 TN    not taken [0:4] cycles [5:6] bus writes [7:9] SP delta (signed);
//           taken the same at [16:25]
// w12 TW    [0:4] branch test bit of W1 ^ TW  [8:15] its inversion mask
//           [16:31] write-data selector (bytes 0-1: first and second written byte)
// w13 CIW   [0:4] carry-in bit of W1 ^ CIW  [5] logic OR term  [6] logic AND term
//           [8:15] subtract mask (0xFF: y complemented)  [16:31] flag-source selector
// w14 SHW   [0:15] shifter funnel selector  [16:20] funnel right shift  [24:31] adder
//           result mask (0xFF)
// w15 DW    bus write addresses: operand address + DW, per 16-bit half (wrapping);
//           for a poll-loop start (FL bit 28, a read): [0:7] the CP constant,
//           [8:9] the JR condition (0 NZ, 1 Z, 2 NC, 3 C); for a block-copy
//           loop start: [31] set
#pragma once
#include <stdint.h>

namespace gbx {

constexpr int kRecWords = 16;
struct Rec {
  uint32_t w[kRecWords];
};

// selector values
enum : uint32_t { P_E = 0, P_D = 1, P_C = 2, P_B = 3, P_A = 4, P_F = 5, P_L = 6, P_H = 7 };
enum : uint32_t { Q_RD0 = 0, Q_RD1 = 1, Q_KL = 2, Q_KH = 3, Q_PCL = 4, Q_PCH = 5, Q_SPL = 6, Q_SPH = 7 };
enum : uint32_t { U_RES = 4, U_FN = 5, U_VL = 6, U_VH = 7 };
enum : uint32_t { S_SEQL = 0, S_SEQH = 1 };
enum : uint32_t { SH_X = 0, SH_X7 = 8, SH_CF = 11 };
enum : uint32_t { FS_X = 0, FS_X7 = 8, FS_T0 = 4, FS_T1 = 5, FS_T2 = 6 };
constexpr uint32_t SEL0 = 12, SELFF = 13;
constexpr uint32_t kZero4 = 0x0C0C0C0Cu;

// flag bits of F
constexpr uint32_t FZ = 0x80, FN = 0x40, FH = 0x20, FC = 0x10, FALL = 0xF0;

// How K is bound from the instruction bytes.
enum KMode : uint32_t { KM_CONST = 0, KM_IMM8, KM_IMM16, KM_HIGH, KM_SEXT, KM_REL };
// Branch condition (bit of W1 ^ TW that decides "taken").
enum Cond : uint32_t { C_NEVER = 0, C_ALWAYS, C_NZ, C_Z, C_NC, C_C };
// Register pairs
enum Pair : uint32_t { PR_BC = 0, PR_DE, PR_HL, PR_SP, PR_AF, PR_PC, PR_K, PR_RD, PR_ZERO };

__host__ __device__ constexpr uint32_t sel4(uint32_t b0, uint32_t b1, uint32_t b2, uint32_t b3) {
  return b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
}
__host__ __device__ constexpr uint32_t set_byte(uint32_t w, uint32_t k, uint32_t v) {
  return (w & ~(0xFFu << (8 * k))) | (v << (8 * k));
}

struct Dec {
  uint32_t len = 1, cyc = 4, cycnt = 0xFF;  // T-cycles; cycnt 0xFF: same as cyc
  uint32_t rap = kZero4, raq = kZero4, nr = 0;
  uint32_t xyp = kZero4, xyq = kZero4, abp = kZero4, abq = kZero4;
  uint32_t fsrc = 1, kmode = KM_CONST, k = 0;
  uint32_t sw0 = 0x03020100u, sw1 = 0x03020000u | (U_FN << 8);
  uint32_t E = 0, M = FALL, X = 0;
  uint32_t ime_set = 0, ime_on = 0, halt = 0, trap = 0, spw = 0, daa = 0;
  uint32_t cond = C_NEVER;
  uint32_t wn = 0, dsp = 0, wn_nt = 0xFF, dsp_nt = 0xFF;  // taken/unconditional; not taken
  uint32_t wv = (SEL0 << 8) | U_RES;
  uint32_t cipos = 9, lor = 0, land = 0, subm = 0, fsel = 0x0C0Cu;
  uint32_t shsel = 0x0C0Cu, sh = 0, madd = 0;
  uint32_t dw = 0;
};

// 8-bit register r in opcode order B C D E H L (HL) A: permute byte, and
// the writeback word (0 W0, 1 W1) and byte it lives in.
__host__ __device__ constexpr uint32_t reg_sel(uint32_t r) {
  return r == 0 ? P_B : r == 1 ? P_C : r == 2 ? P_D : r == 3 ? P_E : r == 4 ? P_H : r == 5 ? P_L : P_A;
}

__host__ __device__ constexpr void wb8(Dec& d, uint32_t r, uint32_t src) {
  const uint32_t s = reg_sel(r);
  if (s < 4) d.sw0 = set_byte(d.sw0, s, src);
  else if (s == P_A) d.sw1 = set_byte(d.sw1, 0, src);
  else d.sw1 = set_byte(d.sw1, s - 4, src);  // L byte 2, H byte 3
}
// 16-bit writeback of v16 to a pair (BC DE HL SP)
__host__ __device__ constexpr void wb16(Dec& d, uint32_t p) {
  if (p == PR_BC) d.sw0 = (d.sw0 & 0x0000FFFFu) | (U_VL << 16) | (U_VH << 24);
  else if (p == PR_DE) d.sw0 = (d.sw0 & 0xFFFF0000u) | U_VL | (U_VH << 8);
  else if (p == PR_HL) d.sw1 = (d.sw1 & 0x0000FFFFu) | (U_VL << 16) | (U_VH << 24);
  else d.spw = 1;
}
// a 16-bit source placed at byte pair `at` (0: A operand / address, 2: B operand)
// of the register-space and bus-space selectors
__host__ __device__ constexpr void src16(uint32_t& p, uint32_t& q, uint32_t at, uint32_t pr) {
  uint32_t lo = SEL0, hi = SEL0, qlo = SEL0, qhi = SEL0;
  if (pr == PR_BC) { lo = P_C; hi = P_B; }
  else if (pr == PR_DE) { lo = P_E; hi = P_D; }
  else if (pr == PR_HL) { lo = P_L; hi = P_H; }
  else if (pr == PR_AF) { lo = P_F; hi = P_A; }
  else if (pr == PR_SP) { qlo = Q_SPL; qhi = Q_SPH; }
  else if (pr == PR_PC) { qlo = Q_PCL; qhi = Q_PCH; }
  else if (pr == PR_K) { qlo = Q_KL; qhi = Q_KH; }
  else if (pr == PR_RD) { qlo = Q_RD0; qhi = Q_RD1; }
  p = set_byte(set_byte(p, at, lo), at + 1, hi);
  q = set_byte(set_byte(q, at, qlo), at + 1, qhi);
}
__host__ __device__ constexpr void set_a16(Dec& d, uint32_t pr) { src16(d.abp, d.abq, 0, pr); }
__host__ __device__ constexpr void set_b16(Dec& d, uint32_t pr) { src16(d.abp, d.abq, 2, pr); }
__host__ __device__ constexpr void set_addr(Dec& d, uint32_t pr) { src16(d.rap, d.raq, 0, pr); }

// ALU operand x (byte 0) or y (byte 1) from register r (6: the bus byte rd0,
// 8: K low byte, 9: rd1)
__host__ __device__ constexpr void set_xy(Dec& d, uint32_t at, uint32_t r) {
  if (r == 6) d.xyq = set_byte(d.xyq, at, Q_RD0);
  else if (r == 8) d.xyq = set_byte(d.xyq, at, Q_KL);
  else if (r == 9) d.xyq = set_byte(d.xyq, at, Q_RD1);
  else d.xyp = set_byte(d.xyp, at, reg_sel(r));
}
__host__ __device__ constexpr void set_x(Dec& d, uint32_t r) { set_xy(d, 0, r); }
__host__ __device__ constexpr void set_y(Dec& d, uint32_t r) { set_xy(d, 1, r); }

// 8-bit destination: register r, or the bus operand (r = 6)
__host__ __device__ constexpr void set_dst(Dec& d, uint32_t r) {
  if (r == 6) d.wn = 1;
  else wb8(d, r, U_RES);
}
// register move / load / store: res = 0 + y
__host__ __device__ constexpr void set_mov(Dec& d) { d.madd = 0xFF; }

// 8-bit ALU op of opcode bits 5-3: ADD ADC SUB SBC AND XOR OR CP (alu.py)
__host__ __device__ constexpr void set_alu(Dec& d, uint32_t y) {
  set_x(d, 7);
  if (y <= 3 || y == 7) {
    const bool sub = y == 2 || y == 3 || y == 7;
    d.madd = 0xFF;
    d.subm = sub ? 0xFF : 0;
    d.cipos = (y == 1 || y == 3) ? 12 : 9;
    d.E = FZ | FH | FC;
    d.M = FZ | FH | FC;  // N forced: set (subtraction) or clear
    d.X = sub ? FN | FH | FC : 0;  // subtraction: borrows are the inverted carries
  } else {
    d.land = (y == 4 || y == 5) ? 1 : 0;
    d.lor = (y == 5 || y == 6) ? 1 : 0;
    d.E = FZ;
    d.M = FZ;
    d.X = y == 4 ? FH : 0;
  }
  if (y != 7) wb8(d, 7, U_RES);
}

// shifter op sub (CB order RLC RRC RL RR SLA SRA SWAP SRL; bitops.py): a
// 16-bit funnel (hi << 8 | lo) shifted right by 7 (left ops), 1 (right ops)
// or 4 (SWAP); the carry out is bit 7 or bit 0 of x.
__host__ __device__ constexpr void set_shift(Dec& d, uint32_t sub) {
  const bool left = sub == 0 || sub == 2 || sub == 4;
  uint32_t lo = SH_X, hi = SH_X, c = FS_X;
  if (sub == 2) lo = SH_CF;
  if (sub == 4) lo = SEL0;
  if (sub == 3) hi = SH_CF;
  if (sub == 5) hi = SH_X7;
  if (sub == 7) hi = SEL0;
  if (left) c = FS_X7;
  if (sub == 6) c = SEL0;
  d.shsel = lo | (hi << 8);
  d.sh = sub == 6 ? 4 : left ? 7 : 1;
  d.fsel = SEL0 | (c << 8);
  d.E = FZ | FC;
  d.M = FZ | FC;
}

// CB-prefixed instruction (second byte cb).  bitops.py: rotates/shifts,
// BIT (flags only), RES, SET; (HL) forms read and write back the bus.
__host__ __device__ constexpr Dec decode_cb(uint32_t cb) {
  Dec d;
  const uint32_t idx = cb & 7u, grp = cb >> 6, sub = (cb >> 3) & 7u;
  d.len = 2;
  set_x(d, idx);
  if (idx == 6) {
    set_addr(d, PR_HL);
    d.nr = 1;
    d.cyc = grp == 1 ? 12 : 16;
  } else {
    d.cyc = 8;
  }
  if (grp == 0) {
    set_shift(d, sub);
    set_dst(d, idx);
  } else {
    set_y(d, 8);
    if (grp == 1) {  // BIT: Z = bit clear, H = 1, C kept
      d.land = 1;
      d.k = 1u << sub;
      d.E = FZ;
      d.M = FZ | FC;
      d.X = FH;
    } else {
      if (grp == 2) {  // RES: x AND ~bit
        d.land = 1;
        d.k = ~(1u << sub) & 0xFFu;
      } else {  // SET: x OR bit
        d.lor = 1;
        d.k = 1u << sub;
      }
      set_dst(d, idx);
    }
  }
  return d;
}

__host__ __device__ constexpr Dec decode_op(uint32_t op) {
  Dec d;
  const uint32_t y = (op >> 3) & 7u, z = op & 7u, p = (op >> 4) & 3u;
  if (op == 0x76u) {  // HALT
    d.halt = 1;
    return d;
  }
  if (op >= 0x40u && op < 0x80u) {  // LD r,r' / LD r,(HL) / LD (HL),r
    set_mov(d);
    set_y(d, z);
    set_dst(d, y);
    if (y == 6 || z == 6) {
      set_addr(d, PR_HL);
      d.cyc = 8;
      d.nr = z == 6 ? 1 : 0;
    }
    return d;
  }
  if (op >= 0x80u && op < 0xC0u) {  // ALU A,r / ALU A,(HL)
    set_alu(d, y);
    set_y(d, z);
    if (z == 6) {
      set_addr(d, PR_HL);
      d.nr = 1;
      d.cyc = 8;
    }
    return d;
  }
  const uint32_t pair = p == 3 ? PR_SP : p;  // BC DE HL SP
  switch (op) {
    case 0x00: return d;  // NOP
    case 0xF3: d.ime_set = 1; return d;                 // DI
    case 0xFB: d.ime_set = 1; d.ime_on = 1; return d;   // EI (immediate)
    case 0x01: case 0x11: case 0x21: case 0x31:  // LD rr,d16
      d.len = 3; d.cyc = 12; d.kmode = KM_IMM16; set_b16(d, PR_K); wb16(d, pair);
      return d;
    case 0x03: case 0x13: case 0x23: case 0x33:  // INC rr
    case 0x0B: case 0x1B: case 0x2B: case 0x3B:  // DEC rr
      d.cyc = 8; set_a16(d, pair); set_b16(d, PR_K); d.k = (op & 8u) ? 0xFFFFu : 1u;
      wb16(d, pair);
      return d;
    case 0x09: case 0x19: case 0x29: case 0x39:  // ADD HL,rr (alu.py:72-111): H bit 11, C bit 15
      d.cyc = 8; set_a16(d, PR_HL); set_b16(d, pair); wb16(d, PR_HL);
      d.fsel = FS_T1 | (FS_T2 << 8); d.E = FH | FC; d.M = FZ | FH | FC;
      return d;
    case 0xF9:  // LD SP,HL
      d.cyc = 8; set_a16(d, PR_HL); d.spw = 1;
      return d;
    case 0x02: case 0x12: case 0x22: case 0x32:  // LD (BC)/(DE)/(HL+)/(HL-),A
      d.cyc = 8; set_mov(d); set_y(d, 7); d.wn = 1;
      set_addr(d, op == 0x02 ? PR_BC : op == 0x12 ? PR_DE : PR_HL);
      if (op == 0x22 || op == 0x32) {
        set_a16(d, PR_HL); set_b16(d, PR_K); d.k = op == 0x22 ? 1u : 0xFFFFu; wb16(d, PR_HL);
      }
      return d;
    case 0x0A: case 0x1A: case 0x2A: case 0x3A:  // LD A,(BC)/(DE)/(HL+)/(HL-)
      d.cyc = 8; set_mov(d); set_y(d, 6); d.nr = 1; wb8(d, 7, U_RES);
      set_addr(d, op == 0x0A ? PR_BC : op == 0x1A ? PR_DE : PR_HL);
      if (op == 0x2A || op == 0x3A) {
        set_a16(d, PR_HL); set_b16(d, PR_K); d.k = op == 0x2A ? 1u : 0xFFFFu; wb16(d, PR_HL);
      }
      return d;
    case 0xEA: case 0xE0: case 0xE2:  // LD (a16),A / LDH (a8),A / LD (C),A
    case 0xFA: case 0xF0: case 0xF2:  // LD A,(a16) / LDH A,(a8) / LD A,(C)
      d.len = (op & 0xFu) == 0xAu ? 3 : (op & 0xFu) == 0x0u ? 2 : 1;
      d.cyc = (op & 0xFu) == 0xAu ? 16 : (op & 0xFu) == 0x0u ? 12 : 8;
      if ((op & 0xFu) == 0x2u) d.rap = sel4(P_C, SELFF, SEL0, SEL0);  // 0xFF00 | C
      else { set_addr(d, PR_K); d.kmode = (op & 0xFu) == 0xAu ? KM_IMM16 : KM_HIGH; }
      set_mov(d);
      if (op < 0xF0u) { set_y(d, 7); d.wn = 1; }
      else { set_y(d, 6); d.nr = 1; wb8(d, 7, U_RES); }
      return d;
    case 0x36:  // LD (HL),d8
      d.len = 2; d.cyc = 12; set_addr(d, PR_HL); set_mov(d); set_y(d, 8); d.kmode = KM_IMM8;
      d.wn = 1;
      return d;
    case 0x06: case 0x0E: case 0x16: case 0x1E: case 0x26: case 0x2E: case 0x3E:  // LD r,d8
      d.len = 2; d.cyc = 8; set_mov(d); set_y(d, 8); d.kmode = KM_IMM8; set_dst(d, y);
      return d;
    case 0x04: case 0x0C: case 0x14: case 0x1C: case 0x24: case 0x2C: case 0x3C:
    case 0x05: case 0x0D: case 0x15: case 0x1D: case 0x25: case 0x2D: case 0x3D:
    case 0x34: case 0x35: {  // INC/DEC r, (HL): alu.py:13-22, 208-217, 913-946
      const bool dec = (op & 1u) != 0u;
      d.madd = 0xFF; d.subm = dec ? 0xFF : 0; set_y(d, 8); d.k = 1;
      set_x(d, y); set_dst(d, y);
      d.E = FZ | FH; d.M = FZ | FH | FC; d.X = dec ? FN | FH : 0;
      if (y == 6) { set_addr(d, PR_HL); d.nr = 1; d.cyc = 12; }
      return d;
    }
    case 0x07: case 0x0F: case 0x17: case 0x1F:  // RLCA RRCA RLA RRA (Z cleared)
      set_shift(d, y); set_x(d, 7); set_dst(d, 7); d.E = FC; d.M = FC;
      return d;
    case 0x27:  // DAA (alu.py:897-950): N kept, H cleared, Z and C computed
      set_x(d, 7); set_mov(d); set_dst(d, 7); d.daa = 1; d.E = FZ | FC; d.M = FZ | FN | FC;
      return d;
    case 0x2F:  // CPL: x XOR 0xFF, N and H set
      set_x(d, 7); set_y(d, 8); d.k = 0xFF; d.lor = 1; d.land = 1; set_dst(d, 7);
      d.M = FZ | FC; d.X = FN | FH;
      return d;
    case 0x37: d.M = FZ; d.X = FC; return d;          // SCF
    case 0x3F: d.M = FZ | FC; d.X = FC; return d;     // CCF
    case 0xC6: case 0xCE: case 0xD6: case 0xDE: case 0xE6: case 0xEE: case 0xF6: case 0xFE:
      d.len = 2; d.cyc = 8; set_alu(d, y); set_y(d, 8); d.kmode = KM_IMM8;
      return d;
    // control flow (jumps.py): the target is the 16-bit sum
    case 0x18: case 0x20: case 0x28: case 0x30: case 0x38:  // JR [cc],e8
      d.len = 2; d.cyc = 12; d.kmode = KM_REL; set_a16(d, PR_PC); set_b16(d, PR_K);
      if (op == 0x18) d.cond = C_ALWAYS;
      else { d.cond = C_NZ + (y & 3u); d.cycnt = 8; }
      return d;
    case 0xC3: case 0xC2: case 0xCA: case 0xD2: case 0xDA:  // JP [cc],a16
      d.len = 3; d.cyc = 16; d.kmode = KM_IMM16; set_b16(d, PR_K);
      if (op == 0xC3) d.cond = C_ALWAYS;
      else { d.cond = C_NZ + (y & 3u); d.cycnt = 12; }
      return d;
    case 0xE9:  // JP HL
      d.cond = C_ALWAYS; set_a16(d, PR_HL);
      return d;
    case 0xCD: case 0xC4: case 0xCC: case 0xD4: case 0xDC:  // CALL [cc],a16: push pc + 3
      d.len = 3; d.cyc = 24; d.kmode = KM_IMM16; set_b16(d, PR_K); set_addr(d, PR_SP);
      d.wn = 2; d.dsp = 0xFFFEu; d.wv = S_SEQH | (S_SEQL << 8); d.dw = 0xFFFEFFFFu;
      if (op == 0xCD) d.cond = C_ALWAYS;
      else { d.cond = C_NZ + (y & 3u); d.cycnt = 12; d.wn_nt = 0; d.dsp_nt = 0; }
      return d;
    case 0xC9: case 0xD9: case 0xC0: case 0xC8: case 0xD0: case 0xD8:  // RET [cc], RETI
      d.cyc = 16; set_addr(d, PR_SP); d.nr = 2; set_b16(d, PR_RD); d.dsp = 2;
      if (op == 0xC9 || op == 0xD9) d.cond = C_ALWAYS;
      else { d.cond = C_NZ + (y & 3u); d.cyc = 20; d.cycnt = 8; d.dsp_nt = 0; }
      if (op == 0xD9) { d.ime_set = 1; d.ime_on = 1; }
      return d;
    case 0xC7: case 0xCF: case 0xD7: case 0xDF: case 0xE7: case 0xEF: case 0xF7: case 0xFF:
      d.cyc = 16; d.cond = C_ALWAYS; set_b16(d, PR_K); d.k = op & 0x38u; set_addr(d, PR_SP);
      d.wn = 2; d.dsp = 0xFFFEu; d.wv = S_SEQH | (S_SEQL << 8); d.dw = 0xFFFEFFFFu;
      return d;
    case 0xC5: case 0xD5: case 0xE5: case 0xF5:  // PUSH rr (stack.py)
      d.cyc = 16; set_a16(d, p == 3 ? PR_AF : p); set_addr(d, PR_SP);
      d.wn = 2; d.dsp = 0xFFFEu; d.wv = U_VH | (U_VL << 8); d.dw = 0xFFFEFFFFu;
      return d;
    case 0xC1: case 0xD1: case 0xE1: case 0xF1:  // POP rr
      d.cyc = 12; set_addr(d, PR_SP); d.nr = 2; set_b16(d, PR_RD); d.dsp = 2;
      if (p == 3) {  // POP AF: A = rd1, F = rd0 & 0xF0
        wb8(d, 7, U_VH); d.fsrc = 4; d.M = FALL;
      } else {
        wb16(d, p);
      }
      return d;
    case 0xE8: case 0xF8:  // ADD SP,e8 / LD HL,SP+e8 (alu.py:114-177): H/C from the low byte
      d.len = 2; d.cyc = op == 0xE8 ? 16 : 12; d.kmode = KM_SEXT; set_a16(d, PR_SP);
      set_b16(d, PR_K); wb16(d, op == 0xE8 ? PR_SP : PR_HL);
      d.fsel = FS_T0 | (FS_T1 << 8); d.E = FH | FC; d.M = FH | FC;
      return d;
    case 0x08:  // LD (a16),SP
      d.len = 3; d.cyc = 20; d.kmode = KM_IMM16; set_addr(d, PR_K); set_a16(d, PR_SP);
      d.wn = 2; d.wv = U_VL | (U_VH << 8); d.dw = 0x00010000u;
      return d;
    default:  // STOP and the 11 unused opcodes: trap, pc frozen (misc.py:42-56)
      d.cyc = 0; d.trap = 1; d.cond = C_ALWAYS; set_a16(d, PR_PC);
      return d;
  }
}

// Branch-test word: bit `pos` of W1 ^ TW decides "taken".  W1 bits 8 and 9
// are F bits 0-1, always 0: bit 8 inverted reads 1 (always), bit 9 reads 0
// (never); Z is W1 bit 15 and C W1 bit 12.
__host__ __device__ constexpr uint32_t cond_word(uint32_t c) {
  return c == C_ALWAYS ? 8u | (1u << 8)
         : c == C_NZ   ? 15u | (1u << 15)
         : c == C_Z    ? 15u
         : c == C_NC   ? 12u | (1u << 12)
         : c == C_C    ? 12u
                       : 9u;
}
__host__ __device__ constexpr uint32_t tn_half(uint32_t cyc, uint32_t wn, uint32_t dsp) {
  return cyc | (wn << 5) | (((dsp & 0xFFFFu) == 0xFFFEu ? 6u : dsp) << 7);
}

__host__ __device__ constexpr Rec pack(Dec d) {
  if (d.cycnt == 0xFF) d.cycnt = d.cyc;
  if (d.wn_nt == 0xFF) d.wn_nt = d.wn;
  if (d.dsp_nt == 0xFF) d.dsp_nt = d.dsp;
  Rec r{};
  r.w[0] = (d.len << 24) | ((d.cyc >> 2) << 26) | ((d.cycnt >> 2) << 29) | d.kmode;
  r.w[1] = d.rap;
  r.w[2] = d.raq;
  r.w[3] = d.xyp;
  r.w[4] = d.xyq;
  r.w[5] = d.abp;
  r.w[6] = d.abq;
  r.w[7] = d.fsrc | (d.nr << 8) | (d.kmode << 12) | ((d.k & 0xFFFFu) << 16);
  r.w[8] = d.sw0;
  r.w[9] = d.sw1;
  r.w[10] = d.E | (d.M << 8) | (d.X << 16) | (d.ime_set << 24) | (d.ime_on << 25) |
            (d.halt << 26) | (d.trap << 27) | (d.spw << 29) | (d.daa << 30);
  // a non-jump is never "taken": its fields live in the not-taken half
  const uint32_t tk = d.cond == C_NEVER ? 0u : tn_half(d.cyc, d.wn, d.dsp);
  r.w[11] = tn_half(d.cond == C_NEVER ? d.cyc : d.cycnt, d.wn_nt, d.dsp_nt) | (tk << 16);
  r.w[12] = cond_word(d.cond) | (d.wv << 16);
  r.w[13] = d.cipos | (d.lor << 5) | (d.land << 6) | (d.subm << 8) | (d.fsel << 16);
  r.w[14] = d.shsel | (d.sh << 16) | (d.madd << 24);
  r.w[15] = d.dw;
  return r;
}

__host__ __device__ constexpr uint32_t sext8(uint32_t v) { return (uint32_t)(int32_t)(int8_t)(v & 0xFFu); }

// LY poll loop: a load of LY into A (LDH A,(44), or LD A,(FF44)), CP d8,
// and a conditional jump back to the load (JR cc with the displacement that
// lands on it, or JP cc,a16).  The record builder marks such a load (FL bit
// 28) with DW = d8 | cc << 8 | (pass cycles / 4) << 10 | JP << 14 | the JP
// target << 16; while LY stays the same every pass leaves the same A and F,
// so the step kernel may advance whole passes at once (3 instructions and
// 32, 36 or 40 cycles each) up to the next event.  A JP's target is only
// known as an address, so the kernel takes passes only when it is the pc of
// the load.  `avail` is the number of bytes readable at p; the result is the
// loop's length in bytes, 0 for no loop.
__host__ __device__ constexpr uint32_t poll_loop_len(const uint8_t* p, uint32_t avail) {
  uint32_t n = 0;  // bytes of the load
  if (avail >= 2u && p[0] == 0xF0u && p[1] == 0x44u) n = 2;
  else if (avail >= 3u && p[0] == 0xFAu && p[1] == 0x44u && p[2] == 0xFFu) n = 3;
  if (n == 0u || avail < n + 4u || p[n] != 0xFEu) return 0;
  const uint32_t j = p[n + 2];
  if ((j == 0x20u || j == 0x28u || j == 0x30u || j == 0x38u) && p[n + 3] == ((0x100u - (n + 4u)) & 0xFFu))
    return n + 4u;
  // (a JP target at or above 0x8000 is never the load's pc: records exist
  // only for ROM and the boot image, and bit 31 of DW marks a copy loop)
  if ((j == 0xC2u || j == 0xCAu || j == 0xD2u || j == 0xDAu) && avail >= n + 5u && p[n + 4] < 0x80u)
    return n + 5u;
  return 0;
}
constexpr uint32_t kPollFlag = 1u << 28;
__host__ __device__ constexpr Rec mark_poll_loop(Rec r, const uint8_t* p) {
  const uint32_t n = p[0] == 0xF0u ? 2u : 3u;
  const uint32_t j = p[n + 2];
  const bool jp = (j & 0xC0u) == 0xC0u;
  const uint32_t cc = ((j & 0x18u) >> 3);  // NZ Z NC C
  const uint32_t cyc = (n == 2u ? 12u : 16u) + 8u + (jp ? 16u : 12u);
  const uint32_t tgt = jp ? (uint32_t)p[n + 3] | ((uint32_t)p[n + 4] << 8) : 0u;
  r.w[10] |= kPollFlag;
  r.w[15] = p[n + 1] | (cc << 8) | ((cyc / 4u) << 10) | ((jp ? 1u : 0u) << 14) | (tgt << 16);
  return r;
}
// The block-copy loop LD A,(HL+); LD (DE),A; INC DE; DEC BC; LD A,B; OR C
// (or LD A,C; OR B); JR NZ back to the LD (displacement -8): its LD A,(HL+)
// carries the same FL bit, and
// bit 31 of its last word (free: the LD writes nothing) tells it from a poll
// loop.
constexpr uint32_t kCopyLoop = 1u << 31;
__host__ __device__ constexpr bool copy_loop_at(const uint8_t* p) {
  return p[0] == 0x2Au && p[1] == 0x12u && p[2] == 0x13u && p[3] == 0x0Bu &&
         ((p[4] == 0x78u && p[5] == 0xB1u) || (p[4] == 0x79u && p[5] == 0xB0u)) && p[6] == 0x20u &&
         p[7] == 0xF8u;
}
__host__ __device__ constexpr Rec mark_copy_loop(Rec r) {
  r.w[10] |= kPollFlag;
  r.w[15] = kCopyLoop;
  return r;
}

// Bind the instruction bytes op, b1, b2 into a record decoded from the
// opcode alone: the bytes go into w0, K into KW per the record's KMode.
__host__ __device__ constexpr Rec bind_bytes(Rec r, uint32_t op, uint32_t b1, uint32_t b2) {
  const uint32_t km = r.w[0] & 7u;
  uint32_t k = r.w[7] >> 16;
  if (km == KM_IMM8) k = b1;
  else if (km == KM_IMM16) k = b1 | (b2 << 8);
  else if (km == KM_HIGH) k = 0xFF00u | b1;
  else if (km == KM_SEXT) k = sext8(b1) & 0xFFFFu;
  else if (km == KM_REL) k = (2u + sext8(b1)) & 0xFFFFu;
  r.w[0] = (r.w[0] & 0xFF000000u) | op | (b1 << 8) | (b2 << 16);
  r.w[7] = (r.w[7] & 0xFFFFu) | (k << 16);
  return r;
}

// Record of an instruction from the opcode (and CB sub-opcode) alone.
__host__ __device__ constexpr Rec decode_base(uint32_t idx) {
  return pack(idx >= 256u ? decode_cb(idx - 256u) : decode_op(idx));
}

// Record of the instruction whose first three bytes are op, b1, b2.
__host__ __device__ constexpr Rec decode_insn(uint32_t op, uint32_t b1, uint32_t b2) {
  return bind_bytes(decode_base(op == 0xCBu ? 256u + b1 : op), op, b1, b2);
}

}  // namespace gbx

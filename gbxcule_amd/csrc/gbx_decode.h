// gbx_decode.h -- SM83 instruction decode into a 40-bit micro-op word.
//
// Every instruction (unprefixed opcode, or CB prefix + second byte) maps to
// one word whose fields drive the step kernel's branch-light datapath:
//
//   bits  0- 1 len      instruction length in bytes (1..3)
//   bits  2- 4 cyc4     cycles / 4 (condition taken, or unconditional)
//   bits  5- 7 cycnt4   cycles / 4 when the branch condition is false
//   bits  8-10 am       bus address mode of the read/write operand (Am)
//   bits 11-12 nr       bus reads (0, 1, or 2 for POP/RET)
//   bits 13-14 hlinc    HL post-update: 0 none, 1 HL+1, 2 HL-1
//   bits 15-18 src      8-bit source: register 0-7 (B C D E H L - A), 6 =
//                       the bus operand, 8 = immediate byte
//   bits 19-21 dst      8-bit destination register, 6 = the bus operand
//   bit  22    xa       first ALU operand is A (else it is dst)
//   bits 23-27 alu      8-bit ALU / load micro-op (Alu)
//   bits 28-30 aux      bit number (BIT/RES/SET) or branch condition
//   bits 31-35 op16     16-bit, stack, control-flow micro-op (Op16)
//   bits 36-37 rr       16-bit source pair: BC DE HL SP (AF for PUSH/POP)
//   bits 38-39 tp       16-bit target pair: BC DE HL SP (AF for POP)
//
// Cycle counts, lengths and operand roles follow the reference opcode table
// (src/gbxcule/core/isa_sm83.py) and the opcode templates under
// src/gbxcule/kernels/cpu_templates/ (loads.py, alu.py, bitops.py,
// jumps.py, stack.py, misc.py).
#pragma once
#include <stdint.h>

namespace gbx {

enum Alu : uint32_t {
  A_NONE = 0, A_MOV,
  // add/subtract family (2..8), then the logic ops (9..11)
  A_ADD, A_ADC, A_SUB, A_SBC, A_CP, A_INC, A_DEC, A_AND, A_XOR, A_OR,
  // CB rotates/shifts in CB sub-opcode order (12 + sub)
  A_RLC, A_RRC, A_RL, A_RR, A_SLA, A_SRA, A_SWAP, A_SRL,
  // accumulator rotates: RLC/RRC/RL/RR with Z forced to 0 (20 + sub)
  A_RLCA, A_RRCA, A_RLA, A_RRA,
  A_BIT, A_RES, A_SET, A_DAA, A_CPL, A_SCF, A_CCF
};
enum Op16 : uint32_t {
  O_NONE = 0, O_LDRR, O_INCRR, O_DECRR, O_ADDHL, O_MOV16, O_ADDSP, O_LDHLSP, O_STSP,
  O_PUSH, O_POP, O_JR, O_JP, O_JPHL, O_CALL, O_RET, O_RETI, O_RST, O_DI, O_EI, O_HALT,
  O_TRAP
};
enum Am : uint32_t { AM_NONE = 0, AM_HL, AM_BC, AM_DE, AM_A16, AM_A8, AM_C, AM_SP };
constexpr uint32_t R_MEM = 6, S_IMM = 8, R_A = 7;

// ALU operation of opcode bits 5-3 in 0x80-0xBF and 0xC6-0xFE
__host__ __device__ constexpr uint32_t alu_of_y(uint32_t y) {
  return y == 0 ? A_ADD : y == 1 ? A_ADC : y == 2 ? A_SUB : y == 3 ? A_SBC
       : y == 4 ? A_AND : y == 5 ? A_XOR : y == 6 ? A_OR : A_CP;
}

struct Dec {
  uint32_t len = 1, cyc4 = 1, cycnt4 = 0, am = AM_NONE, nr = 0, hlinc = 0, src = 0, dst = R_MEM,
           xa = 0, alu = A_NONE, aux = 0, op16 = O_NONE, rr = 0, tp = 0;
};

__host__ __device__ constexpr uint64_t pack_dec(Dec d) {
  if (d.cycnt4 == 0) d.cycnt4 = d.cyc4;
  return (uint64_t)d.len | ((uint64_t)d.cyc4 << 2) | ((uint64_t)d.cycnt4 << 5) |
         ((uint64_t)d.am << 8) | ((uint64_t)d.nr << 11) | ((uint64_t)d.hlinc << 13) |
         ((uint64_t)d.src << 15) | ((uint64_t)d.dst << 19) | ((uint64_t)d.xa << 22) |
         ((uint64_t)d.alu << 23) | ((uint64_t)d.aux << 28) | ((uint64_t)d.op16 << 31) |
         ((uint64_t)d.rr << 36) | ((uint64_t)d.tp << 38);
}

// CB-prefixed instruction (second byte cb).  bitops.py: rotates/shifts,
// BIT (flags only), RES, SET; (HL) forms read and write back the bus.
__host__ __device__ constexpr uint64_t decode_cb(uint32_t cb) {
  Dec d;
  const uint32_t idx = cb & 7u, grp = cb >> 6, sub = (cb >> 3) & 7u;
  d.len = 2;
  d.alu = grp == 0 ? A_RLC + sub : grp == 1 ? A_BIT : grp == 2 ? A_RES : A_SET;
  d.aux = sub;
  d.dst = idx;
  if (idx == R_MEM) {
    d.am = AM_HL;
    d.nr = 1;
    d.cyc4 = grp == 1 ? 3 : 4;
  } else {
    d.cyc4 = 2;
  }
  return pack_dec(d);
}

__host__ __device__ constexpr uint64_t decode_op(uint32_t op) {
  Dec d;
  const uint32_t y = (op >> 3) & 7u, z = op & 7u, p = (op >> 4) & 3u;
  if (op == 0x76u) {  // HALT
    d.op16 = O_HALT;
    return pack_dec(d);
  }
  if (op >= 0x40u && op < 0x80u) {  // LD r,r' / LD r,(HL) / LD (HL),r
    d.alu = A_MOV;
    d.src = z;
    d.dst = y;
    if (y == R_MEM || z == R_MEM) {
      d.am = AM_HL;
      d.cyc4 = 2;
      d.nr = z == R_MEM ? 1 : 0;
    }
    return pack_dec(d);
  }
  if (op >= 0x80u && op < 0xC0u) {  // ALU A,r / ALU A,(HL)
    d.alu = alu_of_y(y);
    d.xa = 1;
    d.dst = R_A;
    d.src = z;
    if (z == R_MEM) {
      d.am = AM_HL;
      d.nr = 1;
      d.cyc4 = 2;
    }
    return pack_dec(d);
  }
  switch (op) {
    case 0x00: return pack_dec(d);  // NOP
    case 0xF3: d.op16 = O_DI; return pack_dec(d);
    case 0xFB: d.op16 = O_EI; return pack_dec(d);
    case 0x01: case 0x11: case 0x21: case 0x31:
      d.len = 3; d.cyc4 = 3; d.op16 = O_LDRR; d.rr = p; d.tp = p; return pack_dec(d);
    case 0x03: case 0x13: case 0x23: case 0x33:
      d.cyc4 = 2; d.op16 = O_INCRR; d.rr = p; d.tp = p; return pack_dec(d);
    case 0x0B: case 0x1B: case 0x2B: case 0x3B:
      d.cyc4 = 2; d.op16 = O_DECRR; d.rr = p; d.tp = p; return pack_dec(d);
    case 0x09: case 0x19: case 0x29: case 0x39:
      d.cyc4 = 2; d.op16 = O_ADDHL; d.rr = p; d.tp = 2; return pack_dec(d);
    case 0xF9: d.cyc4 = 2; d.op16 = O_MOV16; d.rr = 2; d.tp = 3; return pack_dec(d);
    case 0x02: case 0x12: case 0x22: case 0x32:  // LD (BC)/(DE)/(HL+)/(HL-),A
      d.cyc4 = 2; d.alu = A_MOV; d.src = R_A; d.dst = R_MEM;
      d.am = op == 0x02 ? AM_BC : op == 0x12 ? AM_DE : AM_HL;
      d.hlinc = op == 0x22 ? 1 : op == 0x32 ? 2 : 0;
      return pack_dec(d);
    case 0x0A: case 0x1A: case 0x2A: case 0x3A:  // LD A,(BC)/(DE)/(HL+)/(HL-)
      d.cyc4 = 2; d.alu = A_MOV; d.src = R_MEM; d.dst = R_A; d.nr = 1;
      d.am = op == 0x0A ? AM_BC : op == 0x1A ? AM_DE : AM_HL;
      d.hlinc = op == 0x2A ? 1 : op == 0x3A ? 2 : 0;
      return pack_dec(d);
    case 0xEA: case 0xFA:  // LD (a16),A / LD A,(a16)
      d.len = 3; d.cyc4 = 4; d.alu = A_MOV; d.am = AM_A16;
      d.src = op == 0xEA ? R_A : R_MEM; d.dst = op == 0xEA ? R_MEM : R_A; d.nr = op == 0xFA;
      return pack_dec(d);
    case 0xE0: case 0xF0:  // LDH (a8),A / LDH A,(a8)
      d.len = 2; d.cyc4 = 3; d.alu = A_MOV; d.am = AM_A8;
      d.src = op == 0xE0 ? R_A : R_MEM; d.dst = op == 0xE0 ? R_MEM : R_A; d.nr = op == 0xF0;
      return pack_dec(d);
    case 0xE2: case 0xF2:  // LD (C),A / LD A,(C)
      d.cyc4 = 2; d.alu = A_MOV; d.am = AM_C;
      d.src = op == 0xE2 ? R_A : R_MEM; d.dst = op == 0xE2 ? R_MEM : R_A; d.nr = op == 0xF2;
      return pack_dec(d);
    case 0x36:  // LD (HL),d8
      d.len = 2; d.cyc4 = 3; d.alu = A_MOV; d.am = AM_HL; d.src = S_IMM; d.dst = R_MEM;
      return pack_dec(d);
    case 0x06: case 0x0E: case 0x16: case 0x1E: case 0x26: case 0x2E: case 0x3E:
      d.len = 2; d.cyc4 = 2; d.alu = A_MOV; d.src = S_IMM; d.dst = y; return pack_dec(d);
    case 0x04: case 0x0C: case 0x14: case 0x1C: case 0x24: case 0x2C: case 0x3C:
    case 0x05: case 0x0D: case 0x15: case 0x1D: case 0x25: case 0x2D: case 0x3D:
      d.alu = (op & 1u) ? A_DEC : A_INC; d.dst = y; return pack_dec(d);
    case 0x34: case 0x35:  // INC/DEC (HL)
      d.cyc4 = 3; d.alu = op == 0x34 ? A_INC : A_DEC; d.dst = R_MEM; d.am = AM_HL; d.nr = 1;
      return pack_dec(d);
    case 0x07: case 0x0F: case 0x17: case 0x1F:
      d.alu = A_RLCA + y; d.xa = 1; d.dst = R_A; return pack_dec(d);
    case 0x27: d.alu = A_DAA; d.xa = 1; d.dst = R_A; return pack_dec(d);
    case 0x2F: d.alu = A_CPL; d.xa = 1; d.dst = R_A; return pack_dec(d);
    case 0x37: d.alu = A_SCF; d.xa = 1; d.dst = R_A; return pack_dec(d);
    case 0x3F: d.alu = A_CCF; d.xa = 1; d.dst = R_A; return pack_dec(d);
    case 0xC6: case 0xCE: case 0xD6: case 0xDE: case 0xE6: case 0xEE: case 0xF6: case 0xFE:
      d.len = 2; d.cyc4 = 2; d.alu = alu_of_y(y); d.xa = 1; d.dst = R_A; d.src = S_IMM;
      return pack_dec(d);
    // control flow; aux = condition: 0 always, 1 NZ, 2 Z, 3 NC, 4 C
    case 0x18: d.len = 2; d.cyc4 = 3; d.op16 = O_JR; return pack_dec(d);
    case 0x20: case 0x28: case 0x30: case 0x38:
      d.len = 2; d.cyc4 = 3; d.cycnt4 = 2; d.op16 = O_JR; d.aux = (y & 3u) + 1u;
      return pack_dec(d);
    case 0xC3: d.len = 3; d.cyc4 = 4; d.op16 = O_JP; return pack_dec(d);
    case 0xC2: case 0xCA: case 0xD2: case 0xDA:
      d.len = 3; d.cyc4 = 4; d.cycnt4 = 3; d.op16 = O_JP; d.aux = (y & 3u) + 1u;
      return pack_dec(d);
    case 0xE9: d.op16 = O_JPHL; return pack_dec(d);
    case 0xCD: d.len = 3; d.cyc4 = 6; d.op16 = O_CALL; return pack_dec(d);
    case 0xC4: case 0xCC: case 0xD4: case 0xDC:
      d.len = 3; d.cyc4 = 6; d.cycnt4 = 3; d.op16 = O_CALL; d.aux = (y & 3u) + 1u;
      return pack_dec(d);
    case 0xC9: case 0xD9:
      d.cyc4 = 4; d.op16 = op == 0xC9 ? O_RET : O_RETI; d.am = AM_SP; d.nr = 2;
      return pack_dec(d);
    case 0xC0: case 0xC8: case 0xD0: case 0xD8:
      d.cyc4 = 5; d.cycnt4 = 2; d.op16 = O_RET; d.am = AM_SP; d.nr = 2; d.aux = (y & 3u) + 1u;
      return pack_dec(d);
    case 0xC7: case 0xCF: case 0xD7: case 0xDF: case 0xE7: case 0xEF: case 0xF7: case 0xFF:
      d.cyc4 = 4; d.op16 = O_RST; return pack_dec(d);
    case 0xC5: case 0xD5: case 0xE5: case 0xF5:
      d.cyc4 = 4; d.op16 = O_PUSH; d.rr = p; return pack_dec(d);
    case 0xC1: case 0xD1: case 0xE1: case 0xF1:
      d.cyc4 = 3; d.op16 = O_POP; d.tp = p; d.am = AM_SP; d.nr = 2; return pack_dec(d);
    case 0xE8: d.len = 2; d.cyc4 = 4; d.op16 = O_ADDSP; d.tp = 3; return pack_dec(d);
    case 0xF8: d.len = 2; d.cyc4 = 3; d.op16 = O_LDHLSP; d.tp = 2; return pack_dec(d);
    case 0x08: d.len = 3; d.cyc4 = 5; d.op16 = O_STSP; return pack_dec(d);
    case 0xCB: return 0;  // resolved with the second byte (decode_cb)
    default:  // STOP and the 11 unused opcodes: trap, pc frozen (misc.py:42-56)
      d.cyc4 = 0;
      d.op16 = O_TRAP;
      return pack_dec(d);
  }
}

// Decode of the instruction whose first two bytes are op, b1.
__host__ __device__ constexpr uint64_t decode_insn(uint32_t op, uint32_t b1) {
  return op == 0xCBu ? decode_cb(b1) : decode_op(op);
}

}  // namespace gbx

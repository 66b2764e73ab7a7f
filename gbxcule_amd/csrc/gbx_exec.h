// gbx_exec.h -- the step kernel's instruction datapath: one SM83 instruction
// from its 128-bit record (gbx_decode.h), the register file and the bus
// bytes it read, to the new register file, flags, SP, next pc, bus writes and
// cycle count.  Straight-line code: every lane of a wavefront runs the same
// instructions whatever opcode it executes.
//
// Semantics: the opcode templates of the reference
// (src/gbxcule/kernels/cpu_templates/alu.py, bitops.py, loads.py, jumps.py,
// stack.py, misc.py) as bound by core/isa_sm83.py.
#pragma once
#include "gbx_decode.h"

namespace gbx {

struct ExecIn {
  Rec rec;
  uint32_t w0, w1;     // register file: B C D E / H L - A
  uint32_t f, sp, pc;  // F (upper nibble), SP, pc of the instruction
  uint32_t ra;         // operand address (am)
  uint32_t rd0, rd1;   // bus bytes read at ra, ra + 1
};

struct ExecOut {
  uint32_t w0, w1, f, sp, npc;
  uint32_t cycles;
  uint32_t wn, wa0, wv0, wa1, wv1;  // bus writes, in order
  uint32_t ime_set, ime_on;         // DI / EI / RETI
  uint32_t halt, trap;
};

__device__ __forceinline__ uint32_t sext8(uint32_t v) { return (uint32_t)(int32_t)(int8_t)(v & 0xFFu); }

// Operand address of the bus operand (cpu_templates/loads.py address modes).
__device__ __forceinline__ uint32_t operand_address(const Rec& r, uint32_t w0, uint32_t w1,
                                                     uint32_t sp) {
  const uint32_t am = (r.w2 >> 8) & 7u;
  const uint32_t b1 = (r.w0 >> 8) & 0xFFu, imm16 = (r.w0 >> 8) & 0xFFFFu;
  uint32_t ra = sp;
  ra = am == AM_HL ? w1 >> 16 : ra;
  ra = am == AM_BC ? w0 >> 16 : ra;
  ra = am == AM_DE ? w0 & 0xFFFFu : ra;
  ra = am == AM_A16 ? imm16 : ra;
  ra = am == AM_A8 ? 0xFF00u | b1 : ra;
  ra = am == AM_C ? 0xFF00u | ((w0 >> 16) & 0xFFu) : ra;
  return ra;
}

__device__ __forceinline__ ExecOut exec_insn(const ExecIn& in) {
  const uint32_t r0 = in.rec.w0, r1 = in.rec.w1, r2 = in.rec.w2, r3 = in.rec.w3;
  const uint32_t op = r0 & 0xFFu, b1 = (r0 >> 8) & 0xFFu, imm16 = (r0 >> 8) & 0xFFFFu;
  const uint32_t fl = in.f, cin = (fl >> 4) & 1u;
  const uint32_t sp = in.sp, hl = in.w1 >> 16;
  ExecOut o{};

  // ---- 8-bit operands: byte permutes of the register file {w1:w0} ----------
  uint32_t xv = __builtin_amdgcn_perm(in.w1, in.w0, 0x0C0C0C00u | (r1 & 15u));
  xv = (r1 & 0x10u) ? in.rd0 : xv;
  const uint32_t ysrc = (r1 >> 9) & 7u;
  uint32_t yv = __builtin_amdgcn_perm(in.w1, in.w0, 0x0C0C0C00u | ((r1 >> 5) & 15u));
  yv = ysrc == Y_RD0 ? in.rd0 : yv;
  yv = ysrc == Y_CONST ? (r2 & 0xFFu) : yv;
  yv = ysrc == Y_IMM ? b1 : yv;
  yv = ysrc == Y_RD1 ? in.rd1 : yv;

  // ---- adder: ADD ADC SUB SBC CP INC DEC (alu.py) ----------------------------
  // x + (y or ~y) + carry-in; for subtraction the carry out and the half
  // carry out are the inverted borrows.
  const uint32_t sub = (r1 >> 14) & 1u;
  const uint32_t ym = yv ^ (sub * 0xFFu);
  const uint32_t ci = (((r1 >> 15) & 1u) & cin) ^ sub;
  const uint32_t s9 = xv + ym + ci;
  const uint32_t h5 = (xv & 15u) + (ym & 15u) + ci;
  // ---- logic: MOV AND OR XOR CPL RES SET BIT ----------------------------------
  const uint32_t mA = 0u - ((r1 >> 16) & 1u), mX = 0u - ((r1 >> 17) & 1u);
  const uint32_t rl = ((xv & yv) & mA) ^ ((xv ^ yv) & mX);
  // ---- shifter: RLC RRC RL RR SLA SRA SWAP SRL, RLCA RRCA RLA RRA (bitops.py) --
  // a 16-bit funnel (hi << 8 | lo) shifted right: left ops place x high and
  // the in-bit at bit 7, right ops the in-bit high and x low, SWAP x twice.
  const uint32_t inb = ((xv | (cin << 9)) >> ((r1 >> 18) & 15u)) & 1u;
  const uint32_t hi = ((r1 >> 29) & 1u) ? inb : xv;
  const uint32_t lo = ((r1 >> 30) & 1u) ? inb << 7 : xv;
  const uint32_t rs = (((hi << 8) | lo) >> ((r1 >> 22) & 7u)) & 0xFFu;
  const uint32_t cs = (xv >> ((r1 >> 25) & 15u)) & 1u;

  // unit outputs picked with masks (every arm is computed above)
  const uint32_t unit = (r1 >> 12) & 3u;
  const uint32_t madd = 0u - (uint32_t)(unit == U_ADD), msh = 0u - (uint32_t)(unit == U_SHIFT);
  const uint32_t radd = s9 & 0xFFu, hadd = ((h5 >> 4) ^ sub) & 1u, cadd = ((s9 >> 8) ^ sub) & 1u;
  uint32_t res = (radd & madd) | (rs & msh) | (rl & ~(madd | msh));
  uint32_t hcomp = hadd & madd;
  uint32_t ccomp = (cadd & madd) | (cs & msh);
  if (r1 >> 31) {  // DAA (alu.py:897-950)
    const uint32_t nf = (fl >> 6) & 1u, hf = (fl >> 5) & 1u;
    const bool dlo = nf ? hf != 0u : (hf != 0u || (xv & 15u) > 9u);
    const bool dhi = nf ? cin != 0u : (cin != 0u || xv > 0x99u);
    const uint32_t adj = (dlo ? 0x06u : 0u) | (dhi ? 0x60u : 0u);
    res = (nf ? xv - adj : xv + adj) & 0xFFu;
    hcomp = 0;
    ccomp = dhi ? 1u : 0u;
  }

  // ---- 16-bit adder: LD rr,d16, INC/DEC rr, ADD HL,rr, LD SP,HL, ADD SP,e8,
  // LD HL,SP+e8, POP rr ------------------------------------------------------------
  const uint32_t rr = (r3 >> 20) & 3u;
  const uint32_t rsel = rr == 0u ? 0x0C0C0302u : rr == 1u ? 0x0C0C0100u
                        : rr == 2u ? 0x0C0C0706u : 0x0C0C040Cu;
  uint32_t rrv = __builtin_amdgcn_perm(in.w1, in.w0, rsel);
  // pair 3 is AF (record bit 22: A from the perm, F or'ed in) or SP
  const uint32_t maf = 0u - ((r3 >> 22) & 1u);
  const uint32_t msp = (0u - (uint32_t)(rr == 3u)) & ~maf;
  rrv = (rrv & ~msp) | (sp & msp) | (fl & maf);
  const uint32_t a16 = (r3 >> 8) & 3u, b16 = (r3 >> 12) & 7u;
  uint32_t A16 = a16 == 1u ? rrv : a16 == 2u ? hl : a16 == 3u ? sp : 0u;
  const uint32_t rd16 = in.rd0 | (in.rd1 << 8);
  uint32_t B16 = imm16;
  B16 = b16 == 1u ? sext8(r2) : B16;
  B16 = b16 == 2u ? rrv : B16;
  B16 = b16 == 3u ? sext8(b1) : B16;
  B16 = b16 == 4u ? rd16 : B16;
  const uint32_t v16 = (A16 + B16) & 0xFFFFu;
  if ((r3 >> 17) & 1u) {  // ADD HL,rr: H from bit 11, C from bit 15; SP+e8: low nibble/byte
    const bool spadd = (r3 >> 23) & 1u;
    const uint32_t hm = spadd ? 0xFu : 0xFFFu, cm = spadd ? 0xFFu : 0xFFFFu;
    const uint32_t bb = spadd ? b1 : B16;
    hcomp = ((A16 & hm) + (bb & hm)) > hm ? 1u : 0u;
    ccomp = ((A16 & cm) + (bb & cm)) > cm ? 1u : 0u;
  }

  // ---- flags: kept, inverted, set, computed (Z/H/C) ---------------------------
  const uint32_t fw = ((res == 0u ? 1u : 0u) << 7) | (hcomp << 5) | (ccomp << 4);
  uint32_t fn = ((fl & ((r2 >> 8) & 0xF0u)) ^ ((r2 >> 20) & 0xF0u)) | ((r2 >> 16) & 0xF0u) |
                (fw & ((r2 >> 24) & 0xF0u));
  fn = ((r3 >> 24) & 1u) ? in.rd0 & 0xF0u : fn;  // POP AF
  o.f = fn;

  // ---- register writeback: byte permutes with the record's byte masks -------
  const uint32_t hlinc = (r2 >> 18) & 3u;
  const uint32_t hlv = hlinc ? ((hlinc == 1u ? in.ra + 1u : in.ra - 1u) & 0xFFFFu) : v16;
  const uint32_t u8r = res * 0x01010101u;
  const uint32_t u0 = ((r3 >> 16) & 1u) ? v16 | (v16 << 16) : u8r;
  const uint32_t u1 = ((r3 >> 1) & 1u) ? (hlv << 16) | res : u8r;
  o.w0 = __builtin_amdgcn_perm(u0, in.w0, 0x03020100u | (r3 & 0x04040404u));
  o.w1 = __builtin_amdgcn_perm(u1, in.w1, 0x03020100u | ((r3 >> 1) & 0x04040404u));

  // ---- control flow, stack, interrupt enable (jumps.py, stack.py, misc.py) ---
  const uint32_t op16 = (r3 >> 4) & 15u, cc = (r3 >> 28) & 7u;
  const uint32_t cbit = cc <= 2u ? (fl >> 7) & 1u : (fl >> 4) & 1u;
  const bool is_jump = op16 - O_JR <= (uint32_t)(O_RST - O_JR);
  const bool taken = (!is_jump) | (cc == 0u) | (cbit == (uint32_t)((cc & 1u) == 0u));
  const uint32_t seq = (in.pc + ((r0 >> 24) & 3u)) & 0xFFFFu;
  uint32_t target = imm16;  // JP, CALL
  target = op16 == O_JR ? (in.pc + 2u + sext8(b1)) & 0xFFFFu : target;
  target = op16 == O_JPHL ? hl : target;
  target = ((op16 == O_RET) | (op16 == O_RETI)) ? rd16 : target;
  target = op16 == O_RST ? op & 0x38u : target;
  const bool trap = op16 == O_TRAP;
  uint32_t npc = (is_jump & taken) ? target : seq;
  o.npc = trap ? in.pc : npc;
  o.cycles = (taken ? (r0 >> 26) & 7u : r0 >> 29) << 2;

  const bool push = (op16 == O_PUSH) | (((op16 == O_CALL) | (op16 == O_RST)) & taken);
  const uint32_t pushv = op16 == O_PUSH ? rrv : seq;
  const bool stsp = op16 == O_STSP;
  // bus writes as selects: an 8-bit result to the operand, or two bytes
  // (PUSH / CALL / RST / LD (a16),SP)
  const bool w16 = push | stsp;
  const uint32_t wa0_16 = stsp ? imm16 : (sp - 1u) & 0xFFFFu;
  const uint32_t wv0_16 = stsp ? sp & 0xFFu : pushv >> 8;
  o.wn = w16 ? 2u : (r3 & 1u);
  o.wa0 = w16 ? wa0_16 : in.ra;
  o.wv0 = w16 ? wv0_16 : res;
  o.wa1 = stsp ? (imm16 + 1u) & 0xFFFFu : (sp - 2u) & 0xFFFFu;
  o.wv1 = stsp ? (sp >> 8) & 0xFFu : pushv & 0xFFu;
  uint32_t nsp = sp;
  nsp = push ? (sp - 2u) & 0xFFFFu : nsp;
  const uint32_t sp_inc = (sp + 2u) & 0xFFFFu;
  nsp = ((op16 == O_POP) | (((op16 == O_RET) | (op16 == O_RETI)) & taken)) ? sp_inc : nsp;
  nsp = ((r3 >> 15) & 1u) ? v16 : nsp;
  o.sp = nsp;
  o.ime_on = ((op16 == O_EI) | (op16 == O_RETI)) ? 1u : 0u;
  o.ime_set = (o.ime_on | (uint32_t)(op16 == O_DI));
  o.halt = op16 == O_HALT ? 1u : 0u;
  o.trap = trap ? 1u : 0u;
  return o;
}

}  // namespace gbx

// gbx_exec.h -- the step kernel's instruction datapath: one SM83 instruction
// from its 512-bit record (gbx_decode.h), the register file and the bus
// bytes it read, to the new register file, SP, next pc, bus writes and cycle
// count.  Straight-line code: every lane of a wavefront runs the same
// instructions whatever opcode it executes, and the record supplies each
// instruction's operand selectors and masks, so nothing here compares an
// opcode field.
//
// Semantics: the opcode templates of the reference
// (src/gbxcule/kernels/cpu_templates/alu.py, bitops.py, loads.py, jumps.py,
// stack.py, misc.py) as bound by core/isa_sm83.py.
#pragma once
#include "gbx_decode.h"

namespace gbx {

#ifndef GBX_EXEC_HOST_OPS
typedef unsigned short gbx_u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t perm(uint32_t s0, uint32_t s1, uint32_t sel) {
  return __builtin_amdgcn_perm(s0, s1, sel);
}
__device__ __forceinline__ uint32_t ubfe(uint32_t v, uint32_t off, uint32_t width) {
  return __builtin_amdgcn_ubfe(v, off, width);
}
__device__ __forceinline__ uint32_t sbfe(uint32_t v, uint32_t off, uint32_t width) {
  return (uint32_t)__builtin_amdgcn_sbfe((int)v, off, width);
}
// 0 or ~0 from bit `pos` of w.  Kept opaque so that the compiler ANDs with
// it rather than turning it back into a compare and a select.
template <int pos>
__device__ __forceinline__ uint32_t bit_mask(uint32_t w) {
  uint32_t r;
  asm("v_bfe_i32 %0, %1, %2, 1" : "=v"(r) : "v"(w), "i"(pos));
  return r;
}
// per-16-bit-half add, each half wrapping
__device__ __forceinline__ uint32_t add_u16x2(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(gbx_u16x2, a) + __builtin_bit_cast(gbx_u16x2, b));
}
#endif

struct ExecIn {
  uint32_t w0, w1;     // register file: B C D E / H L F A
  uint32_t x1;         // SP << 16 | pc of the instruction
  uint32_t ra;         // operand address
  uint32_t rd0, rd1;   // bus bytes read at ra, ra + 1
};

struct ExecOut {
  uint32_t w0, w1, sp, npc;
  uint32_t cycles;
  uint32_t wn, wa0, wv0, wa1, wv1;  // bus writes, in order
  uint32_t misc;                    // [0] IME write [1] IME value [2] HALT [3] trap [4] poll/copy loop
};

// Operand address of the bus operand (cpu_templates/loads.py address modes):
// a register pair, 0xFF00 | C, SP, or the bound immediate (a16, 0xFF00 | a8).
__device__ __forceinline__ uint32_t operand_address(const Rec& r, uint32_t w0, uint32_t w1, uint32_t x1) {
  return perm(w1, w0, r.w[1]) | perm(x1, r.w[7], r.w[2]);
}

__device__ __forceinline__ ExecOut exec_insn(const Rec& r, const ExecIn& in) {
  const uint32_t R0 = r.w[0], KW = r.w[7], FL = r.w[10], TN = r.w[11], TW = r.w[12];
  const uint32_t CIW = r.w[13], SHW = r.w[14];
  const uint32_t W0 = in.w0, W1 = in.w1, X1 = in.x1;
  const uint32_t X0 = perm(KW, in.rd0 | (in.rd1 << 8), 0x07060100u);  // rd0 rd1 Klo Khi
  ExecOut o{};

  // ---- 8-bit operands: x in byte 0, y in byte 1 ------------------------------
  const uint32_t XY = perm(W1, W0, r.w[3]) | perm(X1, X0, r.w[4]);
  const uint32_t x = XY & 0xFFu;
  const uint32_t ym = ubfe(XY ^ CIW, 8, 8);  // y, complemented for subtraction
  // ---- adder: ADD ADC SUB SBC CP INC DEC and moves (alu.py) ------------------
  // x + (y or ~y) + carry-in; the carry-in is bit `pos` of W1 ^ CIW: F bit 0
  // (always 0) xor the subtract mask, or the C flag (ADC) / its inverse (SBC).
  const uint32_t ci = ubfe(W1 ^ CIW, CIW & 31u, 1);
  const uint32_t s9 = x + ym + ci;
  // ---- logic: AND OR XOR (and CPL, BIT, RES, SET) ------------------------------
  const uint32_t rl = ((x | ym) & bit_mask<5>(CIW)) ^ (x & ym & bit_mask<6>(CIW));
  // ---- shifter: a 16-bit funnel of two selected bytes shifted right (bitops.py)
  const uint32_t XW = x | (x << 8);
  const uint32_t V = perm(W1 << 19, XW, SHW);
  const uint32_t rs = ubfe(V, (SHW >> 16) & 31u, 8);
  uint32_t res = (s9 & (SHW >> 24)) | rs | rl;

  // ---- 16-bit adder: A in bits 0-15, B in bits 16-31 of AB ----------------------
  // (LD rr,d16, INC/DEC rr, ADD HL,rr, SP+e8, POP, PUSH, HL+/-, jump targets)
  const uint32_t AB = perm(W1, W0, r.w[5]) | perm(X1, X0, r.w[6]);
  const uint32_t A16 = AB & 0xFFFFu, B16 = AB >> 16;
  const uint32_t sum = A16 + B16;
  const uint32_t v16 = sum & 0xFFFFu;

  // ---- flags --------------------------------------------------------------------
  // Carry vectors (bit k = carry into bit k) of both adders; the record's
  // flag-source selector moves the 16-bit adder's H/C carries, or the
  // shifter's carry-out, to bits 4 and 8, where the 8-bit adder has them.
  const uint32_t t8 = s9 ^ x ^ ym;
  const uint32_t t16 = sum ^ A16 ^ B16;
  const uint32_t fsv = t8 | perm(t16, XW, CIW >> 16);
  uint32_t cf = ubfe(fsv, 8, 1);
  if (__builtin_expect((FL & (1u << 30)) != 0u, 0)) {  // DAA (alu.py:897-950)
    const uint32_t nf = (W1 >> 14) & 1u, hf = (W1 >> 13) & 1u, cin = (W1 >> 12) & 1u;
    const bool dlo = nf ? hf != 0u : (hf != 0u || (x & 15u) > 9u);
    const bool dhi = nf ? cin != 0u : (cin != 0u || x > 0x99u);
    const uint32_t adj = (dlo ? 0x06u : 0u) | (dhi ? 0x60u : 0u);
    res = (nf ? x - adj : x + adj) & 0xFFu;
    cf = dhi ? 1u : 0u;
  }
  const uint32_t fw = (res == 0u ? 0x80u : 0u) | (ubfe(fsv, 4, 1) << 5) | (cf << 4);
  // kept flags come from F, or from rd0 (POP AF)
  const uint32_t fsrc = perm(X0, W1, KW);
  const uint32_t fn = (((fw & FL) | (fsrc & ~FL)) & ubfe(FL, 8, 8)) ^ ubfe(FL, 16, 8);

  // ---- register writeback: byte permutes of {result, F, v16} and the old words
  const uint32_t U = (sum << 16) | (fn << 8) | res;
  o.w0 = perm(U, W0, r.w[8]);
  o.w1 = perm(U, W1, r.w[9]);

  // ---- control flow, stack (jumps.py, stack.py) --------------------------------
  // "taken" is bit `pos` of W1 ^ TW: a flag, its inverse, 1 (unconditional)
  // or 0 (not a jump); it picks the cycle count, bus writes and SP delta.
  const uint32_t taken = ubfe(W1 ^ TW, TW & 31u, 1);
  const uint32_t sel = TN >> (taken << 4);
  o.cycles = sel & 31u;
  o.wn = ubfe(sel, 5, 2);
  const uint32_t dsp = sbfe(sel, 7, 3);
  const uint32_t seq = ((X1 & 0xFFFFu) + ubfe(R0, 24, 2)) & 0xFFFFu;
  o.npc = taken ? v16 : seq;
  const uint32_t mspw = bit_mask<29>(FL);
  o.sp = (v16 & mspw) | (((X1 >> 16) + dsp) & 0xFFFFu & ~mspw);

  // ---- bus writes: the result to the operand, or two bytes (PUSH, CALL, RST,
  // LD (a16),SP) at operand address + the record's deltas -------------------
  const uint32_t WA = add_u16x2(in.ra | (in.ra << 16), r.w[15]);
  o.wa0 = WA & 0xFFFFu;
  o.wa1 = WA >> 16;
  const uint32_t WV = perm(U, seq, TW >> 16);
  o.wv0 = WV & 0xFFu;
  o.wv1 = ubfe(WV, 8, 8);
  o.misc = ubfe(FL, 24, 5);
  return o;
}

}  // namespace gbx

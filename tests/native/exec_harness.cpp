// Host build of the step kernel's instruction decode (gbx_decode.h) and
// datapath (gbx_exec.h) for CPU tests.  The datapath's byte permute is the
// gfx9 V_PERM_B32 operation, written out here from its ISA definition:
// result byte k = byte sel_k of the 8-byte value {S0:S1} (S1 = bytes 0-3),
// with selector 12 giving 0x00 and 13-15 giving 0xFF.
#include <stdint.h>

#define __host__
#define __device__
#define __forceinline__ inline

static inline uint32_t perm_b32(uint32_t s0, uint32_t s1, uint32_t sel) {
  const uint64_t v = ((uint64_t)s0 << 32) | s1;
  uint32_t r = 0;
  for (int k = 0; k < 4; ++k) {
    const uint32_t s = (sel >> (8 * k)) & 0xFFu;
    uint32_t b = 0;
    if (s < 8) b = (uint32_t)(v >> (8 * s)) & 0xFFu;
    else if (s == 12) b = 0u;
    else if (s >= 13) b = 0xFFu;
    else b = ((v >> (16 * (s - 8) + 15)) & 1u) ? 0xFFu : 0u;  // sign of byte 1, 3, 5, 7
    r |= b << (8 * k);
  }
  return r;
}
#define __builtin_amdgcn_perm perm_b32

#include "../../gbxcule_amd/csrc/gbx_exec.h"

extern "C" {

// out: 4 words of the record for the instruction bytes op, b1, b2
void harness_decode(uint32_t op, uint32_t b1, uint32_t b2, uint32_t* out) {
  const gbx::Rec r = gbx::decode_insn(op, b1, b2);
  out[0] = r.w0;
  out[1] = r.w1;
  out[2] = r.w2;
  out[3] = r.w3;
}

// in: rec[4], w0, w1, f, sp, pc, rd0, rd1 (11 words); the operand address is
// computed here.  out: ra, w0, w1, f, sp, npc, cycles, wn, wa0, wv0, wa1, wv1,
// ime_set, ime_on, halt, trap (16 words).
void harness_exec(const uint32_t* in, uint32_t* out) {
  gbx::ExecIn e{};
  e.rec = gbx::Rec{in[0], in[1], in[2], in[3]};
  e.w0 = in[4];
  e.w1 = in[5];
  e.f = in[6];
  e.sp = in[7];
  e.pc = in[8];
  e.rd0 = in[9];
  e.rd1 = in[10];
  e.ra = gbx::operand_address(e.rec, e.w0, e.w1, e.sp);
  const gbx::ExecOut o = gbx::exec_insn(e);
  const uint32_t v[16] = {e.ra, o.w0, o.w1, o.f, o.sp, o.npc, o.cycles, o.wn, o.wa0,
                          o.wv0, o.wa1, o.wv1, o.ime_set, o.ime_on, o.halt, o.trap};
  for (int k = 0; k < 16; ++k) out[k] = v[k];
}

}  // extern "C"

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
#define GBX_EXEC_HOST_OPS
namespace gbx {
static inline uint32_t perm(uint32_t s0, uint32_t s1, uint32_t sel) { return perm_b32(s0, s1, sel); }
// V_BFE_U32 / V_BFE_I32: offset and width from their low 5 bits
static inline uint32_t ubfe(uint32_t v, uint32_t off, uint32_t width) {
  off &= 31u;
  width &= 31u;
  return width == 0 ? 0u : (v >> off) & ((1u << width) - 1u);
}
static inline uint32_t sbfe(uint32_t v, uint32_t off, uint32_t width) {
  const uint32_t u = ubfe(v, off, width);
  width &= 31u;
  return (width != 0 && (u >> (width - 1)) & 1u) ? u | ~((1u << width) - 1u) : u;
}
template <int pos>
static inline uint32_t bit_mask(uint32_t w) { return 0u - ((w >> pos) & 1u); }
static inline uint32_t add_u16x2(uint32_t a, uint32_t b) {
  return ((a + b) & 0xFFFFu) | (((a >> 16) + (b >> 16)) << 16);
}
}  // namespace gbx

#include "../../gbxcule_amd/csrc/gbx_exec.h"

extern "C" {

// out: the 16 words of the record for the instruction bytes op, b1, b2
void harness_decode(uint32_t op, uint32_t b1, uint32_t b2, uint32_t* out) {
  const gbx::Rec r = gbx::decode_insn(op, b1, b2);
  for (int k = 0; k < gbx::kRecWords; ++k) out[k] = r.w[k];
}

// in: rec[16], w0, w1 (H L F A), sp, pc, rd0, rd1 (22 words); the operand
// address is computed here.  out: ra, w0, w1, sp, npc, cycles, wn, wa0,
// wv0, wa1, wv1, misc (12 words).
void harness_exec(const uint32_t* in, uint32_t* out) {
  gbx::Rec r{};
  for (int k = 0; k < gbx::kRecWords; ++k) r.w[k] = in[k];
  const uint32_t* v = in + gbx::kRecWords;
  gbx::ExecIn e{};
  e.w0 = v[0];
  e.w1 = v[1];
  e.x1 = (v[2] << 16) | v[3];
  e.rd0 = v[4];
  e.rd1 = v[5];
  e.ra = gbx::operand_address(r, e.w0, e.w1, e.x1);
  const gbx::ExecOut o = gbx::exec_insn(r, e);
  const uint32_t res[12] = {e.ra, o.w0, o.w1, o.sp, o.npc, o.cycles, o.wn, o.wa0,
                            o.wv0, o.wa1, o.wv1, o.misc};
  for (int k = 0; k < 12; ++k) out[k] = res[k];
}

// out: [poll-loop length in bytes (0: none), FL word, DW word] of the decoded and marked
// record at p (n bytes readable)
void harness_poll(const uint8_t* p, uint32_t n, uint32_t* out) {
  gbx::Rec r = gbx::decode_insn(p[0], p[1], p[2]);
  const uint32_t len = gbx::poll_loop_len(p, n);
  if (len) r = gbx::mark_poll_loop(r, p);
  out[0] = len;
  out[1] = r.w[10];
  out[2] = r.w[15];
}

// out: [is a block-copy loop start, FL word, DW word] of the decoded and
// marked record at p (8 bytes)
void harness_copy(const uint8_t* p, uint32_t* out) {
  gbx::Rec r = gbx::decode_insn(p[0], p[1], p[2]);
  const bool copy = gbx::copy_loop_at(p);
  if (copy) r = gbx::mark_copy_loop(r);
  out[0] = copy ? 1u : 0u;
  out[1] = r.w[10];
  out[2] = r.w[15];
}

}  // extern "C"

// gbx_step.hip -- the SM83 step kernel for gfx950: one lane per Game Boy.
//
// Semantics are those of the reference's Warp kernel cpu_step
// (src/gbxcule/kernels/cpu_step_builder.py:875-1781 with the opcode bodies of
// kernels/cpu_templates/ and the opcode table core/isa_sm83.py), bit for bit,
// including its documented quirks (EI takes effect at once, IME=0 HALT wake
// skips a byte, OAM DMA reads raw memory, JOYP recomputed only on FF00 writes,
// STAT IRQ edges evaluated at line changes, LCD toggles count as frames).
//
// The implementation is not a translation of that kernel:
//  * memory is interleaved in 64-env blocks (gbx_internal.h mem_index), so a
//    wavefront's lanes reading the same address coalesce into one segment;
//  * CPU registers, the hot IO registers (JOYP, DIV/TIMA/TMA/TAC, IF, IE,
//    LCDC, STAT, LY, LYC, WY) and the cartridge bank offsets live in VGPRs
//    for the whole launch and are written back once;
//  * every instruction goes through one fetch, one table-driven decode, one
//    read phase (<= 2 bus reads), a small per-class execute and one write
//    phase (<= 2 bus writes) shared with interrupt pushes, so a divergent
//    wavefront pays for each bus path once per instruction rather than once
//    per distinct opcode.
#include "gbx_internal.h"

namespace gbx {
namespace {

constexpr int kCyclesPerFrame = 70224;
constexpr int kCyclesPerLine = 456;
constexpr int kLinesPerFrame = 154;
constexpr int kRtcCyclesPerSecond = 4194304;

// ---------------------------------------------------------------------------
// Decode table: one 64-bit record per unprefixed opcode.
// ---------------------------------------------------------------------------
enum Cls : uint32_t {
  K_LD = 0, K_ALU, K_INCDEC, K_R16, K_ACC, K_JUMP, K_STACK, K_SPE8, K_LDA16SP,
  K_CTRL, K_CB, K_TRAP
};
enum Am : uint32_t { AM_NONE = 0, AM_HL, AM_BC, AM_DE, AM_A16, AM_A8, AM_C, AM_SP };
constexpr uint32_t SRC_MEM = 6, SRC_IMM = 8;
enum JumpKind : uint32_t { J_JR = 0, J_JP, J_JPHL, J_CALL, J_RET, J_RETI, J_RST };

// layout: cls[0:4] am[4:7] nr[7:9] len[9:11] cyc[11:16] x[16:20] y[20:24]
//         z[24:28] cyc2[28:33]
constexpr uint64_t rec(uint32_t cls, uint32_t am, uint32_t nr, uint32_t len,
                       uint32_t cyc, uint32_t x = 0, uint32_t y = 0, uint32_t z = 0,
                       uint32_t cyc2 = 0) {
  return (uint64_t)cls | ((uint64_t)am << 4) | ((uint64_t)nr << 7) |
         ((uint64_t)len << 9) | ((uint64_t)cyc << 11) | ((uint64_t)x << 16) |
         ((uint64_t)y << 20) | ((uint64_t)z << 24) | ((uint64_t)cyc2 << 28);
}

constexpr uint64_t decode_op(int op) {
  // 8-bit register file order B C D E H L (HL) A
  if (op == 0x76) return rec(K_CTRL, AM_NONE, 0, 1, 4, 3);  // HALT
  if (op >= 0x40 && op < 0x80) {
    const uint32_t dst = (op >> 3) & 7, src = op & 7;
    if (dst == 6) return rec(K_LD, AM_HL, 0, 1, 8, SRC_MEM, src);
    if (src == 6) return rec(K_LD, AM_HL, 1, 1, 8, dst, SRC_MEM);
    return rec(K_LD, AM_NONE, 0, 1, 4, dst, src);
  }
  if (op >= 0x80 && op < 0xC0) {
    const uint32_t src = op & 7;
    return src == 6 ? rec(K_ALU, AM_HL, 1, 1, 8, (op >> 3) & 7, SRC_MEM)
                    : rec(K_ALU, AM_NONE, 0, 1, 4, (op >> 3) & 7, src);
  }
  switch (op) {
    case 0x00: return rec(K_CTRL, AM_NONE, 0, 1, 4, 0);
    case 0xF3: return rec(K_CTRL, AM_NONE, 0, 1, 4, 1);
    case 0xFB: return rec(K_CTRL, AM_NONE, 0, 1, 4, 2);
    case 0x01: case 0x11: case 0x21: case 0x31:
      return rec(K_R16, AM_NONE, 0, 3, 12, 0, (uint32_t)(op >> 4));
    case 0x03: case 0x13: case 0x23: case 0x33:
      return rec(K_R16, AM_NONE, 0, 1, 8, 1, (uint32_t)(op >> 4));
    case 0x0B: case 0x1B: case 0x2B: case 0x3B:
      return rec(K_R16, AM_NONE, 0, 1, 8, 2, (uint32_t)(op >> 4));
    case 0x09: case 0x19: case 0x29: case 0x39:
      return rec(K_R16, AM_NONE, 0, 1, 8, 3, (uint32_t)(op >> 4));
    case 0xF9: return rec(K_R16, AM_NONE, 0, 1, 8, 4, 0);
    case 0x02: return rec(K_LD, AM_BC, 0, 1, 8, SRC_MEM, 7);
    case 0x12: return rec(K_LD, AM_DE, 0, 1, 8, SRC_MEM, 7);
    case 0x22: return rec(K_LD, AM_HL, 0, 1, 8, SRC_MEM, 7, 1);
    case 0x32: return rec(K_LD, AM_HL, 0, 1, 8, SRC_MEM, 7, 2);
    case 0x0A: return rec(K_LD, AM_BC, 1, 1, 8, 7, SRC_MEM);
    case 0x1A: return rec(K_LD, AM_DE, 1, 1, 8, 7, SRC_MEM);
    case 0x2A: return rec(K_LD, AM_HL, 1, 1, 8, 7, SRC_MEM, 1);
    case 0x3A: return rec(K_LD, AM_HL, 1, 1, 8, 7, SRC_MEM, 2);
    case 0xEA: return rec(K_LD, AM_A16, 0, 3, 16, SRC_MEM, 7);
    case 0xFA: return rec(K_LD, AM_A16, 1, 3, 16, 7, SRC_MEM);
    case 0xE0: return rec(K_LD, AM_A8, 0, 2, 12, SRC_MEM, 7);
    case 0xF0: return rec(K_LD, AM_A8, 1, 2, 12, 7, SRC_MEM);
    case 0xE2: return rec(K_LD, AM_C, 0, 1, 8, SRC_MEM, 7);
    case 0xF2: return rec(K_LD, AM_C, 1, 1, 8, 7, SRC_MEM);
    case 0x36: return rec(K_LD, AM_HL, 0, 2, 12, SRC_MEM, SRC_IMM);
    case 0x06: case 0x0E: case 0x16: case 0x1E: case 0x26: case 0x2E: case 0x3E:
      return rec(K_LD, AM_NONE, 0, 2, 8, (uint32_t)((op >> 3) & 7), SRC_IMM);
    case 0x04: case 0x0C: case 0x14: case 0x1C: case 0x24: case 0x2C: case 0x3C:
      return rec(K_INCDEC, AM_NONE, 0, 1, 4, (uint32_t)((op >> 3) & 7), 0);
    case 0x05: case 0x0D: case 0x15: case 0x1D: case 0x25: case 0x2D: case 0x3D:
      return rec(K_INCDEC, AM_NONE, 0, 1, 4, (uint32_t)((op >> 3) & 7), 1);
    case 0x34: return rec(K_INCDEC, AM_HL, 1, 1, 12, 6, 0);
    case 0x35: return rec(K_INCDEC, AM_HL, 1, 1, 12, 6, 1);
    case 0x07: case 0x0F: case 0x17: case 0x1F: case 0x27: case 0x2F: case 0x37:
    case 0x3F:
      return rec(K_ACC, AM_NONE, 0, 1, 4, (uint32_t)((op >> 3) & 7));
    case 0xC6: case 0xCE: case 0xD6: case 0xDE: case 0xE6: case 0xEE: case 0xF6:
    case 0xFE:
      return rec(K_ALU, AM_NONE, 0, 2, 8, (uint32_t)((op >> 3) & 7), SRC_IMM);
    // control flow: y = condition (0 always, 1 NZ, 2 Z, 3 NC, 4 C)
    case 0x18: return rec(K_JUMP, AM_NONE, 0, 2, 12, J_JR, 0, 0, 12);
    case 0x20: case 0x28: case 0x30: case 0x38:
      return rec(K_JUMP, AM_NONE, 0, 2, 12, J_JR, (uint32_t)(((op >> 3) & 3) + 1), 0, 8);
    case 0xC3: return rec(K_JUMP, AM_NONE, 0, 3, 16, J_JP, 0, 0, 16);
    case 0xC2: case 0xCA: case 0xD2: case 0xDA:
      return rec(K_JUMP, AM_NONE, 0, 3, 16, J_JP, (uint32_t)(((op >> 3) & 3) + 1), 0, 12);
    case 0xE9: return rec(K_JUMP, AM_NONE, 0, 1, 4, J_JPHL, 0, 0, 4);
    case 0xCD: return rec(K_JUMP, AM_NONE, 0, 3, 24, J_CALL, 0, 0, 24);
    case 0xC4: case 0xCC: case 0xD4: case 0xDC:
      return rec(K_JUMP, AM_NONE, 0, 3, 24, J_CALL, (uint32_t)(((op >> 3) & 3) + 1), 0, 12);
    case 0xC9: return rec(K_JUMP, AM_SP, 2, 1, 16, J_RET, 0, 0, 16);
    case 0xD9: return rec(K_JUMP, AM_SP, 2, 1, 16, J_RETI, 0, 0, 16);
    case 0xC0: case 0xC8: case 0xD0: case 0xD8:
      return rec(K_JUMP, AM_SP, 2, 1, 20, J_RET, (uint32_t)(((op >> 3) & 3) + 1), 0, 8);
    case 0xC7: case 0xCF: case 0xD7: case 0xDF: case 0xE7: case 0xEF: case 0xF7:
    case 0xFF:
      return rec(K_JUMP, AM_NONE, 0, 1, 16, J_RST, 0, 0, 16);
    case 0xC5: case 0xD5: case 0xE5: case 0xF5:
      return rec(K_STACK, AM_NONE, 0, 1, 16, 0, (uint32_t)((op >> 4) & 3));
    case 0xC1: case 0xD1: case 0xE1: case 0xF1:
      return rec(K_STACK, AM_SP, 2, 1, 12, 1, (uint32_t)((op >> 4) & 3));
    case 0xE8: return rec(K_SPE8, AM_NONE, 0, 2, 16, 0);
    case 0xF8: return rec(K_SPE8, AM_NONE, 0, 2, 12, 1);
    case 0x08: return rec(K_LDA16SP, AM_NONE, 0, 3, 20);
    case 0xCB: return rec(K_CB, AM_NONE, 0, 2, 8);
    default: return rec(K_TRAP, AM_NONE, 0, 1, 0);  // STOP and the 11 holes
  }
}

struct Table {
  uint64_t e[256];
};
constexpr Table make_table() {
  Table t{};
  for (int i = 0; i < 256; ++i) t.e[i] = decode_op(i);
  return t;
}
__constant__ Table kDecode = make_table();

__device__ __forceinline__ uint32_t fld(uint64_t r, int lo, int bits) {
  return (uint32_t)(r >> lo) & ((1u << bits) - 1u);
}

// ---------------------------------------------------------------------------
// Buffer-resource access.  Every per-env array is reached through a
// wave-uniform descriptor (SGPRs) plus a per-lane 32-bit offset; constant
// addresses go into the scalar offset so no VGPR is spent per address.
// ---------------------------------------------------------------------------
using rsrc_t = __amdgpu_buffer_rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  // word3 0x00020000: untyped raw buffer on gfx9-class MI parts
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
struct Ref8 {
  rsrc_t r;
  uint32_t vo, so;
  __device__ operator uint32_t() const {
    return __builtin_amdgcn_raw_buffer_load_b8(r, (int)vo, (int)so, 0);
  }
  __device__ const Ref8& operator=(uint32_t v) const {
    __builtin_amdgcn_raw_buffer_store_b8((uint8_t)v, r, (int)vo, (int)so, 0);
    return *this;
  }
  __device__ const Ref8& operator=(const Ref8& o) const { return *this = (uint32_t)o; }
};
struct Ref32 {
  rsrc_t r;
  uint32_t vo, so;
  __device__ operator int32_t() const {
    return (int32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)vo, (int)so, 0);
  }
  __device__ const Ref32& operator=(int32_t v) const {
    __builtin_amdgcn_raw_buffer_store_b32((uint32_t)v, r, (int)vo, (int)so, 0);
    return *this;
  }
  __device__ const Ref32& operator=(const Ref32& o) const { return *this = (int32_t)o; }
};

// ---------------------------------------------------------------------------
// Per-lane machine.  Everything here is scalarized into VGPRs.
// ---------------------------------------------------------------------------
struct Lane {
  const DevState& s;
  uint32_t e;           // env index
  uint32_t lane;        // e % 64: position inside the 64-env block
  // wave-uniform descriptors of this wavefront's 64-env block
  rsrc_t rm;            // memory image (4 MiB)
  rsrc_t rcr;           // cartridge RAM
  rsrc_t rsc;           // per-env scalars
  rsrc_t rcs;           // cartridge state
  rsrc_t rrom;          // shared ROM

  // CPU
  uint32_t pc, sp, a, f, w0 /*B C D E*/, w1 /*H L - -*/;
  uint32_t ime, ime_delay, halted;
  // hot IO registers (byte values)
  uint32_t joyp, ff04, tima, tma, tac, ifr, ie, lcdc, stat, lym, lyc, wy;
  // timer
  uint32_t div, pend, delay, tprev;
  // PPU
  uint32_t scan, ly, wl, stat_prev;
  // cartridge
  uint32_t kind, boot_en;
  int rom_lo, rom_hi;   // byte offset of the 0000 / 4000 windows, -1 = open bus
  uint32_t ram_ok, ram_off;
  int rtc_field;        // 0..4 when an RTC register is mapped at A000
  int rtc_sub;
  uint32_t rtc_halt, rtc_dirty;
  // frame loop
  int frames_done, release;
  int32_t action;

  __device__ __forceinline__ Ref32 CS(int slot) const {
    if (__builtin_constant_p(slot)) return Ref32{rcs, lane << 2, (uint32_t)slot << 8};
    return Ref32{rcs, (((uint32_t)slot << kEnvBlockShift) | lane) << 2, 0};
  }
  __device__ __forceinline__ Ref32 SC(int slot) const {
    return Ref32{rsc, lane << 2, (uint32_t)slot << 8};
  }
  __device__ __forceinline__ Ref8 M(uint32_t addr) const {
    if (__builtin_constant_p(addr)) return Ref8{rm, lane, addr << kEnvBlockShift};
    return Ref8{rm, (addr << kEnvBlockShift) | lane, 0};
  }
  __device__ __forceinline__ Ref8 CR(uint32_t off) const {
    return Ref8{rcr, (off << kEnvBlockShift) | lane, 0};
  }

  // -- register file -------------------------------------------------------
  __device__ uint32_t r8(uint32_t idx) const {
    const uint32_t w = (idx & 4) ? w1 : w0;
    return (idx == 7) ? a : (w >> ((~idx & 3u) << 3)) & 0xFFu;
  }
  __device__ void set_r8(uint32_t idx, uint32_t v) {
    if (idx == 7) {
      a = v;
      return;
    }
    const uint32_t sh = (~idx & 3u) << 3;
    const uint32_t m = 0xFFu << sh;
    if (idx & 4) w1 = (w1 & ~m) | (v << sh);
    else w0 = (w0 & ~m) | (v << sh);
  }
  __device__ uint32_t hl() const { return w1 >> 16; }
  __device__ void set_hl(uint32_t v) { w1 = (w1 & 0xFFFFu) | ((v & 0xFFFFu) << 16); }
  __device__ uint32_t rr(uint32_t idx) const {
    switch (idx) {
      case 0: return w0 >> 16;
      case 1: return w0 & 0xFFFFu;
      case 2: return w1 >> 16;
      default: return sp;
    }
  }
  __device__ void set_rr(uint32_t idx, uint32_t v) {
    v &= 0xFFFFu;
    switch (idx) {
      case 0: w0 = (w0 & 0xFFFFu) | (v << 16); break;
      case 1: w0 = (w0 & 0xFFFF0000u) | v; break;
      case 2: w1 = (w1 & 0xFFFFu) | (v << 16); break;
      default: sp = v; break;
    }
  }

  // -- cartridge windows (reference read8 ROM/RAM branches, :565-656) ---------
  __device__ static int clamp_bank(int bank, int count, int mask) {
    if (count <= 0) return 0;
    if (mask >= 0) return bank & mask;
    return bank % count;
  }
  __device__ void refresh_cart() {
    const int lo_raw = CS(CS_ROM_BANK_LO);
    const int lo = lo_raw & 0x1F, hi = CS(CS_ROM_BANK_HI) & 3;
    const int mode = CS(CS_BANK_MODE) & 1;
    int b0 = (kind == MBC_MBC1 && mode) ? (hi & 3) << 5 : 0;
    int b1;
    if (kind == MBC_ROM_ONLY) {
      b1 = 1;
    } else if (kind == MBC_MBC1) {
      b1 = (hi << 5) | lo;
      if (b1 == 0) b1 = 1;
    } else {
      b1 = lo_raw & 0x7F;
      if (b1 == 0) b1 = 1;
    }
    b0 = clamp_bank(b0, s.rom_banks, s.rom_mask);
    b1 = clamp_bank(b1, s.rom_banks, s.rom_mask);
    const int64_t lim = (int64_t)s.rom_banks * 0x4000;
    rom_lo = ((int64_t)b0 * 0x4000 < lim) ? b0 * 0x4000 : -1;
    rom_hi = ((int64_t)b1 * 0x4000 < lim) ? b1 * 0x4000 : -1;
    // cart RAM window
    ram_ok = (s.ram_banks > 0 && CS(CS_RAM_ENABLE) != 0) ? 1u : 0u;
    rtc_field = -1;
    if (kind == MBC_MBC3) {
      const int sel = CS(CS_RTC_SELECT) & 0x0F;
      if (sel >= 0x08 && sel <= 0x0C) rtc_field = sel - 0x08;
    }
    int rb = 0;
    if (kind == MBC_MBC1) {
      if (mode) rb = CS(CS_RAM_BANK) & 3;
    } else if (kind == MBC_MBC3) {
      rb = CS(CS_RAM_BANK) & 3;
    }
    rb = clamp_bank(rb, s.ram_banks, -1);
    ram_off = (uint32_t)rb * 0x2000u;
  }

  // -- bus read (reference read8, cpu_step_builder.py:538-657) ----------------
  __device__ uint32_t io_read(uint32_t addr) {
    switch (addr & 0xFFu) {
      case 0x00: return joyp;
      case 0x04: return ff04;
      case 0x05: return tima;
      case 0x06: return tma;
      case 0x07: return tac;
      case 0x0F: return ifr;
      case 0x40: return lcdc;
      case 0x41: return stat;
      case 0x44: return lym;
      case 0x45: return lyc;
      case 0x4A: return wy;
      case 0xFF: return ie;
      default: return M(addr);
    }
  }
  __device__ uint32_t rom_at(int off) const {
    return __builtin_amdgcn_raw_buffer_load_b8(rrom, off, 0, 0);
  }
  __device__ uint32_t rom_byte(uint32_t addr) const {
    const int off = addr < 0x4000u ? rom_lo : rom_hi;
    return off < 0 ? 0xFFu : rom_at(off + (int)(addr & 0x3FFFu));
  }
  __device__ uint32_t read8(uint32_t addr) {
    uint32_t x = addr & 0xFFFFu;
    if (x - 0xE000u < 0x1E00u) x -= 0x2000u;
    if (x < 0x8000u) {
      if (x < 0x100u && boot_en) return s.boot[x];
      return rom_byte(x);
    }
    if (x >= 0xFF00u) return io_read(x);
    if (x - 0xA000u < 0x2000u) {
      if (!ram_ok) return 0xFFu;
      if (rtc_field >= 0) {
        const bool latched = CS(CS_RTC_LATCH) != 0;
        return (uint32_t)CS((latched ? CS_RTC_L_SECONDS : CS_RTC_SECONDS) + rtc_field) & 0xFFu;
      }
      return CR(ram_off + (x - 0xA000u));
    }
    return M(x);
  }

  // -- timer (cpu_step_builder.py:249-372) -------------------------------------
  __device__ static uint32_t div_bit(uint32_t t) {
    const uint32_t sel = t & 3u;
    return sel == 0 ? 9u : sel == 1 ? 3u : sel == 2 ? 5u : 7u;
  }
  __device__ static uint32_t timer_in(uint32_t d, uint32_t t) {
    return (t & 4u) ? (d >> div_bit(t)) & 1u : 0u;
  }
  __device__ void tima_inc() {
    const uint32_t t = tima;
    tima = (t + 1u) & 0xFFu;
    if (t == 0xFFu) {
      pend = 1;
      delay = 4;
    }
  }
  __device__ void reload_now() {
    tima = tma;
    ifr |= 0x04u;
    pend = 0;
    delay = 0;
  }
  __device__ void timer_tick(int cycles) {
    if (cycles <= 0) return;
    uint32_t d = div & 0xFFFFu;
    if (!(tac & 4u) && !pend) {
      d = (d + (uint32_t)cycles) & 0xFFFFu;  // no edges, no reload: DIV only
    } else {
      int rem = cycles;
      while (rem > 0) {
        if (pend && (int)delay <= 0) reload_now();
        int dt = rem;
        if (pend && (int)delay < dt) dt = (int)delay;
        bool edge = false;
        if (tac & 4u) {
          const int period = 1 << (div_bit(tac) + 1);
          const int edge_dt = period - (int)(d & (uint32_t)(period - 1));
          if (edge_dt < dt) dt = edge_dt;
          edge = dt == edge_dt;
        }
        d = (d + (uint32_t)dt) & 0xFFFFu;
        if (pend) delay = (uint32_t)((int)delay - dt);
        rem -= dt;
        if (edge) tima_inc();
        if (pend && (int)delay <= 0) reload_now();
      }
    }
    div = d;
    ff04 = (d >> 8) & 0xFFu;
    tprev = timer_in(d, tac);
  }

  // -- MBC3 real-time clock (cpu_step_builder.py:374-419) ----------------------
  __device__ void rtc_slow() {
    int dh = CS(CS_RTC_DAYS_HIGH);
    int sec = CS(CS_RTC_SECONDS) & 0xFF, mn = CS(CS_RTC_MINUTES) & 0x3F;
    int hr = CS(CS_RTC_HOURS) & 0x1F;
    int day = ((dh & 1) << 8) | (CS(CS_RTC_DAYS_LOW) & 0xFF);
    while (rtc_sub >= kRtcCyclesPerSecond) {
      rtc_sub -= kRtcCyclesPerSecond;
      if (++sec >= 60) {
        sec = 0;
        if (++mn >= 60) {
          mn = 0;
          if (++hr >= 24) {
            hr = 0;
            if (++day >= 512) {
              day %= 512;
              dh |= 0x80;
            }
          }
        }
      }
    }
    CS(CS_RTC_SECONDS) = sec;
    CS(CS_RTC_MINUTES) = mn;
    CS(CS_RTC_HOURS) = hr;
    CS(CS_RTC_DAYS_LOW) = day & 0xFF;
    CS(CS_RTC_DAYS_HIGH) = (dh & 0xC0) | ((day >> 8) & 1);
    rtc_dirty = 0;
  }
  __device__ void rtc_tick(int cycles) {
    if (cycles <= 0 || kind != MBC_MBC3 || rtc_halt) return;
    if (rtc_sub < 0) rtc_sub = 0;
    rtc_sub += cycles;
    if (rtc_sub >= kRtcCyclesPerSecond || rtc_dirty) rtc_slow();
  }

  // -- JOYP (cpu_step_builder.py:195-247) ----------------------------------------
  __device__ uint32_t joyp_value(uint32_t sel) const {
    const bool pressed = frames_done < release;
    uint32_t dpad = 0, btn = 0;
    if (pressed) {
      dpad = action == 4 ? 4u : action == 5 ? 8u : action == 6 ? 2u : action == 7 ? 1u : 0u;
      btn = action == 1 ? 1u : action == 2 ? 2u : action == 3 ? 8u : 0u;
    }
    const uint32_t p14 = (sel >> 4) & 1u, p15 = (sel >> 5) & 1u;
    uint32_t v = (sel | 0xCFu) & 0xFFu;
    if (p14 && p15) v = 0x0Fu;
    else if (!p14 && !p15) {
    } else if (!p14) v &= 0x0Fu & ~dpad;
    else v &= 0x0Fu & ~btn;
    return v | 0xC0u;
  }

  // -- bus write (reference write8, cpu_step_builder.py:659-873) ----------------
  __device__ void io_write(uint32_t x, uint32_t v) {
    switch (x & 0xFFu) {
      case 0x00: {
        const uint32_t sel = v & 0x30u;
        SC(F_JOYP_SELECT) = (int32_t)sel;
        joyp = joyp_value(sel);
      } break;
      case 0x0F: ifr = v & 0x1Fu; break;
      case 0x02:
        if ((v & 0x80u) && (v & 0x01u)) {
          const int idx = SC(F_SERIAL_LEN);
          if (idx < kSerialMax) {
            s.serial[(size_t)e * kSerialMax + idx] = M(0xFF01);
            SC(F_SERIAL_LEN) = idx + 1;
          } else {
            SC(F_SERIAL_OVERFLOW) = 1;
          }
          M(0xFF02) = (uint8_t)(v & 0x7Fu);
          ifr |= 0x08u;
        } else {
          M(0xFF02) = (uint8_t)v;
        }
        break;
      case 0x50:
        if (v != 0 && boot_en) {
          boot_en = 0;
          CS(CS_BOOTROM_ENABLED) = 0;
        }
        break;
      case 0x04: {
        const uint32_t pre = timer_in(div, tac);
        ff04 = 0;
        div = 0;
        const uint32_t post = timer_in(0, tac);
        tprev = post;
        if (pre && !post) tima_inc();
      } break;
      case 0x05: tima = v; break;
      case 0x06: tma = v; break;
      case 0x07: {
        const uint32_t pre = timer_in(div, tac);
        tac = v & 7u;
        const uint32_t post = timer_in(div, tac);
        tprev = post;
        if (pre && !post) tima_inc();
      } break;
      case 0x46: {
        M(0xFF46) = (uint8_t)v;
        const uint32_t src = v << 8;
#pragma unroll 1
        for (uint32_t k = 0; k < 160; ++k) {
          const uint32_t sa = (src + k) & 0xFFFFu;
          M(0xFE00u + k) = (uint8_t)(sa >= 0xFF00u ? io_read(sa) : M(sa));
        }
      } break;
      case 0xFF: ie = v & 0x1Fu; break;
      case 0x40: lcdc = v; break;
      case 0x41: stat = v; break;
      case 0x44: lym = v; break;
      case 0x45: lyc = v; break;
      case 0x4A: wy = v; break;
      default: M(x) = (uint8_t)v; break;
    }
  }
  __device__ void mbc_write(uint32_t x, uint32_t v) {
    if (kind == MBC_MBC1) {
      if (x < 0x2000u) CS(CS_RAM_ENABLE) = (v & 0x0Fu) == 0x0Au ? 1 : 0;
      else if (x < 0x4000u) CS(CS_ROM_BANK_LO) = (v & 0x1Fu) ? (int)(v & 0x1Fu) : 1;
      else if (x < 0x6000u) {
        CS(CS_ROM_BANK_HI) = (int)(v & 3u);
        CS(CS_RAM_BANK) = (int)(v & 3u);
      } else {
        CS(CS_BANK_MODE) = (int)(v & 1u);
      }
    } else if (kind == MBC_MBC3) {
      if (x < 0x2000u) CS(CS_RAM_ENABLE) = (v & 0x0Fu) == 0x0Au ? 1 : 0;
      else if (x < 0x4000u) CS(CS_ROM_BANK_LO) = (v & 0x7Fu) ? (int)(v & 0x7Fu) : 1;
      else if (x < 0x6000u) {
        const int sel = (int)(v & 0x0Fu);
        CS(CS_RTC_SELECT) = sel;
        if (sel <= 3) CS(CS_RAM_BANK) = sel;
      } else if (v == 0) {
        CS(CS_RTC_LATCH) = 0;
      } else if (v == 1 && CS(CS_RTC_LATCH) == 0) {
        for (int k = 0; k < 5; ++k) CS(CS_RTC_L_SECONDS + k) = CS(CS_RTC_SECONDS + k);
        CS(CS_RTC_LATCH) = 1;
      }
    } else {
      return;
    }
    refresh_cart();
  }
  __device__ void write8(uint32_t addr, uint32_t v) {
    uint32_t x = addr & 0xFFFFu;
    if (x - 0xE000u < 0x1E00u) x -= 0x2000u;
    if (x >= 0xFF00u) {
      io_write(x, v);
    } else if (x - 0xA000u < 0x2000u) {
      if (!ram_ok) return;
      if (rtc_field >= 0) {
        CS(CS_RTC_SECONDS + rtc_field) = (int)v;
        rtc_dirty = 1;
        if (rtc_field == 4) rtc_halt = (v & 0x40u) ? 1u : 0u;
        return;
      }
      CR(ram_off + (x - 0xA000u)) = (uint8_t)v;
    } else if (x < 0x8000u) {
      mbc_write(x, v);
    } else {
      M(x) = (uint8_t)v;
    }
  }

  // -- PPU line bookkeeping (cpu_step_builder.py:421-524, 1406-1500) -----------
  __device__ void latch_env0() {
    if (e != 0 || ly >= (uint32_t)kScreenH) return;
    uint8_t* L = s.latches;
    L[0 * kScreenH + ly] = (uint8_t)lcdc;
    L[1 * kScreenH + ly] = M(0xFF43);
    L[2 * kScreenH + ly] = M(0xFF42);
    L[3 * kScreenH + ly] = M(0xFF47);
    L[4 * kScreenH + ly] = M(0xFF4B);
    L[5 * kScreenH + ly] = (uint8_t)wy;
    L[6 * kScreenH + ly] = (uint8_t)(wl & 0xFFu);
    L[7 * kScreenH + ly] = M(0xFF48);
    L[8 * kScreenH + ly] = M(0xFF49);
  }
  __device__ uint32_t ppu_advance(int cycles) {
    const uint32_t lc = lcdc;
    if (!(lc & 0x80u)) {
      scan = 0;
      ly = 0;
      wl = 0;
      lym = 0;
      stat = (stat & 0xF8u) | ((lyc == 0u) ? 4u : 0u);
      stat_prev = 0;
      return lc;
    }
    int total = (int)scan + cycles;
    int lines = 0;
    while (total >= kCyclesPerLine) {
      total -= kCyclesPerLine;
      ++lines;
    }
    scan = (uint32_t)total;
    if (lines == 0 && scan == 0) latch_env0();
    for (; lines > 0; --lines) {
      const uint32_t prev = ly;
      if (prev < (uint32_t)kScreenH && (lc & 0x20u) && prev >= wy) wl += 1;
      ly = (ly + 1u) % (uint32_t)kLinesPerFrame;
      if (ly == 0) wl = 0;
      lym = ly;
      // ppu_update_stat_irq with mode 0 or 1
      const uint32_t mode = ly >= (uint32_t)kScreenH ? 1u : 0u;
      const uint32_t coin = ly == lyc ? 1u : 0u;
      const uint32_t keep = stat & 0xF8u;
      stat = keep | (coin << 2) | mode;
      const uint32_t cur = (mode == 0 ? 1u : 0u) | (mode == 1 ? 2u : 0u) | (coin << 3);
      const uint32_t en = (keep >> 3) & 0xFu;  // bit0 mode0, bit1 mode1, bit2 mode2, bit3 lyc
      if (en & cur & ~(stat_prev & 0xFu)) ifr |= 0x02u;
      stat_prev = cur;
      if (prev == 143u && ly == 144u) ifr |= 0x01u;
      if (ly < (uint32_t)kScreenH) latch_env0();
    }
    const uint32_t mode = ly >= (uint32_t)kScreenH ? 1u : scan < 80u ? 2u : scan < 250u ? 3u : 0u;
    const uint32_t coin = ly == lyc ? 1u : 0u;
    stat = (stat & 0xF8u) | (coin << 2) | mode;
    stat_prev = (mode == 0 ? 1u : 0u) | (mode == 1 ? 2u : 0u) | (mode == 2 ? 4u : 0u) | (coin << 3);
    return lc;
  }

  // -- 8-bit ALU (cpu_templates/alu.py) ------------------------------------------
  __device__ void alu(uint32_t kind8, uint32_t v) {
    const uint32_t cf = (f >> 4) & 1u;
    switch (kind8) {
      case 0: case 1: {  // ADD / ADC
        const uint32_t cin = kind8 == 1 ? cf : 0u;
        const uint32_t s_ = a + v + cin;
        f = (((s_ & 0xFFu) == 0) << 7) | ((((a & 15u) + (v & 15u) + cin) > 15u) << 5) |
            ((s_ > 0xFFu) << 4);
        a = s_ & 0xFFu;
      } break;
      case 2: case 3: case 7: {  // SUB / SBC / CP
        const uint32_t cin = kind8 == 3 ? cf : 0u;
        const int d = (int)a - (int)v - (int)cin;
        const uint32_t hf = ((int)(a & 15u) - (int)((v & 15u) + cin)) < 0 ? 1u : 0u;
        const uint32_t c_ = a < v + cin ? 1u : 0u;
        f = ((((uint32_t)d & 0xFFu) == 0) << 7) | 0x40u | (hf << 5) | (c_ << 4);
        if (kind8 != 7) a = (uint32_t)d & 0xFFu;
      } break;
      case 4: a &= v; f = ((a == 0) << 7) | 0x20u; break;
      case 5: a = (a ^ v) & 0xFFu; f = (a == 0) << 7; break;
      default: a = (a | v) & 0xFFu; f = (a == 0) << 7; break;
    }
  }
  __device__ bool cond(uint32_t cc) const {
    const uint32_t z = (f >> 7) & 1u, c_ = (f >> 4) & 1u;
    switch (cc) {
      case 0: return true;
      case 1: return z == 0;
      case 2: return z != 0;
      case 3: return c_ == 0;
      default: return c_ != 0;
    }
  }
};

// ---------------------------------------------------------------------------
// The kernel
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void step_kernel(DevState s, StepArgs args) {
  const uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (uint32_t)s.n) return;
  Lane L{s};
  L.e = e;
  L.lane = e & (kEnvBlock - 1);
  const uint32_t blk = __builtin_amdgcn_readfirstlane(e >> kEnvBlockShift);
  L.rm = make_rsrc(s.mem + ((size_t)blk << 22), 1u << 22);
  L.rcr = make_rsrc(s.cram + (size_t)blk * (size_t)s.cram_stride * kEnvBlock,
                    (uint32_t)s.cram_stride * kEnvBlock);
  L.rsc = make_rsrc(s.sc + (size_t)blk * (kNumFields * kEnvBlock), kNumFields * kEnvBlock * 4);
  L.rcs = make_rsrc(s.cs + (size_t)blk * (kCartStateStride * kEnvBlock),
                    kCartStateStride * kEnvBlock * 4);
  L.rrom = make_rsrc(s.rom, (uint32_t)s.rom_len);
  const rsrc_t rcnt = make_rsrc(s.cnt + (size_t)blk * (2 * kEnvBlock), 2 * kEnvBlock * 8);

  // ---- load (cpu_step_builder.py:930-967) ---------------------------------
  L.pc = (uint32_t)L.SC(F_PC) & 0xFFFFu;
  L.sp = (uint32_t)L.SC(F_SP) & 0xFFFFu;
  L.a = (uint32_t)L.SC(F_A) & 0xFFu;
  L.f = (uint32_t)L.SC(F_F) & 0xF0u;
  L.w0 = (((uint32_t)L.SC(F_B) & 0xFFu) << 24) | (((uint32_t)L.SC(F_C) & 0xFFu) << 16) |
         (((uint32_t)L.SC(F_D) & 0xFFu) << 8) | ((uint32_t)L.SC(F_E) & 0xFFu);
  L.w1 = (((uint32_t)L.SC(F_H) & 0xFFu) << 24) | (((uint32_t)L.SC(F_L) & 0xFFu) << 16);
  L.ime = (uint32_t)L.SC(F_IME);
  L.ime_delay = (uint32_t)L.SC(F_IME_DELAY);
  L.halted = (uint32_t)L.SC(F_HALTED);
  L.div = (uint32_t)L.SC(F_DIV_COUNTER);
  L.tprev = (uint32_t)L.SC(F_TIMER_PREV_IN);
  L.pend = (uint32_t)L.SC(F_TIMA_PENDING);
  L.delay = (uint32_t)L.SC(F_TIMA_DELAY);
  L.scan = (uint32_t)L.SC(F_PPU_SCANLINE);
  L.ly = (uint32_t)L.SC(F_PPU_LY);
  L.wl = (uint32_t)L.SC(F_PPU_WINDOW_LINE);
  L.stat_prev = (uint32_t)L.SC(F_PPU_STAT_PREV);
  L.joyp = L.M(0xFF00);
  L.ff04 = L.M(0xFF04);
  L.tima = L.M(0xFF05);
  L.tma = L.M(0xFF06);
  L.tac = L.M(0xFF07);
  L.ifr = L.M(0xFF0F);
  L.lcdc = L.M(0xFF40);
  L.stat = L.M(0xFF41);
  L.lym = L.M(0xFF44);
  L.lyc = L.M(0xFF45);
  L.wy = L.M(0xFF4A);
  L.ie = L.M(0xFFFF);
  L.kind = (uint32_t)L.CS(CS_MBC_KIND);
  L.boot_en = L.CS(CS_BOOTROM_ENABLED) != 0 ? 1u : 0u;
  L.rtc_sub = L.CS(CS_RTC_LAST_CYCLE);
  L.rtc_halt = (L.CS(CS_RTC_DAYS_HIGH) & 0x40) ? 1u : 0u;
  L.rtc_dirty = 1;  // first tick of a launch normalizes like the reference does
  L.refresh_cart();
  L.action = args.actions[e];
  L.release = args.release;
  L.frames_done = 0;

  auto ld64 = [&](uint32_t slot) {
    const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b32(rcnt, (int)(L.lane << 3), (int)(slot << 9), 0);
    const uint32_t hi = __builtin_amdgcn_raw_buffer_load_b32(rcnt, (int)(L.lane << 3), (int)((slot << 9) + 4), 0);
    return (int64_t)(((uint64_t)hi << 32) | lo);
  };
  auto st64 = [&](uint32_t slot, int64_t v) {
    __builtin_amdgcn_raw_buffer_store_b32((uint32_t)v, rcnt, (int)(L.lane << 3), (int)(slot << 9), 0);
    __builtin_amdgcn_raw_buffer_store_b32((uint32_t)((uint64_t)v >> 32), rcnt, (int)(L.lane << 3),
                                          (int)((slot << 9) + 4), 0);
  };
  int64_t instr = ld64(0);
  const int64_t instr_start = instr;
  int64_t cyc = ld64(1);
  int cframe = L.SC(F_CYCLE_IN_FRAME);
  int trap = L.SC(F_TRAP_FLAG), trap_pc = L.SC(F_TRAP_PC);
  int trap_op = L.SC(F_TRAP_OPCODE), trap_kind = L.SC(F_TRAP_KIND);
  const uint32_t watch_val = args.dbg_watch ? (uint32_t)L.M((uint32_t)args.dbg_watch) : 0u;
  const int frames = args.frames;

  while (L.frames_done < frames) {
    if (trap) break;
    const uint32_t lcdc_prev = L.lcdc & 0x80u;
    const bool hiter = L.halted != 0;
    int cycles = 4;
    uint32_t op = 0, b1 = 0;
    const uint32_t pc_before = L.pc;
    // pending bus writes: the instruction's, then the interrupt push
    uint32_t wn = 0, wa0 = 0, wv0 = 0, wa1 = 0, wv1 = 0;
    bool stop = false;

    if (!hiter) {
      // ---- fetch 3 bytes -----------------------------------------------------
      uint32_t b2;
      const uint32_t pc = L.pc;
      if (pc <= 0x7FFDu && (pc & 0x3FFFu) <= 0x3FFDu && !(L.boot_en && pc < 0x100u)) {
        const int off = pc < 0x4000u ? L.rom_lo : L.rom_hi;
        if (off >= 0) {
          const int o = off + (int)(pc & 0x3FFFu);
          op = L.rom_at(o);
          b1 = L.rom_at(o + 1);
          b2 = L.rom_at(o + 2);
        } else {
          op = b1 = b2 = 0xFFu;
        }
      } else {
        b2 = 0;
#pragma unroll 1
        for (uint32_t k = 0; k < 3; ++k) {
          const uint32_t v = L.read8(pc + k);
          if (k == 0) op = v;
          else if (k == 1) b1 = v;
          else b2 = v;
        }
      }
      if (args.dbg_trap_pc && pc == (uint32_t)args.dbg_trap_pc) {
        if (!trap) { trap = 1; trap_pc = (int)pc; trap_op = (int)op; trap_kind = 5; }
        break;
      }
      if (args.dbg_rst38 && op == 0xFFu && pc != 0x0038u) {
        if (!trap) { trap = 1; trap_pc = (int)pc; trap_op = (int)op; trap_kind = 3; }
        break;
      }
      const uint64_t r = kDecode.e[op];
      const uint32_t cls = fld(r, 0, 4);
      uint32_t am = fld(r, 4, 3), nr = fld(r, 7, 2);
      const uint32_t len = fld(r, 9, 2);
      cycles = (int)fld(r, 11, 5);
      const uint32_t x = fld(r, 16, 4), y = fld(r, 20, 4), z = fld(r, 24, 4);
      if (cls == K_CB && (b1 & 7u) == 6u) {
        am = AM_HL;
        nr = 1;
      }
      const uint32_t imm16 = b1 | (b2 << 8);
      // ---- address + read phase ------------------------------------------------
      uint32_t ra;
      switch (am) {
        case AM_HL: ra = L.hl(); break;
        case AM_BC: ra = L.w0 >> 16; break;
        case AM_DE: ra = L.w0 & 0xFFFFu; break;
        case AM_A16: ra = imm16; break;
        case AM_A8: ra = 0xFF00u | b1; break;
        case AM_C: ra = 0xFF00u | ((L.w0 >> 16) & 0xFFu); break;
        default: ra = L.sp; break;
      }
      uint32_t rd0 = 0, rd1 = 0;
#pragma unroll 1
      for (uint32_t k = 0; k < nr; ++k) {
        const uint32_t v = L.read8(ra + k);
        if (k == 0) rd0 = v;
        else rd1 = v;
      }
      // ---- execute ----------------------------------------------------------------
      uint32_t npc = (L.pc + len) & 0xFFFFu;
      switch (cls) {
        case K_LD: {  // loads.py
          const uint32_t v = y == SRC_MEM ? rd0 : y == SRC_IMM ? b1 : L.r8(y);
          if (x == SRC_MEM) {
            wn = 1;
            wa0 = ra;
            wv0 = v;
          } else {
            L.set_r8(x, v);
          }
          if (z) L.set_hl(z == 1 ? ra + 1u : ra - 1u);
        } break;
        case K_ALU:
          L.alu(x, y == SRC_MEM ? rd0 : y == SRC_IMM ? b1 : L.r8(y));
          break;
        case K_INCDEC: {  // alu.py:13-22, 208-217, 913-946
          const uint32_t old = x == 6 ? rd0 : L.r8(x);
          const uint32_t v = (y ? old - 1u : old + 1u) & 0xFFu;
          const uint32_t hf = y ? ((old & 15u) == 0) : ((old & 15u) == 15u);
          L.f = ((v == 0) << 7) | (y << 6) | (hf << 5) | (L.f & 0x10u);
          if (x == 6) {
            wn = 1;
            wa0 = ra;
            wv0 = v;
          } else {
            L.set_r8(x, v);
          }
        } break;
        case K_R16:
          if (x == 0) {
            L.set_rr(y, imm16);
          } else if (x == 1) {
            L.set_rr(y, L.rr(y) + 1u);
          } else if (x == 2) {
            L.set_rr(y, L.rr(y) - 1u);
          } else if (x == 3) {  // ADD HL,rr (alu.py:72-111)
            const uint32_t h = L.hl(), v = L.rr(y), s_ = h + v;
            L.f = (L.f & 0x80u) | ((((h & 0xFFFu) + (v & 0xFFFu)) > 0xFFFu) << 5) |
                  ((s_ > 0xFFFFu) << 4);
            L.set_hl(s_);
          } else {
            L.sp = L.hl();
          }
          break;
        case K_ACC: {  // bitops.py:13-48, alu.py:897-950
          const uint32_t av = L.a, cf = (L.f >> 4) & 1u;
          switch (x) {
            case 0: L.a = ((av << 1) | (av >> 7)) & 0xFFu; L.f = (av >> 7) << 4; break;
            case 1: L.a = (av >> 1) | ((av & 1u) << 7); L.f = (av & 1u) << 4; break;
            case 2: L.a = ((av << 1) | cf) & 0xFFu; L.f = (av >> 7) << 4; break;
            case 3: L.a = (av >> 1) | (cf << 7); L.f = (av & 1u) << 4; break;
            case 4: {  // DAA
              const uint32_t nf = (L.f >> 6) & 1u, hf = (L.f >> 5) & 1u;
              uint32_t adj = 0, carry = cf, v = av;
              if (!nf) {
                if (hf || (v & 15u) > 9u) adj |= 0x06u;
                if (cf || v > 0x99u) {
                  adj |= 0x60u;
                  carry = 1;
                }
                v = (v + adj) & 0xFFu;
              } else {
                if (hf) adj |= 0x06u;
                if (cf) adj |= 0x60u;
                v = (v - adj) & 0xFFu;
              }
              L.f = ((v == 0) << 7) | (nf << 6) | (carry << 4);
              L.a = v;
            } break;
            case 5: L.a = av ^ 0xFFu; L.f = (L.f & 0x90u) | 0x60u; break;
            case 6: L.f = (L.f & 0x80u) | 0x10u; break;
            default: L.f = (L.f & 0x80u) | ((cf ^ 1u) << 4); break;
          }
        } break;
        case K_JUMP: {  // jumps.py, stack.py
          const bool take = L.cond(y);
          uint32_t target;
          switch (x) {
            case J_JR: target = (L.pc + 2u + (uint32_t)(int)(int8_t)b1) & 0xFFFFu; break;
            case J_JPHL: target = L.hl(); break;
            case J_RET: case J_RETI: target = rd0 | (rd1 << 8); break;
            case J_RST: target = op & 0x38u; break;
            default: target = imm16; break;
          }
          if (take) {
            if (x == J_CALL || x == J_RST) {
              const uint32_t ret = npc;
              wn = 2;
              wa0 = (L.sp - 1u) & 0xFFFFu;
              wv0 = ret >> 8;
              wa1 = (L.sp - 2u) & 0xFFFFu;
              wv1 = ret & 0xFFu;
              L.sp = wa1;
            } else if (x == J_RET || x == J_RETI) {
              L.sp = (L.sp + 2u) & 0xFFFFu;
              if (x == J_RETI) {
                L.ime = 1;
                L.ime_delay = 0;
              }
            }
            npc = target;
          } else {
            cycles = (int)fld(r, 28, 5);
          }
        } break;
        case K_STACK:
          if (x == 0) {  // PUSH
            const uint32_t v = y == 3 ? ((L.a << 8) | (L.f & 0xF0u)) : L.rr(y);
            wn = 2;
            wa0 = (L.sp - 1u) & 0xFFFFu;
            wv0 = v >> 8;
            wa1 = (L.sp - 2u) & 0xFFFFu;
            wv1 = v & 0xFFu;
            L.sp = wa1;
          } else {  // POP
            L.sp = (L.sp + 2u) & 0xFFFFu;
            if (y == 3) {
              L.a = rd1;
              L.f = rd0 & 0xF0u;
            } else {
              L.set_rr(y, rd0 | (rd1 << 8));
            }
          }
          break;
        case K_SPE8: {  // alu.py:114-177
          const uint32_t res = (L.sp + (uint32_t)(int)(int8_t)b1) & 0xFFFFu;
          L.f = ((((L.sp & 15u) + (b1 & 15u)) > 15u) << 5) | ((((L.sp & 0xFFu) + b1) > 0xFFu) << 4);
          if (x == 0) L.sp = res;
          else L.set_hl(res);
        } break;
        case K_LDA16SP:  // loads.py template_ld_a16_sp
          wn = 2;
          wa0 = imm16;
          wv0 = L.sp & 0xFFu;
          wa1 = (imm16 + 1u) & 0xFFFFu;
          wv1 = (L.sp >> 8) & 0xFFu;
          break;
        case K_CTRL:  // misc.py
          if (x == 1) {
            L.ime = 0;
            L.ime_delay = 0;
          } else if (x == 2) {
            L.ime = 1;
            L.ime_delay = 0;
          } else if (x == 3) {
            L.halted = 1;
          }
          break;
        case K_CB: {  // bitops.py
          const uint32_t idx = b1 & 7u, grp = b1 >> 6, sub = (b1 >> 3) & 7u;
          uint32_t v = idx == 6 ? rd0 : L.r8(idx);
          const uint32_t cin = (L.f >> 4) & 1u;
          cycles = idx == 6 ? (grp == 1 ? 12 : 16) : 8;
          if (grp == 0) {
            uint32_t cf;
            switch (sub) {
              case 0: cf = v >> 7; v = ((v << 1) | cf) & 0xFFu; break;
              case 1: cf = v & 1u; v = (v >> 1) | (cf << 7); break;
              case 2: cf = v >> 7; v = ((v << 1) | cin) & 0xFFu; break;
              case 3: cf = v & 1u; v = (v >> 1) | (cin << 7); break;
              case 4: cf = v >> 7; v = (v << 1) & 0xFFu; break;
              case 5: cf = v & 1u; v = (v >> 1) | (v & 0x80u); break;
              case 6: cf = 0; v = ((v & 15u) << 4) | (v >> 4); break;
              default: cf = v & 1u; v >>= 1; break;
            }
            L.f = ((v == 0) << 7) | (cf << 4);
          } else if (grp == 1) {
            L.f = ((((v >> sub) & 1u) == 0) << 7) | 0x20u | (cin << 4);
          } else if (grp == 2) {
            v &= ~(1u << sub) & 0xFFu;
          } else {
            v |= 1u << sub;
          }
          if (grp != 1) {
            if (idx == 6) {
              wn = 1;
              wa0 = ra;
              wv0 = v;
            } else {
              L.set_r8(idx, v);
            }
          }
        } break;
        default:  // K_TRAP (misc.py:42-56): freeze the env, pc unchanged
          if (!trap) {
            trap = 1;
            trap_pc = (int)L.pc;
            trap_op = (int)op;
            trap_kind = 1;
          }
          cycles = 0;
          npc = L.pc;
          break;
      }
      L.pc = npc;
    }

    // ---- write phase (instruction writes), then timer/PPU/IRQ; a serviced
    // interrupt queues its two push writes and runs this block once more ----
    int svc = 0;
    uint32_t lcdc_now = L.lcdc;
#pragma unroll 1
    for (int pass = 0; pass < 2; ++pass) {
#pragma unroll 1
      for (uint32_t k = 0; k < wn; ++k) L.write8(k ? wa1 : wa0, k ? wv1 : wv0);
      int tcyc = 20;
      if (pass == 0) {
        if (!hiter) {
          if (args.dbg_rst38 && L.pc >= 0xFE00u) {
            if (!trap) { trap = 1; trap_pc = (int)pc_before; trap_op = (int)op; trap_kind = 4; }
            stop = true;
            break;
          }
          if (trap) {
            stop = true;
            break;
          }
          L.f &= 0xF0u;
          instr += 1;
          if (args.dbg_max_instr > 0 && instr - instr_start >= args.dbg_max_instr) {
            if (!trap) { trap = 1; trap_pc = (int)L.pc; trap_op = (int)op; trap_kind = 6; }
            stop = true;
            break;
          }
          if (args.dbg_watch && (uint32_t)(((uint32_t)args.dbg_watch >= 0xFF00u)
                                               ? L.io_read((uint32_t)args.dbg_watch)
                                               : L.M((uint32_t)args.dbg_watch)) != watch_val) {
            if (!trap) { trap = 1; trap_pc = (int)pc_before; trap_op = (int)op; trap_kind = 7; }
            stop = true;
            break;
          }
        }
        tcyc = cycles;
      }
      L.timer_tick(tcyc);
      if (pass == 0 && !hiter && L.ime_delay) {
        L.ime = 1;
        L.ime_delay = 0;
      }
      lcdc_now = L.ppu_advance(tcyc);
      if (pass == 1) break;
      const uint32_t pending = L.ie & L.ifr & 0x1Fu;
      if (!pending) break;
      L.halted = 0;
      if (!L.ime) {
        if (hiter) L.pc = (L.pc + 1u) & 0xFFFFu;  // IME=0 wake skips a byte
        break;
      }
      // service (cpu_step_builder.py:1502-1600)
      L.ime = 0;
      const uint32_t bit = pending & (0u - pending);
      const uint32_t vec = 0x40u + 8u * (uint32_t)__builtin_ctz(bit);
      L.ifr &= ~bit & 0xFFu;
      wn = 2;
      wa0 = (L.sp - 1u) & 0xFFFFu;
      wv0 = L.pc >> 8;
      wa1 = (L.sp - 2u) & 0xFFFFu;
      wv1 = L.pc & 0xFFu;
      L.sp = wa1;
      L.pc = vec;
      svc = 20;
    }
    if (stop) break;

    const int total = cycles + svc;
    L.rtc_tick(total);
    cyc += total;
    cframe += total;
    if (lcdc_prev && !(lcdc_now & 0x80u)) {
      int tail = 0;
      if (!hiter) {
        tail = total;
        if (op == 0xE0u) {
          const uint32_t imm = L.read8((pc_before + 1u) & 0xFFFFu);
          if (imm == 0x40u && cycles >= 4) tail = total - 4;
        }
      }
      cframe = tail;
      if (++L.frames_done >= frames) break;
      continue;
    }
    if (!hiter && !lcdc_prev && (lcdc_now & 0x80u)) {
      L.scan = 0;
      L.ly = 0;
      L.wl = 0;
      L.lym = 0;
      const uint32_t coin = L.lyc == 0 ? 1u : 0u;
      L.stat = (L.stat & 0xF8u) | (coin << 2) | 2u;
      L.stat_prev = 4u | (coin << 3);
      cframe = 0;
      if (++L.frames_done >= frames) break;
      continue;
    }
    while (cframe >= kCyclesPerFrame) {
      cframe -= kCyclesPerFrame;
      if (++L.frames_done >= frames) break;
    }
  }

  // ---- post-step outputs (cpu_templates/post_step.py) ----------------------
  const int stage = args.stage;
  const uint32_t b_ = L.w0 >> 24, c_ = (L.w0 >> 16) & 0xFFu, d_ = (L.w0 >> 8) & 0xFFu;
  const uint32_t e_ = L.w0 & 0xFFu, h_ = L.w1 >> 24, l_ = (L.w1 >> 16) & 0xFFu;
  if (stage != 0) {
    uint32_t mm[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) mm[k] = L.M(0xC000u + (uint32_t)k);
    if (stage == 2 || stage == 3) {
      float* o = s.obs + (size_t)e * s.obs_dim;
      o[0] = (float)(L.pc & 0xFFFFu) / 65535.0f;
      o[1] = (float)(L.sp & 0xFFFFu) / 65535.0f;
      o[2] = (float)L.a / 255.0f;
      o[3] = (float)L.f / 255.0f;
      o[4] = (float)b_ / 255.0f;
      o[5] = (float)c_ / 255.0f;
      o[6] = (float)d_ / 255.0f;
      o[7] = (float)e_ / 255.0f;
      o[8] = (float)h_ / 255.0f;
      o[9] = (float)l_ / 255.0f;
#pragma unroll
      for (int k = 0; k < 16; ++k) o[10 + k] = (float)mm[k] / 255.0f;
      o[26] = (float)((mm[0] ^ mm[1]) & 0xFFu) / 255.0f;
      o[27] = (float)((mm[2] + mm[3] * 5u) & 0xFFu) / 255.0f;
      o[28] = (float)((mm[4] ^ L.a) & 0xFFu) / 255.0f;
      o[29] = (float)((mm[5] + b_) & 0xFFu) / 255.0f;
      o[30] = (float)((mm[6] ^ c_) & 0xFFu) / 255.0f;
      o[31] = (float)((mm[7] + d_) & 0xFFu) / 255.0f;
    }
    if (stage == 1 || stage == 3) {
      const uint32_t mix = (mm[0] + mm[1] * 3u) & 0xFFu;
      s.reward[e] = (float)((L.a ^ mix) & 0xFFu) / 255.0f;
    }
  }

  // ---- write back --------------------------------------------------------
  L.SC(F_PC) = (int32_t)(L.pc & 0xFFFFu);
  L.SC(F_SP) = (int32_t)(L.sp & 0xFFFFu);
  L.SC(F_A) = (int32_t)L.a;
  L.SC(F_B) = (int32_t)b_;
  L.SC(F_C) = (int32_t)c_;
  L.SC(F_D) = (int32_t)d_;
  L.SC(F_E) = (int32_t)e_;
  L.SC(F_H) = (int32_t)h_;
  L.SC(F_L) = (int32_t)l_;
  L.SC(F_F) = (int32_t)(L.f & 0xF0u);
  st64(0, instr);
  st64(1, cyc);
  L.SC(F_CYCLE_IN_FRAME) = cframe;
  L.SC(F_TRAP_FLAG) = trap;
  L.SC(F_TRAP_PC) = trap_pc;
  L.SC(F_TRAP_OPCODE) = trap_op;
  L.SC(F_TRAP_KIND) = trap_kind;
  L.SC(F_IME) = (int32_t)L.ime;
  L.SC(F_IME_DELAY) = (int32_t)L.ime_delay;
  L.SC(F_HALTED) = (int32_t)L.halted;
  L.SC(F_DIV_COUNTER) = (int32_t)L.div;
  L.SC(F_TIMER_PREV_IN) = (int32_t)L.tprev;
  L.SC(F_TIMA_PENDING) = (int32_t)L.pend;
  L.SC(F_TIMA_DELAY) = (int32_t)L.delay;
  L.SC(F_PPU_SCANLINE) = (int32_t)L.scan;
  L.SC(F_PPU_LY) = (int32_t)L.ly;
  L.SC(F_PPU_WINDOW_LINE) = (int32_t)L.wl;
  L.SC(F_PPU_STAT_PREV) = (int32_t)L.stat_prev;
  L.M(0xFF00) = (uint8_t)L.joyp;
  L.M(0xFF04) = (uint8_t)L.ff04;
  L.M(0xFF05) = (uint8_t)L.tima;
  L.M(0xFF06) = (uint8_t)L.tma;
  L.M(0xFF07) = (uint8_t)L.tac;
  L.M(0xFF0F) = (uint8_t)L.ifr;
  L.M(0xFF40) = (uint8_t)L.lcdc;
  L.M(0xFF41) = (uint8_t)L.stat;
  L.M(0xFF44) = (uint8_t)L.lym;
  L.M(0xFF45) = (uint8_t)L.lyc;
  L.M(0xFF4A) = (uint8_t)L.wy;
  L.M(0xFFFF) = (uint8_t)L.ie;
  if (L.kind == MBC_MBC3) L.CS(CS_RTC_LAST_CYCLE) = L.rtc_sub;
}

}  // namespace

hipError_t launch_step(const DevState& s, const StepArgs& a, hipStream_t st) {
  if (s.n <= 0) return hipSuccess;
  // One wavefront per workgroup: small env counts (16K envs = 256 waves)
  // spread over all CUs instead of packing 4 waves into a quarter of them.
  const int threads = kEnvBlock;
  const int blocks = (s.n + threads - 1) / threads;
  hipLaunchKernelGGL(step_kernel, dim3(blocks), dim3(threads), 0, st, s, a);
  return hipGetLastError();
}

}  // namespace gbx

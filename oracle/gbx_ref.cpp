// gbx_ref.cpp -- TEST INFRASTRUCTURE: the parity oracle (see gbx_ref.h).
//
// A one-env-at-a-time C++ restatement of the reference's Warp CPU backend.
// Each function names the reference code it restates (paths are relative to
// the reference repository root).  Nothing here is optimised or shared with
// the HIP product path; it exists to be obviously the same as the reference.
//
// Pinning (what checks this restatement besides the HIP kernel; expected
// values come from the published SM83/DMG definitions and the reference's
// stated rules, never from this file):
//   - tests/test_oracle_known_answers.py: every unprefixed opcode outside the
//     8-bit ALU block, one instruction from random states, against a model
//     written from the instruction set (loads, 16-bit INC/DEC, stack byte
//     order, jump/call/return targets, rotates of A, CPL/SCF/CCF, DI/EI/RETI);
//     planted mistakes in that model must be caught;
//   - tests/test_oracle_alu.py: every 8-bit ALU/CB op over all operands
//     against closed forms (carries from the full-width result), DAA as BCD;
//   - tests/test_oracle_programs.py: the public cycle table for every opcode,
//     the boot stub's post-boot state, JOYP matrix, timer and LY/STAT/VBlank
//     against cycle-by-cycle brute force, interrupt counts, HALT/EI quirks,
//     MBC1/MBC3 banks and RTC seconds, echo RAM, OAM DMA, IF/IE masks, serial;
//   - tests/test_oracle_timer_ppu.py: STAT requests per frame for all 16
//     source masks against the closed form of the reference's edge rule,
//     LCD on/off frame accounting (LDH (40),A minus-4 tail, interrupt
//     service in the same step, the halted-path variant), obs slots 26-31;
//   - tests/test_oracle_render_reset.py: the reference's renderer known
//     answers, hand-built scenes, an independent numpy renderer, the obs/
//     reward stage known answers and the reset-cache invariants.
#include "gbx_ref.h"

#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <vector>
#ifdef _OPENMP
#include <omp.h>
#endif

namespace {

// src/gbxcule/core/abi.py:33-56, kernels/cpu_step.py:46-58,
// core/cartridge.py:47-76
constexpr int MEM_SIZE = 65536;
constexpr int CYCLES_PER_FRAME = 70224;
constexpr int CYCLES_PER_SCANLINE = 456;
constexpr int LINES_PER_FRAME = 154;
constexpr int SCREEN_H = 144;
constexpr int ROM_LIMIT = 0x8000;
constexpr int CART_RAM_START = 0xA000;
constexpr int CART_RAM_END = 0xC000;
constexpr int ROM_BANK_SIZE = 0x4000;
constexpr int RAM_BANK_SIZE = 0x2000;
constexpr int BOOTROM_SIZE = 0x100;
constexpr int SERIAL_MAX = 1024;
constexpr int RTC_CYCLES_PER_SECOND = 4194304;
constexpr int CS_STRIDE = 20;
enum {
  CS_MBC_KIND = 0, CS_RAM_ENABLE, CS_ROM_BANK_LO, CS_ROM_BANK_HI, CS_RAM_BANK,
  CS_BANK_MODE, CS_BOOTROM_ENABLED, CS_RTC_SELECT, CS_RTC_LATCH, CS_RTC_SECONDS,
  CS_RTC_MINUTES, CS_RTC_HOURS, CS_RTC_DAYS_LOW, CS_RTC_DAYS_HIGH,
  CS_RTC_LAST_CYCLE, CS_RTC_L_SECONDS, CS_RTC_L_MINUTES, CS_RTC_L_HOURS,
  CS_RTC_L_DAYS_LOW, CS_RTC_L_DAYS_HIGH
};
enum { MBC_ROM_ONLY = 0, MBC_MBC1 = 1, MBC_MBC3 = 2 };
constexpr int DS_W = 80, DS_H = 72, DS_WB = 20;

}  // namespace

struct RefMachine {
  int n = 0;
  int obs_dim = 32;
  std::vector<uint8_t> rom, boot;
  int rom_bank_count = 0, rom_bank_mask = -1, ram_bank_count = 0;
  int ram_bytes = 0, ram_stride = 1, mbc_kind = 0;

  std::vector<uint8_t> mem, cart_ram, serial_buf;
  std::vector<int32_t> cart_state;
  std::vector<int32_t> s32[REF_NUM_SCALAR_FIELDS];  // int32 fields
  std::vector<int64_t> instr_count, cycle_count, data_bytes;
  std::vector<uint8_t> joyp_select, serial_overflow, ppu_stat_prev;
  uint8_t latches[9][SCREEN_H];
  std::vector<float> obs, reward;
  std::vector<uint8_t> pix, pix_packed;

  // debug traps (kernels/cpu_step.py:85-114); 0 disables
  int dbg_rst38 = 0, dbg_trap_pc = 0, dbg_max_instr = 0, dbg_watch = 0;

  // ResetCache snapshot (core/reset_cache.py:68-190)
  bool snap_valid = false, snap_has_pix = false;
  std::vector<uint8_t> snap_mem, snap_cart_ram, snap_serial, snap_pix;
  int32_t snap_cart_state[CS_STRIDE];
  int64_t snap_scalar[REF_NUM_SCALAR_FIELDS];
};

namespace {

// Every per-env scalar, read/written as int64 for snapshot/restore.
int64_t get_scalar(const RefMachine& m, int f, int i) {
  switch (f) {
    case REF_INSTR_COUNT: return m.instr_count[i];
    case REF_CYCLE_COUNT: return m.cycle_count[i];
    case REF_JOYP_SELECT: return m.joyp_select[i];
    case REF_SERIAL_OVERFLOW: return m.serial_overflow[i];
    case REF_PPU_STAT_PREV: return m.ppu_stat_prev[i];
    default: return m.s32[f][i];
  }
}

void set_scalar(RefMachine& m, int f, int i, int64_t v) {
  switch (f) {
    case REF_INSTR_COUNT: m.instr_count[i] = v; break;
    case REF_CYCLE_COUNT: m.cycle_count[i] = v; break;
    case REF_JOYP_SELECT: m.joyp_select[i] = (uint8_t)v; break;
    case REF_SERIAL_OVERFLOW: m.serial_overflow[i] = (uint8_t)v; break;
    case REF_PPU_STAT_PREV: m.ppu_stat_prev[i] = (uint8_t)v; break;
    default: m.s32[f][i] = (int32_t)v; break;
  }
}

inline int sign8(int x) { return x >= 128 ? x - 256 : x; }
inline int make_flags(int z, int n, int h, int c) {
  return (z << 7) | (n << 6) | (h << 5) | (c << 4);
}

// kernels/cpu_step_builder.py:195-217
int action_dpad_mask(int action) {
  if (action == 4) return 4;  // UP
  if (action == 5) return 8;  // DOWN
  if (action == 6) return 2;  // LEFT
  if (action == 7) return 1;  // RIGHT
  return 0;
}
int action_button_mask(int action) {
  if (action == 1) return 1;  // A
  if (action == 2) return 2;  // B
  if (action == 3) return 8;  // START
  return 0;
}

// kernels/cpu_step_builder.py:219-247
int joyp_read(int action, int frame_idx, int release, int joyp_sel) {
  int sel = joyp_sel & 0x30;
  int pressed = frame_idx < release;
  int dpad = 0, btn = 0;
  if (pressed) {
    dpad = action_dpad_mask(action);
    btn = action_button_mask(action);
  }
  int directional = 0x0F & ~dpad;
  int standard = 0x0F & ~btn;
  int p14 = (sel >> 4) & 1, p15 = (sel >> 5) & 1;
  int v = (sel | 0xCF) & 0xFF;
  if (p14 && p15) {
    v = 0x0F;
  } else if (!p14 && !p15) {
  } else if (!p14) {
    v &= directional;
  } else {
    v &= standard;
  }
  return v | 0xC0;
}

// kernels/cpu_step_builder.py:249-265
int timer_div_bit(int tac) {
  switch (tac & 3) {
    case 0: return 9;
    case 1: return 3;
    case 2: return 5;
    default: return 7;
  }
}
int timer_in(int div, int tac) {
  if ((tac & 4) == 0) return 0;
  return (div >> timer_div_bit(tac)) & 1;
}

// kernels/cpu_step_builder.py:526-536
int clamp_bank(int bank, int count, int mask) {
  if (count <= 0) return 0;
  if (mask >= 0) return bank & mask;
  return bank % count;
}

// One env's view of the machine during one cpu_step launch
// (kernels/cpu_step_builder.py:875-1781).
//
// During a launch the env's scalar fields, cart state and per-env byte
// counters live in this object (on the stepping thread's stack) and are
// written back at the end: neighbouring envs' fields share cache lines in
// the machine's env-major arrays, and threads stepping neighbours would
// otherwise contend for those lines on every instruction.
struct Env {
  RefMachine& m;
  int i;
  uint8_t* mem;
  int32_t* cs_out;  // the env's row of the machine's cart_state
  int frames_done = 0;
  int release = 0;
  int32_t sl[REF_NUM_SCALAR_FIELDS];
  int32_t cs[CS_STRIDE];
  int64_t data_bytes = 0;
  uint8_t stat_prev = 0, joyp_sel = 0, ser_ovf = 0;

  Env(RefMachine& machine, int env, uint8_t* env_mem, int32_t* env_cs)
      : m(machine), i(env), mem(env_mem), cs_out(env_cs) {
    for (int f = 0; f < REF_NUM_SCALAR_FIELDS; ++f) sl[f] = m.s32[f][i];
    memcpy(cs, cs_out, sizeof(cs));
    data_bytes = m.data_bytes[i];
    stat_prev = m.ppu_stat_prev[i];
    joyp_sel = m.joyp_select[i];
    ser_ovf = m.serial_overflow[i];
  }
  void store() {
    for (int f = 0; f < REF_NUM_SCALAR_FIELDS; ++f) m.s32[f][i] = sl[f];
    memcpy(cs_out, cs, sizeof(cs));
    m.data_bytes[i] = data_bytes;
    m.ppu_stat_prev[i] = stat_prev;
    m.joyp_select[i] = joyp_sel;
    m.serial_overflow[i] = ser_ovf;
  }

  int32_t& S(int f) { return sl[f]; }
  uint8_t& M(int addr) { return mem[addr]; }

  // ---- bus: kernels/cpu_step_builder.py:538-657 ---------------------------
  int read8(int addr) {
    int a = addr & 0xFFFF;
    if (a >= 0xE000 && a < 0xFE00) a -= 0x2000;
    if (a >= 0x8000) data_bytes += 1;
    if (a < BOOTROM_SIZE && cs[CS_BOOTROM_ENABLED] != 0) return m.boot[a];
    if (a < ROM_LIMIT) {
      int kind = cs[CS_MBC_KIND];
      int lo_raw = cs[CS_ROM_BANK_LO];
      int lo = lo_raw & 0x1F;
      int hi = cs[CS_ROM_BANK_HI] & 0x03;
      int mode = cs[CS_BANK_MODE] & 1;
      int bank = 0;
      if (a < 0x4000) {
        if (kind == MBC_MBC1 && mode != 0) bank = (hi & 3) << 5;
      } else if (kind == MBC_ROM_ONLY) {
        bank = 1;
      } else if (kind == MBC_MBC1) {
        bank = (hi << 5) | lo;
        if (bank == 0) bank = 1;
      } else {
        bank = lo_raw & 0x7F;
        if (bank == 0) bank = 1;
      }
      bank = clamp_bank(bank, m.rom_bank_count, m.rom_bank_mask);
      int64_t idx = (int64_t)bank * ROM_BANK_SIZE + (a < 0x4000 ? a : a - 0x4000);
      if (idx < (int64_t)m.rom_bank_count * ROM_BANK_SIZE) return m.rom[idx];
      return 0xFF;
    }
    if (a == 0xFF00) return M(0xFF00);
    if (a >= CART_RAM_START && a < CART_RAM_END) {
      if (m.ram_bank_count <= 0) return 0xFF;
      if (cs[CS_RAM_ENABLE] == 0) return 0xFF;
      int kind = cs[CS_MBC_KIND];
      if (kind == MBC_MBC3) {
        int sel = cs[CS_RTC_SELECT] & 0x0F;
        bool latched = cs[CS_RTC_LATCH] != 0;
        if (sel >= 0x08 && sel <= 0x0C) {
          int live = CS_RTC_SECONDS + (sel - 0x08);
          int held = CS_RTC_L_SECONDS + (sel - 0x08);
          return (latched ? cs[held] : cs[live]) & 0xFF;
        }
      }
      int rb = 0;
      if (kind == MBC_MBC1) {
        if ((cs[CS_BANK_MODE] & 1) != 0) rb = cs[CS_RAM_BANK] & 3;
      } else if (kind == MBC_MBC3) {
        rb = cs[CS_RAM_BANK] & 3;
      }
      rb = clamp_bank(rb, m.ram_bank_count, -1);
      int env_bytes = m.ram_bank_count * RAM_BANK_SIZE;
      if (env_bytes <= 0) return 0xFF;
      int off = rb * RAM_BANK_SIZE + (a - CART_RAM_START);
      if (off >= env_bytes) return 0xFF;
      return m.cart_ram[(int64_t)i * env_bytes + off];
    }
    return M(a);
  }

  // ---- timer: kernels/cpu_step_builder.py:267-372 ---------------------------
  void tima_inc() {
    int t = M(0xFF05);
    M(0xFF05) = (uint8_t)((t + 1) & 0xFF);
    if (t == 0xFF) {
      S(REF_TIMA_RELOAD_PENDING) = 1;
      S(REF_TIMA_RELOAD_DELAY) = 4;
    }
  }
  void tima_reload_now() {
    M(0xFF05) = M(0xFF06);
    M(0xFF0F) = (uint8_t)(M(0xFF0F) | 0x04);
    S(REF_TIMA_RELOAD_PENDING) = 0;
    S(REF_TIMA_RELOAD_DELAY) = 0;
  }
  void timer_tick(int cycles) {
    if (cycles <= 0) return;
    int remaining = cycles;
    int div = S(REF_DIV_COUNTER) & 0xFFFF;
    int32_t& pend = S(REF_TIMA_RELOAD_PENDING);
    int32_t& delay = S(REF_TIMA_RELOAD_DELAY);
    while (remaining > 0) {
      if (pend != 0 && delay <= 0) tima_reload_now();
      int tac = M(0xFF07) & 7;
      int dt = remaining;
      if (pend != 0 && delay < dt) dt = delay;
      bool edge = false;
      if (tac & 4) {
        int period = 1 << (timer_div_bit(tac) + 1);
        int edge_dt = period - (div & (period - 1));
        if (edge_dt < dt) dt = edge_dt;
        if (dt == edge_dt) edge = true;
      }
      div = (div + dt) & 0xFFFF;
      if (pend != 0) delay -= dt;
      remaining -= dt;
      if (edge) tima_inc();
      if (pend != 0 && delay <= 0) tima_reload_now();
    }
    S(REF_DIV_COUNTER) = div;
    M(0xFF04) = (uint8_t)((div >> 8) & 0xFF);
    S(REF_TIMER_PREV_IN) = timer_in(div, M(0xFF07) & 7);
  }

  // ---- MBC3 RTC: kernels/cpu_step_builder.py:374-419 -------------------------
  void rtc_tick(int cycles) {
    if (cycles <= 0) return;
    if (cs[CS_MBC_KIND] != MBC_MBC3) return;
    int dh = cs[CS_RTC_DAYS_HIGH];
    if (dh & 0x40) return;
    int sub = cs[CS_RTC_LAST_CYCLE];
    if (sub < 0) sub = 0;
    sub += cycles;
    int sec = cs[CS_RTC_SECONDS] & 0xFF;
    int mn = cs[CS_RTC_MINUTES] & 0x3F;
    int hr = cs[CS_RTC_HOURS] & 0x1F;
    int day = ((dh & 1) << 8) | (cs[CS_RTC_DAYS_LOW] & 0xFF);
    while (sub >= RTC_CYCLES_PER_SECOND) {
      sub -= RTC_CYCLES_PER_SECOND;
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
    cs[CS_RTC_SECONDS] = sec;
    cs[CS_RTC_MINUTES] = mn;
    cs[CS_RTC_HOURS] = hr;
    cs[CS_RTC_DAYS_LOW] = day & 0xFF;
    cs[CS_RTC_DAYS_HIGH] = (dh & 0xC0) | ((day >> 8) & 1);
    cs[CS_RTC_LAST_CYCLE] = sub;
  }

  // ---- write side effects: kernels/cpu_step_builder.py:659-873 -----------------
  void write8(int addr, int val) {
    int a = addr & 0xFFFF;
    if (a >= 0xE000 && a < 0xFE00) a -= 0x2000;
    if (a >= 0x8000) data_bytes += 1;
    uint8_t v8 = (uint8_t)val;
    if (a == 0xFF00) {
      int sel = v8 & 0x30;
      joyp_sel = (uint8_t)sel;
      M(0xFF00) = (uint8_t)joyp_read(S(REF_ACTIONS), frames_done, release, sel);
      return;
    }
    if (a == 0xFF0F) { M(a) = v8 & 0x1F; return; }
    if (a == 0xFF01) { M(a) = v8; return; }
    if (a == 0xFF02) {
      M(a) = v8;
      if ((val & 0x80) && (val & 0x01)) {
        int sb = M(0xFF01);
        int idx = S(REF_SERIAL_LEN);
        if (idx < SERIAL_MAX) {
          m.serial_buf[(int64_t)i * SERIAL_MAX + idx] = (uint8_t)sb;
          S(REF_SERIAL_LEN) = idx + 1;
        } else {
          ser_ovf = 1;
        }
        M(a) = (uint8_t)(val & 0x7F);
        M(0xFF0F) = (uint8_t)(M(0xFF0F) | 0x08);
      }
      return;
    }
    if (a == 0xFF50) {
      if (val != 0) cs[CS_BOOTROM_ENABLED] = 0;
      return;
    }
    if (a == 0xFF04) {
      int tac = M(0xFF07) & 7;
      int pre = timer_in(S(REF_DIV_COUNTER) & 0xFFFF, tac);
      M(a) = 0;
      S(REF_DIV_COUNTER) = 0;
      int post = timer_in(0, tac);
      S(REF_TIMER_PREV_IN) = post;
      if (pre && !post) tima_inc();
      return;
    }
    if (a == 0xFF05 || a == 0xFF06) { M(a) = v8; return; }
    if (a == 0xFF07) {
      int div = S(REF_DIV_COUNTER) & 0xFFFF;
      int pre = timer_in(div, M(0xFF07) & 7);
      int tac_new = val & 7;
      M(a) = (uint8_t)tac_new;
      int post = timer_in(div, tac_new);
      S(REF_TIMER_PREV_IN) = post;
      if (pre && !post) tima_inc();
      return;
    }
    if (a == 0xFF46) {
      M(a) = v8;
      int src = (val & 0xFF) << 8;
      for (int k = 0; k < 160; ++k) M(0xFE00 + k) = M((src + k) & 0xFFFF);
      data_bytes += 320;
      return;
    }
    if (a == 0xFFFF) { M(a) = v8 & 0x1F; return; }
    if (a >= CART_RAM_START && a < CART_RAM_END) {
      if (m.ram_bank_count <= 0) return;
      if (cs[CS_RAM_ENABLE] == 0) return;
      int kind = cs[CS_MBC_KIND];
      if (kind == MBC_MBC3) {
        int sel = cs[CS_RTC_SELECT] & 0x0F;
        if (sel >= 0x08 && sel <= 0x0C) {
          cs[CS_RTC_SECONDS + (sel - 0x08)] = val & 0xFF;
          return;
        }
      }
      int rb = 0;
      if (kind == MBC_MBC1) {
        if ((cs[CS_BANK_MODE] & 1) != 0) rb = cs[CS_RAM_BANK] & 3;
      } else if (kind == MBC_MBC3) {
        rb = cs[CS_RAM_BANK] & 3;
      }
      rb = clamp_bank(rb, m.ram_bank_count, -1);
      int env_bytes = m.ram_bank_count * RAM_BANK_SIZE;
      if (env_bytes <= 0) return;
      int off = rb * RAM_BANK_SIZE + (a - CART_RAM_START);
      if (off >= env_bytes) return;
      m.cart_ram[(int64_t)i * env_bytes + off] = v8;
      return;
    }
    if (a < ROM_LIMIT) {
      int kind = cs[CS_MBC_KIND];
      if (kind == MBC_MBC1) {
        if (a < 0x2000) {
          cs[CS_RAM_ENABLE] = (val & 0x0F) == 0x0A ? 1 : 0;
        } else if (a < 0x4000) {
          int bank = val & 0x1F;
          cs[CS_ROM_BANK_LO] = bank == 0 ? 1 : bank;
        } else if (a < 0x6000) {
          cs[CS_ROM_BANK_HI] = val & 3;
          cs[CS_RAM_BANK] = val & 3;
        } else {
          cs[CS_BANK_MODE] = val & 1;
        }
      } else if (kind == MBC_MBC3) {
        if (a < 0x2000) {
          cs[CS_RAM_ENABLE] = (val & 0x0F) == 0x0A ? 1 : 0;
        } else if (a < 0x4000) {
          int bank = val & 0x7F;
          cs[CS_ROM_BANK_LO] = bank == 0 ? 1 : bank;
        } else if (a < 0x6000) {
          int sel = val & 0x0F;
          cs[CS_RTC_SELECT] = sel;
          if (sel <= 3) cs[CS_RAM_BANK] = sel;
        } else {
          if (val == 0) {
            cs[CS_RTC_LATCH] = 0;
          } else if (val == 1 && cs[CS_RTC_LATCH] == 0) {
            for (int k = 0; k < 5; ++k) cs[CS_RTC_L_SECONDS + k] = cs[CS_RTC_SECONDS + k];
            cs[CS_RTC_LATCH] = 1;
          }
        }
      }
      return;
    }
    M(a) = v8;
  }

  // ---- PPU: kernels/cpu_step_builder.py:421-524, 1406-1500 ---------------------
  void ppu_update_stat(int ly, int mode) {
    int lyc = M(0xFF45);
    int coincidence = ly == lyc ? 1 : 0;
    int keep = M(0xFF41) & 0xF8;
    M(0xFF41) = (uint8_t)(keep | (coincidence << 2) | mode);
  }
  void ppu_update_stat_irq(int ly, int mode) {
    int lyc = M(0xFF45);
    int coincidence = ly == lyc ? 1 : 0;
    int keep = M(0xFF41) & 0xF8;
    M(0xFF41) = (uint8_t)(keep | (coincidence << 2) | mode);
    int en0 = (keep >> 3) & 1, en1 = (keep >> 4) & 1, en2 = (keep >> 5) & 1,
        enl = (keep >> 6) & 1;
    int c0 = mode == 0, c1 = mode == 1, c2 = mode == 2, cl = coincidence;
    int prev = stat_prev & 0x0F;
    int p0 = prev & 1, p1 = (prev >> 1) & 1, p2 = (prev >> 2) & 1, pl = (prev >> 3) & 1;
    bool edge = (en0 && !p0 && c0) || (en1 && !p1 && c1) || (en2 && !p2 && c2) ||
                (enl && !pl && cl);
    if (edge) M(0xFF0F) = (uint8_t)(M(0xFF0F) | 0x02);
    stat_prev = (uint8_t)(c0 | (c1 << 1) | (c2 << 2) | (cl << 3));
  }
  void capture_latches(int ly, int wl) {
    if (i != 0) return;
    if (ly < 0 || ly >= SCREEN_H) return;
    static const int regs[9] = {0xFF40, 0xFF43, 0xFF42, 0xFF47, 0xFF4B,
                                0xFF4A, -1, 0xFF48, 0xFF49};
    for (int k = 0; k < 9; ++k)
      m.latches[k][ly] = regs[k] < 0 ? (uint8_t)(wl & 0xFF) : M(regs[k]);
  }
  // One of the four identical PPU blocks; returns the LCDC it read.
  int ppu_advance(int cycles, int32_t& scan, int32_t& ly, int32_t& wl) {
    int lcdc = M(0xFF40);
    if ((lcdc & 0x80) == 0) {
      scan = 0;
      ly = 0;
      wl = 0;
      M(0xFF44) = 0;
      ppu_update_stat(0, 0);
      stat_prev = 0;
      return lcdc;
    }
    int total = scan + cycles;
    int lines = total / CYCLES_PER_SCANLINE;
    scan = total - lines * CYCLES_PER_SCANLINE;
    if (lines == 0 && scan == 0) capture_latches(ly, wl);
    while (lines > 0) {
      int prev_ly = ly;
      if (prev_ly < SCREEN_H && (lcdc & 0x20) && prev_ly >= M(0xFF4A)) wl += 1;
      ly = (ly + 1) % LINES_PER_FRAME;
      if (ly == 0) wl = 0;
      M(0xFF44) = (uint8_t)ly;
      ppu_update_stat_irq(ly, ly >= SCREEN_H ? 1 : 0);
      if (prev_ly == 143 && ly == 144) M(0xFF0F) = (uint8_t)(M(0xFF0F) | 0x01);
      if (ly < SCREEN_H) capture_latches(ly, wl);
      --lines;
    }
    int mode = ly >= SCREEN_H ? 1 : scan < 80 ? 2 : scan < 250 ? 3 : 0;
    ppu_update_stat(ly, mode);
    int lyc_eq = ly == M(0xFF45) ? 1 : 0;
    stat_prev =
        (uint8_t)((mode == 0) | ((mode == 1) << 1) | ((mode == 2) << 2) | (lyc_eq << 3));
    return lcdc;
  }

  // ---- interrupt dispatch (kernels/cpu_step_builder.py:1502-1600) -------------
  int irq_vector(int pending, int* bit) {
    if (pending & 1) { *bit = 1; return 0x40; }
    if (pending & 2) { *bit = 2; return 0x48; }
    if (pending & 4) { *bit = 4; return 0x50; }
    if (pending & 8) { *bit = 8; return 0x58; }
    *bit = 0x10;
    return 0x60;
  }

  void run(int frames_to_run, int release_after);
};

// kernels/cpu_step_builder.py:875-1781 with the templates of
// kernels/cpu_templates/ alu, bitops, jumps, loads, stack, misc spliced in
// through the opcode table of core/isa_sm83.py.
void Env::run(int frames_to_run, int release_after) {
  release = release_after;
  int32_t pc = S(REF_PC) & 0xFFFF, sp = S(REF_SP) & 0xFFFF;
  int32_t a = S(REF_A) & 0xFF, b = S(REF_B) & 0xFF, c = S(REF_C) & 0xFF;
  int32_t d = S(REF_D) & 0xFF, e = S(REF_E) & 0xFF, h = S(REF_H) & 0xFF;
  int32_t l = S(REF_L) & 0xFF, f = S(REF_F) & 0xF0;
  int64_t instr = m.instr_count[i];
  const int64_t instr_start = instr;
  int watch_val = m.dbg_watch ? M(m.dbg_watch) : 0;
  int64_t cyc = m.cycle_count[i];
  int32_t cframe = S(REF_CYCLE_IN_FRAME);
  int32_t trap = S(REF_TRAP_FLAG), trap_pc = S(REF_TRAP_PC);
  int32_t trap_op = S(REF_TRAP_OPCODE), trap_kind = S(REF_TRAP_KIND);
  int32_t scan = S(REF_PPU_SCANLINE_CYCLE), ly = S(REF_PPU_LY);
  int32_t wl = S(REF_PPU_WINDOW_LINE);
  int32_t* R[8] = {&b, &c, &d, &e, &h, &l, nullptr, &a};
  frames_done = 0;

  auto set_trap = [&](int tpc, int top, int kind) {
    if (trap == 0) {
      trap = 1;
      trap_pc = tpc & 0xFFFF;
      trap_op = top & 0xFF;
      trap_kind = kind;
    }
  };
  auto push16 = [&](int value) {
    sp = (sp - 1) & 0xFFFF;
    write8(sp, (value >> 8) & 0xFF);
    sp = (sp - 1) & 0xFFFF;
    write8(sp, value & 0xFF);
  };
  auto pop16 = [&]() {
    int lo = read8(sp);
    sp = (sp + 1) & 0xFFFF;
    int hi = read8(sp);
    sp = (sp + 1) & 0xFFFF;
    return ((hi << 8) | lo) & 0xFFFF;
  };
  auto service = [&](int pending) {
    S(REF_IME) = 0;
    int bit;
    int vec = irq_vector(pending, &bit);
    M(0xFF0F) = (uint8_t)(M(0xFF0F) & (0xFF ^ bit));
    push16(pc & 0xFFFF);
    pc = vec;
    timer_tick(20);
  };

  while (frames_done < frames_to_run) {
    if (trap != 0) break;
    int lcdc_prev = M(0xFF40) & 0x80;
    int lcdc;
    if (S(REF_HALTED) != 0) {
      // HALT tick: kernels/cpu_step_builder.py:976-1300
      const int cycles = 4;
      timer_tick(cycles);
      lcdc = ppu_advance(cycles, scan, ly, wl);
      int pending = M(0xFFFF) & M(0xFF0F) & 0x1F;
      int svc = 0;
      if (pending) {
        S(REF_HALTED) = 0;
        if (S(REF_IME) != 0) {
          service(pending);
          svc = 20;
        } else {
          pc = (pc + 1) & 0xFFFF;  // IME=0 wake skips one byte
        }
      }
      if (svc) lcdc = ppu_advance(svc, scan, ly, wl);
      int total = cycles + svc;
      rtc_tick(total);
      cyc += total;
      cframe += total;
      if (lcdc_prev != 0 && (lcdc & 0x80) == 0) {
        cframe = 0;
        if (++frames_done >= frames_to_run) break;
        continue;
      }
      while (cframe >= CYCLES_PER_FRAME) {
        cframe -= CYCLES_PER_FRAME;
        if (++frames_done >= frames_to_run) break;
      }
      continue;
    }

    const int pc_before = pc;
    const int op = read8(pc);
    if (m.dbg_trap_pc != 0 && pc == m.dbg_trap_pc) {
      set_trap(pc, op, 5);
      break;
    }
    if (m.dbg_rst38 != 0 && op == 0xFF && pc != 0x0038) {
      set_trap(pc, op, 3);
      break;
    }
    int cycles = 0;
    if (op == 0xCB) {
      // CB table: bitops.py templates; pc advanced by the skeleton
      const int cb = read8((pc + 1) & 0xFFFF);
      pc = (pc + 2) & 0xFFFF;
      const int ridx = cb & 7;
      const int hl = ((h << 8) | l) & 0xFFFF;
      int val = ridx == 6 ? read8(hl) : *R[ridx];
      const int group = cb >> 6, sub = (cb >> 3) & 7;
      const int carry_in = (f >> 4) & 1;
      bool store = true;
      if (group == 0) {
        int cf = 0;
        switch (sub) {
          case 0: cf = (val >> 7) & 1; val = ((val << 1) & 0xFF) | cf; break;    // RLC
          case 1: cf = val & 1; val = ((val >> 1) & 0xFF) | (cf << 7); break;    // RRC
          case 2: cf = (val >> 7) & 1; val = ((val << 1) & 0xFF) | carry_in; break;  // RL
          case 3: cf = val & 1; val = ((val >> 1) & 0xFF) | (carry_in << 7); break;  // RR
          case 4: cf = (val >> 7) & 1; val = (val << 1) & 0xFF; break;           // SLA
          case 5: cf = val & 1; val = ((val >> 1) & 0x7F) | (val & 0x80); break; // SRA
          case 6: cf = 0; val = ((val & 0x0F) << 4) | ((val & 0xF0) >> 4); break;  // SWAP
          default: cf = val & 1; val = (val >> 1) & 0x7F; break;                 // SRL
        }
        f = make_flags(val == 0, 0, 0, cf);
        cycles = ridx == 6 ? 16 : 8;
      } else if (group == 1) {  // BIT
        f = make_flags(((val >> sub) & 1) == 0, 0, 1, carry_in);
        store = false;
        cycles = ridx == 6 ? 12 : 8;
      } else if (group == 2) {  // RES
        val = val & (0xFF ^ (1 << sub));
        cycles = ridx == 6 ? 16 : 8;
      } else {  // SET
        val = val | (1 << sub);
        cycles = ridx == 6 ? 16 : 8;
      }
      if (store) {
        if (ridx == 6) write8(hl, val);
        else *R[ridx] = val;
      }
    } else {
      auto rd_imm = [&](int k) { return read8((pc + k) & 0xFFFF); };
      auto hlv = [&]() { return ((h << 8) | l) & 0xFFFF; };
      auto set_hl = [&](int v) { h = (v >> 8) & 0xFF; l = v & 0xFF; };
      auto alu = [&](int kind, int v) {
        const int carry = (f >> 4) & 1;
        switch (kind) {
          case 0: {  // ADD  (alu.py template_add_a_*)
            int s = a + v;
            f = make_flags((s & 0xFF) == 0, 0, ((a & 0xF) + (v & 0xF)) > 0xF, s > 0xFF);
            a = s & 0xFF;
          } break;
          case 1: {  // ADC
            int s = a + v + carry;
            f = make_flags((s & 0xFF) == 0, 0, ((a & 0xF) + (v & 0xF) + carry) > 0xF, s > 0xFF);
            a = s & 0xFF;
          } break;
          case 2: {  // SUB
            int s = a - v;
            f = make_flags((s & 0xFF) == 0, 1, ((a & 0xF) - (v & 0xF)) < 0, a < v);
            a = s & 0xFF;
          } break;
          case 3: {  // SBC
            int s = a - v - carry;
            f = make_flags((s & 0xFF) == 0, 1, ((a & 0xF) - ((v & 0xF) + carry)) < 0,
                           a < (v + carry));
            a = s & 0xFF;
          } break;
          case 4: a = (a & v) & 0xFF; f = make_flags(a == 0, 0, 1, 0); break;  // AND
          case 5: a = (a ^ v) & 0xFF; f = make_flags(a == 0, 0, 0, 0); break;  // XOR
          case 6: a = (a | v) & 0xFF; f = make_flags(a == 0, 0, 0, 0); break;  // OR
          default: {  // CP
            int s = a - v;
            f = make_flags((s & 0xFF) == 0, 1, ((a & 0xF) - (v & 0xF)) < 0, a < v);
          } break;
        }
      };
      auto cond = [&](int cc) {  // NZ, Z, NC, C
        int z = (f >> 7) & 1, cf = (f >> 4) & 1;
        switch (cc) {
          case 0: return z == 0;
          case 1: return z != 0;
          case 2: return cf == 0;
          default: return cf != 0;
        }
      };
      auto rr_get = [&](int idx) {
        switch (idx) {
          case 0: return ((b << 8) | c) & 0xFFFF;
          case 1: return ((d << 8) | e) & 0xFFFF;
          case 2: return ((h << 8) | l) & 0xFFFF;
          default: return (int)sp;
        }
      };
      auto rr_set = [&](int idx, int v) {
        v &= 0xFFFF;
        switch (idx) {
          case 0: b = v >> 8; c = v & 0xFF; break;
          case 1: d = v >> 8; e = v & 0xFF; break;
          case 2: h = v >> 8; l = v & 0xFF; break;
          default: sp = v; break;
        }
      };

      if (op >= 0x40 && op < 0x80 && op != 0x76) {
        // LD r,r / LD r,(HL) / LD (HL),r  (loads.py:34-60)
        const int dst = (op >> 3) & 7, src = op & 7;
        if (dst == 6) {
          write8(hlv(), *R[src]);
          cycles = 8;
        } else if (src == 6) {
          *R[dst] = read8(hlv());
          cycles = 8;
        } else {
          *R[dst] = *R[src] & 0xFF;
          cycles = 4;
        }
        pc = (pc + 1) & 0xFFFF;
      } else if (op >= 0x80 && op < 0xC0) {
        // ALU A,r / A,(HL)  (alu.py)
        const int src = op & 7;
        const int v = src == 6 ? read8(hlv()) : *R[src];
        alu((op >> 3) & 7, v);
        pc = (pc + 1) & 0xFFFF;
        cycles = src == 6 ? 8 : 4;
      } else {
        switch (op) {
          case 0x00: pc = (pc + 1) & 0xFFFF; cycles = 4; break;  // NOP
          case 0x01: case 0x11: case 0x21: case 0x31: {  // LD rr,d16
            int lo = rd_imm(1), hi = rd_imm(2);
            rr_set(op >> 4, (hi << 8) | lo);
            pc = (pc + 3) & 0xFFFF;
            cycles = 12;
          } break;
          case 0x02: write8(rr_get(0), a); pc = (pc + 1) & 0xFFFF; cycles = 8; break;
          case 0x12: write8(rr_get(1), a); pc = (pc + 1) & 0xFFFF; cycles = 8; break;
          case 0x22: case 0x32: {  // LDI/LDD (HL),A
            int hl = hlv();
            write8(hl, a);
            set_hl(op == 0x22 ? hl + 1 : hl - 1);
            pc = (pc + 1) & 0xFFFF;
            cycles = 8;
          } break;
          case 0x0A: a = read8(rr_get(0)); pc = (pc + 1) & 0xFFFF; cycles = 8; break;
          case 0x1A: a = read8(rr_get(1)); pc = (pc + 1) & 0xFFFF; cycles = 8; break;
          case 0x2A: case 0x3A: {  // LDI/LDD A,(HL)
            int hl = hlv();
            a = read8(hl);
            set_hl(op == 0x2A ? hl + 1 : hl - 1);
            pc = (pc + 1) & 0xFFFF;
            cycles = 8;
          } break;
          case 0x03: case 0x13: case 0x23: case 0x33:  // INC rr
            rr_set(op >> 4, rr_get(op >> 4) + 1); pc = (pc + 1) & 0xFFFF; cycles = 8; break;
          case 0x0B: case 0x1B: case 0x2B: case 0x3B:  // DEC rr
            rr_set(op >> 4, rr_get(op >> 4) - 1); pc = (pc + 1) & 0xFFFF; cycles = 8; break;
          case 0x04: case 0x0C: case 0x14: case 0x1C: case 0x24: case 0x2C: case 0x3C:
          case 0x34: {  // INC r / INC (HL)  (alu.py:13-22, 913-934)
            int ridx = (op >> 3) & 7;
            int hl = hlv();
            int old = ridx == 6 ? read8(hl) : *R[ridx];
            int v = (old + 1) & 0xFF;
            if (ridx == 6) write8(hl, v); else *R[ridx] = v;
            f = make_flags(v == 0, 0, (old & 0xF) == 0xF, (f >> 4) & 1);
            pc = (pc + 1) & 0xFFFF;
            cycles = ridx == 6 ? 12 : 4;
          } break;
          case 0x05: case 0x0D: case 0x15: case 0x1D: case 0x25: case 0x2D: case 0x3D:
          case 0x35: {  // DEC r / DEC (HL)
            int ridx = (op >> 3) & 7;
            int hl = hlv();
            int old = ridx == 6 ? read8(hl) : *R[ridx];
            int v = (old - 1) & 0xFF;
            if (ridx == 6) write8(hl, v); else *R[ridx] = v;
            f = make_flags(v == 0, 1, (old & 0xF) == 0, (f >> 4) & 1);
            pc = (pc + 1) & 0xFFFF;
            cycles = ridx == 6 ? 12 : 4;
          } break;
          case 0x06: case 0x0E: case 0x16: case 0x1E: case 0x26: case 0x2E: case 0x3E:
            *R[(op >> 3) & 7] = rd_imm(1); pc = (pc + 2) & 0xFFFF; cycles = 8; break;
          case 0x36: {  // LD (HL),d8
            int v = rd_imm(1);
            write8(hlv(), v);
            pc = (pc + 2) & 0xFFFF;
            cycles = 12;
          } break;
          case 0x07: {  // RLCA
            int cf = (a >> 7) & 1;
            a = ((a << 1) & 0xFF) | cf;
            f = make_flags(0, 0, 0, cf);
            pc = (pc + 1) & 0xFFFF; cycles = 4;
          } break;
          case 0x0F: {  // RRCA
            int cf = a & 1;
            a = ((a >> 1) & 0xFF) | (cf << 7);
            f = make_flags(0, 0, 0, cf);
            pc = (pc + 1) & 0xFFFF; cycles = 4;
          } break;
          case 0x17: {  // RLA
            int old = (f >> 4) & 1, cf = (a >> 7) & 1;
            a = ((a << 1) & 0xFF) | old;
            f = make_flags(0, 0, 0, cf);
            pc = (pc + 1) & 0xFFFF; cycles = 4;
          } break;
          case 0x1F: {  // RRA
            int old = (f >> 4) & 1, cf = a & 1;
            a = ((a >> 1) & 0xFF) | (old << 7);
            f = make_flags(0, 0, 0, cf);
            pc = (pc + 1) & 0xFFFF; cycles = 4;
          } break;
          case 0x08: {  // LD (a16),SP
            int lo = rd_imm(1), hi = rd_imm(2);
            int addr = ((hi << 8) | lo) & 0xFFFF;
            write8(addr, sp & 0xFF);
            write8((addr + 1) & 0xFFFF, (sp >> 8) & 0xFF);
            pc = (pc + 3) & 0xFFFF; cycles = 20;
          } break;
          case 0x09: case 0x19: case 0x29: case 0x39: {  // ADD HL,rr (alu.py:72-111)
            int hl = hlv(), rr = rr_get(op >> 4);
            int s = hl + rr;
            int z = (f >> 7) & 1;
            h = (s >> 8) & 0xFF;
            l = s & 0xFF;
            f = make_flags(z, 0, ((hl & 0xFFF) + (rr & 0xFFF)) > 0xFFF, s > 0xFFFF);
            pc = (pc + 1) & 0xFFFF; cycles = 8;
          } break;
          case 0x18: {  // JR
            int off = sign8(rd_imm(1));
            pc = (pc + 2 + off) & 0xFFFF; cycles = 12;
          } break;
          case 0x20: case 0x28: case 0x30: case 0x38: {  // JR cc
            int off = sign8(rd_imm(1));
            bool take = cond((op >> 3) & 3);
            pc = take ? (pc + 2 + off) & 0xFFFF : (pc + 2) & 0xFFFF;
            cycles = take ? 12 : 8;
          } break;
          case 0x27: {  // DAA (alu.py:897-922)
            int av = a & 0xFF, nf = (f >> 6) & 1, hf = (f >> 5) & 1, cf = (f >> 4) & 1;
            int adj = 0, carry = cf;
            if (nf == 0) {
              if (hf || (av & 0xF) > 9) adj |= 0x06;
              if (cf || av > 0x99) { adj |= 0x60; carry = 1; }
              av = (av + adj) & 0xFF;
            } else {
              if (hf) adj |= 0x06;
              if (cf) adj |= 0x60;
              av = (av - adj) & 0xFF;
            }
            f = make_flags(av == 0, nf, 0, carry);
            a = av;
            pc = (pc + 1) & 0xFFFF; cycles = 4;
          } break;
          case 0x2F:  // CPL
            a = a ^ 0xFF;
            f = make_flags((f >> 7) & 1, 1, 1, (f >> 4) & 1);
            pc = (pc + 1) & 0xFFFF; cycles = 4; break;
          case 0x37:  // SCF
            f = make_flags((f >> 7) & 1, 0, 0, 1);
            pc = (pc + 1) & 0xFFFF; cycles = 4; break;
          case 0x3F:  // CCF
            f = make_flags((f >> 7) & 1, 0, 0, ((f >> 4) & 1) ? 0 : 1);
            pc = (pc + 1) & 0xFFFF; cycles = 4; break;
          case 0x76:  // HALT (misc.py:29-33)
            S(REF_HALTED) = 1;
            pc = (pc + 1) & 0xFFFF; cycles = 4; break;
          case 0xC6: case 0xCE: case 0xD6: case 0xDE: case 0xE6: case 0xEE: case 0xF6:
          case 0xFE:  // ALU A,d8
            alu((op >> 3) & 7, rd_imm(1));
            pc = (pc + 2) & 0xFFFF; cycles = 8; break;
          case 0xC0: case 0xC8: case 0xD0: case 0xD8:  // RET cc (stack.py)
            if (cond((op >> 3) & 3)) { pc = pop16(); cycles = 20; }
            else { pc = (pc + 1) & 0xFFFF; cycles = 8; }
            break;
          case 0xC9: pc = pop16(); cycles = 16; break;  // RET
          case 0xD9:  // RETI
            pc = pop16();
            S(REF_IME) = 1;
            S(REF_IME_DELAY) = 0;
            cycles = 16; break;
          case 0xC1: case 0xD1: case 0xE1: {  // POP rr
            int v = pop16();
            rr_set((op >> 4) & 3, v);
            pc = (pc + 1) & 0xFFFF; cycles = 12;
          } break;
          case 0xF1: {  // POP AF
            int v = pop16();
            a = (v >> 8) & 0xFF;
            f = v & 0xF0;
            pc = (pc + 1) & 0xFFFF; cycles = 12;
          } break;
          case 0xC5: case 0xD5: case 0xE5:  // PUSH rr
            push16(rr_get((op >> 4) & 3));
            pc = (pc + 1) & 0xFFFF; cycles = 16; break;
          case 0xF5:  // PUSH AF
            push16((a << 8) | (f & 0xF0));
            pc = (pc + 1) & 0xFFFF; cycles = 16; break;
          case 0xC3: {  // JP
            int lo = rd_imm(1), hi = rd_imm(2);
            pc = ((hi << 8) | lo) & 0xFFFF; cycles = 16;
          } break;
          case 0xC2: case 0xCA: case 0xD2: case 0xDA: {  // JP cc
            int lo = rd_imm(1), hi = rd_imm(2);
            bool take = cond((op >> 3) & 3);
            pc = take ? ((hi << 8) | lo) & 0xFFFF : (pc + 3) & 0xFFFF;
            cycles = take ? 16 : 12;
          } break;
          case 0xE9: pc = hlv(); cycles = 4; break;  // JP (HL)
          case 0xCD: {  // CALL
            int lo = rd_imm(1), hi = rd_imm(2);
            push16((pc + 3) & 0xFFFF);
            pc = ((hi << 8) | lo) & 0xFFFF; cycles = 24;
          } break;
          case 0xC4: case 0xCC: case 0xD4: case 0xDC:  // CALL cc
            if (cond((op >> 3) & 3)) {
              int lo = rd_imm(1), hi = rd_imm(2);
              push16((pc + 3) & 0xFFFF);
              pc = ((hi << 8) | lo) & 0xFFFF; cycles = 24;
            } else {
              pc = (pc + 3) & 0xFFFF; cycles = 12;
            }
            break;
          case 0xC7: case 0xCF: case 0xD7: case 0xDF: case 0xE7: case 0xEF: case 0xF7:
          case 0xFF:  // RST
            push16((pc + 1) & 0xFFFF);
            pc = op & 0x38; cycles = 16; break;
          case 0xE0: {  // LDH (a8),A
            int off = rd_imm(1);
            write8(0xFF00 | off, a);
            pc = (pc + 2) & 0xFFFF; cycles = 12;
          } break;
          case 0xF0: {  // LDH A,(a8)
            int off = rd_imm(1);
            a = read8(0xFF00 | off);
            pc = (pc + 2) & 0xFFFF; cycles = 12;
          } break;
          case 0xE2: write8(0xFF00 | c, a); pc = (pc + 1) & 0xFFFF; cycles = 8; break;
          case 0xF2: a = read8(0xFF00 | c); pc = (pc + 1) & 0xFFFF; cycles = 8; break;
          case 0xE8: case 0xF8: {  // ADD SP,e8 / LD HL,SP+e8 (alu.py:114-177)
            int off = rd_imm(1);
            int off_s = sign8(off), off_u = off & 0xFF;
            int hf = ((sp & 0xF) + (off_u & 0xF)) > 0xF;
            int cf = ((sp & 0xFF) + off_u) > 0xFF;
            int res = (sp + off_s) & 0xFFFF;
            if (op == 0xE8) { sp = res; cycles = 16; }
            else { h = (res >> 8) & 0xFF; l = res & 0xFF; cycles = 12; }
            f = make_flags(0, 0, hf, cf);
            pc = (pc + 2) & 0xFFFF;
          } break;
          case 0xF9: sp = hlv(); pc = (pc + 1) & 0xFFFF; cycles = 8; break;  // LD SP,HL
          case 0xEA: {  // LD (a16),A
            int lo = rd_imm(1), hi = rd_imm(2);
            write8(((hi << 8) | lo) & 0xFFFF, a);
            pc = (pc + 3) & 0xFFFF; cycles = 16;
          } break;
          case 0xFA: {  // LD A,(a16)
            int lo = rd_imm(1), hi = rd_imm(2);
            a = read8(((hi << 8) | lo) & 0xFFFF);
            pc = (pc + 3) & 0xFFFF; cycles = 16;
          } break;
          case 0xF3: S(REF_IME) = 0; S(REF_IME_DELAY) = 0; pc = (pc + 1) & 0xFFFF; cycles = 4; break;
          case 0xFB: S(REF_IME) = 1; S(REF_IME_DELAY) = 0; pc = (pc + 1) & 0xFFFF; cycles = 4; break;
          default:  // STOP, 0xCB handled above, illegal: misc.py:42-56
            set_trap(pc, op, 1);
            cycles = 0;
            break;
        }
      }
    }
    if (m.dbg_rst38 != 0 && pc >= 0xFE00) {
      set_trap(pc_before, op, 4);
      break;
    }
    if (trap != 0) break;

    f &= 0xF0;
    instr += 1;
    if (m.dbg_max_instr > 0 && instr - instr_start >= m.dbg_max_instr) {
      set_trap(pc, op, 6);
      break;
    }
    if (m.dbg_watch != 0 && M(m.dbg_watch) != watch_val) {
      set_trap(pc_before, op, 7);
      break;
    }
    timer_tick(cycles);
    if (S(REF_IME_DELAY) != 0) {
      S(REF_IME) = 1;
      S(REF_IME_DELAY) = 0;
    }
    lcdc = ppu_advance(cycles, scan, ly, wl);
    int pending = M(0xFFFF) & M(0xFF0F) & 0x1F;
    int svc = 0;
    if (pending) {
      if (S(REF_HALTED) != 0) S(REF_HALTED) = 0;
      if (S(REF_IME) != 0) {
        service(pending);
        svc = 20;
        lcdc = ppu_advance(svc, scan, ly, wl);
      }
    }
    int total = cycles + svc;
    rtc_tick(total);
    cyc += total;
    cframe += total;
    if (lcdc_prev != 0 && (lcdc & 0x80) == 0) {
      int tail = total;
      if (op == 0xE0) {
        int imm = read8((pc_before + 1) & 0xFFFF);
        if ((imm & 0xFF) == 0x40 && cycles >= 4) tail = total - 4;
      }
      cframe = tail;
      if (++frames_done >= frames_to_run) break;
      continue;
    } else if (lcdc_prev == 0 && (lcdc & 0x80) != 0) {
      scan = 0;
      ly = 0;
      wl = 0;
      M(0xFF44) = 0;
      ppu_update_stat(0, 2);
      int lyc0 = M(0xFF45) == 0 ? 1 : 0;
      stat_prev = (uint8_t)((1 << 2) | (lyc0 << 3));
      cframe = 0;
      if (++frames_done >= frames_to_run) break;
      continue;
    } else {
      while (cframe >= CYCLES_PER_FRAME) {
        cframe -= CYCLES_PER_FRAME;
        if (++frames_done >= frames_to_run) break;
      }
    }
  }

  S(REF_PC) = pc & 0xFFFF;
  S(REF_SP) = sp & 0xFFFF;
  S(REF_A) = a & 0xFF;
  S(REF_B) = b & 0xFF;
  S(REF_C) = c & 0xFF;
  S(REF_D) = d & 0xFF;
  S(REF_E) = e & 0xFF;
  S(REF_H) = h & 0xFF;
  S(REF_L) = l & 0xFF;
  S(REF_F) = f & 0xF0;
  m.instr_count[i] = instr;
  m.cycle_count[i] = cyc;
  S(REF_CYCLE_IN_FRAME) = cframe;
  S(REF_PPU_SCANLINE_CYCLE) = scan;
  S(REF_PPU_LY) = ly;
  S(REF_PPU_WINDOW_LINE) = wl;
  S(REF_TRAP_FLAG) = trap;
  S(REF_TRAP_PC) = trap_pc;
  S(REF_TRAP_OPCODE) = trap_op;
  S(REF_TRAP_KIND) = trap_kind;
}

// kernels/cpu_templates/post_step.py:11-102 (obs_v0 / reward_v0)
void write_post_step(RefMachine& m, int i, int stage) {
  const uint8_t* mem = &m.mem[(int64_t)i * MEM_SIZE];
  const int pc = m.s32[REF_PC][i], sp = m.s32[REF_SP][i];
  const int a = m.s32[REF_A][i], b = m.s32[REF_B][i], c = m.s32[REF_C][i];
  const int d = m.s32[REF_D][i], e = m.s32[REF_E][i], h = m.s32[REF_H][i];
  const int l = m.s32[REF_L][i], f = m.s32[REF_F][i];
  const bool want_obs = stage == 2 || stage == 3;
  const bool want_reward = stage == 1 || stage == 3;
  int mm[16];
  for (int k = 0; k < 16; ++k) mm[k] = mem[0xC000 + k];
  if (want_obs) {
    float* o = &m.obs[(int64_t)i * m.obs_dim];
    o[0] = (float)(pc & 0xFFFF) / 65535.0f;
    o[1] = (float)(sp & 0xFFFF) / 65535.0f;
    const int rv[8] = {a, f, b, c, d, e, h, l};
    for (int k = 0; k < 8; ++k) o[2 + k] = (float)(rv[k] & 0xFF) / 255.0f;
    for (int k = 0; k < 16; ++k) o[10 + k] = (float)mm[k] / 255.0f;
    const int mix[6] = {(mm[0] ^ mm[1]) & 0xFF,       (mm[2] + mm[3] * 5) & 0xFF,
                        (mm[4] ^ (a & 0xFF)) & 0xFF,  (mm[5] + (b & 0xFF)) & 0xFF,
                        (mm[6] ^ (c & 0xFF)) & 0xFF,  (mm[7] + (d & 0xFF)) & 0xFF};
    for (int k = 0; k < 6; ++k) o[26 + k] = (float)mix[k] / 255.0f;
  }
  if (want_reward) {
    int mix = (mm[0] + mm[1] * 3) & 0xFF;
    m.reward[i] = (float)((a ^ mix) & 0xFF) / 255.0f;
  }
}

// Registers one shade lookup reads.  The snapshot renderer takes them from
// the IO page at render time; the env-0 frame renderer from the per-line
// latches captured during the step.
struct LineRegs {
  int lcdc, scx, scy, bgp, wx, wy, obp0, obp1;
  int win_row;  // window tile-row line: y - WY (snapshot) or the latched window line
};

// Shade of pixel (x, y): background/window then sprites
// (kernels/ppu_render_downsampled.py:27-179; kernels/ppu_step.py:12-171 is
// the same rule with latched registers).
int shade_at(const uint8_t* mem, int x, int y, const LineRegs& r) {
  const int lcdc = r.lcdc, scy = r.scy, scx = r.scx, bgp = r.bgp;
  const int obp0 = r.obp0, obp1 = r.obp1, wy = r.wy, wx = r.wx;
  int shade = 0, bg_color = 0;
  auto tile_row = [&](int tile_id, int row, bool unsigned_data) {
    int addr;
    if (unsigned_data) addr = 0x8000 + tile_id * 16;
    else addr = 0x9000 + (tile_id >= 128 ? tile_id - 256 : tile_id) * 16;
    return addr + row * 2;
  };
  if (lcdc & 0x01) {
    bool use_window = (lcdc & 0x20) && y >= wy && x >= wx - 7;
    int map, px, py;
    if (use_window) {
      px = x - (wx - 7);
      py = r.win_row;
      map = (lcdc & 0x40) ? 0x9C00 : 0x9800;
      px &= 0xFF;
      py &= 0xFF;
    } else {
      px = (x + scx) & 0xFF;
      py = (y + scy) & 0xFF;
      map = (lcdc & 0x08) ? 0x9C00 : 0x9800;
    }
    int tile_id = mem[map + (py >> 3) * 32 + (px >> 3)];
    int ra = tile_row(tile_id, py & 7, (lcdc & 0x10) != 0);
    int lo = mem[ra], hi = mem[ra + 1];
    int bit = 7 - (px & 7);
    bg_color = (((hi >> bit) & 1) << 1) | ((lo >> bit) & 1);
    shade = (bgp >> (bg_color * 2)) & 3;
  }
  if (lcdc & 0x02) {
    const int height = (lcdc & 0x04) ? 16 : 8;
    int on_line = 0, found = 0, best_x = 0, best_oam = 0, best_color = 0, best_attr = 0;
    for (int s = 0; s < 40; ++s) {
      const uint8_t* o = mem + 0xFE00 + s * 4;
      int sy = o[0], sx = o[1], tile = o[2], attr = o[3];
      if (sx == 0 || sy == 0 || sx >= 168 || sy >= 160) continue;
      int top = sy - 16, left = sx - 8;
      if (y < top || y >= top + height) continue;
      if (on_line >= 10) continue;
      ++on_line;
      if (x < left || x >= left + 8) continue;
      int row = y - top;
      if ((attr >> 6) & 1) row = height - 1 - row;
      if (height == 16) {
        tile &= 0xFE;
        if (row >= 8) { tile += 1; row -= 8; }
      }
      int ra = 0x8000 + tile * 16 + row * 2;
      int lo = mem[ra], hi = mem[ra + 1];
      int pxl = x - left;
      int bit = ((attr >> 5) & 1) ? pxl : 7 - pxl;
      int color = (((hi >> bit) & 1) << 1) | ((lo >> bit) & 1);
      if (color == 0) continue;
      if (!found) {
        found = 1; best_x = left; best_oam = s; best_color = color; best_attr = attr;
      } else if (left < best_x) {
        best_x = left; best_oam = s; best_color = color; best_attr = attr;
      } else if (left == best_x && s < best_oam) {
        best_oam = s; best_color = color; best_attr = attr;
      }
    }
    if (found) {
      int prio = (best_attr >> 7) & 1;
      if (!(prio && bg_color != 0)) {
        int pal = ((best_attr >> 4) & 1) ? obp1 : obp0;
        shade = (pal >> (best_color * 2)) & 3;
      }
    }
  }
  return shade;
}

// kernels/ppu_render_downsampled.py:27-179: registers from the IO page
int sample_shade(const uint8_t* mem, int x, int y) {
  LineRegs r;
  r.lcdc = mem[0xFF40];
  r.scy = mem[0xFF42];
  r.scx = mem[0xFF43];
  r.bgp = mem[0xFF47];
  r.obp0 = mem[0xFF48];
  r.obp1 = mem[0xFF49];
  r.wy = mem[0xFF4A];
  r.wx = mem[0xFF4B];
  r.win_row = y - r.wy;
  return shade_at(mem, x, y, r);
}

}  // namespace

extern "C" {

RefMachine* ref_create(int num_envs, const uint8_t* rom, int64_t rom_len,
                       const uint8_t* boot, int boot_len, int obs_dim) {
  if (num_envs <= 0 || !rom || rom_len < 0x150 || !boot || boot_len != BOOTROM_SIZE)
    return nullptr;
  // Header: core/cartridge.py:139-187
  int type = rom[0x147], rom_code = rom[0x148], ram_code = rom[0x149];
  int64_t rom_bytes;
  switch (rom_code) {
    case 0x00: case 0x01: case 0x02: case 0x03: case 0x04: case 0x05: case 0x06:
    case 0x07: case 0x08: rom_bytes = (int64_t)(32 * 1024) << rom_code; break;
    default: return nullptr;
  }
  static const int ram_map[6] = {0, 2048, 8192, 32768, 131072, 65536};
  if (ram_code > 5) return nullptr;
  int ram_bytes = ram_map[ram_code];
  int kind;
  if (type == 0x00) kind = MBC_ROM_ONLY;
  else if (type >= 0x01 && type <= 0x03) kind = MBC_MBC1;
  else if (type >= 0x0F && type <= 0x13) kind = MBC_MBC3;
  else return nullptr;
  if (rom_len < rom_bytes) return nullptr;
  auto* m = new RefMachine();
  m->n = num_envs;
  m->obs_dim = obs_dim;
  m->rom.assign(rom, rom + rom_bytes);
  m->boot.assign(boot, boot + BOOTROM_SIZE);
  m->rom_bank_count = (int)(rom_bytes / ROM_BANK_SIZE);
  m->rom_bank_mask =
      (m->rom_bank_count & (m->rom_bank_count - 1)) == 0 ? m->rom_bank_count - 1 : -1;
  m->ram_bytes = ram_bytes;
  m->ram_bank_count = ram_bytes / RAM_BANK_SIZE;
  m->ram_stride = ram_bytes > 0 ? ram_bytes : 1;
  m->mbc_kind = kind;
  ref_reset(m);
  return m;
}

void ref_destroy(RefMachine* m) { delete m; }
int ref_num_envs(RefMachine* m) { return m ? m->n : 0; }

int ref_set_debug(RefMachine* m, int rst38, int trap_pc, int max_instr, int watch_addr) {
  if (!m) return -1;
  m->dbg_rst38 = rst38 ? 1 : 0;
  m->dbg_trap_pc = trap_pc & 0xFFFF;
  m->dbg_max_instr = max_instr > 0 ? max_instr : 0;
  m->dbg_watch = watch_addr & 0xFFFF;
  return 0;
}

// backends/warp_vec.py:249-513
int ref_reset(RefMachine* m) {
  if (!m) return -1;
  const int n = m->n;
  m->mem.assign((size_t)n * MEM_SIZE, 0);
  for (int i = 0; i < n; ++i)
    memcpy(&m->mem[(size_t)i * MEM_SIZE], m->boot.data(), BOOTROM_SIZE);
  m->cart_ram.assign((size_t)n * m->ram_stride, 0);
  m->serial_buf.assign((size_t)n * SERIAL_MAX, 0);
  m->cart_state.assign((size_t)n * CS_STRIDE, 0);
  for (int i = 0; i < n; ++i) {
    int32_t* cs = &m->cart_state[(size_t)i * CS_STRIDE];
    cs[CS_MBC_KIND] = m->mbc_kind;
    cs[CS_ROM_BANK_LO] = 1;
    cs[CS_BOOTROM_ENABLED] = 1;
  }
  for (int f = 0; f < REF_NUM_SCALAR_FIELDS; ++f) m->s32[f].assign(n, 0);
  m->instr_count.assign(n, 0);
  m->cycle_count.assign(n, 0);
  m->data_bytes.assign(n, 0);
  m->joyp_select.assign(n, 0x30);
  m->serial_overflow.assign(n, 0);
  m->ppu_stat_prev.assign(n, 0);
  memset(m->latches, 0, sizeof(m->latches));
  m->obs.assign((size_t)n * m->obs_dim, 0.0f);
  m->reward.assign(n, 0.0f);
  m->pix.assign((size_t)n * DS_W * DS_H, 0);
  m->pix_packed.assign((size_t)n * DS_WB * DS_H, 0);
  m->snap_valid = false;
  return 0;
}

int ref_step(RefMachine* m, const int32_t* actions, int frames_to_run,
             int release_after_frames, int stage, int env_lo, int env_hi,
             int nthreads) {
  if (!m) return -1;
  if (env_lo < 0) env_lo = 0;
  if (env_hi > m->n || env_hi < 0) env_hi = m->n;
  if (actions)
    for (int i = env_lo; i < env_hi; ++i) m->s32[REF_ACTIONS][i] = actions[i];
#ifdef _OPENMP
  if (nthreads <= 0) nthreads = 1;
#pragma omp parallel for schedule(dynamic, 4) num_threads(nthreads)
#endif
  for (int i = env_lo; i < env_hi; ++i) {
    Env env(*m, i, &m->mem[(size_t)i * MEM_SIZE], &m->cart_state[(size_t)i * CS_STRIDE]);
    env.run(frames_to_run, release_after_frames);
    env.store();
    if (stage != 0) write_post_step(*m, i, stage);
  }
  return 0;
}

int ref_render(RefMachine* m, int packed, int nthreads) {
  if (!m) return -1;
#ifdef _OPENMP
  if (nthreads <= 0) nthreads = 1;
#pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
  for (int i = 0; i < m->n; ++i) {
    const uint8_t* mem = &m->mem[(size_t)i * MEM_SIZE];
    for (int oy = 0; oy < DS_H; ++oy) {
      if (packed) {
        for (int ob = 0; ob < DS_WB; ++ob) {
          int v = 0;
          for (int k = 0; k < 4; ++k) v |= (sample_shade(mem, (ob * 4 + k) * 2, oy * 2) & 3) << (2 * k);
          m->pix_packed[(size_t)i * DS_WB * DS_H + oy * DS_WB + ob] = (uint8_t)v;
        }
      } else {
        for (int ox = 0; ox < DS_W; ++ox)
          m->pix[(size_t)i * DS_W * DS_H + oy * DS_W + ox] =
              (uint8_t)sample_shade(mem, ox * 2, oy * 2);
      }
    }
  }
  return 0;
}

// kernels/ppu_step.py:12-176: env 0's full 160x144 frame from the per-line
// latches (LCDC, SCX, SCY, BGP, WX, WY, window line, OBP0, OBP1) and the
// current VRAM/OAM of env 0.
int ref_render_bg_env0(RefMachine* m, uint8_t* out) {
  if (!m || !out || m->n <= 0) return -1;
  const uint8_t* mem = &m->mem[0];
  for (int y = 0; y < SCREEN_H; ++y) {
    LineRegs r;
    r.lcdc = m->latches[0][y];
    r.scx = m->latches[1][y];
    r.scy = m->latches[2][y];
    r.bgp = m->latches[3][y];
    r.wx = m->latches[4][y];
    r.wy = m->latches[5][y];
    r.win_row = m->latches[6][y];
    r.obp0 = m->latches[7][y];
    r.obp1 = m->latches[8][y];
    for (int x = 0; x < 160; ++x) out[y * 160 + x] = (uint8_t)shade_at(mem, x, y, r);
  }
  return 0;
}

// core/reset_cache.py:68-190 (snapshot of one env)
int ref_snapshot_ex(RefMachine* m, int env, int with_pix) {
  if (!m || env < 0 || env >= m->n) return -1;
  m->snap_mem.assign(m->mem.begin() + (size_t)env * MEM_SIZE,
                     m->mem.begin() + (size_t)(env + 1) * MEM_SIZE);
  m->snap_cart_ram.assign(m->cart_ram.begin() + (size_t)env * m->ram_stride,
                          m->cart_ram.begin() + (size_t)(env + 1) * m->ram_stride);
  m->snap_serial.assign(m->serial_buf.begin() + (size_t)env * SERIAL_MAX,
                        m->serial_buf.begin() + (size_t)(env + 1) * SERIAL_MAX);
  m->snap_has_pix = with_pix != 0;
  if (m->snap_has_pix)
    m->snap_pix.assign(m->pix.begin() + (size_t)env * DS_W * DS_H,
                       m->pix.begin() + (size_t)(env + 1) * DS_W * DS_H);
  memcpy(m->snap_cart_state, &m->cart_state[(size_t)env * CS_STRIDE], sizeof(m->snap_cart_state));
  for (int f = 0; f < REF_NUM_SCALAR_FIELDS; ++f) m->snap_scalar[f] = get_scalar(*m, f, env);
  m->snap_valid = true;
  return 0;
}
int ref_snapshot(RefMachine* m, int env) { return ref_snapshot_ex(m, env, 0); }

// core/reset_cache.py:192-307 (masked restore; packed pixels and env-0
// latches are not part of the snapshot)
int ref_masked_reset(RefMachine* m, const uint8_t* mask) {
  if (!m || !m->snap_valid || !mask) return -1;
  for (int i = 0; i < m->n; ++i) {
    if (!mask[i]) continue;
    memcpy(&m->mem[(size_t)i * MEM_SIZE], m->snap_mem.data(), MEM_SIZE);
    memcpy(&m->cart_ram[(size_t)i * m->ram_stride], m->snap_cart_ram.data(), m->ram_stride);
    memcpy(&m->serial_buf[(size_t)i * SERIAL_MAX], m->snap_serial.data(), SERIAL_MAX);
    if (m->snap_has_pix)
      memcpy(&m->pix[(size_t)i * DS_W * DS_H], m->snap_pix.data(), DS_W * DS_H);
    memcpy(&m->cart_state[(size_t)i * CS_STRIDE], m->snap_cart_state, sizeof(m->snap_cart_state));
    for (int f = 0; f < REF_NUM_SCALAR_FIELDS; ++f) set_scalar(*m, f, i, m->snap_scalar[f]);
  }
  return 0;
}

void* ref_field_ptr(RefMachine* m, int field, int64_t* nbytes, int* elem_size) {
  if (!m) return nullptr;
  auto ret = [&](void* p, int64_t nb, int es) {
    if (nbytes) *nbytes = nb;
    if (elem_size) *elem_size = es;
    return p;
  };
  const int64_t n = m->n;
  switch (field) {
    case REF_INSTR_COUNT: return ret(m->instr_count.data(), n * 8, 8);
    case REF_CYCLE_COUNT: return ret(m->cycle_count.data(), n * 8, 8);
    case REF_JOYP_SELECT: return ret(m->joyp_select.data(), n, 1);
    case REF_SERIAL_OVERFLOW: return ret(m->serial_overflow.data(), n, 1);
    case REF_PPU_STAT_PREV: return ret(m->ppu_stat_prev.data(), n, 1);
    case REF_MEM: return ret(m->mem.data(), n * MEM_SIZE, 1);
    case REF_CART_STATE: return ret(m->cart_state.data(), n * CS_STRIDE * 4, 4);
    case REF_CART_RAM: return ret(m->cart_ram.data(), n * m->ram_stride, 1);
    case REF_SERIAL_BUF: return ret(m->serial_buf.data(), n * SERIAL_MAX, 1);
    case REF_OBS: return ret(m->obs.data(), n * m->obs_dim * 4, 4);
    case REF_REWARD: return ret(m->reward.data(), n * 4, 4);
    case REF_LATCHES: return ret(m->latches, sizeof(m->latches), 1);
    case REF_PIX: return ret(m->pix.data(), n * DS_W * DS_H, 1);
    case REF_PIX_PACKED: return ret(m->pix_packed.data(), n * DS_WB * DS_H, 1);
    case REF_DATA_BYTES: return ret(m->data_bytes.data(), n * 8, 8);
    default:
      if (field >= 0 && field < REF_NUM_SCALAR_FIELDS) return ret(m->s32[field].data(), n * 4, 4);
      return nullptr;
  }
}

}  // extern "C"

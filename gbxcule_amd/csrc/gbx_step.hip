// gbx_step.hip -- the SM83 step kernel for gfx950: one lane per Game Boy.
//
// Semantics are those of the reference's Warp kernel cpu_step
// (src/gbxcule/kernels/cpu_step_builder.py:875-1781 with the opcode bodies of
// kernels/cpu_templates/ and the opcode table core/isa_sm83.py), bit for bit,
// including its documented quirks (EI takes effect at once, IME=0 HALT wake
// skips a byte, OAM DMA reads raw memory, JOYP recomputed only on FF00 writes,
// STAT IRQ edges evaluated at line changes, LCD toggles count as frames).
//
// The implementation is not a translation of that kernel.  A wavefront runs
// up to 64 independent instruction streams, so the loop body is built to
// cost the same whatever mix of opcodes its lanes execute:
//  * fetch + decode is four 16-byte loads of the pre-decoded 64-byte record
//    of the instruction at pc (gbx_decode.h), issued for the next pc while
//    the current instruction's writes, timer and PPU work run;
//  * execute is one straight-line datapath (gbx_exec.h) whose operands are
//    byte permutes of the register file and the bus bytes selected by the
//    record, with one shared adder, logic unit, shifter and 16-bit adder, so
//    no lane waits for another lane's opcode class;
//  * bus reads compute one address per lane (ROM window, boot image,
//    cartridge RAM or the env's memory) and every lane loads its byte, with
//    no branch around the load; only a second byte, IO side effects, MBC and
//    cartridge-RAM writes take divergent branches;
//  * CPU registers, the hot IO registers and the cartridge bank offsets live
//    in VGPRs for the whole launch and are written back once;
//  * a step that reaches no event (timer, scanline, frame end, pending
//    request) takes a fast tail that only advances DIV, the scanline
//    position and the cycle counters; scanline changes that raise no
//    request and TIMA edges short of an overflow are run through without
//    being applied, and are settled before anything observes them (LY,
//    STAT, TIMA and DIV reads derive their values instead);
//  * a halted CPU, an LY poll loop and a block-copy loop advance in one step
//    to the first event the reference's per-instruction loop could observe
//    (ff_horizon), which is exactly equivalent to stepping them one
//    instruction (or 4 halted cycles) at a time;
//  * the rare paths carry branch-probability hints, and those of the
//    per-instruction path a wave-uniform ballot test, so that the common
//    path is laid out as straight fall-through code that keeps its exec
//    mask.
#include "gbx_internal.h"
// after gbx_internal.h, which brings in the HIP runtime
#include "gbx_exec.h"

namespace gbx {
namespace {

constexpr int kCyclesPerFrame = 70224;
constexpr int kCyclesPerLine = 456;
constexpr int kLinesPerFrame = 154;
constexpr int kRtcCyclesPerSecond = 4194304;

// Decode of instructions fetched outside the pre-decoded images (code in
// RAM, the last two bytes of a ROM window): [op] or [256 + CB byte].
struct DecTable {
  Rec e[512];
};
constexpr DecTable make_dec_table() {
  DecTable t{};
  for (uint32_t i = 0; i < 512; ++i) t.e[i] = decode_base(i);
  return t;
}
__constant__ DecTable kDec = make_dec_table();

// ---------------------------------------------------------------------------
// Buffer-resource access for the fixed-address state of a 64-env block: a
// wave-uniform descriptor (SGPRs) plus a per-lane offset; constant addresses
// go into the scalar offset so no VGPR is spent per address.
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
  // byte-to-byte copy through memory (also replaces the implicit member-wise
  // copy assignment, which would only copy the proxy)
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

__device__ __forceinline__ uint32_t sel(bool c, uint32_t a, uint32_t b) { return c ? a : b; }
// c ? a : b for two computed addresses, marked unpredictable: left to
// itself the compiler may turn such a select into a branch around the
// computation of one address, which then sits in front of the load.
__device__ __forceinline__ const uint8_t* sel_ptr(bool c, const uint8_t* a, const uint8_t* b) {
  return __builtin_unpredictable(c) ? a : b;
}
// Lane q's value of v, unsigned (the builtin returns int, which would
// sign-extend when widened).
__device__ __forceinline__ uint32_t lane_value(uint32_t v, uint32_t q) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, (int)q);
}

// Launch-uniform values that the loop only uses in per-lane arithmetic (flat
// base addresses, sizes, limits) are held in VGPRs: the loop body already
// keeps SGPRs busy with buffer descriptors and nested exec masks, and an
// SGPR-held copy would be spilled and reloaded every iteration.
__device__ __forceinline__ uint32_t in_vgpr(uint32_t v) {
  uint32_t r;
  asm("v_mov_b32 %0, %1" : "=v"(r) : "r"(v));
  return r;
}
template <typename T>
__device__ __forceinline__ T* in_vgpr(T* p) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  return reinterpret_cast<T*>(((uint64_t)in_vgpr((uint32_t)(a >> 32)) << 32) | in_vgpr((uint32_t)a));
}

// Loads through flat pointers that are known to be device (global) memory,
// issued as global loads: the compiler then counts them exactly in vmcnt and
// can wait for one load while later ones stay in flight (a flat load could
// also be an LDS access, so waits on flat loads drain every load).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
template <typename T>
__device__ __forceinline__ T ld_global(const T* p) {
  return *(const __attribute__((address_space(1))) T*)p;
}
__device__ __forceinline__ void st_global(const uint8_t* p, uint32_t v) {
  *(__attribute__((address_space(1))) uint8_t*)const_cast<uint8_t*>(p) = (uint8_t)v;
}

// ---------------------------------------------------------------------------
// Per-lane machine.  Everything here is scalarized into VGPRs.
// ---------------------------------------------------------------------------
struct Lane {
  const DevState& s;
  int mbc;        // cartridge kind; a compile-time constant of each kernel variant
  bool cram;      // the cart declares RAM; compile-time too (false: ram_ok never holds)
  uint32_t e;     // env index
  uint32_t lane;  // e % 64: position inside the 64-env block
  rsrc_t rm, rsc, rcs;             // memory image, scalars, cartridge state of the block
  const uint8_t* memb;             // memory image of the block (flat)
  const uint8_t* cramb;            // cartridge RAM of the block (flat)
  const uint8_t* rom;              // ROM buffer (flat)
  uint32_t rom_len;

  // CPU: w0 = B C D E (B in bits 31-24), w1 = H L F A (A in bits 7-0)
  uint32_t pc, sp, w0, w1;
  uint32_t ime, ime_delay, halted;
  // hot IO registers (byte values); FF04 and the STAT mode/coincidence bits
  // are derived from the timer and PPU position (ff04_val, stat_val)
  uint32_t tima, tma, tac, ifr, ie, lcdc, lym, lyc, wy;
  uint32_t stat_full;   // STAT as last written (low 3 bits valid while stat_fresh)
  uint32_t stat_fresh;  // STAT written (or launch start) since the last PPU step
  // timer
  uint32_t div, pend, delay;
  uint32_t tmask;       // no TIMA edge while (div & tmask) + cycles <= tmask
  // DIV when TIMA was last brought up to date: the fast path may run through
  // TIMA edges short of an overflow without applying them (settle_timer)
  uint32_t tdiv;
  uint32_t tp_w;        // DIV or TAC written this launch
  uint32_t ff04_0, tprev0;  // FF04 and timer_prev_in as loaded
  // PPU
  uint32_t scan, ly, wl;
  uint32_t sp0;         // ppu_stat_prev as loaded (until the first PPU step)
  uint32_t lyc_pp;      // LYC at the last PPU step
  uint32_t lcd_pp;      // LCDC bit 7 at the last PPU step; 0x100 before the first
  // Set when the fast path may run through quiet scanline changes (those
  // that raise no request) without applying them: scan then exceeds a line
  // (settle_lines).  Never for env 0, whose latches need every line, nor in
  // the debug variants.
  uint32_t defer;
  uint32_t defer_timer;  // the same for TIMA edges (any env; not in debug variants)
  // cartridge
  uint32_t boot_en;
  uint32_t rom_lo, rom_hi;  // byte offset of the 0000 / 4000 windows in the ROM buffer
  // MBC registers as the step uses them, packed into one word (the
  // cartridge state keeps each value as written): ROM bank bits 0-6, upper
  // bank bits 8-9, banking mode bit 10, RAM enable bit 11, RTC select bits
  // 12-15, RAM bank bits 16-17, RTC latch bit 18.
  uint32_t mbr;
  uint32_t ram_ok;
  int rtc_field;       // 0..4 when an RTC register is mapped at A000
  // The byte the bus reads at A000 (cart_p) and the mask of the row offset
  // of an A000-BFFF address (cart_m): ~0 while a RAM bank is mapped; 0 while
  // an RTC register is (every address reads the low byte of its cartridge
  // state slot) or nothing is (every address reads a byte of the 0xFF filler
  // that follows the boot image in the ROM buffer, which is what disabled or
  // absent cartridge RAM returns).
  const uint8_t* cart_p;
  uint32_t cart_m;
  int rtc_sub;
  uint32_t rtc_halt, rtc_dirty;
  uint32_t map_changed;  // set when a write remaps the fetch windows
  // Cycles a step may take on the fast path (event_budget).  Every event the
  // fast path must not pass sets it to 0: IO and RTC writes with side
  // effects, traps, EI, RETI and HALT with a request pending; the slow path
  // recomputes it.
  int budget;
  // frame loop
  int frames_done, release;
  int32_t action;
  // JOYP: the select bits last written, and the FF00 value for each select
  // (bytes 0-3 for select 0x00, 0x10, 0x20, 0x30), which changes only when
  // the frame count passes the release frame
  uint32_t joyp_sel, joyp_word;

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

  // -- register file (w0 = B C D E, w1 = H L F A) -------------------------------
  __device__ uint32_t a() const { return w1 & 0xFFu; }
  __device__ uint32_t f() const { return (w1 >> 8) & 0xF0u; }

  // -- cartridge windows (reference read8 ROM/RAM branches, :565-656) ----------
  __device__ static int clamp_bank(int bank, int count, int mask) {
    if (count <= 0) return 0;
    if (mask >= 0) return bank & mask;
    return bank % count;
  }
  static constexpr uint32_t kMbrEn = 1u << 11, kMbrLatch = 1u << 18;
  // mbr from the cartridge state slots, masked as the bus uses them
  __device__ uint32_t load_mbr() const {
    uint32_t m = CS(CS_RAM_ENABLE) != 0 ? kMbrEn : 0u;
    if (mbc != MBC_ROM_ONLY) {
      m |= ((uint32_t)CS(CS_ROM_BANK_LO) & 0x7Fu) | (((uint32_t)CS(CS_ROM_BANK_HI) & 3u) << 8) |
           (((uint32_t)CS(CS_BANK_MODE) & 1u) << 10) | (((uint32_t)CS(CS_RAM_BANK) & 3u) << 16);
      if (mbc == MBC_MBC3)
        m |= (((uint32_t)CS(CS_RTC_SELECT) & 0xFu) << 12) | (CS(CS_RTC_LATCH) != 0 ? kMbrLatch : 0u);
    }
    return m;
  }
  __device__ void refresh_cart() {
    const int kind = mbc;
    const int lo_raw = (int)(mbr & 0x7Fu);
    const int lo = lo_raw & 0x1F, hi = (int)((mbr >> 8) & 3u);
    const int mode = (int)((mbr >> 10) & 1u);
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
    // an unmapped bank reads the 0xFF filler that follows the boot image
    const uint32_t open = rom_len + 0x100u;
    rom_lo = ((int64_t)b0 * 0x4000 < lim) ? (uint32_t)b0 * 0x4000u : open;
    rom_hi = ((int64_t)b1 * 0x4000 < lim) ? (uint32_t)b1 * 0x4000u : open;
    // (a runtime value even where cram rules RAM out: folded to a constant
    // it changed the compiler's schedule of the bus read, 1.7% slower)
    ram_ok = ((s.ram_banks > 0) & ((mbr & kMbrEn) != 0u)) ? 1u : 0u;
    rtc_field = -1;
    if (kind == MBC_MBC3) {
      const int sl = (int)((mbr >> 12) & 0xFu);
      if (sl >= 0x08 && sl <= 0x0C) rtc_field = sl - 0x08;
    }
    int rb = 0;
    if (kind == MBC_MBC1) {
      if (mode) rb = (int)((mbr >> 16) & 3u);
    } else if (kind == MBC_MBC3) {
      rb = (int)((mbr >> 16) & 3u);
    }
    rb = clamp_bank(rb, s.ram_banks, -1);
    const size_t blk = e >> kEnvBlockShift;
    const uint8_t* cb = cramb;
    // nothing mapped: a byte of the 0xFF filler after the boot image
    cart_p = rom + (rom_len + 0x100u);
    cart_m = 0u;
    if (ram_ok && rtc_field >= 0) {
      const uint32_t slot = (uint32_t)(((mbr & kMbrLatch) ? CS_RTC_L_SECONDS : CS_RTC_SECONDS) + rtc_field);
      cart_p = reinterpret_cast<const uint8_t*>(s.cs + blk * (kCartStateStride * kEnvBlock)) +
               (((slot << kEnvBlockShift) | lane) << 2);
    } else if (ram_ok) {
      cart_p = cb + ((((uint32_t)rb * 0x2000u) << kEnvBlockShift) | lane);
      cart_m = ~0u;
    }
  }

  // -- bus read (reference read8, cpu_step_builder.py:538-657) ----------------
  // Every IO register the core keeps in a VGPR is also stored to memory when
  // it changes, so the bus reads memory for all of FF00-FFFF except FF04 and
  // the STAT mode/coincidence bits, which follow from the DIV counter and the
  // PPU position.
  __device__ uint32_t io_fix(uint32_t x, uint32_t v) const {
    v = x == 0xFF04u ? ff04_val() : v;
    return x == 0xFF41u ? stat_val() : v;
  }
  __device__ static bool io_derived(uint32_t x) { return (x & 0xFFBAu) == 0xFF00u; }
  // Flat address of the byte the bus returns at x (echo-folded): ROM window,
  // boot image, or the 0xFF filler for an unmapped bank; cartridge RAM, the
  // mapped RTC register, or the 0xFF filler for disabled or absent cartridge
  // RAM; or the env's memory.
  __device__ const uint8_t* bus_ptr(uint32_t x) const {
    const bool rom = x < 0x8000u;
    const bool cart = x - 0xA000u < 0x2000u;
    // bitwise conditions throughout the per-instruction path: each is a
    // select, never a branch
    const bool bootw = (boot_en != 0u) & (x < 0x100u);
    const uint32_t win = (x < 0x4000u ? rom_lo : rom_hi) + (x & 0x3FFFu);
    const uint32_t roff = win + ((rom_len + x - win) & (0u - (uint32_t)bootw));
    // (a cart without RAM never maps any)
    const uint8_t* cp = cram ? cart_p + (((x - 0xA000u) << kEnvBlockShift) & cart_m) : this->rom + (rom_len + 0x100u);
    const uint8_t* p = memb + ((x << kEnvBlockShift) | lane);
    p = cart ? cp : p;
    return sel_ptr(rom, this->rom + roff, p);
  }
  __device__ static uint32_t fold(uint32_t addr) {
    const uint32_t x = addr & 0xFFFFu;
    return x - 0xE000u < 0x1E00u ? x - 0x2000u : x;
  }
  // Value the bus returned for a load v issued at bus_ptr(x).  (Disabled or
  // absent cartridge RAM needs no fix-up: bus_ptr points it at 0xFF.)
  __device__ uint32_t bus_fix(uint32_t x, uint32_t v) const {
    // DIV and STAT, which follow from the timer and PPU position, and TIMA and
    // LY while edges and scanline changes are deferred (FF05 and FF44 hold
    // the values of the last applied ones): FF04 FF05 FF40 FF41 FF44 FF45
    const bool fx = ((x & 0xFFBAu) == 0xFF00u) & (x > 0xFF01u);
    if (__builtin_expect(__ballot(fx) != 0u, 0)) v = fx ? read_ppu(x, v) : v;
    return v;
  }
  __device__ uint32_t read8(uint32_t addr) const {
    const uint32_t x = fold(addr);
    return bus_fix(x, ld_global(bus_ptr(x)));
  }
  __device__ void set_if(uint32_t v) {
    ifr = v;
    M(0xFF0F) = v;
  }

  // -- timer (cpu_step_builder.py:249-372) -------------------------------------
  // TAC select 0..3 -> DIV bit 9, 3, 5, 7 (one nibble each)
  __device__ static uint32_t div_bit(uint32_t t) { return (0x7539u >> ((t & 3u) << 2)) & 0xFu; }
  // x mod 154 for x < 308 (a line number plus fewer than 154 changes)
  __device__ static uint32_t wrap_line(uint32_t x) {
    return x >= (uint32_t)kLinesPerFrame ? x - (uint32_t)kLinesPerFrame : x;
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
  __device__ static uint32_t edge_mask(uint32_t t) {
    return (t & 4u) ? (2u << div_bit(t)) - 1u : 0x7FFFFFFFu;
  }
  // FF04 and timer_prev_in as the reference holds them: derived from the DIV
  // counter once it has ticked or been written this launch.
  __device__ bool timer_live() const { return lcd_pp != 0x100u || tp_w != 0u; }
  __device__ uint32_t ff04_val() const { return timer_live() ? (div >> 8) & 0xFFu : ff04_0; }
  __device__ uint32_t tprev_val() const { return timer_live() ? timer_in(div, tac) : tprev0; }
  __device__ void timer_tick(int cycles) {
    if (cycles <= 0) return;
    uint32_t d = div & 0xFFFFu;
    bool done = false;
    if ((pend == 0u) & ((d & tmask) + (uint32_t)cycles <= tmask)) {
      d = (d + (uint32_t)cycles) & 0xFFFFu;  // no edge, no reload: DIV only
      done = true;
    } else if (pend == 0u) {
      // n falling edges of the selected DIV bit and no overflow: TIMA += n
      const uint32_t n = ((d & tmask) + (uint32_t)cycles) >> (div_bit(tac) + 1u);
      if (tima + n <= 0xFFu) {
        tima += n;
        d = (d + (uint32_t)cycles) & 0xFFFFu;
        M(0xFF05) = tima;
        done = true;
      }
    }
    if (!done) {
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
      M(0xFF05) = tima;
      M(0xFF0F) = ifr;
    }
    div = d;
    // TIMA holds every edge up to here, so a settle later in the same step
    // (an IO write by an interrupt's push) counts none of them again
    tdiv = d;
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
    if (cycles <= 0 || mbc != MBC_MBC3 || rtc_halt) return;
    if (rtc_sub < 0) rtc_sub = 0;
    rtc_sub += cycles;
    if (rtc_sub >= kRtcCyclesPerSecond || rtc_dirty) rtc_slow();
  }

  // -- JOYP (cpu_step_builder.py:195-247) ----------------------------------------
  __device__ void joyp_refresh() {
    joyp_word = joyp_value(0x00u) | (joyp_value(0x10u) << 8) | (joyp_value(0x20u) << 16) |
                (joyp_value(0x30u) << 24);
  }
  __device__ uint32_t joyp_read(uint32_t sl) const { return ubfe(joyp_word, (sl & 0x30u) >> 1, 8); }
  __device__ uint32_t joyp_value(uint32_t sl) const {
    const bool pressed = frames_done < release;
    uint32_t dpad = 0, btn = 0;
    if (pressed) {
      dpad = action == 4 ? 4u : action == 5 ? 8u : action == 6 ? 2u : action == 7 ? 1u : 0u;
      btn = action == 1 ? 1u : action == 2 ? 2u : action == 3 ? 8u : 0u;
    }
    const uint32_t p14 = (sl >> 4) & 1u, p15 = (sl >> 5) & 1u;
    uint32_t v = (sl | 0xCFu) & 0xFFu;
    if (p14 && p15) v = 0x0Fu;
    else if (!p14 && !p15) {
    } else if (!p14) v &= 0x0Fu & ~dpad;
    else v &= 0x0Fu & ~btn;
    return v | 0xC0u;
  }

  // -- bus write (reference write8, cpu_step_builder.py:659-873) ----------------
  // IO bytes with side effects or a VGPR copy: FF02 04-07 0F 40 41 44 45 46
  // 4A 50 and FFFF.  FF00 (JOYP) is a plain store of the joypad value for the
  // written select bits; every other address below FF80 outside ROM and
  // cartridge RAM is a plain store.
  __device__ static bool io_special(uint32_t x) {
    const uint32_t k = x & 0xFFu;
    const uint32_t m = k < 32u ? 0x80F4u : (k - 64u < 32u ? 0x10473u : 0u);
    return (x >= 0xFF00u) & ((k == 0xFFu) | (((m >> (k & 31u)) & 1u) != 0u));
  }
  __device__ void io_write(uint32_t x, uint32_t v) {
    settle();  // the write follows every change and edge the fast path deferred
    budget = 0;  // timer, LCD and PPU registers feed event_budget
    const uint32_t k = x & 0xFFu;
    // plain register copies
    tima = sel(k == 0x05u, v, tima);
    tma = sel(k == 0x06u, v, tma);
    ifr = sel(k == 0x0Fu, v & 0x1Fu, ifr);
    ie = sel(k == 0xFFu, v & 0x1Fu, ie);
    lcdc = sel(k == 0x40u, v, lcdc);
    stat_fresh = sel(k == 0x41u, 1u, stat_fresh);
    stat_full = sel(k == 0x41u, v, stat_full);
    lym = sel(k == 0x44u, v, lym);
    lyc = sel(k == 0x45u, v, lyc);
    wy = sel(k == 0x4Au, v, wy);
    // memory keeps the value the register holds after the write
    uint32_t mv = v;
    mv = sel(k == 0x0Fu, ifr, mv);
    mv = sel(k == 0xFFu, ie, mv);
    mv = sel(k == 0x07u, v & 7u, mv);
    if (k - 0x05u < 3u || k == 0x0Fu || k == 0x40u || k == 0x44u || k == 0x45u || k == 0x4Au ||
        k == 0xFFu)
      M(x) = mv;
    switch (k) {
      case 0x00:
        joyp_sel = v & 0x30u;
        M(0xFF00) = joyp_read(v);
        break;
      case 0x02:
        if ((v & 0x80u) && (v & 0x01u)) {
          const int idx = SC(F_SERIAL_LEN);
          if (idx < kSerialMax) {
            s.serial[(size_t)e * kSerialMax + idx] = (uint8_t)(uint32_t)M(0xFF01);
            SC(F_SERIAL_LEN) = idx + 1;
          } else {
            SC(F_SERIAL_OVERFLOW) = 1;
          }
          M(0xFF02) = v & 0x7Fu;
          set_if(ifr | 0x08u);
        } else {
          M(0xFF02) = v;
        }
        break;
      case 0x50:
        if (v != 0 && boot_en) {
          boot_en = 0;
          CS(CS_BOOTROM_ENABLED) = 0;
          map_changed = 1;
        }
        break;
      case 0x04: {
        const uint32_t pre = timer_in(div, tac);
        div = 0;
        tp_w = 1;
        if (pre && !timer_in(0, tac)) tima_inc();
        M(0xFF05) = tima;
      } break;
      case 0x07: {
        const uint32_t pre = timer_in(div, tac);
        tac = v & 7u;
        tmask = edge_mask(tac);
        tp_w = 1;
        if (pre && !timer_in(div, tac)) tima_inc();
        M(0xFF05) = tima;
      } break;
      case 0x46: {
        M(0xFF46) = v;
        // 160 bytes, 4 loads in flight, then their stores.  Only a source
        // page of FE overlaps the destination, and then batch b reads bytes
        // FE00 + 4b .. that no earlier batch wrote, as the reference's
        // byte-by-byte loop does.
        const uint32_t src = v << 8;
#pragma unroll 1
        for (uint32_t j0 = 0; j0 < 160; j0 += 4) {
          uint32_t b[4];
#pragma unroll
          for (uint32_t t = 0; t < 4; ++t) b[t] = M((src + j0 + t) & 0xFFFFu);
#pragma unroll
          for (uint32_t t = 0; t < 4; ++t) {
            const uint32_t sa = (src + j0 + t) & 0xFFFFu;
            M(0xFE00u + j0 + t) = io_derived(sa) ? io_fix(sa, b[t]) : b[t];
          }
        }
      } break;
      default:
        break;
    }
    tdiv = div;  // a DIV or TAC write starts the count afresh
  }
  // The slots a write changes are stored as the reference stores them, and
  // mbr follows, so that refresh_cart reads no memory.
  __device__ void mbc_write(uint32_t x, uint32_t v) {
    const int kind = mbc;
    if (kind == MBC_ROM_ONLY) return;
    const uint32_t lo_bits = kind == MBC_MBC1 ? 0x1Fu : 0x7Fu;
    if (x < 0x2000u) {
      const uint32_t en = (v & 0x0Fu) == 0x0Au ? 1u : 0u;
      CS(CS_RAM_ENABLE) = (int)en;
      mbr = (mbr & ~kMbrEn) | (en << 11);
    } else if (x < 0x4000u) {
      const uint32_t b = (v & lo_bits) ? (v & lo_bits) : 1u;
      CS(CS_ROM_BANK_LO) = (int)b;
      mbr = (mbr & ~0x7Fu) | b;
    } else if (kind == MBC_MBC1) {
      if (x < 0x6000u) {
        const uint32_t h = v & 3u;
        CS(CS_ROM_BANK_HI) = (int)h;
        CS(CS_RAM_BANK) = (int)h;
        mbr = (mbr & ~0x30300u) | (h << 8) | (h << 16);
      } else {
        CS(CS_BANK_MODE) = (int)(v & 1u);
        mbr = (mbr & ~(1u << 10)) | ((v & 1u) << 10);
      }
    } else if (x < 0x6000u) {
      const uint32_t sl = v & 0x0Fu;
      CS(CS_RTC_SELECT) = (int)sl;
      mbr = (mbr & ~0xF000u) | (sl << 12);
      if (sl <= 3u) {
        CS(CS_RAM_BANK) = (int)sl;
        mbr = (mbr & ~0x30000u) | (sl << 16);
      }
    } else if (v == 0) {
      CS(CS_RTC_LATCH) = 0;
      mbr &= ~kMbrLatch;
    } else if ((v == 1) & ((mbr & kMbrLatch) == 0u)) {
      int r[5];
      for (int k = 0; k < 5; ++k) r[k] = CS(CS_RTC_SECONDS + k);
      for (int k = 0; k < 5; ++k) CS(CS_RTC_L_SECONDS + k) = r[k];
      CS(CS_RTC_LATCH) = 1;
      mbr |= kMbrLatch;
    }
    const uint32_t lo0 = rom_lo, hi0 = rom_hi;
    refresh_cart();
    // write_bus drops the prefetched record only when a fetch window moved:
    // RAM enable, RAM bank, RTC select and latch writes, and bank writes of
    // the bank already mapped, leave every record index as it was.  (Sticky:
    // the first byte of a two-byte write may move a window the second byte
    // leaves alone.)
    map_changed |= ((rom_lo != lo0) | (rom_hi != hi0)) ? 1u : 0u;
  }
  __device__ void write_special(uint32_t x, uint32_t v) {
    if (x < 0x8000u) {
      mbc_write(x, v);
    } else if (x - 0xA000u < 0x2000u) {
      if (!ram_ok) return;
      if (rtc_field >= 0) {
        CS(CS_RTC_SECONDS + rtc_field) = (int)v;
        rtc_dirty = 1;
        budget = 0;
        if (rtc_field == 4) rtc_halt = (v & 0x40u) ? 1u : 0u;
        return;
      }
      st_global(cart_p + ((x - 0xA000u) << kEnvBlockShift), v);  // a RAM bank is mapped
    } else {
      io_write(x, v);
    }
  }
  // A write that is not a plain store to the env's memory: MBC registers,
  // cartridge RAM, IO bytes with side effects.
  __device__ static bool write_is_special(uint32_t x) {
    // 4 KiB regions 0-7 (MBC registers) and A-B (cartridge RAM); x < 0x10000
    return (((0x0CFFu >> (x >> 12)) & 1u) != 0u) | io_special(x);
  }
  __device__ void write8(uint32_t addr, uint32_t v) {
    const uint32_t x = fold(addr);
    // FF00 stores the joypad read for the written select bits (io_write)
    if (!write_is_special(x) & (x != 0xFF00u)) M(x) = v;
    else write_special(x, v);
  }
  // Addresses a write reaches as a plain byte store without side effects:
  // video RAM, work RAM and high RAM (FF80-FFFE) (plain_ram), and for the
  // first byte of a write also FF00, whose store is the joypad value for the
  // written select bits.  Everything else (ROM/MBC registers, cartridge RAM,
  // echo RAM, OAM, IO registers, IE, and FF00 as a second byte, which only a
  // push or LD (a16),SP next to it makes) goes through write8.  x is a
  // 16-bit address.
  __device__ static bool plain_ram(uint32_t x) {
    return (((0x3300u >> (x >> 12)) & 1u) != 0u) | (x - 0xFF80u < 0x7Fu);
  }
  __device__ static bool plain_store(uint32_t x) { return plain_ram(x) | (x == 0xFF00u); }
  // The instruction's bus writes, in order (n = 0, 1 or 2).  When both are
  // plain stores they are stored without a branch; a lane with one write
  // stores its first byte twice.  An MBC bank write clears rv, the validity
  // of the record already fetched for the next pc (the boot ROM switch is an
  // IO write, after which the full sequence drops the record).
  // With cartridge RAM (cram), a byte of a mapped RAM bank is a plain store
  // too, into the cartridge RAM buffer instead of the env's memory.
  __device__ bool cart_plain(uint32_t x) const { return cram & (x - 0xA000u < 0x2000u) & (cart_m != 0u); }
  __device__ uint8_t* store_ptr(uint32_t x, bool c) const {
    return const_cast<uint8_t*>(c ? cart_p + ((x - 0xA000u) << kEnvBlockShift)
                                  : memb + ((x << kEnvBlockShift) | lane));
  }
  __device__ void write_bus(uint32_t n, uint32_t a0, uint32_t v0, uint32_t a1, uint32_t v1, bool& rv) {
    const uint32_t x0 = a0 & 0xFFFFu, x1 = a1 & 0xFFFFu;
    const bool two = n >= 2u;
    const bool c0 = cart_plain(x0), c1 = cart_plain(x1);
    if (__builtin_expect((!(plain_store(x0) | c0)) | (two & !(plain_ram(x1) | c1)), 0)) {
      write8(a0, v0);
      if (two) write8(a1, v1);
      if (mbc != MBC_ROM_ONLY) {
        rv = rv & (map_changed == 0u);
        map_changed = 0;
      }
    } else {
      const bool j0 = x0 == 0xFF00u;
      const uint32_t s0 = j0 ? joyp_read(v0) : v0;
      joyp_sel = j0 ? v0 & 0x30u : joyp_sel;
      if (!cram) {
        M(x0) = s0;
        M(two ? x1 : x0) = two ? v1 : s0;
      } else {
        uint8_t* p0 = store_ptr(x0, c0);
        st_global(p0, s0);
        st_global(two ? store_ptr(x1, c1) : p0, two ? v1 : s0);
      }
    }
  }

  // -- PPU line bookkeeping (cpu_step_builder.py:421-524, 1406-1500) -----------
  // The registers env 0 latches for line l: LCDC, SCX, SCY, BGP, WX, WY,
  // the window line w, OBP0, OBP1.  `io` holds SCX | SCY << 8 | BGP << 16 |
  // WX << 24 and `obp` OBP0 | OBP1 << 8, as read from memory.
  __device__ void store_latches(uint32_t l, uint32_t w, uint32_t io, uint32_t obp) const {
    store_latch_entry(l, w, lcdc, wy, io, obp);
  }
  __device__ void store_latch_entry(uint32_t l, uint32_t w, uint32_t lc, uint32_t wyv, uint32_t io,
                                    uint32_t obp) const {
    // one 16-byte entry per line: LCDC SCX SCY BGP | WX WY WL OBP0 | OBP1
    const uint4 v = make_uint4((lc & 0xFFu) | (io << 8), (io >> 24) | ((wyv & 0xFFu) << 8) |
                                                             ((w & 0xFFu) << 16) | (obp << 24),
                               (obp >> 8) & 0xFFu, 0u);
    *reinterpret_cast<uint4*>(s.latches + (size_t)l * kLatchStride) = v;
  }
  __device__ uint32_t latch_io() const {
    return (uint32_t)M(0xFF43) | ((uint32_t)M(0xFF42) << 8) | ((uint32_t)M(0xFF47) << 16) |
           ((uint32_t)M(0xFF4B) << 24);
  }
  __device__ uint32_t latch_obp() const { return (uint32_t)M(0xFF48) | ((uint32_t)M(0xFF49) << 8); }
  __device__ void latch_env0() {
    if (e != 0 || ly >= (uint32_t)kScreenH) return;
    store_latches(ly, wl, latch_io(), latch_obp());
  }
  // Env 0's latches for the visible lines entered by a run of m line
  // changes (2 <= m <= 154) from line ly.  The run's registers are fixed (no
  // IO write falls between the lines of one step), so they are read once.
  // Each entry has a closed form: change j enters line l = (ly + j + 1) % 154,
  // once each, and leaves the window line counter at wl plus the lines in
  // [ly, l) below 144 and at or past WY (window on), or at the lines in
  // [0, l) once the run has entered line 0.  So every active lane of env 0's
  // wavefront writes a share of the entries; env 0 is lane 0, whose values
  // the others read.  Called by all active lanes when one of them is env 0.
  __device__ void latch_run_wave(uint32_t m) const {
    const auto rl0 = [](uint32_t x) { return (uint32_t)__builtin_amdgcn_readlane((int)x, 0); };
    const uint32_t io = rl0(latch_io()), obp = rl0(latch_obp());
    const uint32_t m0 = rl0(m), l0 = rl0(ly), w0 = rl0(wl), lc = rl0(lcdc), wy0 = rl0(wy);
    const uint64_t act = __ballot(true);
    const uint32_t rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(act >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)act, 0u));
    const uint32_t nact = (uint32_t)__popcll(act);
    auto counted = [&](uint32_t a, uint32_t b) {
      const int hi = min((int)b, kScreenH), lo = max((int)a, (int)wy0);
      return (lc & 0x20u) && hi > lo ? (uint32_t)(hi - lo) : 0u;
    };
    for (uint32_t j = rank; j < m0; j += nact) {
      const uint32_t t = l0 + j + 1u;  // <= 307
      const bool wrapped = t >= (uint32_t)kLinesPerFrame;
      const uint32_t l = wrapped ? t - (uint32_t)kLinesPerFrame : t;
      const uint32_t w = wrapped ? counted(0u, l) : w0 + counted(l0, l);
      if (l < (uint32_t)kScreenH) store_latch_entry(l, w, lc, wy0, io, obp);
    }
  }
  // STAT mode at scanline cycle sc of line l (LCD on)
  __device__ static uint32_t mode_at(uint32_t l, uint32_t sc) {
    return l >= (uint32_t)kScreenH ? 1u : sc < 80u ? 2u : sc < 250u ? 3u : 0u;
  }
  __device__ uint32_t mode_now(uint32_t sc) const { return mode_at(ly, sc); }
  // The line m changes (m < 154) after line ly.
  __device__ uint32_t line_after(uint32_t m) const {
    const uint32_t l = ly + m;
    return l >= (uint32_t)kLinesPerFrame ? l - (uint32_t)kLinesPerFrame : l;
  }
  // Applies the scanline changes the fast path deferred (scan >= 456).  None
  // of them raises a request (event_budget stops short of every change that
  // can), so they change only LY, the window line and FF44, and applying
  // them together gives what applying them one at a time gives.  Everything
  // that observes the PPU position calls this first, except LY and STAT
  // reads, which derive their values (read_ppu).
  __device__ void settle_lines() {
    if (scan < (uint32_t)kCyclesPerLine) return;
    advance_lines(scan / (uint32_t)kCyclesPerLine);
    M(0xFF44) = lym;
  }
  // TIMA edges the fast path ran through since DIV was tdiv (none overflows:
  // event_budget stops at the overflowing edge), counted as timer_tick
  // counts several edges in one step.
  __device__ uint32_t tima_edges() const {
    const uint32_t c = (div - tdiv) & 0xFFFFu;  // the budget keeps it below 65536
    return (tac & 4u) ? ((tdiv & tmask) + c) >> (div_bit(tac) + 1u) : 0u;
  }
  __device__ void settle_timer() {
    const uint32_t n = tima_edges();
    if (n != 0u) {
      tima += n;
      M(0xFF05) = tima;
    }
    tdiv = div;
  }
  // Deferred scanline changes and TIMA edges, applied before anything that
  // observes them other than the reads read_ppu derives.
  __device__ void settle() {
    settle_lines();
    settle_timer();
  }
  // FF04, FF05, FF40, FF41, FF44 and FF45 as the bus reads them: DIV from
  // the counter, TIMA after the deferred edges, STAT from the PPU position,
  // LY after the deferred changes, the others as stored.
  __device__ uint32_t read_ppu(uint32_t x, uint32_t v) const {
    const uint32_t m = scan / (uint32_t)kCyclesPerLine;
    v = ((x == 0xFF44u) & (m != 0u)) ? line_after(m) : v;
    v = x == 0xFF05u ? tima + tima_edges() : v;
    v = x == 0xFF04u ? ff04_val() : v;
    return x == 0xFF41u ? stat_val() : v;
  }
  __device__ static uint32_t stat_bits(uint32_t mode, uint32_t coin) {
    return (mode == 0 ? 1u : 0u) | (mode == 1 ? 2u : 0u) | (mode == 2 ? 4u : 0u) | (coin << 3);
  }
  // STAT as the reference holds it: every PPU step rewrites the low three
  // bits (coincidence, mode) from the position it ends at, so they are
  // derived here from that position instead of being stored per step.
  __device__ uint32_t stat_val() const {
    if (stat_fresh) return stat_full;
    // the position after any deferred scanline changes
    const uint32_t m = scan / (uint32_t)kCyclesPerLine;
    const uint32_t l = line_after(m), sc = scan - m * (uint32_t)kCyclesPerLine;
    const uint32_t coin = l == lyc_pp ? 1u : 0u;
    return (stat_full & 0xF8u) | (coin << 2) | (lcd_pp ? mode_at(l, sc) : 0u);
  }
  // ppu_stat_prev as the reference holds it after the last PPU step that
  // ended at scanline cycle sc.
  __device__ uint32_t stat_prev_at(uint32_t sc) const {
    if (lcd_pp == 0x100u) return sp0;
    if (!lcd_pp) return 0u;
    return stat_bits(mode_now(sc), ly == lyc_pp ? 1u : 0u);
  }
  // Line change(s) after scan reached 456; s0 = scanline cycle before the step.
  // The reference applies each change in turn (cpu_step_builder.py:1436-
  // 1480).  A run of m >= 2 changes, the batched steps of a halted CPU, an LY
  // poll or a block copy, is applied in closed form (ppu_lines_run), after
  // env 0 has recorded the run's scanline latches (latch_run_wave).
  __device__ void ppu_lines(uint32_t s0) {
    uint32_t prev = stat_prev_at(s0);
    // (the run test is one compare; C2-like code never takes it)
    if (__builtin_expect(scan >= 2u * (uint32_t)kCyclesPerLine, 0)) {
      const uint32_t m = scan / (uint32_t)kCyclesPerLine;
      if (__builtin_expect(__ballot(e == 0u) != 0u, 0)) latch_run_wave(m);
      ppu_lines_run(m, prev);
    } else {
      const uint32_t lc = lcdc;
      uint32_t total = scan;
      while (total >= (uint32_t)kCyclesPerLine) {
        total -= kCyclesPerLine;
        const uint32_t pl = ly;
        wl += (uint32_t)((pl < (uint32_t)kScreenH) & ((lc & 0x20u) != 0u) & (pl >= wy));
        ly = wrap_line(ly + 1u);
        wl = ly == 0u ? 0u : wl;
        lym = ly;
        // ppu_update_stat_irq with mode 0 or 1: bit0 mode 0, bit1 mode 1, bit3 LY == LYC
        const uint32_t vb = ly >= (uint32_t)kScreenH ? 1u : 0u;
        const uint32_t cur = (1u << vb) | ((ly == lyc ? 1u : 0u) << 3);
        const uint32_t en = (stat_full >> 3) & 0xFu;  // bit0 mode0, 1 mode1, 2 mode2, 3 lyc
        ifr |= (uint32_t)((en & cur & ~(prev & 0xFu)) != 0u) << 1;
        prev = cur;
        ifr |= (uint32_t)((pl == 143u) & (ly == 144u));
        if ((e == 0u) & (ly < (uint32_t)kScreenH)) latch_env0();
      }
      scan = total;
    }
    M(0xFF44) = lym;
    M(0xFF0F) = ifr;
  }
  // m line changes (2 <= m <= 154) from line ly < 154, with LCDC, STAT, LYC
  // and WY fixed over the run.  Change j enters line l_j = (ly + j) % 154
  // having left l_{j-1}; line t is entered at change j_t = (t - ly - 1) % 154
  // + 1, once, so it is entered in the run iff j_t <= m.  Then:
  //  * the window line counter counts the lines left below 144 and at or
  //    past WY (LCDC bit 5), restarting at 0 when line 0 is entered;
  //  * VBlank is requested iff line 144 is entered (always from line 143);
  //  * a STAT request is raised iff the first change shows an enabled bit
  //    that prev (the bits before the run) lacks, or a later change enters
  //    line 144 (mode-1 source: the line before is below 144), line 0
  //    (mode-0 source: the line before is 153) or line LYC (LYC source:
  //    neighbouring lines differ).  The mode-2 bit is never current at a
  //    change.
  __device__ void ppu_lines_run(uint32_t m, uint32_t prev) {
    const uint32_t nl = (uint32_t)kLinesPerFrame;
    auto entered_at = [&](uint32_t t) {  // j_t for t < 154
      const uint32_t x = t + (nl - 1u) - ly;  // 0 .. 306
      return (x >= nl ? x - nl : x) + 1u;
    };
    const uint32_t en = (stat_full >> 3) & 0xFu;
    const uint32_t l1 = ly + 1u == nl ? 0u : ly + 1u;
    const uint32_t cur1 = (1u << (l1 >= (uint32_t)kScreenH ? 1u : 0u)) | ((l1 == lyc ? 1u : 0u) << 3);
    const uint32_t j144 = entered_at(144u), j0 = entered_at(0u);
    const uint32_t jl = lyc < nl ? entered_at(lyc) : 0xFFFFu;
    const bool stat = ((en & cur1 & ~(prev & 0xFu)) != 0u) | (((en & 2u) != 0u) & (j144 >= 2u) & (j144 <= m)) |
                      (((en & 1u) != 0u) & (j0 >= 2u) & (j0 <= m)) |
                      (((en & 8u) != 0u) & (jl >= 2u) & (jl <= m));
    ifr |= ((uint32_t)stat << 1) | (uint32_t)(j144 <= m);
    advance_lines(m);
  }
  // LY, the window line and the scanline position after m line changes
  // (1 <= m <= 154) from line ly < 154, with LCDC and WY fixed over them:
  // the window line counter counts the lines left below 144 and at or past
  // WY (LCDC bit 5), restarting at 0 when line 0 is entered, which happens
  // iff ly + m reaches 154.
  __device__ void advance_lines(uint32_t m) {
    const uint32_t lf = line_after(m);
    // lines in [a, b) below 144 and at or past WY, with the window on
    auto counted = [&](uint32_t a, uint32_t b) {
      const int hi = min((int)b, kScreenH), lo = max((int)a, (int)wy);
      return (lcdc & 0x20u) && hi > lo ? (uint32_t)(hi - lo) : 0u;
    };
    wl = ly + m >= (uint32_t)kLinesPerFrame ? counted(0u, lf) : wl + counted(ly, lf);
    ly = lf;
    lym = lf;
    scan -= m * (uint32_t)kCyclesPerLine;
  }
  // One PPU step of `cycles` (cycles > 0).
  __device__ uint32_t ppu_advance(int cycles) {
    const uint32_t lc = lcdc;
    if (!(lc & 0x80u)) {
      scan = 0;
      ly = 0;
      wl = 0;
      if (lym) {
        lym = 0;
        M(0xFF44) = 0u;
      }
    } else {
      const uint32_t s0 = scan;
      scan = s0 + (uint32_t)cycles;
      if (scan >= (uint32_t)kCyclesPerLine) ppu_lines(s0);
    }
    stat_fresh = 0;
    lyc_pp = lyc;
    lcd_pp = lc & 0x80u;
    return lc;
  }

  // Cycles from here to the end of the first scanline change that can raise
  // one of the requests in `irq` (bit 0 VBlank, bit 1 STAT): the change into
  // line 144 (VBlank, and the STAT mode-1 source) or into line LYC (the STAT
  // LYC source).  The mode-2 source never fires at a change, and the HBlank
  // source is handled by the caller.
  // (Selects throughout: these run in the rare blocks, where every branch
  // costs the wavefront its exec-mask bookkeeping.)
  __device__ int line_horizon(uint32_t irq) const {
    // changes ahead, 1 = the next one: into line 144 and into line LYC
    const uint32_t n144 = wrap_line(144u + 153u - ly) + 1u;
    const uint32_t nlyc = wrap_line(lyc + 153u - ly) + 1u;  // used only for lyc < 154
    uint32_t n = (((irq & 1u) != 0u) | (((irq & 2u) != 0u) & ((stat_full & 0x10u) != 0u))) ? n144 : 0xFFFFu;
    n = (((irq & 2u) != 0u) & ((stat_full & 0x40u) != 0u) & (lyc < (uint32_t)kLinesPerFrame)) ? min(n, nlyc) : n;
    return n == 0xFFFFu ? kCyclesPerFrame : (kCyclesPerLine - (int)scan) + kCyclesPerLine * (int)(n - 1u);
  }
  // Cycles from here to the nearest event that a batched step must not pass:
  // the frame end, a TIMA overflow or reload, and scanline changes: every
  // one with `every_line`, else those that can raise a request in `irq`
  // (line_horizon).  The PPU step applies several changes in order exactly
  // as the reference's per-instruction steps do, except for one thing: a
  // change compares the new line's STAT bits with those at the start of the
  // step that crosses it.  With the HBlank source enabled that step must
  // start in mode 0 as the reference's last instruction of the line does, so
  // then every change and the mode boundaries count as well.
  __device__ int ff_horizon(int cframe, bool every_line, uint32_t irq) const {
    const int d = kCyclesPerFrame - cframe;
    const bool hsrc = (stat_full & 0x08u) != 0u;
    const bool hbl = hsrc & (ly < (uint32_t)kScreenH);
    const int nb = !hbl ? kCyclesPerLine : scan < 80u ? 80 : scan < 250u ? 250 : kCyclesPerLine;
    const int dl = (every_line | hsrc) ? nb - (int)scan : irq ? line_horizon(irq) : d;
    const int period = 1 << (div_bit(tac) + 1);
    const int edge = period - (int)(div & (uint32_t)(period - 1));
    const int dt = pend ? max((int)delay, 1) : (tac & 4u) ? edge + (int)(255u - tima) * period : d;
    return min(min(d, (lcdc & 0x80u) ? dl : d), dt);
  }
  // No pass may be batched while an interrupt would be serviced after the
  // current instruction or the EI delay is pending.
  __device__ bool ff_blocked() const {
    return (ime_delay != 0u) | ((ime != 0u) & ((ie & ifr & 0x1Fu) != 0u));
  }
  // Whole passes of an LY poll loop (LDH A,(44) or LD A,(FF44); CP d8; JR cc
  // or JP cc back to the load; 32, 36 or 40 cycles) that can be taken in one
  // step from the load at pc that just read ly: 0 unless the jump back is
  // taken (and, for a JP, lands on pc).  The reference runs the loop one
  // instruction at a time with the timer, PPU, interrupt check and frame
  // count after each.  The loop observes only the LY it reads, so the passes
  // run through scanline changes up to the first line whose value ends the
  // loop, and otherwise to the same horizon as a block copy: the frame end, a
  // TIMA overflow, a line change that raises a request that would be
  // serviced, or with the HBlank STAT source on the next mode boundary.  The
  // last pass ends at or before it.  A pass reads the line at its own start:
  // the one read now until the next change, then ly + 1, ly + 2, ...
  // Cycles of one pass of the poll loop whose record word is dw.
  __device__ static uint32_t poll_pass_cycles(uint32_t dw) { return ((dw >> 10) & 0xFu) * 4u; }
  // x / poll_pass_cycles(dw) for 0 <= x < 2^20 as one high multiply by the
  // rounded-up reciprocal (exact for the 32-, 36- and 40-cycle passes there)
  __device__ static uint32_t div_pass(uint32_t x, uint32_t dw) {
    const uint32_t q = (dw >> 10) & 0xFu;  // 8, 9 or 10
    const uint32_t m = q == 8u ? 0x08000000u : q == 9u ? 0x071C71C8u : 0x06666667u;
    return __umulhi(x, m);
  }
  // `ex` is set when the passes stop at the change into a line that ends the
  // loop (not at an event) and the exit also fits before the event horizon:
  // the next pass's load then reads that line, and its CP and the jump not
  // taken can join the step (pass cycles - 4: the jump not taken is 4 cycles
  // shorter), which saves the loop a second entry into this block.
  __device__ int poll_passes(uint32_t dw, uint32_t ly_read, int cframe, uint32_t pc, bool& ex) const {
    const uint32_t d8 = dw & 0xFFu, cc = (dw >> 8) & 3u;
    // cc: 0 NZ, 1 Z, 2 NC, 3 C
    const bool flag = (cc & 2u) ? ly_read < d8 : ly_read == d8;
    const bool back = (flag == ((cc & 1u) != 0u)) & (((dw >> 14) & 1u) == 0u || (dw >> 16) == pc);
    // (with the LCD off ff_horizon ignores the line arguments, and LY stays 0)
    const int h = ff_horizon(cframe, false, ime != 0u ? ie & 0x03u : 0u);
    const int k = (int)div_pass((uint32_t)h, dw);
    // m = line changes ahead to the first line whose value ends the loop
    // (0: none does)
    const uint32_t nl = (uint32_t)kLinesPerFrame;
    const uint32_t v1 = wrap_line(ly + 1u);
    const uint32_t dist = wrap_line(d8 + nl - ly - 1u) + 1u;  // used only for d8 < nl
    uint32_t m = 1u;  // Z: the first change (conservative: stopping early is exact)
    m = cc == 0u ? (d8 < nl ? dist : 0u) : m;                       // NZ: until LY == d8
    m = cc == 2u ? (d8 == 0u ? 0u : v1 < d8 ? 1u : nl - ly) : m;    // NC: until LY < d8
    // C: until LY >= d8.  From line 153 the changes run 0, 1, ..., d8, so d8 + 1
    // of them; (d8 + nl - ly - 1) % nl + 1 counts that and also the case
    // ly == d8 (a program that wrote FF44 reads a smaller LY): nl changes.
    m = cc == 3u ? (d8 >= nl ? 0u : v1 >= d8 ? 1u : dist) : m;
    const int c = (kCyclesPerLine - (int)scan) + kCyclesPerLine * (int)(m - 1u);
    const int km = (int)div_pass((uint32_t)c + poll_pass_cycles(dw) - 1u, dw);  // used only for m != 0
    const bool ends = ((lcdc & 0x80u) != 0u) & (m != 0u);
    const int kk = ends ? min(k, km) : k;
    const int pcyc = (int)poll_pass_cycles(dw);
    const bool none = (!back) | ff_blocked();
    ex = (!none) & ends & (km <= k) & (km * pcyc + pcyc - 4 <= h);
    return none ? 0 : kk;
  }
  // End of the plain RAM window holding x (video RAM, work RAM), else 0.
  __device__ static uint32_t ram_window_end(uint32_t x) {
    return x - 0x8000u < 0x2000u ? 0xA000u : x - 0xC000u < 0x2000u ? 0xE000u : 0u;
  }
  // Whole passes of a block-copy loop (52 cycles, 7 instructions each) that
  // all jump back and can run as one step: bounded by the event horizon, by
  // BC, and by the source and destination staying inside one window each
  // (a ROM bank window above the boot image, video RAM or work RAM for the
  // source; video or work RAM for the destination) where every byte is a
  // plain load or store.  A destination ahead of an overlapping source stops
  // before the first byte a pass would read after an earlier pass wrote it.
  // The loop reads no IO, so a scanline change bounds the passes only when
  // it can raise a VBlank or STAT request that would be serviced.
  __device__ int copy_passes(uint32_t hl, uint32_t de, uint32_t bc, int cframe) const {
    if (ff_blocked()) return 0;
    const uint32_t se = hl < 0x4000u ? (((boot_en != 0u) & (hl < 0x100u)) ? 0u : 0x4000u)
                        : hl < 0x8000u ? 0x8000u : ram_window_end(hl);
    const uint32_t de_end = ram_window_end(de);
    if ((se == 0u) | (de_end == 0u)) return 0;
    int k = ff_horizon(cframe, false, ime != 0u ? ie & 0x03u : 0u) / 52;
    k = min(k, (int)((bc - 1u) & 0xFFFFu));  // BC = 0 runs 65536 passes
    k = min(k, (int)(se - hl));
    k = min(k, (int)(de_end - de));
    if ((hl >= 0x8000u) & (de > hl)) k = min(k, (int)(de - hl));
    return k;
  }
  // Cycles a step may take on the fast path: it must not reach a TIMA
  // edge, the scanline end or the frame end (0 while a switched-off LCD still
  // has PPU state to clear).
  __device__ int event_budget(int cframe) const {
    int b = kCyclesPerFrame - cframe;
    const uint32_t te = tmask - (div & 0xFFFFu & tmask);
    // the next TIMA edge, or with deferral the edge that overflows TIMA
    // (at most 65,535 cycles on, so the DIV difference stays exact)
    const uint32_t tov = ((defer_timer != 0u) & ((tac & 4u) != 0u))
                             ? min(te + 1u + (0xFFu - (tima & 0xFFu)) * (tmask + 1u), 0xFFFFu)
                             : te + 1u;
    b = tov < (uint32_t)b ? (int)tov : b;
    // the scanline end, or with deferral the end of the first change that
    // can raise a request: into line 144 (VBlank, STAT mode 1) or into line
    // LYC with the LYC source on.  With the HBlank source on every change
    // can (its request compares with the STAT bits where the previous
    // instruction ended).
    const bool lazy = (defer != 0u) & ((stat_full & 0x08u) == 0u);
    b = (lcdc & 0x80u) ? min(b, lazy ? line_horizon(3u) : kCyclesPerLine - (int)scan)
                       : ((scan | ly | wl | lym) != 0u ? 0 : b);
    if ((mbc == MBC_MBC3) & (rtc_halt == 0u))  // the next RTC second
      b = ((rtc_dirty != 0u) | (rtc_sub < 0)) ? 0 : min(b, kRtcCyclesPerSecond - rtc_sub);
    // a pending TIMA reload or EI delay, or an interrupt request that IME
    // or HALT lets act on, takes the full sequence every step until it is
    // dealt with.  With IME clear a running CPU leaves a request pending and
    // the step's interrupt check does nothing; EI, RETI and HALT, which
    // change that, zero the budget when a request is pending.
    const uint32_t irq = ((ime | halted) != 0u) ? (ie & ifr & 0x1Fu) : 0u;
    return (pend | ime_delay | irq) != 0u ? 0 : b;
  }
  // Cycles a halted CPU advances in one loop iteration: the reference steps
  // 4 cycles at a time and wakes on IE & IF; nothing it can observe changes
  // before the first event of ff_horizon for the requests IE enables, so it
  // advances straight to the first 4-cycle step that reaches that event.  A
  // request already pending (a launch that ended before its interrupt check,
  // or imported state) wakes the CPU after the first 4 cycles.
  __device__ int halt_cycles(int cframe) const {
    if (ie & ifr & 0x1Fu) return 4;
    const int d = max(ff_horizon(cframe, false, ie & 0x03u), 1);
    return (d + 3) & ~3;
  }

  // -- fetch ---------------------------------------------------------------------
  // A pre-decoded record serves pc when all three instruction bytes lie in
  // one 16 KiB ROM window of a mapped bank, or in the boot image.
  __device__ bool rec_ok(uint32_t p) const {
    const bool bw = (boot_en != 0u) & (p < 0x100u);
    return (bw & (p < 0xFEu)) | (!bw & (p < 0x8000u) & ((p & 0x3FFFu) <= 0x3FFDu));
  }
  __device__ uint32_t rec_index(uint32_t p) const {
    return ((boot_en != 0u) & (p < 0x100u)) ? rom_len + p
                                   : (p < 0x4000u ? rom_lo : rom_hi) + (p & 0x3FFFu);
  }
  // rec_ok and rec_index in one: the record index for p, or 0 when no record
  // serves it (ok false).  Written as selects so that the per-instruction
  // path has no branch for it.
  __device__ uint32_t next_rec(uint32_t p, bool& ok) const {
    const bool bw = (boot_en != 0u) & (p < 0x100u);
    const uint32_t win = sel(p < 0x4000u, rom_lo, rom_hi) + (p & 0x3FFFu);
    ok = (bw & (p < 0xFEu)) | (!bw & (p < 0x8000u) & ((p & 0x3FFFu) <= 0x3FFDu));
    return sel(ok, sel(bw, rom_len + p, win), 0u);
  }
  // Fetch + decode through the bus (code in RAM, window edges, open bus).
  __device__ Rec fetch_slow() const {
    const uint32_t b0 = read8(pc), b1 = read8(pc + 1u), b2 = read8(pc + 2u);
    return bind_bytes(kDec.e[b0 == 0xCBu ? 256u + b1 : b0], b0, b1, b2);
  }
};

// ---------------------------------------------------------------------------
// The kernel
// ---------------------------------------------------------------------------
// One variant per cartridge kind (kMbc), per debug mode (kDbg) and, for
// ROM-only carts, per declared RAM (kCram): the cartridge code of other
// kinds and every debug check compile out.  The variants for MBC carts
// with RAM are built for two wavefronts per SIMD (256 VGPRs): at three they
// spill VGPRs to scratch in the loop, and 131,072 envs in 64-lane
// wavefronts are two per SIMD.
template <int kMbc, bool kDbg, bool kCram = true>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu((kMbc != MBC_ROM_ONLY && kCram) ? 2 : 3))) void step_kernel(DevState s, StepArgs args) {
  const uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (uint32_t)s.n) return;
  Lane L{s};
  L.mbc = kMbc;
  L.cram = kCram;
  L.e = e;
  L.defer = (!kDbg && e != 0u) ? 1u : 0u;
  L.defer_timer = kDbg ? 0u : 1u;
  L.lane = e & (kEnvBlock - 1);
  const uint32_t blk = __builtin_amdgcn_readfirstlane(e >> kEnvBlockShift);
  L.rm = make_rsrc(s.mem + ((size_t)blk << 22), 1u << 22);
  L.memb = in_vgpr(s.mem + ((size_t)blk << 22));
  L.cramb = in_vgpr(s.cram + (size_t)blk * (size_t)s.cram_stride * kEnvBlock);
  L.rom = in_vgpr(s.rom);
  L.rom_len = in_vgpr((uint32_t)s.rom_len);
  L.rsc = make_rsrc(s.sc + (size_t)blk * (kNumFields * kEnvBlock), kNumFields * kEnvBlock * 4);
  L.rcs = make_rsrc(s.cs + (size_t)blk * (kCartStateStride * kEnvBlock),
                    kCartStateStride * kEnvBlock * 4);
  const rsrc_t rcnt = make_rsrc(s.cnt + (size_t)blk * (2 * kEnvBlock), 2 * kEnvBlock * 8);
  const uint4* recs = in_vgpr(reinterpret_cast<const uint4*>(s.recs));  // 4 per record

  // ---- load (cpu_step_builder.py:930-967) ---------------------------------
  L.pc = (uint32_t)L.SC(F_PC) & 0xFFFFu;
  L.sp = (uint32_t)L.SC(F_SP) & 0xFFFFu;
  L.w0 = (((uint32_t)L.SC(F_B) & 0xFFu) << 24) | (((uint32_t)L.SC(F_C) & 0xFFu) << 16) |
         (((uint32_t)L.SC(F_D) & 0xFFu) << 8) | ((uint32_t)L.SC(F_E) & 0xFFu);
  L.w1 = (((uint32_t)L.SC(F_H) & 0xFFu) << 24) | (((uint32_t)L.SC(F_L) & 0xFFu) << 16) |
         (((uint32_t)L.SC(F_F) & 0xF0u) << 8) |
         ((uint32_t)L.SC(F_A) & 0xFFu);
  L.ime = (uint32_t)L.SC(F_IME);
  L.ime_delay = (uint32_t)L.SC(F_IME_DELAY);
  L.halted = (uint32_t)L.SC(F_HALTED);
  L.div = (uint32_t)L.SC(F_DIV_COUNTER);
  L.tprev0 = (uint32_t)L.SC(F_TIMER_PREV_IN);
  L.pend = (uint32_t)L.SC(F_TIMA_PENDING);
  L.delay = (uint32_t)L.SC(F_TIMA_DELAY);
  L.scan = (uint32_t)L.SC(F_PPU_SCANLINE);
  L.ly = (uint32_t)L.SC(F_PPU_LY);
  L.wl = (uint32_t)L.SC(F_PPU_WINDOW_LINE);
  L.sp0 = (uint32_t)L.SC(F_PPU_STAT_PREV);
  L.ff04_0 = L.M(0xFF04);
  L.tima = L.M(0xFF05);
  L.tma = L.M(0xFF06);
  L.tac = L.M(0xFF07);
  L.tmask = Lane::edge_mask(L.tac);
  L.tdiv = L.div;
  L.ifr = L.M(0xFF0F);
  L.lcdc = L.M(0xFF40);
  L.stat_full = L.M(0xFF41);
  L.stat_fresh = 1;
  L.lyc_pp = 0;
  L.lcd_pp = 0x100u;
  L.tp_w = 0;
  L.lym = L.M(0xFF44);
  L.lyc = L.M(0xFF45);
  L.wy = L.M(0xFF4A);
  L.ie = L.M(0xFFFF);
  L.boot_en = L.CS(CS_BOOTROM_ENABLED) != 0 ? 1u : 0u;
  L.rtc_sub = L.CS(CS_RTC_LAST_CYCLE);
  L.rtc_halt = (L.CS(CS_RTC_DAYS_HIGH) & 0x40) ? 1u : 0u;
  L.rtc_dirty = 1;  // first tick of a launch normalizes like the reference does
  L.map_changed = 0;
  L.budget = 0;
  L.mbr = L.load_mbr();
  L.refresh_cart();
  L.action = args.actions[e];
  L.release = (int)in_vgpr((uint32_t)args.release);
  L.frames_done = 0;
  L.joyp_sel = (uint32_t)L.SC(F_JOYP_SELECT);
  L.joyp_refresh();

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
  // per-launch increments, folded into the 64-bit counters at frame ends
  uint32_t ninstr = 0, ncyc = 0;
  int cframe = L.SC(F_CYCLE_IN_FRAME);
  int trap = L.SC(F_TRAP_FLAG), trap_pc = L.SC(F_TRAP_PC);
  int trap_op = L.SC(F_TRAP_OPCODE), trap_kind = L.SC(F_TRAP_KIND);
  const uint32_t dbg_watch = in_vgpr((uint32_t)args.dbg_watch);
  const uint32_t dbg_trap_pc = in_vgpr((uint32_t)args.dbg_trap_pc);
  const uint32_t dbg_rst38 = in_vgpr((uint32_t)args.dbg_rst38);
  const int dbg_max_instr = (int)in_vgpr((uint32_t)args.dbg_max_instr);
  auto watch_read = [&]() -> uint32_t {
    const uint32_t v = L.M(dbg_watch);
    return Lane::io_derived(dbg_watch) ? L.io_fix(dbg_watch, v) : v;
  };
  const uint32_t watch_val = dbg_watch ? watch_read() : 0u;
  const int frames = (int)in_vgpr((uint32_t)args.frames);
  constexpr bool dbg = kDbg;

  // record of the instruction at pc (valid when rv)
  Rec rec{};
  bool rv = false;
  auto load_rec = [&](uint32_t i) {
    const uint4* p = recs + (size_t)i * 4u;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const u32x4 q = ld_global(reinterpret_cast<const u32x4*>(p + k));
      rec.w[4 * k] = q[0];
      rec.w[4 * k + 1] = q[1];
      rec.w[4 * k + 2] = q[2];
      rec.w[4 * k + 3] = q[3];
    }
  };

  // Block copies of the copy-loop fast-forward (bytes cp_src[j * cp_stride]
  // to memory rows cp_dst + j of this lane's env, j < cp_k), done by every
  // active lane of the wavefront together, one copying env after another:
  // a lone lane would make one round trip per 8 bytes while the others
  // wait.  copy_passes bounds k so that no byte is read after the same
  // copy wrote it, so the bytes may be copied in any order.
  uint32_t cp_k = 0, cp_dst = 0, cp_stride = 0;
  const uint8_t* cp_src = nullptr;
  auto coop_copy = [&]() {
    const uint64_t act = __ballot(true);
    uint64_t want = __ballot(cp_k != 0u);
    const uint32_t me = __lane_id();
    const uint32_t rank = (uint32_t)__popcll(act & ((1ull << me) - 1ull));
    const uint32_t nact = (uint32_t)__popcll(act);
    while (want) {
      const uint32_t q = (uint32_t)__builtin_ctzll(want);
      want &= want - 1u;
      const uint32_t k = lane_value(cp_k, q);
      const uint32_t dst = lane_value(cp_dst, q);
      const uint32_t stride = lane_value(cp_stride, q);
      const uint32_t ql = lane_value(L.lane, q);
      const uint64_t sa = reinterpret_cast<uint64_t>(cp_src);
      const uint8_t* src = reinterpret_cast<const uint8_t*>(
          ((uint64_t)lane_value((uint32_t)(sa >> 32), q) << 32) | (uint64_t)lane_value((uint32_t)sa, q));
      for (uint32_t j = rank; j < k; j += 4u * nact) {
        uint32_t v[4];
#pragma unroll
        for (uint32_t t = 0; t < 4u; ++t) {
          const uint32_t jx = j + t * nact;
          v[t] = jx < k ? (uint32_t)ld_global(src + jx * stride) : 0u;
        }
#pragma unroll
        for (uint32_t t = 0; t < 4u; ++t) {
          const uint32_t jx = j + t * nact;
          if (jx < k)
            __builtin_amdgcn_raw_buffer_store_b8((uint8_t)v[t], L.rm, (int)(((dst + jx) << kEnvBlockShift) | ql), 0, 0);
        }
      }
    }
  };

  // One exit: the frame count reached or the env trapped (a trap freezes
  // the env for the rest of the launch, misc.py:42-56).
  while ((L.frames_done < frames) & (trap == 0)) {
    const uint32_t lcdc_prev = L.lcdc & 0x80u;
    const bool hiter = L.halted != 0;
    int cycles = 4;
    // the cycles of a batched step (HALT, poll or copy passes) before its
    // last 4-cycle halted step or last instruction (a taken JR, 12 cycles):
    // the RTC counts them before the step's interrupt check, whose push may
    // write the RTC registers (the reference ticks it after every step)
    int rtc_pre = 0;
    uint32_t op = 0;
    const uint32_t pc_before = L.pc;
    // pending bus writes: the instruction's, then the interrupt push
    uint32_t wn = 0, wa0 = 0, wv0 = 0, wa1 = 0, wv1 = 0;

    if (__builtin_expect(!hiter, 1)) {
      // ---- fetch + decode ------------------------------------------------------
      const uint32_t pc = L.pc;
      // (rare branches of the per-instruction path test a wave-uniform
      // ballot first: when no lane takes them the path keeps its exec mask
      // instead of saving and restoring it around a skipped block)
      if (__builtin_expect(__ballot(!rv) != 0u, 0)) {
        if (!rv) {
          if (L.rec_ok(pc)) load_rec(L.rec_index(pc));
          else rec = L.fetch_slow();
        }
      }
      op = rec.w[0] & 0xFFu;
      if (dbg) {  // debug traps before execution: the instruction does not run
        if (dbg_trap_pc && pc == dbg_trap_pc) {
          trap = 1; trap_pc = (int)pc; trap_op = (int)op; trap_kind = 5;
        } else if (dbg_rst38 && op == 0xFFu && pc != 0x0038u) {
          trap = 1; trap_pc = (int)pc; trap_op = (int)op; trap_kind = 3;
        }
      }
      if (!trap) {
      ExecIn in;
      in.w0 = L.w0;
      in.w1 = L.w1;
      in.x1 = (L.sp << 16) | pc;
      in.ra = operand_address(rec, L.w0, L.w1, in.x1);

      // ---- bus reads ------------------------------------------------------------
      const uint32_t nr = ubfe(rec.w[7], 8, 2);
      {
        // Every lane loads the byte at its operand address, reading or not
        // (a read has no side effect, and the folded address is always on
        // the bus): no branch around the load, which lets it issue as early
        // as its address allows.  A second load only for two-byte reads
        // (POP, RET), issued before either byte is used; that byte sits one
        // address row (64 bytes) after the first when both are in the env's
        // memory.  A lane with one read repeats its first byte.
        const uint32_t x0 = Lane::fold(in.ra);
        const uint8_t* p0 = L.bus_ptr(x0);
        const uint32_t v0 = ld_global(p0);
        uint32_t x1 = x0, v1 = 0;
        if (__builtin_expect(nr > 1u, 0)) {
          x1 = Lane::fold(in.ra + 1u);
          const uint8_t* p1 = p0 + kEnvBlock;
          if ((x1 != x0 + 1u) | (x0 < 0x8000u) | (x0 - 0xA000u < 0x2000u) | (x1 - 0xA000u < 0x2000u))
            p1 = L.bus_ptr(x1);
          v1 = ld_global(p1);
        }
        // DIV, TIMA, STAT and LY (FF04 FF05 FF40 FF41 FF44 FF45, bus_fix's
        // test) for both bytes behind one wave-uniform test, the bytes
        // taken by selects
        const bool h0 = (nr != 0u) & ((x0 & 0xFFBAu) == 0xFF00u) & (x0 > 0xFF01u);
        const bool h1 = (nr > 1u) & ((x1 & 0xFFBAu) == 0xFF00u) & (x1 > 0xFF01u);
        uint32_t r0 = v0, r1 = v1;
        if (__builtin_expect(__ballot(h0 | h1) != 0u, 0)) {
          r0 = h0 ? L.read_ppu(x0, v0) : v0;
          r1 = h1 ? L.read_ppu(x1, v1) : v1;
        }
        in.rd0 = nr != 0u ? r0 : 0u;
        in.rd1 = nr > 1u ? r1 : in.rd0;
      }

      // ---- execute (gbx_exec.h) -------------------------------------------------
      const ExecOut o = exec_insn(rec, in);
      L.w0 = o.w0;
      L.w1 = o.w1;
      L.sp = o.sp;
      cycles = (int)o.cycles;
      wn = o.wn;
      wa0 = o.wa0;
      wv0 = o.wv0;
      wa1 = o.wa1;
      wv1 = o.wv1;
      uint32_t npc = o.npc;
      // (a wave-uniform test, so that the copy below runs with every lane
      // that is executing an instruction)
      if (__builtin_expect(__ballot(o.misc != 0u) != 0u, 0)) {
        if (o.misc != 0u) {  // DI EI RETI HALT, illegal opcodes, poll/copy loops
          L.settle();  // the fast-forwards start from the PPU and timer state
          if (o.misc & 1u) {
            L.ime = (o.misc >> 1) & 1u;
            L.ime_delay = 0;
          }
          if (o.misc & 4u) L.halted = 1;
          // the step's interrupt check services or wakes on a pending request
          if (((L.ime | L.halted) != 0u) & ((L.ie & L.ifr & 0x1Fu) != 0u)) L.budget = 0;
          if (o.misc & 8u) {  // misc.py:42-56: freeze the env, pc unchanged
            trap = 1;
            trap_pc = (int)pc;
            trap_op = (int)op;
            trap_kind = 1;
            L.budget = 0;
          }
          if (!dbg && (o.misc & 16u) && (rec.w[15] & kCopyLoop)) {
            // LD A,(HL+) of a block-copy loop just ran: advance k whole passes
            // (this LD included) in one step.  Each pass copies (HL+) to (DE)
            // and steps DE and BC; OR leaves Z clear (BC stays non-zero), N,
            // H and C clear, so F = 0 and A = B | C.
            const uint32_t hl = in.w1 >> 16, de = in.w0 & 0xFFFFu, bc = in.w0 >> 16;
            const int k = L.copy_passes(hl, de, bc, cframe);
            if (k > 0) {
              // the k bytes are copied below by the whole wavefront
              cp_k = (uint32_t)k;
              cp_dst = de;
              cp_src = L.bus_ptr(hl);
              cp_stride = hl < 0x8000u ? 1u : (uint32_t)kEnvBlock;
              const uint32_t nbc = (bc - (uint32_t)k) & 0xFFFFu;
              L.w0 = (nbc << 16) | (de + (uint32_t)k);
              L.w1 = ((hl + (uint32_t)k) << 16) | ((nbc | (nbc >> 8)) & 0xFFu);
              npc = pc;
              cycles = 52 * k;
              rtc_pre = cycles - 12;
              ninstr += 7u * (uint32_t)k - 1u;
            }
          } else if (!dbg && (o.misc & 16u)) {
            // The load of an LY poll loop just read LY into A; if CP d8 and the
            // jump take it back, every pass until LY or anything else can
            // change reads the same LY and leaves the same A and F: advance k
            // whole passes (this load included) in one step, and when they
            // end at the change into the line that ends the loop (ex), the
            // exit too: the next load reads that line, CP sets F and the jump
            // falls through.
            bool ex = false;
            const int k = L.poll_passes(rec.w[15], in.rd0, cframe, pc, ex);
            if (k > 0) {
              const uint32_t pcyc = Lane::poll_pass_cycles(rec.w[15]);
              const uint32_t jp = (rec.w[15] >> 14) & 1u;
              // A and F as the last pass's load and CP leave them, or with the
              // exit those of the load after the k passes
              const uint32_t off = L.scan + pcyc * (uint32_t)(k - (ex ? 0 : 1));
              const uint32_t ly = ((off < (uint32_t)kCyclesPerLine) | ((L.lcdc & 0x80u) == 0u))
                                      ? in.rd0
                                      : Lane::wrap_line(L.ly + off / (uint32_t)kCyclesPerLine);
              const uint32_t d8 = rec.w[15] & 0xFFu;
              const uint32_t f = ((ly == d8) ? 0x80u : 0u) | 0x40u | (((ly & 15u) < (d8 & 15u)) ? 0x20u : 0u) |
                                 ((ly < d8) ? 0x10u : 0u);
              L.w1 = (L.w1 & 0xFFFF0000u) | (f << 8) | ly;
              // the load (LDH 2 bytes, LD A,(a16) 3), CP d8 and the jump (JR 2, JP 3)
              const uint32_t len = (op == 0xFAu ? 3u : 2u) + 2u + 2u + jp;
              npc = ex ? (pc + len) & 0xFFFFu : pc;
              cycles = (int)pcyc * k + (ex ? (int)pcyc - 4 : 0);
              // the cycles before the last instruction, the jump: taken (JP 16,
              // JR 12) or, after the exit, not taken (JP 12, JR 8)
              rtc_pre = cycles - (jp ? 16 : 12) + (ex ? 4 : 0);
              ninstr += 3u * (uint32_t)k - 1u + (ex ? 3u : 0u);
            }
          }
        }
        if (!dbg && __ballot(cp_k != 0u) != 0u) {
          coop_copy();
          cp_k = 0;
        }
      }
      L.pc = npc;
      // fetch the next record while the writes, timer and PPU run
      load_rec(L.next_rec(npc, rv));
      }
    } else {
      L.settle();
      cycles = L.halt_cycles(cframe);
      rtc_pre = cycles - 4;
    }

    // ---- write phase, debug checks, timer, PPU, interrupt check --------------
    int svc = 0;
    if (__builtin_expect(wn != 0u, 1)) L.write_bus(wn, wa0, wv0, wa1, wv1, rv);
    if (dbg) {
      if (!hiter) {
        if (dbg_rst38 && L.pc >= 0xFE00u && !trap) {
          trap = 1; trap_pc = (int)pc_before; trap_op = (int)op; trap_kind = 4;
        }
        if (!trap) {
          ninstr += 1;
          if (dbg_max_instr > 0 && instr + ninstr - instr_start >= dbg_max_instr) {
            trap = 1; trap_pc = (int)L.pc; trap_op = (int)op; trap_kind = 6;
          } else if (dbg_watch && watch_read() != watch_val) {
            trap = 1; trap_pc = (int)pc_before; trap_op = (int)op; trap_kind = 7;
          }
        }
      }
    } else {
      ninstr += (uint32_t)((!hiter) & (trap == 0));
    }
    // Fast path: when no timer edge or reload, no scanline wrap, no LCD
    // switch, no pending interrupt, no remap, no RTC second and no frame end
    // fall inside this step, the sequence below reduces to DIV, the scanline
    // position and the cycle counters advancing.  The budget is the distance
    // to the nearest of those events, and 0 while any of them is pending or
    // once this step made one (an IO, MBC or RTC write, a trap).
    const uint32_t lc_now = L.lcdc;
    const uint32_t ucyc = (uint32_t)cycles;
    const bool lcd_on = (lc_now & 0x80u) != 0u;
    const bool fast = (trap == 0) & (cycles < L.budget);
    if (__builtin_expect(fast, 1)) {
      // stat_fresh, lyc_pp and lcd_pp already hold what a PPU step would set:
      // STAT, LYC and LCDC writes go through io_write, which zeroes the
      // budget, and a launch starts with the budget at 0
      L.div = (L.div + ucyc) & 0xFFFFu;
      L.scan = lcd_on ? L.scan + ucyc : 0u;
      if (kMbc == MBC_MBC3) L.rtc_sub += L.rtc_halt ? 0 : cycles;
      ncyc += ucyc;
      cframe += cycles;
      L.budget -= cycles;
    } else if (!trap) {
      L.settle();
      L.timer_tick(cycles);
      if (!hiter & (L.ime_delay != 0u)) {
        L.ime = 1;
        L.ime_delay = 0;
      }
      uint32_t lcdc_now = L.ppu_advance(cycles);
      if (kMbc == MBC_MBC3) L.rtc_tick(rtc_pre);
      const uint32_t pending = L.ie & L.ifr & 0x1Fu;
      if (__builtin_expect(pending != 0u, 0)) {
        L.halted = 0;
        if (L.ime) {
          // service (cpu_step_builder.py:1502-1600): push pc, jump to the
          // vector, 20 cycles of timer and PPU
          L.ime = 0;
          const uint32_t bit = pending & (0u - pending);
          L.set_if(L.ifr & ~bit & 0xFFu);
          const uint32_t ret = L.pc;
#pragma unroll 1
          for (uint32_t k = 1; k <= 2; ++k)
            L.write8((L.sp - k) & 0xFFFFu, k == 1 ? ret >> 8 : ret & 0xFFu);
          L.sp = (L.sp - 2u) & 0xFFFFu;
          L.pc = 0x40u + 8u * (uint32_t)__builtin_ctz(bit);
          rv = false;
          svc = 20;
          L.timer_tick(20);
          lcdc_now = L.ppu_advance(20);
        } else if (hiter) {
          L.pc = (L.pc + 1u) & 0xFFFFu;  // IME=0 wake skips a byte
          rv = false;
        }
      }
      if (__builtin_expect(L.map_changed != 0u, 0)) {
        L.map_changed = 0;
        rv = false;
      }

      const int total = cycles + svc;
      L.rtc_tick(total - rtc_pre);
      ncyc += (uint32_t)total;
      cframe += total;
      if (__builtin_expect((((lcdc_prev ^ lcdc_now) & 0x80u) != 0u) | (cframe >= kCyclesPerFrame), 0)) {
        // LCD toggles and frame ends (cpu_step_builder.py frame loop)
        instr += ninstr;
        cyc += ncyc;
        ninstr = 0;
        ncyc = 0;
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
          ++L.frames_done;
          L.joyp_refresh();
        } else if (!hiter && !lcdc_prev && (lcdc_now & 0x80u)) {
          L.scan = 0;
          L.ly = 0;
          L.wl = 0;
          L.lym = 0;
          L.stat_fresh = 0;  // STAT and stat_prev follow from scan 0 of line 0
          cframe = 0;
          ++L.frames_done;
          L.joyp_refresh();
        } else {
          while (cframe >= kCyclesPerFrame && L.frames_done < frames) {
            cframe -= kCyclesPerFrame;
            ++L.frames_done;
          }
          L.joyp_refresh();
        }
      }
      L.budget = L.event_budget(cframe);
    }
  }
  L.settle();
  instr += ninstr;
  cyc += ncyc;

  // ---- post-step outputs (cpu_templates/post_step.py) ----------------------
  const int stage = args.stage;
  const uint32_t a_ = L.a(), b_ = L.w0 >> 24, c_ = (L.w0 >> 16) & 0xFFu, d_ = (L.w0 >> 8) & 0xFFu;
  const uint32_t e_ = L.w0 & 0xFFu, h_ = L.w1 >> 24, l_ = (L.w1 >> 16) & 0xFFu;
  if (stage != 0) {
    uint32_t mm[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) mm[k] = L.M(0xC000u + (uint32_t)k);
    if (stage == 2 || stage == 3) {
      float* o = s.obs + (size_t)e * s.obs_dim;
      o[0] = (float)(L.pc & 0xFFFFu) / 65535.0f;
      o[1] = (float)(L.sp & 0xFFFFu) / 65535.0f;
      o[2] = (float)a_ / 255.0f;
      o[3] = (float)L.f() / 255.0f;
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
      o[28] = (float)((mm[4] ^ a_) & 0xFFu) / 255.0f;
      o[29] = (float)((mm[5] + b_) & 0xFFu) / 255.0f;
      o[30] = (float)((mm[6] ^ c_) & 0xFFu) / 255.0f;
      o[31] = (float)((mm[7] + d_) & 0xFFu) / 255.0f;
    }
    if (stage == 1 || stage == 3) {
      const uint32_t mix = (mm[0] + mm[1] * 3u) & 0xFFu;
      s.reward[e] = (float)((a_ ^ mix) & 0xFFu) / 255.0f;
    }
  }

  // ---- write back --------------------------------------------------------
  L.SC(F_PC) = (int32_t)(L.pc & 0xFFFFu);
  L.SC(F_SP) = (int32_t)(L.sp & 0xFFFFu);
  L.SC(F_A) = (int32_t)a_;
  L.SC(F_B) = (int32_t)b_;
  L.SC(F_C) = (int32_t)c_;
  L.SC(F_D) = (int32_t)d_;
  L.SC(F_E) = (int32_t)e_;
  L.SC(F_H) = (int32_t)h_;
  L.SC(F_L) = (int32_t)l_;
  L.SC(F_F) = (int32_t)L.f();
  st64(0, instr);
  st64(1, cyc);
  L.SC(F_CYCLE_IN_FRAME) = cframe;
  L.SC(F_TRAP_FLAG) = trap;
  L.SC(F_TRAP_PC) = trap_pc;
  L.SC(F_TRAP_OPCODE) = trap_op;
  L.SC(F_TRAP_KIND) = trap_kind;
  L.SC(F_IME) = (int32_t)L.ime;
  L.SC(F_JOYP_SELECT) = (int32_t)L.joyp_sel;
  L.SC(F_IME_DELAY) = (int32_t)L.ime_delay;
  L.SC(F_HALTED) = (int32_t)L.halted;
  L.SC(F_DIV_COUNTER) = (int32_t)L.div;
  L.SC(F_TIMER_PREV_IN) = (int32_t)L.tprev_val();
  L.SC(F_TIMA_PENDING) = (int32_t)L.pend;
  L.SC(F_TIMA_DELAY) = (int32_t)L.delay;
  L.SC(F_PPU_SCANLINE) = (int32_t)L.scan;
  L.SC(F_PPU_LY) = (int32_t)L.ly;
  L.SC(F_PPU_WINDOW_LINE) = (int32_t)L.wl;
  L.SC(F_PPU_STAT_PREV) = (int32_t)L.stat_prev_at(L.scan);
  L.M(0xFF04) = L.ff04_val();
  L.M(0xFF05) = L.tima;
  L.M(0xFF06) = L.tma;
  L.M(0xFF07) = L.tac;
  L.M(0xFF0F) = L.ifr;
  L.M(0xFF40) = L.lcdc;
  L.M(0xFF41) = L.stat_val();
  L.M(0xFF44) = L.lym;
  L.M(0xFF45) = L.lyc;
  L.M(0xFF4A) = L.wy;
  L.M(0xFFFF) = L.ie;
  if (kMbc == MBC_MBC3) L.CS(CS_RTC_LAST_CYCLE) = L.rtc_sub;
}

}  // namespace

hipError_t launch_step(const DevState& s, const StepArgs& a, hipStream_t st) {
  if (s.n <= 0) return hipSuccess;
  // A wavefront carries step_lanes envs (a divisor of the 64-env memory
  // block, so it never straddles two blocks).  Full 64-lane wavefronts go
  // four to a workgroup: the four land on the four SIMDs of one CU, where
  // single-wavefront workgroups left some SIMDs with three wavefronts and
  // others with one (the wavefronts on a crowded SIMD set the launch time).
  // Narrower wavefronts (few envs) stay one to a workgroup, one per SIMD.
  const int threads = s.step_lanes == kEnvBlock ? 4 * kEnvBlock : s.step_lanes;
  const int blocks = (s.n + threads - 1) / threads;
  const bool dbg = a.dbg_rst38 || a.dbg_trap_pc || a.dbg_max_instr > 0 || a.dbg_watch;
  const dim3 g(blocks), b(threads);
  const bool rom_ram = s.mbc_kind == MBC_ROM_ONLY && s.ram_banks > 0;
  switch (s.mbc_kind * 2 + (dbg ? 1 : 0)) {
    case MBC_ROM_ONLY * 2:
      if (rom_ram) hipLaunchKernelGGL((step_kernel<MBC_ROM_ONLY, false, true>), g, b, 0, st, s, a);
      else hipLaunchKernelGGL((step_kernel<MBC_ROM_ONLY, false, false>), g, b, 0, st, s, a);
      break;
    case MBC_ROM_ONLY * 2 + 1:
      if (rom_ram) hipLaunchKernelGGL((step_kernel<MBC_ROM_ONLY, true, true>), g, b, 0, st, s, a);
      else hipLaunchKernelGGL((step_kernel<MBC_ROM_ONLY, true, false>), g, b, 0, st, s, a);
      break;
    // (an MBC cart without RAM gets the variant whose store path has no
    // cartridge RAM; the debug variants keep the general one)
    case MBC_MBC1 * 2:
      if (s.ram_banks > 0) hipLaunchKernelGGL((step_kernel<MBC_MBC1, false, true>), g, b, 0, st, s, a);
      else hipLaunchKernelGGL((step_kernel<MBC_MBC1, false, false>), g, b, 0, st, s, a);
      break;
    case MBC_MBC1 * 2 + 1: hipLaunchKernelGGL((step_kernel<MBC_MBC1, true>), g, b, 0, st, s, a); break;
    case MBC_MBC3 * 2:
      if (s.ram_banks > 0) hipLaunchKernelGGL((step_kernel<MBC_MBC3, false, true>), g, b, 0, st, s, a);
      else hipLaunchKernelGGL((step_kernel<MBC_MBC3, false, false>), g, b, 0, st, s, a);
      break;
    default: hipLaunchKernelGGL((step_kernel<MBC_MBC3, true>), g, b, 0, st, s, a); break;
  }
  return hipGetLastError();
}

}  // namespace gbx

// gbx_internal.h -- device layout shared by the step, render and reset kernels
// and the host API.  Not part of the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace gbx {

constexpr int kMemSize = 65536;
constexpr int kEnvBlockShift = 6;  // 64 envs (one wavefront) per interleave block
constexpr int kEnvBlock = 1 << kEnvBlockShift;
// Env 0's scanline latches on the device, line-major: bytes LCDC, SCX, SCY,
// BGP, WX, WY, window line, OBP0, OBP1 (then padding) of line y at
// y * kLatchStride, written by one 16-byte store per line.  The C ABI and
// the env image carry them as [9][144] (register-major).
constexpr int kLatchStride = 16;
constexpr int kSerialMax = 1024;
constexpr int kCartStateStride = 20;
constexpr int kScreenH = 144;
constexpr int kDsW = 80, kDsH = 72, kDsWB = 20;
constexpr int kScreenW = 160;
constexpr int kNumFields = 32;

// cart_state slots (reference core/cartridge.py:55-76)
enum {
  CS_MBC_KIND = 0, CS_RAM_ENABLE, CS_ROM_BANK_LO, CS_ROM_BANK_HI, CS_RAM_BANK,
  CS_BANK_MODE, CS_BOOTROM_ENABLED, CS_RTC_SELECT, CS_RTC_LATCH, CS_RTC_SECONDS,
  CS_RTC_MINUTES, CS_RTC_HOURS, CS_RTC_DAYS_LOW, CS_RTC_DAYS_HIGH,
  CS_RTC_LAST_CYCLE, CS_RTC_L_SECONDS, CS_RTC_L_MINUTES, CS_RTC_L_HOURS,
  CS_RTC_L_DAYS_LOW, CS_RTC_L_DAYS_HIGH
};
enum { MBC_ROM_ONLY = 0, MBC_MBC1 = 1, MBC_MBC3 = 2 };

// Per-env scalar field slots of the SoA block `sc` (same numbering as the
// C ABI's GBX_FIELD_*).  Slots 10 and 11 (instruction / cycle counters) are
// int64 and live in their own arrays.
enum {
  F_PC = 0, F_SP, F_A, F_B, F_C, F_D, F_E, F_H, F_L, F_F, F_INSTR, F_CYCLES,
  F_CYCLE_IN_FRAME, F_TRAP_FLAG, F_TRAP_PC, F_TRAP_OPCODE, F_TRAP_KIND,
  F_ACTIONS, F_JOYP_SELECT, F_SERIAL_LEN, F_SERIAL_OVERFLOW, F_IME,
  F_IME_DELAY, F_HALTED, F_DIV_COUNTER, F_TIMER_PREV_IN, F_TIMA_PENDING,
  F_TIMA_DELAY, F_PPU_SCANLINE, F_PPU_LY, F_PPU_WINDOW_LINE, F_PPU_STAT_PREV
};

// Byte offset of (env, addr) in the interleaved memory image:
// block (env / 64) owns 4 MiB; inside it, address-major with the 64 envs of
// the block contiguous, so lanes of a wavefront touching one address hit one
// 64-byte segment.
__host__ __device__ inline size_t mem_index(uint32_t env, uint32_t addr) {
  return ((size_t)(env >> kEnvBlockShift) << 22) | ((size_t)addr << kEnvBlockShift) |
         (env & (kEnvBlock - 1));
}
__host__ __device__ inline size_t cram_index(uint32_t env, uint32_t off, uint32_t stride) {
  return (((size_t)(env >> kEnvBlockShift) * stride + off) << kEnvBlockShift) |
         (env & (kEnvBlock - 1));
}
// Per-env scalars, cartridge state and counters use the same 64-env blocking
// (array-of-structures-of-arrays): block (env / 64) holds, for each field,
// the 64 lanes contiguously.  A wavefront then addresses every field from one
// wave-uniform base plus one per-lane offset.
__host__ __device__ inline size_t sc_index(uint32_t env, int field) {
  return (((size_t)(env >> kEnvBlockShift) * kNumFields + field) << kEnvBlockShift) |
         (env & (kEnvBlock - 1));
}
__host__ __device__ inline size_t cs_index(uint32_t env, int slot) {
  return (((size_t)(env >> kEnvBlockShift) * kCartStateStride + slot) << kEnvBlockShift) |
         (env & (kEnvBlock - 1));
}
// int64 counters: slot 0 = instructions, 1 = cycles
__host__ __device__ inline size_t cnt_index(uint32_t env, int slot) {
  return (((size_t)(env >> kEnvBlockShift) * 2 + slot) << kEnvBlockShift) |
         (env & (kEnvBlock - 1));
}

struct DevState {
  uint8_t* mem;         // interleaved, npad * 64 KiB
  uint8_t* cram;        // interleaved, npad * cram_stride
  int32_t* cs;          // cs_index layout, npad * 20
  int32_t* sc;          // sc_index layout, npad * 32
  int64_t* cnt;         // cnt_index layout, npad * 2
  uint8_t* serial;      // [npad][1024] env-major
  int32_t* actions;     // [npad] internal action buffer
  float* obs;           // [n][obs_dim]
  float* reward;        // [n]
  uint8_t* pix;         // [n][72][80]
  uint8_t* pix_packed;  // [n][72][20]
  uint8_t* latches;     // [144][kLatchStride] env-0 scanline latches, one 16-byte entry per line
  uint8_t* frame_bg;    // [144][160] env-0 full-frame shades
  const uint8_t* rom;       // ROM image, the 256-byte boot image, 16 KiB of 0xFF (open bus)
  const uint8_t* boot;
  const uint4* recs;        // pre-decoded instruction record per byte of the ROM buffer
  int n, npad, obs_dim;
  int rom_banks, rom_mask, ram_banks, ram_bytes, cram_stride, mbc_kind;
  int step_lanes;       // envs per step-kernel wavefront: 64, 32, 16 or 8
  int64_t rom_len;
};

struct StepArgs {
  const int32_t* actions;
  int frames, release, stage;
  int dbg_rst38, dbg_trap_pc, dbg_max_instr, dbg_watch;
};

hipError_t launch_step(const DevState& s, const StepArgs& a, hipStream_t st);
hipError_t launch_render(const DevState& s, uint8_t* out, int64_t base, int packed,
                         hipStream_t st);
hipError_t launch_reset(const DevState& s, hipStream_t st);
hipError_t launch_render_bg_env0(const DevState& s, uint8_t* out, hipStream_t st);

}  // namespace gbx

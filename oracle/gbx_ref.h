/*
 * gbx_ref -- CPU restatement of the reference's Warp emulator step.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the parity oracle: a plain, env-major,
 * one-env-at-a-time C++ restatement of gbxcule's Warp CPU backend
 * (src/gbxcule/kernels/cpu_step_builder.py, cpu_templates/ (all files),
 * ppu_render_downsampled.py, core/reset_cache.py, backends/warp_vec.py).
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it, and only as the checker / the timed CPU baseline.  The product path
 * (libgbx_hip.so) never links or calls it.
 *
 * Layout follows the reference ABI: mem[env*65536 + addr], SoA int32/int64
 * per-env arrays, cart_state[env*20 + slot].
 */
#pragma once
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct RefMachine RefMachine;

/* Field ids for ref_field_ptr(); same order as gbx_hip.h's GBX_FIELD_*. */
enum {
  REF_PC = 0, REF_SP, REF_A, REF_B, REF_C, REF_D, REF_E, REF_H, REF_L, REF_F,
  REF_INSTR_COUNT, REF_CYCLE_COUNT, REF_CYCLE_IN_FRAME, REF_TRAP_FLAG,
  REF_TRAP_PC, REF_TRAP_OPCODE, REF_TRAP_KIND, REF_ACTIONS, REF_JOYP_SELECT,
  REF_SERIAL_LEN, REF_SERIAL_OVERFLOW, REF_IME, REF_IME_DELAY, REF_HALTED,
  REF_DIV_COUNTER, REF_TIMER_PREV_IN, REF_TIMA_RELOAD_PENDING,
  REF_TIMA_RELOAD_DELAY, REF_PPU_SCANLINE_CYCLE, REF_PPU_LY,
  REF_PPU_WINDOW_LINE, REF_PPU_STAT_PREV, REF_NUM_SCALAR_FIELDS,
  /* array fields */
  REF_MEM = 100, REF_CART_STATE, REF_CART_RAM, REF_SERIAL_BUF, REF_OBS,
  REF_REWARD, REF_LATCHES, REF_PIX, REF_PIX_PACKED, REF_DATA_BYTES
};

RefMachine* ref_create(int num_envs, const uint8_t* rom, int64_t rom_len,
                       const uint8_t* boot, int boot_len, int obs_dim);
void ref_destroy(RefMachine* m);
/* Initial state of backends/warp_vec.py:249-513 (without the 0-frame launch). */
int ref_reset(RefMachine* m);
/* One launch of cpu_step over envs [lo, hi) with nthreads OpenMP threads.
 * stage: 0 emulate_only, 1 reward_only, 2 obs_only, 3 full_step. */
int ref_step(RefMachine* m, const int32_t* actions, int frames_to_run,
             int release_after_frames, int stage, int env_lo, int env_hi,
             int nthreads);
/* Snapshot renderer into the machine's pix (packed=0) or pix_packed buffer. */
int ref_render(RefMachine* m, int packed, int nthreads);
/* Env 0's 160x144 shade frame from its scanline latches (kernels/ppu_step.py). */
int ref_render_bg_env0(RefMachine* m, uint8_t* out);
int ref_snapshot(RefMachine* m, int env_idx);
int ref_masked_reset(RefMachine* m, const uint8_t* mask);
void* ref_field_ptr(RefMachine* m, int field, int64_t* nbytes, int* elem_size);
int ref_num_envs(RefMachine* m);

#ifdef __cplusplus
}
#endif

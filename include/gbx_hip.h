/*
 * gbx_hip.h -- C ABI of the MI355X (gfx950) vectorized Game Boy core.
 *
 * One context holds N Game Boys.  All state lives in device memory owned by
 * the library; callers pass device pointers for per-step inputs/outputs
 * (actions, masks, observation buffers) and the HIP stream to enqueue on.
 * Launch entry points never synchronize; the export/import helpers do.
 *
 * The reference (bkase/gbxcule) has no C ABI: its operator boundary is
 * wp.launch(cpu_step, dim=N, inputs=[55 arrays]) inside the Python backend
 * src/gbxcule/backends/warp_vec.py.  Each entry point below names the
 * reference method whose effect it reproduces.
 *
 * Every function returns 0 on success or a negative GBX_E* code; the message
 * of the last failure on the calling thread is gbx_last_error().
 */
#ifndef GBX_HIP_H
#define GBX_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gbx_ctx gbx_ctx;

enum {
  GBX_OK = 0,
  GBX_E_INVALID = -1,   /* bad argument (reference: ValueError / TypeError) */
  GBX_E_STATE = -2,     /* call out of order (reference: RuntimeError) */
  GBX_E_HIP = -3,       /* HIP runtime failure */
  GBX_E_UNSUPPORTED = -4 /* cartridge type/size not supported */
};

/* Per-env scalar fields for gbx_export_scalar / gbx_import_scalar, in the
 * order of the reference ABI arrays (backends/warp_vec.py:346-470). */
enum {
  GBX_FIELD_PC = 0, GBX_FIELD_SP, GBX_FIELD_A, GBX_FIELD_B, GBX_FIELD_C,
  GBX_FIELD_D, GBX_FIELD_E, GBX_FIELD_H, GBX_FIELD_L, GBX_FIELD_F,
  GBX_FIELD_INSTR_COUNT, GBX_FIELD_CYCLE_COUNT, GBX_FIELD_CYCLE_IN_FRAME,
  GBX_FIELD_TRAP_FLAG, GBX_FIELD_TRAP_PC, GBX_FIELD_TRAP_OPCODE,
  GBX_FIELD_TRAP_KIND, GBX_FIELD_ACTIONS, GBX_FIELD_JOYP_SELECT,
  GBX_FIELD_SERIAL_LEN, GBX_FIELD_SERIAL_OVERFLOW, GBX_FIELD_IME,
  GBX_FIELD_IME_DELAY, GBX_FIELD_HALTED, GBX_FIELD_DIV_COUNTER,
  GBX_FIELD_TIMER_PREV_IN, GBX_FIELD_TIMA_RELOAD_PENDING,
  GBX_FIELD_TIMA_RELOAD_DELAY, GBX_FIELD_PPU_SCANLINE_CYCLE, GBX_FIELD_PPU_LY,
  GBX_FIELD_PPU_WINDOW_LINE, GBX_FIELD_PPU_STAT_PREV, GBX_NUM_FIELDS
};

/* Stage of the fused post-step (reference kernels/cpu_step.py:328-341). */
enum { GBX_STAGE_EMULATE_ONLY = 0, GBX_STAGE_REWARD_ONLY = 1,
       GBX_STAGE_OBS_ONLY = 2, GBX_STAGE_FULL_STEP = 3 };

/* Buffers exposed for zero-copy views (gbx_buffer). */
enum {
  GBX_BUF_MEM = 0,        /* u8, 64-env blocks: [(N+63)/64][65536][64]; once handed out,
                            gbx_masked_reset also restores the rows the step never
                            writes (below 0x8000, A000-BFFF, E000-FDFF)
                            (gbx_read_mem / gbx_write_mem reach memory without it) */
  GBX_BUF_PIX = 1,        /* u8 [N][72][80] unpacked 2-bit shades */
  GBX_BUF_PIX_PACKED = 2, /* u8 [N][72][20] packed, 4 shades per byte */
  GBX_BUF_OBS = 3,        /* f32 [N][obs_dim] */
  GBX_BUF_REWARD = 4,     /* f32 [N] */
  GBX_BUF_ACTIONS = 5,    /* i32 [N] internal action buffer */
  GBX_BUF_CART_RAM = 6,   /* u8, 64-env blocks: [(N+63)/64][ram_stride][64] */
  GBX_BUF_FRAME_BG = 7    /* u8 [144][160] env-0 frame shades (gbx_render_bg_env0) */
};

/* gbx_info keys. */
enum { GBX_INFO_NUM_ENVS = 0, GBX_INFO_PADDED_ENVS, GBX_INFO_ROM_BANKS,
       GBX_INFO_ROM_BANK_MASK, GBX_INFO_RAM_BANKS, GBX_INFO_RAM_BYTES,
       GBX_INFO_MBC_KIND, GBX_INFO_OBS_DIM, GBX_INFO_CART_RAM_STRIDE,
       GBX_INFO_STEP_LANES };

const char* gbx_last_error(void);
int gbx_version(void);

/* Allocate N Game Boys for a cartridge (header parsed as
 * core/cartridge.py:139-187) and put them in the reset state.  Replaces
 * WarpVecCudaBackend.__init__ + reset() (backends/warp_vec.py:89-513). */
int gbx_create(int32_t num_envs, const uint8_t* rom, int64_t rom_len,
               const uint8_t* boot, int32_t boot_len, int32_t obs_dim,
               gbx_ctx** out);
int gbx_destroy(gbx_ctx* ctx);

/* Power-on state: registers 0, boot ROM overlay on, ROM bank 1,
 * JOYP select 0x30, memory zero but the boot image at 0x0000-0x00FF.
 * Replaces WarpVecBaseBackend.reset (backends/warp_vec.py:249-498). */
int gbx_reset(gbx_ctx* ctx, void* stream);

/* Upload host int32[N] actions into the internal action buffer
 * (replaces the actions.assign(...) of step(), backends/warp_vec.py:538-549). */
int gbx_upload_actions(gbx_ctx* ctx, const int32_t* host_actions, void* stream);

/* Run frames_to_run frames on every env (one cpu_step launch,
 * backends/warp_vec.py:565-650 / step_torch 1234-1269).  actions_dev may be
 * NULL to use the internal buffer.  Writes obs/reward per stage. */
int gbx_step(gbx_ctx* ctx, const int32_t* actions_dev, int32_t frames_to_run,
             int32_t release_after_frames, int32_t stage, void* stream);

/* Snapshot 2x-downsampled render of every env (kernels/
 * ppu_render_downsampled.py:183-234; render_pixels_snapshot_packed_to_torch,
 * backends/warp_vec.py:1293-1352).  out_dev NULL selects the internal pix /
 * pix_packed buffer; base_offset is in bytes. */
int gbx_render(gbx_ctx* ctx, uint8_t* out_dev, int64_t base_offset,
               int32_t packed, void* stream);

/* Env 0's full 160x144 frame of shades 0-3 from the scanline latches its
 * last step captured (kernels/ppu_step.py:12-176, launched after cpu_step
 * when render_bg is set, backends/warp_vec.py:651-670).  out_dev NULL
 * selects the internal GBX_BUF_FRAME_BG buffer. */
int gbx_render_bg_env0(gbx_ctx* ctx, uint8_t* out_dev, void* stream);

/* Capture env_idx as the reset snapshot (ResetCache.from_backend,
 * core/reset_cache.py:68-190); with_pix also snapshots the pix buffer. */
int gbx_snapshot(gbx_ctx* ctx, int32_t env_idx, int32_t with_pix, void* stream);

/* Restore the snapshot into every env whose mask byte is non-zero
 * (ResetCache.apply_mask_torch, core/reset_cache.py:192-307, 381-411). */
int gbx_masked_reset(gbx_ctx* ctx, const uint8_t* mask_dev, void* stream);

/* out_dev[env*k + j] = raw mem byte addrs_dev[j] of env, for all envs
 * (the memory_torch()[:, addr] sense reads of rl/pokered_packed_parcel_env.py
 * :383-391, done as one gather because memory is 64-env interleaved). */
int gbx_gather_mem(gbx_ctx* ctx, const uint16_t* addrs_dev, int32_t k,
                   uint8_t* out_dev, void* stream);

/* Device-to-device copy of memory bytes [lo, hi) of envs [env_lo, env_hi)
 * into out_dev, env-major: out_dev[(env - env_lo) * (hi - lo) + (addr - lo)].
 * It serves the indexing the reference's callers apply to the env-major
 * [N, 65536] memory_torch() view (backends/warp_vec.py:799-810), e.g.
 * mem[:, lo:hi] and mem[:, addr] in rl/pokered_packed_parcel_env.py:
 * 274-291, 387-391.  Enqueued on the stream; never synchronizes. */
int gbx_read_mem(gbx_ctx* ctx, int32_t env_lo, int32_t env_hi, int32_t lo,
                 int32_t hi, uint8_t* out_dev, void* stream);

/* The reverse: in_dev (same env-major layout) into the rectangle.  Writes
 * through the reference's memory_torch() view (mem[:, 0xFF40] |= 0x80,
 * the LCDC override of backends/warp_vec.py:734-757) land here.  A write
 * that reaches a row the step never writes (below 0x8000, A000-BFFF,
 * E000-FDFF) makes gbx_masked_reset restore those rows from then on. */
int gbx_write_mem(gbx_ctx* ctx, int32_t env_lo, int32_t env_hi, int32_t lo,
                  int32_t hi, const uint8_t* in_dev, void* stream);

/* Per-env 64-bit linear hash of mem and registers (no reference
 * counterpart: lets callers compare full state without a readback). */
int gbx_state_hash(gbx_ctx* ctx, uint64_t* out_dev, void* stream);

/* Synchronous readback / writeback helpers (get_cpu_state 947-1009,
 * read_memory 766-797, get_cart_state 1011-1022, read_serial 1409-1431,
 * write_memory 899-911 of backends/warp_vec.py). */
int gbx_export_scalar(gbx_ctx* ctx, int32_t field, int64_t* host_out);
int gbx_import_scalar(gbx_ctx* ctx, int32_t field, const int64_t* host_in);
int gbx_export_mem(gbx_ctx* ctx, int32_t env_lo, int32_t env_hi, int32_t lo,
                   int32_t hi, uint8_t* host_out);
/* gbx_import_mem and gbx_import_env write the rows the step never writes
 * (below 0x8000, A000-BFFF, E000-FDFF) only as data: while every such row
 * still holds the power-on fill (boot image at 0x00-0xFF, zero elsewhere),
 * gbx_masked_reset keeps skipping them. */
int gbx_import_mem(gbx_ctx* ctx, int32_t env, int32_t addr,
                   const uint8_t* host_in, int32_t len);
int gbx_export_cart_state(gbx_ctx* ctx, int32_t* host_out);
int gbx_import_cart_state(gbx_ctx* ctx, const int32_t* host_in);
int gbx_export_cart_ram(gbx_ctx* ctx, int32_t env_lo, int32_t env_hi,
                        uint8_t* host_out);
int gbx_export_serial(gbx_ctx* ctx, uint8_t* host_out);
int gbx_export_latches(gbx_ctx* ctx, uint8_t* host_out);

/* One env's whole state in one synchronous call: scalars[GBX_NUM_FIELDS]
 * (GBX_FIELD_* order), cart_state[20], mem[65536] raw memory image and
 * cart_ram[GBX_INFO_RAM_BYTES] (NULL: not copied).  This is the device side
 * of state_from_warp_backend / apply_state_to_warp_backend
 * (core/state_io.py:662-837, 839-1154), which the reference does with one
 * Warp array copy per field; the savestate file format itself is host code
 * (gbxcule_amd/state_io.py).  gbx_import_env writes every scalar, slot and
 * memory byte given; cart_ram and the env-0 scanline latches (latches[9*144],
 * order LCDC, SCX, SCY, BGP, WX, WY, window line, OBP0, OBP1) are written
 * only when non-NULL. */
int gbx_export_env(gbx_ctx* ctx, int32_t env, int64_t* scalars, int32_t* cart_state,
                   uint8_t* mem, uint8_t* cart_ram);
/* gbx_export_env that allocates nothing: no counterpart in the reference.
 * For callers that cannot allocate device memory (tight serving loops,
 * harnesses that forbid hipMalloc).  The env image is staged in a static
 * 128 KiB device array that each GPU holds until the process ends, so carts
 * with more than 32 KiB of cart RAM are rejected (GBX_E_UNSUPPORTED) and
 * calls that overlap on one GPU race.  Like gbx_export_env it synchronizes
 * the device and copies to host memory synchronously, so it is not for use
 * under stream capture.  Same outputs as gbx_export_env; the context's
 * device must be current. */
int gbx_export_env_noalloc(gbx_ctx* ctx, int32_t env, int64_t* scalars,
                           int32_t* cart_state, uint8_t* mem, uint8_t* cart_ram);
int gbx_import_env(gbx_ctx* ctx, int32_t env, const int64_t* scalars,
                   const int32_t* cart_state, const uint8_t* mem,
                   const uint8_t* cart_ram, const uint8_t* latches);

int gbx_buffer(gbx_ctx* ctx, int32_t which, void** dev_ptr, int64_t* nbytes);
int gbx_info(gbx_ctx* ctx, int32_t key, int64_t* out);

/* Debug traps (kernels/cpu_step.py:85-114, GBXCULE_TRAP_RST38 / _TRAP_PC /
 * _MAX_INSTR / _WATCH_ADDR); zero disables each. */
int gbx_set_debug(gbx_ctx* ctx, int32_t rst38, int32_t trap_pc,
                  int32_t max_instr, int32_t watch_addr);

#ifdef __cplusplus
}
#endif
#endif /* GBX_HIP_H */

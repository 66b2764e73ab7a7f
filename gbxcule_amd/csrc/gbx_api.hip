// gbx_api.hip -- host implementation of the C ABI declared in include/gbx_hip.h.
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/gbx_hip.h"
#include "gbx_aux.h"
#include "gbx_decode.h"

using namespace gbx;

// Static scratch of gbx_export_env_noalloc: one env image (scalars, cart
// state, 64 KiB of memory, cart RAM, scanline latches) staged between the
// gather kernel and the copies to the caller's host buffers.  128 KiB holds
// the image of every cart with at most 32 KiB of cart RAM.  Each GPU the
// library runs on holds its own copy until the process ends; every call on
// one GPU reuses it, so calls that overlap on one GPU race.  In host code the
// name is only a stand-in: kernels get the device address taken once per
// device with hipGetSymbolAddress (scratch_ptr).
constexpr size_t kScratchBytes = 128 * 1024;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

struct gbx_ctx {
  DevState s{};
  int device = 0;  // the device current at gbx_create
  SnapState snap{};
  bool snap_valid = false;
  // Set once anything but the power-on fill may have written a memory row
  // the step never writes: below 0x8000 (ROM-window writes go to the MBC),
  // A000-BFFF (cartridge-RAM writes go to the cartridge RAM buffer) and
  // E000-FDFF (echo writes fold to C000-DDFF).  Set by an import there, a
  // gbx_write_mem there, or the raw memory pointer handed out.  While it is
  // clear every env and the snapshot hold the power-on bytes in those rows,
  // and a masked restore skips them.
  bool dead_rows_dirty = false;
  std::vector<uint8_t> boot_host;  // the power-on fill of rows 0x00-0xFF
  uint64_t* hash_k = nullptr;
  int dbg[4] = {0, 0, 0, 0};
};

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

#define HIP_TRY(expr)                                                              \
  do {                                                                             \
    hipError_t _e = (expr);                                                        \
    if (_e != hipSuccess)                                                          \
      return fail(GBX_E_HIP, std::string(#expr) + ": " + hipGetErrorString(_e));   \
  } while (0)

#define CHECK_CTX(ctx)                                                     \
  do {                                                                     \
    if (!(ctx)) return fail(GBX_E_INVALID, "context is NULL");             \
  } while (0)

uint64_t splitmix(uint64_t i) {
  uint64_t z = (i + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

constexpr int kHashLen = kMemSize + 128;

// Device address of `scratch` per device, taken once per device with that
// device current (gbx_create) and kept for the life of the process.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_setup(int dev) {
  if (dev < 0 || dev >= kMaxDevices) return fail(GBX_E_UNSUPPORTED, "device ordinal out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] != nullptr) return GBX_OK;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || p == nullptr)
    return fail(GBX_E_HIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
  g_scratch_ptr[dev] = p;
  return GBX_OK;
}

void* scratch_ptr(int dev) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  return dev >= 0 && dev < kMaxDevices ? g_scratch_ptr[dev] : nullptr;
}

// Rows of the memory image the step never writes.
bool dead_row(int32_t a) { return a < 0x8000 || (a >= 0xA000 && a < 0xC000) || (a >= 0xE000 && a < 0xFE00); }
// True when bytes [addr, addr + len) of an image differ from the power-on
// fill (boot image at 0x00-0xFF, zero elsewhere) in a dead row.
bool differs_from_fill(const gbx_ctx* c, int32_t addr, const uint8_t* bytes, int32_t len) {
  for (int32_t i = 0; i < len; ++i) {
    const int32_t a = addr + i;
    if (!dead_row(a)) continue;
    const uint8_t fill = a < 0x100 ? c->boot_host[(size_t)a] : 0;
    if (bytes[i] != fill) return true;
  }
  return false;
}

void free_ctx(gbx_ctx* c) {
  DevState& s = c->s;
  void* ptrs[] = {s.mem, s.cram, s.cs, s.sc, s.cnt, s.serial, s.actions, s.obs, s.reward,
                  s.pix, s.pix_packed, s.latches, s.frame_bg, (void*)s.rom, (void*)s.boot, (void*)s.recs,
                  c->snap.mem, c->snap.cram, c->snap.serial, c->snap.pix, c->snap.cs,
                  c->snap.sc, c->snap.cnt, c->hash_k};
  for (void* p : ptrs)
    if (p) (void)hipFree(p);
  delete c;
}

template <typename T>
hipError_t dalloc(T** p, size_t count) {
  return hipMalloc(reinterpret_cast<void**>(p), count * sizeof(T) > 0 ? count * sizeof(T) : 1);
}

// The ROM buffer is the ROM, then the boot image, then one 16 KiB window of
// 0xFF that an unmapped ROM bank reads (open bus).
constexpr int64_t kOpenBusBytes = 0x4000;

// Pre-decoded instruction records for the step kernel's fetch: one 512-bit
// record (gbx_decode.h) per byte of the ROM buffer, built from that byte and
// the next two bytes of the same image.  Bytes past the end of an image read
// as 0; the kernel only uses a record when all three instruction bytes lie
// inside one 16 KiB ROM window or inside the boot image.
std::vector<Rec> build_records(const uint8_t* rom, int64_t rom_bytes, const uint8_t* boot) {
  std::vector<Rec> r((size_t)(rom_bytes + 0x100 + kOpenBusBytes));
  auto fill = [&](const uint8_t* img, int64_t len, size_t base) {
    for (int64_t i = 0; i < len; ++i) {
      const uint32_t op = img[i], b1 = i + 1 < len ? img[i + 1] : 0u,
                     b2 = i + 2 < len ? img[i + 2] : 0u;
      r[base + (size_t)i] = decode_insn(op, b1, b2);
    }
  };
  fill(rom, rom_bytes, 0);
  // LY poll loops and block-copy loops whose bytes lie inside one 16 KiB window
  for (int64_t i = 0; i + 5 < rom_bytes; ++i) {
    const uint32_t pl = poll_loop_len(rom + i, (uint32_t)std::min<int64_t>(8, rom_bytes - i));
    if (pl != 0u && (i & 0x3FFF) + pl <= 0x4000) r[(size_t)i] = mark_poll_loop(r[(size_t)i], rom + i);
    if ((i & 0x3FFF) <= 0x3FF8 && i + 7 < rom_bytes && copy_loop_at(rom + i)) r[(size_t)i] = mark_copy_loop(r[(size_t)i]);
  }
  fill(boot, 0x100, (size_t)rom_bytes);
  const std::vector<uint8_t> ff(kOpenBusBytes, 0xFF);
  fill(ff.data(), kOpenBusBytes, (size_t)rom_bytes + 0x100);
  return r;
}

// Header parse (reference core/cartridge.py:139-187).
int parse_header(const uint8_t* rom, int64_t rom_len, int* kind, int64_t* rom_bytes,
                 int* ram_bytes) {
  if (rom_len < 0x150) return fail(GBX_E_INVALID, "ROM too small for header");
  const int type = rom[0x147], rc = rom[0x148], ramc = rom[0x149];
  if (type == 0x00) *kind = MBC_ROM_ONLY;
  else if (type >= 0x01 && type <= 0x03) *kind = MBC_MBC1;
  else if (type >= 0x0F && type <= 0x13) *kind = MBC_MBC3;
  else return fail(GBX_E_UNSUPPORTED, "unsupported cartridge type " + std::to_string(type));
  if (rc > 0x08) return fail(GBX_E_UNSUPPORTED, "unsupported ROM size code " + std::to_string(rc));
  *rom_bytes = (int64_t)(32 * 1024) << rc;
  static const int ram_map[6] = {0, 2048, 8192, 32768, 131072, 65536};
  if (ramc > 5) return fail(GBX_E_UNSUPPORTED, "unsupported RAM size code " + std::to_string(ramc));
  *ram_bytes = ram_map[ramc];
  if (rom_len < *rom_bytes) return fail(GBX_E_INVALID, "ROM smaller than header advertises");
  return GBX_OK;
}

// Envs per step-kernel wavefront.  Each env is a serial instruction stream,
// so a wavefront's time per emulated instruction is set by its dependent
// memory round trips, not by how many lanes it carries.  Below ~4 wavefronts
// per CU some SIMDs would sit idle, so small env counts are spread over
// narrower workgroups (64 -> 32 -> 16 -> 8 envs) until every SIMD holds one.
// GBX_STEP_LANES=64|32|16|8|4 overrides the choice (for tuning sweeps).
int choose_step_lanes(int n) {
  if (const char* v = getenv("GBX_STEP_LANES")) {
    const int l = atoi(v);
    if (l == 4 || l == 8 || l == 16 || l == 32 || l == 64) return l;
  }
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) {
    int x = 0;
    if (hipDeviceGetAttribute(&x, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && x > 0)
      cus = x;
  }
  int lanes = kEnvBlock;
  while (lanes > 8 && (n + lanes - 1) / lanes < 4 * cus) lanes >>= 1;
  return lanes;
}

// Envs [env_lo, env_hi) x addresses [lo, hi) inside the context.
int check_rect(const gbx_ctx* ctx, int32_t env_lo, int32_t env_hi, int32_t lo, int32_t hi) {
  if (env_lo < 0 || env_hi > ctx->s.n || env_lo > env_hi)
    return fail(GBX_E_INVALID, "env range out of bounds");
  if (lo < 0 || hi > kMemSize || lo > hi) return fail(GBX_E_INVALID, "address range out of bounds");
  return GBX_OK;
}

}  // namespace

extern "C" {

const char* gbx_last_error(void) { return g_err.c_str(); }
int gbx_version(void) { return 1; }

int gbx_create(int32_t num_envs, const uint8_t* rom, int64_t rom_len, const uint8_t* boot,
               int32_t boot_len, int32_t obs_dim, gbx_ctx** out) {
  if (!out) return fail(GBX_E_INVALID, "out is NULL");
  *out = nullptr;
  if (num_envs <= 0) return fail(GBX_E_INVALID, "num_envs must be > 0");
  if (!rom || !boot) return fail(GBX_E_INVALID, "rom/boot is NULL");
  if (boot_len != 0x100) return fail(GBX_E_INVALID, "boot ROM must be 256 bytes");
  if (obs_dim != 32) return fail(GBX_E_INVALID, "obs_dim must be 32");
  int kind, ram_bytes;
  int64_t rom_bytes;
  int rc = parse_header(rom, rom_len, &kind, &rom_bytes, &ram_bytes);
  if (rc) return rc;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(GBX_E_HIP, "hipGetDevice failed");
  if ((rc = scratch_setup(dev)) != GBX_OK) return rc;

  auto* c = new gbx_ctx();
  c->boot_host.assign(boot, boot + 0x100);
  c->device = dev;
  DevState& s = c->s;
  s.n = num_envs;
  s.npad = (num_envs + kEnvBlock - 1) & ~(kEnvBlock - 1);
  s.obs_dim = obs_dim;
  s.rom_banks = (int)(rom_bytes / 0x4000);
  s.rom_mask = (s.rom_banks & (s.rom_banks - 1)) == 0 ? s.rom_banks - 1 : -1;
  s.ram_bytes = ram_bytes;
  s.ram_banks = ram_bytes / 0x2000;
  s.cram_stride = ram_bytes > 0 ? ram_bytes : 1;
  s.mbc_kind = kind;
  s.rom_len = rom_bytes;
  s.step_lanes = choose_step_lanes(num_envs);
  const size_t np = (size_t)s.npad;
  hipError_t e = hipSuccess;
  auto A = [&](hipError_t r) {
    if (e == hipSuccess) e = r;
  };
  A(dalloc(&s.mem, np * kMemSize));
  A(dalloc(&s.cram, np * (size_t)s.cram_stride));
  A(dalloc(&s.cs, np * kCartStateStride));
  A(dalloc(&s.sc, np * kNumFields));
  A(dalloc(&s.cnt, np * 2));
  A(dalloc(&s.serial, np * kSerialMax));
  A(dalloc(&s.actions, np));
  A(dalloc(&s.obs, (size_t)num_envs * obs_dim));
  A(dalloc(&s.reward, (size_t)num_envs));
  A(dalloc(&s.pix, (size_t)num_envs * kDsW * kDsH));
  A(dalloc(&s.pix_packed, (size_t)num_envs * kDsWB * kDsH));
  A(dalloc(&s.latches, (size_t)kScreenH * kLatchStride));
  A(dalloc(&s.frame_bg, (size_t)kScreenW * kScreenH));
  uint8_t *drom = nullptr, *dboot = nullptr;
  Rec* drecs = nullptr;
  A(dalloc(&drom, (size_t)(rom_bytes + 0x100 + kOpenBusBytes)));
  A(dalloc(&dboot, (size_t)0x100));
  A(dalloc(&drecs, (size_t)(rom_bytes + 0x100 + kOpenBusBytes)));
  s.rom = drom;
  s.boot = dboot;
  s.recs = reinterpret_cast<const uint4*>(drecs);
  A(dalloc(&c->snap.mem, (size_t)kMemSize));
  A(dalloc(&c->snap.cram, (size_t)s.cram_stride));
  A(dalloc(&c->snap.serial, (size_t)kSerialMax));
  A(dalloc(&c->snap.pix, (size_t)kDsW * kDsH));
  A(dalloc(&c->snap.cs, (size_t)kCartStateStride));
  A(dalloc(&c->snap.sc, (size_t)kNumFields));
  A(dalloc(&c->snap.cnt, (size_t)2));
  A(dalloc(&c->hash_k, (size_t)kHashLen));
  if (e != hipSuccess) {
    free_ctx(c);
    return fail(GBX_E_HIP, std::string("device allocation failed: ") + hipGetErrorString(e));
  }
  std::vector<uint64_t> k(kHashLen);
  for (int i = 0; i < kHashLen; ++i) k[i] = splitmix((uint64_t)i);
  const std::vector<Rec> recs = build_records(rom, rom_bytes, boot);
  A(hipMemcpy(drom, rom, (size_t)rom_bytes, hipMemcpyHostToDevice));
  A(hipMemcpy(drom + rom_bytes, boot, 0x100, hipMemcpyHostToDevice));
  A(hipMemset(drom + rom_bytes + 0x100, 0xFF, (size_t)kOpenBusBytes));
  A(hipMemcpy(dboot, boot, 0x100, hipMemcpyHostToDevice));
  A(hipMemcpy(drecs, recs.data(), recs.size() * sizeof(Rec), hipMemcpyHostToDevice));
  A(hipMemcpy(c->hash_k, k.data(), k.size() * 8, hipMemcpyHostToDevice));
  if (e != hipSuccess) {
    free_ctx(c);
    return fail(GBX_E_HIP, std::string("upload failed: ") + hipGetErrorString(e));
  }
  rc = gbx_reset(c, nullptr);
  if (rc) {
    free_ctx(c);
    return rc;
  }
  if ((e = hipDeviceSynchronize()) != hipSuccess) {
    free_ctx(c);
    return fail(GBX_E_HIP, std::string("reset failed: ") + hipGetErrorString(e));
  }
  *out = c;
  return GBX_OK;
}

int gbx_destroy(gbx_ctx* ctx) {
  CHECK_CTX(ctx);
  (void)hipDeviceSynchronize();
  free_ctx(ctx);
  return GBX_OK;
}

int gbx_reset(gbx_ctx* ctx, void* stream) {
  CHECK_CTX(ctx);
  DevState& s = ctx->s;
  hipStream_t st = (hipStream_t)stream;
  const size_t np = (size_t)s.npad;
  HIP_TRY(hipMemsetAsync(s.cram, 0, np * (size_t)s.cram_stride, st));
  HIP_TRY(hipMemsetAsync(s.cnt, 0, np * 2 * sizeof(int64_t), st));
  HIP_TRY(hipMemsetAsync(s.serial, 0, np * kSerialMax, st));
  HIP_TRY(hipMemsetAsync(s.actions, 0, np * sizeof(int32_t), st));
  HIP_TRY(hipMemsetAsync(s.obs, 0, (size_t)s.n * s.obs_dim * sizeof(float), st));
  HIP_TRY(hipMemsetAsync(s.reward, 0, (size_t)s.n * sizeof(float), st));
  HIP_TRY(hipMemsetAsync(s.pix, 0, (size_t)s.n * kDsW * kDsH, st));
  HIP_TRY(hipMemsetAsync(s.pix_packed, 0, (size_t)s.n * kDsWB * kDsH, st));
  HIP_TRY(hipMemsetAsync(s.latches, 0, (size_t)kScreenH * kLatchStride, st));
  HIP_TRY(hipMemsetAsync(s.frame_bg, 0, (size_t)kScreenW * kScreenH, st));
  HIP_TRY(launch_reset(s, st));
  return GBX_OK;
}

int gbx_upload_actions(gbx_ctx* ctx, const int32_t* host_actions, void* stream) {
  CHECK_CTX(ctx);
  if (!host_actions) return fail(GBX_E_INVALID, "actions is NULL");
  HIP_TRY(hipMemcpyAsync(ctx->s.actions, host_actions, (size_t)ctx->s.n * sizeof(int32_t),
                         hipMemcpyHostToDevice, (hipStream_t)stream));
  return GBX_OK;
}

int gbx_step(gbx_ctx* ctx, const int32_t* actions_dev, int32_t frames_to_run,
             int32_t release_after_frames, int32_t stage, void* stream) {
  CHECK_CTX(ctx);
  if (frames_to_run < 0) return fail(GBX_E_INVALID, "frames_to_run must be >= 0");
  if (stage < 0 || stage > 3) return fail(GBX_E_INVALID, "stage must be 0..3");
  StepArgs a{};
  a.actions = actions_dev ? actions_dev : ctx->s.actions;
  a.frames = frames_to_run;
  a.release = release_after_frames;
  a.stage = stage;
  a.dbg_rst38 = ctx->dbg[0];
  a.dbg_trap_pc = ctx->dbg[1];
  a.dbg_max_instr = ctx->dbg[2];
  a.dbg_watch = ctx->dbg[3];
  HIP_TRY(launch_step(ctx->s, a, (hipStream_t)stream));
  return GBX_OK;
}

int gbx_render(gbx_ctx* ctx, uint8_t* out_dev, int64_t base_offset, int32_t packed, void* stream) {
  CHECK_CTX(ctx);
  if (base_offset < 0) return fail(GBX_E_INVALID, "base_offset must be >= 0");
  uint8_t* out = out_dev;
  if (!out) {
    if (base_offset != 0) return fail(GBX_E_INVALID, "base_offset needs an output buffer");
    out = packed ? ctx->s.pix_packed : ctx->s.pix;
  }
  HIP_TRY(launch_render(ctx->s, out, base_offset, packed ? 1 : 0, (hipStream_t)stream));
  return GBX_OK;
}

int gbx_render_bg_env0(gbx_ctx* ctx, uint8_t* out_dev, void* stream) {
  CHECK_CTX(ctx);
  HIP_TRY(launch_render_bg_env0(ctx->s, out_dev ? out_dev : ctx->s.frame_bg,
                                (hipStream_t)stream));
  return GBX_OK;
}

int gbx_snapshot(gbx_ctx* ctx, int32_t env_idx, int32_t with_pix, void* stream) {
  CHECK_CTX(ctx);
  if (env_idx < 0 || env_idx >= ctx->s.n)
    return fail(GBX_E_INVALID, "env_idx out of range");
  ctx->snap.has_pix = with_pix ? 1 : 0;
  HIP_TRY(launch_snapshot(ctx->s, ctx->snap, env_idx, ctx->snap.has_pix, (hipStream_t)stream));
  ctx->snap_valid = true;
  return GBX_OK;
}

int gbx_masked_reset(gbx_ctx* ctx, const uint8_t* mask_dev, void* stream) {
  CHECK_CTX(ctx);
  if (!ctx->snap_valid) return fail(GBX_E_STATE, "no snapshot: call gbx_snapshot first");
  if (!mask_dev) return fail(GBX_E_INVALID, "mask is NULL");
  HIP_TRY(launch_masked_reset(ctx->s, ctx->snap, mask_dev, ctx->dead_rows_dirty ? 0 : 1,
                              (hipStream_t)stream));
  return GBX_OK;
}

int gbx_gather_mem(gbx_ctx* ctx, const uint16_t* addrs_dev, int32_t k, uint8_t* out_dev,
                   void* stream) {
  CHECK_CTX(ctx);
  if (k < 0 || (k > 0 && (!addrs_dev || !out_dev)))
    return fail(GBX_E_INVALID, "bad gather arguments");
  HIP_TRY(launch_gather(ctx->s, addrs_dev, k, out_dev, (hipStream_t)stream));
  return GBX_OK;
}

int gbx_read_mem(gbx_ctx* ctx, int32_t env_lo, int32_t env_hi, int32_t lo, int32_t hi,
                 uint8_t* out_dev, void* stream) {
  CHECK_CTX(ctx);
  if (const int rc = check_rect(ctx, env_lo, env_hi, lo, hi)) return rc;
  if (env_lo == env_hi || lo == hi) return GBX_OK;
  if (!out_dev) return fail(GBX_E_INVALID, "out is NULL");
  HIP_TRY(launch_mem_range(ctx->s, env_lo, env_hi - env_lo, lo, hi - lo, out_dev, 0,
                           (hipStream_t)stream));
  return GBX_OK;
}

int gbx_write_mem(gbx_ctx* ctx, int32_t env_lo, int32_t env_hi, int32_t lo, int32_t hi,
                  const uint8_t* in_dev, void* stream) {
  CHECK_CTX(ctx);
  if (const int rc = check_rect(ctx, env_lo, env_hi, lo, hi)) return rc;
  if (env_lo == env_hi || lo == hi) return GBX_OK;
  if (!in_dev) return fail(GBX_E_INVALID, "in is NULL");
  // the bytes are on the device: a write reaching a dead row may change it
  if (lo < 0x8000 || (lo < 0xC000 && hi > 0xA000) || (lo < 0xFE00 && hi > 0xE000)) ctx->dead_rows_dirty = true;
  HIP_TRY(launch_mem_range(ctx->s, env_lo, env_hi - env_lo, lo, hi - lo,
                           const_cast<uint8_t*>(in_dev), 1, (hipStream_t)stream));
  return GBX_OK;
}

int gbx_state_hash(gbx_ctx* ctx, uint64_t* out_dev, void* stream) {
  CHECK_CTX(ctx);
  if (!out_dev) return fail(GBX_E_INVALID, "out is NULL");
  HIP_TRY(launch_hash(ctx->s, ctx->hash_k, out_dev, (hipStream_t)stream));
  return GBX_OK;
}

int gbx_export_scalar(gbx_ctx* ctx, int32_t field, int64_t* host_out) {
  CHECK_CTX(ctx);
  if (!host_out) return fail(GBX_E_INVALID, "out is NULL");
  if (field < 0 || field >= GBX_NUM_FIELDS) return fail(GBX_E_INVALID, "bad field id");
  const DevState& s = ctx->s;
  HIP_TRY(hipDeviceSynchronize());
  if (field == GBX_FIELD_INSTR_COUNT || field == GBX_FIELD_CYCLE_COUNT) {
    std::vector<int64_t> h((size_t)s.npad * 2);
    HIP_TRY(hipMemcpy(h.data(), s.cnt, h.size() * 8, hipMemcpyDeviceToHost));
    const int slot = field == GBX_FIELD_INSTR_COUNT ? 0 : 1;
    for (int e = 0; e < s.n; ++e) host_out[e] = h[cnt_index((uint32_t)e, slot)];
  } else if (field == GBX_FIELD_ACTIONS) {
    std::vector<int32_t> h((size_t)s.n);
    HIP_TRY(hipMemcpy(h.data(), s.actions, h.size() * 4, hipMemcpyDeviceToHost));
    for (int e = 0; e < s.n; ++e) host_out[e] = h[e];
  } else {
    std::vector<int32_t> h((size_t)s.npad * kNumFields);
    HIP_TRY(hipMemcpy(h.data(), s.sc, h.size() * 4, hipMemcpyDeviceToHost));
    for (int e = 0; e < s.n; ++e) host_out[e] = h[sc_index((uint32_t)e, field)];
  }
  return GBX_OK;
}

int gbx_import_scalar(gbx_ctx* ctx, int32_t field, const int64_t* host_in) {
  CHECK_CTX(ctx);
  if (!host_in) return fail(GBX_E_INVALID, "in is NULL");
  if (field < 0 || field >= GBX_NUM_FIELDS) return fail(GBX_E_INVALID, "bad field id");
  const DevState& s = ctx->s;
  HIP_TRY(hipDeviceSynchronize());
  if (field == GBX_FIELD_INSTR_COUNT || field == GBX_FIELD_CYCLE_COUNT) {
    std::vector<int64_t> h((size_t)s.npad * 2);
    HIP_TRY(hipMemcpy(h.data(), s.cnt, h.size() * 8, hipMemcpyDeviceToHost));
    const int slot = field == GBX_FIELD_INSTR_COUNT ? 0 : 1;
    for (int e = 0; e < s.n; ++e) h[cnt_index((uint32_t)e, slot)] = host_in[e];
    HIP_TRY(hipMemcpy(s.cnt, h.data(), h.size() * 8, hipMemcpyHostToDevice));
  } else if (field == GBX_FIELD_ACTIONS) {
    std::vector<int32_t> h((size_t)s.n);
    for (int e = 0; e < s.n; ++e) h[e] = (int32_t)host_in[e];
    HIP_TRY(hipMemcpy(s.actions, h.data(), h.size() * 4, hipMemcpyHostToDevice));
  } else {
    std::vector<int32_t> h((size_t)s.npad * kNumFields);
    HIP_TRY(hipMemcpy(h.data(), s.sc, h.size() * 4, hipMemcpyDeviceToHost));
    for (int e = 0; e < s.n; ++e) h[sc_index((uint32_t)e, field)] = (int32_t)host_in[e];
    HIP_TRY(hipMemcpy(s.sc, h.data(), h.size() * 4, hipMemcpyHostToDevice));
  }
  return GBX_OK;
}

int gbx_export_mem(gbx_ctx* ctx, int32_t env_lo, int32_t env_hi, int32_t lo, int32_t hi,
                   uint8_t* host_out) {
  CHECK_CTX(ctx);
  if (!host_out) return fail(GBX_E_INVALID, "out is NULL");
  if (const int rc = check_rect(ctx, env_lo, env_hi, lo, hi)) return rc;
  const size_t total = (size_t)(env_hi - env_lo) * (size_t)(hi - lo);
  if (total == 0) return GBX_OK;
  uint8_t* tmp = nullptr;
  HIP_TRY(hipDeviceSynchronize());
  HIP_TRY(hipMalloc(&tmp, total));
  hipError_t e = launch_mem_range(ctx->s, env_lo, env_hi - env_lo, lo, hi - lo, tmp, 0, nullptr);
  if (e == hipSuccess) e = hipMemcpy(host_out, tmp, total, hipMemcpyDeviceToHost);
  (void)hipFree(tmp);
  HIP_TRY(e);
  return GBX_OK;
}

int gbx_import_mem(gbx_ctx* ctx, int32_t env, int32_t addr, const uint8_t* host_in, int32_t len) {
  CHECK_CTX(ctx);
  if (!host_in && len > 0) return fail(GBX_E_INVALID, "in is NULL");
  if (env < 0 || env >= ctx->s.n) return fail(GBX_E_INVALID, "env out of range");
  // len > kMemSize - addr, not addr + len > kMemSize: the sum can overflow
  if (addr < 0 || len < 0 || addr > kMemSize || len > kMemSize - addr)
    return fail(GBX_E_INVALID, "write out of range");
  if (len == 0) return GBX_OK;
  if (differs_from_fill(ctx, addr, host_in, len)) ctx->dead_rows_dirty = true;
  uint8_t* tmp = nullptr;
  HIP_TRY(hipDeviceSynchronize());
  HIP_TRY(hipMalloc(&tmp, (size_t)len));
  hipError_t e = hipMemcpy(tmp, host_in, (size_t)len, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = launch_mem_range(ctx->s, env, 1, addr, len, tmp, 1, nullptr);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  (void)hipFree(tmp);
  HIP_TRY(e);
  return GBX_OK;
}

int gbx_export_cart_state(gbx_ctx* ctx, int32_t* host_out) {
  CHECK_CTX(ctx);
  if (!host_out) return fail(GBX_E_INVALID, "out is NULL");
  const DevState& s = ctx->s;
  std::vector<int32_t> h((size_t)s.npad * kCartStateStride);
  HIP_TRY(hipDeviceSynchronize());
  HIP_TRY(hipMemcpy(h.data(), s.cs, h.size() * 4, hipMemcpyDeviceToHost));
  for (int e = 0; e < s.n; ++e)
    for (int k = 0; k < kCartStateStride; ++k)
      host_out[(size_t)e * kCartStateStride + k] = h[cs_index((uint32_t)e, k)];
  return GBX_OK;
}

int gbx_import_cart_state(gbx_ctx* ctx, const int32_t* host_in) {
  CHECK_CTX(ctx);
  if (!host_in) return fail(GBX_E_INVALID, "in is NULL");
  const DevState& s = ctx->s;
  std::vector<int32_t> h((size_t)s.npad * kCartStateStride);
  HIP_TRY(hipDeviceSynchronize());
  HIP_TRY(hipMemcpy(h.data(), s.cs, h.size() * 4, hipMemcpyDeviceToHost));
  for (int e = 0; e < s.n; ++e)
    for (int k = 0; k < kCartStateStride; ++k)
      h[cs_index((uint32_t)e, k)] = host_in[(size_t)e * kCartStateStride + k];
  HIP_TRY(hipMemcpy(s.cs, h.data(), h.size() * 4, hipMemcpyHostToDevice));
  return GBX_OK;
}

int gbx_export_cart_ram(gbx_ctx* ctx, int32_t env_lo, int32_t env_hi, uint8_t* host_out) {
  CHECK_CTX(ctx);
  if (!host_out) return fail(GBX_E_INVALID, "out is NULL");
  if (env_lo < 0 || env_hi > ctx->s.n || env_lo > env_hi)
    return fail(GBX_E_INVALID, "env range out of bounds");
  const size_t total = (size_t)(env_hi - env_lo) * (size_t)ctx->s.cram_stride;
  if (total == 0) return GBX_OK;
  uint8_t* tmp = nullptr;
  HIP_TRY(hipDeviceSynchronize());
  HIP_TRY(hipMalloc(&tmp, total));
  hipError_t e = launch_export_cram(ctx->s, env_lo, env_hi - env_lo, tmp, nullptr);
  if (e == hipSuccess) e = hipMemcpy(host_out, tmp, total, hipMemcpyDeviceToHost);
  (void)hipFree(tmp);
  HIP_TRY(e);
  return GBX_OK;
}

int gbx_export_serial(gbx_ctx* ctx, uint8_t* host_out) {
  CHECK_CTX(ctx);
  if (!host_out) return fail(GBX_E_INVALID, "out is NULL");
  HIP_TRY(hipDeviceSynchronize());
  HIP_TRY(hipMemcpy(host_out, ctx->s.serial, (size_t)ctx->s.n * kSerialMax,
                    hipMemcpyDeviceToHost));
  return GBX_OK;
}

int gbx_export_latches(gbx_ctx* ctx, uint8_t* host_out) {
  CHECK_CTX(ctx);
  if (!host_out) return fail(GBX_E_INVALID, "out is NULL");
  HIP_TRY(hipDeviceSynchronize());
  uint8_t lines[kScreenH * kLatchStride];
  HIP_TRY(hipMemcpy(lines, ctx->s.latches, sizeof(lines), hipMemcpyDeviceToHost));
  for (int k = 0; k < 9; ++k)
    for (int y = 0; y < kScreenH; ++y) host_out[k * kScreenH + y] = lines[y * kLatchStride + k];
  return GBX_OK;
}

int gbx_export_env(gbx_ctx* ctx, int32_t env, int64_t* scalars, int32_t* cart_state,
                   uint8_t* mem, uint8_t* cart_ram) {
  CHECK_CTX(ctx);
  if (!scalars || !cart_state || !mem) return fail(GBX_E_INVALID, "out is NULL");
  if (env < 0 || env >= ctx->s.n) return fail(GBX_E_INVALID, "env out of range");
  const DevState& s = ctx->s;
  const size_t nb = img_bytes(s.ram_bytes);
  std::vector<uint8_t> h(nb);
  uint8_t* img = nullptr;
  HIP_TRY(hipDeviceSynchronize());
  HIP_TRY(hipMalloc(&img, nb));
  hipError_t e = launch_env_image(s, env, img, 0, 0, nullptr);
  if (e == hipSuccess) e = hipMemcpy(h.data(), img, nb, hipMemcpyDeviceToHost);
  (void)hipFree(img);
  HIP_TRY(e);
  memcpy(scalars, h.data(), sizeof(int64_t) * GBX_NUM_FIELDS);
  memcpy(cart_state, h.data() + kImgCart, sizeof(int32_t) * kCartStateStride);
  memcpy(mem, h.data() + kImgMem, kMemSize);
  if (cart_ram && s.ram_bytes > 0) memcpy(cart_ram, h.data() + kImgCram, (size_t)s.ram_bytes);
  return GBX_OK;
}

int gbx_export_env_noalloc(gbx_ctx* ctx, int32_t env, int64_t* scalars, int32_t* cart_state,
                           uint8_t* mem, uint8_t* cart_ram) {
  CHECK_CTX(ctx);
  if (!scalars || !cart_state || !mem) return fail(GBX_E_INVALID, "out is NULL");
  if (env < 0 || env >= ctx->s.n) return fail(GBX_E_INVALID, "env out of range");
  const DevState& s = ctx->s;
  const size_t nb = img_bytes(s.ram_bytes);
  if (nb > kScratchBytes)
    return fail(GBX_E_UNSUPPORTED, "env image of " + std::to_string(nb) + " bytes exceeds the " +
                                       std::to_string(kScratchBytes) +
                                       "-byte static scratch (cart RAM above 32 KiB); use gbx_export_env");
  int dev = -1;
  HIP_TRY(hipGetDevice(&dev));
  if (dev != ctx->device) return fail(GBX_E_STATE, "the context's device is not the current device");
  uint8_t* img = static_cast<uint8_t*>(scratch_ptr(dev));
  if (img == nullptr) return fail(GBX_E_STATE, "static scratch not set up on this device");
  HIP_TRY(hipDeviceSynchronize());
  HIP_TRY(launch_env_image(s, env, img, 0, 0, nullptr));
  // straight from the scratch into the caller's buffers: no staging copy
  HIP_TRY(hipMemcpy(scalars, img, sizeof(int64_t) * GBX_NUM_FIELDS, hipMemcpyDeviceToHost));
  HIP_TRY(hipMemcpy(cart_state, img + kImgCart, sizeof(int32_t) * kCartStateStride,
                    hipMemcpyDeviceToHost));
  HIP_TRY(hipMemcpy(mem, img + kImgMem, kMemSize, hipMemcpyDeviceToHost));
  if (cart_ram && s.ram_bytes > 0)
    HIP_TRY(hipMemcpy(cart_ram, img + kImgCram, (size_t)s.ram_bytes, hipMemcpyDeviceToHost));
  return GBX_OK;
}

int gbx_import_env(gbx_ctx* ctx, int32_t env, const int64_t* scalars, const int32_t* cart_state,
                   const uint8_t* mem, const uint8_t* cart_ram, const uint8_t* latches) {
  CHECK_CTX(ctx);
  if (!scalars || !cart_state || !mem) return fail(GBX_E_INVALID, "in is NULL");
  if (env < 0 || env >= ctx->s.n) return fail(GBX_E_INVALID, "env out of range");
  // dead rows that still hold the power-on fill keep the flag clear
  if (differs_from_fill(ctx, 0, mem, kMemSize)) ctx->dead_rows_dirty = true;
  const DevState& s = ctx->s;
  const size_t nb = img_bytes(s.ram_bytes);
  std::vector<uint8_t> h(nb, 0);
  memcpy(h.data(), scalars, sizeof(int64_t) * GBX_NUM_FIELDS);
  memcpy(h.data() + kImgCart, cart_state, sizeof(int32_t) * kCartStateStride);
  memcpy(h.data() + kImgMem, mem, kMemSize);
  int parts = 0;
  if (cart_ram && s.ram_bytes > 0) {
    memcpy(h.data() + kImgCram, cart_ram, (size_t)s.ram_bytes);
    parts |= IMG_CRAM;
  }
  if (latches) {
    memcpy(h.data() + img_latches_off(s.ram_bytes), latches, kLatchBytes);
    parts |= IMG_LATCHES;
  }
  uint8_t* img = nullptr;
  HIP_TRY(hipDeviceSynchronize());
  HIP_TRY(hipMalloc(&img, nb));
  hipError_t e = hipMemcpy(img, h.data(), nb, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = launch_env_image(s, env, img, 1, parts, nullptr);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  (void)hipFree(img);
  HIP_TRY(e);
  return GBX_OK;
}

int gbx_buffer(gbx_ctx* ctx, int32_t which, void** dev_ptr, int64_t* nbytes) {
  CHECK_CTX(ctx);
  if (!dev_ptr || !nbytes) return fail(GBX_E_INVALID, "out is NULL");
  const DevState& s = ctx->s;
  switch (which) {
    case GBX_BUF_MEM:  // the caller may write any row through it
      *dev_ptr = s.mem;
      *nbytes = (int64_t)s.npad * kMemSize;
      ctx->dead_rows_dirty = true;
      break;
    case GBX_BUF_PIX: *dev_ptr = s.pix; *nbytes = (int64_t)s.n * kDsW * kDsH; break;
    case GBX_BUF_PIX_PACKED: *dev_ptr = s.pix_packed; *nbytes = (int64_t)s.n * kDsWB * kDsH; break;
    case GBX_BUF_FRAME_BG: *dev_ptr = s.frame_bg; *nbytes = (int64_t)kScreenW * kScreenH; break;
    case GBX_BUF_OBS: *dev_ptr = s.obs; *nbytes = (int64_t)s.n * s.obs_dim * 4; break;
    case GBX_BUF_REWARD: *dev_ptr = s.reward; *nbytes = (int64_t)s.n * 4; break;
    case GBX_BUF_ACTIONS: *dev_ptr = s.actions; *nbytes = (int64_t)s.n * 4; break;
    case GBX_BUF_CART_RAM: *dev_ptr = s.cram; *nbytes = (int64_t)s.npad * s.cram_stride; break;
    default: return fail(GBX_E_INVALID, "unknown buffer id");
  }
  return GBX_OK;
}

int gbx_info(gbx_ctx* ctx, int32_t key, int64_t* out) {
  CHECK_CTX(ctx);
  if (!out) return fail(GBX_E_INVALID, "out is NULL");
  const DevState& s = ctx->s;
  switch (key) {
    case GBX_INFO_NUM_ENVS: *out = s.n; break;
    case GBX_INFO_PADDED_ENVS: *out = s.npad; break;
    case GBX_INFO_ROM_BANKS: *out = s.rom_banks; break;
    case GBX_INFO_ROM_BANK_MASK: *out = s.rom_mask; break;
    case GBX_INFO_RAM_BANKS: *out = s.ram_banks; break;
    case GBX_INFO_RAM_BYTES: *out = s.ram_bytes; break;
    case GBX_INFO_MBC_KIND: *out = s.mbc_kind; break;
    case GBX_INFO_OBS_DIM: *out = s.obs_dim; break;
    case GBX_INFO_CART_RAM_STRIDE: *out = s.cram_stride; break;
    case GBX_INFO_STEP_LANES: *out = s.step_lanes; break;
    default: return fail(GBX_E_INVALID, "unknown info key");
  }
  return GBX_OK;
}

int gbx_set_debug(gbx_ctx* ctx, int32_t rst38, int32_t trap_pc, int32_t max_instr,
                  int32_t watch_addr) {
  CHECK_CTX(ctx);
  ctx->dbg[0] = rst38 ? 1 : 0;
  ctx->dbg[1] = trap_pc & 0xFFFF;
  ctx->dbg[2] = max_instr > 0 ? max_instr : 0;
  ctx->dbg[3] = watch_addr & 0xFFFF;
  return GBX_OK;
}

}  // extern "C"

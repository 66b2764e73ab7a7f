// gbx_aux.h -- launch wrappers shared by the kernels and the host API.
#pragma once
#include "gbx_internal.h"

namespace gbx {

// Reset snapshot of one env, env-major (reference core/reset_cache.py).
struct SnapState {
  uint8_t* mem;     // [65536]
  uint8_t* cram;    // [cram_stride]
  uint8_t* serial;  // [1024]
  uint8_t* pix;     // [72*80]
  int32_t* cs;      // [20]
  int32_t* sc;      // [32] (slot F_ACTIONS holds the action buffer entry)
  int64_t* cnt;     // [2]
  int has_pix;
};

// One env's whole state as one flat byte image (state save/load):
//   [0, 256)           int64 per-env scalars in GBX_FIELD_* order
//   [256, 336)         int32 cart state, 20 slots
//   [512, 512 + 64K)   raw memory
//   then ram_bytes of cart RAM, then the 9 x 144 env-0 scanline latches.
constexpr size_t kImgCart = 256;
constexpr size_t kImgMem = 512;
constexpr size_t kImgCram = kImgMem + kMemSize;
constexpr int kLatchBytes = 9 * kScreenH;
__host__ __device__ inline size_t img_latches_off(int ram_bytes) { return kImgCram + (size_t)ram_bytes; }
__host__ __device__ inline size_t img_bytes(int ram_bytes) { return img_latches_off(ram_bytes) + kLatchBytes; }
enum { IMG_CRAM = 1, IMG_LATCHES = 2 };
// to_device = 0: gather env into img (every part); 1: scatter img into env
// (scalars, cart state and memory always; cart RAM / latches per `parts`).
hipError_t launch_env_image(const DevState& s, int env, uint8_t* img, int to_device, int parts,
                            hipStream_t st);

hipError_t launch_snapshot(const DevState& s, const SnapState& snap, int env, int with_pix,
                           hipStream_t st);
hipError_t launch_masked_reset(const DevState& s, const SnapState& snap, const uint8_t* mask,
                               int live, hipStream_t st);
hipError_t launch_gather(const DevState& s, const uint16_t* addrs, int k, uint8_t* out,
                         hipStream_t st);
hipError_t launch_hash(const DevState& s, const uint64_t* K, uint64_t* out, hipStream_t st);
// buf[count][len] env-major <-> memory of envs [env_lo, env_lo + count),
// addresses [lo, lo + len); to_image = 0 reads the image into buf, 1 writes
// buf into the image.  The caller checks the ranges.
hipError_t launch_mem_range(const DevState& s, int env_lo, int count, int lo, int len, uint8_t* buf,
                            int to_image, hipStream_t st);
hipError_t launch_export_cram(const DevState& s, int env_lo, int count, uint8_t* dst,
                              hipStream_t st);

}  // namespace gbx

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

hipError_t launch_snapshot(const DevState& s, const SnapState& snap, int env, int with_pix,
                           hipStream_t st);
hipError_t launch_masked_reset(const DevState& s, const SnapState& snap, const uint8_t* mask,
                               hipStream_t st);
hipError_t launch_gather(const DevState& s, const uint16_t* addrs, int k, uint8_t* out,
                         hipStream_t st);
hipError_t launch_hash(const DevState& s, const uint64_t* K, uint64_t* out, hipStream_t st);
hipError_t launch_export_mem(const DevState& s, int env_lo, int count, int lo, int len,
                             uint8_t* dst, hipStream_t st);
hipError_t launch_import_mem(const DevState& s, int env, int addr, int len, const uint8_t* src,
                             hipStream_t st);
hipError_t launch_export_cram(const DevState& s, int env_lo, int count, uint8_t* dst,
                              hipStream_t st);

}  // namespace gbx

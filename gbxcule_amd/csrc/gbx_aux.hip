// gbx_aux.hip -- kernels around the step: power-on fill, the 2x-downsampled
// snapshot renderer, reset snapshot / masked restore, RAM-sense gather, state
// hash, and the layout converters behind the export/import helpers.
#include <type_traits>
#include <utility>

#include "gbx_aux.h"

namespace gbx {
namespace {

// Streams that pass through once (the masked restore's rows, the render's
// output) go through nontemporal loads and stores, which leave the lines
// the next kernels reuse (records, ROM, the envs' memory rows) in L2.
typedef uint32_t nt4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream(const uint4* p) {
  const nt4 q = __builtin_nontemporal_load(reinterpret_cast<const nt4*>(p));
  return make_uint4(q[0], q[1], q[2], q[3]);
}
__device__ __forceinline__ void st_stream(uint4* p, uint4 v) {
  const nt4 q = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(q, reinterpret_cast<nt4*>(p));
}

__device__ __forceinline__ uint32_t block_of(uint32_t e) {
  return __builtin_amdgcn_readfirstlane(e >> kEnvBlockShift);
}

// ---------------------------------------------------------------------------
// Power-on memory image: zero everywhere except the boot image at 0x00-0xFF
// (reference backends/warp_vec.py:335-340).  One thread per 16 bytes; the 16
// bytes are 16 lanes of one address row, so they share one value.
// ---------------------------------------------------------------------------
__global__ void fill_mem_kernel(uint4* mem, size_t n16, const uint8_t* boot) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n16) return;
  const uint32_t addr = (uint32_t)((i * 16) >> kEnvBlockShift) & 0xFFFFu;
  uint32_t v = 0;
  if (addr < 0x100u) v = (uint32_t)boot[addr] * 0x01010101u;
  mem[i] = make_uint4(v, v, v, v);
}

__global__ void init_state_kernel(int32_t* cs, int32_t* sc, int npad, int mbc_kind) {
  const uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (uint32_t)npad) return;
  for (int k = 0; k < kCartStateStride; ++k) cs[cs_index(e, k)] = 0;
  cs[cs_index(e, CS_MBC_KIND)] = mbc_kind;
  cs[cs_index(e, CS_ROM_BANK_LO)] = 1;
  cs[cs_index(e, CS_BOOTROM_ENABLED)] = 1;
  for (int k = 0; k < kNumFields; ++k) sc[sc_index(e, k)] = 0;
  sc[sc_index(e, F_JOYP_SELECT)] = 0x30;
}

// ---------------------------------------------------------------------------
// Snapshot renderer (reference kernels/ppu_render_downsampled.py:27-234),
// render_kernel below, and env 0's full frame (frame_bg_kernel).  Row reads
// one env's bytes straight from the env-interleaved memory (the full-frame
// renderer's source); the snapshot renderer reads an LDS image (Img).
// ---------------------------------------------------------------------------
struct Row {
  const uint8_t* mb;  // block base
  uint32_t lane;
  __device__ uint32_t M(uint32_t addr) const { return mb[((size_t)addr << kEnvBlockShift) | lane]; }
};

__device__ uint32_t tile_pixel(const Row& r, uint32_t tile_addr, uint32_t row, uint32_t bit) {
  const uint32_t lo = r.M(tile_addr + row * 2u), hi = r.M(tile_addr + row * 2u + 1u);
  return (((hi >> bit) & 1u) << 1) | ((lo >> bit) & 1u);
}

__device__ uint32_t bg_tile_addr(uint32_t lcdc, uint32_t tile_id) {
  if (lcdc & 0x10u) return 0x8000u + tile_id * 16u;
  return (uint32_t)(0x9000 + ((int)tile_id >= 128 ? (int)tile_id - 256 : (int)tile_id) * 16);
}

// The snapshot render reads each env's video RAM, OAM and LCD registers from
// an LDS image of 8 envs (one eighth of a 64-env memory block): address row
// a of the image holds the 8 envs' bytes of address a, as they sit side by
// side in the env-interleaved layout, so one 8-byte load fills a row.
// Gathered straight from memory, every byte a lane needs lies on a 64-byte
// line of its own (the other lanes read other addresses), and the render
// was bound by the cache's line lookups.
constexpr int kImgEnvs = 8;
constexpr uint32_t kImgVram = 0x2000u;  // 8000-9FFF
constexpr uint32_t kImgOam = 0xA0u;     // FE00-FE9F
constexpr uint32_t kImgRegs = 0x0Cu;    // FF40-FF4B
constexpr uint32_t kImgRows = kImgVram + kImgOam + kImgRegs;
constexpr int kImgThreads = kImgEnvs * kDsH;  // one per (env, output row)
// The 9 wavefronts of a workgroup sit on the 4 SIMDs as w mod 4, so SIMD 0
// carries three.  Loads 0 .. kImgLoadsAll-1 of the image come from every
// thread (rows 576k + tid); the rest only from the six wavefronts off SIMD 0
// (384 rows per load), which leaves SIMD 0's three with fewer to issue.
constexpr int kImgLoadsAll = 8;
constexpr int kImgFetchThreads = 384;
constexpr uint32_t kImgRowsAll = (uint32_t)kImgLoadsAll * kImgThreads;
constexpr int kImgLoads =
    kImgLoadsAll + (int)((kImgRows - kImgRowsAll + kImgFetchThreads - 1) / kImgFetchThreads);
constexpr int kTileSlots = 21;     // tile columns one 80-sample row can touch
constexpr int kGroups = kDsW / 4;  // 4-sample groups per row (one output word unpacked)
static_assert(kImgEnvs == 8, "image rows are 8 bytes");
static_assert(kImgThreads == 9 * 64 && kImgFetchThreads == 6 * 64, "nine wavefronts, six off SIMD 0");
// First image row of load k for wavefront w (of all nine with k below
// kImgLoadsAll, else fetch wavefront fw = w - 1 - w/4 of the six); the
// wavefront's 64 lanes take the 64 rows from there.
__host__ __device__ constexpr uint32_t img_row_base(int k, uint32_t w) {
  return k < kImgLoadsAll ? (uint32_t)k * kImgThreads + w * 64u
                          : kImgRowsAll + (uint32_t)(k - kImgLoadsAll) * kImgFetchThreads +
                                (w - 1u - (w >> 2)) * 64u;
}
static_assert(kImgRowsAll <= kImgVram && img_row_base(kImgLoads - 1, 1) <= kImgVram,
              "only the last load reaches past video RAM, and it holds every OAM row");

// The image rows that four envs' renders read, from their LCDC bytes x, as
// a mask of 1 KiB video RAM chunks (bit c: 8000 + 400h * c .. + 3FFh) and
// bit 8 for OAM and the registers: sprite tiles 8000-8FFF with sprites on
// (bit 1); with the BG on (bit 0) the BG and window tile block (8000-8FFF
// with bit 4 set, else 8800-97FF) and the maps the background (bit 3) and
// the window (bits 5 and 6) select.
__device__ __forceinline__ uint32_t image_chunks(uint32_t x) {
  constexpr uint32_t kB = 0x01010101u;
  const uint32_t bg = x & kB, w = bg & (x >> 5);
  const uint32_t lo_tiles = ((x >> 1) | (bg & (x >> 4))) & kB;     // 8000-8FFF
  const uint32_t hi_tiles = bg & ~(x >> 4) & kB;                  // 8800-97FF
  const uint32_t map1 = ((bg & (x >> 3)) | (w & (x >> 6))) & kB;  // 9C00-9FFF
  const uint32_t map0 = ((bg & ~(x >> 3)) | (w & ~(x >> 6))) & kB;
  return (lo_tiles ? 0x0Fu : 0u) | (hi_tiles ? 0x3Cu : 0u) | (map0 ? 0x40u : 0u) | (map1 ? 0x80u : 0u) |
         0x100u;
}

struct Img {
  const uint8_t* p;  // the workgroup's image
  uint32_t env;      // 0..7
  __device__ uint32_t M(uint32_t addr) const { return p[((addr - 0x8000u) << 3) | env]; }  // video RAM
  __device__ uint32_t off(uint32_t addr) const { return ((addr - 0x8000u) << 3) | env; }  // M's byte
  __device__ uint32_t at(uint32_t o) const { return p[o]; }
  // OAM is stored per env (the image's OAM rows transposed): env e's 160
  // bytes from byte 8 * 2000h + 160 e, entry k one aligned word
  __device__ uint32_t oam_entry(uint32_t k) const {
    return *reinterpret_cast<const uint32_t*>(p + (kImgVram << 3) + env * kImgOam + 4u * k);
  }
  __device__ uint32_t reg(uint32_t addr) const { return p[((kImgVram + kImgOam + addr - 0xFF40u) << 3) | env]; }
};

// The four sampled pixels of one tile row word t = lo | hi << 8, colours
// (0..3) one per byte, byte i = the i-th sampled pixel from the left: bits
// 7-p, 5-p, 3-p, 1-p, where p is the layer's sample phase.  After the bit
// reverse, lo bit 7-p-2i sits at 24+p+2i and hi bit 7-p-2i at 16+p+2i, so u
// holds colour i at bits 2i..2i+1; the two multiplies spread the even and the
// odd colours to bytes without overlapping terms.
__device__ __forceinline__ uint32_t spread_tile(uint32_t t, uint32_t p) {
  const uint32_t r = __builtin_bitreverse32(t);
  const uint32_t u = ((r >> (24u + p)) & 0x55u) | ((r >> (15u + p)) & 0xAAu);
  const uint32_t ev = ((u & 0x33u) * 0x1001u) & 0x00030003u;   // colours 0, 2 -> bytes 0, 2
  const uint32_t od = ((u & 0xCCu) * 0x40040u) & 0x03000300u;  // colours 1, 3 -> bytes 1, 3
  return ev | od;
}

// The colours of the four sampled pixels p, p + 2, p + 4, p + 6 (p = 0 or 1,
// from the left) of a sprite's tile row t = lo | hi << 8, one per byte,
// mirrored with xflip: pixel j is bit 7 - j of lo and hi, or bit j.
__device__ __forceinline__ uint32_t sprite_colours(uint32_t t, uint32_t p, bool xflip) {
  // unmirrored as spread_tile; mirrored, lo bit p + 2i and hi bit 8 + p + 2i
  // to bits 2i and 2i + 1 of u directly
  const uint32_t src = xflip ? t : __builtin_bitreverse32(t);
  const uint32_t u = ((src >> (p + (xflip ? 0u : 24u))) & 0x55u) | ((src >> (p + (xflip ? 7u : 15u))) & 0xAAu);
  const uint32_t ev = ((u & 0x33u) * 0x1001u) & 0x00030003u;
  const uint32_t od = ((u & 0xCCu) * 0x40040u) & 0x03000300u;
  return ev | od;
}

// One BG or window layer of a row, for a layer whose sample x reads map pixel
// px = (x + s) & 0xFF (s = SCX for the background, 7 - WX for the window):
// c[j] = the sampled colours (spread_tile) of map column ((s >> 3) + j) & 31.
// Sample ox is then byte ox + ((s & 7) >> 1) of the byte stream c[0], c[1], ...
// The 21 map reads of a layer are independent (layer_ids), then its 42
// tile-data reads are (layer_tiles).
__device__ __forceinline__ void layer_ids(const Img& r, uint32_t map, uint32_t s, uint32_t py,
                                          uint32_t (&id)[kTileSlots]) {
  // map row (py >> 3): its 32 ids are 32 address rows of 8 bytes from an
  // offset whose low 8 bits are the env, column (c + j) & 31 at 8 times that
  const uint32_t row = r.off(map + (py >> 3) * 32u), c8 = s & 0xF8u;
#pragma unroll
  for (int j = 0; j < kTileSlots; ++j) id[j] = r.at(((c8 + 8u * (uint32_t)j) & 0xF8u) | row);
}
// Tile id's row in the block LCDC bit 4 selects: 8000 + 16 id, or with
// signed ids 9000 + 16 (int8)id = 8800 + 16 (id ^ 80h); in the image, the
// row's low byte at offset((8000 or 8800) + 2 * row) + ((id ^ x) << 7), its
// high byte 8 further (one address row).
__device__ __forceinline__ void layer_tiles(const Img& r, uint32_t lcdc, uint32_t s, uint32_t py,
                                            const uint32_t (&id)[kTileSlots], uint32_t (&c)[kTileSlots]) {
  const bool unsigned_ids = (lcdc & 0x10u) != 0u;
  const uint32_t x = unsigned_ids ? 0u : 0x80u;
  const uint32_t b = r.off((unsigned_ids ? 0x8000u : 0x8800u) + (py & 7u) * 2u);
#pragma unroll
  for (int j = 0; j < kTileSlots; ++j) {
    const uint32_t o = b + ((id[j] ^ x) << 7);
    c[j] = spread_tile(r.at(o) | (r.at(o + 8u) << 8), s & 1u);
  }
}

// One workgroup per 8 envs: it copies their image rows into LDS (every
// thread issues all its loads before its LDS stores; the 1 KiB video RAM
// chunks that none of the 8 envs' LCDC lets the render read are skipped),
// then renders one (env, output row) per thread.  Each image load brings a
// 128-byte line for 16 useful bytes, so the CU's supply of L1 misses, not
// HBM, bounds the copy: fewer lines and loads spread over the group are
// what speed it up.  The 8 workgroups of a 64-env block are dealt to one
// XCD (the hardware deals workgroup i to XCD i mod 8), so each 64-byte line
// comes from HBM about once and its other reads hit that XCD's L2.  Per
// row, the sprites (the first 10 OAM entries covering the line,
// counted before the x test) are resolved into a line buffer of the 80
// samples: each sample keeps the opaque sprite pixel with the lowest x
// (ties: the lower OAM index, the earlier entry), as the reference's
// per-sample search over OAM selects it; a thread walks only its covering
// entries, two per round.  The BG and window tile rows are read for all 21
// tile columns at once; the samples are then shaded four at a time, one per
// byte: the group's colours are a byte window of the layer's colour stream,
// the window layer is blended in by a byte mask, BGP maps colours to shades
// through a byte permute, and the sprite overlay is a byte mask.  The output
// words are staged in LDS in output order and stored by each wavefront
// along the rows of its 8 envs.
template <bool packed>
__global__ __launch_bounds__(kImgThreads) void render_kernel(DevState s, uint8_t* out, int64_t base,
                                                             uint32_t rounds) {
  // One LDS block, the image first: at LDS address 0 its data-dependent
  // reads need no base added to their offsets.
  constexpr size_t kImgBytes = (size_t)kImgRows * kImgEnvs;
  constexpr size_t kObjBytes = (size_t)kGroups * kImgThreads * 4 * sizeof(uint16_t);
  static_assert(kImgBytes % 16 == 0, "the sprite line buffer stays 16-byte aligned");
  __shared__ uint4 lds[(kImgBytes + kObjBytes + (size_t)kDsH * kImgEnvs * sizeof(uint64_t)) / 16];
  uint8_t* const img = reinterpret_cast<uint8_t*>(lds);
  // sprite line buffer, 4 samples per (group, thread): bits [0:1] the
  // sample's sprite shade (palette applied), [2] behind non-zero BG, [3] set
  // (a sprite pixel), [8:15] that sprite's OAM x (its left edge + 8), 0xFF00
  // while no sprite pixel is set; reused as the output stage
  auto obj = reinterpret_cast<uint16_t(*)[kImgThreads][4]>(img + kImgBytes);
  // OAM entries covering each (env, output row): bit k = entry k
  auto cover = reinterpret_cast<uint64_t(*)[kImgEnvs]>(img + kImgBytes + kObjBytes);
  const uint32_t tid0 = threadIdx.x;
  const uint32_t nblk = (uint32_t)s.npad >> kEnvBlockShift;
  // Group `it` of this workgroup: (64-env block, eighth).  With rounds > 1
  // the grid is a multiple of 64 workgroups, each rendering `rounds` groups;
  // in round `it` the workgroups of one XCD render whole blocks.
  auto group = [&](uint32_t it, uint32_t& blk, uint32_t& part) {
    const uint32_t w = blockIdx.x;
    if (rounds > 1u) {
      const uint32_t c = w >> 3, per_xcd = gridDim.x >> 3;
      blk = ((it * (per_xcd >> 3) + (c >> 3)) << 3) | (w & 7u);
      part = c & 7u;
    } else if ((nblk & 7u) == 0u) {
      blk = (((w >> 3) >> 3) << 3) | (w & 7u);
      part = (w >> 3) & 7u;
    } else {
      blk = w >> 3;
      part = w & 7u;
    }
  };
  // image rows k0 <= k < k1 of each thread for a group, the loads issued
  // together, those in chunks outside `need` (image_chunks) skipped: the
  // LDS rows they would fill get zeros no render of the group reads.  A
  // wavefront's 64 rows of one load are 64-aligned, so they lie in one
  // chunk and the test is wavefront-uniform.  The loads address the 64-env
  // block as a raw buffer, a skipped one at an offset past its end, which
  // returns zeros without a memory request (a branch around the load would
  // make the compiler drain every outstanding load before the next one).
  uint2 v[kImgLoads];
  // wavefront index; those with w mod 4 != 0 (off SIMD 0) take the loads
  // past kImgLoadsAll
  const uint32_t wv = __builtin_amdgcn_readfirstlane(tid0 >> 6);
  auto fetch = [&](uint32_t blk, uint32_t part, uint32_t need, auto k0, auto k1) {
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        s.mem + ((size_t)blk << 22), 0, 1 << 22, 0x00020000);  // untyped raw buffer
    // (recomputed per call: kept across the loop, the offsets would hold
    // registers the render needs)
    uint32_t t = tid0, w = wv;
    asm volatile("" : "+v"(t), "+s"(w));
    const uint32_t f = t - 64u - ((w >> 2) << 6);  // row of load kImgLoadsAll, less kImgRowsAll
    auto one = [&](int k) {
      const uint32_t r0 = img_row_base(k, w);
      const uint32_t i0 = k < kImgLoadsAll ? t + (uint32_t)k * kImgThreads
                                           : f + img_row_base(k, 1u);
      const uint32_t i = k == kImgLoads - 1 ? min(i0, kImgRows - 1u) : i0;
      const uint32_t a = k < kImgLoads - 1 || i < kImgVram ? 0x8000u + i
                         : i < kImgVram + kImgOam          ? 0xFE00u + (i - kImgVram)
                                                           : 0xFF40u + (i - kImgVram - kImgOam);
      const bool want = (need >> (r0 >> 10)) & 1u;
      const auto w = __builtin_amdgcn_raw_buffer_load_b64(rb, (int)(want ? a << kEnvBlockShift : 0x80000000u),
                                                          (int)(part * (uint32_t)kImgEnvs), 0);
      v[k] = make_uint2(w[0], w[1]);
    };
    constexpr int a0 = decltype(k0)::value, a1 = decltype(k1)::value;
#pragma unroll
    for (int k = a0; k < (a1 < kImgLoadsAll ? a1 : kImgLoadsAll); ++k) one(k);
    if ((w & 3u) != 0u) {
#pragma unroll
      for (int k = a0 > kImgLoadsAll ? a0 : kImgLoadsAll; k < a1; ++k) one(k);
    }
  };
  // a group's 8 LCDC bytes (one broadcast load), for its chunk mask
  auto lcdc_row = [&](uint32_t blk, uint32_t part) {
    return *reinterpret_cast<const uint2*>(s.mem + ((size_t)blk << 22) + part * (uint32_t)kImgEnvs +
                                           ((size_t)0xFF40u << kEnvBlockShift));
  };
  auto chunks_of = [](uint2 x) {
    return image_chunks(__builtin_amdgcn_readfirstlane(x.x)) | image_chunks(__builtin_amdgcn_readfirstlane(x.y));
  };
  uint32_t blk, part;
  using K0 = std::integral_constant<int, 0>;
  using K4 = std::integral_constant<int, 4>;
  using K8 = std::integral_constant<int, kImgLoadsAll>;
  using KN = std::integral_constant<int, kImgLoads>;
  group(0u, blk, part);
  fetch(blk, part, 0x1FFu, K0{}, KN{});
  // the LCDC bytes of group it + 1 load one group ahead of its rows
  uint2 lc_next = make_uint2(0u, 0u);
  if (rounds > 1u) {
    uint32_t b1, p1;
    group(1u, b1, p1);
    lc_next = lcdc_row(b1, p1);
  }
#pragma unroll 1
  for (uint32_t it = 0; it < rounds; ++it) {
    // (derived per round: kept across the loop, the addresses that follow
    // from the thread index would hold registers the render needs)
    uint32_t tid = tid0, w = wv;
    asm volatile("" : "+v"(tid), "+s"(w));
    const uint32_t f = tid - 64u - ((w >> 2) << 6);
    auto put = [&](int k) {
      const uint32_t i = k < kImgLoadsAll ? tid + (uint32_t)k * kImgThreads : f + img_row_base(k, 1u);
      if (k == kImgLoads - 1 && i - kImgVram < kImgOam) {
        // an OAM row: its 8 envs' bytes to their per-env OAM copies
#pragma unroll
        for (int e = 0; e < kImgEnvs; ++e)
          img[(kImgVram << 3) + (uint32_t)e * kImgOam + (i - kImgVram)] =
              (uint8_t)((e < 4 ? v[k].x : v[k].y) >> (8 * (e & 3)));
      } else if (k < kImgLoads - 1 || i < kImgRows) {
        *reinterpret_cast<uint2*>(img + (size_t)i * kImgEnvs) = v[k];
      }
    };
#pragma unroll
    for (int k = 0; k < kImgLoadsAll; ++k) put(k);
    if ((w & 3u) != 0u) {
#pragma unroll
      for (int k = kImgLoadsAll; k < kImgLoads; ++k) put(k);
    }
    // The next group's rows load while this one renders, in three parts:
    // loads 0-3 once the coverage is marked, 4-7 after the sprites (the last
    // of SIMD 0's wavefronts), the rest after the BG and window layers (their
    // tile rows then no longer hold registers).  Issued at once,
    // the loads of the 9 wavefronts queue in the CU's memory pipeline and
    // hold each wavefront at the issue of its last one; spread over the
    // group, they stream beside the render.
    uint32_t nblk_next = 0, npart = 0, need = 0;
    const bool more = it + 1u < rounds;
    if (more) {
      group(it + 1u, nblk_next, npart);
      need = chunks_of(lc_next);
      if (it + 2u < rounds) {
        uint32_t b2, p2;
        group(it + 2u, b2, p2);
        lc_next = lcdc_row(b2, p2);
      }
    }
    const uint32_t env = tid & (uint32_t)(kImgEnvs - 1);
    // Wavefront w renders the 8 output rows of row block perm[w].  The 9
    // wavefronts sit on the 4 SIMDs as w mod 4, so SIMD 0 carries three of
    // them: it gets the three top blocks, and the bottom blocks, where a
    // status-bar window adds a second layer, go to SIMDs with two.
    constexpr uint64_t kRowBlock = 0x267815430ull;  // perm = 0 3 4 5 1 8 7 6 2
    const uint32_t rblk = (uint32_t)(kRowBlock >> (4u * (tid >> 6))) & 0xFu;
    const uint32_t oy = rblk * 8u + ((tid >> 3) & 7u);
    const uint32_t y = oy * 2u;
#pragma unroll
    for (int g = 0; g < kGroups; ++g) *reinterpret_cast<uint2*>(&obj[g][tid][0]) = make_uint2(0xFF00FF00u, 0xFF00FF00u);
    cover[oy][env] = 0u;
    __syncthreads();
    const Img r{img, env};
    // entry k of env e (thread 40e + k) marks the output rows it covers:
    // position valid, screen row 2*oy inside [sy - 16, sy - 16 + height)
    if (tid < 40u * (uint32_t)kImgEnvs) {
      const uint32_t e = tid / 40u, k = tid % 40u;
      const Img o{img, e};
      const uint32_t oe = o.oam_entry(k), sy = oe & 0xFFu, sx = (oe >> 8) & 0xFFu;
      const uint32_t ht = (o.reg(0xFF40) & 0x04u) ? 16u : 8u;
      if ((sx != 0u) & (sy != 0u) & (sx < 168u) & (sy < 160u)) {
        const uint32_t first = (sy > 16u ? sy - 16u : 0u) >> 1;
#pragma unroll
        for (uint32_t j = 0; j < 9u; ++j) {
          const uint32_t row = first + j;
          if ((row < (uint32_t)kDsH) & (2u * row + 16u - sy < ht))
            atomicOr(reinterpret_cast<unsigned long long*>(&cover[row][e]), 1ull << k);
        }
      }
    }
    __syncthreads();
    if (more) fetch(nblk_next, npart, need, K0{}, K4{});
    const uint32_t lcdc = r.reg(0xFF40);
    const uint32_t height = (lcdc & 0x04u) ? 16u : 8u;
    const uint32_t scy = r.reg(0xFF42), scx = r.reg(0xFF43);
    const uint32_t bgp = r.reg(0xFF47), obp0 = r.reg(0xFF48), obp1 = r.reg(0xFF49);
    const uint32_t wy = r.reg(0xFF4A), wx = r.reg(0xFF4B);
    // OBP0 and OBP1 as byte tables: byte c = shade of colour c
    const uint32_t ptab0 = (obp0 & 3u) | (((obp0 >> 2) & 3u) << 8) | (((obp0 >> 4) & 3u) << 16) |
                           (((obp0 >> 6) & 3u) << 24);
    const uint32_t ptab1 = (obp1 & 3u) | (((obp1 >> 2) & 3u) << 8) | (((obp1 >> 4) & 3u) << 16) |
                           (((obp1 >> 6) & 3u) << 24);
    if (lcdc & 0x02u) {
      // the entries covering this row (position valid, row inside their 8 or
      // 16 lines) in OAM order, then only the first 10
      uint64_t vis = cover[oy][env];
      if (__builtin_expect(__ballot(__popcll(vis) > 10) != 0u, 0)) {
        uint64_t rest = vis;
#pragma unroll
        for (int j = 0; j < 10; ++j) rest &= rest - 1u;  // clears the lowest 10
        vis &= ~rest;
      }
      // each thread's covering entries, lowest OAM index first, two per round
      // (their tile-row reads issued together)
#pragma unroll 1
      while (__ballot(vis != 0u) != 0u) {
        uint32_t ent[2], lo[2], hi[2];
        bool on[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          on[t] = vis != 0u;
          const uint32_t k = on[t] ? (uint32_t)__builtin_ctzll(vis) : 0u;
          vis &= vis - 1u;
          ent[t] = r.oam_entry(k);
        }
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          // the sprite's line for this row, mirrored with y-flip; 8x16: the
          // even tile above, the odd one below.  (A lane without a second
          // entry reads entry 0's row and skips the merge.)
          const uint32_t sy = ent[t] & 0xFFu, attr = ent[t] >> 24;
          uint32_t row = (y + 16u - sy) & 15u;
          row = ((attr >> 6) & 1u) ? (height - 1u - row) & 15u : row;
          const uint32_t tile = height == 16u ? ((ent[t] >> 16) & 0xFEu) | (row >> 3) : (ent[t] >> 16) & 0xFFu;
          const uint32_t o = r.off(0x8000u) + (tile << 7) + ((row & 7u) << 4);  // the row's low byte
          lo[t] = r.at(o);
          hi[t] = r.at(o + 8u);
        }
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          if (!on[t]) continue;
          const uint32_t sx = (ent[t] >> 8) & 0xFFu;
          const uint32_t attr = ent[t] >> 24;
          const uint32_t tag = (sx << 8) | 0x08u | (((attr >> 7) & 1u) << 2);
          // The sampled columns x = 2 ox inside [sx - 8, sx): ox0 .. ox0 + 3,
          // the sprite's pixels p + 2i (p = sx & 1), colours one per byte.
          // They go to the four slots from oc = ox0 clamped to [0, 76],
          // sample i to slot i + ox0 - oc: a sample off the screen falls
          // outside the four, its colour byte shifted out (transparent).
          // The slots are distinct, so all four are read, then all four
          // written (the old entry where the sample does not change it).
          const int ox0 = ((int)sx - 7) >> 1;
          const int oc = min(max(ox0, 0), kDsW - 4), d = ox0 - oc;  // d in -3 .. 4
          const uint32_t c0 = sprite_colours(lo[t] | (hi[t] << 8), sx & 1u, ((attr >> 5) & 1u) != 0u);
          const uint32_t cols = (uint32_t)(((uint64_t)c0 << 32) >> (32 - 8 * d));  // c0 shifted by 8d
          const uint32_t shades = __builtin_amdgcn_perm(0u, ((attr >> 4) & 1u) ? ptab1 : ptab0, cols);
          const uint32_t q = (uint32_t)oc & 3u;
          uint16_t* const w0 = &obj[0][tid][q] + __umul24((uint32_t)oc >> 2, 4u * (uint32_t)kImgThreads);
          uint16_t* slot[4];
          uint32_t cur[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            slot[j] = w0 + j + (q + (uint32_t)j >= 4u ? 4 * kImgThreads - 4 : 0);  // the next group's
            cur[j] = *slot[j];
          }
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const bool upd = (((cols >> (8 * j)) & 3u) != 0u) & (sx < (cur[j] >> 8));  // empty: x 0xFF
            *slot[j] = (uint16_t)(upd ? tag | ((shades >> (8 * j)) & 3u) : cur[j]);
          }
        }
      }
    }

    if (more) fetch(nblk_next, npart, need, K4{}, K8{});
    const uint32_t bg_on = (lcdc & 0x01u) ? ~0u : 0u;
    const bool win = (lcdc & 0x20u) && y >= wy;
    const int wx7 = (int)wx - 7;
    const uint32_t sw = (7u - wx) & 0xFFu;  // window: px = (x - (WX - 7)) & 0xFF
    // A layer not drawn leaves its colours unset (defined by an empty asm,
    // no instruction): the shading masks them out of every sample (the BG
    // off clears all; a window covering the row takes every sample from
    // the window, one starting past the row none).
    uint32_t cb[kTileSlots], cw[kTileSlots];
#pragma unroll
    for (int j = 0; j < kTileSlots; ++j) {
      asm volatile("" : "=v"(cb[j]));
      asm volatile("" : "=v"(cw[j]));
    }
    if (bg_on) {
      // the background unless the window covers the whole row
      const bool do_bg = !(win && wx7 <= 0), do_win = win && wx7 < 2 * kDsW - 1;
      const uint32_t pyb = (y + scy) & 0xFFu, pyw = (y - wy) & 0xFFu;
      // one layer after the other (from LDS the reads need no batching
      // across layers, and the tile ids of one layer fewer hold registers)
      uint32_t id[kTileSlots];
      if (do_bg) {
        layer_ids(r, (lcdc & 0x08u) ? 0x9C00u : 0x9800u, scx, pyb, id);
        layer_tiles(r, lcdc, scx, pyb, id, cb);
      }
      if (do_win) {
        layer_ids(r, (lcdc & 0x40u) ? 0x9C00u : 0x9800u, sw, pyw, id);
        layer_tiles(r, lcdc, sw, pyw, id, cw);
      }
    }
    if (more) fetch(nblk_next, npart, need, K8{}, KN{});
    const uint32_t qb = (scx & 7u) >> 1, qw = (sw & 7u) >> 1;
    // BGP as a byte table: byte c = shade of colour c (all zero with the BG off)
    const uint32_t pbg = ((bgp & 3u) | (((bgp >> 2) & 3u) << 8) | (((bgp >> 4) & 3u) << 16) |
                          (((bgp >> 6) & 3u) << 24)) & bg_on;
    // Samples x = 2 ox >= WX - 7 show the window: ox >= h = (WX - 6) >> 1,
    // so byte i of group g when 4g + i >= h (h = 80, none, without it).
    const int h8 = win ? 8 * ((wx7 + 1) >> 1) : 8 * kDsW;
    uint32_t word[kGroups] = {};
    uint32_t pword = 0;
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
      // colours of samples 4g..4g+3, one per byte
      uint32_t col = __builtin_amdgcn_alignbyte(cb[g + 1], cb[g], qb);
      const uint32_t m = (uint32_t)(~0ull << min(max(h8 - 32 * g, 0), 32));  // the window's bytes
      col = (col & ~m) | (__builtin_amdgcn_alignbyte(cw[g + 1], cw[g], qw) & m);
      col &= bg_on;
      uint32_t shade = __builtin_amdgcn_perm(0u, pbg, col);
      const uint2 ob = *reinterpret_cast<const uint2*>(&obj[g][tid][0]);
      const uint32_t w = __builtin_amdgcn_perm(ob.y, ob.x, 0x06040200u);  // low byte of each entry
      const uint32_t nz = (col | (col >> 1)) & 0x01010101u;
      const uint32_t show = (w >> 3) & ~((w >> 2) & nz) & 0x01010101u;
      const uint32_t sm = (show << 8) - show;
      shade = (sm & w & 0x03030303u) | (~sm & shade);
      // shades s0..s3 to s0 | s1 << 2 | s2 << 4 | s3 << 6 (no overlapping terms)
      pword |= ((shade * 0x01041040u) >> 24) << (8 * (g & 3));
      if ((g & 3) == 3) {
        if (packed) word[g >> 2] = pword;
        pword = 0;
      }
      if (!packed) word[g] = shade;
    }
    // The stage: per wavefront (8 output rows of the 8 envs) its words in
    // output order, env by env, row by row, in the wavefront's own sprite
    // line slots: stage word d in the 128 words of obj[d >> 7][64 wave ..
    // 64 wave + 63].  No other wavefront touches them, so staging needs no
    // barrier, and a wavefront done early stores its rows while the others
    // still render.
    const uint32_t wave = tid >> 6, lane = tid & 63u, r8 = oy & 7u;
    uint32_t* const slots = reinterpret_cast<uint32_t*>(&obj[0][0][0]) + wave * 128u;
    auto stage = [&](uint32_t d) { return slots + (d >> 7) * (2u * (uint32_t)kImgThreads) + (d & 127u); };
    constexpr uint32_t nw = packed ? (uint32_t)kDsWB / 4u : (uint32_t)kGroups;  // words per row
    static_assert(64u * nw <= 128u * (uint32_t)kGroups, "a wavefront's stage fits its slots");
    const uint32_t mine = (env * 8u + r8) * nw;
#pragma unroll
    for (int g = 0; g < kGroups; ++g)
      if ((uint32_t)g < nw) *stage(mine + (uint32_t)g) = word[g];
    constexpr size_t env_bytes = (size_t)nw * 4u * kDsH;
    const uint32_t env0 = blk * (uint32_t)kEnvBlock + part * (uint32_t)kImgEnvs;
    // The wavefront's words in output order: env e's 8 rows are 8 * nw
    // consecutive words of its output, from byte wave * 32 * nw on.
    const uintptr_t ob = (uintptr_t)(out + base);
    if ((ob & 15u) == 0u) {
      // 16 bytes per lane (an env's words are a multiple of 4)
#pragma unroll
      for (uint32_t d = 4u * lane; d < 64u * nw; d += 256u) {
        const uint32_t e = d / (8u * nw), w2 = d % (8u * nw);
        if (env0 + e < (uint32_t)s.n)
          st_stream(reinterpret_cast<uint4*>(out + base + (size_t)(env0 + e) * env_bytes + rblk * 32u * nw + 4u * w2),
                    *reinterpret_cast<const uint4*>(stage(d)));
      }
    } else {
      const bool aligned = (ob & 3u) == 0u;
#pragma unroll
      for (uint32_t d = lane; d < 64u * nw; d += 64u) {
        const uint32_t e = d / (8u * nw), w2 = d % (8u * nw);
        if (env0 + e < (uint32_t)s.n) {
          const uint32_t wd = *stage(d);
          uint8_t* p = out + base + (size_t)(env0 + e) * env_bytes + rblk * 32u * nw + 4u * w2;
          if (aligned) {
            *reinterpret_cast<uint32_t*>(p) = wd;
          } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) p[q] = (uint8_t)(wd >> (8 * q));
          }
        }
      }
    }
    // every wavefront is done with the image and the stage
    __syncthreads();
    blk = nblk_next;
    part = npart;
  }
}

// ---------------------------------------------------------------------------
// Env 0's full 160x144 frame from its scanline latches (reference
// kernels/ppu_step.py:12-176): LCDC, SCX, SCY, BGP, WX, WY, the window line,
// OBP0 and OBP1 of each line as the step captured them; VRAM and OAM as they
// are now.  One workgroup per line.  Wavefront 0 selects the line's sprites
// first (the first 10 OAM entries that overlap the line, counted before the
// x test) with one ballot, into LDS in OAM order; then every thread renders
// one pixel against at most those 10.
// ---------------------------------------------------------------------------
constexpr int kFrameThreads = 192;  // 160 pixels, three wavefronts

__global__ __launch_bounds__(kFrameThreads) void frame_bg_kernel(DevState s, uint8_t* out) {
  __shared__ uint32_t cand[10];
  __shared__ uint32_t ncand;
  const uint32_t y = blockIdx.x;
  const uint32_t x = threadIdx.x;
  const Row r{s.mem, 0u};  // env 0: block 0, lane 0
  const uint8_t* L = s.latches + (size_t)y * kLatchStride;
  const uint32_t lcdc = L[0], scx = L[1], scy = L[2], bgp = L[3], wx = L[4], wy = L[5];
  const uint32_t win_line = L[6], obp0 = L[7], obp1 = L[8];
  const uint32_t height = (lcdc & 0x04u) ? 16u : 8u;
  if (x < 64u) {
    bool on = false;
    if (x < 40u && (lcdc & 0x02u)) {
      const uint32_t sy = r.M(0xFE00u + 4u * x), sx = r.M(0xFE01u + 4u * x);
      const int top = (int)sy - 16;
      on = sx != 0 && sy != 0 && sx < 168u && sy < 160u && (int)y >= top &&
           (int)y < top + (int)height;
    }
    const uint64_t mask = __ballot(on);
    const uint32_t rank = (uint32_t)__builtin_popcountll(mask & ((1ull << x) - 1ull));
    if (on && rank < 10u) cand[rank] = x;
    if (x == 0) {
      const uint32_t total = (uint32_t)__builtin_popcountll(mask);
      ncand = total < 10u ? total : 10u;
    }
  }
  __syncthreads();
  if (x >= (uint32_t)kScreenW) return;

  uint32_t shade = 0, bg_color = 0;
  if (lcdc & 0x01u) {
    uint32_t px, py, map;
    if ((lcdc & 0x20u) && y >= wy && (int)x >= (int)wx - 7) {
      px = (uint32_t)((int)x - ((int)wx - 7)) & 0xFFu;
      py = win_line & 0xFFu;
      map = (lcdc & 0x40u) ? 0x9C00u : 0x9800u;
    } else {
      px = (x + scx) & 0xFFu;
      py = (y + scy) & 0xFFu;
      map = (lcdc & 0x08u) ? 0x9C00u : 0x9800u;
    }
    const uint32_t tile_id = r.M(map + (py >> 3) * 32u + (px >> 3));
    bg_color = tile_pixel(r, bg_tile_addr(lcdc, tile_id), py & 7u, 7u - (px & 7u));
    shade = (bgp >> (bg_color * 2u)) & 3u;
  }
  const uint32_t nc = ncand;
  bool found = false;
  int best_x = 0;
  uint32_t best_color = 0, best_attr = 0;
  for (uint32_t c = 0; c < nc; ++c) {  // OAM order: an x tie keeps the lower index
    const uint32_t k = cand[c];
    const int left = (int)r.M(0xFE01u + 4u * k) - 8;
    if ((int)x < left || (int)x >= left + 8) continue;
    const int top = (int)r.M(0xFE00u + 4u * k) - 16;
    uint32_t tile = r.M(0xFE02u + 4u * k);
    const uint32_t attr = r.M(0xFE03u + 4u * k);
    uint32_t row = (uint32_t)((int)y - top);
    if ((attr >> 6) & 1u) row = height - 1u - row;
    if (height == 16u) {
      tile &= 0xFEu;
      if (row >= 8u) {
        tile += 1u;
        row -= 8u;
      }
    }
    const uint32_t pxl = (uint32_t)((int)x - left);
    const uint32_t bit = ((attr >> 5) & 1u) ? pxl : 7u - pxl;
    const uint32_t color = tile_pixel(r, 0x8000u + tile * 16u, row, bit);
    if (color == 0) continue;
    if (!found || left < best_x) {
      found = true;
      best_x = left;
      best_color = color;
      best_attr = attr;
    }
  }
  if (found && !(((best_attr >> 7) & 1u) && bg_color != 0)) {
    const uint32_t pal = ((best_attr >> 4) & 1u) ? obp1 : obp0;
    shade = (pal >> (best_color * 2u)) & 3u;
  }
  out[y * (uint32_t)kScreenW + x] = (uint8_t)shade;
}

// ---------------------------------------------------------------------------
// Reset snapshot (core/reset_cache.py:68-190): one env into env-major buffers.
// ---------------------------------------------------------------------------
__global__ void snapshot_kernel(DevState s, SnapState snap, uint32_t env, int with_pix) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < (uint32_t)kMemSize) snap.mem[i] = s.mem[mem_index(env, i)];
  if (i < (uint32_t)s.cram_stride) snap.cram[i] = s.cram[cram_index(env, i, (uint32_t)s.cram_stride)];
  if (i < (uint32_t)kSerialMax) snap.serial[i] = s.serial[(size_t)env * kSerialMax + i];
  if (with_pix && i < (uint32_t)(kDsW * kDsH)) snap.pix[i] = s.pix[(size_t)env * kDsW * kDsH + i];
  if (i < (uint32_t)kCartStateStride) snap.cs[i] = s.cs[cs_index(env, (int)i)];
  if (i < (uint32_t)kNumFields)
    snap.sc[i] = i == (uint32_t)F_ACTIONS ? s.actions[env] : s.sc[sc_index(env, (int)i)];
  if (i < 2u) snap.cnt[i] = s.cnt[cnt_index(env, (int)i)];
}

// Masked restore of the interleaved images (mem + cart RAM).  An address
// row holds one byte of each of the block's 64 envs, so the restore works
// on whole rows: four lanes (a quad) take one 64-byte row, 16 envs each,
// load it with one 16-byte load per lane, put the snapshot byte into the
// positions of the masked envs (a byte mask built once from the block's
// mask bits) and store the row back, as four 16-byte stores covering all 64
// bytes, only when one of its bytes changed.  Every masked env of the block
// is restored in the same pass, each row is read once, and no row is written
// partially.  A workgroup of 256 threads covers kResetRows rows of one block,
// four rows per thread in flight.  With `live` set only the rows the step
// writes are restored (8000-9FFF, C000-DFFF, FE00-FFFF, then cartridge RAM):
// the caller knows that the others still hold the power-on bytes in every
// env and in the snapshot.  Blocks without a masked env leave at once.
constexpr uint32_t kResetRows = 1024;
constexpr int kResetBatch = 4;
// Row of restore index i: every row of mem then of cartridge RAM, or with
// `live` the live rows 8000-9FFF, C000-DFFF, FE00-FFFF then cartridge RAM.
__device__ __forceinline__ uint32_t restore_row(uint32_t i, bool live) {
  return !live ? i : i < 0x2000u ? 0x8000u + i : i < 0x4000u ? 0xA000u + i : 0xBE00u + i;
}
__host__ __device__ inline uint32_t restore_rows(uint32_t cram_stride, bool live) {
  return (live ? 0x4200u : (uint32_t)kMemSize) + cram_stride;
}
__global__ __launch_bounds__(256) void masked_mem_kernel(DevState s, const uint8_t* snap_mem,
                                                         const uint8_t* snap_cram, const uint8_t* mask,
                                                         int live) {
  const uint32_t b = blockIdx.x, t = threadIdx.x;
  const uint32_t e = (b << kEnvBlockShift) | (t & (kEnvBlock - 1));
  const uint64_t bits = __ballot(e < (uint32_t)s.n && mask[e] != 0);
  if (bits == 0) return;
  // this lane's 16 envs (16k .. 16k + 15 of the block) as a byte mask
  const uint32_t k = t & 3u;
  const uint32_t m16 = (uint32_t)(bits >> (16u * k)) & 0xFFFFu;
  uint32_t mw[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t n4 = (m16 >> (4 * j)) & 0xFu;
    mw[j] = ((n4 & 1u) ? 0xFFu : 0u) | ((n4 & 2u) ? 0xFF00u : 0u) | ((n4 & 4u) ? 0xFF0000u : 0u) |
            ((n4 & 8u) ? 0xFF000000u : 0u);
  }
  const uint32_t count = restore_rows((uint32_t)s.cram_stride, live != 0);
  const uint32_t r0 = blockIdx.y * kResetRows + (t >> 2);
  const uint32_t r1 = min(count, (blockIdx.y + 1u) * kResetRows);
  const size_t cram_base = (size_t)b * (size_t)s.cram_stride;
  for (uint32_t r = r0; r < r1; r += 64u * kResetBatch) {
    uint4* p[kResetBatch];
    uint4 cur[kResetBatch];
    uint32_t w[kResetBatch];
#pragma unroll
    for (int i = 0; i < kResetBatch; ++i) {
      const uint32_t ii = r + 64u * (uint32_t)i;
      const bool ok = ii < r1;
      const uint32_t ri = restore_row(ii, live != 0);
      const bool in_mem = ri < (uint32_t)kMemSize;
      const uint32_t off = ri - (uint32_t)kMemSize;
      uint8_t* row = in_mem ? s.mem + ((size_t)b << 22) + ((size_t)ri << kEnvBlockShift)
                            : s.cram + ((cram_base + off) << kEnvBlockShift);
      p[i] = ok ? reinterpret_cast<uint4*>(row) + k : nullptr;
      w[i] = (ok ? (uint32_t)(in_mem ? snap_mem[ri] : snap_cram[off]) : 0u) * 0x01010101u;
      cur[i] = ok ? ld_stream(p[i]) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < kResetBatch; ++i) {
      uint4 nv;
      nv.x = (cur[i].x & ~mw[0]) | (w[i] & mw[0]);
      nv.y = (cur[i].y & ~mw[1]) | (w[i] & mw[1]);
      nv.z = (cur[i].z & ~mw[2]) | (w[i] & mw[2]);
      nv.w = (cur[i].w & ~mw[3]) | (w[i] & mw[3]);
      uint32_t d = (nv.x ^ cur[i].x) | (nv.y ^ cur[i].y) | (nv.z ^ cur[i].z) | (nv.w ^ cur[i].w);
      // the row changed if any of its quad's lanes changed (quad_perm OR)
      d |= (uint32_t)__builtin_amdgcn_mov_dpp((int)d, 0xB1, 0xF, 0xF, true);
      d |= (uint32_t)__builtin_amdgcn_mov_dpp((int)d, 0x4E, 0xF, 0xF, true);
      if (p[i] != nullptr && d != 0u) st_stream(p[i], nv);
    }
  }
}

// One workgroup per 256 envs (a launch of one per env spent its time
// dispatching workgroups that found their env unmasked): the masked envs
// are listed in LDS, then each gets the snapshot's serial buffer, pixels
// (16 bytes a thread), cart state, scalars, counters and action from the
// whole workgroup.
static_assert(kSerialMax % 16 == 0 && (kDsW * kDsH) % 16 == 0, "serial and pixel rows are 16-byte multiples");
__global__ __launch_bounds__(256) void masked_state_kernel(DevState s, SnapState snap, const uint8_t* mask,
                                                           int with_pix) {
  __shared__ uint32_t list[256];
  __shared__ uint32_t count;
  const uint32_t t = threadIdx.x, e0 = blockIdx.x * 256u + t;
  if (t == 0) count = 0;
  __syncthreads();
  if (e0 < (uint32_t)s.n && mask[e0]) list[atomicAdd(&count, 1u)] = e0;
  __syncthreads();
  const uint32_t m = count;
  for (uint32_t i = 0; i < m; ++i) {
    const uint32_t e = list[i];
    for (uint32_t q = t; q < (uint32_t)kSerialMax / 16u; q += 256u)
      reinterpret_cast<uint4*>(s.serial + (size_t)e * kSerialMax)[q] = reinterpret_cast<const uint4*>(snap.serial)[q];
    if (with_pix)
      for (uint32_t q = t; q < (uint32_t)(kDsW * kDsH) / 16u; q += 256u)
        reinterpret_cast<uint4*>(s.pix + (size_t)e * kDsW * kDsH)[q] = reinterpret_cast<const uint4*>(snap.pix)[q];
    if (t < (uint32_t)kCartStateStride) s.cs[cs_index(e, (int)t)] = snap.cs[t];
    if (t < (uint32_t)kNumFields) s.sc[sc_index(e, (int)t)] = snap.sc[t];
    if (t < 2u) s.cnt[cnt_index(e, (int)t)] = snap.cnt[t];
    if (t == 0) s.actions[e] = snap.sc[F_ACTIONS];
  }
}

// RAM senses: out[e*k + j] = raw byte addrs[j] of env e.
__global__ void gather_kernel(DevState s, const uint16_t* addrs, int k, uint8_t* out) {
  const uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (uint32_t)s.n) return;
  const uint8_t* mb = s.mem + ((size_t)block_of(e) << 22);
  const uint32_t lane = e & (kEnvBlock - 1);
  auto byte = [&](int j) { return (uint32_t)mb[((size_t)addrs[j] << kEnvBlockShift) | lane]; };
  if (((reinterpret_cast<uintptr_t>(out) | (uintptr_t)k) & 15u) == 0u) {
    // the env's bytes 16-byte aligned: one 16-byte store per 16 (not one
    // byte store per sense, 64 lanes k bytes apart)
    for (int j0 = 0; j0 < k; j0 += 16) {
      uint32_t w[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        w[q] = byte(j0 + 4 * q) | (byte(j0 + 4 * q + 1) << 8) | (byte(j0 + 4 * q + 2) << 16) |
               (byte(j0 + 4 * q + 3) << 24);
      *reinterpret_cast<uint4*>(out + (size_t)e * k + j0) = make_uint4(w[0], w[1], w[2], w[3]);
    }
  } else {
    for (int j = 0; j < k; ++j) out[(size_t)e * k + j] = (uint8_t)byte(j);
  }
}

// Per-env linear hash: sum of byte * K[addr] over memory, plus the scalar
// fields, counters and cartridge state weighted by further K entries
// (wrapping uint64 arithmetic; K = splitmix64(index)).
__global__ void hash_kernel(DevState s, const uint64_t* K, uint64_t* out) {
  const uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (uint32_t)s.n) return;
  const uint8_t* mb = s.mem + ((size_t)block_of(e) << 22);
  const uint32_t lane = e & (kEnvBlock - 1);
  uint64_t h = 0;
  for (uint32_t a = 0; a < (uint32_t)kMemSize; ++a)
    h += (uint64_t)mb[((size_t)a << kEnvBlockShift) | lane] * K[a];
  for (int f = 0; f < kNumFields; ++f) {
    if (f == F_INSTR || f == F_CYCLES) continue;
    const int32_t v = f == F_ACTIONS ? s.actions[e] : s.sc[sc_index(e, f)];
    h += (uint64_t)(uint32_t)v * K[kMemSize + f];
  }
  h += (uint64_t)s.cnt[cnt_index(e, 0)] * K[kMemSize + F_INSTR];
  h += (uint64_t)s.cnt[cnt_index(e, 1)] * K[kMemSize + F_CYCLES];
  for (int k = 0; k < kCartStateStride; ++k)
    h += (uint64_t)(uint32_t)s.cs[cs_index(e, k)] * K[kMemSize + 64 + k];
  out[e] = h;
}

// Layout converters for the synchronous export/import helpers.
// Copies between a rectangle of the interleaved image (envs [env_lo, env_lo
// + count), addresses [lo, lo + len)) and an env-major buffer buf[count][len].
// One workgroup per tile of 64 envs x 64 addresses, staged in LDS: the image
// side is read or written one address row (64 neighbouring env bytes) per
// wavefront instruction and the buffer side one env row of 64 addresses, so
// both sides stay coalesced.  Rows are padded to 65 bytes so the transposed
// LDS accesses of a wavefront fall into different banks.
constexpr int kTile = 64;
constexpr int kTileThreads = 256;
__global__ __launch_bounds__(kTileThreads) void mem_range_kernel(DevState s, uint32_t env_lo,
                                                                 uint32_t count, uint32_t lo,
                                                                 uint32_t len, uint8_t* buf,
                                                                 int to_image) {
  __shared__ uint8_t tile[kTile][kTile + 1];  // [address][env]
  const uint32_t e0 = blockIdx.x * kTile, a0 = blockIdx.y * kTile, t = threadIdx.x;
  if (!to_image) {
    for (uint32_t i = t; i < (uint32_t)(kTile * kTile); i += kTileThreads) {
      const uint32_t ai = i / kTile, ei = i % kTile;  // lanes run over envs
      if (a0 + ai < len && e0 + ei < count)
        tile[ai][ei] = s.mem[mem_index(env_lo + e0 + ei, lo + a0 + ai)];
    }
    __syncthreads();
    for (uint32_t i = t; i < (uint32_t)(kTile * kTile); i += kTileThreads) {
      const uint32_t ei = i / kTile, ai = i % kTile;  // lanes run over addresses
      if (a0 + ai < len && e0 + ei < count) buf[(size_t)(e0 + ei) * len + a0 + ai] = tile[ai][ei];
    }
  } else {
    for (uint32_t i = t; i < (uint32_t)(kTile * kTile); i += kTileThreads) {
      const uint32_t ei = i / kTile, ai = i % kTile;
      if (a0 + ai < len && e0 + ei < count) tile[ai][ei] = buf[(size_t)(e0 + ei) * len + a0 + ai];
    }
    __syncthreads();
    for (uint32_t i = t; i < (uint32_t)(kTile * kTile); i += kTileThreads) {
      const uint32_t ai = i / kTile, ei = i % kTile;
      if (a0 + ai < len && e0 + ei < count)
        s.mem[mem_index(env_lo + e0 + ei, lo + a0 + ai)] = tile[ai][ei];
    }
  }
}
__global__ void export_cram_kernel(DevState s, uint32_t env_lo, uint32_t count, uint8_t* dst) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t stride = (uint32_t)s.cram_stride;
  if (i >= (size_t)count * stride) return;
  const uint32_t ei = (uint32_t)(i / stride), off = (uint32_t)(i % stride);
  dst[i] = s.cram[cram_index(env_lo + ei, off, stride)];
}

// One thread per element of the image: 32 scalars, 20 cart slots, then the
// bytes of memory, cart RAM and latches.
__global__ void env_image_kernel(DevState s, uint32_t env, uint8_t* img, int to_device,
                                 int parts) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t ram = (uint32_t)s.ram_bytes;
  const uint32_t n_mem = 52u + (uint32_t)kMemSize;
  int64_t* isc = reinterpret_cast<int64_t*>(img);
  int32_t* ics = reinterpret_cast<int32_t*>(img + kImgCart);
  if (i < 32u) {
    const int f = (int)i;
    if (f == F_INSTR || f == F_CYCLES) {
      int64_t& d = s.cnt[cnt_index(env, f - F_INSTR)];
      if (to_device) d = isc[f]; else isc[f] = d;
    } else if (f == F_ACTIONS) {
      if (to_device) s.actions[env] = (int32_t)isc[f]; else isc[f] = s.actions[env];
    } else {
      int32_t& d = s.sc[sc_index(env, f)];
      if (to_device) d = (int32_t)isc[f]; else isc[f] = d;
    }
  } else if (i < 52u) {
    int32_t& d = s.cs[cs_index(env, (int)(i - 32u))];
    if (to_device) d = ics[i - 32u]; else ics[i - 32u] = d;
  } else if (i < n_mem) {
    const uint32_t a = i - 52u;
    uint8_t& d = s.mem[mem_index(env, a)];
    if (to_device) d = img[kImgMem + a]; else img[kImgMem + a] = d;
  } else if (i < n_mem + ram) {
    const uint32_t off = i - n_mem;
    uint8_t& d = s.cram[cram_index(env, off, (uint32_t)s.cram_stride)];
    if (!to_device) img[kImgCram + off] = d;
    else if (parts & IMG_CRAM) d = img[kImgCram + off];
  } else if (i < n_mem + ram + (uint32_t)kLatchBytes) {
    const uint32_t k = i - n_mem - ram;  // [9][144] in the image
    uint8_t* src = img + img_latches_off((int)ram);
    uint8_t& d = s.latches[(k % (uint32_t)kScreenH) * kLatchStride + k / (uint32_t)kScreenH];
    if (!to_device) src[k] = d;
    else if (parts & IMG_LATCHES) d = src[k];
  }
}

}  // namespace

hipError_t launch_env_image(const DevState& s, int env, uint8_t* img, int to_device, int parts,
                            hipStream_t st) {
  const uint32_t total = 52u + (uint32_t)kMemSize + (uint32_t)s.ram_bytes + (uint32_t)kLatchBytes;
  hipLaunchKernelGGL(env_image_kernel, dim3((total + 255) / 256), dim3(256), 0, st, s,
                     (uint32_t)env, img, to_device, parts);
  return hipGetLastError();
}

hipError_t launch_reset(const DevState& s, hipStream_t st) {
  const size_t mem_bytes = (size_t)s.npad * kMemSize;
  const size_t n16 = mem_bytes / 16;
  hipLaunchKernelGGL(fill_mem_kernel, dim3((unsigned)((n16 + 255) / 256)), dim3(256), 0, st,
                     reinterpret_cast<uint4*>(s.mem), n16, s.boot);
  hipLaunchKernelGGL(init_state_kernel, dim3((unsigned)((s.npad + 255) / 256)), dim3(256), 0, st,
                     s.cs, s.sc, s.npad, s.mbc_kind);
  return hipGetLastError();
}

hipError_t launch_render_bg_env0(const DevState& s, uint8_t* out, hipStream_t st) {
  hipLaunchKernelGGL(frame_bg_kernel, dim3(kScreenH), dim3(kFrameThreads), 0, st, s, out);
  return hipGetLastError();
}

hipError_t launch_render(const DevState& s, uint8_t* out, int64_t base, int packed,
                         hipStream_t st) {
  if (s.n <= 0) return hipSuccess;
  // One workgroup fills a CU's LDS: with the blocks a multiple of 8 and the
  // groups spread evenly, one workgroup per CU (rounded down to a multiple
  // of 64) renders several groups, loading each next image while it renders
  // the current one; otherwise one group per workgroup.
  const uint32_t groups = (uint32_t)(s.npad / kImgEnvs);
  int dev = 0, cus = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err == hipSuccess) err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (err != hipSuccess) return err;
  uint32_t wgs = groups, rounds = 1;
  if (((s.npad >> kEnvBlockShift) & 7) == 0) {
    for (uint32_t w = ((uint32_t)cus / 64u) * 64u; w >= 64u; w -= 64u) {
      if (groups % w == 0 && groups / w >= 2u) {
        wgs = w;
        rounds = groups / w;
        break;
      }
    }
  }
  if (packed)
    hipLaunchKernelGGL(render_kernel<true>, dim3(wgs), dim3(kImgThreads), 0, st, s, out, base, rounds);
  else
    hipLaunchKernelGGL(render_kernel<false>, dim3(wgs), dim3(kImgThreads), 0, st, s, out, base, rounds);
  return hipGetLastError();
}

hipError_t launch_snapshot(const DevState& s, const SnapState& snap, int env, int with_pix,
                           hipStream_t st) {
  hipLaunchKernelGGL(snapshot_kernel, dim3(kMemSize / 256 + ((s.cram_stride + 255) / 256) + 1),
                     dim3(256), 0, st, s, snap, (uint32_t)env, with_pix);
  return hipGetLastError();
}

hipError_t launch_masked_reset(const DevState& s, const SnapState& snap, const uint8_t* mask,
                               int live, hipStream_t st) {
  if (s.n <= 0) return hipSuccess;
  const uint32_t chunks = (restore_rows((uint32_t)s.cram_stride, live != 0) + kResetRows - 1) / kResetRows;
  hipLaunchKernelGGL(masked_mem_kernel, dim3((unsigned)((s.n + kEnvBlock - 1) / kEnvBlock), chunks),
                     dim3(256), 0, st, s, snap.mem, snap.cram, mask, live);
  hipLaunchKernelGGL(masked_state_kernel, dim3((unsigned)((s.n + 255) / 256)), dim3(256), 0, st, s, snap,
                     mask, snap.has_pix);
  return hipGetLastError();
}

hipError_t launch_gather(const DevState& s, const uint16_t* addrs, int k, uint8_t* out,
                         hipStream_t st) {
  if (s.n <= 0 || k <= 0) return hipSuccess;
  hipLaunchKernelGGL(gather_kernel, dim3((unsigned)((s.n + 255) / 256)), dim3(256), 0, st, s, addrs,
                     k, out);
  return hipGetLastError();
}

hipError_t launch_hash(const DevState& s, const uint64_t* K, uint64_t* out, hipStream_t st) {
  if (s.n <= 0) return hipSuccess;
  hipLaunchKernelGGL(hash_kernel, dim3((unsigned)((s.n + 255) / 256)), dim3(256), 0, st, s, K, out);
  return hipGetLastError();
}

hipError_t launch_mem_range(const DevState& s, int env_lo, int count, int lo, int len, uint8_t* buf,
                            int to_image, hipStream_t st) {
  if (count <= 0 || len <= 0) return hipSuccess;
  // callers have checked env_lo + count <= n and lo + len <= 65536
  // envs on x (unbounded), address tiles on y (at most 1024)
  const dim3 grid((unsigned)((count + kTile - 1) / kTile), (unsigned)((len + kTile - 1) / kTile));
  hipLaunchKernelGGL(mem_range_kernel, grid, dim3(kTileThreads), 0, st, s, (uint32_t)env_lo,
                     (uint32_t)count, (uint32_t)lo, (uint32_t)len, buf, to_image);
  return hipGetLastError();
}

hipError_t launch_export_cram(const DevState& s, int env_lo, int count, uint8_t* dst,
                              hipStream_t st) {
  const size_t total = (size_t)count * (size_t)s.cram_stride;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(export_cram_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, s,
                     (uint32_t)env_lo, (uint32_t)count, dst);
  return hipGetLastError();
}

}  // namespace gbx

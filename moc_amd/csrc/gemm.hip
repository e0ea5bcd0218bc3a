// MFMA GEMM engine for the MoC FFN on gfx950.
//
//   C[M,N] = sum_k A(m,k) B(k,n)  [+ sum_k A2(m,k) B2(k,n)]
//
// The reference runs its nine FFN GEMMs through torch/cuBLAS
// (moc/ffn.py:141,146,163,203-254,389,394,414,447-494); here they run on the
// CDNA4 matrix cores (v_mfma_f32_32x32x16_bf16, f32 accumulation).  The
// optional second product lets dX = gG*W_gate + gU*W_up (moc/ffn.py:486,
// 491-494) accumulate in one pass instead of a GEMM plus an addmm.
//
// Operand layouts.  Each operand is K-contiguous ("KC": A(m,k) at
// A[m*lda + k], B(k,n) at B[n*ldb + k]) or MN-contiguous ("MN": A(m,k) at
// A[k*lda + m], B(k,n) at B[k*ldb + n]).  Tiles keep the layout they have in
// HBM: a KC tile is 256 rows x 64 k (128 B rows), an MN tile 64 k-rows x 256
// columns (512 B rows).  MFMA fragments (8 consecutive k of one row/column
// per lane) come out of a KC tile with one ds_read_b128 and out of an MN
// tile with two ds_read_b64_tr_b16 transposing reads, so no operand is ever
// transposed in registers or in HBM.
//
// Data movement.  Full K tiles travel HBM -> LDS with buffer_load_dwordx4
// ... lds (no VGPR staging).  Each wave instruction writes 1 KB of
// contiguous LDS, so bank-conflict freedom comes from an XOR swizzle of the
// 16-byte chunks inside a row, applied on the global-address side.  The
// swizzles keep the fragment reads conflict-free whether the LDS serves 8
// lanes x 16 B (32 banks) or 16 lanes x 16 B (64 banks) per clock:
//   KC: chunk c of tile row r lives in slot c ^ (r & 7) ^ ((r >> 3) & 1)
//       (b128 reads: 16 lanes = 16 rows, one logical chunk)
//   MN: chunk c of k-row r lives in slot c ^ f(r & 3), f = {0, 4, 10, 14}
//       (tr reads: 16 lanes = 4 k-rows x 32 B; 32 lanes = 4 k-rows x 64 B)
// Rows beyond the operand's extent are out of range of the buffer resource
// and read as zero; MN tiles need nothing else.  The last K tile of a KC
// operand whose K is not a multiple of 64 goes through registers with
// element masking (one tile per launch).
//
// Tiling: 256x256 C tile per workgroup, K step 64.  The main kernel
// (gemm_pp_kernel) runs eight waves of 128x64, two per SIMD, that alternate
// between MFMA phases and LDS/memory phases, its K tiles staged as halves in
// a five-slot LDS ring (160 KB; see there); a
// four-wave kernel (128x128 per wave, one barrier per K step) covers operands
// whose buffer offsets could wrap 32 bits.  Workgroup ids are remapped so
// that each XCD (ids are dealt round-robin over the 8 XCDs) works on a
// contiguous, M-grouped run of tiles that shares its L2.
//
// f32 operands use a plain FMA kernel (parity path for f32 models).
#include <algorithm>

#include "abi.h"
#include "common.h"

namespace moc {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x16_t __attribute__((ext_vector_type(16)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;

constexpr int kBM = 256, kBN = 256, kBK = 64, kThreads = 256;
constexpr int kStages = 2;                      // K tiles resident in LDS
constexpr int kPrefetch = 2;                    // L2 prefetch distance beyond the loaded tile
constexpr int kTileBytes = 256 * kBK * 2;       // one operand tile
constexpr int kBOffset = kStages * kTileBytes;  // LDS: A stages | B stages | prefetch sink
constexpr int kSinkOffset = 2 * kStages * kTileBytes;
constexpr int kLdsBytes = kSinkOffset + 1024;
constexpr int kLoads = kTileBytes / (kThreads * 16);  // 16-byte loads per thread per tile
constexpr int kCpr = kBK / 8;                   // 16-byte chunks per KC tile row
constexpr int kRowsPerLoad = 64 / kCpr;         // KC rows one wave instruction covers
constexpr int kBufferFlags = 0x00020000;        // raw buffer, 32-bit dwords
constexpr int kGroupM = 4;                      // M tiles per L2 group
constexpr uint32_t kOob = 0x80000000u;          // a buffer offset that reads as zero

static_assert(kLdsBytes <= 160 * 1024, "LDS budget");
static_assert(kLoads == 2 * (kBK / 16), "each k16 step issues two loads per operand");
// The 512-thread kernel's LDS ring: five 32 KB slots, each holding one half
// of a K tile of A (its first 16 KB) and of B (the next 16 KB).  A half is
// what one wave group loads:
// loads [0, kLoads / 2) or [kLoads / 2, kLoads) of each operand, i.e. rows
// 0-127 or 128-255 of a KC tile (0-63 or 64-127 of a 128-row A tile) and
// k-rows 0-31 or 32-63 of an MN tile.  Five slots let group 1 request its
// half of K tile t + 2 while tiles t and t + 1 are resident.
constexpr int kSlots = 5;
constexpr int kSlotBytes = 32 * 1024;
constexpr int kSlotB = 16 * 1024;  // B's half inside a slot
constexpr int kRingBytes = kSlots * kSlotBytes;
static_assert(kRingBytes <= 160 * 1024, "LDS budget");
// Structured-sparse product: a half's A region holds its 128 rows of
// 2:4-packed values (32 per 64-channel K tile: 64 bytes a row) and then
// their positions (8 bytes a row).
constexpr int kSpAHalf = 128 * 32 * 2;
static_assert(kSpAHalf + 128 * 8 <= kSlotB, "SP: packed rows and positions share a half's A region");
// The fix-up's LDS flag word after the main loop: past every epilogue's
// staging area (at most 128 KB)
constexpr int kFlagOffset = kRingBytes - 64;

struct Operand {
  const uint16_t* p;
  int64_t ld;   // elements between consecutive storage rows
  int ext;      // extent of M (A) or N (B)
  int K;
  int bytes;    // size of the buffer resource (rows * ld * 2, < 2^31)
};

struct GemmArgs {
  Operand a[2], b[2];
  int nk[2];    // K tiles of each product (nk[1] = 0: single product)
  int M, N;
  void* C;
  int64_t ldc;
  int tiles_m, tiles_n;
  int vec_store;  // C rows are 16-byte aligned: vector epilogue stores
  int pp;         // the 512-thread kernel may run this product
  int ksplit;     // workgroups per C tile (split-K; 512-thread kernel only)
  int kper;       // K tiles per split
  int64_t ws_stride;  // f32 elements between the partial C matrices of two splits
  // Tail fix-up (512-thread kernel, fix_tail > 0): workgroups [0, fix_full)
  // run whole tiles; each of the fix_tail tiles after them runs as two
  // workgroups, over K tiles [0, fix_split) and [fix_split, nk), and the
  // second to finish adds the other's partial (fix_part, [fix_tail][2]
  // partial tiles) and writes C.  fix_cnt: arrival counters [fix_tail],
  // zero at launch and left zero.
  int fix_full, fix_tail, fix_split;
  char* fix_part;
  int* fix_cnt;
  // MoC 2:8 gate/up launch (gemm_pp_kernel<..., GU = true>): B rows [0, 128)
  // of a tile are W_gate rows (b[0]), rows [128, 256) the same W_up rows
  // (b[1]); the epilogue writes top-2-of-8 indices and SiLU(g) u values.
  int64_t* gu_idx;
  uint16_t* gu_sz;
  int gu_inter;
  // Column-concatenated pair (512-thread kernel, ncat_tn > 0, single
  // product, no split): tile columns [0, ncat_tn) compute C = A b[0], tile
  // columns ncat_tn.. compute C2 = A b[1] (extent N2, row pitch ldc2), so two
  // products that share A fill the CUs as one launch.
  int ncat_tn, N2, vec_store2;
  void* C2;
  int64_t ldc2;
  // MoC 2:8 compacted Down (gemm_pp_kernel<..., SP = true>): a[0] holds the
  // activations 2:4-packed (two stored values per 4 channels: 32 values per
  // 64-channel K tile, a[0].K = 32 nk[0]) and sp_meta the stored values'
  // positions inside their 4-channel groups, laid out [nk][sp_rows][2] u32:
  // word h of row r for K tile t holds 2 bits per stored value, those of
  // channels 64t + 16h .. +16 in bits 0-15 and of 64t + 32 + 16h .. +16 in
  // bits 16-31 (the two 32-channel steps of the tile).
  const uint32_t* sp_meta;
  int sp_rows;
  // MoC 2:8 gate/up launch writing the 2:4-packed form of its selection
  // (gu_ap != nullptr) instead of (gu_idx, gu_sz): values ap[M, gu_ld_ap],
  // positions gu_meta in the sp_meta layout ([gu_nt][gu_meta_rows][2]).
  uint16_t* gu_ap;
  int64_t gu_ld_ap;
  uint32_t* gu_meta;
  int gu_meta_rows, gu_nt;
  // bf16 output plus a residual: C = bf16(bf16(A B) + R), R [M, N] bf16 with
  // rows ldres apart (16-byte aligned rows); null: plain C = bf16(A B).  The
  // decoder block's x + ffn(...) in the Down GEMM's epilogue.
  const uint16_t* res;
  int64_t ldres;
  // Grouped split-K launch (gemm_pp_kernel<..., DUAL = false, SPLIT = true>,
  // grp_wgs > 0): workgroups [0, grp_wgs) run the product above, the ones
  // after them a second product of the same operand layouts with operands
  // a[1], b[1] (nk[1] stays 0) and its own K tiles, extents, tiles, split
  // and partial slices (grp_C, rows grp_ldc apart, grp_ws_stride apart).
  int grp_wgs;
  int grp_nk, grp_M, grp_N, grp_tiles_m, grp_tiles_n, grp_ksplit, grp_kper;
  void* grp_C;
  int64_t grp_ldc, grp_ws_stride;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const Operand& o) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(o.p), (short)0, o.bytes,
                                           kBufferFlags);
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>((uintptr_t)((__attribute__((address_space(3))) const char*)p));
}

// One direct-to-LDS 16-byte load per lane: lane l's chunk lands at LDS byte
// m0 + 16 l.  The full byte offset travels in the VGPR (soffset 0) so the
// buffer range check covers it: offsets >= the resource size read as zero.
// Inline asm keeps the compiler from ordering these loads against each other
// or waiting for them before unrelated LDS reads; the kernel counts them
// itself (s_waitcnt vmcnt) before the barrier that publishes a stage.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, uint32_t m0, uint32_t voff) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen lds"
      :
      : "s"(m0), "v"(voff), "s"(rsrc)
      : "memory");
}

// Wait until the loads of a K tile have landed while the loads of the n
// newer tiles (2 kLoads each) and, with pf, the 2 newest prefetches may still
// be in flight (vector memory loads complete in issue order).
__device__ __forceinline__ void wait_tiles(int n, bool pf) {
  if (pf) {
    switch (n) {
      case 0: asm volatile("s_waitcnt vmcnt(2)" ::: "memory"); break;
      case 1: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * kLoads + 2) : "memory"); break;
      default: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * kLoads + 2) : "memory"); break;
    }
  } else {
    switch (n) {
      case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
      case 1: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * kLoads) : "memory"); break;
      default: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * kLoads) : "memory"); break;
    }
  }
}

// Swizzle terms (see the header): KC slot = c ^ kc_swz(row & 15), MN slot =
// c ^ mn_swz(k-row & 3).
__device__ __forceinline__ int kc_swz(int r) {
  return kCpr == 8 ? ((r & 7) ^ ((r >> 3) & 1)) : (((r >> 1) ^ (r >> 3)) & 3);
}
__device__ __forceinline__ int mn_swz(int r) { return ((r & 1) << 2) + ((r >> 1) & 1) * 10; }
// 2:4-packed A tile (64-byte rows of four 16-byte chunks): chunk c of row r
// in slot c ^ sp_swz(r & 15).  Rows r .. r + 15 reading one logical chunk hit
// 16 distinct 16-byte bank groups, and rows r .. r + 7 eight distinct ones
// within their 128 bytes.
__device__ __forceinline__ int sp_swz(int r) { return ((r >> 1) ^ (r >> 3)) & 3; }

// -------------------------------------------------------------- tile loading
// Thread (wave w, lane l) moves kLoads chunks of 16 bytes per operand tile;
// wave instruction j fills LDS bytes [(4j + w) KB, +1 KB) of the tile.
//   KC tile (256 rows x kBK k): instruction j covers rows R(4j + w) .. +R,
//     R = 64 / kCpr; lane l: row +l/kCpr, slot l%kCpr, logical chunk
//     c = slot ^ kc_swz(row)  (row & 15 depends on w and l only).
//   MN tile (32 k-rows x 256 columns, 512-byte rows): instruction j covers
//     k-rows 2(4j + w) .. +2; lane l: k-row +l/32, slot l%32, logical chunk
//     c = (l%32) ^ mn_swz(row).
template <bool KC>
struct TileMap {
  uint32_t voff[kLoads];  // byte offsets at k = 0 (kOob for rows beyond the extent)
  int kchunk;             // KC: first k of this lane's chunk within a tile

  __device__ __forceinline__ void init(const Operand& o, int row0, int wave, int lane) {
    kchunk = 8 * ((lane % kCpr) ^ kc_swz((wave * kRowsPerLoad + lane / kCpr) & 15));
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
      if (KC) {
        const int r = row0 + (j * 4 + wave) * kRowsPerLoad + lane / kCpr;
        const int64_t e = static_cast<int64_t>(r) * o.ld + kchunk;
        voff[j] = (r < o.ext) ? static_cast<uint32_t>(e * 2) : kOob;
      } else {
        const int r = (j * 4 + wave) * 2 + (lane >> 5);
        const int c = (lane & 31) ^ mn_swz(r);
        const int64_t e = static_cast<int64_t>(r) * o.ld + row0 + c * 8;
        voff[j] = static_cast<uint32_t>(e * 2);
      }
    }
  }

  // Issue loads j0, j0+1 of the K tile at k0 into the tile at LDS byte
  // `tile`.  KC: chunks at k >= K read as zero (a chunk straddling K is fixed
  // up by zero_straddle once it has landed).  MN: k-rows >= K lie past the
  // end of the buffer and read as zero.
  __device__ __forceinline__ void issue2(__amdgpu_buffer_rsrc_t rsrc, const Operand& o, int k0,
                                         uint32_t tile, int wave, int j0) const {
    const uint32_t kofs = KC ? static_cast<uint32_t>(k0) * 2u
                             : static_cast<uint32_t>(static_cast<int64_t>(k0) * o.ld * 2);
    const bool dead = KC && (k0 + kchunk >= o.K);
#pragma unroll
    for (int j = j0; j < j0 + 2; ++j) {
      const uint32_t m0 = __builtin_amdgcn_readfirstlane(tile + (j * 4 + wave) * 1024);
      dma16(rsrc, m0, dead ? kOob : voff[j] + kofs);
    }
  }

  // Pull the K tile at k0 into L2 ahead of its real loads: one 16-byte load
  // per 128-byte line of the tile, landing in a shared LDS sink.  KC: one
  // tile row per thread; MN: a quarter k-row (128 bytes) per thread.
  static __device__ __forceinline__ void prefetch(__amdgpu_buffer_rsrc_t rsrc, const Operand& o,
                                                  int k0, int row0, uint32_t sink, int tid) {
    uint32_t off;
    if (KC) {
      const int r = row0 + tid;
      off = (r < o.ext && k0 < o.K)
                ? static_cast<uint32_t>((static_cast<int64_t>(r) * o.ld + k0) * 2)
                : kOob;
    } else {
      const int64_t e = static_cast<int64_t>(k0 + (tid >> 2)) * o.ld + row0 + 64 * (tid & 3);
      off = (tid >> 2) < kBK ? static_cast<uint32_t>(e * 2) : kOob;
    }
    dma16(rsrc, __builtin_amdgcn_readfirstlane(sink), off);
  }

  // KC, K % 8 != 0: zero the elements k >= K of the chunk that straddles K
  // (its loads must have landed).
  __device__ __forceinline__ void zero_straddle(char* lds, const Operand& o, int k0,
                                                uint32_t tile, int wave, int lane) const {
    const int k = k0 + kchunk;
    if (!(k < o.K && o.K < k + 8)) return;
    const int valid = o.K - k;
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
      uint16_t* q = reinterpret_cast<uint16_t*>(lds + tile + (j * 4 + wave) * 1024 + lane * 16);
      for (int e = valid; e < 8; ++e) q[e] = 0;
    }
  }
};

// ------------------------------------------------------------ fragment reads
// 32x32x16 MFMA operand fragment: lane l holds 8 consecutive k (8*(l/32)..)
// of row/column (l % 32) of a 32-wide block.  Per-lane base offsets are
// computed once; block, k step and stage enter as added offsets.
template <bool KC>
struct FragMap {
  // Byte address of the lane's fragment for block 0, k16 step 0, stage 0.
  // The other fragments differ only in bits that no other term touches, so
  // they are one XOR away: KC fragments of k16 step ks at base ^ 32 ks (the
  // swizzled chunk index (2 ks + l/32) ^ swz = ((l/32) ^ swz) ^ 2 ks), MN
  // fragments of block bi at base ^ 64 bi (the chunk index c + 4 bi, c % 4 =
  // c, sets bits 2-3 of c when the wave's offset is a multiple of 128, or for
  // bi < 2).  Keeping one register per operand matters for the 512-thread
  // kernel, whose 256-register budget holds 128 accumulators and a K tile of
  // fragments.
  uint32_t base;

  // region: LDS byte of this operand's stage-0 tile; wofs: the wave's row
  // offset inside the 256-row tile (a multiple of 64; of 128 if blocks 2-3
  // of an MN operand are read)
  __device__ __forceinline__ void init(uint32_t region, int wofs, int lane) {
    if (KC) {
      // rows wofs + 32 blk + (lane & 31): row & 15 = lane & 15
      const uint32_t row = static_cast<uint32_t>(wofs + (lane & 31)) * (kBK * 2);
      const int swz = kc_swz(lane & 15);
      base = region + row + static_cast<uint32_t>(((lane >> 5) ^ swz) * 16);
    } else {
      // lane = 16 g + i reads k-row 8(g >> 1) + i/4 (+16 ks) and columns
      // m = blk + 16(g & 1) + 4(i & 3) .. +3 of chunk m/8
      const int i = lane & 15, g = lane >> 4;
      const int r = 8 * (g >> 1) + (i >> 2);
      const int swz = mn_swz(i >> 2);
      const int c = (wofs + 16 * (g & 1) + 4 * (i & 3)) >> 3;
      base = region + r * 512 + 8 * (i & 1) + 16 * (c ^ swz);
    }
  }

  // so: byte offset of the stage's tile (a multiple of 32 KB, so adding it
  // before the XOR is the same as after).  ring: so is the ring slot of the
  // half that holds the fragment; an MN half holds two k16 steps.
  __device__ __forceinline__ bf16x8_t read(const char* lds, int blk, int ks, uint32_t so,
                                           bool ring = false) const {
    if (KC) {
      const char* p = lds + ((base + so) ^ (32u * ks)) + blk * (32 * kBK * 2);
      return __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(p));
    } else {
      const char* p = lds + ((base + so) ^ (64u * blk)) + (ring ? (ks & 1) : ks) * 8192;
      const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)p);
      const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(p + 4 * 512));
      const i16x4_t v[2] = {lo, hi};
      return __builtin_bit_cast(bf16x8_t, v);
    }
  }
};

// -------------------------------------------------------------- tile order
__device__ __forceinline__ void tile_coords(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  const int per = total / 8;
  int t = bid;
  if (bid < per * 8) t = (bid & 7) * per + (bid >> 3);
  const int span = kGroupM * tiles_n;
  const int grp = t / span;
  const int first = grp * kGroupM;
  const int gsize = min(tiles_m - first, kGroupM);
  const int in = t - grp * span;
  tm = first + in % gsize;
  tn = in / gsize;
}

// ---------------------------------------------------------------- epilogue
// Each wave stages 32 rows x 128 columns of its results in its own LDS
// region and writes them back as 16-byte row segments.  The accumulators
// hold transposed blocks, so a lane's four consecutive elements r = 4q..4q+3
// are four consecutive columns of one row: one packed conversion pair and one
// 8-byte (bf16) or 16-byte (f32) LDS write each.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}

// Eight bf16 values of C (a 16-byte segment) plus the residual's eight at
// r (n < 8: only the first n are read), each bf16(c + r).
__device__ __forceinline__ uint4 add_residual8(uint4 v, const uint16_t* r, int n) {
  uint32_t rw[4];
  if (n >= 8) {
    const uint4 t = *reinterpret_cast<const uint4*>(r);
    rw[0] = t.x;
    rw[1] = t.y;
    rw[2] = t.z;
    rw[3] = t.w;
  } else {
    for (int q = 0; q < 4; ++q) {
      const uint32_t lo = 2 * q < n ? r[2 * q] : 0u, hi = 2 * q + 1 < n ? r[2 * q + 1] : 0u;
      rw[q] = lo | (hi << 16);
    }
  }
  const uint32_t cw[4] = {v.x, v.y, v.z, v.w};
  uint32_t o[4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
    o[q] = pack_bf16x2(__uint_as_float(cw[q] << 16) + __uint_as_float(rw[q] << 16),
                       __uint_as_float(cw[q] & 0xFFFF0000u) + __uint_as_float(rw[q] & 0xFFFF0000u));
  return make_uint4(o[0], o[1], o[2], o[3]);
}

template <bool OUT_F32, int NJ, int MI = 4>
__device__ __forceinline__ void store_tile_w(const GemmArgs& g, char* lds, const f32x16_t (&acc)[MI][NJ],
                                             int row0, int col0, int wm, int wn, int wave, int lane) {
  constexpr int kEsz = OUT_F32 ? 4 : 2;
  constexpr int kCols = 32 * NJ;  // columns of the wave's tile
  // row pitch: 16-byte aligned, +16 bytes so that rows r and r + 1 start on
  // different banks
  constexpr int kPitch = kCols * kEsz + 16;
  char* reg = lds + wave * (32 * kPitch);
  const bool vec = g.vec_store != 0;
#pragma unroll
  for (int i = 0; i < MI; ++i) {
    char* rowp = reg + (lane & 31) * kPitch;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        char* dst = rowp + (32 * j + 8 * q + 4 * (lane >> 5)) * kEsz;
        const f32x16_t& a = acc[i][j];
        if (OUT_F32) {
          *reinterpret_cast<float4*>(dst) = make_float4(a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]);
        } else {
          *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf16x2(a[4 * q], a[4 * q + 1]),
                                                      pack_bf16x2(a[4 * q + 2], a[4 * q + 3]));
        }
      }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes are done
    // read back: 16-byte segments
    constexpr int kSegs = kCols * kEsz / 16;        // per row
    constexpr int kIters = 32 * kSegs / 64;
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      const int e = it * 64 + lane;
      const int row = e / kSegs, seg = e % kSegs;
      uint4 v = *reinterpret_cast<const uint4*>(reg + row * kPitch + seg * 16);
      const int grow = row0 + wm + 32 * i + row;
      const int gcol = col0 + wn + seg * (16 / kEsz);
      if (grow >= g.M || gcol >= g.N) continue;
      if constexpr (!OUT_F32) {
        if (g.res != nullptr) v = add_residual8(v, g.res + static_cast<int64_t>(grow) * g.ldres + gcol, g.N - gcol);
      }
      char* dst = static_cast<char*>(g.C) + (static_cast<int64_t>(grow) * g.ldc + gcol) * kEsz;
      if (vec && gcol + 16 / kEsz <= g.N) {
        *reinterpret_cast<uint4*>(dst) = v;
      } else {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
        if (OUT_F32) {
          for (int q = 0; q < 4 && gcol + q < g.N; ++q)
            reinterpret_cast<float*>(dst)[q] = __uint_as_float(w[q]);
        } else {
          for (int q = 0; q < 8 && gcol + q < g.N; ++q)
            reinterpret_cast<uint16_t*>(dst)[q] = static_cast<uint16_t>(w[q >> 1] >> (16 * (q & 1)));
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
  }
}

// The same write-back for accumulators in the MFMA's own orientation (the
// structured-sparse product, whose sparse operand must come first): lane l
// holds column 32 j + (l & 31) of rows 8q + 4(l >> 5) + r.  Each element is
// staged with its own LDS write, then rows go out as 16-byte segments.
template <bool OUT_F32, int NJ>
__device__ __forceinline__ void store_tile_t(const GemmArgs& g, char* lds, const f32x16_t (&acc)[4][NJ],
                                             int row0, int col0, int wm, int wn, int wave, int lane) {
  constexpr int kEsz = OUT_F32 ? 4 : 2;
  constexpr int kCols = 32 * NJ;
  constexpr int kPitch = kCols * kEsz + 16;
  char* reg = lds + wave * (32 * kPitch);
  const bool vec = g.vec_store != 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          char* dst = reg + (8 * q + 4 * (lane >> 5) + r) * kPitch + (32 * j + (lane & 31)) * kEsz;
          const float v = acc[i][j][4 * q + r];
          if (OUT_F32) *reinterpret_cast<float*>(dst) = v;
          else *reinterpret_cast<uint16_t*>(dst) = static_cast<uint16_t>(pack_bf16x2(v, 0.f) & 0xFFFFu);
        }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    constexpr int kSegs = kCols * kEsz / 16;
    constexpr int kIters = 32 * kSegs / 64;
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      const int e = it * 64 + lane;
      const int row = e / kSegs, seg = e % kSegs;
      uint4 v = *reinterpret_cast<const uint4*>(reg + row * kPitch + seg * 16);
      const int grow = row0 + wm + 32 * i + row;
      const int gcol = col0 + wn + seg * (16 / kEsz);
      if (grow >= g.M || gcol >= g.N) continue;
      if constexpr (!OUT_F32) {
        if (g.res != nullptr) v = add_residual8(v, g.res + static_cast<int64_t>(grow) * g.ldres + gcol, g.N - gcol);
      }
      char* dst = static_cast<char*>(g.C) + (static_cast<int64_t>(grow) * g.ldc + gcol) * kEsz;
      if (vec && gcol + 16 / kEsz <= g.N) {
        *reinterpret_cast<uint4*>(dst) = v;
      } else {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
        if (OUT_F32) {
          for (int q = 0; q < 4 && gcol + q < g.N; ++q)
            reinterpret_cast<float*>(dst)[q] = __uint_as_float(w[q]);
        } else {
          for (int q = 0; q < 8 && gcol + q < g.N; ++q)
            reinterpret_cast<uint16_t*>(dst)[q] = static_cast<uint16_t>(w[q >> 1] >> (16 * (q & 1)));
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
  }
}

template <bool A_KC, bool B_KC, bool OUT_F32, bool DUAL>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm_bf16_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(1024))) char lds[kLdsBytes];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int tm, tn;
  tile_coords(blockIdx.x, g.tiles_m, g.tiles_n, tm, tn);
  const int row0 = tm * kBM;
  const int col0 = tn * kBN;
  const int wm = (wave >> 1) * 128;
  const int wn = (wave & 1) * 128;
  const uint32_t lds0 = lds_addr(lds);

  const int nk0 = g.nk[0];
  const int nk = nk0 + (DUAL ? g.nk[1] : 0);

  TileMap<A_KC> ma0, ma1;
  TileMap<B_KC> mb0, mb1;
  ma0.init(g.a[0], row0, wave, lane);
  mb0.init(g.b[0], col0, wave, lane);
  const __amdgpu_buffer_rsrc_t ra0 = make_rsrc(g.a[0]), rb0 = make_rsrc(g.b[0]);
  __amdgpu_buffer_rsrc_t ra1 = ra0, rb1 = rb0;
  if (DUAL) {
    ma1.init(g.a[1], row0, wave, lane);
    mb1.init(g.b[1], col0, wave, lane);
    ra1 = make_rsrc(g.a[1]);
    rb1 = make_rsrc(g.b[1]);
  }
  FragMap<A_KC> fa_map;
  FragMap<B_KC> fb_map;
  fa_map.init(0, wm, lane);
  fb_map.init(kBOffset, wn, lane);

  // Issue share h (loads 2h, 2h+1 of A and of B) of K tile t into stage st.
  auto stage_load = [&](int t, int st, int h) {
    const uint32_t at = lds0 + st * kTileBytes, bt = lds0 + kBOffset + st * kTileBytes;
    if (DUAL && t >= nk0) {
      const int k0 = (t - nk0) * kBK;
      ma1.issue2(ra1, g.a[1], k0, at, wave, 2 * h);
      mb1.issue2(rb1, g.b[1], k0, bt, wave, 2 * h);
    } else {
      const int k0 = t * kBK;
      ma0.issue2(ra0, g.a[0], k0, at, wave, 2 * h);
      mb0.issue2(rb0, g.b[0], k0, bt, wave, 2 * h);
    }
  };
  // L2 prefetch of K tile t (A and B: two loads per thread).
  auto tile_prefetch = [&](int t) {
    const uint32_t sink = lds0 + kSinkOffset;
    if (DUAL && t >= nk0) {
      const int k0 = (t - nk0) * kBK;
      ma1.prefetch(ra1, g.a[1], k0, row0, sink, tid);
      mb1.prefetch(rb1, g.b[1], k0, col0, sink, tid);
    } else {
      const int k0 = t * kBK;
      ma0.prefetch(ra0, g.a[0], k0, row0, sink, tid);
      mb0.prefetch(rb0, g.b[0], k0, col0, sink, tid);
    }
  };
  // After tile t's loads have landed: zero KC elements beyond a K that is
  // not a multiple of 8 (only the last tile of a product can need it).
  auto stage_fix = [&](int t, int st) {
    const uint32_t at = st * kTileBytes, bt = kBOffset + st * kTileBytes;
    const bool p1 = DUAL && t >= nk0;
    const Operand& oa = p1 ? g.a[1] : g.a[0];
    const int k0 = (p1 ? t - nk0 : t) * kBK;
    if (k0 + kBK <= oa.K || (oa.K & 7) == 0) return;
    // kchunk depends on the lane only, so the product-0 maps serve both
    if (A_KC) ma0.zero_straddle(lds, oa, k0, at, wave, lane);
    if (B_KC) mb0.zero_straddle(lds, p1 ? g.b[1] : g.b[0], k0, bt, wave, lane);
  };

  f32x16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // kBK/16 k16 steps of 16 MFMAs per K tile.  The other work of a step -
  // reading the next step's 8 fragments from LDS and issuing a share of the
  // loads of K tile `tnext` (plus, after the last share, the L2 prefetch of
  // tile tpf) - is interleaved one instruction group per MFMA, so it issues
  // in the shadow of the matrix pipeline instead of between MFMA bursts
  // (sched_barrier pins the order).
  auto compute = [&](int st, int tnext, int tpf) {
    const uint32_t so = st * kTileBytes;
    bf16x8_t fa[2][4], fb[2][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) fa[0][i] = fa_map.read(lds, i, 0, so);
#pragma unroll
    for (int j = 0; j < 4; ++j) fb[0][j] = fb_map.read(lds, j, 0, so);
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      const int cb = ks & 1;
      const bool more = ks + 1 < kBK / 16;
#pragma unroll
      for (int idx = 0; idx < 16; ++idx) {
        const int i = idx >> 2, j = idx & 3;
        // B as the MFMA's first operand: acc[i][j] holds the block transposed,
        // lane l: row 32 i + l % 32, columns 32 j + 8(r/4) + 4(l/32) + r % 4
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[cb][j], fa[cb][i], acc[i][j], 0, 0, 0);
        if (more && idx < 4) fa[cb ^ 1][idx] = fa_map.read(lds, idx, ks + 1, so);
        if (more && idx >= 4 && idx < 8) fb[cb ^ 1][idx - 4] = fb_map.read(lds, idx - 4, ks + 1, so);
        if (idx == 9 && tnext < nk) stage_load(tnext, tnext % kStages, ks);
        if (idx == 13 && ks == kBK / 16 - 1 && tpf < nk) tile_prefetch(tpf);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };

  // prologue: tiles 0 .. kStages-2 in flight
#pragma unroll
  for (int p = 0; p < kStages - 1; ++p)
    if (p < nk) {
#pragma unroll
      for (int h = 0; h < kLoads / 2; ++h) stage_load(p, p, h);
    }

  for (int t = 0; t < nk; ++t) {
    const int st = t % kStages;
    // tiles t+1 .. t+kStages-2 may stay in flight (kLoads*2 loads each), and
    // the prefetch issued by the previous trip
    wait_tiles(min(kStages - 2, nk - 1 - t), t > 0 && t + kStages - 2 + kPrefetch < nk);
    stage_fix(t, st);
    __syncthreads();  // tile t visible to all waves; tile t-1's stage is free
    compute(st, t + kStages - 1, t + kStages - 1 + kPrefetch);
  }
  __syncthreads();  // every wave is done with the LDS stages
  store_tile_w<OUT_F32, 4>(g, lds, acc, row0, col0, wm, wn, wave, lane);
}

// ---------------------------------------------------------------------------
// Ping-pong variant: 512 threads, two waves per SIMD.
//
// The same 256x256 C tile and 64-deep K tiles in the same two LDS stages, but
// eight waves of 128x64 (4x2 blocks of 32x32, 128 accumulators per lane) in
// two groups.  Waves 0-3 (group 0) and 4-7 (group 1) sit one per SIMD each,
// and the groups alternate between a compute phase (the 32 MFMAs of one K
// tile, fragments already in registers) and a memory phase (all fragments of
// the next K tile from LDS, plus, for group 0, the direct-to-LDS loads of the
// tile after it; for group 1 the L2 prefetch), with one workgroup barrier
// between phases:
//   phase 2t:    group 0 reads K tile t, loads tile t+1   | group 1 MFMAs tile t-1
//   phase 2t+1:  group 0 MFMAs tile t                     | group 1 reads K tile t
// so each SIMD's matrix pipe is fed by one wave while the other waits on LDS
// and memory.  Tile t+1 lands in the stage of tile t-1, whose last reader
// (group 1, phase 2t-1) is past a barrier; group 0 waits for its loads at the
// end of its compute phase, a whole K tile after issuing them.
// ---------------------------------------------------------------------------
constexpr int kPpThreads = 512;
constexpr int kShortMaxKTiles = 40;  // longest K (in 64-deep tiles) run on 128-row tiles
// Direct-to-LDS load offsets of one operand for a wave (index 0-3 within its
// group): the eight loads of a tile differ by a uniform stride, so only load
// 0 is kept.
template <bool KC>
struct LoadMap {
  uint32_t voff0;  // byte offset of load 0 at k = 0
  int kchunk;      // KC: first k of this lane's chunk within a tile

  // Rows past the extent (KC) and k-rows past K (MN) are not checked here:
  // their offsets land past the end of the buffer resource and read as zero.
  // The host guarantees that no such offset wraps around 2^32.
  __device__ __forceinline__ void init(const Operand& o, int row0, int wave, int lane) {
    if (KC) {
      kchunk = 8 * ((lane % kCpr) ^ kc_swz((wave * kRowsPerLoad + lane / kCpr) & 15));
      const int r = row0 + wave * kRowsPerLoad + lane / kCpr;
      voff0 = static_cast<uint32_t>((static_cast<int64_t>(r) * o.ld + kchunk) * 2);
    } else {
      kchunk = 0;
      const int r = wave * 2 + (lane >> 5);
      const int c = (lane & 31) ^ mn_swz(r);
      voff0 = static_cast<uint32_t>((static_cast<int64_t>(r) * o.ld + row0 + c * 8) * 2);
    }
  }

  // Lane offset of load 0 of the K tile at k0; a KC chunk at k >= K reads as
  // zero (kOob + j * stride stays >= 2^31).
  __device__ __forceinline__ uint32_t tile_base(const Operand& o, int k0) const {
    const uint32_t kofs = KC ? static_cast<uint32_t>(k0) * 2u
                             : static_cast<uint32_t>(static_cast<int64_t>(k0) * o.ld * 2);
    uint32_t b = voff0 + kofs;
    if (KC && k0 + kchunk >= o.K) b = kOob;
    // opaque: keeps the compiler from hoisting the per-load offsets out of
    // the K loop (they would stay live in registers the 512-thread kernel
    // lacks)
    asm volatile("" : "+v"(b));
    return b;
  }

  // Load j of the K tile whose tile_base is b into the tile at LDS byte
  // `tile` (the placement of TileMap::issue2), counted from load jbase: the
  // loads of one half of a tile in an LDS ring slot.
  __device__ __forceinline__ void issue(__amdgpu_buffer_rsrc_t rsrc, const Operand& o, uint32_t b,
                                        uint32_t tile, int wave, int j, int jbase = 0) const {
    const uint32_t jstride = KC ? static_cast<uint32_t>(4 * kRowsPerLoad * o.ld * 2)
                                : static_cast<uint32_t>(8 * o.ld * 2);
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(tile + ((j - jbase) * 4 + wave) * 1024);
    dma16(rsrc, m0, b + j * jstride);
  }

  // KC, K % 8 != 0: zero the elements k >= K of the chunk that straddles K
  // (its loads must have landed); loads [j0, j1) placed as by issue.
  __device__ __forceinline__ void zero_straddle(char* lds, const Operand& o, int k0, uint32_t tile, int wave,
                                                int lane, int j0, int j1, int jbase = 0) const {
    const int k = k0 + kchunk;
    if (!(k < o.K && o.K < k + 8)) return;
    const int valid = o.K - k;  // 1 .. 7 elements stay
    uint32_t keep[4];
#pragma unroll
    for (int d = 0; d < 4; ++d)
      keep[d] = 2 * d + 1 < valid ? 0xFFFFFFFFu : (2 * d < valid ? 0x0000FFFFu : 0u);
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
      if (j < j0 || j >= j1) continue;
      uint4* q = reinterpret_cast<uint4*>(lds + tile + ((j - jbase) * 4 + wave) * 1024 + lane * 16);
      uint4 v = *q;
      v.x &= keep[0];
      v.y &= keep[1];
      v.z &= keep[2];
      v.w &= keep[3];
      *q = v;
    }
  }
};

// ------------------------------------------------------------ tail fix-up
// A tile of the last, partial round of a launch (every tile when a launch
// has fewer tiles than CUs) runs as two workgroups: part 0 over K tiles
// [0, fix_kper), part 1 over the rest.  The one that finishes first stores
// its f32 partial tile in accumulator order (16-byte word (b, q, tid) =
// acc[b / 2][b % 2][4q .. 4q+3] of thread tid: one wave instruction covers
// 1 KB) with device-coherent stores, waits for them and bumps the tile's
// arrival counter (an agent-scope release); the one that finishes second
// (it finds the counter at 1, or its own increment returns 1, each an
// agent-scope acquire) reads that partial back with device-coherent loads,
// adds it to its registers (a + b = b + a, so the
// result does not depend on which part came second), writes C and resets
// the counter.  Nothing waits on another workgroup.
constexpr int kPartBytes = 8 * 4 * kPpThreads * 16;  // one partial tile (256 KB)
constexpr int kFixCounterBytes = MOC_GEMM_WS_COUNTER_BYTES;  // arrival counters at the workspace start
constexpr int kCoherent = 16;                         // buffer op cache policy: sc1

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// Returns true in the second workgroup of the tile; acc then holds the sum
// of both parts.  flag: one LDS word.
template <int MI = 4>
__device__ __forceinline__ bool fix_arrive(const GemmArgs& g, f32x16_t (&acc)[MI][2], int slot, int part,
                                           int tid, int* flag) {
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      g.fix_part + static_cast<int64_t>(slot) * 2 * kPartBytes, (short)0, 2 * kPartBytes, kBufferFlags);
  int* cnt = g.fix_cnt + slot;
  // acquire: if the other part has arrived, its partial is visible to the
  // loads below (on this GPU the L2 of each XCD is private, so the two parts
  // of a tile need the agent-scope release/acquire pair, not just coherent
  // data stores, whichever XCDs they run on)
  if (tid == 0) *flag = __hip_atomic_load(cnt, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (*flag == 0) {
    // first so far: publish the partial, then arrive
#pragma unroll
    for (int b = 0; b < 2 * MI; ++b)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x16_t& a = acc[b >> 1][b & 1];
        const u32x4_t v = {__float_as_uint(a[4 * q]), __float_as_uint(a[4 * q + 1]),
                           __float_as_uint(a[4 * q + 2]), __float_as_uint(a[4 * q + 3])};
        __builtin_amdgcn_raw_buffer_store_b128(
            v, rsrc, static_cast<uint32_t>(part * kPartBytes + ((b * 4 + q) * kPpThreads + tid) * 16), 0,
            kCoherent);
      }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partial is stored
    __syncthreads();
    if (tid == 0) *flag = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (*flag == 0) return false;
  }
  // second: the other part's partial plus ours
  const uint32_t other = static_cast<uint32_t>((1 - part) * kPartBytes);
#pragma unroll
  for (int b = 0; b < 2 * MI; ++b) {
    f32x16_t& a = acc[b >> 1][b & 1];
    u32x4_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
      w[q] = __builtin_amdgcn_raw_buffer_load_b128(
          rsrc, other + static_cast<uint32_t>(((b * 4 + q) * kPpThreads + tid) * 16), 0, kCoherent);
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int c = 0; c < 4; ++c) a[4 * q + c] += __uint_as_float(w[q][c]);
  }
  if (tid == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // for the next call
  return true;
}

// ------------------------------------------------------ MoC 2:8 epilogue
// The C tile of a gate/up launch holds, for 256 tokens, the gate values of
// 128 channels (columns 0-127) and their up values (columns 128-255).  They
// are rounded to bf16 and staged in LDS (G then U, 256 B rows whose 16-byte
// chunks are XOR-swizzled by row), then each thread selects the top 2 of a
// (token, group of 8 channels) item and writes its two indices (int64) and
// two SiLU(g) u values (bf16) in the reference's compacted layout
// [token][group][top-1, top-2].
__device__ __forceinline__ void gu28_epilogue(const GemmArgs& g, char* lds, const f32x16_t (&acc)[4][2],
                                              int row0, int col0, int wm, int wn, int tid, int lane) {
  constexpr int kU = 256 * 256;  // byte offset of the U rows
  __syncthreads();               // every wave is done with the LDS stages
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = wm + 32 * i + (lane & 31);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = wn + 32 * j;
      char* base = lds + (col < 128 ? 0 : kU) + row * 256;
      const f32x16_t& a = acc[i][j];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int cc = (col & 127) + 8 * q + 4 * (lane >> 5);
        *reinterpret_cast<uint2*>(base + (((cc >> 3) ^ (row & 15)) << 4) + (cc & 7) * 2) =
            make_uint2(pack_bf16x2(a[4 * q], a[4 * q + 1]), pack_bf16x2(a[4 * q + 2], a[4 * q + 3]));
      }
    }
  }
  __syncthreads();
  const int kout = g.gu_inter / 4;
  if (g.gu_ap != nullptr) {
    // packed form: item (token, 8-group G) writes its four stored values
    // (8 bytes) and its positions byte; the four 8-groups of one position
    // word sit in lanes l, l ^ 1, l ^ 4, l ^ 5 (G & 15 = l & 15), which
    // combine it before one of them stores it.
#pragma unroll 2
    for (int item = tid; item < 256 * 16; item += kPpThreads) {
      const int tr = item >> 4, grp8 = item & 15;
      const int tok = row0 + tr, cg = col0 + grp8 * 8;
      const int G = cg >> 3;
      uint16_t q[4] = {0, 0, 0, 0};
      uint32_t pos = kPackEmpty2of8;
      if (tok < g.M && cg < g.gu_inter) {
        const int off = tr * 256 + ((grp8 ^ (tr & 15)) << 4);
        const uint4 gv = *reinterpret_cast<const uint4*>(lds + off);
        const uint4 uv = *reinterpret_cast<const uint4*>(lds + kU + off);
        const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
        int b1, b2;
        uint16_t s1, s2;
        select_group_top2_bits(gw, uw, b1, b2, s1, s2);
        pos = pack_group_2of8(b1, s1, b2, s2, q);
      }
      // 64-channel tile t = G / 8; G % 8 = 4s + 2h + jj
      const int t = G >> 3, s = (G >> 2) & 1, h = (G >> 1) & 1, jj = G & 1;
      uint32_t w = pos << (16 * s + 8 * jj);
      w |= __shfl_xor(w, 1);
      w |= __shfl_xor(w, 4);
      if (tok < g.M && t < g.gu_nt) {
        *reinterpret_cast<uint2*>(g.gu_ap + static_cast<int64_t>(tok) * g.gu_ld_ap + 4 * G) =
            make_uint2(q[0] | (static_cast<uint32_t>(q[1]) << 16), q[2] | (static_cast<uint32_t>(q[3]) << 16));
        if (s == 0 && jj == 0) g.gu_meta[(static_cast<int64_t>(t) * g.gu_meta_rows + tok) * 2 + h] = w;
      }
    }
    return;
  }
#pragma unroll 2
  for (int item = tid; item < 256 * 16; item += kPpThreads) {
    const int tr = item >> 4, grp8 = item & 15;
    const int tok = row0 + tr, cg = col0 + grp8 * 8;
    if (tok >= g.M || cg >= g.gu_inter) continue;
    const int off = tr * 256 + ((grp8 ^ (tr & 15)) << 4);
    const uint4 gv = *reinterpret_cast<const uint4*>(lds + off);
    const uint4 uv = *reinterpret_cast<const uint4*>(lds + kU + off);
    const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
    const int64_t o = static_cast<int64_t>(tok) * kout + (cg / 8) * 2;
    select_group_emit_bits(gw, uw, cg, g.gu_idx + o, g.gu_sz + o);
  }
}

// SPLIT: split-K launch (f32 partial tiles into the workspace slices).
// GU: MoC 2:8 gate/up launch (see GemmArgs::gu_idx).
// SP: A is 2:4-packed (see GemmArgs::sp_meta) and each 32-channel step of a
// K tile runs on v_smfmac_f32_32x32x32_bf16: half the MFMA instructions and
// half the A bytes of the dense form.  A K tile of A is then 256 rows x 32
// stored values (16 KB, 64-byte rows, chunks swizzled by sp_swz) plus 2 KB of
// positions, both in the A stage; B and everything else are unchanged.  The
// sparse operand is the MFMA's first, so the accumulators come out in the
// MFMA's orientation and leave through store_tile_t.
template <bool A_KC, bool B_KC, bool OUT_F32, bool DUAL, bool SPLIT, bool GU = false, bool SP = false,
          bool SHORT = false>
__global__ __launch_bounds__(kPpThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void gemm_pp_kernel(GemmArgs g) {
  static_assert(!SHORT || (A_KC && !GU && !SP), "128-row tiles: K-contiguous A, plain products");
  // SHORT: 128 x 256 C tiles (the A tile half as tall; wave tiles 64 x 64)
  constexpr int MI = SHORT ? 2 : 4;  // 32-row blocks of a wave's tile
  // K tiles staged as halves in the five-slot LDS ring (kSlots)
  __shared__ __attribute__((aligned(1024))) char lds[kRingBytes];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2;
  const int sw = wave & 3;
  int bid = static_cast<int>(blockIdx.x);
  if constexpr (SPLIT && !DUAL) {
    if (g.grp_wgs > 0 && bid >= g.grp_wgs) {  // the grouped launch's second product
      bid -= g.grp_wgs;
      g.a[0] = g.a[1];
      g.b[0] = g.b[1];
      g.nk[0] = g.grp_nk;
      g.M = g.grp_M;
      g.N = g.grp_N;
      g.tiles_m = g.grp_tiles_m;
      g.tiles_n = g.grp_tiles_n;
      g.ksplit = g.grp_ksplit;
      g.kper = g.grp_kper;
      g.C = g.grp_C;
      g.ldc = g.grp_ldc;
      g.ws_stride = g.grp_ws_stride;
    }
  }
  // split-K: workgroup bid runs K tiles [split * kper, +kper) of its tile
  // and writes an f32 partial tile into slice `split` of the workspace
  const int split = SPLIT ? bid % g.ksplit : 0;
  int tbid = SPLIT ? bid / g.ksplit : bid;
  // tail fix-up: workgroup fix_full + part * fix_tail + slot runs part
  // `part` of the K range of tile fix_full + slot
  int part = -1, slot = 0;
  if (!SPLIT && g.fix_tail > 0 && tbid >= g.fix_full) {
    const int j = tbid - g.fix_full;
    part = j / g.fix_tail;
    slot = j - part * g.fix_tail;
    tbid = g.fix_full + slot;
  }
  int tm, tn;
  tile_coords(tbid, g.tiles_m, g.tiles_n, tm, tn);
  if (!GU && !DUAL && !SPLIT && g.ncat_tn > 0 && tn >= g.ncat_tn) {
    tn -= g.ncat_tn;
    g.b[0] = g.b[1];
    g.C = g.C2;
    g.N = g.N2;
    g.ldc = g.ldc2;
    g.vec_store = g.vec_store2;
  }
  const int row0 = tm * (SHORT ? 128 : kBM);
  const int col0 = GU ? tn * 128 : tn * kBN;  // GU: channel base of the gate and up halves
  const int wm = (sw >> 1) * (SHORT ? 64 : 128);
  const int wn = (sw & 1) * 128 + grp * 64;
  const uint32_t lds0 = lds_addr(lds);

  const int nk0 = g.nk[0];
  const int nk_all = nk0 + (DUAL ? g.nk[1] : 0);
  // first K tile of this workgroup and one past its last
  const int kt0 = SPLIT ? split * g.kper : (part == 1 ? g.fix_split : 0);
  const int nk = SPLIT ? min(nk_all, kt0 + g.kper) : (part == 0 ? g.fix_split : nk_all);

  FragMap<A_KC> fa_map;
  FragMap<B_KC> fb_map;
  // The rows of a KC operand that a wave reads lie in one half of the tile
  // (ha, hb), addressed inside that half's region of a slot; an MN
  // operand's k16 steps 0-1 and 2-3 lie in halves 0 and 1
  constexpr int kHalfRowsA = SHORT ? 64 : 128;
  const int ha = A_KC ? wm / kHalfRowsA : 0;
  const int hb = B_KC ? wn / 128 : 0;
  fa_map.init(0, wm - ha * kHalfRowsA, lane);
  fb_map.init(kSlotB, wn - hb * 128, lane);

  f32x16_t acc[MI][2];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  bf16x8_t fa[4][MI], fb[4][2];  // [k16 step][block]  (SP: fa[32-channel step][block])
  uint32_t fm[4];               // SP: positions of the stored A values, per block
  // SP: a half's A region holds its 128 packed rows (8 KB, kSpAHalf) and
  // then their positions (1 KB).  The lane's A fragment of block 0, step 0
  // (row wm + (lane & 31) of the tile, logical chunk lane >> 5); step s is
  // chunk 2s + (lane >> 5), one XOR away; and its positions word
  const int wr = wm - ha * 128 + (lane & 31);  // row inside the half
  const uint32_t spa_base = static_cast<uint32_t>(wr * 64 + (((lane >> 5) ^ sp_swz(lane & 15)) << 4));
  const uint32_t spm_base = static_cast<uint32_t>(kSpAHalf + wr * 8 + (lane >> 5) * 4);
  // LDS byte of the slot of half h of K tile t.  Halves are requested
  // in the order H1(kt0), H0(kt0), H1(kt0 + 1), H0(kt0 + 1), ... (sequence
  // number 2 (t - kt0) + 1 - h) and take the slots round-robin; the schedule
  // below has each half dead before its slot comes round again.
  auto slot_of = [&](int t, int h) -> uint32_t {
    return static_cast<uint32_t>((2 * (t - kt0) + 1 - h) % kSlots) * kSlotBytes;
  };
  auto read_frags = [&](int t) {
    const uint32_t s0 = slot_of(t, 0), s1 = slot_of(t, 1);
    const uint32_t sa = ha ? s1 : s0, sb = hb ? s1 : s0;
    if constexpr (SP) {
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          fa[s][i] = __builtin_bit_cast(
              bf16x8_t, *reinterpret_cast<const uint4*>(lds + ((spa_base + sa) ^ (32u * s)) + i * 2048));
#pragma unroll
      for (int i = 0; i < 4; ++i) fm[i] = *reinterpret_cast<const uint32_t*>(lds + sa + spm_base + i * 256);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int j = 0; j < 2; ++j) fb[ks][j] = fb_map.read(lds, j, ks, B_KC ? sb : (ks < 2 ? s0 : s1), true);
      return;
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const uint32_t sk = ks < 2 ? s0 : s1;
#pragma unroll
      for (int i = 0; i < MI; ++i) fa[ks][i] = fa_map.read(lds, i, ks, A_KC ? sa : sk, true);
#pragma unroll
      for (int j = 0; j < 2; ++j) fb[ks][j] = fb_map.read(lds, j, ks, B_KC ? sb : sk, true);
    }
  };
  // The 32 MFMAs of a K tile (order pinned); SP: 16 structured-sparse ones,
  // B of a 32-channel step being the two k16 fragments of the dense form
  // (the operand layout of v_smfmac_f32_32x32x32_bf16: lane l's B holds
  // channels 8(l >> 5) .. +8 and 16 + 8(l >> 5) .. +8 of column l & 31).
  auto compute = [&]() {
    if constexpr (SP) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const bf16x16_t b = __builtin_shufflevector(fb[0][j], fb[1][j], 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10,
                                                      11, 12, 13, 14, 15);
          acc[i][j] = __builtin_amdgcn_smfmac_f32_32x32x32_bf16(fa[0][i], b, acc[i][j], fm[i], 0, 0);
          __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const bf16x16_t b = __builtin_shufflevector(fb[2][j], fb[3][j], 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10,
                                                      11, 12, 13, 14, 15);
          acc[i][j] = __builtin_amdgcn_smfmac_f32_32x32x32_bf16(fa[1][i], b, acc[i][j], fm[i], 0, 1);
          __builtin_amdgcn_sched_barrier(0);
        }
    } else {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[ks][j], fa[ks][i], acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
          }
    }
  };

  // Workgroup barrier between phases; the scheduling fences keep the compiler
  // from moving MFMAs or LDS reads across it (they touch registers only, so
  // it otherwise would), which would merge the two phases.
  auto phase_end = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
  };

  LoadMap<A_KC> ma0, ma1;
  LoadMap<B_KC> mb0, mb1;
  ma0.init(g.a[0], row0, sw, lane);
  mb0.init(g.b[0], col0, sw, lane);
  const __amdgpu_buffer_rsrc_t ra0 = make_rsrc(g.a[0]), rb0 = make_rsrc(g.b[0]);
  __amdgpu_buffer_rsrc_t ra1 = ra0, rb1 = rb0;
  if (DUAL) {
    ma1.init(g.a[1], row0, sw, lane);
    mb1.init(g.b[1], col0, sw, lane);
    ra1 = make_rsrc(g.a[1]);
    rb1 = make_rsrc(g.b[1]);
  }
  if (GU) {
    // loads 4-7 fill tile rows 128-255 from the W_up rows col0.. (the
    // offsets of the loads < 4 of this map, never issued, may wrap)
    mb1.init(g.b[1], col0 - 128, sw, lane);
    rb1 = make_rsrc(g.b[1]);
  }
  // SP: the 16 wave loads of a packed A tile (load L fills tile rows
  // 16L .. 16L + 15: lane l row 16L + l/4, slot l % 4; eight per half) and
  // the 2 of its positions (load L covers rows 128L .. 128L + 127, two per
  // lane; one per half).
  const __amdgpu_buffer_rsrc_t rm = SP ? __builtin_amdgcn_make_buffer_rsrc(
                                             const_cast<uint32_t*>(g.sp_meta), (short)0,
                                             g.nk[0] * g.sp_rows * 8, kBufferFlags)
                                       : ra0;
  const uint32_t spa_voff = static_cast<uint32_t>(
      (static_cast<int64_t>(row0 + (lane >> 2)) * g.a[0].ld + 8 * ((lane & 3) ^ sp_swz(lane >> 2))) * 2);
  // Half h of K tile t into its slot (kRingHalfLoads loads per wave: A
  // loads [h JA, h JA + JA) and B loads [4h, 4h + 4); SP: see there), and
  // the K-straddle fix of that half once it has landed (only the last tile
  // of a product can need it; kchunk depends on the lane only, so the
  // product-0 maps serve both products).
  constexpr int JA = SHORT ? kLoads / 4 : kLoads / 2;
  constexpr int kRingHalfLoads = JA + kLoads / 2;
  auto load_half = [&](int t, int h) {
    const uint32_t sl = lds0 + slot_of(t, h);
    if constexpr (SP) {
      // the packed A rows 128h .. +127 (two loads per wave), their positions
      // (one load, wave 2 of the group) and B's k-rows of the half
      const uint32_t kofs = static_cast<uint32_t>(t) * 64u;
      const uint32_t rstride = static_cast<uint32_t>(16 * g.a[0].ld * 2);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int L = 8 * h + 4 * u + sw;
        uint32_t off = spa_voff + kofs + static_cast<uint32_t>(L) * rstride;
        asm volatile("" : "+v"(off));
        dma16(ra0, __builtin_amdgcn_readfirstlane(sl + (4 * u + sw) * 1024), off);
      }
      if (sw == 2) {
        const uint32_t off = static_cast<uint32_t>(
            ((static_cast<int64_t>(t) * g.sp_rows + row0 + 128 * h + 2 * lane) * 8));
        dma16(rm, __builtin_amdgcn_readfirstlane(sl + kSpAHalf), off);
      }
      const uint32_t bb = mb0.tile_base(g.b[0], t * kBK);
#pragma unroll
      for (int jj = 0; jj < kLoads / 2; ++jj) mb0.issue(rb0, g.b[0], bb, sl + kSlotB, sw, 4 * h + jj, 4 * h);
      return;
    }
    const bool p1 = DUAL && t >= nk0;
    const int k0 = (p1 ? t - nk0 : t) * kBK;
    const Operand& oa = p1 ? g.a[1] : g.a[0];
    const Operand& ob = p1 ? g.b[1] : g.b[0];
    const LoadMap<A_KC>& la = p1 ? ma1 : ma0;
    const LoadMap<B_KC>& lb = p1 ? mb1 : mb0;
    const uint32_t ba = la.tile_base(oa, k0);
    // GU: half 1 of the B tile is the W_up rows
    const bool up = GU && h == 1;
    const uint32_t bb = up ? mb1.tile_base(g.b[1], k0) : lb.tile_base(ob, k0);
#pragma unroll
    for (int jj = 0; jj < kLoads / 2; ++jj) {
      if (jj < JA) la.issue(p1 ? ra1 : ra0, oa, ba, sl, sw, h * JA + jj, h * JA);
      if (up) mb1.issue(rb1, g.b[1], bb, sl + kSlotB, sw, 4 * h + jj, 4 * h);
      else lb.issue(p1 ? rb1 : rb0, ob, bb, sl + kSlotB, sw, 4 * h + jj, 4 * h);
    }
  };
  auto fix_half = [&](int t, int h) {
    const bool p1 = DUAL && t >= nk0;
    const Operand& oa = p1 ? g.a[1] : g.a[0];
    const int k0 = (p1 ? t - nk0 : t) * kBK;
    if constexpr (SP) {  // packed A tiles are whole; only a KC B can straddle K
      if (B_KC && k0 + kBK > g.b[0].K && (g.b[0].K & 7) != 0)
        mb0.zero_straddle(lds, g.b[0], k0, slot_of(t, h) + kSlotB, sw, lane, 4 * h, 4 * h + 4, 4 * h);
      return;
    }
    if (k0 + kBK <= oa.K || (oa.K & 7) == 0) return;
    const uint32_t sl = slot_of(t, h);
    if (A_KC) ma0.zero_straddle(lds, oa, k0, sl, sw, lane, h * JA, h * JA + JA, h * JA);
    if (B_KC) mb0.zero_straddle(lds, p1 ? g.b[1] : g.b[0], k0, sl + kSlotB, sw, lane, 4 * h, 4 * h + 4, 4 * h);
  };

  // The loads of a K tile are split between the groups, half 0 from group
  // 0 and half 1 from group 1, each issued at the start of the group's
  // memory phase (issuing a whole tile from one group stalls that group's
  // phase: the address unit accepts a 1 KB load every ~25 cycles, 64 per
  // tile).  In phase 2t group 0 requests H0(t + 1) and waits for it at the
  // end of phase 2t + 1; in phase 2t + 1 group 1 requests H1(t + 2) and
  // waits for H1(t + 1), requested a phase earlier, so neither group waits
  // out a load's latency in the phase that issued it.  Slot reuse: H0(t + 1)
  // takes the slot of H1(t - 1) and H1(t + 2) that of H0(t - 1), both last
  // read in phase 2t - 1.
  if (grp == 0) {
    load_half(kt0, 0);
    load_half(kt0, 1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    fix_half(kt0, 0);
    fix_half(kt0, 1);
    phase_end();
    for (int t = kt0; t < nk; ++t) {
      if (t + 1 < nk) load_half(t + 1, 0);
      read_frags(t);
      phase_end();  // phase 2t -> 2t+1
      compute();
      if (t + 1 < nk) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        fix_half(t + 1, 0);
      }
      phase_end();  // phase 2t+1 -> 2t+2
    }
  } else {
    if (kt0 + 1 < nk) load_half(kt0 + 1, 1);
    phase_end();
    for (int t = kt0; t < nk; ++t) {
      if (t > kt0) compute();
      phase_end();  // phase 2t -> 2t+1
      const bool ahead = t + 2 < nk;
      if (ahead) load_half(t + 2, 1);
      read_frags(t);
      if (t + 1 < nk) {
        // H1(t + 1) has landed once at most the loads just issued are in
        // flight (vector memory loads complete in issue order)
        if (!ahead) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        else if (SP && sw == 2) asm volatile("s_waitcnt vmcnt(7)" ::: "memory");  // + the positions
        else if constexpr (kRingHalfLoads == 8 && !SP) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
        fix_half(t + 1, 1);
      }
      phase_end();  // phase 2t+1 -> 2t+2
    }
    compute();
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  if constexpr (GU) {
    gu28_epilogue(g, lds, acc, row0, col0, wm, wn, tid, lane);
  } else if constexpr (SPLIT) {
    GemmArgs gs = g;
    gs.C = static_cast<float*>(g.C) + split * g.ws_stride;
    if constexpr (SP) store_tile_t<OUT_F32, 2>(gs, lds, acc, row0, col0, wm, wn, wave, lane);
    else store_tile_w<OUT_F32, 2, MI>(gs, lds, acc, row0, col0, wm, wn, wave, lane);
  } else {
    if (part >= 0 && !fix_arrive<MI>(g, acc, slot, part, tid, reinterpret_cast<int*>(lds + kFlagOffset)))
      return;
    if constexpr (SP) store_tile_t<OUT_F32, 2>(g, lds, acc, row0, col0, wm, wn, wave, lane);
    else store_tile_w<OUT_F32, 2, MI>(g, lds, acc, row0, col0, wm, wn, wave, lane);
  }
}

// Sum of the ksplit f32 partial tiles of a split-K GEMM, in split order (the
// result does not depend on timing), converted to the output type.  One
// thread per four consecutive columns of a row.
template <bool OUT_F32>
__device__ __forceinline__ void splitk_reduce_quad(int64_t q, const float* __restrict__ ws, int64_t stride,
                                                   int ksplit, int M, int N, int64_t ldw, void* __restrict__ C,
                                                   int64_t ldc, int vec, const uint16_t* __restrict__ res,
                                                   int64_t ldres) {
  const int qpr = (N + 3) / 4;
  if (q >= static_cast<int64_t>(M) * qpr) return;
  const int row = static_cast<int>(q / qpr), c = static_cast<int>(q % qpr) * 4;
  const float* p = ws + row * ldw + c;
  float4 s = *reinterpret_cast<const float4*>(p);
  for (int i = 1; i < ksplit; ++i) {
    const float4 v = *reinterpret_cast<const float4*>(p + i * stride);
    s.x += v.x;
    s.y += v.y;
    s.z += v.z;
    s.w += v.w;
  }
  float r[4] = {s.x, s.y, s.z, s.w};
  if (!OUT_F32 && res != nullptr) {
    // bf16(bf16(sum) + residual), the rounding of x + bf16 GEMM output
    const uint16_t* rp = res + row * ldres + c;
    for (int e = 0; e < 4; ++e)
      if (c + e < N)
        r[e] = __uint_as_float(pack_bf16x2(r[e], 0.0f) << 16) + __uint_as_float(static_cast<uint32_t>(rp[e]) << 16);
  }
  if (OUT_F32) {
    float* dst = static_cast<float*>(C) + row * ldc + c;
    if (vec && c + 4 <= N) {
      *reinterpret_cast<float4*>(dst) = s;
    } else {
      for (int e = 0; e < 4 && c + e < N; ++e) dst[e] = r[e];
    }
  } else {
    uint16_t* dst = static_cast<uint16_t*>(C) + row * ldc + c;
    if (vec && c + 4 <= N) {
      *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf16x2(r[0], r[1]), pack_bf16x2(r[2], r[3]));
    } else {
      for (int e = 0; e < 4 && c + e < N; ++e)
        dst[e] = static_cast<uint16_t>(pack_bf16x2(r[e], 0.0f) & 0xFFFF);
    }
  }
}

template <bool OUT_F32>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ ws, int64_t stride,
                                                            int ksplit, int M, int N, int64_t ldw,
                                                            void* __restrict__ C, int64_t ldc, int vec,
                                                            const uint16_t* __restrict__ res = nullptr,
                                                            int64_t ldres = 0) {
  splitk_reduce_quad<OUT_F32>(static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x, ws, stride, ksplit, M, N,
                              ldw, C, ldc, vec, res, ldres);
}

// The sums of a grouped split-K launch's two products in one launch:
// workgroups [0, blocks0) reduce the first, the rest the second.
struct ReduceJob {
  const float* ws;
  int64_t stride;
  int ksplit, M, N;
  int64_t ldw;
  void* C;
  int64_t ldc;
  int vec;
};

template <bool OUT_F32>
__global__ __launch_bounds__(256) void splitk_reduce_pair_kernel(ReduceJob j0, ReduceJob j1, int blocks0) {
  const bool second = static_cast<int>(blockIdx.x) >= blocks0;
  const ReduceJob& j = second ? j1 : j0;
  const int64_t q = static_cast<int64_t>(static_cast<int>(blockIdx.x) - (second ? blocks0 : 0)) * 256 + threadIdx.x;
  splitk_reduce_quad<OUT_F32>(q, j.ws, j.stride, j.ksplit, j.M, j.N, j.ldw, j.C, j.ldc, j.vec, nullptr, 0);
}

// ---------------------------------------------------------------------------
// f32 path: 64x64 tile, 256 threads x (4x4) outputs, K step 16, any strides.
// ---------------------------------------------------------------------------
struct GemmArgsF32 {
  int M, N, K1, K2;
  const float* A1;
  const float* B1;
  const float* A2;
  const float* B2;
  int64_t a1m, a1k, b1k, b1n, a2m, a2k, b2k, b2n;
  float* C;
  int64_t ldc;
  // pair (ncat > 0, tiled kernel only): column tiles from ncat on compute
  // Cp = A Bp^T with Bp laid out as B1
  const float* Bp;
  float* Cp;
  int ncat;
};

__global__ __launch_bounds__(256) void gemm_f32_kernel(GemmArgsF32 g) {
  __shared__ float As[16][65];
  __shared__ float Bs[16][65];
  const int tid = threadIdx.x;
  const int tr = tid / 16, tc = tid % 16;
  const int row0 = blockIdx.y * 64, col0 = blockIdx.x * 64;
  float acc[4][4] = {};
  for (int pass = 0; pass < 2; ++pass) {
    const float* A = pass ? g.A2 : g.A1;
    const float* B = pass ? g.B2 : g.B1;
    const int K = pass ? g.K2 : g.K1;
    if (A == nullptr || K == 0) continue;
    const int64_t am = pass ? g.a2m : g.a1m, ak = pass ? g.a2k : g.a1k;
    const int64_t bk = pass ? g.b2k : g.b1k, bn = pass ? g.b2n : g.b1n;
    for (int k0 = 0; k0 < K; k0 += 16) {
      for (int e = tid; e < 16 * 64; e += 256) {
        const int kk = e / 64, mm = e % 64;
        const int gm = row0 + mm, gn = col0 + mm, gk = k0 + kk;
        As[kk][mm] = (gm < g.M && gk < K) ? A[gm * am + gk * ak] : 0.0f;
        Bs[kk][mm] = (gn < g.N && gk < K) ? B[gk * bk + gn * bn] : 0.0f;
      }
      __syncthreads();
#pragma unroll
      for (int kk = 0; kk < 16; ++kk) {
        float a[4], b[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = As[kk][tr * 4 + i];
#pragma unroll
        for (int j = 0; j < 4; ++j) b[j] = Bs[kk][tc * 4 + j];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
      }
      __syncthreads();
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = row0 + tr * 4 + i, c = col0 + tc * 4 + j;
      if (r < g.M && c < g.N) g.C[static_cast<int64_t>(r) * g.ldc + c] = acc[i][j];
    }
}

// f32 tiled path on the fp32 MFMA (v_mfma_f32_32x32x2_f32): 64x64 C tile
// per 512-thread workgroup.  Waves w and w + 4 share the 32x32 block w of
// the tile and split each 32-deep K step between them (two waves per SIMD:
// one's LDS reads and barrier wait overlap the other's MFMAs, which one wave
// per SIMD leaves exposed when the tiles fill each CU once); their sums are
// added through LDS at the end.  Each step's two 8 KB operand tiles come in
// by direct-to-LDS buffer loads (1 KB per wave instruction, 16 per step)
// into four LDS stages, the loads of steps i + 1 .. i + 3 in flight while
// step i multiplies.  Rows beyond the extent and K beyond the product's K
// read as zeros through out-of-range buffer offsets (the dispatch keeps the
// contiguous extent a multiple of 4, so a 16-byte chunk is all in range or
// all out).  MFMA step s (0-7) of wave group g multiplies K values
// 8 g + s (lanes 0-31) and 16 + 8 g + s (lanes 32-63): the order of the K
// sum is the hardware's, so results agree with a scalar loop to f32
// rounding.  The K range (both products concatenated, the first's K a
// multiple of 32) can be split over gridDim.z workgroups: split z adds
// [z kchunk, (z+1) kchunk) and writes its f32 partial tile to ws + z stride,
// summed in split order by splitk_reduce_kernel.  KC: operand contiguous
// along K; else along M (A) or N (B).
//
// LDS of an operand tile (8 rows of 1 KB, one per load instruction):
// KC: tile row r (M or N) at (r / 8) * 1024 + (r % 8) * 128, its 16-byte K
//     chunk c in slot c ^ ((r >> 1) & 7) — the 16-byte reads of one chunk
//     of 16 consecutive rows are free of bank conflicts;
// MN: K row k at (k / 4) * 1056 + (k % 4) * 256, 64 floats of M or N — the
//     32-byte skew per load puts rows k and k + 16, read by the two lane
//     halves of one MFMA step, on different banks.
constexpr int kF32BM = 64, kF32BK = 32, kF32Stages = 4;
constexpr int kF32OpBytes = 8 * 1056;
constexpr int kF32StageBytes = 2 * kF32OpBytes;

template <bool KC>
struct F32Load {
  static constexpr int kPitch = KC ? 1024 : 1056;  // LDS bytes per load instruction
  // byte offset of lane `lane`'s 16 bytes of load j (0-7) of the tile of K
  // step k0 (K the product's), or kOob
  __device__ __forceinline__ static uint32_t offset(int j, int lane, int row0, int ext, int64_t ld, int k0,
                                                    int K) {
    if (KC) {
      const int r = 8 * j + (lane >> 3);
      const int c = (lane & 7) ^ ((r >> 1) & 7);
      const int k = k0 + 4 * c;
      const bool ok = row0 + r < ext && k < K;
      return ok ? static_cast<uint32_t>(((row0 + r) * ld + k) * 4) : kOob;
    }
    const int k = k0 + 4 * j + (lane >> 4);
    const int m = row0 + 4 * (lane & 15);
    const bool ok = k < K && m < ext;
    return ok ? static_cast<uint32_t>((k * ld + m) * 4) : kOob;
  }
  // the lane's operands of the 8 MFMA steps of wave group g: tile row `row`,
  // K values 16 h + 8 g + s (x4[j] holds steps 4j .. 4j + 3)
  __device__ __forceinline__ static void read(const char* tile, int row, int h, int g, float4 (&x4)[2]) {
    if (KC) {
      const char* rp = tile + (row >> 3) * 1024 + (row & 7) * 128;
#pragma unroll
      for (int j = 0; j < 2; ++j)
        x4[j] = *reinterpret_cast<const float4*>(rp + (((4 * h + 2 * g + j) ^ ((row >> 1) & 7)) << 4));
    } else {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int k = 16 * h + 8 * g + 4 * j + e;
          v[e] = *reinterpret_cast<const float*>(tile + (k >> 2) * 1056 + (k & 3) * 256 + row * 4);
        }
        x4[j] = make_float4(v[0], v[1], v[2], v[3]);
      }
    }
  }
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t f32_rsrc(const float* p, int64_t rows, int64_t ld,
                                                           int64_t cols) {
  const int64_t bytes = rows > 0 && cols > 0 ? ((rows - 1) * ld + cols) * 4 : 0;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), (short)0, static_cast<int>(bytes),
                                           kBufferFlags);
}

template <bool A_KC, bool B_KC>
__global__ __launch_bounds__(512) void gemm_f32_tiled_kernel(GemmArgsF32 g, int kchunk, float* ws,
                                                             int64_t ws_stride, int64_t ldw) {
  __shared__ __attribute__((aligned(1024))) char lds[kF32Stages * kF32StageBytes];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int grp = wave >> 2, blk = wave & 3;
  int bx = blockIdx.x;
  if (g.ncat > 0 && bx >= g.ncat) {  // the pair's second product
    bx -= g.ncat;
    g.B1 = g.Bp;
    g.C = g.Cp;
  }
  const int m0 = blockIdx.y * kF32BM, n0 = bx * kF32BM;
  const int bm = (blk >> 1) * 32, bn = (blk & 1) * 32;
  const int ktot = g.K1 + g.K2;
  const int klo = blockIdx.z * kchunk;
  const int khi = min(ktot, klo + kchunk);
  const int nsteps = klo < khi ? (khi - klo + kF32BK - 1) / kF32BK : 0;
  // operand resources: KC rows of K values, else K rows of M (N) values
  const __amdgpu_buffer_rsrc_t ra1 = A_KC ? f32_rsrc(g.A1, g.M, g.a1m, g.K1) : f32_rsrc(g.A1, g.K1, g.a1k, g.M);
  const __amdgpu_buffer_rsrc_t rb1 = B_KC ? f32_rsrc(g.B1, g.N, g.b1n, g.K1) : f32_rsrc(g.B1, g.K1, g.b1k, g.N);
  const __amdgpu_buffer_rsrc_t ra2 = A_KC ? f32_rsrc(g.A2, g.M, g.a2m, g.K2) : f32_rsrc(g.A2, g.K2, g.a2k, g.M);
  const __amdgpu_buffer_rsrc_t rb2 = B_KC ? f32_rsrc(g.B2, g.N, g.b2n, g.K2) : f32_rsrc(g.B2, g.K2, g.b2k, g.N);
  const uint32_t lds0 = lds_addr(lds);
  // the two loads of K step i (this wave's load `wave` of each operand
  // tile) into stage i % 4
  auto issue = [&](int i) {
    const int kk = klo + i * kF32BK;
    const bool p2 = kk >= g.K1;
    const int k0 = p2 ? kk - g.K1 : kk;
    const int K = p2 ? g.K2 : g.K1;
    const __amdgpu_buffer_rsrc_t ra = p2 ? ra2 : ra1, rb = p2 ? rb2 : rb1;
    const int64_t lda = A_KC ? (p2 ? g.a2m : g.a1m) : (p2 ? g.a2k : g.a1k);
    const int64_t ldb = B_KC ? (p2 ? g.b2n : g.b1n) : (p2 ? g.b2k : g.b1k);
    const uint32_t st = lds0 + (i % kF32Stages) * kF32StageBytes;
    dma16(ra, __builtin_amdgcn_readfirstlane(st + wave * F32Load<A_KC>::kPitch),
          F32Load<A_KC>::offset(wave, lane, m0, g.M, lda, k0, K));
    dma16(rb, __builtin_amdgcn_readfirstlane(st + kF32OpBytes + wave * F32Load<B_KC>::kPitch),
          F32Load<B_KC>::offset(wave, lane, n0, g.N, ldb, k0, K));
  };
  // wait until the loads of all but the `newer` most recent steps have landed
  auto wait_steps = [](int newer) {
    if (newer >= 2) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    else if (newer == 1) asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  };
  // two accumulation chains (even and odd MFMAs of a step)
  f32x16_t acc0, acc1;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc0[r] = acc1[r] = 0.0f;
  for (int i = 0; i < kF32Stages - 1 && i < nsteps; ++i) issue(i);
  wait_steps(min(nsteps, kF32Stages - 1) - 1);
  __syncthreads();
  const int h = lane >> 5;
  for (int i = 0; i < nsteps; ++i) {
    const char* st = lds + (i % kF32Stages) * kF32StageBytes;
    float4 a4[2], b4[2];
    F32Load<A_KC>::read(st, bm + (lane & 31), h, grp, a4);
    F32Load<B_KC>::read(st + kF32OpBytes, bn + (lane & 31), h, grp, b4);
    // step i + 3 into the stage step i - 1 used (all its reads ended at the
    // barrier that closed step i - 1)
    if (i + kF32Stages - 1 < nsteps) issue(i + kF32Stages - 1);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a4[j].x, b4[j].x, acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a4[j].y, b4[j].y, acc1, 0, 0, 0);
      acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a4[j].z, b4[j].z, acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a4[j].w, b4[j].w, acc1, 0, 0, 0);
    }
    // step i + 1's loads have landed (those of the steps after it may be in flight)
    wait_steps(min(nsteps - 1, i + kF32Stages - 1) - (i + 1));
    __syncthreads();
  }
  // group 1 hands its sums to group 0 through LDS (stage memory, free after
  // the loop's last barrier): lane-major, 16 KB
  float* red = reinterpret_cast<float*>(lds);
  if (grp == 1) {
#pragma unroll
    for (int r = 0; r < 16; ++r) red[(blk * 16 + r) * 64 + lane] = acc0[r] + acc1[r];
  }
  __syncthreads();
  if (grp == 1) return;
  // lane l holds column l & 31 of the wave's block, rows 8 (r / 4) + 4 (l / 32) + r % 4
  float* dst = ws ? ws + blockIdx.z * ws_stride : g.C;
  const int64_t ld = ws ? ldw : g.ldc;
  const int c = n0 + bn + (lane & 31);
  if (c < g.N) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = m0 + bm + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      if (row < g.M) dst[static_cast<int64_t>(row) * ld + c] = (acc0[r] + acc1[r]) + red[(blk * 16 + r) * 64 + lane];
    }
  }
}

// Split of an f32 GEMM over K.  A CU's MFMA pipes run its workgroups'
// steps one after another whatever their number, so the time of the
// busiest CU is ceil(tiles * splits / CUs) workgroups of ceil(steps /
// splits) K steps; a split adds the reduction of the f32 partials (a
// launch of ~4 us, ~9 K steps).  The split count minimising that wins.
struct F32Split {
  int ksplit, kchunk;
  int64_t ldw, bytes;
};

template <bool A_KC, bool B_KC>
void launch_bf16(const GemmArgs& a, bool out_f32, hipStream_t st, bool short_m = false) {
  const int64_t units = a.fix_tail > 0 ? a.fix_full + 2 * static_cast<int64_t>(a.fix_tail)
                                       : static_cast<int64_t>(a.tiles_m) * a.tiles_n * a.ksplit;
  const dim3 grid(static_cast<unsigned>(units)), block(kThreads);
  const bool dual = a.nk[1] > 0;
  if constexpr (A_KC) {
    if (a.pp && short_m) {  // 128 x 256 tiles, whole or with the two-part fix-up (no split)
      const dim3 pblock(kPpThreads);
      if (out_f32) {
        if (dual) gemm_pp_kernel<A_KC, B_KC, true, true, false, false, false, true><<<grid, pblock, 0, st>>>(a);
        else gemm_pp_kernel<A_KC, B_KC, true, false, false, false, false, true><<<grid, pblock, 0, st>>>(a);
      } else {
        if (dual) gemm_pp_kernel<A_KC, B_KC, false, true, false, false, false, true><<<grid, pblock, 0, st>>>(a);
        else gemm_pp_kernel<A_KC, B_KC, false, false, false, false, false, true><<<grid, pblock, 0, st>>>(a);
      }
      return;
    }
  }
  if (a.pp) {
    const dim3 pblock(kPpThreads);
    if (a.ksplit > 1) {  // partial tiles are f32
      if (dual) gemm_pp_kernel<A_KC, B_KC, true, true, true><<<grid, pblock, 0, st>>>(a);
      else gemm_pp_kernel<A_KC, B_KC, true, false, true><<<grid, pblock, 0, st>>>(a);
    } else if (out_f32) {
      if (dual) gemm_pp_kernel<A_KC, B_KC, true, true, false><<<grid, pblock, 0, st>>>(a);
      else gemm_pp_kernel<A_KC, B_KC, true, false, false><<<grid, pblock, 0, st>>>(a);
    } else {
      if (dual) gemm_pp_kernel<A_KC, B_KC, false, true, false><<<grid, pblock, 0, st>>>(a);
      else gemm_pp_kernel<A_KC, B_KC, false, false, false><<<grid, pblock, 0, st>>>(a);
    }
    return;
  }
  if (out_f32) {
    if (dual) gemm_bf16_kernel<A_KC, B_KC, true, true><<<grid, block, 0, st>>>(a);
    else gemm_bf16_kernel<A_KC, B_KC, true, false><<<grid, block, 0, st>>>(a);
  } else {
    if (dual) gemm_bf16_kernel<A_KC, B_KC, false, true><<<grid, block, 0, st>>>(a);
    else gemm_bf16_kernel<A_KC, B_KC, false, false><<<grid, block, 0, st>>>(a);
  }
}

// Returns +1 for K-contiguous, 0 for MN-contiguous, -1 if neither.
int layout_of(int64_t s_mn, int64_t s_k, int64_t mn, int64_t k) {
  if (s_k == 1 || k <= 1) return 1;
  if (s_mn == 1 || mn <= 1) return 0;
  return -1;
}

// Describe one bf16 operand for the kernel; returns false if it cannot be
// addressed by a 32-bit buffer resource.
bool make_operand(const void* p, int64_t ld, bool kc, int64_t ext, int64_t K, Operand& o) {
  o.p = static_cast<const uint16_t*>(p);
  o.ld = ld;
  o.ext = static_cast<int>(ext);
  o.K = static_cast<int>(K);
  const int64_t rows = kc ? ext : K;
  const int64_t bytes = rows * ld * 2;
  if (bytes >= (1LL << 31) - 1024) return false;
  o.bytes = static_cast<int>(bytes);
  return true;
}


F32Split plan_f32(int64_t M, int64_t N, int64_t K, int64_t K2) {
  constexpr int64_t kReduceSteps = 9;
  F32Split p{1, 0, 0, 0};
  const int64_t ktot = K + K2;
  const int64_t tiles = ((M + kF32BM - 1) / kF32BM) * ((N + kF32BM - 1) / kF32BM);
  const int64_t steps = (ktot + kF32BK - 1) / kF32BK;
  p.kchunk = static_cast<int>(steps * kF32BK);
  const int64_t cus = cu_count();
  if (steps < 4 || tiles <= 0) return p;
  int64_t best = (tiles + cus - 1) / cus * steps, best_per = steps;
  for (int64_t ks = 2; ks <= 16 && 2 * ks <= steps; ++ks) {
    const int64_t per = (steps + ks - 1) / ks;
    const int64_t n = (steps + per - 1) / per;
    const int64_t cost = (tiles * n + cus - 1) / cus * per + kReduceSteps;
    if (cost < best) {
      best = cost;
      best_per = per;
    }
  }
  if (best_per == steps) return p;
  p.kchunk = static_cast<int>(best_per * kF32BK);
  p.ksplit = static_cast<int>((steps + best_per - 1) / best_per);
  p.ldw = (N + 3) / 4 * 4;
  p.bytes = static_cast<int64_t>(p.ksplit) * M * p.ldw * 4;
  return p;
}

// Split-K plan of a bf16 GEMM: a product whose 256x256 tiles fill at most a
// third of the CUs runs each tile as `ksplit` (>= 3) workgroups over
// consecutive ranges of at least 4 K tiles.  ldw: row pitch of the f32
// partials.
struct SplitPlan {
  int ksplit = 1;
  int kper = 0;
  int64_t ldw = 0;
  int64_t bytes = 0;
};

SplitPlan plan_split(int64_t M, int64_t N, int nk) {
  SplitPlan p;
  p.kper = nk;
  const int64_t tiles = ((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN);
  const int cus = cu_count();
  if (tiles <= 0 || 3 * tiles > cus) return p;
  int ks = static_cast<int>(std::min<int64_t>(cus / tiles, nk / 4));
  if (ks < 2) return p;
  const int kper = (nk + ks - 1) / ks;
  ks = (nk + kper - 1) / kper;
  if (ks < 2) return p;
  p.ksplit = ks;
  p.kper = kper;
  p.ldw = (N + 3) & ~3LL;
  p.bytes = kFixCounterBytes + static_cast<int64_t>(ks) * M * p.ldw * 4;  // partials after the counters
  return p;
}

// Fix-up plan of a bf16 GEMM whose n tiles fill more than a third of the
// CUs but not all of them (the weight gradients at the 1b shape: 176 tiles
// on 256 CUs, K = 16384; the 2:8 down projection: 128 tiles).  Each tile
// runs as two workgroups: part 0 over K tiles [0, s) on n CUs, part 1 over
// [s, nk) on the h = CUs - n others, which take w = ceil(n / h) of them in
// turn (w = 1 up to half the CUs).  s balances the two sides,
// s + kFix ~ w (nk - s + kStore), in K-tile times (kUnit of prologue and
// epilogue per workgroup, kFix for reading and adding the other partial,
// kStore for storing one); the plan is kept if it beats whole tiles.
// Launches with more tiles than CUs run whole tiles only: splitting the
// tiles of their last, partial round measured no faster (the half-empty
// last round already runs its K tiles faster, with less contention for L2
// and HBM, and the partial stores of a whole round at once are HBM-bound).
struct FixPlan {
  int full = 0, tail = 0, split = 0;
  int64_t bytes = 0;
};

FixPlan plan_fix_tiles(int64_t tiles, int nk) {
  constexpr int64_t kUnit = 5, kFix = 4, kStore = 3;
  FixPlan f;
  const int64_t cus = cu_count();
  if (tiles <= 0 || 3 * tiles <= cus || tiles >= cus || nk < 8 || tiles * 4 > kFixCounterBytes) return f;
  const int64_t w = (tiles + (cus - tiles) - 1) / (cus - tiles);
  int64_t best = nk + kUnit, best_s = 0;
  for (int64_t r = 4; 2 * r <= nk; ++r) {
    const int64_t s = nk - r;
    const int64_t cost = std::max(s + kUnit + kFix, w * (r + kUnit + kStore));
    if (cost < best) {
      best = cost;
      best_s = s;
    }
  }
  if (best_s == 0) return f;
  f.tail = static_cast<int>(tiles);
  f.split = static_cast<int>(best_s);
  f.bytes = kFixCounterBytes + tiles * 2 * kPartBytes;
  return f;
}

FixPlan plan_fix(int64_t M, int64_t N, int nk) {
  return plan_fix_tiles(((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN), nk);
}

// A product whose 256x256 tiles fill at most a third of the CUs (split-K
// territory) but whose 128-row tiles fill more: the 128-row tiles with the
// two-part fix-up instead, no f32 partial tiles of the whole K range and no
// reduction launch (the fix-up's partials are one per split tile).  Up to
// kShortFixMaxKTiles: a 128-row K tile moves the B tile of a 256-row one for
// half its MFMA work, so over a longer K the K split and its reduction win
// (350m layer: D, 43 K tiles, 39.3 against 33.4 + 11.2 us; dX, 86, 62.4
// against 49.0 + 12.0 us).
constexpr int kShortFixMaxKTiles = 64;
FixPlan plan_fix_short(int64_t M, int64_t N, int nk) {
  const int64_t tiles256 = ((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN);
  if (3 * tiles256 > cu_count() || nk > kShortFixMaxKTiles) return FixPlan();
  return plan_fix_tiles(((M + 127) / 128) * ((N + kBN - 1) / kBN), nk);
}

// Two split-K products in one launch (the layer backward's weight gradients
// at the 130m shape: dW_gu 48 tiles and dWd 24 tiles over K = 8192).  Apart,
// each splits K until its tiles alone fill the CUs (5 and 10 ways: 63 MB of
// f32 partials each, two GEMM and two reduction launches); together they
// share the CUs with fewer splits (3 and 3: 57 MB of partials, one launch
// of each kind).  Costs in K-tile times: kRound per launch (prologue,
// epilogue, turnover), kReduce per reduction launch, and the partials'
// bytes written and read back at kTileBytes per K-tile time.  Kept when it
// beats the two products apart; bytes = 0 otherwise.
struct PairSplitPlan {
  SplitPlan p[2];
  int64_t bytes = 0;  // arrival counters + both products' partials
};

PairSplitPlan plan_split_pair(int64_t M1, int64_t N1, int nk1, int64_t M2, int64_t N2, int nk2) {
  constexpr double kRound = 5.0, kReduce = 1.0, kTileBytes = 8.7e6;
  PairSplitPlan r;
  const SplitPlan sep[2] = {plan_split(M1, N1, nk1), plan_split(M2, N2, nk2)};
  if (sep[0].ksplit < 2 || sep[1].ksplit < 2) return r;
  const int64_t cus = cu_count();
  const int64_t M[2] = {M1, M2};
  const int64_t ldw[2] = {(N1 + 3) & ~3LL, (N2 + 3) & ~3LL};
  const int64_t t[2] = {((M1 + kBM - 1) / kBM) * ((N1 + kBN - 1) / kBN), ((M2 + kBM - 1) / kBM) * ((N2 + kBN - 1) / kBN)};
  const int nk[2] = {nk1, nk2};
  auto part_bytes = [&](int i, int ks) { return static_cast<double>(ks) * M[i] * ldw[i] * 4; };
  double best = 0;
  for (int i = 0; i < 2; ++i) best += kRound + sep[i].kper + kReduce + 2 * part_bytes(i, sep[i].ksplit) / kTileBytes;
  int pick[2] = {0, 0}, per[2] = {0, 0};
  for (int a = 2; a <= std::max(2, nk1 / 4); ++a) {
    for (int b = 2; b <= std::max(2, nk2 / 4); ++b) {
      const int kp[2] = {(nk1 + a - 1) / a, (nk2 + b - 1) / b};
      const int ks[2] = {(nk1 + kp[0] - 1) / kp[0], (nk2 + kp[1] - 1) / kp[1]};
      if (t[0] * ks[0] + t[1] * ks[1] > cus) continue;
      const double cost =
          kRound + std::max(kp[0], kp[1]) + kReduce + 2 * (part_bytes(0, ks[0]) + part_bytes(1, ks[1])) / kTileBytes;
      if (cost < best) {
        best = cost;
        pick[0] = ks[0], pick[1] = ks[1];
        per[0] = kp[0], per[1] = kp[1];
      }
    }
  }
  if (pick[0] == 0) return r;
  r.bytes = kFixCounterBytes;
  for (int i = 0; i < 2; ++i) {
    r.p[i].ksplit = pick[i];
    r.p[i].kper = per[i];
    r.p[i].ldw = ldw[i];
    r.p[i].bytes = static_cast<int64_t>(pick[i]) * M[i] * ldw[i] * 4;
    r.bytes += r.p[i].bytes;
  }
  return r;
}

}  // namespace

// MoC 2:8 gate/up projection + top-2-of-8 on the 512-thread GEMM kernel
// (256 tokens x 128 channels of gate and of up per workgroup).  Returns 1
// without launching when an operand is too large for its 32-bit buffer
// offsets (the caller then uses its own kernel).
int launch_gate_up_2of8(const void* x, int64_t nb, int64_t hidden, const void* wg, const void* wu,
                        int64_t inter, int64_t* idx, uint16_t* sz, hipStream_t st, uint16_t* ap,
                        int64_t ld_ap, uint32_t* meta, int64_t meta_rows) {
  GemmArgs a{};
  const bool ok = make_operand(x, hidden, true, nb, hidden, a.a[0]) &&
                  make_operand(wg, hidden, true, inter, hidden, a.b[0]) &&
                  make_operand(wu, hidden, true, inter, hidden, a.b[1]);
  auto no_wrap = [](const Operand& o) {
    return static_cast<int64_t>(o.bytes) + 512 * o.ld + 4096 < (1LL << 32) && 512 * o.ld < (1LL << 31);
  };
  if (!ok || !no_wrap(a.a[0]) || !no_wrap(a.b[0]) || !no_wrap(a.b[1])) return 1;
  a.a[1] = a.a[0];
  a.nk[0] = static_cast<int>((hidden + kBK - 1) / kBK);
  a.nk[1] = 0;
  a.M = static_cast<int>(nb);
  a.N = static_cast<int>(2 * inter);
  a.tiles_m = static_cast<int>((nb + kBM - 1) / kBM);
  a.tiles_n = static_cast<int>((inter + 127) / 128);
  a.pp = 1;
  a.ksplit = 1;
  a.gu_idx = idx;
  a.gu_sz = sz;
  a.gu_inter = static_cast<int>(inter);
  a.gu_ap = ap;
  a.gu_ld_ap = ld_ap;
  a.gu_meta = meta;
  a.gu_meta_rows = static_cast<int>(meta_rows);
  a.gu_nt = static_cast<int>((inter + kBK - 1) / kBK);
  const dim3 grid(static_cast<unsigned>(static_cast<int64_t>(a.tiles_m) * a.tiles_n));
  gemm_pp_kernel<true, true, false, false, false, true><<<grid, dim3(kPpThreads), 0, st>>>(a);
  return check_launch("gemm_pp_kernel (2:8 gate/up)");
}

template <bool W_KC>
void launch_sparse_down_kernel(const GemmArgs& run, bool split, hipStream_t st) {
  const int64_t units = run.fix_tail > 0 ? run.fix_full + 2 * static_cast<int64_t>(run.fix_tail)
                                         : static_cast<int64_t>(run.tiles_m) * run.tiles_n * run.ksplit;
  const dim3 grid(static_cast<unsigned>(units)), block(kPpThreads);
  if (split) gemm_pp_kernel<true, W_KC, true, false, true, false, true><<<grid, block, 0, st>>>(run);
  else gemm_pp_kernel<true, W_KC, false, false, false, false, true><<<grid, block, 0, st>>>(run);
}

}  // namespace moc

using namespace moc;

extern "C" int64_t moc_gemm_workspace_size(int dtype, int64_t M, int64_t N, int64_t K, int64_t K2) {
  if (M <= 0 || N <= 0 || K < 0 || K2 < 0) return 0;
  if (dtype == MOC_F32) {
    // f32 partial tiles after the counter block the bf16 forms keep zero
    if (K2 > 0 && K % kF32BK != 0) return 0;
    const int64_t b = plan_f32(M, N, K, K2).bytes;
    return b > 0 ? MOC_GEMM_WS_COUNTER_BYTES + b : 0;
  }
  if (dtype != MOC_BF16) return 0;
  const int nk = static_cast<int>((K + kBK - 1) / kBK + (K2 + kBK - 1) / kBK);
  return std::max({plan_split(M, N, nk).bytes, plan_fix(M, N, nk).bytes, plan_fix_short(M, N, nk).bytes});
}

// MoC 2:8 compacted Down on the structured-sparse MFMA:
//   y[nb, hidden] = A[nb, inter] W^T,  A 2:4-packed (ap, meta; see GemmArgs::sp_meta)
// w: W_down [hidden, inter] (w_kc = 1, rows of ldw elements) or W_down^T
// [inter, hidden] (w_kc = 0).  Tiles, split-K and the tail fix-up follow
// moc_gemm_ws (same workspace size as the dense [nb, hidden, inter] GEMM).
extern "C" int64_t moc_sparse28_down_workspace_size(int64_t nb, int64_t inter, int64_t hidden) {
  return moc_gemm_workspace_size(MOC_BF16, nb, hidden, inter, 0);
}

extern "C" int moc_sparse28_down_bf16(const void* ap, int64_t ld_ap, const uint32_t* meta, int64_t meta_rows,
                                      int64_t nb, int64_t inter, const void* w, int64_t ldw, int w_kc,
                                      int64_t hidden, void* y, int64_t ldy, void* workspace,
                                      int64_t workspace_bytes, void* stream) {
  MOC_REQUIRE(nb >= 0 && inter >= 1 && hidden >= 1 && inter < (1LL << 30) && hidden < (1LL << 30) &&
                  nb < (1LL << 30),
              "moc_sparse28_down_bf16: bad shape");
  if (nb == 0) return MOC_OK;
  MOC_REQUIRE(ap && meta && w && y, "moc_sparse28_down_bf16: null pointer");
  const int64_t nt = (inter + kBK - 1) / kBK;
  const int64_t tiles_m = (nb + kBM - 1) / kBM;
  MOC_REQUIRE(ld_ap >= 32 * nt && ld_ap % 8 == 0,
              "moc_sparse28_down_bf16: ld_ap must be a multiple of 8 and >= 32 * ceil(inter / 64)");
  MOC_REQUIRE(meta_rows >= tiles_m * kBM, "moc_sparse28_down_bf16: meta_rows must be >= nb rounded up to 256");
  MOC_REQUIRE(ldw % 8 == 0 && ldw >= (w_kc ? inter : ((hidden + 7) & ~7LL)),
              "moc_sparse28_down_bf16: bad ldw");
  MOC_REQUIRE(ldy >= hidden, "moc_sparse28_down_bf16: ldy < hidden");
  MOC_REQUIRE(aligned16(ap) && aligned16(meta) && aligned16(w),
              "moc_sparse28_down_bf16: operands must be 16-byte aligned");
  MOC_REQUIRE(nt * meta_rows * 8 < (1LL << 31), "moc_sparse28_down_bf16: position array too large");
  GemmArgs a{};
  bool ok = make_operand(ap, ld_ap, true, nb, 32 * nt, a.a[0]) && make_operand(w, ldw, w_kc != 0, hidden, inter, a.b[0]);
  auto no_wrap = [](const Operand& o) {
    return static_cast<int64_t>(o.bytes) + 512 * o.ld + 4096 < (1LL << 32) && 512 * o.ld < (1LL << 31);
  };
  MOC_REQUIRE(ok && no_wrap(a.a[0]) && no_wrap(a.b[0]),
              "moc_sparse28_down_bf16: an operand exceeds 32-bit buffer addressing");
  a.a[1] = a.a[0];
  a.b[1] = a.b[0];
  a.nk[0] = static_cast<int>(nt);
  a.nk[1] = 0;
  a.M = static_cast<int>(nb);
  a.N = static_cast<int>(hidden);
  a.C = y;
  a.ldc = ldy;
  a.vec_store = (reinterpret_cast<uintptr_t>(y) % 16 == 0 && (ldy * 2) % 16 == 0) ? 1 : 0;
  a.tiles_m = static_cast<int>(tiles_m);
  a.tiles_n = static_cast<int>((hidden + kBN - 1) / kBN);
  a.pp = 1;
  a.ksplit = 1;
  a.kper = a.nk[0];
  a.sp_meta = meta;
  a.sp_rows = static_cast<int>(meta_rows);
  const SplitPlan sp = plan_split(nb, hidden, a.nk[0]);
  const bool split = sp.ksplit > 1 && workspace != nullptr && workspace_bytes >= sp.bytes &&
                     reinterpret_cast<uintptr_t>(workspace) % 16 == 0;
  GemmArgs run = a;
  if (split) {
    run.ksplit = sp.ksplit;
    run.kper = sp.kper;
    run.ws_stride = nb * sp.ldw;
    run.C = static_cast<char*>(workspace) + kFixCounterBytes;
    run.ldc = sp.ldw;
    run.vec_store = 1;
  }
  const FixPlan fp = split ? FixPlan() : plan_fix(nb, hidden, a.nk[0]);
  if (fp.tail > 0 && workspace != nullptr && workspace_bytes >= fp.bytes &&
      reinterpret_cast<uintptr_t>(workspace) % 256 == 0) {
    run.fix_full = fp.full;
    run.fix_tail = fp.tail;
    run.fix_split = fp.split;
    run.fix_cnt = static_cast<int*>(workspace);
    run.fix_part = static_cast<char*>(workspace) + kFixCounterBytes;
  }
  hipStream_t st = as_stream(stream);
  if (w_kc) launch_sparse_down_kernel<true>(run, split, st);
  else launch_sparse_down_kernel<false>(run, split, st);
  if (!split) return check_launch("gemm_pp_kernel (2:8 sparse down)");
  const int rc = check_launch("gemm_pp_kernel (2:8 sparse down, split)");
  if (rc != MOC_OK) return rc;
  const int64_t quads = nb * ((hidden + 3) / 4);
  splitk_reduce_kernel<false><<<dim3(static_cast<unsigned>((quads + 255) / 256)), 256, 0, st>>>(
      static_cast<const float*>(run.C), run.ws_stride, sp.ksplit, (int)nb, (int)hidden, sp.ldw, y, ldy,
      a.vec_store);
  return check_launch("splitk_reduce_kernel");
}

// Two products of one A in one launch: C1 = A W1^T, C2 = A W2^T (the gate
// and up projections of the FFN input).  The tile grid is the two products'
// grids side by side (gemm_pp_kernel's ncat_tn), so a pair whose grids each
// end in a partial round of the CUs runs as one launch with fewer partial
// rounds.  Pairs whose tiles do not fill the CUs, or whose operands the
// 512-thread kernel cannot address, run as two moc_gemm_ws calls.
extern "C" int moc_gemm_pair(int64_t M, int64_t K, const void* A, int64_t lda, const void* W1,
                             int64_t ldw1, int64_t N1, void* C1, int64_t ldc1, const void* W2,
                             int64_t ldw2, int64_t N2, void* C2, int64_t ldc2, void* workspace,
                             int64_t workspace_bytes, void* stream) {
  MOC_REQUIRE(M >= 0 && K >= 0 && N1 >= 0 && N2 >= 0, "moc_gemm_pair: negative extent");
  MOC_REQUIRE(M < (1LL << 31) && K < (1LL << 31) && N1 < (1LL << 31) && N2 < (1LL << 31),
              "moc_gemm_pair: extent too large");
  MOC_REQUIRE(ldc1 >= N1 && ldc2 >= N2, "moc_gemm_pair: ldc < N");
  if (M == 0) return MOC_OK;
  const int64_t tm = (M + kBM - 1) / kBM, tn1 = (N1 + kBN - 1) / kBN, tn2 = (N2 + kBN - 1) / kBN;
  GemmArgs a{};
  bool pair = K > 0 && N1 > 0 && N2 > 0 && tm * (tn1 + tn2) >= cu_count() &&
              tm * (tn1 + tn2) < (1LL << 31) && C1 != nullptr && C2 != nullptr && A != nullptr &&
              W1 != nullptr && W2 != nullptr && aligned16(A) && aligned16(W1) && aligned16(W2) &&
              lda % 8 == 0 && ldw1 % 8 == 0 && ldw2 % 8 == 0 && lda >= K && ldw1 >= K && ldw2 >= K;
  if (pair) {
    pair = make_operand(A, lda, true, M, K, a.a[0]) && make_operand(W1, ldw1, true, N1, K, a.b[0]) &&
           make_operand(W2, ldw2, true, N2, K, a.b[1]);
    auto no_wrap = [](const Operand& o) {
      return static_cast<int64_t>(o.bytes) + 512 * o.ld + 4096 < (1LL << 32) && 512 * o.ld < (1LL << 31);
    };
    pair = pair && no_wrap(a.a[0]) && no_wrap(a.b[0]) && no_wrap(a.b[1]);
  }
  if (!pair) {
    int rc = moc_gemm_ws(MOC_BF16, M, N1, K, A, lda, 1, W1, 1, ldw1, 0, nullptr, 0, 0, nullptr, 0, 0,
                         C1, ldc1, MOC_BF16, workspace, workspace_bytes, stream);
    if (rc == MOC_OK)
      rc = moc_gemm_ws(MOC_BF16, M, N2, K, A, lda, 1, W2, 1, ldw2, 0, nullptr, 0, 0, nullptr, 0, 0,
                       C2, ldc2, MOC_BF16, workspace, workspace_bytes, stream);
    return rc;
  }
  a.a[1] = a.a[0];
  a.nk[0] = static_cast<int>((K + kBK - 1) / kBK);
  a.nk[1] = 0;
  a.M = static_cast<int>(M);
  a.N = static_cast<int>(N1);
  a.C = C1;
  a.ldc = ldc1;
  a.vec_store = (reinterpret_cast<uintptr_t>(C1) % 16 == 0 && (ldc1 * 2) % 16 == 0) ? 1 : 0;
  a.tiles_m = static_cast<int>(tm);
  a.tiles_n = static_cast<int>(tn1 + tn2);
  a.pp = 1;
  a.ksplit = 1;
  a.kper = a.nk[0];
  a.ncat_tn = static_cast<int>(tn1);
  a.N2 = static_cast<int>(N2);
  a.C2 = C2;
  a.ldc2 = ldc2;
  a.vec_store2 = (reinterpret_cast<uintptr_t>(C2) % 16 == 0 && (ldc2 * 2) % 16 == 0) ? 1 : 0;
  const dim3 grid(static_cast<unsigned>(tm * (tn1 + tn2)));
  gemm_pp_kernel<true, true, false, false, false><<<grid, dim3(kPpThreads), 0, as_stream(stream)>>>(a);
  return check_launch("gemm_pp_kernel (pair)");
}

extern "C" int moc_gemm(int dtype, int64_t M, int64_t N, int64_t K, const void* A, int64_t a_sm,
                        int64_t a_sk, const void* B, int64_t b_sk, int64_t b_sn, int64_t K2,
                        const void* A2, int64_t a2_sm, int64_t a2_sk, const void* B2,
                        int64_t b2_sk, int64_t b2_sn, void* C, int64_t ldc, int c_dtype,
                        void* stream) {
  return moc_gemm_ws(dtype, M, N, K, A, a_sm, a_sk, B, b_sk, b_sn, K2, A2, a2_sm, a2_sk, B2, b2_sk,
                     b2_sn, C, ldc, c_dtype, nullptr, 0, stream);
}

namespace {

// moc_gemm_ws with an optional bf16 residual R added to a bf16 C (res may be
// null): C = bf16(bf16(A B (+ A2 B2)) + R).
int gemm_ws_impl(int dtype, int64_t M, int64_t N, int64_t K, const void* A, int64_t a_sm, int64_t a_sk,
                 const void* B, int64_t b_sk, int64_t b_sn, int64_t K2, const void* A2, int64_t a2_sm,
                 int64_t a2_sk, const void* B2, int64_t b2_sk, int64_t b2_sn, void* C, int64_t ldc, int c_dtype,
                 void* workspace, int64_t workspace_bytes, void* stream, const void* res, int64_t ldres) {
  MOC_REQUIRE(dtype == MOC_BF16 || dtype == MOC_F32, "moc_gemm: dtype must be bf16 or f32");
  MOC_REQUIRE(res == nullptr || (dtype == MOC_BF16 && c_dtype == MOC_BF16 && aligned16(res) && ldres % 8 == 0 &&
                                 ldres >= N),
              "moc_gemm: a residual needs bf16 operands and output and 16-byte aligned rows (ldres a multiple "
              "of 8, >= N)");
  MOC_REQUIRE(M >= 0 && N >= 0 && K >= 0 && K2 >= 0, "moc_gemm: negative extent");
  MOC_REQUIRE(M < (1LL << 31) && N < (1LL << 31) && K < (1LL << 31) && K2 < (1LL << 31),
              "moc_gemm: extent too large");
  MOC_REQUIRE(ldc >= N, "moc_gemm: ldc < N");
  const bool second = A2 != nullptr && K2 > 0;
  MOC_REQUIRE(!second || B2 != nullptr, "moc_gemm: A2 given without B2");
  if (M == 0 || N == 0) return MOC_OK;
  MOC_REQUIRE(C != nullptr, "moc_gemm: null C");
  MOC_REQUIRE(K == 0 || (A != nullptr && B != nullptr), "moc_gemm: null operand");
  hipStream_t st = as_stream(stream);

  if (dtype == MOC_F32) {
    MOC_REQUIRE(c_dtype == MOC_F32, "moc_gemm: f32 operands need an f32 output");
    GemmArgsF32 a{(int)M, (int)N, (int)K, second ? (int)K2 : 0,
                  (const float*)A, (const float*)B, second ? (const float*)A2 : nullptr,
                  second ? (const float*)B2 : nullptr, a_sm, a_sk, b_sk, b_sn, a2_sm, a2_sk,
                  b2_sk, b2_sn, (float*)C, ldc};
    const dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64));
    MOC_REQUIRE(grid.y <= 65535, "moc_gemm: M too large for the f32 grid");
    // tiled path: each operand contiguous along K or along M/N with 16-byte
    // rows and that extent (K, or M/N) a multiple of 4, both products with
    // the same layouts, the first product's K a multiple of the K step when
    // there is a second
    auto f32_layout = [](const void* p, int64_t s_mn, int64_t s_k, int64_t mn, int64_t k) -> int {
      if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return -1;
      if (s_k == 1 && s_mn % 4 == 0 && k % 4 == 0) return 1;  // KC
      if (s_mn == 1 && s_k % 4 == 0 && mn % 4 == 0) return 0;  // MN
      return -1;
    };
    int la = K > 0 ? f32_layout(A, a_sm, a_sk, M, K) : 1, lb = K > 0 ? f32_layout(B, b_sn, b_sk, N, K) : 1;
    if (second) {
      if (f32_layout(A2, a2_sm, a2_sk, M, K2) != la || f32_layout(B2, b2_sn, b2_sk, N, K2) != lb ||
          K % kF32BK != 0)
        la = -1;
    }
    // and its bytes addressable by 32-bit buffer offsets below kOob
    auto fits = [](int kc, int64_t mn, int64_t s_mn, int64_t s_k, int64_t k) {
      if (mn <= 0 || k <= 0) return true;
      const int64_t bytes = kc ? ((mn - 1) * s_mn + k) * 4 : ((k - 1) * s_k + mn) * 4;
      return bytes < static_cast<int64_t>(kOob) - 16;
    };
    if (la >= 0 && lb >= 0 &&
        !(fits(la, M, a_sm, a_sk, K) && fits(lb, N, b_sn, b_sk, K) &&
          (!second || (fits(la, M, a2_sm, a2_sk, K2) && fits(lb, N, b2_sn, b2_sk, K2)))))
      la = -1;
    if (la < 0 || lb < 0 || K + (second ? K2 : 0) == 0) {
      gemm_f32_kernel<<<grid, 256, 0, st>>>(a);
      return check_launch("gemm_f32_kernel");
    }
    F32Split sp = plan_f32(M, N, K, second ? K2 : 0);
    float* ws = nullptr;
    if (sp.ksplit > 1) {
      if (workspace != nullptr && workspace_bytes >= MOC_GEMM_WS_COUNTER_BYTES + sp.bytes &&
          reinterpret_cast<uintptr_t>(workspace) % 16 == 0) {
        ws = reinterpret_cast<float*>(static_cast<char*>(workspace) + MOC_GEMM_WS_COUNTER_BYTES);
      } else {  // no room for partial tiles: one workgroup per tile
        sp.ksplit = 1;
        sp.kchunk = static_cast<int>((K + (second ? K2 : 0) + kF32BK - 1) / kF32BK * kF32BK);
      }
    }
    const dim3 g3(grid.x, grid.y, static_cast<unsigned>(sp.ksplit));
    const int64_t stride = M * sp.ldw;
#define MOC_F32T(AK, BK)                                                                          \
  gemm_f32_tiled_kernel<AK, BK><<<g3, 512, 0, st>>>(a, sp.kchunk, ws, stride, sp.ldw)
    if (la == 1 && lb == 1) MOC_F32T(true, true);
    else if (la == 1) MOC_F32T(true, false);
    else if (lb == 1) MOC_F32T(false, true);
    else MOC_F32T(false, false);
#undef MOC_F32T
    int rc = check_launch("gemm_f32_tiled_kernel");
    if (rc != MOC_OK || ws == nullptr) return rc;
    const int64_t quads = M * ((N + 3) / 4);
    const int vec = (reinterpret_cast<uintptr_t>(C) % 16 == 0 && ldc % 4 == 0) ? 1 : 0;
    splitk_reduce_kernel<true><<<dim3(static_cast<unsigned>((quads + 255) / 256)), 256, 0, st>>>(
        ws, stride, sp.ksplit, (int)M, (int)N, sp.ldw, C, ldc, vec);
    return check_launch("splitk_reduce_kernel (f32)");
  }

  MOC_REQUIRE(c_dtype == MOC_BF16 || c_dtype == MOC_F32, "moc_gemm: bad output dtype");
  const int la = layout_of(a_sm, a_sk, M, K);
  const int lb = layout_of(b_sn, b_sk, N, K);
  MOC_REQUIRE(la >= 0 && lb >= 0, "moc_gemm: each operand needs a unit stride along M/N or K");
  const int64_t lda = la ? a_sm : a_sk;
  const int64_t ldb = lb ? b_sn : b_sk;
  MOC_REQUIRE(K == 0 || (aligned16(A) && aligned16(B)), "moc_gemm: bf16 operands must be 16-byte aligned");
  MOC_REQUIRE(lda % 8 == 0 && ldb % 8 == 0,
              "moc_gemm: bf16 leading dimensions must be multiples of 8 (lda=%lld ldb=%lld)",
              (long long)lda, (long long)ldb);
  // an operand row must hold its logical extent (rounded to 8 for MN tiles)
  MOC_REQUIRE(lda >= (la ? K : ((M + 7) & ~7LL)) && ldb >= (lb ? K : ((N + 7) & ~7LL)),
              "moc_gemm: leading dimension smaller than the operand extent");
  GemmArgs a{};
  bool ok = make_operand(A, lda, la == 1, M, K, a.a[0]) && make_operand(B, ldb, lb == 1, N, K, a.b[0]);
  a.nk[0] = static_cast<int>((K + kBK - 1) / kBK);
  a.nk[1] = 0;
  if (second) {
    const int la2 = layout_of(a2_sm, a2_sk, M, K2);
    const int lb2 = layout_of(b2_sn, b2_sk, N, K2);
    MOC_REQUIRE(la2 == la && lb2 == lb, "moc_gemm: second product must share the operand layouts");
    const int64_t lda2 = la2 ? a2_sm : a2_sk;
    const int64_t ldb2 = lb2 ? b2_sn : b2_sk;
    MOC_REQUIRE(aligned16(A2) && aligned16(B2), "moc_gemm: bf16 operands must be 16-byte aligned");
    MOC_REQUIRE(lda2 % 8 == 0 && ldb2 % 8 == 0, "moc_gemm: bf16 leading dimensions must be multiples of 8");
    MOC_REQUIRE(lda2 >= (la ? K2 : ((M + 7) & ~7LL)) && ldb2 >= (lb ? K2 : ((N + 7) & ~7LL)),
                "moc_gemm: leading dimension smaller than the operand extent");
    ok = ok && make_operand(A2, lda2, la == 1, M, K2, a.a[1]) &&
         make_operand(B2, ldb2, lb == 1, N, K2, a.b[1]);
    a.nk[1] = static_cast<int>((K2 + kBK - 1) / kBK);
  } else {
    a.a[1] = a.a[0];
    a.b[1] = a.b[0];
  }
  MOC_REQUIRE(ok, "moc_gemm: an operand exceeds 2 GiB (32-bit buffer addressing)");
  a.M = static_cast<int>(M);
  a.N = static_cast<int>(N);
  a.C = C;
  a.ldc = ldc;
  a.res = static_cast<const uint16_t*>(res);
  a.ldres = ldres;
  a.vec_store = (reinterpret_cast<uintptr_t>(C) % 16 == 0 &&
                 (ldc * (c_dtype == MOC_F32 ? 4 : 2)) % 16 == 0) ? 1 : 0;
  a.tiles_m = static_cast<int>((M + kBM - 1) / kBM);
  a.tiles_n = static_cast<int>((N + kBN - 1) / kBN);
  MOC_REQUIRE(static_cast<int64_t>(a.tiles_m) * a.tiles_n < (1LL << 31), "moc_gemm: too many tiles");
  const bool of = c_dtype == MOC_F32;
  // The 512-thread kernel relies on the buffer range check for rows past an
  // operand's extent: every offset it forms must stay below 2^32.
  auto no_wrap = [](const Operand& o) {
    return static_cast<int64_t>(o.bytes) + 512 * o.ld + 4096 < (1LL << 32) && 512 * o.ld < (1LL << 31);
  };
  a.pp = no_wrap(a.a[0]) && no_wrap(a.b[0]) && no_wrap(a.a[1]) && no_wrap(a.b[1]);
  // 128-row tiles when 256 x 256 tiles would fill more than a quarter but at
  // most half of the CUs and K is short (the 130m layer's D: 96 tiles, 32 K
  // tiles): twice the tiles run whole, where 256 x 256 tiles need a two-part
  // K split whose f32 partial tile (256 KB) passes through one CU per tile
  // (45 -> 40 us).  A 128-row tile runs its K tiles at ~0.7 of the 256-row
  // tile's rate per FLOP (half the MFMA work per phase, more than half the
  // fragment reads), so for long K the split wins (the 130m dX, 64 K tiles:
  // 72 us split against 78 us).
  const int64_t cus = cu_count();
  const int64_t tiles256 = static_cast<int64_t>(a.tiles_m) * a.tiles_n;
  const bool short_whole = a.pp && la == 1 && 4 * tiles256 > cus && 2 * tiles256 <= cus &&
                           a.nk[0] + a.nk[1] <= kShortMaxKTiles;
  // 128-row tiles in two K parts instead of a K split (see plan_fix_short)
  const FixPlan sfp = a.pp && la == 1 && !short_whole ? plan_fix_short(M, N, a.nk[0] + a.nk[1]) : FixPlan();
  const bool short_fix = sfp.tail > 0 && workspace != nullptr && workspace_bytes >= sfp.bytes &&
                         reinterpret_cast<uintptr_t>(workspace) % 256 == 0;
  const bool short_m = short_whole || short_fix;
  if (short_m) a.tiles_m = static_cast<int>((M + 127) / 128);
  a.ksplit = 1;
  a.kper = a.nk[0] + a.nk[1];
  a.ws_stride = 0;
  const SplitPlan sp = short_m ? SplitPlan() : plan_split(M, N, a.nk[0] + a.nk[1]);
  const bool split = a.pp && sp.ksplit > 1 && workspace != nullptr && workspace_bytes >= sp.bytes &&
                     reinterpret_cast<uintptr_t>(workspace) % 16 == 0;
  GemmArgs run = a;
  if (split) {
    // partial tiles in f32 go to the workspace; the reduction writes C
    run.ksplit = sp.ksplit;
    run.kper = sp.kper;
    run.ws_stride = M * sp.ldw;
    run.C = static_cast<char*>(workspace) + kFixCounterBytes;
    run.ldc = sp.ldw;
    run.vec_store = 1;
  }
  const FixPlan fp = short_fix ? sfp : (split || short_m) ? FixPlan() : plan_fix(M, N, a.nk[0] + a.nk[1]);
  const bool fix = a.pp && fp.tail > 0 && workspace != nullptr && workspace_bytes >= fp.bytes &&
                   reinterpret_cast<uintptr_t>(workspace) % 256 == 0;
  if (fix) {
    run.fix_full = fp.full;
    run.fix_tail = fp.tail;
    run.fix_split = fp.split;
    run.fix_cnt = static_cast<int*>(workspace);
    run.fix_part = static_cast<char*>(workspace) + kFixCounterBytes;
  }
  const bool of_run = split ? true : of;
  if (la && lb) launch_bf16<true, true>(run, of_run, st, short_m);
  else if (la && !lb) launch_bf16<true, false>(run, of_run, st, short_m);
  else if (!la && lb) launch_bf16<false, true>(run, of_run, st);
  else launch_bf16<false, false>(run, of_run, st);
  if (!split) return check_launch("gemm_bf16_kernel");
  {
    const int rc = check_launch("gemm_bf16_kernel");
    if (rc != MOC_OK) return rc;
    const int64_t quads = M * ((N + 3) / 4);
    const dim3 grid(static_cast<unsigned>((quads + 255) / 256));
    const float* parts = static_cast<const float*>(run.C);
    if (of)
      splitk_reduce_kernel<true><<<grid, 256, 0, st>>>(parts, run.ws_stride, sp.ksplit, (int)M, (int)N, sp.ldw,
                                                       C, ldc, a.vec_store);
    else
      splitk_reduce_kernel<false><<<grid, 256, 0, st>>>(parts, run.ws_stride, sp.ksplit, (int)M, (int)N, sp.ldw,
                                                        C, ldc, a.vec_store, a.res, a.ldres);
    return check_launch("splitk_reduce_kernel");
  }
}

}  // namespace

extern "C" int moc_gemm_ws(int dtype, int64_t M, int64_t N, int64_t K, const void* A, int64_t a_sm,
                           int64_t a_sk, const void* B, int64_t b_sk, int64_t b_sn, int64_t K2,
                           const void* A2, int64_t a2_sm, int64_t a2_sk, const void* B2,
                           int64_t b2_sk, int64_t b2_sn, void* C, int64_t ldc, int c_dtype,
                           void* workspace, int64_t workspace_bytes, void* stream) {
  return gemm_ws_impl(dtype, M, N, K, A, a_sm, a_sk, B, b_sk, b_sn, K2, A2, a2_sm, a2_sk, B2, b2_sk, b2_sn, C,
                      ldc, c_dtype, workspace, workspace_bytes, stream, nullptr, 0);
}

// C = bf16(bf16(A B) + R): moc_gemm_ws for bf16 operands and output with the
// residual R [M, N] (rows ldres apart) added in the epilogue (the decoder
// block's x + Down(z) in one pass).
extern "C" int moc_gemm_residual_bf16(int64_t M, int64_t N, int64_t K, const void* A, int64_t a_sm, int64_t a_sk,
                                      const void* B, int64_t b_sk, int64_t b_sn, void* C, int64_t ldc,
                                      const void* res, int64_t ldres, void* workspace, int64_t workspace_bytes,
                                      void* stream) {
  MOC_REQUIRE(res != nullptr, "moc_gemm_residual_bf16: null residual");
  return gemm_ws_impl(MOC_BF16, M, N, K, A, a_sm, a_sk, B, b_sk, b_sn, 0, nullptr, 0, 0, nullptr, 0, 0, C, ldc,
                      MOC_BF16, workspace, workspace_bytes, stream, res, ldres);
}

namespace moc {

// f32 pair C1 = A W1^T and C2 = A W2^T (W1, W2: [N, K] rows of ldw, C1, C2
// rows of ldc, A [M, K] rows of lda) as one launch of the tiled kernel,
// their column tiles side by side.  Returns 1 without launching when the
// shapes do not suit it (a layout the tiled kernel does not take, or
// products the split plan would cut over K on their own); the caller then
// issues two GEMMs.  Where each product alone runs unsplit, the pair runs
// unsplit too: the same steps per tile, two workgroups sharing a CU where
// one product's tiles would leave CUs idle.
int f32_gemm_pair(int64_t M, int64_t N, int64_t K, const float* A, int64_t lda, const float* W1,
                  const float* W2, int64_t ldw, float* C1, float* C2, int64_t ldc, hipStream_t st) {
  auto al = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  if (M <= 0 || N <= 0 || K <= 0 || M >= (1LL << 31) || N >= (1LL << 30) || K % 4 != 0 || lda % 4 != 0 ||
      ldw % 4 != 0 || !al(A) || !al(W1) || !al(W2) || C1 == nullptr || C2 == nullptr)
    return 1;
  if (((M - 1) * lda + K) * 4 >= static_cast<int64_t>(kOob) - 16 ||
      ((N - 1) * ldw + K) * 4 >= static_cast<int64_t>(kOob) - 16)
    return 1;
  const int64_t tn = (N + kF32BM - 1) / kF32BM, tm = (M + kF32BM - 1) / kF32BM;
  if (tm > 65535 || plan_f32(M, N, K, 0).ksplit != 1) return 1;
  GemmArgsF32 a{(int)M, (int)N, (int)K, 0, A, W1, nullptr, nullptr, lda, 1, 1, ldw, 0, 0, 0, 0, C1, ldc};
  a.Bp = W2;
  a.Cp = C2;
  a.ncat = static_cast<int>(tn);
  const dim3 grid(static_cast<unsigned>(2 * tn), static_cast<unsigned>(tm), 1);
  gemm_f32_tiled_kernel<true, true><<<grid, 512, 0, st>>>(a, static_cast<int>((K + kF32BK - 1) / kF32BK * kF32BK),
                                                          nullptr, 0, 0);
  return check_launch("gemm_f32_tiled_kernel (pair)");
}

namespace {

// One bf16 product of a grouped launch: C [M, N] = A B over K, strides as
// in moc_gemm_ws.  False when the 512-thread split kernel cannot take it.
bool pair_product(int64_t M, int64_t N, int64_t K, const void* A, int64_t a_sm, int64_t a_sk, const void* B,
                  int64_t b_sk, int64_t b_sn, int& la, int& lb, Operand& oa, Operand& ob) {
  if (M <= 0 || N <= 0 || K <= 0 || M >= (1LL << 31) || N >= (1LL << 31) || K >= (1LL << 31)) return false;
  la = layout_of(a_sm, a_sk, M, K);
  lb = layout_of(b_sn, b_sk, N, K);
  if (la < 0 || lb < 0 || !aligned16(A) || !aligned16(B)) return false;
  const int64_t lda = la ? a_sm : a_sk, ldb = lb ? b_sn : b_sk;
  if (lda % 8 != 0 || ldb % 8 != 0 || lda < (la ? K : ((M + 7) & ~7LL)) || ldb < (lb ? K : ((N + 7) & ~7LL)))
    return false;
  if (!make_operand(A, lda, la == 1, M, K, oa) || !make_operand(B, ldb, lb == 1, N, K, ob)) return false;
  auto no_wrap = [](const Operand& o) {
    return static_cast<int64_t>(o.bytes) + 512 * o.ld + 4096 < (1LL << 32) && 512 * o.ld < (1LL << 31);
  };
  return no_wrap(oa) && no_wrap(ob);
}

}  // namespace

int64_t gemm_split_pair_workspace(int64_t M1, int64_t N1, int64_t K1, int64_t M2, int64_t N2, int64_t K2) {
  if (M1 <= 0 || N1 <= 0 || K1 <= 0 || M2 <= 0 || N2 <= 0 || K2 <= 0) return 0;
  return plan_split_pair(M1, N1, static_cast<int>((K1 + kBK - 1) / kBK), M2, N2,
                         static_cast<int>((K2 + kBK - 1) / kBK))
      .bytes;
}

int gemm_split_pair(int64_t M1, int64_t N1, int64_t K1, const void* A1, int64_t a1_sm, int64_t a1_sk,
                    const void* B1, int64_t b1_sk, int64_t b1_sn, void* C1, int64_t ldc1, int64_t M2, int64_t N2,
                    int64_t K2, const void* A2, int64_t a2_sm, int64_t a2_sk, const void* B2, int64_t b2_sk,
                    int64_t b2_sn, void* C2, int64_t ldc2, int c_dtype, void* workspace, int64_t workspace_bytes,
                    hipStream_t st) {
  if (c_dtype != MOC_BF16 && c_dtype != MOC_F32) return 1;
  if (C1 == nullptr || C2 == nullptr || ldc1 < N1 || ldc2 < N2) return 1;
  const int nk1 = static_cast<int>((K1 + kBK - 1) / kBK), nk2 = static_cast<int>((K2 + kBK - 1) / kBK);
  const PairSplitPlan plan = K1 > 0 && K2 > 0 ? plan_split_pair(M1, N1, nk1, M2, N2, nk2) : PairSplitPlan();
  if (plan.bytes == 0 || workspace == nullptr || workspace_bytes < plan.bytes || !aligned16(workspace)) return 1;
  GemmArgs a{};
  int la1, lb1, la2, lb2;
  if (!pair_product(M1, N1, K1, A1, a1_sm, a1_sk, B1, b1_sk, b1_sn, la1, lb1, a.a[0], a.b[0]) ||
      !pair_product(M2, N2, K2, A2, a2_sm, a2_sk, B2, b2_sk, b2_sn, la2, lb2, a.a[1], a.b[1]) || la1 != la2 ||
      lb1 != lb2)
    return 1;
  const SplitPlan& p1 = plan.p[0];
  const SplitPlan& p2 = plan.p[1];
  float* ws1 = reinterpret_cast<float*>(static_cast<char*>(workspace) + kFixCounterBytes);
  float* ws2 = reinterpret_cast<float*>(reinterpret_cast<char*>(ws1) + p1.bytes);
  a.nk[0] = nk1;
  a.nk[1] = 0;
  a.M = static_cast<int>(M1);
  a.N = static_cast<int>(N1);
  a.C = ws1;
  a.ldc = p1.ldw;
  a.tiles_m = static_cast<int>((M1 + kBM - 1) / kBM);
  a.tiles_n = static_cast<int>((N1 + kBN - 1) / kBN);
  a.vec_store = 1;
  a.pp = 1;
  a.ksplit = p1.ksplit;
  a.kper = p1.kper;
  a.ws_stride = M1 * p1.ldw;
  a.grp_wgs = a.tiles_m * a.tiles_n * p1.ksplit;
  a.grp_nk = nk2;
  a.grp_M = static_cast<int>(M2);
  a.grp_N = static_cast<int>(N2);
  a.grp_tiles_m = static_cast<int>((M2 + kBM - 1) / kBM);
  a.grp_tiles_n = static_cast<int>((N2 + kBN - 1) / kBN);
  a.grp_ksplit = p2.ksplit;
  a.grp_kper = p2.kper;
  a.grp_C = ws2;
  a.grp_ldc = p2.ldw;
  a.grp_ws_stride = M2 * p2.ldw;
  const dim3 grid(static_cast<unsigned>(a.grp_wgs + a.grp_tiles_m * a.grp_tiles_n * p2.ksplit)), block(kPpThreads);
  if (la1 && lb1) gemm_pp_kernel<true, true, true, false, true><<<grid, block, 0, st>>>(a);
  else if (la1) gemm_pp_kernel<true, false, true, false, true><<<grid, block, 0, st>>>(a);
  else if (lb1) gemm_pp_kernel<false, true, true, false, true><<<grid, block, 0, st>>>(a);
  else gemm_pp_kernel<false, false, true, false, true><<<grid, block, 0, st>>>(a);
  int rc = check_launch("gemm_pp_kernel (grouped split-K)");
  if (rc != MOC_OK) return rc;
  const int64_t esz = c_dtype == MOC_F32 ? 4 : 2;
  auto vec = [&](const void* c, int64_t ldc) { return aligned16(c) && (ldc * esz) % 16 == 0 ? 1 : 0; };
  const ReduceJob j1{ws1, M1 * p1.ldw, p1.ksplit, static_cast<int>(M1), static_cast<int>(N1), p1.ldw, C1, ldc1,
                     vec(C1, ldc1)};
  const ReduceJob j2{ws2, M2 * p2.ldw, p2.ksplit, static_cast<int>(M2), static_cast<int>(N2), p2.ldw, C2, ldc2,
                     vec(C2, ldc2)};
  const int64_t b1 = (M1 * ((N1 + 3) / 4) + 255) / 256, b2 = (M2 * ((N2 + 3) / 4) + 255) / 256;
  const dim3 rgrid(static_cast<unsigned>(b1 + b2));
  if (c_dtype == MOC_F32) splitk_reduce_pair_kernel<true><<<rgrid, 256, 0, st>>>(j1, j2, static_cast<int>(b1));
  else splitk_reduce_pair_kernel<false><<<rgrid, 256, 0, st>>>(j1, j2, static_cast<int>(b1));
  return check_launch("splitk_reduce_pair_kernel");
}

}  // namespace moc

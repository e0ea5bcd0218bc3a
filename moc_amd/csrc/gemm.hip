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
// Tiling: 256x256 C tile per 256-thread workgroup, four waves of 128x128
// (4x4 blocks of 32x32), K step 64, two LDS stages (128 KB), one barrier per
// K step; the next tile's loads are in flight during the MFMAs.  Workgroup
// ids are remapped so that each XCD (ids are dealt round-robin over the 8
// XCDs) works on a contiguous, M-grouped run of tiles that shares its L2.
//
// f32 operands use a plain FMA kernel (parity path for f32 models).
#include "abi.h"
#include "common.h"

namespace moc {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
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
  __device__ __forceinline__ void prefetch(__amdgpu_buffer_rsrc_t rsrc, const Operand& o, int k0,
                                           int row0, uint32_t sink, int tid) const {
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
  uint32_t base[4];   // KC: one per k16 step; MN: one per 32-wide block

  // region: LDS byte of this operand's stage-0 tile; wofs: the wave's 128-row
  // offset inside the 256-row tile
  __device__ __forceinline__ void init(uint32_t region, int wofs, int lane) {
    if (KC) {
      // rows wofs + 32 blk + (lane & 31): row & 15 = lane & 15
      const uint32_t row = static_cast<uint32_t>(wofs + (lane & 31)) * (kBK * 2);
      const int swz = kc_swz(lane & 15);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        base[ks] = (ks < kBK / 16)
                       ? region + row + static_cast<uint32_t>(((2 * ks + (lane >> 5)) ^ swz) * 16)
                       : 0;
    } else {
      // lane = 16 g + i reads k-row 8(g >> 1) + i/4 (+16 ks) and columns
      // m = blk + 16(g & 1) + 4(i & 3) .. +3 of chunk m/8
      const int i = lane & 15, g = lane >> 4;
      const int r = 8 * (g >> 1) + (i >> 2);
      const int swz = mn_swz(i >> 2);
      const uint32_t b = region + r * 512 + 8 * (i & 1);
#pragma unroll
      for (int bi = 0; bi < 4; ++bi) {
        const int c = (wofs + 32 * bi + 16 * (g & 1) + 4 * (i & 3)) >> 3;
        base[bi] = b + 16 * (c ^ swz);
      }
    }
  }

  // so: byte offset of the stage's tile
  __device__ __forceinline__ bf16x8_t read(const char* lds, int blk, int ks, uint32_t so) const {
    if (KC) {
      const char* p = lds + (base[ks] + so) + blk * (32 * kBK * 2);
      return __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(p));
    } else {
      const char* p = lds + (base[blk] + so) + ks * 8192;
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

template <bool OUT_F32>
__device__ __forceinline__ void store_tile(const GemmArgs& g, char* lds, const f32x16_t (&acc)[4][4],
                                           int row0, int col0, int wm, int wn, int wave, int lane) {
  constexpr int kEsz = OUT_F32 ? 4 : 2;
  // row pitch: 16-byte aligned, +16 bytes so that rows r and r + 1 start on
  // different banks
  constexpr int kPitch = 128 * kEsz + 16;
  char* reg = lds + wave * (32 * kPitch);
  const bool vec = g.vec_store != 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    char* rowp = reg + (lane & 31) * kPitch;
#pragma unroll
    for (int j = 0; j < 4; ++j)
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
    // read back: 16-byte segments, 16 per row (bf16: 8 per row)
    constexpr int kSegs = 128 * kEsz / 16;          // per row
    constexpr int kIters = 32 * kSegs / 64;
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      const int e = it * 64 + lane;
      const int row = e / kSegs, seg = e % kSegs;
      const uint4 v = *reinterpret_cast<const uint4*>(reg + row * kPitch + seg * 16);
      const int grow = row0 + wm + 32 * i + row;
      const int gcol = col0 + wn + seg * (16 / kEsz);
      if (grow >= g.M || gcol >= g.N) continue;
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
  store_tile<OUT_F32>(g, lds, acc, row0, col0, wm, wn, wave, lane);
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

template <bool A_KC, bool B_KC>
void launch_bf16(const GemmArgs& a, bool out_f32, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(a.tiles_m * a.tiles_n)), block(kThreads);
  const bool dual = a.nk[1] > 0;
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

}  // namespace
}  // namespace moc

using namespace moc;

extern "C" int moc_gemm(int dtype, int64_t M, int64_t N, int64_t K, const void* A, int64_t a_sm,
                        int64_t a_sk, const void* B, int64_t b_sk, int64_t b_sn, int64_t K2,
                        const void* A2, int64_t a2_sm, int64_t a2_sk, const void* B2,
                        int64_t b2_sk, int64_t b2_sn, void* C, int64_t ldc, int c_dtype,
                        void* stream) {
  MOC_REQUIRE(dtype == MOC_BF16 || dtype == MOC_F32, "moc_gemm: dtype must be bf16 or f32");
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
    gemm_f32_kernel<<<grid, 256, 0, st>>>(a);
    return check_launch("gemm_f32_kernel");
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
  a.vec_store = (reinterpret_cast<uintptr_t>(C) % 16 == 0 &&
                 (ldc * (c_dtype == MOC_F32 ? 4 : 2)) % 16 == 0) ? 1 : 0;
  a.tiles_m = static_cast<int>((M + kBM - 1) / kBM);
  a.tiles_n = static_cast<int>((N + kBN - 1) / kBN);
  MOC_REQUIRE(static_cast<int64_t>(a.tiles_m) * a.tiles_n < (1LL << 31), "moc_gemm: too many tiles");
  const bool of = c_dtype == MOC_F32;
  if (la && lb) launch_bf16<true, true>(a, of, st);
  else if (la && !lb) launch_bf16<true, false>(a, of, st);
  else if (!la && lb) launch_bf16<false, true>(a, of, st);
  else launch_bf16<false, false>(a, of, st);
  return check_launch("gemm_bf16_kernel");
}

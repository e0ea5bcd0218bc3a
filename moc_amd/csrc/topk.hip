// Row-wise channel selection for the MoC FFN on gfx950.
//
//  * moc_topk_rows   - global Top-K over each row of gate logits G.  Replaces
//    torch.topk(g, k, sorted=False) on the training path (moc/ffn.py:144,392)
//    and the CUB block-radix-sort kernels of the decode path
//    (moc/inference/cuda/optimized_global_moc_ext.cu:39-125).
//  * moc_select_2of8 - structured top-2 of every aligned 8-channel group
//    (moc/ffn.py:62-108).
//
// Selection rule (both): order by value descending, ties broken toward the
// lower channel index; -0.0 equals +0.0; NaN ranks above +inf.  Top-K writes
// the selected channels in ascending channel order (the reference leaves the
// order unspecified, sorted=False), so row r of idx is strictly increasing.
//
// Top-K algorithm: one wave per row (up to four rows per workgroup, no
// workgroup barrier).  The row's order keys are staged in the wave's LDS
// (16-byte loads).  An MSB-first radix *select* with 4-bit digits over
// lane-private histograms (4 passes over the keys for bf16 scores, 8 for f32;
// select.h) finds the exact threshold key T and the number r of T-valued
// channels still to take.  One walk over the row in chunks of 64 channels
// then ranks the selected channels by ballots (the r lowest-index T-valued
// channels are taken) and writes them in channel order, with the bit mask
// words straight from the chunk ballots.
#include <algorithm>
#include <type_traits>

#include "abi.h"
#include "common.h"
#include "select.h"

namespace moc {
namespace {

constexpr int kTopkThreads = 256;
constexpr int kMaxTopkInter = 16384;
// Histogram copies: 4 keeps a row's LDS small enough for three workgroups
// per CU, which beats the cheaper atomics of more copies here.
constexpr int kTopkCopies = 4;

// Order key of a raw score (bf16 or f32 bits); transform 1 ranks by
// |SiLU(g)| rounded to the score dtype (moc/ffn.py:335).
template <bool BF16>
__device__ __forceinline__ uint32_t score_key(uint32_t raw, int transform) {
  if (BF16) {
    uint16_t b = static_cast<uint16_t>(raw);
    if (transform == 1) b = f32_to_bf16(fabsf(silu_f32(bf16_to_f32(b))));
    return bf16_order_key(b);
  } else {
    uint32_t u = raw;
    if (transform == 1) u = __float_as_uint(fabsf(silu_f32(__uint_as_float(u))));
    return f32_order_key(u);
  }
}

template <bool BF16>
__device__ __forceinline__ uint32_t load_key(const void* base, int64_t i, int transform) {
  const uint32_t raw = BF16 ? static_cast<uint32_t>(static_cast<const uint16_t*>(base)[i])
                            : static_cast<const uint32_t*>(base)[i];
  return score_key<BF16>(raw, transform);
}

// Row-group shape: NW waves select one row; a workgroup holds RPW groups.
template <int NW>
constexpr int topk_rows_per_wg() {
  return NW == 1 ? 4 : 1;
}

// Thread t of a row group holds channels [t L, t L + L) (select.h).  Per
// group LDS: first the staged row, then, in the same space, the select's
// histograms, the row's mask words (mask output only; assembled with LDS OR
// and stored coalesced) and the list of the k selected channel ids in rank
// order (stored coalesced).
template <bool BF16, int NW, int L>
__global__ __launch_bounds__(kTopkThreads) void topk_rows_kernel(
    const void* __restrict__ scores, int64_t ld, int64_t rows, int inter, int k, int transform,
    int vec, int group_dwords, void* __restrict__ vals, void* __restrict__ idx, int idx_dtype,
    uint32_t* __restrict__ mask, int64_t mask_ld) {
  constexpr int ESZ = BF16 ? 2 : 4;
  constexpr int GT = 64 * NW;  // threads per row group
  constexpr int D = (L + 31) / 32;
  extern __shared__ __attribute__((aligned(16))) uint32_t lds_dyn[];
  const int grp = threadIdx.x / GT, t = threadIdx.x % GT;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * topk_rows_per_wg<NW>() + grp;
  if (row >= rows) return;  // whole row groups only; NW > 1 has one group per workgroup
  uint32_t* lds = lds_dyn + grp * group_dwords;
  const char* src = static_cast<const char*>(scores) + row * ld * ESZ;
  const int c0 = t * L;
  const int mwords = (inter + 31) / 32;
  const int mask_dwords = mask != nullptr ? (mwords + 3) / 4 * 4 : 0;

  // 1. order keys of this thread's channels (coalesced through LDS)
  uint32_t w[sel_words<BF16, L>()];
  load_row_raw_staged<NW, BF16, L>(src, inter, t, vec != 0, lds, w);
  raw_to_keys<BF16, L>(inter, c0, transform, [](uint32_t r) { return score_key<BF16>(r, 1); }, w);

  // 2. threshold and the selected channels of this thread
  uint32_t thr, krem, take[D], first;
  select_threshold<NW, kTopkCopies, sel_words<BF16, L>(), BF16 ? 16 : 32>(w, static_cast<uint32_t>(k), lds,
                                                             thr, krem);
  select_ranks<NW, kTopkCopies, L, BF16>(w, thr, krem, lds, take, first);

  // 3. selected channels in channel order: ids into the group's LDS list
  //    (rank order), then out to HBM coalesced, with values and the index
  //    type conversion
  uint16_t* list = reinterpret_cast<uint16_t*>(lds + select_lds_dwords<NW, kTopkCopies>() + mask_dwords);
  select_emit<L>(take, c0, first, [&](int c, uint32_t pos) { list[pos] = static_cast<uint16_t>(c); });
  if constexpr (NW > 1) __syncthreads(); else __builtin_amdgcn_wave_barrier();
  using KT = typename std::conditional<BF16, uint16_t, uint32_t>::type;
  const KT* raw = reinterpret_cast<const KT*>(src);
  auto copy_out = [&](auto* idx_row) {
    using IT = typename std::remove_pointer<decltype(idx_row)>::type;
    for (int e = t; e < k; e += GT) idx_row[e] = static_cast<IT>(list[e]);
  };
  if (idx_dtype == MOC_I16) copy_out(static_cast<int16_t*>(idx) + row * k);
  else if (idx_dtype == MOC_I32) copy_out(static_cast<int32_t*>(idx) + row * k);
  else copy_out(static_cast<int64_t*>(idx) + row * k);
  if (vals != nullptr) {
    KT* vals_row = static_cast<KT*>(vals) + row * k;
    for (int e = t; e < k; e += GT) vals_row[e] = raw[list[e]];
  }

  // 4. optional bit mask
  if (mask != nullptr) {
    uint32_t* mw = lds + select_lds_dwords<NW, kTopkCopies>();
    for (int i = t; i < mwords; i += GT) mw[i] = 0;
    if constexpr (NW > 1) __syncthreads(); else __builtin_amdgcn_wave_barrier();
    const int sh = c0 & 31;
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const uint32_t bits = take[d];
      if (bits != 0u) {
        const int word = (c0 + 32 * d) >> 5;
        atomicOr(&mw[word], bits << sh);
        if (sh != 0 && (bits >> (32 - sh)) != 0u) atomicOr(&mw[word + 1], bits >> (32 - sh));
      }
    }
    if constexpr (NW > 1) __syncthreads(); else __builtin_amdgcn_wave_barrier();
    uint32_t* mask_row = mask + row * mask_ld;
    for (int i = t; i < mwords; i += GT) mask_row[i] = mw[i];
  }
}

template <bool BF16, int NW, int L>
int launch_topk_kernel(const void* scores, int64_t rows, int inter, int64_t ld, int k,
                       int transform, void* vals, void* idx, int idx_dtype, uint32_t* mask,
                       int64_t mask_ld, hipStream_t st) {
  constexpr int esz = BF16 ? 2 : 4;
  constexpr int rpw = topk_rows_per_wg<NW>();
  const int mwords = (inter + 31) / 32;
  const int sel_dwords = select_lds_dwords<NW, kTopkCopies>() + (mask != nullptr ? (mwords + 3) / 4 * 4 : 0) +
                         (k + 1) / 2;
  const int stage_dwords = 64 * NW * L * esz / 4;
  const int group_dwords = (std::max(sel_dwords, stage_dwords) + 3) / 4 * 4;
  const size_t lds = static_cast<size_t>(group_dwords) * 4 * rpw;
  const int vec = (reinterpret_cast<uintptr_t>(scores) % 16 == 0 && (ld * esz) % 16 == 0) ? 1 : 0;
  const dim3 grid(static_cast<unsigned>((rows + rpw - 1) / rpw)), block(64 * NW * rpw);
  topk_rows_kernel<BF16, NW, L><<<grid, block, lds, st>>>(scores, ld, rows, inter, k, transform, vec,
                                                          group_dwords, vals, idx, idx_dtype, mask,
                                                          mask_ld);
  return check_launch("topk_rows_kernel");
}

// One wave per row while a thread's share fits 128 (f32) or 256 (bf16)
// channels in registers; wider f32 rows, f32 rows of more than 960 channels
// when there are fewer rows than SIMDs, and bf16 rows of 961-4032 channels
// use two waves per row, bf16 rows of 4033-8192 channels four (each row's
// dependent chain shortens; four waves on the 130m and 350m rows of 2048
// and 2736 measured slower than two).
template <bool BF16>
int launch_topk(const void* scores, int64_t rows, int inter, int64_t ld, int k, int transform,
                void* vals, void* idx, int idx_dtype, uint32_t* mask, int64_t mask_ld,
                hipStream_t st) {
#define MOC_TOPK(NW, L) \
  return launch_topk_kernel<BF16, NW, L>(scores, rows, inter, ld, k, transform, vals, idx, idx_dtype, mask, mask_ld, st)
#define MOC_TOPK_L8(NW, per)                                             \
  switch ((per + 7) / 8) {                                               \
    case 1: MOC_TOPK(NW, 8);   case 2: MOC_TOPK(NW, 16);                 \
    case 3: MOC_TOPK(NW, 24);  case 4: MOC_TOPK(NW, 32);                 \
    case 5: MOC_TOPK(NW, 40);  case 6: MOC_TOPK(NW, 48);                 \
    case 7: MOC_TOPK(NW, 56);  case 8: MOC_TOPK(NW, 64);                 \
    case 9: MOC_TOPK(NW, 72);  case 10: MOC_TOPK(NW, 80);                \
    case 11: MOC_TOPK(NW, 88); case 12: MOC_TOPK(NW, 96);                \
    case 13: MOC_TOPK(NW, 104); case 14: MOC_TOPK(NW, 112);              \
    case 15: MOC_TOPK(NW, 120); default: MOC_TOPK(NW, 128);              \
  }
  const int per1 = (inter + 63) / 64;
  if constexpr (!BF16) {
    // few rows (under one row-wave per SIMD): two waves per row halve each
    // row's dependent chain (same selection)
    if (rows < 4LL * cu_count() && per1 >= 16) {
      const int per2 = (inter + 127) / 128;
      MOC_TOPK_L8(2, per2);
    }
  }
  if constexpr (BF16) {
    if (per1 >= 64 && per1 <= 128) {
      const int per4 = (inter + 255) / 256;
      MOC_TOPK_L8(4, per4);
    }
    if (per1 >= 16 && per1 <= 128) {
      const int per2 = (inter + 127) / 128;
      MOC_TOPK_L8(2, per2);
    }
  }
  if (per1 <= 128) {
    MOC_TOPK_L8(1, per1);
  }
  if constexpr (BF16) {
    if (per1 <= 160) MOC_TOPK(1, 160);
    if (per1 <= 192) MOC_TOPK(1, 192);
    if (per1 <= 224) MOC_TOPK(1, 224);
    MOC_TOPK(1, 256);
  } else {
    const int per2 = (inter + 127) / 128;
    MOC_TOPK_L8(2, per2);
  }
#undef MOC_TOPK_L8
#undef MOC_TOPK
}

// ---------------------------------------------------------------------------
// 2:8 structured selection: one thread per (row, group of 8 channels).  The
// trailing partial group of `tail` channels keeps top-min(2, tail).
// Output per group: (top-1, top-2), top-1 = max with lowest index among equal
// maxima, top-2 = max of the remaining seven with the same rule.
// ---------------------------------------------------------------------------
template <bool BF16, typename IdxT>
__global__ __launch_bounds__(256) void select_2of8_kernel(
    const void* __restrict__ scores, int64_t rows, int64_t ld, int inter, int kout,
    void* __restrict__ vals, IdxT* __restrict__ idx) {
  const int groups = (inter + 7) / 8;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= rows * groups) return;
  const int64_t row = gid / groups;
  const int g = static_cast<int>(gid - row * groups);
  const int c0 = g * 8;
  const int cn = min(8, inter - c0);
  const size_t esz = BF16 ? 2 : 4;
  const char* src = static_cast<const char*>(scores) + (row * ld + c0) * esz;
  uint32_t key[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) key[j] = (j < cn) ? load_key<BF16>(src, j, 0) : 0u;
  int b1 = 0;
#pragma unroll
  for (int j = 1; j < 8; ++j)
    if (j < cn && key[j] > key[b1]) b1 = j;
  int b2 = (b1 == 0) ? 1 : 0;
#pragma unroll
  for (int j = 0; j < 8; ++j)
    if (j < cn && j != b1 && key[j] > key[b2]) b2 = j;
  const int64_t o = row * kout + 2 * g;
  const int take = min(2, cn);
  idx[o] = static_cast<IdxT>(c0 + b1);
  if (take > 1) idx[o + 1] = static_cast<IdxT>(c0 + b2);
  if (vals != nullptr) {
    if (BF16) {
      const uint16_t* s = reinterpret_cast<const uint16_t*>(src);
      static_cast<uint16_t*>(vals)[o] = s[b1];
      if (take > 1) static_cast<uint16_t*>(vals)[o + 1] = s[b2];
    } else {
      const uint32_t* s = reinterpret_cast<const uint32_t*>(src);
      static_cast<uint32_t*>(vals)[o] = s[b1];
      if (take > 1) static_cast<uint32_t*>(vals)[o + 1] = s[b2];
    }
  }
}

// ---------------------------------------------------------------------------
// Bit mask -> channel indices: row r's set bits in ascending channel order,
// the first k of them (a mask from moc_topk_rows has exactly k).  One
// workgroup of 256 threads per row; thread t owns the W consecutive mask
// words [t W, t W + W), counts their bits, and a block scan gives the
// thread's first output slot.  Slots a short row leaves empty get channel 0
// (always in range).
// ---------------------------------------------------------------------------
template <typename IdxT>
__global__ __launch_bounds__(256) void mask_to_idx_kernel(const uint32_t* __restrict__ mask, int words,
                                                          int64_t ldw, int k, int W,
                                                          IdxT* __restrict__ idx) {
  __shared__ uint32_t tot_w[4];
  __shared__ uint32_t total;
  const int64_t r = blockIdx.x;
  const uint32_t* m = mask + r * ldw;
  IdxT* out = idx + r * static_cast<int64_t>(k);
  const int w0 = static_cast<int>(threadIdx.x) * W;
  uint32_t cnt = 0;
  for (int i = 0; i < W; ++i)
    if (w0 + i < words) cnt += __popc(m[w0 + i]);
  uint32_t t;
  uint32_t pos = block_exclusive_scan(cnt, tot_w, &t);
  for (int i = 0; i < W; ++i) {
    if (w0 + i >= words) break;
    uint32_t bits = m[w0 + i];
    while (bits) {
      const int b = __ffs(bits) - 1;
      if (pos < static_cast<uint32_t>(k)) out[pos] = static_cast<IdxT>(32 * (w0 + i) + b);
      ++pos;
      bits &= bits - 1u;
    }
  }
  for (uint32_t j = t + threadIdx.x; j < static_cast<uint32_t>(k); j += 256) out[j] = static_cast<IdxT>(0);
  (void)total;
}

}  // namespace
}  // namespace moc

using namespace moc;

extern "C" int moc_mask_to_idx(const void* mask, int64_t rows, int64_t inter, int64_t ld_words,
                               int64_t k, void* idx, int idx_dtype, void* stream) {
  MOC_REQUIRE(rows >= 0 && inter >= 1 && k >= 1 && k <= inter && inter < (1LL << 30),
              "moc_mask_to_idx: bad shape");
  const int64_t words = (inter + 31) / 32;
  MOC_REQUIRE(ld_words >= words, "moc_mask_to_idx: ld_words < ceil(inter / 32)");
  MOC_REQUIRE(idx_dtype == MOC_I16 || idx_dtype == MOC_I32 || idx_dtype == MOC_I64,
              "moc_mask_to_idx: bad index dtype");
  MOC_REQUIRE(idx_dtype != MOC_I16 || inter - 1 <= 32767,
              "topk_idx range [0, %lld] cannot be stored as torch.int16", (long long)(inter - 1));
  MOC_REQUIRE(rows < (1LL << 31), "moc_mask_to_idx: too many rows");
  if (rows == 0) return MOC_OK;
  MOC_REQUIRE(mask && idx, "moc_mask_to_idx: null pointer");
  const int W = static_cast<int>((words + 255) / 256);
  const dim3 grid(static_cast<unsigned>(rows)), block(256);
  hipStream_t st = as_stream(stream);
  const uint32_t* m = static_cast<const uint32_t*>(mask);
  if (idx_dtype == MOC_I16)
    mask_to_idx_kernel<int16_t><<<grid, block, 0, st>>>(m, (int)words, ld_words, (int)k, W, (int16_t*)idx);
  else if (idx_dtype == MOC_I32)
    mask_to_idx_kernel<int32_t><<<grid, block, 0, st>>>(m, (int)words, ld_words, (int)k, W, (int32_t*)idx);
  else
    mask_to_idx_kernel<int64_t><<<grid, block, 0, st>>>(m, (int)words, ld_words, (int)k, W, (int64_t*)idx);
  return check_launch("mask_to_idx_kernel");
}

extern "C" int moc_topk_rows(int dtype, const void* scores, int64_t rows, int64_t inter,
                             int64_t ld, int64_t k, int score_transform, void* vals_out,
                             void* idx_out, int idx_dtype, uint32_t* mask_out, int64_t mask_ld,
                             void* stream) {
  MOC_REQUIRE(dtype == MOC_BF16 || dtype == MOC_F32, "moc_topk_rows: scores must be bf16 or f32");
  MOC_REQUIRE(rows >= 0, "moc_topk_rows: rows must be >= 0");
  MOC_REQUIRE(inter >= 1 && inter <= kMaxTopkInter,
              "moc_topk_rows: intermediate size %lld outside [1, %d]", (long long)inter, kMaxTopkInter);
  MOC_REQUIRE(k >= 1 && k <= inter, "invalid k: k=%lld must be in [1, %lld]", (long long)k,
              (long long)inter);
  MOC_REQUIRE(ld >= inter, "moc_topk_rows: ld (%lld) < intermediate size (%lld)", (long long)ld,
              (long long)inter);
  MOC_REQUIRE(idx_dtype == MOC_I16 || idx_dtype == MOC_I32 || idx_dtype == MOC_I64,
              "moc_topk_rows: bad index dtype");
  MOC_REQUIRE(idx_dtype != MOC_I16 || inter - 1 <= 32767,
              "topk_idx range [0, %lld] cannot be stored as torch.int16", (long long)(inter - 1));
  MOC_REQUIRE(score_transform == 0 || score_transform == 1, "moc_topk_rows: bad score transform");
  MOC_REQUIRE(mask_out == nullptr || mask_ld >= (inter + 31) / 32, "moc_topk_rows: mask_ld too small");
  MOC_REQUIRE(rows == 0 || (scores != nullptr && idx_out != nullptr), "moc_topk_rows: null pointer");
  if (rows == 0) return MOC_OK;
  hipStream_t st = as_stream(stream);
  if (dtype == MOC_BF16)
    return launch_topk<true>(scores, rows, (int)inter, ld, (int)k, score_transform, vals_out,
                             idx_out, idx_dtype, mask_out, mask_ld, st);
  return launch_topk<false>(scores, rows, (int)inter, ld, (int)k, score_transform, vals_out,
                            idx_out, idx_dtype, mask_out, mask_ld, st);
}

extern "C" int64_t moc_moc28_effective_k(int64_t inter) {
  if (inter < 0) return -1;
  const int64_t full = inter / 8, tail = inter % 8;
  return full * 2 + (tail < 2 ? tail : 2);
}

extern "C" int moc_select_2of8(int dtype, const void* scores, int64_t rows, int64_t inter,
                               int64_t ld, void* vals_out, void* idx_out, int idx_dtype,
                               void* stream) {
  MOC_REQUIRE(dtype == MOC_BF16 || dtype == MOC_F32, "moc_select_2of8: scores must be bf16 or f32");
  MOC_REQUIRE(rows >= 0 && inter >= 1, "moc_select_2of8: bad shape");
  MOC_REQUIRE(inter <= (int64_t)1 << 30, "moc_select_2of8: intermediate size too large");
  MOC_REQUIRE(ld >= inter, "moc_select_2of8: ld < intermediate size");
  MOC_REQUIRE(idx_dtype == MOC_I16 || idx_dtype == MOC_I32 || idx_dtype == MOC_I64,
              "moc_select_2of8: bad index dtype");
  MOC_REQUIRE(idx_dtype != MOC_I16 || inter - 1 <= 32767,
              "topk_idx range [0, %lld] cannot be stored as torch.int16", (long long)(inter - 1));
  MOC_REQUIRE(rows == 0 || (scores != nullptr && idx_out != nullptr), "moc_select_2of8: null pointer");
  if (rows == 0) return MOC_OK;
  const int kout = (int)moc_moc28_effective_k(inter);
  const int64_t groups = (inter + 7) / 8;
  const int64_t total = rows * groups;
  const dim3 grid(static_cast<unsigned>((total + 255) / 256)), block(256);
  hipStream_t st = as_stream(stream);
#define MOC_LAUNCH_2OF8(BF, T)                                                            \
  select_2of8_kernel<BF, T><<<grid, block, 0, st>>>(scores, rows, ld, (int)inter, kout, \
                                                     vals_out, static_cast<T*>(idx_out))
  const bool bf = dtype == MOC_BF16;
  if (idx_dtype == MOC_I16) { if (bf) MOC_LAUNCH_2OF8(true, int16_t); else MOC_LAUNCH_2OF8(false, int16_t); }
  else if (idx_dtype == MOC_I32) { if (bf) MOC_LAUNCH_2OF8(true, int32_t); else MOC_LAUNCH_2OF8(false, int32_t); }
  else { if (bf) MOC_LAUNCH_2OF8(true, int64_t); else MOC_LAUNCH_2OF8(false, int64_t); }
#undef MOC_LAUNCH_2OF8
  return check_launch("select_2of8_kernel");
}

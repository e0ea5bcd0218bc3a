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
// Top-K algorithm: one workgroup per row.  The row's order keys are staged in
// LDS, each thread then owns a contiguous chunk in registers.  An MSB-first
// radix *select* (8-bit digits, 2 passes for bf16 keys, 4 for f32) finds the
// exact threshold key T and the number r of T-valued channels that still have
// to be taken.  Two block scans then give each thread (a) how many T-valued
// channels precede its chunk, which resolves the lower-index tie rule, and
// (b) its output offset, which compacts the selection in channel order.
#include "abi.h"
#include "common.h"

namespace moc {
namespace {

constexpr int kTopkThreads = 256;
constexpr int kMaxTopkInter = 16384;

template <bool BF16>
__device__ __forceinline__ uint32_t load_key(const void* base, int64_t i, int transform) {
  if (BF16) {
    uint16_t b = static_cast<const uint16_t*>(base)[i];
    if (transform == 1) {  // |SiLU(g)| rounded to the score dtype (moc/ffn.py:335)
      b = f32_to_bf16(fabsf(silu_f32(bf16_to_f32(b))));
    }
    return bf16_order_key(b);
  } else {
    uint32_t u = static_cast<const uint32_t*>(base)[i];
    if (transform == 1) u = __float_as_uint(fabsf(silu_f32(__uint_as_float(u))));
    return f32_order_key(u);
  }
}

template <bool BF16, int ITEMS, typename IdxT>
__global__ __launch_bounds__(kTopkThreads) void topk_rows_kernel(
    const void* __restrict__ scores, int64_t ld, int inter, int k, int transform,
    void* __restrict__ vals, IdxT* __restrict__ idx, uint32_t* __restrict__ mask,
    int64_t mask_ld) {
  constexpr int KEY_BITS = BF16 ? 16 : 32;
  extern __shared__ uint32_t lds_dyn[];  // keys staging, later reused as flags
  __shared__ uint32_t hist[256];
  __shared__ uint32_t wtot[16];
  __shared__ uint32_t pick[2];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int64_t row = blockIdx.x;
  const size_t esz = BF16 ? 2 : 4;
  const void* src = static_cast<const char*>(scores) + row * ld * esz;

  // 1. stage order keys (coalesced), 2. pull my contiguous chunk to registers
  uint16_t* keys16 = reinterpret_cast<uint16_t*>(lds_dyn);
  for (int i = tid; i < inter; i += kTopkThreads) {
    const uint32_t key = load_key<BF16>(src, i, transform);
    if (BF16) keys16[i] = static_cast<uint16_t>(key); else lds_dyn[i] = key;
  }
  __syncthreads();
  const int chunk = (inter + kTopkThreads - 1) / kTopkThreads;
  const int beg = min(tid * chunk, inter);
  const int n = min(beg + chunk, inter) - beg;
  uint32_t key[ITEMS];
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    key[j] = 0;
    if (j < n) key[j] = BF16 ? static_cast<uint32_t>(keys16[beg + j]) : lds_dyn[beg + j];
  }

  // 3. MSB-first radix select of the k-th largest key
  uint32_t prefix = 0, pmask = 0;
  uint32_t krem = static_cast<uint32_t>(k);
#pragma unroll
  for (int shift = KEY_BITS - 8; shift >= 0; shift -= 8) {
    hist[tid] = 0;  // kTopkThreads == 256 bins
    __syncthreads();
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
      if (j < n && (key[j] & pmask) == prefix) atomicAdd(&hist[(key[j] >> shift) & 255u], 1u);
    }
    __syncthreads();
    // thread t looks at bin 255-t; inclusive scan over t = #elements with digit >= bin
    const uint32_t h = hist[255 - tid];
    const uint32_t inc = wave_inclusive_scan(h);
    if (lane == kWave - 1) wtot[wave] = inc;
    __syncthreads();
    uint32_t before = 0;
    for (int w = 0; w < wave; ++w) before += wtot[w];
    const uint32_t ge = before + inc;
    const uint32_t gt = ge - h;
    if (gt < krem && ge >= krem) {
      pick[0] = 255u - tid;
      pick[1] = krem - gt;
    }
    __syncthreads();
    prefix |= pick[0] << shift;
    pmask |= 255u << shift;
    krem = pick[1];
    __syncthreads();
  }
  const uint32_t thr = prefix;

  // 4. tie resolution + compaction in channel order
  uint32_t cgt = 0, ceq = 0;
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    if (j < n) {
      cgt += key[j] > thr;
      ceq += key[j] == thr;
    }
  }
  uint32_t total;
  const uint32_t eq_before = block_exclusive_scan(ceq, wtot, &total);
  const uint32_t take_eq = (krem > eq_before) ? min(krem - eq_before, ceq) : 0u;
  uint32_t pos = block_exclusive_scan(cgt + take_eq, wtot, &total);

  uint8_t* flags = reinterpret_cast<uint8_t*>(lds_dyn);
  IdxT* idx_row = idx + row * k;
  uint32_t eq_seen = 0;
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    if (j < n) {
      bool sel = key[j] > thr;
      if (key[j] == thr) {
        sel = (eq_before + eq_seen) < krem;
        ++eq_seen;
      }
      const int ch = beg + j;
      if (sel) {
        idx_row[pos] = static_cast<IdxT>(ch);
        if (vals != nullptr) {
          if (BF16) static_cast<uint16_t*>(vals)[row * k + pos] = static_cast<const uint16_t*>(src)[ch];
          else static_cast<uint32_t*>(vals)[row * k + pos] = static_cast<const uint32_t*>(src)[ch];
        }
        ++pos;
      }
      flags[ch] = sel ? 1 : 0;
    }
  }
  if (mask != nullptr) {
    __syncthreads();
    const int words = (inter + 31) / 32;
    for (int w = tid; w < words; w += kTopkThreads) {
      uint32_t bits = 0;
      const int c0 = w * 32;
      const int cn = min(32, inter - c0);
      for (int b = 0; b < cn; ++b) bits |= static_cast<uint32_t>(flags[c0 + b]) << b;
      mask[row * mask_ld + w] = bits;
    }
  }
}

template <bool BF16, int ITEMS>
int launch_topk_items(const void* scores, int64_t rows, int inter, int64_t ld, int k,
                      int transform, void* vals, void* idx, int idx_dtype, uint32_t* mask,
                      int64_t mask_ld, hipStream_t st) {
  const size_t lds = static_cast<size_t>(inter) * (BF16 ? 2 : 4);
  const dim3 grid(static_cast<unsigned>(rows)), block(kTopkThreads);
  switch (idx_dtype) {
    case MOC_I16:
      topk_rows_kernel<BF16, ITEMS, int16_t><<<grid, block, lds, st>>>(
          scores, ld, inter, k, transform, vals, static_cast<int16_t*>(idx), mask, mask_ld);
      break;
    case MOC_I32:
      topk_rows_kernel<BF16, ITEMS, int32_t><<<grid, block, lds, st>>>(
          scores, ld, inter, k, transform, vals, static_cast<int32_t*>(idx), mask, mask_ld);
      break;
    default:
      topk_rows_kernel<BF16, ITEMS, int64_t><<<grid, block, lds, st>>>(
          scores, ld, inter, k, transform, vals, static_cast<int64_t*>(idx), mask, mask_ld);
      break;
  }
  return check_launch("topk_rows_kernel");
}

template <bool BF16>
int launch_topk(const void* scores, int64_t rows, int inter, int64_t ld, int k, int transform,
                void* vals, void* idx, int idx_dtype, uint32_t* mask, int64_t mask_ld,
                hipStream_t st) {
  const int chunk = (inter + kTopkThreads - 1) / kTopkThreads;
  if (chunk <= 8)
    return launch_topk_items<BF16, 8>(scores, rows, inter, ld, k, transform, vals, idx, idx_dtype, mask, mask_ld, st);
  if (chunk <= 16)
    return launch_topk_items<BF16, 16>(scores, rows, inter, ld, k, transform, vals, idx, idx_dtype, mask, mask_ld, st);
  if (chunk <= 32)
    return launch_topk_items<BF16, 32>(scores, rows, inter, ld, k, transform, vals, idx, idx_dtype, mask, mask_ld, st);
  return launch_topk_items<BF16, 64>(scores, rows, inter, ld, k, transform, vals, idx, idx_dtype, mask, mask_ld, st);
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

}  // namespace
}  // namespace moc

using namespace moc;

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

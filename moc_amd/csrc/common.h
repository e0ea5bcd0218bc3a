// Shared device helpers for the MoC gfx950 kernels.
//
// Everything here is written for CDNA4 (gfx950, wave64).  bf16 values travel
// as raw uint16_t bit patterns so that the kernels never depend on a vendor
// bf16 header; conversions follow the IEEE-754 definition of round to nearest,
// ties to even, with NaN mapped to the canonical quiet NaN 0x7FC0 (the same
// result torch's float->bfloat16 cast produces).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moc {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// bf16 <-> f32
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;  // any NaN
  const uint32_t bias = 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>((u + bias) >> 16);
}

// Round an f32 to the nearest bf16 and return it widened back to f32.
__device__ __forceinline__ float round_bf16(float f) {
  return bf16_to_f32(f32_to_bf16(f));
}

// RNE to bf16 with the gfx950 packed conversion; NaN keeps the canonical
// 0x7FC0 of f32_to_bf16 (same bits as f32_to_bf16 for every input).
typedef float cvt_f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 cvt_bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint16_t bf16_rne(float f) {
  const uint32_t w =
      __builtin_bit_cast(uint32_t, __builtin_convertvector((cvt_f32x2_t){f, 0.0f}, cvt_bf16x2_t));
  return f != f ? uint16_t(0x7FC0u) : static_cast<uint16_t>(w & 0xFFFFu);
}
__device__ __forceinline__ float bf16_rnd(float f) { return bf16_to_f32(bf16_rne(f)); }

// Backward of one selected entry of the sparse SwiGLU (bf16 chain of
// moc/training/triton_sparse_aux.py:376-400): g, u the saved gate/up values,
// gz the gradient of z = SiLU(g) * u; s = SiLU(g) as saved (bf16), or, when
// have_s is false, recomputed as bf16(g / (1 + exp(-g))) (F.silu's formula,
// moc/ffn.py:435-436).  One exp serves both SiLU and the sigmoid.
__device__ __forceinline__ void sparse_bwd_entry(float g, float u, bool have_s, float s_saved,
                                                 float gz, uint16_t& grad_g, uint16_t& grad_u) {
  const float den = 1.0f + expf(-g);
  const float s = have_s ? s_saved : bf16_rnd(g / den);
  const float gs = bf16_rnd(u * gz);
  const float gu = bf16_rnd(s * gz);
  const float sig = bf16_rnd(1.0f / den);
  const float t1 = bf16_rnd(1.0f - sig);
  const float t2 = bf16_rnd(g * t1);
  const float t3 = bf16_rnd(1.0f + t2);
  const float d = bf16_rnd(sig * t3);
  grad_g = bf16_rne(gs * d);
  grad_u = bf16_rne(gu);
}

// ---------------------------------------------------------------------------
// Order keys: unsigned integers whose natural order is the IEEE order of the
// values.  -0.0 and +0.0 map to the same key (they compare equal as numbers)
// and every NaN maps to the largest key, so a NaN ranks above +inf.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t bf16_order_key(uint16_t b) {
  if ((b & 0x7FFFu) > 0x7F80u) return 0xFFFFu;  // NaN
  if (b == 0x8000u) b = 0;                       // -0 -> +0
  return (b & 0x8000u) ? (static_cast<uint32_t>(~b) & 0xFFFFu)
                       : (static_cast<uint32_t>(b) | 0x8000u);
}

__device__ __forceinline__ uint32_t f32_order_key(uint32_t u) {
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0xFFFFFFFFu;  // NaN
  if (u == 0x80000000u) u = 0;                                 // -0 -> +0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// ---------------------------------------------------------------------------
// SiLU and its derivative, in f32.  expf is the accurate device exp.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float sigmoid_f32(float g) { return 1.0f / (1.0f + expf(-g)); }

// MoC 2:8: top-2 of one group of 8 channels from its bf16 gate and up
// values (gw, uw: channel 2e in the low half of word e, 2e + 1 in the high
// half): top-1 is the largest gate value with the lowest index among equal
// maxima, top-2 the largest of the other seven under the same rule (NaN
// above +inf, -0 equal to +0), sz = bf16((g * sigmoid(g)) * u) in f32
// (moc/inference/triton_fused_ffn_kernels.py:103-114,126-129).
// Each channel's key is its 16-bit order key (0x8000 + |v| for v >= 0,
// 0x8000 - |v| for v < 0, NaN 0xFFFF) above 7 - index, so the eight keys
// are distinct, a larger key is the better channel, and the top two come
// out of a max/min tournament.
typedef unsigned short g8_u16x2 __attribute__((ext_vector_type(2)));
typedef short g8_s16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void select_group_top2_bits(const uint32_t (&gw)[4], const uint32_t (&uw)[4],
                                                       int& b1, int& b2, uint16_t& s1, uint16_t& s2) {
  uint32_t k[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const g8_u16x2 v = __builtin_bit_cast(g8_u16x2, gw[e]);
    const g8_u16x2 m = __builtin_bit_cast(g8_u16x2, __builtin_bit_cast(g8_s16x2, gw[e]) >> 15);
    const g8_u16x2 a = v & static_cast<unsigned short>(0x7FFF);
    uint32_t key2 = __builtin_bit_cast(uint32_t, ((a ^ m) + static_cast<unsigned short>(0x8000)) - m);
    // NaN: |v| > 0x7F80 in either half -> key 0xFFFF
    const uint32_t lo_nan = (a.x > 0x7F80u) ? 0xFFFFu : 0u, hi_nan = (a.y > 0x7F80u) ? 0xFFFF0000u : 0u;
    key2 |= lo_nan | hi_nan;
    k[2 * e] = (key2 << 16) | static_cast<uint32_t>(7 - 2 * e);
    k[2 * e + 1] = (key2 & 0xFFFF0000u) | static_cast<uint32_t>(6 - 2 * e);
  }
  uint32_t f[4], sc[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    f[p] = max(k[2 * p], k[2 * p + 1]);
    sc[p] = min(k[2 * p], k[2 * p + 1]);
  }
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const uint32_t hi = max(f[2 * p], f[2 * p + 1]), lo = min(f[2 * p], f[2 * p + 1]);
    sc[p] = max(lo, max(sc[2 * p], sc[2 * p + 1]));
    f[p] = hi;
  }
  const uint32_t F = max(f[0], f[1]);
  const uint32_t S = max(min(f[0], f[1]), max(sc[0], sc[1]));
  b1 = 7 - static_cast<int>(F & 7u);
  b2 = 7 - static_cast<int>(S & 7u);
  auto value_of = [](const uint32_t (&w4)[4], int b) {
    const uint32_t w = (b >> 1) == 0 ? w4[0] : (b >> 1) == 1 ? w4[1] : (b >> 1) == 2 ? w4[2] : w4[3];
    return __uint_as_float((b & 1) ? (w & 0xFFFF0000u) : (w << 16));
  };
  const float g1 = value_of(gw, b1), g2 = value_of(gw, b2);
  s1 = bf16_rne((g1 * sigmoid_f32(g1)) * value_of(uw, b1));
  s2 = bf16_rne((g2 * sigmoid_f32(g2)) * value_of(uw, b2));
}

// The same from bf16-exact f32 values g[8], u[8].
__device__ __forceinline__ void select_group_top2(const float* g, const float* u, int& b1, int& b2,
                                                  uint16_t& s1, uint16_t& s2) {
  uint32_t gw[4], uw[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    gw[e] = (__float_as_uint(g[2 * e]) >> 16) | (__float_as_uint(g[2 * e + 1]) & 0xFFFF0000u);
    uw[e] = (__float_as_uint(u[2 * e]) >> 16) | (__float_as_uint(u[2 * e + 1]) & 0xFFFF0000u);
  }
  select_group_top2_bits(gw, uw, b1, b2, s1, s2);
}

__device__ __forceinline__ void select_group_emit_bits(const uint32_t (&gw)[4], const uint32_t (&uw)[4],
                                                       int64_t c0, int64_t* __restrict__ idx_out,
                                                       uint16_t* __restrict__ sz_out) {
  int b1, b2;
  uint16_t s1, s2;
  select_group_top2_bits(gw, uw, b1, b2, s1, s2);
  idx_out[0] = c0 + b1;
  idx_out[1] = c0 + b2;
  sz_out[0] = s1;
  sz_out[1] = s2;
}

__device__ __forceinline__ void select_group_emit(const float* g, const float* u, int64_t c0,
                                                  int64_t* __restrict__ idx_out,
                                                  uint16_t* __restrict__ sz_out) {
  int b1, b2;
  uint16_t s1, s2;
  select_group_top2(g, u, b1, b2, s1, s2);
  idx_out[0] = c0 + b1;
  idx_out[1] = c0 + b2;
  sz_out[0] = s1;
  sz_out[1] = s2;
}

// 2:4 packing of one 8-channel group holding two selected channels at
// positions p1 != p2 (0-7) with values v1, v2: each 4-channel half keeps two
// stored values (its selected values in channel order, zeros for the rest,
// at distinct positions).  out: lo0, lo1, hi0, hi1; the return value holds
// the four 2-bit positions in the same order (bits 0-7).
__device__ __forceinline__ uint32_t pack_group_2of8(int p1, uint16_t v1, int p2, uint16_t v2,
                                                    uint16_t (&out)[4]) {
  // branch-free: (qa, va) the lower position, (qb, vb) the higher
  const bool sw = p2 < p1;
  const int qa = sw ? p2 : p1, qb = sw ? p1 : p2;
  const uint16_t va = sw ? v2 : v1, vb = sw ? v1 : v2;
  const bool lo_both = qb < 4, hi_both = qa >= 4, split = !lo_both && !hi_both;
  // low half: both there -> (qa, qb); none -> zeros at (0, 1); qa alone ->
  // stored at 0 when qa is 0 (zero at 1), else zero at 0 and qa
  const uint32_t l0 = lo_both ? static_cast<uint32_t>(qa) : 0u;
  const uint32_t l1 = lo_both ? static_cast<uint32_t>(qb) : hi_both ? 1u : static_cast<uint32_t>(max(qa, 1));
  out[0] = (lo_both || (split && qa == 0)) ? va : uint16_t(0);
  out[1] = lo_both ? vb : (split && qa != 0) ? va : uint16_t(0);
  // high half, the same with qb alone in the split case
  const uint32_t h0 = hi_both ? static_cast<uint32_t>(qa - 4) : 0u;
  const uint32_t h1 = hi_both ? static_cast<uint32_t>(qb - 4) : lo_both ? 1u : static_cast<uint32_t>(max(qb - 4, 1));
  out[2] = hi_both ? va : (split && qb == 4) ? vb : uint16_t(0);
  out[3] = (hi_both || (split && qb != 4)) ? vb : uint16_t(0);
  return l0 | (l1 << 2) | (h0 << 4) | (h1 << 6);
}

// Positions byte of an 8-group with nothing to pack (zeros at 0, 1 per half).
constexpr uint32_t kPackEmpty2of8 = 0x44u;

// Dot product of 8 bf16 pairs (two 16-byte chunks) accumulated in f32: one
// v_dot2c_f32_bf16 per packed pair (acc + a0 b0 + a1 b1; the bf16 products
// are exact in f32), where unpacking each half and an FMA per product took
// six VALU instructions per pair.
typedef __bf16 dot_bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(dot_bf16x2_t, a),
                                         __builtin_bit_cast(dot_bf16x2_t, b), acc, false);
}

__device__ __forceinline__ float dot8(uint4 a, uint4 b, float acc) {
  acc = dot2_bf16(a.x, b.x, acc);
  acc = dot2_bf16(a.y, b.y, acc);
  acc = dot2_bf16(a.z, b.z, acc);
  return dot2_bf16(a.w, b.w, acc);
}

// RMSNorm of 8 bf16 values with the row's factor r = 1 / sqrt(mean(x^2) +
// eps) and the norm weights w: bf16(bf16(x * r) * w), the rounding points of
// (x.float() * r).to(bf16) * w (benchmark_decode.py:101-109).
__device__ __forceinline__ uint4 rmsnorm8(uint4 xv, uint4 wv, float r) {
  const uint32_t a[4] = {xv.x, xv.y, xv.z, xv.w}, w[4] = {wv.x, wv.y, wv.z, wv.w};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float lo = round_bf16(round_bf16(__uint_as_float(a[i] << 16) * r) * __uint_as_float(w[i] << 16));
    const float hi = round_bf16(round_bf16(__uint_as_float(a[i] & 0xFFFF0000u) * r) *
                                __uint_as_float(w[i] & 0xFFFF0000u));
    o[i] = (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + expf(-g)); }

// ---------------------------------------------------------------------------
// Wave64 reductions / scans with DPP row operations (VALU, no LDS round
// trip), rows of 16 lanes joined with row_bcast / readlane.
// ---------------------------------------------------------------------------
template <int CTRL, int ROW_MASK = 0xF, int BANK_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  // lanes whose source is outside the row, or in a masked row, read 0
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, ROW_MASK, BANK_MASK, true));
}

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}

__device__ __forceinline__ uint32_t wave_read_lane(uint32_t v, int lane) {
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), lane));
}

// Sum over the 64 lanes, returned to every lane.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f32<0x141>(v);  // row_half_mirror
  v += dpp_f32<0x140>(v);  // row_mirror: every lane holds its row's sum
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

// Inclusive prefix sum over lanes 0..63 (Hillis-Steele within rows, then
// row 0's total into row 1 and rows 0-1's total into rows 2-3).
__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t v) {
  v += dpp_u32<0x111>(v);       // row_shr:1
  v += dpp_u32<0x112>(v);       // row_shr:2
  v += dpp_u32<0x114>(v);       // row_shr:4
  v += dpp_u32<0x118>(v);       // row_shr:8
  v += dpp_u32<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
  v += dpp_u32<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}

// Exclusive scan over the whole block of blockDim.x threads (a multiple of 64,
// at most 1024).  `wave_tot` is LDS scratch of at least 16 words.  Returns the
// exclusive prefix and writes the block total to *total.  Contains barriers:
// every thread of the block must call it.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* wave_tot,
                                                         uint32_t* total) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int nwaves = blockDim.x / kWave;
  const uint32_t inc = wave_inclusive_scan(v);
  if (lane == kWave - 1) wave_tot[wave] = inc;
  __syncthreads();
  if (wave == 0) {
    uint32_t w = (lane < nwaves) ? wave_tot[lane] : 0u;
    w = wave_inclusive_scan(w);
    if (lane < nwaves) wave_tot[lane] = w;  // inclusive totals
  }
  __syncthreads();
  const uint32_t before_wave = (wave > 0) ? wave_tot[wave - 1] : 0u;
  *total = wave_tot[nwaves - 1];
  __syncthreads();
  return before_wave + inc - v;
}

}  // namespace moc

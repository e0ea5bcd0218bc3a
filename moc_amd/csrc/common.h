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
__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + expf(-g)); }

// ---------------------------------------------------------------------------
// Wave64 reductions / scans through cross-lane shuffles.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t v) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const uint32_t t = __shfl_up(v, off, kWave);
    if (lane >= off) v += t;
  }
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

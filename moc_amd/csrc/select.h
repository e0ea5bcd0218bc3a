// Selection of the k largest order keys of one row, by a group of NW waves
// (NW = 1: one wave selects on its own, with no workgroup barrier; NW > 1:
// the NW waves of a workgroup select one row together).
//
// Thread t of the group holds the order keys of the L contiguous channels
// [t L, t L + L) in registers (L a multiple of 8; two 16-bit keys per
// register for bf16 scores, one 32-bit key for f32).  Channels past the row
// end hold the key 0, which no real value produces (real bf16/f32 keys are
// >= 0x80 / 0x800000), so a padding key is never the k-th largest and
// counting padding keys in the lowest bin never moves the threshold.
//
// select_threshold finds the k-th largest key T and how many T-valued
// channels still have to be taken (krem) by an MSB-first radix select with
// 8-bit digits (2 passes over the registers for 16-bit keys, 4 for 32-bit;
// with 16-bit keys one wave (select_threshold_window) or a group of waves
// (select_threshold_window_group) first tries two passes over the 4096 keys
// below the row's largest).
// The group counts into one 256-bin LDS histogram kept in C copies (lane % C
// picks the copy): LDS atomics serialise on lanes of one instruction that
// hit the same address, and real scores pile into a few exponent bins, so
// 16 copies make an atomic about twice as fast as 4 (at four times the
// LDS to clear and read back).  A key
// whose higher digits do not match the prefix found so far is counted into
// a spare bin of its lane instead (a branch-free unsigned min), so no pass
// needs a compare per key.  With NW = 1 the wave's own program order orders
// its LDS operations; with NW > 1 workgroup barriers separate clearing,
// counting and reading.
//
// select_ranks turns T into per-thread bit masks of the selected channels:
// every channel above T, and the krem lowest-index T-valued channels (the
// reference's tie rule), with the thread's first rank from one scan of the
// packed (count > T, count == T) pair over the group.  select_emit then
// visits the set bits, so the cost of the emit grows with the number of
// selected channels a thread holds, not with L.
#pragma once

#include "common.h"

namespace moc {

typedef unsigned short sel_u16x2 __attribute__((ext_vector_type(2)));
typedef short sel_s16x2 __attribute__((ext_vector_type(2)));

constexpr int kSelBins = 256;

// Histogram layout for C copies (lane % C picks the copy): 256 bins, one
// spare bin per lane sharing the copy, pad dwords up to a multiple of four
// (every copy starts 16-byte aligned, so a scan reads four bins at once; the
// copies' bin b still fall in distinct LDS banks for C = 4 and 8).
template <int C>
constexpr int sel_copy_pitch() {
  return (kSelBins + 64 / C + 1 + 3) / 4 * 4;
}

// The second pass of a group's windowed threshold counts the 16 keys of one
// window bin into its own small histogram (C copies, a spare bin per lane
// sharing the copy, one pad dword), so it needs no barrier to clear the
// first pass's counts while other waves still read them.
template <int C>
constexpr int sel_copy_pitch16() {
  return 16 + 64 / C + 1;
}

// LDS dwords the selection of a group of NW waves needs: the histogram, a
// per-wave table, and (NW > 1) the 16-bin histogram of the window's second
// pass.
template <int NW, int C>
constexpr int select_lds_dwords() {
  return C * sel_copy_pitch<C>() + (NW > 1 ? NW + C * sel_copy_pitch16<C>() : 0);
}

// Order keys of two packed bf16 values: 0x8000 + |v| for v >= 0 (and -0),
// 0x8000 - |v| for v < 0, so keys compare as the values do; five packed
// 16-bit operations for the pair.  NaN is fixed up by bf16x2_fix_nan.
__device__ __forceinline__ uint32_t bf16x2_order_keys(uint32_t w, sel_u16x2& amax) {
  const sel_u16x2 v = __builtin_bit_cast(sel_u16x2, w);
  const sel_u16x2 m = __builtin_bit_cast(sel_u16x2, __builtin_bit_cast(sel_s16x2, w) >> 15);
  const sel_u16x2 a = v & static_cast<unsigned short>(0x7FFF);
  amax = __builtin_elementwise_max(amax, a);
  return __builtin_bit_cast(uint32_t, ((a ^ m) + static_cast<unsigned short>(0x8000)) - m);
}

// NaN (either sign) ranks above +inf (key 0xFF80) and all NaNs are equal:
// bf16x2_order_keys maps a NaN to (0xFF80, 0xFFFF] or [0x0001, 0x007F],
// ranges no number reaches; both become 0xFFFF.
__device__ __forceinline__ uint32_t bf16x2_fix_nan(uint32_t key2) {
  uint32_t r = key2;
  const uint32_t lo = key2 & 0xFFFFu, hi = key2 >> 16;
  if (lo > 0xFF80u || (lo != 0u && lo < 0x80u)) r |= 0xFFFFu;
  if (hi > 0xFF80u || (hi != 0u && hi < 0x80u)) r |= 0xFFFF0000u;
  return r;
}

// Order key of one f32 value with the same rules (NaN -> 0xFFFFFFFF, -0 ->
// +0): 0x80000000 + |v| for v >= 0, 0x80000000 - |v| for v < 0.
__device__ __forceinline__ uint32_t f32_fast_order_key(uint32_t u) {
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return 0xFFFFFFFFu;
  return (u & 0x80000000u) ? 0x80000000u - a : 0x80000000u + a;
}

// Words per thread: two 16-bit keys or one 32-bit key per register.
template <bool BF16, int L>
constexpr int sel_words() {
  return BF16 ? L / 2 : L;
}

// Raw scores of channels [c0, c0 + L) of a row of n channels (BF16: uint16
// bits, else f32 bits) into w, 0 past n; loaded by this thread directly.
// vec: the row is 16-byte aligned, so whole 8-channel chunks load as
// 16-byte vectors.
template <bool BF16, int L>
__device__ __forceinline__ void load_row_raw(const void* src, int n, int c0, bool vec,
                                             uint32_t (&w)[sel_words<BF16, L>()]) {
  static_assert(L % 8 == 0, "L must be a multiple of 8");
  constexpr int W = sel_words<BF16, L>();
  constexpr int WPC = BF16 ? 4 : 8;  // words per 8-channel chunk
  constexpr int ESZ = BF16 ? 2 : 4;
  const char* s = static_cast<const char*>(src);
  if (vec) {
#pragma unroll
    for (int i = 0; i < L / 8; ++i) {
      const int c = c0 + 8 * i;
      if (c + 8 <= n) {
        const uint4 a = *reinterpret_cast<const uint4*>(s + static_cast<int64_t>(c) * ESZ);
        w[WPC * i + 0] = a.x; w[WPC * i + 1] = a.y; w[WPC * i + 2] = a.z; w[WPC * i + 3] = a.w;
        if constexpr (!BF16) {
          const uint4 b = *reinterpret_cast<const uint4*>(s + static_cast<int64_t>(c) * ESZ + 16);
          w[WPC * i + 4] = b.x; w[WPC * i + 5] = b.y; w[WPC * i + 6] = b.z; w[WPC * i + 7] = b.w;
        }
      } else {
#pragma unroll
        for (int q = 0; q < WPC; ++q) w[WPC * i + q] = 0;
      }
    }
  }
  // element loads: everything without vec, else only the chunk that
  // straddles the row end
  if (!vec || (c0 < n && c0 + L > n)) {
#pragma unroll
    for (int j = 0; j < W; ++j) {
      const int chunk_end = c0 + 8 * (j / WPC) + 8;
      if (!vec || chunk_end > n) {
        if constexpr (BF16) {
          const int c = c0 + 2 * j;
          const uint16_t* e = reinterpret_cast<const uint16_t*>(s);
          const uint32_t lo = c < n ? e[c] : 0u, hi = c + 1 < n ? e[c + 1] : 0u;
          w[j] = lo | (hi << 16);
        } else {
          const int c = c0 + j;
          w[j] = c < n ? reinterpret_cast<const uint32_t*>(s)[c] : 0u;
        }
      }
    }
  }
}

// The same through LDS: the group of NW waves (thread t) loads the row
// coalesced into stage (64 NW L channels, 16-byte aligned), then each thread
// reads its own L channels back with 16-byte LDS reads.  Used where a
// thread's share is long: direct loads of long per-thread runs touch every
// cache line from many load instructions.  stage may alias the select's
// histograms: with reuse, a last barrier orders the reads before that.
template <int NW, bool BF16, int L>
__device__ __forceinline__ void load_row_raw_staged(const void* src, int n, int t, bool vec,
                                                    uint32_t* stage,
                                                    uint32_t (&w)[sel_words<BF16, L>()],
                                                    bool reuse = true) {
  constexpr int GT = 64 * NW;
  constexpr int EPC = BF16 ? 8 : 4;        // elements per 16 bytes
  constexpr int CPT = L / EPC;             // 16-byte chunks per thread
  constexpr int ESZ = BF16 ? 2 : 4;
  const char* s = static_cast<const char*>(src);
  uint4* st4 = reinterpret_cast<uint4*>(stage);
  if (vec) {
    const int nfull = n / EPC;
    uint4 v[CPT];
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int ch = t + GT * i;
      if (ch < nfull) {
        v[i] = *reinterpret_cast<const uint4*>(s + static_cast<int64_t>(ch) * 16);
      } else {
        uint32_t e[4] = {0u, 0u, 0u, 0u};
        if (ch == nfull) {  // the chunk that straddles the row end
#pragma unroll
          for (int q = 0; q < EPC; ++q) {
            const int c = ch * EPC + q;
            if (c < n) {
              if (BF16) e[q / 2] |= static_cast<uint32_t>(reinterpret_cast<const uint16_t*>(s)[c]) << (16 * (q & 1));
              else e[q] = reinterpret_cast<const uint32_t*>(s)[c];
            }
          }
        }
        v[i] = make_uint4(e[0], e[1], e[2], e[3]);
      }
    }
#pragma unroll
    for (int i = 0; i < CPT; ++i) st4[t + GT * i] = v[i];
  } else {
    constexpr int EPT = L;  // elements per thread, coalesced over the group
    uint32_t v[EPT];
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const int c = t + GT * i;
      v[i] = c < n ? (BF16 ? static_cast<uint32_t>(reinterpret_cast<const uint16_t*>(s)[c])
                           : reinterpret_cast<const uint32_t*>(s)[c])
                   : 0u;
    }
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const int c = t + GT * i;
      if (BF16) reinterpret_cast<uint16_t*>(stage)[c] = static_cast<uint16_t>(v[i]);
      else stage[c] = v[i];
    }
  }
  if constexpr (NW > 1) __syncthreads(); else __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const uint4 a = st4[t * CPT + i];
    w[4 * i + 0] = a.x; w[4 * i + 1] = a.y; w[4 * i + 2] = a.z; w[4 * i + 3] = a.w;
  }
  (void)ESZ;
  if (reuse) {
    if constexpr (NW > 1) __syncthreads(); else __builtin_amdgcn_wave_barrier();
  }
}

// Raw scores in w (channels [c0, c0 + L)) -> order keys, key 0 past n.
// transform 1 ranks by |SiLU(v)| rounded to the score type instead of v
// (key_of gives that key for one raw value).
template <bool BF16, int L, typename KeyOf>
__device__ __forceinline__ void raw_to_keys(int n, int c0, int transform, KeyOf key_of,
                                            uint32_t (&w)[sel_words<BF16, L>()]) {
  constexpr int W = sel_words<BF16, L>();
  if (transform == 0) {
    if constexpr (BF16) {
      sel_u16x2 amax = {0, 0};
#pragma unroll
      for (int j = 0; j < W; ++j) w[j] = bf16x2_order_keys(w[j], amax);
      if (__builtin_expect(amax.x > 0x7F80 || amax.y > 0x7F80, 0)) {
#pragma unroll
        for (int j = 0; j < W; ++j) w[j] = bf16x2_fix_nan(w[j]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < W; ++j) w[j] = f32_fast_order_key(w[j]);
    }
  } else {
#pragma unroll
    for (int j = 0; j < W; ++j)
      w[j] = BF16 ? (key_of(w[j] & 0xFFFFu) | (key_of(w[j] >> 16) << 16)) : key_of(w[j]);
  }
  // padding channels -> key 0
  if (c0 + L > n) {
#pragma unroll
    for (int j = 0; j < W; ++j) {
      if constexpr (BF16) {
        const int c = c0 + 2 * j;
        if (c >= n) w[j] = 0;
        else if (c + 1 >= n) w[j] &= 0xFFFFu;
      } else {
        if (c0 + j >= n) w[j] = 0;
      }
    }
  }
}

// Scan of one histogram (C copies summed) from the top bin down: the bin pb
// holding the krem-th largest counted key and the count gt of keys in the
// bins above it.  Lane l owns bins 255 - 64 m - l (m = 0..3): every m a run
// of 64 descending bins in lane order, so the reads are bank-conflict free.
// Returns false (pb, gt untouched) when fewer than krem keys were counted.
template <int C>
__device__ __forceinline__ bool sel_scan_bins(const uint32_t* hist, int lane, uint32_t krem, uint32_t& pb,
                                              uint32_t& gt) {
  constexpr int kPitch = sel_copy_pitch<C>();
  uint32_t s[4], ge[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int bin = kSelBins - 1 - 64 * m - lane;
    uint32_t v = 0;
#pragma unroll
    for (int c = 0; c < C; ++c) v += hist[c * kPitch + bin];
    s[m] = v;
  }
  // keys in bins >= bin
  uint32_t base = 0;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const uint32_t incl = wave_inclusive_scan(s[m]);
    ge[m] = base + incl;
    base += wave_read_lane(incl, 63);
  }
  int hit_m = -1;
  uint32_t hit_gt = 0;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const uint32_t g = ge[m] - s[m];
    if (g < krem && ge[m] >= krem) {
      hit_m = m;
      hit_gt = g;
    }
  }
  const unsigned long long hits = __ballot(hit_m >= 0);
  if (hits == 0ull) return false;
  const int src = __ffsll(hits) - 1;
  pb = kSelBins - 1 - 64 * wave_read_lane(static_cast<uint32_t>(hit_m), src) - src;
  gt = wave_read_lane(hit_gt, src);
  return true;
}

// The same scan with lane l owning the four contiguous bins 252 - 4l ...
// 255 - 4l: one 16-byte LDS read per copy and one wave scan (hist must be
// 16-byte aligned).
template <int C>
__device__ __forceinline__ bool sel_scan_bins4(const uint32_t* hist, int lane, uint32_t krem, uint32_t& pb,
                                               uint32_t& gt) {
  constexpr int kPitch = sel_copy_pitch<C>();
  uint32_t s0 = 0, s1 = 0, s2 = 0, s3 = 0;  // bins 252 - 4l ... 255 - 4l
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const uint4 v = *reinterpret_cast<const uint4*>(hist + c * kPitch + kSelBins - 4 - 4 * lane);
    s0 += v.x; s1 += v.y; s2 += v.z; s3 += v.w;
  }
  const uint32_t tot = s0 + s1 + s2 + s3;
  const uint32_t incl = wave_inclusive_scan(tot);
  uint32_t g = incl - tot;  // keys in the bins above this lane's four
  const unsigned long long hits = __ballot(g < krem && incl >= krem);
  if (hits == 0ull) return false;
  const int src = __ffsll(hits) - 1;
  uint32_t j = 3;  // from the top bin down: the first whose count reaches krem
  if (g + s3 >= krem) j = 0;
  else if (g + s3 + s2 >= krem) { j = 1; g += s3; }
  else if (g + s3 + s2 + s1 >= krem) { j = 2; g += s3 + s2; }
  else g += s3 + s2 + s1;
  pb = kSelBins - 1 - 4 * src - wave_read_lane(j, src);
  gt = wave_read_lane(g, src);
  return true;
}

// Largest value over the 64 lanes, returned to every lane.
__device__ __forceinline__ uint32_t sel_wave_max(uint32_t v) {
  v = max(v, dpp_u32<0xB1>(v));   // quad_perm [1,0,3,2]
  v = max(v, dpp_u32<0x4E>(v));   // quad_perm [2,3,0,1]
  v = max(v, dpp_u32<0x141>(v));  // row_half_mirror
  v = max(v, dpp_u32<0x140>(v));  // row_mirror: every lane holds its row's max
  return max(max(wave_read_lane(v, 0), wave_read_lane(v, 16)), max(wave_read_lane(v, 32), wave_read_lane(v, 48)));
}

// One wave, 16-bit keys: the threshold in two passes over a window below the
// row's largest key hi, when the k-th largest key lies in [hi - 4095, hi]
// (32 binades below the largest value).  Pass 1 counts bins of 16 keys (a
// sixteenth of a binade) over the window, pass 2 the 16 keys of the bin
// found.  The top byte of a key (sign and seven exponent bits) puts two
// binades in one bin, a quarter of a Gaussian row's keys, and the atomic
// adds of the 16 lanes that share a copy serialise on that address; a
// sixteenth of a binade spreads the same keys over 32 bins.  Keys outside
// the counted range go to the lane's spare bin: as unsigned values,
// (key - base) >> 4 in pass 1 and (key - base) << 4 in pass 2 (in-bin keys
// on every 16th bin) are then at least 256 (no key lies above the window).
// Returns false, with nothing decided, when fewer than k keys lie in the
// window (the caller then runs the byte-digit passes).
template <int C, int W>
__device__ __forceinline__ bool select_threshold_window(const uint32_t (&w)[W], uint32_t k, uint32_t* hist,
                                                        uint32_t& thr, uint32_t& krem) {
  constexpr int kPitch = sel_copy_pitch<C>();
  constexpr int kHist = C * kPitch;
  const int lane = threadIdx.x & 63;
  uint32_t* mine = hist + (lane % C) * kPitch;
  const uint32_t spare = kSelBins + lane / C;
  auto bump = [&](uint32_t bin) {
    __hip_atomic_fetch_add(&mine[bin], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  };
  sel_u16x2 m2 = {0, 0};
#pragma unroll
  for (int j = 0; j < W; ++j) m2 = __builtin_elementwise_max(m2, __builtin_bit_cast(sel_u16x2, w[j]));
  const uint32_t hi = sel_wave_max(max(static_cast<uint32_t>(m2.x), static_cast<uint32_t>(m2.y)));
  // the lowest real key is 0x80; padding keys (0) fall below the window
  const int lo = max(static_cast<int>(hi) - 4095, 1);
  for (int i = lane; i < kHist; i += 64) hist[i] = 0;
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int j = 0; j < W; ++j) {
    bump(min(static_cast<uint32_t>(static_cast<int>(w[j] & 0xFFFFu) - lo) >> 4, spare));
    bump(min(static_cast<uint32_t>(static_cast<int>(w[j] >> 16) - lo) >> 4, spare));
  }
  __builtin_amdgcn_wave_barrier();
  uint32_t pb, gt;
  if (!sel_scan_bins<C>(hist, lane, k, pb, gt)) return false;
  krem = k - gt;
  const int kb = lo + 16 * static_cast<int>(pb);  // the bin holds keys [kb, kb + 16)
  __builtin_amdgcn_wave_barrier();
  for (int i = lane; i < kHist; i += 64) hist[i] = 0;
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int j = 0; j < W; ++j) {
    bump(min(static_cast<uint32_t>(static_cast<int>(w[j] & 0xFFFFu) - kb) << 4, spare));
    bump(min(static_cast<uint32_t>(static_cast<int>(w[j] >> 16) - kb) << 4, spare));
  }
  __builtin_amdgcn_wave_barrier();
  sel_scan_bins<C>(hist, lane, krem, pb, gt);  // krem of the bin's keys lie in the bin
  thr = static_cast<uint32_t>(kb) + (pb >> 4);
  krem -= gt;
  return true;
}

// The same window for a group of NW > 1 waves selecting one row together
// (thread t of the group holds channels [t L, t L + L)), in three steps so
// that a kernel can do its own work between them:
//  - sel_window_pass1: the row's largest key (per-wave maxima through the
//    table behind the histogram, which is cleared meanwhile, with the 16-bin
//    one), the first pass and its scan, two workgroup barriers; every wave
//    scans the counts itself.  Gives the bin [kb, kb + 16) that holds the
//    k-th largest key and krem, the number of keys to take from it; returns
//    false, uniformly over the group, when fewer than k keys lie in the
//    window;
//  - sel_window_pass2_count: the keys of that bin into the 16-bin histogram
//    (no barrier: the caller puts one before the scan);
//  - sel_window_pass2_scan: the threshold T and krem within T's keys.
template <int NW, int C, int W>
__device__ __forceinline__ bool sel_window_pass1(const uint32_t (&w)[W], uint32_t k, uint32_t* hist,
                                                 int& kb, uint32_t& krem) {
  constexpr int kPitch = sel_copy_pitch<C>();
  constexpr int kPitch16 = sel_copy_pitch16<C>();
  constexpr int kHist = C * kPitch;
  uint32_t* tab = hist + kHist;
  uint32_t* hist16 = tab + NW;
  const int t = static_cast<int>(threadIdx.x), lane = t & 63, wave = t >> 6;
  uint32_t* mine = hist + (lane % C) * kPitch;
  const uint32_t spare = kSelBins + lane / C;
  for (int i = t; i < kHist; i += 64 * NW) hist[i] = 0;
  for (int i = t; i < C * kPitch16; i += 64 * NW) hist16[i] = 0;
  sel_u16x2 m2 = {0, 0};
#pragma unroll
  for (int j = 0; j < W; ++j) m2 = __builtin_elementwise_max(m2, __builtin_bit_cast(sel_u16x2, w[j]));
  const uint32_t wmax = sel_wave_max(max(static_cast<uint32_t>(m2.x), static_cast<uint32_t>(m2.y)));
  if (lane == 0) tab[wave] = wmax;
  __syncthreads();
  uint32_t hi = tab[0];
#pragma unroll
  for (int q = 1; q < NW; ++q) hi = max(hi, tab[q]);
  // the lowest real key is 0x80; padding keys (0) fall below the window
  const int lo = max(static_cast<int>(hi) - 4095, 1);
#pragma unroll
  for (int j = 0; j < W; ++j) {
    const uint32_t b0 = min(static_cast<uint32_t>(static_cast<int>(w[j] & 0xFFFFu) - lo) >> 4, spare);
    const uint32_t b1 = min(static_cast<uint32_t>(static_cast<int>(w[j] >> 16) - lo) >> 4, spare);
    __hip_atomic_fetch_add(&mine[b0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    __hip_atomic_fetch_add(&mine[b1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  __syncthreads();
  uint32_t pb, gt;
  if (!sel_scan_bins4<C>(hist, lane, k, pb, gt)) return false;
  krem = k - gt;
  kb = lo + 16 * static_cast<int>(pb);
  return true;
}

template <int NW, int C, int W>
__device__ __forceinline__ void sel_window_pass2_count(const uint32_t (&w)[W], int kb, uint32_t* hist) {
  constexpr int kPitch16 = sel_copy_pitch16<C>();
  uint32_t* mine16 = hist + C * sel_copy_pitch<C>() + NW + (threadIdx.x % C) * kPitch16;
#pragma unroll
  for (int j = 0; j < W; ++j) {
    const uint32_t d0 = static_cast<uint32_t>(static_cast<int>(w[j] & 0xFFFFu) - kb);
    const uint32_t d1 = static_cast<uint32_t>(static_cast<int>(w[j] >> 16) - kb);
    if (d0 < 16u) __hip_atomic_fetch_add(&mine16[d0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (d1 < 16u) __hip_atomic_fetch_add(&mine16[d1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
}

template <int NW, int C>
__device__ __forceinline__ void sel_window_pass2_scan(const uint32_t* hist, int kb, uint32_t& thr,
                                                      uint32_t& krem) {
  constexpr int kPitch16 = sel_copy_pitch16<C>();
  const uint32_t* hist16 = hist + C * sel_copy_pitch<C>() + NW;
  const int lane = threadIdx.x & 63;
  // lane l < 16 holds key kb + 15 - l; the krem-th largest of the bin's keys
  uint32_t s = 0;
  if (lane < 16) {
#pragma unroll
    for (int c = 0; c < C; ++c) s += hist16[c * kPitch16 + 15 - lane];
  }
  const uint32_t incl = wave_inclusive_scan(s);
  const unsigned long long hits = __ballot(lane < 16 && incl >= krem);
  const int src = __ffsll(hits) - 1;  // the bin holds krem of its keys
  thr = static_cast<uint32_t>(kb + 15 - src);
  krem -= wave_read_lane(incl - s, src);
}

template <int NW, int C, int W>
__device__ __forceinline__ bool select_threshold_window_group(const uint32_t (&w)[W], uint32_t k,
                                                              uint32_t* hist, uint32_t& thr,
                                                              uint32_t& krem) {
  int kb;
  if (!sel_window_pass1<NW, C, W>(w, k, hist, kb, krem)) return false;
  sel_window_pass2_count<NW, C, W>(w, kb, hist);
  __syncthreads();
  sel_window_pass2_scan<NW, C>(hist, kb, thr, krem);
  return true;
}

// The MSB-first radix passes alone (no window).
template <int NW, int C, int W, int KEY_BITS>
__device__ __forceinline__ void select_threshold_bytes(const uint32_t (&w)[W], uint32_t k,
                                                       uint32_t* hist, uint32_t& thr, uint32_t& krem) {
  static_assert(C == 4 || C == 8 || C == 16, "4, 8 or 16 histogram copies");
  constexpr int kPitch = sel_copy_pitch<C>();
  constexpr int kHist = C * kPitch;
  const int t = (NW > 1) ? static_cast<int>(threadIdx.x) : static_cast<int>(threadIdx.x & 63);
  const int lane = t & 63;
  uint32_t* mine = hist + (lane % C) * kPitch;
  const uint32_t spare = kSelBins + lane / C;  // this lane's spare bin in its copy
  auto group_sync = [] {
    if constexpr (NW > 1) __syncthreads(); else __builtin_amdgcn_wave_barrier();
  };
  uint32_t prefix = 0;
  krem = k;
#pragma unroll
  for (int pass = 0; pass < KEY_BITS / 8; ++pass) {
    const int shift = KEY_BITS - 8 * (pass + 1);
    const uint32_t phi = (pass == 0) ? 0u : prefix >> (shift + 8);
    if (pass > 0) group_sync();  // every wave is done reading the last counts
    for (int i = t; i < kHist; i += 64 * NW) hist[i] = 0;
    group_sync();
    auto bump = [&](uint32_t bin) {
      __hip_atomic_fetch_add(&mine[bin], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    };
#pragma unroll
    for (int j = 0; j < W; ++j) {
      if constexpr (KEY_BITS == 16) {
        if (pass == 0) {
          // padding channels (key 0) are never counted: they would all hit
          // bin 0 of their copy at once (a serialised atomic per lane), and
          // bin 0 holds no real key
          if ((w[j] & 0xFFFFu) != 0u) bump((w[j] >> 8) & 0xFFu);
          if ((w[j] >> 16) != 0u) bump(w[j] >> 24);
        } else {
          // (key - phi:00) per half; off-prefix keys land at >= 256 -> spare
          const sel_u16x2 x = __builtin_elementwise_min(
              __builtin_bit_cast(sel_u16x2, w[j]) - static_cast<unsigned short>(phi << 8),
              sel_u16x2{static_cast<unsigned short>(spare), static_cast<unsigned short>(spare)});
          bump(x.x);
          bump(x.y);
        }
      } else {
        const uint32_t x = (w[j] >> shift) - (phi << 8);
        bump(pass == 0 ? x : min(x, spare));
      }
    }
    group_sync();
    uint32_t pb = 0, gt = 0;
    sel_scan_bins<C>(hist, lane, krem, pb, gt);  // the keys counted include the krem-th
    krem -= gt;
    prefix |= pb << shift;
  }
  thr = prefix;
}

template <int NW, int C, int W, int KEY_BITS>
__device__ __forceinline__ void select_threshold(const uint32_t (&w)[W], uint32_t k,
                                                 uint32_t* hist, uint32_t& thr, uint32_t& krem) {
  if constexpr (NW == 1 && KEY_BITS == 16) {
    if (select_threshold_window<C, W>(w, k, hist, thr, krem)) return;
    __builtin_amdgcn_wave_barrier();
  }
  if constexpr (NW > 1 && KEY_BITS == 16) {
    if (select_threshold_window_group<NW, C, W>(w, k, hist, thr, krem)) return;
    __syncthreads();  // every wave is done reading the window's counts
  }
  select_threshold_bytes<NW, C, W, KEY_BITS>(w, k, hist, thr, krem);
}

// take[d] bit i: channel c0 + 32 d + i is selected; first: rank of the
// thread's first selected channel.  With NW > 1 this uses the table behind
// the histograms and one workgroup barrier.
template <int NW, int C, int L, bool BF16>
__device__ __forceinline__ void select_ranks(const uint32_t (&w)[sel_words<BF16, L>()],
                                             uint32_t thr, uint32_t krem, uint32_t* lds,
                                             uint32_t (&take)[(L + 31) / 32], uint32_t& first) {
  constexpr int D = (L + 31) / 32;
  uint32_t eqb[D];
#pragma unroll
  for (int d = 0; d < D; ++d) take[d] = eqb[d] = 0;
#pragma unroll
  for (int i = 0; i < L; ++i) {
    const uint32_t key = BF16 ? ((w[i / 2] >> (16 * (i & 1))) & 0xFFFFu) : w[i];
    take[i / 32] |= (key > thr ? 1u : 0u) << (i % 32);
    eqb[i / 32] |= (key == thr ? 1u : 0u) << (i % 32);
  }
  uint32_t cgt = 0, ceq = 0;
#pragma unroll
  for (int d = 0; d < D; ++d) {
    cgt += __popc(take[d]);
    ceq += __popc(eqb[d]);
  }
  // one scan of the packed pair (group totals stay below 2^16)
  const uint32_t v = (cgt << 16) | ceq;
  const uint32_t incl = wave_inclusive_scan(v);
  uint32_t ex = incl - v;
  if constexpr (NW > 1) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t* tab = lds + C * sel_copy_pitch<C>();
    if (lane == 63) tab[wave] = incl;
    __syncthreads();
    for (int q = 0; q < wave; ++q) ex += tab[q];
  }
  const uint32_t gt_before = ex >> 16, eq_before = ex & 0xFFFFu;
  first = gt_before + min(krem, eq_before);
  uint32_t allow = krem > eq_before ? krem - eq_before : 0u;
  // the lowest-index `allow` T-valued channels of this thread
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const uint32_t n = __popc(eqb[d]);
    if (allow >= n) {
      take[d] |= eqb[d];
      allow -= n;
    } else {
      uint32_t e = eqb[d];
      for (uint32_t q = 0; q < allow; ++q) {
        take[d] |= e & (0u - e);
        e &= e - 1u;
      }
      allow = 0;
    }
  }
}

// Calls on_sel(channel, rank) for every selected channel of the thread, in
// channel order.
template <int L, typename OnSel>
__device__ __forceinline__ void select_emit(const uint32_t (&take)[(L + 31) / 32], int c0,
                                            uint32_t first, OnSel&& on_sel) {
  uint32_t pos = first;
#pragma unroll
  for (int d = 0; d < (L + 31) / 32; ++d) {
    uint32_t bits = take[d];
    while (bits) {
      const int i = __ffs(bits) - 1;
      on_sel(c0 + 32 * d + i, pos);
      ++pos;
      bits &= bits - 1u;
    }
  }
}

}  // namespace moc

// Shared MFMA GEMM building blocks for gfx950: the 128-row x 64-k operand
// tile that is staged global -> registers -> LDS (K-contiguous in LDS, row
// pitch kPitch bf16).  Used by the GEMM engine and by the fused 2:8 gate/up
// kernel.
#pragma once

#include "common.h"

namespace moc {
namespace tile {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kBM = 128, kBN = 128, kBK = 64, kPitch = 72, kThreads = 256;



// One operand tile of 128 rows (M or N) x 64 k, staged through registers.
template <bool KC>
struct TileLoader {
  uint4 r[4];

  // rows: extent of the M/N dimension, K: extent of k, (row0, k0): tile origin
  __device__ __forceinline__ void load(const uint16_t* __restrict__ p, int64_t ld, int rows, int K,
                                       int row0, int k0, int tid) {
    if (KC) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int v = tid + kThreads * i;
        const int gr = row0 + (v >> 3);
        const int gk = k0 + (v & 7) * 8;
        if (gr < rows && gk + 8 <= K) {
          r[i] = *reinterpret_cast<const uint4*>(p + static_cast<int64_t>(gr) * ld + gk);
        } else {
          uint16_t e[8];
#pragma unroll
          for (int j = 0; j < 8; ++j)
            e[j] = (gr < rows && gk + j < K) ? p[static_cast<int64_t>(gr) * ld + gk + j] : 0;
          r[i] = make_uint4(e[0] | (uint32_t(e[1]) << 16), e[2] | (uint32_t(e[3]) << 16),
                            e[4] | (uint32_t(e[5]) << 16), e[6] | (uint32_t(e[7]) << 16));
        }
      }
    } else {
      const int kq = tid & 15;   // which 4 k's
      const int mch = tid >> 4;  // which 8 rows
      const int gm = row0 + mch * 8;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int gk = k0 + kq * 4 + i;
        if (gk < K && gm + 8 <= rows) {
          r[i] = *reinterpret_cast<const uint4*>(p + static_cast<int64_t>(gk) * ld + gm);
        } else {
          uint16_t e[8];
#pragma unroll
          for (int j = 0; j < 8; ++j)
            e[j] = (gk < K && gm + j < rows) ? p[static_cast<int64_t>(gk) * ld + gm + j] : 0;
          r[i] = make_uint4(e[0] | (uint32_t(e[1]) << 16), e[2] | (uint32_t(e[3]) << 16),
                            e[4] | (uint32_t(e[5]) << 16), e[6] | (uint32_t(e[7]) << 16));
        }
      }
    }
  }

  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = make_uint4(0, 0, 0, 0);
  }

  __device__ __forceinline__ void store(uint16_t* __restrict__ lds, int tid) const {
    if (KC) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int v = tid + kThreads * i;
        *reinterpret_cast<uint4*>(lds + (v >> 3) * kPitch + (v & 7) * 8) = r[i];
      }
    } else {
      const int kq = tid & 15;
      const int mch = tid >> 4;
      // r[i] holds rows mch*8..+8 at k = kq*4+i; emit row-major 4-k runs.
      const uint32_t w[4][4] = {{r[0].x, r[0].y, r[0].z, r[0].w},
                                {r[1].x, r[1].y, r[1].z, r[1].w},
                                {r[2].x, r[2].y, r[2].z, r[2].w},
                                {r[3].x, r[3].y, r[3].z, r[3].w}};
#pragma unroll
      for (int mm = 0; mm < 8; ++mm) {
        const int pidx = mm >> 1;
        const int sh = (mm & 1) * 16;
        uint2 o;
        o.x = ((w[0][pidx] >> sh) & 0xFFFFu) | (((w[1][pidx] >> sh) & 0xFFFFu) << 16);
        o.y = ((w[2][pidx] >> sh) & 0xFFFFu) | (((w[3][pidx] >> sh) & 0xFFFFu) << 16);
        *reinterpret_cast<uint2*>(lds + (mch * 8 + mm) * kPitch + kq * 4) = o;
      }
    }
  }
};

}  // namespace tile
}  // namespace moc

// MFMA GEMM engine for the MoC FFN on gfx950.
//
//   C[M,N] = sum_k A(m,k) B(k,n)  [+ sum_k A2(m,k) B2(k,n)]
//
// The reference runs its nine FFN GEMMs through torch/cuBLAS
// (moc/ffn.py:141,146,163,203-254,389,394,414,447-494); here they run on the
// CDNA4 matrix cores through v_mfma_f32_32x32x16_bf16 with f32 accumulation.
// The optional second product lets dX = gG*W_gate + gU*W_up (moc/ffn.py:486,
// 491-494) accumulate in one pass instead of a GEMM plus an addmm.
//
// Operand layouts: each operand is either K-contiguous ("KC", A(m,k) at
// A[m*lda + k], B(k,n) at B[n*ldb + k]) or MN-contiguous (A(m,k) at
// A[k*lda + m], B(k,n) at B[k*ldb + n]).  Both land in LDS K-contiguous so
// one MFMA fragment is one 16-byte ds_read.  MN-contiguous tiles are
// transposed in registers on their way to LDS (8x4 blocks per thread).
//
// Tiling: 128x128 C tile per 256-thread workgroup (four waves of 64x64, each
// 2x2 MFMA 32x32 blocks), K step 64, LDS double buffer with one barrier per
// step; the next tile's global loads are in flight during the MFMAs.
// LDS row pitch is 72 bf16 (36 dwords): with the lane mappings below the
// fragment reads and both kinds of LDS stores are free of bank conflicts.
//
// f32 operands use a plain FMA kernel (parity path for f32 models).
#include "abi.h"
#include "common.h"
#include "gemm_tile.h"

namespace moc {
namespace {

using namespace tile;

struct GemmArgs {
  int M, N;
  int K1, K2;
  const uint16_t* A1;
  const uint16_t* B1;
  const uint16_t* A2;
  const uint16_t* B2;
  int64_t lda1, ldb1, lda2, ldb2;  // the non-unit stride of each operand
  void* C;
  int64_t ldc;
};

template <bool A_KC, bool B_KC, bool OUT_F32>
__global__ __launch_bounds__(kThreads) void gemm_bf16_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][kBM * kPitch];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][kBN * kPitch];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int row0 = blockIdx.y * kBM;
  const int col0 = blockIdx.x * kBN;
  const int wm = (wave >> 1) * 64;
  const int wn = (wave & 1) * 64;

  const int nk1 = (g.K1 + kBK - 1) / kBK;
  const int nk2 = (g.A2 != nullptr) ? (g.K2 + kBK - 1) / kBK : 0;
  const int nk = nk1 + nk2;

  TileLoader<A_KC> la;
  TileLoader<B_KC> lb;
  auto load = [&](int t) {
    if (t < nk1) {
      la.load(g.A1, g.lda1, g.M, g.K1, row0, t * kBK, tid);
      lb.load(g.B1, g.ldb1, g.N, g.K1, col0, t * kBK, tid);
    } else {
      const int k0 = (t - nk1) * kBK;
      la.load(g.A2, g.lda2, g.M, g.K2, row0, k0, tid);
      lb.load(g.B2, g.ldb2, g.N, g.K2, col0, k0, tid);
    }
  };

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  if (nk > 0) {
    load(0);
    la.store(As[0], tid);
    lb.store(Bs[0], tid);
  }
  __syncthreads();

  const int frow = lane & 31;
  const int fk = (lane >> 5) * 8;
  for (int t = 0; t < nk; ++t) {
    const int cur = t & 1;
    if (t + 1 < nk) load(t + 1);
    const uint16_t* as = As[cur];
    const uint16_t* bs = Bs[cur];
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      bf16x8_t a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const uint4 va =
            *reinterpret_cast<const uint4*>(as + (wm + 32 * i + frow) * kPitch + ks * 16 + fk);
        a[i] = __builtin_bit_cast(bf16x8_t, va);
        const uint4 vb =
            *reinterpret_cast<const uint4*>(bs + (wn + 32 * i + frow) * kPitch + ks * 16 + fk);
        b[i] = __builtin_bit_cast(bf16x8_t, vb);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (t + 1 < nk) {
      la.store(As[cur ^ 1], tid);
      lb.store(Bs[cur ^ 1], tid);
    }
    __syncthreads();
  }

  // 32x32 accumulator layout: lane l, element r -> row 8*(r/4) + 4*(l/32) + r%4, col l%32
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = col0 + wn + 32 * j + (lane & 31);
      if (col >= g.N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = row0 + wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row < g.M) {
          if (OUT_F32)
            static_cast<float*>(g.C)[static_cast<int64_t>(row) * g.ldc + col] = acc[i][j][r];
          else
            static_cast<uint16_t*>(g.C)[static_cast<int64_t>(row) * g.ldc + col] =
                f32_to_bf16(acc[i][j][r]);
        }
      }
    }
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
  const dim3 grid((a.N + kBN - 1) / kBN, (a.M + kBM - 1) / kBM), block(kThreads);
  if (out_f32)
    gemm_bf16_kernel<A_KC, B_KC, true><<<grid, block, 0, st>>>(a);
  else
    gemm_bf16_kernel<A_KC, B_KC, false><<<grid, block, 0, st>>>(a);
}

// Returns +1 for K-contiguous, 0 for MN-contiguous, -1 if neither.
int layout_of(int64_t s_mn, int64_t s_k, int64_t mn, int64_t k) {
  if (s_k == 1 || k <= 1) return 1;
  if (s_mn == 1 || mn <= 1) return 0;
  return -1;
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
  int64_t lda2 = 0, ldb2 = 0;
  if (second) {
    const int la2 = layout_of(a2_sm, a2_sk, M, K2);
    const int lb2 = layout_of(b2_sn, b2_sk, N, K2);
    MOC_REQUIRE(la2 == la && lb2 == lb, "moc_gemm: second product must share the operand layouts");
    lda2 = la2 ? a2_sm : a2_sk;
    ldb2 = lb2 ? b2_sn : b2_sk;
    MOC_REQUIRE(aligned16(A2) && aligned16(B2), "moc_gemm: bf16 operands must be 16-byte aligned");
    MOC_REQUIRE(lda2 % 8 == 0 && ldb2 % 8 == 0, "moc_gemm: bf16 leading dimensions must be multiples of 8");
  }
  MOC_REQUIRE((M + kBM - 1) / kBM <= 65535, "moc_gemm: M too large");
  GemmArgs a{(int)M, (int)N, (int)K, second ? (int)K2 : 0, (const uint16_t*)A, (const uint16_t*)B,
             second ? (const uint16_t*)A2 : nullptr, second ? (const uint16_t*)B2 : nullptr,
             lda, ldb, lda2, ldb2, C, ldc};
  const bool of = c_dtype == MOC_F32;
  if (la && lb) launch_bf16<true, true>(a, of, st);
  else if (la && !lb) launch_bf16<true, false>(a, of, st);
  else if (!la && lb) launch_bf16<false, true>(a, of, st);
  else launch_bf16<false, false>(a, of, st);
  return check_launch("gemm_bf16_kernel");
}

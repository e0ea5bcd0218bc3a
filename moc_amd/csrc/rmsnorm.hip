// The FFN's pre-norm as row kernels (gfx950): the RMSNorm of the decoder
// block that feeds the MoC FFN (moc/model.py:20-28, used at :83-86 as
// x + ffn(ffn_norm(x))), forward and backward, for bf16 activations.
//
//   forward   y = bf16(bf16(x * r) * w),  r = 1 / sqrt(mean(x^2) + eps)  (f32)
//             (the rounding points of (x.float() * r).to(bf16) * weight)
//   backward  with dy the gradient of y and dres a gradient that reaches x
//             around the norm (the block's residual branch):
//             dx = dres + r * (dy * w) - (r^3 / d) * x * sum_j(dy_j w_j x_j)
//             dw = sum over rows of dy * bf16(x * r)
//             summed in f32 and rounded once (the reference's autograd rounds
//             its two bf16 branch gradients and their sum; within 1-2 ulp).
//
// One wave per row: lane l holds 16-byte chunks l, l + 64, ... of the row in
// registers, so a row is read once per pass and its sums are one DPP wave
// reduction.  The backward keeps each wave's dw contribution for its lane's
// columns in registers across the rows it handles, adds the four waves of a
// workgroup through LDS and writes one f32 partial row per workgroup; a
// second kernel sums the partial rows column by column in a fixed order, so
// dw does not depend on timing.  HBM-bound: the forward moves 2 d bytes
// in and 2 d + 4 bytes out per row, the backward 6 d in and 2 d out.
#include <algorithm>

#include "abi.h"
#include "common.h"

namespace moc {
namespace {

constexpr int kRmsWaves = 4;     // waves (rows in flight) per workgroup
constexpr int kRmsMaxBlocks = 512;  // workgroups of the backward (partial dw rows)

__device__ __forceinline__ float lo16(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi16(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return static_cast<uint32_t>(bf16_rne(lo)) | (static_cast<uint32_t>(bf16_rne(hi)) << 16);
}

// NC: 16-byte chunks per lane (d <= 512 NC); chunk c = lane + 64 i, valid
// while c < d / 8.
template <int NC>
__global__ __launch_bounds__(64 * kRmsWaves) void rmsnorm_rows_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int rows, int d, const uint16_t* __restrict__ w, float eps,
    uint16_t* __restrict__ y, int64_t ldy, float* __restrict__ rstd) {
  const int lane = threadIdx.x & 63;
  const int nchunk = d >> 3;
  uint4 wv[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = lane + 64 * i;
    wv[i] = c < nchunk ? *reinterpret_cast<const uint4*>(w + 8 * c) : make_uint4(0, 0, 0, 0);
  }
  const int waves = gridDim.x * kRmsWaves;
  for (int row = blockIdx.x * kRmsWaves + (threadIdx.x >> 6); row < rows; row += waves) {
    const uint16_t* xr = x + static_cast<int64_t>(row) * ldx;
    uint4 xv[NC];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = lane + 64 * i;
      xv[i] = c < nchunk ? *reinterpret_cast<const uint4*>(xr + 8 * c) : make_uint4(0, 0, 0, 0);
      const uint32_t e[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        ss = fmaf(lo16(e[q]), lo16(e[q]), ss);
        ss = fmaf(hi16(e[q]), hi16(e[q]), ss);
      }
    }
    ss = wave_sum(ss);
    const float r = 1.0f / sqrtf(ss / static_cast<float>(d) + eps);
    uint16_t* yr = y + static_cast<int64_t>(row) * ldy;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = lane + 64 * i;
      if (c < nchunk) *reinterpret_cast<uint4*>(yr + 8 * c) = rmsnorm8(xv[i], wv[i], r);
    }
    if (lane == 0 && rstd != nullptr) rstd[row] = r;
  }
}

template <int NC>
__global__ __launch_bounds__(64 * kRmsWaves) void rmsnorm_bwd_rows_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int rows, int d, const uint16_t* __restrict__ w,
    const float* __restrict__ rstd, const uint16_t* __restrict__ dy, int64_t lddy,
    const uint16_t* __restrict__ dres, int64_t ldres, uint16_t* __restrict__ dx, int64_t lddx,
    float* __restrict__ dw_part) {
  __shared__ float red[kRmsWaves][64 * 8];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nchunk = d >> 3;
  uint4 wv[NC];
  float dwa[NC][8];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = lane + 64 * i;
    wv[i] = c < nchunk ? *reinterpret_cast<const uint4*>(w + 8 * c) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int q = 0; q < 8; ++q) dwa[i][q] = 0.f;
  }
  const float inv_d = 1.0f / static_cast<float>(d);
  const int waves = gridDim.x * kRmsWaves;
  for (int row = blockIdx.x * kRmsWaves + wave; row < rows; row += waves) {
    const uint16_t* xr = x + static_cast<int64_t>(row) * ldx;
    const uint16_t* gr = dy + static_cast<int64_t>(row) * lddy;
    const float r = rstd[row];
    uint4 xv[NC], gv[NC];
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = lane + 64 * i;
      const bool ok = c < nchunk;
      xv[i] = ok ? *reinterpret_cast<const uint4*>(xr + 8 * c) : make_uint4(0, 0, 0, 0);
      gv[i] = ok ? *reinterpret_cast<const uint4*>(gr + 8 * c) : make_uint4(0, 0, 0, 0);
      const uint32_t xe[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
      const uint32_t ge[4] = {gv[i].x, gv[i].y, gv[i].z, gv[i].w};
      const uint32_t we[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        s = fmaf(lo16(ge[q]) * lo16(we[q]), lo16(xe[q]), s);
        s = fmaf(hi16(ge[q]) * hi16(we[q]), hi16(xe[q]), s);
        // dw: dy times the forward's first rounding point bf16(x * r)
        dwa[i][2 * q] = fmaf(lo16(ge[q]), round_bf16(lo16(xe[q]) * r), dwa[i][2 * q]);
        dwa[i][2 * q + 1] = fmaf(hi16(ge[q]), round_bf16(hi16(xe[q]) * r), dwa[i][2 * q + 1]);
      }
    }
    s = wave_sum(s);
    const float c3 = s * r * r * r * inv_d;
    const uint16_t* rr = dres != nullptr ? dres + static_cast<int64_t>(row) * ldres : nullptr;
    uint16_t* dr = dx + static_cast<int64_t>(row) * lddx;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = lane + 64 * i;
      if (c >= nchunk) continue;
      const uint4 rv = rr != nullptr ? *reinterpret_cast<const uint4*>(rr + 8 * c) : make_uint4(0, 0, 0, 0);
      const uint32_t xe[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
      const uint32_t ge[4] = {gv[i].x, gv[i].y, gv[i].z, gv[i].w};
      const uint32_t we[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
      const uint32_t re[4] = {rv.x, rv.y, rv.z, rv.w};
      uint32_t o[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float lo = lo16(re[q]) + (r * (lo16(ge[q]) * lo16(we[q])) - c3 * lo16(xe[q]));
        const float hi = hi16(re[q]) + (r * (hi16(ge[q]) * hi16(we[q])) - c3 * hi16(xe[q]));
        o[q] = pack2(lo, hi);
      }
      *reinterpret_cast<uint4*>(dr + 8 * c) = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
  // the workgroup's dw partial row: waves summed in wave order through LDS,
  // chunk by chunk
#pragma unroll
  for (int i = 0; i < NC; ++i) {
#pragma unroll
    for (int q = 0; q < 8; ++q) red[wave][lane * 8 + q] = dwa[i][q];
    __syncthreads();
    // element e of the slice is column 8 (e / 8 + 64 i) + e % 8 = 512 i + e
    for (int e = threadIdx.x; e < 64 * 8; e += 64 * kRmsWaves) {
      const int col = 512 * i + e;
      if (col < d) {
        float t = red[0][e];
#pragma unroll
        for (int v = 1; v < kRmsWaves; ++v) t += red[v][e];
        dw_part[static_cast<int64_t>(blockIdx.x) * d + col] = t;
      }
    }
    __syncthreads();
  }
}

// dw[col] = sum over the partial rows, in w's dtype.  A workgroup of 16 waves
// takes 64 columns: wave w adds partial rows w, w + 16, ... for its lane's
// column (each step one coalesced 256-byte row segment; eight loads in
// flight), then the 16 wave sums are added in wave order through LDS, so
// the result is the same on every run.
constexpr int kDwWaves = 16;
template <bool OUT_F32>
__global__ __launch_bounds__(64 * kDwWaves) void rmsnorm_dw_reduce_kernel(const float* __restrict__ part,
                                                                          int nblocks, int d, void* __restrict__ dw) {
  __shared__ float red[kDwWaves][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = blockIdx.x * 64 + lane;
  float t[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (col < d) {
    int b = wave;
    for (; b + 7 * kDwWaves < nblocks; b += 8 * kDwWaves) {
#pragma unroll
      for (int u = 0; u < 8; ++u) t[u] += part[static_cast<int64_t>(b + u * kDwWaves) * d + col];
    }
    for (; b < nblocks; b += kDwWaves) t[0] += part[static_cast<int64_t>(b) * d + col];
  }
  red[wave][lane] = ((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]));
  __syncthreads();
  if (wave == 0 && col < d) {
    float s = red[0][lane];
#pragma unroll
    for (int v = 1; v < kDwWaves; ++v) s += red[v][lane];
    if (OUT_F32) static_cast<float*>(dw)[col] = s;
    else static_cast<uint16_t*>(dw)[col] = bf16_rne(s);
  }
}

int rms_blocks(int64_t rows) {
  return static_cast<int>(std::min<int64_t>((rows + kRmsWaves - 1) / kRmsWaves, kRmsMaxBlocks));
}

bool rows_ok(const void* p, int64_t ld, int64_t d) {
  return p != nullptr && aligned16(p) && ld % 8 == 0 && ld >= d;
}

}  // namespace
}  // namespace moc

using namespace moc;

extern "C" int moc_rmsnorm_rows_bf16(const void* x, int64_t ldx, int64_t rows, int64_t d, const void* w,
                                     float eps, void* y, int64_t ldy, float* rstd, void* stream) {
  MOC_REQUIRE(rows >= 0 && rows < (1LL << 31), "moc_rmsnorm_rows_bf16: bad row count");
  MOC_REQUIRE(d >= 8 && d % 8 == 0 && d <= 8192, "moc_rmsnorm_rows_bf16: hidden must be a multiple of 8 in [8, 8192]");
  MOC_REQUIRE(eps >= 0.f, "moc_rmsnorm_rows_bf16: eps must be >= 0");
  if (rows == 0) return MOC_OK;
  MOC_REQUIRE(rows_ok(x, ldx, d) && rows_ok(y, ldy, d) && w != nullptr && aligned16(w),
              "moc_rmsnorm_rows_bf16: x, y and w need 16-byte aligned rows (leading dimensions multiples of 8)");
  const int blocks = static_cast<int>(std::min<int64_t>((rows + kRmsWaves - 1) / kRmsWaves, 8 * cu_count()));
  const auto* xp = static_cast<const uint16_t*>(x);
  const auto* wp = static_cast<const uint16_t*>(w);
  auto* yp = static_cast<uint16_t*>(y);
  hipStream_t st = as_stream(stream);
  const int nc = static_cast<int>((d / 8 + 63) / 64);
#define MOC_RMS_FWD(NC) \
  rmsnorm_rows_kernel<NC><<<blocks, 64 * kRmsWaves, 0, st>>>(xp, ldx, (int)rows, (int)d, wp, eps, yp, ldy, rstd)
  if (nc <= 1) MOC_RMS_FWD(1);
  else if (nc <= 2) MOC_RMS_FWD(2);
  else if (nc <= 4) MOC_RMS_FWD(4);
  else if (nc <= 8) MOC_RMS_FWD(8);
  else MOC_RMS_FWD(16);
#undef MOC_RMS_FWD
  return check_launch("rmsnorm_rows_kernel");
}

extern "C" int64_t moc_rmsnorm_backward_workspace_size(int64_t rows, int64_t d) {
  if (rows <= 0 || d <= 0) return 0;
  return (static_cast<int64_t>(rms_blocks(rows)) * d * 4 + 255) / 256 * 256;
}

extern "C" int moc_rmsnorm_backward_bf16(const void* x, int64_t ldx, int64_t rows, int64_t d, const void* w,
                                         const float* rstd, const void* dy, int64_t lddy, const void* dres,
                                         int64_t ldres, void* dx, int64_t lddx, void* dw, int dw_dtype,
                                         void* workspace, int64_t workspace_bytes, void* stream) {
  MOC_REQUIRE(rows >= 0 && rows < (1LL << 31), "moc_rmsnorm_backward_bf16: bad row count");
  MOC_REQUIRE(d >= 8 && d % 8 == 0 && d <= 4096,
              "moc_rmsnorm_backward_bf16: hidden must be a multiple of 8 in [8, 4096]");
  MOC_REQUIRE(dw_dtype == MOC_BF16 || dw_dtype == MOC_F32, "moc_rmsnorm_backward_bf16: dw dtype bf16 or f32");
  MOC_REQUIRE(dw != nullptr && w != nullptr && aligned16(w), "moc_rmsnorm_backward_bf16: null or unaligned w/dw");
  if (rows == 0) {
    return moc_fill_zero(dw, d * (dw_dtype == MOC_F32 ? 4 : 2), stream);
  }
  MOC_REQUIRE(rows_ok(x, ldx, d) && rows_ok(dy, lddy, d) && rows_ok(dx, lddx, d) &&
                  (dres == nullptr || rows_ok(dres, ldres, d)) && rstd != nullptr,
              "moc_rmsnorm_backward_bf16: x, dy, dres and dx need 16-byte aligned rows (leading dimensions "
              "multiples of 8)");
  const int64_t need = moc_rmsnorm_backward_workspace_size(rows, d);
  MOC_REQUIRE(workspace != nullptr && workspace_bytes >= need && aligned16(workspace),
              "moc_rmsnorm_backward_bf16: workspace of %lld bytes required", (long long)need);
  const int blocks = rms_blocks(rows);
  auto* part = static_cast<float*>(workspace);
  hipStream_t st = as_stream(stream);
  const int nc = static_cast<int>((d / 8 + 63) / 64);
  const auto* xp = static_cast<const uint16_t*>(x);
  const auto* wp = static_cast<const uint16_t*>(w);
  const auto* gp = static_cast<const uint16_t*>(dy);
  const auto* rp = static_cast<const uint16_t*>(dres);
  auto* op = static_cast<uint16_t*>(dx);
#define MOC_RMS_BWD(NC)                                                                                   \
  rmsnorm_bwd_rows_kernel<NC><<<blocks, 64 * kRmsWaves, 0, st>>>(xp, ldx, (int)rows, (int)d, wp, rstd, gp, \
                                                                 lddy, rp, ldres, op, lddx, part)
  if (nc <= 1) MOC_RMS_BWD(1);
  else if (nc <= 2) MOC_RMS_BWD(2);
  else if (nc <= 4) MOC_RMS_BWD(4);
  else MOC_RMS_BWD(8);
#undef MOC_RMS_BWD
  int rc = check_launch("rmsnorm_bwd_rows_kernel");
  if (rc != MOC_OK) return rc;
  const dim3 grid(static_cast<unsigned>((d + 63) / 64));
  if (dw_dtype == MOC_F32) rmsnorm_dw_reduce_kernel<true><<<grid, 64 * kDwWaves, 0, st>>>(part, blocks, (int)d, dw);
  else rmsnorm_dw_reduce_kernel<false><<<grid, 64 * kDwWaves, 0, st>>>(part, blocks, (int)d, dw);
  return check_launch("rmsnorm_dw_reduce_kernel");
}

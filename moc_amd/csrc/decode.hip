// Global-MoC decode kernels (gfx950): a handful of tokens (nb <= 16) through
// one MoC FFN layer.  Every kernel here is bound by HBM bandwidth: the gate
// projection streams all of W_gate, the selected Up/Down kernels stream only
// the K selected rows of W_up and W_down^T.
//
//  moc_gemv_bf16              gate projection G = x W_gate^T on MFMA 16x16x32
//                             (tokens are the N dimension, zero-padded to 16)
//  moc_selected_up_silu_bf16  one wave per (token, selected channel)
//  moc_selected_down_bf16     split-K over selected rows + fixed-order reduce
//  moc_global_after_gate_bf16 Top-K -> selected Up -> selected Down
//
// Reference: moc/inference/cuda/optimized_global_moc_ext.cu:127-540 and the
// masked_reference oracle moc/inference/inference_ffn.py:169-180, whose
// rounding points (U, SiLU(G) and Z materialised in bf16) these kernels keep.
#include "abi.h"
#include "common.h"

extern "C" int moc_topk_rows(int dtype, const void* scores, int64_t rows, int64_t inter,
                             int64_t ld, int64_t k, int score_transform, void* vals_out,
                             void* idx_out, int idx_dtype, uint32_t* mask_out, int64_t mask_ld,
                             void* stream);

namespace moc {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float dot8(uint4 a, uint4 b, float acc) {
  const uint32_t aw[4] = {a.x, a.y, a.z, a.w};
  const uint32_t bw[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    acc = fmaf(__uint_as_float(aw[i] << 16), __uint_as_float(bw[i] << 16), acc);
    acc = fmaf(__uint_as_float(aw[i] & 0xFFFF0000u), __uint_as_float(bw[i] & 0xFFFF0000u), acc);
  }
  return acc;
}

template <typename IdxT>
__device__ __forceinline__ int64_t load_idx(const void* p, int64_t e) {
  return static_cast<int64_t>(static_cast<const IdxT*>(p)[e]);
}

// ---------------------------------------------------------------------------
// Gate GEMV: workgroup = 16 rows of W, four waves split the hidden dimension
// in interleaved 32-wide k steps, an LDS reduction joins the waves.
// ---------------------------------------------------------------------------
constexpr int kGemvUnroll = 8;

__global__ __launch_bounds__(256) void gemv16_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                     int nb, const uint16_t* __restrict__ W,
                                                     int64_t ldw, int rows, int hidden,
                                                     uint16_t* __restrict__ y, int64_t ldy) {
  __shared__ f32x4_t red[4][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r0 = blockIdx.x * 16;
  const int row = r0 + (lane & 15);
  const int tok = lane & 15;
  const int kq = (lane >> 4) * 8;
  const bool row_ok = row < rows;
  const bool tok_ok = tok < nb;
  const uint16_t* wrow = W + static_cast<int64_t>(row_ok ? row : 0) * ldw + kq;
  const uint16_t* xrow = x + static_cast<int64_t>(tok_ok ? tok : 0) * ldx + kq;
  const int nsteps = (hidden + 31) / 32;

  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = wave; s0 < nsteps; s0 += 4 * kGemvUnroll) {
    uint4 wv[kGemvUnroll], xv[kGemvUnroll];
#pragma unroll
    for (int u = 0; u < kGemvUnroll; ++u) {
      const int s = s0 + 4 * u;
      const int k = s * 32 + kq;
      const bool kin = s < nsteps && k < hidden;
      wv[u] = (kin && row_ok) ? *reinterpret_cast<const uint4*>(wrow + s * 32) : make_uint4(0, 0, 0, 0);
      xv[u] = (kin && tok_ok) ? *reinterpret_cast<const uint4*>(xrow + s * 32) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kGemvUnroll; ++u)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, wv[u]),
                                                    __builtin_bit_cast(bf16x8_t, xv[u]), acc, 0, 0, 0);
  }
  red[wave][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    f32x4_t t = red[0][lane];
#pragma unroll
    for (int w = 1; w < 4; ++w) {
      const f32x4_t o = red[w][lane];
      t[0] += o[0]; t[1] += o[1]; t[2] += o[2]; t[3] += o[3];
    }
    // 16x16 accumulator layout: lane l element j -> row 4*(l/16)+j, column l%16
    const int n = lane & 15;
    if (n < nb) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = r0 + 4 * (lane >> 4) + j;
        if (r < rows) y[static_cast<int64_t>(n) * ldy + r] = f32_to_bf16(t[j]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Selected Up * SiLU: one wave per (token, selected channel).
// ---------------------------------------------------------------------------
template <typename IdxT>
__global__ __launch_bounds__(256) void selected_up_silu_kernel(
    const uint16_t* __restrict__ x, int nb, int hidden, const uint16_t* __restrict__ vals,
    const void* __restrict__ idx, int k, const uint16_t* __restrict__ w_up, int inter,
    uint16_t* __restrict__ z) {
  const int64_t item = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (item >= static_cast<int64_t>(nb) * k) return;
  const int64_t b = item / k;
  int64_t ch = load_idx<IdxT>(idx, item);
  if (ch < 0 || ch >= inter) {  // malformed index: contributes nothing
    if (lane == 0) z[item] = 0;
    return;
  }
  const uint16_t* wr = w_up + ch * hidden;
  const uint16_t* xr = x + b * hidden;
  const int chunks = hidden / 8;
  float acc = 0.f;
  int c = lane;
  for (; c + 192 < chunks; c += 256) {
    uint4 w0 = *reinterpret_cast<const uint4*>(wr + c * 8);
    uint4 w1 = *reinterpret_cast<const uint4*>(wr + (c + 64) * 8);
    uint4 w2 = *reinterpret_cast<const uint4*>(wr + (c + 128) * 8);
    uint4 w3 = *reinterpret_cast<const uint4*>(wr + (c + 192) * 8);
    acc = dot8(w0, *reinterpret_cast<const uint4*>(xr + c * 8), acc);
    acc = dot8(w1, *reinterpret_cast<const uint4*>(xr + (c + 64) * 8), acc);
    acc = dot8(w2, *reinterpret_cast<const uint4*>(xr + (c + 128) * 8), acc);
    acc = dot8(w3, *reinterpret_cast<const uint4*>(xr + (c + 192) * 8), acc);
  }
  for (; c < chunks; c += 64)
    acc = dot8(*reinterpret_cast<const uint4*>(wr + c * 8), *reinterpret_cast<const uint4*>(xr + c * 8), acc);
  acc = wave_sum(acc);
  if (lane == 0) {
    const float u = round_bf16(acc);
    const float s = round_bf16(silu_f32(bf16_to_f32(vals[item])));
    z[item] = f32_to_bf16(s * u);
  }
}

// ---------------------------------------------------------------------------
// Selected Down, split over the k selected rows.  Workgroup (split, h-chunk,
// token): 4 waves stride over the split's rows, each lane owns 8 columns.
// Partials [splits, nb, hidden] f32 are summed in split order by a second
// kernel, so the result does not depend on scheduling.
// ---------------------------------------------------------------------------
struct DownPlan {
  int splits;
  int rows_per_split;
  int hchunks;
};

__host__ __device__ inline DownPlan down_plan(int64_t nb, int64_t k, int64_t hidden) {
  DownPlan p;
  p.hchunks = static_cast<int>((hidden + 511) / 512);
  const int64_t target = 512;  // workgroups to fill 256 CUs twice
  int64_t s = (target + p.hchunks * nb - 1) / (p.hchunks * nb);
  const int64_t smax = (k + 3) / 4;  // at least 4 rows (one per wave) per split
  if (s > smax) s = smax;
  if (s < 1) s = 1;
  p.rows_per_split = static_cast<int>((k + s - 1) / s);
  p.splits = static_cast<int>((k + p.rows_per_split - 1) / p.rows_per_split);
  return p;
}

template <typename IdxT>
__global__ __launch_bounds__(256) void selected_down_partial_kernel(
    const uint16_t* __restrict__ z, const void* __restrict__ idx, int k, int hidden,
    const uint16_t* __restrict__ wdt, int inter, int rows_per_split, int nb,
    float* __restrict__ part) {
  __shared__ float red[4][512];
  const int split = blockIdx.x;
  const int hc = blockIdx.y;
  const int b = blockIdx.z;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = hc * 512 + lane * 8;
  const bool col_ok = col < hidden;
  const int kbeg = split * rows_per_split;
  const int kend = min(k, kbeg + rows_per_split);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const int64_t zb = static_cast<int64_t>(b) * k;
  int kk = kbeg + wave;
  for (; kk + 4 < kend; kk += 8) {
    const int64_t r0 = load_idx<IdxT>(idx, zb + kk);
    const int64_t r1 = load_idx<IdxT>(idx, zb + kk + 4);
    const float z0 = bf16_to_f32(z[zb + kk]);
    const float z1 = bf16_to_f32(z[zb + kk + 4]);
    uint4 w0 = make_uint4(0, 0, 0, 0), w1 = make_uint4(0, 0, 0, 0);
    if (col_ok && r0 >= 0 && r0 < inter) w0 = *reinterpret_cast<const uint4*>(wdt + r0 * hidden + col);
    if (col_ok && r1 >= 0 && r1 < inter) w1 = *reinterpret_cast<const uint4*>(wdt + r1 * hidden + col);
    const uint32_t a0[4] = {w0.x, w0.y, w0.z, w0.w};
    const uint32_t a1[4] = {w1.x, w1.y, w1.z, w1.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] = fmaf(z0, __uint_as_float(a0[i] << 16), acc[2 * i]);
      acc[2 * i + 1] = fmaf(z0, __uint_as_float(a0[i] & 0xFFFF0000u), acc[2 * i + 1]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] = fmaf(z1, __uint_as_float(a1[i] << 16), acc[2 * i]);
      acc[2 * i + 1] = fmaf(z1, __uint_as_float(a1[i] & 0xFFFF0000u), acc[2 * i + 1]);
    }
  }
  for (; kk < kend; kk += 4) {
    const int64_t r0 = load_idx<IdxT>(idx, zb + kk);
    const float z0 = bf16_to_f32(z[zb + kk]);
    uint4 w0 = make_uint4(0, 0, 0, 0);
    if (col_ok && r0 >= 0 && r0 < inter) w0 = *reinterpret_cast<const uint4*>(wdt + r0 * hidden + col);
    const uint32_t a0[4] = {w0.x, w0.y, w0.z, w0.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] = fmaf(z0, __uint_as_float(a0[i] << 16), acc[2 * i]);
      acc[2 * i + 1] = fmaf(z0, __uint_as_float(a0[i] & 0xFFFF0000u), acc[2 * i + 1]);
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) red[wave][lane * 8 + i] = acc[i];
  __syncthreads();
  if (wave == 0 && col_ok) {
    float* dst = part + (static_cast<int64_t>(split) * nb + b) * hidden + col;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      dst[i] = ((red[0][lane * 8 + i] + red[1][lane * 8 + i]) + red[2][lane * 8 + i]) +
               red[3][lane * 8 + i];
  }
}

__global__ __launch_bounds__(256) void split_reduce_kernel(const float* __restrict__ part,
                                                           int splits, int64_t n,
                                                           uint16_t* __restrict__ y) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= n) return;
  float s = 0.f;
  for (int i = 0; i < splits; ++i) s += part[static_cast<int64_t>(i) * n + e];
  y[e] = f32_to_bf16(s);
}

bool idx_ok(int d) { return d == MOC_I16 || d == MOC_I32 || d == MOC_I64; }

int launch_selected_down(const void* z, const void* idx, int idx_dtype, int64_t nb, int64_t k,
                         const void* wdt, int64_t inter, int64_t hidden, void* y, void* ws,
                         hipStream_t st) {
  const DownPlan p = down_plan(nb, k, hidden);
  float* part = static_cast<float*>(ws);
  const dim3 grid(p.splits, p.hchunks, static_cast<unsigned>(nb)), block(256);
#define MOC_DOWN(T)                                                                         \
  selected_down_partial_kernel<T><<<grid, block, 0, st>>>(                                  \
      (const uint16_t*)z, idx, (int)k, (int)hidden, (const uint16_t*)wdt, (int)inter,       \
      p.rows_per_split, (int)nb, part)
  if (idx_dtype == MOC_I16) MOC_DOWN(int16_t);
  else if (idx_dtype == MOC_I32) MOC_DOWN(int32_t);
  else MOC_DOWN(int64_t);
#undef MOC_DOWN
  int rc = check_launch("selected_down_partial_kernel");
  if (rc != MOC_OK) return rc;
  const int64_t n = nb * hidden;
  split_reduce_kernel<<<dim3(static_cast<unsigned>((n + 255) / 256)), 256, 0, st>>>(
      part, p.splits, n, static_cast<uint16_t*>(y));
  return check_launch("split_reduce_kernel");
}

inline int64_t align256(int64_t b) { return (b + 255) & ~int64_t(255); }

}  // namespace
}  // namespace moc

using namespace moc;

extern "C" int moc_gemv_bf16(const void* x, int64_t ldx, int64_t nb, const void* W, int64_t ldw,
                             int64_t rows, int64_t hidden, void* y, int64_t ldy, void* stream) {
  MOC_REQUIRE(nb >= 0 && nb <= 16, "moc_gemv_bf16: 0 <= nb <= 16 tokens (got %lld)", (long long)nb);
  MOC_REQUIRE(rows >= 0 && hidden >= 1 && rows < (1LL << 31) && hidden < (1LL << 30),
              "moc_gemv_bf16: bad shape");
  MOC_REQUIRE(hidden % 8 == 0, "moc_gemv_bf16: hidden must be a multiple of 8");
  MOC_REQUIRE(ldx >= hidden && ldw >= hidden && ldy >= rows, "moc_gemv_bf16: bad leading dimension");
  MOC_REQUIRE(ldx % 8 == 0 && ldw % 8 == 0, "moc_gemv_bf16: ldx/ldw must be multiples of 8");
  if (nb == 0 || rows == 0) return MOC_OK;
  MOC_REQUIRE(x && W && y, "moc_gemv_bf16: null pointer");
  MOC_REQUIRE(aligned16(x) && aligned16(W), "moc_gemv_bf16: x and W must be 16-byte aligned");
  const dim3 grid(static_cast<unsigned>((rows + 15) / 16)), block(256);
  gemv16_kernel<<<grid, block, 0, as_stream(stream)>>>(
      (const uint16_t*)x, ldx, (int)nb, (const uint16_t*)W, ldw, (int)rows, (int)hidden,
      (uint16_t*)y, ldy);
  return check_launch("gemv16_kernel");
}

extern "C" int moc_selected_up_silu_bf16(const void* x, int64_t nb, int64_t hidden,
                                         const void* topk_vals, const void* idx, int idx_dtype,
                                         int64_t k, const void* w_up, int64_t inter, void* z,
                                         void* stream) {
  MOC_REQUIRE(idx_ok(idx_dtype), "moc_selected_up_silu_bf16: bad index dtype");
  MOC_REQUIRE(nb >= 0 && k >= 1 && inter >= 1 && hidden >= 1, "moc_selected_up_silu_bf16: bad shape");
  MOC_REQUIRE(hidden % 8 == 0, "moc_selected_up_silu_bf16: hidden must be a multiple of 8");
  MOC_REQUIRE(nb * k < (1LL << 31), "moc_selected_up_silu_bf16: too many items");
  if (nb == 0) return MOC_OK;
  MOC_REQUIRE(x && topk_vals && idx && w_up && z, "moc_selected_up_silu_bf16: null pointer");
  MOC_REQUIRE(aligned16(x) && aligned16(w_up), "moc_selected_up_silu_bf16: x/w_up must be 16-byte aligned");
  const int64_t items = nb * k;
  const dim3 grid(static_cast<unsigned>((items * 64 + 255) / 256)), block(256);
  hipStream_t st = as_stream(stream);
#define MOC_UP(T)                                                                              \
  selected_up_silu_kernel<T><<<grid, block, 0, st>>>((const uint16_t*)x, (int)nb, (int)hidden, \
                                                     (const uint16_t*)topk_vals, idx, (int)k,  \
                                                     (const uint16_t*)w_up, (int)inter,        \
                                                     (uint16_t*)z)
  if (idx_dtype == MOC_I16) MOC_UP(int16_t);
  else if (idx_dtype == MOC_I32) MOC_UP(int32_t);
  else MOC_UP(int64_t);
#undef MOC_UP
  return check_launch("selected_up_silu_kernel");
}

extern "C" int64_t moc_selected_down_workspace_size(int64_t nb, int64_t k, int64_t hidden) {
  if (nb <= 0 || k <= 0 || hidden <= 0) return 0;
  const DownPlan p = down_plan(nb, k, hidden);
  return align256(static_cast<int64_t>(p.splits) * nb * hidden * 4);
}

extern "C" int moc_selected_down_bf16(const void* z, const void* idx, int idx_dtype, int64_t nb,
                                      int64_t k, const void* w_down_t, int64_t inter,
                                      int64_t hidden, void* y, void* workspace,
                                      int64_t workspace_bytes, void* stream) {
  MOC_REQUIRE(idx_ok(idx_dtype), "moc_selected_down_bf16: bad index dtype");
  MOC_REQUIRE(nb >= 0 && k >= 1 && inter >= 1 && hidden >= 1, "moc_selected_down_bf16: bad shape");
  MOC_REQUIRE(hidden % 8 == 0, "moc_selected_down_bf16: hidden must be a multiple of 8");
  MOC_REQUIRE(nb <= 65535, "moc_selected_down_bf16: nb too large");
  if (nb == 0) return MOC_OK;
  MOC_REQUIRE(z && idx && w_down_t && y, "moc_selected_down_bf16: null pointer");
  MOC_REQUIRE(aligned16(w_down_t), "moc_selected_down_bf16: w_down_t must be 16-byte aligned");
  const int64_t need = moc_selected_down_workspace_size(nb, k, hidden);
  MOC_REQUIRE(workspace != nullptr && workspace_bytes >= need,
              "moc_selected_down_bf16: workspace of %lld bytes required", (long long)need);
  return launch_selected_down(z, idx, idx_dtype, nb, k, w_down_t, inter, hidden, y, workspace,
                              as_stream(stream));
}

extern "C" int64_t moc_global_after_gate_workspace_size(int64_t nb, int64_t inter, int64_t k,
                                                        int64_t hidden) {
  if (nb <= 0 || k <= 0 || hidden <= 0 || inter <= 0) return 0;
  return align256(nb * k * 4) + 2 * align256(nb * k * 2) +
         moc_selected_down_workspace_size(nb, k, hidden);
}

extern "C" int moc_global_after_gate_bf16(const void* x, const void* gate_scores, int64_t nb,
                                          int64_t inter, int64_t hidden, const void* w_up,
                                          const void* w_down_t, int64_t k, void* y,
                                          void* workspace, int64_t workspace_bytes,
                                          void* stream) {
  MOC_REQUIRE(nb >= 0 && inter >= 1 && hidden >= 1, "moc_global_after_gate_bf16: bad shape");
  MOC_REQUIRE(k >= 1 && k <= inter, "invalid k");
  if (nb == 0) return MOC_OK;
  const int64_t need = moc_global_after_gate_workspace_size(nb, inter, k, hidden);
  MOC_REQUIRE(workspace != nullptr && workspace_bytes >= need,
              "moc_global_after_gate_bf16: workspace of %lld bytes required", (long long)need);
  char* ws = static_cast<char*>(workspace);
  void* idx = ws;
  ws += align256(nb * k * 4);
  void* vals = ws;
  ws += align256(nb * k * 2);
  void* z = ws;
  ws += align256(nb * k * 2);
  int rc = moc_topk_rows(MOC_BF16, gate_scores, nb, inter, inter, k, 0, vals, idx, MOC_I32,
                         nullptr, 0, stream);
  if (rc != MOC_OK) return rc;
  rc = moc_selected_up_silu_bf16(x, nb, hidden, vals, idx, MOC_I32, k, w_up, inter, z, stream);
  if (rc != MOC_OK) return rc;
  return moc_selected_down_bf16(z, idx, MOC_I32, nb, k, w_down_t, inter, hidden, y, ws,
                                moc_selected_down_workspace_size(nb, k, hidden), stream);
}

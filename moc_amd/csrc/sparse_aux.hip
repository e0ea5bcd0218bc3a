// Sparse helper kernels of the MoC training path (gfx950).
//
// These move data between the compact per-token selection [rows, K] (values
// paired with channel indices) and the dense [rows, I] activations that the
// GEMMs consume.  Each entry point restates one launcher of
// moc/training/triton_sparse_aux.py with the same bf16 rounding points:
//
//   moc_sparse_forward_aux     <- sparse_forward_aux      (:197-231, kernel :17-49)
//   moc_scatter_sparse_to_dense<- scatter_sparse_to_dense (:266-290, kernel :71-87)
//   moc_gather_dense_to_sparse <- gather_dense_to_sparse  (:234-263, kernel :52-68)
//   moc_sparse_backward_aux    <- sparse_backward_aux     (:363-423; bf16 chain :376-400,
//                                                          fp32 kernel :139-182)
//   moc_gcp_recompute          <- _MoCGCPFunction.backward recompute (moc/ffn.py:435-436)
//   moc_gcp_recompute_scatter  <- the same recompute followed by the scatter of z
//                                 (moc/ffn.py:435-437) in one pass
//
// bf16 with 16-byte aligned dense rows (the FFN's padded buffers) runs the
// row form: one workgroup per row, dense rows staged and built in LDS and
// moved with 16-byte accesses, zeros included.  Otherwise dense outputs are
// cleared by a fill kernel inside the same entry point (no hipMemsetAsync,
// so the calls stay valid inside a captured HIP graph) and elementwise work
// is one thread per selected entry.  Every kernel is bound by HBM traffic.
#include <algorithm>

#include "abi.h"
#include "common.h"

extern "C" int moc_fill_zero(void* dst, int64_t bytes, void* stream);

namespace moc {
namespace {

template <bool BF16>
struct Elem;
template <>
struct Elem<true> {
  using T = uint16_t;
  __device__ static float ld(T v) { return bf16_to_f32(v); }
  __device__ static T st(float f) { return f32_to_bf16(f); }
  __device__ static float rnd(float f) { return round_bf16(f); }
};
template <>
struct Elem<false> {
  using T = float;
  __device__ static float ld(T v) { return v; }
  __device__ static T st(float f) { return f; }
  __device__ static float rnd(float f) { return f; }
};

template <bool BF16, typename IdxT>
__global__ __launch_bounds__(256) void sparse_forward_aux_kernel(
    const typename Elem<BF16>::T* __restrict__ vals, const IdxT* __restrict__ idx,
    const typename Elem<BF16>::T* __restrict__ u_full, int64_t u_ld, int64_t n, int k,
    typename Elem<BF16>::T* __restrict__ u_s, typename Elem<BF16>::T* __restrict__ s_s,
    typename Elem<BF16>::T* __restrict__ z_s, typename Elem<BF16>::T* __restrict__ z_full,
    int64_t z_ld, int64_t inter) {
  using E = Elem<BF16>;
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= n) return;
  const int64_t row = e / k;
  const int64_t ch = static_cast<int64_t>(idx[e]);
  if (ch < 0 || ch >= inter) return;  // malformed index: never touch memory
  const float g = E::ld(vals[e]);
  const typename E::T u_raw = u_full[row * u_ld + ch];
  const float u = E::ld(u_raw);
  // Triton: s = g * sigmoid(g); bf16: s rounded, z = bf16(s_bf16 * u)
  const float s = E::rnd(g * sigmoid_f32(g));
  const typename E::T z = E::st(s * u);
  if (u_s) u_s[e] = u_raw;
  if (s_s) s_s[e] = E::st(s);
  if (z_s) z_s[e] = z;
  if (z_full) z_full[row * z_ld + ch] = z;
}

template <typename T, typename IdxT>
__global__ __launch_bounds__(256) void scatter_kernel(const T* __restrict__ sparse,
                                                      const IdxT* __restrict__ idx, int64_t n,
                                                      int k, T* __restrict__ dense, int64_t ld,
                                                      int64_t inter) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= n) return;
  const int64_t row = e / k;
  const int64_t ch = static_cast<int64_t>(idx[e]);
  if (ch < 0 || ch >= inter) return;
  dense[row * ld + ch] = sparse[e];
}

template <typename T, typename IdxT>
__global__ __launch_bounds__(256) void gather_kernel(const T* __restrict__ dense, int64_t ld,
                                                     const IdxT* __restrict__ idx, int64_t n,
                                                     int k, T* __restrict__ sparse, int64_t inter) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= n) return;
  const int64_t row = e / k;
  const int64_t ch = static_cast<int64_t>(idx[e]);
  sparse[e] = (ch >= 0 && ch < inter) ? dense[row * ld + ch] : T(0);
}

// GCP recompute.  torch F.silu on a bf16 tensor evaluates g / (1 + exp(-g))
// in f32 and rounds; the product is another rounded bf16 op.
template <bool BF16>
__global__ __launch_bounds__(256) void gcp_recompute_kernel(
    const typename Elem<BF16>::T* __restrict__ g_s, const typename Elem<BF16>::T* __restrict__ u_s,
    int64_t n, typename Elem<BF16>::T* __restrict__ s_s, typename Elem<BF16>::T* __restrict__ z_s) {
  using E = Elem<BF16>;
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= n) return;
  const float s = E::rnd(silu_f32(E::ld(g_s[e])));
  if (s_s) s_s[e] = E::st(s);
  if (z_s) z_s[e] = E::st(s * E::ld(u_s[e]));
}

// Backward aux.  bf16 follows the reference's correctness-first chain where
// every elementwise op materialises a bf16 tensor:
//   grad_s = bf16(u*gz), grad_u = bf16(s*gz), sig = bf16(sigmoid(g)),
//   t1 = bf16(1-sig), t2 = bf16(g*t1), t3 = bf16(1+t2), d = bf16(sig*t3),
//   grad_g = bf16(grad_s*d).
// f32 is the fused kernel: grad_g = u*gz*sig*(1+g*(1-sig)), grad_u = s*gz.
// A null s_s recomputes s = silu(g) as the GCP variant does.
template <bool BF16, typename IdxT>
__global__ __launch_bounds__(256) void sparse_backward_aux_kernel(
    const IdxT* __restrict__ idx, const typename Elem<BF16>::T* __restrict__ g_s,
    const typename Elem<BF16>::T* __restrict__ u_s, const typename Elem<BF16>::T* __restrict__ s_s,
    const typename Elem<BF16>::T* __restrict__ gz_full, int64_t gz_ld, int64_t n, int k,
    typename Elem<BF16>::T* __restrict__ grad_g, typename Elem<BF16>::T* __restrict__ grad_u,
    int64_t out_ld, int64_t inter) {
  using E = Elem<BF16>;
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= n) return;
  const int64_t row = e / k;
  const int64_t ch = static_cast<int64_t>(idx[e]);
  if (ch < 0 || ch >= inter) return;
  const float gz = E::ld(gz_full[row * gz_ld + ch]);
  const float g = E::ld(g_s[e]);
  const float u = E::ld(u_s[e]);
  const float s = s_s ? E::ld(s_s[e]) : E::rnd(silu_f32(g));
  float gg, gu;
  if (BF16) {
    const float gs = round_bf16(u * gz);
    gu = round_bf16(s * gz);
    const float sig = round_bf16(sigmoid_f32(g));
    const float t1 = round_bf16(1.0f - sig);
    const float t2 = round_bf16(g * t1);
    const float t3 = round_bf16(1.0f + t2);
    const float d = round_bf16(sig * t3);
    gg = round_bf16(gs * d);
  } else {
    const float sig = sigmoid_f32(g);
    const float d = sig * (1.0f + g * (1.0f - sig));
    gg = u * gz * d;
    gu = s * gz;
  }
  grad_g[row * out_ld + ch] = E::st(gg);
  grad_u[row * out_ld + ch] = E::st(gu);
}

// ---------------------------------------------------------------------------
// Row form (bf16, dense rows 16-byte aligned with a pitch that is a multiple
// of 8 and <= kRowMaxLd): one workgroup per row.  Dense inputs are staged in
// LDS with 16-byte loads, dense outputs are built in LDS (zeros plus the
// selected values) and written back whole with 16-byte stores, so the dense
// tensors are read and written once, coalesced, and need no separate
// zero-fill launch.  The per-entry arithmetic is the same as above.
// ---------------------------------------------------------------------------
// Threads per row: 256 (the backward row at 512 measured 118.9 against
// 116-117 us on 16384 rows of 5461 and 33.7 against 26-27 us on 8192 rows of
// 2048; the other row kernels at 512, 49.6 against 67 us for the GCP
// recompute + scatter at 16384 x 5461).
constexpr int kRowThreadsBwd = 256;
constexpr int kRowThreads = 256;
// Rows of at most kNarrowRow channels run the forward and backward row
// kernels on 128 threads (130m rows of 2048: forward 16.9 -> 15.8 us,
// backward 25.2 -> 23.4 us; 16384 rows of 5461 at 128: 82 -> 91 and 119 ->
// 152 us, so wider rows keep 256).
constexpr int64_t kNarrowRow = 2048;
constexpr int64_t kRowMaxLd = 8192;  // three staged rows fit the default 64 KB of LDS

// Elements of an output row the row kernels write: inter rounded up to a
// multiple of 8, at most the row pitch.
__host__ __device__ inline int64_t out_row_width(int64_t inter, int64_t out_ld) {
  const int64_t w = (inter + 7) / 8 * 8;
  return w < out_ld ? w : out_ld;
}

template <int NT>
__device__ __forceinline__ void row_zero(uint16_t* buf, int64_t ld) {
  for (int64_t c = threadIdx.x; c < ld / 8; c += NT)
    reinterpret_cast<uint4*>(buf)[c] = make_uint4(0, 0, 0, 0);
}
// All of a thread's (<= 4) 16-byte loads are issued before any is stored, so
// staging a row costs one memory latency.
template <int NT>
__device__ __forceinline__ void row_load(uint16_t* buf, const uint16_t* src, int64_t ld) {
  constexpr int kMax = static_cast<int>(kRowMaxLd / 8 / NT);
  uint4 v[kMax];
#pragma unroll
  for (int q = 0; q < kMax; ++q) {
    const int64_t c = threadIdx.x + static_cast<int64_t>(NT) * q;
    v[q] = c < ld / 8 ? reinterpret_cast<const uint4*>(src)[c] : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int q = 0; q < kMax; ++q) {
    const int64_t c = threadIdx.x + static_cast<int64_t>(NT) * q;
    if (c < ld / 8) reinterpret_cast<uint4*>(buf)[c] = v[q];
  }
}
template <int NT>
__device__ __forceinline__ void row_store(uint16_t* dst, const uint16_t* buf, int64_t ld) {
  for (int64_t c = threadIdx.x; c < ld / 8; c += NT)
    reinterpret_cast<uint4*>(dst)[c] = reinterpret_cast<const uint4*>(buf)[c];
}

// Row-form arithmetic: RNE to bf16 with the gfx950 packed conversion.
__device__ __forceinline__ uint16_t to_bf16(float f) { return bf16_rne(f); }
__device__ __forceinline__ float rnd(float f) { return bf16_rnd(f); }

// The entries of a row are taken kRowPer per thread at a time; the first
// group's sparse loads are issued before the dense row is staged, so the two
// memory latencies overlap.
constexpr int kRowPer = 4;

// VEC: the thread's kRowPer entries are consecutive (e0 + kRowPer threadIdx.x
// + q), so each sparse tensor arrives in one 8-byte load (the indices in
// kRowPer sizeof(IdxT) bytes) instead of kRowPer 2-byte ones; the caller
// guarantees k % kRowPer == 0 and aligned rows.  Otherwise the entries are
// e0 + threadIdx.x + NT q (element loads, any k).
template <typename IdxT, int NT, bool VEC = false>
struct RowEntries {
  int64_t ch[kRowPer];
  uint16_t a[kRowPer], b[kRowPer], c[kRowPer];
  __device__ __forceinline__ static int entry(int e0, int q) {
    return VEC ? e0 + kRowPer * static_cast<int>(threadIdx.x) + q : e0 + static_cast<int>(threadIdx.x) + NT * q;
  }
  __device__ __forceinline__ static void load4(const uint16_t* p, int64_t i, bool ok, uint16_t (&v)[kRowPer]) {
    const uint2 w = (ok && p) ? *reinterpret_cast<const uint2*>(p + i) : make_uint2(0, 0);
    v[0] = static_cast<uint16_t>(w.x);
    v[1] = static_cast<uint16_t>(w.x >> 16);
    v[2] = static_cast<uint16_t>(w.y);
    v[3] = static_cast<uint16_t>(w.y >> 16);
  }
  // entries of row `row` from entry(e0, .); a/b/c from up to three sparse
  // [rows, k] tensors (null: not loaded)
  __device__ __forceinline__ void load(const IdxT* idx, const uint16_t* pa, const uint16_t* pb,
                                       const uint16_t* pc, int64_t row, int k, int e0) {
    if constexpr (VEC) {
      static_assert(kRowPer == 4, "vector entry loads take four entries");
      const int e = entry(e0, 0);
      const int64_t i = row * k + e;
      const bool ok = e < k;
      load4(pa, i, ok, a);
      load4(pb, i, ok, b);
      load4(pc, i, ok, c);
      if constexpr (sizeof(IdxT) == 2) {
        uint16_t t[kRowPer];
        load4(reinterpret_cast<const uint16_t*>(idx), i, ok, t);
#pragma unroll
        for (int q = 0; q < kRowPer; ++q) ch[q] = ok ? static_cast<int64_t>(static_cast<int16_t>(t[q])) : -1;
      } else {
#pragma unroll
        for (int q = 0; q < kRowPer; ++q) ch[q] = ok ? static_cast<int64_t>(idx[i + q]) : -1;
      }
    } else {
#pragma unroll
      for (int q = 0; q < kRowPer; ++q) {
        const int e = entry(e0, q);
        const int64_t i = row * k + e;
        const bool ok = e < k;
        ch[q] = ok ? static_cast<int64_t>(idx[i]) : -1;
        a[q] = (ok && pa) ? pa[i] : uint16_t(0);
        b[q] = (ok && pb) ? pb[i] : uint16_t(0);
        c[q] = (ok && pc) ? pc[i] : uint16_t(0);
      }
    }
  }
};

// Stores kRowPer bf16 values of consecutive entries e .. e + 3 (VEC form).
__device__ __forceinline__ void store4(uint16_t* p, const uint16_t (&v)[kRowPer]) {
  *reinterpret_cast<uint2*>(p) = make_uint2(v[0] | (static_cast<uint32_t>(v[1]) << 16),
                                            v[2] | (static_cast<uint32_t>(v[3]) << 16));
}

template <typename IdxT>
__global__ __launch_bounds__(kRowThreads) void scatter_rows_kernel(
    const uint16_t* __restrict__ sparse, const IdxT* __restrict__ idx, int k, int64_t inter,
    uint16_t* __restrict__ dense, int64_t ld) {
  extern __shared__ __attribute__((aligned(16))) uint16_t rbuf[];
  const int64_t row = blockIdx.x;
  RowEntries<IdxT, kRowThreads> r;
  r.load(idx, sparse, nullptr, nullptr, row, k, 0);
  row_zero<kRowThreads>(rbuf, ld);
  __syncthreads();
  for (int e0 = 0; e0 < k; e0 += kRowThreads * kRowPer) {
    if (e0 > 0) r.load(idx, sparse, nullptr, nullptr, row, k, e0);
#pragma unroll
    for (int q = 0; q < kRowPer; ++q)
      if (r.ch[q] >= 0 && r.ch[q] < inter) rbuf[r.ch[q]] = r.a[q];
  }
  __syncthreads();
  row_store<kRowThreads>(dense + row * ld, rbuf, ld);
}

// GCP recompute fused with the scatter of z: s = bf16(SiLU(g)),
// z = bf16(s * u) per selected entry (torch's F.silu and product on bf16
// tensors), s to s_s, z into the dense row.
template <typename IdxT, bool VEC>
__global__ __launch_bounds__(kRowThreads) void gcp_scatter_rows_kernel(
    const uint16_t* __restrict__ g_s, const uint16_t* __restrict__ u_s,
    const IdxT* __restrict__ idx, int k, int64_t inter, uint16_t* __restrict__ s_s,
    uint16_t* __restrict__ z_full, int64_t ld) {
  extern __shared__ __attribute__((aligned(16))) uint16_t rbuf[];
  const int64_t row = blockIdx.x;
  RowEntries<IdxT, kRowThreads, VEC> r;
  r.load(idx, g_s, u_s, nullptr, row, k, 0);
  row_zero<kRowThreads>(rbuf, ld);
  __syncthreads();
  for (int e0 = 0; e0 < k; e0 += kRowThreads * kRowPer) {
    if (e0 > 0) r.load(idx, g_s, u_s, nullptr, row, k, e0);
    uint16_t sv[kRowPer];
#pragma unroll
    for (int q = 0; q < kRowPer; ++q) {
      const int e = r.entry(e0, q);
      const float s = rnd(silu_f32(bf16_to_f32(r.a[q])));
      sv[q] = to_bf16(s);
      if (!VEC && s_s && e < k) s_s[row * k + e] = sv[q];
      if (r.ch[q] >= 0 && r.ch[q] < inter) rbuf[r.ch[q]] = to_bf16(s * bf16_to_f32(r.b[q]));
    }
    if (VEC && s_s && r.entry(e0, 0) < k) store4(s_s + row * k + r.entry(e0, 0), sv);
  }
  __syncthreads();
  row_store<kRowThreads>(z_full + row * ld, rbuf, ld);
}

template <typename IdxT, bool VEC, int NT = kRowThreads>
__global__ __launch_bounds__(NT) void forward_aux_rows_kernel(
    const uint16_t* __restrict__ vals, const IdxT* __restrict__ idx,
    const uint16_t* __restrict__ u_full, int64_t u_ld, int k, int64_t inter,
    uint16_t* __restrict__ u_s, uint16_t* __restrict__ s_s, uint16_t* __restrict__ z_s,
    uint16_t* __restrict__ z_full, int64_t z_ld) {
  extern __shared__ __attribute__((aligned(16))) uint16_t rbuf[];
  uint16_t* urow = rbuf;        // [u_ld]
  uint16_t* zrow = rbuf + u_ld;  // [z_ld]
  const int64_t row = blockIdx.x;
  RowEntries<IdxT, NT, VEC> r;
  r.load(idx, vals, nullptr, nullptr, row, k, 0);
  row_load<NT>(urow, u_full + row * u_ld, u_ld);
  row_zero<NT>(zrow, z_ld);
  __syncthreads();
  for (int e0 = 0; e0 < k; e0 += NT * kRowPer) {
    if (e0 > 0) r.load(idx, vals, nullptr, nullptr, row, k, e0);
    uint16_t uv[kRowPer], sv[kRowPer], zv[kRowPer];
    bool all = true;  // every entry of the group valid (VEC: vector stores)
#pragma unroll
    for (int q = 0; q < kRowPer; ++q) {
      const int64_t ch = r.ch[q];
      uv[q] = sv[q] = zv[q] = 0;
      if (ch < 0 || ch >= inter) {  // malformed index or past k: never touch memory
        all = false;
        continue;
      }
      const int64_t i = row * k + r.entry(e0, q);
      const float g = bf16_to_f32(r.a[q]);
      const uint16_t u_raw = urow[ch];
      const float s = rnd(g * sigmoid_f32(g));
      const uint16_t z = to_bf16(s * bf16_to_f32(u_raw));
      uv[q] = u_raw;
      sv[q] = to_bf16(s);
      zv[q] = z;
      if (!VEC) {
        if (u_s) u_s[i] = u_raw;
        if (s_s) s_s[i] = sv[q];
        if (z_s) z_s[i] = z;
      }
      zrow[ch] = z;
    }
    if (VEC) {
      const int e = r.entry(e0, 0);
      if (all) {
        const int64_t i = row * k + e;
        if (u_s) store4(u_s + i, uv);
        if (s_s) store4(s_s + i, sv);
        if (z_s) store4(z_s + i, zv);
      } else {
#pragma unroll
        for (int q = 0; q < kRowPer; ++q) {
          if (r.ch[q] < 0 || r.ch[q] >= inter) continue;
          const int64_t i = row * k + e + q;
          if (u_s) u_s[i] = uv[q];
          if (s_s) s_s[i] = sv[q];
          if (z_s) z_s[i] = zv[q];
        }
      }
    }
  }
  __syncthreads();
  row_store<NT>(z_full + row * z_ld, zrow, z_ld);
}

// f32 form of forward_aux_rows_kernel (rows of at most kRowMaxLdF32 floats,
// pitches multiples of 4): the element kernel's f32 arithmetic, the U row
// staged in LDS and the dense Z row built there and written whole (no
// zero-fill launch).
constexpr int64_t kRowMaxLdF32 = 4096;

template <typename IdxT>
__global__ __launch_bounds__(kRowThreads) void forward_aux_rows_f32_kernel(
    const float* __restrict__ vals, const IdxT* __restrict__ idx, const float* __restrict__ u_full,
    int64_t u_ld, int k, int64_t inter, float* __restrict__ u_s, float* __restrict__ s_s,
    float* __restrict__ z_s, float* __restrict__ z_full, int64_t z_ld) {
  extern __shared__ __attribute__((aligned(16))) float fbuf[];
  float* urow = fbuf;        // [u_ld]
  float* zrow = fbuf + u_ld;  // [z_ld]
  const int64_t row = blockIdx.x;
  constexpr int kMax = static_cast<int>(kRowMaxLdF32 / 4 / kRowThreads);
  // the first entries' loads, then the U row's, before any is used
  int64_t ch[kRowPer];
  float gv[kRowPer];
#pragma unroll
  for (int q = 0; q < kRowPer; ++q) {
    const int e = threadIdx.x + kRowThreads * q;
    ch[q] = e < k ? static_cast<int64_t>(idx[row * k + e]) : -1;
    gv[q] = e < k ? vals[row * k + e] : 0.0f;
  }
  float4 v[kMax];
#pragma unroll
  for (int q = 0; q < kMax; ++q) {
    const int64_t c = threadIdx.x + static_cast<int64_t>(kRowThreads) * q;
    v[q] = c < u_ld / 4 ? reinterpret_cast<const float4*>(u_full + row * u_ld)[c] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
#pragma unroll
  for (int q = 0; q < kMax; ++q) {
    const int64_t c = threadIdx.x + static_cast<int64_t>(kRowThreads) * q;
    if (c < u_ld / 4) reinterpret_cast<float4*>(urow)[c] = v[q];
  }
  for (int64_t c = threadIdx.x; c < z_ld / 4; c += kRowThreads)
    reinterpret_cast<float4*>(zrow)[c] = make_float4(0.f, 0.f, 0.f, 0.f);
  __syncthreads();
  for (int e0 = 0; e0 < k; e0 += kRowThreads * kRowPer) {
    if (e0 > 0) {
#pragma unroll
      for (int q = 0; q < kRowPer; ++q) {
        const int e = e0 + threadIdx.x + kRowThreads * q;
        ch[q] = e < k ? static_cast<int64_t>(idx[row * k + e]) : -1;
        gv[q] = e < k ? vals[row * k + e] : 0.0f;
      }
    }
#pragma unroll
    for (int q = 0; q < kRowPer; ++q) {
      if (ch[q] < 0 || ch[q] >= inter) continue;  // malformed index or past k: never touch memory
      const int64_t i = row * k + e0 + threadIdx.x + kRowThreads * q;
      const float g = gv[q];
      const float u = urow[ch[q]];
      const float sv = g * sigmoid_f32(g);
      const float z = sv * u;
      if (u_s) u_s[i] = u;
      if (s_s) s_s[i] = sv;
      if (z_s) z_s[i] = z;
      zrow[ch[q]] = z;
    }
  }
  __syncthreads();
  for (int64_t c = threadIdx.x; c < z_ld / 4; c += kRowThreads)
    reinterpret_cast<float4*>(z_full + row * z_ld)[c] = reinterpret_cast<const float4*>(zrow)[c];
}

// ZOUT: the same pass also writes the dense Z rows that the weight gradient
// dWd = dD^T Z reads (z_full, rows z_ld apart): z = bf16(S u) from the
// recomputed S (GCP, the bits of gcp_scatter_rows_kernel) or the saved z_s
// (the bits of the scatter), so no separate scatter launch is needed when
// dWd runs after this kernel.
template <typename IdxT, bool VEC, bool ZOUT = false, int NT = kRowThreadsBwd>
__global__ __launch_bounds__(NT) void backward_aux_rows_kernel(
    const IdxT* __restrict__ idx, const uint16_t* __restrict__ g_s,
    const uint16_t* __restrict__ u_s, const uint16_t* __restrict__ s_s,
    const uint16_t* gz_full, int64_t gz_ld, int k, int64_t inter,
    uint16_t* __restrict__ grad_g, uint16_t* grad_u, int64_t out_ld,
    const uint16_t* __restrict__ z_s = nullptr, uint16_t* __restrict__ z_full = nullptr, int64_t z_ld = 0) {
  extern __shared__ __attribute__((aligned(16))) uint16_t rbuf[];
  // an output row is inter values plus zeros up to a multiple of 8; rows
  // are out_ld apart (out_ld may leave room for another tensor's rows).
  // gz_full may be grad_u itself (gz_ld == out_ld): the row's gZ values are
  // staged whole before the barrier that precedes the row's stores.
  const int64_t width = out_row_width(inter, out_ld);
  const int64_t gz_w = out_row_width(inter, gz_ld);
  const int64_t z_w = ZOUT ? out_row_width(inter, z_ld) : 0;
  uint16_t* gzrow = rbuf;                 // [gz_w]
  uint16_t* ggrow = rbuf + gz_w;          // [width]
  uint16_t* gurow = rbuf + gz_w + width;  // [width]
  uint16_t* zrow = gurow + width;         // [z_w] (ZOUT)
  const int64_t row = blockIdx.x;
  RowEntries<IdxT, NT, VEC> r;
  r.load(idx, g_s, u_s, s_s, row, k, 0);
  row_load<NT>(gzrow, gz_full + row * gz_ld, gz_w);
  row_zero<NT>(ggrow, width);
  row_zero<NT>(gurow, width);
  if constexpr (ZOUT) row_zero<NT>(zrow, z_w);
  __syncthreads();
  for (int e0 = 0; e0 < k; e0 += NT * kRowPer) {
    if (e0 > 0) r.load(idx, g_s, u_s, s_s, row, k, e0);
    uint16_t zv[kRowPer];
    if constexpr (ZOUT) {
      if (z_s != nullptr) {
        if constexpr (VEC) {
          r.load4(z_s, row * k + r.entry(e0, 0), r.entry(e0, 0) < k, zv);
        } else {
#pragma unroll
          for (int q = 0; q < kRowPer; ++q) zv[q] = r.entry(e0, q) < k ? z_s[row * k + r.entry(e0, q)] : uint16_t(0);
        }
      }
    }
#pragma unroll
    for (int q = 0; q < kRowPer; ++q) {
      const int64_t ch = r.ch[q];
      if (ch < 0 || ch >= inter) continue;
      const float g = bf16_to_f32(r.a[q]), u = bf16_to_f32(r.b[q]);
      sparse_bwd_entry(g, u, s_s != nullptr, bf16_to_f32(r.c[q]), bf16_to_f32(gzrow[ch]), ggrow[ch], gurow[ch]);
      if constexpr (ZOUT) zrow[ch] = z_s != nullptr ? zv[q] : to_bf16(rnd(silu_f32(g)) * u);
    }
  }
  __syncthreads();
  row_store<NT>(grad_g + row * out_ld, ggrow, width);
  row_store<NT>(grad_u + row * out_ld, gurow, width);
  if constexpr (ZOUT) row_store<NT>(z_full + row * z_ld, zrow, z_w);
}

// Zeros columns [0, width) of rows x ld elements of esz bytes (16-byte
// stores where the row start and width allow, else element stores).
__global__ __launch_bounds__(256) void zero_rows_kernel(char* __restrict__ p, int64_t rows,
                                                        int64_t width_bytes, int64_t ld_bytes) {
  const int64_t row = blockIdx.y;
  char* r = p + row * ld_bytes;
  const bool vec = ((reinterpret_cast<uintptr_t>(r) | static_cast<uintptr_t>(width_bytes)) & 15) == 0;
  if (vec) {
    for (int64_t c = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; c < width_bytes / 16;
         c += static_cast<int64_t>(gridDim.x) * 256)
      reinterpret_cast<uint4*>(r)[c] = make_uint4(0, 0, 0, 0);
  } else {
    for (int64_t c = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; c < width_bytes;
         c += static_cast<int64_t>(gridDim.x) * 256)
      r[c] = 0;
  }
}

// The row form applies to bf16 dense rows that are 16-byte aligned with a
// pitch that is a multiple of 8 elements and at most kRowMaxLd.
inline bool row_form_ok(const void* p, int64_t ld) {
  return ld % 8 == 0 && ld <= kRowMaxLd && reinterpret_cast<uintptr_t>(p) % 16 == 0;
}

inline dim3 grid_for(int64_t n) { return dim3(static_cast<unsigned>((n + 255) / 256)); }

bool idx_ok(int d) { return d == MOC_I16 || d == MOC_I32 || d == MOC_I64; }

// The row kernels' vector entry loads: k a multiple of kRowPer, the bf16
// sparse tensors 8-byte aligned (a row of k entries then starts aligned
// too) and the indices aligned to kRowPer of their width.
bool entries_vec_ok(int64_t k, int idx_dtype, const void* idx, const void* a, const void* b, const void* c) {
  const uintptr_t isz = idx_dtype == MOC_I16 ? 2 : idx_dtype == MOC_I32 ? 4 : 8;
  auto al = [](const void* p, uintptr_t n) { return p == nullptr || reinterpret_cast<uintptr_t>(p) % n == 0; };
  return k % kRowPer == 0 && al(idx, kRowPer * isz) && al(a, 8) && al(b, 8) && al(c, 8);
}

}  // namespace
}  // namespace moc

using namespace moc;

#define MOC_IDX_DISPATCH(IDX_DTYPE, MACRO)       \
  do {                                           \
    if ((IDX_DTYPE) == MOC_I16) {                \
      MACRO(int16_t);                            \
    } else if ((IDX_DTYPE) == MOC_I32) {         \
      MACRO(int32_t);                            \
    } else {                                     \
      MACRO(int64_t);                            \
    }                                            \
  } while (0)

extern "C" int moc_sparse_forward_aux(int dtype, const void* topk_vals, const void* idx,
                                      int idx_dtype, const void* u_full, int64_t u_ld,
                                      int64_t rows, int64_t k, int64_t inter, void* u_sparse,
                                      void* s_sparse, void* z_sparse, void* z_full, int64_t z_ld,
                                      void* stream) {
  MOC_REQUIRE(dtype == MOC_BF16 || dtype == MOC_F32, "moc_sparse_forward_aux: bad dtype");
  MOC_REQUIRE(idx_ok(idx_dtype), "moc_sparse_forward_aux: bad index dtype");
  MOC_REQUIRE(rows >= 0 && k >= 1 && inter >= k, "moc_sparse_forward_aux: bad shape");
  MOC_REQUIRE(u_ld >= inter && (z_full == nullptr || z_ld >= inter),
              "moc_sparse_forward_aux: bad leading dimension");
  const int64_t n = rows * k;
  if (n == 0) return MOC_OK;
  MOC_REQUIRE(topk_vals && idx && u_full, "moc_sparse_forward_aux: null input");
  hipStream_t st = as_stream(stream);
  const size_t esz = dtype == MOC_BF16 ? 2 : 4;
  if (dtype == MOC_BF16 && z_full != nullptr && rows < (1LL << 31) && row_form_ok(z_full, z_ld) &&
      row_form_ok(u_full, u_ld)) {
    const size_t lds = static_cast<size_t>(u_ld + z_ld) * 2;
    // vector entry loads and stores: the inputs and every sparse output aligned
    const bool vec = entries_vec_ok(k, idx_dtype, idx, topk_vals, u_sparse, s_sparse) &&
                     entries_vec_ok(k, idx_dtype, nullptr, z_sparse, nullptr, nullptr);
#define MOC_FWDR_NT(T, V, NT)                                                                        \
  forward_aux_rows_kernel<T, V, NT><<<dim3(static_cast<unsigned>(rows)), NT, lds, st>>>(              \
      (const uint16_t*)topk_vals, (const T*)idx, (const uint16_t*)u_full, u_ld, (int)k, inter,       \
      (uint16_t*)u_sparse, (uint16_t*)s_sparse, (uint16_t*)z_sparse, (uint16_t*)z_full, z_ld)
#define MOC_FWDR(T)                                                 \
  {                                                                 \
    if (inter <= kNarrowRow) {                                      \
      if (vec) MOC_FWDR_NT(T, true, 128);                           \
      else MOC_FWDR_NT(T, false, 128);                              \
    } else {                                                        \
      if (vec) MOC_FWDR_NT(T, true, kRowThreads);                   \
      else MOC_FWDR_NT(T, false, kRowThreads);                      \
    }                                                               \
  }
    MOC_IDX_DISPATCH(idx_dtype, MOC_FWDR);
#undef MOC_FWDR
#undef MOC_FWDR_NT
    return check_launch("forward_aux_rows_kernel");
  }
  auto f32_row_ok = [](const void* p, int64_t ld) {
    return ld % 4 == 0 && ld <= kRowMaxLdF32 && reinterpret_cast<uintptr_t>(p) % 16 == 0;
  };
  if (dtype == MOC_F32 && z_full != nullptr && rows < (1LL << 31) && f32_row_ok(z_full, z_ld) &&
      f32_row_ok(u_full, u_ld)) {
    const size_t lds = static_cast<size_t>(u_ld + z_ld) * 4;
#define MOC_FWDRF(T)                                                                           \
  forward_aux_rows_f32_kernel<T><<<dim3(static_cast<unsigned>(rows)), kRowThreads, lds, st>>>( \
      (const float*)topk_vals, (const T*)idx, (const float*)u_full, u_ld, (int)k, inter,        \
      (float*)u_sparse, (float*)s_sparse, (float*)z_sparse, (float*)z_full, z_ld)
    MOC_IDX_DISPATCH(idx_dtype, MOC_FWDRF);
#undef MOC_FWDRF
    return check_launch("forward_aux_rows_f32_kernel");
  }
  if (z_full) {
    const int rc = moc_fill_zero(z_full, rows * z_ld * static_cast<int64_t>(esz), stream);
    if (rc != MOC_OK) return rc;
  }
#define MOC_FWD(T)                                                                          \
  if (dtype == MOC_BF16)                                                                    \
    sparse_forward_aux_kernel<true, T><<<grid_for(n), 256, 0, st>>>(                        \
        (const uint16_t*)topk_vals, (const T*)idx, (const uint16_t*)u_full, u_ld, n, (int)k, \
        (uint16_t*)u_sparse, (uint16_t*)s_sparse, (uint16_t*)z_sparse, (uint16_t*)z_full,   \
        z_ld, inter);                                                                       \
  else                                                                                      \
    sparse_forward_aux_kernel<false, T><<<grid_for(n), 256, 0, st>>>(                       \
        (const float*)topk_vals, (const T*)idx, (const float*)u_full, u_ld, n, (int)k,      \
        (float*)u_sparse, (float*)s_sparse, (float*)z_sparse, (float*)z_full, z_ld, inter)
  MOC_IDX_DISPATCH(idx_dtype, MOC_FWD);
#undef MOC_FWD
  return check_launch("sparse_forward_aux_kernel");
}

extern "C" int moc_scatter_sparse_to_dense(int dtype, const void* sparse, const void* idx,
                                           int idx_dtype, int64_t rows, int64_t k, int64_t inter,
                                           void* dense, int64_t ld, void* stream) {
  MOC_REQUIRE(dtype == MOC_BF16 || dtype == MOC_F32, "moc_scatter_sparse_to_dense: bad dtype");
  MOC_REQUIRE(idx_ok(idx_dtype), "moc_scatter_sparse_to_dense: bad index dtype");
  MOC_REQUIRE(rows >= 0 && k >= 1 && inter >= k && ld >= inter,
              "moc_scatter_sparse_to_dense: bad shape");
  if (rows == 0) return MOC_OK;
  MOC_REQUIRE(sparse && idx && dense, "moc_scatter_sparse_to_dense: null pointer");
  hipStream_t st = as_stream(stream);
  if (dtype == MOC_BF16 && rows < (1LL << 31) && row_form_ok(dense, ld)) {
    const size_t lds = static_cast<size_t>(ld) * 2;
#define MOC_SCATR(T)                                                                          \
  scatter_rows_kernel<T><<<dim3(static_cast<unsigned>(rows)), kRowThreads, lds, st>>>(         \
      (const uint16_t*)sparse, (const T*)idx, (int)k, inter, (uint16_t*)dense, ld)
    MOC_IDX_DISPATCH(idx_dtype, MOC_SCATR);
#undef MOC_SCATR
    return check_launch("scatter_rows_kernel");
  }
  const size_t esz = dtype == MOC_BF16 ? 2 : 4;
  int rc = moc_fill_zero(dense, rows * ld * static_cast<int64_t>(esz), stream);
  if (rc != MOC_OK) return rc;
  const int64_t n = rows * k;
#define MOC_SCAT(T)                                                                              \
  if (dtype == MOC_BF16)                                                                         \
    scatter_kernel<uint16_t, T><<<grid_for(n), 256, 0, st>>>((const uint16_t*)sparse, (const T*)idx, \
                                                             n, (int)k, (uint16_t*)dense, ld, inter); \
  else                                                                                           \
    scatter_kernel<float, T><<<grid_for(n), 256, 0, st>>>((const float*)sparse, (const T*)idx, n,  \
                                                          (int)k, (float*)dense, ld, inter)
  MOC_IDX_DISPATCH(idx_dtype, MOC_SCAT);
#undef MOC_SCAT
  return check_launch("scatter_kernel");
}

extern "C" int moc_gather_dense_to_sparse(int dtype, const void* dense, int64_t ld,
                                          const void* idx, int idx_dtype, int64_t rows,
                                          int64_t k, void* sparse, void* stream) {
  MOC_REQUIRE(dtype == MOC_BF16 || dtype == MOC_F32, "moc_gather_dense_to_sparse: bad dtype");
  MOC_REQUIRE(idx_ok(idx_dtype), "moc_gather_dense_to_sparse: bad index dtype");
  MOC_REQUIRE(rows >= 0 && k >= 1 && ld >= k, "moc_gather_dense_to_sparse: bad shape");
  const int64_t n = rows * k;
  if (n == 0) return MOC_OK;
  MOC_REQUIRE(sparse && idx && dense, "moc_gather_dense_to_sparse: null pointer");
  const int64_t inter = ld;  // indices beyond the row pitch read as zero
  hipStream_t st = as_stream(stream);
#define MOC_GATH(T)                                                                            \
  if (dtype == MOC_BF16)                                                                       \
    gather_kernel<uint16_t, T><<<grid_for(n), 256, 0, st>>>((const uint16_t*)dense, ld,        \
                                                            (const T*)idx, n, (int)k,          \
                                                            (uint16_t*)sparse, inter);         \
  else                                                                                         \
    gather_kernel<float, T><<<grid_for(n), 256, 0, st>>>((const float*)dense, ld, (const T*)idx, \
                                                         n, (int)k, (float*)sparse, inter)
  MOC_IDX_DISPATCH(idx_dtype, MOC_GATH);
#undef MOC_GATH
  return check_launch("gather_kernel");
}

extern "C" int moc_gcp_recompute(int dtype, const void* g_sparse, const void* u_sparse, int64_t n,
                                 void* s_sparse, void* z_sparse, void* stream) {
  MOC_REQUIRE(dtype == MOC_BF16 || dtype == MOC_F32, "moc_gcp_recompute: bad dtype");
  MOC_REQUIRE(n >= 0, "moc_gcp_recompute: bad size");
  if (n == 0) return MOC_OK;
  MOC_REQUIRE(g_sparse && u_sparse, "moc_gcp_recompute: null input");
  hipStream_t st = as_stream(stream);
  if (dtype == MOC_BF16)
    gcp_recompute_kernel<true><<<grid_for(n), 256, 0, st>>>(
        (const uint16_t*)g_sparse, (const uint16_t*)u_sparse, n, (uint16_t*)s_sparse,
        (uint16_t*)z_sparse);
  else
    gcp_recompute_kernel<false><<<grid_for(n), 256, 0, st>>>(
        (const float*)g_sparse, (const float*)u_sparse, n, (float*)s_sparse, (float*)z_sparse);
  return check_launch("gcp_recompute_kernel");
}

extern "C" int moc_sparse_backward_aux(int dtype, const void* idx, int idx_dtype,
                                       const void* g_sparse, const void* u_sparse,
                                       const void* s_sparse, const void* gz_full, int64_t gz_ld,
                                       int64_t rows, int64_t k, int64_t inter, void* grad_g,
                                       void* grad_u, int64_t out_ld, void* stream) {
  MOC_REQUIRE(dtype == MOC_BF16 || dtype == MOC_F32, "moc_sparse_backward_aux: bad dtype");
  MOC_REQUIRE(idx_ok(idx_dtype), "moc_sparse_backward_aux: bad index dtype");
  MOC_REQUIRE(rows >= 0 && k >= 1 && inter >= k && gz_ld >= inter && out_ld >= inter,
              "moc_sparse_backward_aux: bad shape");
  if (rows == 0) return MOC_OK;
  MOC_REQUIRE(idx && g_sparse && u_sparse && gz_full && grad_g && grad_u,
              "moc_sparse_backward_aux: null pointer");
  const bool in_place = gz_full == grad_u;
  MOC_REQUIRE(gz_full != grad_g && (!in_place || gz_ld == out_ld),
              "moc_sparse_backward_aux: gz_full may only be grad_u itself, with gz_ld == out_ld");
  if (dtype == MOC_BF16 && rows < (1LL << 31) && row_form_ok(gz_full, gz_ld) &&
      row_form_ok(grad_g, out_ld) && row_form_ok(grad_u, out_ld)) {
    hipStream_t st = as_stream(stream);
    const size_t lds = static_cast<size_t>(out_row_width(inter, gz_ld) + 2 * out_row_width(inter, out_ld)) * 2;
    const bool vec = entries_vec_ok(k, idx_dtype, idx, g_sparse, u_sparse, s_sparse);
#define MOC_BWDR_NT(T, V, NT)                                                                        \
  backward_aux_rows_kernel<T, V, false, NT><<<dim3(static_cast<unsigned>(rows)), NT, lds, st>>>(      \
      (const T*)idx, (const uint16_t*)g_sparse, (const uint16_t*)u_sparse, (const uint16_t*)s_sparse, \
      (const uint16_t*)gz_full, gz_ld, (int)k, inter, (uint16_t*)grad_g, (uint16_t*)grad_u, out_ld)
#define MOC_BWDR(T)                                                 \
  {                                                                 \
    if (inter <= kNarrowRow) {                                      \
      if (vec) MOC_BWDR_NT(T, true, 128);                           \
      else MOC_BWDR_NT(T, false, 128);                              \
    } else {                                                        \
      if (vec) MOC_BWDR_NT(T, true, kRowThreadsBwd);                \
      else MOC_BWDR_NT(T, false, kRowThreadsBwd);                   \
    }                                                               \
  }
    MOC_IDX_DISPATCH(idx_dtype, MOC_BWDR);
#undef MOC_BWDR
#undef MOC_BWDR_NT
    return check_launch("backward_aux_rows_kernel");
  }
  MOC_REQUIRE(!in_place, "moc_sparse_backward_aux: gZ in grad_u's rows needs the bf16 row form (16-byte aligned "
                         "rows, pitch a multiple of 8 and <= %lld)", (long long)kRowMaxLd);
  const int64_t esz = dtype == MOC_BF16 ? 2 : 4;
  MOC_REQUIRE(rows <= 65535 || out_row_width(inter, out_ld) == out_ld,
              "moc_sparse_backward_aux: more than 65535 rows need out_ld = inter rounded to 8");
  hipStream_t st = as_stream(stream);
  int rc = MOC_OK;
  if (out_row_width(inter, out_ld) == out_ld) {
    rc = moc_fill_zero(grad_g, rows * out_ld * esz, stream);
    if (rc == MOC_OK) rc = moc_fill_zero(grad_u, rows * out_ld * esz, stream);
  } else {
    // rows out_ld apart that leave room for other data: zero only the rows
    const int64_t wb = out_row_width(inter, out_ld) * esz;
    const dim3 zgrid(static_cast<unsigned>(std::min<int64_t>((wb / 16 + 255) / 256, 64)),
                     static_cast<unsigned>(rows));
    zero_rows_kernel<<<zgrid, 256, 0, st>>>(static_cast<char*>(grad_g), rows, wb, out_ld * esz);
    zero_rows_kernel<<<zgrid, 256, 0, st>>>(static_cast<char*>(grad_u), rows, wb, out_ld * esz);
    rc = check_launch("zero_rows_kernel");
  }
  if (rc != MOC_OK) return rc;
  const int64_t n = rows * k;
#define MOC_BWD(T)                                                                            \
  if (dtype == MOC_BF16)                                                                      \
    sparse_backward_aux_kernel<true, T><<<grid_for(n), 256, 0, st>>>(                         \
        (const T*)idx, (const uint16_t*)g_sparse, (const uint16_t*)u_sparse,                  \
        (const uint16_t*)s_sparse, (const uint16_t*)gz_full, gz_ld, n, (int)k,                \
        (uint16_t*)grad_g, (uint16_t*)grad_u, out_ld, inter);                                 \
  else                                                                                        \
    sparse_backward_aux_kernel<false, T><<<grid_for(n), 256, 0, st>>>(                        \
        (const T*)idx, (const float*)g_sparse, (const float*)u_sparse, (const float*)s_sparse, \
        (const float*)gz_full, gz_ld, n, (int)k, (float*)grad_g, (float*)grad_u, out_ld, inter)
  MOC_IDX_DISPATCH(idx_dtype, MOC_BWD);
#undef MOC_BWD
  return check_launch("sparse_backward_aux_kernel");
}

extern "C" int moc_gcp_recompute_scatter(int dtype, const void* g_sparse, const void* u_sparse,
                                         const void* idx, int idx_dtype, int64_t rows, int64_t k,
                                         int64_t inter, void* s_sparse, void* z_full, int64_t ld,
                                         void* stream) {
  MOC_REQUIRE(dtype == MOC_BF16, "moc_gcp_recompute_scatter: bf16 only");
  MOC_REQUIRE(idx_ok(idx_dtype), "moc_gcp_recompute_scatter: bad index dtype");
  MOC_REQUIRE(rows >= 0 && rows < (1LL << 31) && k >= 1 && inter >= k && ld >= inter,
              "moc_gcp_recompute_scatter: bad shape");
  if (rows == 0) return MOC_OK;
  MOC_REQUIRE(g_sparse && u_sparse && idx && z_full, "moc_gcp_recompute_scatter: null pointer");
  MOC_REQUIRE(row_form_ok(z_full, ld),
              "moc_gcp_recompute_scatter: z_full rows must be 16-byte aligned, pitch a multiple of 8 "
              "and <= %lld", (long long)kRowMaxLd);
  hipStream_t st = as_stream(stream);
  const size_t lds = static_cast<size_t>(ld) * 2;
  const bool vec = entries_vec_ok(k, idx_dtype, idx, g_sparse, u_sparse, s_sparse);
#define MOC_GCPS(T)                                                                                  \
  if (vec)                                                                                           \
    gcp_scatter_rows_kernel<T, true><<<dim3(static_cast<unsigned>(rows)), kRowThreads, lds, st>>>(   \
        (const uint16_t*)g_sparse, (const uint16_t*)u_sparse, (const T*)idx, (int)k, inter,         \
        (uint16_t*)s_sparse, (uint16_t*)z_full, ld);                                                 \
  else                                                                                               \
    gcp_scatter_rows_kernel<T, false><<<dim3(static_cast<unsigned>(rows)), kRowThreads, lds, st>>>(  \
        (const uint16_t*)g_sparse, (const uint16_t*)u_sparse, (const T*)idx, (int)k, inter,         \
        (uint16_t*)s_sparse, (uint16_t*)z_full, ld)
  MOC_IDX_DISPATCH(idx_dtype, MOC_GCPS);
#undef MOC_GCPS
  return check_launch("gcp_scatter_rows_kernel");
}

namespace moc {

// moc_sparse_backward_aux (bf16 row form) that also writes the dense Z rows
// (z_full, pitch z_ld) from the recomputed S (z_sparse NULL: GCP) or from the
// saved z_sparse: the scatter of Z fused into the gradient pass for a
// backward that runs dWd after it.  Returns 1 without launching where the
// row form does not apply.
int sparse_backward_aux_z(const void* idx, int idx_dtype, const void* g_sparse, const void* u_sparse,
                          const void* s_sparse, const void* z_sparse, const void* gz_full, int64_t gz_ld,
                          int64_t rows, int64_t k, int64_t inter, void* grad_g, void* grad_u, int64_t out_ld,
                          void* z_full, int64_t z_ld, hipStream_t st) {
  if (!idx_ok(idx_dtype) || rows <= 0 || rows >= (1LL << 31) || k < 1 || inter < k || gz_ld < inter ||
      out_ld < inter || z_ld < inter)
    return 1;
  if (!idx || !g_sparse || !u_sparse || !gz_full || !grad_g || !grad_u || !z_full) return 1;
  if (gz_full == grad_g || (gz_full == grad_u && gz_ld != out_ld)) return 1;
  if (!row_form_ok(gz_full, gz_ld) || !row_form_ok(grad_g, out_ld) || !row_form_ok(grad_u, out_ld) ||
      !row_form_ok(z_full, z_ld))
    return 1;
  const size_t lds = static_cast<size_t>(out_row_width(inter, gz_ld) + 2 * out_row_width(inter, out_ld) +
                                         out_row_width(inter, z_ld)) * 2;
  if (lds > 64 * 1024) return 1;
  const bool vec = entries_vec_ok(k, idx_dtype, idx, g_sparse, u_sparse, s_sparse) &&
                   reinterpret_cast<uintptr_t>(z_sparse) % 8 == 0;
#define MOC_BWDZ_NT(T, V, NT)                                                                        \
  backward_aux_rows_kernel<T, V, true, NT><<<dim3(static_cast<unsigned>(rows)), NT, lds, st>>>(       \
      (const T*)idx, (const uint16_t*)g_sparse, (const uint16_t*)u_sparse, (const uint16_t*)s_sparse, \
      (const uint16_t*)gz_full, gz_ld, (int)k, inter, (uint16_t*)grad_g, (uint16_t*)grad_u, out_ld,   \
      (const uint16_t*)z_sparse, (uint16_t*)z_full, z_ld)
#define MOC_BWDZ(T)                                                 \
  {                                                                 \
    if (inter <= kNarrowRow) {                                      \
      if (vec) MOC_BWDZ_NT(T, true, 128);                           \
      else MOC_BWDZ_NT(T, false, 128);                              \
    } else {                                                        \
      if (vec) MOC_BWDZ_NT(T, true, kRowThreadsBwd);                \
      else MOC_BWDZ_NT(T, false, kRowThreadsBwd);                   \
    }                                                               \
  }
  MOC_IDX_DISPATCH(idx_dtype, MOC_BWDZ);
#undef MOC_BWDZ
#undef MOC_BWDZ_NT
  return check_launch("backward_aux_rows_kernel (with Z)");
}

}  // namespace moc

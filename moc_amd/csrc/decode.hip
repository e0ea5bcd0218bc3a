// Global-MoC decode kernels (gfx950): a handful of tokens (nb <= 16) through
// one MoC FFN layer.  Every kernel here is bound by HBM bandwidth or by
// memory latency: the gate projection streams all of W_gate, the selected
// Up/Down kernels stream only the selected rows of W_up and W_down^T.
//
//  moc_gemv_bf16              gate projection G = x W_gate^T.  Up to 4
//                             tokens: one wave per row, whole rows in flight,
//                             f32 FMA.  More tokens: a workgroup owns <= 32
//                             consecutive rows, pulls all of them into LDS
//                             with direct-to-LDS loads in one go, then runs
//                             MFMA 16x16x32 (tokens padded to 16)
//  moc_global_after_gate_bf16 one launch: every workgroup of a token ranks
//                             the token's Top-K from G (radix select, lower
//                             index on ties), computes z = bf16(bf16(SiLU(g))
//                             bf16(x.W_up[c])) for its slice of the ranks and
//                             the Down contribution of that slice to its
//                             column block; partials are added in a fixed
//                             order by the last workgroup of each block
//  moc_selected_down_bf16     y[b] = sum_j z[b,j] W_down^T[idx[b,j]]: a
//                             workgroup per (64-column block, 128 selected
//                             rows), 128-byte row segments, partial sums
//                             reduced in a fixed order by the last workgroup
//                             of each column block to arrive
//  moc_selected_up_silu_bf16  one wave per (token, selected channel)
//
// Reference: moc/inference/cuda/optimized_global_moc_ext.cu:127-540 and the
// masked_reference oracle moc/inference/inference_ffn.py:169-180, whose
// rounding points (U, SiLU(G) and Z materialised in bf16) these kernels keep.
#include "abi.h"
#include "common.h"
#include "select.h"

extern "C" int moc_fill_zero(void* dst, int64_t bytes, void* stream);

namespace moc {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;

constexpr uint32_t kOob = 0x80000000u;  // buffer offset that reads as zero

template <typename IdxT>
__device__ __forceinline__ int64_t load_idx(const void* p, int64_t e) {
  return static_cast<int64_t>(static_cast<const IdxT*>(p)[e]);
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>((uintptr_t)((__attribute__((address_space(3))) const char*)p));
}

// One direct-to-LDS 16-byte load per lane (lane l -> LDS byte m0 + 16 l);
// the counter is waited for with an explicit vmcnt(0).
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, uint32_t m0, uint32_t voff) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen lds"
      :
      : "s"(m0), "v"(voff), "s"(rsrc)
      : "memory");
}

// ---------------------------------------------------------------------------
// Gate GEMV, streaming form.  Workgroup w owns rows [w*rows/nwg, ...) (<= 32).
// Row r of the workgroup sits at LDS byte r * 2*hidden; its 16-byte chunk c
// is stored in slot c ^ (r & 15), so the 16 lanes of an MFMA fragment read
// (16 rows, one chunk) hit 16 distinct bank groups.
// ---------------------------------------------------------------------------
constexpr int kGvMaxRows = 32;
constexpr int kGvLdsBytes = 128 * 1024;
constexpr int kGvMaxHidden = 2048;
constexpr int kGvMaxSteps = kGvMaxHidden / 32 / 4;  // k steps per wave

// Pair form (W2 != nullptr): workgroups nwg .. gridDim.x - 1 do the same for
// a second matrix W2 [rows2, hidden] into y2, so two projections of the same
// tokens stream in one launch.
__global__ __launch_bounds__(256) void gemv_stream_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int nb, const uint16_t* __restrict__ W,
    int64_t ldw, int rows, int hidden, int nwg, uint16_t* __restrict__ y, int64_t ldy,
    int wbytes, const uint16_t* __restrict__ W2, int64_t ldw2, int rows2, uint16_t* __restrict__ y2,
    int64_t ldy2, int wbytes2) {
  __shared__ __attribute__((aligned(1024))) char lw[kGvLdsBytes];
  __shared__ f32x4_t red[2][4][64];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int blk = static_cast<int>(blockIdx.x);
  if (W2 != nullptr && blk >= nwg) {
    blk -= nwg;
    nwg = static_cast<int>(gridDim.x) - nwg;
    W = W2;
    ldw = ldw2;
    rows = rows2;
    y = y2;
    ldy = ldy2;
    wbytes = wbytes2;
  }
  const int r_lo = static_cast<int>(static_cast<int64_t>(blk) * rows / nwg);
  const int r_hi = static_cast<int>(static_cast<int64_t>(blk + 1) * rows / nwg);
  const int nr = r_hi - r_lo;
  const int cpr = hidden / 8;  // 16-byte chunks per row (a multiple of 16)

  // 1. every chunk of the workgroup's rows in flight at once
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(W), (short)0, wbytes, 0x00020000);
  const uint32_t lbase = lds_addr(lw);
  const int ninstr = (nr * cpr + 63) / 64;
  // linear chunk q = 64 i + lane of the workgroup's rows -> (row r, slot s);
  // i advances by 4 per trip, so (r, s) advance by 256 chunks incrementally
  int r = (wave * 64 + lane) / cpr;
  int s = wave * 64 + lane - r * cpr;
  const uint32_t rowb = static_cast<uint32_t>(ldw * 2);
  uint32_t rowoff = static_cast<uint32_t>((static_cast<int64_t>(r_lo + r) * ldw) * 2);
  for (int i = wave; i < ninstr; i += 4) {
    const int c = s ^ (r & 15);
    const uint32_t off = (r < nr) ? rowoff + static_cast<uint32_t>(c * 16) : kOob;
    dma16(rs, __builtin_amdgcn_readfirstlane(lbase + i * 1024), off);
    s += 256;
    while (s >= cpr) {
      s -= cpr;
      ++r;
      rowoff += rowb;
    }
  }
  // the wave's x fragments (L2-resident) load while the rows stream in
  const int tok = lane & 15, kq = lane >> 4;
  const bool tok_ok = tok < nb;
  const uint16_t* xr = x + static_cast<int64_t>(tok_ok ? tok : 0) * ldx;
  const int steps = hidden / 32;
  const int s_lo = wave * steps / 4, s_hi = (wave + 1) * steps / 4;
  uint4 xf[kGvMaxSteps];
#pragma unroll
  for (int u = 0; u < kGvMaxSteps; ++u) {
    const int c = (s_lo + u) * 4 + kq;
    xf[u] = (tok_ok && s_lo + u < s_hi) ? *reinterpret_cast<const uint4*>(xr + c * 8)
                                        : make_uint4(0, 0, 0, 0);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  // 2. MFMA 16x16x32: A = W rows (lane: row l%16, k 8(l/16)..), B = x
  //    (lane: token l%16); the four waves split the k steps
  f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  const int r0 = lane & 15;
#pragma unroll
  for (int u = 0; u < kGvMaxSteps; ++u) {
    if (s_lo + u >= s_hi) break;
    const int c = (s_lo + u) * 4 + kq;
    const bf16x8_t xb = __builtin_bit_cast(bf16x8_t, xf[u]);
    const uint4 w0 = *reinterpret_cast<const uint4*>(lw + r0 * (2 * hidden) + ((c ^ r0) * 16));
    acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, w0), xb, acc0, 0, 0, 0);
    if (nr > 16) {
      const int r1 = 16 + r0;
      const uint4 w1 = *reinterpret_cast<const uint4*>(lw + r1 * (2 * hidden) + ((c ^ (r1 & 15)) * 16));
      acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, w1), xb, acc1, 0, 0, 0);
    }
  }
  red[0][wave][lane] = acc0;
  red[1][wave][lane] = acc1;
  __syncthreads();
  // 3. sum the four waves' partials in a fixed order; 16x16 accumulator
  //    layout: lane l element j -> row 4(l/16) + j, column (token) l%16
  if (wave < 2 && (wave == 0 || nr > 16)) {
    f32x4_t t = red[wave][0][lane];
#pragma unroll
    for (int w = 1; w < 4; ++w) {
      const f32x4_t o = red[wave][w][lane];
      t[0] += o[0]; t[1] += o[1]; t[2] += o[2]; t[3] += o[3];
    }
    if (tok_ok) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = 16 * wave + 4 * (lane >> 4) + j;
        if (r < nr) y[static_cast<int64_t>(tok) * ldy + r_lo + r] = f32_to_bf16(t[j]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Gate GEMV for 5..16 tokens, pipelined: one workgroup per CU walks a run of
// 16-row blocks (of W, then of W2 in the pair form).  A block's rows (64 KB
// at hidden 2048; chunk c of row r in slot c ^ (r & 15), as above) stream
// into one of two LDS buffers by direct-to-LDS loads while the previous block
// is multiplied (MFMA 16x16x32, the four waves splitting k as the streaming
// kernel does, so both give the same bits).  Every wave issues exactly
// kGpLoads loads per block (the ones past the block's bytes land in a sink),
// so the wait for a block is one constant vmcnt.
constexpr int kGpRows = 16;
constexpr int kGpMaxHidden = 2048;
constexpr int kGpBufBytes = kGpRows * 2 * kGpMaxHidden;          // 64 KB
constexpr int kGpLoads = kGpBufBytes / 1024 / 4;                 // per wave and block: 16
constexpr int kGpMaxSteps = kGpMaxHidden / 32 / 4;               // k steps per wave

__global__ __launch_bounds__(256) void gemv_pipe_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int nb, const uint16_t* __restrict__ W, int64_t ldw,
    int rows, int hidden, uint16_t* __restrict__ y, int64_t ldy, int wbytes, int nblk1, int nblk,
    const uint16_t* __restrict__ W2, int64_t ldw2, int rows2, uint16_t* __restrict__ y2, int64_t ldy2,
    int wbytes2) {
  __shared__ __attribute__((aligned(1024))) char lw[2 * kGpBufBytes + 1024];  // two buffers, a sink
  __shared__ f32x4_t red[4][64];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b_lo = static_cast<int>(static_cast<int64_t>(blockIdx.x) * nblk / gridDim.x);
  const int b_hi = static_cast<int>(static_cast<int64_t>(blockIdx.x + 1) * nblk / gridDim.x);
  const int cpr = hidden / 8;  // 16-byte chunks per row
  const __amdgpu_buffer_rsrc_t rs1 =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(W), (short)0, wbytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs2 =
      W2 != nullptr ? __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(W2), (short)0, wbytes2, 0x00020000)
                    : rs1;
  const uint32_t lbase = lds_addr(lw);
  // the loads of block bi into buffer buf
  // linear chunk q = 64 i + lane of a block -> (row rr, slot sl); i advances
  // by 4 per load, so (rr, sl) advance by 256 chunks incrementally
  const int q0 = wave * 64 + lane;
  const int rr0 = q0 / cpr, sl0 = q0 - rr0 * cpr;
  auto issue = [&](int bi, int buf) {
    const bool second = bi >= nblk1;
    const int r0 = (second ? bi - nblk1 : bi) * kGpRows;
    const int nr = min(kGpRows, (second ? rows2 : rows) - r0);
    const uint32_t rowb = static_cast<uint32_t>((second ? ldw2 : ldw) * 2);
    const int nq = (nr * cpr + 63) / 64;  // wave instructions that carry rows
    const __amdgpu_buffer_rsrc_t rs = second ? rs2 : rs1;
    int rr = rr0, sl = sl0;
    uint32_t rowoff = static_cast<uint32_t>(r0 + rr0) * rowb;
    for (int u = 0; u < kGpLoads; ++u) {
      const int i = wave + 4 * u;
      const bool real = i < nq;
      const uint32_t off = (real && rr < nr) ? rowoff + static_cast<uint32_t>(((sl ^ (rr & 15)) * 16)) : kOob;
      const uint32_t m0 = real ? lbase + buf * kGpBufBytes + i * 1024 : lbase + 2 * kGpBufBytes;
      dma16(rs, __builtin_amdgcn_readfirstlane(m0), off);
      sl += 256;
      while (sl >= cpr) {
        sl -= cpr;
        ++rr;
        rowoff += rowb;
      }
    }
  };
  // the wave's x fragments, kept for every block
  const int tok = lane & 15, kq = lane >> 4;
  const bool tok_ok = tok < nb;
  const uint16_t* xr = x + static_cast<int64_t>(tok_ok ? tok : 0) * ldx;
  const int steps = hidden / 32;
  const int s_lo = wave * steps / 4, s_hi = (wave + 1) * steps / 4;
  uint4 xf[kGpMaxSteps];
#pragma unroll
  for (int u = 0; u < kGpMaxSteps; ++u) {
    const int c = (s_lo + u) * 4 + kq;
    xf[u] = (tok_ok && s_lo + u < s_hi) ? *reinterpret_cast<const uint4*>(xr + c * 8) : make_uint4(0, 0, 0, 0);
  }
  if (b_lo < b_hi) issue(b_lo, 0);
  const int r0l = lane & 15;
  for (int bi = b_lo; bi < b_hi; ++bi) {
    const int buf = (bi - b_lo) & 1;
    if (bi + 1 < b_hi) {
      issue(bi + 1, buf ^ 1);
      asm volatile("s_waitcnt vmcnt(16)" ::: "memory");  // kGpLoads: block bi has landed
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();
    const char* lb = lw + buf * kGpBufBytes;
    uint4 wf[kGpMaxSteps];
#pragma unroll
    for (int u = 0; u < kGpMaxSteps; ++u) {
      const int c = (s_lo + u) * 4 + kq;
      wf[u] = s_lo + u < s_hi ? *reinterpret_cast<const uint4*>(lb + r0l * (2 * hidden) + ((c ^ r0l) * 16))
                              : make_uint4(0, 0, 0, 0);
    }
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < kGpMaxSteps; ++u)
      if (s_lo + u < s_hi)  // wave-uniform
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, wf[u]),
                                                      __builtin_bit_cast(bf16x8_t, xf[u]), acc, 0, 0, 0);
    red[wave][lane] = acc;
    __syncthreads();
    if (wave == 0 && tok_ok) {
      f32x4_t t = red[0][lane];
#pragma unroll
      for (int w = 1; w < 4; ++w) {
        const f32x4_t o = red[w][lane];
        t[0] += o[0]; t[1] += o[1]; t[2] += o[2]; t[3] += o[3];
      }
      const bool second = bi >= nblk1;
      const int r0 = (second ? bi - nblk1 : bi) * kGpRows;
      const int nrows = second ? rows2 : rows;
      uint16_t* yy = second ? y2 : y;
      const int64_t ly = second ? ldy2 : ldy;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = r0 + 4 * kq + j;
        if (row < nrows) yy[static_cast<int64_t>(tok) * ly + row] = f32_to_bf16(t[j]);
      }
    }
  }
}

// Fallback gate GEMV for shapes the streaming kernel does not take
// (hidden not a multiple of 128 or larger than the LDS row budget).
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
// Gate GEMV for 1..4 tokens: one wave per row, the whole row requested at
// once (lane l: 16-byte chunks l + 64 i), x in registers, f32 FMA dot
// products and a wave reduction.  With ~one row per wave every byte of W is
// in flight within one memory latency.
// ---------------------------------------------------------------------------
// NORM: the tokens go through RMSNorm first (the FFN's pre-norm,
// benchmark_decode.py:101-109,303): xn = bf16(bf16(x * r) * w) with
// r = 1 / sqrt(mean(x^2) + eps) in f32; every wave normalises its own copy
// of x, and wave 0 of workgroup 0 also writes xn for the kernels after it.
// Pair form (W2 != nullptr): the waves from row2_start on (a workgroup
// boundary) take the rows of a second matrix W2 [rows2, hidden] into y2 (two
// projections of the same tokens in one launch).
template <int NB, int CHN, bool NORM>
__global__ __launch_bounds__(256) void gemv_rows_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                        const uint16_t* __restrict__ W, int64_t ldw,
                                                        int rows, int hidden,
                                                        uint16_t* __restrict__ y, int64_t ldy,
                                                        const uint16_t* __restrict__ norm_w, float eps,
                                                        uint16_t* __restrict__ xn, int64_t ldxn,
                                                        const uint16_t* __restrict__ W2, int64_t ldw2,
                                                        int row2_start, int rows2, uint16_t* __restrict__ y2,
                                                        int64_t ldy2) {
  const int lane = threadIdx.x & 63;
  int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (W2 != nullptr && row >= row2_start) {
    row -= row2_start;
    rows = rows2;
    W = W2;
    ldw = ldw2;
    y = y2;
    ldy = ldy2;
  }
  if (row >= rows) return;
  const int nch = hidden / 8;
  uint4 wv[CHN];
#pragma unroll
  for (int i = 0; i < CHN; ++i) {
    const int c = lane + 64 * i;
    wv[i] = c < nch ? *reinterpret_cast<const uint4*>(W + static_cast<int64_t>(row) * ldw + c * 8)
                    : make_uint4(0, 0, 0, 0);
  }
  uint4 nwv[NORM ? CHN : 1];  // norm weight chunks, requested with the row
  if (NORM) {
#pragma unroll
    for (int i = 0; i < CHN; ++i) {
      const int c = lane + 64 * i;
      nwv[i] = c < nch ? *reinterpret_cast<const uint4*>(norm_w + c * 8) : make_uint4(0, 0, 0, 0);
    }
  }
  float acc[NB];
#pragma unroll
  for (int t = 0; t < NB; ++t) {
    acc[t] = 0.f;
    uint4 xv[CHN];
#pragma unroll
    for (int i = 0; i < CHN; ++i) {
      const int c = lane + 64 * i;
      xv[i] = c < nch ? *reinterpret_cast<const uint4*>(x + t * ldx + c * 8) : make_uint4(0, 0, 0, 0);
    }
    if (NORM) {
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < CHN; ++i) {
        const uint32_t a[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float lo = __uint_as_float(a[j] << 16), hi = __uint_as_float(a[j] & 0xFFFF0000u);
          ss = fmaf(lo, lo, ss);
          ss = fmaf(hi, hi, ss);
        }
      }
      const float r = rsqrtf(wave_sum(ss) / static_cast<float>(hidden) + eps);
#pragma unroll
      for (int i = 0; i < CHN; ++i) {
        const int c = lane + 64 * i;
        xv[i] = rmsnorm8(xv[i], nwv[NORM ? i : 0], r);
        if (blockIdx.x == 0 && threadIdx.x < 64 && c < nch)
          *reinterpret_cast<uint4*>(xn + t * ldxn + c * 8) = xv[i];
      }
    }
#pragma unroll
    for (int i = 0; i < CHN; ++i) acc[t] = dot8(wv[i], xv[i], acc[t]);
  }
#pragma unroll
  for (int t = 0; t < NB; ++t) {
    const float tot = wave_sum(acc[t]);
    if (lane == 0) y[t * ldy + row] = f32_to_bf16(tot);
  }
}

// The gate and up projections of the same channels in one wave: wave r
// requests row r of both W and W2 at once (two 4 KB rows at hidden 2048)
// and writes y[., r] and y2[., r].  Half the waves of the two-range pair
// form above, so the whole launch is resident in one round.  Same lane
// split, dot products and wave sums as gemv_rows_kernel: same bits.
template <int NB, int CHN>
__global__ __launch_bounds__(256) void gemv_dual_rows_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                             const uint16_t* __restrict__ W,
                                                             const uint16_t* __restrict__ W2, int64_t ldw,
                                                             int rows, int hidden, uint16_t* __restrict__ y,
                                                             uint16_t* __restrict__ y2, int64_t ldy) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int nch = hidden / 8;
  uint4 wv[CHN], wv2[CHN];
#pragma unroll
  for (int i = 0; i < CHN; ++i) {
    const int c = lane + 64 * i;
    const int64_t o = static_cast<int64_t>(row) * ldw + c * 8;
    wv[i] = c < nch ? *reinterpret_cast<const uint4*>(W + o) : make_uint4(0, 0, 0, 0);
    wv2[i] = c < nch ? *reinterpret_cast<const uint4*>(W2 + o) : make_uint4(0, 0, 0, 0);
  }
  float acc[NB], acc2[NB];
#pragma unroll
  for (int t = 0; t < NB; ++t) {
    acc[t] = 0.f;
    acc2[t] = 0.f;
#pragma unroll
    for (int i = 0; i < CHN; ++i) {
      const int c = lane + 64 * i;
      const uint4 xv = c < nch ? *reinterpret_cast<const uint4*>(x + t * ldx + c * 8) : make_uint4(0, 0, 0, 0);
      acc[t] = dot8(wv[i], xv, acc[t]);
      acc2[t] = dot8(wv2[i], xv, acc2[t]);
    }
  }
#pragma unroll
  for (int t = 0; t < NB; ++t) {
    const float tot = wave_sum(acc[t]), tot2 = wave_sum(acc2[t]);
    if (lane == 0) {
      y[t * ldy + row] = f32_to_bf16(tot);
      y2[t * ldy + row] = f32_to_bf16(tot2);
    }
  }
}

template <int NB>
void launch_gemv_dual_rows(const void* x, int64_t ldx, const void* W, const void* W2, int64_t ldw, int rows,
                           int hidden, void* y, void* y2, int64_t ldy, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>((rows + 3) / 4)), block(256);
  const int chn = (hidden / 8 + 63) / 64;
#define MOC_GD(C)                                                                                      \
  gemv_dual_rows_kernel<NB, C><<<grid, block, 0, st>>>((const uint16_t*)x, ldx, (const uint16_t*)W,     \
                                                       (const uint16_t*)W2, ldw, rows, hidden, (uint16_t*)y, \
                                                       (uint16_t*)y2, ldy)
  if (chn <= 1) MOC_GD(1);
  else if (chn <= 2) MOC_GD(2);
  else if (chn <= 4) MOC_GD(4);
  else MOC_GD(8);
#undef MOC_GD
}

template <int NB, bool NORM = false>
void launch_gemv_rows(const void* x, int64_t ldx, const void* W, int64_t ldw, int rows, int hidden,
                      void* y, int64_t ldy, hipStream_t st, const void* norm_w = nullptr,
                      float eps = 0.f, void* xn = nullptr, int64_t ldxn = 0, const void* W2 = nullptr,
                      int64_t ldw2 = 0, int rows2 = 0, void* y2 = nullptr, int64_t ldy2 = 0) {
  // the pair's second row range starts at a workgroup boundary
  const int wg1 = (rows + 3) / 4, wg2 = W2 != nullptr ? (rows2 + 3) / 4 : 0;
  const dim3 grid(static_cast<unsigned>(wg1 + wg2)), block(256);
  const int chn = (hidden / 8 + 63) / 64;
#define MOC_GR(C)                                                                                  \
  gemv_rows_kernel<NB, C, NORM><<<grid, block, 0, st>>>((const uint16_t*)x, ldx, (const uint16_t*)W, \
                                                         ldw, rows, hidden, (uint16_t*)y, ldy,       \
                                                         (const uint16_t*)norm_w, eps, (uint16_t*)xn, ldxn, \
                                                         (const uint16_t*)W2, ldw2, wg1 * 4, rows2, (uint16_t*)y2, \
                                                         ldy2)
  if (chn <= 1) MOC_GR(1);
  else if (chn <= 2) MOC_GR(2);
  else if (chn <= 4) MOC_GR(4);
  else MOC_GR(8);
#undef MOC_GR
}

// ---------------------------------------------------------------------------
// Decode after the gate, one launch.  Workgroup (b, p, cb): token b, slice p
// of P of the k selected ranks, column block cb of CB (CW = hidden / CB
// columns of y); about one workgroup per CU.
//  (0) token b's gate row, staged in LDS, as order keys in registers; the
//      k-th largest key and the ranks of the selected channels in ascending
//      channel order, ties toward the lower index (select.h; the same rule
//      and result as moc_topk_rows).  Every workgroup of the token ranks the
//      row itself (cheaper than a separate launch plus a round trip through
//      HBM) and keeps its ranks [p k / P, (p+1) k / P);
//  (1) the W_down^T row segments [cb CW, cb CW + CW) of the slice's channels
//      are requested first, then u = x_b . W_up[c] (whole rows, four
//      channels in flight per wave; or, with up_ld > 0, u read from the
//      token's dense U row that w_up then points to) and
//      z = bf16(bf16(SiLU(g)) * bf16(u));
//  (2) the segment sums over the slice are written to part[b][p] with
//      device-coherent stores; the last of the P workgroups of (b, cb) to
//      arrive adds the P partials in a fixed order and writes y[b, cb CW ..].
// The CB workgroups of one (b, p) are numbered nb P apart, so with nb P a
// multiple of 8 they share an XCD (and its L2) and read the W_up rows they
// all need from HBM once.  Arrival counters must be zero when a call starts;
// every call leaves them zero.
// ---------------------------------------------------------------------------
constexpr int kUdThreads = 512;
constexpr int kSelWaves = kUdThreads / 64;
constexpr int kSelCopies = 8;
constexpr int kFusedMaxSel = 256;  // ranks per workgroup (k / P)
constexpr int kUpPerWave = 4;      // W_up rows in flight per wave
constexpr int kDownBatch = 4;      // W_down^T segments in flight per thread

template <int L, int CW>
__global__ __launch_bounds__(kUdThreads) void select_up_down_kernel(
    const uint16_t* __restrict__ x, int hidden, const uint16_t* __restrict__ gate, int inter,
    int k, int P, int CB, const uint16_t* __restrict__ w_up, int64_t up_ld, const uint16_t* __restrict__ wdt,
    int64_t ldd,
    float* __restrict__ part, int* __restrict__ cnt, uint16_t* __restrict__ y,
    const uint16_t* __restrict__ res, int* __restrict__ idx_out) {
  constexpr int QN = CW / 8;            // 16-byte chunks per row segment
  constexpr int S = kUdThreads / QN;    // row segments summed in parallel
  static_assert(S * QN == kUdThreads, "CW / 8 must divide the workgroup");
  constexpr int NW = kUdThreads / 64;
  __shared__ __attribute__((aligned(16))) uint32_t sel_lds[select_lds_dwords<kSelWaves, kSelCopies>()];
  __shared__ __attribute__((aligned(16))) uint32_t row_lds[kUdThreads * L / 2];  // raw gate row
  __shared__ int sch[kFusedMaxSel];
  __shared__ float sv[kFusedMaxSel];  // bf16(SiLU(g)), then z
  __shared__ float red[S][CW + 1];
  __shared__ int last;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nbp = static_cast<int>(gridDim.x) / CB;
  const int cb = static_cast<int>(blockIdx.x) / nbp, bp = static_cast<int>(blockIdx.x) - cb * nbp;
  const int b = bp / P, p = bp - b * P;
  const int lo = static_cast<int>(static_cast<int64_t>(p) * k / P);
  const int hi = static_cast<int>(static_cast<int64_t>(p + 1) * k / P);
  const int nsel = hi - lo;

  // 0. selection; this workgroup's ranks [lo, hi)
  {
    const uint16_t* grow = gate + static_cast<int64_t>(b) * inter;
    const int c0 = tid * L;
    uint32_t w[sel_words<true, L>()];
    load_row_raw_staged<kSelWaves, true, L>(grow, inter, tid,
                                            (reinterpret_cast<uintptr_t>(grow) & 15) == 0, row_lds, w,
                                            false);
    raw_to_keys<true, L>(inter, c0, 0, [](uint32_t r) { return r; }, w);
    uint32_t thr, krem, take[(L + 31) / 32], first;
    select_threshold<kSelWaves, kSelCopies, sel_words<true, L>(), 16>(w, static_cast<uint32_t>(k),
                                                                      sel_lds, thr, krem);
    select_ranks<kSelWaves, kSelCopies, L, true>(w, thr, krem, sel_lds, take, first);
    // only threads holding ranks of the slice list their channels (ids
    // only: SiLU is taken where z is formed, in parallel)
    uint32_t cnt = 0;
#pragma unroll
    for (int d = 0; d < (L + 31) / 32; ++d) cnt += __popc(take[d]);
    if (static_cast<int>(first) < hi && static_cast<int>(first + cnt) > lo) {
      select_emit<L>(take, c0, first, [&](int c, uint32_t pos) {
        if (static_cast<int>(pos) >= lo && static_cast<int>(pos) < hi) sch[pos - lo] = c;
      });
    }
  }
  __syncthreads();
  const uint16_t* raw = reinterpret_cast<const uint16_t*>(row_lds);
  // the selection itself, written once per token (column block 0)
  if (idx_out != nullptr && cb == 0) {
    for (int e = tid; e < nsel; e += kUdThreads) idx_out[static_cast<int64_t>(b) * k + lo + e] = sch[e];
  }

  // 1. first batch of W_down^T segments in flight, then selected Up * SiLU
  const int q = tid % QN, sl = tid / QN;
  const int col = cb * CW + q * 8;
  uint4 dv[kDownBatch];
#pragma unroll
  for (int j = 0; j < kDownBatch; ++j) {
    const int e = sl + S * j;
    dv[j] = e < nsel ? *reinterpret_cast<const uint4*>(wdt + static_cast<int64_t>(sch[e]) * ldd + col)
                     : make_uint4(0, 0, 0, 0);
  }
  const int nch = hidden / 8;
  const uint16_t* xb = x + static_cast<int64_t>(b) * hidden;
  // z = bf16(bf16(SiLU(g)) * bf16(u))
  auto silu_g = [&](int e) { return round_bf16(silu_f32(bf16_to_f32(raw[sch[e]]))); };
  if (up_ld > 0) {  // w_up holds the tokens' dense U rows [nb, up_ld]
    for (int e = tid; e < nsel; e += kUdThreads)
      sv[e] = round_bf16(silu_g(e) * bf16_to_f32(w_up[static_cast<int64_t>(b) * up_ld + sch[e]]));
  }
  for (int e0 = wave * kUpPerWave; up_ld == 0 && e0 < nsel; e0 += kUpPerWave * NW) {
    float acc[kUpPerWave] = {};
    for (int cbase = 0; cbase < nch; cbase += 256) {
      uint4 wv[kUpPerWave][4], xv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = cbase + lane + 64 * i;
        xv[i] = c < nch ? *reinterpret_cast<const uint4*>(xb + c * 8) : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int u = 0; u < kUpPerWave; ++u) {
          const int e = e0 + u;
          wv[u][i] = (e < nsel && c < nch)
                         ? *reinterpret_cast<const uint4*>(w_up + static_cast<int64_t>(sch[e]) * hidden + c * 8)
                         : make_uint4(0, 0, 0, 0);
        }
      }
#pragma unroll
      for (int u = 0; u < kUpPerWave; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[u] = dot8(wv[u][i], xv[i], acc[u]);
    }
#pragma unroll
    for (int u = 0; u < kUpPerWave; ++u) {
      const float tot = wave_sum(acc[u]);
      const int e = e0 + u;
      if (lane == 0 && e < nsel) sv[e] = round_bf16(silu_g(e) * round_bf16(tot));
    }
  }
  __syncthreads();

  // 2. segment sums of z_e W_down^T[c_e, col .. col + 8) over this slot's e
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int e0 = 0; e0 < nsel; e0 += S * kDownBatch) {
    if (e0 > 0) {
#pragma unroll
      for (int j = 0; j < kDownBatch; ++j) {
        const int e = e0 + sl + S * j;
        dv[j] = e < nsel ? *reinterpret_cast<const uint4*>(wdt + static_cast<int64_t>(sch[e]) * ldd + col)
                         : make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int j = 0; j < kDownBatch; ++j) {
      const int e = e0 + sl + S * j;
      const float zz = e < nsel ? sv[e] : 0.f;
      const uint32_t a[4] = {dv[j].x, dv[j].y, dv[j].z, dv[j].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] = fmaf(zz, __uint_as_float(a[i] << 16), acc[2 * i]);
        acc[2 * i + 1] = fmaf(zz, __uint_as_float(a[i] & 0xFFFF0000u), acc[2 * i + 1]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) red[sl][q * 8 + i] = acc[i];
  __syncthreads();
  // Partials go through to the device-coherent level (agent-scope atomic
  // stores) and are waited for before the arrival count is bumped; the last
  // workgroup reads them back with agent-scope loads.
  if (tid < CW) {
    float t = 0.f;
    for (int r = 0; r < S; ++r) t += red[r][tid];
    __hip_atomic_store(part + static_cast<int64_t>(bp) * hidden + cb * CW + tid, t, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    const int prev = atomicAdd(&cnt[b * CB + cb], 1);
    last = (prev == P - 1);
  }
  __syncthreads();
  if (!last) return;
  // Thread (g, c) of G = 512 / CW groups sums partials p = g, g + G, ...
  // of column c, 16 independent loads in flight at a time; the G group sums
  // are then added in group order.
  {
    constexpr int G = kUdThreads / CW;
    constexpr int kLoads = 16;
    const int c = tid % CW, g = tid / CW;
    const float* p0 = part + static_cast<int64_t>(b) * P * hidden + cb * CW + c;
    float t = 0.f;
    for (int pi0 = g; pi0 < P; pi0 += G * kLoads) {
      float v[kLoads];
#pragma unroll
      for (int u = 0; u < kLoads; ++u) {
        const int pi = pi0 + G * u;
        v[u] = pi < P ? __hip_atomic_load(p0 + static_cast<int64_t>(pi) * hidden, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT)
                      : 0.f;
      }
#pragma unroll
      for (int u = 0; u < kLoads; ++u) t += v[u];
    }
    reinterpret_cast<float*>(red)[tid] = t;  // red holds S (CW + 1) >= 512 floats
  }
  __syncthreads();
  if (tid < CW) {
    constexpr int G = kUdThreads / CW;
    const float* flat = reinterpret_cast<const float*>(red);
    float t = 0.f;
#pragma unroll
    for (int g = 0; g < G; ++g) t += flat[g * CW + tid];
    const int64_t o = static_cast<int64_t>(b) * hidden + cb * CW + tid;
    // with a residual: the layer's x + FFN(x), both bf16 as in the reference
    // (benchmark_decode.py:303)
    y[o] = res ? f32_to_bf16(bf16_to_f32(res[o]) + round_bf16(t)) : f32_to_bf16(t);
  }
  if (tid == 0) cnt[b * CB + cb] = 0;  // ready for the next call
}

// ---------------------------------------------------------------------------
// Decode after the gate from the tokens' dense U rows (written together with
// G by the gate/up GEMV pair).  Workgroup (b, cb): token b and the CW output
// columns [cb CW, cb CW + CW), over every selected channel of the token.
//  (0) token b's G and U rows are staged in LDS with one round of loads; the
//      order keys of G and the selection as in select_up_down_kernel
//      (select.h), every selected channel listed in rank (= channel) order;
//  (1) thread (r, q) requests the W_down^T row segments (8 columns q of the
//      block) of the ranks r, r + R, ... (up to kSdBatch in flight), and
//      while they are in flight z_e = bf16(bf16(SiLU(g_c)) * bf16(u_c)) is
//      formed for every rank e, one rank per thread;
//  (2) y[b, cols] = sum_e z_e W_down^T[c_e, cols]: the R slot sums of each
//      column are added in slot order.
// Every workgroup of a token ranks the row itself; the output of a column
// block is summed inside one workgroup, so no partial sums, arrival counters
// or final-sum step follow (the selected-row kernel above needs all three:
// its workgroups split the ranks of a column block).  Workgroups are ordered
// so that the column blocks of one XCD are contiguous (CB a multiple of 8):
// the tokens' workgroups of a block, which read the same W_down^T rows where
// their selections meet, and blocks sharing 128-byte lines use one L2.
// Rows of G and U: pitch ld (a multiple of 8), 16-byte aligned; inter <=
// kSdMaxInter, k <= kSdMaxK; idx_out (optional) int32.
// G28 (MoC 2:8): the selection in (0) is the top 2 of every group of 8
// channels instead (select_group_top2_bits: the tie rule and the single
// rounding z = bf16(SiLU(g) u) of moc_grouped_top2_up_silu_bf16): thread t's
// L channels are whole groups, so group g's two channels become list
// entries 2g, 2g + 1 (top-1, then top-2: the reference's order) with their
// z, and no threshold, ranks, scan or step-(1) z pass are needed; k =
// inter / 4; idx_out (optional) int64.
// ---------------------------------------------------------------------------
constexpr int kSdThreads = 512;
constexpr int kSdMaxInter = 8192;
constexpr int kSdMaxK = 4096;
constexpr int kSdBatch = 16;

template <int L, int CW, bool G28>
__global__ __launch_bounds__(kSdThreads) void select_down_kernel(
    const uint16_t* __restrict__ gate, const uint16_t* __restrict__ up, int64_t ld, int inter, int k,
    int hidden, int CB, const uint16_t* __restrict__ wdt, int64_t ldd, uint16_t* __restrict__ y,
    const uint16_t* __restrict__ res, void* __restrict__ idx_out) {
  constexpr int NW = kSdThreads / 64;
  constexpr int CPT = L / 8;          // 16-byte chunks of a row per thread
  constexpr int Q = CW / 8;           // 16-byte chunks per row segment
  constexpr int R = kSdThreads / Q;   // rank slots summed in parallel
  static_assert(R * Q == kSdThreads && R * (CW + 1) >= kSdThreads, "CW / 8 must divide the workgroup");
  __shared__ __attribute__((aligned(16))) uint32_t sel_lds[select_lds_dwords<NW, kSelCopies>()];
  __shared__ __attribute__((aligned(16))) uint4 g_st[kSdThreads * CPT];
  __shared__ __attribute__((aligned(16))) uint4 u_st[kSdThreads * CPT];
  __shared__ uint16_t sch[kSdMaxK];
  __shared__ float zs[kSdMaxK];
  __shared__ float red[R][CW + 1];

  const int tid = threadIdx.x;
  int b, cb;
  if (CB % 8 == 0) {
    const int xcd = static_cast<int>(blockIdx.x) & 7, s = static_cast<int>(blockIdx.x) >> 3;
    const int per = CB / 8;
    cb = xcd * per + s % per;
    b = s / per;
  } else {
    b = static_cast<int>(blockIdx.x) / CB;
    cb = static_cast<int>(blockIdx.x) - b * CB;
  }

  // 0. the token's G and U rows in LDS, G's keys in registers, selection
  const uint4* g4 = reinterpret_cast<const uint4*>(gate + static_cast<int64_t>(b) * ld);
  const uint4* u4 = reinterpret_cast<const uint4*>(up + static_cast<int64_t>(b) * ld);
  const int nch = (inter + 7) / 8;
  {
    uint4 gv[CPT], uv[CPT];
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int ch = tid + kSdThreads * i;
      gv[i] = ch < nch ? g4[ch] : make_uint4(0, 0, 0, 0);
      uv[i] = ch < nch ? u4[ch] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      g_st[tid + kSdThreads * i] = gv[i];
      u_st[tid + kSdThreads * i] = uv[i];
    }
  }
  __syncthreads();
  if constexpr (G28) {
    const int c0 = tid * L;
    int64_t* io = (idx_out != nullptr && cb == 0) ? static_cast<int64_t*>(idx_out) + static_cast<int64_t>(b) * k
                                                   : nullptr;
#pragma unroll
    for (int q8 = 0; q8 < L / 8; ++q8) {
      const int c = c0 + 8 * q8;
      if (c < inter) {  // inter is a multiple of 8: whole groups
        const uint4 ga = g_st[c / 8], ua = u_st[c / 8];
        const uint32_t gw[4] = {ga.x, ga.y, ga.z, ga.w}, uw[4] = {ua.x, ua.y, ua.z, ua.w};
        int b1, b2;
        uint16_t s1, s2;
        select_group_top2_bits(gw, uw, b1, b2, s1, s2);
        const int e = c / 4;
        sch[e] = static_cast<uint16_t>(c + b1);
        sch[e + 1] = static_cast<uint16_t>(c + b2);
        zs[e] = bf16_to_f32(s1);
        zs[e + 1] = bf16_to_f32(s2);
        if (io != nullptr) {
          io[e] = c + b1;
          io[e + 1] = c + b2;
        }
      }
    }
  } else {
    const int c0 = tid * L;
    uint32_t w[sel_words<true, L>()];
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const uint4 a = g_st[tid * CPT + i];
      w[4 * i + 0] = a.x; w[4 * i + 1] = a.y; w[4 * i + 2] = a.z; w[4 * i + 3] = a.w;
    }
    raw_to_keys<true, L>(inter, c0, 0, [](uint32_t r) { return r; }, w);
    uint32_t thr, krem, take[(L + 31) / 32], first;
    select_threshold<NW, kSelCopies, sel_words<true, L>(), 16>(w, static_cast<uint32_t>(k), sel_lds, thr,
                                                               krem);
    select_ranks<NW, kSelCopies, L, true>(w, thr, krem, sel_lds, take, first);
    select_emit<L>(take, c0, first, [&](int c, uint32_t pos) { sch[pos] = static_cast<uint16_t>(c); });
  }
  __syncthreads();

  // 1. the first batch of W_down^T segments in flight, then z for every rank
  //    (and the selection itself, once per token)
  const int q = tid % Q, r = tid / Q;
  const int col = cb * CW + q * 8;
  uint4 dv[kSdBatch];
#pragma unroll
  for (int j = 0; j < kSdBatch; ++j) {
    const int e = r + R * j;
    dv[j] = e < k ? *reinterpret_cast<const uint4*>(wdt + static_cast<int64_t>(sch[e]) * ldd + col)
                  : make_uint4(0, 0, 0, 0);
  }
  if constexpr (!G28) {
    const uint16_t* graw = reinterpret_cast<const uint16_t*>(g_st);
    const uint16_t* uraw = reinterpret_cast<const uint16_t*>(u_st);
    int* io = (idx_out != nullptr && cb == 0) ? static_cast<int*>(idx_out) + static_cast<int64_t>(b) * k : nullptr;
    for (int e = tid; e < k; e += kSdThreads) {
      const int c = sch[e];
      zs[e] = round_bf16(round_bf16(silu_f32(bf16_to_f32(graw[c]))) * bf16_to_f32(uraw[c]));
      if (io != nullptr) io[e] = c;
    }
    __syncthreads();
  }

  // 2. column sums over the ranks
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int e0 = r;; e0 += R * kSdBatch) {
#pragma unroll
    for (int j = 0; j < kSdBatch; ++j) {
      const int e = e0 + R * j;
      const float zz = e < k ? zs[e] : 0.f;
      const uint32_t a[4] = {dv[j].x, dv[j].y, dv[j].z, dv[j].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] = fmaf(zz, __uint_as_float(a[i] << 16), acc[2 * i]);
        acc[2 * i + 1] = fmaf(zz, __uint_as_float(a[i] & 0xFFFF0000u), acc[2 * i + 1]);
      }
    }
    if (e0 + R * kSdBatch >= k) break;
#pragma unroll
    for (int j = 0; j < kSdBatch; ++j) {
      const int e = e0 + R * kSdBatch + R * j;
      dv[j] = e < k ? *reinterpret_cast<const uint4*>(wdt + static_cast<int64_t>(sch[e]) * ldd + col)
                    : make_uint4(0, 0, 0, 0);
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) red[r][q * 8 + i] = acc[i];
  __syncthreads();
  // thread (g, c) of G = 512 / CW groups adds the slots g, g + G, ... of
  // column c; then the G group sums in group order
  constexpr int G = kSdThreads / CW;
  {
    const int c = tid % CW, g = tid / CW;
    float t = 0.f;
    for (int rr = g; rr < R; rr += G) t += red[rr][c];
    __syncthreads();
    reinterpret_cast<float*>(red)[tid] = t;  // red holds R (CW + 1) >= 512 floats
  }
  __syncthreads();
  if (tid < CW) {
    const float* flat = reinterpret_cast<const float*>(red);
    float t = 0.f;
#pragma unroll
    for (int g = 0; g < G; ++g) t += flat[g * CW + tid];
    const int64_t o = static_cast<int64_t>(b) * hidden + cb * CW + tid;
    y[o] = res ? f32_to_bf16(bf16_to_f32(res[o]) + round_bf16(t)) : f32_to_bf16(t);
  }
}

// ---------------------------------------------------------------------------
// Selected Down.  Workgroup (cb, gg): columns [64 cb, 64 cb + 64) of y and
// group gg = b G + g of 128 selected rows of token b (G = ceil(k / 128)).
// Thread t: row slot t/8 (+32 per pass), 8 columns (16 bytes) at 8 (t%8).
// Column sums of the group go to part[gg][64 cb ..]; the last of the G
// workgroups of (b, cb) to arrive adds the G partials in group order.
// ---------------------------------------------------------------------------
constexpr int kDownRows = 128;

template <typename IdxT>
__global__ __launch_bounds__(256) void selected_down_kernel(
    const uint16_t* __restrict__ z, const void* __restrict__ idx, int k, int hidden,
    const uint16_t* __restrict__ wdt, int64_t ldd, int inter, int G, float* __restrict__ part,
    int* __restrict__ cnt, uint16_t* __restrict__ y, const uint16_t* __restrict__ res) {
  __shared__ float red[32][65];
  __shared__ int last;
  const int tid = threadIdx.x;
  const int cb = blockIdx.x, gg = blockIdx.y;
  const int b = gg / G, g = gg - b * G;
  const int rs = tid >> 3, q = tid & 7;
  const int col = cb * 64 + q * 8;
  const int64_t zb = static_cast<int64_t>(b) * k;

  int64_t ch[4];
  float zz[4];
#pragma unroll
  for (int ps = 0; ps < 4; ++ps) {
    const int j = g * kDownRows + ps * 32 + rs;
    const bool ok = j < k;
    ch[ps] = ok ? load_idx<IdxT>(idx, zb + j) : -1;
    zz[ps] = ok ? bf16_to_f32(z[zb + j]) : 0.f;
  }
  uint4 wv[4];
#pragma unroll
  for (int ps = 0; ps < 4; ++ps)
    wv[ps] = (ch[ps] >= 0 && ch[ps] < inter)
                 ? *reinterpret_cast<const uint4*>(wdt + ch[ps] * ldd + col)
                 : make_uint4(0, 0, 0, 0);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ps = 0; ps < 4; ++ps) {
    const uint32_t a[4] = {wv[ps].x, wv[ps].y, wv[ps].z, wv[ps].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] = fmaf(zz[ps], __uint_as_float(a[i] << 16), acc[2 * i]);
      acc[2 * i + 1] = fmaf(zz[ps], __uint_as_float(a[i] & 0xFFFF0000u), acc[2 * i + 1]);
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) red[rs][q * 8 + i] = acc[i];
  __syncthreads();
  // Partials are written through to the device-coherent level (agent-scope
  // atomic stores) and waited for before the arrival count is bumped; the
  // last workgroup reads them back with agent-scope loads.  No full L2
  // write-back or invalidate (what a __threadfence() costs) is needed.
  float* prow = part + static_cast<int64_t>(gg) * hidden + cb * 64;
  if (tid < 64) {
    float s = 0.f;
    for (int r = 0; r < 32; ++r) s += red[r][tid];
    __hip_atomic_store(prow + tid, s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    const int prev = atomicAdd(&cnt[b * (hidden / 64) + cb], 1);
    last = (prev == G - 1);
  }
  __syncthreads();
  if (!last) return;
  if (tid < 64) {
    const float* p0 = part + static_cast<int64_t>(b) * G * hidden + cb * 64 + tid;
    float s = 0.f;
    for (int gi = 0; gi < G; ++gi)
      s += __hip_atomic_load(p0 + static_cast<int64_t>(gi) * hidden, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    const int64_t o = static_cast<int64_t>(b) * hidden + cb * 64 + tid;
    // with a residual: the layer's x + FFN(x), both bf16 as in the reference
    y[o] = res ? f32_to_bf16(bf16_to_f32(res[o]) + round_bf16(s)) : f32_to_bf16(s);
  }
  if (tid == 0) cnt[b * (hidden / 64) + cb] = 0;  // ready for the next call
}

// ---------------------------------------------------------------------------
// Selected Up * SiLU from given (vals, idx): one wave per (token, channel).
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

bool idx_ok(int d) { return d == MOC_I16 || d == MOC_I32 || d == MOC_I64; }

inline int64_t align256(int64_t b) { return (b + 255) & ~int64_t(255); }

// Down workspace: partials [nb * G][hidden] f32, then counters [nb][hidden/64].
struct DownWs {
  int G;
  int64_t part_bytes, cnt_bytes;
};
inline DownWs down_ws(int64_t nb, int64_t k, int64_t hidden) {
  DownWs w;
  w.G = static_cast<int>((k + kDownRows - 1) / kDownRows);
  w.part_bytes = align256(nb * w.G * hidden * 4);
  w.cnt_bytes = align256(nb * (hidden / 64) * 4);
  return w;
}

int launch_selected_down(const void* z, const void* idx, int idx_dtype, int64_t nb, int64_t k,
                         const void* wdt, int64_t ldd, int64_t inter, int64_t hidden, void* y, void* ws,
                         hipStream_t st, const void* res = nullptr) {
  const DownWs w = down_ws(nb, k, hidden);
  float* part = static_cast<float*>(ws);
  int* cnt = reinterpret_cast<int*>(static_cast<char*>(ws) + w.part_bytes);
  const dim3 grid(static_cast<unsigned>(hidden / 64), static_cast<unsigned>(nb * w.G)), block(256);
#define MOC_DOWN(T)                                                                         \
  selected_down_kernel<T><<<grid, block, 0, st>>>((const uint16_t*)z, idx, (int)k, (int)hidden, \
                                                  (const uint16_t*)wdt, ldd, (int)inter, w.G, part, \
                                                  cnt, (uint16_t*)y, (const uint16_t*)res)
  if (idx_dtype == MOC_I16) MOC_DOWN(int16_t);
  else if (idx_dtype == MOC_I32) MOC_DOWN(int32_t);
  else MOC_DOWN(int64_t);
#undef MOC_DOWN
  return check_launch("selected_down_kernel");
}

// Launch shape: CW = 256 columns per block when hidden allows (else 64), P
// (a power of two, <= k, with k / P <= kFusedMaxSel) rank slices so that
// nb P CB is about 256 workgroups (one per CU).
struct FusedShape {
  int CW, CB, P;
};

inline FusedShape fused_shape(int64_t nb, int64_t k, int64_t hidden) {
  FusedShape f;
  f.CW = (hidden % 256 == 0) ? 256 : 64;
  f.CB = static_cast<int>(hidden / f.CW);
  int64_t P = 256 / (nb * f.CB);
  int64_t p2 = 1;
  while (p2 * 2 <= P) p2 *= 2;
  P = p2 < 1 ? 1 : p2;
  while ((k + P - 1) / P > kFusedMaxSel) P *= 2;
  if (P > k) P = k;
  f.P = static_cast<int>(P);
  return f;
}

template <int CW>
void launch_fused(const void* x, int hidden, const void* gate, int inter, int k, int nb,
                  const FusedShape& f, const void* w_up, int64_t up_ld, const void* wdt, int64_t ldd,
                  float* part, int* cnt, void* y, const void* res, int* idx_out, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(nb * f.P * f.CB)), block(kUdThreads);
  const int per = (inter + kUdThreads - 1) / kUdThreads;
#define MOC_FU(N)                                                                               \
  select_up_down_kernel<N, CW><<<grid, block, 0, st>>>((const uint16_t*)x, hidden,               \
                                                       (const uint16_t*)gate, inter, k, f.P, f.CB, \
                                                       (const uint16_t*)w_up, up_ld, (const uint16_t*)wdt, \
                                                       ldd, part, cnt, (uint16_t*)y, (const uint16_t*)res, \
                                                       idx_out)
  if (per <= 8) MOC_FU(8);
  else if (per <= 16) MOC_FU(16);
  else if (per <= 24) MOC_FU(24);
  else MOC_FU(32);
#undef MOC_FU
}

// Column-owning after-gate launch (select_down_kernel), CW columns per
// workgroup.
template <int CW, bool G28 = false>
void launch_select_down_cw(const void* g, const void* u, int64_t ld, int nb, int inter, int k, int hidden,
                           const void* wdt, int64_t ldd, void* y, const void* res, void* idx_out,
                           hipStream_t st) {
  const int CB = hidden / CW;
  const dim3 grid(static_cast<unsigned>(nb * CB)), block(kSdThreads);
  const int per = (inter + kSdThreads - 1) / kSdThreads;
#define MOC_SD(N)                                                                                  \
  select_down_kernel<N, CW, G28><<<grid, block, 0, st>>>((const uint16_t*)g, (const uint16_t*)u, ld, inter, k, \
                                                     hidden, CB, (const uint16_t*)wdt, ldd, (uint16_t*)y, \
                                                     (const uint16_t*)res, idx_out)
  if (per <= 8) MOC_SD(8);
  else MOC_SD(16);
#undef MOC_SD
}

}  // namespace
}  // namespace moc

using namespace moc;

namespace moc {
// One GEMV launch for W [rows, hidden] -> y, or (W2 != nullptr) for W and a
// second matrix W2 [rows2, hidden] -> y2 of the same tokens; shapes checked
// by the callers.  The streaming form needs each matrix within 2 GiB.
int gemv_launch(const void* x, int64_t ldx, int64_t nb, const void* W, int64_t ldw, int64_t rows,
                int64_t hidden, void* y, int64_t ldy, const void* W2, int64_t ldw2, int64_t rows2, void* y2,
                int64_t ldy2, hipStream_t st) {
  if (nb <= 4 && hidden <= 4096) {
    switch (nb) {
      case 1: launch_gemv_rows<1>(x, ldx, W, ldw, (int)rows, (int)hidden, y, ldy, st, nullptr, 0.f, nullptr, 0, W2, ldw2, (int)rows2, y2, ldy2); break;
      case 2: launch_gemv_rows<2>(x, ldx, W, ldw, (int)rows, (int)hidden, y, ldy, st, nullptr, 0.f, nullptr, 0, W2, ldw2, (int)rows2, y2, ldy2); break;
      case 3: launch_gemv_rows<3>(x, ldx, W, ldw, (int)rows, (int)hidden, y, ldy, st, nullptr, 0.f, nullptr, 0, W2, ldw2, (int)rows2, y2, ldy2); break;
      default: launch_gemv_rows<4>(x, ldx, W, ldw, (int)rows, (int)hidden, y, ldy, st, nullptr, 0.f, nullptr, 0, W2, ldw2, (int)rows2, y2, ldy2); break;
    }
    return check_launch("gemv_rows_kernel");
  }
  const int64_t wbytes = rows * ldw * 2, wbytes2 = W2 != nullptr ? rows2 * ldw2 * 2 : 0;
  // the pair (gate and dense U, ~2.7 blocks of 16 rows per CU) on the
  // pipelined kernel: 35.3 -> 30.9 us per 16-token layer, 31.6 -> 27.9 at 8;
  // one projection (~1.3 blocks per CU, nothing to overlap) stays on the
  // streaming kernel (8.9 against 9.6 us at 16 tokens); both give the same bits
  if (W2 != nullptr && hidden % 128 == 0 && hidden <= kGpMaxHidden && wbytes < (1LL << 31) - 1024 &&
      wbytes2 < (1LL << 31) - 1024) {
    const int64_t nblk1 = (rows + kGpRows - 1) / kGpRows;
    const int64_t nblk = nblk1 + (W2 != nullptr ? (rows2 + kGpRows - 1) / kGpRows : 0);
    const int64_t grid = std::min<int64_t>(nblk, cu_count());
    gemv_pipe_kernel<<<dim3(static_cast<unsigned>(grid)), 256, 0, st>>>(
        (const uint16_t*)x, ldx, (int)nb, (const uint16_t*)W, ldw, (int)rows, (int)hidden, (uint16_t*)y, ldy,
        (int)wbytes, (int)nblk1, (int)nblk, (const uint16_t*)W2, ldw2, (int)rows2, (uint16_t*)y2, ldy2,
        (int)wbytes2);
    return check_launch("gemv_pipe_kernel");
  }
  const int64_t max_rows = kGvLdsBytes / (2 * hidden);
  if (hidden % 128 == 0 && hidden <= kGvMaxHidden && max_rows >= 16 && wbytes < (1LL << 31) - 1024 &&
      wbytes2 < (1LL << 31) - 1024) {
    // balanced split over >= 256 workgroups (per matrix) with <= min(32,
    // max_rows) rows each
    const int64_t cap = max_rows < kGvMaxRows ? max_rows : kGvMaxRows;
    auto split = [&](int64_t r) {
      int64_t n = (r + cap - 1) / cap;
      if (n < 256) n = r < 256 ? r : 256;
      return n;
    };
    const int64_t nwg = split(rows), nwg2 = W2 != nullptr ? split(rows2) : 0;
    gemv_stream_kernel<<<dim3(static_cast<unsigned>(nwg + nwg2)), 256, 0, st>>>(
        (const uint16_t*)x, ldx, (int)nb, (const uint16_t*)W, ldw, (int)rows, (int)hidden,
        (int)nwg, (uint16_t*)y, ldy, (int)wbytes, (const uint16_t*)W2, ldw2, (int)rows2, (uint16_t*)y2, ldy2,
        (int)wbytes2);
    return check_launch("gemv_stream_kernel");
  }
  const dim3 grid(static_cast<unsigned>((rows + 15) / 16)), block(256);
  gemv16_kernel<<<grid, block, 0, st>>>((const uint16_t*)x, ldx, (int)nb, (const uint16_t*)W, ldw,
                                        (int)rows, (int)hidden, (uint16_t*)y, ldy);
  int rc = check_launch("gemv16_kernel");
  if (rc != MOC_OK || W2 == nullptr) return rc;
  const dim3 grid2(static_cast<unsigned>((rows2 + 15) / 16));
  gemv16_kernel<<<grid2, block, 0, st>>>((const uint16_t*)x, ldx, (int)nb, (const uint16_t*)W2, ldw2,
                                         (int)rows2, (int)hidden, (uint16_t*)y2, ldy2);
  return check_launch("gemv16_kernel");
}
}  // namespace moc

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
  return gemv_launch(x, ldx, nb, W, ldw, rows, hidden, y, ldy, nullptr, 0, 0, nullptr, 0, as_stream(stream));
}

extern "C" int moc_gemv_rmsnorm_bf16(const void* x, int64_t ldx, int64_t nb, const void* norm_w,
                                     float eps, void* xn, int64_t ldxn, const void* W, int64_t ldw,
                                     int64_t rows, int64_t hidden, void* y, int64_t ldy, void* stream) {
  MOC_REQUIRE(nb >= 0 && nb <= 4, "moc_gemv_rmsnorm_bf16: 0 <= nb <= 4 tokens (got %lld)", (long long)nb);
  MOC_REQUIRE(rows >= 0 && rows < (1LL << 31) && hidden >= 8 && hidden <= 4096 && hidden % 8 == 0,
              "moc_gemv_rmsnorm_bf16: hidden must be a multiple of 8 in [8, 4096]");
  MOC_REQUIRE(ldx >= hidden && ldw >= hidden && ldy >= rows && ldxn >= hidden,
              "moc_gemv_rmsnorm_bf16: bad leading dimension");
  MOC_REQUIRE(ldx % 8 == 0 && ldw % 8 == 0 && ldxn % 8 == 0,
              "moc_gemv_rmsnorm_bf16: ldx/ldw/ldxn must be multiples of 8");
  MOC_REQUIRE(eps >= 0.f, "moc_gemv_rmsnorm_bf16: eps must be >= 0");
  if (nb == 0 || rows == 0) return MOC_OK;
  MOC_REQUIRE(x && norm_w && xn && W && y, "moc_gemv_rmsnorm_bf16: null pointer");
  MOC_REQUIRE(aligned16(x) && aligned16(W) && aligned16(norm_w) && aligned16(xn),
              "moc_gemv_rmsnorm_bf16: x, norm_w, xn and W must be 16-byte aligned");
  hipStream_t st = as_stream(stream);
  switch (nb) {
    case 1: launch_gemv_rows<1, true>(x, ldx, W, ldw, (int)rows, (int)hidden, y, ldy, st, norm_w, eps, xn, ldxn); break;
    case 2: launch_gemv_rows<2, true>(x, ldx, W, ldw, (int)rows, (int)hidden, y, ldy, st, norm_w, eps, xn, ldxn); break;
    case 3: launch_gemv_rows<3, true>(x, ldx, W, ldw, (int)rows, (int)hidden, y, ldy, st, norm_w, eps, xn, ldxn); break;
    default: launch_gemv_rows<4, true>(x, ldx, W, ldw, (int)rows, (int)hidden, y, ldy, st, norm_w, eps, xn, ldxn); break;
  }
  return check_launch("gemv_rows_kernel (rmsnorm)");
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
  const DownWs w = down_ws(nb, k, hidden);
  return w.part_bytes + w.cnt_bytes;
}

namespace moc {
int selected_down_impl(const void* z, const void* idx, int idx_dtype, int64_t nb, int64_t k,
                       const void* w_down_t, int64_t ldw_down, int64_t inter, int64_t hidden, const void* res,
                       void* y, void* workspace, int64_t workspace_bytes, void* stream) {
  MOC_REQUIRE(idx_ok(idx_dtype), "moc_selected_down_bf16: bad index dtype");
  MOC_REQUIRE(nb >= 0 && k >= 1 && inter >= 1 && hidden >= 1, "moc_selected_down_bf16: bad shape");
  MOC_REQUIRE(hidden % 64 == 0, "moc_selected_down_bf16: hidden must be a multiple of 64");
  MOC_REQUIRE(nb <= 65535 && nb * k < (1LL << 31), "moc_selected_down_bf16: too many rows");
  if (nb == 0) return MOC_OK;
  MOC_REQUIRE(z && idx && w_down_t && y, "moc_selected_down_bf16: null pointer");
  MOC_REQUIRE(aligned16(w_down_t), "moc_selected_down_bf16: w_down_t must be 16-byte aligned");
  MOC_REQUIRE(ldw_down >= hidden && ldw_down % 8 == 0,
              "moc_selected_down_bf16: ldw_down must be a multiple of 8 and >= hidden");
  const int64_t need = moc_selected_down_workspace_size(nb, k, hidden);
  MOC_REQUIRE(workspace != nullptr && workspace_bytes >= need,
              "moc_selected_down_bf16: workspace of %lld bytes required", (long long)need);
  const DownWs w = down_ws(nb, k, hidden);
  int rc = moc_fill_zero(static_cast<char*>(workspace) + w.part_bytes, w.cnt_bytes, stream);
  if (rc != MOC_OK) return rc;
  return launch_selected_down(z, idx, idx_dtype, nb, k, w_down_t, ldw_down, inter, hidden, y, workspace,
                              as_stream(stream), res);
}
}  // namespace moc

extern "C" int moc_selected_down_bf16(const void* z, const void* idx, int idx_dtype, int64_t nb,
                                      int64_t k, const void* w_down_t, int64_t ldw_down, int64_t inter,
                                      int64_t hidden, void* y, void* workspace,
                                      int64_t workspace_bytes, void* stream) {
  return selected_down_impl(z, idx, idx_dtype, nb, k, w_down_t, ldw_down, inter, hidden, nullptr, y, workspace,
                            workspace_bytes, stream);
}

// Workspace: a fixed 64 KB block of arrival counters (so the counters of one
// call shape never overlap other data of another shape that reuses the
// workspace), then the partial sums.
constexpr int64_t kFusedCounterBytes = kAfterGateCounterBytes;

// From this many tokens on, U = x W_up^T is computed densely for all
// channels by the gate GEMV kernel before the after-gate kernel: the union of
// the tokens' selections then covers most channels (about 3080 of 5461 at 4
// tokens of the 1b shape, 5250 at 16), so one streaming pass over W_up
// replaces every column block re-reading each token's selected rows
// (measured at the 1b shape: 4 tokens 33.9 -> 31.2 us, 16 tokens 61.7 ->
// 37.5 us per layer; 2 tokens stay faster without it).
constexpr int64_t kDenseUpMinTokens = 4;

inline int64_t dense_up_bytes(int64_t nb, int64_t inter) {
  return nb >= kDenseUpMinTokens ? ((nb * inter * 2 + 255) / 256) * 256 : 0;
}

extern "C" int64_t moc_global_after_gate_workspace_size(int64_t nb, int64_t inter, int64_t k,
                                                        int64_t hidden) {
  if (nb <= 0 || k <= 0 || hidden < 64 || inter <= 0) return 0;
  const FusedShape f = fused_shape(nb, k, hidden);
  return kFusedCounterBytes + nb * f.P * hidden * 4 + dense_up_bytes(nb, inter);
}

namespace moc {
int global_after_gate(const void* x, const void* gate_scores, int64_t nb, int64_t inter, int64_t hidden,
                      const void* w_up, const void* w_down_t, int64_t ldw_down, int64_t k, const void* res,
                      void* y, void* idx_out, void* workspace, int64_t workspace_bytes, void* stream,
                      bool up_ready) {
  MOC_REQUIRE(nb >= 0 && nb <= 16, "moc_global_after_gate_bf16: 0 <= nb <= 16 tokens");
  MOC_REQUIRE(inter >= 1 && inter <= 16384 && hidden >= 64, "moc_global_after_gate_bf16: bad shape");
  MOC_REQUIRE(hidden % 64 == 0, "moc_global_after_gate_bf16: hidden must be a multiple of 64");
  MOC_REQUIRE(k >= 1 && k <= inter, "invalid k");
  if (nb == 0) return MOC_OK;
  MOC_REQUIRE(x && gate_scores && w_up && w_down_t && y, "moc_global_after_gate_bf16: null pointer");
  MOC_REQUIRE(aligned16(x) && aligned16(w_up) && aligned16(w_down_t),
              "moc_global_after_gate_bf16: x and weights must be 16-byte aligned");
  MOC_REQUIRE(ldw_down >= hidden && ldw_down % 8 == 0,
              "moc_global_after_gate_bf16: ldw_down must be a multiple of 8 and >= hidden");
  const int64_t need = moc_global_after_gate_workspace_size(nb, inter, k, hidden);
  MOC_REQUIRE(workspace != nullptr && workspace_bytes >= need,
              "moc_global_after_gate_bf16: workspace of %lld bytes required", (long long)need);
  const FusedShape f = fused_shape(nb, k, hidden);
  MOC_REQUIRE(nb * f.CB * 4 <= kFusedCounterBytes, "moc_global_after_gate_bf16: hidden too large");
  char* ws = static_cast<char*>(workspace);
  int* cnt = reinterpret_cast<int*>(ws);
  float* part = reinterpret_cast<float*>(ws + kFusedCounterBytes);
  hipStream_t st = as_stream(stream);
  const void* up = w_up;
  int64_t up_ld = 0;
  if (dense_up_bytes(nb, inter) > 0) {
    // up_ready: the caller's pair GEMV has already written U there
    void* u = ws + kFusedCounterBytes + nb * f.P * hidden * 4;
    if (!up_ready) {
      const int rc = moc_gemv_bf16(x, hidden, nb, w_up, hidden, inter, hidden, u, inter, stream);
      if (rc != MOC_OK) return rc;
    }
    up = u;
    up_ld = inter;
  }
  int* io = static_cast<int*>(idx_out);
  if (f.CW == 256)
    launch_fused<256>(x, (int)hidden, gate_scores, (int)inter, (int)k, (int)nb, f, up, up_ld, w_down_t,
                      ldw_down, part, cnt, y, res, io, st);
  else
    launch_fused<64>(x, (int)hidden, gate_scores, (int)inter, (int)k, (int)nb, f, up, up_ld, w_down_t,
                     ldw_down, part, cnt, y, res, io, st);
  return check_launch("select_up_down_kernel");
}
}  // namespace moc

extern "C" int moc_global_after_gate_bf16(const void* x, const void* gate_scores, int64_t nb,
                                          int64_t inter, int64_t hidden, const void* w_up,
                                          const void* w_down_t, int64_t ldw_down, int64_t k, void* y,
                                          void* idx_out, void* workspace, int64_t workspace_bytes,
                                          void* stream) {
  return global_after_gate(x, gate_scores, nb, inter, hidden, w_up, w_down_t, ldw_down, k, nullptr, y, idx_out,
                           workspace, workspace_bytes, stream);
}

// The whole decode layer from x.  Where select_down_kernel fits the shape:
// G and the dense U of every token in one GEMV launch (two projections of
// one x stream), then the column-owning after-gate kernel; G and U rows at
// a pitch of a multiple of 8, after the after-gate workspace's counters
// (which this path leaves as they are).  Otherwise: the gate projection
// (with, from 4 tokens on, the dense U in the same launch), then
// select_up_down_kernel; workspace: the after-gate workspace, then G.
namespace {
inline int64_t sd_pitch(int64_t inter) { return (inter + 7) / 8 * 8; }

inline bool sd_fits(int64_t nb, int64_t inter, int64_t k, int64_t hidden) {
  return nb >= 1 && nb <= 16 && inter <= kSdMaxInter && k <= kSdMaxK && hidden % 256 == 0;
}
}  // namespace

namespace {
// The column-owning layer: G and U of every token (of RMSNorm(x) when
// norm_w != nullptr) in one GEMV launch, then select_down_kernel (with the
// residual added when res != nullptr).  Workspace after the counters: U, G
// (pitch sd_pitch(inter)), then xn [nb, hidden].  g28: the MoC 2:8
// selection (top 2 of every 8 channels, k = inter / 4, idx_out int64) in
// place of the global Top-K (idx_out int32).
int global_decode_sd(const void* x, int64_t nb, int64_t hidden, const void* norm_w, float eps,
                     const void* w_gate, const void* w_up, int64_t inter, const void* w_down_t, int64_t ldw_down,
                     int64_t k, const void* res, void* y, void* idx_out, char* ws, hipStream_t st,
                     bool g28 = false) {
  const int64_t pitch = sd_pitch(inter);
  void* u = ws + kFusedCounterBytes;
  void* gs = ws + kFusedCounterBytes + align256(nb * pitch * 2);
  void* xn = ws + kFusedCounterBytes + 2 * align256(nb * pitch * 2);
  const int in = static_cast<int>(inter), hd = static_cast<int>(hidden);
  int rc;
  if (norm_w != nullptr) {
    // gate rows, then the up rows as the pair's second range; every wave
    // normalises its own copy of x (nb <= 4, checked by the caller)
    switch (nb) {
      case 1: launch_gemv_rows<1, true>(x, hidden, w_gate, hidden, in, hd, gs, pitch, st, norm_w, eps, xn, hidden, w_up, hidden, in, u, pitch); break;
      case 2: launch_gemv_rows<2, true>(x, hidden, w_gate, hidden, in, hd, gs, pitch, st, norm_w, eps, xn, hidden, w_up, hidden, in, u, pitch); break;
      case 3: launch_gemv_rows<3, true>(x, hidden, w_gate, hidden, in, hd, gs, pitch, st, norm_w, eps, xn, hidden, w_up, hidden, in, u, pitch); break;
      default: launch_gemv_rows<4, true>(x, hidden, w_gate, hidden, in, hd, gs, pitch, st, norm_w, eps, xn, hidden, w_up, hidden, in, u, pitch); break;
    }
    rc = check_launch("gemv_rows_kernel");
  } else if (nb >= 3 && nb <= 4 && hidden <= 4096) {
    // 3-4 tokens: one wave per (gate row, up row) pair measured faster
    // (4 tokens 24.3 -> 23.1 us per layer); 1-2 tokens: the two-range form
    if (nb == 3) launch_gemv_dual_rows<3>(x, hidden, w_gate, w_up, hidden, in, hd, gs, u, pitch, st);
    else launch_gemv_dual_rows<4>(x, hidden, w_gate, w_up, hidden, in, hd, gs, u, pitch, st);
    rc = check_launch("gemv_dual_rows_kernel");
  } else {
    rc = gemv_launch(x, hidden, nb, w_gate, hidden, inter, hidden, gs, pitch, w_up, hidden, inter, u, pitch, st);
  }
  if (rc != MOC_OK) return rc;
  // 16 columns per workgroup for one token (128 workgroups at hidden 2048:
  // a quarter of the W_down^T bytes through each CU; 64 columns 18.42, 32
  // 18.21-18.28, 16 18.11-18.13 us per layer), 32 for 2-4 tokens (64
  // against 32: 19.80-19.83 -> 19.65 us at 2, 22.07-22.09 -> 21.98-22.00 at
  // 4), 64 up to 8 tokens (<= 256 workgroups), 128 beyond (12-16 tokens:
  // 32.0-32.5 -> 26.5-26.9 us per layer)
  if (g28 && nb == 1)
    launch_select_down_cw<16, true>(gs, u, pitch, (int)nb, in, (int)k, hd, w_down_t, ldw_down, y, res, idx_out, st);
  else if (!g28 && nb == 1)
    launch_select_down_cw<16>(gs, u, pitch, (int)nb, in, (int)k, hd, w_down_t, ldw_down, y, res, idx_out, st);
  else if (g28 && nb <= 4)
    launch_select_down_cw<32, true>(gs, u, pitch, (int)nb, in, (int)k, hd, w_down_t, ldw_down, y, res, idx_out, st);
  else if (!g28 && nb <= 4)
    launch_select_down_cw<32>(gs, u, pitch, (int)nb, in, (int)k, hd, w_down_t, ldw_down, y, res, idx_out, st);
  else if (g28 && nb <= 8)
    launch_select_down_cw<64, true>(gs, u, pitch, (int)nb, in, (int)k, hd, w_down_t, ldw_down, y, res, idx_out, st);
  else if (g28)
    launch_select_down_cw<128, true>(gs, u, pitch, (int)nb, in, (int)k, hd, w_down_t, ldw_down, y, res, idx_out, st);
  else if (nb <= 8)
    launch_select_down_cw<64>(gs, u, pitch, (int)nb, in, (int)k, hd, w_down_t, ldw_down, y, res, idx_out, st);
  else
    launch_select_down_cw<128>(gs, u, pitch, (int)nb, in, (int)k, hd, w_down_t, ldw_down, y, res, idx_out, st);
  return check_launch("select_down_kernel");
}
}  // namespace

extern "C" int64_t moc_global_decode_workspace_size(int64_t nb, int64_t inter, int64_t k, int64_t hidden) {
  const int64_t a = moc_global_after_gate_workspace_size(nb, inter, k, hidden);
  if (a <= 0) return 0;
  const int64_t legacy = a + align256(nb * inter * 2);
  const int64_t sd = kFusedCounterBytes + 2 * align256(nb * sd_pitch(inter) * 2) + align256(nb * hidden * 2);
  return legacy > sd ? legacy : sd;
}

extern "C" int moc_global_decode_bf16(const void* x, int64_t nb, int64_t hidden, const void* w_gate,
                                      const void* w_up, int64_t inter, const void* w_down_t, int64_t ldw_down,
                                      int64_t k, void* y, void* idx_out, void* workspace,
                                      int64_t workspace_bytes, void* stream) {
  MOC_REQUIRE(nb >= 0 && nb <= 16, "moc_global_decode_bf16: 0 <= nb <= 16 tokens");
  MOC_REQUIRE(inter >= 1 && inter <= 16384 && hidden >= 64 && hidden % 64 == 0 && hidden < (1LL << 30),
              "moc_global_decode_bf16: bad shape");
  MOC_REQUIRE(k >= 1 && k <= inter, "invalid k");
  if (nb == 0) return MOC_OK;
  MOC_REQUIRE(x && w_gate && w_up && w_down_t && y, "moc_global_decode_bf16: null pointer");
  MOC_REQUIRE(aligned16(x) && aligned16(w_gate) && aligned16(w_up) && aligned16(w_down_t),
              "moc_global_decode_bf16: x and weights must be 16-byte aligned");
  MOC_REQUIRE(ldw_down >= hidden && ldw_down % 8 == 0,
              "moc_global_decode_bf16: ldw_down must be a multiple of 8 and >= hidden");
  const int64_t need = moc_global_decode_workspace_size(nb, inter, k, hidden);
  MOC_REQUIRE(workspace != nullptr && workspace_bytes >= need,
              "moc_global_decode_bf16: workspace of %lld bytes required", (long long)need);
  const int64_t abytes = moc_global_after_gate_workspace_size(nb, inter, k, hidden);
  char* ws = static_cast<char*>(workspace);
  hipStream_t st = as_stream(stream);
  int rc;
  if (sd_fits(nb, inter, k, hidden))
    return global_decode_sd(x, nb, hidden, nullptr, 0.f, w_gate, w_up, inter, w_down_t, ldw_down, k, nullptr, y,
                            idx_out, ws, st);
  void* g = ws + abytes;
  const bool pair = dense_up_bytes(nb, inter) > 0;
  if (pair) {
    const FusedShape f = fused_shape(nb, k, hidden);
    void* u = ws + kFusedCounterBytes + nb * f.P * hidden * 4;
    rc = gemv_launch(x, hidden, nb, w_gate, hidden, inter, hidden, g, inter, w_up, hidden, inter, u, inter, st);
  } else {
    rc = gemv_launch(x, hidden, nb, w_gate, hidden, inter, hidden, g, inter, nullptr, 0, 0, nullptr, 0, st);
  }
  if (rc != MOC_OK) return rc;
  return global_after_gate(x, g, nb, inter, hidden, w_up, w_down_t, ldw_down, k, nullptr, y, idx_out, workspace,
                           abytes, stream, pair);
}

// The decoder layer's FFN half x + FFN(RMSNorm(x)) for <= 4 tokens in two
// launches: the norm inside the gate/up GEMV pair, the residual add in the
// last step of the column-owning after-gate kernel.
extern "C" int moc_global_decode_rmsnorm_residual_bf16(const void* x, int64_t nb, int64_t hidden,
                                                       const void* norm_w, float eps, const void* w_gate,
                                                       const void* w_up, int64_t inter, const void* w_down_t,
                                                       int64_t ldw_down, int64_t k, void* y, void* idx_out,
                                                       void* workspace, int64_t workspace_bytes, void* stream) {
  MOC_REQUIRE(nb >= 0 && nb <= 4, "moc_global_decode_rmsnorm_residual_bf16: 0 <= nb <= 4 tokens");
  MOC_REQUIRE(inter >= 1 && hidden >= 8 && hidden <= 4096,
              "moc_global_decode_rmsnorm_residual_bf16: bad shape");
  MOC_REQUIRE(k >= 1 && k <= inter, "invalid k");
  MOC_REQUIRE(sd_fits(nb < 1 ? 1 : nb, inter, k, hidden),
              "moc_global_decode_rmsnorm_residual_bf16: needs hidden %% 256 == 0, inter <= %d, k <= %d",
              kSdMaxInter, kSdMaxK);
  MOC_REQUIRE(eps >= 0.f, "moc_global_decode_rmsnorm_residual_bf16: eps must be >= 0");
  if (nb == 0) return MOC_OK;
  MOC_REQUIRE(x && norm_w && w_gate && w_up && w_down_t && y,
              "moc_global_decode_rmsnorm_residual_bf16: null pointer");
  MOC_REQUIRE(aligned16(x) && aligned16(norm_w) && aligned16(w_gate) && aligned16(w_up) && aligned16(w_down_t),
              "moc_global_decode_rmsnorm_residual_bf16: x, norm_w and weights must be 16-byte aligned");
  MOC_REQUIRE(ldw_down >= hidden && ldw_down % 8 == 0,
              "moc_global_decode_rmsnorm_residual_bf16: ldw_down must be a multiple of 8 and >= hidden");
  MOC_REQUIRE(y != x, "moc_global_decode_rmsnorm_residual_bf16: y must not alias x");
  const int64_t need = moc_global_decode_workspace_size(nb, inter, k, hidden);
  MOC_REQUIRE(workspace != nullptr && workspace_bytes >= need,
              "moc_global_decode_rmsnorm_residual_bf16: workspace of %lld bytes required", (long long)need);
  return global_decode_sd(x, nb, hidden, norm_w, eps, w_gate, w_up, inter, w_down_t, ldw_down, k, x, y, idx_out,
                          static_cast<char*>(workspace), as_stream(stream));
}

extern "C" int64_t moc_moc28_decode_workspace_size(int64_t nb, int64_t inter, int64_t hidden) {
  if (nb < 0 || inter < 8 || hidden < 1) return 0;
  return kFusedCounterBytes + 2 * align256(nb * sd_pitch(inter) * 2) + align256(nb * hidden * 2);
}

// The MoC 2:8 decode layer (moc::fused_grouped_top2_up_silu followed by
// moc::selected_grouped_down, moc/inference/triton_grouped_moc_ops.py:26-131)
// in two launches: G and U of every token (of RMSNorm(x) when norm_w is
// given) in one GEMV launch, then select_down_kernel with the top 2 of every
// 8 channels, the residual added in its last step when given.
extern "C" int moc_moc28_decode_bf16(const void* x, int64_t nb, int64_t hidden, const void* norm_w, float eps,
                                     const void* w_gate, const void* w_up, int64_t inter, const void* w_down_t,
                                     int64_t ldw_down, const void* residual, void* y, void* idx_out,
                                     void* workspace, int64_t workspace_bytes, void* stream) {
  MOC_REQUIRE(nb >= 0 && nb <= 16, "moc_moc28_decode_bf16: 0 <= nb <= 16 tokens");
  MOC_REQUIRE(norm_w == nullptr || nb <= 4, "moc_moc28_decode_bf16: the fused RMSNorm takes nb <= 4 tokens");
  MOC_REQUIRE(inter >= 8 && inter % 8 == 0 && inter <= kSdMaxInter,
              "moc_moc28_decode_bf16: inter must be a multiple of 8 and <= %d", kSdMaxInter);
  MOC_REQUIRE(hidden >= 256 && hidden % 256 == 0 && hidden < (1LL << 30) && (norm_w == nullptr || hidden <= 4096),
              "moc_moc28_decode_bf16: hidden must be a multiple of 256 (<= 4096 with the fused RMSNorm)");
  MOC_REQUIRE(eps >= 0.f, "moc_moc28_decode_bf16: eps must be >= 0");
  if (nb == 0) return MOC_OK;
  MOC_REQUIRE(x && w_gate && w_up && w_down_t && y, "moc_moc28_decode_bf16: null pointer");
  MOC_REQUIRE(aligned16(x) && aligned16(w_gate) && aligned16(w_up) && aligned16(w_down_t) &&
                  (norm_w == nullptr || aligned16(norm_w)),
              "moc_moc28_decode_bf16: x, norm_w and weights must be 16-byte aligned");
  MOC_REQUIRE(ldw_down >= hidden && ldw_down % 8 == 0,
              "moc_moc28_decode_bf16: ldw_down must be a multiple of 8 and >= hidden");
  MOC_REQUIRE(y != x && (residual == nullptr || residual != y),
              "moc_moc28_decode_bf16: y must not alias x or the residual");
  const int64_t need = moc_moc28_decode_workspace_size(nb, inter, hidden);
  MOC_REQUIRE(workspace != nullptr && workspace_bytes >= need,
              "moc_moc28_decode_bf16: workspace of %lld bytes required", (long long)need);
  return global_decode_sd(x, nb, hidden, norm_w, eps, w_gate, w_up, inter, w_down_t, ldw_down, inter / 4, residual,
                          y, idx_out, static_cast<char*>(workspace), as_stream(stream), true);
}

extern "C" int moc_global_after_gate_residual_bf16(const void* x, const void* gate_scores, int64_t nb,
                                                   int64_t inter, int64_t hidden, const void* w_up,
                                                   const void* w_down_t, int64_t ldw_down, int64_t k,
                                                   const void* residual, void* y, void* idx_out, void* workspace,
                                                   int64_t workspace_bytes, void* stream) {
  MOC_REQUIRE(nb == 0 || residual != nullptr, "moc_global_after_gate_residual_bf16: null residual");
  return global_after_gate(x, gate_scores, nb, inter, hidden, w_up, w_down_t, ldw_down, k, residual, y, idx_out,
                           workspace, workspace_bytes, stream);
}


// MoC 2:8 inference kernels (gfx950): every aligned group of 8 channels keeps
// its two largest gate values.
//
//  moc_grouped_top2_up_silu_bf16  fused gate+up projection + top-2-of-8 +
//      SiLU(g)*u, writing only idx[nb, K'] and sz[nb, K'].  Replaces
//      moc::fused_grouped_top2_up_silu (moc/inference/triton_grouped_moc_ops.py:
//      26-78; kernel moc/inference/triton_fused_ffn_kernels.py:29-156).
//      Semantics kept from that kernel: G and U accumulate in f32 and are
//      rounded to bf16 before selection (:95-97,117-118); top-1 is the max
//      with the lowest index among equal maxima, top-2 the max of the other
//      seven under the same rule (:103-114); sz = (g*sigmoid(g))*u in f32,
//      stored bf16 (:126-129); idx int64 ordered (top-1, top-2) per group.
//      nb <= 16: a workgroup owns 16 channels (two groups) and all tokens,
//      G/U through MFMA 16x16x32 with the waves splitting the hidden dim.
//      nb  > 16: a 128-token x 64-channel MFMA GEMM tile computes G and U
//      side by side (B tile = 64 W_gate rows + the same 64 W_up rows); the
//      epilogue stages bf16 G/U in LDS and selects per (token, group).
//  moc_selected_grouped_down_bf16  y = sz * W_down^T[idx] (moc::selected_grouped_down,
//      triton_grouped_moc_ops.py:96-131, kernel triton_fused_ffn_kernels.py:228-267).
//      nb <= 64: split-K gathered GEMV; nb > 64: sz is scattered into a dense
//      zero-filled [nb, inter] tile and multiplied on MFMA (dense-equivalent
//      work: 4x the compacted FLOPs).
#include "abi.h"
#include "common.h"
#include "gemm_tile.h"

extern "C" int moc_selected_down_bf16(const void* z, const void* idx, int idx_dtype, int64_t nb,
                                      int64_t k, const void* w_down_t, int64_t ldw_down, int64_t inter,
                                      int64_t hidden, void* y, void* workspace,
                                      int64_t workspace_bytes, void* stream);
extern "C" int64_t moc_selected_down_workspace_size(int64_t nb, int64_t k, int64_t hidden);
extern "C" int moc_scatter_sparse_to_dense(int dtype, const void* sparse, const void* idx,
                                           int idx_dtype, int64_t rows, int64_t k, int64_t inter,
                                           void* dense, int64_t ld, void* stream);
extern "C" int moc_gemm_ws(int dtype, int64_t M, int64_t N, int64_t K, const void* A, int64_t a_sm,
                           int64_t a_sk, const void* B, int64_t b_sk, int64_t b_sn, int64_t K2,
                           const void* A2, int64_t a2_sm, int64_t a2_sk, const void* B2,
                           int64_t b2_sk, int64_t b2_sn, void* C, int64_t ldc, int c_dtype,
                           void* workspace, int64_t workspace_bytes, void* stream);
extern "C" int64_t moc_gemm_workspace_size(int dtype, int64_t M, int64_t N, int64_t K, int64_t K2);
extern "C" int64_t moc_sparse28_down_workspace_size(int64_t nb, int64_t inter, int64_t hidden);
extern "C" int moc_sparse28_down_bf16(const void* ap, int64_t ld_ap, const uint32_t* meta, int64_t meta_rows,
                                      int64_t nb, int64_t inter, const void* w, int64_t ldw, int w_kc,
                                      int64_t hidden, void* y, int64_t ldy, void* workspace,
                                      int64_t workspace_bytes, void* stream);
extern "C" int moc_pack28_bf16(const void* sz, const void* idx, int64_t nb, int64_t inter, void* ap,
                               int64_t ld_ap, uint32_t* meta, int64_t meta_rows, void* zero4k,
                               void* stream);

namespace moc {
namespace {

using namespace tile;

typedef float f32x4_t __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// nb <= 16 path.
// ---------------------------------------------------------------------------
constexpr int kDecUnroll = 4;

__global__ __launch_bounds__(256) void grouped_decode_kernel(
    const uint16_t* __restrict__ x, int nb, int hidden, const uint16_t* __restrict__ wg,
    const uint16_t* __restrict__ wu, int inter, int64_t* __restrict__ idx,
    uint16_t* __restrict__ sz) {
  __shared__ f32x4_t red[2][4][64];
  __shared__ float gu[2][16][17];  // [g|u][channel][token]
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c0 = blockIdx.x * 16;
  const int ch = c0 + (lane & 15);
  const int tok = lane & 15;
  const int kq = (lane >> 4) * 8;
  const bool ch_ok = ch < inter;
  const bool tok_ok = tok < nb;
  const uint16_t* gr = wg + static_cast<int64_t>(ch_ok ? ch : 0) * hidden + kq;
  const uint16_t* ur = wu + static_cast<int64_t>(ch_ok ? ch : 0) * hidden + kq;
  const uint16_t* xr = x + static_cast<int64_t>(tok_ok ? tok : 0) * hidden + kq;
  const int nsteps = (hidden + 31) / 32;
  f32x4_t ag = {0.f, 0.f, 0.f, 0.f}, au = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = wave; s0 < nsteps; s0 += 4 * kDecUnroll) {
    uint4 gv[kDecUnroll], uv[kDecUnroll], xv[kDecUnroll];
#pragma unroll
    for (int q = 0; q < kDecUnroll; ++q) {
      const int s = s0 + 4 * q;
      const bool kin = s < nsteps && s * 32 + kq < hidden;
      const uint4 zero = make_uint4(0, 0, 0, 0);
      gv[q] = (kin && ch_ok) ? *reinterpret_cast<const uint4*>(gr + s * 32) : zero;
      uv[q] = (kin && ch_ok) ? *reinterpret_cast<const uint4*>(ur + s * 32) : zero;
      xv[q] = (kin && tok_ok) ? *reinterpret_cast<const uint4*>(xr + s * 32) : zero;
    }
#pragma unroll
    for (int q = 0; q < kDecUnroll; ++q) {
      const bf16x8_t xb = __builtin_bit_cast(bf16x8_t, xv[q]);
      ag = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, gv[q]), xb, ag, 0, 0, 0);
      au = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, uv[q]), xb, au, 0, 0, 0);
    }
  }
  red[0][wave][lane] = ag;
  red[1][wave][lane] = au;
  __syncthreads();
  if (wave < 2) {
    f32x4_t t = red[wave][0][lane];
#pragma unroll
    for (int w = 1; w < 4; ++w) {
      const f32x4_t o = red[wave][w][lane];
      t[0] += o[0]; t[1] += o[1]; t[2] += o[2]; t[3] += o[3];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) gu[wave][4 * (lane >> 4) + j][lane & 15] = round_bf16(t[j]);
  }
  __syncthreads();
  // 16 tokens x 2 groups
  if (threadIdx.x < 32) {
    const int t = threadIdx.x & 15;
    const int grp = threadIdx.x >> 4;
    const int cg = c0 + grp * 8;
    if (t < nb && cg < inter) {
      float g[8], u[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        g[j] = gu[0][grp * 8 + j][t];
        u[j] = gu[1][grp * 8 + j][t];
      }
      const int kout = inter / 4;
      const int64_t o = static_cast<int64_t>(t) * kout + (cg / 8) * 2;
      select_group_emit(g, u, cg, idx + o, sz + o);
    }
  }
}

// ---------------------------------------------------------------------------
// nb <= 4 path, row streaming: a workgroup of 8 waves covers 16 channels (two
// groups of 8); wave w owns channels c0 + 2w and c0 + 2w + 1 and requests
// their W_gate and W_up rows whole (lane l: 16-byte chunks l + 64 i), so
// every byte of the four rows is in flight within one memory latency (the
// gate GEMV's scheme).  NORM: the tokens go through the FFN's RMSNorm first
// (rmsnorm8; every wave normalises its own copy of x).  G and U are rounded
// to bf16 and the two groups selected from LDS.
// ---------------------------------------------------------------------------
template <int NB, int CHN, bool NORM>
__global__ __launch_bounds__(512) void grouped_rows_kernel(
    const uint16_t* __restrict__ x, int hidden, const uint16_t* __restrict__ wg,
    const uint16_t* __restrict__ wu, int inter, int64_t* __restrict__ idx, uint16_t* __restrict__ sz,
    const uint16_t* __restrict__ norm_w, float eps) {
  __shared__ float gu[2][16][NB];  // [g | u][channel][token]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c0 = blockIdx.x * 16;
  const int nch = hidden / 8;
  uint4 w[4][CHN];  // gate ch0, gate ch1, up ch0, up ch1
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int ch = c0 + 2 * wave + (r & 1);
    const uint16_t* row = (r < 2 ? wg : wu) + static_cast<int64_t>(ch < inter ? ch : 0) * hidden;
#pragma unroll
    for (int i = 0; i < CHN; ++i) {
      const int c = lane + 64 * i;
      w[r][i] = (ch < inter && c < nch) ? *reinterpret_cast<const uint4*>(row + c * 8) : make_uint4(0, 0, 0, 0);
    }
  }
  uint4 nwv[NORM ? CHN : 1];
  if (NORM) {
#pragma unroll
    for (int i = 0; i < CHN; ++i) {
      const int c = lane + 64 * i;
      nwv[i] = c < nch ? *reinterpret_cast<const uint4*>(norm_w + c * 8) : make_uint4(0, 0, 0, 0);
    }
  }
#pragma unroll
  for (int t = 0; t < NB; ++t) {
    uint4 xv[CHN];
#pragma unroll
    for (int i = 0; i < CHN; ++i) {
      const int c = lane + 64 * i;
      xv[i] = c < nch ? *reinterpret_cast<const uint4*>(x + static_cast<int64_t>(t) * hidden + c * 8)
                      : make_uint4(0, 0, 0, 0);
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
      const float rr = rsqrtf(wave_sum(ss) / static_cast<float>(hidden) + eps);
#pragma unroll
      for (int i = 0; i < CHN; ++i) xv[i] = rmsnorm8(xv[i], nwv[NORM ? i : 0], rr);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float a = 0.f;
#pragma unroll
      for (int i = 0; i < CHN; ++i) a = dot8(w[r][i], xv[i], a);
      a = wave_sum(a);
      if (lane == 0) gu[r >> 1][2 * wave + (r & 1)][t] = round_bf16(a);
    }
  }
  __syncthreads();
  if (threadIdx.x < 2 * NB) {
    const int t = threadIdx.x % NB, grp = threadIdx.x / NB;
    const int cg = c0 + grp * 8;
    if (cg < inter) {
      float g[8], u[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        g[j] = gu[0][grp * 8 + j][t];
        u[j] = gu[1][grp * 8 + j][t];
      }
      const int64_t o = static_cast<int64_t>(t) * (inter / 4) + (cg / 8) * 2;
      select_group_emit(g, u, cg, idx + o, sz + o);
    }
  }
}

template <int NB, bool NORM>
void launch_grouped_rows(const void* x, int hidden, const void* wg, const void* wu, int inter, void* idx,
                         void* sz, const void* norm_w, float eps, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>((inter + 15) / 16)), block(512);
  const int chn = (hidden / 8 + 63) / 64;
#define MOC_GRW(C)                                                                                    \
  grouped_rows_kernel<NB, C, NORM><<<grid, block, 0, st>>>((const uint16_t*)x, hidden,                \
                                                            (const uint16_t*)wg, (const uint16_t*)wu, \
                                                            inter, (int64_t*)idx, (uint16_t*)sz,      \
                                                            (const uint16_t*)norm_w, eps)
  if (chn <= 1) MOC_GRW(1);
  else if (chn <= 2) MOC_GRW(2);
  else if (chn <= 4) MOC_GRW(4);
  else MOC_GRW(8);
#undef MOC_GRW
}

template <bool NORM>
void launch_grouped_rows_nb(int nb, const void* x, int hidden, const void* wg, const void* wu, int inter,
                            void* idx, void* sz, const void* norm_w, float eps, hipStream_t st) {
  switch (nb) {
    case 1: launch_grouped_rows<1, NORM>(x, hidden, wg, wu, inter, idx, sz, norm_w, eps, st); break;
    case 2: launch_grouped_rows<2, NORM>(x, hidden, wg, wu, inter, idx, sz, norm_w, eps, st); break;
    case 3: launch_grouped_rows<3, NORM>(x, hidden, wg, wu, inter, idx, sz, norm_w, eps, st); break;
    default: launch_grouped_rows<4, NORM>(x, hidden, wg, wu, inter, idx, sz, norm_w, eps, st); break;
  }
}

// B tile of the fused gate/up GEMM: rows [0, 64) are W_gate rows c0.., rows
// [64, 128) the same W_up rows; same thread mapping and LDS layout as the
// K-contiguous TileLoader.
struct DualLoader : TileLoader<true> {
  __device__ __forceinline__ void load(const uint16_t* __restrict__ wg,
                                       const uint16_t* __restrict__ wu, int hidden, int cvalid,
                                       int c0, int k0, int tid) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int v = tid + kThreads * i;
      const int row = v >> 3;
      const int rr = row & 63;
      const uint16_t* p = (row < 64 ? wg : wu) + static_cast<int64_t>(c0 + rr) * hidden;
      const int gk = k0 + (v & 7) * 8;
      if (rr < cvalid && gk + 8 <= hidden) {
        r[i] = *reinterpret_cast<const uint4*>(p + gk);
      } else {
        uint16_t e[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) e[j] = (rr < cvalid && gk + j < hidden) ? p[gk + j] : 0;
        r[i] = make_uint4(e[0] | (uint32_t(e[1]) << 16), e[2] | (uint32_t(e[3]) << 16),
                          e[4] | (uint32_t(e[5]) << 16), e[6] | (uint32_t(e[7]) << 16));
      }
    }
  }
};

// ---------------------------------------------------------------------------
// nb > 16 path: 128 tokens x 64 channels per workgroup.
// ---------------------------------------------------------------------------
constexpr int kGroupPitch = 130;  // bf16 per staged row in the epilogue

__global__ __launch_bounds__(kThreads) void grouped_prefill_kernel(
    const uint16_t* __restrict__ x, int nb, int hidden, const uint16_t* __restrict__ wg,
    const uint16_t* __restrict__ wu, int inter, int64_t* __restrict__ idx,
    uint16_t* __restrict__ sz) {
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * (kBM + kBN) * kPitch];
  auto As = [&](int b) { return smem + b * (kBM * kPitch); };
  auto Bs = [&](int b) { return smem + 2 * kBM * kPitch + b * (kBN * kPitch); };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int row0 = blockIdx.y * kBM;  // tokens
  const int c0 = blockIdx.x * 64;     // channels
  const int wm = (wave >> 1) * 64;
  const int wn = (wave & 1) * 64;     // 0: gate half, 64: up half
  const int nk = (hidden + kBK - 1) / kBK;
  const int cvalid = min(64, inter - c0);

  TileLoader<true> la;
  DualLoader lb;
  auto load = [&](int t) {
    la.load(x, hidden, nb, hidden, row0, t * kBK, tid);
    lb.load(wg, wu, hidden, cvalid, c0, t * kBK, tid);
  };
  auto store = [&](int buf) {
    la.store(As(buf), tid);
    lb.store(Bs(buf), tid);
  };

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  load(0);
  store(0);
  __syncthreads();
  const int frow = lane & 31;
  const int fk = (lane >> 5) * 8;
  for (int t = 0; t < nk; ++t) {
    const int cur = t & 1;
    if (t + 1 < nk) load(t + 1);
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      bf16x8_t a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        a[i] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(
                                                As(cur) + (wm + 32 * i + frow) * kPitch + ks * 16 + fk));
        b[i] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(
                                                Bs(cur) + (wn + 32 * i + frow) * kPitch + ks * 16 + fk));
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (t + 1 < nk) store(cur ^ 1);
    __syncthreads();
  }

  // stage bf16-rounded G (cols 0..63) and U (cols 64..127) per token row
  uint16_t* q = smem;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = wn + 32 * j + (lane & 31);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        q[row * kGroupPitch + col] = f32_to_bf16(acc[i][j][r]);
      }
    }
  __syncthreads();
  const int kout = inter / 4;
  for (int p = tid; p < kBM * 8; p += kThreads) {
    const int tr = p >> 3;
    const int grp = p & 7;
    const int tok = row0 + tr;
    const int cg = c0 + grp * 8;
    if (tok >= nb || cg >= inter) continue;
    float g[8], u[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      g[j] = bf16_to_f32(q[tr * kGroupPitch + grp * 8 + j]);
      u[j] = bf16_to_f32(q[tr * kGroupPitch + 64 + grp * 8 + j]);
    }
    const int64_t o = static_cast<int64_t>(tok) * kout + (cg / 8) * 2;
    select_group_emit(g, u, cg, idx + o, sz + o);
  }
}

inline int64_t align256(int64_t b) { return (b + 255) & ~int64_t(255); }

// ---------------------------------------------------------------------------
// 2:4 packing of a 2:8 selection for the compacted Down on the structured-
// sparse MFMA (moc_sparse28_down_bf16; layout in include/moc_amd.h).  Each
// group of 8 channels holds two selected channels; its two 4-channel halves
// get two stored values each (pack_group_2of8), so the packed row is half as
// wide as the dense one.  A lane packs one 8-group G of one row: it reads
// the group's (top-1, top-2) indices (16 bytes) and values (4 bytes) and
// writes its four stored values (8 bytes), so a wave covers 64 consecutive
// groups (8 channel tiles) of a row with contiguous loads and stores.  The
// positions byte of G goes into bits 8(G & 1) + 16((G >> 2) & 1) of word
// h = (G >> 1) & 1 of its tile G >> 3; lanes G, G ^ 1, G ^ 4, G ^ 5 combine
// that word, which is staged in LDS and leaves as 128-byte runs of one tile
// (16 rows).  An index outside its own group, or both equal, cannot be
// packed: the group's values become NaN, so the token's output row is NaN
// rather than silently wrong.  Workgroup: 16 rows x 64 groups, a wave per
// row at a time.
// ---------------------------------------------------------------------------
constexpr int kPackRows = 16, kPackTiles = 8;

__global__ __launch_bounds__(256) void pack28_kernel(const uint16_t* __restrict__ sz,
                                                      const int64_t* __restrict__ idx, int nb, int inter,
                                                      int nt, uint16_t* __restrict__ ap, int64_t ld_ap,
                                                      uint32_t* __restrict__ meta, int meta_rows,
                                                      uint32_t* __restrict__ zero4k) {
  __shared__ uint32_t words[kPackTiles][kPackRows * 2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (zero4k != nullptr && blockIdx.x == 0 && blockIdx.y == 0)
    reinterpret_cast<uint4*>(zero4k)[tid] = make_uint4(0, 0, 0, 0);  // 4 KB of GEMM counters
  const int kp = inter / 4;       // entries per row
  const int ngroups = inter / 8;  // 8-groups
  const int G = blockIdx.x * 64 + lane;
  const int t = G >> 3;
#pragma unroll
  for (int i = 0; i < kPackRows / 4; ++i) {
    const int rl = wave * (kPackRows / 4) + i;
    const int row = blockIdx.y * kPackRows + rl;
    uint16_t q[4] = {0, 0, 0, 0};
    uint32_t pos = kPackEmpty2of8;
    if (row < nb && G < ngroups) {
      const int64_t e = static_cast<int64_t>(row) * kp + 2 * G;
      const int64_t p1 = idx[e] - 8 * static_cast<int64_t>(G), p2 = idx[e + 1] - 8 * static_cast<int64_t>(G);
      const uint32_t v = *reinterpret_cast<const uint32_t*>(sz + e);  // e is even: 4-byte aligned
      if (p1 < 0 || p1 > 7 || p2 < 0 || p2 > 7 || p1 == p2) {
        q[0] = q[1] = q[2] = q[3] = 0x7FC0;  // NaN
      } else {
        pos = pack_group_2of8(static_cast<int>(p1), static_cast<uint16_t>(v & 0xFFFFu), static_cast<int>(p2),
                              static_cast<uint16_t>(v >> 16), q);
      }
    }
    uint32_t w = pos << (16 * ((G >> 2) & 1) + 8 * (G & 1));
    w |= __shfl_xor(w, 1);
    w |= __shfl_xor(w, 4);
    if (row < nb && t < nt)
      *reinterpret_cast<uint2*>(ap + static_cast<int64_t>(row) * ld_ap + 4 * G) =
          make_uint2(q[0] | (static_cast<uint32_t>(q[1]) << 16), q[2] | (static_cast<uint32_t>(q[3]) << 16));
    if ((lane & 5) == 0) words[(lane >> 3)][rl * 2 + ((lane >> 1) & 1)] = w;
  }
  __syncthreads();
  const int wt = tid >> 5, wi = tid & 31;  // tile, (row, h) of the write-out
  const int ot = blockIdx.x * kPackTiles + wt, orow = blockIdx.y * kPackRows + (wi >> 1);
  if (ot < nt && orow < meta_rows)
    meta[(static_cast<int64_t>(ot) * meta_rows + orow) * 2 + (wi & 1)] = words[wt][wi];
}

}  // namespace
}  // namespace moc

using namespace moc;

extern "C" int moc_pack28_bf16(const void* sz, const void* idx, int64_t nb, int64_t inter, void* ap,
                               int64_t ld_ap, uint32_t* meta, int64_t meta_rows, void* zero4k,
                               void* stream) {
  MOC_REQUIRE(nb >= 0 && inter >= 8 && inter % 8 == 0 && inter < (1LL << 30) && nb < (1LL << 30),
              "moc_pack28_bf16: bad shape (intermediate must be a multiple of 8)");
  if (nb == 0) return MOC_OK;
  MOC_REQUIRE(sz && idx && ap && meta, "moc_pack28_bf16: null pointer");
  MOC_REQUIRE(reinterpret_cast<uintptr_t>(sz) % 4 == 0 && reinterpret_cast<uintptr_t>(idx) % 8 == 0,
              "moc_pack28_bf16: sz must be 4-byte and idx 8-byte aligned");
  const int64_t nt = (inter + 63) / 64;
  MOC_REQUIRE(ld_ap >= 32 * nt && ld_ap % 8 == 0 && aligned16(ap),
              "moc_pack28_bf16: ap needs 16-byte aligned rows of >= 32 * ceil(inter / 64) values");
  MOC_REQUIRE(meta_rows >= nb && meta_rows % 64 == 0, "moc_pack28_bf16: meta_rows must be >= nb, a multiple of 64");
  MOC_REQUIRE(zero4k == nullptr || aligned16(zero4k), "moc_pack28_bf16: unaligned counter block");
  const dim3 grid(static_cast<unsigned>((nt + kPackTiles - 1) / kPackTiles),
                  static_cast<unsigned>(meta_rows / kPackRows));
  MOC_REQUIRE(grid.y <= 65535, "moc_pack28_bf16: too many rows");
  pack28_kernel<<<grid, 256, 0, as_stream(stream)>>>(
      static_cast<const uint16_t*>(sz), static_cast<const int64_t*>(idx), (int)nb, (int)inter, (int)nt,
      static_cast<uint16_t*>(ap), ld_ap, meta, (int)meta_rows, static_cast<uint32_t*>(zero4k));
  return check_launch("pack28_kernel");
}

extern "C" int moc_grouped_top2_up_silu_bf16(const void* x, int64_t nb, int64_t hidden,
                                             const void* w_gate, const void* w_up, int64_t inter,
                                             void* idx, void* sz, void* stream) {
  MOC_REQUIRE(nb >= 0 && hidden >= 1 && inter >= 8, "moc_grouped_top2_up_silu_bf16: bad shape");
  MOC_REQUIRE(inter % 8 == 0, "intermediate=%lld must be divisible by 8", (long long)inter);
  MOC_REQUIRE(hidden % 8 == 0, "moc_grouped_top2_up_silu_bf16: hidden must be a multiple of 8");
  MOC_REQUIRE(inter < (1LL << 30) && hidden < (1LL << 30), "moc_grouped_top2_up_silu_bf16: too large");
  if (nb == 0) return MOC_OK;
  MOC_REQUIRE(x && w_gate && w_up && idx && sz, "moc_grouped_top2_up_silu_bf16: null pointer");
  MOC_REQUIRE(aligned16(x) && aligned16(w_gate) && aligned16(w_up),
              "moc_grouped_top2_up_silu_bf16: x and weights must be 16-byte aligned");
  hipStream_t st = as_stream(stream);
  if (nb <= 4 && hidden <= 4096) {
    launch_grouped_rows_nb<false>((int)nb, x, (int)hidden, w_gate, w_up, (int)inter, idx, sz, nullptr, 0.f, st);
    return check_launch("grouped_rows_kernel");
  }
  if (nb <= 16) {
    grouped_decode_kernel<<<dim3(static_cast<unsigned>((inter + 15) / 16)), 256, 0, st>>>(
        (const uint16_t*)x, (int)nb, (int)hidden, (const uint16_t*)w_gate, (const uint16_t*)w_up,
        (int)inter, (int64_t*)idx, (uint16_t*)sz);
    return check_launch("grouped_decode_kernel");
  }
  {
    const int rc = launch_gate_up_2of8(x, nb, hidden, w_gate, w_up, inter, static_cast<int64_t*>(idx),
                                       static_cast<uint16_t*>(sz), st);
    if (rc != 1) return rc;
  }
  MOC_REQUIRE((nb + kBM - 1) / kBM <= 65535, "moc_grouped_top2_up_silu_bf16: too many tokens");
  const dim3 grid(static_cast<unsigned>((inter + 63) / 64), static_cast<unsigned>((nb + kBM - 1) / kBM));
  grouped_prefill_kernel<<<grid, kThreads, 0, st>>>((const uint16_t*)x, (int)nb, (int)hidden,
                                                    (const uint16_t*)w_gate, (const uint16_t*)w_up,
                                                    (int)inter, (int64_t*)idx, (uint16_t*)sz);
  return check_launch("grouped_prefill_kernel");
}

// Layout of the 2:4-packed operand inside the workspace of the prefill path.
namespace {
struct Packed28 {
  int64_t nt, ld_ap, meta_rows, ap_bytes, meta_bytes;
};
Packed28 packed28_layout(int64_t nb, int64_t inter) {
  Packed28 p;
  p.nt = (inter + 63) / 64;
  p.ld_ap = 32 * p.nt;
  p.meta_rows = (nb + 255) / 256 * 256;
  p.ap_bytes = align256(nb * p.ld_ap * 2);
  p.meta_bytes = align256(p.nt * p.meta_rows * 8);
  return p;
}

// The compacted (structured-sparse) prefill form applies to the 2:8 layout:
// k = inter / 4 entries per token, (top-1, top-2) of each 8-group.
bool sparse28_applies(int64_t nb, int64_t k, int64_t inter) {
  return nb > 64 && inter % 8 == 0 && k == inter / 4;
}
}  // namespace

extern "C" int moc_grouped_top2_up_silu_packed_bf16(const void* x, int64_t nb, int64_t hidden,
                                                    const void* w_gate, const void* w_up, int64_t inter,
                                                    void* ap, int64_t ld_ap, uint32_t* meta,
                                                    int64_t meta_rows, void* stream) {
  MOC_REQUIRE(nb >= 0 && hidden >= 1 && inter >= 8, "moc_grouped_top2_up_silu_packed_bf16: bad shape");
  MOC_REQUIRE(inter % 8 == 0, "intermediate=%lld must be divisible by 8", (long long)inter);
  MOC_REQUIRE(hidden % 8 == 0, "moc_grouped_top2_up_silu_packed_bf16: hidden must be a multiple of 8");
  MOC_REQUIRE(inter < (1LL << 30) && hidden < (1LL << 30) && nb < (1LL << 30),
              "moc_grouped_top2_up_silu_packed_bf16: too large");
  if (nb == 0) return MOC_OK;
  MOC_REQUIRE(x && w_gate && w_up && ap && meta, "moc_grouped_top2_up_silu_packed_bf16: null pointer");
  MOC_REQUIRE(aligned16(x) && aligned16(w_gate) && aligned16(w_up) && aligned16(ap) && aligned16(meta),
              "moc_grouped_top2_up_silu_packed_bf16: operands must be 16-byte aligned");
  const int64_t nt = (inter + 63) / 64;
  MOC_REQUIRE(ld_ap >= 32 * nt && ld_ap % 8 == 0,
              "moc_grouped_top2_up_silu_packed_bf16: ld_ap must be a multiple of 8 and >= 32 * ceil(inter / 64)");
  MOC_REQUIRE(meta_rows >= nb && nt * meta_rows * 8 < (1LL << 31),
              "moc_grouped_top2_up_silu_packed_bf16: bad meta_rows");
  const int rc = launch_gate_up_2of8(x, nb, hidden, w_gate, w_up, inter, nullptr, nullptr, as_stream(stream),
                                     static_cast<uint16_t*>(ap), ld_ap, meta, meta_rows);
  MOC_REQUIRE(rc != 1, "moc_grouped_top2_up_silu_packed_bf16: operands exceed 32-bit buffer addressing");
  return rc;
}

extern "C" int64_t moc_selected_grouped_down_workspace_size(int64_t nb, int64_t k, int64_t inter,
                                                            int64_t hidden) {
  if (nb <= 0 || k <= 0 || inter <= 0 || hidden <= 0) return 0;
  if (nb <= 64) return moc_selected_down_workspace_size(nb, k, hidden);
  if (sparse28_applies(nb, k, inter)) {
    // packed values and positions, then the sparse down GEMM's workspace
    const Packed28 p = packed28_layout(nb, inter);
    return p.ap_bytes + p.meta_bytes + moc_sparse28_down_workspace_size(nb, inter, hidden);
  }
  // dense z, then the down GEMM's own workspace
  return align256(nb * inter * 2) + moc_gemm_workspace_size(MOC_BF16, nb, hidden, inter, 0);
}

extern "C" int moc_selected_grouped_down_bf16(const void* sz, const void* idx, int64_t nb,
                                              int64_t k, const void* w_down_t, int64_t ldw_down,
                                              int64_t inter, int64_t hidden, void* y, void* workspace,
                                              int64_t workspace_bytes, void* stream) {
  MOC_REQUIRE(nb >= 0 && k >= 1 && inter >= k && hidden >= 1, "moc_selected_grouped_down_bf16: bad shape");
  MOC_REQUIRE(hidden % 8 == 0, "moc_selected_grouped_down_bf16: hidden must be a multiple of 8");
  MOC_REQUIRE(ldw_down >= hidden && ldw_down % 8 == 0,
              "moc_selected_grouped_down_bf16: ldw_down must be a multiple of 8 and >= hidden");
  if (nb == 0) return MOC_OK;
  const int64_t need = moc_selected_grouped_down_workspace_size(nb, k, inter, hidden);
  MOC_REQUIRE(workspace != nullptr && workspace_bytes >= need,
              "moc_selected_grouped_down_bf16: workspace of %lld bytes required", (long long)need);
  if (nb <= 64)
    return moc_selected_down_bf16(sz, idx, MOC_I64, nb, k, w_down_t, ldw_down, inter, hidden, y, workspace,
                                  workspace_bytes, stream);
  MOC_REQUIRE(inter % 8 == 0, "moc_selected_grouped_down_bf16: intermediate must be a multiple of 8");
  if (sparse28_applies(nb, k, inter)) {
    // pack (sz, idx) 2:4, clearing the GEMM's counters on the way, then the
    // structured-sparse GEMM over W_down^T
    const Packed28 p = packed28_layout(nb, inter);
    char* base = static_cast<char*>(workspace);
    uint32_t* meta = reinterpret_cast<uint32_t*>(base + p.ap_bytes);
    char* gws = base + p.ap_bytes + p.meta_bytes;
    const int64_t gbytes = moc_sparse28_down_workspace_size(nb, inter, hidden);
    int rc = moc_pack28_bf16(sz, idx, nb, inter, base, p.ld_ap, meta, p.meta_rows,
                             gbytes > 0 ? gws : nullptr, stream);
    if (rc != MOC_OK) return rc;
    return moc_sparse28_down_bf16(base, p.ld_ap, meta, p.meta_rows, nb, inter, w_down_t, ldw_down, 0, hidden,
                                  y, hidden, gbytes > 0 ? gws : nullptr, gbytes, stream);
  }
  int rc = moc_scatter_sparse_to_dense(MOC_BF16, sz, idx, MOC_I64, nb, k, inter, workspace, inter,
                                       stream);
  if (rc != MOC_OK) return rc;
  // The GEMM's workspace starts with arrival counters that must be zero;
  // this entry point's workspace carries nothing between calls, so they are
  // cleared here.
  char* gws = static_cast<char*>(workspace) + align256(nb * inter * 2);
  const int64_t gbytes = moc_gemm_workspace_size(MOC_BF16, nb, hidden, inter, 0);
  if (gbytes > 0) {
    rc = moc_fill_zero(gws, MOC_GEMM_WS_COUNTER_BYTES, stream);
    if (rc != MOC_OK) return rc;
  }
  // y[nb, hidden] = z[nb, inter] (K-contiguous) x W_down^T[inter, hidden] (N-contiguous)
  return moc_gemm_ws(MOC_BF16, nb, hidden, inter, workspace, inter, 1, w_down_t, ldw_down, 1, 0,
                     nullptr, 0, 0, nullptr, 0, 0, y, hidden, MOC_BF16, gbytes > 0 ? gws : nullptr,
                     gbytes, stream);
}

extern "C" int moc_grouped_top2_up_silu_rmsnorm_bf16(const void* x, int64_t nb, int64_t hidden,
                                                     const void* norm_w, float eps, const void* w_gate,
                                                     const void* w_up, int64_t inter, void* idx, void* sz,
                                                     void* stream) {
  MOC_REQUIRE(nb >= 0 && nb <= 4, "moc_grouped_top2_up_silu_rmsnorm_bf16: 0 <= nb <= 4 tokens");
  MOC_REQUIRE(hidden >= 8 && hidden <= 4096 && hidden % 8 == 0,
              "moc_grouped_top2_up_silu_rmsnorm_bf16: hidden must be a multiple of 8 in [8, 4096]");
  MOC_REQUIRE(inter >= 8 && inter % 8 == 0 && inter < (1LL << 30),
              "intermediate=%lld must be divisible by 8", (long long)inter);
  MOC_REQUIRE(eps >= 0.f, "moc_grouped_top2_up_silu_rmsnorm_bf16: eps must be >= 0");
  if (nb == 0) return MOC_OK;
  MOC_REQUIRE(x && norm_w && w_gate && w_up && idx && sz, "moc_grouped_top2_up_silu_rmsnorm_bf16: null pointer");
  MOC_REQUIRE(aligned16(x) && aligned16(norm_w) && aligned16(w_gate) && aligned16(w_up),
              "moc_grouped_top2_up_silu_rmsnorm_bf16: x, norm_w and weights must be 16-byte aligned");
  launch_grouped_rows_nb<true>((int)nb, x, (int)hidden, w_gate, w_up, (int)inter, idx, sz, norm_w, eps,
                               as_stream(stream));
  return check_launch("grouped_rows_kernel (rmsnorm)");
}

extern "C" int moc_selected_grouped_down_residual_bf16(const void* sz, const void* idx, int64_t nb,
                                                       int64_t k, const void* w_down_t, int64_t ldw_down,
                                                       int64_t inter, int64_t hidden, const void* residual, void* y,
                                                       void* workspace, int64_t workspace_bytes,
                                                       void* stream) {
  MOC_REQUIRE(nb >= 0 && nb <= 64, "moc_selected_grouped_down_residual_bf16: 0 <= nb <= 64 tokens");
  MOC_REQUIRE(k >= 1 && inter >= k && hidden >= 1 && hidden % 64 == 0,
              "moc_selected_grouped_down_residual_bf16: bad shape");
  if (nb == 0) return MOC_OK;
  MOC_REQUIRE(residual != nullptr, "moc_selected_grouped_down_residual_bf16: null residual");
  return selected_down_impl(sz, idx, MOC_I64, nb, k, w_down_t, ldw_down, inter, hidden, residual, y, workspace,
                            workspace_bytes, stream);
}

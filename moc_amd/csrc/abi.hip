// Error plumbing and small memory utilities of the C-ABI.
//
// No entry point throws across the ABI: each returns MOC_OK or a negative
// status, and the message of the last failure on the calling thread is kept
// for moc_last_error().  The library allocates no device memory; callers own
// every buffer, so each entry point can be recorded into a HIP graph.
#include <stdio.h>

#include "abi.h"
#include "common.h"

namespace moc {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: HIP launch failed: %s", what, hipGetErrorString(e));
    return MOC_ERR_HIP;
  }
  return MOC_OK;
}

namespace {

// Grid-stride zero fill with 16-byte stores where the pointer allows.
__global__ void fill_zero_kernel(uint8_t* __restrict__ p, int64_t bytes) {
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t n16 = bytes / 16;
  uint4* p16 = reinterpret_cast<uint4*>(p);
  for (int64_t i = tid; i < n16; i += stride) p16[i] = make_uint4(0, 0, 0, 0);
  for (int64_t i = n16 * 16 + tid; i < bytes; i += stride) p[i] = 0;
}

// 2-D copy of a row-major [rows, cols] block into a destination with its own
// leading dimension; columns [cols, dst_cols) of the destination are zeroed.
template <typename T>
__global__ void copy_pad_2d_kernel(const T* __restrict__ src, int64_t rows, int64_t cols,
                                   int64_t src_ld, T* __restrict__ dst, int64_t dst_ld,
                                   int64_t dst_cols) {
  const int64_t total = rows * dst_cols;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
       e += stride) {
    const int64_t r = e / dst_cols;
    const int64_t c = e - r * dst_cols;
    dst[r * dst_ld + c] = (c < cols) ? src[r * src_ld + c] : T(0);
  }
}

// bf16 copy into 16-byte aligned destination rows (dst_ld a multiple of 8):
// row blockIdx.y, each thread one 8-element chunk of it, written with one
// 16-byte store; the source (any alignment) is read element by element,
// coalesced across the threads of the row.
__global__ __launch_bounds__(256) void copy_pad_rows16_kernel(const uint16_t* __restrict__ src,
                                                              int64_t cols, int64_t src_ld,
                                                              uint16_t* __restrict__ dst,
                                                              int64_t dst_ld, int64_t dst_cols) {
  const int64_t r = blockIdx.y;
  const int64_t c0 = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 8;
  if (c0 >= dst_cols) return;
  const uint16_t* s = src + r * src_ld;
  uint16_t v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = (c0 + j < cols) ? s[c0 + j] : uint16_t(0);
  uint4 o;
  o.x = v[0] | (uint32_t(v[1]) << 16);
  o.y = v[2] | (uint32_t(v[3]) << 16);
  o.z = v[4] | (uint32_t(v[5]) << 16);
  o.w = v[6] | (uint32_t(v[7]) << 16);
  *reinterpret_cast<uint4*>(dst + r * dst_ld + c0) = o;
}

}  // namespace
}  // namespace moc

using namespace moc;

extern "C" const char* moc_last_error(void) { return g_last_error; }

extern "C" int moc_abi_version(void) { return MOC_ABI_VERSION; }

extern "C" int moc_fill_zero(void* dst, int64_t bytes, void* stream) {
  MOC_REQUIRE(bytes >= 0, "moc_fill_zero: negative size");
  MOC_REQUIRE(bytes == 0 || dst != nullptr, "moc_fill_zero: null pointer");
  if (bytes == 0) return MOC_OK;
  MOC_REQUIRE(aligned16(dst), "moc_fill_zero: destination must be 16-byte aligned");
  int64_t blocks = (bytes / 16 + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 4096) blocks = 4096;
  fill_zero_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, as_stream(stream)>>>(
      static_cast<uint8_t*>(dst), bytes);
  return check_launch("fill_zero_kernel");
}

extern "C" int moc_copy_pad_2d(int dtype, const void* src, int64_t rows, int64_t cols,
                               int64_t src_ld, void* dst, int64_t dst_ld, int64_t dst_cols,
                               void* stream) {
  MOC_REQUIRE(dtype == MOC_BF16 || dtype == MOC_F32, "moc_copy_pad_2d: bad dtype");
  MOC_REQUIRE(rows >= 0 && cols >= 0 && dst_cols >= cols, "moc_copy_pad_2d: bad shape");
  MOC_REQUIRE(src_ld >= cols && dst_ld >= dst_cols, "moc_copy_pad_2d: bad leading dimension");
  if (rows == 0 || dst_cols == 0) return MOC_OK;
  MOC_REQUIRE(dst != nullptr && (cols == 0 || src != nullptr), "moc_copy_pad_2d: null pointer");
  int64_t blocks = (rows * dst_cols + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  const dim3 grid(static_cast<unsigned>(blocks)), block(256);
  hipStream_t st = as_stream(stream);
  if (dtype == MOC_BF16 && dst_ld % 8 == 0 && dst_cols % 8 == 0 && aligned16(dst) && rows <= 65535) {
    const int64_t chunks = dst_cols / 8;
    const dim3 g2(static_cast<unsigned>((chunks + 255) / 256), static_cast<unsigned>(rows));
    copy_pad_rows16_kernel<<<g2, 256, 0, st>>>(static_cast<const uint16_t*>(src), cols, src_ld,
                                              static_cast<uint16_t*>(dst), dst_ld, dst_cols);
    return check_launch("copy_pad_rows16_kernel");
  }
  if (dtype == MOC_BF16)
    copy_pad_2d_kernel<uint16_t><<<grid, block, 0, st>>>(static_cast<const uint16_t*>(src), rows,
                                                         cols, src_ld, static_cast<uint16_t*>(dst),
                                                         dst_ld, dst_cols);
  else
    copy_pad_2d_kernel<uint32_t><<<grid, block, 0, st>>>(static_cast<const uint32_t*>(src), rows,
                                                         cols, src_ld, static_cast<uint32_t*>(dst),
                                                         dst_ld, dst_cols);
  return check_launch("copy_pad_2d_kernel");
}

// Allocation-free global-MoC after-gate entry point.  Its workspace is `scratch`, a
// file-scope device array of MOC_NOALLOC_SCRATCH_BYTES that each GPU the
// library runs on holds until the process ends.  On the host the array's name
// is only a stand-in: the array's device address on a GPU comes from
// hipGetSymbolAddress, taken once per device with that device current, and
// only that address is handed to kernels.  Layout as the caller workspace of
// moc_global_after_gate_bf16: arrival counters, partial sums, dense U.  The
// counters are cleared once, by the first call on a device, which then waits
// for the clear to finish before it goes on (so every later call, on any
// stream, finds them zero; every call leaves them zero).  That first call must
// therefore not be made while its stream is being captured into a HIP graph:
// it returns an error instead; calls after it may be captured and replayed.
// Every call on a GPU shares that GPU's array, so calls that overlap on one
// GPU (two streams, two threads, graph replays beside eager calls) race.

#include <mutex>

#include "abi.h"

static __device__ __align__(256) unsigned char scratch[MOC_NOALLOC_SCRATCH_BYTES];

namespace moc {
namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_of_current_device(void** out, void* stream) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("moc_global_after_gate_noalloc_bf16: hipGetDevice failed: %s", hipGetErrorString(e));
    return MOC_ERR_HIP;
  }
  MOC_REQUIRE(dev >= 0 && dev < kMaxDevices, "moc_global_after_gate_noalloc_bf16: device %d out of range",
              dev);
  if (stream != nullptr) {
    int sdev = -1;
    e = hipStreamGetDevice(as_stream(stream), &sdev);
    if (e != hipSuccess) {
      set_error("moc_global_after_gate_noalloc_bf16: hipStreamGetDevice failed: %s", hipGetErrorString(e));
      return MOC_ERR_HIP;
    }
    MOC_REQUIRE(sdev == dev,
                "moc_global_after_gate_noalloc_bf16: the stream belongs to device %d, the current "
                "device is %d", sdev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error("moc_global_after_gate_noalloc_bf16: hipGetSymbolAddress(scratch) failed: %s",
                hipGetErrorString(e));
      return MOC_ERR_HIP;
    }
    // the arrival counters must be zero before the first call: cleared on
    // this stream and waited for, so that no later call on another stream
    // can run ahead of the clear (and never recorded into a graph)
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(as_stream(stream), &cap);
    if (e != hipSuccess) {
      set_error("moc_global_after_gate_noalloc_bf16: hipStreamIsCapturing failed: %s", hipGetErrorString(e));
      return MOC_ERR_HIP;
    }
    MOC_REQUIRE(cap == hipStreamCaptureStatusNone,
                "moc_global_after_gate_noalloc_bf16: the first call on a device clears the scratch "
                "counters and waits for it, so it cannot run under HIP graph capture; make one call "
                "outside the capture first");
    const int rc = moc_fill_zero(p, kAfterGateCounterBytes, stream);
    if (rc != MOC_OK) return rc;
    e = hipStreamSynchronize(as_stream(stream));
    if (e != hipSuccess) {
      set_error("moc_global_after_gate_noalloc_bf16: waiting for the scratch clear failed: %s",
                hipGetErrorString(e));
      return MOC_ERR_HIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MOC_OK;
}
}  // namespace
}  // namespace moc

using namespace moc;

extern "C" int moc_global_after_gate_noalloc_bf16(const void* x, const void* gate_scores, int64_t nb,
                                                  int64_t inter, int64_t hidden, const void* w_up,
                                                  const void* w_down_t, int64_t ldw_down, int64_t k,
                                                  const void* residual, void* y, void* idx_out, void* stream) {
  MOC_REQUIRE(nb >= 0 && nb <= 16, "moc_global_after_gate_noalloc_bf16: 0 <= nb <= 16 tokens");
  MOC_REQUIRE(inter >= 1 && inter <= 16384 && hidden >= 64 && hidden % 64 == 0,
              "moc_global_after_gate_noalloc_bf16: bad shape");
  MOC_REQUIRE(k >= 1 && k <= inter, "invalid k");
  if (nb == 0) return MOC_OK;
  const int64_t need = moc_global_after_gate_workspace_size(nb, inter, k, hidden);
  MOC_REQUIRE(need <= MOC_NOALLOC_SCRATCH_BYTES,
              "moc_global_after_gate_noalloc_bf16: this shape needs %lld bytes of scratch, more than "
              "the library's fixed %lld (use moc_global_after_gate_bf16 with a workspace)",
              (long long)need, (long long)MOC_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  const int rc = scratch_of_current_device(&ws, stream);
  if (rc != MOC_OK) return rc;
  return global_after_gate(x, gate_scores, nb, inter, hidden, w_up, w_down_t, ldw_down, k, residual, y, idx_out, ws,
                           MOC_NOALLOC_SCRATCH_BYTES, stream);
}

// qlin_gemm_i8_noalloc: qlin_gemm_i8 with its split-K scratch in a static device array
// instead of a caller-supplied workspace, for callers that cannot allocate device memory
// (code under HIP graph capture, serving loops, harnesses that forbid allocation).
//
// The array `scratch` (kScratchBytes: 1 MiB of arrival counters, 4 MiB of polling-exchange
// slots, then 8 MiB of fp32 partial sums, the workspace's layout; zero at load, and the
// counters and slots are left zero by every call) exists once per GPU for the life of
// the process.
// Its device address is taken once per device with hipGetSymbolAddress, with that device
// current, and kept per device; host code uses only that address, never the array's
// name (in host code the name is a host-side stand-in, not a device address).  Every
// call clears the arrival counters it can touch with a fill kernel on the caller's
// stream (no memset node, so the call can be captured) and runs the qlin_gemm_i8 plan
// on the scratch.  Calls that overlap in time on one GPU share the array and race.
#include <stdio.h>

#include <mutex>

#include "../../include/qlin.h"
#include "qlin_internal.h"

namespace {

constexpr size_t kScratchPartialBytes = size_t(8) << 20;
constexpr size_t kScratchBytes = (size_t(1) << 20) + (size_t(4) << 20) + kScratchPartialBytes;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

void* g_scratch[kMaxDevices] = {};
std::mutex g_scratch_mu;

// The device address of the current device's `scratch`.
int scratch_ptr(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess && (dev < 0 || dev >= kMaxDevices)) e = hipErrorInvalidDevice;
  if (e == hipSuccess) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch[dev]) {
      void* p = nullptr;
      e = hipGetSymbolAddress((void**)&p, HIP_SYMBOL(scratch));
      if (e == hipSuccess) g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
  }
  if (e == hipSuccess) return QLIN_OK;
  char msg[200];
  snprintf(msg, sizeof(msg), "qlin_gemm_i8_noalloc: scratch address: HIP error %d (%s)", (int)e,
           hipGetErrorString(e));
  return qlin::set_error(QLIN_ERR_HIP, msg);
}

}  // namespace

extern "C" int qlin_gemm_i8_noalloc(const int8_t* a_q, const float* a_s, int M, int K, const int8_t* b,
                                    const void* b_s, int bs_dtype, int N, void* out, int64_t ldo,
                                    const void* residual, int64_t ldr, void* stream) {
  if (qlin::counter_bytes() + qlin::poll_bytes() + kScratchPartialBytes != kScratchBytes)
    return qlin::set_error(QLIN_ERR_WORKSPACE, "qlin_gemm_i8_noalloc: scratch layout mismatch");
  void* ptr = nullptr;
  const int rc = scratch_ptr(&ptr);
  if (rc != QLIN_OK) return rc;
  return qlin::gemm_i8_scratch("qlin_gemm_i8_noalloc", a_q, a_s, M, K, b, b_s, bs_dtype, N, out, ldo, residual,
                               ldr, ptr, kScratchBytes, stream);
}

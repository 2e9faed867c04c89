// psgdk_norm_lower_bound_full_noalloc: psgdk_norm_lower_bound_full for callers that cannot allocate device memory
// (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc). Its scratch is a file-scope device
// array of kNoallocScratchBytes that every GPU the library runs on holds until the process ends; the call allocates
// nothing and takes no workspace argument.
//
// The array's name is a host-side stand-in in host code, not a device address: the address is looked up once per
// device with hipGetSymbolAddress (with that device current) and only that pointer is handed to the kernels.
// Every call on one GPU shares that GPU's array: calls that overlap on one GPU (two streams, or two host threads)
// race on it. The norm bound pipeline writes every scratch element before reading it, so nothing is cleared
// between calls.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <mutex>

#include "../../include/psgdk.h"

namespace psgdk {
int set_error(int code, const char* msg);
}

namespace {

constexpr size_t kNoallocScratchBytes = size_t(PSGDK_NOALLOC_SCRATCH_MIB) << 20;
static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's copy of the scratch array (looked up on the device's first call).
int scratch_for_current_device(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return psgdk::set_error(PSGDK_EHIP, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return psgdk::set_error(PSGDK_EINVAL, "device index beyond the scratch table");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      char msg[160];
      snprintf(msg, sizeof msg, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
      return psgdk::set_error(PSGDK_EHIP, msg);
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return PSGDK_OK;
}

}  // namespace

extern "C" int psgdk_norm_lower_bound_full_noalloc(int64_t n, int sign, int nb, const void* const* A, int64_t lda,
                                                   int a_dtype, const float* const* V, float* const* out,
                                                   psgdk_stream_t stream) {
  size_t need = 0;
  int rc = psgdk_norm_lower_bound_full(n, sign, nb, A, lda, a_dtype, V, out, nullptr, &need, stream);
  if (rc != PSGDK_OK) return rc;
  if (need > kNoallocScratchBytes) {
    char msg[200];
    snprintf(msg, sizeof msg, "n = %lld, nb = %d needs %zu bytes of scratch; the static scratch holds %zu",
             (long long)n, nb, need, kNoallocScratchBytes);
    return psgdk::set_error(PSGDK_ESHAPE, msg);
  }
  void* ws = nullptr;
  rc = scratch_for_current_device(&ws);
  if (rc != PSGDK_OK) return rc;
  size_t have = kNoallocScratchBytes;
  return psgdk_norm_lower_bound_full(n, sign, nb, A, lda, a_dtype, V, out, ws, &have, stream);
}

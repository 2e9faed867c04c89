// Measurement kernels (no counterpart in the reference): the read rate of the memory hierarchy and the engine clock
// during a run, the ceilings the optimizer's launches are compared against.
#include "common.h"

namespace psgdk {

// Each workgroup of 256 threads reads `iters` 4 KiB blocks of uint4: block (blockIdx * iters + i) * stride, its
// index wrapped into the buffer by `mask` (the buffer's uint4 count minus one, a power of two), so every load lies
// inside the buffer. stride 1 with grid * iters blocks = the buffer reads every byte once (HBM); an odd stride over a
// small buffer keeps it in the caches. The XOR of the loaded words is stored only when it equals a value that a
// buffer of one repeated byte never gives, so the loads stay and nothing is written.
__global__ void __launch_bounds__(256) read_rate_kernel(const uint4* __restrict__ buf, unsigned long long mask,
                                                        int iters, unsigned long long stride, unsigned* sink) {
  unsigned acc = 0;
#pragma unroll 8
  for (int i = 0; i < iters; ++i) {
    const unsigned long long blk = ((unsigned long long)blockIdx.x * (unsigned long long)iters + i) * stride;
    const uint4 v = buf[(blk * 256ull + threadIdx.x) & mask];
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == 0x9e3779b9u) sink[blockIdx.x] = acc;
}

hipError_t read_rate_launch(const void* buf, long long bytes, int wgs, int iters, long long stride, unsigned* sink,
                            hipStream_t st) {
  const unsigned long long mask = (unsigned long long)bytes / 16 - 1;
  hipLaunchKernelGGL(read_rate_kernel, dim3(wgs), dim3(256), 0, st, reinterpret_cast<const uint4*>(buf), mask, iters,
                     (unsigned long long)stride, sink);
  return hipGetLastError();
}

// One thread samples the engine clock: every step it sleeps (s_sleep 127, about 8 thousand cycles), then records
// the cycle counter and the constant-rate wall counter (out[2 i], out[2 i + 1]), for `samples` steps; the ratio of
// their increments times the wall counter's rate is the clock of the CU it runs on. Launched on a stream of its own
// beside the work being timed, it takes one wave of one CU.
__global__ void __launch_bounds__(64) clock_sample_kernel(int samples, unsigned long long* out) {
  if (threadIdx.x != 0) return;
  for (int i = 0; i < samples; ++i) {
    __builtin_amdgcn_s_sleep(127);
    out[2 * i] = (unsigned long long)clock64();
    out[2 * i + 1] = (unsigned long long)wall_clock64();
  }
}

// out[0] = the wall counter when the stream reaches this launch (marks a region for clock_sample_kernel's samples)
__global__ void __launch_bounds__(64) wall_mark_kernel(unsigned long long* out) {
  if (threadIdx.x == 0) out[0] = (unsigned long long)wall_clock64();
}

hipError_t clock_sample_launch(int samples, unsigned long long* out, hipStream_t st) {
  hipLaunchKernelGGL(clock_sample_kernel, dim3(1), dim3(64), 0, st, samples, out);
  return hipGetLastError();
}

hipError_t wall_mark_launch(unsigned long long* out, hipStream_t st) {
  hipLaunchKernelGGL(wall_mark_kernel, dim3(1), dim3(64), 0, st, out);
  return hipGetLastError();
}

}  // namespace psgdk

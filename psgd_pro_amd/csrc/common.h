// Shared device helpers for the psgdk kernels (gfx950 / CDNA4, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace psgdk {

typedef uint16_t bf16_t;  // bfloat16 storage (raw bits)
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr float kSmallestNormal = 1.17549435e-38f;  // torch.finfo(torch.float32).smallest_normal

// The calling thread's last MFMA-engine launch, for the launch profiler: the workgroups it launched and how many of
// its kernel's workgroups one CU holds at once (the runtime's occupancy query for its block and LDS size; 0 when
// that query fails). The launchers call note_launch after their hipGetLastError, and it does nothing unless the
// calling thread is profiling.
struct LaunchShape {
  int workgroups = 0, per_cu = 0;
};
void note_launch(const void* fn, long long workgroups, int threads, int lds_bytes);
LaunchShape last_launch();

// Operand element addressing of a GEMM operand viewed as X[mn][k]:
//   KC  : X[mn][k] at mn * ld + k   (k contiguous: A row-major M x K, or B given as N x K)
//   MC  : X[mn][k] at k * ld + mn   (mn contiguous: A given as K x M, or B row-major K x N)
//   SYM : X[mn][k] = S[min][max] read from the upper triangle of a square S; the strict lower part is sign * the
//         transposed upper element: sign = +1 symmetric, -1 skew-symmetric (diagonal read as 0), 0 upper-triangular
//         (lower part is zero, TRMM).
enum OpMode : int { KC = 0, MC = 1, SYM = 2 };

__device__ __forceinline__ float bf16_to_f32(bf16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

// float -> bfloat16 with round-to-nearest-even (NaN stays NaN).
__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (bf16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (bf16_t)(u >> 16);
}

__device__ __forceinline__ uint32_t pack2(bf16_t lo, bf16_t hi) { return (uint32_t)lo | ((uint32_t)hi << 16); }

template <typename T> __device__ __forceinline__ float to_f32(T v);
template <> __device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ float to_f32<bf16_t>(bf16_t v) { return bf16_to_f32(v); }
template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ bf16_t from_f32<bf16_t>(float v) { return f32_to_bf16(v); }

// wave64 reductions
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Raw buffer resource over [base, base + bytes): loads at offsets >= bytes (clamped to 2^31 - 1) return zero,
// so a lane with nothing to load passes offset 0x7fffffff instead of branching.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, long long bytes) {
  const int n = bytes > 0x7fffffffLL ? 0x7fffffff : (int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}
constexpr int kOob = 0x7fffffff;

// Block-wide reductions for blockDim.x a multiple of 64 (<= 1024). `red` holds >= 16 floats of LDS.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < nw; ++i) t += red[i];  // fixed order: deterministic
  return t;
}
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float t = -INFINITY;
  for (int i = 0; i < nw; ++i) t = fmaxf(t, red[i]);
  return t;
}

}  // namespace psgdk

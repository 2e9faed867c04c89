// Small products on the k-contiguous operand contract of the bf16 kernel (bf16 operands, or fp32 ones stored
// k-contiguous), plain-store epilogue only.
//
// A launch whose 128 x 128 tiles leave most of the 256 CUs idle is bound by the chain of global-load round trips of
// its few workgroups: the pipelined kernels keep one k tile of 64 in flight, so a 128-tile at K = 512 waits for
// eight round trips in a row. Here a workgroup owns a 64 x 64 output tile (four times as many workgroups) and moves k
// in chunks of 512 bytes per row (256 bf16 or 128 fp32), two chunks in flight in registers: K = 512 bf16 is one
// wait. Four waves of 32 x 32 (2 x 2 MFMA tiles of 16 x 16). The chunk passes through one LDS stage of 64 rows x
// 512 bytes per operand, 16-byte pieces XOR-swizzled by row (piece p of row r at slot p ^ (r % 16): the 16 rows of a
// fragment read fall on 16 distinct bank groups; the 32 lanes that store one row still fill its 32 slots).
// fp32 operands feed four v_mfma_f32_16x16x4f32 per 16-byte fragment pair (lane group g holds k = 4 g + s of both
// operands) and sum k in blocks of 128 (one chunk) into a second accumulator set, as the other fp32 paths do.
// Epilogue straight from the accumulators: C (fp32) and / or Cb (bf16) at (row, col), CTb (bf16) / CT (fp32) at
// (col, row); a SYRK writes row <= col, and with out_mode 1 also (col, row) for row < col.
#include <cstring>

#include "gemm_bf16.h"

namespace psgdk {

namespace {

constexpr int SM_T = 64;                    // output tile
constexpr int SM_ROWB = 512;                // bytes per row per chunk
constexpr int SM_NV = SM_T * (SM_ROWB / 16) / 256;  // 16-byte pieces per thread per operand per chunk (8)

// One operand's chunk in registers: thread t owns piece t % 32 of rows t / 32 + 8 i.
struct SmChunk {
  uint4 r[SM_NV];
};

template <typename T>
__device__ __forceinline__ void sm_load(SmChunk& c, __amdgpu_buffer_rsrc_t rs, const int (&off)[SM_NV], int k0, int K,
                                        int piece) {
  constexpr int CE = 16 / sizeof(T);
  const bool kin = k0 + piece * CE < K;
#pragma unroll
  for (int i = 0; i < SM_NV; ++i)
    c.r[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, kin ? off[i] : kOob,
                                                                              k0 * (int)sizeof(T), 0));
}

__device__ __forceinline__ void sm_store(const SmChunk& c, unsigned char* lds, int rr, int piece) {
#pragma unroll
  for (int i = 0; i < SM_NV; ++i) {
    const int row = rr + 8 * i;
    *reinterpret_cast<uint4*>(lds + row * SM_ROWB + ((piece ^ (row & 15)) << 4)) = c.r[i];
  }
}

}  // namespace

template <typename T>
__global__ void __launch_bounds__(256) gemm_small_kernel(const GB16Args p) {
  constexpr bool BF = sizeof(T) == 2;
  constexpr int CE = 16 / sizeof(T);          // elements per piece
  constexpr int KC = (SM_ROWB / 16) * CE;     // k per chunk
  extern __shared__ __align__(16) unsigned char smem[];
  unsigned char* const As = smem;
  unsigned char* const Bs = smem + SM_T * SM_ROWB;

  const int b = blockIdx.x / p.ntiles, tile = blockIdx.x % p.ntiles;
  int ti, tj;
  if (p.tri) {
    ti = 0;
    int rem = tile, rowlen = p.tiles_m;
    while (rem >= rowlen) { rem -= rowlen; ++ti; --rowlen; }
    tj = ti + rem;
  } else {
    ti = tile / p.tiles_n;
    tj = tile % p.tiles_n;
  }
  const int m0 = ti * SM_T, n0 = tj * SM_T;
  const int rowsB = p.tri ? p.M : p.N;
  const T* __restrict__ Ap = reinterpret_cast<const T*>(p.A[b]);
  const T* __restrict__ Bp = reinterpret_cast<const T*>(p.tri ? p.A[b] : p.B[b]);
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(Ap, (long long)p.M * p.lda * (long long)sizeof(T));
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(Bp, (long long)rowsB * p.ldb * (long long)sizeof(T));
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1, r16 = lane & 15, g = lane >> 4;
  const int rr = tid >> 5, piece = tid & 31;
  int oa[SM_NV], ob[SM_NV];
#pragma unroll
  for (int i = 0; i < SM_NV; ++i) {
    const int row = rr + 8 * i;
    oa[i] = m0 + row < p.M ? (int)(((long long)(m0 + row) * p.lda + piece * CE) * (long long)sizeof(T)) : kOob;
    ob[i] = n0 + row < rowsB ? (int)(((long long)(n0 + row) * p.ldb + piece * CE) * (long long)sizeof(T)) : kOob;
  }

  f32x4_t acc[2][2], part[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = part[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  auto& dst = BF ? acc : part;

  // chunk c from LDS: 8 fragment steps of 16 bytes per lane (32 bf16 or 16 fp32 of k)
  auto compute = [&]() {
#pragma unroll
    for (int s = 0; s < SM_ROWB / 64; ++s) {
      const int pc = s * 4 + g;
      uint4 af[2], bfr[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int row = wm * 32 + i * 16 + r16;
        af[i] = *reinterpret_cast<const uint4*>(As + row * SM_ROWB + ((pc ^ (row & 15)) << 4));
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int row = wn * 32 + j * 16 + r16;
        bfr[j] = *reinterpret_cast<const uint4*>(Bs + row * SM_ROWB + ((pc ^ (row & 15)) << 4));
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          if constexpr (BF) {
            dst[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, af[i]),
                                                                __builtin_bit_cast(bf16x8_t, bfr[j]), dst[i][j], 0, 0, 0);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              dst[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float((&af[i].x)[e]),
                                                               __uint_as_float((&bfr[j].x)[e]), dst[i][j], 0, 0, 0);
          }
        }
    }
    if constexpr (!BF) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          acc[i][j] += part[i][j];
          part[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        }
    }
  };

  // two register sets, the loop unrolled by two so that each set's index is static
  const int nc = (p.K + KC - 1) / KC;
  SmChunk a0, b0, a1, b1;
  sm_load<T>(a0, ra, oa, 0, p.K, piece);
  sm_load<T>(b0, rb, ob, 0, p.K, piece);
  if (nc > 1) {
    sm_load<T>(a1, ra, oa, KC, p.K, piece);
    sm_load<T>(b1, rb, ob, KC, p.K, piece);
  }
  for (int c = 0; c < nc; c += 2) {
    if (c > 0) __syncthreads();  // every wave is done with the previous chunk
    sm_store(a0, As, rr, piece);
    sm_store(b0, Bs, rr, piece);
    __syncthreads();
    if (c + 2 < nc) {
      sm_load<T>(a0, ra, oa, (c + 2) * KC, p.K, piece);
      sm_load<T>(b0, rb, ob, (c + 2) * KC, p.K, piece);
    }
    compute();
    if (c + 1 >= nc) break;
    __syncthreads();
    sm_store(a1, As, rr, piece);
    sm_store(b1, Bs, rr, piece);
    __syncthreads();
    if (c + 3 < nc) {
      sm_load<T>(a1, ra, oa, (c + 3) * KC, p.K, piece);
      sm_load<T>(b1, rb, ob, (c + 3) * KC, p.K, piece);
    }
    compute();
  }

  // Epilogue: lane (r16, g) of wave (wm, wn) holds rows 4 g + e of column r16 of MFMA tile (i, j)
  float* __restrict__ C = p.C[b];
  bf16_t* __restrict__ Cb = p.Cb[b];
  bf16_t* __restrict__ CTb = p.CTb[b];
  float* __restrict__ CT = p.CT[b];
  const bool mirror = p.tri && p.out_mode == 1;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = m0 + wm * 32 + i * 16 + 4 * g + e, col = n0 + wn * 32 + j * 16 + r16;
        if (row >= p.M || col >= p.N || (p.tri && row > col)) continue;
        const float v = p.alpha * acc[i][j][e];
        if (C) C[(long long)row * p.ldc + col] = v;
        if (Cb) Cb[(long long)row * p.ldcb + col] = f32_to_bf16(v);
        if (CTb) CTb[(long long)col * p.ldct + row] = f32_to_bf16(v);
        if (CT) CT[(long long)col * p.ldct + row] = v;
        if (mirror && row < col) {
          if (C) C[(long long)col * p.ldc + row] = v;
          if (Cb) Cb[(long long)col * p.ldcb + row] = f32_to_bf16(v);
        }
      }
}

// ------------------------------------------------------------------------------------------------------------
// Tiny products: a launch whose 64-tiles would fill only a fraction of the CUs (one 512 x 512 SYRK: 36 workgroups)
// is bound by one workgroup's chain: its loads, a pass through LDS per chunk, the epilogue. Here a workgroup owns a
// 32 x 32 output tile (four times as many workgroups again) and its four waves split k: wave w takes the k batches
// w, w + 4, ... of 256 bytes per row (128 bf16 or 64 fp32), so each wave loads half the bytes a whole-k quarter
// tile would (one 512 x 512 SYRK: 5.4 us against 6.7 us in the kernel trace). A lane loads its MFMA fragments
// straight from global memory into registers (lane (r, g) holds k = 32 s + 8 g .. + 7 of row r for step s: bf16,
// one v_mfma_f32_16x16x32_bf16 per fragment pair; fp32 k = 16 s + 4 g + e, four v_mfma_f32_16x16x4f32), two batches
// in flight, no LDS staging. The four partial tiles meet in LDS and are added in the order w = 0..3 (fp32: each
// batch summed on its own first): deterministic, but rounded in another order than the other kernels' k-order
// chains. The epilogue writes what gemm_small_kernel writes. Its own argument block carries at most TY_MAXB
// problems (a launch of more is split), about 450 bytes of kernel arguments.
namespace {

constexpr int TY_T = 32;    // output tile
constexpr int TY_NS = 4;    // fragment steps (16 bytes per lane) per batch
constexpr int TY_MAXB = 8;  // problems per launch

struct TinyArgs {
  int M, N, K, tri, out_mode, tiles_m, tiles_n, ntiles;
  long long lda, ldb, ldc, ldcb, ldct;
  float alpha;
  const void* A[TY_MAXB];
  const void* B[TY_MAXB];
  float* C[TY_MAXB];
  bf16_t* Cb[TY_MAXB];
  bf16_t* CTb[TY_MAXB];
  float* CT[TY_MAXB];
};

struct TyBatch {
  uint4 a[2][TY_NS], b[2][TY_NS];
};

// batch at k0: step s of row half i reads 16 bytes at k = k0 + s KS + g CE (zero past K or past the last row)
template <typename T>
__device__ __forceinline__ void ty_load(TyBatch& x, __amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rb,
                                        const int (&oa)[2], const int (&ob)[2], int k0, int K, int g) {
  constexpr int CE = 16 / sizeof(T), KS = 4 * CE;
#pragma unroll
  for (int s = 0; s < TY_NS; ++s) {
    const bool kin = k0 + s * KS + g * CE < K;
    const int soff = (k0 + s * KS) * (int)sizeof(T);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      x.a[i][s] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(ra, kin ? oa[i] : kOob, soff, 0));
      x.b[i][s] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rb, kin ? ob[i] : kOob, soff, 0));
    }
  }
}

template <typename T>
__device__ __forceinline__ void ty_mma(const TyBatch& x, f32x4_t (&acc)[2][2]) {
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int s = 0; s < TY_NS; ++s)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, x.a[i][s]),
                                                              __builtin_bit_cast(bf16x8_t, x.b[j][s]), acc[i][j], 0, 0,
                                                              0);
  } else {
    f32x4_t part[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) part[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < TY_NS; ++s)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            part[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float((&x.a[i][s].x)[e]),
                                                              __uint_as_float((&x.b[j][s].x)[e]), part[i][j], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] += part[i][j];
  }
}

}  // namespace

template <typename T>
__global__ void __launch_bounds__(256) gemm_tiny_kernel(const TinyArgs p) {
  constexpr int CE = 16 / sizeof(T);
  constexpr int KB = TY_NS * 4 * CE;  // k per batch
  __shared__ float red[4][TY_T][TY_T + 1];

  const int b = blockIdx.x / p.ntiles, tile = blockIdx.x % p.ntiles;
  int ti, tj;
  if (p.tri) {
    ti = 0;
    int rem = tile, rowlen = p.tiles_m;
    while (rem >= rowlen) { rem -= rowlen; ++ti; --rowlen; }
    tj = ti + rem;
  } else {
    ti = tile / p.tiles_n;
    tj = tile % p.tiles_n;
  }
  const int m0 = ti * TY_T, n0 = tj * TY_T;
  const int rowsB = p.tri ? p.M : p.N;
  const T* __restrict__ Ap = reinterpret_cast<const T*>(p.A[b]);
  const T* __restrict__ Bp = reinterpret_cast<const T*>(p.tri ? p.A[b] : p.B[b]);
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(Ap, (long long)p.M * p.lda * (long long)sizeof(T));
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(Bp, (long long)rowsB * p.ldb * (long long)sizeof(T));
  const int lane = threadIdx.x & 63, r16 = lane & 15, g = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: the batches' offsets stay scalar
  int oa[2], ob[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int ra_ = m0 + 16 * i + r16, rb_ = n0 + 16 * i + r16;
    oa[i] = ra_ < p.M ? (int)(((long long)ra_ * p.lda + g * CE) * (long long)sizeof(T)) : kOob;
    ob[i] = rb_ < rowsB ? (int)(((long long)rb_ * p.ldb + g * CE) * (long long)sizeof(T)) : kOob;
  }

  f32x4_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // wave w: batches w, w + 4, w + 8, ...; two register sets, the loop unrolled by two so each set's index is static
  const int nbat = (p.K + KB - 1) / KB;
  TyBatch x0, x1;
  if (w < nbat) ty_load<T>(x0, ra, rb, oa, ob, w * KB, p.K, g);
  if (w + 4 < nbat) ty_load<T>(x1, ra, rb, oa, ob, (w + 4) * KB, p.K, g);
  for (int bt = w; bt < nbat; bt += 8) {
    ty_mma<T>(x0, acc);
    if (bt + 8 < nbat) ty_load<T>(x0, ra, rb, oa, ob, (bt + 8) * KB, p.K, g);
    if (bt + 4 >= nbat) break;
    ty_mma<T>(x1, acc);
    if (bt + 12 < nbat) ty_load<T>(x1, ra, rb, oa, ob, (bt + 12) * KB, p.K, g);
  }

  // lane (r16, g) holds rows 4 g + e of column r16 of MFMA tile (i, j)
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) red[w][16 * i + 4 * g + e][16 * j + r16] = acc[i][j][e];
  __syncthreads();

  // thread t: row t / 8, columns 4 (t % 8) .. + 3 of the tile
  const int rl = threadIdx.x >> 3, cl = (threadIdx.x & 7) * 4;
  const int row = m0 + rl;
  if (row >= p.M) return;
  float* __restrict__ C = p.C[b];
  bf16_t* __restrict__ Cb = p.Cb[b];
  bf16_t* __restrict__ CTb = p.CTb[b];
  float* __restrict__ CT = p.CT[b];
  const bool mirror = p.tri && p.out_mode == 1;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int col = n0 + cl + q;
    if (col >= p.N || (p.tri && row > col)) continue;
    const float v = p.alpha * (((red[0][rl][cl + q] + red[1][rl][cl + q]) + red[2][rl][cl + q]) + red[3][rl][cl + q]);
    if (C) C[(long long)row * p.ldc + col] = v;
    if (Cb) Cb[(long long)row * p.ldcb + col] = f32_to_bf16(v);
    if (CTb) CTb[(long long)col * p.ldct + row] = f32_to_bf16(v);
    if (CT) CT[(long long)col * p.ldct + row] = v;
    if (mirror && row < col) {
      if (C) C[(long long)col * p.ldc + row] = v;
      if (Cb) Cb[(long long)col * p.ldcb + row] = f32_to_bf16(v);
    }
  }
}

int gemm_tiny_tiles(long long M, long long N, int tri) {
  const long long tm = (M + TY_T - 1) / TY_T, tn = (N + TY_T - 1) / TY_T;
  return (int)(tri ? tm * (tm + 1) / 2 : tm * tn);
}

hipError_t gemm_tiny_launch(const GB16Args& a, int esz, hipStream_t st) {
  if (a.epi != EPI_STORE || a.kbeg || a.amc || a.bmc) return hipErrorInvalidValue;
  TinyArgs t;
  std::memset(&t, 0, sizeof t);
  t.M = a.M; t.N = a.N; t.K = a.K; t.tri = a.tri; t.out_mode = a.out_mode;
  t.lda = a.lda; t.ldb = a.ldb; t.ldc = a.ldc; t.ldcb = a.ldcb; t.ldct = a.ldct; t.alpha = a.alpha;
  t.tiles_m = (a.M + TY_T - 1) / TY_T;
  t.tiles_n = (a.N + TY_T - 1) / TY_T;
  t.ntiles = a.tri ? t.tiles_m * (t.tiles_m + 1) / 2 : t.tiles_m * t.tiles_n;
  void (*fn)(TinyArgs) = esz == 4 ? gemm_tiny_kernel<float> : gemm_tiny_kernel<bf16_t>;
  for (int b0 = 0; b0 < a.nb; b0 += TY_MAXB) {
    const int nb = a.nb - b0 < TY_MAXB ? a.nb - b0 : TY_MAXB;
    for (int b = 0; b < nb; ++b) {
      t.A[b] = a.A[b0 + b]; t.B[b] = a.B[b0 + b];
      t.C[b] = a.C[b0 + b]; t.Cb[b] = a.Cb[b0 + b]; t.CTb[b] = a.CTb[b0 + b]; t.CT[b] = a.CT[b0 + b];
    }
    hipLaunchKernelGGL(fn, dim3(t.ntiles * nb), dim3(256), 0, st, t);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  note_launch(reinterpret_cast<const void*>(fn), (long long)t.ntiles * a.nb, 256, 0);
  return hipSuccess;
}

int gemm_small_tiles(long long M, long long N, int tri) {
  const long long tm = (M + SM_T - 1) / SM_T, tn = (N + SM_T - 1) / SM_T;
  return (int)(tri ? tm * (tm + 1) / 2 : tm * tn);
}

hipError_t gemm_small_launch(GB16Args& a, int esz, hipStream_t st) {
  constexpr int smem = 2 * SM_T * SM_ROWB;  // one stage of A and B: 64 KB
  void (*fn)(GB16Args) = esz == 4 ? gemm_small_kernel<float> : gemm_small_kernel<bf16_t>;
  static const hipError_t attr_b =
      hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_small_kernel<bf16_t>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, smem);
  static const hipError_t attr_f =
      hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_small_kernel<float>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, smem);
  if (attr_b != hipSuccess) return attr_b;
  if (attr_f != hipSuccess) return attr_f;
  if (a.epi != EPI_STORE || a.kbeg || a.amc || a.bmc) return hipErrorInvalidValue;
  a.tiles_m = (a.M + SM_T - 1) / SM_T;
  a.tiles_n = (a.N + SM_T - 1) / SM_T;
  a.ntiles = a.tri ? a.tiles_m * (a.tiles_m + 1) / 2 : a.tiles_m * a.tiles_n;
  hipLaunchKernelGGL(fn, dim3(a.ntiles * a.nb), dim3(256), smem, st, a);
  const hipError_t e = hipGetLastError();
  note_launch(reinterpret_cast<const void*>(fn), (long long)a.ntiles * a.nb, 256, smem);
  return e;
}

}  // namespace psgdk

// CDNA4 MFMA GEMM / SYRK / SYMM / TRMM engine.
//
// One kernel template computes C = op(A) op(B) for up to MAXB same-shape problems per launch (grouped launch: the
// problems' pointers travel by value in the kernel arguments). Both operands are viewed as X[mn][k] and staged in
// LDS k-contiguous, one 144-byte row per mn (64 bf16 or 32 fp32 plus a 16-byte pad that spreads consecutive rows
// over the LDS banks), double-buffered with one barrier per k-tile.
//
// Loads (global -> registers -> LDS):
//   KC operands: one 16-byte vector of k per thread per step (coalesced along k).
//   MC operands: each thread loads CE rows of 4 consecutive mn (coalesced along mn) and transposes the CE x 4 block
//                in registers into four k-contiguous LDS vectors.
//   SYM operands: tiles strictly above the diagonal are KC loads of the stored upper triangle, tiles strictly below
//                 are MC loads of the mirrored upper tile (times the sign); tiles crossing the diagonal and ragged
//                 edge tiles take an element-wise guarded path. The strict lower triangle is never read.
// Math: bf16 inputs use v_mfma_f32_16x16x32_bf16, fp32 inputs v_mfma_f32_16x16x4_f32; fp32 accumulation.
// Each wave owns an (BM/WM) x (BN/WN) block of 16x16 MFMA tiles.
// Work mapping: the (problem, tile) list is dealt out so that each XCD (workgroups are dispatched round-robin
// over the 8 XCDs) receives a contiguous run of tiles, so tiles sharing operand panels share one L2.
#include "gemm.h"

namespace psgdk {

enum LoadHow : int { LD_KC = 0, LD_MC = 1, LD_SCALAR = 2, LD_ZERO = 3 };

constexpr int KCHUNK = 128;  // k per accumulation chunk

template <int PREC> struct Prec;
template <> struct Prec<0> { static constexpr int BK = 32, CE = 4, ESZ = 4; };
template <> struct Prec<1> { static constexpr int BK = 64, CE = 8, ESZ = 2; };

// CE fp32 values -> one 16-byte LDS vector in the compute type
template <int PREC> __device__ __forceinline__ uint4 pack_vec(const float* v);
template <> __device__ __forceinline__ uint4 pack_vec<0>(const float* v) {
  return make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3]));
}
template <> __device__ __forceinline__ uint4 pack_vec<1>(const float* v) {
  return make_uint4(pack2(f32_to_bf16(v[0]), f32_to_bf16(v[1])), pack2(f32_to_bf16(v[2]), f32_to_bf16(v[3])),
                    pack2(f32_to_bf16(v[4]), f32_to_bf16(v[5])), pack2(f32_to_bf16(v[6]), f32_to_bf16(v[7])));
}

// Element (mn, k) of an operand (KC: p[mn][k]; MC: p[k][mn]; SYM: the upper triangle, the lower one mirrored with
// `sign`, zero for sign 0, a zero diagonal for sign < 0), zero past rows or K. Branch-free: the offset and a scale
// (0, 1 or sign) are selected first and the load is unconditional (element 0 for an element that is not read, the
// scale then selecting zero rather than multiplying, so that a non-finite element 0 cannot leak in).
template <typename T>
__device__ __forceinline__ float fetch(const T* __restrict__ p, int mode, int sign, long long ld, int mn, int k,
                                       int rows, int K) {
  const bool in = mn < rows && k < K;
  const bool up = mode == KC || (mode == SYM && mn < k);
  const long long off = !in ? 0 : up ? (long long)mn * ld + k : (long long)k * ld + mn;
  const float sc = !in ? 0.f
                 : mode != SYM || mn < k ? 1.f
                 : mn > k ? (float)sign
                          : (sign < 0 ? 0.f : 1.f);
  const float v = to_f32<T>(p[off]);
  return sc != 0.f ? sc * v : 0.f;
}

// Loads CE consecutive k of row mn (KC addressing) and converts them to the compute type.
template <int PREC, typename T>
__device__ __forceinline__ uint4 load_kc_vec(const T* __restrict__ p) {
  if constexpr (PREC == 1 && sizeof(T) == 2) {
    return *reinterpret_cast<const uint4*>(p);
  } else if constexpr (PREC == 1) {
    const float4 x = reinterpret_cast<const float4*>(p)[0], y = reinterpret_cast<const float4*>(p)[1];
    const float v[8] = {x.x, x.y, x.z, x.w, y.x, y.y, y.z, y.w};
    return pack_vec<1>(v);
  } else if constexpr (sizeof(T) == 4) {
    return *reinterpret_cast<const uint4*>(p);
  } else {
    const uint2 x = *reinterpret_cast<const uint2*>(p);
    const float v[4] = {bf16_to_f32((bf16_t)(x.x & 0xffff)), bf16_to_f32((bf16_t)(x.x >> 16)),
                        bf16_to_f32((bf16_t)(x.y & 0xffff)), bf16_to_f32((bf16_t)(x.y >> 16))};
    return pack_vec<0>(v);
  }
}

// Loads 4 consecutive mn of row k (MC addressing) as fp32.
template <typename T>
__device__ __forceinline__ void load_mc4(const T* __restrict__ p, float* v) {
  if constexpr (sizeof(T) == 4) {
    const float4 x = *reinterpret_cast<const float4*>(p);
    v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
  } else {
    const uint2 x = *reinterpret_cast<const uint2*>(p);
    v[0] = bf16_to_f32((bf16_t)(x.x & 0xffff)); v[1] = bf16_to_f32((bf16_t)(x.x >> 16));
    v[2] = bf16_to_f32((bf16_t)(x.y & 0xffff)); v[3] = bf16_to_f32((bf16_t)(x.y >> 16));
  }
}

template <int PREC, typename T, int ROWS, int NT>
struct TileLoader {
  static constexpr int BK = Prec<PREC>::BK, CE = Prec<PREC>::CE, ESZ = Prec<PREC>::ESZ, KP = BK + CE;
  static constexpr int KV = BK / CE;                    // 16-byte vectors per LDS row
  static constexpr int NVEC = ROWS * KV;                // vectors per tile (KC mapping)
  static constexpr int NV_KC = (NVEC + NT - 1) / NT;
  static constexpr int NBLK = KV * (ROWS / 4);          // CE(k) x 4(mn) blocks (MC mapping)
  static constexpr int NB_MC = (NBLK + NT - 1) / NT;
  static constexpr int NREG = NV_KC > 4 * NB_MC ? NV_KC : 4 * NB_MC;
  uint4 reg[NREG];
  int how;

  __device__ __forceinline__ void load(const T* __restrict__ p, int mode, int sign, long long ld, int mn0, int k0,
                                       int rows, int K, int vec_ok) {
    const int tid = threadIdx.x;
    const bool full = mn0 + ROWS <= rows && k0 + BK <= K;
    int h = LD_SCALAR;
    if (mode == SYM && sign == 0 && mn0 >= k0 + BK) h = LD_ZERO;
    else if (full && vec_ok) {
      if (mode == KC) h = LD_KC;
      else if (mode == MC) h = LD_MC;
      else if (mn0 + ROWS <= k0) h = LD_KC;
      else if (mn0 >= k0 + BK) h = LD_MC;
    }
    how = h;
    if (h == LD_KC) {
#pragma unroll
      for (int i = 0; i < NV_KC; ++i) {
        const int v = tid + NT * i;
        if (NVEC % NT == 0 || v < NVEC) {
          const int row = v / KV, kv = v % KV;
          reg[i] = load_kc_vec<PREC, T>(p + (long long)(mn0 + row) * ld + k0 + kv * CE);
        }
      }
    } else if (h == LD_MC) {
      const float sg = mode == SYM ? (float)sign : 1.f;
#pragma unroll
      for (int bi = 0; bi < NB_MC; ++bi) {
        const int blk = tid + NT * bi;
        if (NBLK % NT == 0 || blk < NBLK) {
          const int mnb = blk % (ROWS / 4), kb = blk / (ROWS / 4);
          float e[CE][4];
          const T* q = p + (long long)(k0 + kb * CE) * ld + mn0 + mnb * 4;
#pragma unroll
          for (int j = 0; j < CE; ++j) load_mc4<T>(q + (long long)j * ld, e[j]);
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            float v[CE];
#pragma unroll
            for (int j = 0; j < CE; ++j) v[j] = sg * e[j][c];
            reg[bi * 4 + c] = pack_vec<PREC>(v);
          }
        }
      }
    } else if (h == LD_SCALAR) {
#pragma unroll
      for (int i = 0; i < NV_KC; ++i) {
        const int v = tid + NT * i;
        if (NVEC % NT == 0 || v < NVEC) {
          const int row = v / KV, kv = v % KV;
          float x[CE];
#pragma unroll
          for (int e = 0; e < CE; ++e) x[e] = fetch<T>(p, mode, sign, ld, mn0 + row, k0 + kv * CE + e, rows, K);
          reg[i] = pack_vec<PREC>(x);
        }
      }
    }
  }

  __device__ __forceinline__ void store(unsigned char* lds) const {
    const int tid = threadIdx.x;
    if (how == LD_MC) {
#pragma unroll
      for (int bi = 0; bi < NB_MC; ++bi) {
        const int blk = tid + NT * bi;
        if (NBLK % NT == 0 || blk < NBLK) {
          const int mnb = blk % (ROWS / 4), kb = blk / (ROWS / 4);
#pragma unroll
          for (int c = 0; c < 4; ++c)
            *reinterpret_cast<uint4*>(lds + ((mnb * 4 + c) * KP + kb * CE) * ESZ) = reg[bi * 4 + c];
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < NV_KC; ++i) {
        const int v = tid + NT * i;
        if (NVEC % NT == 0 || v < NVEC) {
          const int row = v / KV, kv = v % KV;
          *reinterpret_cast<uint4*>(lds + (row * KP + kv * CE) * ESZ) = how == LD_ZERO ? make_uint4(0, 0, 0, 0) : reg[i];
        }
      }
    }
  }
};

// Maps the flattened workgroup id to (problem, tile) so that each XCD gets a contiguous run of the tile list.
__device__ __forceinline__ int xcd_remap(int w, int G) {
  const int cnt = G / 8, rem = G % 8, xcd = w % 8, slot = w / 8;
  return xcd < rem ? xcd * (cnt + 1) + slot : rem * (cnt + 1) + (xcd - rem) * cnt + slot;
}

template <int PREC, typename TA, typename TB, int BM, int BN, int WM, int WN>
__global__ void __launch_bounds__(WM * WN * 64) gemm_kernel(const GemmArgs p) {
  constexpr int NT = WM * WN * 64;
  constexpr int BK = Prec<PREC>::BK, CE = Prec<PREC>::CE, ESZ = Prec<PREC>::ESZ, KP = BK + CE;
  constexpr int FM = BM / WM / 16, FN = BN / WN / 16;
  static_assert(FM >= 1 && FN >= 1, "wave tile");
  extern __shared__ __align__(16) unsigned char smem[];
  unsigned char* const As0 = smem;
  unsigned char* const Bs0 = smem + 2 * BM * KP * ESZ;
  constexpr int ASZ = BM * KP * ESZ, BSZ = BN * KP * ESZ;

  const int G = p.ntiles * p.nb * p.splitk;
  const int logical0 = xcd_remap(blockIdx.x, G);
  const int split = logical0 % p.splitk;
  const int logical = logical0 / p.splitk;
  const int b = logical / p.ntiles;
  const int tile = logical % p.ntiles;
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
  const int m0 = ti * BM, n0 = tj * BN;
  const TA* __restrict__ Ap = reinterpret_cast<const TA*>(p.A[b]);
  const TB* __restrict__ Bp = reinterpret_cast<const TB*>(p.B[b]);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int r = lane & 15, g = lane >> 4;

  f32x4_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  int kbeg = split * p.kchunk;
  const int kend = min(p.K, kbeg + p.kchunk);
  if (p.kbeg_tri) kbeg = max(kbeg, (m0 / BK) * BK);
  const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;

  TileLoader<PREC, TA, BM, NT> la;
  TileLoader<PREC, TB, BN, NT> lb;
  if (nk > 0) {
    la.load(Ap, p.amode, p.asign, p.lda, m0, kbeg, p.M, kend, p.avec);
    lb.load(Bp, p.bmode, p.bsign, p.ldb, n0, kbeg, p.N, kend, p.bvec);
    la.store(As0);
    lb.store(Bs0);
  }
  __syncthreads();

  // The k loop accumulates KCHUNK-wide chunks in `part` and folds each chunk into `acc`: one long fp32 FMA chain over
  // all of K carries several times the rounding error of blocked summation against an fp64 product.
  constexpr int KC_TILES = KCHUNK / BK;
  f32x4_t part[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) part[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      const int k0 = kbeg + (kt + 1) * BK;
      la.load(Ap, p.amode, p.asign, p.lda, m0, k0, p.M, kend, p.avec);
      lb.load(Bp, p.bmode, p.bsign, p.ldb, n0, k0, p.N, kend, p.bvec);
    }
    const unsigned char* As = As0 + cur * ASZ;
    const unsigned char* Bs = Bs0 + cur * BSZ;
    if constexpr (PREC == 1) {
#pragma unroll
      for (int ks = 0; ks < BK / 32; ++ks) {
        bf16x8_t af[FM], bfr[FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
          af[i] = *reinterpret_cast<const bf16x8_t*>(As + ((wm * FM * 16 + i * 16 + r) * KP + ks * 32 + g * 8) * ESZ);
#pragma unroll
        for (int j = 0; j < FN; ++j)
          bfr[j] = *reinterpret_cast<const bf16x8_t*>(Bs + ((wn * FN * 16 + j * 16 + r) * KP + ks * 32 + g * 8) * ESZ);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j) part[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], part[i][j], 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int kq = 0; kq < BK / 16; ++kq) {
        f32x4_t af[FM], bfr[FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
          af[i] = *reinterpret_cast<const f32x4_t*>(As + ((wm * FM * 16 + i * 16 + r) * KP + kq * 16 + g * 4) * ESZ);
#pragma unroll
        for (int j = 0; j < FN; ++j)
          bfr[j] = *reinterpret_cast<const f32x4_t*>(Bs + ((wn * FN * 16 + j * 16 + r) * KP + kq * 16 + g * 4) * ESZ);
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) part[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][s], bfr[j][s], part[i][j], 0, 0, 0);
      }
    }
    if ((kt + 1) % KC_TILES == 0 || !more) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          acc[i][j] += part[i][j];
          part[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        }
    }
    if (more) {
      la.store(As0 + (cur ^ 1) * ASZ);
      lb.store(Bs0 + (cur ^ 1) * BSZ);
    }
    __syncthreads();
  }

  // Epilogue. Lane (r, g) of wave (wm, wn) holds rows 4g..4g+3 of column r of each 16x16 tile.
  float* __restrict__ C = p.C[b] + (long long)split * p.M * p.ldc;
  const float* __restrict__ X1 = p.X1[b];
  const float* __restrict__ X2 = p.X2[b];
  float s0 = 0.f, s1 = 0.f;
  if (p.epi != EPI_STORE && p.epi != EPI_SUMSQ) {
    s0 = p.s[b][0];
    if (p.epi == EPI_FACTOR || p.epi == EPI_PROC) s1 = p.s[b][1];
  }
  const long long ldc = p.ldc, ldx = p.ldx;
  float t1 = 0.f, t2 = 0.f;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int col = n0 + wn * FN * 16 + j * 16 + r;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = m0 + wm * FM * 16 + i * 16 + g * 4 + e;
        if (row >= p.M || col >= p.N) continue;
        if (p.tri && row > col) continue;
        const float a = acc[i][j][e];
        float v;
        const long long off = (long long)row * ldc + col;
        switch (p.epi) {
          case EPI_FACTOR: { const float q = X1[(long long)row * ldx + col]; v = q - s0 * (a - s1 * q); break; }
          case EPI_PROC: {
            const long long xo = (long long)row * ldx + col;
            v = X1[xo] + s0 * X2[xo] + 0.5f * s0 * s0 * s1 * a;
            break;
          }
          case EPI_SCALE: v = s0 * a; break;
          case EPI_RQ: {
            v = s0 * a;
            if (row == col) t1 += v;
            t2 += s0 * X1[(long long)col * ldx + row] * v;
            break;
          }
          case EPI_SUMSQ: v = p.alpha * a; t1 += v * v; break;
          case EPI_STRACE: {  // tri: element (row, col), row <= col, stands for (col, row) too
            v = (s0 * a) * s0;
            t2 += v * (X1[(long long)row * ldx + col] + (row != col ? X1[(long long)col * ldx + row] : 0.f));
            break;
          }
          default: v = p.beta != 0.f ? p.alpha * a + p.beta * C[off] : p.alpha * a; break;
        }
        if (p.tri) {
          if (p.out_mode == 2) {
            C[(long long)row * p.N - (long long)row * (row - 1) / 2 + (col - row)] = v;
          } else {
            C[off] = v;
            if (p.out_mode == 1 && row != col) C[(long long)col * ldc + row] = v;
          }
        } else {
          C[off] = v;
        }
      }
    }
  }
  if (p.epi == EPI_RQ || p.epi == EPI_SUMSQ || p.epi == EPI_STRACE) {
    __shared__ float red[16];
    t1 = block_sum(t1, red);
    if (p.epi == EPI_RQ || p.epi == EPI_STRACE) t2 = block_sum(t2, red);
    if (tid == 0) {
      p.part[b][2 * tile] = t1;
      p.part[b][2 * tile + 1] = t2;
    }
  }
}

// One MFMA on a single wave with operands placed by the lane layout the GEMM assumes; the host compares C with
// A @ B (layout check of the compiler builtins).
__global__ void psgdk_debug_mfma_kernel(const float* A, const float* B, float* C, int prec) {
  // A: 16 x K row-major, B: K x 16 row-major, C: 16 x 16, K = 32 (bf16) or 4 (fp32); one wave. prec 2: the 32 x 32
  // bf16 shape, A 32 x 16, B 16 x 32, C 32 x 32: lane l holds A[l % 32][8 (l / 32) + e] and B[8 (l / 32) + e][l % 32],
  // and accumulator m of lane l is C[8 (m / 4) + 4 (l / 32) + m % 4][l % 32].
  const int lane = threadIdx.x, r = lane & 15, g = lane >> 4;
  if (prec == 2) {
    const int c = lane & 31, h = lane >> 5;
    bf16x8_t a, b;
    for (int e = 0; e < 8; ++e) {
      a[e] = __builtin_bit_cast(__bf16, f32_to_bf16(A[c * 16 + 8 * h + e]));
      b[e] = __builtin_bit_cast(__bf16, f32_to_bf16(B[(8 * h + e) * 32 + c]));
    }
    f32x16_t acc;
    for (int m = 0; m < 16; ++m) acc[m] = 0.f;
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
    for (int m = 0; m < 16; ++m) C[(8 * (m >> 2) + 4 * h + (m & 3)) * 32 + c] = acc[m];
    return;
  }
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  if (prec == 1) {
    bf16x8_t a, b;
    for (int e = 0; e < 8; ++e) {
      a[e] = __builtin_bit_cast(__bf16, f32_to_bf16(A[r * 32 + g * 8 + e]));
      b[e] = __builtin_bit_cast(__bf16, f32_to_bf16(B[(g * 8 + e) * 16 + r]));
    }
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
  } else {
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(A[r * 4 + g], B[g * 16 + r], acc, 0, 0, 0);
  }
  for (int e = 0; e < 4; ++e) C[(g * 4 + e) * 16 + r] = acc[e];
}

// The bf16 MFMA rate this GPU sustains at the moment of the call: each wave issues `iters` rounds of 32
// independent v_mfma_f32_16x16x32_bf16 (no memory traffic in the loop; operands from the lane index), and lane 0 of
// each wave writes the sum of its accumulators' first element to out[wave id] so that nothing is optimised away.
// 16384 flops per MFMA. One wave per SIMD issuing this instruction stays near 1.4-1.55 PFLOP/s however many
// independent accumulators it cycles through; two waves per SIMD with 32 each reach about 2.36 (measured): launch
// two workgroups per CU.
__global__ void __launch_bounds__(256, 2) psgdk_mfma_rate_kernel(int iters, float* out) {
  const int lane = threadIdx.x & 63;
  bf16x8_t a, b;
  for (int e = 0; e < 8; ++e) {
    a[e] = __builtin_bit_cast(__bf16, f32_to_bf16(1.f + 1e-3f * (lane + e)));
    b[e] = __builtin_bit_cast(__bf16, f32_to_bf16(1.f - 1e-3f * (lane ^ e)));
  }
  f32x4_t acc[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 32; ++i) acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[i], 0, 0, 0);
  }
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) t += acc[i][0];
  if (lane == 0) out[blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)] = t;
}

// ---------------------------------------------------------------------------------------------------------------
// host launchers

template <int PREC, typename TA, typename TB, int BM, int BN, int WM, int WN>
static hipError_t launch_cfg(const GemmArgs& a, hipStream_t st) {
  constexpr int BK = Prec<PREC>::BK, CE = Prec<PREC>::CE, ESZ = Prec<PREC>::ESZ, KP = BK + CE;
  constexpr int smem = 2 * (BM + BN) * KP * ESZ;
  auto fn = gemm_kernel<PREC, TA, TB, BM, BN, WM, WN>;
  // once per instantiation (a function-local static is initialised once, also under concurrent first calls)
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize, smem);
  if (attr != hipSuccess) return attr;
  const int G = a.ntiles * a.nb * a.splitk;
  hipLaunchKernelGGL(fn, dim3(G), dim3(WM * WN * 64), smem, st, a);
  const hipError_t e = hipGetLastError();
  note_launch(reinterpret_cast<const void*>(fn), G, WM * WN * 64, smem);
  return e;
}

template <int PREC, typename TA, typename TB>
static hipError_t launch_prec(GemmArgs& a, int cfg, hipStream_t st) {
  if (cfg == 1) {  // skinny M: 32 x 128 tiles
    a.tiles_m = (a.M + 31) / 32; a.tiles_n = (a.N + 127) / 128;
    a.ntiles = a.tri ? a.tiles_m * (a.tiles_m + 1) / 2 : a.tiles_m * a.tiles_n;
    return launch_cfg<PREC, TA, TB, 32, 128, 1, 4>(a, st);
  }
  a.tiles_m = (a.M + 127) / 128; a.tiles_n = (a.N + 127) / 128;
  a.ntiles = a.tri ? a.tiles_m * (a.tiles_m + 1) / 2 : a.tiles_m * a.tiles_n;
  return launch_cfg<PREC, TA, TB, 128, 128, 2, 2>(a, st);
}

// dtype codes: 0 fp32, 1 bf16
hipError_t gemm_launch(GemmArgs& a, int prec, int adt, int bdt, int cfg, hipStream_t st) {
  if (prec == 1) {
    if (adt == 0 && bdt == 0) return launch_prec<1, float, float>(a, cfg, st);
    if (adt == 0 && bdt == 1) return launch_prec<1, float, bf16_t>(a, cfg, st);
    if (adt == 1 && bdt == 0) return launch_prec<1, bf16_t, float>(a, cfg, st);
    return launch_prec<1, bf16_t, bf16_t>(a, cfg, st);
  }
  if (adt == 0 && bdt == 0) return launch_prec<0, float, float>(a, cfg, st);
  if (adt == 0 && bdt == 1) return launch_prec<0, float, bf16_t>(a, cfg, st);
  if (adt == 1 && bdt == 0) return launch_prec<0, bf16_t, float>(a, cfg, st);
  return launch_prec<0, bf16_t, bf16_t>(a, cfg, st);
}

hipError_t mfma_rate_launch(int iters, int wgs, float* out, hipStream_t st) {
  hipLaunchKernelGGL(psgdk_mfma_rate_kernel, dim3(wgs), dim3(256), 0, st, iters, out);
  return hipGetLastError();
}

hipError_t debug_mfma_launch(const float* A, const float* B, float* C, int prec, hipStream_t st) {
  hipLaunchKernelGGL(psgdk_debug_mfma_kernel, dim3(1), dim3(64), 0, st, A, B, C, prec);
  return hipGetLastError();
}

}  // namespace psgdk

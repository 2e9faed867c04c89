// Elementwise and small reduction kernels of the PSGD-Kron step. All reductions are deterministic: fixed-order
// partial sums, no float atomics.
#include "elem.h"

namespace psgdk {

template <typename T> __device__ __forceinline__ float ld_as_f32(const void* p, long long i) {
  return to_f32<T>(reinterpret_cast<const T*>(p)[i]);
}
__device__ __forceinline__ float ldv(const void* p, int dt, long long i) {
  return dt ? ld_as_f32<bf16_t>(p, i) : ld_as_f32<float>(p, i);
}

constexpr int EW_THREADS = 256;
constexpr int EW_PER_THREAD = 8;

__device__ __forceinline__ void ew_range(long long total, int blocks_per, long long& beg, long long& end) {
  const long long chunk = (total + blocks_per - 1) / blocks_per;
  beg = (long long)(blockIdx.x % blocks_per) * chunk;
  end = beg + chunk < total ? beg + chunk : total;
}

// Eight consecutive elements at a 16-byte aligned address, as floats / from floats.
__device__ __forceinline__ void ew_load8(const bf16_t* src, float (&x)[8]) {
  const uint4 u = *reinterpret_cast<const uint4*>(src);
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    x[2 * e] = __uint_as_float(w[e] << 16);
    x[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
  }
}
__device__ __forceinline__ void ew_load8(const float* src, float (&x)[8]) {
  const float4 p = reinterpret_cast<const float4*>(src)[0], q = reinterpret_cast<const float4*>(src)[1];
  x[0] = p.x; x[1] = p.y; x[2] = p.z; x[3] = p.w; x[4] = q.x; x[5] = q.y; x[6] = q.z; x[7] = q.w;
}
__device__ __forceinline__ void ew_store8(bf16_t* dst, const float (&x)[8]) {
  *reinterpret_cast<uint4*>(dst) = make_uint4(pack2(f32_to_bf16(x[0]), f32_to_bf16(x[1])),
                                              pack2(f32_to_bf16(x[2]), f32_to_bf16(x[3])),
                                              pack2(f32_to_bf16(x[4]), f32_to_bf16(x[5])),
                                              pack2(f32_to_bf16(x[6]), f32_to_bf16(x[7])));
}
__device__ __forceinline__ void ew_store8(float* dst, const float (&x)[8]) {
  reinterpret_cast<float4*>(dst)[0] = make_float4(x[0], x[1], x[2], x[3]);
  reinterpret_cast<float4*>(dst)[1] = make_float4(x[4], x[5], x[6], x[7]);
}

static int ew_blocks(long long total) {
  long long b = (total + (long long)EW_THREADS * EW_PER_THREAD - 1) / ((long long)EW_THREADS * EW_PER_THREAD);
  if (b < 1) b = 1;
  if (b > 4096) b = 4096;
  return (int)b;
}

// ---------------------------------------------------------------------------------------------------------------
// x of the lane that DPP control C names (a move inside a row of 16 lanes; no LDS traffic, unlike a shuffle)
template <int C>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), C, 0xf, 0xf, false));
}
// Sum and max over each row of 16 lanes, every lane getting the row's result: quad_perm(1,0,3,2) and (2,3,0,1) make
// quad results, row_half_mirror combines the two quads of each half, row_mirror the two halves.
__device__ __forceinline__ void row16_sum_max(float& s, float& m) {
  s += dpp<0xB1>(s); m = fmaxf(m, dpp<0xB1>(m));
  s += dpp<0x4E>(s); m = fmaxf(m, dpp<0x4E>(m));
  s += dpp<0x141>(s); m = fmaxf(m, dpp<0x141>(m));
  s += dpp<0x140>(s); m = fmaxf(m, dpp<0x140>(m));
}

// 8 consecutive elements of a bf16 (dt = 1) or fp32 buffer at element offset i (16-byte aligned), as floats
__device__ __forceinline__ void ew_load8_dt(const void* p, int dt, long long i, float (&x)[8]) {
  if (dt) ew_load8(reinterpret_cast<const bf16_t*>(p) + i, x);
  else ew_load8(reinterpret_cast<const float*>(p) + i, x);
}
__device__ __forceinline__ bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// The elementwise kernels take 8 elements per thread and step (16- and 32-byte accesses) when the element count
// is a multiple of 8 and every base is 16-byte aligned; each workgroup owns a contiguous range of 8-element groups.
__device__ __forceinline__ void ew_range8(long long total, int blocks_per, long long& beg, long long& end) {
  ew_range(total >> 3, blocks_per, beg, end);
}

// ---------------------------------------------------------------------------------------------------------------
// Standard normals from a counter-based generator: Philox4x32 with 10 rounds (Salmon, Moraes, Dror and Shaw,
// "Parallel random numbers: as easy as 1, 2, 3", SC 2011), key = the 64-bit seed, counter = (block b of four
// outputs, as two 32-bit words; the 64-bit stream id as two words). A round multiplies words 0 and 2 by the
// published constants 0xD2511F53 and 0xCD9E8D57, keeps the low halves and XORs the high halves with words 1, 3 and
// the key; the key is bumped by the Weyl increments 0x9E3779B9 and 0xBB67AE85 between rounds. Each word x gives
// the uniform u = (floor(x / 256) + 1/2) 2^-24 in (0, 1), exact in fp32 (so ln u keeps its precision next to 1),
// and each pair (u0, u1) two normals by the Box-Muller transform,
// sqrt(-2 ln u0) (cos 2 pi u1, sin 2 pi u1). Output b covers elements 4 b .. 4 b + 3 (fp32, or bf16 rounded from
// the fp32 value).
__device__ __forceinline__ void philox4x32_10(uint32_t (&c)[4], uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    // one 32 x 32 -> 64-bit product per word (one v_mad_u64_u32) rather than separate low and high multiplies
    const uint64_t p0 = (uint64_t)0xD2511F53u * c[0], p1 = (uint64_t)0xCD9E8D57u * c[2];
    const uint32_t lo0 = (uint32_t)p0, hi0 = (uint32_t)(p0 >> 32);
    const uint32_t lo1 = (uint32_t)p1, hi1 = (uint32_t)(p1 >> 32);
    c[0] = hi1 ^ c[1] ^ k0;
    c[1] = lo1;
    c[2] = hi0 ^ c[3] ^ k1;
    c[3] = lo0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
}

// The four normals of output block blk (elements 4 blk .. 4 blk + 3) as normal_fill_kernel computes them, before
// the storage rounding.
__device__ __forceinline__ void philox_normals4(unsigned long long blk, uint32_t k0, uint32_t k1, uint32_t s0,
                                                uint32_t s1, float (&z)[4]) {
  uint32_t c[4] = {(uint32_t)blk, (uint32_t)(blk >> 32), s0, s1};
  philox4x32_10(c, k0, k1);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const float u0 = ((float)(c[2 * h] >> 8) + 0.5f) * 5.9604644775390625e-8f;  // 2^-24
    const float u1 = ((float)(c[2 * h + 1] >> 8) + 0.5f) * 5.9604644775390625e-8f;
    // the hardware transcendentals: v_log_f32 (log2), v_sqrt_f32, and v_sin_f32 / v_cos_f32, which take their
    // argument in revolutions (sin 2 pi u1 directly); -2 ln u0 = -2 ln 2 log2 u0
    const float r = __builtin_amdgcn_sqrtf(-1.3862943611198906f * __builtin_amdgcn_logf(u0));
    z[2 * h] = r * __builtin_amdgcn_cosf(u1);
    z[2 * h + 1] = r * __builtin_amdgcn_sinf(u1);
  }
}
// a normal as stored in dtype dt (0 fp32, 1 bf16) and read back as float, as the noise kernels read a filled buffer
__device__ __forceinline__ float stored_normal(float z, int dt) { return dt ? bf16_to_f32(f32_to_bf16(z)) : z; }
// element j of the drawn sequence, as stored in dtype dt (the block's four normals computed for one of them)
__device__ __forceinline__ float drawn_normal(const EwArgs& a, unsigned long long j, int dt) {
  float z[4];
  philox_normals4(j >> 2, a.dk0, a.dk1, a.ds0, a.ds1, z);
  const int e = (int)(j & 3);
  return stored_normal(e == 0 ? z[0] : e == 1 ? z[1] : e == 2 ? z[2] : z[3], dt);
}

__global__ void __launch_bounds__(EW_THREADS) noise_kernel(const EwArgs a, int blocks_per) {
  const int b = blockIdx.x / blocks_per;
  long long beg, end;
  const void* G = a.in[b];
  const void* N = a.in2[b];  // the noise, in G's dtype
  float* X = a.out[b];
  bf16_t* Xb = reinterpret_cast<bf16_t*>(a.out2[b]);
  const float* rsc = a.in3[b];  // optional row scale (a diagonal P1 folded into the input of P1 X P2)
  const long long total = a.m * a.n;
  const bool drawn = a.draw != 0;
  const unsigned long long doff = drawn ? (unsigned long long)a.doff[b] : 0ull;
  if ((total & 7) == 0 && (a.n & 7) == 0 && al16(G) && (!N || al16(N)) && (!X || al16(X)) && (!Xb || al16(Xb))) {
    ew_range8(total, blocks_per, beg, end);
    for (long long v = beg + threadIdx.x; v < end; v += EW_THREADS) {
      float g[8], nz[8];
      ew_load8_dt(G, a.dt, 8 * v, g);
      if (drawn) {  // elements doff + 8 v .. + 7: two whole blocks (doff is a multiple of 4)
        float z[4];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          philox_normals4((doff >> 2) + 2ull * (unsigned long long)v + q, a.dk0, a.dk1, a.ds0, a.ds1, z);
#pragma unroll
          for (int e = 0; e < 4; ++e) nz[4 * q + e] = stored_normal(z[e], a.dt);
        }
      } else if (N) {
        ew_load8_dt(N, a.dt, 8 * v, nz);
      }
      if (drawn || N) {
#pragma unroll
        for (int e = 0; e < 8; ++e) g[e] = g[e] + (a.f0 + a.f1 * fabsf(g[e])) * nz[e];
      }
      if (rsc) {
        const float r = rsc[(8 * v) / a.n];  // n % 8 == 0: the 8 elements share a row
#pragma unroll
        for (int e = 0; e < 8; ++e) g[e] *= r;
      }
      if (X) ew_store8(X + 8 * v, g);
      if (Xb) ew_store8(Xb + 8 * v, g);
    }
    return;
  }
  ew_range(total, blocks_per, beg, end);
  for (long long i = beg + threadIdx.x; i < end; i += EW_THREADS) {
    const float g = ldv(G, a.dt, i);
    float x = drawn ? g + (a.f0 + a.f1 * fabsf(g)) * drawn_normal(a, doff + (unsigned long long)i, a.dt)
              : N   ? g + (a.f0 + a.f1 * fabsf(g)) * ldv(N, a.dt, i)
                    : g;
    if (rsc) x *= rsc[i / a.n];
    if (X) X[i] = x;
    if (Xb) Xb[i] = f32_to_bf16(x);
  }
}
hipError_t noise_launch(const EwArgs& a, hipStream_t st) {
  const int bp = ew_blocks(a.m * a.n);
  hipLaunchKernelGGL(noise_kernel, dim3(bp * a.nb), dim3(EW_THREADS), 0, st, a, bp);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// out2 = bf16 of (X diag(c))^T (n x m) with X = G + (f0 + f1 |G|) N (N optional) and the column scale c = in3
// (optional): the transposed bf16 operand of P1 (X P2) when P2 is diagonal. 64 x 64 tiles through LDS: row-wise
// reads of G and N, row-wise (along m) writes of the transpose. grid: nb * ceil(m / 64) * ceil(n / 64).
__global__ void __launch_bounds__(256) noise_t_kernel(const EwArgs a) {
  __shared__ float t[64][65];
  const long long m = a.m, n = a.n;
  const int tm = (int)((m + 63) / 64), tn = (int)((n + 63) / 64);
  const int b = blockIdx.x / (tm * tn), tile = blockIdx.x % (tm * tn);
  const int I = tile / tn, J = tile % tn;
  const void* G = a.in[b];
  const void* N = a.in2[b];  // the noise, in G's dtype
  const float* csc = a.in3[b];
  bf16_t* __restrict__ Y = reinterpret_cast<bf16_t*>(a.out2[b]);
  const int tid = threadIdx.x, c = tid & 63, r0 = tid >> 6;
  const long long gj = (long long)J * 64 + c;
  // this thread's 16 rows r0 + 4 q: their G (and a read noise's) values are loaded together, an element outside
  // the matrix reading element 0 and being discarded (loads behind the bounds branch waited for each in turn)
  const bool rd = !a.draw && N;
  float gv[16], nv[16];
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const long long gi = (long long)I * 64 + r0 + 4 * q;
    const long long o = gi < m && gj < n ? gi * n + gj : 0;
    gv[q] = ldv(G, a.dt, o);
    nv[q] = 0.f;
  }
  if (rd) {  // uniform over the launch
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const long long gi = (long long)I * 64 + r0 + 4 * q;
      nv[q] = ldv(N, a.dt, gi < m && gj < n ? gi * n + gj : 0);
    }
  }
  const float cs = csc && gj < n ? csc[gj] : 1.f;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int r = r0 + 4 * q;
    const long long gi = (long long)I * 64 + r;
    float x = 0.f;
    if (gi < m && gj < n) {
      const long long o = gi * n + gj;
      const float g = gv[q];
      x = a.draw ? g + (a.f0 + a.f1 * fabsf(g)) * drawn_normal(a, (unsigned long long)a.doff[b] + o, a.dt)
          : N    ? g + (a.f0 + a.f1 * fabsf(g)) * nv[q]
                 : g;
      if (csc) x *= cs;
    }
    t[r][c] = x;
  }
  __syncthreads();
  const long long oi = (long long)I * 64 + c;  // output column (an input row)
#pragma unroll 4
  for (int r = r0; r < 64; r += 4) {
    const long long oj = (long long)J * 64 + r;  // output row (an input column)
    if (oj < n && oi < m) Y[oj * m + oi] = f32_to_bf16(t[c][r]);
  }
}
hipError_t noise_t_launch(const EwArgs& a, hipStream_t st) {
  const long long tm = (a.m + 63) / 64, tn = (a.n + 63) / 64;
  hipLaunchKernelGGL(noise_t_kernel, dim3((unsigned)(tm * tn * a.nb)), dim3(256), 0, st, a);
  return hipGetLastError();
}

// out[b][i] = sum_j X[i][j]^2 over the rows of a bf16 m x n matrix X = in[b] (one wave per row; 16-byte loads when
// n % 8 == 0 and the base is 16-byte aligned): a diagonal factor's term1 from the bf16 Pg (rows) or Pg^T (columns).
__global__ void __launch_bounds__(256) rowsq_kernel(const EwArgs a) {
  const long long nrb = (a.m + 3) / 4;
  const int b = (int)(blockIdx.x / nrb);
  const long long i = (blockIdx.x % nrb) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (i >= a.m) return;
  const bf16_t* row = reinterpret_cast<const bf16_t*>(a.in[b]) + i * a.n;
  float s = 0.f;
  if ((a.n & 7) == 0 && al16(a.in[b])) {
    for (long long c = lane; c < a.n / 8; c += 64) {
      float x[8];
      ew_load8(row + 8 * c, x);
#pragma unroll
      for (int e = 0; e < 8; ++e) s += x[e] * x[e];
    }
  } else {
    for (long long c = lane; c < a.n; c += 64) {
      const float x = bf16_to_f32(row[c]);
      s += x * x;
    }
  }
  s = wave_sum(s);
  if (lane == 0) a.out[b][i] = s;
}
hipError_t rowsq_launch(const EwArgs& a, hipStream_t st) {
  const long long nrb = (a.m + 3) / 4;
  hipLaunchKernelGGL(rowsq_kernel, dim3((unsigned)(nrb * a.nb)), dim3(256), 0, st, a);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// R[i][j] = sign * (Q[j][i] - Q[i][j]) and R[j][i] = -R[i][j] from one read of each 64 x 64 tile pair (I <= J):
// both tiles are staged in LDS (16-byte loads when rows are 16-byte aligned), each output tile is written
// row-major from there, 4 consecutive columns per thread (16-byte fp32 / 8-byte bf16 stores). Outputs: R fp32
// (out, optional) and R bf16 (out2, optional); with sc[b] set, sc[b][pair] = sum of R_ij Q_ij over the pair's
// elements (fp32 values, a fixed-order block sum; the r2 Procrustes trace). Pairs are numbered p = b np + pair
// (np = T (T + 1) / 2, T = ceil(d / 64)); workgroup w takes p = w, w + G, w + 2 G, ... (G = the grid) and loads
// the next pair's two tiles into registers while it writes the current one, so that every workgroup keeps loads
// in flight through its output phase. grid: min(nb np, RF_GRID).
constexpr int RF_GRID = 1024;  // 4 workgroups (34 KB of LDS each) on each of 256 CUs

__global__ void __launch_bounds__(256) rform_kernel(const EwArgs a) {
  constexpr int TP = 65;        // LDS pitch (floats): column reads of the transposed tile are conflict-free
  __shared__ float qa[64 * TP];  // Q[I block][J block]
  __shared__ float qb[64 * TP];  // Q[J block][I block]
  __shared__ float rsq[2][64], rmx[2][64];  // row statistics of the two tiles, written out as 256-byte runs
  __shared__ float red[16];
  const int d = (int)a.m, T = (d + 63) / 64, np = T * (T + 1) / 2, total = np * a.nb;
  const long long ld = a.ld;
  const float sg = (float)a.i0;
  const int tid = threadIdx.x, c4 = (tid & 15) * 4, r0 = tid >> 4;  // 4 columns, rows r0 + 16 k
  auto decode = [&](int p, int& b, int& I, int& J) {
    b = p / np;
    int t = p % np, i = 0;
    while (t >= T - i) { t -= T - i; ++i; }
    I = i;
    J = i + t;
  };
  float pv[2][4][4];  // the pair's tiles (I, J) and (J, I) as this thread stages them: [tile][k][column]
  auto fetch = [&](int p) {
    int b, I, J;
    decode(p, b, I, J);
    const float* __restrict__ Q = reinterpret_cast<const float*>(a.in[b]);
    const bool vec = (I + 1) * 64 <= d && (J + 1) * 64 <= d && (ld & 3) == 0 &&
                     (reinterpret_cast<uintptr_t>(Q) & 15) == 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int rb = h ? J : I, cb = h ? I : J;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int gi = rb * 64 + r0 + 16 * k, gj = cb * 64 + c4;
        if (vec) {
          const float4 q = *reinterpret_cast<const float4*>(Q + (long long)gi * ld + gj);
          pv[h][k][0] = q.x; pv[h][k][1] = q.y; pv[h][k][2] = q.z; pv[h][k][3] = q.w;
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) pv[h][k][e] = (gi < d && gj + e < d) ? Q[(long long)gi * ld + gj + e] : 0.f;
        }
      }
    }
  };
  if ((int)blockIdx.x < total) fetch(blockIdx.x);
  for (int p = blockIdx.x; p < total; p += gridDim.x) {
    int b, I, J;
    decode(p, b, I, J);
    const int pair = p - b * np;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int e = 0; e < 4; ++e) (h ? qb : qa)[(r0 + 16 * k) * TP + c4 + e] = pv[h][k][e];
    __syncthreads();
    if (p + (int)gridDim.x < total) fetch(p + gridDim.x);
    const float* __restrict__ Q = reinterpret_cast<const float*>(a.in[b]);
    float* __restrict__ R = a.out[b];
    bf16_t* __restrict__ Rb = reinterpret_cast<bf16_t*>(a.out2[b]);
    const bool vec = (I + 1) * 64 <= d && (J + 1) * 64 <= d && (ld & 3) == 0 &&
                     (reinterpret_cast<uintptr_t>(Q) & 15) == 0 && (reinterpret_cast<uintptr_t>(R) & 15) == 0 &&
                     (reinterpret_cast<uintptr_t>(Rb) & 7) == 0;
    // out(rb, cb)[r][c] = sg (src_t[c][r] - src[r][c]): (I, J) from (qb, qa), (J, I) from (qa, qb)
    float tr = 0.f;  // sum of R_ij Q_ij (out-of-range elements are zero in both staged tiles)
    float* __restrict__ st = a.aux[b];
    auto emit = [&](const float* src, const float* srct, int rb, int cb) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int r = r0 + 16 * k, gi = rb * 64 + r, gj = cb * 64 + c4;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = sg * (srct[(c4 + e) * TP + r] - src[r * TP + c4 + e]);
          tr += v[e] * src[r * TP + c4 + e];
        }
        if (st) {  // row statistics of the bf16 R over this tile's 64 columns (the 16 lanes of row r), fixed tree
          float s2 = 0.f, mx = 0.f;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float q = bf16_to_f32(f32_to_bf16(v[e]));
            s2 += q * q;
            mx = fmaxf(mx, fabsf(q));
          }
          row16_sum_max(s2, mx);
          if ((tid & 15) == 0) {
            const int t = rb == I ? 0 : 1;  // tile (I, J) or (J, I)
            rsq[t][r] = s2;
            rmx[t][r] = mx;
          }
        }
        const long long o = (long long)gi * ld + gj;
        if (vec) {
          if (R) *reinterpret_cast<float4*>(R + o) = make_float4(v[0], v[1], v[2], v[3]);
          if (Rb)
            *reinterpret_cast<uint2*>(Rb + o) = make_uint2(pack2(f32_to_bf16(v[0]), f32_to_bf16(v[1])),
                                                          pack2(f32_to_bf16(v[2]), f32_to_bf16(v[3])));
        } else if (gi < d) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (gj + e < d) {
              if (R) R[o + e] = v[e];
              if (Rb) Rb[o + e] = f32_to_bf16(v[e]);
            }
        }
      }
    };
    emit(qa, qb, I, J);
    if (I != J) emit(qb, qa, J, I);
    if (st) {
      __syncthreads();
      const int t = tid >> 6, r = tid & 63;  // threads 0-63: tile (I, J), 64-127: tile (J, I)
      const int rb = t ? J : I, cb = t ? I : J, gi = rb * 64 + r;
      if (t < 2 && (t == 0 || I != J) && gi < d) {
        st[(long long)cb * d + gi] = rsq[t][r];
        st[(long long)(T + cb) * d + gi] = rmx[t][r];
      }
    }
    if (a.sc[b]) {
      tr = block_sum(tr, red);
      if (tid == 0) a.sc[b][pair] = tr;
    }
    __syncthreads();  // the next pair rewrites qa, qb, rsq, rmx and red
  }
}
// rform_kernel for the layout the optimizer uses: d a multiple of 64, 16-byte aligned rows, R in bf16 only, no
// trace partials, row statistics for every matrix or for none (STATS). Every iteration issues the same stores on
// every path, so the wait for the next pair's loads (issued before this pair's stores) leaves the stores in flight:
// with the branches of the general kernel the compiler cannot count them and waits for them too. The same values;
// a diagonal pair writes its tile and statistics twice (the same values to the same places), and the pair fetched
// after a workgroup's last one is clamped to an existing pair and never read.
template <bool STATS>
__global__ void __launch_bounds__(256) rform_fast_kernel(const EwArgs a) {
  constexpr int TP = 65;
  __shared__ float qa[64 * TP];
  __shared__ float qb[64 * TP];
  __shared__ float rsq[2][64], rmx[2][64];
  const int d = (int)a.m, T = d / 64, np = T * (T + 1) / 2, total = np * a.nb;
  const long long ld = a.ld;
  const float sg = (float)a.i0;
  const int tid = threadIdx.x, c4 = (tid & 15) * 4, r0 = tid >> 4;
  auto decode = [&](int p, int& b, int& I, int& J) {
    b = p / np;
    int t = p % np, i = 0;
    while (t >= T - i) { t -= T - i; ++i; }
    I = i;
    J = i + t;
  };
  float pv[2][4][4];
  auto fetch = [&](int p) {
    int b, I, J;
    decode(p, b, I, J);
    const float* __restrict__ Q = reinterpret_cast<const float*>(a.in[b]);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int rb = h ? J : I, cb = h ? I : J;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float4 q = *reinterpret_cast<const float4*>(Q + (long long)(rb * 64 + r0 + 16 * k) * ld + cb * 64 + c4);
        pv[h][k][0] = q.x; pv[h][k][1] = q.y; pv[h][k][2] = q.z; pv[h][k][3] = q.w;
      }
    }
  };
  auto stage = [&]() {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int e = 0; e < 4; ++e) (h ? qb : qa)[(r0 + 16 * k) * TP + c4 + e] = pv[h][k][e];
  };
  fetch(blockIdx.x);
  stage();
  for (int p = blockIdx.x; p < total; p += gridDim.x) {
    int b, I, J;
    decode(p, b, I, J);
    __syncthreads();  // qa, qb hold pair p
    const int pn = p + (int)gridDim.x;
    fetch(pn < total ? pn : total - 1);
    bf16_t* __restrict__ Rb = reinterpret_cast<bf16_t*>(a.out2[b]);
    auto emit = [&](const float* src, const float* srct, int rb, int cb, int t) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int r = r0 + 16 * k;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = sg * (srct[(c4 + e) * TP + r] - src[r * TP + c4 + e]);
        if constexpr (STATS) {
          float s2 = 0.f, mx = 0.f;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float q = bf16_to_f32(f32_to_bf16(v[e]));
            s2 += q * q;
            mx = fmaxf(mx, fabsf(q));
          }
          row16_sum_max(s2, mx);
          if ((tid & 15) == 0) {
            rsq[t][r] = s2;
            rmx[t][r] = mx;
          }
        }
        *reinterpret_cast<uint2*>(Rb + (long long)(rb * 64 + r) * ld + cb * 64 + c4) =
            make_uint2(pack2(f32_to_bf16(v[0]), f32_to_bf16(v[1])), pack2(f32_to_bf16(v[2]), f32_to_bf16(v[3])));
      }
    };
    emit(qa, qb, I, J, 0);
    emit(qb, qa, J, I, 1);  // a diagonal pair (I = J): the same tile and statistics again
    __syncthreads();  // rsq, rmx complete; qa, qb no longer read
    if constexpr (STATS) {
      float* __restrict__ stt = a.aux[b];
      const int t = (tid >> 6) & 1, r = tid & 63;  // waves 2, 3 repeat the stores of waves 0, 1
      const int rb = t ? J : I, cb = t ? I : J, gi = rb * 64 + r;
      stt[(long long)cb * d + gi] = rsq[t][r];
      stt[(long long)(T + cb) * d + gi] = rmx[t][r];
    }
    stage();  // the next pair (its loads were issued before this pair's stores)
  }
}

hipError_t rform_launch(const EwArgs& a, hipStream_t st) {
  const long long T = (a.m + 63) / 64, total = T * (T + 1) / 2 * a.nb;
  if (total > 0x7fffffffLL) return hipErrorInvalidValue;
  const unsigned grid = (unsigned)(total < RF_GRID ? total : RF_GRID);
  bool fast = total > 0 && a.m % 64 == 0 && (a.ld & 3) == 0;
  int stats = -1;
  for (int b = 0; fast && b < a.nb; ++b) {
    fast = a.out[b] == nullptr && a.out2[b] != nullptr && a.sc[b] == nullptr &&
           (reinterpret_cast<uintptr_t>(a.in[b]) & 15) == 0 &&
           (reinterpret_cast<uintptr_t>(a.out2[b]) & 7) == 0;
    const int s_b = a.aux[b] != nullptr;
    if (stats < 0) stats = s_b;
    fast = fast && stats == s_b;
  }
  if (fast && stats) hipLaunchKernelGGL(rform_fast_kernel<true>, dim3(grid), dim3(256), 0, st, a);
  else if (fast) hipLaunchKernelGGL(rform_fast_kernel<false>, dim3(grid), dim3(256), 0, st, a);
  else hipLaunchKernelGGL(rform_kernel, dim3(grid), dim3(256), 0, st, a);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// in2[b] = trace partials (2 per tile, i0 tiles), sc[b][0] = 1 / (bound + smallest normal).
// out[b] = {a, scale}: a = min(-tr(RQ)/tr(RRQ), f0) if tr(RRQ) < 0 else f0.
__global__ void __launch_bounds__(256) proc_scalar_kernel(const EwArgs a) {
  __shared__ float red[16];
  const int b = blockIdx.x;
  const float* part = a.in2[b];
  float t1 = 0.f, t2 = 0.f;
  for (int t = threadIdx.x; t < a.i0; t += blockDim.x) { t1 += part[2 * t]; t2 += part[2 * t + 1]; }
  t1 = block_sum(t1, red);
  t2 = block_sum(t2, red);
  if (threadIdx.x == 0) {
    float step = a.f0;
    if (t2 < 0.f) {
      const float x = -t1 / t2;
      step = x > a.f0 ? a.f0 : x;
    }
    a.out[b][0] = step;
    a.out[b][1] = a.sc[b][0];
    a.out[b][2] = t1;
    a.out[b][3] = t2;
  }
}
hipError_t proc_scalar_launch(const EwArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(proc_scalar_kernel, dim3(a.nb), dim3(256), 0, st, a);
  return hipGetLastError();
}

// Step size of procrustes_step_r2 (psgd_pro_fast.py:141-153) from R = Q^T - Q (unscaled; the reference's
// Rn = Q - Q^T scaled by rs = sc[b][0] = 1 / (bound + smallest normal) is -rs R) and S = Rn^T Rn = rs^2 R R^T
// (already scaled by the SYRK epilogue): in2[b] = the i0 partials of sum R_ij Q_ij, in3[b] = the i1 SYRK trace
// partials (sum S_ij Q_ij at odd slots). tr(RQ) = sum(Rn * Q) = -rs sum(R * Q), tr(RRQ) = -sum(S * Q);
// a = min(-tr(RQ) / tr(RRQ), f0) if tr(RRQ) < 0 else f0. Q - (a Rn + a^2/2 S) Q = Q + M Q with
// M = a rs R - a^2/2 S: out[b] = {a rs, -a^2/2, -1, 0, a, tr(RQ), tr(RRQ)} (slots 2, 3: the coefficients that
// turn the factor-update epilogue X1 - s0 (acc - s1 X1) into X1 + acc). rs^2 is never formed: R = 0 (a
// symmetric Q, bound 0, rs = 1 / smallest normal) gives S = 0, tr = 0, M = 0 and Q unchanged, as in the
// reference, where Rn is scaled before it is squared.
__global__ void __launch_bounds__(256) proc_scalar_r2_kernel(const EwArgs a) {
  __shared__ float red[16];
  const int b = blockIdx.x;
  float t1 = 0.f, t2 = 0.f;
  for (int t = threadIdx.x; t < a.i0; t += blockDim.x) t1 += a.in2[b][t];
  for (int t = threadIdx.x; t < a.i1; t += blockDim.x) t2 += a.in3[b][2 * t + 1];
  t1 = block_sum(t1, red);
  t2 = block_sum(t2, red);
  if (threadIdx.x == 0) {
    const float rs = a.sc[b][0];
    const float trq = -rs * t1, trrq = -t2;
    float step = a.f0;
    if (trrq < 0.f) {
      const float x = -trq / trrq;
      step = x > a.f0 ? a.f0 : x;
    }
    float* o = a.out[b];
    o[0] = step * rs;
    o[1] = -0.5f * step * step;
    o[2] = -1.f;
    o[3] = 0.f;
    o[4] = step;
    o[5] = trq;
    o[6] = trrq;
  }
}
hipError_t proc_scalar_r2_launch(const EwArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(proc_scalar_r2_kernel, dim3(a.nb), dim3(256), 0, st, a);
  return hipGetLastError();
}

// M = c0 R + c1 S over m x n contiguous elements, c = sc[b][0..1]; R = in[b], S = in2 (as `in`'s dtype dt), M =
// out2[b] in the same dtype (bf16 or fp32). 8 elements per thread and step (16-byte access when m n % 8 == 0 and
// the bases are 16-byte aligned).
template <typename T>
__global__ void __launch_bounds__(EW_THREADS) mform_kernel(const EwArgs a, int blocks_per) {
  const int b = blockIdx.x / blocks_per;
  const long long total = a.m * a.n;
  const T* __restrict__ R = reinterpret_cast<const T*>(a.in[b]);
  const T* __restrict__ S = reinterpret_cast<const T*>(a.in2[b]);
  T* __restrict__ M = reinterpret_cast<T*>(a.out2[b]);
  const float c0 = a.sc[b][0], c1 = a.sc[b][1];
  const bool vec = (total & 7) == 0 && ((reinterpret_cast<uintptr_t>(R) | reinterpret_cast<uintptr_t>(S) |
                                         reinterpret_cast<uintptr_t>(M)) & 15) == 0;
  if (vec) {
    const long long nv = total >> 3;
    const long long chunk = (nv + blocks_per - 1) / blocks_per;
    const long long beg = (long long)(blockIdx.x % blocks_per) * chunk, end = min(nv, beg + chunk);
    for (long long i = beg + threadIdx.x; i < end; i += EW_THREADS) {
      float r[8], s[8];
      ew_load8(R + 8 * i, r);
      ew_load8(S + 8 * i, s);
#pragma unroll
      for (int e = 0; e < 8; ++e) r[e] = c0 * r[e] + c1 * s[e];
      ew_store8(M + 8 * i, r);
    }
  } else {
    long long beg, end;
    ew_range(total, blocks_per, beg, end);
    for (long long i = beg + threadIdx.x; i < end; i += EW_THREADS)
      M[i] = from_f32<T>(c0 * to_f32<T>(R[i]) + c1 * to_f32<T>(S[i]));
  }
}
hipError_t mform_launch(const EwArgs& a, hipStream_t st) {
  const int bp = ew_blocks(a.m * a.n / 8 + 1);
  if (a.dt) hipLaunchKernelGGL(mform_kernel<bf16_t>, dim3(bp * a.nb), dim3(EW_THREADS), 0, st, a, bp);
  else hipLaunchKernelGGL(mform_kernel<float>, dim3(bp * a.nb), dim3(EW_THREADS), 0, st, a, bp);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(EW_THREADS) diag_scale_kernel(const EwArgs a, int blocks_per) {
  const int b = blockIdx.x / blocks_per;
  long long beg, end;
  ew_range(a.m * a.n, blocks_per, beg, end);
  const void* X = a.in[b];
  const float* pr = a.in2[b];
  const float* pc = a.in3[b];
  float* Y = a.out[b];
  for (long long i = beg + threadIdx.x; i < end; i += EW_THREADS) {
    const long long r = i / a.n, c = i % a.n;
    float v = ldv(X, a.dt, i);
    if (pr) v *= pr[r];
    if (pc) v *= pc[c];
    Y[i] = v;
  }
}
hipError_t diag_scale_launch(const EwArgs& a, hipStream_t st) {
  const int bp = ew_blocks(a.m * a.n);
  hipLaunchKernelGGL(diag_scale_kernel, dim3(bp * a.nb), dim3(EW_THREADS), 0, st, a, bp);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// rows (i0 = 0): one wave per row; columns (i0 = 1): one thread per column.
__global__ void __launch_bounds__(256) diag_term1_rows_kernel(const EwArgs a, int blocks_per) {
  const int b = blockIdx.x / blocks_per, blk = blockIdx.x % blocks_per;
  const float* X = reinterpret_cast<const float*>(a.in[b]);
  float* out = a.out[b];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (long long r = (long long)blk * 4 + w; r < a.m; r += (long long)blocks_per * 4) {
    float s = 0.f;
    for (long long c = lane; c < a.n; c += 64) { const float v = X[r * a.n + c]; s += v * v; }
    s = wave_sum(s);
    if (lane == 0) out[r] = s;
  }
}
__global__ void __launch_bounds__(256) diag_term1_cols_kernel(const EwArgs a, int blocks_per) {
  const int b = blockIdx.x / blocks_per, blk = blockIdx.x % blocks_per;
  const float* X = reinterpret_cast<const float*>(a.in[b]);
  float* out = a.out[b];
  for (long long c = (long long)blk * 256 + threadIdx.x; c < a.n; c += (long long)blocks_per * 256) {
    float s = 0.f;
    for (long long r = 0; r < a.m; ++r) { const float v = X[r * a.n + c]; s += v * v; }
    out[c] = s;
  }
}
hipError_t diag_term1_launch(const EwArgs& a, hipStream_t st) {
  if (a.i0 == 0) {
    int bp = (int)((a.m + 3) / 4);
    if (bp > 1024) bp = 1024;
    hipLaunchKernelGGL(diag_term1_rows_kernel, dim3(bp * a.nb), dim3(256), 0, st, a, bp);
  } else {
    int bp = (int)((a.n + 255) / 256);
    if (bp > 1024) bp = 1024;
    hipLaunchKernelGGL(diag_term1_cols_kernel, dim3(bp * a.nb), dim3(256), 0, st, a, bp);
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// One workgroup per factor: in2 = term1 (m values), out = q (in place), out2 = P = q * q, sc = L (1 float).
// f0 = lr, f1 = beta, f2 = term2.
__global__ void __launch_bounds__(1024) diag_update_kernel(const EwArgs a) {
  __shared__ float red[16];
  __shared__ float s_c;
  const int b = blockIdx.x;
  const float* t1 = a.in2[b];
  float* q = a.out[b];
  float* P = reinterpret_cast<float*>(a.out2[b]);
  float mx = -INFINITY;
  for (long long i = threadIdx.x; i < a.m; i += blockDim.x) mx = fmaxf(mx, t1[i]);
  mx = block_max(mx, red);
  if (threadIdx.x == 0) {
    const float ell = mx + a.f2;
    float* L = a.sc[b];
    const float Ln = fmaxf(a.f1 * L[0] + (1.f - a.f1) * ell, ell);
    L[0] = Ln;
    s_c = a.f0 / Ln;
  }
  __syncthreads();
  const float c = s_c;
  for (long long i = threadIdx.x; i < a.m; i += blockDim.x) {
    const float v = q[i] * (1.f - c * (t1[i] - a.f2));
    q[i] = v;
    if (P) P[i] = v * v;
  }
}
hipError_t diag_update_launch(const EwArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(diag_update_kernel, dim3(a.nb), dim3(1024), 0, st, a);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// Clamp to [-amp, amp] with torch.clamp's semantics (psgd_pro.py:380): NaN stays NaN (fminf / fmaxf would replace
// it by a bound), +-inf goes to the bound.
__device__ __forceinline__ float clamp_keep_nan(float x, float amp) { return x < -amp ? -amp : (x > amp ? amp : x); }

// pre -> clip -> param update (psgd_pro.py:371-381): RMS from the sum-of-squares partials; rescale by amp / RMS when
// RMS > amp (a NaN RMS does not rescale, an inf RMS rescales by 0, as the reference's comparison and multiply do),
// then the elementwise clamp.
// in = param (dtype dt, m*n), in2 = pre (fp32), in3 = sum-of-squares partials (value at [2 t], i0 partials),
// out2 (optional) = the clipped gradient. f0 = max average amplitude, f1 = max element amplitude, f2 = lr.
__global__ void __launch_bounds__(EW_THREADS) clip_update_kernel(const EwArgs a, int blocks_per) {
  __shared__ float red[16];
  const int b = blockIdx.x / blocks_per;
  const float* part = a.in3[b];
  float s = 0.f;
  for (int t = threadIdx.x; t < a.i0; t += blockDim.x) s += part[2 * t];
  s = block_sum(s, red);
  const long long total = a.m * a.n;
  const float avg = sqrtf(s / (float)total);
  const bool scale = avg > a.f0;
  const float sc = a.f0 / avg;
  long long beg, end;
  const float* pre = a.in2[b];
  void* prm = const_cast<void*>(a.in[b]);
  float* gout = reinterpret_cast<float*>(a.out2[b]);
  if ((total & 7) == 0 && al16(pre) && al16(prm) && (!gout || al16(gout))) {
    ew_range8(total, blocks_per, beg, end);
    for (long long v = beg + threadIdx.x; v < end; v += EW_THREADS) {
      float g[8], w[8];
      ew_load8(pre + 8 * v, g);
      ew_load8_dt(prm, a.dt, 8 * v, w);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (scale) g[e] *= sc;
        g[e] = clamp_keep_nan(g[e], a.f1);
        w[e] = w[e] - a.f2 * g[e];
      }
      if (gout) ew_store8(gout + 8 * v, g);
      if (a.dt) ew_store8(reinterpret_cast<bf16_t*>(prm) + 8 * v, w);
      else ew_store8(reinterpret_cast<float*>(prm) + 8 * v, w);
    }
    return;
  }
  ew_range(total, blocks_per, beg, end);
  for (long long i = beg + threadIdx.x; i < end; i += EW_THREADS) {
    float g = pre[i];
    if (scale) g *= sc;
    g = clamp_keep_nan(g, a.f1);
    if (gout) gout[i] = g;
    if (a.dt) {
      bf16_t* p = reinterpret_cast<bf16_t*>(prm);
      p[i] = f32_to_bf16(bf16_to_f32(p[i]) - a.f2 * g);
    } else {
      float* p = reinterpret_cast<float*>(prm);
      p[i] = p[i] - a.f2 * g;
    }
  }
}
hipError_t clip_update_launch(const EwArgs& a, hipStream_t st) {
  const int bp = ew_blocks(a.m * a.n);
  hipLaunchKernelGGL(clip_update_kernel, dim3(bp * a.nb), dim3(EW_THREADS), 0, st, a, bp);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// out[b][blk] = max |in[b][i]| over the block's range (i0 = blocks per problem).
__global__ void __launch_bounds__(EW_THREADS) absmax_kernel(const EwArgs a, int blocks_per) {
  __shared__ float red[16];
  const int b = blockIdx.x / blocks_per;
  long long beg, end;
  ew_range(a.m * a.n, blocks_per, beg, end);
  const float* x = reinterpret_cast<const float*>(a.in[b]);
  const long long total = a.m * a.n;
  float m = 0.f;
  if ((total & 3) == 0 && al16(x)) {  // 16-byte loads: each workgroup owns a contiguous range of float4s
    ew_range(total >> 2, blocks_per, beg, end);
    const float4* x4 = reinterpret_cast<const float4*>(x);
#pragma unroll 4
    for (long long v = beg + threadIdx.x; v < end; v += EW_THREADS) {
      const float4 q = x4[v];
      m = fmaxf(m, fmaxf(fmaxf(fabsf(q.x), fabsf(q.y)), fmaxf(fabsf(q.z), fabsf(q.w))));
    }
  } else {
    for (long long i = beg + threadIdx.x; i < end; i += EW_THREADS) m = fmaxf(m, fabsf(x[i]));
  }
  m = block_max(m, red);
  if (threadIdx.x == 0) a.out[b][blockIdx.x % blocks_per] = m;
}
hipError_t absmax_launch(const EwArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(absmax_kernel, dim3(a.i0 * a.nb), dim3(EW_THREADS), 0, st, a, a.i0);
  return hipGetLastError();
}

// One workgroup per parameter: in2[b] = partial maxima of its i1 factors (i0 partials each, factor-major);
// out[b][f] = gmean / max|q_f| with gmean = (prod_f max|q_f|)^(1/i1).
__global__ void __launch_bounds__(64) balance_scalar_kernel(const EwArgs a) {
  const int b = blockIdx.x, lane = threadIdx.x;
  const float* part = a.in2[b];
  float norms[8];
  float prod = 1.f;
  for (int f = 0; f < a.i1; ++f) {
    float m = 0.f;
    for (int t = lane; t < a.i0; t += 64) m = fmaxf(m, part[f * a.i0 + t]);
    m = wave_max(m);
    norms[f] = m;
    prod *= m;
  }
  const float g = powf(prod, 1.f / (float)a.i1);
  if (lane == 0)
    for (int f = 0; f < a.i1; ++f) a.out[b][f] = g / norms[f];
}
hipError_t balance_scalar_launch(const EwArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(balance_scalar_kernel, dim3(a.nb), dim3(64), 0, st, a);
  return hipGetLastError();
}

// out[b][i] *= sc[b][i1]
__global__ void __launch_bounds__(EW_THREADS) scale_by_dev_kernel(const EwArgs a, int blocks_per) {
  const int b = blockIdx.x / blocks_per;
  long long beg, end;
  ew_range(a.m * a.n, blocks_per, beg, end);
  const float s = a.sc[b][a.i1];
  float* x = a.out[b];
  for (long long i = beg + threadIdx.x; i < end; i += EW_THREADS) x[i] *= s;
}
hipError_t scale_by_dev_launch(const EwArgs& a, hipStream_t st) {
  const int bp = ew_blocks(a.m * a.n);
  hipLaunchKernelGGL(scale_by_dev_kernel, dim3(bp * a.nb), dim3(EW_THREADS), 0, st, a, bp);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(EW_THREADS) momentum_kernel(const EwArgs a, int blocks_per) {
  const int b = blockIdx.x / blocks_per;
  long long beg, end;
  ew_range(a.m * a.n, blocks_per, beg, end);
  const void* g = a.in[b];
  float* m = a.out[b];
  for (long long i = beg + threadIdx.x; i < end; i += EW_THREADS) m[i] = m[i] * a.f0 + (1.f - a.f0) * ldv(g, a.dt, i);
}
hipError_t momentum_launch(const EwArgs& a, hipStream_t st) {
  const int bp = ew_blocks(a.m * a.n);
  hipLaunchKernelGGL(momentum_kernel, dim3(bp * a.nb), dim3(EW_THREADS), 0, st, a, bp);
  return hipGetLastError();
}

// Each workgroup takes a contiguous slice of the concatenated range in groups of 4 elements (a group never spans two
// tensors: each tensor starts at a multiple of 4); a thread's groups only grow, so the tensor holding them is found by
// walking the offsets forward. 16-byte m and g accesses where every tensor is aligned for them. The arithmetic is
// momentum_kernel's.
__global__ void __launch_bounds__(EW_THREADS) momentum_multi_kernel(const MomList a) {
  const long long total = a.off[a.nb] / 4;
  const long long chunk = (total + gridDim.x - 1) / gridDim.x;
  const long long beg = (long long)blockIdx.x * chunk, end = beg + chunk < total ? beg + chunk : total;
  int t = 0;
  for (long long q = beg + threadIdx.x; q < end; q += EW_THREADS) {
    const long long e = 4 * q;
    while (e >= a.off[t + 1]) ++t;
    const long long j = e - a.off[t], n = a.n[t];
    if (j >= n) continue;  // the padding of tensor t
    float* m = a.m[t];
    if (a.vec && j + 4 <= n) {
      float4 mv = *reinterpret_cast<const float4*>(m + j);
      float gv[4];
      if (a.dt[t]) {
        const uint2 h = *reinterpret_cast<const uint2*>(reinterpret_cast<const bf16_t*>(a.g[t]) + j);
        gv[0] = bf16_to_f32((bf16_t)(h.x & 0xffff)); gv[1] = bf16_to_f32((bf16_t)(h.x >> 16));
        gv[2] = bf16_to_f32((bf16_t)(h.y & 0xffff)); gv[3] = bf16_to_f32((bf16_t)(h.y >> 16));
      } else {
        const float4 f = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(a.g[t]) + j);
        gv[0] = f.x; gv[1] = f.y; gv[2] = f.z; gv[3] = f.w;
      }
      mv.x = mv.x * a.beta + (1.f - a.beta) * gv[0];
      mv.y = mv.y * a.beta + (1.f - a.beta) * gv[1];
      mv.z = mv.z * a.beta + (1.f - a.beta) * gv[2];
      mv.w = mv.w * a.beta + (1.f - a.beta) * gv[3];
      *reinterpret_cast<float4*>(m + j) = mv;
    } else {
      for (long long i = j; i < j + 4 && i < n; ++i) m[i] = m[i] * a.beta + (1.f - a.beta) * ldv(a.g[t], a.dt[t], i);
    }
  }
}
hipError_t momentum_multi_launch(const MomList& a, hipStream_t st) {
  const long long total = a.off[a.nb] / 4;  // groups of 4 elements
  const long long want = (total + EW_THREADS * 4 - 1) / (EW_THREADS * 4);
  const int blocks = (int)(want < 1 ? 1 : want > 1024 ? 1024 : want);
  hipLaunchKernelGGL(momentum_multi_kernel, dim3(blocks), dim3(EW_THREADS), 0, st, a);
  return hipGetLastError();
}

__global__ void __launch_bounds__(EW_THREADS) normal_fill_kernel(void* out, long long n, int dt, uint32_t k0,
                                                                   uint32_t k1, uint32_t s0, uint32_t s1) {
  const long long nblk = (n + 3) / 4;
  for (long long blk = (long long)blockIdx.x * EW_THREADS + threadIdx.x; blk < nblk;
       blk += (long long)gridDim.x * EW_THREADS) {
    float z[4];
    philox_normals4((unsigned long long)blk, k0, k1, s0, s1, z);
    const long long i0 = 4 * blk;
    if (dt == 1) {  // bf16 storage (dtype codes: 0 fp32, 1 bf16)
      bf16_t* o = reinterpret_cast<bf16_t*>(out) + i0;
      if (i0 + 4 <= n) {
        *reinterpret_cast<uint2*>(o) = make_uint2(pack2(f32_to_bf16(z[0]), f32_to_bf16(z[1])),
                                                  pack2(f32_to_bf16(z[2]), f32_to_bf16(z[3])));
      } else {
        for (int e = 0; i0 + e < n; ++e) o[e] = f32_to_bf16(z[e]);
      }
    } else {
      float* o = reinterpret_cast<float*>(out) + i0;
      if (i0 + 4 <= n) *reinterpret_cast<float4*>(o) = make_float4(z[0], z[1], z[2], z[3]);
      else
        for (int e = 0; i0 + e < n; ++e) o[e] = z[e];
    }
  }
}
hipError_t normal_fill_launch(void* out, long long n, int dt, unsigned long long seed, unsigned long long stream_id,
                              hipStream_t st) {
  const long long nblk = (n + 3) / 4;
  const long long want = (nblk + EW_THREADS * 4 - 1) / (EW_THREADS * 4);
  const int blocks = (int)(want < 1 ? 1 : want > 4096 ? 4096 : want);
  hipLaunchKernelGGL(normal_fill_kernel, dim3(blocks), dim3(EW_THREADS), 0, st, out, n, dt, (uint32_t)seed,
                     (uint32_t)(seed >> 32), (uint32_t)stream_id, (uint32_t)(stream_id >> 32));
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(EW_THREADS) splitk_sum_kernel(const EwArgs a, int blocks_per) {
  const int b = blockIdx.x / blocks_per;
  long long beg, end;
  const long long mn = a.m * a.n;
  ew_range(mn, blocks_per, beg, end);
  const float* in = a.in2[b];
  float* out = a.out[b];
  for (long long i = beg + threadIdx.x; i < end; i += EW_THREADS) {
    float s = 0.f;
    for (int k = 0; k < a.i0; ++k) s += in[(long long)k * mn + i];
    out[i] = s;
  }
}
hipError_t splitk_sum_launch(const EwArgs& a, hipStream_t st) {
  const int bp = ew_blocks(a.m * a.n);
  hipLaunchKernelGGL(splitk_sum_kernel, dim3(bp * a.nb), dim3(EW_THREADS), 0, st, a, bp);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// out[b][2 blk] = sum of squares over the block's range, out[b][2 blk + 1] = 0 (i0 = blocks per problem).
__global__ void __launch_bounds__(EW_THREADS) sumsq_kernel(const EwArgs a, int blocks_per) {
  __shared__ float red[16];
  const int b = blockIdx.x / blocks_per;
  long long beg, end;
  ew_range(a.m * a.n, blocks_per, beg, end);
  const float* x = reinterpret_cast<const float*>(a.in[b]);
  float s = 0.f;
  for (long long i = beg + threadIdx.x; i < end; i += EW_THREADS) s += x[i] * x[i];
  s = block_sum(s, red);
  if (threadIdx.x == 0) {
    a.out[b][2 * (blockIdx.x % blocks_per)] = s;
    a.out[b][2 * (blockIdx.x % blocks_per) + 1] = 0.f;
  }
}
hipError_t sumsq_launch(const EwArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(sumsq_kernel, dim3(a.i0 * a.nb), dim3(EW_THREADS), 0, st, a, a.i0);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// Full symmetric n x n (ld) from the row-major packed upper triangle.
__global__ void __launch_bounds__(EW_THREADS) unpack_kernel(const EwArgs a, int blocks_per) {
  const int b = blockIdx.x / blocks_per;
  long long beg, end;
  const long long n = a.n;
  ew_range(n * n, blocks_per, beg, end);
  const float* pk = a.in2[b];
  float* C = a.out[b];
  for (long long i = beg + threadIdx.x; i < end; i += EW_THREADS) {
    const long long r = i / n, c = i % n;
    const long long lo = r < c ? r : c, hi = r < c ? c : r;
    C[r * a.ld + c] = pk[lo * n - lo * (lo - 1) / 2 + (hi - lo)];
  }
}
hipError_t unpack_launch(const EwArgs& a, hipStream_t st) {
  const int bp = ew_blocks(a.n * a.n);
  hipLaunchKernelGGL(unpack_kernel, dim3(bp * a.nb), dim3(EW_THREADS), 0, st, a, bp);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// out2[b] (bf16, m x n row-major, leading dimension n) = bf16(in[b]) (i0 = 0) or bf16(in[b]^T) (i0 = 1, in is
// n x m with leading dimension a.ld); with out[b] set, the same copy in fp32 into out[b] instead. 64 x 64 tiles
// through LDS. grid: tiles * nb.
__global__ void __launch_bounds__(256) to_bf16_kernel(const EwArgs a) {
  __shared__ float t[64][65];
  const int TM = (int)((a.m + 63) / 64), TN = (int)((a.n + 63) / 64);
  const int b = blockIdx.x / (TM * TN), tile = blockIdx.x % (TM * TN);
  const int I = tile / TN, J = tile % TN;  // output tile (rows I, cols J)
  const void* __restrict__ X = a.in[b];
  auto xat = [&](long long idx) {
    return a.dt ? bf16_to_f32(reinterpret_cast<const bf16_t*>(X)[idx]) : reinterpret_cast<const float*>(X)[idx];
  };
  bf16_t* __restrict__ Y = reinterpret_cast<bf16_t*>(a.out2[b]);
  float* __restrict__ Yf = a.out[b];
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  if (a.i0 == 0) {
    for (int r = ty; r < 64; r += 4) {
      const long long gi = (long long)I * 64 + r, gj = (long long)J * 64 + tx;
      if (gi < a.m && gj < a.n) {
        const float v = a.i1 && gj < gi ? 0.f : xat(gi * a.ld + gj);  // i1: the strict lower part is not read
        if (Yf) Yf[gi * a.n + gj] = v;
        else Y[gi * a.n + gj] = f32_to_bf16(v);
      }
    }
    return;
  }
  // transposed: output (gi, gj) = in (gj, gi); load in rows J-block, cols I-block
  for (int r = ty; r < 64; r += 4) {
    const long long si = (long long)J * 64 + r, sj = (long long)I * 64 + tx;
    t[r][tx] = (si < a.n && sj < a.m) ? xat(si * a.ld + sj) : 0.f;
  }
  __syncthreads();
  for (int r = ty; r < 64; r += 4) {
    const long long gi = (long long)I * 64 + r, gj = (long long)J * 64 + tx;
    if (gi < a.m && gj < a.n) {
      if (Yf) Yf[gi * a.n + gj] = t[tx][r];
      else Y[gi * a.n + gj] = f32_to_bf16(t[tx][r]);
    }
  }
}
hipError_t to_bf16_launch(const EwArgs& a, hipStream_t st) {
  const int TM = (int)((a.m + 63) / 64), TN = (int)((a.n + 63) / 64);
  hipLaunchKernelGGL(to_bf16_kernel, dim3(TM * TN * a.nb), dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace psgdk

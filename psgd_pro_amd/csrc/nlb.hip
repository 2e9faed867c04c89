// Norm lower bounds of symmetric (SPD) and skew-symmetric matrices read from their upper triangle.
//
// nlb(A, V) = nf * max_r || V4_r || with nf = max diag(A) (SPD) or max |A_ij| (skew) plus the smallest normal,
// V0 = a_j + sgn(<a_j, V_r>) V_r (a_j = row j of A/nf, j = the largest row), V1 = V0 A/nf, V2 = (V1/|V1|) A/nf,
// V3 = V2 A/nf, V4 = (V3/|V3|) A/nf. Stages (each a grouped launch over up to MAXB matrices):
//   tri_rownorm : one pass over the stored upper triangle in 64x64 tiles: per-tile row and column sums of squares
//                 (deterministic partial slots, no float atomics), per-tile max |A_ij| and max diagonal
//   nlb_init    : one workgroup per matrix: squared row norms, argmax (first maximum), nf, V0
//   V A products: the GEMM engine (M = 32, B read from the triangle), split over k, partials in ws
//   nlb_reduce  : sums the k-split partials in a fixed order, scales the rows by 1/nf and by the input row
//                 normalisation 1/(|V_in,r| + smallest normal) (exact: the product is linear in each row of V),
//                 and writes per-(row, column block) sums of squares of the result
//   nlb_final   : nf * max_r |V4_r| and the consumer's scalars (L EMA and lr/L, or the Procrustes scale)
#include "nlb.h"

namespace psgdk {

constexpr int RT = 64;  // row-norm tile side

// grid: nb * T(T+1)/2 workgroups of 256 threads; T = ceil(n / 64).
// rpart[b][(X * T + Y) * 64 + i] = contribution to squared row norm 64 X + i from the stored tile pair {X, Y}.
// tmax[b][t] = max |A_ij| over stored tile t, dmax[b][t] = max diagonal element over tile t (-inf if none).
__global__ void __launch_bounds__(256) tri_rownorm_kernel(const NlbArgs p) {
  __shared__ float sq[RT][RT + 1];
  __shared__ float red[16];
  const int T = p.T, ntri = T * (T + 1) / 2;
  const int b = blockIdx.x / ntri, t = blockIdx.x % ntri;
  int I = 0, rem = t, rowlen = T;
  while (rem >= rowlen) { rem -= rowlen; ++I; --rowlen; }
  const int J = I + rem;
  const float* __restrict__ A = p.A[b];
  const long long ld = p.lda;
  const int n = p.n, tid = threadIdx.x;
  const int lr = tid >> 2, lc0 = (tid & 3) * 16;
  const int gi = I * RT + lr;
  float rs = 0.f, am = 0.f, dm = -INFINITY;
  // the 16 loads go out together: each reads a valid address (element 0 in place of one outside the stored
  // triangle) and the value is selected afterwards (a load behind a per-element branch waited for each in turn)
  float a16[16];
#pragma unroll
  for (int c = 0; c < 16; ++c) {
    const int gj = J * RT + lc0 + c;
    const bool ok = gi < n && gj < n && gi <= gj;
    a16[c] = A[ok ? (long long)gi * ld + gj : 0];
  }
#pragma unroll
  for (int c = 0; c < 16; ++c) {
    const int gj = J * RT + lc0 + c;
    const float v0 = a16[c];
    float v = gi < n && gj < n && gi <= gj ? v0 : 0.f;
    if (gi == gj && gi < n) {
      dm = fmaxf(dm, v);
      if (p.sign < 0) v = 0.f;  // skew: the diagonal is zero by definition
    }
    const float s = v * v;
    sq[lr][lc0 + c] = (gi < gj) ? s : 0.f;  // strictly-upper elements also count for the column's row norm
    rs += s;
    am = fmaxf(am, fabsf(v));
  }
  rs += __shfl_xor(rs, 1, 64);
  rs += __shfl_xor(rs, 2, 64);
  float* __restrict__ rp = p.rpart[b];
  if ((tid & 3) == 0) rp[((long long)I * T + J) * RT + lr] = rs;
  __syncthreads();
  if (I != J && tid < RT) {
    float cs = 0.f;
    for (int i = 0; i < RT; ++i) cs += sq[i][tid];
    rp[((long long)J * T + I) * RT + tid] = cs;
  } else if (I == J && tid < RT) {
    float cs = 0.f;
    for (int i = 0; i < RT; ++i) cs += sq[i][tid];
    p.cpart[b][(long long)I * RT + tid] = cs;  // diagonal tile: its column sums get a slot of their own
  }
  am = block_max(am, red);
  dm = block_max(dm, red);
  if (tid == 0) {
    p.tmax[b][t] = am;
    p.dmax[b][t] = dm;
  }
}

// One workgroup (1024 threads) per matrix.
__global__ void __launch_bounds__(1024) nlb_init_kernel(const NlbArgs p) {
  __shared__ float red[16];
  __shared__ float sval[16];
  __shared__ int sidx[16];
  __shared__ float snf;
  __shared__ int sj;
  const int b = blockIdx.x, tid = threadIdx.x, nt = blockDim.x;
  const int n = p.n, T = p.T, ntri = T * (T + 1) / 2;
  const float* __restrict__ A = p.A[b];
  const long long ld = p.lda;
  const float* __restrict__ rp = p.rpart[b];
  const float* __restrict__ cp = p.cpart[b];
  float* __restrict__ rn2 = p.rn2[b];
  // squared row norms (fixed summation order over the partner blocks) and their argmax (first maximum)
  float best = -1.f;
  int bi = 0x7fffffff;
  for (int i = tid; i < n; i += nt) {
    const int X = i / RT, li = i % RT;
    float s = 0.f;
    for (int Y = 0; Y < T; ++Y) s += rp[((long long)X * T + Y) * RT + li];
    s += cp[(long long)X * RT + li];
    rn2[i] = s;
    if (s > best) { best = s; bi = i; }  // i increases: first maximum per thread
  }
  // block argmax: max value, then smallest index among equals
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (ov > best || (ov == best && oi < bi)) { best = ov; bi = oi; }
  }
  if ((tid & 63) == 0) { sval[tid >> 6] = best; sidx[tid >> 6] = bi; }
  float am = 0.f, dm = -INFINITY;
  for (int t = tid; t < ntri; t += nt) { am = fmaxf(am, p.tmax[b][t]); dm = fmaxf(dm, p.dmax[b][t]); }
  __syncthreads();
  if (tid == 0) {
    float bv = sval[0];
    int bj = sidx[0];
    for (int w = 1; w < nt / 64; ++w)
      if (sval[w] > bv || (sval[w] == bv && sidx[w] < bj)) { bv = sval[w]; bj = sidx[w]; }
    sj = bj < n ? bj : 0;
  }
  am = block_max(am, red);
  dm = block_max(dm, red);
  if (tid == 0) {
    const float nf = (p.sign > 0 ? dm : am) + kSmallestNormal;
    snf = nf;
    p.scal[b][NLB_NF] = nf;
    p.scal[b][NLB_J] = (float)sj;
    if (p.amax_out[b]) p.amax_out[b][0] = am;
  }
  __syncthreads();
  if (p.Vin[b] == nullptr) return;  // row norms only
  const int j = sj;
  // a_j[k] = A_sym[j][k] / nf from the triangle; V0[r] = a_j + sgn(<a_j, V_r>) V_r
  const float* __restrict__ Vin = p.Vin[b];
  float* __restrict__ V0 = p.Vout[b];
  auto aj = [&](int k) -> float {
    float v;
    if (k > j) v = A[(long long)j * ld + k];
    else if (k < j) v = (float)p.sign * A[(long long)k * ld + j];
    else v = p.sign < 0 ? 0.f : A[(long long)j * ld + j];
    return v / snf;
  };
  const int wave = tid >> 6, lane = tid & 63, nw = nt >> 6;
  for (int r = wave; r < NLB_K; r += nw) {
    float d = 0.f;
    for (int k = lane; k < n; k += 64) d += aj(k) * Vin[(long long)r * n + k];
    d = wave_sum(d);
    const float sg = d > 0.f ? 1.f : (d < 0.f ? -1.f : 0.f);
    for (int k = lane; k < n; k += 64) V0[(long long)r * n + k] = aj(k) + sg * Vin[(long long)r * n + k];
  }
}

// grid: nb * ceil(n / 64) workgroups of 256 threads (4 waves x 8 rows, 64 columns).
// out[r][c] = rowscale_r / nf * sum_s part[s][r][c]; ss[r][cb] = sum over the block's 64 columns of out^2.
__global__ void __launch_bounds__(256) nlb_reduce_kernel(const NlbArgs p, int normalize_in) {
  const int nbk = (p.n + 63) / 64;
  const int b = blockIdx.x / nbk, cb = blockIdx.x % nbk;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = p.n, c = cb * 64 + lane;
  const float nf = p.scal[b][NLB_NF];
  const float* __restrict__ part = p.part[b];
  const float* __restrict__ ssin = p.ssin[b];
  float* __restrict__ out = p.Vout[b];
  float* __restrict__ ss = p.ssout[b];
  for (int rr = 0; rr < 8; ++rr) {
    const int r = wave * 8 + rr;
    float sc = 1.f / nf;
    if (normalize_in) {
      float s = 0.f;
      for (int q = 0; q < nbk; ++q) s += ssin[r * nbk + q];
      sc = sc / (sqrtf(s) + kSmallestNormal);
    }
    float v = 0.f;
    if (c < n) {
      float acc = 0.f;
      for (int s = 0; s < p.splits; ++s) acc += part[((long long)s * NLB_K + r) * n + c];
      v = acc * sc;
      out[(long long)r * n + c] = v;
    }
    const float t = wave_sum(v * v);
    if (lane == 0) ss[r * nbk + cb] = t;
  }
}

// One workgroup (64 threads) per matrix: bound = nf * max_r |V4_r|, then the consumer's scalars.
__global__ void __launch_bounds__(64) nlb_final_kernel(const NlbArgs p, NlbFinal f) {
  const int b = blockIdx.x, lane = threadIdx.x;
  const int nbk = (p.n + p.ssc - 1) / p.ssc;
  const float* __restrict__ ss = p.ssin[b];
  float m = 0.f;
  if (lane < NLB_K) {
    float s = 0.f;
    for (int q = 0; q < nbk; ++q) s += ss[lane * nbk + q];
    m = sqrtf(s);
  }
  m = wave_max(m);
  if (lane == 0) {
    const float nf = p.scal[b][NLB_NF];
    const float bound = nf * m;
    p.scal[b][NLB_BOUND] = bound;
    if (f.mode == NLB_FINAL_FACTOR) {
      // psgd_pro.py:132-135: ell = bound + term2; L = max(beta L + (1 - beta) ell, ell); coef = lr / L, term2
      const float ell = bound + f.term2[b];
      float* L = f.L[b];
      const float Ln = fmaxf(f.beta * L[0] + (1.f - f.beta) * ell, ell);
      L[0] = Ln;
      f.coef[b][0] = f.lr / Ln;
      f.coef[b][1] = f.term2[b];
    } else if (f.mode == NLB_FINAL_SCALE) {
      // psgd_pro.py:88: R / (bound + smallest normal)
      f.coef[b][0] = 1.f / (bound + kSmallestNormal);
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------

hipError_t nlb_rownorm_launch(const NlbArgs& a, hipStream_t st) {
  const int ntri = a.T * (a.T + 1) / 2;
  hipLaunchKernelGGL(tri_rownorm_kernel, dim3(ntri * a.nb), dim3(256), 0, st, a);
  return hipGetLastError();
}
hipError_t nlb_init_launch(const NlbArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(nlb_init_kernel, dim3(a.nb), dim3(1024), 0, st, a);
  return hipGetLastError();
}
hipError_t nlb_reduce_launch(const NlbArgs& a, int normalize_in, hipStream_t st) {
  const int nbk = (a.n + 63) / 64;
  hipLaunchKernelGGL(nlb_reduce_kernel, dim3(nbk * a.nb), dim3(256), 0, st, a, normalize_in);
  return hipGetLastError();
}
hipError_t nlb_final_launch(const NlbArgs& a, const NlbFinal& f, hipStream_t st) {
  hipLaunchKernelGGL(nlb_final_kernel, dim3(a.nb), dim3(64), 0, st, a, f);
  return hipGetLastError();
}


// ================================================================================================================
// Norm lower bounds of fully stored matrices (fp32 or bf16 storage): row-parallel row norms, an init kernel that
// reads them directly, and split-K V A products whose partials a second kernel sums in a fixed order (the
// input-row normalisation and 1/nf are folded into that epilogue, which also writes the sums of squares the next
// product normalises with).

// Row statistics of a fully stored matrix, one wave per row: rn2[i] = sum_j A_ij^2, rpart[i] = max_j |A_ij|,
// cpart[i] = A_ii (skew: the diagonal counts as zero, psgd_pro.py:50 takes max |A| of a matrix whose diagonal is
// zero). Rows are read in 16-byte chunks when every row start is 16-byte aligned.
template <typename T>
__global__ void __launch_bounds__(256) rownorm_full_kernel(const NlbArgs p) {
  constexpr int ACH = 16 / sizeof(T);
  const int nrb = (p.n + 3) / 4;
  const int b = blockIdx.x / nrb, rb = blockIdx.x % nrb;
  const int lane = threadIdx.x & 63, i = rb * 4 + (threadIdx.x >> 6);
  if (i >= p.n) return;
  const int n = p.n;
  const T* __restrict__ A = reinterpret_cast<const T*>(p.A[b]);
  const T* __restrict__ row = A + (long long)i * p.lda;
  const bool va = (p.lda % ACH) == 0 && (reinterpret_cast<uintptr_t>(A) & 15) == 0;
  float s = 0.f, m = 0.f;
  int j0 = 0;
  if (va) {
    const int nv = n / ACH;
    for (int c = lane; c < nv; c += 64) {
      const uint4 u = reinterpret_cast<const uint4*>(row)[c];
      const T* t = reinterpret_cast<const T*>(&u);
#pragma unroll
      for (int e = 0; e < ACH; ++e) {
        float v = to_f32<T>(t[e]);
        if (p.sign < 0 && c * ACH + e == i) v = 0.f;
        s += v * v;
        m = fmaxf(m, fabsf(v));
      }
    }
    j0 = nv * ACH;
  }
  for (int j = j0 + lane; j < n; j += 64) {
    float v = to_f32<T>(row[j]);
    if (p.sign < 0 && j == i) v = 0.f;
    s += v * v;
    m = fmaxf(m, fabsf(v));
  }
  s = wave_sum(s);
  m = wave_max(m);
  if (lane == 0) {
    p.rn2[b][i] = s;
    p.rpart[b][i] = m;
    p.cpart[b][i] = to_f32<T>(row[i]);
  }
}

// The same row statistics from per-(row, 64-column block) partials in part[b] that the producer of a skew matrix
// left (rform: sums of squares at part[cb n + i], then maxima of |.| at part[(T + cb) n + i]). 64 rows per
// workgroup, four threads per row over quarters of the blocks, combined through LDS in quarter order. The diagonal
// of R = +-(Q^T - Q) is zero. grid: nb * ceil(n / 64).
__global__ void __launch_bounds__(256) rowstats_reduce_kernel(const NlbArgs p) {
  __shared__ float ps[4][64], pm[4][64];
  const int n = p.n, T = (n + 63) / 64, nrb = (n + 63) / 64;
  const int b = blockIdx.x / nrb, r = threadIdx.x & 63, q = threadIdx.x >> 6;
  const int i = (blockIdx.x % nrb) * 64 + r;
  const float* __restrict__ S = p.part[b];
  const int c0 = q * T / 4, c1 = (q + 1) * T / 4;
  float s = 0.f, m = 0.f;
  if (i < n) {
#pragma unroll 4
    for (int c = c0; c < c1; ++c) {
      s += S[(long long)c * n + i];
      m = fmaxf(m, S[(long long)(T + c) * n + i]);
    }
  }
  ps[q][r] = s;
  pm[q][r] = m;
  __syncthreads();
  if (q == 0 && i < n) {
    p.rn2[b][i] = ((ps[0][r] + ps[1][r]) + ps[2][r]) + ps[3][r];
    p.rpart[b][i] = fmaxf(fmaxf(pm[0][r], pm[1][r]), fmaxf(pm[2][r], pm[3][r]));
    p.cpart[b][i] = 0.f;
  }
}

// Eight consecutive elements of T at a 16-byte aligned address, as floats.
__device__ __forceinline__ void load8(const bf16_t* src, float (&x)[8]) {
  const uint4 u = *reinterpret_cast<const uint4*>(src);
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    x[2 * e] = __uint_as_float(w[e] << 16);
    x[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
  }
}
__device__ __forceinline__ void load8(const float* src, float (&x)[8]) {
  const float4 a = reinterpret_cast<const float4*>(src)[0], c = reinterpret_cast<const float4*>(src)[1];
  x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = c.x; x[5] = c.y; x[6] = c.z; x[7] = c.w;
}
__device__ __forceinline__ void store8(bf16_t* dst, const float (&x)[8]) {
  uint4 u;
  u.x = pack2(f32_to_bf16(x[0]), f32_to_bf16(x[1]));
  u.y = pack2(f32_to_bf16(x[2]), f32_to_bf16(x[3]));
  u.z = pack2(f32_to_bf16(x[4]), f32_to_bf16(x[5]));
  u.w = pack2(f32_to_bf16(x[6]), f32_to_bf16(x[7]));
  *reinterpret_cast<uint4*>(dst) = u;
}
__device__ __forceinline__ void store8(float* dst, const float (&x)[8]) {
  reinterpret_cast<float4*>(dst)[0] = make_float4(x[0], x[1], x[2], x[3]);
  reinterpret_cast<float4*>(dst)[1] = make_float4(x[4], x[5], x[6], x[7]);
}
__device__ __forceinline__ void store4(bf16_t* dst, const float (&x)[4]) {
  *reinterpret_cast<uint2*>(dst) = make_uint2(pack2(f32_to_bf16(x[0]), f32_to_bf16(x[1])),
                                              pack2(f32_to_bf16(x[2]), f32_to_bf16(x[3])));
}
__device__ __forceinline__ void store4(float* dst, const float (&x)[4]) {
  *reinterpret_cast<float4*>(dst) = make_float4(x[0], x[1], x[2], x[3]);
}

// One workgroup per (matrix, row r of V): argmax of rn2 (first maximum), nf = max diagonal (SPD) or max |A|
// (skew) + smallest normal, then V0[r] = a_j + sgn(<a_j, V_r>) V_r with a_j = row j of A / nf (psgd_pro.py:25-33,
// :49-57). Workgroup r = 0 also publishes nf and j. The scans read 4 (statistics) or 8 (rows) elements per thread
// and step with the loads of several steps in flight; the rows take the element path unless n % 8 == 0, A's row
// stride is a multiple of 16 bytes and the bases are 16-byte aligned.
template <typename T>
__global__ void __launch_bounds__(256) nlb_init_full_kernel(const NlbArgs p) {
  __shared__ float red[4];
  __shared__ float sval[4];
  __shared__ int sidx[4];
  __shared__ float snf;
  __shared__ int sj;
  const int b = blockIdx.x / NLB_K, r = blockIdx.x % NLB_K;
  const int tid = threadIdx.x, n = p.n;
  const float* __restrict__ rn2 = p.rn2[b];
  const float* __restrict__ rmax = p.rpart[b];
  const float* __restrict__ diag = p.cpart[b];
  float best = -1.f, am = 0.f, dm = -INFINITY;
  int bi = 0x7fffffff;
  if ((n & 3) == 0) {  // workspace arrays: 256-byte aligned bases
    const int n4 = n >> 2;
#pragma unroll 4
    for (int i = tid; i < n4; i += 256) {
      const float4 s = reinterpret_cast<const float4*>(rn2)[i];
      const float4 a = reinterpret_cast<const float4*>(rmax)[i];
      const float4 c = reinterpret_cast<const float4*>(diag)[i];
      const float sv[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (sv[e] > best) { best = sv[e]; bi = 4 * i + e; }  // indices increase: first maximum per thread
      am = fmaxf(am, fmaxf(fmaxf(a.x, a.y), fmaxf(a.z, a.w)));
      dm = fmaxf(dm, fmaxf(fmaxf(c.x, c.y), fmaxf(c.z, c.w)));
    }
  } else {
    for (int i = tid; i < n; i += 256) {
      const float s = rn2[i];
      if (s > best) { best = s; bi = i; }
      am = fmaxf(am, rmax[i]);
      dm = fmaxf(dm, diag[i]);
    }
  }
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (ov > best || (ov == best && oi < bi)) { best = ov; bi = oi; }
  }
  if ((tid & 63) == 0) { sval[tid >> 6] = best; sidx[tid >> 6] = bi; }
  am = block_max(am, red);
  dm = block_max(dm, red);
  if (tid == 0) {
    float bv = sval[0];
    int bj = sidx[0];
    for (int w = 1; w < 4; ++w)
      if (sval[w] > bv || (sval[w] == bv && sidx[w] < bj)) { bv = sval[w]; bj = sidx[w]; }
    sj = bj < n ? bj : 0;
    const float nf = (p.sign > 0 ? dm : am) + kSmallestNormal;
    snf = nf;
    if (r == 0) {
      p.scal[b][NLB_NF] = nf;
      p.scal[b][NLB_J] = (float)sj;
    }
  }
  __syncthreads();
  const T* __restrict__ arow = reinterpret_cast<const T*>(p.A[b]) + (long long)sj * p.lda;
  const int j = sj;
  const float nf = snf;
  const float* __restrict__ vr = p.Vin[b] + (long long)r * n;
  T* __restrict__ v0 = reinterpret_cast<T*>(p.Vout[b]);
  // element k of row r of V0: row-major, or in 16-column blocks (vblk)
  auto vat = [&](int k) { return p.vblk ? ((long long)(k >> 4) * NLB_K + r) * 16 + (k & 15) : (long long)r * n + k; };
  const bool vec = (n & 7) == 0 && (p.lda * (long long)sizeof(T)) % 16 == 0 &&
                   (reinterpret_cast<uintptr_t>(p.A[b]) & 15) == 0 && (reinterpret_cast<uintptr_t>(p.Vin[b]) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(p.Vout[b]) & 15) == 0;
  auto aval = [&](float a, int k) { return (p.sign < 0 && k == j ? 0.f : a) / nf; };
  float d = 0.f;
  if (vec) {
#pragma unroll 2
    for (int c = tid; c < (n >> 3); c += 256) {
      float a[8], v[8];
      load8(arow + 8 * c, a);
      load8(vr + 8 * c, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) d += aval(a[e], 8 * c + e) * v[e];
    }
  } else {
    for (int k = tid; k < n; k += 256) d += aval(to_f32<T>(arow[k]), k) * vr[k];
  }
  d = block_sum(d, red);
  const float sg = d > 0.f ? 1.f : (d < 0.f ? -1.f : 0.f);
  if (vec) {
#pragma unroll 2
    for (int c = tid; c < (n >> 3); c += 256) {
      float a[8], v[8];
      load8(arow + 8 * c, a);
      load8(vr + 8 * c, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) a[e] = aval(a[e], 8 * c + e) + sg * v[e];
      store8(v0 + vat(8 * c), a);  // 8 columns inside one 16-column block
    }
  } else {
    for (int k = tid; k < n; k += 256) v0[vat(k)] = from_f32<T>(aval(to_f32<T>(arow[k]), k) + sg * vr[k]);
  }
}

// W = V A^T * (1 / nf) * (normalize ? 1 / (|V_r| + smallest normal) : 1) for symmetric or skew A read in full;
// A^T = +-A, and a sign flip of every product leaves every row norm of the iteration, hence the bound, unchanged.
// Reading A^T makes both operands k-contiguous: rows c of A for output columns c, rows r of V.
// Workgroup: 32 rows x 128 columns x one k slice (kslice, a multiple of 64), 4 waves of 32 columns (2 x 2 MFMA
// tiles of 16 x 16). Every operand element is used by one wave only (V rows are shared through the caches), so the
// lanes load their MFMA fragments as 16-byte pieces straight from memory, 4 k steps at a time: no LDS staging and
// no barriers, and the loads in flight are bounded by registers only. V is stored in A's type T (the init kernel
// and the epilogues write it so): bf16 with v_mfma_f32_16x16x32_bf16, fp32 with v_mfma_f32_16x16x4_f32.
// ksplit > 1: each workgroup stores its 32 x 128 partial in part[b][s] and vmm_reduce_kernel sums the slices in
// order s = 0, 1, ... and runs the epilogue. A single-workgroup handshake (a device-scope fence and an arrival
// counter) would need an L2 write-back and invalidate per workgroup on this multi-XCD part, which costs more than
// the separate launch. Epilogue: W, and ssout[r][cb] = sum over the block's columns of W[r][c]^2.
// grid: nb * ceil(n / 128) * ksplit, the k slice fastest.
constexpr int VMM_C = 128;

// 1 / nf, times 1 / (|W_r| + smallest normal) of the previous product when normalize (psgd_pro.py:36-38). The
// row's nbk partial sums are added in order q = 0, 1, ..., loaded 32 at a time so that their latencies overlap
// (entries past nbk count as +0, which leaves the non-negative sum unchanged).
__device__ __forceinline__ float vmm_row_scale(const NlbArgs& p, int b, int r, int nbk, int normalize) {
  float sc = 1.f / p.scal[b][NLB_NF];
  if (normalize) {
    const float* ss = p.ssin[b] + (long long)r * nbk;
    float s = 0.f;
    for (int q = 0; q < nbk; q += 32) {
      float t[32];
#pragma unroll
      for (int e = 0; e < 32; ++e) {
        const float v = ss[q + e < nbk ? q + e : nbk - 1];  // unconditional: no branch per load
        t[e] = q + e < nbk ? v : 0.f;
      }
#pragma unroll
      for (int e = 0; e < 32; ++e) s += t[e];
    }
    sc = sc / (sqrtf(s) + kSmallestNormal);
  }
  return sc;
}

template <typename T, int U>  // U: MFMA steps whose loads are issued together
__global__ void __launch_bounds__(256) vmm_full_kernel(const NlbArgs p, int normalize) {
  constexpr bool BF = sizeof(T) == 2;
  constexpr int ACH = 16 / sizeof(T);  // elements per 16-byte piece
  constexpr int KS = 4 * ACH;          // k per MFMA step: lane group g holds pieces at k + g ACH
  __shared__ float rs[NLB_K];
  __shared__ float ssw[4][NLB_K];
  const int nbk = (p.n + VMM_C - 1) / VMM_C;
  const int ks = blockIdx.x % p.ksplit, bc = blockIdx.x / p.ksplit;
  const int b = bc / nbk, cb = bc % nbk;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  const int n = p.n, c0 = cb * VMM_C;
  const T* __restrict__ A = reinterpret_cast<const T*>(p.A[b]);
  const T* __restrict__ V = reinterpret_cast<const T*>(p.Vin[b]);
  if (tid < NLB_K) rs[tid] = vmm_row_scale(p, b, tid, nbk, normalize);
  // 16-byte buffer loads (out-of-range lanes read zero, no branches) where every row start is 16-byte aligned and
  // both matrices span < 2^31 bytes (uniform per launch); element loads otherwise
  const bool va = (p.lda % ACH) == 0 && (n % ACH) == 0 && (reinterpret_cast<uintptr_t>(A) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(V) & 15) == 0 && (long long)n * p.lda * sizeof(T) < kOob &&
                  (long long)NLB_K * n * sizeof(T) < kOob;
  // MFMA operands straight from memory: V rows i*16 + r16 (A operand), A rows = output columns (B operand)
  int cj[2];
  bool aok[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    cj[j] = c0 + wave * 32 + j * 16 + r16;
    aok[j] = cj[j] < n;
  }
  f32x4_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  auto mma = [&](const uint4 (&vf)[2], const uint4 (&af)[2]) {
    if constexpr (BF) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, vf[i]),
                                                              __builtin_bit_cast(bf16x8_t, af[j]), acc[i][j], 0, 0, 0);
    } else {  // element s of every lane's piece: k = kk + 4 g + s, the same map for both operands
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float((&vf[i].x)[s4]),
                                                             __uint_as_float((&af[j].x)[s4]), acc[i][j], 0, 0, 0);
    }
  };
  const int kbeg = ks * p.kslice, kend = min(n, kbeg + p.kslice);
  if (va) {
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(V, (long long)NLB_K * n * sizeof(T));
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(A, (long long)n * p.lda * sizeof(T));
    int vo[2], ao[2];  // byte offsets of this lane's pieces at k = 0
#pragma unroll
    for (int i = 0; i < 2; ++i) vo[i] = ((i * 16 + r16) * n + g * ACH) * (int)sizeof(T);
#pragma unroll
    for (int j = 0; j < 2; ++j) ao[j] = (int)(((long long)cj[j] * p.lda + g * ACH) * sizeof(T));
    for (int k0 = kbeg; k0 < kend; k0 += U * KS) {
      uint4 vf[U][2], af[U][2];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int kk = k0 + u * KS, so = kk * (int)sizeof(T);
        const bool in = kk + g * ACH < kend;
#pragma unroll
        for (int i = 0; i < 2; ++i)
          vf[u][i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rv, in ? vo[i] : kOob, so, 0));
#pragma unroll
        for (int j = 0; j < 2; ++j)
          af[u][j] = __builtin_bit_cast(uint4,
                                        __builtin_amdgcn_raw_buffer_load_b128(ra, in && aok[j] ? ao[j] : kOob, so, 0));
      }
      __builtin_amdgcn_sched_barrier(0);  // keep all U steps' loads ahead of the first MFMA
#pragma unroll
      for (int u = 0; u < U; ++u) mma(vf[u], af[u]);
    }
  } else {
    for (int k0 = kbeg; k0 < kend; k0 += KS) {
      uint4 vf[2], af[2];
      const int kl = k0 + g * ACH;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        T t[ACH];
        const T* src = V + (long long)(i * 16 + r16) * n + kl;
#pragma unroll
        for (int e = 0; e < ACH; ++e) t[e] = kl + e < kend ? src[e] : T(0);
        vf[i] = *reinterpret_cast<const uint4*>(t);
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        T t[ACH];
        const T* src = A + (long long)(aok[j] ? cj[j] : 0) * p.lda + kl;
#pragma unroll
        for (int e = 0; e < ACH; ++e) t[e] = aok[j] && kl + e < kend ? src[e] : T(0);
        af[j] = *reinterpret_cast<const uint4*>(t);
      }
      mma(vf, af);
    }
  }
  __syncthreads();  // rs
  // lane holds rows i*16 + 4g + e of column wave*32 + j*16 + r16
  if (p.ksplit > 1) {  // partial product of this k slice; vmm_reduce_kernel finishes the column block
    float* __restrict__ P = p.part[b];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = c0 + wave * 32 + j * 16 + r16;
      if (col < n) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e) P[((long long)ks * NLB_K + i * 16 + g * 4 + e) * n + col] = acc[i][j][e];
      }
    }
    return;
  }
  T* __restrict__ W = reinterpret_cast<T*>(p.Vout[b]);
  float sq[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) sq[i][e] = 0.f;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int col = c0 + wave * 32 + j * 16 + r16;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = i * 16 + g * 4 + e;
        const float w = acc[i][j][e] * rs[row];
        if (col < n) {
          W[(long long)row * n + col] = from_f32<T>(w);
          sq[i][e] += w * w;
        }
      }
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float v = sq[i][e];
      for (int o = 1; o < 16; o <<= 1) v += __shfl_xor(v, o, 64);
      sq[i][e] = v;
    }
  if (r16 == 0) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) ssw[wave][i * 16 + g * 4 + e] = sq[i][e];
  }
  __syncthreads();
  if (tid < NLB_K) p.ssout[b][tid * nbk + cb] = ssw[0][tid] + ssw[1][tid] + ssw[2][tid] + ssw[3][tid];
}

// Sum of the ksplit (<= VMM_MAXS) partial products of 8 rows x 128 columns in slice order, then the epilogue of
// vmm_full_kernel (row scale, W in the storage type T, per-row sums of squares of the fp32 values over the block's
// columns). Thread (rg, c) owns rows r0 + rg + 2t (t < 4) of column c and issues the loads of all slices and rows
// at once (slices >= ksplit read zero through the buffer range check; adding zeros keeps the sum). grid: nb *
// ceil(n / 128) * 4.
constexpr int VMM_MAXS = 8;

template <typename T>
__global__ void __launch_bounds__(256) vmm_reduce_kernel(const NlbArgs p, int normalize) {
  __shared__ float rs[8];
  __shared__ float ssw[4][4];
  const int nbk = (p.n + VMM_C - 1) / VMM_C;
  const int b = blockIdx.x / (nbk * 4), cb = (blockIdx.x / 4) % nbk, r0 = (blockIdx.x % 4) * 8;
  const int tid = threadIdx.x, n = p.n;
  if (tid < 8) rs[tid] = vmm_row_scale(p, b, r0 + tid, nbk, normalize);
  const int col = cb * VMM_C + (tid & 127), rg = tid >> 7;
  const bool ok = col < n;
  const __amdgpu_buffer_rsrc_t rp = make_rsrc(p.part[b], (long long)p.ksplit * NLB_K * n * 4);
  const int vo = ok ? ((r0 + rg) * n + col) * 4 : kOob;
  float x[VMM_MAXS][4];
#pragma unroll
  for (int q = 0; q < VMM_MAXS; ++q)
#pragma unroll
    for (int t = 0; t < 4; ++t)
      x[q][t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                              rp, q < p.ksplit ? vo : kOob, (q * NLB_K + 2 * t) * n * 4, 0));
  float w[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    w[t] = x[0][t];
#pragma unroll
    for (int q = 1; q < VMM_MAXS; ++q) w[t] += x[q][t];
  }
  __syncthreads();
  T* __restrict__ W = reinterpret_cast<T*>(p.Vout[b]);
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int lr = rg + 2 * t;
    const float v = ok ? w[t] * rs[lr] : 0.f;
    if (ok) W[(long long)(r0 + lr) * n + col] = from_f32<T>(v);
    const float sq = wave_sum(v * v);
    if ((tid & 63) == 0) ssw[tid >> 6][t] = sq;
  }
  __syncthreads();
  if (tid < 8) {
    const int g = tid & 1, t = tid >> 1;  // local row tid = g + 2 t: waves 2g and 2g + 1
    p.ssout[b][(r0 + tid) * nbk + cb] = ssw[2 * g][t] + ssw[2 * g + 1][t];
  }
}

// W = V A^T * row scale (the product of vmm_full_kernel) with one workgroup per 64 output columns of one matrix
// over the whole k range, so that no partial products leave the workgroup and no reduce kernel follows. Wave w
// multiplies the k quarter [w kq, (w + 1) kq) for all 32 x 64 outputs (2 x 4 MFMA tiles of 16 x 16, each V
// fragment used by four A fragments); the four partial blocks are summed through LDS in the fixed order w = 0..3.
// Operands come from 16-byte buffer loads straight into MFMA fragments, U steps issued together (the 16-byte layout
// is required: n and the row stride multiples of 16 bytes, aligned bases, each matrix < 2 GiB; the host checks).
// Epilogue: thread t owns row t / 8 and 8 consecutive columns: W in T (one 16- or 32-byte store) and
// ssout[r][cb] = sum over the block's columns of W[r][c]^2 (dot: of W[r][c] times the scaled input), reduced over
// the row's 8 lanes in a fixed tree. Rectangular products (kdim > 0): V is 32 x kdim, A is n x kdim, W is 32 x n;
// plain: no row scale and no sums of squares (the Gram route's start U0 = V0 Pc).
// grid: nb * ceil(n / 64).
constexpr int VMC = 64;     // output columns per workgroup
constexpr int VMC_LD = 68;  // LDS row stride (floats) of the partial blocks

template <typename T, int U>
__global__ void __launch_bounds__(256) vmm_cols_kernel(const NlbArgs p, int normalize) {
  constexpr bool BF = sizeof(T) == 2;
  constexpr int ACH = 16 / sizeof(T);  // elements per 16-byte piece
  constexpr int KS = 4 * ACH;          // k per MFMA step: lane group g holds pieces at k + g ACH
  __shared__ float rs[NLB_K];
  __shared__ __attribute__((aligned(16))) float red[4][NLB_K][VMC_LD];
  const int n = p.n, nbk = (n + VMC - 1) / VMC;
  const int K = p.kdim ? p.kdim : n;  // k extent (rectangular products: V is 32 x K, A is n x K)
  const int b = blockIdx.x / nbk, cb = blockIdx.x % nbk;
  // the wave index sets the k range, hence the loads' scalar offset: readfirstlane makes it provably uniform
  // (otherwise every load becomes a waterfall loop)
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int c0 = cb * VMC;
  const T* __restrict__ A = reinterpret_cast<const T*>(p.A[b]);
  const T* __restrict__ V = reinterpret_cast<const T*>(p.Vin[b]);
  if (tid < NLB_K) rs[tid] = p.plain ? 1.f : vmm_row_scale(p, b, tid, nbk, normalize);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(V, (long long)NLB_K * K * sizeof(T));
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(A, (long long)n * p.lda * sizeof(T));
  int vo[2], ao[4];  // byte offsets of this lane's pieces at k = 0 (kOob: a column past n reads zero)
#pragma unroll
  for (int i = 0; i < 2; ++i) vo[i] = ((i * 16 + r16) * K + g * ACH) * (int)sizeof(T);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = c0 + j * 16 + r16;
    ao[j] = c < n ? (int)(((long long)c * p.lda + g * ACH) * sizeof(T)) : kOob;
  }
  f32x4_t acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const int kq = ((K + 3) / 4 + KS - 1) / KS * KS;
  const int kbeg = wave * kq, kend = min(K, kbeg + kq);
  for (int k0 = kbeg; k0 < kend; k0 += U * KS) {
    uint4 vf[U][2], af[U][4];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kk = k0 + u * KS, so = kk * (int)sizeof(T);
      const bool in = kk + g * ACH < kend;
#pragma unroll
      for (int i = 0; i < 2; ++i)
        vf[u][i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rv, in ? vo[i] : kOob, so, 0));
#pragma unroll
      for (int j = 0; j < 4; ++j)
        af[u][j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(ra, in ? ao[j] : kOob, so, 0));
    }
    __builtin_amdgcn_sched_barrier(0);  // keep all U steps' loads ahead of the first MFMA
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if constexpr (BF) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, vf[u][i]),
                                                                __builtin_bit_cast(bf16x8_t, af[u][j]), acc[i][j], 0, 0, 0);
      } else {  // element s of every lane's piece: k = kk + 4 g + s, the same map for both operands
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float((&vf[u][i].x)[s4]),
                                                               __uint_as_float((&af[u][j].x)[s4]), acc[i][j], 0, 0, 0);
      }
    }
  }
  // lane holds rows i*16 + 4g + e of columns j*16 + r16
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) red[wave][i * 16 + 4 * g + e][j * 16 + r16] = acc[i][j][e];
  __syncthreads();
  const int row = tid >> 3, cl = (tid & 7) * 8, col = c0 + cl;
  float w[8];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const float4 x0 = *reinterpret_cast<const float4*>(&red[0][row][cl + 4 * h]);
    const float4 x1 = *reinterpret_cast<const float4*>(&red[1][row][cl + 4 * h]);
    const float4 x2 = *reinterpret_cast<const float4*>(&red[2][row][cl + 4 * h]);
    const float4 x3 = *reinterpret_cast<const float4*>(&red[3][row][cl + 4 * h]);
    w[4 * h + 0] = ((x0.x + x1.x) + x2.x) + x3.x;
    w[4 * h + 1] = ((x0.y + x1.y) + x2.y) + x3.y;
    w[4 * h + 2] = ((x0.z + x1.z) + x2.z) + x3.z;
    w[4 * h + 3] = ((x0.w + x1.w) + x2.w) + x3.w;
  }
  const float sc = rs[row];
  float x[8];  // dot: the scaled input row at these columns (square products: V is 32 x n)
  if (p.dot) {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = col + e < n ? sc * to_f32(V[(long long)row * n + col + e]) : 0.f;
  }
  float sq = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    w[e] *= sc;
    if (col + e < n) sq += w[e] * (p.dot ? x[e] : w[e]);
  }
  T* __restrict__ W = reinterpret_cast<T*>(p.Vout[b]) + (long long)row * n + col;
  if (col + 8 <= n) {
    store8(W, w);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (col + e < n) W[e] = from_f32<T>(w[e]);
  }
  if (p.plain) return;
  sq += __shfl_xor(sq, 1, 64);
  sq += __shfl_xor(sq, 2, 64);
  sq += __shfl_xor(sq, 4, 64);
  if ((tid & 7) == 0) p.ssout[b][row * nbk + cb] = sq;
}

// The product of vmm_cols_kernel with A staged through LDS: the workgroup's 64 rows of A are read in chunks of
// 64 rows x 512 bytes (256 bf16 or 128 fp32 of k), each row's 512 bytes by 32 consecutive lanes (row-contiguous
// runs, as a row-norm pass reads them; the MFMA fragment layout would read 64-byte pieces of 16 rows per load),
// stored in unpadded 512-byte rows whose 16-byte pieces are XOR-swizzled by the row (piece p of row r at
// p ^ (r % 16): the 16 fragment rows of a read land on 16 distinct 16-byte bank groups, and the 32 lanes writing
// one row still cover its 32 slots) and read back as MFMA fragments. Wave w multiplies the k quarter w of every
// chunk (2 MFMA steps, V fragments straight from global memory; fp32: four 16x16x4 MFMAs per fragment pair,
// element s of every lane's piece at k = kk + 4 g + s for both operands); the next chunk's A and V loads are in
// flight while a chunk is multiplied. The four waves' partial blocks are summed through LDS in the fixed order
// w = 0..3, 16 rows of W at a time, and each row is scaled, stored and its sum of squares (of this column block)
// written. The 32 KB of LDS (the staging buffer, which the epilogue reuses) would let five workgroups share a CU;
// the 136 registers of the bf16 instantiation (three waves per SIMD) let three.
// grid: nb * ceil(n / 64).
constexpr int VR_ROWB = 512;                   // bytes of one row per chunk
constexpr int VR_SMEM = VMC * VR_ROWB;         // the staging buffer: 64 rows x 512 bytes
static_assert(4 * 16 * VMC_LD * 4 + NLB_K * 4 <= VR_SMEM, "epilogue blocks and row scales fit in the staging buffer");

template <typename T>
__global__ void __launch_bounds__(256) vmm_rows_kernel(const NlbArgs p, int normalize) {
  constexpr int CE = 16 / sizeof(T);          // elements per 16-byte piece
  constexpr int VRK = VR_ROWB / sizeof(T);    // k per chunk
  constexpr int KS = 4 * CE;                  // k per MFMA step
  __shared__ __attribute__((aligned(16))) unsigned char sm[VR_SMEM];
  T* const As = reinterpret_cast<T*>(sm);
  const int n = p.n, nbk = (n + VMC - 1) / VMC;
  const int K = p.kdim ? p.kdim : n;
  const int b = blockIdx.x / nbk, cb = blockIdx.x % nbk;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int c0 = cb * VMC;
  const T* __restrict__ A = reinterpret_cast<const T*>(p.A[b]);
  const T* __restrict__ V = reinterpret_cast<const T*>(p.Vin[b]);
  // the row scale of V row tid (threads < 32), kept in a register until the epilogue
  const float my_rs = tid < NLB_K ? (p.plain ? 1.f : vmm_row_scale(p, b, tid, nbk, normalize)) : 0.f;
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(V, (long long)NLB_K * K * sizeof(T));
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(A, (long long)n * p.lda * sizeof(T));
  // A staging: thread t owns the 16-byte piece t % 32 of rows t / 32 + 8 i (i < 8) of the chunk
  const int rr = tid >> 5, pc = tid & 31;
  int ao[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    ao[i] = c0 + rr + 8 * i < n ? (int)(((long long)(c0 + rr + 8 * i) * p.lda + pc * CE) * sizeof(T)) : kOob;
  int vo[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) vo[i] = ((i * 16 + r16) * K + g * CE) * (int)sizeof(T);
  uint4 st[8], vn[2][2];
  auto load = [&](int kc) {  // chunk at k = kc: A pieces into st, this wave's V fragments into vn
    const bool kin = kc + pc * CE < K;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      st[i] = __builtin_bit_cast(
          uint4, __builtin_amdgcn_raw_buffer_load_b128(ra, kin ? ao[i] : kOob, kc * (int)sizeof(T), 0));
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int kk = kc + wave * (VRK / 4) + s * KS;
      const bool vin = kk + g * CE < K;
#pragma unroll
      for (int i = 0; i < 2; ++i)
        vn[s][i] = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(rv, vin ? vo[i] : kOob, kk * (int)sizeof(T), 0));
    }
  };
  f32x4_t acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  load(0);
  for (int kc = 0; kc < K; kc += VRK) {
    // row rr + 8 i has (rr + 8 i) % 16 = rr + 8 (i % 2)
#pragma unroll
    for (int i = 0; i < 8; ++i)
      *reinterpret_cast<uint4*>(As + (rr + 8 * i) * VRK + ((pc ^ (rr + 8 * (i & 1))) * CE)) = st[i];
    uint4 vc[2][2];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int i = 0; i < 2; ++i) vc[s][i] = vn[s][i];
    __syncthreads();
    if (kc + VRK < K) load(kc + VRK);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int piece = wave * 8 + s * 4 + g;  // 16-byte piece of the row this lane's fragment reads
      uint4 af[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) af[j] = *reinterpret_cast<const uint4*>(As + (j * 16 + r16) * VRK + (piece ^ r16) * CE);
      if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, vc[s][i]),
                                                                __builtin_bit_cast(bf16x8_t, af[j]), acc[i][j], 0, 0, 0);
      } else {
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float((&vc[s][i].x)[s4]),
                                                               __uint_as_float((&af[j].x)[s4]), acc[i][j], 0, 0, 0);
      }
    }
    __syncthreads();
  }
  // Epilogue in the staging buffer (free after the loop's last barrier): rows 16 h .. 16 h + 15 of the four waves'
  // partial blocks, then the row scales after them. Lane holds rows i * 16 + 4 g + e of columns j * 16 + r16.
  float (*red)[16][VMC_LD] = reinterpret_cast<float (*)[16][VMC_LD]>(sm);
  float* const rsl = reinterpret_cast<float*>(sm) + 4 * 16 * VMC_LD;
  if (tid < NLB_K) rsl[tid] = my_rs;
  const int lr = tid >> 4, cl = (tid & 15) * 4, col = c0 + cl;  // this thread: row lr of the half, 4 columns
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if (h) __syncthreads();  // the first half's reads are done
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) red[wave][4 * g + e][j * 16 + r16] = acc[h][j][e];
    __syncthreads();
    const int row = 16 * h + lr;
    const float4 x0 = *reinterpret_cast<const float4*>(&red[0][lr][cl]);
    const float4 x1 = *reinterpret_cast<const float4*>(&red[1][lr][cl]);
    const float4 x2 = *reinterpret_cast<const float4*>(&red[2][lr][cl]);
    const float4 x3 = *reinterpret_cast<const float4*>(&red[3][lr][cl]);
    float w[4] = {((x0.x + x1.x) + x2.x) + x3.x, ((x0.y + x1.y) + x2.y) + x3.y, ((x0.z + x1.z) + x2.z) + x3.z,
                  ((x0.w + x1.w) + x2.w) + x3.w};
    const float sc = rsl[row];
    float x[4];  // dot: the scaled input row at these columns (square products: V is 32 x n)
    if (p.dot) {
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = col + e < n ? sc * to_f32(V[(long long)row * n + col + e]) : 0.f;
    }
    float sq = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      w[e] *= sc;
      if (col + e < n) sq += w[e] * (p.dot ? x[e] : w[e]);
    }
    T* __restrict__ W = reinterpret_cast<T*>(p.Vout[b]) + (long long)row * n + col;
    if (col + 4 <= n) {
      store4(W, w);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (col + e < n) W[e] = from_f32<T>(w[e]);
    }
    if (!p.plain) {
      sq += __shfl_xor(sq, 1, 64);
      sq += __shfl_xor(sq, 2, 64);
      sq += __shfl_xor(sq, 4, 64);
      sq += __shfl_xor(sq, 8, 64);
      if ((tid & 15) == 0) p.ssout[b][row * nbk + cb] = sq;
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Norm bound of term1 = P P^T from its factor P (d x k, k < d / 2 on the bf16 update's Pg route). With H = P^T P:
// ||row i of P P^T||^2 = P_i H P_i^T = sum_c (P H)_ic P_ic, (P P^T)_ii = ||P_i||^2, row j of P P^T = P P_j^T.

// One wave per row i: rn2[i] = sum_c W_ic P_ic, diag[i] = sum_c P_ic^2, rmax[i] = 0 (16-byte loads; k % 8 == 0 and
// 16-byte aligned rows, which the host checks). grid: nb * ceil(d / 4).
__global__ void __launch_bounds__(256) gram_stats_kernel(const GramArgs p) {
  const int nrb = (p.d + 3) / 4;
  const int b = blockIdx.x / nrb, i = (blockIdx.x % nrb) * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (i >= p.d) return;
  const bf16_t* __restrict__ pr = p.P[b] + (long long)i * p.k;
  const bf16_t* __restrict__ wr = p.W[b] + (long long)i * p.k;
  float s = 0.f, q = 0.f;
  for (int c = lane; c < p.k / 8; c += 64) {
    float x[8], w[8];
    load8(pr + 8 * c, x);
    load8(wr + 8 * c, w);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      s += w[e] * x[e];
      q += x[e] * x[e];
    }
  }
  s = wave_sum(s);
  q = wave_sum(q);
  if (lane == 0) {
    p.rn2[b][i] = s;
    p.diag[b][i] = q;
    p.rmax[b][i] = 0.f;
  }
}

// One workgroup per matrix: j = the first maximum of rn2 (the init kernel's rule) into scal[NLB_J].
__global__ void __launch_bounds__(256) gram_argmax_kernel(const GramArgs p) {
  __shared__ float sval[4];
  __shared__ int sidx[4];
  const int b = blockIdx.x, tid = threadIdx.x;
  const float* __restrict__ rn2 = p.rn2[b];
  float best = -1.f;
  int bi = 0x7fffffff;
  for (int i = tid; i < p.d; i += 256) {
    const float v = rn2[i];
    if (v > best) { best = v; bi = i; }
  }
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (ov > best || (ov == best && oi < bi)) { best = ov; bi = oi; }
  }
  if ((tid & 63) == 0) { sval[tid >> 6] = best; sidx[tid >> 6] = bi; }
  __syncthreads();
  if (tid == 0) {
    float bv = sval[0];
    int bj = sidx[0];
    for (int w = 1; w < 4; ++w)
      if (sval[w] > bv || (sval[w] == bv && sidx[w] < bj)) { bv = sval[w]; bj = sidx[w]; }
    p.scal[b][NLB_J] = (float)(bj < p.d ? bj : 0);
  }
}

// One wave per row c: aj[c] = sum_k P_ck P_jk (row j of P P^T, rounded to bf16 like the matrices the bound reads).
// grid: nb * ceil(d / 4).
__global__ void __launch_bounds__(256) gram_row_kernel(const GramArgs p) {
  const int nrb = (p.d + 3) / 4;
  const int b = blockIdx.x / nrb, c = (blockIdx.x % nrb) * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (c >= p.d) return;
  const int j = (int)p.scal[b][NLB_J];
  const bf16_t* __restrict__ pc = p.P[b] + (long long)c * p.k;
  const bf16_t* __restrict__ pj = p.P[b] + (long long)j * p.k;
  float s = 0.f;
  for (int q = lane; q < p.k / 8; q += 64) {
    float x[8], y[8];
    load8(pc + 8 * q, x);
    load8(pj + 8 * q, y);
#pragma unroll
    for (int e = 0; e < 8; ++e) s += x[e] * y[e];
  }
  s = wave_sum(s);
  if (lane == 0) p.aj[b][c] = f32_to_bf16(s);
}

hipError_t gram_launch(const GramArgs& a, int stage, hipStream_t st) {
  const int nrb = (a.d + 3) / 4;
  if (stage == 0) hipLaunchKernelGGL(gram_stats_kernel, dim3(nrb * a.nb), dim3(256), 0, st, a);
  else if (stage == 1) hipLaunchKernelGGL(gram_argmax_kernel, dim3(a.nb), dim3(256), 0, st, a);
  else hipLaunchKernelGGL(gram_row_kernel, dim3(nrb * a.nb), dim3(256), 0, st, a);
  return hipGetLastError();
}

// The product of vmm_rows_kernel (W = V A^T with its row scales and per-(row, 64-column block) sums of squares) for
// a symmetric or skew bf16 matrix stored in full, read from its upper 64 x 64 tiles only. Workgroup J (output
// columns 64 J ..) needs the tiles (J, s) of A for every s; tile (J, s) with J > s is sign * (s, J)^T, so every
// upper tile serves two workgroups. They read it in the same round: round r pairs workgroup J with s = sigma_r(J),
// the circle method of a round-robin tournament on T = n / 64 players (T even; round T - 1 is the diagonal tile),
// and all T workgroups of a matrix run on one XCD (workgroups go round-robin over the 8 XCDs: matrix b on XCD
// b % 8), so the second read of a tile is an L2 hit. A loads-only probe of 24 matrices of 3072^2 read this way took
// 34.5 us against 74.3 us for their full rows. A round stages the tile in LDS as stored (16-byte writes), then wave w
// multiplies its k quarter of it with one v_mfma_f32_32x32x16_bf16 per 32-column half (V's 32 rows are one M tile;
// V fragments straight from global memory, where V is kept in 16-column blocks (NlbArgs::vblk) so that a wave's
// fragment is one contiguous 1 KB read): a tile (J, s) is [column][k] and its B fragments are 16-byte reads, a
// tile (s, J) is [k][column] and its fragments come from gfx950's transposing LDS reads (ds_read_b64_tr_b16), the
// sign folded in. VT_D rounds' loads are in flight, issued unconditionally (loads
// past the last round re-read it) so that the compiler can count them; one barrier per round (two LDS buffers). The
// four waves' partial blocks are summed through LDS in the order w = 0..3, 16 rows at a time, as in vmm_rows_kernel.
// grid: 8 * ceil(nb / 8) * T (workgroups of matrices past nb exit at once).
constexpr int VT_LD = 72;  // LDS row pitch (bf16) of a staged tile: 144-byte rows, 16-byte aligned

__device__ __forceinline__ int vt_partner(int J, int r, int T) {
  if (r == T - 1) return J;  // the diagonal round
  if (J == T - 1) return r;
  if (J == r) return T - 1;
  return ((2 * r - J) % (T - 1) + (T - 1)) % (T - 1);
}

// Five waves per SIMD (the accumulators in arch VGPRs, 96 registers in all): 1280 workgroups fit at once, so 24
// matrices of 3072 columns (1152 workgroups) run in one round; at four per SIMD 128 of them formed a second round.
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(5))) vmm_tri_kernel(const NlbArgs p,
                                                                                               int normalize) {
  const int n = p.n, T = n / VMC;
  const int xcd = blockIdx.x % 8, slot = blockIdx.x / 8;
  const int b = xcd + 8 * (slot / T), J = slot % T;
  if (b >= p.nb) return;
  __shared__ __attribute__((aligned(16))) unsigned char sm[2 * VMC * VT_LD * 2];  // 2 tiles; the epilogue reuses it
  __shared__ float rsl[NLB_K];
  bf16_t* const lt = reinterpret_cast<bf16_t*>(sm);
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, h = lane >> 5;
  const bf16_t* __restrict__ A = reinterpret_cast<const bf16_t*>(p.A[b]);
  const bf16_t* __restrict__ V = reinterpret_cast<const bf16_t*>(p.Vin[b]);
  const long long lda = p.lda;
  const uint32_t flip = p.sign < 0 ? 0x80008000u : 0u;
  // a round's operands in registers: this thread's two 16-byte pieces of the tile (rows v / 8, chunk v % 8 for
  // v = tid, tid + 256) and this lane's V fragment (row c, k = 64 s + 16 w + 8 h .. + 7)
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));  // not uint4, whose copies go through memory
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x4_v __attribute__((__vector_size__(4 * sizeof(__bf16))));
  typedef __attribute__((address_space(3))) bf16x4_v lds_bf16x4;  // an LDS address, as the transposing read takes
  struct Rd {
    u32x4 t0, t1, v;
  };
  auto load = [&](int r, Rd& x) {
    r = r < T ? r : T - 1;
    const int s = vt_partner(J, r, T), lo = J < s ? J : s, hi = J < s ? s : J;
    const bf16_t* const t = A + (long long)(lo * VMC + (tid >> 3)) * lda + hi * VMC + (tid & 7) * 8;
    x.t0 = *reinterpret_cast<const u32x4*>(t);
    x.t1 = *reinterpret_cast<const u32x4*>(t + 32 * lda);  // v = tid + 256: 32 rows further
    // V in 16-column blocks: this wave's fragment (rows 0..31, k = 64 s + 16 w ..) is one contiguous 1 KB
    x.v = *reinterpret_cast<const u32x4*>(V + ((long long)(4 * s + w) * NLB_K + c) * 16 + 8 * h);
  };
  f32x16_t acc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[j][i] = 0.f;
  auto do_round = [&](int r, const Rd& x) {
    const int s = vt_partner(J, r, T);
    bf16_t* const L = lt + (r & 1) * VMC * VT_LD;
    bf16_t* const st = L + (tid >> 3) * VT_LD + (tid & 7) * 8;
    *reinterpret_cast<u32x4*>(st) = x.t0;
    *reinterpret_cast<u32x4*>(st + 32 * VT_LD) = x.t1;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      u32x4 bf;
      if (J <= s) {  // tile (J, s): row 32 j + c, k = 16 w + 8 h .. + 7
        bf = *reinterpret_cast<const u32x4*>(L + (32 * j + c) * VT_LD + 16 * w + 8 * h);
      } else {  // tile (s, J): column 32 j + c of rows 16 w + 8 h .. + 7, times sign, by two transposing reads
        // (each: 16 lanes read a 4 x 16 block, lane i the 4 elements at row i / 4, columns 4 (i % 4) ..; lane i
        // receives column i of the block, rows 0..3)
        const int i = lane & 15;
        const bf16_t* const tb = L + (16 * w + 8 * h + (i >> 2)) * VT_LD + 32 * j + 16 * (c >> 4) + 4 * (i & 3);
        const u32x2 lo = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)tb));
        const u32x2 hi =
            __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(tb + 4 * VT_LD)));
        bf = u32x4{lo[0], lo[1], hi[0], hi[1]} ^ flip;
      }
      acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, x.v), __builtin_bit_cast(bf16x8_t, bf),
                                                       acc[j], 0, 0, 0);
    }
  };
  Rd x0, x1, x2, x3;  // four rounds in flight (named registers: an array of them is not kept in registers)
  load(0, x0);
  load(1, x1);
  load(2, x2);
  load(3, x3);
  for (int r0 = 0; r0 < T; r0 += 4) {
    do_round(r0, x0);
    load(r0 + 4, x0);
    do_round(r0 + 1, x1);
    load(r0 + 5, x1);
    if (r0 + 2 < T) {  // T is even; the branch holds no memory loads
      do_round(r0 + 2, x2);
      do_round(r0 + 3, x3);
    }
    load(r0 + 6, x2);
    load(r0 + 7, x3);
  }
  // The row scales, read after the epilogue's first barrier. Computed here, where the rounds' operand registers are
  // free, the helper's loads go out together; before the rounds (x0..x3 in flight) the compiler issued them one at a
  // time, each waited for, and the first round's barrier waited out that chain of T dependent loads.
  if (tid < NLB_K) rsl[tid] = vmm_row_scale(p, b, tid, T, normalize);
  // Epilogue: lane (c, h) holds rows 8 (i / 4) + 4 h + i % 4 of column 32 j + c; rows 0-15 are i < 8
  float (*red)[16][VMC] = reinterpret_cast<float (*)[16][VMC]>(sm);
  const int lr = tid >> 4, cl = (tid & 15) * 4, col = J * VMC + cl;
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    __syncthreads();  // the last round's reads (hf = 0) or the first half's (hf = 1) are done
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int ii = 8 * hf + i;
        red[w][8 * (i >> 2) + 4 * h + (i & 3)][32 * j + c] = acc[j][ii];
      }
    __syncthreads();
    const int row = 16 * hf + lr;
    const float4 x0_ = *reinterpret_cast<const float4*>(&red[0][lr][cl]);
    const float4 x1_ = *reinterpret_cast<const float4*>(&red[1][lr][cl]);
    const float4 x2_ = *reinterpret_cast<const float4*>(&red[2][lr][cl]);
    const float4 x3_ = *reinterpret_cast<const float4*>(&red[3][lr][cl]);
    float wv[4] = {((x0_.x + x1_.x) + x2_.x) + x3_.x, ((x0_.y + x1_.y) + x2_.y) + x3_.y,
                   ((x0_.z + x1_.z) + x2_.z) + x3_.z, ((x0_.w + x1_.w) + x2_.w) + x3_.w};
    const float sc = rsl[row];
    float sq = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      wv[e] *= sc;
      sq += wv[e] * wv[e];
    }
    // W in 16-column blocks, as this kernel reads its V (4 columns inside one block)
    store4(reinterpret_cast<bf16_t*>(p.Vout[b]) + ((long long)(col >> 4) * NLB_K + row) * 16 + (col & 15), wv);
    sq += __shfl_xor(sq, 1, 64);
    sq += __shfl_xor(sq, 2, 64);
    sq += __shfl_xor(sq, 4, 64);
    sq += __shfl_xor(sq, 8, 64);
    if ((tid & 15) == 0) p.ssout[b][row * T + J] = sq;
  }
}

hipError_t nlb_full_launch(const NlbArgs& a, int stage, int a_bf16, int normalize, hipStream_t st) {
  if (stage == 3) {
    hipLaunchKernelGGL(rowstats_reduce_kernel, dim3(((a.n + 63) / 64) * a.nb), dim3(256), 0, st, a);
  } else if (stage == 0) {
    const int nrb = (a.n + 3) / 4;
    if (a_bf16) hipLaunchKernelGGL(rownorm_full_kernel<bf16_t>, dim3(nrb * a.nb), dim3(256), 0, st, a);
    else hipLaunchKernelGGL(rownorm_full_kernel<float>, dim3(nrb * a.nb), dim3(256), 0, st, a);
  } else if (stage == 1) {
    if (a_bf16) hipLaunchKernelGGL(nlb_init_full_kernel<bf16_t>, dim3(a.nb * NLB_K), dim3(256), 0, st, a);
    else hipLaunchKernelGGL(nlb_init_full_kernel<float>, dim3(a.nb * NLB_K), dim3(256), 0, st, a);
  } else if (a.vmm_cols) {
    const dim3 grid(((a.n + VMC - 1) / VMC) * a.nb);
    if (a.vmm_cols == 3) {  // bf16, square, n a multiple of 128 (an even number of 64-tiles)
      const int T = a.n / VMC;
      hipLaunchKernelGGL(vmm_tri_kernel, dim3(8 * ((a.nb + 7) / 8) * T), dim3(256), 0, st, a, normalize);
    } else if (a.vmm_cols == 2) {
      if (a_bf16) hipLaunchKernelGGL(vmm_rows_kernel<bf16_t>, grid, dim3(256), 0, st, a, normalize);
      else hipLaunchKernelGGL(vmm_rows_kernel<float>, grid, dim3(256), 0, st, a, normalize);
    } else if (a_bf16) {
      if (a.vmm_u == 2) hipLaunchKernelGGL((vmm_cols_kernel<bf16_t, 2>), grid, dim3(256), 0, st, a, normalize);
      else hipLaunchKernelGGL((vmm_cols_kernel<bf16_t, 4>), grid, dim3(256), 0, st, a, normalize);
    } else {
      if (a.vmm_u == 2) hipLaunchKernelGGL((vmm_cols_kernel<float, 2>), grid, dim3(256), 0, st, a, normalize);
      else hipLaunchKernelGGL((vmm_cols_kernel<float, 4>), grid, dim3(256), 0, st, a, normalize);
    }
  } else {
    const int nbk = (a.n + VMM_C - 1) / VMM_C;
    if (a.ksplit < 1 || a.ksplit > VMM_MAXS || a.kslice % 64 != 0 || (long long)a.ksplit * a.kslice < a.n)
      return hipErrorInvalidValue;
    const dim3 grid(nbk * a.nb * a.ksplit);
    if (a_bf16) {
      if (a.vmm_u == 8) hipLaunchKernelGGL((vmm_full_kernel<bf16_t, 8>), grid, dim3(256), 0, st, a, normalize);
      else if (a.vmm_u == 2) hipLaunchKernelGGL((vmm_full_kernel<bf16_t, 2>), grid, dim3(256), 0, st, a, normalize);
      else hipLaunchKernelGGL((vmm_full_kernel<bf16_t, 4>), grid, dim3(256), 0, st, a, normalize);
      if (a.ksplit > 1) hipLaunchKernelGGL(vmm_reduce_kernel<bf16_t>, dim3(nbk * a.nb * 4), dim3(256), 0, st, a, normalize);
    } else {
      if (a.vmm_u == 8) hipLaunchKernelGGL((vmm_full_kernel<float, 8>), grid, dim3(256), 0, st, a, normalize);
      else if (a.vmm_u == 2) hipLaunchKernelGGL((vmm_full_kernel<float, 2>), grid, dim3(256), 0, st, a, normalize);
      else hipLaunchKernelGGL((vmm_full_kernel<float, 4>), grid, dim3(256), 0, st, a, normalize);
      if (a.ksplit > 1) hipLaunchKernelGGL(vmm_reduce_kernel<float>, dim3(nbk * a.nb * 4), dim3(256), 0, st, a, normalize);
    }
  }
  return hipGetLastError();
}

}  // namespace psgdk

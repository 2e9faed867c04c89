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
#pragma unroll
  for (int c = 0; c < 16; ++c) {
    const int gj = J * RT + lc0 + c;
    float v = 0.f;
    if (gi < n && gj < n && gi <= gj) v = A[(long long)gi * ld + gj];
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
  const int nbk = (p.n + 63) / 64;
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
      const float ell = bound + f.term2;
      float* L = f.L[b];
      const float Ln = fmaxf(f.beta * L[0] + (1.f - f.beta) * ell, ell);
      L[0] = Ln;
      f.coef[b][0] = f.lr / Ln;
      f.coef[b][1] = f.term2;
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

}  // namespace psgdk

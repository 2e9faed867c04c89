// Elementwise and reduction kernels around the contractions: argument blocks and launchers.
#pragma once
#include "common.h"
#include "gemm.h"

namespace psgdk {

struct EwArgs {
  int nb;
  long long m, n;          // matrix shape (rows, cols) of the operands
  long long ld;            // leading dimension of the (square) operand for tile kernels
  int dt;                  // storage dtype of `in` (0 fp32, 1 bf16)
  float f0, f1, f2, f3;    // kernel-specific host scalars
  int i0, i1;              // kernel-specific ints
  const void* in[MAXB];
  const float* in2[MAXB];
  const float* in3[MAXB];
  float* out[MAXB];
  void* out2[MAXB];
  float* sc[MAXB];         // device scalars
  float* aux[MAXB];        // kernel-specific extra output
  // noise kernels: draw = 1 generates the noise N instead of reading in2: problem b's element i is normal
  // doff[b] + i of the Philox4x32-10 sequence keyed (dk0, dk1) on counter words (ds0, ds1) (normal_fill_launch's)
  int draw;
  unsigned dk0, dk1, ds0, ds1;
  long long doff[MAXB];
};

// X = G + (damping + eps |G|) * N  (fp32 into out and / or bf16 into out2; N in G's dtype dt; N null: X = G)
// (psgd_pro.py:121-123);
// in3 (optional): a row scale applied to X (a diagonal P1 of P1 X P2)
hipError_t noise_launch(const EwArgs& a, hipStream_t st);
// out2 = bf16 (X diag(in3))^T with X as noise_launch (a diagonal P2 folded into the transposed operand of P1 X P2)
hipError_t noise_t_launch(const EwArgs& a, hipStream_t st);
// out[i] = sum_j X[i][j]^2 of a bf16 m x n matrix (a diagonal factor's term1 from the bf16 Pg or Pg^T)
hipError_t rowsq_launch(const EwArgs& a, hipStream_t st);
// R = Q^T - Q (sign = +1) or Q - Q^T (sign = -1), square d x d, plus an optional bf16 copy in out2
// (psgd_pro.py:87; psgd_pro_fast.py:147); aux (optional, with out2): per (row, 64-column block) sums of squares and
// maxima of |.| of the bf16 R, block-major: aux[cb d + i], then aux[T d + cb d + i] (T = ceil(d / 64))
hipError_t rform_launch(const EwArgs& a, hipStream_t st);
// Procrustes step size from the trace partials     (psgd_pro.py:91-93)
hipError_t proc_scalar_launch(const EwArgs& a, hipStream_t st);
// procrustes_step_r2 step size and the coefficients of M = a Rn + a^2/2 S   (psgd_pro_fast.py:141-153)
hipError_t proc_scalar_r2_launch(const EwArgs& a, hipStream_t st);
// M = c0 R + c1 S (bf16 or fp32, elementwise)       (psgd_pro_fast.py:153)
hipError_t mform_launch(const EwArgs& a, hipStream_t st);
// out = in * p_row[i] * p_col[j] (diagonal factors' P = q * q; null pointer = 1)
hipError_t diag_scale_launch(const EwArgs& a, hipStream_t st);
// diagonal factor term1: sums of squares along rows (i0 = 0) or columns (i0 = 1) of Pg  (psgd_pro.py:125-126)
hipError_t diag_term1_launch(const EwArgs& a, hipStream_t st);
// diagonal factor update: ell, L EMA, q *= 1 - lr/L (term1 - term2), P = q * q  (psgd_pro.py:127-130)
hipError_t diag_update_launch(const EwArgs& a, hipStream_t st);
// clip + parameter update from the sum-of-squares partials  (psgd_pro.py:371-381)
hipError_t clip_update_launch(const EwArgs& a, hipStream_t st);
// max |x| partials and scaling for balancing (psgd_pro.py:96-105)
hipError_t absmax_launch(const EwArgs& a, hipStream_t st);
hipError_t balance_scalar_launch(const EwArgs& a, hipStream_t st);
hipError_t scale_by_dev_launch(const EwArgs& a, hipStream_t st);
// m = beta m + (1 - beta) g                           (psgd_pro.py:340-341)
hipError_t momentum_launch(const EwArgs& a, hipStream_t st);
// The same for nb tensors of their own sizes and gradient dtypes in one launch: tensor t holds elements
// off[t] .. off[t + 1] - 1 of the concatenated index range.
struct MomList {
  int nb;
  int vec;                  // every m 16-byte and every g 16-byte (fp32) / 8-byte (bf16) aligned: 4 elements per access
  float beta;
  long long off[MAXB + 1];  // tensor t's elements at off[t] .. off[t] + n[t] of the concatenated range (off[t] a
                            // multiple of 4: each tensor's length is rounded up to 4 there)
  long long n[MAXB];
  int dt[MAXB];
  const void* g[MAXB];
  float* m[MAXB];
};
hipError_t momentum_multi_launch(const MomList& a, hipStream_t st);
// out[0 .. n) = standard normals (fp32 or bf16 storage, dt) from Philox4x32-10 keyed by seed on stream stream_id,
// four per counter value (Box-Muller); out 16-byte aligned for fp32, 8-byte for bf16
hipError_t normal_fill_launch(void* out, long long n, int dt, unsigned long long seed, unsigned long long stream_id,
                              hipStream_t st);
// sum of the split partials: out[i] = sum_s in[s * m * n + i]
hipError_t splitk_sum_launch(const EwArgs& a, hipStream_t st);
// sum-of-squares partials in the GEMM's EPI_SUMSQ format (i0 blocks per problem)
hipError_t sumsq_launch(const EwArgs& a, hipStream_t st);
// full symmetric matrix from the packed upper triangle
hipError_t unpack_launch(const EwArgs& a, hipStream_t st);
// bf16 copy (i0 = 0) or bf16 transposed copy (i0 = 1) of an fp32 (dt 0) or bf16 (dt 1) matrix with leading dimension
// ld into out2 (m x n, leading dimension n); with out set, the fp32 copy into out. i1 = 1 (with i0 = 0): the upper
// triangle only, zeros written below the diagonal without reading the input there
hipError_t to_bf16_launch(const EwArgs& a, hipStream_t st);

}  // namespace psgdk

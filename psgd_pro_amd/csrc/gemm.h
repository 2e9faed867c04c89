// MFMA GEMM engine: argument block shared by the host launcher and the kernels.
#pragma once
#include "common.h"

namespace psgdk {

constexpr int MAXB = 64;  // problems per grouped launch (pointer arrays in the kernel arguments, by value; the
                          // largest argument block, the norm bound's final stage, is about 8 KB)

// Epilogues. acc is op(A) op(B) accumulated in fp32; s = the problem's device scalars.
enum Epi : int {
  EPI_STORE = 0,   // C = alpha * acc + beta * C
  EPI_FACTOR = 1,  // C = X1 - s[0] * (acc - s[1] * X1)              (Q - lr/L (term1 Q - term2 Q))
  EPI_PROC = 2,    // C = X1 + a X2 + a^2/2 * s[1] * acc, a = s[0]    (Procrustes: Q + a RQ + a^2/2 R RQ)
  EPI_SCALE = 3,   // C = s[0] * acc
  EPI_RQ = 4,      // C = s[0] * acc and trace partials of tr(C), tr(s[0] X1 C) into part[]  (Procrustes RQ)
  EPI_SUMSQ = 5,   // C = alpha * acc and partial sums of C^2 into part[]                    (apply + clip stats)
  EPI_PROCB = 7,   // bf16 kernel only: EPI_PROC with X2 = (R Q)^T in bf16, row stride ldx (the transposed copy
                   // that is also the product's B operand), read at (col, row)
  EPI_STRACE = 6,  // SYRK only: C = (s[0] acc) s[0] (the scale applied twice, so that acc = 0 gives 0 for any
                   // finite s[0]), and partials of sum_ij C_ij X1_ij over the whole symmetric C into part[2 t + 1]
                   // (part[2 t] = 0)                                    (Procrustes r2: S = Rn^T Rn, sum(S * Q))
};

struct GemmArgs {
  int M, N, K;
  int amode, bmode;     // OpMode of A (rows m) and B (rows n), both viewed as X[mn][k]
  int asign, bsign;     // SYM sign
  long long lda, ldb, ldc, ldx;
  float alpha, beta;
  int epi;
  int tri;              // 1: upper-triangular tile grid (SYRK: M == N, B is A)
  int out_mode;         // tri: 0 upper triangle only, 1 mirrored full matrix, 2 packed upper triangle
  int tiles_m, tiles_n, ntiles;
  int avec, bvec;       // 16-byte vector loads allowed for A / B (alignment of base and ld)
  int kbeg_tri;         // A is upper-triangular (SYM, sign 0): start the k loop at the tile's first row
  int splitk, kchunk;   // split-K (EPI_STORE only): split s covers k in [s kchunk, (s+1) kchunk) and writes its
                        // partial product to C + s * M * ldc
  int nb;
  const void* A[MAXB];
  const void* B[MAXB];
  float* C[MAXB];
  const float* X1[MAXB];
  const float* X2[MAXB];
  const float* s[MAXB];
  float* part[MAXB];
};

}  // namespace psgdk

// bf16 MFMA GEMM with k-contiguous bf16 operands: argument block shared by the host launcher and the kernel.
#pragma once
#include "gemm.h"

namespace psgdk {

// C = op over acc = A B^T where A is M x K and B is N x K, both row-major bf16 with k contiguous (X[mn][k]).
// Outputs (each optional per launch): C (fp32, row-major, ldc), Cb (bf16, row-major, ldcb), CTb (bf16 of C^T,
// row-major N x M, ldct), CT (fp32 of C^T, ldct; the fp32 kernel). Epilogues as in gemm.h (EPI_STORE uses alpha only), except that EPI_RQ reads X1 (R) as
// bf16.
struct GB16Args {
  int M, N, K;
  long long lda, ldb, ldc, ldcb, ldct, ldx;
  float alpha;
  int epi;
  int tri, out_mode;  // tri: SYRK (B is A); out_mode 0 upper, 1 mirrored
  int tiles_m, tiles_n, ntiles, nb;
  int vec;            // 0: problem-major order (WG id = tile); 1: tiles dealt to XCDs in contiguous runs; 2: as 1,
                      // with tile rows grouped by 4 inside each problem
  int amc, bmc;       // fp32 kernel: A / B stored m- / n-contiguous (rows of the buffer are k; M / N a multiple of 4)
  int kbeg;           // 1: A is upper-triangular (A[i][k] = 0 for k < i, zeros stored): a tile of rows m0.. starts its
                      // k loop at the k tile holding m0 (TRMM)
  int kper;           // 1: problem b has its own K = kp[b], with lda = ldb = kp[b] (k-contiguous rows of exactly K)
  int kp[MAXB];
  const bf16_t* A[MAXB];
  const bf16_t* B[MAXB];
  float* C[MAXB];
  bf16_t* Cb[MAXB];
  bf16_t* CTb[MAXB];
  float* CT[MAXB];      // fp32 kernel: fp32 copy of C^T (row stride ldct)
  const float* X1[MAXB];
  const float* X2[MAXB];
  const float* s[MAXB];
  float* part[MAXB];
};

// cfg 0: 256 x 256 tiles (8 waves), cfg 1: 128 x 128 tiles (4 waves), cfg 2: 256 x 256 tiles (4 waves), cfg 3:
// 256 x 256 tiles (8 MFMA waves on 32 x 32 x 16 and 4 load-only waves), cfg 4: 128 x 128 tiles (4 MFMA waves on
// 32 x 32 x 16 and 4 load-only waves)
hipError_t gemm_bf16_launch(GB16Args& a, int cfg, hipStream_t st);
// The same kernel for k-contiguous fp32 operands (A, B reinterpreted as float; K, leading dimensions multiples of 4;
// always the 128-tile configuration, with k summed in blocks of 128; operands k-contiguous or, with amc / bmc,
// m- / n-contiguous; EPI_RQ reads R as fp32; every epilogue but EPI_PROCB, which reads a bf16 X operand)
hipError_t gemm_f32kc_launch(GB16Args& a, int cfg, hipStream_t st);
int gemm_bf16_tiles(long long M, long long N, int tri, int cfg);
// Small products (plain-store epilogue, k-contiguous operands, bf16 (esz 2) or fp32 (esz 4)): 64 x 64 tiles, k in
// chunks of 512 bytes per row with two chunks in flight (gemm_small.hip).
hipError_t gemm_small_launch(GB16Args& a, int esz, hipStream_t st);
int gemm_small_tiles(long long M, long long N, int tri);
// Tiny products (same contract): 32 x 32 tiles whose four waves split k, fragments loaded straight into registers;
// launches of more than 8 problems are split (gemm_small.hip).
hipError_t gemm_tiny_launch(const GB16Args& a, int esz, hipStream_t st);
int gemm_tiny_tiles(long long M, long long N, int tri);

}  // namespace psgdk

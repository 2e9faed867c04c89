// Norm lower bound stages: argument blocks shared by the host launchers and the kernels.
#pragma once
#include "common.h"
#include "gemm.h"

namespace psgdk {

constexpr int NLB_K = 32;  // rows of the random start V

// per-matrix device scalars (scal[b][...])
enum : int { NLB_NF = 0, NLB_J = 1, NLB_BOUND = 2, NLB_NSCAL = 4 };

struct NlbArgs {
  int nb, n, T, sign, splits;
  int ssc;                  // columns per sum-of-squares block of the V A outputs (64: split-K path, 128: full path)
  int vmm_u;                // full path: MFMA steps per load batch of the V A kernel (2, 4 or 8)
  int ksplit, kslice;       // full path: k slices per V A product and their length (a multiple of 64); part holds
                            // ksplit x 32 x n partial products
  int vmm_cols;             // full path: 1 = one workgroup per 64 output columns over the whole k range (no
                            // partials, ssc = 64); 2 = the same with A staged through LDS in row-contiguous
                            // runs; 3 = square bf16 matrices read from their upper 64-tiles in
                            // tournament-paired rounds (ssc = 64); 0 = split-K products plus a reduce kernel
                            // (ssc = 128)
  int kdim;                 // column kernel: k extent of a rectangular product (0: n)
  int vblk;                 // init and upper-tile kernels: V (32 x n) stored in 16-column blocks, element (r, c)
                            // at ((c / 16) 32 + r) 16 + c % 16, so that a wave's MFMA fragment of 32 rows x 16 k
                            // is one contiguous 1 KB (n a multiple of 16)
  int plain;                // column kernel: no row scale and no sums of squares
  int dot;                  // column and row kernels (square: kdim 0): the per-(row, column block) partials are
                            // sum_c W[r][c] * s_r Vin[r][c] (s_r the row scale) instead of sum_c W[r][c]^2: with A
                            // the Gram matrix H = P^T P of a factor P and X = s Vin, row r of X P^T has squared
                            // norm X_r H X_r^T = sum_c (X H)_rc X_rc
  long long lda;
  const float* A[MAXB];     // n x n, upper triangle read
  const float* Vin[MAXB];   // init: the random start (32 x n)
  float* Vout[MAXB];        // init: V0; reduce: the scaled product
  float* part[MAXB];        // reduce input: splits x 32 x n partial products
  const float* ssin[MAXB];  // reduce (normalize_in) / final: per-(row, column block) sums of squares of the input
  float* ssout[MAXB];       // reduce output sums of squares
  float* rpart[MAXB];       // T x T x 64 row-norm partials
  float* cpart[MAXB];       // T x 64 diagonal-tile column partials
  float* tmax[MAXB];        // per stored tile max |A_ij|
  float* dmax[MAXB];        // per stored tile max diagonal
  float* rn2[MAXB];         // n squared row norms
  float* scal[MAXB];        // NLB_NSCAL scalars
  float* amax_out[MAXB];    // optional: max |A_ij| of the stored triangle (init)
};

enum : int { NLB_FINAL_NONE = 0, NLB_FINAL_FACTOR = 1, NLB_FINAL_SCALE = 2 };

struct NlbFinal {
  int mode;
  float lr, beta;
  float term2[MAXB];  // factor: numel / d of each problem
  float* L[MAXB];     // factor: the smoothness EMA (1 float)
  float* coef[MAXB];  // factor: {lr / L, term2}; scale: {1 / (bound + smallest normal)}
};

// The norm bound of term1 = P P^T (d x d) from its factor P (d x k bf16 rows, k contiguous), without forming term1:
// the statistics the init kernel reads and row j of P P^T.
struct GramArgs {
  int nb, d, k;
  const bf16_t* P[MAXB];  // d x k, row stride k
  const bf16_t* W[MAXB];  // d x k: P H with H = P^T P (row stride k)
  float* rn2[MAXB];       // out: squared row norms of P P^T
  float* rmax[MAXB];      // out: zero (the row maxima are read by skew bounds only)
  float* diag[MAXB];      // out: the diagonal of P P^T
  float* scal[MAXB];      // NLB scalars: the argmax kernel writes NLB_J
  bf16_t* aj[MAXB];       // out: row j of P P^T (d values)
};
// stage 0: rn2 = rowsum(W * P), diag = rowsum(P * P); 1: argmax of rn2 (first maximum) into scal; 2: aj
hipError_t gram_launch(const GramArgs& a, int stage, hipStream_t st);

hipError_t nlb_rownorm_launch(const NlbArgs& a, hipStream_t st);
hipError_t nlb_init_launch(const NlbArgs& a, hipStream_t st);
hipError_t nlb_reduce_launch(const NlbArgs& a, int normalize_in, hipStream_t st);
hipError_t nlb_final_launch(const NlbArgs& a, const NlbFinal& f, hipStream_t st);
// fully stored matrices: stage 0 row norms (rn2, rpart = row max |A|, cpart = diagonal), 1 init, 2 one V A product,
// 3 the stage-0 outputs of a skew matrix from the per-(row, 64-column block) partials its producer left in part
hipError_t nlb_full_launch(const NlbArgs& a, int stage, int a_bf16, int normalize, hipStream_t st);
hipError_t gemm_launch(GemmArgs& a, int prec, int adt, int bdt, int cfg, hipStream_t st);
hipError_t debug_mfma_launch(const float* A, const float* B, float* C, int prec, hipStream_t st);

}  // namespace psgdk

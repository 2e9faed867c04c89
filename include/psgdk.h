/* psgdk: MI355X (gfx950) kernels for the PSGD-Kron preconditioner update + gradient apply.
 *
 * C ABI. Every pointer argument named as device memory is a device address (HIP), every array of pointers
 * (`const T* const* X`, one entry per problem of a grouped call) is a HOST array of `nb` device addresses. All
 * matrices are row-major with the given leading dimension (elements). Outputs are caller-allocated. Work is enqueued
 * on `stream` (NULL = the default stream); no call synchronizes the host, allocates device memory or frees caller
 * memory. Calls that need scratch memory take (ws, ws_bytes): with ws == NULL they only store the required size in
 * *ws_bytes and return PSGDK_OK; otherwise *ws_bytes must be at least that size.
 * Return value: PSGDK_OK or an error code; psgdk_last_error() describes the last error of the calling thread.
 *
 * Precision: prec = PSGDK_PREC_F32 multiplies fp32 inputs on the fp32 MFMA path; PSGDK_PREC_BF16 rounds the inputs
 * of every contraction to bfloat16 (round to nearest even) and multiplies on the bf16 MFMA path. Accumulation and
 * all outputs are fp32 in both cases. Operand storage dtypes (PSGDK_F32 / PSGDK_BF16) are independent of prec.
 *
 * Each entry point names the reference interface (dlyr3/psgd_pro, file:line) whose role it takes.
 */
#ifndef PSGDK_H
#define PSGDK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* psgdk_stream_t; /* hipStream_t */
typedef struct ihipEvent_t* psgdk_event_t;   /* hipEvent_t */

#define PSGDK_VERSION 4
#define PSGDK_MAXB 16 /* problems per grouped call */
#define PSGDK_MAX_GROUPS 64 /* groups per psgdk_kron2d_update_groups call */
#define PSGDK_NLB_K 32 /* rows of the random start of the norm lower bounds */

enum { PSGDK_OK = 0, PSGDK_EINVAL = 1, PSGDK_ESHAPE = 2, PSGDK_EHIP = 3, PSGDK_EWORKSPACE = 4 };
enum { PSGDK_F32 = 0, PSGDK_BF16 = 1 };
enum { PSGDK_PREC_F32 = 0, PSGDK_PREC_BF16 = 1 };
enum { PSGDK_OUT_UPPER = 0, PSGDK_OUT_MIRROR = 1, PSGDK_OUT_PACKED = 2 };
enum { PSGDK_FACTOR_NONE = 0, PSGDK_FACTOR_DIAG = 1, PSGDK_FACTOR_DENSE = 2 };

/* Message of the calling thread's last error ("" if none). */
const char* psgdk_last_error(void);
/* PSGDK_VERSION of the library. */
int psgdk_version(void);

/* ---------------------------------------------------------------------------------------------------------------
 * Level 1: the kernels behind the reference's custom ops (kernels/ops.py:24-116).
 * ------------------------------------------------------------------------------------------------------------ */

/* C = A A^T (trans = 0, A is n x k) or A^T A (trans = 1, A is k x n), computing only the upper-triangle tiles.
 * out_mode PSGDK_OUT_UPPER writes the upper triangle (the strict lower triangle of C is not touched),
 * PSGDK_OUT_MIRROR the full symmetric matrix, PSGDK_OUT_PACKED the row-major packed upper triangle
 * (n(n+1)/2 values, row i at i n - i(i-1)/2; ldc ignored).
 * Replaces cublasSsyrk (kernels/blas.cpp:21-33, psgd::syrk_cublas kernels/ops.py:55-63) and the Triton SYRKs
 * psgd::syrk / syrk2 / syrk2p (kernels/ops.py:66-109, kernels/k2.py:17-39,48-85,106-137). */
int psgdk_syrk(int prec, int trans, int out_mode, int64_t n, int64_t k, int a_dtype, int nb,
               const void* const* A, int64_t lda, float* const* C, int64_t ldc, psgdk_stream_t stream);

/* Symmetric matmul reading S (n x n) from its upper triangle only (the strict lower triangle is never read):
 * side 0: C (n x p) = S B with B n x p;  side 1: C (p x n) = B S with B p x n.
 * sign +1: S symmetric; -1: S skew-symmetric (diagonal taken as 0); 0: S upper-triangular (TRMM, see below).
 * Replaces cublasSsymm side-right / side-left (kernels/blas.cpp:36-65; psgd::symm, psgd::symm_right
 * kernels/ops.py:45-52,90-97). */
int psgdk_symm(int prec, int side, int sign, int64_t n, int64_t p, int b_dtype, int nb, const float* const* S,
               int64_t lds, const void* const* B, int64_t ldb, float* const* C, int64_t ldc, psgdk_stream_t stream);

/* C (n x p) = triu(Q) B: Q's strict lower triangle is neither read nor multiplied (k loop starts at the tile's
 * first row). No reference counterpart beyond the triangle-reading SYMM above; the literal triangular product of
 * the microbenchmark specification. */
int psgdk_trmm(int prec, int64_t n, int64_t p, int b_dtype, int nb, const float* const* Q, int64_t ldq,
               const void* const* B, int64_t ldb, float* const* C, int64_t ldc, psgdk_stream_t stream);

/* psgdk_trmm with a workspace: the operands are converted once (triu(Q) with zeros below the diagonal, and for
 * prec bf16 B^T, in bf16) and multiplied on the k-contiguous MFMA kernel, each output tile's k loop starting at the
 * diagonal (n(n+1)p flops in place of 2 n^2 p). Needs n and p multiples of 8 (bf16) or 4 (fp32, with fp32 B and n
 * > 32); other shapes take psgdk_trmm and need no workspace. Q's strict lower triangle is never read. */
int psgdk_trmm_ws(int prec, int64_t n, int64_t p, int b_dtype, int nb, const float* const* Q, int64_t ldq,
                  const void* const* B, int64_t ldb, float* const* C, int64_t ldc, void* ws, size_t* ws_bytes,
                  psgdk_stream_t stream);

/* C (m x n) = alpha op(A) op(B) + beta C, op(X) = X (trans = 0) or X^T (trans = 1); A is m x k (or k x m),
 * B is k x n (or n x k). The dense contractions of the reference's hot path that have no custom kernel there
 * (R @ Q and R @ RQ in procrustes_step2, psgd_pro.py:89-90; term1 @ q, psgd_pro.py:135; the exprP chain,
 * psgd_pro.py:112,123). */
int psgdk_gemm(int prec, int trans_a, int trans_b, int64_t m, int64_t n, int64_t k, float alpha, int a_dtype,
               int b_dtype, int nb, const void* const* A, int64_t lda, const void* const* B, int64_t ldb, float beta,
               float* const* C, int64_t ldc, psgdk_stream_t stream);

/* Squared row norms rn2 (n) and max |A_ij| (*amax, one float per problem) of the symmetric (sign +1) or
 * skew-symmetric (sign -1) matrix held in the upper triangle of A (n x n, fp32).
 * Replaces psgd::tri_rownorm2 (kernels/ops.py:34-42, kernels/k1.cu:84-181,297-307). */
int psgdk_tri_rownorm2(int64_t n, int sign, int nb, const float* const* A, int64_t lda, float* const* rn2,
                       float* const* amax, void* ws, size_t* ws_bytes, psgdk_stream_t stream);

/* W (32 x n) = V A_sym, V 32 x n contiguous fp32, A_sym read from the upper triangle of A (sign as above).
 * Replaces psgd::tri_vmm (kernels/ops.py:24-31, kernels/k1.cu:189-268,282-294). */
int psgdk_tri_vmm(int64_t n, int sign, int nb, const float* const* V, const float* const* A, int64_t lda,
                  float* const* W, void* ws, size_t* ws_bytes, psgdk_stream_t stream);

/* Norm lower bound of the SPD (sign +1) or skew-symmetric (sign -1) matrix held in the upper triangle of A, with
 * the random start V (32 x n) passed in; out[b] (device, one float) receives the bound. Computed entirely on the
 * device (no host synchronization).
 * Replaces norm_lower_bound_spd / _skh (psgd_pro.py:19-65, psgd_pro_fast.py:32-51) and nlb_tri
 * (kernels/ops.py:124-136, kernels/k1.py:19-33). */
int psgdk_norm_lower_bound(int64_t n, int sign, int nb, const float* const* A, int64_t lda, const float* const* V,
                           float* const* out, void* ws, size_t* ws_bytes, psgdk_stream_t stream);

/* Norm lower bound of the fully stored SPD (sign +1) or skew-symmetric (sign -1) n x n matrix A (row-major, lda;
 * a_dtype PSGDK_F32 or PSGDK_BF16; both triangles stored: the row-norm pass reads both, and with bf16 storage and
 * n a multiple of 128 the products V A may read the upper 64 x 64 tiles only, option 4), random start V (32 x n
 * fp32); out[b] (device, one float) receives the bound. With bf16 storage the products V A run in bf16 with fp32
 * accumulation.
 * Replaces norm_lower_bound_spd / _skh (psgd_pro.py:19-41, :43-65) on full matrices. */
int psgdk_norm_lower_bound_full(int64_t n, int sign, int nb, const void* const* A, int64_t lda, int a_dtype,
                                const float* const* V, float* const* out, void* ws, size_t* ws_bytes,
                                psgdk_stream_t stream);

/* psgdk_norm_lower_bound_full without the workspace arguments, for callers that cannot allocate device memory
 * (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc). No counterpart in the reference.
 * Scratch comes from a static device array of PSGDK_NOALLOC_SCRATCH_MIB MiB that each GPU the library runs on holds
 * until the process ends; a call allocates nothing. A problem whose workspace (the size psgdk_norm_lower_bound_full
 * reports) exceeds the array is refused with PSGDK_ESHAPE (e.g. n = 3072 fits up to nb = 4 bf16 matrices). Every
 * call on one GPU shares that GPU's array, which keeps the last call's contents: calls that overlap on one GPU (two
 * streams, or two host threads) race. */
#define PSGDK_NOALLOC_SCRATCH_MIB 32
int psgdk_norm_lower_bound_full_noalloc(int64_t n, int sign, int nb, const void* const* A, int64_t lda, int a_dtype,
                                        const float* const* V, float* const* out, psgdk_stream_t stream);

/* norm_lower_bound_spd (psgd_pro.py:19-41) of P P^T (d x d) given P (d x k bf16, rows k-contiguous) and Pt = P^T
 * (k x d bf16), without forming P P^T: the squared row norms come from P (P^T P), the diagonal from the rows of P,
 * row j from P P_j^T. The subspace iteration runs in k-space: with X = V P, the product V (P P^T) is (X H) P^T for
 * H = P^T P (k x k), and row r of V has squared norm X_r H X_r^T. So the start V0 is multiplied by P once and the
 * four products are k x k products with H. The bound the bf16 update takes for term1 = Pg Pg^T or Pg^T Pg when the
 * other side k is under half of d. d and k multiples of 8, 16-byte aligned operands. */
int psgdk_norm_lower_bound_gram(int64_t d, int64_t k, int nb, const void* const* P, const void* const* Pt,
                                const float* const* V, float* const* out, void* ws, size_t* ws_bytes,
                                psgdk_stream_t stream);

/* Full symmetric n x n matrix from its row-major packed upper triangle.
 * Replaces psgd::unpack (kernels/ops.py:112-116, kernels/k2.py:88-103). */
int psgdk_unpack(int64_t n, int nb, const float* const* Pk, float* const* C, int64_t ldc, psgdk_stream_t stream);

/* ---------------------------------------------------------------------------------------------------------------
 * Level 2: the optimizer step over a group of same-shape parameters. A parameter is viewed as an m x n gradient
 * (a vector as 1 x n, a scalar as 1 x 1) with one factor kind per dimension.
 * ------------------------------------------------------------------------------------------------------------ */

typedef struct psgdk_kron2d {
  int32_t nb;                /* parameters in the group, 1..PSGDK_MAXB */
  int32_t prec;              /* PSGDK_PREC_* of the contractions */
  int64_t m, n;              /* gradient shape (row-major, contiguous) */
  int32_t kind[2];           /* PSGDK_FACTOR_* of dimension 0 (rows) and 1 (columns) */
  int32_t g_dtype;           /* storage dtype of G */
  int32_t p_dtype;           /* storage dtype of the parameters (apply) */
  const void* G[PSGDK_MAXB]; /* gradient (or momentum) m x n */
  float* Q[2][PSGDK_MAXB];   /* dense: d x d; diagonal: d values; none: unused */
  float* P[2][PSGDK_MAXB];   /* Q^T Q (dense: full symmetric, or upper triangle with tri bit 1) or q * q */
  float* L[2][PSGDK_MAXB];   /* one float each: the factor's Lipschitz smoothness EMA */
  /* bf16 shadows of dense factors for prec = PSGDK_PREC_BF16 (optional: NULL selects the general path): Qt16 is
   * Q^T and P16 is P in bfloat16, d x d row-major. The library keeps them in step with Q (update, refresh,
   * balance); psgdk_kron2d_refresh_p rebuilds both from the fp32 state. With shadows (and tri = 0) the update
   * refreshes only P16, the copy its readers use; fp32 P is current after psgdk_kron2d_refresh_p and
   * psgdk_kron2d_balance, so a caller that reads P between them calls psgdk_kron2d_refresh_p first. */
  void* Qt16[2][PSGDK_MAXB];
  void* P16[2][PSGDK_MAXB];
} psgdk_kron2d_t;

typedef struct psgdk_update_opts {
  float lr;       /* lr_preconditioner */
  float betaL;
  float damping;
  float grad_eps; /* eps of the damping scale (torch.finfo(gradient dtype).eps in the reference) */
  int32_t tri;    /* bit 0: term1 kept as its upper triangle; bit 1: P kept as its upper triangle */
  int32_t r2;     /* 0: procrustes_step2 (psgd_pro.py:71-94); 1: procrustes_step_r2 (psgd_pro_fast.py:141-153) */
} psgdk_update_opts_t;

typedef struct psgdk_apply_opts {
  float lr_params;
  float max_avg_amp;     /* grad_clip_max_amps[0] */
  float max_element_amp; /* grad_clip_max_amps[1] */
  int32_t tri;           /* bit 1: P kept as its upper triangle */
} psgdk_apply_opts_t;

/* One preconditioner update of every parameter in the group: update_2d (psgd_pro_fast.py:168-192), i.e.
 * update_precond_kron_whiten_q0p5eq1p5 (psgd_pro.py:114-137) with P = Q^T Q cached: Pg = P1 (G + (damping +
 * grad_eps |G|) noise) P2; per factor: term1 (SYRK or sums of squares), norm lower bound, L EMA, Q update,
 * Procrustes rotation (psgd_pro.py:71-94); then P refresh. Draws are passed in: noise[b] is m x n N(0,1) stored in
 * the gradient's dtype (g_dtype), as randn_like(G) draws it (psgd_pro_fast.py:202); V[b] (fp32) holds, per dense
 * factor in dimension order, two 32 x d blocks (the SPD bound's start, then the skew bound's).
 * The balancing coin (psgd_pro.py:138-139) is the caller's (psgdk_kron2d_balance). */
int psgdk_kron2d_update(const psgdk_kron2d_t* g, const psgdk_update_opts_t* o, const void* const* noise,
                        const float* const* V, void* ws, size_t* ws_bytes, psgdk_stream_t stream);

/* The update of several groups in one call: the same operation as psgdk_kron2d_update on each group, with the
 * factor work of all groups batched by factor side (each launch covers up to 64 factors of one side, from any
 * group and either dimension). Every group must be on the bf16 path (prec bf16, two factors, dense or diagonal with
 * at least one dense, every dense factor with its Qt16 / P16 shadows, sides multiples of 8, tri = 0); lr, betaL,
 * r2 and tri must agree across opts[]; damping and grad_eps
 * are per group. noise[g] and V[g] are the group's arrays as in psgdk_kron2d_update. Each factor goes through the
 * operations of psgdk_kron2d_update; a launch that batches more problems may take another tile configuration or k
 * split (the size rule looks at the whole launch), which changes only the order of the sums, so the results match
 * one psgdk_kron2d_update per group to the bf16 path's rounding (bitwise where the launches take the same
 * configurations). The work runs on side streams the library creates once per device (default priority;
 * psgdk_set_option 6), forked from and joined back to `stream` with events (concurrent calls from several host
 * threads take turns on them); while `stream` is being captured into a HIP graph, everything runs on `stream`
 * itself. Results do not depend on the number of side streams. Replaces the per-parameter
 * loop of update_2d calls
 * (psgd_pro_fast.py:351-368; the reference's batch=True stacks same-shape parameters, psgd_pro_fast.py:327-349). */
int psgdk_kron2d_update_groups(int ngroups, const psgdk_kron2d_t* const* groups,
                               const psgdk_update_opts_t* const* opts, const void* const* const* noise,
                               const float* const* const* V, void* ws, size_t* ws_bytes, psgdk_stream_t stream);
/* psgdk_kron2d_update_groups that also records, for each group g with group_done[g] non-NULL, the caller's event
 * group_done[g] once that group's factors, L, P and bf16 shadows are final (the batches holding its factors done),
 * so that work on one group (its balance and apply) can start while other groups' batches still run. The call still
 * joins all its work back to `stream`. Events are created by the caller (hipEventCreate) and re-recorded by every
 * call. No counterpart in the reference (its per-parameter loop runs in order, psgd_pro_fast.py:351-368). */
int psgdk_kron2d_update_groups_ev(int ngroups, const psgdk_kron2d_t* const* groups,
                                  const psgdk_update_opts_t* const* opts, const void* const* const* noise,
                                  const float* const* const* V, void* ws, size_t* ws_bytes, psgdk_stream_t stream,
                                  psgdk_event_t const* group_done);

/* A group's noise drawn inside the update instead of read from a buffer: problem b's m x n noise (row-major) is
 * the normals offset[b] .. offset[b] + m n - 1 of the sequence psgdk_fill_normal(.., seed, stream_id, ..) writes,
 * rounded to the group's g_dtype as that call rounds them, so the update equals, bit for bit, the one that reads a
 * buffer filled by psgdk_fill_normal at those offsets. offset[b] >= 0, a multiple of 4. */
typedef struct psgdk_draws {
  uint64_t seed;
  uint64_t stream_id;
  int64_t offset[PSGDK_MAXB];
} psgdk_draws_t;

/* psgdk_kron2d_update_groups_ev where each group takes its noise either from noise[g] (device pointers, as there)
 * or, with noise NULL or noise[g] NULL, from draws[g]: the normals are generated by the kernel that forms the
 * noisy gradient, so the step writes and reads no noise buffer. group_done may be NULL (no events). Replaces
 * psgd_pro.py:123 / psgd_pro_fast.py:200-206 (torch.randn_like(G) into memory, then G + (damping + eps |G|) V). */
int psgdk_kron2d_update_groups_drawn(int ngroups, const psgdk_kron2d_t* const* groups,
                                     const psgdk_update_opts_t* const* opts, const void* const* const* noise,
                                     const psgdk_draws_t* const* draws, const float* const* const* V, void* ws,
                                     size_t* ws_bytes, psgdk_stream_t stream, psgdk_event_t const* group_done);

/* Precondition, clip and update: pre = P1 G P2 (apply_2d, psgd_pro_fast.py:156-161 = precond_grad_kron,
 * psgd_pro.py:107-112), clip to RMS <= max_avg_amp and |.| <= max_element_amp, param -= lr_params * clipped
 * (psgd_pro.py:371-381). pre_out[b] / clipped_out[b] (m x n fp32, optional: NULL array or NULL entries) receive
 * the unclipped and clipped gradients. */
int psgdk_kron2d_apply(const psgdk_kron2d_t* g, const psgdk_apply_opts_t* o, void* const* params,
                       float* const* pre_out, float* const* clipped_out, void* ws, size_t* ws_bytes,
                       psgdk_stream_t stream);

/* One dense factor update per problem given its term1 (full symmetric d x d fp32, or its upper triangle with
 * term1_tri): ell = norm_lower_bound_spd(term1, V) + term2, L = max(betaL L + (1 - betaL) ell, ell) (L: one
 * device float each, updated), Q_out = Q - lr/L (term1 Q - term2 Q), Q_out not aliasing Q. prec PSGDK_PREC_F32
 * or _BF16 (MFMA inputs). Replaces the factor update of update_precond_kron_whiten_q0p5eq1p5 (psgd_pro.py:132-135,
 * psgd_pro_fast.py:186-189). */
int psgdk_factor_update(int prec, int64_t d, int nb, const float* const* term1, int term1_tri,
                        const float* const* Q, float* const* Q_out, float* const* L, const float* const* V, float lr,
                        float betaL, float term2, void* ws, size_t* ws_bytes, psgdk_stream_t stream);

/* Q_out = procrustes_step2(Q) (psgd_pro.py:71-94; psgd_pro_fast.py:129-138): R = Q^T - Q normalized by
 * norm_lower_bound_skh(R, V) + smallest normal, a = min(-tr(RQ)/tr(RRQ), 1/8) when tr(RRQ) < 0 else 1/8,
 * Q_out = Q + a (RQ + a/2 RRQ), all on the device. Q_out must not alias Q (the reference updates in place). */
int psgdk_procrustes(int prec, int64_t d, int nb, const float* const* Q, float* const* Q_out, const float* const* V,
                     void* ws, size_t* ws_bytes, psgdk_stream_t stream);

/* Q_out = procrustes_step_r2(Q) (psgd_pro_fast.py:141-153): the same rotation with R R formed once by a symmetric
 * rank-d product (3 d^3 flops instead of 4 d^3): Rn = Q - Q^T normalized by its skew norm bound, S = Rn^T Rn,
 * tr(RQ) = sum(Rn * Q), tr(RRQ) = -sum(S * Q), Q_out = Q - (a Rn + a^2/2 S) Q. Arguments as psgdk_procrustes. */
int psgdk_procrustes_r2(int prec, int64_t d, int nb, const float* const* Q, float* const* Q_out,
                        const float* const* V, void* ws, size_t* ws_bytes, psgdk_stream_t stream);

/* apply_2d + clip + update (psgd_pro_fast.py:156-161,426-438): the same operation as psgdk_kron2d_apply. */
int psgdk_apply2d(const psgdk_kron2d_t* g, const psgdk_apply_opts_t* o, void* const* params, float* const* pre_out,
                  float* const* clipped_out, void* ws, size_t* ws_bytes, psgdk_stream_t stream);

/* P = Q^T Q (dense) or q * q (diagonal) for the factors selected by factor_mask (bit f = factor f):
 * gram_2d (psgd_pro_fast.py:164-165,191-192,447-449). tri bit 1: P written as its upper triangle. With bf16
 * shadows, Qt16 = bf16(Q^T) is rebuilt first and P16 written with P. */
int psgdk_kron2d_refresh_p(const psgdk_kron2d_t* g, int factor_mask, int tri, psgdk_stream_t stream);

/* Balance the factors of the parameters whose flag is set (host array of nb ints): q_f *= gmean / max|q_f|,
 * gmean = (prod_f max|q_f|)^(1/order) over the group's non-NONE factors, then refresh their P
 * (balance_kron_precond, psgd_pro.py:96-105; psgd_pro_fast.py:390-397). */
int psgdk_kron2d_balance(const psgdk_kron2d_t* g, const int32_t* flags, int tri, void* ws, size_t* ws_bytes,
                         psgdk_stream_t stream);

/* m = beta m + (1 - beta) g for nb tensors of numel elements (psgd_pro.py:340-341). */
int psgdk_momentum(int64_t numel, float beta, int g_dtype, int nb, float* const* mom, const void* const* g,
                   psgdk_stream_t stream);

/* The same update for nb (1 .. 64) tensors of their own element counts numel[t] and gradient dtypes g_dtype[t]
 * (host arrays), in one launch: the momentum EMA of every parameter of an optimizer step at once
 * (psgd_pro.py:340-341 loops over the parameters). Each element's arithmetic is psgdk_momentum's. */
int psgdk_momentum_multi(int nb, const int64_t* numel, float beta, const int32_t* g_dtype, float* const* mom,
                         const void* const* g, psgdk_stream_t stream);

/* out[0 .. n) = standard normal samples (fp32 or bf16 storage, dtype) from the counter-based Philox4x32-10
 * generator (Salmon et al., SC 2011) keyed by seed on stream stream_id, through the Box-Muller transform (fp32 with
 * the hardware log2, square root, sine and cosine: within 2e-5 (1 + |z|) of the exact transform): element i
 * depends only on (seed, stream_id, i), so a call is reproducible and calls with different (seed, stream_id) are
 * independent. The device draws of an optimizer step (the noise and the norm bounds' random starts, which
 * psgd_pro_fast.py:200-206 and 482-483 draw with torch.randn on the device). out: 16-byte aligned (fp32) or 8-byte
 * (bf16). */
int psgdk_fill_normal(void* out, int64_t n, int dtype, uint64_t seed, uint64_t stream_id, psgdk_stream_t stream);

/* Launch profiling (diagnostic, per host thread): after psgdk_profile_start every MFMA-engine launch the thread makes is
 * bracketed by a pair of HIP events on its stream. psgdk_profile_stop ends the recording and, with out non-NULL,
 * waits for the recorded events and fills one record per launch: the kernel instantiation id
 * (general engine: cfg * 1000 + prec * 100 + a_dtype * 10 + b_dtype, cfg 0 = 128 x 128 tiles, 1 = 32 x 128;
 * bf16 engine: 5000 + cfg * 10 + epilogue, cfg as option 1 below, epilogue 0 = store, 1 = factor update, 2 = Procrustes
 * step, 3 = scale, 4 = R Q with its trace partials, 5 = store with sums of squares, 6 = the r2 trace SYRK's scale
 * applied twice, 7 = Procrustes step reading (R Q)^T in bf16;
 * its fp32 twin: 6000 + cfg * 10 + epilogue; the small-problem kernels: 7000 / 7001 on 64 x 64 tiles, 7002 / 7003
 * the tiny-product kernel, bf16 / fp32 operands), whether it was a
 * SYRK (triangular grid), the problems in the launch, its device time, its algorithmic flop count (SYRK n(n+1)k,
 * TRMM n(n+1)p, GEMM 2mnk, per problem) and its algorithmic bytes (operands read once, outputs written once). With out NULL only *n_records is set (records kept). */
typedef struct psgdk_prof_record {
  int32_t kernel_id;
  int32_t tri;
  int32_t nb;
  float ms;
  double flops;
  double bytes; /* algorithmic HBM bytes: each operand read once, each output written once, epilogue reads */
  int64_t m, n, k;    /* each problem's output rows and columns (a SYRK: n = m) and k extent (the largest one) */
  int32_t workgroups; /* workgroups launched */
  int32_t per_cu;     /* workgroups of this kernel that one CU holds at once (HIP's occupancy query; 0 unknown) */
} psgdk_prof_record_t;
int psgdk_profile_start(void);
int psgdk_profile_stop(psgdk_prof_record_t* out, int max_records, int* n_records);

/* Tuning switches, one set per host thread (a thread's settings apply to the calls it makes and never change
 * another thread's results; a new thread starts from the defaults, so a switch set on one thread does not reach
 * calls that other threads make, such as a framework's worker threads): option 0 = tile order of the bf16 kernel (0 problem-major, 1 contiguous runs per
 * XCD, 2 = 1 with tile rows grouped by 4 so that the tiles an XCD runs at once share operand panels; default 2);
 * option 1 = its tile configuration (-1 chosen by size, 0 = 256 x 256 on 8 waves, 1 = 128 x 128, 2 = 256 x 256 on 4
 * waves, 3 = 256 x 256 on 8 MFMA waves fed by 4 load-only waves, 4 = 128 x 128 on 4 MFMA waves fed by 4 load-only
 * waves; other values are refused); option 2 = workgroups
 * per split-K V A product of the norm lower bound (default 1024); option 3 = MFMA steps per load batch of the V A
 * kernels (2, 4 or 8; default 4; the column-block kernel takes 2 or 4); option 4 = the V A kernel of full-storage
 * norm bounds (-1 by shape: 3 for bf16 launches of at least 16 matrices and 512 workgroups, else 2; 0 split-K products plus a reduce kernel, 1 one workgroup
 * per 64 output columns over the whole k range, 2 the same with A staged through LDS in row-contiguous runs, 3 bf16
 * matrices of an even number of 64-tiles read from their upper tiles only, in tournament-paired rounds (else as 2);
 * shapes the column kernels cannot read take the split-K kernel); option 5 = how the bf16 update
 * forms term1 Q for a factor whose other side m is under half of its side d (1, default: Pg^T (Pg Q) or Pg (Pg^T Q),
 * 4 m d^2 flops; 0: term1 Q, 2 d^3 flops); option 6 = side streams of psgdk_kron2d_update_groups (default 3; 0 or
 * 1: everything on the caller's stream); option 7 = whether the bf16 update keeps R Q (the Procrustes correction)
 * in bf16 (1, default: only the bf16 (R Q)^T, which the Q update also reads) or fp32 (0) between its two
 * products; option 8 = whether fp32 products with k- or m/n-contiguous operands (M > 32, one k range, no packed
 * output) take the k-contiguous kernel's fp32 twin (1, default) or the general engine (0); option 9 = the most
 * factors of one side >= 2048 that psgdk_kron2d_update_groups batches into one launch (1 .. 64, default 64; smaller
 * batches of one side run on different side streams); option 10 = plain-store bf16 GEMMs on k-contiguous operands
 * whose launch has fewer 128 x 128 tiles than this take the small-problem kernel (64 x 64 tiles, k in chunks of 512
 * bytes per row with two in flight); bf16 SYRKs below 1.5 times it and fp32 products below 3 times it (default 128,
 * 0: never; not with a forced tile configuration, option 1); option 11 = of those, a launch with fewer 64 x 64 tiles
 * than this takes the tiny-product kernel (32 x 32 tiles whose four waves split k; results rounded in another
 * order than the other kernels' k-order sums; default 64, 0: never); option 12 = whether launches given 256 x 256
 * or 128 x 128 tiles by size take the configurations with load-only waves (option 1 values 3 and 4) rather than 0
 * and 1, except launches with epilogues 1, 2, 6 and 7 of the profiling ids above (the factor update, both Procrustes
 * steps and the r2 trace SYRK), whose registers spill in configuration 3 (three waves per SIMD) and in configuration 4
 * exceed the 128 of two workgroups per CU (1, default; 0: never). On gfx950
 * configurations 0, 1, 3 and 4 round the same sums (their k steps of 32 and 16 accumulate in one order:
 * bitwise-equal products). */
int psgdk_set_option(int option, int value);
/* The calling thread's value of a psgdk_set_option switch. */
int psgdk_get_option(int option, int* value);

/* Measurement (no counterpart in the reference): wgs workgroups of 4 waves, each wave issuing iters x 32
 * independent bf16 MFMAs of 16 x 16 x 32 (16384 flops each) with no memory traffic; out receives one float per wave
 * (4 wgs). Timed at two workgroups per CU it gives the bf16 MFMA rate the GPU sustains at its current clock, the
 * ceiling a kernel can reach there. */
int psgdk_mfma_rate(int iters, int wgs, float* out, psgdk_stream_t stream);

/* Measurement (no counterpart in the reference): wgs workgroups of 256 threads, each reading iters blocks of 4 KiB
 * of buf (device memory of `bytes` bytes, a power of two >= 4096): block (workgroup * iters + i) * stride, wrapped
 * into the buffer. stride 1 with wgs * iters * 4096 = bytes reads the buffer once (the HBM read rate when it is far
 * larger than the caches); an odd stride over a small buffer gives the cache read rate. sink: device memory of wgs
 * uint32 (practically never written). */
int psgdk_read_rate(const void* buf, int64_t bytes, int wgs, int iters, int64_t stride, uint32_t* sink,
                    psgdk_stream_t stream);

/* Measurement (no counterpart in the reference): one wave that, `samples` times, sleeps about 8 thousand cycles and
 * then writes the cycle counter (out[2 i]) and the constant-rate wall counter (out[2 i + 1]; its rate is the
 * device's hipDeviceAttributeWallClockRate). Launched on a stream of its own next to other work, it gives the engine
 * clock while that work runs. out: device memory of 2 * samples uint64. */
int psgdk_clock_sample(int samples, uint64_t* out, psgdk_stream_t stream);
/* Measurement: the wall counter's rate of the current device in kHz (hipDeviceAttributeWallClockRate; host query). */
int psgdk_wall_clock_rate(int* khz);
/* Measurement: out[0] = the wall counter when `stream` reaches this call (marks the ends of a timed region). */
int psgdk_wall_mark(uint64_t* out, psgdk_stream_t stream);

/* Debug: one MFMA with operands placed by the lane layout the kernels assume (A 16 x K, B K x 16 row-major fp32,
 * K = 32 for bf16, 4 for fp32), C (16 x 16) = A B; prec 2: the 32 x 32 x 16 bf16 shape (A 32 x 16, B 16 x 32,
 * C 32 x 32). Checks the compiler builtins' lane layout. */
int psgdk_debug_mfma(int prec, const float* A, const float* B, float* C, psgdk_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* PSGDK_H */

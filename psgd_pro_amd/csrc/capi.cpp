// The C ABI (include/psgdk.h): argument validation, workspace layout and the sequencing of the grouped kernel
// launches of each stage. Host code only; every launch goes to the caller's stream, nothing synchronizes.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/psgdk.h"
#include "elem.h"
#include "gemm.h"
#include "gemm_bf16.h"
#include "nlb.h"

namespace psgdk {
hipError_t gemm_launch(GemmArgs& a, int prec, int adt, int bdt, int cfg, hipStream_t st);
hipError_t debug_mfma_launch(const float* A, const float* B, float* C, int prec, hipStream_t st);
hipError_t mfma_rate_launch(int iters, int wgs, float* out, hipStream_t st);
hipError_t read_rate_launch(const void* buf, long long bytes, int wgs, int iters, long long stride, unsigned* sink,
                            hipStream_t st);
hipError_t clock_sample_launch(int samples, unsigned long long* out, hipStream_t st);
hipError_t wall_mark_launch(unsigned long long* out, hipStream_t st);
int set_error(int code, const char* msg);  // for entry points defined in other source files
}  // namespace psgdk

using namespace psgdk;

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(PSGDK_EHIP, "%s: %s", what, hipGetErrorString(e));
  return PSGDK_OK;
}

#define PSGDK_TRY(expr)          \
  do {                           \
    const int _rc = (expr);      \
    if (_rc != PSGDK_OK) return _rc; \
  } while (0)
#define PSGDK_HIP(expr, what) PSGDK_TRY(hip_check((expr), what))

// Bump allocator over the caller's workspace; with base == nullptr it only measures.
struct Ws {
  char* base;
  size_t off = 0;
  explicit Ws(void* b) : base(static_cast<char*>(b)) {}
  template <typename T>
  T* take(size_t count) {
    off = (off + 255) & ~size_t(255);
    T* p = base ? reinterpret_cast<T*>(base + off) : nullptr;
    off += count * sizeof(T);
    return p;
  }
};

size_t esize(int dt) { return dt == PSGDK_BF16 ? 2 : 4; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <typename P>
bool vec_ok(P const* ptrs, int nb, int64_t ld, int dt) {
  if ((ld * (int64_t)esize(dt)) % 16 != 0) return false;
  for (int b = 0; b < nb; ++b)
    if (!aligned16(ptrs[b])) return false;
  return true;
}

int check_nb(int nb) {  // problems per public call (a launch may batch several calls' problems, up to MAXB)
  if (nb < 1 || nb > PSGDK_MAXB) return fail(PSGDK_EINVAL, "nb = %d: must be in 1..%d", nb, PSGDK_MAXB);
  return PSGDK_OK;
}
int check_prec(int prec) {
  if (prec != PSGDK_PREC_F32 && prec != PSGDK_PREC_BF16) return fail(PSGDK_EINVAL, "prec = %d", prec);
  return PSGDK_OK;
}
int check_dt(int dt, const char* name) {
  if (dt != PSGDK_F32 && dt != PSGDK_BF16) return fail(PSGDK_EINVAL, "%s dtype = %d", name, dt);
  return PSGDK_OK;
}
template <typename P>
int check_ptrs(P const* ptrs, int nb, const char* name) {
  if (!ptrs) return fail(PSGDK_EINVAL, "%s: null pointer array", name);
  for (int b = 0; b < nb; ++b)
    if (!ptrs[b]) return fail(PSGDK_EINVAL, "%s[%d]: null device pointer", name, b);
  return PSGDK_OK;
}
int check_dims(int64_t v, const char* name) {
  if (v < 1 || v > (int64_t)1 << 30) return fail(PSGDK_ESHAPE, "%s = %lld out of range", name, (long long)v);
  return PSGDK_OK;
}

// ------------------------------------------------------------------------------------------------------------
// Launch profiling (psgdk_profile_start / _stop): a HIP event pair around every MFMA-engine launch, recorded on the
// launch's stream, with the launch's kernel instantiation and its algorithmic flop and byte counts. Diagnostic.
struct ProfRec {
  int kernel_id, tri, nb;
  double flops, bytes;
  int64_t m = 0, n = 0, k = 0;
  LaunchShape shape;
  hipEvent_t a, b;
};
struct Prof {  // one per host thread: a thread's records cover its own launches
  bool on = false;
  std::vector<ProfRec> recs;
  std::vector<hipEvent_t> pool;
  hipEvent_t ev() {
    if (!pool.empty()) { hipEvent_t e = pool.back(); pool.pop_back(); return e; }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
  }
};
thread_local Prof g_prof;
thread_local LaunchShape g_last_launch;  // set by psgdk::note_launch (end of this file)

// Instantiation id of gemm_kernel<PREC, TA, TB, tile config>: cfg * 1000 + prec * 100 + adt * 10 + bdt.
int kernel_id(int prec, int adt, int bdt, int cfg) { return cfg * 1000 + prec * 100 + adt * 10 + bdt; }

void gemm_init(GemmArgs& a) {
  std::memset(&a, 0, sizeof a);
  a.alpha = 1.f;
  a.splitk = 1;
}

// Operand description for the GEMM launcher.
struct Opnd {
  int mode = KC, sign = 1, dt = PSGDK_F32;
  int64_t ld = 0;
  const void* p[MAXB] = {};
};

struct EpiSpec {
  int epi = EPI_STORE;
  float alpha = 1.f, beta = 0.f;
  int64_t ldx = 0;
  const float* X1[MAXB] = {};
  const float* X2[MAXB] = {};
  const float* s[MAXB] = {};
  float* part[MAXB] = {};
};

int gemm_cfg(int64_t M) { return M <= 32 ? 1 : 0; }
int gemm_tiles(int64_t M, int64_t N, int tri) {
  const int cfg = gemm_cfg(M);
  const int64_t tm = cfg ? (M + 31) / 32 : (M + 127) / 128, tn = (N + 127) / 128;
  return (int)(tri ? tm * (tm + 1) / 2 : tm * tn);
}

// The general engine (gemm.hip): every operand mode, precision, split-K and triangular option.
int run_gemm_general(int prec, int nb, int64_t M, int64_t N, int64_t K, const Opnd& A, const Opnd& B,
                     float* const* C, int64_t ldc, const EpiSpec& e, int tri, int out_mode, int kbeg_tri, int splitk,
                     int64_t kchunk, hipStream_t st) {
  GemmArgs a;
  gemm_init(a);
  a.M = (int)M; a.N = (int)N; a.K = (int)K;
  a.amode = A.mode; a.asign = A.sign; a.lda = A.ld;
  a.bmode = B.mode; a.bsign = B.sign; a.ldb = B.ld;
  a.ldc = ldc; a.ldx = e.ldx;
  a.alpha = e.alpha; a.beta = e.beta; a.epi = e.epi;
  a.tri = tri; a.out_mode = out_mode; a.kbeg_tri = kbeg_tri;
  a.splitk = splitk; a.kchunk = (int)(splitk > 1 ? kchunk : K);
  a.avec = vec_ok(A.p, nb, A.ld, A.dt);
  a.bvec = vec_ok(B.p, nb, B.ld, B.dt);
  a.nb = nb;
  for (int b = 0; b < nb; ++b) {
    a.A[b] = A.p[b]; a.B[b] = B.p[b]; a.C[b] = C[b];
    a.X1[b] = e.X1[b]; a.X2[b] = e.X2[b]; a.s[b] = e.s[b]; a.part[b] = e.part[b];
  }
  const int cfg = gemm_cfg(M);
  if (!g_prof.on) return hip_check(gemm_launch(a, prec, A.dt, B.dt, cfg, st), "gemm launch");
  ProfRec r;
  r.kernel_id = kernel_id(prec, A.dt, B.dt, cfg);
  r.tri = tri;
  r.nb = nb;
  if (tri) r.flops = (double)M * (M + 1) * K * nb;                    // SYRK: n(n+1)k
  else if (kbeg_tri) r.flops = (double)M * (M + 1) * N * nb;         // TRMM: n(n+1)p
  else r.flops = 2.0 * M * N * K * nb;
  {  // operands once (a triangle-read operand: its triangle), outputs once, epilogue reads and a beta read of C
    auto opnd = [&](const Opnd& o, int64_t mn) {
      const double el = o.mode == SYM ? (double)K * (K + 1) / 2 : (double)mn * K;
      return el * (double)esize(o.dt);
    };
    const double out = tri ? (out_mode == PSGDK_OUT_MIRROR ? (double)M * M : (double)M * (M + 1) / 2) : (double)M * N;
    double x = 0;
    if (e.X1[0]) x += out;
    if (e.X2[0]) x += out;
    r.bytes = nb * (opnd(A, M) + (tri ? 0.0 : opnd(B, N)) + 4.0 * out * (1 + (e.beta != 0.f) + x / out));
  }
  r.a = g_prof.ev();
  r.b = g_prof.ev();
  if (!r.a || !r.b) return fail(PSGDK_EHIP, "profiling: hipEventCreate failed");
  g_last_launch = LaunchShape();
  PSGDK_HIP(hipEventRecord(r.a, st), "profiling event");
  PSGDK_TRY(hip_check(gemm_launch(a, prec, A.dt, B.dt, cfg, st), "gemm launch"));
  PSGDK_HIP(hipEventRecord(r.b, st), "profiling event");
  r.m = M;
  r.n = tri ? M : N;
  r.k = K;
  r.shape = last_launch();
  g_prof.recs.push_back(r);
  return PSGDK_OK;
}
// run_gemm_general, or the k-contiguous kernel's fp32 twin where it applies (defined after run_b16)
int run_gemm(int prec, int nb, int64_t M, int64_t N, int64_t K, const Opnd& A, const Opnd& B, float* const* C,
             int64_t ldc, const EpiSpec& e, int tri, int out_mode, int kbeg_tri, int splitk, int64_t kchunk,
             hipStream_t st);

// ------------------------------------------------------------------------------------------------------------
// bf16 k-contiguous GEMM (gemm_bf16.hip). A: M x K rows, B: N x K rows (bf16, k contiguous); C = acc A B^T.
struct B16Out {
  float* C[MAXB] = {};
  bf16_t* Cb[MAXB] = {};
  bf16_t* CTb[MAXB] = {};
  float* CT[MAXB] = {};  // fp32 kernel only
  int64_t ldc = 0, ldcb = 0, ldct = 0;
};

// Tuning options (psgdk_set_option): one set per host thread, so that a thread's settings never change another
// thread's results.
thread_local int g_tile_order = 2;  // option 0: 0 problem-major, 1 XCD-contiguous runs, 2 runs + grouped rows
thread_local int g_force_cfg = -1;  // option 1: -1 by size, else the bf16 kernel's tile config
thread_local int g_ws = 1;          // option 12: the main loop of the 256 x 256 tiles chosen by size (0 cfg 0, 1 cfg 3)
thread_local int g_nlb_target = 1024;  // option 2: workgroups per full-storage V A product (split-K target)
thread_local int g_vmm_u = 4;          // option 3: MFMA steps per load batch of the V A kernel (2, 4 or 8)
thread_local int g_vmm_cols = -1;      // option 4: V A kernel: -1 by shape (3 for bf16 launches of >= 16
                                       // matrices and >= 512 workgroups, else 2 where the layout holds, else 0),
                                       // 0 split-K + reduce, 1 column blocks, 2 column blocks with A staged in LDS,
                                       // 3 upper tiles only in tournament-paired rounds (bf16 full-storage
                                       // matrices of an even number of 64-tiles; else 2)
thread_local int g_t1q_pg = 1;  // option 5: bf16 update forms term1 Q through Pg where cheaper (1) or never (0)
thread_local int g_upd_streams = 3;  // option 6: side streams of psgdk_kron2d_update_groups (0: the caller's only)
thread_local int g_rq16 = 1;   // option 7: the bf16 update keeps R Q in bf16 (1) or fp32 (0) for the Q update
thread_local int g_f32kc = 1;  // option 8: fp32 products with k-contiguous operands take the k-contiguous kernel
thread_local int g_big_batch = MAXB;  // option 9: items per batch of the grouped update for factor sides >= 2048
thread_local int g_small = 128;       // option 10: bf16 plain-store GEMMs with fewer 128 x 128 tiles than this (over
                                      // the launch) take the small-problem kernel; bf16 SYRKs below 1.5 times it, fp32
                                      // products below 3 times it (0: never)
thread_local int g_tiny = 64;         // option 11: of those, launches with fewer 64 x 64 tiles than this take the
                                      // tiny-product kernel (32-tiles, k split over the four waves; 0: never)

// Side streams (default priority, non-blocking) and events of the grouped update, created once per device and kept
// until the process ends. A call forks from the caller's stream with an event and joins back with one event per
// side stream, so it stays ordered with the caller's other work. The table is shared by every host thread: a call
// holds side_stream_mutex() from its fork to its join, so concurrent calls from several threads queue their side
// work one call after the other instead of mixing their events.
struct SideStreams {
  std::vector<hipStream_t> s;
  std::vector<hipEvent_t> ev;  // 1 fork + per side stream 2 (phase join, final join)
  std::vector<hipEvent_t> bev;  // the end of each batch of a grouped update (per-group completion events)
};
std::mutex& side_stream_mutex() {
  static std::mutex m;
  return m;
}
// Caller holds side_stream_mutex().
int side_streams(int n, SideStreams** out) {
  static std::vector<SideStreams> per_dev;
  int dev = 0;
  PSGDK_HIP(hipGetDevice(&dev), "hipGetDevice");
  if ((int)per_dev.size() <= dev) per_dev.resize(dev + 1);
  SideStreams& ss = per_dev[dev];
  while ((int)ss.s.size() < n) {
    hipStream_t t;
    PSGDK_HIP(hipStreamCreateWithFlags(&t, hipStreamNonBlocking), "side stream");
    ss.s.push_back(t);
  }
  while ((int)ss.ev.size() < 1 + 2 * n) {
    hipEvent_t e;
    PSGDK_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming), "side stream event");
    ss.ev.push_back(e);
  }
  *out = &ss;
  return PSGDK_OK;
}
// Caller holds side_stream_mutex(): at least n batch events in ss.
int batch_events(SideStreams* ss, size_t n) {
  while (ss->bev.size() < n) {
    hipEvent_t e;
    PSGDK_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming), "batch event");
    ss->bev.push_back(e);
  }
  return PSGDK_OK;
}

// The 256-tile configuration needs most of the 256 CUs busy; with K >= 4096 its faster main loop pays for a
// half-empty chip down to 128 tiles (one 4096 x 4096 SYRK, 136 tiles: 117 us against 133 us on 528 128-tiles).
// Its warp-specialized main loop (cfg 3, option 12) gives the same sums; it is taken except for four epilogues:
// the factor update (EPI_FACTOR, reading X1), both Procrustes steps (EPI_PROC, EPI_PROCB, reading X1 and X2) and
// the r2 trace SYRK (EPI_STRACE). At three waves per SIMD their registers spill (11 to 118 registers per lane in
// the code objects' metadata), they run at half the epilogue's load depth, and they lose more than the main loop
// gains (measured on the ViT-B step: the d = 3072 SYRKs 907 -> 840 us, the PROCB products 1676 -> 1759 us). The
// 128-tile launches take the same loop on 128 x 128 tiles (cfg 4) under the same rule (16 SYRKs of 768 x 3072:
// 67.9 -> 58.5 us); there those four epilogues would exceed the 128 registers of two workgroups per CU.
int b16_cfg(int64_t M, int64_t N, int64_t K, int tri, int nb, int epi) {
  if (g_force_cfg >= 0) return g_force_cfg;
  // the load-only-wave configurations 3 and 4, not for the epilogues that spill at their three waves per SIMD
  const bool ws = g_ws && epi != EPI_FACTOR && epi != EPI_PROCB && epi != EPI_STRACE && epi != EPI_PROC;
  const int64_t t0 = gemm_bf16_tiles(M, N, tri, 0) * nb;
  if (!(t0 >= 160 || (t0 >= 128 && K >= 4096))) return ws ? 4 : 1;
  // a SYRK of at most nine 256-tile rows: a fifth or more of its 256-tiles straddle the diagonal and compute a whole
  // block for half of one; its 128-tiles waste half as much, which outweighs their slower main loop (12 SYRKs of
  // 2304 x 2304: 227.5 -> 210.1 us on cfg 4; 16 of 3072, twelve rows: 530 -> 611 us, so not there)
  if (tri && M <= 2304) return ws ? 4 : 1;
  return ws ? 3 : 0;
}

// Operand contract of the k-contiguous kernel (gemm_bf16, esz 2; its fp32 twin, esz 4): 16-byte aligned bases,
// leading dimensions multiples of one 16-byte chunk, each operand under 2 GiB (buffer extent); a k-contiguous
// operand (rows of the buffer: m or n) needs K a multiple of a chunk, an m/n-contiguous one (fp32 only, amc / bmc:
// rows of the buffer: k) M or N a multiple of 4.
template <typename P>
bool b16_operands_ok(int nb, int64_t M, int64_t N, int64_t K, P const* A, int64_t lda, P const* B, int64_t ldb,
                     int esz = 2, bool amc = false, bool bmc = false) {
  const int64_t ce = 16 / esz, big = (int64_t)1 << 31;
  auto one = [&](int64_t mn, int64_t ld, bool mc) {
    if (ld % ce) return false;
    if (mc) return mn % ce == 0 && ld >= mn && K * ld * esz < big;
    return K % ce == 0 && ld >= K && mn * ld * esz < big;
  };
  if (!one(M, lda, amc) || !one(N, ldb, bmc)) return false;
  for (int b = 0; b < nb; ++b)
    if (!aligned16(A[b]) || !aligned16(B[b])) return false;
  return true;
}

// The k-contiguous kernel on bf16 (esz 2) or fp32 (esz 4) operands.
// kbeg: A is upper-triangular with its zeros stored; each tile starts its k loop at its first row (TRMM).
// kper (optional, bf16 k-contiguous operands): problem b has its own K = kper[b] with lda = ldb = kper[b]; K is then
// the largest of them (the size rule's K).
int run_b16(int nb, int64_t M, int64_t N, int64_t K, const void* const* A, int64_t lda, const void* const* B,
            int64_t ldb, const B16Out& o, const EpiSpec& e, int tri, int out_mode, int* ntiles, hipStream_t st,
            int esz = 2, bool amc = false, bool bmc = false, int kbeg = 0, const int* kper = nullptr) {
  if (kper) {
    if (esz != 2 || amc || bmc || kbeg) return fail(PSGDK_EINVAL, "per-problem K: bf16 k-contiguous operands only");
    for (int b = 0; b < nb; ++b) {
      const void* Ab[1] = {A[b]};
      const void* Bb[1] = {tri ? A[b] : B[b]};
      if (kper[b] < 1 || kper[b] > K || !b16_operands_ok(1, M, tri ? M : N, kper[b], Ab, kper[b], Bb, kper[b]))
        return fail(PSGDK_EINVAL, "k-contiguous kernel operand contract violated (problem %d, K = %d)", b, kper[b]);
    }
  } else if (!b16_operands_ok(nb, M, tri ? M : N, K, A, lda, tri ? A : B, ldb, esz, amc, tri ? amc : bmc)) {
    return fail(PSGDK_EINVAL, "k-contiguous kernel operand contract violated (K, leading dimensions, alignment or size)");
  }
  GB16Args a;
  std::memset(&a, 0, sizeof a);
  a.M = (int)M; a.N = (int)N; a.K = (int)K;
  a.lda = lda; a.ldb = ldb; a.ldc = o.ldc; a.ldcb = o.ldcb; a.ldct = o.ldct; a.ldx = e.ldx;
  a.alpha = e.alpha; a.epi = e.epi; a.tri = tri; a.out_mode = out_mode; a.nb = nb;
  a.vec = g_tile_order;
  a.amc = amc; a.bmc = tri ? amc : bmc;
  a.kbeg = kbeg;
  a.kper = kper ? 1 : 0;
  for (int b = 0; b < nb; ++b) {
    a.kp[b] = kper ? kper[b] : (int)K;
    a.A[b] = reinterpret_cast<const bf16_t*>(A[b]);
    a.B[b] = reinterpret_cast<const bf16_t*>(B[b]);
    a.C[b] = o.C[b]; a.Cb[b] = o.Cb[b]; a.CTb[b] = o.CTb[b]; a.CT[b] = o.CT[b];
    a.X1[b] = e.X1[b]; a.X2[b] = e.X2[b]; a.s[b] = e.s[b]; a.part[b] = e.part[b];
  }
  int cfg = b16_cfg(M, N, K, tri, nb, e.epi);
  if (esz == 4) cfg = 1;  // the fp32 kernel: the 128-tile configuration
  // a plain store whose 128-tiles would leave most of the chip idle: the small-problem kernel (64-tiles, k in
  // 512-byte chunks, two in flight). Measured crossovers against the pipelined kernels (launch of nb problems, in
  // 128-tiles): bf16 GEMMs about 130, bf16 SYRKs (whose triangle the 64-tiles follow more closely) about 200, fp32
  // products about 400 (the fp32 twin's main loop is the slower one there).
  const int64_t t128 = (int64_t)gemm_bf16_tiles(M, N, tri, 1) * nb;
  const int64_t small_max = esz == 4 ? 3 * (int64_t)g_small : tri ? 3 * (int64_t)g_small / 2 : g_small;
  const bool small = e.epi == EPI_STORE && !kbeg && !kper && !amc && !(tri ? amc : bmc) && g_force_cfg < 0 &&
                     t128 < small_max;
  // ... and one whose 64-tiles would still fill only a fraction of the CUs: the tiny-product kernel
  const bool tiny = small && (int64_t)gemm_small_tiles(M, N, tri) * nb < g_tiny;
  if (ntiles)
    *ntiles = tiny ? gemm_tiny_tiles(M, N, tri) : small ? gemm_small_tiles(M, N, tri) : gemm_bf16_tiles(M, N, tri, cfg);
  auto launch = [&]() {
    if (tiny) return gemm_tiny_launch(a, esz, st);
    if (small) return gemm_small_launch(a, esz, st);
    return esz == 4 ? gemm_f32kc_launch(a, cfg, st) : gemm_bf16_launch(a, cfg, st);
  };
  if (!g_prof.on) return hip_check(launch(), "k-contiguous gemm launch");
  ProfRec r;
  r.kernel_id = small ? 7000 + (tiny ? 2 : 0) + (esz == 4 ? 1 : 0) : (esz == 4 ? 6000 : 5000) + cfg * 10 + a.epi;
  r.tri = tri;
  r.nb = nb;
  double ksum = (double)K * nb;  // the problems' k extents summed
  if (kper) {
    ksum = 0;
    for (int b = 0; b < nb; ++b) ksum += kper[b];
  }
  const double kavg = ksum / nb;
  r.flops = tri ? (double)M * (M + 1) * ksum : kbeg ? (double)M * (M + 1) * N * nb : 2.0 * M * N * ksum;
  {  // operands once (kbeg: A's upper triangle), each output written once, each epilogue operand read once
    const double out = tri ? (out_mode == PSGDK_OUT_MIRROR ? (double)M * M : (double)M * (M + 1) / 2) : (double)M * N;
    const double a_el = kbeg ? (double)M * (M + 1) / 2 : (double)M * kavg;
    double by = a_el * esz + (tri ? 0.0 : (double)N * kavg * esz);
    if (o.C[0]) by += 4 * out;
    if (o.Cb[0]) by += 2 * out;
    if (o.CTb[0]) by += 2 * out;
    if (o.CT[0]) by += 4 * out;
    const int ep = e.epi;
    if (e.X1[0]) by += (ep == EPI_RQ ? esz : 4) * out;  // EPI_RQ reads R in the operand type
    if (e.X2[0]) by += (ep == EPI_PROCB ? 2 : 4) * out;  // EPI_PROCB reads the bf16 (R Q)^T
    r.bytes = by * nb;
  }
  r.a = g_prof.ev();
  r.b = g_prof.ev();
  if (!r.a || !r.b) return fail(PSGDK_EHIP, "profiling: hipEventCreate failed");
  g_last_launch = LaunchShape();
  PSGDK_HIP(hipEventRecord(r.a, st), "profiling event");
  PSGDK_TRY(hip_check(launch(), "k-contiguous gemm launch"));
  PSGDK_HIP(hipEventRecord(r.b, st), "profiling event");
  r.m = M;
  r.n = tri ? M : N;
  r.k = kper ? 0 : K;  // with k per problem: the largest
  if (kper)
    for (int b = 0; b < nb; ++b) r.k = kper[b] > r.k ? kper[b] : r.k;
  r.shape = last_launch();
  g_prof.recs.push_back(r);
  return PSGDK_OK;
}

int run_gemm(int prec, int nb, int64_t M, int64_t N, int64_t K, const Opnd& A, const Opnd& B, float* const* C,
             int64_t ldc, const EpiSpec& e, int tri, int out_mode, int kbeg_tri, int splitk, int64_t kchunk,
             hipStream_t st) {
  // fp32 products on the k-contiguous kernel's fp32 twin: fp32 operands stored k- or m/n-contiguous (not a triangle),
  // M > 32 (the general engine's 128 x 128 tiles, so that per-tile partials count the same), one k range, no packed
  // output, a plain store only without beta, and a SYRK's single operand.
  const bool kc_epi = e.epi == EPI_FACTOR || e.epi == EPI_PROC || e.epi == EPI_SCALE || e.epi == EPI_RQ ||
                      e.epi == EPI_SUMSQ || e.epi == EPI_STRACE || (e.epi == EPI_STORE && e.beta == 0.f);
  if (g_f32kc && prec == PSGDK_PREC_F32 && A.dt == PSGDK_F32 && B.dt == PSGDK_F32 && M > 32 && splitk == 1 &&
      !kbeg_tri && out_mode != PSGDK_OUT_PACKED && kc_epi && A.mode != SYM && B.mode != SYM &&
      (!tri || A.mode == B.mode) &&
      b16_operands_ok(nb, M, tri ? M : N, K, A.p, A.ld, tri ? A.p : B.p, tri ? A.ld : B.ld, 4, A.mode == MC,
                      (tri ? A.mode : B.mode) == MC)) {
    B16Out o;
    o.ldc = ldc;
    for (int b = 0; b < nb; ++b) o.C[b] = C[b];
    return run_b16(nb, M, N, K, A.p, A.ld, tri ? A.p : B.p, tri ? A.ld : B.ld, o, e, tri, out_mode, nullptr, st, 4,
                   A.mode == MC, (tri ? A.mode : B.mode) == MC);
  }
  return run_gemm_general(prec, nb, M, N, K, A, B, C, ldc, e, tri, out_mode, kbeg_tri, splitk, kchunk, st);
}

// ------------------------------------------------------------------------------------------------------------
// Norm lower bound pipeline (see nlb.hip). full = the matrix is stored in full (read by contiguous loads);
// otherwise only its upper triangle is read.
// tile pairs of rform (64 x 64 tiles, I <= J): its trace partials
int64_t rform_pairs(int64_t d) {
  const int64_t T = (d + 63) / 64;
  return T * (T + 1) / 2;
}

struct NlbWs {
  float *vb0[MAXB], *vb1[MAXB], *part[MAXB], *ss0[MAXB], *ss1[MAXB];
  float *rpart[MAXB], *cpart[MAXB], *tmax[MAXB], *dmax[MAXB], *rn2[MAXB], *scal[MAXB];
  int splits;
  int64_t kchunk;
  int64_t part_cols;  // capacity of part[b] in columns of 32 rows
};

void nlb_plan(int64_t n, int nb, int& splits, int64_t& kchunk) {
  const int tiles = (int)((n + 127) / 128);
  int s = (512 + tiles * nb - 1) / (tiles * nb);
  const int maxs = (int)std::max<int64_t>(1, (n + 63) / 64);
  s = std::max(1, std::min(s, maxs));
  kchunk = ((n + s - 1) / s + 63) / 64 * 64;
  splits = (int)((n + kchunk - 1) / kchunk);
}

// Split of the full-storage V A products: about g_nlb_target workgroups of 32 x 128 outputs, k slices of at least
// 128, at most 8 slices (the reduce kernel's unrolled width), within the partial capacity (columns of 32 rows per
// matrix).
void nlb_full_plan(int64_t n, int nb, int64_t part_cols, int& ksplit, int& kslice) {
  const int64_t ncb = (n + 127) / 128;
  int64_t s = (g_nlb_target + ncb * nb - 1) / (ncb * nb);
  s = std::min(s, std::max<int64_t>(1, (n + 127) / 128));
  s = std::max<int64_t>(1, std::min({s, part_cols / n, (int64_t)8}));
  kslice = (int)(((n + s - 1) / s + 63) / 64 * 64);
  ksplit = (int)((n + kslice - 1) / kslice);
}

void nlb_take(Ws& w, int64_t n, int nb, NlbWs& o) {
  nlb_plan(n, nb, o.splits, o.kchunk);
  const int64_t T = (n + 63) / 64, nbk = T, ntri = T * (T + 1) / 2;
  o.part_cols = std::max<int64_t>(o.splits, 8) * n;
  for (int b = 0; b < nb; ++b) {
    o.vb0[b] = w.take<float>(NLB_K * n);
    o.vb1[b] = w.take<float>(NLB_K * n);
    o.part[b] = w.take<float>((size_t)o.part_cols * NLB_K);
    o.ss0[b] = w.take<float>(NLB_K * nbk);
    o.ss1[b] = w.take<float>(NLB_K * nbk);
    o.rpart[b] = w.take<float>((size_t)T * T * 64);
    o.cpart[b] = w.take<float>((size_t)T * 64);
    o.tmax[b] = w.take<float>(ntri);
    o.dmax[b] = w.take<float>(ntri);
    o.rn2[b] = w.take<float>(n);
    o.scal[b] = w.take<float>(NLB_NSCAL);
  }
}

// Whether rform_kernel's row statistics of an n x n matrix (2 n ceil(n / 64) floats) fit in a bound's part buffer.
bool rform_stats_fit(int64_t n, const NlbWs& w) { return 2 * n * ((n + 63) / 64) <= w.part_cols * NLB_K; }

NlbArgs nlb_args(int64_t n, int sign, int nb, const float* const* A, int64_t lda, const NlbWs& w) {
  NlbArgs a;
  std::memset(&a, 0, sizeof a);
  a.nb = nb; a.n = (int)n; a.T = (int)((n + 63) / 64); a.sign = sign; a.splits = w.splits; a.lda = lda;
  a.ssc = 64;
  for (int b = 0; b < nb; ++b) {
    a.A[b] = A[b];
    a.rpart[b] = w.rpart[b]; a.cpart[b] = w.cpart[b]; a.tmax[b] = w.tmax[b]; a.dmax[b] = w.dmax[b];
    a.rn2[b] = w.rn2[b]; a.scal[b] = w.scal[b]; a.part[b] = w.part[b];
  }
  return a;
}

// One V A_sym product into the split partials.
int nlb_vmm(int64_t n, int sign, int nb, const float* const* A, int64_t lda, bool full, float* const* Vin,
            const NlbWs& w, hipStream_t st) {
  Opnd oa, ob;
  oa.mode = KC; oa.ld = n;
  for (int b = 0; b < nb; ++b) { oa.p[b] = Vin[b]; ob.p[b] = A[b]; }
  ob.ld = lda;
  if (full) { ob.mode = MC; } else { ob.mode = SYM; ob.sign = sign; }
  EpiSpec e;
  float* C[MAXB];
  for (int b = 0; b < nb; ++b) C[b] = w.part[b];
  return run_gemm(PSGDK_PREC_F32, nb, NLB_K, n, n, oa, ob, C, n, e, 0, 0, 0, w.splits, w.kchunk, st);
}

int run_nlb(int64_t n, int sign, int nb, const float* const* A, int64_t lda, bool full, const float* const* V,
            const NlbFinal& fin, const NlbWs& w, hipStream_t st) {
  NlbArgs a = nlb_args(n, sign, nb, A, lda, w);
  PSGDK_HIP(nlb_rownorm_launch(a, st), "tri_rownorm");
  for (int b = 0; b < nb; ++b) { a.Vin[b] = V[b]; a.Vout[b] = w.vb0[b]; }
  PSGDK_HIP(nlb_init_launch(a, st), "nlb_init");
  float* const* vb[2] = {w.vb0, w.vb1};
  float* const* ss[2] = {w.ss0, w.ss1};
  // V1 = V0 A / nf; V2 = (V1/|V1|) A / nf; V3 = V2 A / nf; V4 = (V3/|V3|) A / nf
  int cur = 0;
  for (int it = 0; it < 4; ++it) {
    PSGDK_TRY(nlb_vmm(n, sign, nb, A, lda, full, vb[cur], w, st));
    const int normalize = it & 1;
    for (int b = 0; b < nb; ++b) {
      a.Vout[b] = vb[cur ^ 1][b];
      a.ssin[b] = ss[0][b];
      a.ssout[b] = ss[normalize][b];
    }
    PSGDK_HIP(nlb_reduce_launch(a, normalize, st), "nlb_reduce");
    cur ^= 1;
  }
  for (int b = 0; b < nb; ++b) a.ssin[b] = ss[1][b];
  PSGDK_HIP(nlb_final_launch(a, fin, st), "nlb_final");
  return PSGDK_OK;
}

// Norm lower bound of fully stored matrices (fp32 or bf16): row norms, init, 4 V A products with folded scaling,
// final. 7 launches.
// The column-block V A kernel needs the 16-byte operand layout (n and the row stride multiples of 16 bytes,
// 16-byte aligned matrices and V buffers, each matrix < 2 GiB).
bool vmm_cols_ok(int64_t n, int nb, const void* const* A, int64_t lda, int esz, const NlbWs& w) {
  const int64_t ach = 16 / esz;
  if (n % ach || lda % ach || n * lda * esz >= ((int64_t)1 << 31) || NLB_K * n * esz >= ((int64_t)1 << 31)) return false;
  for (int b = 0; b < nb; ++b)
    if (!aligned16(A[b]) || !aligned16(w.vb0[b]) || !aligned16(w.vb1[b])) return false;
  return true;
}

// stats_in_part: the producer of the (skew) matrices left per-(row, column block) row statistics in w.part
// (rform_kernel's aux output; rform_stats_fit says where they fit), reduced here instead of a pass over A.
int run_nlb_full(int64_t n, int sign, int nb, const void* const* A, int64_t lda, int a_bf16, const float* const* V,
                 const NlbFinal& fin, const NlbWs& w, hipStream_t st, bool stats_in_part = false) {
  const float* Af[MAXB];
  for (int b = 0; b < nb; ++b) Af[b] = reinterpret_cast<const float*>(A[b]);
  NlbArgs a = nlb_args(n, sign, nb, Af, lda, w);
  nlb_full_plan(n, nb, w.part_cols, a.ksplit, a.kslice);
  a.vmm_u = g_vmm_u;
  a.vmm_cols = g_vmm_cols != 0 && vmm_cols_ok(n, nb, A, lda, a_bf16 ? 2 : 4, w) ? (g_vmm_cols != 1 ? 2 : 1) : 0;
  // bf16 matrices of an even number of 64-tiles: the kernel that reads the upper tiles only. It keeps a matrix on
  // one XCD, so by shape (option 4 = -1) it takes launches of at least 16 matrices (two per XCD or more) and 512
  // workgroups; smaller sets ran faster on the row kernel (measured crossovers), and option 4 = 3 forces it.
  const bool tri_ok = a.vmm_cols == 2 && a_bf16 && n % 128 == 0;
  if (tri_ok && (g_vmm_cols == 3 || (g_vmm_cols == -1 && nb >= 16 && (int64_t)nb * (n / 64) >= 512))) a.vmm_cols = 3;
  a.vblk = a.vmm_cols == 3;  // the upper-tile kernel's V layout, from the init kernel on
  a.ssc = a.vmm_cols ? 64 : 128;
  if (a.vmm_cols && a.vmm_u == 8) a.vmm_u = 4;
  if (stats_in_part) PSGDK_HIP(nlb_full_launch(a, 3, a_bf16, 0, st), "row norms from partials");
  else PSGDK_HIP(nlb_full_launch(a, 0, a_bf16, 0, st), "row norms");
  for (int b = 0; b < nb; ++b) { a.Vin[b] = V[b]; a.Vout[b] = w.vb0[b]; }
  PSGDK_HIP(nlb_full_launch(a, 1, a_bf16, 0, st), "nlb init");
  float* const* vb[2] = {w.vb0, w.vb1};
  float* const* ss[2] = {w.ss0, w.ss1};
  int cur = 0;
  for (int it = 0; it < 4; ++it) {
    const int normalize = it & 1;
    for (int b = 0; b < nb; ++b) {
      a.Vin[b] = vb[cur][b];
      a.Vout[b] = vb[cur ^ 1][b];
      a.ssin[b] = ss[0][b];
      a.ssout[b] = ss[normalize][b];
    }
    PSGDK_HIP(nlb_full_launch(a, 2, a_bf16, normalize, st), "V A");
    cur ^= 1;
  }
  for (int b = 0; b < nb; ++b) a.ssin[b] = ss[1][b];
  PSGDK_HIP(nlb_final_launch(a, fin, st), "nlb_final");
  return PSGDK_OK;
}

// The SPD bound of term1 = Pc Pc^T (d x d) from its factor Pc (d x k bf16 rows; Pr = Pc^T, k x d rows), without
// forming term1: the same bound (psgd_pro.py:19-41) on the same matrix, its products carried out in k-space.
//   H = Pr Pr^T = Pc^T Pc (k x k, SYRK) -> Hb; W = Pc H -> Wb (d x k); row statistics of term1 (squared row norms
//   rowsum(W * Pc), diagonal rowsum(Pc * Pc)); argmax j; row j of term1 = Pc Pc_j^T; V0 from it; U0 = V0 Pc.
//   The bound's iterate V (32 x d) is X Pc^T with X = V Pc (32 x k): V term1 / nf = (X H / nf) Pc^T, and row r of
//   V has squared norm X_r H X_r^T. So its four products V <- s (V term1 / nf) (s: the row normalization, every
//   second product) are X <- s (X H / nf) on the k x k matrix H, starting from U0, with the row dots X H X^T in
//   place of the sums of squares (the V A kernels' dot epilogue); the bound nf max_r ||V_r|| reads the last ones.
//   One d x k read of Pc and four of the k x k H, against eight of Pc with the products through Pc and Pc^T.
// Needs k, d multiples of 8 and 16-byte aligned operands (the bf16 update's Pg route: k < d / 2).
int run_nlb_gram(int64_t d, int64_t k, int nb, const bf16_t* const* Pc, const bf16_t* const* Pr, bf16_t* const* Hb,
                 bf16_t* const* Wb, const float* const* V, const NlbFinal& fin, const NlbWs& w, hipStream_t st) {
  const void *A[MAXB], *B[MAXB];
  {  // H = Pr Pr^T (k x k, mirrored bf16)
    B16Out out;
    out.ldcb = k;
    for (int b = 0; b < nb; ++b) { A[b] = Pr[b]; out.Cb[b] = Hb[b]; }
    EpiSpec e;
    PSGDK_TRY(run_b16(nb, k, k, d, A, d, A, d, out, e, 1, PSGDK_OUT_MIRROR, nullptr, st));
  }
  {  // W = Pc H (d x k bf16)
    B16Out out;
    out.ldcb = k;
    for (int b = 0; b < nb; ++b) { A[b] = Pc[b]; B[b] = Hb[b]; out.Cb[b] = Wb[b]; }
    EpiSpec e;
    PSGDK_TRY(run_b16(nb, d, k, k, A, k, B, k, out, e, 0, 0, nullptr, st));
  }
  GramArgs ga;
  std::memset(&ga, 0, sizeof ga);
  ga.nb = nb; ga.d = (int)d; ga.k = (int)k;
  for (int b = 0; b < nb; ++b) {
    ga.P[b] = Pc[b]; ga.W[b] = Wb[b]; ga.rn2[b] = w.rn2[b]; ga.rmax[b] = w.rpart[b]; ga.diag[b] = w.cpart[b];
    ga.scal[b] = w.scal[b]; ga.aj[b] = reinterpret_cast<bf16_t*>(w.vb1[b]);  // vb1 is free until the first product
  }
  for (int stage = 0; stage < 3; ++stage) PSGDK_HIP(gram_launch(ga, stage, st), "gram statistics");
  const float* Af[MAXB];
  for (int b = 0; b < nb; ++b) Af[b] = reinterpret_cast<const float*>(ga.aj[b]);
  NlbArgs a = nlb_args(d, 1, nb, Af, 0, w);  // row stride 0: the init kernel's "row j" is aj itself
  a.vmm_cols = g_vmm_cols == 1 ? 1 : 2; a.ssc = 64; a.vmm_u = g_vmm_u == 2 ? 2 : 4;
  for (int b = 0; b < nb; ++b) { a.Vin[b] = V[b]; a.Vout[b] = w.vb0[b]; }
  PSGDK_HIP(nlb_full_launch(a, 1, 1, 0, st), "nlb init");
  {
    NlbArgs h1 = a;  // U0 = V0 Pc: A = Pr (k rows of d), 32 x k, no scale
    h1.n = (int)k; h1.kdim = (int)d; h1.lda = d; h1.plain = 1;
    for (int b = 0; b < nb; ++b) { h1.A[b] = reinterpret_cast<const float*>(Pr[b]); h1.Vin[b] = w.vb0[b]; h1.Vout[b] = w.part[b]; }
    PSGDK_HIP(nlb_full_launch(h1, 2, 1, 0, st), "V Pc");
  }
  NlbArgs hx = a;  // X <- s (X H / nf): A = Hb (k x k, both triangles), row dots for the norms
  hx.n = (int)k; hx.lda = k; hx.dot = 1;
  float* const* vb[2] = {w.vb0, w.vb1};
  float* const* ss[2] = {w.ss0, w.ss1};
  int cur = 0;
  for (int it = 0; it < 4; ++it) {
    const int normalize = it & 1;
    for (int b = 0; b < nb; ++b) {
      hx.A[b] = reinterpret_cast<const float*>(Hb[b]);
      hx.Vin[b] = it == 0 ? w.part[b] : vb[cur][b];
      hx.Vout[b] = vb[cur ^ 1][b];
      hx.ssin[b] = ss[0][b];
      hx.ssout[b] = ss[normalize][b];
    }
    PSGDK_HIP(nlb_full_launch(hx, 2, 1, normalize, st), "X H");
    cur ^= 1;
  }
  for (int b = 0; b < nb; ++b) hx.ssin[b] = ss[1][b];  // k-space partials: ceil(k / 64) per row
  PSGDK_HIP(nlb_final_launch(hx, fin, st), "nlb_final");
  return PSGDK_OK;
}

// ------------------------------------------------------------------------------------------------------------
// Kron 2-D group helpers

int check_group(const psgdk_kron2d_t* g, bool need_g = true) {
  if (!g) return fail(PSGDK_EINVAL, "null group");
  PSGDK_TRY(check_nb(g->nb));
  PSGDK_TRY(check_prec(g->prec));
  PSGDK_TRY(check_dims(g->m, "m"));
  PSGDK_TRY(check_dims(g->n, "n"));
  PSGDK_TRY(check_dt(g->g_dtype, "G"));
  PSGDK_TRY(check_dt(g->p_dtype, "param"));
  const int64_t d[2] = {g->m, g->n};
  for (int f = 0; f < 2; ++f) {
    const int k = g->kind[f];
    if (k != PSGDK_FACTOR_NONE && k != PSGDK_FACTOR_DIAG && k != PSGDK_FACTOR_DENSE)
      return fail(PSGDK_EINVAL, "kind[%d] = %d", f, k);
    if (k == PSGDK_FACTOR_NONE && d[f] != 1) return fail(PSGDK_ESHAPE, "factor %d is NONE but its size is %lld", f, (long long)d[f]);
    if (k != PSGDK_FACTOR_NONE) {
      PSGDK_TRY(check_ptrs(g->Q[f], g->nb, "Q"));
      PSGDK_TRY(check_ptrs(g->P[f], g->nb, "P"));
      PSGDK_TRY(check_ptrs(g->L[f], g->nb, "L"));
    }
  }
  if (need_g) PSGDK_TRY(check_ptrs(g->G, g->nb, "G"));
  return PSGDK_OK;
}

int64_t dense_max(const psgdk_kron2d_t* g) {
  int64_t d = 0;
  if (g->kind[0] == PSGDK_FACTOR_DENSE) d = std::max(d, g->m);
  if (g->kind[1] == PSGDK_FACTOR_DENSE) d = std::max(d, g->n);
  return d;
}

// out = P1 X P2 over the factor kinds (dense: GEMM with P; diagonal: scaling by q * q; none: identity).
// tmp: m x n scratch. With part non-null, sum-of-squares partials of out are written there and their count to
// *npart.
int precondition(const psgdk_kron2d_t* g, const void* const* X, int xdt, float* const* tmp, float* const* out,
                 float* const* part, int ptri, int* npart, hipStream_t st) {
  const int nb = g->nb, k0 = g->kind[0], k1 = g->kind[1];
  const int64_t m = g->m, n = g->n;
  *npart = 0;
  const void* cur[MAXB];
  int curdt = xdt;
  for (int b = 0; b < nb; ++b) cur[b] = X[b];
  bool sumsq_done = false;
  float* const* dst1 = k1 != PSGDK_FACTOR_NONE ? tmp : out;
  if (g->prec == PSGDK_PREC_F32 && curdt == PSGDK_BF16 && g_f32kc && k0 == PSGDK_FACTOR_DENSE &&
      k1 == PSGDK_FACTOR_DENSE && m > 32) {
    // bf16 X on the fp32 path: widened into `out` (free until the second product) so that P1 X takes the fp32
    // twin of the k-contiguous kernel (the general engine, reading the bf16 X, ran 12 products of 768 x 3072 x 768
    // at 27.5 TFLOP/s)
    EwArgs a;
    std::memset(&a, 0, sizeof a);
    a.nb = nb; a.m = m; a.n = n; a.dt = curdt;
    for (int b = 0; b < nb; ++b) { a.in[b] = cur[b]; a.out[b] = out[b]; }
    PSGDK_HIP(noise_launch(a, st), "X to fp32");
    curdt = PSGDK_F32;
    for (int b = 0; b < nb; ++b) cur[b] = out[b];
  }
  // rows: P1 X
  if (k0 == PSGDK_FACTOR_DENSE) {
    Opnd A, B;
    if (ptri & 2) { A.mode = SYM; A.sign = 1; } else { A.mode = KC; }
    A.ld = m;
    B.mode = MC; B.ld = n; B.dt = curdt;
    for (int b = 0; b < nb; ++b) { A.p[b] = g->P[0][b]; B.p[b] = cur[b]; }
    EpiSpec e;
    if (k1 == PSGDK_FACTOR_NONE && part) {
      e.epi = EPI_SUMSQ;
      for (int b = 0; b < nb; ++b) e.part[b] = part[b];
      sumsq_done = true;
      *npart = gemm_tiles(m, n, 0);
    }
    PSGDK_TRY(run_gemm(g->prec, nb, m, n, m, A, B, dst1, n, e, 0, 0, 0, 1, 0, st));
    curdt = PSGDK_F32;
    for (int b = 0; b < nb; ++b) cur[b] = dst1[b];
  } else if (k0 == PSGDK_FACTOR_DIAG || k1 == PSGDK_FACTOR_NONE) {
    EwArgs a;
    std::memset(&a, 0, sizeof a);
    a.nb = nb; a.m = m; a.n = n; a.dt = curdt;
    for (int b = 0; b < nb; ++b) {
      a.in[b] = cur[b];
      a.in2[b] = k0 == PSGDK_FACTOR_DIAG ? g->P[0][b] : nullptr;
      a.out[b] = dst1[b];
    }
    PSGDK_HIP(diag_scale_launch(a, st), "diag_scale rows");
    curdt = PSGDK_F32;
    for (int b = 0; b < nb; ++b) cur[b] = dst1[b];
  }
  // columns: (.) P2
  if (k1 == PSGDK_FACTOR_DENSE) {
    Opnd A, B;
    A.mode = KC; A.ld = n; A.dt = curdt;
    if (ptri & 2) { B.mode = SYM; B.sign = 1; } else { B.mode = KC; }
    B.ld = n;
    for (int b = 0; b < nb; ++b) { A.p[b] = cur[b]; B.p[b] = g->P[1][b]; }
    EpiSpec e;
    if (part) {
      e.epi = EPI_SUMSQ;
      for (int b = 0; b < nb; ++b) e.part[b] = part[b];
      sumsq_done = true;
      *npart = gemm_tiles(m, n, 0);
    }
    PSGDK_TRY(run_gemm(g->prec, nb, m, n, n, A, B, out, n, e, 0, 0, 0, 1, 0, st));
  } else if (k1 == PSGDK_FACTOR_DIAG) {
    EwArgs a;
    std::memset(&a, 0, sizeof a);
    a.nb = nb; a.m = m; a.n = n; a.dt = curdt;
    for (int b = 0; b < nb; ++b) { a.in[b] = cur[b]; a.in3[b] = g->P[1][b]; a.out[b] = out[b]; }
    PSGDK_HIP(diag_scale_launch(a, st), "diag_scale cols");
  }
  if (part && !sumsq_done) {
    EwArgs a;
    std::memset(&a, 0, sizeof a);
    a.nb = nb; a.m = m; a.n = n;
    a.i0 = (int)std::min<int64_t>(256, std::max<int64_t>(1, (m * n + 2047) / 2048));
    for (int b = 0; b < nb; ++b) { a.in[b] = out[b]; a.out[b] = part[b]; }
    PSGDK_HIP(sumsq_launch(a, st), "sumsq");
    *npart = a.i0;
  }
  return PSGDK_OK;
}

// The bf16 path with k-contiguous bf16 operands applies to groups with two dense factors, or one dense and one
// diagonal factor, bf16 shadows for every dense factor, rows of whole 16-byte vectors and full (not triangle)
// storage.
bool b16_group(const psgdk_kron2d_t* g, int tri) {
  if (g->prec != PSGDK_PREC_BF16 || tri) return false;
  const int k0 = g->kind[0], k1 = g->kind[1];
  const bool dd = k0 == PSGDK_FACTOR_DENSE && k1 == PSGDK_FACTOR_DENSE;
  const bool mixed = (k0 == PSGDK_FACTOR_DENSE && k1 == PSGDK_FACTOR_DIAG) ||
                     (k0 == PSGDK_FACTOR_DIAG && k1 == PSGDK_FACTOR_DENSE);
  if (!dd && !mixed) return false;
  if (g->m % 8 || g->n % 8) return false;
  for (int f = 0; f < 2; ++f) {
    if (g->kind[f] != PSGDK_FACTOR_DENSE) continue;
    const int64_t d = f == 0 ? g->m : g->n;
    if (d * d * 2 >= ((int64_t)1 << 31)) return false;
    for (int b = 0; b < g->nb; ++b)
      if (!g->Qt16[f][b] || !g->P16[f][b] || !aligned16(g->Qt16[f][b]) || !aligned16(g->P16[f][b])) return false;
  }
  // G's alignment does not matter: the update reads G through the noise kernel and the apply copies a misaligned
  // bf16 G into aligned workspace, so a group's path depends on its own storage only (the bf16 path keeps fp32 P
  // current at refresh points only, and no other path may run on the group in between)
  if (g->m * g->n * 2 >= ((int64_t)1 << 31)) return false;
  return true;
}

bool has_shadows(const psgdk_kron2d_t* g, int f, const int* sel, int nsel) {
  if (g->prec != PSGDK_PREC_BF16 || g->kind[f] != PSGDK_FACTOR_DENSE) return false;
  const int64_t d = f == 0 ? g->m : g->n;
  if (d % 8 || d * d * 2 >= ((int64_t)1 << 31)) return false;
  for (int i = 0; i < nsel; ++i)
    if (!g->Qt16[f][sel[i]] || !g->P16[f][sel[i]] || !aligned16(g->Qt16[f][sel[i]]) || !aligned16(g->P16[f][sel[i]]))
      return false;
  return true;
}

int refresh_p_dense(const psgdk_kron2d_t* g, int f, int tri, const int* sel, int nsel, hipStream_t st) {
  const int64_t d = f == 0 ? g->m : g->n;
  if (!(tri & 2) && has_shadows(g, f, sel, nsel)) {
    // Qt16 = bf16(Q^T), then P = Qt16 Qt16^T (= Q^T Q) with its bf16 copy
    EwArgs c;
    std::memset(&c, 0, sizeof c);
    c.nb = nsel; c.m = d; c.n = d; c.ld = d; c.i0 = 1;
    for (int i = 0; i < nsel; ++i) { c.in[i] = g->Q[f][sel[i]]; c.out2[i] = g->Qt16[f][sel[i]]; }
    PSGDK_HIP(to_bf16_launch(c, st), "Q^T shadow");
    const void* A[MAXB];
    B16Out o;
    o.ldc = d; o.ldcb = d;
    for (int i = 0; i < nsel; ++i) {
      A[i] = g->Qt16[f][sel[i]];
      o.C[i] = g->P[f][sel[i]];
      o.Cb[i] = reinterpret_cast<bf16_t*>(g->P16[f][sel[i]]);
    }
    EpiSpec e;
    return run_b16(nsel, d, d, d, A, d, A, d, o, e, 1, PSGDK_OUT_MIRROR, nullptr, st);
  }
  Opnd A;
  A.mode = MC; A.ld = d;
  float* C[MAXB];
  for (int i = 0; i < nsel; ++i) { A.p[i] = g->Q[f][sel[i]]; C[i] = g->P[f][sel[i]]; }
  EpiSpec e;
  return run_gemm(g->prec, nsel, d, d, d, A, A, C, d, e, 1, (tri & 2) ? PSGDK_OUT_UPPER : PSGDK_OUT_MIRROR, 0, 1, 0, st);
}

int refresh_p_diag(const psgdk_kron2d_t* g, int f, const int* sel, int nsel, hipStream_t st) {
  const int64_t d = f == 0 ? g->m : g->n;
  EwArgs a;
  std::memset(&a, 0, sizeof a);
  a.nb = nsel; a.m = 1; a.n = d; a.dt = PSGDK_F32;
  for (int i = 0; i < nsel; ++i) { a.in[i] = g->Q[f][sel[i]]; a.in3[i] = g->Q[f][sel[i]]; a.out[i] = g->P[f][sel[i]]; }
  return hip_check(diag_scale_launch(a, st), "diag P refresh");
}

// One preconditioner update of bf16-path groups (b16_group): every contraction on gemm_bf16 with k-contiguous bf16
// operands; producers write the bf16 (and transposed) copies their consumers read.
//   per group:  X  = G + (damping + eps |G|) N                      -> Xb
//               Y  = X P2            (A = Xb,   B = P2 shadow)      -> Y^T bf16
//               Pg = P1 Y            (A = P1 shadow, B = Y^T)       -> Pg bf16, Pg^T bf16
//   per dense factor of every parameter (an item), batched over the items of one factor side d (all groups,
//   both factors, up to MAXB items per launch): term1 = SYRK (Pg or Pg^T) -> bf16; bound, L, lr/L;
//   Qn = Q - lr/L (term1 Q - term2 Q) (B = Q^T shadow; when the other side is under half of d, term1 Q is formed
//   as Pg^T (Pg Q) or Pg (Pg^T Q)) -> fp32 + Qn^T bf16; R = Qn^T - Qn -> bf16; skew bound; RQ (B = Qn^T) -> fp32 +
//   RQ^T bf16 + traces; step size; Q = Qn + a RQ + a^2/2 R RQ (B = RQ^T) -> Q fp32 + Q^T shadow (r2: S = Rn^T Rn
//   by SYRK, Q + M Q); P = Q^T Q (SYRK of the Q^T shadow) -> P shadow.
// The items are independent after Pg, and every kernel computes each problem of a launch on its own, so the
// results do not depend on how the items are batched.
struct B16Item {
  int gi = 0;  // the item's group in the call
  int64_t d = 0, other = 0;
  float term2 = 0.f;
  const bf16_t* pcol = nullptr;  // d x other rows (k = other): term1 = pcol pcol^T
  const bf16_t* prow = nullptr;  // other x d rows (k = d): term1 = pcol prow
  float* Q = nullptr;
  float* L = nullptr;
  bf16_t* Qt16 = nullptr;
  bf16_t* P16 = nullptr;
  const float* Vs = nullptr;  // 32 x d starts of the SPD and the skew bound
  const float* Vk = nullptr;
  bf16_t *T1b = nullptr, *QnTb = nullptr, *Rb = nullptr, *RQTb = nullptr;
  float *Qn = nullptr, *RQ = nullptr, *coef = nullptr, *rs = nullptr, *pc = nullptr, *tpart = nullptr,
        *rtp = nullptr;
};

// Phases of one batch of items with a common side d (n <= MAXB).
int b16_items(const std::vector<B16Item*>& it, const psgdk_update_opts_t* o, const NlbWs& nw, hipStream_t st) {
  const int nb = (int)it.size();
  const int64_t d = it[0]->d;
  const void *A[MAXB], *B[MAXB];
  // The SPD bound of term1 = pcol pcol^T. Items whose other side is under half of d (the Pg route: term1 Q goes
  // through pcol) bound term1 from pcol without forming it (run_nlb_gram, one launch sequence per other side, H in
  // the T1b buffer and pcol H in the Rb buffer, both free until later phases); the others form term1 by SYRK (one
  // launch for all of them) and share one full-storage bound.
  std::vector<int> full;
  {  // term1 = pcol pcol^T, full symmetric bf16 (its only consumers read bf16), for every item that forms it: one
     // launch whatever the other sides (K = other per problem). The problems go longest K first, dealt in snake
     // order over 8 runs, one per XCD (the kernel gives each XCD a contiguous run of tiles), so that every XCD
     // gets a like share of long and short problems.
    std::vector<int> sy;
    for (int i = 0; i < nb; ++i)
      if (!(g_t1q_pg && 2 * it[i]->other < d)) { sy.push_back(i); full.push_back(i); }
    if (!sy.empty()) {
      std::stable_sort(sy.begin(), sy.end(), [&](int x, int y) { return it[x]->other > it[y]->other; });
      std::vector<int> run[8];
      for (size_t j = 0; j < sy.size(); ++j) {
        const size_t r = j % 16;
        run[r < 8 ? r : 15 - r].push_back(sy[j]);
      }
      int k = 0, kp[MAXB];
      int64_t kmax = 0;
      B16Out out;
      out.ldcb = d;
      for (auto& rn : run)
        for (int i : rn) {
          A[k] = it[i]->pcol; out.Cb[k] = it[i]->T1b; kp[k] = (int)it[i]->other;
          kmax = std::max<int64_t>(kmax, it[i]->other);
          ++k;
        }
      EpiSpec e;
      PSGDK_TRY(run_b16(k, d, d, kmax, A, kmax, A, kmax, out, e, 1, PSGDK_OUT_MIRROR, nullptr, st, 2, false, false,
                        0, kp));
    }
  }
  for (int i0 = 0; i0 < nb;) {
    int k = 0;
    int idx[MAXB];
    const int64_t other = it[i0]->other;
    for (int i = i0; i < nb; ++i)
      if (it[i]->other == other) idx[k++] = i;
    while (i0 < nb && it[i0]->other == other) ++i0;  // items arrive sorted by other side within a batch
    if (g_t1q_pg && 2 * other < d) {
      NlbFinal fin;
      std::memset(&fin, 0, sizeof fin);
      fin.mode = NLB_FINAL_FACTOR; fin.lr = o->lr; fin.beta = o->betaL;
      const bf16_t *Pc[MAXB], *Pr[MAXB];
      bf16_t *Hb[MAXB], *Wb[MAXB];
      const float* Vs[MAXB];
      for (int j = 0; j < k; ++j) {
        const B16Item* x = it[idx[j]];
        fin.L[j] = x->L; fin.coef[j] = x->coef; fin.term2[j] = x->term2;
        Pc[j] = x->pcol; Pr[j] = x->prow; Hb[j] = x->T1b; Wb[j] = x->Rb; Vs[j] = x->Vs;
      }
      PSGDK_TRY(run_nlb_gram(d, other, k, Pc, Pr, Hb, Wb, Vs, fin, nw, st));
    }
  }
  if (!full.empty()) {
    NlbFinal fin;
    std::memset(&fin, 0, sizeof fin);
    fin.mode = NLB_FINAL_FACTOR; fin.lr = o->lr; fin.beta = o->betaL;
    const void* T1c[MAXB];
    const float* Vs[MAXB];
    for (size_t j = 0; j < full.size(); ++j) {
      const B16Item* x = it[full[j]];
      fin.L[j] = x->L; fin.coef[j] = x->coef; fin.term2[j] = x->term2;
      T1c[j] = x->T1b; Vs[j] = x->Vs;
    }
    PSGDK_TRY(run_nlb_full(d, 1, (int)full.size(), T1c, d, 1, Vs, fin, nw, st));
  }
  // Qn = Q - lr/L (term1 Q - term2 Q) -> fp32 + Qn^T bf16; items whose other side is under half of d form
  // term1 Q = pcol (prow Q): 4 other d^2 flops instead of 2 d^3, the same product associated the other way, one
  // launch sequence per other side; every other item multiplies term1 Q (d x d x d whatever its other side), and all
  // of those go in one launch (at ViT-B, the 60 factors of side 768: one launch instead of three)
  {
    int k = 0;
    B16Out out;
    out.ldc = d; out.ldct = d;
    EpiSpec e;
    e.epi = EPI_FACTOR; e.ldx = d;
    for (int i = 0; i < nb; ++i) {
      const B16Item* x = it[i];
      if (g_t1q_pg && 2 * x->other < d) continue;
      A[k] = x->T1b; B[k] = x->Qt16; out.C[k] = x->Qn; out.CTb[k] = x->QnTb; e.X1[k] = x->Q; e.s[k] = x->coef;
      ++k;
    }
    if (k) PSGDK_TRY(run_b16(k, d, d, d, A, d, B, d, out, e, 0, 0, nullptr, st));
  }
  for (int i0 = 0; i0 < nb;) {
    const int64_t other = it[i0]->other;
    int k = 0;
    int idx[MAXB];
    for (int i = i0; i < nb; ++i)
      if (it[i]->other == other) idx[k++] = i;
    while (i0 < nb && it[i0]->other == other) ++i0;
    B16Out out;
    out.ldc = d; out.ldct = d;
    EpiSpec e;
    e.epi = EPI_FACTOR; e.ldx = d;
    if (g_t1q_pg && 2 * other < d) {
      {  // Z = prow Q (other x d; B = Q^T shadow) -> Z^T bf16 (d x other) in the RQ^T buffer
        B16Out zo;
        zo.ldct = other;
        for (int j = 0; j < k; ++j) { A[j] = it[idx[j]]->prow; B[j] = it[idx[j]]->Qt16; zo.CTb[j] = it[idx[j]]->RQTb; }
        EpiSpec ze;
        PSGDK_TRY(run_b16(k, other, d, d, A, d, B, d, zo, ze, 0, 0, nullptr, st));
      }
      for (int j = 0; j < k; ++j) {
        const B16Item* x = it[idx[j]];
        A[j] = x->pcol; B[j] = x->RQTb; out.C[j] = x->Qn; out.CTb[j] = x->QnTb; e.X1[j] = x->Q; e.s[j] = x->coef;
      }
      PSGDK_TRY(run_b16(k, d, d, other, A, other, B, other, out, e, 0, 0, nullptr, st));
    }
  }
  // R = Qn^T - Qn -> bf16 (r2: and the partials of sum R * Qn), with the skew bound's row statistics of the bf16 R
  // as a by-product (no separate pass over R)
  const bool rstats = rform_stats_fit(d, nw);
  {
    EwArgs a;
    std::memset(&a, 0, sizeof a);
    a.nb = nb; a.m = d; a.n = d; a.ld = d; a.i0 = 1;
    for (int b = 0; b < nb; ++b) {
      a.in[b] = it[b]->Qn; a.out2[b] = it[b]->Rb; a.sc[b] = o->r2 ? it[b]->rtp : nullptr;
      a.aux[b] = rstats ? nw.part[b] : nullptr;
    }
    PSGDK_HIP(rform_launch(a, st), "R = Q^T - Q");
  }
  {
    NlbFinal fin;
    std::memset(&fin, 0, sizeof fin);
    fin.mode = NLB_FINAL_SCALE;
    const void* Rc[MAXB];
    const float* Vk[MAXB];
    for (int b = 0; b < nb; ++b) { fin.coef[b] = it[b]->rs; Rc[b] = it[b]->Rb; Vk[b] = it[b]->Vk; }
    PSGDK_TRY(run_nlb_full(d, -1, nb, Rc, d, 1, Vk, fin, nw, st, rstats));
  }
  if (o->r2) {  // procrustes_step_r2 (psgd_pro_fast.py:141-153)
    // S = rs^2 R R^T in the RQ^T buffer (bf16); M = a rs R - a^2/2 S in the (unused) fp32 RQ buffer, as bf16
    int nt = 0;
    {  // S = rs^2 R R^T (SYRK of R's rows, scaled in the epilogue) -> bf16 mirrored, partials of sum S * Qn
      B16Out out;
      out.ldcb = d;
      EpiSpec e;
      e.epi = EPI_STRACE; e.ldx = d;
      for (int b = 0; b < nb; ++b) {
        A[b] = it[b]->Rb; out.Cb[b] = it[b]->RQTb; e.X1[b] = it[b]->Qn; e.s[b] = it[b]->rs; e.part[b] = it[b]->tpart;
      }
      PSGDK_TRY(run_b16(nb, d, d, d, A, d, A, d, out, e, 1, PSGDK_OUT_MIRROR, &nt, st));
    }
    {
      EwArgs a;
      std::memset(&a, 0, sizeof a);
      a.nb = nb; a.i0 = (int)rform_pairs(d); a.i1 = nt; a.f0 = 0.125f;
      for (int b = 0; b < nb; ++b) {
        a.in2[b] = it[b]->rtp; a.in3[b] = it[b]->tpart; a.sc[b] = it[b]->rs; a.out[b] = it[b]->pc;
      }
      PSGDK_HIP(proc_scalar_r2_launch(a, st), "procrustes r2 step size");
    }
    {
      EwArgs a;
      std::memset(&a, 0, sizeof a);
      a.nb = nb; a.m = d; a.n = d; a.dt = PSGDK_BF16;
      for (int b = 0; b < nb; ++b) {
        a.in[b] = it[b]->Rb; a.in2[b] = reinterpret_cast<const float*>(it[b]->RQTb); a.out2[b] = it[b]->RQ;
        a.sc[b] = it[b]->pc;
      }
      PSGDK_HIP(mform_launch(a, st), "M = a rs R - a^2/2 S");
    }
    {  // Q = Qn + M Qn -> Q fp32 + Q^T shadow
      B16Out out;
      out.ldc = d; out.ldct = d;
      EpiSpec e;
      e.epi = EPI_FACTOR; e.ldx = d;
      for (int b = 0; b < nb; ++b) {
        A[b] = it[b]->RQ; B[b] = it[b]->QnTb; out.C[b] = it[b]->Q; out.CTb[b] = it[b]->Qt16;
        e.X1[b] = it[b]->Qn; e.s[b] = it[b]->pc + 2;
      }
      PSGDK_TRY(run_b16(nb, d, d, d, A, d, B, d, out, e, 0, 0, nullptr, st));
    }
  } else {
    int nt = 0;
    {  // RQ = R Qn / (bound + sn) -> RQ^T bf16 (and, option 7 = 0, RQ fp32), trace partials (tr(R RQ) reads the
       // bf16 R of the product). RQ enters the Q update as the correction a RQ, read from the bf16 RQ^T that the
       // second product takes as its B operand; the product already comes from bf16 operands, so its bf16 rounding
       // adds an error of the same size, and no second copy of RQ is written
      B16Out out;
      out.ldc = d; out.ldct = d;
      EpiSpec e;
      e.epi = EPI_RQ; e.ldx = d;
      for (int b = 0; b < nb; ++b) {
        A[b] = it[b]->Rb; B[b] = it[b]->QnTb; out.CTb[b] = it[b]->RQTb;
        if (!g_rq16) out.C[b] = it[b]->RQ;
        e.X1[b] = reinterpret_cast<const float*>(it[b]->Rb); e.s[b] = it[b]->rs; e.part[b] = it[b]->tpart;
      }
      PSGDK_TRY(run_b16(nb, d, d, d, A, d, B, d, out, e, 0, 0, &nt, st));
    }
    {
      EwArgs a;
      std::memset(&a, 0, sizeof a);
      a.nb = nb; a.i0 = nt; a.f0 = 0.125f;
      for (int b = 0; b < nb; ++b) { a.in2[b] = it[b]->tpart; a.sc[b] = it[b]->rs; a.out[b] = it[b]->pc; }
      PSGDK_HIP(proc_scalar_launch(a, st), "procrustes step size");
    }
    {  // Q = Qn + a RQ + a^2/2 R RQ -> Q fp32 + Q^T shadow
      B16Out out;
      out.ldc = d; out.ldct = d;
      EpiSpec e;
      e.epi = g_rq16 ? EPI_PROCB : EPI_PROC; e.ldx = d;
      for (int b = 0; b < nb; ++b) {
        A[b] = it[b]->Rb; B[b] = it[b]->RQTb; out.C[b] = it[b]->Q; out.CTb[b] = it[b]->Qt16;
        e.X1[b] = it[b]->Qn; e.s[b] = it[b]->pc;
        e.X2[b] = g_rq16 ? reinterpret_cast<const float*>(it[b]->RQTb) : it[b]->RQ;
      }
      PSGDK_TRY(run_b16(nb, d, d, d, A, d, B, d, out, e, 0, 0, nullptr, st));
    }
  }
  {  // P16 = bf16(Q^T Q) from the fresh Q^T shadow (its only per-step reader reads bf16; fp32 P is written by
     // psgdk_kron2d_refresh_p / _balance from the same shadow)
    B16Out out;
    out.ldcb = d;
    for (int b = 0; b < nb; ++b) { A[b] = it[b]->Qt16; out.Cb[b] = it[b]->P16; }
    EpiSpec e;
    PSGDK_TRY(run_b16(nb, d, d, d, A, d, A, d, out, e, 1, PSGDK_OUT_MIRROR, nullptr, st));
  }
  return PSGDK_OK;
}

// The update of ng bf16-path groups: per-group noise, Y and Pg, then the items of every dense factor in batches of
// one side d (largest first), the items of a batch ordered by their other side.
// group_done (optional): per group an event recorded once that group's factors, L and shadows are final (its
// items' batches done), so that a caller can start work on one group before the whole call has finished.
// draws (optional): group gi with no noise pointers (noise or noise[gi] null) generates its noise from draws[gi].
int b16_update_groups(int ng, const psgdk_kron2d_t* const* gs, const psgdk_update_opts_t* const* os,
                      const void* const* const* noise, const float* const* const* V, void* ws, size_t* ws_bytes,
                      hipStream_t st, const hipEvent_t* group_done = nullptr,
                      const psgdk_draws_t* const* draws = nullptr) {
  Ws w(ws);
  std::vector<std::vector<bf16_t*>> Xb(ng), YTb(ng), Pgb(ng), PgTb(ng);
  std::vector<std::vector<float*>> dterm(ng);  // a diagonal factor's term1
  std::vector<B16Item> items;
  for (int gi = 0; gi < ng; ++gi) {
    const psgdk_kron2d_t* g = gs[gi];
    const int64_t mn = g->m * g->n;
    for (int b = 0; b < g->nb; ++b) {
      Xb[gi].push_back(w.take<bf16_t>(mn));
      YTb[gi].push_back(w.take<bf16_t>(mn));
      Pgb[gi].push_back(w.take<bf16_t>(mn));
      PgTb[gi].push_back(w.take<bf16_t>(mn));
      dterm[gi].push_back(w.take<float>(std::max(g->m, g->n)));
    }
    for (int b = 0; b < g->nb; ++b) {
      int64_t voff = 0;
      for (int f = 0; f < 2; ++f) {
        if (g->kind[f] != PSGDK_FACTOR_DENSE) continue;  // a diagonal factor is updated in the per-group phase
        B16Item x;
        x.gi = gi;
        x.d = f == 0 ? g->m : g->n;
        x.other = f == 0 ? g->n : g->m;
        x.term2 = (float)mn / (float)x.d;
        x.pcol = f == 0 ? Pgb[gi][b] : PgTb[gi][b];
        x.prow = f == 0 ? PgTb[gi][b] : Pgb[gi][b];
        x.Q = g->Q[f][b]; x.L = g->L[f][b];
        x.Qt16 = reinterpret_cast<bf16_t*>(g->Qt16[f][b]); x.P16 = reinterpret_cast<bf16_t*>(g->P16[f][b]);
        if (V) { x.Vs = V[gi][b] + voff; x.Vk = V[gi][b] + voff + NLB_K * x.d; }
        voff += 2 * NLB_K * x.d;
        const int64_t dd = x.d * x.d;
        x.T1b = w.take<bf16_t>(dd); x.QnTb = w.take<bf16_t>(dd); x.Rb = w.take<bf16_t>(dd); x.RQTb = w.take<bf16_t>(dd);
        x.Qn = w.take<float>(dd); x.RQ = w.take<float>(dd);
        x.coef = w.take<float>(4); x.rs = w.take<float>(4); x.pc = w.take<float>(8);
        x.tpart = w.take<float>(2 * (size_t)gemm_bf16_tiles(x.d, x.d, 0, 1));
        x.rtp = w.take<float>(rform_pairs(x.d));
        items.push_back(x);
      }
    }
  }
  // batches: items sorted by (d descending, other), cut into runs of one d of at most MAXB
  std::vector<B16Item*> order;
  for (auto& x : items) order.push_back(&x);
  std::stable_sort(order.begin(), order.end(), [](const B16Item* a, const B16Item* b) {
    return a->d != b->d ? a->d > b->d : a->other < b->other;
  });
  std::vector<std::vector<B16Item*>> batches;
  for (size_t i = 0; i < order.size();) {
    std::vector<B16Item*> bt;
    const int64_t d = order[i]->d;
    const int cap = d >= 2048 ? std::min(g_big_batch, MAXB) : MAXB;
    while (i < order.size() && order[i]->d == d && (int)bt.size() < cap) bt.push_back(order[i++]);
    batches.push_back(bt);
  }
  std::vector<NlbWs> nws(batches.size());
  for (size_t k = 0; k < batches.size(); ++k) nlb_take(w, batches[k][0]->d, (int)batches[k].size(), nws[k]);
  if (!ws) { *ws_bytes = w.off; return PSGDK_OK; }
  if (*ws_bytes < w.off) return fail(PSGDK_EWORKSPACE, "workspace %zu < %zu bytes", *ws_bytes, w.off);
  // group gi's noise: noise[gi] when given, else draws[gi]
  auto drawn = [&](int gi) { return (!noise || !noise[gi]) ? draws[gi] : nullptr; };
  for (int gi = 0; gi < ng; ++gi) {
    if (!noise || !noise[gi]) {
      if (!draws || !draws[gi]) return fail(PSGDK_EINVAL, "group %d: neither noise pointers nor draws", gi);
      for (int b = 0; b < gs[gi]->nb; ++b)
        if (draws[gi]->offset[b] < 0 || draws[gi]->offset[b] % 4 || draws[gi]->offset[b] > ((int64_t)1 << 60))
          return fail(PSGDK_EINVAL, "group %d: draw offset[%d] = %lld (a multiple of 4 in 0 .. 2^60)", gi, b,
                      (long long)draws[gi]->offset[b]);
    } else {
      PSGDK_TRY(check_ptrs(noise[gi], gs[gi]->nb, "noise"));
    }
    PSGDK_TRY(check_ptrs(V[gi], gs[gi]->nb, "V"));
  }
  // the noise of group gi into a noise kernel's arguments
  auto set_noise = [&](EwArgs& a, int gi) {
    const psgdk_draws_t* d = drawn(gi);
    if (d) {
      a.draw = 1;
      a.dk0 = (unsigned)d->seed; a.dk1 = (unsigned)(d->seed >> 32);
      a.ds0 = (unsigned)d->stream_id; a.ds1 = (unsigned)(d->stream_id >> 32);
    }
    for (int b = 0; b < gs[gi]->nb; ++b) {
      if (d) a.doff[b] = d->offset[b];
      else a.in2[b] = reinterpret_cast<const float*>(noise[gi][b]);
    }
  };
  // streams: the per-group phase of group gi and batch k run on side stream gi % S and k % S; every batch starts
  // after every group's Pg exists. Under HIP graph capture everything stays on the caller's stream: a capture that
  // forked onto these side streams ended in a host-side crash inside the end of the capture, so that combination
  // is not used.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  PSGDK_HIP(hipStreamIsCapturing(st, &cap), "capture status");
  const int S = cap != hipStreamCaptureStatusNone ? 1 : std::min<int>(g_upd_streams, std::max<int>(ng, (int)batches.size()));
  SideStreams* ss = nullptr;
  std::unique_lock<std::mutex> ss_lock;
  // An error return between the fork and the join still joins: the caller's stream then waits for whatever was
  // queued on the side streams, and a capture sees no unjoined stream.
  struct Joiner {
    SideStreams* ss = nullptr;
    int S = 0;
    hipStream_t st = nullptr;
    ~Joiner() {
      if (!ss) return;
      for (int i = 0; i < S; ++i)
        if (hipEventRecord(ss->ev[1 + S + i], ss->s[i]) == hipSuccess) (void)hipStreamWaitEvent(st, ss->ev[1 + S + i], 0);
    }
  } joiner;
  if (S > 1) {
    ss_lock = std::unique_lock<std::mutex>(side_stream_mutex());
    PSGDK_TRY(side_streams(S, &ss));
    PSGDK_HIP(hipEventRecord(ss->ev[0], st), "fork");
    for (int i = 0; i < S; ++i) PSGDK_HIP(hipStreamWaitEvent(ss->s[i], ss->ev[0], 0), "fork wait");
    joiner.ss = ss; joiner.S = S; joiner.st = st;
  }
  auto lane = [&](int i) { return S > 1 ? ss->s[i % S] : st; };
  for (int gi = 0; gi < ng; ++gi) {
    const psgdk_kron2d_t* g = gs[gi];
    const int nb = g->nb;
    const int64_t m = g->m, n = g->n;
    hipStream_t st = lane(gi);
    const bool d0 = g->kind[0] == PSGDK_FACTOR_DENSE, d1 = g->kind[1] == PSGDK_FACTOR_DENSE;
    const void *A[MAXB], *B[MAXB];
    if (d0 && !d1) {  // P2 diagonal: Pg = P1 (X diag(p2)), the scaled X transposed to bf16 by the noise kernel
      EwArgs a;
      std::memset(&a, 0, sizeof a);
      a.nb = nb; a.m = m; a.n = n; a.dt = g->g_dtype; a.f0 = os[gi]->damping; a.f1 = os[gi]->grad_eps;
      for (int b = 0; b < nb; ++b) {
        a.in[b] = g->G[b]; a.in3[b] = g->P[1][b];
        a.out2[b] = Xb[gi][b];
      }
      set_noise(a, gi);
      PSGDK_HIP(noise_t_launch(a, st), "noise (transposed, column-scaled)");
      B16Out out;
      out.ldcb = n; out.ldct = m;
      for (int b = 0; b < nb; ++b) { A[b] = g->P16[0][b]; B[b] = Xb[gi][b]; out.Cb[b] = Pgb[gi][b]; out.CTb[b] = PgTb[gi][b]; }
      EpiSpec e;
      PSGDK_TRY(run_b16(nb, m, n, m, A, m, B, m, out, e, 0, 0, nullptr, st));
    } else {
      {  // X (P1 diagonal: diag(p1) X) -> bf16
        EwArgs a;
        std::memset(&a, 0, sizeof a);
        a.nb = nb; a.m = m; a.n = n; a.dt = g->g_dtype; a.f0 = os[gi]->damping; a.f1 = os[gi]->grad_eps;
        for (int b = 0; b < nb; ++b) {
          a.in[b] = g->G[b]; a.out2[b] = Xb[gi][b];
          a.in3[b] = d0 ? nullptr : g->P[0][b];
        }
        set_noise(a, gi);
        PSGDK_HIP(noise_launch(a, st), "noise");
      }
      if (d0) {
        {  // Y = X P2 -> Y^T
          B16Out out;
          out.ldct = m;
          for (int b = 0; b < nb; ++b) { A[b] = Xb[gi][b]; B[b] = g->P16[1][b]; out.CTb[b] = YTb[gi][b]; }
          EpiSpec e;
          PSGDK_TRY(run_b16(nb, m, n, n, A, n, B, n, out, e, 0, 0, nullptr, st));
        }
        {  // Pg = P1 Y -> Pg, Pg^T
          B16Out out;
          out.ldcb = n; out.ldct = m;
          for (int b = 0; b < nb; ++b) { A[b] = g->P16[0][b]; B[b] = YTb[gi][b]; out.Cb[b] = Pgb[gi][b]; out.CTb[b] = PgTb[gi][b]; }
          EpiSpec e;
          PSGDK_TRY(run_b16(nb, m, n, m, A, m, B, m, out, e, 0, 0, nullptr, st));
        }
      } else {  // Pg = (diag(p1) X) P2 -> Pg, Pg^T
        B16Out out;
        out.ldcb = n; out.ldct = m;
        for (int b = 0; b < nb; ++b) { A[b] = Xb[gi][b]; B[b] = g->P16[1][b]; out.Cb[b] = Pgb[gi][b]; out.CTb[b] = PgTb[gi][b]; }
        EpiSpec e;
        PSGDK_TRY(run_b16(nb, m, n, n, A, n, B, n, out, e, 0, 0, nullptr, st));
      }
    }
    for (int f = 0; f < 2; ++f) {  // a diagonal factor (psgd_pro.py:126-130): term1 = row sums of squares of Pg
      if (g->kind[f] != PSGDK_FACTOR_DIAG) continue;  // (f = 0) or of Pg^T (f = 1), read in bf16; L EMA, q, P = q^2
      const int64_t d = f == 0 ? m : n, other = f == 0 ? n : m;
      EwArgs a;
      std::memset(&a, 0, sizeof a);
      a.nb = nb; a.m = d; a.n = other;
      for (int b = 0; b < nb; ++b) { a.in[b] = f == 0 ? Pgb[gi][b] : PgTb[gi][b]; a.out[b] = dterm[gi][b]; }
      PSGDK_HIP(rowsq_launch(a, st), "diagonal factor term1");
      EwArgs u;
      std::memset(&u, 0, sizeof u);
      u.nb = nb; u.m = d; u.f0 = os[gi]->lr; u.f1 = os[gi]->betaL; u.f2 = (float)(m * n) / (float)d;
      for (int b = 0; b < nb; ++b) { u.in2[b] = dterm[gi][b]; u.out[b] = g->Q[f][b]; u.out2[b] = g->P[f][b]; u.sc[b] = g->L[f][b]; }
      PSGDK_HIP(diag_update_launch(u, st), "diagonal factor update");
    }
  }
  if (S > 1) {
    for (int i = 0; i < S; ++i) PSGDK_HIP(hipEventRecord(ss->ev[1 + i], ss->s[i]), "phase join");
    for (int i = 0; i < S; ++i)
      for (int j = 0; j < S; ++j)
        if (i != j) PSGDK_HIP(hipStreamWaitEvent(ss->s[i], ss->ev[1 + j], 0), "phase join wait");
  }
  if (group_done && S > 1) PSGDK_TRY(batch_events(ss, batches.size()));
  for (size_t k = 0; k < batches.size(); ++k) {
    PSGDK_TRY(b16_items(batches[k], os[0], nws[k], lane((int)k)));
    if (group_done && S > 1) PSGDK_HIP(hipEventRecord(ss->bev[k], lane((int)k)), "batch end");
  }
  if (group_done) {
    // group gi is final once every batch holding one of its items is: its event is recorded on the lane of its last
    // such batch after that lane waits for the others' end events (every group has an item: b16_group needs a
    // dense factor; its diagonal factors were updated before the phase join)
    for (int gi = 0; gi < ng; ++gi) {
      if (!group_done[gi]) continue;
      if (S == 1) {
        PSGDK_HIP(hipEventRecord(group_done[gi], st), "group done");
        continue;
      }
      int last = -1;
      for (size_t k = 0; k < batches.size(); ++k)
        for (const B16Item* x : batches[k])
          if (x->gi == gi) last = (int)k;
      if (last < 0) return fail(PSGDK_EINVAL, "group %d has no dense factor", gi);
      hipStream_t L = lane(last);
      for (size_t k = 0; k < batches.size(); ++k) {
        if ((int)k == last || lane((int)k) == L) continue;
        bool has = false;
        for (const B16Item* x : batches[k]) has = has || x->gi == gi;
        if (has) PSGDK_HIP(hipStreamWaitEvent(L, ss->bev[k], 0), "group done wait");
      }
      PSGDK_HIP(hipEventRecord(group_done[gi], L), "group done");
    }
  }
  if (S > 1) {
    joiner.ss = nullptr;
    for (int i = 0; i < S; ++i) {
      PSGDK_HIP(hipEventRecord(ss->ev[1 + S + i], ss->s[i]), "join");
      PSGDK_HIP(hipStreamWaitEvent(st, ss->ev[1 + S + i], 0), "join wait");
    }
  }
  return PSGDK_OK;
}

int b16_update(const psgdk_kron2d_t* g, const psgdk_update_opts_t* o, const void* const* noise,
               const float* const* V, void* ws, size_t* ws_bytes, hipStream_t st) {
  return b16_update_groups(1, &g, &o, &noise, &V, ws, ws_bytes, st);
}

// Precondition + clip + update of a bf16-path group: Y = G P2 (A = G bf16, B = P2 shadow) -> Y^T bf16;
// pre = P1 Y (A = P1 shadow, B = Y^T) -> fp32 + sum-of-squares partials; clip + update.
int b16_apply(const psgdk_kron2d_t* g, const psgdk_apply_opts_t* o, void* const* params, float* const* pre_out,
              float* const* clipped_out, void* ws, size_t* ws_bytes, hipStream_t st) {
  const int nb = g->nb;
  const int64_t m = g->m, n = g->n, mn = m * n;
  Ws w(ws);
  bf16_t *Gb[MAXB], *YTb[MAXB];
  float *pre[MAXB], *part[MAXB];
  const int np_max = gemm_bf16_tiles(m, n, 0, 1);
  bool conv = g->g_dtype != PSGDK_BF16;  // fp32 G, or a bf16 G the kernel cannot read in place: copy to bf16
  for (int b = 0; b < nb; ++b) conv = conv || !aligned16(g->G[b]);
  for (int b = 0; b < nb; ++b) {
    Gb[b] = conv ? w.take<bf16_t>(mn) : nullptr;
    YTb[b] = w.take<bf16_t>(mn);
    pre[b] = w.take<float>(mn);
    part[b] = w.take<float>(2 * (size_t)np_max);
  }
  if (!ws) { *ws_bytes = w.off; return PSGDK_OK; }
  if (*ws_bytes < w.off) return fail(PSGDK_EWORKSPACE, "workspace %zu < %zu bytes", *ws_bytes, w.off);
  PSGDK_TRY(check_ptrs(params, nb, "params"));
  for (int b = 0; b < nb; ++b)
    if (pre_out && pre_out[b]) pre[b] = pre_out[b];
  const void *A[MAXB], *B[MAXB];
  const bool d0 = g->kind[0] == PSGDK_FACTOR_DENSE, d1 = g->kind[1] == PSGDK_FACTOR_DENSE;
  int np = 0;
  if (d0 && d1) {
    if (conv) {
      EwArgs a;
      std::memset(&a, 0, sizeof a);
      a.nb = nb; a.m = m; a.n = n; a.dt = g->g_dtype;
      for (int b = 0; b < nb; ++b) { a.in[b] = g->G[b]; a.out2[b] = Gb[b]; }
      PSGDK_HIP(noise_launch(a, st), "G to bf16");
    }
    {
      B16Out out;
      out.ldct = m;
      for (int b = 0; b < nb; ++b) { A[b] = conv ? (const void*)Gb[b] : g->G[b]; B[b] = g->P16[1][b]; out.CTb[b] = YTb[b]; }
      EpiSpec e;
      PSGDK_TRY(run_b16(nb, m, n, n, A, n, B, n, out, e, 0, 0, nullptr, st));
    }
    B16Out out;
    out.ldc = n;
    EpiSpec e;
    e.epi = EPI_SUMSQ;
    for (int b = 0; b < nb; ++b) { A[b] = g->P16[0][b]; B[b] = YTb[b]; out.C[b] = pre[b]; e.part[b] = part[b]; }
    PSGDK_TRY(run_b16(nb, m, n, m, A, m, B, m, out, e, 0, 0, &np, st));
  } else {
    // one diagonal factor: its P scales G's rows (P1) or columns (P2) on the way to the bf16 operand, and one GEMM
    // with the dense factor's P shadow gives pre; P2 diagonal needs the operand transposed (Gb holds m n bf16)
    EwArgs a;
    std::memset(&a, 0, sizeof a);
    a.nb = nb; a.m = m; a.n = n; a.dt = g->g_dtype;
    for (int b = 0; b < nb; ++b) { a.in[b] = g->G[b]; a.out2[b] = YTb[b]; a.in3[b] = d0 ? g->P[1][b] : g->P[0][b]; }
    if (d0) PSGDK_HIP(noise_t_launch(a, st), "G diag(p2) transposed to bf16");
    else PSGDK_HIP(noise_launch(a, st), "diag(p1) G to bf16");
    B16Out out;
    out.ldc = n;
    EpiSpec e;
    e.epi = EPI_SUMSQ;
    for (int b = 0; b < nb; ++b) {
      A[b] = d0 ? (const void*)g->P16[0][b] : (const void*)YTb[b];
      B[b] = d0 ? (const void*)YTb[b] : (const void*)g->P16[1][b];
      out.C[b] = pre[b]; e.part[b] = part[b];
    }
    if (d0) PSGDK_TRY(run_b16(nb, m, n, m, A, m, B, m, out, e, 0, 0, &np, st));  // P1 (G diag(p2))
    else PSGDK_TRY(run_b16(nb, m, n, n, A, n, B, n, out, e, 0, 0, &np, st));     // (diag(p1) G) P2
  }
  EwArgs a;
  std::memset(&a, 0, sizeof a);
  a.nb = nb; a.m = m; a.n = n; a.dt = g->p_dtype; a.i0 = np;
  a.f0 = o->max_avg_amp; a.f1 = o->max_element_amp; a.f2 = o->lr_params;
  for (int b = 0; b < nb; ++b) {
    a.in[b] = params[b]; a.in2[b] = pre[b]; a.in3[b] = part[b];
    a.out2[b] = clipped_out ? clipped_out[b] : nullptr;
  }
  return hip_check(clip_update_launch(a, st), "clip + update");
}

// ------------------------------------------------------------------------------------------------------------
// Dense factor steps of the general engine, shared by psgdk_kron2d_update and the per-factor entry points.

struct FacWs {
  float *R[MAXB], *RQ[MAXB], *coef[MAXB], *rs[MAXB], *pc[MAXB], *tpart[MAXB], *rtp[MAXB];
  float *Ta[MAXB], *Tb[MAXB];  // fp32 transposed operands of the k-contiguous kernel (Q^T / (R Q)^T, Qn^T)
  NlbWs nw;
};

void fac_take(Ws& w, int64_t d, int nb, FacWs& o) {
  const int tp = gemm_tiles(d, d, 0);
  for (int b = 0; b < nb; ++b) {
    o.R[b] = w.take<float>(d * d);
    o.RQ[b] = w.take<float>(d * d);
    o.coef[b] = w.take<float>(4);
    o.rs[b] = w.take<float>(4);
    o.pc[b] = w.take<float>(8);
    o.tpart[b] = w.take<float>(2 * (size_t)tp);
    o.rtp[b] = w.take<float>(rform_pairs(d));
    o.Ta[b] = w.take<float>(d * d);
    o.Tb[b] = w.take<float>(d * d);
  }
  nlb_take(w, d, nb, o.nw);
}

// Whether the fp32 factor products of a d x d group take the k-contiguous kernel's fp32 twin with transposed
// fp32 copies of their n-contiguous operands (Q, Qn, R Q): fp32 arithmetic, d > 32 (the general engine's
// 128 x 128 tiles, so that per-tile partials count the same), d a multiple of 4, 16-byte aligned matrices.
bool fac_kc(int prec, int64_t d, int nb, std::initializer_list<const void* const*> ptrs) {
  if (prec != PSGDK_PREC_F32 || !g_f32kc || d <= 32 || d % 4 || d * d * 4 >= ((int64_t)1 << 31)) return false;
  for (auto p : ptrs)
    for (int b = 0; b < nb; ++b)
      if (!aligned16(p[b])) return false;
  return true;
}

// fp32 transposed copies dst[b] = src[b]^T of d x d matrices
int transpose_f32(int nb, int64_t d, const float* const* src, float* const* dst, hipStream_t st) {
  EwArgs a;
  std::memset(&a, 0, sizeof a);
  a.nb = nb; a.m = d; a.n = d; a.ld = d; a.i0 = 1;
  for (int b = 0; b < nb; ++b) { a.in[b] = src[b]; a.out[b] = dst[b]; }
  return hip_check(to_bf16_launch(a, st), "fp32 transpose");
}

// ell = nlb_spd(term1, V) + term2; L = max(betaL L + (1 - betaL) ell, ell); Qout = Q - lr/L (term1 Q - term2 Q)
// (psgd_pro.py:132-135). term1: full symmetric, or its upper triangle when t1_tri. Qout must not alias Q.
// qn_t (optional): set when Qout^T was also written, into w.Tb (the fp32 k-contiguous route; procrustes_run reads
// it from there)
int factor_update_run(int prec, int nb, int64_t d, const float* const* T1, int t1_tri, const float* const* Q,
                      float* const* Qout, float* const* Lv, const float* const* V, float lr, float betaL, float term2,
                      const FacWs& w, hipStream_t st, bool* qn_t = nullptr) {
  {
    NlbFinal fin;
    std::memset(&fin, 0, sizeof fin);
    fin.mode = NLB_FINAL_FACTOR; fin.lr = lr; fin.beta = betaL;
    for (int b = 0; b < nb; ++b) { fin.L[b] = Lv[b]; fin.coef[b] = w.coef[b]; fin.term2[b] = term2; }
    if (t1_tri) PSGDK_TRY(run_nlb(d, 1, nb, T1, d, false, V, fin, w.nw, st));
    else PSGDK_TRY(run_nlb_full(d, 1, nb, reinterpret_cast<const void* const*>(T1), d, 0, V, fin, w.nw, st));
  }
  Opnd a, bq;
  if (t1_tri) { a.mode = SYM; a.sign = 1; } else { a.mode = KC; }
  a.ld = d;
  bq.mode = MC; bq.ld = d;
  EpiSpec e;
  e.epi = EPI_FACTOR; e.ldx = d;
  for (int b = 0; b < nb; ++b) { a.p[b] = T1[b]; bq.p[b] = Q[b]; e.X1[b] = Q[b]; e.s[b] = w.coef[b]; }
  if (qn_t && !t1_tri && fac_kc(prec, d, nb, {reinterpret_cast<const void* const*>(T1), reinterpret_cast<const void* const*>(Q),
                                              reinterpret_cast<const void* const*>(Qout), reinterpret_cast<const void* const*>(w.Ta),
                                              reinterpret_cast<const void* const*>(w.Tb)})) {
    // Q^T into Ta; Qn = Q - c (term1 Q - term2 Q) with term1 and Q^T k-contiguous, Qn^T into Tb on the way out
    PSGDK_TRY(transpose_f32(nb, d, Q, w.Ta, st));
    B16Out o;
    o.ldc = d; o.ldct = d;
    const void *Ac[MAXB], *Bc[MAXB];
    for (int b = 0; b < nb; ++b) { Ac[b] = T1[b]; Bc[b] = w.Ta[b]; o.C[b] = Qout[b]; o.CT[b] = w.Tb[b]; }
    *qn_t = true;
    return run_b16(nb, d, d, d, Ac, d, Bc, d, o, e, 0, 0, nullptr, st, 4);
  }
  return run_gemm(prec, nb, d, d, d, a, bq, Qout, d, e, 0, 0, 0, 1, 0, st);
}

// Qout = procrustes_step2(Q) (psgd_pro.py:71-94): R = Q^T - Q, R /= nlb_skh(R, V) + sn, RQ = R Q, RRQ = R RQ,
// a = min(-tr(RQ)/tr(RRQ), 1/8) if tr(RRQ) < 0 else 1/8, Qout = Q + a (RQ + a/2 RRQ). Qout must not alias Q.
// procrustes_step_r2 (psgd_pro_fast.py:141-153) on the fp32 engine, after R = Q^T - Q (with the partials of
// sum R * Q) and its norm bound: S = rs^2 R R^T (SYRK, mirrored, with the partials of sum S * Q), the step size and
// M's coefficients, M = a rs R - a^2/2 S (in R's buffer), Qout = Q + M Q.
int procrustes_r2_tail(int prec, int nb, int64_t d, const float* const* Q, float* const* Qout, const FacWs& w,
                       hipStream_t st) {
  {
    Opnd a;
    a.mode = KC; a.ld = d;
    EpiSpec e;
    e.epi = EPI_STRACE; e.ldx = d;
    for (int b = 0; b < nb; ++b) { a.p[b] = w.R[b]; e.X1[b] = Q[b]; e.s[b] = w.rs[b]; e.part[b] = w.tpart[b]; }
    PSGDK_TRY(run_gemm(prec, nb, d, d, d, a, a, w.RQ, d, e, 1, PSGDK_OUT_MIRROR, 0, 1, 0, st));
  }
  {
    EwArgs a;
    std::memset(&a, 0, sizeof a);
    a.nb = nb; a.i0 = (int)rform_pairs(d); a.i1 = gemm_tiles(d, d, 1); a.f0 = 0.125f;
    for (int b = 0; b < nb; ++b) { a.in2[b] = w.rtp[b]; a.in3[b] = w.tpart[b]; a.sc[b] = w.rs[b]; a.out[b] = w.pc[b]; }
    PSGDK_HIP(proc_scalar_r2_launch(a, st), "procrustes r2 step size");
  }
  {
    EwArgs a;
    std::memset(&a, 0, sizeof a);
    a.nb = nb; a.m = d; a.n = d; a.dt = PSGDK_F32;
    for (int b = 0; b < nb; ++b) { a.in[b] = w.R[b]; a.in2[b] = w.RQ[b]; a.out2[b] = w.R[b]; a.sc[b] = w.pc[b]; }
    PSGDK_HIP(mform_launch(a, st), "M = a rs R - a^2/2 S");
  }
  Opnd a, bq;
  a.mode = KC; a.ld = d;
  bq.mode = MC; bq.ld = d;
  EpiSpec e;
  e.epi = EPI_FACTOR; e.ldx = d;  // X1 - (-1) (acc - 0 X1) = Q + M Q
  for (int b = 0; b < nb; ++b) { a.p[b] = w.R[b]; bq.p[b] = Q[b]; e.X1[b] = Q[b]; e.s[b] = w.pc[b] + 2; }
  return run_gemm(prec, nb, d, d, d, a, bq, Qout, d, e, 0, 0, 0, 1, 0, st);
}

// q_t: w.Tb already holds Q^T (written by factor_update_run)
int procrustes_run(int prec, int nb, int64_t d, const float* const* Q, float* const* Qout, const float* const* V,
                   const FacWs& w, hipStream_t st, bool r2 = false, bool q_t = false) {
  {
    EwArgs a;
    std::memset(&a, 0, sizeof a);
    a.nb = nb; a.m = d; a.n = d; a.ld = d; a.i0 = 1;
    for (int b = 0; b < nb; ++b) { a.in[b] = Q[b]; a.out[b] = w.R[b]; a.sc[b] = r2 ? w.rtp[b] : nullptr; }
    PSGDK_HIP(rform_launch(a, st), "R = Q^T - Q");
  }
  {
    NlbFinal fin;
    std::memset(&fin, 0, sizeof fin);
    fin.mode = NLB_FINAL_SCALE;
    for (int b = 0; b < nb; ++b) fin.coef[b] = w.rs[b];
    const void* Rc[MAXB];
    for (int b = 0; b < nb; ++b) Rc[b] = w.R[b];
    PSGDK_TRY(run_nlb_full(d, -1, nb, Rc, d, 0, V, fin, w.nw, st));
  }
  if (r2) return procrustes_r2_tail(prec, nb, d, Q, Qout, w, st);
  if (fac_kc(prec, d, nb, {reinterpret_cast<const void* const*>(Q), reinterpret_cast<const void* const*>(Qout),
                           reinterpret_cast<const void* const*>(w.R), reinterpret_cast<const void* const*>(w.RQ),
                           reinterpret_cast<const void* const*>(w.Ta), reinterpret_cast<const void* const*>(w.Tb)})) {
    // k-contiguous operands: Q^T (Tb), then R Q -> RQ and (R Q)^T (Ta), then R RQ with (R Q)^T
    if (!q_t) PSGDK_TRY(transpose_f32(nb, d, Q, w.Tb, st));
    const void *Ac[MAXB], *Bc[MAXB];
    {
      B16Out o;
      o.ldc = d; o.ldct = d;
      EpiSpec e;
      e.epi = EPI_RQ; e.ldx = d;
      for (int b = 0; b < nb; ++b) {
        Ac[b] = w.R[b]; Bc[b] = w.Tb[b]; o.C[b] = w.RQ[b]; o.CT[b] = w.Ta[b];
        e.X1[b] = w.R[b]; e.s[b] = w.rs[b]; e.part[b] = w.tpart[b];
      }
      PSGDK_TRY(run_b16(nb, d, d, d, Ac, d, Bc, d, o, e, 0, 0, nullptr, st, 4));
    }
    {
      EwArgs a;
      std::memset(&a, 0, sizeof a);
      a.nb = nb; a.i0 = gemm_tiles(d, d, 0); a.f0 = 0.125f;
      for (int b = 0; b < nb; ++b) { a.in2[b] = w.tpart[b]; a.sc[b] = w.rs[b]; a.out[b] = w.pc[b]; }
      PSGDK_HIP(proc_scalar_launch(a, st), "procrustes step size");
    }
    B16Out o;
    o.ldc = d;
    EpiSpec e;
    e.epi = EPI_PROC; e.ldx = d;
    for (int b = 0; b < nb; ++b) {
      Ac[b] = w.R[b]; Bc[b] = w.Ta[b]; o.C[b] = Qout[b];
      e.X1[b] = Q[b]; e.X2[b] = w.RQ[b]; e.s[b] = w.pc[b];
    }
    return run_b16(nb, d, d, d, Ac, d, Bc, d, o, e, 0, 0, nullptr, st, 4);
  }
  {
    Opnd a, bq;
    a.mode = KC; a.ld = d;
    bq.mode = MC; bq.ld = d;
    EpiSpec e;
    e.epi = EPI_RQ; e.ldx = d;
    for (int b = 0; b < nb; ++b) { a.p[b] = w.R[b]; bq.p[b] = Q[b]; e.X1[b] = w.R[b]; e.s[b] = w.rs[b]; e.part[b] = w.tpart[b]; }
    PSGDK_TRY(run_gemm(prec, nb, d, d, d, a, bq, w.RQ, d, e, 0, 0, 0, 1, 0, st));
  }
  {
    EwArgs a;
    std::memset(&a, 0, sizeof a);
    a.nb = nb; a.i0 = gemm_tiles(d, d, 0); a.f0 = 0.125f;
    for (int b = 0; b < nb; ++b) { a.in2[b] = w.tpart[b]; a.sc[b] = w.rs[b]; a.out[b] = w.pc[b]; }
    PSGDK_HIP(proc_scalar_launch(a, st), "procrustes step size");
  }
  Opnd a, bq;
  a.mode = KC; a.ld = d;
  bq.mode = MC; bq.ld = d;
  EpiSpec e;
  e.epi = EPI_PROC; e.ldx = d;
  for (int b = 0; b < nb; ++b) { a.p[b] = w.R[b]; bq.p[b] = w.RQ[b]; e.X1[b] = Q[b]; e.X2[b] = w.RQ[b]; e.s[b] = w.pc[b]; }
  return run_gemm(prec, nb, d, d, d, a, bq, Qout, d, e, 0, 0, 0, 1, 0, st);
}

}  // namespace

// The launchers in the kernel source files report each launch here (declared in common.h).
void psgdk::note_launch(const void* fn, long long workgroups, int threads, int lds_bytes) {
  if (!g_prof.on) return;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, lds_bytes) != hipSuccess) {
    per_cu = 0;
    (void)hipGetLastError();  // the query's error is not the launch's
  }
  g_last_launch.workgroups = (int)workgroups;
  g_last_launch.per_cu = per_cu;
}
psgdk::LaunchShape psgdk::last_launch() { return g_last_launch; }

int psgdk::set_error(int code, const char* msg) { return fail(code, "%s", msg); }

// ==============================================================================================================
extern "C" {

const char* psgdk_last_error(void) { return g_err.c_str(); }
int psgdk_version(void) { return PSGDK_VERSION; }

int psgdk_syrk(int prec, int trans, int out_mode, int64_t n, int64_t k, int a_dtype, int nb, const void* const* A,
               int64_t lda, float* const* C, int64_t ldc, psgdk_stream_t stream) {
  PSGDK_TRY(check_nb(nb));
  PSGDK_TRY(check_prec(prec));
  PSGDK_TRY(check_dt(a_dtype, "A"));
  PSGDK_TRY(check_dims(n, "n"));
  PSGDK_TRY(check_dims(k, "k"));
  PSGDK_TRY(check_ptrs(A, nb, "A"));
  PSGDK_TRY(check_ptrs(C, nb, "C"));
  if (out_mode < 0 || out_mode > 2) return fail(PSGDK_EINVAL, "out_mode = %d", out_mode);
  if (lda < (trans ? n : k)) return fail(PSGDK_ESHAPE, "lda = %lld too small", (long long)lda);
  if (out_mode != PSGDK_OUT_PACKED && ldc < n) return fail(PSGDK_ESHAPE, "ldc = %lld < n", (long long)ldc);
  if (prec == PSGDK_PREC_BF16 && a_dtype == PSGDK_BF16 && !trans && out_mode != PSGDK_OUT_PACKED &&
      b16_operands_ok(nb, n, n, k, A, lda, A, lda)) {
    B16Out o;
    o.ldc = ldc;
    for (int b = 0; b < nb; ++b) o.C[b] = C[b];
    EpiSpec e;
    return run_b16(nb, n, n, k, A, lda, A, lda, o, e, 1, out_mode, nullptr, (hipStream_t)stream);
  }
  Opnd a;
  a.mode = trans ? MC : KC; a.ld = lda; a.dt = a_dtype;
  for (int b = 0; b < nb; ++b) a.p[b] = A[b];
  EpiSpec e;
  return run_gemm(prec, nb, n, n, k, a, a, C, out_mode == PSGDK_OUT_PACKED ? n : ldc, e, 1, out_mode, 0, 1, 0,
                  (hipStream_t)stream);
}

int psgdk_symm(int prec, int side, int sign, int64_t n, int64_t p, int b_dtype, int nb, const float* const* S,
               int64_t lds, const void* const* B, int64_t ldb, float* const* C, int64_t ldc, psgdk_stream_t stream) {
  PSGDK_TRY(check_nb(nb));
  PSGDK_TRY(check_prec(prec));
  PSGDK_TRY(check_dt(b_dtype, "B"));
  PSGDK_TRY(check_dims(n, "n"));
  PSGDK_TRY(check_dims(p, "p"));
  PSGDK_TRY(check_ptrs(S, nb, "S"));
  PSGDK_TRY(check_ptrs(B, nb, "B"));
  PSGDK_TRY(check_ptrs(C, nb, "C"));
  if (sign < -1 || sign > 1) return fail(PSGDK_EINVAL, "sign = %d", sign);
  if (lds < n) return fail(PSGDK_ESHAPE, "lds < n");
  Opnd os, ob;
  os.mode = SYM; os.sign = sign; os.ld = lds;
  for (int b = 0; b < nb; ++b) { os.p[b] = S[b]; ob.p[b] = B[b]; }
  ob.dt = b_dtype; ob.ld = ldb;
  EpiSpec e;
  if (side == 0) {  // C (n x p) = S B: A = S, B operand rows p read B[k][j] (mn-contiguous)
    if (ldb < p || ldc < p) return fail(PSGDK_ESHAPE, "ldb/ldc < p");
    ob.mode = MC;
    return run_gemm(prec, nb, n, p, n, os, ob, C, ldc, e, 0, 0, sign == 0, 1, 0, (hipStream_t)stream);
  }
  if (side != 1) return fail(PSGDK_EINVAL, "side = %d", side);
  if (sign == 0) return fail(PSGDK_EINVAL, "side 1 with sign 0 (right TRMM) is not provided");
  // C (p x n) = B S: A = B (k-contiguous rows), B operand X[j][k] = S[k][j] = sign * S_sym[j][k]
  if (ldb < n || ldc < n) return fail(PSGDK_ESHAPE, "ldb/ldc < n");
  ob.mode = KC;
  e.alpha = (float)sign;
  return run_gemm(prec, nb, p, n, n, ob, os, C, ldc, e, 0, 0, 0, 1, 0, (hipStream_t)stream);
}

int psgdk_trmm(int prec, int64_t n, int64_t p, int b_dtype, int nb, const float* const* Q, int64_t ldq,
               const void* const* B, int64_t ldb, float* const* C, int64_t ldc, psgdk_stream_t stream) {
  return psgdk_symm(prec, 0, 0, n, p, b_dtype, nb, Q, ldq, B, ldb, C, ldc, stream);
}

int psgdk_trmm_ws(int prec, int64_t n, int64_t p, int b_dtype, int nb, const float* const* Q, int64_t ldq,
                  const void* const* B, int64_t ldb, float* const* C, int64_t ldc, void* ws, size_t* ws_bytes,
                  psgdk_stream_t stream) {
  PSGDK_TRY(check_nb(nb));
  PSGDK_TRY(check_prec(prec));
  PSGDK_TRY(check_dt(b_dtype, "B"));
  PSGDK_TRY(check_dims(n, "n"));
  PSGDK_TRY(check_dims(p, "p"));
  if (!ws_bytes) return fail(PSGDK_EINVAL, "ws_bytes is null");
  if (ldq < n || ldb < p || ldc < p) return fail(PSGDK_ESHAPE, "leading dimension too small");
  // The k-contiguous kernel with the triangle's k range: bf16 takes bf16 copies of triu(Q) (zeros below the
  // diagonal) and of B^T; fp32 takes an fp32 copy of triu(Q) and reads B as it is (n-contiguous rows of k).
  const bool bf = prec == PSGDK_PREC_BF16;
  const bool fast = (bf ? (n % 8 == 0 && p % 8 == 0) : (b_dtype == PSGDK_F32 && n % 4 == 0 && p % 4 == 0 && n > 32 &&
                                                        g_f32kc && (ldb * 4) % 16 == 0)) &&
                    n * n * 4 < ((int64_t)1 << 31) && n * p * 4 < ((int64_t)1 << 31);
  Ws w(ws);
  void *Qc[MAXB], *Bt[MAXB];
  for (int b = 0; b < nb; ++b) {
    Qc[b] = fast ? (bf ? (void*)w.take<bf16_t>(n * n) : (void*)w.take<float>(n * n)) : nullptr;
    Bt[b] = fast && bf ? (void*)w.take<bf16_t>(p * n) : nullptr;
  }
  if (!ws) { *ws_bytes = w.off; return PSGDK_OK; }
  if (*ws_bytes < w.off) return fail(PSGDK_EWORKSPACE, "workspace %zu < %zu bytes", *ws_bytes, w.off);
  PSGDK_TRY(check_ptrs(Q, nb, "Q"));
  PSGDK_TRY(check_ptrs(B, nb, "B"));
  PSGDK_TRY(check_ptrs(C, nb, "C"));
  bool b_aligned = true;  // the fp32 route reads B in place
  for (int b = 0; b < nb; ++b) b_aligned = b_aligned && aligned16(B[b]);
  if (!fast || (!bf && !b_aligned)) return psgdk_trmm(prec, n, p, b_dtype, nb, Q, ldq, B, ldb, C, ldc, stream);
  hipStream_t st = (hipStream_t)stream;
  {  // triu(Q), zeros below the diagonal (never read there)
    EwArgs a;
    std::memset(&a, 0, sizeof a);
    a.nb = nb; a.m = n; a.n = n; a.ld = ldq; a.dt = PSGDK_F32; a.i1 = 1;
    for (int b = 0; b < nb; ++b) {
      a.in[b] = Q[b];
      if (bf) a.out2[b] = Qc[b];
      else a.out[b] = static_cast<float*>(Qc[b]);
    }
    PSGDK_HIP(to_bf16_launch(a, st), "triu(Q) copy");
  }
  if (bf) {  // B^T in bf16 (p x n)
    EwArgs a;
    std::memset(&a, 0, sizeof a);
    a.nb = nb; a.m = p; a.n = n; a.ld = ldb; a.dt = b_dtype; a.i0 = 1;
    for (int b = 0; b < nb; ++b) { a.in[b] = B[b]; a.out2[b] = Bt[b]; }
    PSGDK_HIP(to_bf16_launch(a, st), "B^T to bf16");
  }
  B16Out o;
  o.ldc = ldc;
  const void *Ac[MAXB], *Bc[MAXB];
  for (int b = 0; b < nb; ++b) { o.C[b] = C[b]; Ac[b] = Qc[b]; Bc[b] = bf ? (const void*)Bt[b] : B[b]; }
  EpiSpec e;
  if (bf) return run_b16(nb, n, p, n, Ac, n, Bc, n, o, e, 0, 0, nullptr, st, 2, false, false, 1);
  return run_b16(nb, n, p, n, Ac, n, Bc, ldb, o, e, 0, 0, nullptr, st, 4, false, true, 1);
}

int psgdk_gemm(int prec, int trans_a, int trans_b, int64_t m, int64_t n, int64_t k, float alpha, int a_dtype,
               int b_dtype, int nb, const void* const* A, int64_t lda, const void* const* B, int64_t ldb, float beta,
               float* const* C, int64_t ldc, psgdk_stream_t stream) {
  PSGDK_TRY(check_nb(nb));
  PSGDK_TRY(check_prec(prec));
  PSGDK_TRY(check_dt(a_dtype, "A"));
  PSGDK_TRY(check_dt(b_dtype, "B"));
  PSGDK_TRY(check_dims(m, "m"));
  PSGDK_TRY(check_dims(n, "n"));
  PSGDK_TRY(check_dims(k, "k"));
  PSGDK_TRY(check_ptrs(A, nb, "A"));
  PSGDK_TRY(check_ptrs(B, nb, "B"));
  PSGDK_TRY(check_ptrs(C, nb, "C"));
  if (lda < (trans_a ? m : k) || ldb < (trans_b ? k : n) || ldc < n) return fail(PSGDK_ESHAPE, "leading dimension too small");
  if (prec == PSGDK_PREC_BF16 && a_dtype == PSGDK_BF16 && b_dtype == PSGDK_BF16 && !trans_a && trans_b &&
      beta == 0.f && b16_operands_ok(nb, m, n, k, A, lda, B, ldb)) {  // k-contiguous bf16 operands: bf16 kernel
    B16Out o;
    o.ldc = ldc;
    for (int b = 0; b < nb; ++b) o.C[b] = C[b];
    EpiSpec e;
    e.alpha = alpha;
    return run_b16(nb, m, n, k, A, lda, B, ldb, o, e, 0, 0, nullptr, (hipStream_t)stream);
  }
  Opnd oa, ob;
  oa.mode = trans_a ? MC : KC; oa.ld = lda; oa.dt = a_dtype;
  ob.mode = trans_b ? KC : MC; ob.ld = ldb; ob.dt = b_dtype;
  for (int b = 0; b < nb; ++b) { oa.p[b] = A[b]; ob.p[b] = B[b]; }
  EpiSpec e;
  e.alpha = alpha; e.beta = beta;
  return run_gemm(prec, nb, m, n, k, oa, ob, C, ldc, e, 0, 0, 0, 1, 0, (hipStream_t)stream);
}

int psgdk_tri_rownorm2(int64_t n, int sign, int nb, const float* const* A, int64_t lda, float* const* rn2,
                       float* const* amax, void* ws, size_t* ws_bytes, psgdk_stream_t stream) {
  PSGDK_TRY(check_nb(nb));
  PSGDK_TRY(check_dims(n, "n"));
  if (!ws_bytes) return fail(PSGDK_EINVAL, "ws_bytes is null");
  Ws w(ws);
  NlbWs nw;
  nlb_take(w, n, nb, nw);
  if (!ws) { *ws_bytes = w.off; return PSGDK_OK; }
  if (*ws_bytes < w.off) return fail(PSGDK_EWORKSPACE, "workspace %zu < %zu bytes", *ws_bytes, w.off);
  PSGDK_TRY(check_ptrs(A, nb, "A"));
  PSGDK_TRY(check_ptrs(rn2, nb, "rn2"));
  PSGDK_TRY(check_ptrs(amax, nb, "amax"));
  if (sign != 1 && sign != -1) return fail(PSGDK_EINVAL, "sign = %d", sign);
  if (lda < n) return fail(PSGDK_ESHAPE, "lda < n");
  NlbArgs a = nlb_args(n, sign, nb, A, lda, nw);
  for (int b = 0; b < nb; ++b) { a.rn2[b] = rn2[b]; a.amax_out[b] = amax[b]; a.Vin[b] = nullptr; }
  hipStream_t st = (hipStream_t)stream;
  PSGDK_HIP(nlb_rownorm_launch(a, st), "tri_rownorm");
  PSGDK_HIP(nlb_init_launch(a, st), "rownorm reduce");
  return PSGDK_OK;
}

int psgdk_tri_vmm(int64_t n, int sign, int nb, const float* const* V, const float* const* A, int64_t lda,
                  float* const* W, void* ws, size_t* ws_bytes, psgdk_stream_t stream) {
  PSGDK_TRY(check_nb(nb));
  PSGDK_TRY(check_dims(n, "n"));
  if (!ws_bytes) return fail(PSGDK_EINVAL, "ws_bytes is null");
  int splits;
  int64_t kchunk;
  nlb_plan(n, nb, splits, kchunk);
  Ws w(ws);
  float* part[MAXB];
  for (int b = 0; b < nb; ++b) part[b] = w.take<float>((size_t)splits * NLB_K * n);
  if (!ws) { *ws_bytes = w.off; return PSGDK_OK; }
  if (*ws_bytes < w.off) return fail(PSGDK_EWORKSPACE, "workspace %zu < %zu bytes", *ws_bytes, w.off);
  PSGDK_TRY(check_ptrs(V, nb, "V"));
  PSGDK_TRY(check_ptrs(A, nb, "A"));
  PSGDK_TRY(check_ptrs(W, nb, "W"));
  if (sign != 1 && sign != -1) return fail(PSGDK_EINVAL, "sign = %d", sign);
  if (lda < n) return fail(PSGDK_ESHAPE, "lda < n");
  hipStream_t st = (hipStream_t)stream;
  Opnd oa, ob;
  oa.mode = KC; oa.ld = n;
  ob.mode = SYM; ob.sign = sign; ob.ld = lda;
  for (int b = 0; b < nb; ++b) { oa.p[b] = V[b]; ob.p[b] = A[b]; }
  EpiSpec e;
  e.alpha = (float)sign;  // X[j][k] = A_sym[k][j] = sign * A_sym[j][k]
  PSGDK_TRY(run_gemm(PSGDK_PREC_F32, nb, NLB_K, n, n, oa, ob, part, n, e, 0, 0, 0, splits, kchunk, st));
  EwArgs s;
  std::memset(&s, 0, sizeof s);
  s.nb = nb; s.m = NLB_K; s.n = n; s.i0 = splits;
  for (int b = 0; b < nb; ++b) { s.in2[b] = part[b]; s.out[b] = W[b]; }
  return hip_check(splitk_sum_launch(s, st), "split-k sum");
}

int psgdk_norm_lower_bound(int64_t n, int sign, int nb, const float* const* A, int64_t lda, const float* const* V,
                           float* const* out, void* ws, size_t* ws_bytes, psgdk_stream_t stream) {
  PSGDK_TRY(check_nb(nb));
  PSGDK_TRY(check_dims(n, "n"));
  if (!ws_bytes) return fail(PSGDK_EINVAL, "ws_bytes is null");
  Ws w(ws);
  NlbWs nw;
  nlb_take(w, n, nb, nw);
  if (!ws) { *ws_bytes = w.off; return PSGDK_OK; }
  if (*ws_bytes < w.off) return fail(PSGDK_EWORKSPACE, "workspace %zu < %zu bytes", *ws_bytes, w.off);
  PSGDK_TRY(check_ptrs(A, nb, "A"));
  PSGDK_TRY(check_ptrs(V, nb, "V"));
  PSGDK_TRY(check_ptrs(out, nb, "out"));
  if (sign != 1 && sign != -1) return fail(PSGDK_EINVAL, "sign = %d", sign);
  if (lda < n) return fail(PSGDK_ESHAPE, "lda < n");
  hipStream_t st = (hipStream_t)stream;
  NlbFinal fin;
  std::memset(&fin, 0, sizeof fin);
  fin.mode = NLB_FINAL_NONE;
  PSGDK_TRY(run_nlb(n, sign, nb, A, lda, false, V, fin, nw, st));
  for (int b = 0; b < nb; ++b)
    PSGDK_HIP(hipMemcpyAsync(out[b], nw.scal[b] + NLB_BOUND, sizeof(float), hipMemcpyDeviceToDevice, st), "copy bound");
  return PSGDK_OK;
}

int psgdk_norm_lower_bound_full(int64_t n, int sign, int nb, const void* const* A, int64_t lda, int a_dtype,
                                const float* const* V, float* const* out, void* ws, size_t* ws_bytes,
                                psgdk_stream_t stream) {
  PSGDK_TRY(check_nb(nb));
  PSGDK_TRY(check_dims(n, "n"));
  PSGDK_TRY(check_dt(a_dtype, "A"));
  if (!ws_bytes) return fail(PSGDK_EINVAL, "ws_bytes is null");
  Ws w(ws);
  NlbWs nw;
  nlb_take(w, n, nb, nw);
  if (!ws) { *ws_bytes = w.off; return PSGDK_OK; }
  if (*ws_bytes < w.off) return fail(PSGDK_EWORKSPACE, "workspace %zu < %zu bytes", *ws_bytes, w.off);
  PSGDK_TRY(check_ptrs(A, nb, "A"));
  PSGDK_TRY(check_ptrs(V, nb, "V"));
  PSGDK_TRY(check_ptrs(out, nb, "out"));
  if (sign != 1 && sign != -1) return fail(PSGDK_EINVAL, "sign = %d", sign);
  if (lda < n) return fail(PSGDK_ESHAPE, "lda < n");
  hipStream_t st = (hipStream_t)stream;
  NlbFinal fin;
  std::memset(&fin, 0, sizeof fin);
  fin.mode = NLB_FINAL_NONE;
  PSGDK_TRY(run_nlb_full(n, sign, nb, A, lda, a_dtype == PSGDK_BF16, V, fin, nw, st));
  for (int b = 0; b < nb; ++b)
    PSGDK_HIP(hipMemcpyAsync(out[b], nw.scal[b] + NLB_BOUND, sizeof(float), hipMemcpyDeviceToDevice, st), "copy bound");
  return PSGDK_OK;
}

int psgdk_norm_lower_bound_gram(int64_t d, int64_t k, int nb, const void* const* P, const void* const* Pt,
                                const float* const* V, float* const* out, void* ws, size_t* ws_bytes,
                                psgdk_stream_t stream) {
  PSGDK_TRY(check_nb(nb));
  PSGDK_TRY(check_dims(d, "d"));
  PSGDK_TRY(check_dims(k, "k"));
  if (!ws_bytes) return fail(PSGDK_EINVAL, "ws_bytes is null");
  if (d % 8 || k % 8) return fail(PSGDK_ESHAPE, "d = %lld and k = %lld must be multiples of 8", (long long)d, (long long)k);
  if (d * k * 2 >= ((int64_t)1 << 31) || k * k * 2 >= ((int64_t)1 << 31)) return fail(PSGDK_ESHAPE, "operands over 2 GiB");
  Ws w(ws);
  bf16_t *Hb[MAXB], *Wb[MAXB];
  for (int b = 0; b < nb; ++b) { Hb[b] = w.take<bf16_t>(k * k); Wb[b] = w.take<bf16_t>(d * k); }
  NlbWs nw;
  nlb_take(w, d, nb, nw);
  if (!ws) { *ws_bytes = w.off; return PSGDK_OK; }
  if (*ws_bytes < w.off) return fail(PSGDK_EWORKSPACE, "workspace %zu < %zu bytes", *ws_bytes, w.off);
  PSGDK_TRY(check_ptrs(P, nb, "P"));
  PSGDK_TRY(check_ptrs(Pt, nb, "Pt"));
  PSGDK_TRY(check_ptrs(V, nb, "V"));
  PSGDK_TRY(check_ptrs(out, nb, "out"));
  const bf16_t *Pc[MAXB], *Pr[MAXB];
  for (int b = 0; b < nb; ++b) {
    if (!aligned16(P[b]) || !aligned16(Pt[b])) return fail(PSGDK_EINVAL, "P[%d] / Pt[%d] not 16-byte aligned", b, b);
    Pc[b] = reinterpret_cast<const bf16_t*>(P[b]); Pr[b] = reinterpret_cast<const bf16_t*>(Pt[b]);
  }
  hipStream_t st = (hipStream_t)stream;
  NlbFinal fin;
  std::memset(&fin, 0, sizeof fin);
  fin.mode = NLB_FINAL_NONE;
  PSGDK_TRY(run_nlb_gram(d, k, nb, Pc, Pr, Hb, Wb, V, fin, nw, st));
  for (int b = 0; b < nb; ++b)
    PSGDK_HIP(hipMemcpyAsync(out[b], nw.scal[b] + NLB_BOUND, sizeof(float), hipMemcpyDeviceToDevice, st), "copy bound");
  return PSGDK_OK;
}

int psgdk_unpack(int64_t n, int nb, const float* const* Pk, float* const* C, int64_t ldc, psgdk_stream_t stream) {
  PSGDK_TRY(check_nb(nb));
  PSGDK_TRY(check_dims(n, "n"));
  PSGDK_TRY(check_ptrs(Pk, nb, "Pk"));
  PSGDK_TRY(check_ptrs(C, nb, "C"));
  if (ldc < n) return fail(PSGDK_ESHAPE, "ldc < n");
  EwArgs a;
  std::memset(&a, 0, sizeof a);
  a.nb = nb; a.n = n; a.ld = ldc;
  for (int b = 0; b < nb; ++b) { a.in2[b] = Pk[b]; a.out[b] = C[b]; }
  return hip_check(unpack_launch(a, (hipStream_t)stream), "unpack");
}

// ------------------------------------------------------------------------------------------------------------
int psgdk_kron2d_update(const psgdk_kron2d_t* g, const psgdk_update_opts_t* o, const void* const* noise,
                        const float* const* V, void* ws, size_t* ws_bytes, psgdk_stream_t stream) {
  PSGDK_TRY(check_group(g));
  if (!o) return fail(PSGDK_EINVAL, "null options");
  if (!ws_bytes) return fail(PSGDK_EINVAL, "ws_bytes is null");
  if (o->r2 != 0 && o->r2 != 1) return fail(PSGDK_EINVAL, "r2 = %d (0: procrustes_step2, 1: procrustes_step_r2)", o->r2);
  if (b16_group(g, o->tri)) return b16_update(g, o, noise, V, ws, ws_bytes, (hipStream_t)stream);
  const int nb = g->nb;
  const int64_t m = g->m, n = g->n, mn = m * n, dmx = dense_max(g);
  const int64_t dims[2] = {m, n};
  Ws w(ws);
  float *X[MAXB], *Y[MAXB], *Pg[MAXB], *T1[MAXB], *Qn[MAXB], *dterm[MAXB];
  for (int b = 0; b < nb; ++b) {
    X[b] = w.take<float>(mn);
    Y[b] = w.take<float>(mn);
    Pg[b] = w.take<float>(mn);
    T1[b] = w.take<float>(dmx * dmx);
    Qn[b] = w.take<float>(dmx * dmx);
    dterm[b] = w.take<float>(std::max(m, n));
  }
  FacWs fw;
  if (dmx) fac_take(w, dmx, nb, fw);
  if (!ws) { *ws_bytes = w.off; return PSGDK_OK; }
  if (*ws_bytes < w.off) return fail(PSGDK_EWORKSPACE, "workspace %zu < %zu bytes", *ws_bytes, w.off);
  PSGDK_TRY(check_ptrs(noise, nb, "noise"));
  if (dmx) PSGDK_TRY(check_ptrs(V, nb, "V"));
  hipStream_t st = (hipStream_t)stream;

  // X = G + (damping + eps |G|) N   (psgd_pro.py:121-123)
  {
    EwArgs a;
    std::memset(&a, 0, sizeof a);
    a.nb = nb; a.m = m; a.n = n; a.dt = g->g_dtype; a.f0 = o->damping; a.f1 = o->grad_eps;
    for (int b = 0; b < nb; ++b) { a.in[b] = g->G[b]; a.in2[b] = reinterpret_cast<const float*>(noise[b]); a.out[b] = X[b]; }
    PSGDK_HIP(noise_launch(a, st), "noise");
  }
  // Pg = P1 X P2
  int np = 0;
  {
    const void* Xc[MAXB];
    for (int b = 0; b < nb; ++b) Xc[b] = X[b];
    PSGDK_TRY(precondition(g, Xc, PSGDK_F32, Y, Pg, nullptr, o->tri, &np, st));
  }
  const float term_numel = (float)mn;
  int64_t voff = 0;
  for (int f = 0; f < 2; ++f) {
    const int kind = g->kind[f];
    const int64_t d = dims[f], other = dims[1 - f];
    const float term2 = term_numel / (float)d;
    if (kind == PSGDK_FACTOR_DIAG) {
      EwArgs a;
      std::memset(&a, 0, sizeof a);
      a.nb = nb; a.m = m; a.n = n; a.i0 = f;
      for (int b = 0; b < nb; ++b) { a.in[b] = Pg[b]; a.out[b] = dterm[b]; }
      PSGDK_HIP(diag_term1_launch(a, st), "diag term1");
      EwArgs u;
      std::memset(&u, 0, sizeof u);
      u.nb = nb; u.m = d; u.f0 = o->lr; u.f1 = o->betaL; u.f2 = term2;
      for (int b = 0; b < nb; ++b) { u.in2[b] = dterm[b]; u.out[b] = g->Q[f][b]; u.out2[b] = g->P[f][b]; u.sc[b] = g->L[f][b]; }
      PSGDK_HIP(diag_update_launch(u, st), "diag update");
      continue;
    }
    if (kind != PSGDK_FACTOR_DENSE) continue;
    const int term_tri = o->tri & 1;
    // term1 = Pg Pg^T (f = 0) or Pg^T Pg (f = 1)   (psgd_pro.py:125)
    {
      Opnd a;
      a.mode = f == 0 ? KC : MC; a.ld = n;
      for (int b = 0; b < nb; ++b) a.p[b] = Pg[b];
      EpiSpec e;
      PSGDK_TRY(run_gemm(g->prec, nb, d, d, other, a, a, T1, d, e, 1,
                         term_tri ? PSGDK_OUT_UPPER : PSGDK_OUT_MIRROR, 0, 1, 0, st));
    }
    const float* Vs[MAXB];
    const float* Vk[MAXB];
    for (int b = 0; b < nb; ++b) { Vs[b] = V[b] + voff; Vk[b] = V[b] + voff + NLB_K * d; }
    voff += 2 * NLB_K * d;
    // Qn = Q - lr/L (term1 Q - term2 Q) with L's EMA (psgd_pro.py:132-135), then the Procrustes step on Qn into Q
    const float* T1c[MAXB];
    const float* Qc[MAXB];
    const float* Qnc[MAXB];
    for (int b = 0; b < nb; ++b) { T1c[b] = T1[b]; Qc[b] = g->Q[f][b]; Qnc[b] = Qn[b]; }
    bool qn_t = false;
    PSGDK_TRY(factor_update_run(g->prec, nb, d, T1c, term_tri, Qc, Qn, g->L[f], Vs, o->lr, o->betaL, term2, fw, st,
                                &qn_t));
    PSGDK_TRY(procrustes_run(g->prec, nb, d, Qnc, g->Q[f], Vk, fw, st, o->r2 != 0, qn_t));
  }
  // P refresh (psgd_pro_fast.py:191-192)
  int sel[MAXB];
  for (int b = 0; b < nb; ++b) sel[b] = b;
  for (int f = 0; f < 2; ++f)
    if (g->kind[f] == PSGDK_FACTOR_DENSE) PSGDK_TRY(refresh_p_dense(g, f, o->tri, sel, nb, st));
  return PSGDK_OK;
}

int psgdk_kron2d_update_groups(int ngroups, const psgdk_kron2d_t* const* groups,
                               const psgdk_update_opts_t* const* opts, const void* const* const* noise,
                               const float* const* const* V, void* ws, size_t* ws_bytes, psgdk_stream_t stream) {
  if (ngroups < 1 || ngroups > PSGDK_MAX_GROUPS)
    return fail(PSGDK_EINVAL, "ngroups = %d: must be in 1..%d", ngroups, PSGDK_MAX_GROUPS);
  if (!groups || !opts) return fail(PSGDK_EINVAL, "null groups or options");
  if (!ws_bytes) return fail(PSGDK_EINVAL, "ws_bytes is null");
  for (int i = 0; i < ngroups; ++i) {
    PSGDK_TRY(check_group(groups[i]));
    const psgdk_update_opts_t* o = opts[i];
    if (!o) return fail(PSGDK_EINVAL, "null options of group %d", i);
    if (o->r2 != 0 && o->r2 != 1) return fail(PSGDK_EINVAL, "r2 = %d (0: procrustes_step2, 1: procrustes_step_r2)", o->r2);
    if (o->lr != opts[0]->lr || o->betaL != opts[0]->betaL || o->r2 != opts[0]->r2 || o->tri != opts[0]->tri)
      return fail(PSGDK_EINVAL, "group %d: lr, betaL, r2 and tri must be the same for every group of one call", i);
    if (!b16_group(groups[i], o->tri))
      return fail(PSGDK_EINVAL, "group %d is not a bf16-path group (bf16 precision, two dense factors with bf16 "
                  "shadows, sides multiples of 8, full storage)", i);
  }
  if (ws && (!noise || !V)) return fail(PSGDK_EINVAL, "null noise or V");
  return b16_update_groups(ngroups, groups, opts, noise, V, ws, ws_bytes, (hipStream_t)stream);
}

int psgdk_kron2d_update_groups_drawn(int ngroups, const psgdk_kron2d_t* const* groups,
                                     const psgdk_update_opts_t* const* opts, const void* const* const* noise,
                                     const psgdk_draws_t* const* draws, const float* const* const* V, void* ws,
                                     size_t* ws_bytes, psgdk_stream_t stream, psgdk_event_t const* group_done) {
  // the checks of psgdk_kron2d_update_groups (its size query takes no noise), then the call
  size_t need = 0;
  PSGDK_TRY(psgdk_kron2d_update_groups(ngroups, groups, opts, nullptr, nullptr, nullptr, &need, stream));
  if (!ws) { *ws_bytes = need; return PSGDK_OK; }
  if (*ws_bytes < need) return fail(PSGDK_EWORKSPACE, "workspace %zu < %zu bytes", *ws_bytes, need);
  if (!V) return fail(PSGDK_EINVAL, "null V");
  if (!noise && !draws) return fail(PSGDK_EINVAL, "null noise and draws");
  return b16_update_groups(ngroups, groups, opts, noise, V, ws, ws_bytes, (hipStream_t)stream,
                           reinterpret_cast<const hipEvent_t*>(group_done), draws);
}

int psgdk_kron2d_update_groups_ev(int ngroups, const psgdk_kron2d_t* const* groups,
                                  const psgdk_update_opts_t* const* opts, const void* const* const* noise,
                                  const float* const* const* V, void* ws, size_t* ws_bytes, psgdk_stream_t stream,
                                  psgdk_event_t const* group_done) {
  if (!group_done) return fail(PSGDK_EINVAL, "null group_done array");
  if (!ws) return psgdk_kron2d_update_groups(ngroups, groups, opts, noise, V, ws, ws_bytes, stream);
  // the checks of psgdk_kron2d_update_groups, then the call with the completion events
  size_t need = 0;
  PSGDK_TRY(psgdk_kron2d_update_groups(ngroups, groups, opts, noise, V, nullptr, &need, stream));
  if (*ws_bytes < need) return fail(PSGDK_EWORKSPACE, "workspace %zu < %zu bytes", *ws_bytes, need);
  if (!noise || !V) return fail(PSGDK_EINVAL, "null noise or V");
  return b16_update_groups(ngroups, groups, opts, noise, V, ws, ws_bytes, (hipStream_t)stream,
                           reinterpret_cast<const hipEvent_t*>(group_done));
}

int psgdk_kron2d_apply(const psgdk_kron2d_t* g, const psgdk_apply_opts_t* o, void* const* params,
                       float* const* pre_out, float* const* clipped_out, void* ws, size_t* ws_bytes,
                       psgdk_stream_t stream) {
  PSGDK_TRY(check_group(g));
  if (!o) return fail(PSGDK_EINVAL, "null options");
  if (!ws_bytes) return fail(PSGDK_EINVAL, "ws_bytes is null");
  if (b16_group(g, o->tri)) return b16_apply(g, o, params, pre_out, clipped_out, ws, ws_bytes, (hipStream_t)stream);
  const int nb = g->nb;
  const int64_t m = g->m, n = g->n, mn = m * n;
  Ws w(ws);
  float *tmp[MAXB], *pre[MAXB], *part[MAXB];
  const int np_max = std::max(gemm_tiles(m, n, 0), 256);
  for (int b = 0; b < nb; ++b) {
    tmp[b] = w.take<float>(mn);
    pre[b] = w.take<float>(mn);
    part[b] = w.take<float>(2 * (size_t)np_max);
  }
  if (!ws) { *ws_bytes = w.off; return PSGDK_OK; }
  if (*ws_bytes < w.off) return fail(PSGDK_EWORKSPACE, "workspace %zu < %zu bytes", *ws_bytes, w.off);
  PSGDK_TRY(check_ptrs(params, nb, "params"));
  hipStream_t st = (hipStream_t)stream;
  for (int b = 0; b < nb; ++b)
    if (pre_out && pre_out[b]) pre[b] = pre_out[b];
  int np = 0;
  PSGDK_TRY(precondition(g, g->G, g->g_dtype, tmp, pre, part, o->tri, &np, st));
  EwArgs a;
  std::memset(&a, 0, sizeof a);
  a.nb = nb; a.m = m; a.n = n; a.dt = g->p_dtype; a.i0 = np;
  a.f0 = o->max_avg_amp; a.f1 = o->max_element_amp; a.f2 = o->lr_params;
  for (int b = 0; b < nb; ++b) {
    a.in[b] = params[b]; a.in2[b] = pre[b]; a.in3[b] = part[b];
    a.out2[b] = clipped_out ? clipped_out[b] : nullptr;
  }
  return hip_check(clip_update_launch(a, st), "clip + update");
}

int psgdk_factor_update(int prec, int64_t d, int nb, const float* const* term1, int term1_tri,
                        const float* const* Q, float* const* Q_out, float* const* L, const float* const* V, float lr,
                        float betaL, float term2, void* ws, size_t* ws_bytes, psgdk_stream_t stream) {
  PSGDK_TRY(check_prec(prec));
  PSGDK_TRY(check_nb(nb));
  PSGDK_TRY(check_dims(d, "d"));
  if (!ws_bytes) return fail(PSGDK_EINVAL, "ws_bytes is null");
  Ws w(ws);
  FacWs fw;
  fac_take(w, d, nb, fw);
  if (!ws) { *ws_bytes = w.off; return PSGDK_OK; }
  if (*ws_bytes < w.off) return fail(PSGDK_EWORKSPACE, "workspace %zu < %zu bytes", *ws_bytes, w.off);
  PSGDK_TRY(check_ptrs(term1, nb, "term1"));
  PSGDK_TRY(check_ptrs(Q, nb, "Q"));
  PSGDK_TRY(check_ptrs(Q_out, nb, "Q_out"));
  PSGDK_TRY(check_ptrs(L, nb, "L"));
  PSGDK_TRY(check_ptrs(V, nb, "V"));
  for (int b = 0; b < nb; ++b)
    if (Q_out[b] == Q[b]) return fail(PSGDK_EINVAL, "Q_out[%d] aliases Q[%d]", b, b);
  return factor_update_run(prec, nb, d, term1, term1_tri ? 1 : 0, Q, Q_out, L, V, lr, betaL, term2, fw,
                           (hipStream_t)stream);
}

static int procrustes_entry(int prec, int64_t d, int nb, const float* const* Q, float* const* Q_out,
                            const float* const* V, void* ws, size_t* ws_bytes, hipStream_t st, bool r2) {
  PSGDK_TRY(check_prec(prec));
  PSGDK_TRY(check_nb(nb));
  PSGDK_TRY(check_dims(d, "d"));
  if (!ws_bytes) return fail(PSGDK_EINVAL, "ws_bytes is null");
  Ws w(ws);
  FacWs fw;
  fac_take(w, d, nb, fw);
  if (!ws) { *ws_bytes = w.off; return PSGDK_OK; }
  if (*ws_bytes < w.off) return fail(PSGDK_EWORKSPACE, "workspace %zu < %zu bytes", *ws_bytes, w.off);
  PSGDK_TRY(check_ptrs(Q, nb, "Q"));
  PSGDK_TRY(check_ptrs(Q_out, nb, "Q_out"));
  PSGDK_TRY(check_ptrs(V, nb, "V"));
  for (int b = 0; b < nb; ++b)
    if (Q_out[b] == Q[b]) return fail(PSGDK_EINVAL, "Q_out[%d] aliases Q[%d]", b, b);
  return procrustes_run(prec, nb, d, Q, Q_out, V, fw, st, r2);
}

int psgdk_procrustes_r2(int prec, int64_t d, int nb, const float* const* Q, float* const* Q_out,
                        const float* const* V, void* ws, size_t* ws_bytes, psgdk_stream_t stream) {
  return procrustes_entry(prec, d, nb, Q, Q_out, V, ws, ws_bytes, (hipStream_t)stream, true);
}

int psgdk_procrustes(int prec, int64_t d, int nb, const float* const* Q, float* const* Q_out, const float* const* V,
                     void* ws, size_t* ws_bytes, psgdk_stream_t stream) {
  return procrustes_entry(prec, d, nb, Q, Q_out, V, ws, ws_bytes, (hipStream_t)stream, false);
}

int psgdk_apply2d(const psgdk_kron2d_t* g, const psgdk_apply_opts_t* o, void* const* params, float* const* pre_out,
                  float* const* clipped_out, void* ws, size_t* ws_bytes, psgdk_stream_t stream) {
  return psgdk_kron2d_apply(g, o, params, pre_out, clipped_out, ws, ws_bytes, stream);
}

int psgdk_kron2d_refresh_p(const psgdk_kron2d_t* g, int factor_mask, int tri, psgdk_stream_t stream) {
  PSGDK_TRY(check_group(g, false));
  int sel[MAXB];
  for (int b = 0; b < g->nb; ++b) sel[b] = b;
  for (int f = 0; f < 2; ++f) {
    if (!(factor_mask & (1 << f))) continue;
    if (g->kind[f] == PSGDK_FACTOR_DENSE) PSGDK_TRY(refresh_p_dense(g, f, tri, sel, g->nb, (hipStream_t)stream));
    else if (g->kind[f] == PSGDK_FACTOR_DIAG) PSGDK_TRY(refresh_p_diag(g, f, sel, g->nb, (hipStream_t)stream));
  }
  return PSGDK_OK;
}

int psgdk_kron2d_balance(const psgdk_kron2d_t* g, const int32_t* flags, int tri, void* ws, size_t* ws_bytes,
                         psgdk_stream_t stream) {
  PSGDK_TRY(check_group(g, false));
  if (!ws_bytes) return fail(PSGDK_EINVAL, "ws_bytes is null");
  constexpr int PB = 1024;  // partial maxima per factor (workgroups of its max |q| pass)
  Ws w(ws);
  float *part[MAXB], *sc[MAXB];
  for (int b = 0; b < g->nb; ++b) { part[b] = w.take<float>(2 * PB); sc[b] = w.take<float>(4); }
  if (!ws) { *ws_bytes = w.off; return PSGDK_OK; }
  if (*ws_bytes < w.off) return fail(PSGDK_EWORKSPACE, "workspace %zu < %zu bytes", *ws_bytes, w.off);
  if (!flags) return fail(PSGDK_EINVAL, "null flags");
  int fac[2], order = 0;
  for (int f = 0; f < 2; ++f)
    if (g->kind[f] != PSGDK_FACTOR_NONE) fac[order++] = f;
  if (order < 2) return PSGDK_OK;  // psgd_pro.py:101: a single factor is left alone
  int sel[MAXB], nsel = 0;
  for (int b = 0; b < g->nb; ++b)
    if (flags[b]) sel[nsel++] = b;
  if (!nsel) return PSGDK_OK;
  hipStream_t st = (hipStream_t)stream;
  const int64_t dims[2] = {g->m, g->n};
  for (int i = 0; i < order; ++i) {
    const int f = fac[i];
    const int64_t sz = g->kind[f] == PSGDK_FACTOR_DENSE ? dims[f] * dims[f] : dims[f];
    EwArgs a;
    std::memset(&a, 0, sizeof a);
    a.nb = nsel; a.m = 1; a.n = sz; a.i0 = PB;
    for (int j = 0; j < nsel; ++j) { a.in[j] = g->Q[f][sel[j]]; a.out[j] = part[sel[j]] + i * PB; }
    PSGDK_HIP(absmax_launch(a, st), "balance absmax");
  }
  {
    EwArgs a;
    std::memset(&a, 0, sizeof a);
    a.nb = nsel; a.i0 = PB; a.i1 = order;
    for (int j = 0; j < nsel; ++j) { a.in2[j] = part[sel[j]]; a.out[j] = sc[sel[j]]; }
    PSGDK_HIP(balance_scalar_launch(a, st), "balance scalars");
  }
  for (int i = 0; i < order; ++i) {
    const int f = fac[i];
    const int64_t sz = g->kind[f] == PSGDK_FACTOR_DENSE ? dims[f] * dims[f] : dims[f];
    EwArgs a;
    std::memset(&a, 0, sizeof a);
    a.nb = nsel; a.m = 1; a.n = sz; a.i1 = i;
    for (int j = 0; j < nsel; ++j) { a.out[j] = g->Q[f][sel[j]]; a.sc[j] = sc[sel[j]]; }
    PSGDK_HIP(scale_by_dev_launch(a, st), "balance scale");
  }
  for (int i = 0; i < order; ++i) {
    const int f = fac[i];
    if (g->kind[f] == PSGDK_FACTOR_DENSE) PSGDK_TRY(refresh_p_dense(g, f, tri, sel, nsel, st));
    else PSGDK_TRY(refresh_p_diag(g, f, sel, nsel, st));
  }
  return PSGDK_OK;
}

int psgdk_momentum(int64_t numel, float beta, int g_dtype, int nb, float* const* mom, const void* const* g,
                   psgdk_stream_t stream) {
  PSGDK_TRY(check_nb(nb));
  PSGDK_TRY(check_dims(numel, "numel"));
  PSGDK_TRY(check_dt(g_dtype, "g"));
  PSGDK_TRY(check_ptrs(mom, nb, "mom"));
  PSGDK_TRY(check_ptrs(g, nb, "g"));
  EwArgs a;
  std::memset(&a, 0, sizeof a);
  a.nb = nb; a.m = 1; a.n = numel; a.dt = g_dtype; a.f0 = beta;
  for (int b = 0; b < nb; ++b) { a.in[b] = g[b]; a.out[b] = mom[b]; }
  return hip_check(momentum_launch(a, (hipStream_t)stream), "momentum");
}

int psgdk_fill_normal(void* out, int64_t n, int dtype, uint64_t seed, uint64_t stream_id, psgdk_stream_t stream) {
  PSGDK_TRY(check_dt(dtype, "out"));
  if (n < 0) return fail(PSGDK_ESHAPE, "n = %lld: must be >= 0", (long long)n);
  if (n == 0) return PSGDK_OK;
  if (!out) return fail(PSGDK_EINVAL, "null out");
  if (reinterpret_cast<uintptr_t>(out) % (dtype == PSGDK_BF16 ? 8 : 16))
    return fail(PSGDK_EINVAL, "out must be %d-byte aligned", dtype == PSGDK_BF16 ? 8 : 16);
  return hip_check(normal_fill_launch(out, n, dtype, seed, stream_id, (hipStream_t)stream), "normal fill");
}

int psgdk_momentum_multi(int nb, const int64_t* numel, float beta, const int32_t* g_dtype, float* const* mom,
                         const void* const* g, psgdk_stream_t stream) {
  if (nb < 1 || nb > MAXB) return fail(PSGDK_EINVAL, "nb = %d: must be in 1..%d", nb, MAXB);
  if (!numel || !g_dtype) return fail(PSGDK_EINVAL, "null numel or g_dtype array");
  PSGDK_TRY(check_ptrs(mom, nb, "mom"));
  PSGDK_TRY(check_ptrs(g, nb, "g"));
  MomList a;
  std::memset(&a, 0, sizeof a);
  a.nb = nb; a.beta = beta; a.vec = 1;
  for (int t = 0; t < nb; ++t) {
    PSGDK_TRY(check_dims(numel[t], "numel"));
    PSGDK_TRY(check_dt(g_dtype[t], "g"));
    a.off[t + 1] = a.off[t] + (numel[t] + 3) / 4 * 4;
    a.n[t] = numel[t];
    a.dt[t] = g_dtype[t]; a.g[t] = g[t]; a.m[t] = mom[t];
    const uintptr_t ga = reinterpret_cast<uintptr_t>(g[t]), ma = reinterpret_cast<uintptr_t>(mom[t]);
    if (ma % 16 || ga % (g_dtype[t] == PSGDK_BF16 ? 8 : 16)) a.vec = 0;
  }
  return hip_check(momentum_multi_launch(a, (hipStream_t)stream), "momentum (multi-tensor)");
}

int psgdk_set_option(int option, int value) {
  if (option == 0) {
    if (value < 0 || value > 2) return fail(PSGDK_EINVAL, "option 0 (bf16 tile order) must be 0 .. 2");
    g_tile_order = value;
    return PSGDK_OK;
  }
  if (option == 1) {
    if (value < -1 || value > 4) return fail(PSGDK_EINVAL, "option 1 (bf16 tile config) must be -1 .. 4");
    g_force_cfg = value;
    return PSGDK_OK;
  }
  if (option == 2) {
    if (value < 1) return fail(PSGDK_EINVAL, "option 2 (V A workgroup target) must be >= 1");
    g_nlb_target = value;
    return PSGDK_OK;
  }
  if (option == 3) {
    if (value != 2 && value != 4 && value != 8) return fail(PSGDK_EINVAL, "option 3 (V A load batch) must be 2, 4 or 8");
    g_vmm_u = value;
    return PSGDK_OK;
  }
  if (option == 8) {
    if (value < 0 || value > 1) return fail(PSGDK_EINVAL, "option 8 (fp32 k-contiguous kernel) must be 0 or 1");
    g_f32kc = value;
    return PSGDK_OK;
  }
  if (option == 4) {
    if (value < -1 || value > 3) return fail(PSGDK_EINVAL, "option 4 (V A kernel) must be -1 .. 3");
    g_vmm_cols = value;
    return PSGDK_OK;
  }
  if (option == 5) {
    if (value != 0 && value != 1) return fail(PSGDK_EINVAL, "option 5 (term1 Q through Pg) must be 0 or 1");
    g_t1q_pg = value;
    return PSGDK_OK;
  }
  if (option == 7) {
    if (value != 0 && value != 1) return fail(PSGDK_EINVAL, "option 7 (R Q in bf16) must be 0 or 1");
    g_rq16 = value;
    return PSGDK_OK;
  }
  if (option == 9) {
    if (value < 1 || value > MAXB) return fail(PSGDK_EINVAL, "option 9 (items per large-side batch) must be 1 .. %d", MAXB);
    g_big_batch = value;
    return PSGDK_OK;
  }
  if (option == 10) {
    if (value < 0) return fail(PSGDK_EINVAL, "option 10 (small-problem kernel threshold) must be >= 0");
    g_small = value;
    return PSGDK_OK;
  }
  if (option == 11) {
    if (value < 0) return fail(PSGDK_EINVAL, "option 11 (tiny-product kernel threshold) must be >= 0");
    g_tiny = value;
    return PSGDK_OK;
  }
  if (option == 12) {
    if (value != 0 && value != 1) return fail(PSGDK_EINVAL, "option 12 (warp-specialized main loop) must be 0 or 1");
    g_ws = value;
    return PSGDK_OK;
  }
  if (option == 6) {
    if (value < 0 || value > 8) return fail(PSGDK_EINVAL, "option 6 (grouped update side streams) must be 0 .. 8");
    g_upd_streams = value;
    return PSGDK_OK;
  }
  return fail(PSGDK_EINVAL, "unknown option %d", option);
}

int psgdk_get_option(int option, int* value) {
  if (!value) return fail(PSGDK_EINVAL, "value is null");
  const int* opts[] = {&g_tile_order, &g_force_cfg,   &g_nlb_target, &g_vmm_u, &g_vmm_cols,
                       &g_t1q_pg,     &g_upd_streams, &g_rq16,       &g_f32kc, &g_big_batch, &g_small,
                       &g_tiny,       &g_ws};
  if (option < 0 || option >= (int)(sizeof opts / sizeof opts[0])) return fail(PSGDK_EINVAL, "unknown option %d", option);
  *value = *opts[option];
  return PSGDK_OK;
}

int psgdk_profile_start(void) {
  for (auto& r : g_prof.recs) { g_prof.pool.push_back(r.a); g_prof.pool.push_back(r.b); }
  g_prof.recs.clear();
  g_prof.on = true;
  return PSGDK_OK;
}

int psgdk_profile_stop(psgdk_prof_record_t* out, int max_records, int* n_records) {
  g_prof.on = false;
  if (!n_records) return fail(PSGDK_EINVAL, "n_records is null");
  const int n = (int)g_prof.recs.size();
  *n_records = n;
  if (!out) return PSGDK_OK;
  if (max_records < n) return fail(PSGDK_EINVAL, "max_records %d < %d records", max_records, n);
  for (int i = 0; i < n; ++i) {
    ProfRec& r = g_prof.recs[i];
    PSGDK_HIP(hipEventSynchronize(r.b), "profiling sync");
    float ms = 0.f;
    PSGDK_HIP(hipEventElapsedTime(&ms, r.a, r.b), "profiling elapsed");
    out[i].kernel_id = r.kernel_id;
    out[i].tri = r.tri;
    out[i].nb = r.nb;
    out[i].ms = ms;
    out[i].flops = r.flops;
    out[i].bytes = r.bytes;
    out[i].m = r.m;
    out[i].n = r.n;
    out[i].k = r.k;
    out[i].workgroups = r.shape.workgroups;
    out[i].per_cu = r.shape.per_cu;
  }
  return PSGDK_OK;
}

int psgdk_mfma_rate(int iters, int wgs, float* out, psgdk_stream_t stream) {
  if (iters < 1 || wgs < 1) return fail(PSGDK_EINVAL, "iters = %d, wgs = %d: both must be >= 1", iters, wgs);
  if (!out) return fail(PSGDK_EINVAL, "null pointer");
  return hip_check(mfma_rate_launch(iters, wgs, out, (hipStream_t)stream), "mfma rate");
}

int psgdk_read_rate(const void* buf, int64_t bytes, int wgs, int iters, int64_t stride, uint32_t* sink,
                    psgdk_stream_t stream) {
  if (!buf || !sink) return fail(PSGDK_EINVAL, "null pointer");
  if (bytes < 4096 || (bytes & (bytes - 1)) != 0)
    return fail(PSGDK_EINVAL, "bytes = %lld: must be a power of two >= 4096", (long long)bytes);
  if (wgs < 1 || iters < 1 || stride < 1)
    return fail(PSGDK_EINVAL, "wgs = %d, iters = %d, stride = %lld: each must be >= 1", wgs, iters, (long long)stride);
  return hip_check(read_rate_launch(buf, bytes, wgs, iters, stride, sink, (hipStream_t)stream), "read rate");
}

int psgdk_clock_sample(int samples, uint64_t* out, psgdk_stream_t stream) {
  if (!out) return fail(PSGDK_EINVAL, "null pointer");
  if (samples < 1 || samples > (1 << 24)) return fail(PSGDK_EINVAL, "samples = %d: must be in 1 .. 2^24", samples);
  return hip_check(clock_sample_launch(samples, reinterpret_cast<unsigned long long*>(out), (hipStream_t)stream),
                   "clock sample");
}

int psgdk_wall_clock_rate(int* khz) {
  if (!khz) return fail(PSGDK_EINVAL, "null pointer");
  int dev = 0;
  PSGDK_HIP(hipGetDevice(&dev), "hipGetDevice");
  PSGDK_HIP(hipDeviceGetAttribute(khz, hipDeviceAttributeWallClockRate, dev), "wall clock rate");
  return PSGDK_OK;
}

int psgdk_wall_mark(uint64_t* out, psgdk_stream_t stream) {
  if (!out) return fail(PSGDK_EINVAL, "null pointer");
  return hip_check(wall_mark_launch(reinterpret_cast<unsigned long long*>(out), (hipStream_t)stream), "wall mark");
}

int psgdk_debug_mfma(int prec, const float* A, const float* B, float* C, psgdk_stream_t stream) {
  if (prec != 2) PSGDK_TRY(check_prec(prec));
  if (!A || !B || !C) return fail(PSGDK_EINVAL, "null pointer");
  return hip_check(debug_mfma_launch(A, B, C, prec, (hipStream_t)stream), "debug mfma");
}

}  // extern "C"

// bf16 MFMA GEMM for k-contiguous bf16 operands (the bf16 path of the Kron update and apply).
//
// Every operand arrives in HBM as bf16 rows with k contiguous (producers write transposed copies where a consumer
// needs one), so the main loop is only 16-byte global loads, 16-byte LDS stores and 16-byte LDS fragment reads: no
// conversion, no in-register transposes. Macro tile BM x BN x 64 with WGM x WGN waves, each wave owning a
// (BM/WGM) x (BN/WGN) block of v_mfma_f32_16x16x32_bf16 tiles. The large configuration runs 8 waves of 128 x 64
// (128 fp32 accumulators per lane, two waves per SIMD): while one wave waits on LDS, a barrier or the epilogue's
// memory traffic, the other keeps the SIMD's MFMA pipe busy.
// LDS holds two stages of A and B in 128-byte rows with XOR-swizzled 16-byte chunks (conflict-free fragment
// reads and row writes). Global loads for tile k+1 are in flight while tile k is
// multiplied; one barrier per k tile. The (problem, tile) list is dealt out so each XCD gets a contiguous run.
// Operands: K a multiple of 8, leading dimensions multiples of 8, 16-byte aligned bases, under 2 GiB each (the host
// routes anything else to the general engine); ragged M, N and K edges read zeros through the buffer extent.
#include <type_traits>

#include "gemm_bf16.h"

namespace psgdk {

namespace {

// Element traits of the k-contiguous operands. A k tile is 8 chunks of 16 bytes (one 128-byte LDS row per m or n,
// chunks XOR-swizzled by row, swz): 64 bf16 or 32 fp32. CE: elements per chunk; MPF: MFMAs per pair of 16-byte
// fragments (one v_mfma_f32_16x16x32_bf16, or four v_mfma_f32_16x16x4f32 over the fragment's 4 k values, lane group
// g holding k = 4 g + s for both operands).
template <typename T> struct Kc;
template <> struct Kc<bf16_t> { static constexpr int CE = 8, MPF = 1; using F = bf16x8_t; };
template <> struct Kc<float> { static constexpr int CE = 4, MPF = 4; using F = f32x4_t; };

// Row pitch (floats) of a wave's parked epilogue block of hr x wc: unpadded and swizzled for 64 x 64 blocks (see ei
// in the kernel), padded by 4 otherwise.
constexpr int epi_pitch(int hr, int wc) { return hr == 64 && wc == 64 ? wc : wc + 4; }

__device__ __forceinline__ int remap_xcd(int w, int G) {
  const int cnt = G / 8, rem = G % 8, xcd = w % 8, slot = w / 8;
  return xcd < rem ? xcd * (cnt + 1) + slot : rem * (cnt + 1) + (xcd - rem) * cnt + slot;
}


// LDS slot of the 16-byte k chunk c (0..7) of tile row `row`. Rows are 128 bytes with no padding; the XOR spreads
// the 16 rows of an MFMA fragment read (16 lanes, one chunk each) over 16 distinct 16-byte bank groups, which
// the LDS serves without conflicts (measured: 4 cycles per ds_read_b128, against 8 with rows padded to 144
// bytes); the 8 lanes that write one row still cover its 8 slots.
__device__ __forceinline__ int swz(int row, int c) { return c ^ (row & 7); }
// The 32 x 32 x 16 MFMA's fragment read: 16 lanes read one chunk of 16 consecutive rows. XORing with row bits 1-3
// spreads them over 16 distinct bank groups (with row bits 0-2, rows r and r + 8 met: 2-way conflicts).
__device__ __forceinline__ int swz32(int row, int c) { return c ^ ((row >> 1) & 7); }

// Global -> register -> LDS staging of one ROWS x (8 chunks) tile with buffer loads. Lane `tid` owns the 16-byte
// k chunk tid % 8 of rows tid / 8 + 32 i (i < NV): the lane part of the byte offset is the VGPR offset, the row
// group and the tile's k origin are the scalar offset. A lane whose row is past the operand or whose k chunk is
// past K (K is a multiple of a chunk) gets an offset beyond the buffer extent: it reads zero (or, where the scalar
// part wraps the 32-bit sum, some element of the same buffer), and either way only feeds outputs that are not
// stored.
template <typename T, int ROWS, int NT, bool SW32 = false>
struct Ld {
  static constexpr int CE = Kc<T>::CE, KP = 8 * CE;
  static constexpr int NV = ROWS * 8 / NT;  // 16-byte vectors per thread
  uint4 r[NV];

  // t: the thread's index among the NT threads that load this tile
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, int voff, long long ld, int mn0, int rows, int k0,
                                       int K, int t) {
    const int lrow = t >> 3;
    const bool kok = k0 + (t & 7) * CE < K;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int base = mn0 + i * (NT / 8);
      const bool ok = kok && base + lrow < rows;
      const int soff = (int)(((long long)base * ld + k0) * (long long)sizeof(T));
      r[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, ok ? voff : 0x7fffffff, soff, 0));
    }
  }

  // load() for the producer waves of the warp-specialized loop: the same loads, with the lane's offset passed
  // through an empty asm statement so that the compiler cannot hoist the eight per-row selects out of the k loop
  // (kept across it they take eight more registers per operand, which the producer's two register sets leave no
  // room for)
  __device__ __forceinline__ void load_pinned(__amdgpu_buffer_rsrc_t rs, int voff, long long ld, int mn0, int rows,
                                              int k0, int K, int t) {
    asm volatile("" : "+v"(voff));
    load(rs, voff, ld, mn0, rows, k0, K, t);
  }

  __device__ __forceinline__ void store(T* lds, int t) const {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int v = t + NT * i, row = v >> 3, kv = v & 7;
      *reinterpret_cast<uint4*>(lds + row * KP + (SW32 ? swz32(row, kv) : swz(row, kv)) * CE) = r[i];
    }
  }

  // An fp32 operand stored m- or n-contiguous, X[k][mn] with row stride ld (the rows of the buffer are k): thread t
  // owns the 4 x 4 block of k chunk (t / 4) % 8 and tile rows 4 nb .. + 3, nb = 4 (t / 32) + t % 4. Four 16-byte
  // loads (k rows: each group of 4 lanes reads 64 contiguous bytes, the 8 lanes of one k chunk in a wave 128) are
  // transposed in registers into the block's four k-contiguous chunks, stored in the same swizzled layout (at most
  // 2-way bank conflicts). One block per thread (ROWS = NT / 2); rows past the operand and k past K read zero.
  __device__ __forceinline__ void load_mc(__amdgpu_buffer_rsrc_t rs, long long ld, int mn0, int rows, int k0, int K,
                                          int t) {
    static_assert(std::is_same_v<T, float> && NV == 4 && ROWS * 2 == NT, "m/n-contiguous loader: fp32, one block");
    const int kc = (t >> 2) & 7, nb = (t >> 5) * 4 + (t & 3);
    const bool nok = mn0 + nb * 4 < rows;
    const int soff = (int)(((long long)k0 * ld + mn0) * 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = kc * 4 + i;
      const int voff = (int)(((long long)k * ld + nb * 4) * 4);
      r[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, nok && k0 + k < K ? voff : 0x7fffffff,
                                                                                soff, 0));
    }
  }
  __device__ __forceinline__ void store_mc(T* lds, int t) const {
    const int kc = (t >> 2) & 7, nb = (t >> 5) * 4 + (t & 3);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = nb * 4 + j;
      const uint4 x = make_uint4((&r[0].x)[j], (&r[1].x)[j], (&r[2].x)[j], (&r[3].x)[j]);
      *reinterpret_cast<uint4*>(lds + row * KP + swz(row, kc) * CE) = x;
    }
  }
};

}  // namespace

// WGM x WGN waves, each owning a TM x TN block (TM = BM / WGM, TN = BN / WGN) of 16 x 16 MFMA tiles; T = bf16_t
// (the bf16 kernel) or float (its fp32 twin for k-contiguous fp32 operands: the same tiles, LDS layout, schedule
// and epilogues, four fp32 MFMAs per fragment pair).
// LAY (fp32 only): bit 0 set = A stored m-contiguous, bit 1 = B stored n-contiguous (the buffer's rows are k).
// PW > 0 (bf16, 256 x 256 tiles on 2 x 4 waves): PW further waves only stage the operands (warp-specialized main
// loop; see below); the WGM x WGN waves multiply on 32 x 32 x 16 MFMAs and run the epilogue.
template <typename T, int BM, int BN, int WGM, int WGN, int EPI, int LAY = 0, int PW = 0>
__device__ __forceinline__ void gemm_kc_body(const GB16Args& p) {
  constexpr int CE = Kc<T>::CE, BK = 8 * CE, KP = BK, MPF = Kc<T>::MPF;
  using F = typename Kc<T>::F;
  constexpr int NT = 64 * WGM * WGN;  // the multiplying waves' threads
  constexpr int TM = BM / WGM, TN = BN / WGN;
  constexpr bool WS = PW > 0;                       // warp-specialized: producer and MFMA waves
  constexpr bool PP = !WS && WGM == 2 && WGN == 4;  // ping-pong main loop (8 waves, two groups of 4)
  static_assert(!WS || (std::is_same_v<T, bf16_t> && PW == 4 &&
                        ((BM == 256 && BN == 256 && WGM == 2 && WGN == 4) || (BM == 128 && BN == 128 && WGM == 2 && WGN == 2))),
                "warp-specialized main loop: bf16, 256 x 256 tiles on 8 MFMA waves or 128 x 128 on 4, 4 producer waves");
  constexpr int FM = TM / 16, FN = TN / 16;  // 16x16 tiles per wave along m, n
  extern __shared__ __align__(16) unsigned char smem[];
  T* const As0 = reinterpret_cast<T*>(smem);
  T* const Bs0 = As0 + 2 * BM * KP;

  const int G = p.ntiles * p.nb;
  const int logical = p.vec ? remap_xcd(blockIdx.x, G) : (int)blockIdx.x;
  const int b = logical / p.ntiles, tile = logical % p.ntiles;
  // this problem's k extent and leading dimensions (kper: its own K, rows of exactly K)
  const int K = p.kper ? p.kp[b] : p.K;
  const long long lda = p.kper ? (long long)K : p.lda, ldb = p.kper ? (long long)K : p.ldb;
  int ti, tj;
  if (p.tri) {
    ti = 0;
    int rem = tile, rowlen = p.tiles_m;
    while (rem >= rowlen) { rem -= rowlen; ++ti; --rowlen; }
    tj = ti + rem;
  } else if (p.vec == 2) {
    // groups of GM tile rows, column-major inside a group: the 32 workgroups an XCD runs at once cover a
    // GM x 8 block of tiles, so each k step fetches GM + 8 operand panel slices into that XCD's L2
    constexpr int GM = 4;
    const int grp = tile / (GM * p.tiles_n), r0 = grp * GM;
    const int gm = min(GM, p.tiles_m - r0), idx = tile - r0 * p.tiles_n;
    ti = r0 + idx % gm;
    tj = idx / gm;
  } else {
    ti = tile / p.tiles_n;
    tj = tile % p.tiles_n;
  }
  const int m0 = ti * BM, n0 = tj * BN;
  const T* __restrict__ Ap = reinterpret_cast<const T*>(p.A[b]);
  const T* __restrict__ Bp = reinterpret_cast<const T*>(p.tri ? p.A[b] : p.B[b]);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // a producer wave (WS): the test is on a scalar copy of the wave index, so both roles are scalar branches
  const bool producer = WS && __builtin_amdgcn_readfirstlane(wave) >= WGM * WGN;
  const int wm = wave / WGN, wn = wave % WGN;
  const int r = lane & 15, g = lane >> 4;

  f32x4_t acc[FM][FN];
  // fp32 operands sum k in blocks of 128 (four k tiles) into `part`, folded into `acc` after each block, as the
  // general fp32 engine does: one fp32 chain over all of K carries several times the rounding error against an
  // fp64 product (measured 7.6x at K = 3072). The 128-tile configuration has the registers for the second set.
  constexpr bool BLK = std::is_same_v<T, float>;
  static_assert(!BLK || !PP, "blocked fp32 summation needs the 128-tile configuration");
  constexpr int KC_TILES = 128 / BK;
  f32x4_t part[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = part[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  auto& dst = BLK ? part : acc;  // the MFMA accumulators of the main loop
  // WS: FM32 x FN32 tiles of 32 x 32 per wave (element m of lane l at row 8 (m / 4) + 4 (l / 32) + m % 4, column
  // l % 32)
  constexpr int FM32 = WS ? TM / 32 : 1, FN32 = WS ? TN / 32 : 1;
  f32x16_t acc32[FM32][FN32];
  if constexpr (WS) {
#pragma unroll
    for (int i = 0; i < FM32; ++i)
#pragma unroll
      for (int j = 0; j < FN32; ++j)
#pragma unroll
        for (int m = 0; m < 16; ++m) acc32[i][j][m] = 0.f;
  }

  // k tiles of this output tile: all of K, or (kbeg: A upper-triangular, zero left of the tile's first row) from the
  // k tile holding m0; kb is the k origin of the first one
  const int kfirst = p.kbeg ? m0 / BK : 0, kb = kfirst * BK;
  const int nk = (K + BK - 1) / BK - kfirst;
  // fp32 operands may be stored m- / n-contiguous (amc, bmc: the buffer's rows are k)
  constexpr bool amc = (LAY & 1) != 0, bmc = (LAY & 2) != 0;  // a SYRK (B = A) has both bits or neither
  static_assert(LAY == 0 || std::is_same_v<T, float>, "m/n-contiguous operands: fp32 only");
  const __amdgpu_buffer_rsrc_t rsA =
      make_rsrc(Ap, (long long)(amc ? K : p.M) * lda * (long long)sizeof(T));
  const __amdgpu_buffer_rsrc_t rsB =
      make_rsrc(Bp, (long long)(bmc ? K : (p.tri ? p.M : p.N)) * ldb * (long long)sizeof(T));
  // acc += a b over one pair of 16-byte fragments (32 k of bf16, or 16 k of fp32 in four steps)
  auto mma = [](f32x4_t& c, const F& a, const F& bb) {
    if constexpr (MPF == 1) {
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bb, c, 0, 0, 0);
    } else {
#pragma unroll
      for (int s = 0; s < MPF; ++s) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], bb[s], c, 0, 0, 0);
    }
  };
  const int rowsB = p.tri ? p.M : p.N;
  // 2 steps of 4 chunks per k tile from LDS (B fragments held, A fragments streamed one row ahead)
  auto mma_tile = [&](const T* As, const T* Bs) {
#pragma unroll 1
    for (int ks = 0; ks < 2; ++ks) {
      // fragment rows are 16-aligned plus r, so their swizzle is that of r
      const int ko = swz(r, ks * 4 + g) * CE;
      F bfr[FN];
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bfr[j] = *reinterpret_cast<const F*>(Bs + (wn * TN + j * 16 + r) * KP + ko);
      F a_cur = *reinterpret_cast<const F*>(As + (wm * TM + r) * KP + ko);
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        F a_nxt = a_cur;
        if (i + 1 < FM)
          a_nxt = *reinterpret_cast<const F*>(As + (wm * TM + (i + 1) * 16 + r) * KP + ko);
#pragma unroll
        for (int j = 0; j < FN; ++j) mma(dst[i][j], a_cur, bfr[j]);
        a_cur = a_nxt;
      }
    }
  };
  // Ping-pong compute phase: the other wave on the SIMD is moving data, so this wave alone must keep the MFMA
  // pipe fed. All 2 x FM A rows of the tile are streamed 3 rows ahead of their MFMAs; the second step's B
  // fragments are read during the first step. sched_group_barrier pins the order: reads go out ahead of the
  // MFMAs that hide their latency.
  auto mma_tile_pp = [&](const T* As, const T* Bs) {
    constexpr int NQ = 2 * FM, LA = 3;
    F bq[2][FN], aq[NQ];
    auto rd_b = [&](int ks) {
      const int ko = swz(r, ks * 4 + g) * CE;
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bq[ks][j] = *reinterpret_cast<const F*>(Bs + (wn * TN + j * 16 + r) * KP + ko);
    };
    auto rd_a = [&](int q) {
      const int ks = q / FM, i = q % FM;
      aq[q] = *reinterpret_cast<const F*>(As + (wm * TM + i * 16 + r) * KP + swz(r, ks * 4 + g) * CE);
    };
    rd_b(0);
#pragma unroll
    for (int q = 0; q < LA; ++q) rd_a(q);
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      if (q + LA < NQ) rd_a(q + LA);
      if (q == FM / 2) rd_b(1);
      const int ks = q / FM, i = q % FM;
#pragma unroll
      for (int j = 0; j < FN; ++j)
        mma(acc[i][j], aq[q], bq[ks][j]);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, FN + LA, 0);
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      if (q + LA < NQ && q == FM / 2) __builtin_amdgcn_sched_group_barrier(0x100, FN + 1, 0);
      else if (q + LA < NQ) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      else if (q == FM / 2) __builtin_amdgcn_sched_group_barrier(0x100, FN, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, FN * MPF, 0);
    }
  };
  if constexpr (WS) {
    // Warp-specialized: the PW = 4 producer waves (one per SIMD) move every operand tile from HBM into LDS and
    // multiply nothing; the 8 MFMA waves (two per SIMD, each 128 x 64 of the output as 4 x 2 tiles of 32 x 32)
    // multiply from LDS and load nothing. One barrier per k tile: in the phase of tile kt the MFMA waves read LDS
    // stage kt & 1 while the producers write tile kt + 1 into stage (kt + 1) & 1 and then request tile kt + 3. The
    // producers hold two tiles in registers (two sets of 16 x 16 bytes per thread), so a tile's loads have two phases
    // to arrive; the roles live in separate loops, so no wave holds both the accumulators and the staging registers.
    // LDS rows are swizzled for the 32-row fragment reads (swz32). Loads past the last tile read zeros and their
    // stage is never read.
    if (producer) {
      constexpr int NTP = 64 * PW;
      const int t = tid - NT;
      const int voffA = (int)(((long long)(t >> 3) * lda + (t & 7) * CE) * (long long)sizeof(T));
      const int voffB = (int)(((long long)(t >> 3) * ldb + (t & 7) * CE) * (long long)sizeof(T));
      Ld<T, BM, NTP, true> la0, la1;
      Ld<T, BN, NTP, true> lb0, lb1;
      la0.load_pinned(rsA, voffA, lda, m0, p.M, kb, K, t);
      lb0.load_pinned(rsB, voffB, ldb, n0, rowsB, kb, K, t);
      la1.load_pinned(rsA, voffA, lda, m0, p.M, kb + BK, K, t);
      lb1.load_pinned(rsB, voffB, ldb, n0, rowsB, kb + BK, K, t);
      la0.store(As0, t);
      lb0.store(Bs0, t);
      la0.load_pinned(rsA, voffA, lda, m0, p.M, kb + 2 * BK, K, t);
      lb0.load_pinned(rsB, voffB, ldb, n0, rowsB, kb + 2 * BK, K, t);
      __syncthreads();
      // Two phases per trip, so that the register set of each is static: the first stores set 1 (tile kt + 1),
      // the second set 0. Both are unconditional inside the loop and an odd last phase is peeled after it: with a
      // conditional second phase the compiler's wait counts at the loop head merge a path on which set 1 holds the
      // newest loads, and the first phase then waits for every load in flight (vmcnt(0)), not for its own set only.
      int kt = 0;
      for (; kt + 1 < nk; kt += 2) {
        la1.store(As0 + BM * KP, t);
        lb1.store(Bs0 + BN * KP, t);
        la1.load_pinned(rsA, voffA, lda, m0, p.M, kb + (kt + 3) * BK, K, t);
        lb1.load_pinned(rsB, voffB, ldb, n0, rowsB, kb + (kt + 3) * BK, K, t);
        __syncthreads();
        la0.store(As0, t);
        lb0.store(Bs0, t);
        la0.load_pinned(rsA, voffA, lda, m0, p.M, kb + (kt + 4) * BK, K, t);
        lb0.load_pinned(rsB, voffB, ldb, n0, rowsB, kb + (kt + 4) * BK, K, t);
        __syncthreads();
      }
      if (kt < nk) {
        la1.store(As0 + BM * KP, t);
        lb1.store(Bs0 + BN * KP, t);
        __syncthreads();
      }
    } else {
      // four k steps of 16 per tile; lane (c, hh) reads chunk 2 ks + hh of fragment rows c (row offsets are
      // multiples of 32, so the swizzle is that of c)
      const int c = lane & 31, hh = lane >> 5;
      __syncthreads();
      for (int kt = 0; kt < nk; ++kt) {
        const T* As = As0 + (kt & 1) * BM * KP;
        const T* Bs = Bs0 + (kt & 1) * BN * KP;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const int ko = swz32(c, 2 * ks + hh) * CE;
          F bq[FN32], aq[FM32];
#pragma unroll
          for (int j = 0; j < FN32; ++j) bq[j] = *reinterpret_cast<const F*>(Bs + (wn * TN + 32 * j + c) * KP + ko);
#pragma unroll
          for (int i = 0; i < FM32; ++i) aq[i] = *reinterpret_cast<const F*>(As + (wm * TM + 32 * i + c) * KP + ko);
#pragma unroll
          for (int i = 0; i < FM32; ++i)
#pragma unroll
            for (int j = 0; j < FN32; ++j)
              acc32[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aq[i], bq[j], acc32[i][j], 0, 0, 0);
        }
        __syncthreads();
      }
    }
  } else if constexpr (!PP) {
    const int voffA = (int)(((long long)(tid >> 3) * lda + (tid & 7) * CE) * (long long)sizeof(T));
    const int voffB = (int)(((long long)(tid >> 3) * ldb + (tid & 7) * CE) * (long long)sizeof(T));
    Ld<T, BM, NT> la;
    Ld<T, BN, NT> lb;
    auto load = [&](int k0) {
      if constexpr (amc) la.load_mc(rsA, lda, m0, p.M, k0, K, tid);
      else la.load(rsA, voffA, lda, m0, p.M, k0, K, tid);
      if constexpr (bmc) lb.load_mc(rsB, ldb, n0, rowsB, k0, K, tid);
      else lb.load(rsB, voffB, ldb, n0, rowsB, k0, K, tid);
    };
    auto store = [&](T* as, T* bs) {
      if constexpr (amc) la.store_mc(as, tid);
      else la.store(as, tid);
      if constexpr (bmc) lb.store_mc(bs, tid);
      else lb.store(bs, tid);
    };
    load(kb);
    store(As0, Bs0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int cur = kt & 1;
      const bool more = kt + 1 < nk;
      if (more) load(kb + (kt + 1) * BK);
      mma_tile(As0 + cur * BM * KP, Bs0 + cur * BN * KP);
      if constexpr (BLK) {
        if ((kt + 1) % KC_TILES == 0 || !more) {
#pragma unroll
          for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) {
              acc[i][j] += part[i][j];
              part[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            }
        }
      }
      if (more) store(As0 + (cur ^ 1) * BM * KP, Bs0 + (cur ^ 1) * BN * KP);
      __syncthreads();
    }
  } else {
    // Ping-pong: wave group h = wave / 4 (one wave of each group per SIMD) owns output rows 128 h .. 128 h + 127
    // and loads rows 128 h .. of both operand tiles. The groups run half a tile apart:
    //   group 0: compute(kt) | barrier | memory(kt) | barrier
    //   group 1: memory(kt)  | barrier | compute(kt) | barrier
    // memory(kt) writes the group's half of tile kt + 1 (in registers since two phases) into LDS stage
    // (kt + 1) & 1 and requests its half of tile kt + 2. Between two barriers one group multiplies while the other
    // moves data, so each SIMD's MFMA pipe has a wave with work; the stage being written is never the one read in
    // the same phase. Past the last tile the loads read zeros and their LDS stage is not read again.
    // The group's row offset rides in the lane index t (t / 8 is the tile row), not in the loads' scalar offset:
    // h is uniform per wave but not provably so, and a scalar offset derived from it would be waterfalled.
    const int h = wave >> 2, t = (tid & 255) + h * (NT / 2) * 4;  // rows h * 128 + (tid & 255) / 8 (+ 32 i)
    static_assert(BM == BN && (NT / 2) * 4 == (BM / 2) * 8, "ping-pong loader: one group loads half the rows");
    const int voffA = (int)(((long long)(t >> 3) * lda + (t & 7) * CE) * (long long)sizeof(T));
    const int voffB = (int)(((long long)(t >> 3) * ldb + (t & 7) * CE) * (long long)sizeof(T));
    Ld<T, BM / 2, NT / 2> la;
    Ld<T, BN / 2, NT / 2> lb;
    la.load(rsA, voffA, lda, m0, p.M, kb, K, t);
    lb.load(rsB, voffB, ldb, n0, rowsB, kb, K, t);
    la.store(As0, t);
    lb.store(Bs0, t);
    la.load(rsA, voffA, lda, m0, p.M, kb + BK, K, t);
    lb.load(rsB, voffB, ldb, n0, rowsB, kb + BK, K, t);
    __syncthreads();
    auto memory = [&](int kt) {
      const int nxt = (kt + 1) & 1;
      la.store(As0 + nxt * BM * KP, t);
      lb.store(Bs0 + nxt * BN * KP, t);
      la.load(rsA, voffA, lda, m0, p.M, kb + (kt + 2) * BK, K, t);
      lb.load(rsB, voffB, ldb, n0, rowsB, kb + (kt + 2) * BK, K, t);
    };
    for (int kt = 0; kt < nk; ++kt) {
      const int cur = kt & 1;
      if (h == 0) mma_tile_pp(As0 + cur * BM * KP, Bs0 + cur * BN * KP);
      else memory(kt);
      __syncthreads();
      if (h == 0) memory(kt);
      else mma_tile_pp(As0 + cur * BM * KP, Bs0 + cur * BN * KP);
      __syncthreads();
    }
  }

  // Epilogue through LDS (idle after the main loop), in two halves of each wave's rows so that every wave's
  // (TM/2 x TN) fp32 fit: (1) the wave parks half of its accumulators in its own LDS slot (static register
  // indices only); (2) row pass: each lane takes 4 consecutive columns of a row, applies the epilogue, writes the
  // value back to LDS and stores C / Cb rows (16- and 8-byte stores); (3) column pass: each lane takes 4
  // consecutive rows of a column for the transposed bf16 copy, the SYRK mirror and the Procrustes trace.
  constexpr int HR = TM / 2;       // rows per wave per half
  constexpr int WC = TN;           // columns per wave
  constexpr int EP = epi_pitch(HR, WC);  // LDS row pitch (floats)
  float* const ep = reinterpret_cast<float*>(smem) + wave * HR * EP;
  // LDS slot of element (row, col) of the wave's parked block. For 64 x 64 blocks: rows of 64 floats, the float4
  // group of the column XORed with the row's 4-row group k (its two 2-bit halves swapped), so that parking (16
  // consecutive columns of rows 4 apart), the row pass (whole rows as float4) and the column passes (one column of
  // 16 rows 4 apart) each touch 64 distinct banks; with a padded pitch of 68 the column passes met 4-way conflicts.
  // Other shapes keep the padded pitch.
  auto ei = [](int row, int col) {
    if constexpr (EP == 64) {
      const int k = (row >> 2) & 15, sw = ((k & 3) << 2) | (k >> 2);
      return row * EP + (col ^ (sw << 2));
    } else {
      return row * EP + col;
    }
  };
  float* __restrict__ C = p.C[b];
  bf16_t* __restrict__ Cb = p.Cb[b];
  bf16_t* __restrict__ CTb = p.CTb[b];
  float* __restrict__ CTf = p.CT[b];
  const float* __restrict__ X1 = p.X1[b];
  const float* __restrict__ X2 = p.X2[b];
  float s0 = 0.f, s1 = 0.f;
  if constexpr (EPI == EPI_FACTOR || EPI == EPI_PROC || EPI == EPI_PROCB || EPI == EPI_SCALE || EPI == EPI_RQ ||
                EPI == EPI_STRACE)
    s0 = p.s[b][0];
  if constexpr (EPI == EPI_FACTOR || EPI == EPI_PROC || EPI == EPI_PROCB) s1 = p.s[b][1];
  const bool mirror = p.tri && p.out_mode == 1;
  const bool colpass = CTb != nullptr || CTf != nullptr || mirror || EPI == EPI_RQ || EPI == EPI_STRACE;
  auto al = [](const void* q, int bytes) { return (reinterpret_cast<uintptr_t>(q) & (bytes - 1)) == 0; };
  const bool fast = m0 + BM <= p.M && n0 + BN <= p.N && (!p.tri || ti < tj) &&
                    (!C || ((p.ldc & 3) == 0 && al(C, 16))) && (!Cb || ((p.ldcb & 3) == 0 && al(Cb, 8))) &&
                    (!CTb || ((p.ldct & 3) == 0 && al(CTb, 8))) && (!CTf || ((p.ldct & 3) == 0 && al(CTf, 16))) &&
                    (p.ldx & 3) == 0 &&
                    (!X1 || al(X1, EPI == EPI_RQ && !std::is_same_v<T, float> ? 8 : 16)) && (!X2 || al(X2, 16));
  float t1 = 0.f, t2 = 0.f;
  // one half of each wave's rows; h is a template constant so that the accumulator indices stay static (a loop
  // over h is too large to be unrolled, and a dynamic index would move the accumulators to scratch)
  auto half = [&](auto h_c) {
    constexpr int h = decltype(h_c)::value;
    // (1) park accumulators: tile (i, j) of this half at local row (i - h FM/2) * 16 + 4g + e, column 16 j + r
    // (WS: 32 x 32 tile (i, j) of this half, i = h FM32/2 + ii, element m at local row ii * 32 + 8 (m / 4) + 4 hh +
    // m % 4, column 32 j + c)
    if constexpr (WS) {
      const int c = lane & 31, hh = lane >> 5;
#pragma unroll
      for (int ii = 0; ii < FM32 / 2; ++ii)
#pragma unroll
        for (int j = 0; j < FN32; ++j)
#pragma unroll
          for (int m = 0; m < 16; ++m)
            ep[ei(ii * 32 + 8 * (m >> 2) + 4 * hh + (m & 3), j * 32 + c)] = acc32[h * (FM32 / 2) + ii][j][m];
    } else {
#pragma unroll
      for (int ii = 0; ii < FM / 2; ++ii)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) ep[ei(ii * 16 + g * 4 + e, j * 16 + r)] = acc[h * (FM / 2) + ii][j][e];
    }
    __syncthreads();
    const int grow0 = m0 + wm * TM + h * HR;  // global row of local row 0
    const int gcol0 = n0 + wn * TN;
    // (2) row pass, (3) column pass. An interior tile (fast: inside M and N, strictly above the diagonal for a
    // SYRK, every leading dimension and base 16-byte compatible) needs no per-element checks: its loads and stores
    // are whole vectors (row_pass_fast). Edge tiles check each element (row_pass).
    // The element-wise epilogue of 4 consecutive columns of one row (acc values in v, X1 / X2 values in q1 / q2).
    auto epi_math = [&](float* v, const float* q1, const float* q2, const bool* ok, int row, int col) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if constexpr (EPI == EPI_FACTOR) {
          v[e] = q1[e] - s0 * (v[e] - s1 * q1[e]);
        } else if constexpr (EPI == EPI_PROC) {
          v[e] = ok[e] ? q1[e] + s0 * q2[e] + 0.5f * s0 * s0 * s1 * v[e] : 0.f;
        } else if constexpr (EPI == EPI_PROCB) {  // v holds a RQ + a^2/2 s1 acc (tcol_pass)
          v[e] = ok[e] ? q1[e] + v[e] : 0.f;
        } else if constexpr (EPI == EPI_STRACE) {
          v[e] = (s0 * v[e]) * s0;
        } else if constexpr (EPI == EPI_SCALE || EPI == EPI_RQ) {
          v[e] = s0 * v[e];
          if (EPI == EPI_RQ && ok[e] && row == col + e) t1 += v[e];
        } else {
          v[e] = p.alpha * v[e];
          if (EPI == EPI_SUMSQ && ok[e]) t1 += v[e] * v[e];
        }
      }
    };
    auto row_pass = [&]() {
      constexpr int IT = HR * (WC / 4) / 64;
      static_assert(IT * 64 == HR * (WC / 4), "row pass: whole iterations");
#pragma unroll 4
      for (int it = 0; it < IT; ++it) {
        const int idx = lane + 64 * it;
        const int lr = idx / (WC / 4), lc = (idx % (WC / 4)) * 4;
        const int row = grow0 + lr, col = gcol0 + lc;
        const float4 a = *reinterpret_cast<const float4*>(ep + ei(lr, lc));
        float v[4] = {a.x, a.y, a.z, a.w};
        bool ok[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) ok[e] = row < p.M && col + e < p.N && !(p.tri && row > col + e);
        const long long xo = (long long)row * p.ldx + col;
        float q1[4] = {0.f, 0.f, 0.f, 0.f}, q2[4] = {0.f, 0.f, 0.f, 0.f};
        if constexpr (EPI == EPI_FACTOR || EPI == EPI_PROC || EPI == EPI_PROCB) {
#pragma unroll
          for (int e = 0; e < 4; ++e) q1[e] = ok[e] ? X1[xo + e] : 0.f;
        }
        if constexpr (EPI == EPI_PROC) {
#pragma unroll
          for (int e = 0; e < 4; ++e) q2[e] = ok[e] ? X2[xo + e] : 0.f;
        }
        epi_math(v, q1, q2, ok, row, col);
        if constexpr (EPI == EPI_STRACE) {  // sum C_ij X1_ij over the stored (upper) elements, diagonal included
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (ok[e]) t2 += v[e] * X1[xo + e];
        }
        *reinterpret_cast<float4*>(ep + ei(lr, lc)) = make_float4(v[0], v[1], v[2], v[3]);
        const bool all = ok[0] && ok[1] && ok[2] && ok[3];
        if (C) {
          float* dst = C + (long long)row * p.ldc + col;
          if (all && (p.ldc & 3) == 0) *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
          else
#pragma unroll
            for (int e = 0; e < 4; ++e) if (ok[e]) dst[e] = v[e];
        }
        if (Cb) {
          bf16_t* dst = Cb + (long long)row * p.ldcb + col;
          if (all && (p.ldcb & 3) == 0)
            *reinterpret_cast<uint2*>(dst) = make_uint2(pack2(f32_to_bf16(v[0]), f32_to_bf16(v[1])),
                                                         pack2(f32_to_bf16(v[2]), f32_to_bf16(v[3])));
          else
#pragma unroll
            for (int e = 0; e < 4; ++e) if (ok[e]) dst[e] = f32_to_bf16(v[e]);
        }
      }
    };
    // Interior tiles: the X1 / X2 loads of the next U iterations go out before the current U are processed (two
    // register sets; the batch loop is unrolled so that the set index is static). Stores sit behind branches on
    // C / Cb, which the scheduler does not move loads across, so without this each wave would have only one
    // iteration's loads in flight and the epilogue would run at the latency of HBM.
    // hc, hcb: whether C / Cb are stored, as types when the epilogue loads X1 (then every iteration issues the same
    // stores on every path, so the compiler counts them and each wait covers the one load it needs; with the
    // stores behind branches it cannot, and from the middle of the pass on its waits also cover earlier stores)
    auto row_pass_fast = [&](auto hc, auto hcb) {
      // (two fp32 operands in flight take 4 iterations ahead, within the register budget)
      // (the warp-specialized kernel's three waves per SIMD leave fewer registers: half the depth)
      constexpr int IT = HR * (WC / 4) / 64, U = (EPI == EPI_PROC ? 4 : 8) / (WS ? 2 : 1), NBT = IT / U;
      static_assert(IT % U == 0, "row pass: whole batches");
      constexpr bool L1 = EPI == EPI_FACTOR || EPI == EPI_PROC || EPI == EPI_PROCB || EPI == EPI_STRACE;
      constexpr int HC = decltype(hc)::value, HCB = decltype(hcb)::value;  // 1 stored, 0 not, -1 known at run time
      float4 x1[2][U], x2[2][U];
      auto issue = [&](int set, int it0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int idx = lane + 64 * (it0 + u);
          const int lr = idx / (WC / 4), lc = (idx % (WC / 4)) * 4;
          const long long xo = (long long)(grow0 + lr) * p.ldx + gcol0 + lc;
          if constexpr (L1) x1[set][u] = *reinterpret_cast<const float4*>(X1 + xo);
          if constexpr (EPI == EPI_PROC) x2[set][u] = *reinterpret_cast<const float4*>(X2 + xo);
        }
      };
      // one iteration: 4 columns of one row, X1 / X2 values from register set `set`, slot u
      auto step = [&](int it, int set, int u) {
        const int idx = lane + 64 * it;
        const int lr = idx / (WC / 4), lc = (idx % (WC / 4)) * 4;
        const int row = grow0 + lr, col = gcol0 + lc;
        const float4 a = *reinterpret_cast<const float4*>(ep + ei(lr, lc));
        float v[4] = {a.x, a.y, a.z, a.w};
        const bool ok[4] = {true, true, true, true};
        float q1[4] = {0.f, 0.f, 0.f, 0.f}, q2[4] = {0.f, 0.f, 0.f, 0.f};
        if constexpr (L1) {
          q1[0] = x1[set][u].x; q1[1] = x1[set][u].y; q1[2] = x1[set][u].z; q1[3] = x1[set][u].w;
        }
        if constexpr (EPI == EPI_PROC) {
          q2[0] = x2[set][u].x; q2[1] = x2[set][u].y; q2[2] = x2[set][u].z; q2[3] = x2[set][u].w;
        }
        epi_math(v, q1, q2, ok, row, col);
        if constexpr (EPI == EPI_STRACE) t2 += v[0] * q1[0] + v[1] * q1[1] + v[2] * q1[2] + v[3] * q1[3];
        *reinterpret_cast<float4*>(ep + ei(lr, lc)) = make_float4(v[0], v[1], v[2], v[3]);
        if (HC == 1 || (HC < 0 && C))
          *reinterpret_cast<float4*>(C + (long long)row * p.ldc + col) = make_float4(v[0], v[1], v[2], v[3]);
        if (HCB == 1 || (HCB < 0 && Cb))
          *reinterpret_cast<uint2*>(Cb + (long long)row * p.ldcb + col) =
              make_uint2(pack2(f32_to_bf16(v[0]), f32_to_bf16(v[1])), pack2(f32_to_bf16(v[2]), f32_to_bf16(v[3])));
      };
      if constexpr (L1) {
        issue(0, 0);
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) {
          const int set = bt & 1;
          if (bt + 1 < NBT) issue(set ^ 1, (bt + 1) * U);
#pragma unroll
          for (int u = 0; u < U; ++u) step(bt * U + u, set, u);
        }
      } else {  // nothing to load: a rolled loop (the fully unrolled form measured slower for store-only epilogues)
#pragma unroll 4
        for (int it = 0; it < IT; ++it) step(it, 0, 0);
      }
    };
    // EPI_PROCB: X2 = (R Q)^T in bf16 (the product's own B operand, row stride ldx), so R Q at (row, col) is read at
    // (col, row): a column pass (4 consecutive rows of one column, 8 contiguous bytes) folds a RQ + a^2/2 s1 acc
    // into the parked values before the row pass adds Qn. Interior tiles issue the loads 8 iterations ahead.
    auto tcol_pass = [&](auto fast_c) {
      constexpr bool FAST = decltype(fast_c)::value;
      constexpr int IT = WC * (HR / 4) / 64, U = WS ? 4 : 8, NBT = IT / U;
      static_assert(IT % U == 0, "transposed column pass: whole batches");
      const float c2 = 0.5f * s0 * s0 * s1;
      const bf16_t* __restrict__ X2b = reinterpret_cast<const bf16_t*>(X2);
      auto fold = [&](int it, const float* q2) {
        const int idx = lane + 64 * it;
        const int lc = idx / (HR / 4), lr = (idx % (HR / 4)) * 4;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float& x = ep[ei(lr + e, lc)];
          x = s0 * q2[e] + c2 * x;
        }
      };
      if constexpr (FAST) {
        uint2 xb[2][U];
        auto issue = [&](int set, int it0) {
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const int idx = lane + 64 * (it0 + u);
            const int lc = idx / (HR / 4), lr = (idx % (HR / 4)) * 4;
            xb[set][u] = *reinterpret_cast<const uint2*>(X2b + (long long)(gcol0 + lc) * p.ldx + grow0 + lr);
          }
        };
        issue(0, 0);
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) {
          const int set = bt & 1;
          if (bt + 1 < NBT) issue(set ^ 1, (bt + 1) * U);
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const uint2 t = xb[set][u];
            const float q2[4] = {bf16_to_f32((bf16_t)(t.x & 0xffff)), bf16_to_f32((bf16_t)(t.x >> 16)),
                                 bf16_to_f32((bf16_t)(t.y & 0xffff)), bf16_to_f32((bf16_t)(t.y >> 16))};
            fold(bt * U + u, q2);
          }
        }
      } else {
#pragma unroll 4
        for (int it = 0; it < IT; ++it) {
          const int idx = lane + 64 * it;
          const int lc = idx / (HR / 4), lr = (idx % (HR / 4)) * 4;
          const int col = gcol0 + lc, row = grow0 + lr;
          float q2[4];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            q2[e] = row + e < p.M && col < p.N ? bf16_to_f32(X2b[(long long)col * p.ldx + row + e]) : 0.f;
          fold(it, q2);
        }
      }
    };
    auto col_pass = [&](auto fast_c) {
      constexpr bool FAST = decltype(fast_c)::value;
      constexpr int IT = WC * (HR / 4) / 64;
      static_assert(IT * 64 == WC * (HR / 4), "column pass: whole iterations");
#pragma unroll 4
      for (int it = 0; it < IT; ++it) {
        const int idx = lane + 64 * it;
        const int lc = idx / (HR / 4), lr = (idx % (HR / 4)) * 4;
        const int col = gcol0 + lc, row = grow0 + lr;
        float v[4];
        bool ok[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = ep[ei(lr + e, lc)];
          ok[e] = FAST || (row + e < p.M && col < p.N && !(p.tri && row + e > col));
        }
        const bool all = ok[0] && ok[1] && ok[2] && ok[3];
        if constexpr (EPI == EPI_RQ && std::is_same_v<T, float>) {  // X1: R in fp32, read at (col, row..row+3)
          const float* x = X1 + (long long)col * p.ldx + row;
          if constexpr (FAST) {
            const float4 t = *reinterpret_cast<const float4*>(x);
            t2 += s0 * (t.x * v[0] + t.y * v[1] + t.z * v[2] + t.w * v[3]);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (ok[e]) t2 += s0 * x[e] * v[e];
          }
        } else if constexpr (EPI == EPI_RQ) {  // X1: R in bf16, read at (col, row..row+3)
          const bf16_t* x = reinterpret_cast<const bf16_t*>(X1) + (long long)col * p.ldx + row;
          if constexpr (FAST) {
            const uint2 t = *reinterpret_cast<const uint2*>(x);
            t2 += s0 * (bf16_to_f32((bf16_t)(t.x & 0xffff)) * v[0] + bf16_to_f32((bf16_t)(t.x >> 16)) * v[1] +
                        bf16_to_f32((bf16_t)(t.y & 0xffff)) * v[2] + bf16_to_f32((bf16_t)(t.y >> 16)) * v[3]);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (ok[e]) t2 += s0 * bf16_to_f32(x[e]) * v[e];
          }
        }
        if constexpr (EPI == EPI_STRACE) {  // the mirrored elements (col, row + e), strictly below the diagonal
          const float* x = X1 + (long long)col * p.ldx + row;
          if constexpr (FAST) {
            const float4 t = *reinterpret_cast<const float4*>(x);
            t2 += v[0] * t.x + v[1] * t.y + v[2] * t.z + v[3] * t.w;
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (ok[e] && row + e < col) t2 += v[e] * x[e];
          }
        }
        if (CTf) {
          float* dst = CTf + (long long)col * p.ldct + row;
          if (FAST || (all && (p.ldct & 3) == 0)) *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
          else
#pragma unroll
            for (int e = 0; e < 4; ++e) if (ok[e]) dst[e] = v[e];
        }
        if (CTb) {
          bf16_t* dst = CTb + (long long)col * p.ldct + row;
          if (FAST || (all && (p.ldct & 3) == 0))
            *reinterpret_cast<uint2*>(dst) = make_uint2(pack2(f32_to_bf16(v[0]), f32_to_bf16(v[1])),
                                                         pack2(f32_to_bf16(v[2]), f32_to_bf16(v[3])));
          else
#pragma unroll
            for (int e = 0; e < 4; ++e) if (ok[e]) dst[e] = f32_to_bf16(v[e]);
        }
        if (mirror) {  // element (row, col) with row < col also at (col, row): rows row..row+3 are contiguous there
          if (FAST || (all && row + 3 < col)) {
            if (C) {
              float* dst = C + (long long)col * p.ldc + row;
              if (FAST || (p.ldc & 3) == 0) *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
              else
#pragma unroll
                for (int e = 0; e < 4; ++e) dst[e] = v[e];
            }
            if (Cb) {
              bf16_t* dst = Cb + (long long)col * p.ldcb + row;
              if (FAST || (p.ldcb & 3) == 0)
                *reinterpret_cast<uint2*>(dst) = make_uint2(pack2(f32_to_bf16(v[0]), f32_to_bf16(v[1])),
                                                             pack2(f32_to_bf16(v[2]), f32_to_bf16(v[3])));
              else
#pragma unroll
                for (int e = 0; e < 4; ++e) dst[e] = f32_to_bf16(v[e]);
            }
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              if (!ok[e] || row + e == col) continue;
              if (C) C[(long long)col * p.ldc + row + e] = v[e];
              if (Cb) Cb[(long long)col * p.ldcb + row + e] = f32_to_bf16(v[e]);
            }
          }
        }
      }
    };
    if constexpr (EPI == EPI_PROCB) {
      if (fast) tcol_pass(std::true_type{});
      else tcol_pass(std::false_type{});
      __syncthreads();
    }
    if (fast) {
      using I1 = std::integral_constant<int, 1>;
      using I0 = std::integral_constant<int, 0>;
      if constexpr (EPI == EPI_FACTOR || EPI == EPI_PROC || EPI == EPI_PROCB || EPI == EPI_STRACE) {
        if (C && Cb) row_pass_fast(I1{}, I1{});
        else if (C) row_pass_fast(I1{}, I0{});
        else if (Cb) row_pass_fast(I0{}, I1{});
        else row_pass_fast(I0{}, I0{});
      } else {
        row_pass_fast(std::integral_constant<int, -1>{}, std::integral_constant<int, -1>{});
      }
    } else {
      row_pass();
    }
    __syncthreads();
    if (colpass) {
      if (fast) col_pass(std::true_type{});
      else col_pass(std::false_type{});
      __syncthreads();
    }
  };
  if (!producer) {
    half(std::integral_constant<int, 0>{});
    half(std::integral_constant<int, 1>{});
  } else {  // producer waves (WS): the epilogue's barriers, nothing else (each half: parking, row pass, and the
            // transposed and column passes where the epilogue has them)
    const int nbar = 2 * (2 + (EPI == EPI_PROCB ? 1 : 0) + (colpass ? 1 : 0));
    for (int i = 0; i < nbar; ++i) __syncthreads();
  }
  if constexpr (EPI == EPI_RQ || EPI == EPI_SUMSQ || EPI == EPI_STRACE) {
    __shared__ float red[16];
    t1 = block_sum(t1, red);
    if constexpr (EPI == EPI_RQ || EPI == EPI_STRACE) t2 = block_sum(t2, red);
    if (tid == 0) {
      p.part[b][2 * tile] = t1;
      p.part[b][2 * tile + 1] = t2;
    }
  }
}

template <int BM, int BN, int WGM, int WGN, int EPI, int PW = 0>
__global__ void __launch_bounds__(64 * (WGM * WGN + PW)) gemm_bf16_kernel(const GB16Args p) {
  gemm_kc_body<bf16_t, BM, BN, WGM, WGN, EPI, 0, PW>(p);
}

// two workgroups per CU (two waves per SIMD): the register budget of every layout
template <int BM, int BN, int WGM, int WGN, int EPI, int LAY>
__global__ void __launch_bounds__(64 * WGM * WGN, 2) gemm_f32kc_kernel(const GB16Args p) {
  gemm_kc_body<float, BM, BN, WGM, WGN, EPI, LAY>(p);
}

int gemm_bf16_tiles(long long M, long long N, int tri, int cfg) {
  const int T = cfg == 1 || cfg == 4 ? 128 : 256;
  const long long tm = (M + T - 1) / T, tn = (N + T - 1) / T;
  return (int)(tri ? tm * (tm + 1) / 2 : tm * tn);
}

template <typename T, int BM, int BN, int WGM, int WGN, int EPI, int LAY = 0, int PW = 0>
static hipError_t launch_b16(GB16Args& a, hipStream_t st) {
  constexpr int NW = WGM * WGN;
  constexpr int smem_main = 2 * (BM + BN) * 128,
                smem_epi = NW * (BM / WGM / 2) * epi_pitch(BM / WGM / 2, BN / WGN) * 4;
  constexpr int smem = smem_main > smem_epi ? smem_main : smem_epi;
  void (*fn)(GB16Args) = nullptr;
  if constexpr (std::is_same_v<T, bf16_t>) fn = gemm_bf16_kernel<BM, BN, WGM, WGN, EPI, PW>;
  else fn = gemm_f32kc_kernel<BM, BN, WGM, WGN, EPI, LAY>;
  // once per instantiation (a function-local static is initialised once, also under concurrent first calls)
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize, smem);
  if (attr != hipSuccess) return attr;
  a.tiles_m = (a.M + BM - 1) / BM;
  a.tiles_n = (a.N + BN - 1) / BN;
  a.ntiles = a.tri ? a.tiles_m * (a.tiles_m + 1) / 2 : a.tiles_m * a.tiles_n;
  hipLaunchKernelGGL(fn, dim3(a.ntiles * a.nb), dim3(64 * (NW + PW)), smem, st, a);
  const hipError_t e = hipGetLastError();
  note_launch(reinterpret_cast<const void*>(fn), (long long)a.ntiles * a.nb, 64 * (NW + PW), smem);
  return e;
}

template <typename T, int BM, int BN, int WGM, int WGN, int LAY = 0, int PW = 0>
static hipError_t launch_epi(GB16Args& a, hipStream_t st) {
  constexpr bool B16 = std::is_same_v<T, bf16_t>;
  switch (a.epi) {
    case EPI_FACTOR: return launch_b16<T, BM, BN, WGM, WGN, EPI_FACTOR, LAY, PW>(a, st);
    case EPI_PROC: return launch_b16<T, BM, BN, WGM, WGN, EPI_PROC, LAY, PW>(a, st);
    case EPI_SCALE: return launch_b16<T, BM, BN, WGM, WGN, EPI_SCALE, LAY, PW>(a, st);
    case EPI_SUMSQ: return launch_b16<T, BM, BN, WGM, WGN, EPI_SUMSQ, LAY, PW>(a, st);
    case EPI_STRACE: return launch_b16<T, BM, BN, WGM, WGN, EPI_STRACE, LAY, PW>(a, st);
    case EPI_STORE: return launch_b16<T, BM, BN, WGM, WGN, EPI_STORE, LAY, PW>(a, st);
    case EPI_RQ: return launch_b16<T, BM, BN, WGM, WGN, EPI_RQ, LAY, PW>(a, st);  // R read as T
    default: break;
  }
  if constexpr (B16) {  // reads a bf16 X operand
    if (a.epi == EPI_PROCB) return launch_b16<T, BM, BN, WGM, WGN, EPI_PROCB, LAY, PW>(a, st);
  }
  return hipErrorInvalidValue;
}

// cfg 0: 256 x 256 tiles, 8 waves (2 per SIMD) of 128 x 64; cfg 1: 128 x 128 tiles, 4 waves of 64 x 64;
// cfg 2: 256 x 256 tiles, 4 waves of 128 x 128 (one wave per SIMD); cfg 3: 256 x 256 tiles, 8 MFMA waves of
// 128 x 64 on 32 x 32 x 16 MFMAs plus 4 producer waves (warp-specialized main loop); cfg 4: the same on 128 x 128
// tiles, 4 MFMA waves of 64 x 64
hipError_t gemm_bf16_launch(GB16Args& a, int cfg, hipStream_t st) {
  if (cfg == 1) return launch_epi<bf16_t, 128, 128, 2, 2>(a, st);
  if (cfg == 4) return launch_epi<bf16_t, 128, 128, 2, 2, 0, 4>(a, st);
  if (cfg == 2) return launch_epi<bf16_t, 256, 256, 2, 2>(a, st);
  if (cfg == 3) return launch_epi<bf16_t, 256, 256, 2, 4, 0, 4>(a, st);
  return launch_epi<bf16_t, 256, 256, 2, 4>(a, st);
}

// fp32: the 128-tile configuration only (its waves hold the blocked-summation accumulators)
hipError_t gemm_f32kc_launch(GB16Args& a, int cfg, hipStream_t st) {
  (void)cfg;
  if (a.tri && a.amc != a.bmc) return hipErrorInvalidValue;  // a SYRK reads one operand
  switch ((a.amc ? 1 : 0) | (a.bmc ? 2 : 0)) {
    case 1: return launch_epi<float, 128, 128, 2, 2, 1>(a, st);
    case 2: return launch_epi<float, 128, 128, 2, 2, 2>(a, st);
    case 3: return launch_epi<float, 128, 128, 2, 2, 3>(a, st);
    default: return launch_epi<float, 128, 128, 2, 2, 0>(a, st);
  }
}

}  // namespace psgdk

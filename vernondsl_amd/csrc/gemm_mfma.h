// Shared main loop of the MFMA GEMMs (bf16 and int8) for gfx950: C[m][n] = sum_k A[m][k] B[n][k]
// with both operands K-contiguous ("NT").
//
// Both instruction shapes used here consume a 16-byte fragment per lane and 32 bytes of K per row
// per instruction:
//   v_mfma_f32_32x32x16_bf16: lane l holds A[row = l%32][k = 8*(l/32) .. +7]   (8 bf16)
//   v_mfma_i32_32x32x32_i8:   lane l holds A[row = l%32][k = 16*(l/32) .. +15] (16 int8)
// (B likewise with row -> column), and accumulator element r of lane l is
// C[8*(r/4) + 4*(l/32) + r%4][l%32].  So one byte-level tile machinery serves both.
//
// Block tile BM x BN, K advancing BKB bytes per stage.  WGM x WGN waves each own a
// (BM/WGM) x (BN/WGN) wave tile = FM x FN accumulators.  LDS holds two stages of A [BM][BKB+16]
// and B [BN][BKB+16] bytes (the 16-byte row pad staggers fragment rows across banks), so one
// barrier per K stage suffices: stage s+1 is written while other waves may still read stage s.
// The next stage's global loads are issued into registers before the current stage's MFMAs.
// Blocks are re-numbered so that the ids the hardware dispatches to one XCD (congruent mod 8)
// walk neighbouring tiles, and tiles are visited in groups of 8 tile-rows so consecutive blocks
// share B columns in that XCD's L2.
#pragma once

#include <type_traits>

#include "common.h"

namespace vdsl {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

struct MfmaBf16 {
  using Frag = bf16x8;
  using Acc = f32x16;
  static constexpr int kElemBytes = 2;
  __device__ static __forceinline__ Acc mma(const Frag& a, const Frag& b, const Acc& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  __device__ static __forceinline__ Acc zero() {
    Acc z;
#pragma unroll
    for (int r = 0; r < 16; ++r) z[r] = 0.0f;
    return z;
  }
};

struct MfmaI8 {
  using Frag = i32x4;
  using Acc = i32x16;
  static constexpr int kElemBytes = 1;
  __device__ static __forceinline__ Acc mma(const Frag& a, const Frag& b, const Acc& c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  }
  __device__ static __forceinline__ Acc zero() {
    Acc z;
#pragma unroll
    for (int r = 0; r < 16; ++r) z[r] = 0;
    return z;
  }
};

__device__ __forceinline__ int xcd_remap(int b, int nb) {
  if (nb % 8) return b;
  return (b % 8) * (nb / 8) + (b / 8);
}

// Tile coordinates of linear tile id t: groups of G tile-rows, walked column-major inside a group.
__device__ __forceinline__ void tile_coords(int t, int tiles_m, int tiles_n, int& tm, int& tn) {
  constexpr int G = 8;
  const int group = t / (G * tiles_n);
  const int first_m = group * G;
  const int gsize = min(G, tiles_m - first_m);
  const int in_group = t - group * G * tiles_n;
  tm = first_m + in_group % gsize;
  tn = in_group / gsize;
}

template <class T, int BM_, int BN_, int BKB_, int WGM_, int WGN_>
struct GemmConfig {
  static constexpr int BM = BM_, BN = BN_, BKB = BKB_, WGM = WGM_, WGN = WGN_;
  static constexpr int NT = WGM * WGN * 64;
  static constexpr int WTM = BM / WGM, WTN = BN / WGN;
  static constexpr int FM = WTM / 32, FN = WTN / 32;
  static constexpr int ROW = BKB + 16;  // padded LDS row, bytes
  static constexpr int CPR = BKB / 16;  // 16-byte chunks per row
  static constexpr int A_PER_T = BM * CPR / NT, B_PER_T = BN * CPR / NT;
  static constexpr int STAGE = (BM + BN) * ROW;
  static constexpr int LDS_BYTES = 2 * STAGE;
  // blocks per CU the kernel is built for (__launch_bounds__): two when their LDS fits the CU's
  // 160 KiB, else one (asking for two then only caps the registers for nothing)
  static constexpr int MIN_BLOCKS = 2 * LDS_BYTES <= 160 * 1024 ? 2 : 1;
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be whole 32x32 MFMA tiles");
  static_assert(BKB % 32 == 0, "a stage must hold whole MFMA K steps");
  static_assert((BM * CPR) % NT == 0 && (BN * CPR) % NT == 0, "loads must split evenly over lanes");
  static_assert(LDS_BYTES <= 160 * 1024, "gfx950 workgroup LDS limit");
};

// Per-lane view of the global->LDS copy of one operand tile: lane t moves chunks c = t + NT*i,
// row c / CPR = t / CPR + i * (NT / CPR), K byte (t % CPR) * 16.  One base pointer per operand;
// the per-chunk offsets i * (NT / CPR) * Kb are uniform.
// (Prefetch registers are clang vectors, not HIP's uint4 class: a class copy can become a memcpy
// through a stack slot, which the compiler then fails to promote to registers.)
template <class Cfg, int ROWS, bool EDGE>
__device__ __forceinline__ void gemm_load_tile(u32x4 (&r)[ROWS * Cfg::CPR / Cfg::NT], const char* base, int Kb, int kb,
                                               bool kin, int row0, int rows_valid) {
  constexpr int RPP = Cfg::NT / Cfg::CPR;
#pragma unroll
  for (int i = 0; i < ROWS * Cfg::CPR / Cfg::NT; ++i) {
    const char* p = base + static_cast<size_t>(i * RPP) * Kb + kb;
    if (EDGE) {
      const u32x4 z = {0u, 0u, 0u, 0u};
      r[i] = (kin && row0 + i * RPP < rows_valid) ? *reinterpret_cast<const u32x4*>(p) : z;
    } else {
      r[i] = *reinterpret_cast<const u32x4*>(p);
    }
  }
}

template <class Cfg, int ROWS>
__device__ __forceinline__ void gemm_store_tile(const u32x4 (&r)[ROWS * Cfg::CPR / Cfg::NT], char* s, int tid) {
#pragma unroll
  for (int i = 0; i < ROWS * Cfg::CPR / Cfg::NT; ++i) {
    const int c = tid + Cfg::NT * i;
    *reinterpret_cast<u32x4*>(s + (c / Cfg::CPR) * Cfg::ROW + (c % Cfg::CPR) * 16) = r[i];
  }
}

// MFMAs of one LDS stage for this wave.  The fragments of k-step kk+1 are read before the MFMAs
// of k-step kk (two fragment sets in turn), so LDS latency hides behind FM*FN MFMAs; scheduling
// barriers keep that order (left alone, the compiler moves each read next to its first use).
// sched_group_barrier masks: 0x008 MFMA, 0x100 DS read.
template <class T, class Cfg>
__device__ __forceinline__ void gemm_compute_stage(const char* sa, const char* sb, typename T::Acc (&acc)[Cfg::FM][Cfg::FN]) {
  using Frag = typename T::Frag;
  constexpr int FM = Cfg::FM, FN = Cfg::FN, KS = Cfg::BKB / 32;
  Frag a0[FM], b0[FN], a1[FM], b1[FN];
#define VDSL_GEMM_READ(A_, B_, KK)                                                              \
  do {                                                                                          \
    _Pragma("unroll") for (int i = 0; i < FM; ++i)                                              \
      A_[i] = *reinterpret_cast<const Frag*>(sa + i * 32 * Cfg::ROW + (KK) * 32);               \
    _Pragma("unroll") for (int j = 0; j < FN; ++j)                                              \
      B_[j] = *reinterpret_cast<const Frag*>(sb + j * 32 * Cfg::ROW + (KK) * 32);               \
  } while (0)
#define VDSL_GEMM_MMA(A_, B_)                                                                   \
  do {                                                                                          \
    _Pragma("unroll") for (int i = 0; i < FM; ++i)                                              \
      _Pragma("unroll") for (int j = 0; j < FN; ++j) acc[i][j] = T::mma(A_[i], B_[j], acc[i][j]); \
  } while (0)
#define VDSL_GEMM_ORDER()                                                                       \
  do {                                                                                          \
    __builtin_amdgcn_sched_group_barrier(0x100, FM + FN, 0);                                    \
    __builtin_amdgcn_sched_group_barrier(0x008, FM * FN, 0);                                    \
    __builtin_amdgcn_sched_barrier(0);                                                          \
  } while (0)
  VDSL_GEMM_READ(a0, b0, 0);
#pragma unroll
  for (int kk = 0; kk < KS; kk += 2) {
    if (kk + 1 < KS) VDSL_GEMM_READ(a1, b1, kk + 1);
    VDSL_GEMM_MMA(a0, b0);
    VDSL_GEMM_ORDER();
    if (kk + 1 < KS) {
      if (kk + 2 < KS) VDSL_GEMM_READ(a0, b0, kk + 2);
      VDSL_GEMM_MMA(a1, b1);
      VDSL_GEMM_ORDER();
    }
  }
#undef VDSL_GEMM_ORDER
#undef VDSL_GEMM_MMA
#undef VDSL_GEMM_READ
}

// Runs the K loop over bytes [kb_begin, kb_end) of rows m0.. and n0.. and leaves the wave's
// accumulators in acc.  Kb = row stride of A and B in bytes (K * element size); kb_end <= Kb.
// Requires Kb % 16 == 0.  EDGE = false is the fast path for launches whose every block tile and K
// stage are in range (no load predicates); with EDGE = true out-of-range rows and K bytes read
// as 0.  The host picks one per launch (gemm_needs_edge).
//
// Pipeline: two register sets (0 and 1) of prefetched global data.  At the start of stage kt
// (S = kt & 1), LDS stage S holds tile kt, register set S^1 holds (or is still receiving) tile
// kt+1 and set S is free; the stage issues the loads of tile kt+2 into set S, runs its MFMAs,
// stores set S^1 into LDS stage S^1 and meets the barrier.  So two stages of HBM latency hide
// behind MFMAs.  The loop is unrolled by two so every register index is a compile-time constant.
template <class T, class Cfg, bool EDGE>
__device__ __forceinline__ void gemm_mainloop(const char* __restrict__ A, const char* __restrict__ B, int M, int N,
                                              int Kb, int kb_begin, int kb_end, int m0, int n0, char* smem,
                                              typename T::Acc (&acc)[Cfg::FM][Cfg::FN]) {
  static_assert(Cfg::NT % Cfg::CPR == 0, "a pass of all lanes must cover whole rows");
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / Cfg::WGN, wn = wave % Cfg::WGN;
#pragma unroll
  for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
    for (int j = 0; j < Cfg::FN; ++j) acc[i][j] = T::zero();

  const int trow = tid / Cfg::CPR;
  const int tk = (tid % Cfg::CPR) * 16;
  const char* pa = A + static_cast<size_t>(m0 + trow) * Kb + tk;
  const char* pb = B + static_cast<size_t>(n0 + trow) * Kb + tk;
  u32x4 ra0[Cfg::A_PER_T], rb0[Cfg::B_PER_T], ra1[Cfg::A_PER_T], rb1[Cfg::B_PER_T];
  const int frow = lane & 31;
  const int fk = (lane >> 5) * 16;
  const char* fa = smem + (wm * Cfg::WTM + frow) * Cfg::ROW + fk;
  const char* fb = smem + Cfg::BM * Cfg::ROW + (wn * Cfg::WTN + frow) * Cfg::ROW + fk;

#define VDSL_GEMM_LOAD(RA, RB, KB)                                                              \
  do {                                                                                          \
    const bool kin_ = !EDGE || (KB) + tk < kb_end;                                              \
    gemm_load_tile<Cfg, Cfg::BM, EDGE>(RA, pa, Kb, (KB), kin_, m0 + trow, M);                   \
    gemm_load_tile<Cfg, Cfg::BN, EDGE>(RB, pb, Kb, (KB), kin_, n0 + trow, N);                   \
  } while (0)
#define VDSL_GEMM_STORE(RA, RB, ST)                                                             \
  do {                                                                                          \
    gemm_store_tile<Cfg, Cfg::BM>(RA, smem + (ST) * Cfg::STAGE, tid);                           \
    gemm_store_tile<Cfg, Cfg::BN>(RB, smem + (ST) * Cfg::STAGE + Cfg::BM * Cfg::ROW, tid);      \
  } while (0)
// Stage kt computed from LDS stage CUR; RA/RB_L receive tile kt+2; RA/RB_S (tile kt+1) go to
// LDS stage CUR ^ 1.  The loads and the store are unconditional: past the last tile they repeat
// it (kb clamped to kb_last) and that copy is never read.  A branch around them would make the
// compiler's wait counts conservative at the join: it then waits for every outstanding load at
// the top of each stage, which leaves one stage of prefetch instead of two.
// The scheduling barrier after the loads keeps the compiler from sinking them below the store
// of the previous tile (it does so otherwise, and the store then waits for every load).
#define VDSL_GEMM_STEP(KT, CUR, RA_L, RB_L, RA_S, RB_S)                                         \
  do {                                                                                          \
    VDSL_GEMM_LOAD(RA_L, RB_L, min(kb_begin + ((KT) + 2) * Cfg::BKB, kb_last));                \
    __builtin_amdgcn_sched_barrier(0);                                                          \
    gemm_compute_stage<T, Cfg>(fa + (CUR) * Cfg::STAGE, fb + (CUR) * Cfg::STAGE, acc);          \
    VDSL_GEMM_STORE(RA_S, RB_S, (CUR) ^ 1);                                                     \
    __syncthreads();                                                                            \
    __builtin_amdgcn_sched_barrier(0);                                                          \
  } while (0)

  const int nk = (kb_end - kb_begin + Cfg::BKB - 1) / Cfg::BKB;
  if (nk <= 0) return;
  const int kb_last = kb_begin + (nk - 1) * Cfg::BKB;
  VDSL_GEMM_LOAD(ra0, rb0, kb_begin);
  VDSL_GEMM_LOAD(ra1, rb1, min(kb_begin + Cfg::BKB, kb_last));
  VDSL_GEMM_STORE(ra0, rb0, 0);
  __syncthreads();
  // Unrolled by two so every register set index is a constant; no early exit inside the loop
  // (the accumulators then stay in one register class across the back edge).
  int kt = 0;
  for (; kt + 2 <= nk; kt += 2) {
    VDSL_GEMM_STEP(kt, 0, ra0, rb0, ra1, rb1);
    VDSL_GEMM_STEP(kt + 1, 1, ra1, rb1, ra0, rb0);
  }
  if (kt < nk) VDSL_GEMM_STEP(kt, 0, ra0, rb0, ra1, rb1);
#undef VDSL_GEMM_STEP
#undef VDSL_GEMM_STORE
#undef VDSL_GEMM_LOAD
}

// True when some block tile or K stage of the launch would reach past the operands.
template <class Cfg>
inline bool gemm_needs_edge(int64_t M, int64_t N, int64_t kbytes_per_block) {
  return (M % Cfg::BM) != 0 || (N % Cfg::BN) != 0 || (kbytes_per_block % Cfg::BKB) != 0;
}

// Row / column of accumulator element r of fragment (i, j) for this lane.
template <class Cfg>
__device__ __forceinline__ int acc_row(int m0, int i, int r) {
  const int lane = threadIdx.x & 63;
  const int wm = (threadIdx.x >> 6) / Cfg::WGN;
  return m0 + wm * Cfg::WTM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
}
template <class Cfg>
__device__ __forceinline__ int acc_col(int n0, int j) {
  const int lane = threadIdx.x & 63;
  const int wn = (threadIdx.x >> 6) % Cfg::WGN;
  return n0 + wn * Cfg::WTN + j * 32 + (lane & 31);
}

// Host side: GEMM tile configuration chosen for a shape.  VDSL_GEMM_CONFIG=<index> forces one
// (used for tuning sweeps); an out-of-range index falls back to the heuristic.
int gemm_config_override();

}  // namespace vdsl

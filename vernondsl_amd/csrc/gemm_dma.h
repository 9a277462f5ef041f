// Direct-to-LDS MFMA main loop for gfx950: C[m][n] = sum_k A[m][k] B[n][k], both operands
// K-contiguous, for launches whose K range is a whole number of 64-byte stages.
//
// Global -> LDS copies use global_load_lds_dwordx4: each lane's 16 bytes go straight into LDS at
// (wave-uniform base + 16 * lane), with no VGPR round trip and no ds_write.  Freed of prefetch
// registers, the loop keeps NS stages of LDS in flight (NS-1 stages of global latency hidden).
//
// LDS layout, per operand and stage: 64 K bytes (4 chunks of 16 B) of each row, in 1 KiB blocks
// of 16 rows.  Within a block row r occupies 64 bytes at 64 * (r % 16) and its chunk c sits in
// slot c ^ ((r >> 2) & 3).  Both sides of that choice are measured constraints of the hardware:
//   - the address unit coalesces 4 consecutive lanes; the copy gives lanes 4q..4q+3 one row's 4
//     chunks (a whole 64-byte sector, in swizzled order), so a copy instruction touches 16 sectors;
//   - an MFMA fragment read has lane l take row l % 32, chunk 2 * kk + l / 32; the 16 lanes read
//     together land in 16 distinct 16-byte bank groups (rows 4 apart share a 64-byte bank window
//     and the XOR gives them distinct slots), so fragment reads are free of bank conflicts.
//
// A stage is BKB = 64 or 128 K bytes: one or two 64-byte sub-stages, each laid out as above.
// Pipeline per stage t (ring of NS LDS stages): issue the copy of stage t+NS-1 (into the slot
// stage t-1 used), read fragments k-step by k-step one step ahead of the MFMAs, then before the
// MFMAs of the last k-step wait for this wave's copy of stage t+1 (vmcnt = copies issued after
// it) and meet the block barrier, so stage t+1's first fragment reads overlap those MFMAs.  A
// 128-byte stage halves the barriers per MFMA.  The
// barrier also orders every wave's reads of stage t before the copy that overwrites it (issued
// at stage t+1).  Rows past M or N are clamped to the last row (their products only reach
// outputs that are not stored).
//
// K-major B (BKN, bf16 only): B stored [K][N] (N contiguous), the layout of an activation that a
// weight-gradient GEMM takes as is (dW = g^T x with x [batch][in]), so no transpose kernel runs
// first.  A sub-stage's B area then holds the 32 K rows of the tile, each 2 BN bytes, with chunk
// c of row k in slot c ^ kn_swz(k); the copies move whole 64-byte runs of a row, and a B fragment
// is assembled by two transposing LDS reads (ds_read_b64_tr_b16): within each group of 16 lanes,
// result lane i, element e is element i % 4 of the 8 bytes addressed by lane 4 e + i / 4, so
// pointing lane j at row k0 + j / 4, columns 4 (j % 4) .. + 3 hands lane i the 4 K values of
// column i (measured on gfx950 with an in-bounds lane-layout probe).  Same products in the same
// order as the NT form of the transposed B, so the same results bit for bit.
#pragma once

#include "gemm_mfma.h"

namespace vdsl {

template <class T, int BM_, int BN_, int WGM_, int WGN_, int NS_, int BKB_ = 64>
struct DmaConfig {
  static constexpr int BM = BM_, BN = BN_, WGM = WGM_, WGN = WGN_, NS = NS_;
  static constexpr int BKB = BKB_;                   // K bytes per stage (one barrier per stage)
  static constexpr int KSUB = BKB / 64;              // 64-byte sub-stages per stage
  static constexpr int KS = BKB / 32;                // MFMA k-steps per stage
  static constexpr int RPB = 16;                     // rows per 1 KiB LDS block
  static constexpr int NT = WGM * WGN * 64, NW = WGM * WGN;
  static constexpr int WTM = BM / WGM, WTN = BN / WGN;
  static constexpr int FM = WTM / 32, FN = WTN / 32;
  static constexpr int SUB = (BM + BN) * 64;         // bytes of one sub-stage
  static constexpr int STAGE = KSUB * SUB;
  static constexpr int LDS_BYTES = NS * STAGE;
  // blocks per CU the kernel is built for (__launch_bounds__): two 4-wave blocks when their LDS
  // fits the CU's 160 KiB, else one
  static constexpr int MIN_BLOCKS = (NT < 512 && 2 * LDS_BYTES <= 160 * 1024) ? 2 : 1;
  static constexpr int NBLK = (BM + BN) / RPB;       // 1 KiB copy blocks per sub-stage
  static constexpr int BPW = NBLK / NW;              // copy instructions per wave per sub-stage
  static constexpr int CPW = KSUB * BPW;             // copy instructions per wave per stage
  static_assert(BKB % 64 == 0 && BKB > 0, "a stage is a whole number of 64-byte sub-stages");
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be whole 32x32 MFMA tiles");
  static_assert(BM % RPB == 0 && BN % RPB == 0 && NBLK % NW == 0, "copy blocks must split evenly over waves");
  static_assert(NS >= 3, "the loop keeps two stages in flight beyond the one being read");
  static_assert(LDS_BYTES <= 160 * 1024, "gfx950 workgroup LDS limit");
};

typedef __attribute__((address_space(3))) void lds_void_t;

// LDS offset (within a stage's operand area) of chunk c of row r.
__device__ __forceinline__ int dma_slot(int r, int c) {
  return (r >> 4) * 1024 + (r & 15) * 64 + ((c ^ ((r >> 2) & 3)) << 4);
}

// The gfx950-only builtins sit in plain (non-template) device functions: inside a function
// template, clang's host pass marks the specialization invalid on first instantiation and then
// rejects every later call to it.
__device__ __forceinline__ void lds_copy16(const char* g, char* l) {
  __builtin_amdgcn_global_load_lds(g, (lds_void_t*)l, 16, 0, 0);
}

typedef short i16x4_t __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16 at an 8-byte aligned LDS address (see the K-major B note above).
__device__ __forceinline__ i16x4_t lds_read_tr16(const char* l) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4_t*)(l));
}

// K-major B: the 16-byte slot XOR of K row k (0..31 within a sub-stage), in chunk units.  It flips
// bits 2-4 of the chunk index, so a row's 64-byte runs stay whole; the 8 rows one transposing read
// touches (k0 + 0..3 and k0 + 8..11, k0 % 4 == 0) get 8 distinct 64-byte windows of a 512-byte row.
__device__ __forceinline__ int kn_swz(int k) { return ((k & 7) ^ ((k >> 1) & 4)) << 2; }

// s_waitcnt vmcnt(n) lgkmcnt(0) (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt 6:4 left at
// its no-wait value 7, lgkmcnt 11:8 = 0).  The count must be a constant.
#define VDSL_WAIT_VM_LGKM0(n) dma_wait<(n)>()
template <int N>
__device__ __forceinline__ void dma_wait();
#define VDSL_DMA_WAIT_CASE(n) \
  template <> __device__ __forceinline__ void dma_wait<n>() { __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (((n) >> 4) << 14) | (0x7 << 4)); }
VDSL_DMA_WAIT_CASE(0)
VDSL_DMA_WAIT_CASE(3)
VDSL_DMA_WAIT_CASE(4)
VDSL_DMA_WAIT_CASE(6)
VDSL_DMA_WAIT_CASE(8)
VDSL_DMA_WAIT_CASE(9)
VDSL_DMA_WAIT_CASE(12)
VDSL_DMA_WAIT_CASE(16)
VDSL_DMA_WAIT_CASE(18)
VDSL_DMA_WAIT_CASE(24)
#undef VDSL_DMA_WAIT_CASE

// Block barrier without the full memory fence of __syncthreads (which would also wait for the
// copies still meant to be in flight); the empty asm statements stop the compiler from moving
// memory accesses across it.
__device__ __forceinline__ void dma_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// K loop over bytes [kb_begin, kb_end) for the tile at (m0, n0).  Requires kb_begin % 16 == 0 and
// (kb_end - kb_begin) % BKB == 0; Kb = row stride of A and B in bytes.
// BKN: B is stored [K][N] with row stride Nb bytes (needs BN == 256, bf16, and the tile's N range
// inside N: the caller launches it only for N % 256 == 0).  AKM: likewise A stored [K][M] with row
// stride Mb bytes (BM == 256, M % 256 == 0): the same copies and transposing reads as K-major B,
// since an MFMA A fragment has B's lane layout (lane l: row l % 32, K values 8 (l / 32) .. + 7).
template <class T, class Cfg, class AccT, int FM_, int FN_, bool BKN = false, bool AKM = false>
__device__ __forceinline__ void dma_mainloop(const char* __restrict__ A, const char* __restrict__ B, int M, int N, int Kb,
                                             int kb_begin, int kb_end, int m0, int n0, char* smem, AccT (&acc)[FM_][FN_],
                                             int Nb = 0, int Mb = 0) {
  static_assert(FM_ == Cfg::FM && FN_ == Cfg::FN, "accumulator array must match the configuration");
  static_assert(!BKN || (Cfg::BN == 256 && std::is_same<T, MfmaBf16>::value), "K-major B: bf16, 256-wide tiles");
  static_assert(!AKM || (Cfg::BM == 256 && std::is_same<T, MfmaBf16>::value), "K-major A: bf16, 256-tall tiles");
  using Frag = typename T::Frag;
  constexpr int FM = Cfg::FM, FN = Cfg::FN, NS = Cfg::NS, BPW = Cfg::BPW, STAGE = Cfg::STAGE, SUB = Cfg::SUB;
  constexpr int KS = Cfg::KS, KSUB = Cfg::KSUB, CPW = Cfg::CPW;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / Cfg::WGN, wn = wave % Cfg::WGN;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = T::zero();

  // Copy block b = wave * BPW + u of a sub-stage: blocks [0, BM/16) are A rows 16b.., the rest B.
  // Lane l copies row 16 * (b') + l / 4, LDS slot l % 4, i.e. global chunk (l % 4) ^ swizzle.
  const char* src[BPW];
  size_t kmul[BPW];  // K-major B: bytes of source per K byte of the stage offset (1 for row-major rows)
#pragma unroll
  for (int u = 0; u < BPW; ++u) {
    const int b = wave * BPW + u;
    const bool is_a = b < Cfg::BM / Cfg::RPB;
    if (AKM && is_a) {  // as K-major B below, over the A area's 16 blocks
      const int k = 2 * b + (lane >> 5);
      const int c = (lane & 31) ^ kn_swz(k);
      src[u] = A + static_cast<size_t>(kb_begin / 2 + k) * Mb + static_cast<size_t>(m0) * 2 + c * 16;
      kmul[u] = static_cast<size_t>(Mb) / 2;
      continue;
    }
    if (BKN && !is_a) {
      // 1 KiB block j holds K rows 2j, 2j+1 of the sub-stage; lane l fills slot l % 32 of row
      // 2j + l / 32 with global chunk (l % 32) ^ kn_swz(row) of that row's 512-byte run.
      const int k = 2 * (b - Cfg::BM / Cfg::RPB) + (lane >> 5);
      const int c = (lane & 31) ^ kn_swz(k);
      src[u] = B + static_cast<size_t>(kb_begin / 2 + k) * Nb + static_cast<size_t>(n0) * 2 + c * 16;
      kmul[u] = static_cast<size_t>(Nb) / 2;
      continue;
    }
    const int r = Cfg::RPB * (is_a ? b : b - Cfg::BM / Cfg::RPB) + (lane >> 2);
    const int c = (lane & 3) ^ ((r >> 2) & 3);
    const size_t row = is_a ? static_cast<size_t>(min(m0 + r, M - 1)) : static_cast<size_t>(min(n0 + r, N - 1));
    src[u] = (is_a ? A : B) + row * Kb + kb_begin + c * 16;
    kmul[u] = 1;
  }
  (void)kmul;
  char* const dst = smem + wave * BPW * 1024;
  // This lane's fragment rows (within a sub-stage's A and B areas).
  const int ra = wm * Cfg::WTM + (lane & 31);
  const int rb = wn * Cfg::WTN + (lane & 31);
  const int hk = lane >> 5;
  const char* const fa = smem;
  const char* const fb = smem + Cfg::BM * 64;
  // K-major B: offsets of this lane's two transposing reads (r = K values 0-3 / 4-7 of its half)
  // of fragment j in the first k-step of a sub-stage; the second k-step is 16 rows further.
  int tro[2][FN];
  if constexpr (BKN) {
    const int g = lane >> 4, i = lane & 15;
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int k = 8 * (g >> 1) + 4 * r + (i >> 2);
        const int n = wn * Cfg::WTN + 32 * j + 16 * (g & 1) + 4 * (i & 3);
        tro[r][j] = k * (2 * Cfg::BN) + (((n >> 3) ^ kn_swz(k)) << 4) + ((n >> 2) & 1) * 8;
      }
  }
  int tra[2][FM];  // K-major A: the same offsets over the A area (row stride 2 BM)
  if constexpr (AKM) {
    const int g = lane >> 4, i = lane & 15;
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int f = 0; f < FM; ++f) {
        const int k = 8 * (g >> 1) + 4 * r + (i >> 2);
        const int m = wm * Cfg::WTM + 32 * f + 16 * (g & 1) + 4 * (i & 3);
        tra[r][f] = k * (2 * Cfg::BM) + (((m >> 3) ^ kn_swz(k)) << 4) + ((m >> 2) & 1) * 8;
      }
  }
  constexpr int NRD = (AKM ? 2 : 1) * FM + (BKN ? 2 : 1) * FN;  // LDS read instructions per k-step

#define VDSL_DMA_SRC(U, KOFF) ((BKN || AKM) ? src[U] + static_cast<size_t>(KOFF) * kmul[U] : src[U] + (KOFF))
#define VDSL_DMA_COPY(ST, KB)                                                                     \
  do {                                                                                            \
    _Pragma("unroll") for (int sb = 0; sb < KSUB; ++sb)                                           \
      _Pragma("unroll") for (int u = 0; u < BPW; ++u)                                             \
        lds_copy16(VDSL_DMA_SRC(u, (KB) + 64 * sb), dst + (ST) * STAGE + sb * SUB + u * 1024);    \
  } while (0)
// Copies [I0, I1) of a stage's CPW copies (copy i = sub-stage i / BPW, block i % BPW).
#define VDSL_DMA_COPY_PART(ST, KB, I0, I1)                                                        \
  do {                                                                                            \
    _Pragma("unroll") for (int i = (I0); i < (I1); ++i)                                           \
      lds_copy16(VDSL_DMA_SRC(i % BPW, (KB) + 64 * (i / BPW)), dst + (ST) * STAGE + (i / BPW) * SUB + \
                 (i % BPW) * 1024);                                                               \
  } while (0)
// Fragments of k-step KK (32 K bytes) of stage ST: sub-stage KK / 2, chunks 2 (KK % 2) + hk.
#define VDSL_DMA_READ(A_, B_, ST, KK)                                                             \
  do {                                                                                            \
    if constexpr (AKM) {                                                                          \
      _Pragma("unroll") for (int i = 0; i < FM; ++i) {                                            \
        const char* const ka_ = fa + (ST) * STAGE + ((KK) >> 1) * SUB + ((KK) & 1) * 32 * Cfg::BM; \
        const i16x4_t lo_ = lds_read_tr16(ka_ + tra[0][i]), hi_ = lds_read_tr16(ka_ + tra[1][i]); \
        A_[i] = __builtin_bit_cast(Frag, __builtin_shufflevector(lo_, hi_, 0, 1, 2, 3, 4, 5, 6, 7)); \
      }                                                                                           \
    } else {                                                                                      \
      _Pragma("unroll") for (int i = 0; i < FM; ++i)                                              \
        A_[i] = *reinterpret_cast<const Frag*>(fa + (ST) * STAGE + ((KK) >> 1) * SUB +            \
                                               dma_slot(ra + 32 * i, 2 * ((KK) & 1) + hk));        \
    }                                                                                             \
    if constexpr (BKN) {                                                                          \
      _Pragma("unroll") for (int j = 0; j < FN; ++j) {                                            \
        const char* const kb_ = fb + (ST) * STAGE + ((KK) >> 1) * SUB + ((KK) & 1) * 32 * Cfg::BN; \
        const i16x4_t lo_ = lds_read_tr16(kb_ + tro[0][j]), hi_ = lds_read_tr16(kb_ + tro[1][j]); \
        B_[j] = __builtin_bit_cast(Frag, __builtin_shufflevector(lo_, hi_, 0, 1, 2, 3, 4, 5, 6, 7)); \
      }                                                                                           \
    } else {                                                                                      \
      _Pragma("unroll") for (int j = 0; j < FN; ++j)                                              \
        B_[j] = *reinterpret_cast<const Frag*>(fb + (ST) * STAGE + ((KK) >> 1) * SUB +            \
                                               dma_slot(rb + 32 * j, 2 * ((KK) & 1) + hk));        \
    }                                                                                             \
  } while (0)
#define VDSL_DMA_MMA(A_, B_)                                                                      \
  do {                                                                                            \
    _Pragma("unroll") for (int i = 0; i < FM; ++i)                                                \
      _Pragma("unroll") for (int j = 0; j < FN; ++j) acc[i][j] = T::mma(A_[i], B_[j], acc[i][j]); \
  } while (0)
// Reads of the next k-step first, then the MFMAs (sched_group_barrier masks: 0x100 DS read,
// 0x008 MFMA); the scheduling barrier keeps each k-step's instructions together.
#define VDSL_DMA_ORDER()                                                                          \
  do {                                                                                            \
    __builtin_amdgcn_sched_group_barrier(0x100, NRD, 0);                                      \
    __builtin_amdgcn_sched_group_barrier(0x008, FM * FN, 0);                                      \
    __builtin_amdgcn_sched_barrier(0);                                                            \
  } while (0)
// First k-step of a stage: one MFMA ahead of the reads.  At the loop top the compiler waits for
// every outstanding LDS read before the first MFMA (lgkmcnt(0)); issuing the next k-step's reads
// after that MFMA keeps them out of that wait.
#define VDSL_DMA_ORDER_LATE()                                                                     \
  do {                                                                                            \
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                            \
    __builtin_amdgcn_sched_group_barrier(0x100, NRD, 0);                                      \
    __builtin_amdgcn_sched_group_barrier(0x008, FM * FN - 1, 0);                                  \
    __builtin_amdgcn_sched_barrier(0);                                                            \
  } while (0)
// A k-step that also issues NC copies (VMEM, mask 0x020): reads first (after one MFMA when
// LATE), then each copy between MFMAs, so the copies of all waves do not reach the address unit
// in one burst while no MFMA issues.
#define VDSL_DMA_ORDER_COPIES(LATE, NC)                                                           \
  do {                                                                                            \
    if (LATE) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                  \
    __builtin_amdgcn_sched_group_barrier(0x100, NRD, 0);                                      \
    _Pragma("unroll") for (int c = 0; c < (NC); ++c) {                                            \
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                                          \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                          \
    }                                                                                             \
    __builtin_amdgcn_sched_group_barrier(0x008, FM * FN, 0);                                      \
    __builtin_amdgcn_sched_barrier(0);                                                            \
  } while (0)

// Wave priority (s_setprio, the issue arbiter's per-wave priority) is raised while a wave issues
// its fragment reads and MFMAs and dropped for its copies, waits and barrier, so of the two waves
// sharing a SIMD the one with MFMAs ready issues first (int8 512x8192x8192: 1123 -> 1231 TOP/s;
// bf16 unchanged within noise).
#define VDSL_DMA_PRIO(P)                                                                          \
  do {                                                                                            \
    __builtin_amdgcn_s_setprio(P);                                                                \
    __builtin_amdgcn_sched_barrier(0);                                                            \
  } while (0)

  const int nk = (kb_end - kb_begin) / Cfg::BKB;
  if (nk <= 0) return;
#pragma unroll
  for (int s = 0; s < NS - 1; ++s) VDSL_DMA_COPY(s, min(s, nk - 1) * Cfg::BKB);
  VDSL_WAIT_VM_LGKM0((NS - 2) * CPW);
  dma_barrier();
  if constexpr (KS == 4) {
    // 128-byte stages: fragments are read two k-steps ahead (four register sets, k-step kk in set
    // kk), so an LDS read has two k-steps of MFMAs to land.  The barrier moves one k-step earlier:
    // it precedes the first read of stage kt+1 (k-step 2's group).
    Frag af[4][FM], bf[4][FN];
    VDSL_DMA_READ(af[0], bf[0], 0, 0);
    VDSL_DMA_READ(af[1], bf[1], 0, 1);
    int st = 0;
    for (int kt = 0; kt < nk; ++kt) {
      const int nst = st + 1 == NS ? 0 : st + 1;
      const int cst = st == 0 ? NS - 1 : st - 1;
      const int kb_copy = min(kt + NS - 1, nk - 1) * Cfg::BKB;
      __builtin_amdgcn_sched_barrier(0);
      VDSL_DMA_PRIO(1);
      VDSL_DMA_READ(af[2], bf[2], st, 2);
      VDSL_DMA_MMA(af[0], bf[0]);
      VDSL_DMA_COPY_PART(cst, kb_copy, 0, CPW / 2);
      VDSL_DMA_ORDER_COPIES(true, CPW / 2);
      VDSL_DMA_READ(af[3], bf[3], st, 3);
      VDSL_DMA_MMA(af[1], bf[1]);
      VDSL_DMA_COPY_PART(cst, kb_copy, CPW / 2, CPW);
      VDSL_DMA_ORDER_COPIES(true, CPW - CPW / 2);
      VDSL_DMA_PRIO(0);
      VDSL_WAIT_VM_LGKM0((NS - 2) * CPW);
      dma_barrier();
      __builtin_amdgcn_sched_barrier(0);
      VDSL_DMA_PRIO(1);
      VDSL_DMA_READ(af[0], bf[0], nst, 0);
      VDSL_DMA_MMA(af[2], bf[2]);
      VDSL_DMA_ORDER_LATE();
      VDSL_DMA_READ(af[1], bf[1], nst, 1);
      VDSL_DMA_MMA(af[3], bf[3]);
      VDSL_DMA_ORDER_LATE();
      VDSL_DMA_PRIO(0);
      st = nst;
    }
    VDSL_WAIT_VM_LGKM0(0);
    return;
  }
  // Fragment double buffer: k-step kk of a stage computes from set kk % 2 while set (kk + 1) % 2
  // is read (KS is even, so every stage starts on set 0).
  Frag af[2][FM], bf[2][FN];
  VDSL_DMA_READ(af[0], bf[0], 0, 0);
  int st = 0;
  for (int kt = 0; kt < nk; ++kt) {
    const int nst = st + 1 == NS ? 0 : st + 1;
    const int cst = st == 0 ? NS - 1 : st - 1;  // = (kt + NS - 1) % NS
    // The copy of stage kt+NS-1 (into the slot stage kt-1 used, whose reads all ended before the
    // last barrier) is spread over the k-steps before the last, between MFMAs.  Past the last
    // stage it repeats that stage (never read): the copy count per stage stays fixed, which is
    // what the vmcnt in the wait below counts on.
    const int kb_copy = min(kt + NS - 1, nk - 1) * Cfg::BKB;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kk = 0; kk < KS - 1; ++kk) {
      constexpr int kParts = KS - 1;
      const int c0 = kk * CPW / kParts, c1 = (kk + 1) * CPW / kParts;
      VDSL_DMA_PRIO(1);
      VDSL_DMA_READ(af[(kk + 1) & 1], bf[(kk + 1) & 1], st, kk + 1);
      VDSL_DMA_MMA(af[kk & 1], bf[kk & 1]);
      VDSL_DMA_COPY_PART(cst, kb_copy, c0, c1);
      VDSL_DMA_ORDER_COPIES(kk == 0, c1 - c0);
      VDSL_DMA_PRIO(0);
    }
    // Before the last k-step: this wave's copy of stage kt+1 has landed, and every wave's has
    // once all meet the barrier (which also ends all reads of the slot the next copy overwrites).
    VDSL_WAIT_VM_LGKM0((NS - 2) * CPW);
    dma_barrier();
    __builtin_amdgcn_sched_barrier(0);
    VDSL_DMA_PRIO(1);
    VDSL_DMA_READ(af[0], bf[0], nst, 0);
    VDSL_DMA_MMA(af[1], bf[1]);
    VDSL_DMA_ORDER();
    VDSL_DMA_PRIO(0);
    st = nst;
  }
  // Drain the copies of the stages past the end before the block's LDS can be reused or freed.
  VDSL_WAIT_VM_LGKM0(0);
#undef VDSL_DMA_PRIO
#undef VDSL_DMA_ORDER_COPIES
#undef VDSL_DMA_ORDER_LATE
#undef VDSL_DMA_ORDER
#undef VDSL_DMA_MMA
#undef VDSL_DMA_READ
#undef VDSL_DMA_COPY_PART
#undef VDSL_DMA_COPY
#undef VDSL_DMA_SRC
}

// True when the direct-to-LDS loop with `bkb` K bytes per stage can run this K range.
inline bool dma_k_ok(int64_t kb_begin, int64_t kbytes, int64_t bkb = 64) {
  return kb_begin % 16 == 0 && kbytes % bkb == 0 && kbytes > 0;
}

}  // namespace vdsl

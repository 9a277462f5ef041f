// MFMA main loop for gfx950 with the B operand read from a packed fragment layout straight into
// registers, and only A staged through LDS: C[m][n] = sum_k A[m][k] B[n][k].
//
// Packed B ("fragment order"): unit (nb, kb) is the 32 x 32-byte block B[32 nb .. +31][32 kb ..
// +31] stored as the register image of one MFMA B fragment: 1 KiB, lane l's 16 bytes at 16 l hold
// B[32 nb + l % 32][32 kb + 16 (l / 32) .. +15].  Units are ordered nb-major: unit (nb, kb) starts
// at byte (nb * Kb / 32 + kb) * 1024.  A wave's fragment load is then one fully coalesced 1 KiB
// global_load_dwordx4 (a row-major B read in fragment layout touches 64 sectors per instruction
// instead of 16, which measured address-unit bound).
//
// Why B skips LDS: a block's W waves split N only (wave w owns columns 64 w .. of the block, all
// BM rows), so no two waves use the same B fragment and there is nothing to share; every wave
// reads every A fragment, which LDS shares.  LDS traffic per k-step is then BM*32 bytes written
// plus W*BM*32 read for W*FM*FN MFMAs (1/FN KiB per MFMA), against (FM+FN)/(FM*FN) KiB read plus
// the copies of both operands when both go through LDS.
//
// Pipeline, per 128-byte K stage t (ring of NS = PD+1 LDS slots for A and PD+1 register sets for
// B): the wave reads A fragments two k-steps ahead of the MFMAs, issues its B loads for stage t+PD
// during k-steps 0-1 and its A copies for stage t+PD during k-steps 2-3, each spread evenly between
// MFMAs, and before the MFMAs of k-step 2 waits (vmcnt) for its own loads of stage t+1 and meets
// the block barrier.  Spreading matters: with the stage's 12 loads and copies issued back to back
// the address unit backs up and stalls the wave's MFMA issue (2048x4096x4096 bf16: 60-62 us
// against 56-57 spread over the four k-steps).  The loop body is unrolled over the PD+1 stages of
// the ring so every register-set index is a constant; the stage count of a launch must be a
// multiple of PD+1.
// Rows of A past M are clamped to the last row and fragments of B past N to the last unit (their
// products only reach outputs that are not stored).
//
// A kernel using this loop must declare no __shared__ variable besides `smem`: with a second one
// the compiler tags LDS accesses with alias scopes, cannot tell a copy's destination slot from the
// slot being read, and waits for every copy in flight (vmcnt(0)) before each fragment read.
#pragma once

#include "gemm_dma.h"

namespace vdsl {

template <class T, int FM_, int FN_, int W_, int PD_>
struct BpkConfig {
  static constexpr int FM = FM_, FN = FN_, W = W_, PD = PD_;
  static constexpr int BM = 32 * FM, BN = 32 * FN * W, NT = 64 * W;
  // The wave grid in the terms the shared epilogues use (1 x W waves, each BM x 32 FN).
  static constexpr int WGM = 1, WGN = W, NW = W, WTM = BM, WTN = 32 * FN;
  static constexpr int BKB = 128, KS = 4;   // K bytes and MFMA k-steps per stage
  static constexpr int NR = PD + 1;         // LDS slots = B register sets = stages per loop trip
  static constexpr int SUB = BM * 64;       // one 64-byte sub-stage of A
  static constexpr int STAGE = 2 * SUB;
  static constexpr int LDS_BYTES = NR * STAGE;
  static constexpr int CPS = BM / 16;       // 1 KiB copy blocks per sub-stage
  static constexpr int CPW = 2 * CPS / W;   // copies per wave per stage
  static constexpr int BPW = KS * FN;       // B fragment loads per wave per stage
  static constexpr int VPS = CPW + BPW;     // vector-memory instructions per wave per stage
  static_assert((2 * CPS) % W == 0 && CPW >= 1, "A copy blocks must split evenly over the waves");
  static_assert(PD >= 2, "the loop keeps loads of at least two stages in flight");
  static_assert((PD - 1) * VPS <= 63, "s_waitcnt vmcnt holds at most 63");
  static_assert(LDS_BYTES <= 160 * 1024, "gfx950 workgroup LDS limit");
};

// s_waitcnt vmcnt(N) lgkmcnt(0): this wave's LDS reads have ended too, so no read of a slot can
// still be pending when another wave's copy into that slot is issued after the next barrier.
template <int N>
__device__ __forceinline__ void bpk_wait_vm() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4));
}

// Orders one k-step's instructions: one MFMA, the D fragment reads (LDS), then the other NM - 1
// MFMAs with V vector-memory instructions spread evenly between them (sched_group_barrier masks:
// 0x008 MFMA, 0x100 DS read, 0x020 VMEM read).  The MFMA ahead of the reads works on fragments
// read earlier, so the wait the compiler puts before it covers only those older reads.
template <int NM, int D, int V>
__device__ __forceinline__ void bpk_sched_kstep() {
  __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
  if constexpr (D > 0) __builtin_amdgcn_sched_group_barrier(0x100, D, 0);
  if constexpr (NM > 1) {
#pragma unroll
    for (int i = 0; i < NM - 1; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
#pragma unroll
      for (int v = i * V / (NM - 1); v < (i + 1) * V / (NM - 1); ++v) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
  }
  if constexpr (NM == 1 && V > 0) __builtin_amdgcn_sched_group_barrier(0x020, V, 0);
  __builtin_amdgcn_sched_barrier(0);
}

// K loop over bytes [kb_begin, kb_end) of the tile at (m0, n0): ((kb_end - kb_begin) / 128) must
// be a positive multiple of Cfg::NR.  A: row-major, Kb bytes per row.  Bp: packed (see above),
// Kb / 32 units per 32-row group.  nblk = N / 32 (B units per K column).
template <class T, class Cfg>
__device__ __forceinline__ void bpk_mainloop(const char* __restrict__ A, const char* __restrict__ Bp, int M, int nblk, int Kb,
                                             int kb_begin, int kb_end, int m0, int n0, char* smem,
                                             typename T::Acc (&acc)[Cfg::FM][Cfg::FN]) {
  using Frag = typename T::Frag;
  constexpr int FM = Cfg::FM, FN = Cfg::FN, NR = Cfg::NR, PD = Cfg::PD, KS = Cfg::KS;
  constexpr int SUB = Cfg::SUB, STAGE = Cfg::STAGE, CPS = Cfg::CPS, CPW = Cfg::CPW;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = T::zero();

  // A copies: stage copy c = wave * CPW + u covers sub-stage c / CPS, 16-row block c % CPS; lane l
  // moves row 16 (c % CPS) + l / 4, global chunk (l % 4) ^ ((l >> 4) & 3) into LDS slot l % 4
  // (gemm_dma.h's swizzle: chunk c of row r sits in slot c ^ ((r >> 2) & 3)).
  const char* asrc[CPW];
  int adst[CPW];
#pragma unroll
  for (int u = 0; u < CPW; ++u) {
    const int c = wave * CPW + u;
    const int r = 16 * (c % CPS) + (lane >> 2);
    const int ch = (lane & 3) ^ ((lane >> 4) & 3);
    asrc[u] = A + static_cast<size_t>(min(m0 + r, M - 1)) * Kb + kb_begin + (c / CPS) * 64 + ch * 16;
    adst[u] = (c / CPS) * SUB + (c % CPS) * 1024;
  }
  // B fragments: this wave's FN units of each k-step.
  const int kblk = Kb / 32;
  const char* bsrc[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int nb = min(n0 / 32 + FN * wave + j, nblk - 1);
    bsrc[j] = Bp + (static_cast<size_t>(nb) * kblk + kb_begin / 32) * 1024 + lane * 16;
  }
  const int ra = lane & 31, hk = lane >> 5;

  Frag bq[NR][KS][FN];
  Frag af[4][FM];
  const int nk = (kb_end - kb_begin) / Cfg::BKB;

  // B fragment loads of k-steps [K0, K1) and A copies [U0, U1) of stage ST.
#define VDSL_BPK_LOAD_B(SET, ST, K0, K1)                                                         \
  do {                                                                                           \
    _Pragma("unroll") for (int kk = (K0); kk < (K1); ++kk)                                       \
      _Pragma("unroll") for (int j = 0; j < FN; ++j)                                             \
        bq[SET][kk][j] = *reinterpret_cast<const Frag*>(bsrc[j] + static_cast<size_t>((ST) * KS + kk) * 1024); \
  } while (0)
#define VDSL_BPK_COPY_A(SLOT, ST, U0, U1)                                                        \
  do {                                                                                           \
    _Pragma("unroll") for (int u = (U0); u < (U1); ++u)                                          \
      lds_copy16(asrc[u] + (ST) * Cfg::BKB, smem + (SLOT) * STAGE + adst[u]);                    \
  } while (0)
#define VDSL_BPK_READ_A(DST, SLOT, KK)                                                           \
  do {                                                                                           \
    _Pragma("unroll") for (int i = 0; i < FM; ++i)                                               \
      DST[i] = *reinterpret_cast<const Frag*>(smem + (SLOT) * STAGE + ((KK) >> 1) * SUB +        \
                                             dma_slot(ra + 32 * i, 2 * ((KK) & 1) + hk));          \
  } while (0)
#define VDSL_BPK_MMA(AF, SET, KK)                                                                \
  do {                                                                                           \
    _Pragma("unroll") for (int i = 0; i < FM; ++i)                                               \
      _Pragma("unroll") for (int j = 0; j < FN; ++j) acc[i][j] = T::mma(AF[i], bq[SET][KK][j], acc[i][j]); \
  } while (0)

  // Prologue: stages 0 .. PD-1 (B loads, then A copies, per stage, as in the loop).  Loads from
  // a read-only __restrict__ kernel argument may otherwise be moved past the wait and barrier
  // below, which would make the vmcnt of the wait count the wrong instructions: the scheduling
  // barriers pin them (as do the ones around every group in the loop).
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int s = 0; s < PD; ++s) {
    const int st = min(s, nk - 1);
    VDSL_BPK_LOAD_B(s, st, 0, KS);
    VDSL_BPK_COPY_A(s, st, 0, CPW);
  }
  __builtin_amdgcn_sched_barrier(0);
  bpk_wait_vm<(PD - 1) * Cfg::VPS>();
  dma_barrier();
  VDSL_BPK_READ_A(af[0], 0, 0);
  VDSL_BPK_READ_A(af[1], 0, 1);

  // do-while: the launch guarantees nk >= NR, and a loop guard here would let the compiler sink
  // the prologue's B loads below the barrier into the guarded block.
  constexpr int NM = FM * FN, HB = KS / 2, HC = CPW / 2;
  int kt = 0;
  do {
#pragma unroll
    for (int s = 0; s < NR; ++s) {
      const int nslot = (s + 1) % NR;
      const int pslot = (s + PD) % NR;  // the slot and register set stage kt+s-1 used
      const int pst = min(kt + s + PD, nk - 1);
      __builtin_amdgcn_sched_barrier(0);
      VDSL_BPK_READ_A(af[2], s, 2);
      VDSL_BPK_MMA(af[0], s, 0);
      VDSL_BPK_LOAD_B(pslot, pst, 0, HB);
      bpk_sched_kstep<NM, FM, HB * FN>();
      VDSL_BPK_READ_A(af[3], s, 3);
      VDSL_BPK_MMA(af[1], s, 1);
      VDSL_BPK_LOAD_B(pslot, pst, HB, KS);
      bpk_sched_kstep<NM, FM, (KS - HB) * FN>();
      // This wave's loads of stage kt+s+1 have landed once only later ones are outstanding: the
      // B loads and A copies of stages kt+s+2 .. kt+s+PD-1 and the B loads of stage kt+s+PD (its
      // A copies follow below).  After the barrier every wave's A copies of that stage have too.
      bpk_wait_vm<(PD - 2) * Cfg::VPS + Cfg::BPW>();
      dma_barrier();
      __builtin_amdgcn_sched_barrier(0);
      VDSL_BPK_READ_A(af[0], nslot, 0);
      VDSL_BPK_MMA(af[2], s, 2);
      VDSL_BPK_COPY_A(pslot, pst, 0, HC);
      bpk_sched_kstep<NM, FM, HC>();
      VDSL_BPK_READ_A(af[1], nslot, 1);
      VDSL_BPK_MMA(af[3], s, 3);
      VDSL_BPK_COPY_A(pslot, pst, HC, CPW);
      bpk_sched_kstep<NM, FM, CPW - HC>();
    }
    kt += NR;
  } while (kt < nk);
  // Drain the loads and copies issued past the last stage before the LDS is reused or freed.
  bpk_wait_vm<0>();
#undef VDSL_BPK_MMA
#undef VDSL_BPK_READ_A
#undef VDSL_BPK_COPY_A
#undef VDSL_BPK_LOAD_B
}

// Packs B [N][K] (row-major, Kb bytes per row; N % 32 == 0, Kb % 32 == 0) into fragment order:
// thread u writes 16-byte chunk u of the packed array.  Internal linkage: each source file that
// includes this header launches its own copy.
static __global__ __launch_bounds__(256) void bpk_pack_kernel(const char* __restrict__ B, char* __restrict__ Bp, int64_t nblk,
                                                       int64_t kblk, int64_t Kb) {
  const int64_t chunks = nblk * kblk * 64;
  for (int64_t u = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; u < chunks;
       u += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t unit = u >> 6;
    const int l = static_cast<int>(u & 63);
    const int64_t nb = unit / kblk, kb = unit % kblk;
    const int64_t row = nb * 32 + (l & 31);
    const int64_t col = kb * 32 + 16 * (l >> 5);
    *reinterpret_cast<u32x4*>(Bp + u * 16) = *reinterpret_cast<const u32x4*>(B + row * Kb + col);
  }
}

}  // namespace vdsl

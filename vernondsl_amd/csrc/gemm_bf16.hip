// Op class 4: dense bf16 x bf16 -> f32-accumulate GEMM on gfx950 MFMA, with fused epilogues.
//
// No reference code (the north-star op class: the dense matmuls of the MLP graph, forward and
// autodiff-generated backward).
//
// Native layout "NT": C[m][n] = sum_k A[m][k] * B[n][k], both operands K-contiguous (B is a
// weight in [out][in] form).  The other layouts are reduced to it by transposing the strided
// operand into caller-provided workspace first (vdsl_gemm_bf16_workspace_bytes).  The main loop
// (tiling, LDS double buffering, MFMA fragment layout, XCD-aware order) is gemm_mfma.h; this file
// adds the epilogue (GELU / ReLU, optional f32 pre-activation, f32 or bf16 C) and the choice of
// tile configuration per shape.

#include <atomic>
#include <cstdlib>

#include "gemm_mfma.h"
#include "gemm_bpk.h"
#include "gemm_dma.h"

namespace vdsl {

// Defined in layout.hip.
int launch_transpose(const void* src, void* dst, int64_t rows, int64_t cols, int dtype, hipStream_t s);
// Defined in autodiff.hip: the one-block, fixed-order sum of MSE partials into the loss.
int launch_mse_finish(const double* partials, int64_t n_partials, float* loss, double inv_n, hipStream_t s);

namespace {
std::atomic<int> g_gemm_config{-2};  // -2: not yet read from the environment
}  // namespace

int gemm_config_override() {
  int v = g_gemm_config.load(std::memory_order_relaxed);
  if (v == -2) {
    const char* e = std::getenv("VDSL_GEMM_CONFIG");
    g_gemm_config.compare_exchange_strong(v, e ? std::atoi(e) : -1);
    v = g_gemm_config.load(std::memory_order_relaxed);
  }
  return v;
}

namespace {


// Tile configurations (block M x N, K bytes per stage, wave grid).
using Bf0 = GemmConfig<MfmaBf16, 128, 128, 128, 2, 2>;  // wave tile 64x64
using Bf1 = GemmConfig<MfmaBf16, 256, 128, 128, 2, 2>;  // wave tile 128x64
using Bf2 = GemmConfig<MfmaBf16, 128, 256, 128, 2, 2>;  // wave tile 64x128
using Bf3 = GemmConfig<MfmaBf16, 64, 64, 128, 2, 2>;    // wave tile 32x32: small outputs
using Bf4 = GemmConfig<MfmaBf16, 256, 256, 64, 4, 2>;   // 8 waves, wave tile 64x128
using Bf5 = GemmConfig<MfmaBf16, 256, 128, 128, 4, 2>;  // 8 waves, wave tile 64x64
using Bf6 = GemmConfig<MfmaBf16, 128, 128, 256, 2, 2>;  // 128 bf16 of K per stage
using Bf7 = GemmConfig<MfmaBf16, 128, 64, 128, 2, 2>;   // wave tile 64x32: twice the blocks of 128x128
using Bf8 = GemmConfig<MfmaBf16, 64, 128, 128, 2, 2>;   // wave tile 32x64
using Bf9 = GemmConfig<MfmaBf16, 128, 128, 64, 2, 2>;   // 64 K bytes per stage: 3 blocks per CU fit in LDS
using Bf10 = GemmConfig<MfmaBf16, 256, 128, 64, 2, 2>;  // wave tile 128x64, 2 blocks per CU
using Bf11 = GemmConfig<MfmaBf16, 128, 256, 64, 2, 2>;  // wave tile 64x128, 2 blocks per CU
using Bf12 = GemmConfig<MfmaBf16, 256, 256, 64, 2, 4>;  // 8 waves, wave tile 128x64
using Bf13 = GemmConfig<MfmaBf16, 256, 128, 64, 4, 2>;  // 8 waves, wave tile 64x64, 2 blocks per CU
// Direct-to-LDS loop (gemm_dma.h), configurations 14..: <BM, BN, WGM, WGN, LDS stages>
using Dm14 = DmaConfig<MfmaBf16, 128, 256, 2, 4, 4>;  // 8 waves of 64x64
using Dm15 = DmaConfig<MfmaBf16, 256, 256, 2, 4, 3>;  // 8 waves of 128x64
using Dm16 = DmaConfig<MfmaBf16, 128, 256, 2, 4, 3>;  // 8 waves of 64x64, 3 LDS stages
using Dm17 = DmaConfig<MfmaBf16, 128, 128, 2, 2, 4>;  // 4 waves of 64x64, 2 blocks per CU
using Dm18 = DmaConfig<MfmaBf16, 128, 256, 2, 4, 5>;  // 8 waves of 64x64, 5 LDS stages
using Dm19 = DmaConfig<MfmaBf16, 256, 128, 2, 2, 4>;  // 4 waves of 128x64
using Dm20 = DmaConfig<MfmaBf16, 128, 256, 2, 2, 4>;  // 4 waves of 64x128
using Dm21 = DmaConfig<MfmaBf16, 128, 256, 2, 2, 3>;  // 4 waves of 64x128, 3 LDS stages
using Dm22 = DmaConfig<MfmaBf16, 128, 256, 2, 2, 5>;  // 4 waves of 64x128, 5 LDS stages
// 128-byte stages (one barrier per 64 bf16 of K); need K % 64 == 0
using Dm23 = DmaConfig<MfmaBf16, 128, 256, 2, 4, 3, 128>;  // 8 waves of 64x64
using Dm24 = DmaConfig<MfmaBf16, 128, 256, 2, 2, 3, 128>;  // 4 waves of 64x128
using Dm25 = DmaConfig<MfmaBf16, 128, 128, 2, 2, 4, 128>;  // 4 waves of 64x64
using Dm26 = DmaConfig<MfmaBf16, 256, 128, 2, 2, 3, 128>;  // 4 waves of 128x64
constexpr int kNumConfigs = 27;
constexpr int kFirstDma = 14, kFirstDma128 = 23;

// Internal epilogue code of vdsl_op_gemm_bf16_gelu_bwd: C (bf16) = v * GELU'(pre) with `pre` an
// input, and the same values transposed into `ctr` ([N][M], optional).
constexpr int kEpiGeluBwd = 100;
// OR-ed into a kernel's `epi` argument when its f32 output is bound as VDSL_BIND_OUTPUT (a result
// for the host that no later device work reads soon): the LDS-staged epilogue then stores it with
// non-temporal hints.  In the config-4 step the weight gradients (2 x 64 MB of f32) stored that way
// no longer leave dirty lines for the next GEMMs to write back: step 372-376 -> 355-358 us.
constexpr int kEpiStreamOut = 0x1000;

// Backward epilogue modes (template argument BWD): 0 = forward (epi selects it), 1 = C = v *
// GELU'(pre) (vdsl_op_gemm_bf16_gelu_bwd), 2 = C = v * g with the factor g given in `pre`
// (vdsl_op_gemm_bf16_mul_packed).  With g = GELU'(pre) from the forward epilogue
// VDSL_EPI_GELU_DERIV, modes 1 and 2 compute the same product and round it the same way.
template <int BWD>
__device__ __forceinline__ float bwd_factor(float p) {
  if constexpr (BWD == 2) return p;
  else return gelu_grad_f(p);
}

// Epilogue of one accumulator element at (row, col), shared by both main loops.  DERIV: the
// kernel runs VDSL_EPI_GELU_DERIV only (a separate instantiation: in the shared forward kernels
// its code made the register allocator spill).
template <int BWD, bool DERIV = false>
__device__ __forceinline__ void bf16_epilogue(float v, int row, int col, int M, int N, void* __restrict__ C,
                                              float* __restrict__ pre, int epi, int c_dtype, uint16_t* __restrict__ ctr) {
  if (row < M && col < N) {
    const size_t o = static_cast<size_t>(row) * N + col;
    if constexpr (BWD != 0) {
      const uint16_t h = f32_to_bf16(v * bwd_factor<BWD>(pre[o]));
      static_cast<uint16_t*>(C)[o] = h;
      if (ctr) ctr[static_cast<size_t>(col) * M + row] = h;
      return;
    }
    if constexpr (DERIV) {
      pre[o] = gelu_grad_f(v);
      static_cast<uint16_t*>(C)[o] = f32_to_bf16(gelu_f(v));
      return;
    }
    if (pre) pre[o] = v;
    float y = v;
    if (epi == VDSL_EPI_GELU) y = gelu_f(v);
    else if (epi == VDSL_EPI_RELU) y = v > 0.0f ? v : 0.0f;
    if (c_dtype == VDSL_F32) static_cast<float*>(C)[o] = y;
    else static_cast<uint16_t*>(C)[o] = f32_to_bf16(y);
  }
}

// Whole-tile epilogue with the variant fixed at compile time: no bounds checks and no per-element
// branches (the generic per-element form costs ~6000 instructions of branchy code per tile).
// Variants: 0 = f32 C, no activation, no pre-activation; 1 = bf16 C = GELU(v) with f32 pre-activation.
template <class Cfg, int VARIANT>
__device__ __forceinline__ void bf16_epilogue_tile(const f32x16 (&acc)[Cfg::FM][Cfg::FN], int m0, int n0, int N,
                                                   void* __restrict__ C, float* __restrict__ pre) {
#pragma unroll
  for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
    for (int j = 0; j < Cfg::FN; ++j) {
      const int col = acc_col<Cfg>(n0, j);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const size_t o = static_cast<size_t>(acc_row<Cfg>(m0, i, r)) * N + col;
        const float v = acc[i][j][r];
        if (VARIANT == 0) {
          static_cast<float*>(C)[o] = v;
        } else {
          pre[o] = v;
          static_cast<uint16_t*>(C)[o] = f32_to_bf16(gelu_f(v));
        }
      }
    }
}

// Picks the whole-tile variant when one applies, else the generic per-element epilogue.
template <class Cfg, int BWD, bool DERIV = false>
__device__ __forceinline__ void bf16_store_tile(const f32x16 (&acc)[Cfg::FM][Cfg::FN], int m0, int n0, int M, int N,
                                                void* __restrict__ C, float* __restrict__ pre, int epi, int c_dtype,
                                                uint16_t* __restrict__ ctr) {
  const bool whole = m0 + Cfg::BM <= M && n0 + Cfg::BN <= N;
  if (DERIV) {
#pragma unroll
    for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
      for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          bf16_epilogue<0, true>(acc[i][j][r], acc_row<Cfg>(m0, i, r), acc_col<Cfg>(n0, j), M, N, C, pre, epi, c_dtype, ctr);
  } else if (BWD != 0) {
#pragma unroll
    for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
      for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          bf16_epilogue<BWD>(acc[i][j][r], acc_row<Cfg>(m0, i, r), acc_col<Cfg>(n0, j), M, N, C, pre, epi, c_dtype, ctr);
  } else if (whole && epi == VDSL_EPI_NONE && c_dtype == VDSL_F32 && !pre) {
    bf16_epilogue_tile<Cfg, 0>(acc, m0, n0, N, C, pre);
  } else if (whole && epi == VDSL_EPI_GELU && c_dtype == VDSL_BF16 && pre) {
    bf16_epilogue_tile<Cfg, 1>(acc, m0, n0, N, C, pre);
  } else {
#pragma unroll
    for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
      for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          bf16_epilogue<0>(acc[i][j][r], acc_row<Cfg>(m0, i, r), acc_col<Cfg>(n0, j), M, N, C, pre, epi, c_dtype, ctr);
  }
}

// Whole-tile epilogue staged through LDS (after the main loop, when the block's LDS is free):
// each wave writes one 32-row block of its accumulators to a private LDS area (row stride WTN + 8
// floats: the lanes of one accumulator store, 32 columns x rows 4 apart, hit 64 distinct banks),
// reads it back as 4 consecutive columns per lane and stores 16-byte runs of the f32 output (or
// of the pre-activation) and 8-byte runs of the bf16 output, instead of one 4- or 2-byte store
// per accumulator element.  Needs N % 4 == 0 (aligned runs) and NW * 32 * (WTN + 8) floats of
// LDS; the caller has synchronised the block after the main loop.
template <class Cfg>
constexpr bool kLdsEpilogue = Cfg::NW * 32 * (Cfg::WTN + 8) * 4 <= Cfg::LDS_BYTES;


template <class Cfg, int VARIANT>
__device__ __forceinline__ void bf16_epilogue_tile_lds(const f32x16 (&acc)[Cfg::FM][Cfg::FN], int m0, int n0, int N,
                                                       void* __restrict__ C, float* __restrict__ pre, char* smem) {
  constexpr int WTN = Cfg::WTN, LD = WTN + 8;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / Cfg::WGN, wn = wave % Cfg::WGN;
  float* const area = reinterpret_cast<float*>(smem) + wave * 32 * LD;
  const int row0 = m0 + wm * Cfg::WTM, col0 = n0 + wn * WTN;
#pragma unroll
  for (int i = 0; i < Cfg::FM; ++i) {
#pragma unroll
    for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) area[(8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * LD + 32 * j + (lane & 31)] = acc[i][j][r];
    constexpr int Q = WTN / 4;  // 16-byte units per row
#pragma unroll
    for (int k = 0; k < 32 * Q / 64; ++k) {
      const int u = lane + 64 * k, row = u / Q, c4 = u % Q;
      const f32x4 v = *reinterpret_cast<const f32x4*>(area + row * LD + 4 * c4);
      const size_t o = static_cast<size_t>(row0 + 32 * i + row) * N + col0 + 4 * c4;
      if (VARIANT == 0) {
        *reinterpret_cast<f32x4*>(static_cast<float*>(C) + o) = v;
      } else if (VARIANT == 3) {  // VARIANT 0 with streaming stores (kEpiStreamOut)
        __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(static_cast<float*>(C) + o));
      } else {
        if (VARIANT == 1) {
          *reinterpret_cast<f32x4*>(pre + o) = v;
        } else {  // GELU'(v) for the backward pass; erfc(-v / sqrt2) is shared with GELU(v) below
          f32x4 d;
#pragma unroll
          for (int e = 0; e < 4; ++e) d[e] = gelu_grad_f(v[e]);
          *reinterpret_cast<f32x4*>(pre + o) = d;
        }
        uint2 h;
        h.x = pack_bf16x2(gelu_f(v[0]), gelu_f(v[1]));
        h.y = pack_bf16x2(gelu_f(v[2]), gelu_f(v[3]));
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(C) + o) = h;
      }
    }
  }
}

// Whole-tile GELU-backward epilogue (vdsl_op_gemm_bf16_gelu_bwd), also through each wave's LDS
// area: C = bf16(v * GELU'(pre)) stored as 8-byte runs; the f32 products go back into the area and,
// if `ctr` is set, each lane then reads one column of the 32-row block (64 lanes, 64 consecutive
// floats per read: no bank conflict) and writes it as a 64-byte run of the transposed output
// ctr[N][M] (needs M % 8 == 0 and WTN % 64 == 0).  `pre` is usually cold (written by the forward
// pass long before): every load of it for the wave's whole tile is issued first, before the block
// barrier that ends the main loop, so the tile pays one memory latency instead of one per unit
// (in a training step the per-unit form made this GEMM 38 us slower than without the epilogue).
template <class Cfg, int LDS_AVAIL = Cfg::LDS_BYTES, int BWD = 1>
__device__ __forceinline__ void bf16_epilogue_bwd_lds(const f32x16 (&acc)[Cfg::FM][Cfg::FN], int m0, int n0, int M,
                                                      int N, void* __restrict__ C, const float* __restrict__ pre,
                                                      char* smem, uint16_t* __restrict__ ctr) {
  constexpr int WTN = Cfg::WTN, LD = WTN + 8, Q = WTN / 4, UPL = 32 * Q / 64;  // 16-byte units per lane per row block
  // Rows of the wave's area: the whole wave tile when it fits in the block's LDS (LDS_AVAIL bytes;
  // then each lane's transposed run is WTM * 2 bytes, whole 128-byte lines), else 32.
  constexpr int AR = Cfg::NW * Cfg::WTM * LD * 4 <= LDS_AVAIL ? Cfg::WTM : 32;
  static_assert(WTN % 64 == 0, "the transposed store takes whole columns per lane");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / Cfg::WGN, wn = wave % Cfg::WGN;
  float* const area = reinterpret_cast<float*>(smem) + wave * AR * LD;
  const int row0 = m0 + wm * Cfg::WTM, col0 = n0 + wn * WTN;
  f32x4 x[Cfg::FM][UPL];
#pragma unroll
  for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
    for (int k = 0; k < UPL; ++k) {
      const int u = lane + 64 * k, row = u / Q, c4 = u % Q;
      x[i][k] = __builtin_nontemporal_load(
          reinterpret_cast<const f32x4*>(pre + static_cast<size_t>(row0 + 32 * i + row) * N + col0 + 4 * c4));
    }
  dma_barrier();  // every wave's last fragment reads of the main loop are done
  // The transposed output of rows [r0, r0 + AR) of the wave tile: lane c takes column c and writes
  // AR bf16 (AR * 2 bytes) of ctr row col0 + c.
  auto store_transposed = [&](int r0) {
#pragma unroll
    for (int cc = 0; cc < WTN / 64; ++cc) {
      const int c = lane + 64 * cc;
      u32x4* dst = reinterpret_cast<u32x4*>(ctr + static_cast<size_t>(col0 + c) * M + row0 + r0);
#pragma unroll
      for (int q4 = 0; q4 < AR / 8; ++q4) {
        u32x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = pack_bf16x2(area[(8 * q4 + 2 * e) * LD + c], area[(8 * q4 + 2 * e + 1) * LD + c]);
        dst[q4] = w;
      }
    }
  };
#pragma unroll
  for (int i = 0; i < Cfg::FM; ++i) {
    float* const blk = area + (AR == 32 ? 0 : 32 * i) * LD;  // this 32-row block's rows of the area
#pragma unroll
    for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) blk[(8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * LD + 32 * j + (lane & 31)] = acc[i][j][r];
#pragma unroll
    for (int k = 0; k < UPL; ++k) {
      const int u = lane + 64 * k, row = u / Q, c4 = u % Q;
      const f32x4 v = *reinterpret_cast<const f32x4*>(blk + row * LD + 4 * c4);
      const size_t o = static_cast<size_t>(row0 + 32 * i + row) * N + col0 + 4 * c4;
      f32x4 d;
#pragma unroll
      for (int e = 0; e < 4; ++e) d[e] = v[e] * bwd_factor<BWD>(x[i][k][e]);
      uint2 h;
      h.x = pack_bf16x2(d[0], d[1]);
      h.y = pack_bf16x2(d[2], d[3]);
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(C) + o) = h;
      if (ctr) *reinterpret_cast<f32x4*>(blk + row * LD + 4 * c4) = d;
    }
    if (AR == 32 && ctr) store_transposed(32 * i);
  }
  if (AR != 32 && ctr) store_transposed(0);
}

// Whole-tile MSE epilogue (vdsl_op_gemm_bf16_mse_packed), through each wave's LDS area like the
// GELU-backward one: with y the accumulator and d = y - t, dy = bf16(d * scale) as 8-byte runs, y
// as 16-byte runs (if wanted), dy^T through the area (each lane one column, AR * 2-byte runs of
// dy_t[N][M]), and the wave's sum of d^2 in f64 (lane order: 32-row block, unit, component; then a
// butterfly over the wave) into *part.  t, like `pre` there, is cold: every load of the wave's
// tile is issued before the block barrier that ends the main loop.  The arithmetic of d, dy and
// its rounding is that of mse_tile_vec (autodiff.hip), so dy and dy_t equal the unfused op's.
template <class Cfg, int LDS_AVAIL>
__device__ __forceinline__ void bf16_epilogue_mse_lds(const f32x16 (&acc)[Cfg::FM][Cfg::FN], int m0, int n0, int M, int N,
                                                      const float* __restrict__ t, float scale, float* __restrict__ y,
                                                      uint16_t* __restrict__ dy, uint16_t* __restrict__ dyt,
                                                      double* __restrict__ part, char* smem) {
  constexpr int WTN = Cfg::WTN, LD = WTN + 8, Q = WTN / 4, UPL = 32 * Q / 64;
  constexpr int AR = Cfg::NW * Cfg::WTM * LD * 4 <= LDS_AVAIL ? Cfg::WTM : 32;
  static_assert(WTN % 64 == 0, "the transposed store takes whole columns per lane");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / Cfg::WGN, wn = wave % Cfg::WGN;
  float* const area = reinterpret_cast<float*>(smem) + wave * AR * LD;
  const int row0 = m0 + wm * Cfg::WTM, col0 = n0 + wn * WTN;
  f32x4 x[Cfg::FM][UPL];
#pragma unroll
  for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
    for (int k = 0; k < UPL; ++k) {
      const int u = lane + 64 * k, row = u / Q, c4 = u % Q;
      x[i][k] = __builtin_nontemporal_load(
          reinterpret_cast<const f32x4*>(t + static_cast<size_t>(row0 + 32 * i + row) * N + col0 + 4 * c4));
    }
  dma_barrier();  // every wave's last fragment reads of the main loop are done
  auto store_transposed = [&](int r0) {
#pragma unroll
    for (int cc = 0; cc < WTN / 64; ++cc) {
      const int c = lane + 64 * cc;
      u32x4* dst = reinterpret_cast<u32x4*>(dyt + static_cast<size_t>(col0 + c) * M + row0 + r0);
#pragma unroll
      for (int q4 = 0; q4 < AR / 8; ++q4) {
        u32x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = pack_bf16x2(area[(8 * q4 + 2 * e) * LD + c], area[(8 * q4 + 2 * e + 1) * LD + c]);
        dst[q4] = w;
      }
    }
  };
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < Cfg::FM; ++i) {
    float* const blk = area + (AR == 32 ? 0 : 32 * i) * LD;
#pragma unroll
    for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) blk[(8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * LD + 32 * j + (lane & 31)] = acc[i][j][r];
#pragma unroll
    for (int k = 0; k < UPL; ++k) {
      const int u = lane + 64 * k, row = u / Q, c4 = u % Q;
      const f32x4 v = *reinterpret_cast<const f32x4*>(blk + row * LD + 4 * c4);
      const size_t o = static_cast<size_t>(row0 + 32 * i + row) * N + col0 + 4 * c4;
      f32x4 g;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float d = v[e] - x[i][k][e];
        s += static_cast<double>(d) * static_cast<double>(d);
        g[e] = d * scale;
      }
      uint2 h;
      h.x = pack_bf16x2(g[0], g[1]);
      h.y = pack_bf16x2(g[2], g[3]);
      *reinterpret_cast<uint2*>(dy + o) = h;
      if (y) *reinterpret_cast<f32x4*>(y + o) = v;
      if (dyt) *reinterpret_cast<f32x4*>(blk + row * LD + 4 * c4) = g;
    }
    if (AR == 32 && dyt) store_transposed(32 * i);
  }
  if (AR != 32 && dyt) store_transposed(0);
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m, 64);
  if (lane == 0) *part = s;
}

template <class Cfg, bool EDGE, bool BWD>
__global__ __launch_bounds__(Cfg::NT, Cfg::MIN_BLOCKS) void gemm_bf16_nt(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                                                        void* __restrict__ C, float* __restrict__ pre, int M, int N, int K,
                                                        int epi, int c_dtype, uint16_t* __restrict__ ctr) {
  __shared__ __attribute__((aligned(16))) char smem[Cfg::LDS_BYTES];
  epi &= ~kEpiStreamOut;  // this kernel's epilogue stores per element, with plain stores
  const int tiles_m = (M + Cfg::BM - 1) / Cfg::BM, tiles_n = (N + Cfg::BN - 1) / Cfg::BN;
  int tm, tn;
  tile_coords(xcd_remap(blockIdx.x, gridDim.x), tiles_m, tiles_n, tm, tn);
  const int m0 = tm * Cfg::BM, n0 = tn * Cfg::BN;
  f32x16 acc[Cfg::FM][Cfg::FN];
  gemm_mainloop<MfmaBf16, Cfg, EDGE>(reinterpret_cast<const char*>(A), reinterpret_cast<const char*>(B), M, N, K * 2, 0, K * 2,
                               m0, n0, smem, acc);
  bf16_store_tile<Cfg, BWD>(acc, m0, n0, M, N, C, pre, epi, c_dtype, ctr);
}

// Direct-to-LDS kernel (gemm_dma.h).  Blocks of 8 waves are sized for one block per CU, blocks
// of 4 waves for two.  BKN: B stored [K][N] (the "NN" form, no transpose first; N % 256 == 0).
// AKM: A stored [K][M] (trans_a; M % 256 == 0), read K-major as well.
template <class Cfg, bool BWD, bool BKN = false, bool AKM = false>
__global__ __launch_bounds__(Cfg::NT, Cfg::MIN_BLOCKS) void gemm_bf16_dma(const uint16_t* __restrict__ A,
                                                                               const uint16_t* __restrict__ B,
                                                                               void* __restrict__ C, float* __restrict__ pre,
                                                                               int M, int N, int K, int epi, int c_dtype,
                                                                               uint16_t* __restrict__ ctr) {
  __shared__ __attribute__((aligned(1024))) char smem[Cfg::LDS_BYTES];
  const bool stream = (epi & kEpiStreamOut) != 0;
  epi &= ~kEpiStreamOut;
  const int tiles_m = (M + Cfg::BM - 1) / Cfg::BM, tiles_n = (N + Cfg::BN - 1) / Cfg::BN;
  int tm, tn;
  tile_coords(xcd_remap(blockIdx.x, gridDim.x), tiles_m, tiles_n, tm, tn);
  const int m0 = tm * Cfg::BM, n0 = tn * Cfg::BN;
  f32x16 acc[Cfg::FM][Cfg::FN];
  dma_mainloop<MfmaBf16, Cfg, f32x16, Cfg::FM, Cfg::FN, BKN, AKM>(reinterpret_cast<const char*>(A),
                                                                  reinterpret_cast<const char*>(B), M, N, K * 2, 0, K * 2, m0,
                                                                  n0, smem, acc, N * 2, M * 2);
  if constexpr (kLdsEpilogue<Cfg>) {
    // Block-uniform: the tile is whole, N allows aligned runs, and the epilogue is one the LDS path has.
    const bool whole = m0 + Cfg::BM <= M && n0 + Cfg::BN <= N && N % 4 == 0;
    if constexpr (BWD) {
      if constexpr (Cfg::WTN % 64 == 0 && Cfg::FM * Cfg::WTN / 2 <= 64) {  // pre prefetch: FM * WTN / 2 VGPRs
        if (whole && (!ctr || M % 8 == 0)) {
          bf16_epilogue_bwd_lds<Cfg>(acc, m0, n0, M, N, C, pre, smem, ctr);
          return;
        }
      }
    } else {
      const bool v0 = epi == VDSL_EPI_NONE && c_dtype == VDSL_F32 && !pre;
      const bool v1 = epi == VDSL_EPI_GELU && c_dtype == VDSL_BF16 && pre;
      if (whole && (v0 || v1)) {
        dma_barrier();  // every wave's last fragment reads of the main loop are done
        if (v0 && stream) bf16_epilogue_tile_lds<Cfg, 3>(acc, m0, n0, N, C, pre, smem);
        else if (v0) bf16_epilogue_tile_lds<Cfg, 0>(acc, m0, n0, N, C, pre, smem);
        else bf16_epilogue_tile_lds<Cfg, 1>(acc, m0, n0, N, C, pre, smem);
        return;
      }
    }
  }
  bf16_store_tile<Cfg, BWD>(acc, m0, n0, M, N, C, pre, epi, c_dtype, ctr);
}

// Any K (including K % 8 != 0): one lane per output, f32 accumulate in k order.
__global__ __launch_bounds__(256) void gemm_bf16_nt_simple(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                                                           void* __restrict__ C, float* __restrict__ pre, int M, int N,
                                                           int K, int epi, int c_dtype, uint16_t* __restrict__ ctr) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= static_cast<int64_t>(M) * N) return;
  epi &= ~kEpiStreamOut;
  const int row = static_cast<int>(idx / N), col = static_cast<int>(idx % N);
  float v = 0.0f;
  for (int k = 0; k < K; ++k)
    v = __builtin_fmaf(bf16_to_f32(A[static_cast<size_t>(row) * K + k]), bf16_to_f32(B[static_cast<size_t>(col) * K + k]), v);
  if (epi == kEpiGeluBwd) {
    const uint16_t h = f32_to_bf16(v * gelu_grad_f(pre[idx]));
    static_cast<uint16_t*>(C)[idx] = h;
    if (ctr) ctr[static_cast<size_t>(col) * M + row] = h;
    return;
  }
  if (pre) pre[idx] = v;
  float y = v;
  if (epi == VDSL_EPI_GELU) y = gelu_f(v);
  else if (epi == VDSL_EPI_RELU) y = v > 0.0f ? v : 0.0f;
  if (c_dtype == VDSL_F32) static_cast<float*>(C)[idx] = y;
  else static_cast<uint16_t*>(C)[idx] = f32_to_bf16(y);
}

// ---- packed-weight form (gemm_bpk.h main loop): B in MFMA fragment order, A through LDS --------
// For constant weights (forward GEMMs on [out][in] weights): the weight is packed once and each
// wave loads its B fragments straight into registers.  Same k-steps in the same order with the same
// MFMA as every other configuration, so the same results bit for bit.  Measured standalone on
// 2048x4096x4096 (random bf16, f32 out): 61-63 us against 66-68 us for the direct-to-LDS kernel.
using Pb0 = BpkConfig<MfmaBf16, 4, 2, 4, 3>;  // 128 x 256 blocks, 4 waves of 128 x 64

// BWD: the backward epilogues (1: vdsl_op_gemm_bf16_gelu_bwd_packed, C = da, pre an input, ctr =
// da^T; 2: vdsl_op_gemm_bf16_mul_packed, the factor given); their LDS is enlarged so the whole wave
// tile stages at once (whole-line transposed stores).
template <class Cfg, bool BWD>
constexpr int bpk_bf16_smem() {
  return BWD && Cfg::NW * Cfg::WTM * (Cfg::WTN + 8) * 4 > Cfg::LDS_BYTES ? Cfg::NW * Cfg::WTM * (Cfg::WTN + 8) * 4
                                                                          : Cfg::LDS_BYTES;
}

// BWD: the backward epilogue mode (bf16_epilogue); DERIV: the forward VDSL_EPI_GELU_DERIV kernel.
template <class Cfg, int BWD, bool DERIV = false>
__global__ __launch_bounds__(Cfg::NT, 1) void gemm_bf16_bpk(const uint16_t* __restrict__ A, const uint16_t* __restrict__ Bp,
                                                         void* __restrict__ C, float* __restrict__ pre, int M, int N, int K,
                                                         int epi, int c_dtype, uint16_t* __restrict__ ctr) {
  // The only __shared__ variable (see gemm_bpk.h); after the main loop it stages the epilogue.
  __shared__ __attribute__((aligned(1024))) char smem[bpk_bf16_smem<Cfg, BWD != 0>()];
  const bool stream = (epi & kEpiStreamOut) != 0;
  epi &= ~kEpiStreamOut;
  // Tiles in groups of 8 tile-rows, walked column-major (tile_coords): the 32 blocks one XCD runs
  // (congruent ids, made consecutive by xcd_remap) then cover 8 row tiles x 4 column panels, so
  // each XCD's L2 fetches 1/2 of A and 1/4 of B (2048x4096x4096: 128 MB fetched in all, against
  // 168 MB when each XCD took 16 row tiles x 2 panels).
  const int tiles_m = (M + Cfg::BM - 1) / Cfg::BM, tiles_n = (N + Cfg::BN - 1) / Cfg::BN;
  int tm, tn;
  tile_coords(xcd_remap(blockIdx.x, gridDim.x), tiles_m, tiles_n, tm, tn);
  const int m0 = tm * Cfg::BM, n0 = tn * Cfg::BN;
  f32x16 acc[Cfg::FM][Cfg::FN];
  bpk_mainloop<MfmaBf16, Cfg>(reinterpret_cast<const char*>(A), reinterpret_cast<const char*>(Bp), M, N / 32, K * 2, 0, K * 2,
                              m0, n0, smem, acc);
  static_assert(kLdsEpilogue<Cfg>, "the LDS-staged epilogue must fit the main loop's LDS");
  const bool whole = m0 + Cfg::BM <= M && n0 + Cfg::BN <= N && N % 4 == 0;
  if constexpr (BWD != 0) {
    if (whole && (!ctr || M % 8 == 0)) {
      bf16_epilogue_bwd_lds<Cfg, bpk_bf16_smem<Cfg, true>(), BWD>(acc, m0, n0, M, N, C, pre, smem, ctr);
      return;
    }
  } else if constexpr (DERIV) {
    if (whole) {
      __syncthreads();  // every wave is past its last read of the main loop's LDS
      bf16_epilogue_tile_lds<Cfg, 2>(acc, m0, n0, N, C, pre, smem);
      return;
    }
  } else {
    const bool v0 = epi == VDSL_EPI_NONE && c_dtype == VDSL_F32 && !pre;
    const bool v1 = epi == VDSL_EPI_GELU && c_dtype == VDSL_BF16 && pre;
    if (whole && (v0 || v1)) {
      __syncthreads();  // every wave is past its last read of the main loop's LDS
      if (v0 && stream) bf16_epilogue_tile_lds<Cfg, 3>(acc, m0, n0, N, C, pre, smem);
      else if (v0) bf16_epilogue_tile_lds<Cfg, 0>(acc, m0, n0, N, C, pre, smem);
      else bf16_epilogue_tile_lds<Cfg, 1>(acc, m0, n0, N, C, pre, smem);
      return;
    }
  }
  bf16_store_tile<Cfg, BWD, DERIV>(acc, m0, n0, M, N, C, pre, epi, c_dtype, ctr);
}

// The packed GEMM fused with the MSE loss of its f32 output (vdsl_op_gemm_bf16_mse_packed): whole
// tiles only; partials[tile * W + wave] receives each wave's sum of squared differences.
template <class Cfg>
__global__ __launch_bounds__(Cfg::NT, 1) void gemm_bf16_bpk_mse(const uint16_t* __restrict__ A, const uint16_t* __restrict__ Bp,
                                                             const float* __restrict__ t, float* __restrict__ y,
                                                             uint16_t* __restrict__ dy, uint16_t* __restrict__ dyt,
                                                             double* __restrict__ partials, int M, int N, int K, float scale) {
  __shared__ __attribute__((aligned(1024))) char smem[bpk_bf16_smem<Cfg, true>()];
  const int tiles_m = M / Cfg::BM, tiles_n = N / Cfg::BN;
  int tm, tn;
  tile_coords(xcd_remap(blockIdx.x, gridDim.x), tiles_m, tiles_n, tm, tn);
  const int m0 = tm * Cfg::BM, n0 = tn * Cfg::BN;
  f32x16 acc[Cfg::FM][Cfg::FN];
  bpk_mainloop<MfmaBf16, Cfg>(reinterpret_cast<const char*>(A), reinterpret_cast<const char*>(Bp), M, N / 32, K * 2, 0, K * 2,
                              m0, n0, smem, acc);
  double* const part = partials + (static_cast<size_t>(tm) * tiles_n + tn) * Cfg::W + (threadIdx.x >> 6);
  bf16_epilogue_mse_lds<Cfg, bpk_bf16_smem<Cfg, true>()>(acc, m0, n0, M, N, t, scale, y, dy, dyt, part, smem);
}

template <class Cfg>
int launch_cfg(const uint16_t* A, const uint16_t* B, void* C, float* pre, int M, int N, int K, int epi, int ct, hipStream_t s,
               uint16_t* ctr) {
  const int64_t tiles = static_cast<int64_t>((M + Cfg::BM - 1) / Cfg::BM) * ((N + Cfg::BN - 1) / Cfg::BN);
  const dim3 g(static_cast<unsigned>(tiles)), b(Cfg::NT);
  const bool edge = gemm_needs_edge<Cfg>(M, N, static_cast<int64_t>(K) * 2);
  if (epi == kEpiGeluBwd) {
    if (edge) hipLaunchKernelGGL((gemm_bf16_nt<Cfg, true, true>), g, b, 0, s, A, B, C, pre, M, N, K, epi, ct, ctr);
    else hipLaunchKernelGGL((gemm_bf16_nt<Cfg, false, true>), g, b, 0, s, A, B, C, pre, M, N, K, epi, ct, ctr);
  } else {
    if (edge) hipLaunchKernelGGL((gemm_bf16_nt<Cfg, true, false>), g, b, 0, s, A, B, C, pre, M, N, K, epi, ct, ctr);
    else hipLaunchKernelGGL((gemm_bf16_nt<Cfg, false, false>), g, b, 0, s, A, B, C, pre, M, N, K, epi, ct, ctr);
  }
  return check_launch("gemm_bf16_nt");
}

template <class Cfg>
int launch_dma(const uint16_t* A, const uint16_t* B, void* C, float* pre, int M, int N, int K, int epi, int ct, hipStream_t s,
               uint16_t* ctr) {
  const int64_t tiles = static_cast<int64_t>((M + Cfg::BM - 1) / Cfg::BM) * ((N + Cfg::BN - 1) / Cfg::BN);
  if (epi == kEpiGeluBwd)
    hipLaunchKernelGGL((gemm_bf16_dma<Cfg, true>), dim3(static_cast<unsigned>(tiles)), dim3(Cfg::NT), 0, s, A, B, C, pre, M, N, K, epi,
                       ct, ctr);
  else
    hipLaunchKernelGGL((gemm_bf16_dma<Cfg, false>), dim3(static_cast<unsigned>(tiles)), dim3(Cfg::NT), 0, s, A, B, C, pre, M, N, K,
                       epi, ct, ctr);
  return check_launch("gemm_bf16_dma");
}

// The "NN" form (B stored [K][N]) without a transpose: the direct-to-LDS configurations with
// 256-wide tiles read B K-major (gemm_dma.h) when every tile is whole along N.  With akm, the "TN"
// form (A stored [K][M] as well, e.g. dW = g^T x with g [batch][out] as stored): the 256 x 256
// configuration reads both operands K-major when M % 256 == 0 too.  Returns 1 (never a status)
// when the shape needs the transpose path instead.
bool dma_kn_runs(int cfg, int64_t M, int64_t N, bool akm) {
  if (N % 256 != 0) return false;
  return akm ? (M % 256 == 0 && cfg == 15) : (cfg == 15 || cfg == 23);
}

int launch_dma_kn(int cfg, const uint16_t* A, const uint16_t* B, void* C, float* pre, int M, int N, int K, int epi, int ct,
                  hipStream_t s, bool akm = false) {
  if (!dma_kn_runs(cfg, M, N, akm)) return 1;
  auto go = [&](auto cfg_tag, auto akm_tag) {
    using Cfg = decltype(cfg_tag);
    constexpr bool kAkm = decltype(akm_tag)::value;
    const int64_t tiles = static_cast<int64_t>((M + Cfg::BM - 1) / Cfg::BM) * (N / Cfg::BN);
    hipLaunchKernelGGL((gemm_bf16_dma<Cfg, false, true, kAkm>), dim3(static_cast<unsigned>(tiles)), dim3(Cfg::NT), 0, s, A, B, C,
                       pre, M, N, K, epi, ct, nullptr);
    return check_launch(kAkm ? "gemm_bf16_dma<K-major A and B>" : "gemm_bf16_dma<K-major B>");
  };
  if (akm) return go(Dm15{}, std::true_type{});
  if (cfg == 15) return go(Dm15{}, std::false_type{});
  if (cfg == 23) return go(Dm23{}, std::false_type{});
  return 1;
}

// Configuration for a shape.  The direct-to-LDS loop (14..) runs whenever K is a whole number of
// its 64-byte stages (K % 32 == 0); measured on MI355X with random operands (bf16, f32 out):
// 128x256 blocks of 8 waves are fastest while they still give every CU a block, with 128-byte
// stages and fragments read two k-steps ahead when K % 64 == 0 (2048x4096x4096: 890-915 TFLOP/s
// against 845-860 with 64-byte stages), 256x256 blocks once those do (4096x4096x2048: 955 against
// 870).  Smaller launches take 128x128 blocks, two per CU.  Other K use the register-staged loop
// (0..13), where 128x128 tiles are fastest below 512 tiles of 256x128 and 256x128 tiles of 8
// waves above.
int choose_config(int64_t M, int64_t N, int64_t K) {
  const bool dma = dma_k_ok(0, K * 2), dma128 = dma_k_ok(0, K * 2, 128);
  const int o = gemm_config_override();
  if (o >= 0 && o < kNumConfigs && (o < kFirstDma || (o < kFirstDma128 ? dma : dma128))) return o;
  if (dma) {
    const int64_t t256 = ((M + 255) / 256) * ((N + 255) / 256);
    const int64_t t128x256 = ((M + 127) / 128) * ((N + 255) / 256);
    if (t256 >= 240) return 15;
    if (t128x256 >= 128) return dma128 ? 23 : 14;
    return 17;
  }
  const int64_t tiles_256x128 = ((M + 255) / 256) * ((N + 127) / 128);
  return tiles_256x128 >= 512 ? 13 : 0;
}

int launch_nt(const uint16_t* A, const uint16_t* B, void* C, float* pre, int M, int N, int K, int epi, int ct, hipStream_t s,
              uint16_t* ctr = nullptr) {
  if (K % 8 != 0) {
    const int64_t blocks = (static_cast<int64_t>(M) * N + 255) / 256;
    hipLaunchKernelGGL(gemm_bf16_nt_simple, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, A, B, C, pre, M, N, K, epi, ct, ctr);
    return check_launch("gemm_bf16_nt_simple");
  }
  switch (choose_config(M, N, K)) {
    case 1: return launch_cfg<Bf1>(A, B, C, pre, M, N, K, epi, ct, s, ctr);
    case 2: return launch_cfg<Bf2>(A, B, C, pre, M, N, K, epi, ct, s, ctr);
    case 3: return launch_cfg<Bf3>(A, B, C, pre, M, N, K, epi, ct, s, ctr);
    case 4: return launch_cfg<Bf4>(A, B, C, pre, M, N, K, epi, ct, s, ctr);
    case 5: return launch_cfg<Bf5>(A, B, C, pre, M, N, K, epi, ct, s, ctr);
    case 6: return launch_cfg<Bf6>(A, B, C, pre, M, N, K, epi, ct, s, ctr);
    case 7: return launch_cfg<Bf7>(A, B, C, pre, M, N, K, epi, ct, s, ctr);
    case 8: return launch_cfg<Bf8>(A, B, C, pre, M, N, K, epi, ct, s, ctr);
    case 9: return launch_cfg<Bf9>(A, B, C, pre, M, N, K, epi, ct, s, ctr);
    case 10: return launch_cfg<Bf10>(A, B, C, pre, M, N, K, epi, ct, s, ctr);
    case 11: return launch_cfg<Bf11>(A, B, C, pre, M, N, K, epi, ct, s, ctr);
    case 12: return launch_cfg<Bf12>(A, B, C, pre, M, N, K, epi, ct, s, ctr);
    case 13: return launch_cfg<Bf13>(A, B, C, pre, M, N, K, epi, ct, s, ctr);
    case 14: return launch_dma<Dm14>(A, B, C, pre, M, N, K, epi, ct, s, ctr);
    case 15: return launch_dma<Dm15>(A, B, C, pre, M, N, K, epi, ct, s, ctr);
    case 16: return launch_dma<Dm16>(A, B, C, pre, M, N, K, epi, ct, s, ctr);
    case 17: return launch_dma<Dm17>(A, B, C, pre, M, N, K, epi, ct, s, ctr);
    case 18: return launch_dma<Dm18>(A, B, C, pre, M, N, K, epi, ct, s, ctr);
    case 19: return launch_dma<Dm19>(A, B, C, pre, M, N, K, epi, ct, s, ctr);
    case 20: return launch_dma<Dm20>(A, B, C, pre, M, N, K, epi, ct, s, ctr);
    case 21: return launch_dma<Dm21>(A, B, C, pre, M, N, K, epi, ct, s, ctr);
    case 22: return launch_dma<Dm22>(A, B, C, pre, M, N, K, epi, ct, s, ctr);
    case 23: return launch_dma<Dm23>(A, B, C, pre, M, N, K, epi, ct, s, ctr);
    case 24: return launch_dma<Dm24>(A, B, C, pre, M, N, K, epi, ct, s, ctr);
    case 25: return launch_dma<Dm25>(A, B, C, pre, M, N, K, epi, ct, s, ctr);
    case 26: return launch_dma<Dm26>(A, B, C, pre, M, N, K, epi, ct, s, ctr);
    default: return launch_cfg<Bf0>(A, B, C, pre, M, N, K, epi, ct, s, ctr);
  }
}

// Whether a GEMM's result leaves through streaming stores: a plain f32 output bound as an output.
bool stream_out(vdsl_buffer C, int epilogue, int c_dtype) {
  return epilogue == VDSL_EPI_NONE && c_dtype == VDSL_F32 && C->binding == VDSL_BIND_OUTPUT;
}

// kSizeOverflow when the re-layout copies' size does not fit size_t.
// Workspace of the transpose path: none when B is stored [K][N] and a configuration that reads the
// operands K-major runs the shape (vdsl_op_gemm_bf16 then transposes nothing).
size_t workspace_bytes(int ta, int tb, int64_t M, int64_t N, int64_t K) {
  if (!tb && K % 8 == 0 && M <= 0x7fffffff && N <= 0x7fffffff && dma_kn_runs(choose_config(M, N, K), M, N, ta)) return 0;
  const size_t a = ta ? nbytes(M, K, 2) : 0, b = tb ? 0 : nbytes(N, K, 2);
  if (a == kSizeOverflow || b == kSizeOverflow || a > kSizeOverflow - 1 - b) return kSizeOverflow;
  return a + b;
}

}  // namespace
}  // namespace vdsl

using namespace vdsl;

extern "C" int vdsl_gemm_bf16_workspace_bytes(int32_t trans_a, int32_t trans_b, int64_t M, int64_t N, int64_t K,
                                              size_t* bytes) {
  if (!bytes) return fail(VDSL_ERR_INVALID_ARG, "bytes is null");
  if (M < 0 || N < 0 || K < 0) return fail(VDSL_ERR_INVALID_ARG, "negative GEMM extent");
  const size_t ws = workspace_bytes(trans_a != 0, trans_b != 0, M, N, K);
  if (ws == kSizeOverflow) return fail(VDSL_ERR_SHAPE, "GEMM workspace size overflows (extents too large)");
  *bytes = ws;
  return VDSL_OK;
}

extern "C" int vdsl_op_gemm_bf16(vdsl_queue q, int32_t trans_a, int32_t trans_b, int64_t M, int64_t N, int64_t K,
                                 vdsl_buffer A, vdsl_buffer B, vdsl_buffer C, int32_t c_dtype, int32_t epilogue,
                                 vdsl_buffer pre_act, vdsl_buffer workspace) {
  VDSL_TRY(enter_queue(q));
  if (M < 0 || N < 0 || K < 0) return fail(VDSL_ERR_INVALID_ARG, "negative GEMM extent");
  if (M > 0x7fffffff || N > 0x7fffffff || K > 0x3fffffff) return fail(VDSL_ERR_UNSUPPORTED, "GEMM extent too large");
  if (c_dtype != VDSL_F32 && c_dtype != VDSL_BF16) return fail(VDSL_ERR_UNSUPPORTED, "C must be f32 or bf16");
  if (epilogue < VDSL_EPI_NONE || epilogue > VDSL_EPI_RELU) return fail(VDSL_ERR_INVALID_ARG, "unknown epilogue");
  const bool ta = trans_a != 0, tb = trans_b != 0;
  VDSL_TRY(check_buffer(q, A, nbytes(M, K, 2), "A", false));
  VDSL_TRY(check_buffer(q, B, nbytes(N, K, 2), "B", false));
  VDSL_TRY(check_buffer(q, C, nbytes(M, N, dtype_size(c_dtype)), "C", true));
  if (pre_act) VDSL_TRY(check_buffer(q, pre_act, nbytes(M, N, 4), "pre_act", true));
  // checked here, for the path this call takes (the K-major configurations need none)
  const size_t ws = workspace_bytes(ta, tb, M, N, K);
  if (ws == kSizeOverflow) return fail(VDSL_ERR_SHAPE, "GEMM workspace size overflows (extents too large)");
  if (ws) VDSL_TRY(check_buffer(q, workspace, ws, "workspace", true));
  if (M == 0 || N == 0) return VDSL_OK;

  const uint16_t* a = static_cast<const uint16_t*>(A->ptr);
  const uint16_t* b = static_cast<const uint16_t*>(B->ptr);
  float* pre = pre_act ? static_cast<float*>(pre_act->ptr) : nullptr;
  const int epi = epilogue | (stream_out(C, epilogue, c_dtype) ? kEpiStreamOut : 0);
  if (ws == 0 && !tb) {  // B stored [K][N] (and A [K][M] if ta): read K-major by a 256-wide configuration
    return launch_dma_kn(choose_config(M, N, K), a, b, C->ptr, pre, static_cast<int>(M), static_cast<int>(N),
                         static_cast<int>(K), epi, c_dtype, q->stream, ta);
  }
  char* w = ws ? static_cast<char*>(workspace->ptr) : nullptr;
  if (ta) {  // A stored [K][M] -> [M][K]
    VDSL_TRY(launch_transpose(a, w, K, M, VDSL_BF16, q->stream));
    a = reinterpret_cast<const uint16_t*>(w);
    w += static_cast<size_t>(M) * K * 2;
  }
  if (!tb) {  // B stored [K][N] -> [N][K]
    VDSL_TRY(launch_transpose(b, w, K, N, VDSL_BF16, q->stream));
    b = reinterpret_cast<const uint16_t*>(w);
  }
  return launch_nt(a, b, C->ptr, pre, static_cast<int>(M), static_cast<int>(N), static_cast<int>(K), epi, c_dtype,
                   q->stream);
}

extern "C" int vdsl_debug_gemm_config(int32_t config) {
  vdsl::gemm_config_override();  // consume the environment value first, so it cannot override this
  vdsl::g_gemm_config.store(config < 0 ? -1 : config, std::memory_order_relaxed);
  return VDSL_OK;
}

extern "C" int vdsl_op_gemm_bf16_gelu_bwd(vdsl_queue q, int64_t M, int64_t N, int64_t K, vdsl_buffer A, vdsl_buffer B,
                                          vdsl_buffer pre, vdsl_buffer da, vdsl_buffer da_t) {
  VDSL_TRY(enter_queue(q));
  if (M < 0 || N < 0 || K < 0) return fail(VDSL_ERR_INVALID_ARG, "negative GEMM extent");
  if (M > 0x7fffffff || N > 0x7fffffff || K > 0x3fffffff) return fail(VDSL_ERR_UNSUPPORTED, "GEMM extent too large");
  VDSL_TRY(check_buffer(q, A, nbytes(M, K, 2), "A", false));
  VDSL_TRY(check_buffer(q, B, nbytes(N, K, 2), "B", false));
  VDSL_TRY(check_buffer(q, pre, nbytes(M, N, 4), "pre", false));
  VDSL_TRY(check_buffer(q, da, nbytes(M, N, 2), "da", true));
  if (da_t) VDSL_TRY(check_buffer(q, da_t, nbytes(M, N, 2), "da_t", true));
  if (M == 0 || N == 0) return VDSL_OK;
  return launch_nt(static_cast<const uint16_t*>(A->ptr), static_cast<const uint16_t*>(B->ptr), da->ptr,
                   static_cast<float*>(pre->ptr), static_cast<int>(M), static_cast<int>(N), static_cast<int>(K), kEpiGeluBwd,
                   VDSL_BF16, q->stream, da_t ? static_cast<uint16_t*>(da_t->ptr) : nullptr);
}

extern "C" int vdsl_op_pack_bf16_weights(vdsl_queue q, int64_t N, int64_t K, vdsl_buffer w, vdsl_buffer wp) {
  VDSL_TRY(enter_queue(q));
  if (N < 0 || K < 0) return fail(VDSL_ERR_INVALID_ARG, "negative weight extent");
  if (N % 32 || K % 16) return fail(VDSL_ERR_UNSUPPORTED, "packed bf16 weights need N % 32 == 0 and K % 16 == 0");
  const size_t n = nbytes(N, K, 2);
  VDSL_TRY(check_buffer(q, w, n, "w", false));
  VDSL_TRY(check_buffer(q, wp, n, "wp", true));
  if (w == wp) return fail(VDSL_ERR_INVALID_ARG, "w and wp must be different buffers");
  if (n == 0) return VDSL_OK;
  int64_t blocks = (static_cast<int64_t>(n / 16) + 255) / 256;
  if (blocks > 16384) blocks = 16384;
  hipLaunchKernelGGL(bpk_pack_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, q->stream,
                     static_cast<const char*>(w->ptr), static_cast<char*>(wp->ptr), N / 32, 2 * K / 32, 2 * K);
  return check_launch("bpk_pack_kernel");
}

extern "C" int vdsl_op_gemm_bf16_packed(vdsl_queue q, int64_t M, int64_t N, int64_t K, vdsl_buffer A, vdsl_buffer Bp,
                                        vdsl_buffer C, int32_t c_dtype, int32_t epilogue, vdsl_buffer pre_act) {
  VDSL_TRY(enter_queue(q));
  if (M < 0 || N < 0 || K < 0) return fail(VDSL_ERR_INVALID_ARG, "negative GEMM extent");
  if (M > 0x7fffffff || N > 0x7fffffff || K > 0x3fffffff) return fail(VDSL_ERR_UNSUPPORTED, "GEMM extent too large");
  if (N % 32) return fail(VDSL_ERR_UNSUPPORTED, "packed GEMM needs N % 32 == 0");
  if ((2 * K) % (128 * Pb0::NR) || K == 0) return fail(VDSL_ERR_UNSUPPORTED, "packed bf16 GEMM needs K % 256 == 0 and K > 0");
  if (c_dtype != VDSL_F32 && c_dtype != VDSL_BF16) return fail(VDSL_ERR_UNSUPPORTED, "C must be f32 or bf16");
  if (epilogue < VDSL_EPI_NONE || epilogue > VDSL_EPI_GELU_DERIV) return fail(VDSL_ERR_INVALID_ARG, "unknown epilogue");
  if (epilogue == VDSL_EPI_GELU_DERIV && (!pre_act || c_dtype != VDSL_BF16))
    return fail(VDSL_ERR_INVALID_ARG, "VDSL_EPI_GELU_DERIV needs pre_act and a bf16 C");
  VDSL_TRY(check_buffer(q, A, nbytes(M, K, 2), "A", false));
  VDSL_TRY(check_buffer(q, Bp, nbytes(N, K, 2), "Bp", false));
  VDSL_TRY(check_buffer(q, C, nbytes(M, N, dtype_size(c_dtype)), "C", true));
  if (pre_act) VDSL_TRY(check_buffer(q, pre_act, nbytes(M, N, 4), "pre_act", true));
  if (M == 0 || N == 0) return VDSL_OK;
  const int64_t tiles = ((M + Pb0::BM - 1) / Pb0::BM) * ((N + Pb0::BN - 1) / Pb0::BN);
  auto* kern = epilogue == VDSL_EPI_GELU_DERIV ? gemm_bf16_bpk<Pb0, 0, true> : gemm_bf16_bpk<Pb0, 0, false>;
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(tiles)), dim3(Pb0::NT), 0, q->stream,
                     static_cast<const uint16_t*>(A->ptr), static_cast<const uint16_t*>(Bp->ptr), C->ptr,
                     pre_act ? static_cast<float*>(pre_act->ptr) : nullptr, static_cast<int>(M), static_cast<int>(N),
                     static_cast<int>(K), epilogue | (stream_out(C, epilogue, c_dtype) ? kEpiStreamOut : 0), c_dtype, nullptr);
  return check_launch("gemm_bf16_bpk");
}

extern "C" int vdsl_op_gemm_bf16_gelu_bwd_packed(vdsl_queue q, int64_t M, int64_t N, int64_t K, vdsl_buffer A,
                                                 vdsl_buffer Bp, vdsl_buffer pre, vdsl_buffer da, vdsl_buffer da_t) {
  VDSL_TRY(enter_queue(q));
  if (M < 0 || N < 0 || K < 0) return fail(VDSL_ERR_INVALID_ARG, "negative GEMM extent");
  if (M > 0x7fffffff || N > 0x7fffffff || K > 0x3fffffff) return fail(VDSL_ERR_UNSUPPORTED, "GEMM extent too large");
  if (N % 32) return fail(VDSL_ERR_UNSUPPORTED, "packed GEMM needs N % 32 == 0");
  if ((2 * K) % (128 * Pb0::NR) || K == 0) return fail(VDSL_ERR_UNSUPPORTED, "packed bf16 GEMM needs K % 256 == 0 and K > 0");
  VDSL_TRY(check_buffer(q, A, nbytes(M, K, 2), "A", false));
  VDSL_TRY(check_buffer(q, Bp, nbytes(N, K, 2), "Bp", false));
  VDSL_TRY(check_buffer(q, pre, nbytes(M, N, 4), "pre", false));
  VDSL_TRY(check_buffer(q, da, nbytes(M, N, 2), "da", true));
  if (da_t) VDSL_TRY(check_buffer(q, da_t, nbytes(M, N, 2), "da_t", true));
  if (M == 0 || N == 0) return VDSL_OK;
  const int64_t tiles = ((M + Pb0::BM - 1) / Pb0::BM) * ((N + Pb0::BN - 1) / Pb0::BN);
  hipLaunchKernelGGL((gemm_bf16_bpk<Pb0, 1>), dim3(static_cast<unsigned>(tiles)), dim3(Pb0::NT), 0, q->stream,
                     static_cast<const uint16_t*>(A->ptr), static_cast<const uint16_t*>(Bp->ptr), da->ptr,
                     static_cast<float*>(pre->ptr), static_cast<int>(M), static_cast<int>(N), static_cast<int>(K),
                     kEpiGeluBwd, VDSL_BF16, da_t ? static_cast<uint16_t*>(da_t->ptr) : nullptr);
  return check_launch("gemm_bf16_bpk<gelu_bwd>");
}

extern "C" int vdsl_op_gemm_bf16_mul_packed(vdsl_queue q, int64_t M, int64_t N, int64_t K, vdsl_buffer A, vdsl_buffer Bp,
                                            vdsl_buffer g, vdsl_buffer c, vdsl_buffer c_t) {
  VDSL_TRY(enter_queue(q));
  if (M < 0 || N < 0 || K < 0) return fail(VDSL_ERR_INVALID_ARG, "negative GEMM extent");
  if (M > 0x7fffffff || N > 0x7fffffff || K > 0x3fffffff) return fail(VDSL_ERR_UNSUPPORTED, "GEMM extent too large");
  if (N % 32) return fail(VDSL_ERR_UNSUPPORTED, "packed GEMM needs N % 32 == 0");
  if ((2 * K) % (128 * Pb0::NR) || K == 0) return fail(VDSL_ERR_UNSUPPORTED, "packed bf16 GEMM needs K % 256 == 0 and K > 0");
  VDSL_TRY(check_buffer(q, A, nbytes(M, K, 2), "A", false));
  VDSL_TRY(check_buffer(q, Bp, nbytes(N, K, 2), "Bp", false));
  VDSL_TRY(check_buffer(q, g, nbytes(M, N, 4), "g", false));
  VDSL_TRY(check_buffer(q, c, nbytes(M, N, 2), "c", true));
  if (c_t) VDSL_TRY(check_buffer(q, c_t, nbytes(M, N, 2), "c_t", true));
  if (M == 0 || N == 0) return VDSL_OK;
  const int64_t tiles = ((M + Pb0::BM - 1) / Pb0::BM) * ((N + Pb0::BN - 1) / Pb0::BN);
  hipLaunchKernelGGL((gemm_bf16_bpk<Pb0, 2>), dim3(static_cast<unsigned>(tiles)), dim3(Pb0::NT), 0, q->stream,
                     static_cast<const uint16_t*>(A->ptr), static_cast<const uint16_t*>(Bp->ptr), c->ptr,
                     static_cast<float*>(g->ptr), static_cast<int>(M), static_cast<int>(N), static_cast<int>(K),
                     kEpiGeluBwd, VDSL_BF16, c_t ? static_cast<uint16_t*>(c_t->ptr) : nullptr);
  return check_launch("gemm_bf16_bpk<mul>");
}

extern "C" int vdsl_op_gemm_bf16_mse_packed(vdsl_queue q, int64_t M, int64_t N, int64_t K, vdsl_buffer A, vdsl_buffer Bp,
                                            vdsl_buffer t, vdsl_buffer y, vdsl_buffer loss, vdsl_buffer dy, vdsl_buffer dy_t,
                                            vdsl_buffer partials) {
  VDSL_TRY(enter_queue(q));
  if (M <= 0 || N <= 0 || K <= 0) return fail(VDSL_ERR_INVALID_ARG, "GEMM + MSE needs positive extents");
  if (M > 0x7fffffff || N > 0x7fffffff || K > 0x3fffffff) return fail(VDSL_ERR_UNSUPPORTED, "GEMM extent too large");
  if (M % Pb0::BM || N % Pb0::BN) return fail(VDSL_ERR_UNSUPPORTED, "GEMM + MSE needs M % 128 == 0 and N % 256 == 0");
  if ((2 * K) % (128 * Pb0::NR)) return fail(VDSL_ERR_UNSUPPORTED, "packed bf16 GEMM needs K % 256 == 0");
  VDSL_TRY(check_buffer(q, A, nbytes(M, K, 2), "A", false));
  VDSL_TRY(check_buffer(q, Bp, nbytes(N, K, 2), "Bp", false));
  VDSL_TRY(check_buffer(q, t, nbytes(M, N, 4), "t", false));
  if (y) VDSL_TRY(check_buffer(q, y, nbytes(M, N, 4), "y", true));
  VDSL_TRY(check_buffer(q, loss, 4, "loss", true));
  VDSL_TRY(check_buffer(q, dy, nbytes(M, N, 2), "dy", true));
  if (dy_t) VDSL_TRY(check_buffer(q, dy_t, nbytes(M, N, 2), "dy_t", true));
  const int64_t tiles = (M / Pb0::BM) * (N / Pb0::BN), n_part = tiles * Pb0::W;
  VDSL_TRY(check_buffer(q, partials, nbytes(vdsl_mse_partials_count(M, N), 4), "partials", true));
  if (static_cast<int64_t>(n_part * 2) > vdsl_mse_partials_count(M, N))
    return fail(VDSL_ERR_UNSUPPORTED, "GEMM + MSE: partial sums exceed the MSE scratch size");
  const size_t n = static_cast<size_t>(M) * static_cast<size_t>(N);
  const float scale = 2.0f / static_cast<float>(n);  // as vdsl_op_mse_fwd_bwd
  double* part = static_cast<double*>(partials->ptr);
  hipLaunchKernelGGL((gemm_bf16_bpk_mse<Pb0>), dim3(static_cast<unsigned>(tiles)), dim3(Pb0::NT), 0, q->stream,
                     static_cast<const uint16_t*>(A->ptr), static_cast<const uint16_t*>(Bp->ptr),
                     static_cast<const float*>(t->ptr), y ? static_cast<float*>(y->ptr) : nullptr,
                     static_cast<uint16_t*>(dy->ptr), dy_t ? static_cast<uint16_t*>(dy_t->ptr) : nullptr, part,
                     static_cast<int>(M), static_cast<int>(N), static_cast<int>(K), scale);
  VDSL_TRY(check_launch("gemm_bf16_bpk_mse"));
  return launch_mse_finish(part, n_part, static_cast<float*>(loss->ptr), 1.0 / static_cast<double>(n), q->stream);
}

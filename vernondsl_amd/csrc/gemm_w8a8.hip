// Op class 5: int8 W8A8 GEMM with fused dequant (+ ReLU), and per-row activation quantisation,
// on gfx950 MFMA.
//
// No reference code (north-star op class).  Arithmetic shared with the CPU oracle, bit for bit:
//   quantise: s = max|x_row| / 127 (f32), q = clamp(rint(x / s), -127, 127), q = 0 when s = 0;
//   GEMM:     acc = sum_k xq[m][k] * w[n][k] in int32 (exact: |acc| <= K * 127 * 127 < 2^31
//             for K < 133,000), y = relu?((float(acc) * xs[m]) * ws[n]), RNE to bf16.
//
// The main loop is gemm_mfma.h's, shared byte for byte with the bf16 GEMM: the
// v_mfma_i32_32x32x32_i8 fragment is 16 int8 per lane (A[row = l%32][k = 16*(l/32) .. +15]) and
// the accumulator layout is the f32 one.  This file adds the dequant epilogue and the split-K path.
//
// Narrow outputs (too few tiles to fill 256 CUs, e.g. the 1024-wide last layer at batch 512)
// split K across blocks: each block adds its int32 partial tile into a zeroed int32 workspace
// with atomics - integer addition is exact and order-independent, so the result is still
// deterministic - and a second kernel applies the dequant epilogue.

#include "gemm_bpk.h"
#include "gemm_dma.h"
#include "gemm_mfma.h"

namespace vdsl {
namespace {

// Tile configurations (block M x N, K bytes per stage, wave grid); K bytes = K int8 elements.
using I0 = GemmConfig<MfmaI8, 128, 128, 128, 2, 2>;
using I1 = GemmConfig<MfmaI8, 256, 128, 128, 2, 2>;
using I2 = GemmConfig<MfmaI8, 128, 256, 128, 2, 2>;
using I3 = GemmConfig<MfmaI8, 64, 64, 128, 2, 2>;   // wave tile 32x32: small outputs
using I4 = GemmConfig<MfmaI8, 256, 256, 64, 4, 2>;  // 8 waves, wave tile 64x128
using I5 = GemmConfig<MfmaI8, 256, 128, 128, 4, 2>;
using I6 = GemmConfig<MfmaI8, 128, 128, 256, 2, 2>;
using I7 = GemmConfig<MfmaI8, 128, 64, 128, 2, 2>;   // wave tile 64x32: twice the blocks of 128x128
using I8 = GemmConfig<MfmaI8, 64, 128, 128, 2, 2>;   // wave tile 32x64
using I9 = GemmConfig<MfmaI8, 128, 128, 64, 2, 2>;   // 64 K bytes per stage: 3 blocks per CU fit in LDS
using I10 = GemmConfig<MfmaI8, 256, 128, 64, 2, 2>;  // wave tile 128x64, 2 blocks per CU
using I11 = GemmConfig<MfmaI8, 128, 256, 64, 2, 2>;  // wave tile 64x128, 2 blocks per CU
using I12 = GemmConfig<MfmaI8, 256, 256, 64, 2, 4>;  // 8 waves, wave tile 128x64
using I13 = GemmConfig<MfmaI8, 256, 128, 64, 4, 2>;  // 8 waves, wave tile 64x64, 2 blocks per CU
// Direct-to-LDS loop (gemm_dma.h), configurations 14..: <BM, BN, WGM, WGN, LDS stages>
using Di14 = DmaConfig<MfmaI8, 128, 256, 2, 4, 4>;  // 8 waves of 64x64
using Di15 = DmaConfig<MfmaI8, 256, 256, 2, 4, 3>;  // 8 waves of 128x64
using Di16 = DmaConfig<MfmaI8, 64, 128, 2, 2, 4>;   // 4 waves of 32x64, two blocks per CU
using Di17 = DmaConfig<MfmaI8, 128, 128, 2, 2, 4>;  // 4 waves of 64x64, 2 blocks per CU
using Di18 = DmaConfig<MfmaI8, 128, 128, 2, 4, 4>;  // 8 waves of 64x32
using Di19 = DmaConfig<MfmaI8, 128, 64, 2, 2, 4>;   // 4 waves of 64x32
// 128-byte stages (one barrier per 128 int8 of K); need K % 128 == 0
using Di20 = DmaConfig<MfmaI8, 128, 128, 2, 4, 4, 128>;  // 8 waves of 64x32
using Di21 = DmaConfig<MfmaI8, 128, 128, 2, 2, 4, 128>;  // 4 waves of 64x64
using Di22 = DmaConfig<MfmaI8, 64, 128, 2, 2, 4, 128>;   // 4 waves of 32x64
constexpr int kNumConfigs = 23;
constexpr int kFirstDma = 14, kFirstDma128 = 20;

__device__ __forceinline__ void store_y(void* y, int out_dtype, size_t o, float v) {
  if (out_dtype == VDSL_F32) static_cast<float*>(y)[o] = v;
  else static_cast<uint16_t*>(y)[o] = f32_to_bf16(v);
}

__device__ __forceinline__ float dequant(int32_t acc, float xs, float ws, int relu) {
  float v = static_cast<float>(acc) * xs;
  v = v * ws;
  if (relu && !(v > 0.0f)) v = 0.0f;
  return v;
}

// SPLIT: block (x, z) covers K range [z*k_per, (z+1)*k_per) and adds its int32 tile into ws_acc.
template <class Cfg, bool SPLIT, bool EDGE>
__global__ __launch_bounds__(Cfg::NT, Cfg::MIN_BLOCKS) void gemm_w8a8_nt(const int8_t* __restrict__ A, const int8_t* __restrict__ B,
                                                        const float* __restrict__ xs, const float* __restrict__ wsc,
                                                        void* __restrict__ y, int out_dtype, int relu,
                                                        int32_t* __restrict__ acc_out, int32_t* __restrict__ ws_acc, int M,
                                                        int N, int K, int k_per) {
  __shared__ __attribute__((aligned(16))) char smem[Cfg::LDS_BYTES];
  const int tiles_m = (M + Cfg::BM - 1) / Cfg::BM, tiles_n = (N + Cfg::BN - 1) / Cfg::BN;
  int tm, tn;
  tile_coords(xcd_remap(blockIdx.x, gridDim.x), tiles_m, tiles_n, tm, tn);
  const int m0 = tm * Cfg::BM, n0 = tn * Cfg::BN;
  const int k_begin = SPLIT ? blockIdx.y * k_per : 0;
  const int k_end = SPLIT ? min(K, k_begin + k_per) : K;
  i32x16 acc[Cfg::FM][Cfg::FN];
  gemm_mainloop<MfmaI8, Cfg, EDGE>(reinterpret_cast<const char*>(A), reinterpret_cast<const char*>(B), M, N, K, k_begin, k_end,
                             m0, n0, smem, acc);
#pragma unroll
  for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
    for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = acc_row<Cfg>(m0, i, r), col = acc_col<Cfg>(n0, j);
        if (row < M && col < N) {
          const size_t o = static_cast<size_t>(row) * N + col;
          const int32_t a = acc[i][j][r];
          if (SPLIT) {
            atomicAdd(ws_acc + o, a);
          } else {
            if (acc_out) acc_out[o] = a;
            store_y(y, out_dtype, o, dequant(a, xs[row], wsc[col], relu));
          }
        }
      }
}

// Direct-to-LDS variant (gemm_dma.h); same epilogue and split-K contract as gemm_w8a8_nt.
template <class Cfg, bool SPLIT>
__global__ __launch_bounds__(Cfg::NT, Cfg::MIN_BLOCKS) void gemm_w8a8_dma(
    const int8_t* __restrict__ A, const int8_t* __restrict__ B, const float* __restrict__ xs, const float* __restrict__ wsc,
    void* __restrict__ y, int out_dtype, int relu, int32_t* __restrict__ acc_out, int32_t* __restrict__ ws_acc, int M, int N,
    int K, int k_per) {
  __shared__ __attribute__((aligned(1024))) char smem[Cfg::LDS_BYTES];
  const int tiles_m = (M + Cfg::BM - 1) / Cfg::BM, tiles_n = (N + Cfg::BN - 1) / Cfg::BN;
  int tm, tn;
  tile_coords(xcd_remap(blockIdx.x, gridDim.x), tiles_m, tiles_n, tm, tn);
  const int m0 = tm * Cfg::BM, n0 = tn * Cfg::BN;
  const int k_begin = SPLIT ? static_cast<int>(blockIdx.y) * k_per : 0;
  const int k_end = SPLIT ? (K < k_begin + k_per ? K : k_begin + k_per) : K;
  i32x16 acc[Cfg::FM][Cfg::FN];
  dma_mainloop<MfmaI8, Cfg>(reinterpret_cast<const char*>(A), reinterpret_cast<const char*>(B), M, N, K, k_begin, k_end, m0,
                            n0, smem, acc);
#pragma unroll
  for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
    for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = acc_row<Cfg>(m0, i, r), col = acc_col<Cfg>(n0, j);
        if (row < M && col < N) {
          const size_t o = static_cast<size_t>(row) * N + col;
          const int32_t a = acc[i][j][r];
          if (SPLIT) {
            atomicAdd(ws_acc + o, a);
          } else {
            if (acc_out) acc_out[o] = a;
            store_y(y, out_dtype, o, dequant(a, xs[row], wsc[col], relu));
          }
        }
      }
}

__global__ __launch_bounds__(256) void w8a8_epilogue(const int32_t* __restrict__ ws_acc, const float* __restrict__ xs,
                                                     const float* __restrict__ wsc, void* __restrict__ y, int out_dtype,
                                                     int relu, int32_t* __restrict__ acc_out, int M, int N) {
  const int64_t n = static_cast<int64_t>(M) * N;
  for (int64_t o = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; o < n; o += static_cast<int64_t>(gridDim.x) * 256) {
    const int row = static_cast<int>(o / N), col = static_cast<int>(o % N);
    const int32_t a = ws_acc[o];
    if (acc_out) acc_out[o] = a;
    store_y(y, out_dtype, static_cast<size_t>(o), dequant(a, xs[row], wsc[col], relu));
  }
}

// One 256-lane block per row; 16-byte vectors (PV elements) per lane; pass 1 finds max|x| (lane
// max, wave butterfly, 4-wave combine in LDS), pass 2 re-reads the row (from L2) and quantises.
template <int DT>
__global__ __launch_bounds__(256) void quantize_rows_vec(const void* __restrict__ x, int8_t* __restrict__ q,
                                                         float* __restrict__ scale, int64_t cols) {
  constexpr int PV = DT == VDSL_F32 ? 4 : 8;
  __shared__ float wmax[4];
  const int64_t row = blockIdx.x;
  const int64_t nvec = cols / PV;
  const uint4* src = reinterpret_cast<const uint4*>(static_cast<const char*>(x) + row * cols * (DT == VDSL_F32 ? 4 : 2));
  auto unpack = [](const uint4& v, float (&o)[PV]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    if (DT == VDSL_F32) {
#pragma unroll
      for (int k = 0; k < 4; ++k) o[k] = __uint_as_float(w[k]);
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        o[2 * k] = __uint_as_float(w[k] << 16);
        o[2 * k + 1] = __uint_as_float(w[k] & 0xFFFF0000u);
      }
    }
  };
  float amax = 0.0f;
  for (int64_t v = threadIdx.x; v < nvec; v += 256) {
    float e[PV];
    unpack(src[v], e);
#pragma unroll
    for (int k = 0; k < PV; ++k) amax = fmaxf(amax, fabsf(e[k]));
  }
  amax = wave_max(amax);
  if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  const float s = amax / 127.0f;
  if (threadIdx.x == 0) scale[row] = s;
  int8_t* dst = q + row * cols;
  for (int64_t v = threadIdx.x; v < nvec; v += 256) {
    float e[PV];
    unpack(src[v], e);
    uint32_t packed[PV / 4];
#pragma unroll
    for (int w = 0; w < PV / 4; ++w) packed[w] = 0;
#pragma unroll
    for (int k = 0; k < PV; ++k) {
      int iv = 0;
      if (s > 0.0f) {
        float t = rintf(e[k] / s);
        t = fminf(fmaxf(t, -127.0f), 127.0f);
        iv = static_cast<int>(t);
      }
      packed[k / 4] |= (static_cast<uint32_t>(iv) & 0xFFu) << (8 * (k % 4));
    }
    if (PV == 4) *reinterpret_cast<uint32_t*>(dst + v * PV) = packed[0];
    else *reinterpret_cast<uint2*>(dst + v * PV) = make_uint2(packed[0], packed[PV / 4 - 1]);
  }
}

// Rows of exactly NV 16-byte vectors per lane (BT lanes, one block per row): the row is read once
// and held in registers across the block max, so it is never fetched twice.  With few rows (512
// in config 5) the kernel is one load-reduce-store chain per block: 1024 lanes of one vector each
// (bf16 [512][8192]: NV = 1) shorten it against 256 lanes of four (config-5 step ~1 us faster).
template <int DT, int NV, int BT>
__global__ __launch_bounds__(BT) void quantize_rows_resident(const void* __restrict__ x, int8_t* __restrict__ q,
                                                              float* __restrict__ scale) {
  constexpr int PV = DT == VDSL_F32 ? 4 : 8;
  constexpr int64_t COLS = static_cast<int64_t>(NV) * BT * PV;
  __shared__ float wmax[BT / 64];
  const int64_t row = blockIdx.x;
  const u32x4* src = reinterpret_cast<const u32x4*>(static_cast<const char*>(x) + row * COLS * (DT == VDSL_F32 ? 4 : 2));
  u32x4 v[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) v[k] = __builtin_nontemporal_load(src + threadIdx.x + BT * k);
  auto elem = [&](int k, int e) -> float {
    const uint32_t w = v[k][DT == VDSL_F32 ? e : e >> 1];
    if (DT == VDSL_F32) return __uint_as_float(w);
    return __uint_as_float((e & 1) ? (w & 0xFFFF0000u) : (w << 16));
  };
  float amax = 0.0f;
#pragma unroll
  for (int k = 0; k < NV; ++k)
#pragma unroll
    for (int e = 0; e < PV; ++e) amax = fmaxf(amax, fabsf(elem(k, e)));
  amax = wave_max(amax);
  if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = wmax[0];
#pragma unroll
  for (int w = 1; w < BT / 64; ++w) amax = fmaxf(amax, wmax[w]);
  const float s = amax / 127.0f;
  if (threadIdx.x == 0) scale[row] = s;
  int8_t* dst = q + row * COLS;
  // rint(x / s) without a division per element: q = x * rcp(s) lies within 2.7e-5 of x / s (|x / s|
  // <= 127, rcp within 1 ulp, one rounding of the product), and fl(x / s) within 3.8e-6 (half an
  // ulp at 127), so both round to the same integer unless x / s is within 3.1e-5 of a half-integer.
  // A lane with a quotient within 1.2e-4 of one (or a row whose s is outside [2^-120, 2^120], where
  // the reciprocal may flush or lose accuracy) takes the IEEE division instead: the same bits as
  // rintf(x / s) throughout.
  const float rs = __builtin_amdgcn_rcpf(s);
  const bool fast = s >= 0x1p-120f && s <= 0x1p120f;
  float tq[NV][PV];
  bool near = !fast;
#pragma unroll
  for (int k = 0; k < NV; ++k)
#pragma unroll
    for (int e = 0; e < PV; ++e) {
      const float qv = elem(k, e) * rs;
      tq[k][e] = rintf(qv);
      near |= fabsf(fabsf(qv - tq[k][e]) - 0.5f) < 0x1p-13f;
    }
  if (near) {
#pragma unroll
    for (int k = 0; k < NV; ++k)
#pragma unroll
      for (int e = 0; e < PV; ++e) tq[k][e] = rintf(elem(k, e) / s);
  }
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    uint32_t packed[PV / 4];
#pragma unroll
    for (int w = 0; w < PV / 4; ++w) packed[w] = 0;
#pragma unroll
    for (int e = 0; e < PV; ++e) {
      int iv = 0;
      if (s > 0.0f) iv = static_cast<int>(fminf(fmaxf(tq[k][e], -127.0f), 127.0f));
      packed[e / 4] |= (static_cast<uint32_t>(iv) & 0xFFu) << (8 * (e % 4));
    }
    const int64_t vi = threadIdx.x + BT * k;
    if (PV == 4) *reinterpret_cast<uint32_t*>(dst + vi * PV) = packed[0];
    else *reinterpret_cast<uint2*>(dst + vi * PV) = make_uint2(packed[0], packed[PV / 4 - 1]);
  }
}

// Any width: one wave per row, element at a time, same arithmetic.
template <int DT>
__global__ __launch_bounds__(256) void quantize_rows_kernel(const void* __restrict__ x, int8_t* __restrict__ q,
                                                            float* __restrict__ scale, int64_t rows, int64_t cols) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = row * cols;
  auto ld = [&](int64_t c) -> float {
    if (DT == VDSL_F32) return static_cast<const float*>(x)[base + c];
    return bf16_to_f32(static_cast<const uint16_t*>(x)[base + c]);
  };
  float amax = 0.0f;
  for (int64_t c = lane; c < cols; c += 64) amax = fmaxf(amax, fabsf(ld(c)));
  amax = wave_max(amax);
  const float s = amax / 127.0f;
  if (lane == 0) scale[row] = s;
  for (int64_t c = lane; c < cols; c += 64) {
    int v = 0;
    if (s > 0.0f) {
      float t = rintf(ld(c) / s);
      t = fminf(fmaxf(t, -127.0f), 127.0f);
      v = static_cast<int>(t);
    }
    q[base + c] = static_cast<int8_t>(v);
  }
}

int64_t tiles_for(int bm, int bn, int64_t M, int64_t N) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); }

// Configuration for a shape.  The direct-to-LDS loop (14..) runs when K is a multiple of its
// 64-byte stage (128-byte stages, 20..: K % 128 == 0).  Measured on MI355X with random int8
// (config-5 shapes, clocks warm): 128x128 blocks of 8 waves when they give every CU a block
// (512x8192x8192: 1438-1460 TOP/s with 128-byte stages, 1424-1426 with 64-byte ones, 1366 with 4
// waves), else 64x128 blocks with split-K (512x1024x8192: 460, the same with 128-byte stages).
// Other K use the register-staged loop, where 128x64 tiles measured fastest.
int choose_config(int64_t M, int64_t N, int64_t K) {
  const bool dma = K % 64 == 0 && K > 0, dma128 = K % 128 == 0 && K > 0;
  const int o = gemm_config_override();
  if (o >= 0 && o < kNumConfigs && (o < kFirstDma || (o < kFirstDma128 ? dma : dma128))) return o;
  if (!dma) return 7;
  if (((M + 127) / 128) * ((N + 127) / 128) >= 256) return dma128 ? 20 : 18;
  return 16;
}

void config_tile(int c, int& bm, int& bn) {
  static const int t[kNumConfigs][2] = {{128, 128}, {256, 128}, {128, 256}, {64, 64}, {256, 256}, {256, 128}, {128, 128},
                                          {128, 64},  {64, 128},  {128, 128}, {256, 128}, {128, 256}, {256, 256}, {256, 128},
                                          {128, 256}, {256, 256}, {64, 128},  {128, 128}, {128, 128}, {128, 64},
                                          {128, 128}, {128, 128}, {64, 128}};
  bm = t[c][0];
  bn = t[c][1];
}

// K splits for outputs with fewer tiles than the 256 CUs (the split-K path).
int split_of(int64_t M, int64_t N, int64_t K) {
  int bm, bn;
  config_tile(choose_config(M, N, K), bm, bn);
  const int64_t tiles = tiles_for(bm, bn, M, N);
  if (tiles >= 256 || K < 256) return 1;
  int64_t s = 256 / tiles;
  const int64_t kt = (K + 127) / 128;
  if (s > kt) s = kt;
  return static_cast<int>(s < 1 ? 1 : s);
}

template <class Cfg>
int launch_cfg(const int8_t* a, const int8_t* b, const float* xs, const float* wsc, void* y, int out_dtype, int relu,
               int32_t* ao, int32_t* wacc, int m, int n, int k, int split, hipStream_t s) {
  const int64_t tiles = tiles_for(Cfg::BM, Cfg::BN, m, n);
  if (split == 1) {
    if (gemm_needs_edge<Cfg>(m, n, k))
      hipLaunchKernelGGL((gemm_w8a8_nt<Cfg, false, true>), dim3(static_cast<unsigned>(tiles), 1), dim3(Cfg::NT), 0, s, a, b, xs,
                         wsc, y, out_dtype, relu, ao, nullptr, m, n, k, k);
    else
      hipLaunchKernelGGL((gemm_w8a8_nt<Cfg, false, false>), dim3(static_cast<unsigned>(tiles), 1), dim3(Cfg::NT), 0, s, a, b, xs,
                         wsc, y, out_dtype, relu, ao, nullptr, m, n, k, k);
    return check_launch("gemm_w8a8_nt");
  }
  // k_per: a multiple of the K stage so every split starts on a stage boundary
  const int kt = (k + Cfg::BKB - 1) / Cfg::BKB;
  const int k_per = ((kt + split - 1) / split) * Cfg::BKB;
  const int nsplit = (k + k_per - 1) / k_per;
  // the last split may be shorter than k_per: it takes the edge path
  hipLaunchKernelGGL((gemm_w8a8_nt<Cfg, true, true>), dim3(static_cast<unsigned>(tiles), static_cast<unsigned>(nsplit)), dim3(Cfg::NT),
                     0, s, a, b, xs, wsc, y, out_dtype, relu, ao, wacc, m, n, k, k_per);
  return check_launch("gemm_w8a8_nt<split>");
}

template <class Cfg>
int launch_dma(const int8_t* a, const int8_t* b, const float* xs, const float* wsc, void* y, int out_dtype, int relu,
               int32_t* ao, int32_t* wacc, int m, int n, int k, int split, hipStream_t s) {
  const int64_t tiles = tiles_for(Cfg::BM, Cfg::BN, m, n);
  if (split == 1) {
    hipLaunchKernelGGL((gemm_w8a8_dma<Cfg, false>), dim3(static_cast<unsigned>(tiles), 1), dim3(Cfg::NT), 0, s, a, b, xs, wsc, y,
                       out_dtype, relu, ao, nullptr, m, n, k, k);
    return check_launch("gemm_w8a8_dma");
  }
  // k_per: a multiple of the stage (BKB bytes), so with K % BKB == 0 every split is whole stages
  const int kt = (k + Cfg::BKB - 1) / Cfg::BKB;
  const int k_per = ((kt + split - 1) / split) * Cfg::BKB;
  const int nsplit = (k + k_per - 1) / k_per;
  hipLaunchKernelGGL((gemm_w8a8_dma<Cfg, true>), dim3(static_cast<unsigned>(tiles), static_cast<unsigned>(nsplit)), dim3(Cfg::NT),
                     0, s, a, b, xs, wsc, y, out_dtype, relu, ao, wacc, m, n, k, k_per);
  return check_launch("gemm_w8a8_dma<split>");
}

int launch_w8a8(const int8_t* a, const int8_t* b, const float* xs, const float* wsc, void* y, int out_dtype, int relu,
                int32_t* ao, int32_t* wacc, int m, int n, int k, int split, hipStream_t s) {
  switch (choose_config(m, n, k)) {
    case 14: return launch_dma<Di14>(a, b, xs, wsc, y, out_dtype, relu, ao, wacc, m, n, k, split, s);
    case 15: return launch_dma<Di15>(a, b, xs, wsc, y, out_dtype, relu, ao, wacc, m, n, k, split, s);
    case 16: return launch_dma<Di16>(a, b, xs, wsc, y, out_dtype, relu, ao, wacc, m, n, k, split, s);
    case 17: return launch_dma<Di17>(a, b, xs, wsc, y, out_dtype, relu, ao, wacc, m, n, k, split, s);
    case 18: return launch_dma<Di18>(a, b, xs, wsc, y, out_dtype, relu, ao, wacc, m, n, k, split, s);
    case 19: return launch_dma<Di19>(a, b, xs, wsc, y, out_dtype, relu, ao, wacc, m, n, k, split, s);
    case 20: return launch_dma<Di20>(a, b, xs, wsc, y, out_dtype, relu, ao, wacc, m, n, k, split, s);
    case 21: return launch_dma<Di21>(a, b, xs, wsc, y, out_dtype, relu, ao, wacc, m, n, k, split, s);
    case 22: return launch_dma<Di22>(a, b, xs, wsc, y, out_dtype, relu, ao, wacc, m, n, k, split, s);
    case 1: return launch_cfg<I1>(a, b, xs, wsc, y, out_dtype, relu, ao, wacc, m, n, k, split, s);
    case 2: return launch_cfg<I2>(a, b, xs, wsc, y, out_dtype, relu, ao, wacc, m, n, k, split, s);
    case 3: return launch_cfg<I3>(a, b, xs, wsc, y, out_dtype, relu, ao, wacc, m, n, k, split, s);
    case 4: return launch_cfg<I4>(a, b, xs, wsc, y, out_dtype, relu, ao, wacc, m, n, k, split, s);
    case 5: return launch_cfg<I5>(a, b, xs, wsc, y, out_dtype, relu, ao, wacc, m, n, k, split, s);
    case 6: return launch_cfg<I6>(a, b, xs, wsc, y, out_dtype, relu, ao, wacc, m, n, k, split, s);
    case 7: return launch_cfg<I7>(a, b, xs, wsc, y, out_dtype, relu, ao, wacc, m, n, k, split, s);
    case 8: return launch_cfg<I8>(a, b, xs, wsc, y, out_dtype, relu, ao, wacc, m, n, k, split, s);
    case 9: return launch_cfg<I9>(a, b, xs, wsc, y, out_dtype, relu, ao, wacc, m, n, k, split, s);
    case 10: return launch_cfg<I10>(a, b, xs, wsc, y, out_dtype, relu, ao, wacc, m, n, k, split, s);
    case 11: return launch_cfg<I11>(a, b, xs, wsc, y, out_dtype, relu, ao, wacc, m, n, k, split, s);
    case 12: return launch_cfg<I12>(a, b, xs, wsc, y, out_dtype, relu, ao, wacc, m, n, k, split, s);
    case 13: return launch_cfg<I13>(a, b, xs, wsc, y, out_dtype, relu, ao, wacc, m, n, k, split, s);
    default: return launch_cfg<I0>(a, b, xs, wsc, y, out_dtype, relu, ao, wacc, m, n, k, split, s);
  }
}


// ---- packed-weight GEMM (gemm_bpk.h main loop) ------------------------------------------------
// Weights in fragment order (bpk_pack_kernel), activations row-major through LDS.  A launch of
// tiles * S blocks: block (tile, z) covers K bytes [z K/S, (z+1) K/S) of its tile.  With S == 1 the
// block runs the dequant epilogue itself; with S > 1 it stores its int32 partial tile to the
// workspace in accumulator order (each wave's fragments as 16-byte runs: 1 KiB per store
// instruction) and w8a8_bpk_reduce adds the S partials and runs the epilogue.  Integer addition
// is exact and order-free, so the result is the unsplit one, bit for bit.
//
// Measured on MI355X, 512x8192x8192, clocks warm.  The MFMA rate depends on the operand bits:
// the main loop alone ran 41.1 us on random full-range int8, 38.3 us on bytes 0..127 and 33.4 us
// on bytes 0..15.  On bytes 0..127: 64 x 256 blocks, no split, 35.8 us; 128 x 256 blocks split in
// two with the partials exchanged inside the kernel (counters, last block adds) 46.3 us; 128 x
// 256 unsplit on 128 CUs 47.0 us.  The 1024-wide last layer (32 tiles of 64 x 256): the last
// block of each tile adding S - 1 partials alone took 18.5 us (S = 4) to 28.6 us on full-range
// data; the separate reduce spreads that work over the whole GPU.
using P0 = BpkConfig<MfmaI8, 4, 2, 4, 3>;  // 128 x 256 blocks, 4 waves of 128 x 64
using P1 = BpkConfig<MfmaI8, 2, 2, 4, 3>;  // 64 x 256 blocks, 4 waves of 64 x 64
using P2 = BpkConfig<MfmaI8, 2, 2, 4, 7>;  // P1 with loads 7 stages ahead (stages % 8 == 0)
// 128 x 128 blocks, 4 waves of 128 x 32: the same outputs per block as 64 x 256 with 32 KiB of
// operands per 128-byte stage instead of 40 (A 16 + B 16 against 8 + 32), for twice the LDS
// reads (every wave reads all 128 rows of A).  512x8192x8192 with weights rotating through three
// matrices, same box: 36.6 us against 40.3 us for P2 (4-layer step 162 against 173 us).
using P3 = BpkConfig<MfmaI8, 4, 1, 4, 3>;
// 64 x 128 blocks, 4 waves of 64 x 32: a quarter of P0's outputs per block, for narrow outputs
// split along K over every CU.
using P4 = BpkConfig<MfmaI8, 2, 1, 4, 3>;
// 32 x 64 blocks of 2 waves of 32 x 32 and 32 x 128 blocks of 4 waves: narrow outputs without a
// K split (512 x 1024: 256 and 128 tiles), each block streaming its operands over the whole K.
using P5 = BpkConfig<MfmaI8, 1, 1, 2, 3>;
using P6 = BpkConfig<MfmaI8, 1, 1, 4, 3>;

// Whole-tile bf16 epilogue through LDS: each wave writes its dequantised fragments as bf16 into a
// [BM][EPI_ROW] staging tile (2-byte writes; the row stride 528 = 512 + 16 puts the rows r and
// r + 4 that one store instruction covers into disjoint 16-bank windows), then every thread
// stores 16-byte runs of whole rows.
constexpr int kEpiRow = 528;
template <class Cfg>
constexpr int bpk_smem_bytes() {
  return Cfg::LDS_BYTES > Cfg::BM * kEpiRow ? Cfg::LDS_BYTES : Cfg::BM * kEpiRow;
}

template <class Cfg>
__global__ __launch_bounds__(Cfg::NT, 1) void gemm_w8a8_bpk(const int8_t* __restrict__ A, const int8_t* __restrict__ Bp,
                                                         const float* __restrict__ xs, const float* __restrict__ wsc,
                                                         void* __restrict__ y, int out_dtype, int relu,
                                                         int32_t* __restrict__ acc_out, char* __restrict__ part, int M,
                                                         int N, int K, int S) {
  constexpr int FM = Cfg::FM, FN = Cfg::FN, W = Cfg::W;
  constexpr size_t WAVE_BYTES = static_cast<size_t>(FM) * FN * 4096;
  // The only __shared__ variable (see gemm_bpk.h); after the main loop it stages the epilogue.
  __shared__ __attribute__((aligned(1024))) char smem[bpk_smem_bytes<Cfg>()];
  const int tiles_m = (M + Cfg::BM - 1) / Cfg::BM;
  const int w = xcd_remap(blockIdx.x, gridDim.x);
  const int tile = w / S, z = w % S;
  const int m0 = (tile % tiles_m) * Cfg::BM, n0 = (tile / tiles_m) * Cfg::BN;
  const int kper = K / S;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  i32x16 acc[FM][FN];
  bpk_mainloop<MfmaI8, Cfg>(reinterpret_cast<const char*>(A), reinterpret_cast<const char*>(Bp), M, N / 32, K, z * kper,
                            (z + 1) * kper, m0, n0, smem, acc);
  if (S > 1) {
    char* const mine = part + ((static_cast<size_t>(tile) * S + z) * W + wave) * WAVE_BYTES + lane * 16;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const i32x4 v = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
          *reinterpret_cast<i32x4*>(mine + ((i * FN + j) * 4 + q) * 1024) = v;
        }
    return;
  }
  if (out_dtype == VDSL_BF16 && !acc_out && m0 + Cfg::BM <= M && n0 + Cfg::BN <= N) {
    __syncthreads();  // every wave is past its last read of the main loop's LDS
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int c = Cfg::WTN * wave + 32 * j + (lane & 31);
        const float wcol = wsc[n0 + c];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int rr = 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          *reinterpret_cast<uint16_t*>(smem + rr * kEpiRow + 2 * c) = f32_to_bf16(dequant(acc[i][j][r], xs[m0 + rr], wcol, relu));
        }
      }
    __syncthreads();
    constexpr int CHUNKS = Cfg::BM * (Cfg::BN * 2 / 16);  // 16-byte runs of the tile
    char* const yb = static_cast<char*>(y);
#pragma unroll
    for (int k = 0; k < CHUNKS / Cfg::NT; ++k) {
      const int idx = threadIdx.x + Cfg::NT * k;
      const int rr = idx / (Cfg::BN * 2 / 16), ch = idx % (Cfg::BN * 2 / 16);
      const u32x4 v = *reinterpret_cast<const u32x4*>(smem + rr * kEpiRow + ch * 16);
      *reinterpret_cast<u32x4*>(yb + (static_cast<size_t>(m0 + rr) * N + n0) * 2 + ch * 16) = v;
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int col = n0 + Cfg::WTN * wave + 32 * j + (lane & 31);
      if (col >= N) continue;
      const float wcol = wsc[col];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row < M) {
          const size_t o = static_cast<size_t>(row) * N + col;
          const int32_t a = acc[i][j][r];
          if (acc_out) acc_out[o] = a;
          store_y(y, out_dtype, o, dequant(a, xs[row], wcol, relu));
        }
      }
    }
}

// Sum of the S partial tiles of a split launch, then the dequant epilogue.  Thread u takes 16-byte
// chunk u of one partial (tile, wave, fragment, quarter q, lane): accumulators 4q .. 4q+3 of
// that lane, i.e. rows 8q + 4 (lane / 32) + 0..3 of column lane % 32 of the fragment.
template <class Cfg>
__global__ __launch_bounds__(256) void w8a8_bpk_reduce(const char* __restrict__ part, const float* __restrict__ xs,
                                                       const float* __restrict__ wsc, void* __restrict__ y, int out_dtype,
                                                       int relu, int32_t* __restrict__ acc_out, int M, int N, int S,
                                                       int64_t tiles) {
  constexpr int FM = Cfg::FM, FN = Cfg::FN, W = Cfg::W;
  constexpr int64_t WAVE_CHUNKS = static_cast<int64_t>(FM) * FN * 4 * 64;  // 16-byte chunks per wave
  const int tiles_m = (M + Cfg::BM - 1) / Cfg::BM;
  const int64_t total = tiles * W * WAVE_CHUNKS;
  for (int64_t u = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; u < total; u += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t tw = u / WAVE_CHUNKS;  // tile * W + wave
    const int rem = static_cast<int>(u % WAVE_CHUNKS);
    const int tile = static_cast<int>(tw / W), wave = static_cast<int>(tw % W);
    const int lane = rem & 63, fq = rem >> 6;  // fq = (i * FN + j) * 4 + q
    const int q = fq & 3, f = fq >> 2, i = f / FN, j = f % FN;
    const char* p = part + (static_cast<size_t>(tile) * S * W + wave) * (WAVE_CHUNKS * 16) + static_cast<size_t>(rem) * 16;
    i32x4 sum = *reinterpret_cast<const i32x4*>(p);
    for (int z = 1; z < S; ++z) sum += *reinterpret_cast<const i32x4*>(p + static_cast<size_t>(z) * W * WAVE_CHUNKS * 16);
    const int m0 = (tile % tiles_m) * Cfg::BM, n0 = (tile / tiles_m) * Cfg::BN;
    const int col = n0 + Cfg::WTN * wave + 32 * j + (lane & 31);
    if (col >= N) continue;
    const float wcol = wsc[col];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = m0 + 32 * i + 8 * q + 4 * (lane >> 5) + e;
      if (row < M) {
        const size_t o = static_cast<size_t>(row) * N + col;
        if (acc_out) acc_out[o] = sum[e];
        store_y(y, out_dtype, o, dequant(sum[e], xs[row], wcol, relu));
      }
    }
  }
}

// Launch plan of the packed GEMM for a shape: configuration, K split S, tiles.  128 x 256 tiles
// when they alone give every CU a block; else 128 x 128 when those do; else, with M >= 128, 64 x
// 128 tiles with K split into about 256 blocks; else 64 x 256, with K split only when those are
// fewer than 256, into about 256 blocks; each split part is a whole number of loop trips (NR
// stages of 128 bytes).
struct BpkPlan {
  int cfg, split;  // cfg: 0 = P0, 1 = P1, 2 = P2, 3 = P3, 4 = P4, 5 = P5, 6 = P6
  int64_t tiles;
};
std::atomic<int> g_bpk_plan{-1};  // debug override: cfg * 256 + split, or -1

template <class Cfg>
int64_t bpk_tiles(int64_t M, int64_t N) {
  return ((M + Cfg::BM - 1) / Cfg::BM) * ((N + Cfg::BN - 1) / Cfg::BN);
}

BpkPlan bpk_plan(int64_t M, int64_t N, int64_t K) {
  BpkPlan p;
  const int o = g_bpk_plan.load(std::memory_order_relaxed);
  if (o >= 0) {  // a forced plan, when its stages split evenly: K % (128 * NR * split) == 0
    const int cfg = o >> 8, split = o & 255;
    const int nr = cfg == 2 ? P2::NR : P0::NR;
    if (cfg >= 0 && cfg <= 6 && split >= 1 && K % (static_cast<int64_t>(128) * nr * split) == 0) {
      p.cfg = cfg;
      p.split = split;
      p.tiles = cfg == 0   ? bpk_tiles<P0>(M, N)
                : cfg == 3 ? bpk_tiles<P3>(M, N)
                : cfg == 4 ? bpk_tiles<P4>(M, N)
                : cfg == 5 ? bpk_tiles<P5>(M, N)
                : cfg == 6 ? bpk_tiles<P6>(M, N)
                           : bpk_tiles<P1>(M, N);
      return p;
    }
  }
  const int64_t t0 = ((M + P0::BM - 1) / P0::BM) * ((N + P0::BN - 1) / P0::BN);
  const int64_t t3 = ((M + P3::BM - 1) / P3::BM) * ((N + P3::BN - 1) / P3::BN);
  if (t0 < 256 && t3 >= 256) {
    p.cfg = 3;
    p.tiles = t3;
    p.split = 1;
    return p;
  }
  const int64_t trips = K / (128 * P0::NR);
  if (t0 < 256 && M >= 128) {
    // Narrow outputs: 64 x 128 tiles with K split into about 256 blocks.  512x1024x8192 with
    // weights rotating through 16 copies, same box: 64 x 128 split 4 (256 blocks) 13.8 us, split 2
    // 14.8, split 8 16.6, unsplit 19.1; 128 x 128 split 4 (128 blocks, the plan before) 14.4-14.8,
    // split 2 18.5, split 8 16.5-16.9; 64 x 256 split 4 15.0.  A larger split costs more in the
    // partials' round trip through memory and the reduce than its extra blocks gain.
    const int64_t t4 = bpk_tiles<P4>(M, N);
    p.cfg = 4;
    p.tiles = t4;
    int64_t s = t4 >= 256 ? 1 : 256 / t4;
    if (s > trips) s = trips;
    while (s > 1 && trips % s) --s;
    p.split = static_cast<int>(s < 1 ? 1 : s);
    return p;
  }
  p.cfg = t0 >= 256 ? 0 : 1;
  p.tiles = p.cfg == 0 ? t0 : ((M + P1::BM - 1) / P1::BM) * ((N + P1::BN - 1) / P1::BN);
  int64_t s = p.tiles >= 256 ? 1 : (256 + p.tiles - 1) / p.tiles;
  if (s > trips) s = trips;
  while (s > 1 && trips % s) --s;
  p.split = static_cast<int>(s < 1 ? 1 : s);
  if (p.cfg == 1 && (K / p.split / 128) % P2::NR == 0) p.cfg = 2;
  return p;
}
size_t bpk_workspace_bytes(const BpkPlan& p) {
  if (p.split == 1) return 0;
  const size_t tile_bytes = p.cfg == 0   ? static_cast<size_t>(P0::BM) * P0::BN * 4
                            : p.cfg == 3 ? static_cast<size_t>(P3::BM) * P3::BN * 4
                            : p.cfg == 4 ? static_cast<size_t>(P4::BM) * P4::BN * 4
                            : p.cfg == 5 ? static_cast<size_t>(P5::BM) * P5::BN * 4
                            : p.cfg == 6 ? static_cast<size_t>(P6::BM) * P6::BN * 4
                                         : static_cast<size_t>(P1::BM) * P1::BN * 4;
  return static_cast<size_t>(p.tiles) * p.split * tile_bytes;
}

template <class Cfg>
int launch_bpk(const BpkPlan& p, const int8_t* a, const int8_t* b, const float* xs, const float* wsc, void* y, int out_dtype,
               int relu, int32_t* ao, char* part, int m, int n, int k, hipStream_t s) {
  hipLaunchKernelGGL(gemm_w8a8_bpk<Cfg>, dim3(static_cast<unsigned>(p.tiles * p.split)), dim3(Cfg::NT), 0, s, a, b, xs, wsc, y,
                     out_dtype, relu, p.split > 1 ? nullptr : ao, part, m, n, k, p.split);
  VDSL_TRY(check_launch("gemm_w8a8_bpk"));
  if (p.split == 1) return VDSL_OK;
  const int64_t chunks = p.tiles * Cfg::W * Cfg::FM * Cfg::FN * 4 * 64;
  int64_t blocks = (chunks + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(w8a8_bpk_reduce<Cfg>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, part, xs, wsc, y, out_dtype,
                     relu, ao, m, n, p.split, p.tiles);
  return check_launch("w8a8_bpk_reduce");
}

}  // namespace
}  // namespace vdsl

using namespace vdsl;

extern "C" int vdsl_op_quantize_rows_i8(vdsl_queue q, int64_t rows, int64_t cols, int32_t x_dtype, vdsl_buffer x,
                                        vdsl_buffer qx, vdsl_buffer scale) {
  VDSL_TRY(enter_queue(q));
  if (rows < 0 || cols < 0) return fail(VDSL_ERR_INVALID_ARG, "negative shape");
  if (x_dtype != VDSL_F32 && x_dtype != VDSL_BF16) return fail(VDSL_ERR_UNSUPPORTED, "quantize input must be f32 or bf16");
  VDSL_TRY(check_buffer(q, x, nbytes(rows, cols, dtype_size(x_dtype)), "x", false));
  VDSL_TRY(check_buffer(q, qx, nbytes(rows, cols), "qx", true));
  VDSL_TRY(check_buffer(q, scale, nbytes(rows, 4), "scale", true));
  if (rows == 0) return VDSL_OK;
  const int pv = x_dtype == VDSL_F32 ? 4 : 8;
  if (rows <= 0x7fffffff && (cols == 256 * pv * 4 || cols == 256 * pv * 8)) {  // register-resident rows
    const dim3 g(static_cast<unsigned>(rows));
    auto* qp = static_cast<int8_t*>(qx->ptr);
    auto* sp = static_cast<float*>(scale->ptr);
    const bool nv4 = cols == 256 * pv * 4;
    const dim3 b4(1024);
    if (x_dtype == VDSL_F32) {
      if (nv4) hipLaunchKernelGGL((quantize_rows_resident<VDSL_F32, 1, 1024>), g, b4, 0, q->stream, x->ptr, qp, sp);
      else hipLaunchKernelGGL((quantize_rows_resident<VDSL_F32, 2, 1024>), g, b4, 0, q->stream, x->ptr, qp, sp);
    } else {
      if (nv4) hipLaunchKernelGGL((quantize_rows_resident<VDSL_BF16, 1, 1024>), g, b4, 0, q->stream, x->ptr, qp, sp);
      else hipLaunchKernelGGL((quantize_rows_resident<VDSL_BF16, 2, 1024>), g, b4, 0, q->stream, x->ptr, qp, sp);
    }
    return check_launch("quantize_rows_resident");
  }
  if (cols % pv == 0 && rows <= 0x7fffffff) {  // rows of whole 16-byte vectors (hipMalloc bases are aligned)
    if (x_dtype == VDSL_F32)
      hipLaunchKernelGGL(quantize_rows_vec<VDSL_F32>, dim3(static_cast<unsigned>(rows)), dim3(256), 0, q->stream, x->ptr,
                         static_cast<int8_t*>(qx->ptr), static_cast<float*>(scale->ptr), cols);
    else
      hipLaunchKernelGGL(quantize_rows_vec<VDSL_BF16>, dim3(static_cast<unsigned>(rows)), dim3(256), 0, q->stream, x->ptr,
                         static_cast<int8_t*>(qx->ptr), static_cast<float*>(scale->ptr), cols);
    return check_launch("quantize_rows_vec");
  }
  const int64_t blocks = (rows + 3) / 4;
  if (x_dtype == VDSL_F32)
    hipLaunchKernelGGL(quantize_rows_kernel<VDSL_F32>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, q->stream, x->ptr,
                       static_cast<int8_t*>(qx->ptr), static_cast<float*>(scale->ptr), rows, cols);
  else
    hipLaunchKernelGGL(quantize_rows_kernel<VDSL_BF16>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, q->stream, x->ptr,
                       static_cast<int8_t*>(qx->ptr), static_cast<float*>(scale->ptr), rows, cols);
  return check_launch("quantize_rows_kernel");
}

extern "C" int vdsl_gemm_w8a8_workspace_bytes(int64_t M, int64_t N, int64_t K, size_t* bytes) {
  if (!bytes) return fail(VDSL_ERR_INVALID_ARG, "bytes is null");
  if (M < 0 || N < 0 || K < 0) return fail(VDSL_ERR_INVALID_ARG, "negative GEMM extent");
  const size_t ws = split_of(M, N, K) > 1 ? nbytes(M, N, 4) : 0;
  if (ws == kSizeOverflow) return fail(VDSL_ERR_SHAPE, "GEMM workspace size overflows (extents too large)");
  *bytes = ws;
  return VDSL_OK;
}

extern "C" int vdsl_op_gemm_w8a8(vdsl_queue q, int64_t M, int64_t N, int64_t K, vdsl_buffer xq, vdsl_buffer x_scale,
                                 vdsl_buffer w, vdsl_buffer w_scale, vdsl_buffer y, int32_t out_dtype, int32_t relu,
                                 vdsl_buffer acc_out, vdsl_buffer workspace) {
  VDSL_TRY(enter_queue(q));
  if (M < 0 || N < 0 || K < 0) return fail(VDSL_ERR_INVALID_ARG, "negative GEMM extent");
  if (M > 0x7fffffff || N > 0x7fffffff || K > 133000) return fail(VDSL_ERR_UNSUPPORTED, "extent too large (K <= 133000 keeps int32 exact)");
  if (out_dtype != VDSL_F32 && out_dtype != VDSL_BF16) return fail(VDSL_ERR_UNSUPPORTED, "y must be f32 or bf16");
  if (K % 16) return fail(VDSL_ERR_UNSUPPORTED, "K must be a multiple of 16 (16-byte int8 rows)");
  VDSL_TRY(check_buffer(q, xq, nbytes(M, K), "xq", false));
  VDSL_TRY(check_buffer(q, x_scale, nbytes(M, 4), "x_scale", false));
  VDSL_TRY(check_buffer(q, w, nbytes(N, K), "w", false));
  VDSL_TRY(check_buffer(q, w_scale, nbytes(N, 4), "w_scale", false));
  VDSL_TRY(check_buffer(q, y, nbytes(M, N, dtype_size(out_dtype)), "y", true));
  if (acc_out) VDSL_TRY(check_buffer(q, acc_out, nbytes(M, N, 4), "acc_out", true));
  const int split = split_of(M, N, K);
  if (split > 1) VDSL_TRY(check_buffer(q, workspace, nbytes(M, N, 4), "workspace", true));
  if (M == 0 || N == 0) return VDSL_OK;
  const int m = static_cast<int>(M), n = static_cast<int>(N), k = static_cast<int>(K);
  int32_t* ao = acc_out ? static_cast<int32_t*>(acc_out->ptr) : nullptr;
  const auto* a = static_cast<const int8_t*>(xq->ptr);
  const auto* b = static_cast<const int8_t*>(w->ptr);
  const auto* xs = static_cast<const float*>(x_scale->ptr);
  const auto* wsc = static_cast<const float*>(w_scale->ptr);
  if (split == 1) return launch_w8a8(a, b, xs, wsc, y->ptr, out_dtype, relu, ao, nullptr, m, n, k, 1, q->stream);
  VDSL_TRY(vdsl_buffer_fill_u32(q, workspace, 0, static_cast<size_t>(M) * N * 4, 0u));
  int32_t* wacc = static_cast<int32_t*>(workspace->ptr);
  VDSL_TRY(launch_w8a8(a, b, xs, wsc, y->ptr, out_dtype, relu, ao, wacc, m, n, k, split, q->stream));
  int64_t blocks = (static_cast<int64_t>(M) * N + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(w8a8_epilogue, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, q->stream, wacc, xs, wsc, y->ptr,
                     out_dtype, relu, ao, m, n);
  return check_launch("w8a8_epilogue");
}


extern "C" int vdsl_op_pack_w8a8_weights(vdsl_queue q, int64_t N, int64_t K, vdsl_buffer w, vdsl_buffer wp) {
  VDSL_TRY(enter_queue(q));
  if (N < 0 || K < 0) return fail(VDSL_ERR_INVALID_ARG, "negative weight extent");
  if (N % 32 || K % 32) return fail(VDSL_ERR_UNSUPPORTED, "packed weights need N % 32 == 0 and K % 32 == 0");
  const size_t n = nbytes(N, K);
  VDSL_TRY(check_buffer(q, w, n, "w", false));
  VDSL_TRY(check_buffer(q, wp, n, "wp", true));
  if (w == wp) return fail(VDSL_ERR_INVALID_ARG, "w and wp must be different buffers");
  if (n == 0) return VDSL_OK;
  const int64_t chunks = static_cast<int64_t>(n / 16);
  int64_t blocks = (chunks + 255) / 256;
  if (blocks > 16384) blocks = 16384;
  hipLaunchKernelGGL(bpk_pack_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, q->stream,
                     static_cast<const char*>(w->ptr), static_cast<char*>(wp->ptr), N / 32, K / 32, K);
  return check_launch("bpk_pack_kernel");
}

static int packed_shape_ok(int64_t M, int64_t N, int64_t K) {
  if (M < 0 || N < 0 || K < 0) return fail(VDSL_ERR_INVALID_ARG, "negative GEMM extent");
  if (M > 0x7fffffff || N > 0x7fffffff || K > 133000)
    return fail(VDSL_ERR_UNSUPPORTED, "extent too large (K <= 133000 keeps int32 exact)");
  if (N % 32) return fail(VDSL_ERR_UNSUPPORTED, "packed GEMM needs N % 32 == 0");
  if (K % (128 * P0::NR)) return fail(VDSL_ERR_UNSUPPORTED, "packed GEMM needs K % 512 == 0");
  return VDSL_OK;
}

extern "C" int vdsl_gemm_w8a8_packed_workspace_bytes(int64_t M, int64_t N, int64_t K, size_t* bytes) {
  if (!bytes) return fail(VDSL_ERR_INVALID_ARG, "bytes is null");
  VDSL_TRY(packed_shape_ok(M, N, K));
  *bytes = (M == 0 || N == 0 || K == 0) ? 0 : bpk_workspace_bytes(bpk_plan(M, N, K));
  return VDSL_OK;
}

// Operand checks shared by the packed entry points (everything but the split-K scratch).
static int packed_operands_ok(vdsl_queue q, int64_t M, int64_t N, int64_t K, vdsl_buffer xq, vdsl_buffer x_scale,
                              vdsl_buffer wp, vdsl_buffer w_scale, vdsl_buffer y, int32_t out_dtype, vdsl_buffer acc_out) {
  VDSL_TRY(packed_shape_ok(M, N, K));
  if (out_dtype != VDSL_F32 && out_dtype != VDSL_BF16) return fail(VDSL_ERR_UNSUPPORTED, "y must be f32 or bf16");
  VDSL_TRY(check_buffer(q, xq, nbytes(M, K), "xq", false));
  VDSL_TRY(check_buffer(q, x_scale, nbytes(M, 4), "x_scale", false));
  VDSL_TRY(check_buffer(q, wp, nbytes(N, K), "wp", false));
  VDSL_TRY(check_buffer(q, w_scale, nbytes(N, 4), "w_scale", false));
  VDSL_TRY(check_buffer(q, y, nbytes(M, N, dtype_size(out_dtype)), "y", true));
  if (acc_out) VDSL_TRY(check_buffer(q, acc_out, nbytes(M, N, 4), "acc_out", true));
  if (M != 0 && N != 0 && K == 0) return fail(VDSL_ERR_UNSUPPORTED, "packed GEMM needs K > 0");
  return VDSL_OK;
}

// Launches the plan's GEMM (and, split, its reduce) with the split-K partials at `part`.
static int packed_launch(vdsl_queue q, const BpkPlan& p, int64_t M, int64_t N, int64_t K, vdsl_buffer xq,
                         vdsl_buffer x_scale, vdsl_buffer wp, vdsl_buffer w_scale, vdsl_buffer y, int32_t out_dtype,
                         int32_t relu, vdsl_buffer acc_out, char* part) {
  int32_t* ao = acc_out ? static_cast<int32_t*>(acc_out->ptr) : nullptr;
  const auto* a = static_cast<const int8_t*>(xq->ptr);
  const auto* b = static_cast<const int8_t*>(wp->ptr);
  const auto* xs = static_cast<const float*>(x_scale->ptr);
  const auto* wsc = static_cast<const float*>(w_scale->ptr);
  const int m = static_cast<int>(M), n = static_cast<int>(N), k = static_cast<int>(K);
  if (p.cfg == 0) return launch_bpk<P0>(p, a, b, xs, wsc, y->ptr, out_dtype, relu, ao, part, m, n, k, q->stream);
  if (p.cfg == 3) return launch_bpk<P3>(p, a, b, xs, wsc, y->ptr, out_dtype, relu, ao, part, m, n, k, q->stream);
  if (p.cfg == 4) return launch_bpk<P4>(p, a, b, xs, wsc, y->ptr, out_dtype, relu, ao, part, m, n, k, q->stream);
  if (p.cfg == 5) return launch_bpk<P5>(p, a, b, xs, wsc, y->ptr, out_dtype, relu, ao, part, m, n, k, q->stream);
  if (p.cfg == 6) return launch_bpk<P6>(p, a, b, xs, wsc, y->ptr, out_dtype, relu, ao, part, m, n, k, q->stream);
  if (p.cfg == 2) return launch_bpk<P2>(p, a, b, xs, wsc, y->ptr, out_dtype, relu, ao, part, m, n, k, q->stream);
  return launch_bpk<P1>(p, a, b, xs, wsc, y->ptr, out_dtype, relu, ao, part, m, n, k, q->stream);
}

extern "C" int vdsl_debug_w8a8_packed_plan(int32_t cfg, int32_t split) {
  if (cfg < 0) {
    g_bpk_plan.store(-1, std::memory_order_relaxed);
    return VDSL_OK;
  }
  if (cfg > 6 || split < 1 || split > 255) return fail(VDSL_ERR_INVALID_ARG, "plan: cfg 0..6, split 1..255");
  g_bpk_plan.store(cfg * 256 + split, std::memory_order_relaxed);
  return VDSL_OK;
}

extern "C" int vdsl_op_gemm_w8a8_packed(vdsl_queue q, int64_t M, int64_t N, int64_t K, vdsl_buffer xq, vdsl_buffer x_scale,
                                        vdsl_buffer wp, vdsl_buffer w_scale, vdsl_buffer y, int32_t out_dtype, int32_t relu,
                                        vdsl_buffer acc_out, vdsl_buffer workspace) {
  VDSL_TRY(enter_queue(q));
  VDSL_TRY(packed_operands_ok(q, M, N, K, xq, x_scale, wp, w_scale, y, out_dtype, acc_out));
  if (M == 0 || N == 0) return VDSL_OK;
  const BpkPlan p = bpk_plan(M, N, K);
  const size_t wsb = bpk_workspace_bytes(p);
  if (wsb) VDSL_TRY(check_buffer(q, workspace, wsb, "workspace", true));
  return packed_launch(q, p, M, N, K, xq, x_scale, wp, w_scale, y, out_dtype, relu, acc_out,
                       wsb ? static_cast<char*>(workspace->ptr) : nullptr);
}

// ---- allocation-free entry point ------------------------------------------------------------------
// vdsl_op_gemm_w8a8_packed_noalloc keeps the split-K partials in `scratch`, a file-scope device
// array, so it calls no allocator.  Every GPU that loads the library holds its own copy until the
// process ends.  In host code the name `scratch` is a host-side stand-in, not a device address:
// the array's address on a device comes from hipGetSymbolAddress, called once per device with that
// device current (w8a8_noalloc_setup, from vdsl_device_open), kept in g_scratch_addr, and only that
// address is handed to kernels.  Nothing in the array needs to start at zero: a split launch
// writes every partial it later reads.  Calls that overlap in time on one GPU (two queues) share
// the array and race.
namespace vdsl {
static __device__ __align__(256) char scratch[VDSL_W8A8_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kScratchDevices = 64;
std::atomic<char*> g_scratch_addr[kScratchDevices];

// The device address of `scratch` on device `ordinal`, which must be the current device.
int scratch_address(int ordinal, char** out) {
  if (ordinal < 0 || ordinal >= kScratchDevices)
    return fail(VDSL_ERR_UNSUPPORTED, "allocation-free GEMM: device ordinal beyond the library's table");
  char* p = g_scratch_addr[ordinal].load(std::memory_order_acquire);
  if (!p) {
    void* addr = nullptr;
    VDSL_TRY(check_hip(hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)"));
    if (!addr) return fail(VDSL_ERR_DEVICE, "hipGetSymbolAddress(scratch) returned a null address");
    p = static_cast<char*>(addr);
    g_scratch_addr[ordinal].store(p, std::memory_order_release);
  }
  *out = p;
  return VDSL_OK;
}
}  // namespace

void w8a8_noalloc_setup(int ordinal) {
  char* p = nullptr;
  // A failure is not fatal to the device: the entry point tries again and reports the HIP error.
  (void)scratch_address(ordinal, &p);
}
}  // namespace vdsl

extern "C" int vdsl_op_gemm_w8a8_packed_noalloc(vdsl_queue q, int64_t M, int64_t N, int64_t K, vdsl_buffer xq,
                                                vdsl_buffer x_scale, vdsl_buffer wp, vdsl_buffer w_scale, vdsl_buffer y,
                                                int32_t out_dtype, int32_t relu, vdsl_buffer acc_out) {
  VDSL_TRY(enter_queue(q));
  VDSL_TRY(packed_operands_ok(q, M, N, K, xq, x_scale, wp, w_scale, y, out_dtype, acc_out));
  if (M == 0 || N == 0) return VDSL_OK;
  const BpkPlan p = bpk_plan(M, N, K);
  const size_t wsb = bpk_workspace_bytes(p);
  if (wsb > VDSL_W8A8_NOALLOC_SCRATCH_BYTES)
    return fail(VDSL_ERR_UNSUPPORTED, "allocation-free GEMM: this shape needs " + std::to_string(wsb) +
                                          " bytes of split-K scratch, the library's array holds " +
                                          std::to_string(VDSL_W8A8_NOALLOC_SCRATCH_BYTES) +
                                          "; use vdsl_op_gemm_w8a8_packed with a workspace");
  char* part = nullptr;
  if (wsb) VDSL_TRY(scratch_address(q->dev->ordinal, &part));
  return packed_launch(q, p, M, N, K, xq, x_scale, wp, w_scale, y, out_dtype, relu, acc_out, part);
}

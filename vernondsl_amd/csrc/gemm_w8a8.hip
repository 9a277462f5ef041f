// Op class 5: int8 W8A8 GEMM with fused dequant (+ ReLU), and per-row activation quantisation,
// on gfx950 MFMA.
//
// No reference code (north-star op class).  Arithmetic shared with the CPU oracle, bit for bit:
//   quantise: s = max|x_row| / 127 (f32), q = clamp(rint(x / s), -127, 127), q = 0 when s = 0;
//   GEMM:     acc = sum_k xq[m][k] * w[n][k] in int32 (exact: |acc| <= K * 127 * 127 < 2^31
//             for K < 133,000), y = relu?((float(acc) * xs[m]) * ws[n]), RNE to bf16.
//
// Tiling mirrors the bf16 kernel byte for byte: a 256-lane block computes a 128x128 tile; K
// advances 128 int8 (128 bytes) per LDS tile, so A/B tiles are [128][128+16] bytes.  Each wave
// owns 64x64 as 2x2 v_mfma_i32_32x32x32_i8 accumulators; lane l supplies A[row = l%32][k =
// 16*(l/32) .. +15] (one 16-byte fragment) and B likewise; accumulator element r of lane l is
// C[8*(r/4) + 4*(l/32) + r%4][l%32].
//
// Narrow outputs (too few tiles to fill 256 CUs, e.g. the 1024-wide last layer at batch 512)
// split K across blocks: each block adds its int32 partial tile into a zeroed int32 workspace
// with atomics - integer addition is exact and order-independent, so the result is still
// deterministic - and a second kernel applies the dequant epilogue.

#include "common.h"

namespace vdsl {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BKB = 128, LDB = BKB + 16;  // BKB: K bytes per tile

__device__ __forceinline__ int remap_xcd(int b, int nb) {
  if (nb % 8) return b;
  return (b % 8) * (nb / 8) + (b / 8);
}

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

// SPLIT: this block covers K range [kz*k_per, (kz+1)*k_per) and adds into ws_acc.
template <bool SPLIT>
__global__ __launch_bounds__(256, 2) void gemm_w8a8_nt(const int8_t* __restrict__ A, const int8_t* __restrict__ B,
                                                       const float* __restrict__ xs, const float* __restrict__ wsc,
                                                       void* __restrict__ y, int out_dtype, int relu,
                                                       int32_t* __restrict__ acc_out, int32_t* __restrict__ ws_acc, int M,
                                                       int N, int K, int k_per) {
  __shared__ __attribute__((aligned(16))) int8_t As[BM * LDB];
  __shared__ __attribute__((aligned(16))) int8_t Bs[BN * LDB];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  const int t = remap_xcd(blockIdx.x, gridDim.x);
  constexpr int G = 8;
  const int group = t / (G * tiles_n);
  const int first_m = group * G;
  const int gsize = min(G, tiles_m - first_m);
  const int in_group = t - group * G * tiles_n;
  const int tile_m = first_m + in_group % gsize;
  const int tile_n = in_group / gsize;
  const int m0 = tile_m * BM, n0 = tile_n * BN;
  const int k_begin = SPLIT ? blockIdx.y * k_per : 0;
  const int k_end = SPLIT ? min(K, k_begin + k_per) : K;

  i32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  uint4 ra[4], rb[4];
  auto load_tiles = [&](int kb) {  // kb: first K index of the tile
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i;
      const int row = c >> 3;
      const int k = kb + (c & 7) * 16;
      const int gm = m0 + row, gn = n0 + row;
      ra[i] = (gm < M && k < k_end) ? *reinterpret_cast<const uint4*>(A + static_cast<size_t>(gm) * K + k) : make_uint4(0, 0, 0, 0);
      rb[i] = (gn < N && k < k_end) ? *reinterpret_cast<const uint4*>(B + static_cast<size_t>(gn) * K + k) : make_uint4(0, 0, 0, 0);
    }
  };
  auto store_tiles = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i;
      const int row = c >> 3;
      const int kc = (c & 7) * 16;
      *reinterpret_cast<uint4*>(&As[row * LDB + kc]) = ra[i];
      *reinterpret_cast<uint4*>(&Bs[row * LDB + kc]) = rb[i];
    }
  };

  const int nk = (k_end - k_begin + BKB - 1) / BKB;
  if (nk > 0) {
    load_tiles(k_begin);
    store_tiles();
  }
  __syncthreads();
  const int frag_row = lane & 31;
  const int frag_k = (lane >> 5) * 16;
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) load_tiles(k_begin + (kt + 1) * BKB);
#pragma unroll
    for (int kk = 0; kk < BKB; kk += 32) {
      i32x4 a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        a[i] = *reinterpret_cast<const i32x4*>(&As[(wm * 64 + i * 32 + frag_row) * LDB + kk + frag_k]);
        b[i] = *reinterpret_cast<const i32x4*>(&Bs[(wn * 64 + i * 32 + frag_row) * LDB + kk + frag_k]);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
    if (kt + 1 < nk) {
      store_tiles();
      __syncthreads();
    }
  }

#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const int col = n0 + wn * 64 + j * 32 + (lane & 31);
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

// One wave per row: pass 1 finds max|x|, pass 2 quantises.
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

int split_of(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  if (tiles >= 128 || K < 2 * BKB) return 1;
  int64_t s = 256 / tiles;
  const int64_t kt = (K + BKB - 1) / BKB;
  if (s > kt) s = kt;
  return static_cast<int>(s < 1 ? 1 : s);
}

}  // namespace
}  // namespace vdsl

using namespace vdsl;

extern "C" int vdsl_op_quantize_rows_i8(vdsl_queue q, int64_t rows, int64_t cols, int32_t x_dtype, vdsl_buffer x,
                                        vdsl_buffer qx, vdsl_buffer scale) {
  VDSL_TRY(enter_queue(q));
  if (rows < 0 || cols < 0) return fail(VDSL_ERR_INVALID_ARG, "negative shape");
  if (x_dtype != VDSL_F32 && x_dtype != VDSL_BF16) return fail(VDSL_ERR_UNSUPPORTED, "quantize input must be f32 or bf16");
  const size_t n = static_cast<size_t>(rows) * static_cast<size_t>(cols);
  VDSL_TRY(check_buffer(q, x, n * dtype_size(x_dtype), "x", false));
  VDSL_TRY(check_buffer(q, qx, n, "qx", true));
  VDSL_TRY(check_buffer(q, scale, static_cast<size_t>(rows) * 4, "scale", true));
  if (rows == 0) return VDSL_OK;
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
  *bytes = split_of(M, N, K) > 1 ? static_cast<size_t>(M) * static_cast<size_t>(N) * 4 : 0;
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
  VDSL_TRY(check_buffer(q, xq, static_cast<size_t>(M) * K, "xq", false));
  VDSL_TRY(check_buffer(q, x_scale, static_cast<size_t>(M) * 4, "x_scale", false));
  VDSL_TRY(check_buffer(q, w, static_cast<size_t>(N) * K, "w", false));
  VDSL_TRY(check_buffer(q, w_scale, static_cast<size_t>(N) * 4, "w_scale", false));
  VDSL_TRY(check_buffer(q, y, static_cast<size_t>(M) * N * dtype_size(out_dtype), "y", true));
  if (acc_out) VDSL_TRY(check_buffer(q, acc_out, static_cast<size_t>(M) * N * 4, "acc_out", true));
  const int split = split_of(M, N, K);
  if (split > 1) VDSL_TRY(check_buffer(q, workspace, static_cast<size_t>(M) * N * 4, "workspace", true));
  if (M == 0 || N == 0) return VDSL_OK;
  const int m = static_cast<int>(M), n = static_cast<int>(N), k = static_cast<int>(K);
  const int64_t tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  int32_t* ao = acc_out ? static_cast<int32_t*>(acc_out->ptr) : nullptr;
  const auto* a = static_cast<const int8_t*>(xq->ptr);
  const auto* b = static_cast<const int8_t*>(w->ptr);
  const auto* xs = static_cast<const float*>(x_scale->ptr);
  const auto* wsc = static_cast<const float*>(w_scale->ptr);
  if (split == 1) {
    hipLaunchKernelGGL(gemm_w8a8_nt<false>, dim3(static_cast<unsigned>(tiles), 1), dim3(256), 0, q->stream, a, b, xs, wsc,
                       y->ptr, out_dtype, relu, ao, nullptr, m, n, k, k);
    return check_launch("gemm_w8a8_nt");
  }
  // k_per: a multiple of the K tile so every split starts on a tile boundary
  const int kt = (k + BKB - 1) / BKB;
  const int k_per = ((kt + split - 1) / split) * BKB;
  const int nsplit = (k + k_per - 1) / k_per;
  VDSL_TRY(vdsl_buffer_fill_u32(q, workspace, 0, static_cast<size_t>(M) * N * 4, 0u));
  int32_t* wacc = static_cast<int32_t*>(workspace->ptr);
  hipLaunchKernelGGL(gemm_w8a8_nt<true>, dim3(static_cast<unsigned>(tiles), static_cast<unsigned>(nsplit)), dim3(256), 0,
                     q->stream, a, b, xs, wsc, y->ptr, out_dtype, relu, ao, wacc, m, n, k, k_per);
  VDSL_TRY(check_launch("gemm_w8a8_nt<split>"));
  int64_t blocks = (static_cast<int64_t>(M) * N + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(w8a8_epilogue, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, q->stream, wacc, xs, wsc, y->ptr,
                     out_dtype, relu, ao, m, n);
  return check_launch("w8a8_epilogue");
}

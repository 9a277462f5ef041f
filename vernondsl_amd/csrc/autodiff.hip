// Autodiff building blocks of the execution graph on gfx950: GELU and ReLU backward, MSE
// forward+backward, and the elementwise sum (residual adds, gradients of a value read twice).
//
// No reference code (north-star op class: "compiler-generated backward").  Both kernels are
// elementwise over [rows][cols] and also emit the transposed gradient, because the weight
// gradients dW = G^T X need G K-contiguous along the batch: a 256-lane block reads a 64x64 tile
// (coalesced), writes the row-major result directly and the transposed result through an LDS
// tile (coalesced along the transposed rows), so the transpose costs no extra HBM pass.
//
// MSE: loss = mean((y - t)^2) as a deterministic two-stage reduction - each tile writes one f64
// partial sum, then one block adds the partials in tile order - and dy = (y - t) * (2 / n) in
// f32, rounded to bf16.

#include <algorithm>

#include "common.h"

namespace vdsl {
namespace {


// Vector forms of the two kernels below, for rows % 8 == 0 and cols % 4 == 0 (every base is a
// whole hipMalloc buffer, 256-byte aligned): a 64x64 tile per 256-lane block, each lane loads two
// units of 2 rows x 4 columns with 16-byte loads (all loads issued before any arithmetic), stores
// the row-major result as 8-byte runs and hands the transposed result to LDS as row pairs, which
// go out as 16-byte runs of the transposed rows (store_pair_tile_transposed).

// Unit k of this lane: source rows r0 + 2q, r0 + 2q + 1, columns c0 + 4t .. c0 + 4t + 3.
__device__ __forceinline__ void unit_of(int k, int& q, int& t) {
  const int u = static_cast<int>(threadIdx.x) + 256 * k;
  q = u >> 4;
  t = u & 15;
}

// Packs the bf16 results of one unit: row-major words (2 per row) and the 4 column pairs.
__device__ __forceinline__ void pack_unit(const float (&v)[2][4], uint32_t (&row)[2][2], uint32_t (&pair)[4]) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    row[i][0] = pack_bf16x2(v[i][0], v[i][1]);
    row[i][1] = pack_bf16x2(v[i][2], v[i][3]);
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    pair[2 * h] = (row[0][h] & 0xFFFFu) | (row[1][h] << 16);
    pair[2 * h + 1] = (row[0][h] >> 16) | (row[1][h] & 0xFFFF0000u);
  }
}

// The activation backward of y = act(pre): dL/dpre = dL/dy * act'(pre).  ACT 0: GELU' (the erfc
// form of gelu_grad_f); ACT 1: ReLU', dL/dy where pre > 0, else +0 (pre <= 0 and NaN: 0, as
// torch's threshold backward; a select, so an infinite dL/dy at pre <= 0 gives 0, not NaN).
enum { kActGelu = 0, kActRelu = 1 };
template <int ACT>
__device__ __forceinline__ float act_bwd(float g, float pre) {
  if constexpr (ACT == kActGelu) return g * gelu_grad_f(pre);
  else return pre > 0.0f ? g : 0.0f;
}

template <int ACT>
__global__ __launch_bounds__(256) void act_bwd_vec(const float* __restrict__ dh, const float* __restrict__ pre,
                                                   uint16_t* __restrict__ da, uint16_t* __restrict__ da_t,
                                                   int64_t rows, int64_t cols) {
  __shared__ __align__(16) uint32_t tile[kPairTileWords];
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 64, c0 = static_cast<int64_t>(blockIdx.x) * 64;
  f32x4 g[2][2], x[2][2];
  bool ok[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    int q, t;
    unit_of(k, q, t);
    ok[k] = r0 + 2 * q < rows && c0 + 4 * t < cols;
    const int64_t o = (r0 + 2 * q) * cols + c0 + 4 * t;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      if (ok[k]) {
        g[k][i] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(dh + o + i * cols));
        x[k][i] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(pre + o + i * cols));
      }
    }
  }
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    if (!ok[k]) continue;
    int q, t;
    unit_of(k, q, t);
    float v[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) v[i][j] = act_bwd<ACT>(g[k][i][j], x[k][i][j]);
    uint32_t row[2][2], pair[4];
    pack_unit(v, row, pair);
    const int64_t o = (r0 + 2 * q) * cols + c0 + 4 * t;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      uint2 w;
      w.x = row[i][0];
      w.y = row[i][1];
      *reinterpret_cast<uint2*>(da + o + i * cols) = w;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) tile[pair_slot(4 * t + j, q)] = pair[j];
  }
  if (!da_t) return;  // uniform across the block
  __syncthreads();
  store_pair_tile_transposed(tile, da_t, rows, cols, r0, c0);
}

__global__ __launch_bounds__(256) void mse_tile_vec(const float* __restrict__ y, const float* __restrict__ t_in,
                                                    uint16_t* __restrict__ dy, uint16_t* __restrict__ dy_t,
                                                    double* __restrict__ partials, int64_t rows, int64_t cols,
                                                    float scale) {
  __shared__ __align__(16) uint32_t tile[kPairTileWords];
  __shared__ double wsum[4];
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 64, c0 = static_cast<int64_t>(blockIdx.x) * 64;
  f32x4 a[2][2], b[2][2];
  bool ok[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    int q, t;
    unit_of(k, q, t);
    ok[k] = r0 + 2 * q < rows && c0 + 4 * t < cols;
    const int64_t o = (r0 + 2 * q) * cols + c0 + 4 * t;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      if (ok[k]) {
        a[k][i] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(y + o + i * cols));
        b[k][i] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(t_in + o + i * cols));
      }
    }
  }
  double s = 0.0;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    if (!ok[k]) continue;
    int q, t;
    unit_of(k, q, t);
    float v[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float d = a[k][i][j] - b[k][i][j];
        s += static_cast<double>(d) * static_cast<double>(d);
        v[i][j] = d * scale;
      }
    uint32_t row[2][2], pair[4];
    pack_unit(v, row, pair);
    const int64_t o = (r0 + 2 * q) * cols + c0 + 4 * t;
    if (dy) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        uint2 w;
        w.x = row[i][0];
        w.y = row[i][1];
        *reinterpret_cast<uint2*>(dy + o + i * cols) = w;
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) tile[pair_slot(4 * t + j, q)] = pair[j];
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m, 64);
  if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0)
    partials[static_cast<int64_t>(blockIdx.y) * gridDim.x + blockIdx.x] = ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
  if (!dy_t) return;
  store_pair_tile_transposed(tile, dy_t, rows, cols, r0, c0);
}

template <int ACT>
__global__ __launch_bounds__(256) void act_bwd_kernel(const float* __restrict__ dh, const float* __restrict__ pre,
                                                      uint16_t* __restrict__ da, uint16_t* __restrict__ da_t,
                                                      int64_t rows, int64_t cols) {
  __shared__ uint16_t tile[64][66];
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 64, c0 = static_cast<int64_t>(blockIdx.x) * 64;
#pragma unroll 4
  for (int p = 0; p < 16; ++p) {
    const int64_t r = r0 + ty + 4 * p, c = c0 + tx;
    if (r < rows && c < cols) {
      const int64_t o = r * cols + c;
      const uint16_t h = f32_to_bf16(act_bwd<ACT>(dh[o], pre[o]));
      da[o] = h;
      tile[ty + 4 * p][tx] = h;
    }
  }
  if (!da_t) return;  // uniform across the block
  __syncthreads();
#pragma unroll 4
  for (int p = 0; p < 16; ++p) {
    const int64_t c = c0 + ty + 4 * p, r = r0 + tx;
    if (r < rows && c < cols) da_t[c * rows + r] = tile[tx][ty + 4 * p];
  }
}

__global__ __launch_bounds__(256) void mse_tile_kernel(const float* __restrict__ y, const float* __restrict__ t,
                                                       uint16_t* __restrict__ dy, uint16_t* __restrict__ dy_t,
                                                       double* __restrict__ partials, int64_t rows, int64_t cols,
                                                       float scale) {
  __shared__ uint16_t tile[64][66];
  __shared__ double wsum[4];
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 64, c0 = static_cast<int64_t>(blockIdx.x) * 64;
  double s = 0.0;
#pragma unroll 4
  for (int p = 0; p < 16; ++p) {
    const int64_t r = r0 + ty + 4 * p, c = c0 + tx;
    if (r < rows && c < cols) {
      const int64_t o = r * cols + c;
      const float d = y[o] - t[o];
      s += static_cast<double>(d) * static_cast<double>(d);
      const uint16_t h = f32_to_bf16(d * scale);
      if (dy) dy[o] = h;
      tile[ty + 4 * p][tx] = h;
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m, 64);
  if (tx == 0) wsum[ty] = s;
  __syncthreads();
  if (threadIdx.x == 0)
    partials[static_cast<int64_t>(blockIdx.y) * gridDim.x + blockIdx.x] = ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
  if (!dy_t) return;
#pragma unroll 4
  for (int p = 0; p < 16; ++p) {
    const int64_t c = c0 + ty + 4 * p, r = r0 + tx;
    if (r < rows && c < cols) dy_t[c * rows + r] = tile[tx][ty + 4 * p];
  }
}

// One block: lane-strided f64 sums of the partials, then a fixed-order combine.
__global__ __launch_bounds__(256) void mse_finish_kernel(const double* __restrict__ partials, int64_t n_partials,
                                                         float* __restrict__ loss, double inv_n) {
  __shared__ double wsum[4];
  double s = 0.0;
  for (int64_t i = threadIdx.x; i < n_partials; i += 256) s += partials[i];
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m, 64);
  if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) loss[0] = static_cast<float>((((wsum[0] + wsum[1]) + wsum[2]) + wsum[3]) * inv_n);
}

int64_t tiles_of(int64_t rows, int64_t cols) { return ((rows + 63) / 64) * ((cols + 63) / 64); }

}  // namespace

int launch_mse_finish(const double* partials, int64_t n_partials, float* loss, double inv_n, hipStream_t s) {
  hipLaunchKernelGGL(mse_finish_kernel, dim3(1), dim3(256), 0, s, partials, n_partials, loss, inv_n);
  return check_launch("mse_finish_kernel");
}

}  // namespace vdsl

using namespace vdsl;

namespace vdsl {
namespace {
template <int ACT>
int launch_act_bwd(vdsl_queue q, int64_t rows, int64_t cols, vdsl_buffer dh, vdsl_buffer pre, vdsl_buffer da,
                   vdsl_buffer da_t, const char* name) {
  VDSL_TRY(enter_queue(q));
  if (rows < 0 || cols < 0) return fail(VDSL_ERR_INVALID_ARG, "negative shape");
  VDSL_TRY(check_buffer(q, dh, nbytes(rows, cols, 4), "dh", false));
  VDSL_TRY(check_buffer(q, pre, nbytes(rows, cols, 4), "pre", false));
  VDSL_TRY(check_buffer(q, da, nbytes(rows, cols, 2), "da", true));
  if (da_t) VDSL_TRY(check_buffer(q, da_t, nbytes(rows, cols, 2), "da_t", true));
  const size_t n = static_cast<size_t>(rows) * static_cast<size_t>(cols);  // fits: checked above
  if (n == 0) return VDSL_OK;
  const int64_t gx = (cols + 63) / 64, gy = (rows + 63) / 64;
  if (gy > 65535 || gx > 0x7fffffff) return fail(VDSL_ERR_UNSUPPORTED, std::string(name) + ": tensor too large");
  const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy));
  const float* g = static_cast<const float*>(dh->ptr);
  const float* x = static_cast<const float*>(pre->ptr);
  uint16_t* a = static_cast<uint16_t*>(da->ptr);
  uint16_t* at = da_t ? static_cast<uint16_t*>(da_t->ptr) : nullptr;
  if (rows % 8 == 0 && cols % 4 == 0) {
    hipLaunchKernelGGL(act_bwd_vec<ACT>, grid, dim3(256), 0, q->stream, g, x, a, at, rows, cols);
    return check_launch("act_bwd_vec");
  }
  hipLaunchKernelGGL(act_bwd_kernel<ACT>, grid, dim3(256), 0, q->stream, g, x, a, at, rows, cols);
  return check_launch("act_bwd_kernel");
}
}  // namespace
}  // namespace vdsl

extern "C" int vdsl_op_gelu_bwd(vdsl_queue q, int64_t rows, int64_t cols, vdsl_buffer dh, vdsl_buffer pre, vdsl_buffer da,
                                vdsl_buffer da_t) {
  return launch_act_bwd<kActGelu>(q, rows, cols, dh, pre, da, da_t, "gelu_bwd");
}

extern "C" int vdsl_op_relu_bwd(vdsl_queue q, int64_t rows, int64_t cols, vdsl_buffer dh, vdsl_buffer pre, vdsl_buffer da,
                                vdsl_buffer da_t) {
  return launch_act_bwd<kActRelu>(q, rows, cols, dh, pre, da, da_t, "relu_bwd");
}

extern "C" int64_t vdsl_mse_partials_count(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  return 2 * tiles_of(rows, cols);  // one f64 (two f32 slots) per 64x64 tile
}

namespace vdsl {
namespace {
// Grid-stride elementwise GELU (erfc form, branch-free; the accurate variant, since f32 results
// are held to 1e-5 relative).
template <int XT, int YT>
__global__ __launch_bounds__(256) void gelu_fwd_kernel(const void* __restrict__ x, void* __restrict__ y, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256) {
    const float v = XT == VDSL_F32 ? static_cast<const float*>(x)[i] : bf16_to_f32(static_cast<const uint16_t*>(x)[i]);
    const float g = gelu_f_acc(v);
    if (YT == VDSL_F32) static_cast<float*>(y)[i] = g;
    else static_cast<uint16_t*>(y)[i] = f32_to_bf16(g);
  }
}
}  // namespace
}  // namespace vdsl

extern "C" int vdsl_op_gelu_fwd(vdsl_queue q, int64_t n, int32_t x_dtype, vdsl_buffer x, int32_t y_dtype, vdsl_buffer y) {
  VDSL_TRY(enter_queue(q));
  if (n < 0) return fail(VDSL_ERR_INVALID_ARG, "negative element count");
  const bool ok = (x_dtype == VDSL_F32 || x_dtype == VDSL_BF16) && (y_dtype == VDSL_F32 || y_dtype == VDSL_BF16);
  if (!ok) return fail(VDSL_ERR_UNSUPPORTED, "gelu_fwd supports f32 and bf16");
  VDSL_TRY(check_buffer(q, x, nbytes(n, dtype_size(x_dtype)), "x", false));
  VDSL_TRY(check_buffer(q, y, nbytes(n, dtype_size(y_dtype)), "y", true));
  if (x == y && x_dtype != y_dtype) return fail(VDSL_ERR_INVALID_ARG, "in-place gelu_fwd needs one dtype");
  if (n == 0) return VDSL_OK;
  const int64_t blocks = std::min<int64_t>((n + 255) / 256, 256 * 32);
  const dim3 g(static_cast<unsigned>(blocks)), b(256);
  if (x_dtype == VDSL_F32 && y_dtype == VDSL_F32) hipLaunchKernelGGL((gelu_fwd_kernel<VDSL_F32, VDSL_F32>), g, b, 0, q->stream, x->ptr, y->ptr, n);
  else if (x_dtype == VDSL_F32) hipLaunchKernelGGL((gelu_fwd_kernel<VDSL_F32, VDSL_BF16>), g, b, 0, q->stream, x->ptr, y->ptr, n);
  else if (y_dtype == VDSL_F32) hipLaunchKernelGGL((gelu_fwd_kernel<VDSL_BF16, VDSL_F32>), g, b, 0, q->stream, x->ptr, y->ptr, n);
  else hipLaunchKernelGGL((gelu_fwd_kernel<VDSL_BF16, VDSL_BF16>), g, b, 0, q->stream, x->ptr, y->ptr, n);
  return check_launch("gelu_fwd_kernel");
}

extern "C" int vdsl_op_mse_fwd_bwd(vdsl_queue q, int64_t rows, int64_t cols, vdsl_buffer y, vdsl_buffer t, vdsl_buffer loss,
                                   vdsl_buffer dy, vdsl_buffer dy_t, vdsl_buffer partials) {
  VDSL_TRY(enter_queue(q));
  if (rows <= 0 || cols <= 0) return fail(VDSL_ERR_INVALID_ARG, "MSE needs a non-empty tensor");
  VDSL_TRY(check_buffer(q, y, nbytes(rows, cols, 4), "y", false));
  VDSL_TRY(check_buffer(q, t, nbytes(rows, cols, 4), "t", false));
  VDSL_TRY(check_buffer(q, loss, 4, "loss", true));
  if (dy) VDSL_TRY(check_buffer(q, dy, nbytes(rows, cols, 2), "dy", true));
  if (dy_t) VDSL_TRY(check_buffer(q, dy_t, nbytes(rows, cols, 2), "dy_t", true));
  const size_t n = static_cast<size_t>(rows) * static_cast<size_t>(cols);  // fits: checked above
  const int64_t np = tiles_of(rows, cols);
  VDSL_TRY(check_buffer(q, partials, nbytes(np, 8), "partials", true));
  const int64_t gx = (cols + 63) / 64, gy = (rows + 63) / 64;
  if (gy > 65535 || gx > 0x7fffffff) return fail(VDSL_ERR_UNSUPPORTED, "mse: tensor too large");
  const float scale = 2.0f / static_cast<float>(n);
  double* part = static_cast<double*>(partials->ptr);
  const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy));
  if (rows % 8 == 0 && cols % 4 == 0)
    hipLaunchKernelGGL(mse_tile_vec, grid, dim3(256), 0, q->stream, static_cast<const float*>(y->ptr),
                       static_cast<const float*>(t->ptr), dy ? static_cast<uint16_t*>(dy->ptr) : nullptr,
                       dy_t ? static_cast<uint16_t*>(dy_t->ptr) : nullptr, part, rows, cols, scale);
  else
    hipLaunchKernelGGL(mse_tile_kernel, grid, dim3(256), 0, q->stream,
                       static_cast<const float*>(y->ptr), static_cast<const float*>(t->ptr),
                       dy ? static_cast<uint16_t*>(dy->ptr) : nullptr, dy_t ? static_cast<uint16_t*>(dy_t->ptr) : nullptr, part,
                       rows, cols, scale);
  VDSL_TRY(check_launch("mse_tile_kernel"));
  hipLaunchKernelGGL(mse_finish_kernel, dim3(1), dim3(256), 0, q->stream, part, np, static_cast<float*>(loss->ptr),
                     1.0 / static_cast<double>(n));
  return check_launch("mse_finish_kernel");
}

namespace vdsl {
namespace {
// Four consecutive elements of an F32 or BF16 array, widened to f32 (exact), from one 16- or
// 8-byte load; and their store, rounded once (RNE) to the output dtype.
template <int T>
__device__ __forceinline__ void load4(const void* __restrict__ p, int64_t i, float (&v)[4]) {
  if constexpr (T == VDSL_F32) {
    const f32x4 x = *reinterpret_cast<const f32x4*>(static_cast<const float*>(p) + i);
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = x[j];
  } else {
    const uint2 w = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p) + i);
    v[0] = __uint_as_float(w.x << 16);
    v[1] = __uint_as_float(w.x & 0xFFFF0000u);
    v[2] = __uint_as_float(w.y << 16);
    v[3] = __uint_as_float(w.y & 0xFFFF0000u);
  }
}

template <int T>
__device__ __forceinline__ void store4(void* __restrict__ p, int64_t i, const float (&v)[4]) {
  if constexpr (T == VDSL_F32) {
    const f32x4 x = {v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4*>(static_cast<float*>(p) + i) = x;
  } else {
    uint2 w;
    w.x = pack_bf16x2(v[0], v[1]);
    w.y = pack_bf16x2(v[2], v[3]);
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p) + i) = w;
  }
}

template <int T>
__device__ __forceinline__ float load1(const void* __restrict__ p, int64_t i) {
  if constexpr (T == VDSL_F32) return static_cast<const float*>(p)[i];
  else return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
}

// out = a + b elementwise: one f32 addition per element, rounded once to out's dtype.  VEC (n %
// 4 == 0; every buffer is a whole 256-byte-aligned allocation): four elements per lane and trip.
// A lane reads its elements before it writes them, so out may be a or b (same dtype).
template <int AT, int BT, int OT, bool VEC>
__global__ __launch_bounds__(256) void add_kernel(const void* a, const void* b, void* out, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if constexpr (VEC) {
    for (int64_t u = first; u < n / 4; u += stride) {
      float x[4], y[4], z[4];
      load4<AT>(a, 4 * u, x);
      load4<BT>(b, 4 * u, y);
#pragma unroll
      for (int j = 0; j < 4; ++j) z[j] = x[j] + y[j];
      store4<OT>(out, 4 * u, z);
    }
  } else {
    for (int64_t i = first; i < n; i += stride) {
      const float z = load1<AT>(a, i) + load1<BT>(b, i);
      if constexpr (OT == VDSL_F32) static_cast<float*>(out)[i] = z;
      else static_cast<uint16_t*>(out)[i] = f32_to_bf16(z);
    }
  }
}

typedef void (*AddKernel)(const void*, const void*, void*, int64_t);
template <int AT, int BT, int OT>
AddKernel add_pick(bool vec) {
  return vec ? add_kernel<AT, BT, OT, true> : add_kernel<AT, BT, OT, false>;
}
template <int AT, int BT>
AddKernel add_pick(int ot, bool vec) {
  return ot == VDSL_F32 ? add_pick<AT, BT, VDSL_F32>(vec) : add_pick<AT, BT, VDSL_BF16>(vec);
}
template <int AT>
AddKernel add_pick(int bt, int ot, bool vec) {
  return bt == VDSL_F32 ? add_pick<AT, VDSL_F32>(ot, vec) : add_pick<AT, VDSL_BF16>(ot, vec);
}
}  // namespace
}  // namespace vdsl

extern "C" int vdsl_op_add(vdsl_queue q, int64_t n, int32_t a_dtype, vdsl_buffer a, int32_t b_dtype, vdsl_buffer b,
                           int32_t out_dtype, vdsl_buffer out) {
  VDSL_TRY(enter_queue(q));
  if (n < 0) return fail(VDSL_ERR_INVALID_ARG, "negative element count");
  auto fb = [](int32_t t) { return t == VDSL_F32 || t == VDSL_BF16; };
  if (!fb(a_dtype) || !fb(b_dtype) || !fb(out_dtype)) return fail(VDSL_ERR_UNSUPPORTED, "add supports f32 and bf16");
  VDSL_TRY(check_buffer(q, a, nbytes(n, dtype_size(a_dtype)), "a", false));
  VDSL_TRY(check_buffer(q, b, nbytes(n, dtype_size(b_dtype)), "b", false));
  VDSL_TRY(check_buffer(q, out, nbytes(n, dtype_size(out_dtype)), "out", true));
  if ((out == a && a_dtype != out_dtype) || (out == b && b_dtype != out_dtype))
    return fail(VDSL_ERR_INVALID_ARG, "in-place add needs the output's dtype on the operand it overwrites");
  if (n == 0) return VDSL_OK;
  const bool vec = n % 4 == 0;
  const int64_t units = vec ? n / 4 : n;
  const int64_t blocks = std::min<int64_t>((units + 255) / 256, 256 * 16);
  const AddKernel k = a_dtype == VDSL_F32 ? add_pick<VDSL_F32>(b_dtype, out_dtype, vec)
                                          : add_pick<VDSL_BF16>(b_dtype, out_dtype, vec);
  hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, q->stream, a->ptr, b->ptr, out->ptr, n);
  return check_launch("add_kernel");
}

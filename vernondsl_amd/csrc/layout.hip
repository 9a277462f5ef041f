// Layout ops: 2-D transpose (f32 / bf16) and f32 <-> bf16 conversion, on gfx950.
//
// No reference code.  The GEMMs of op class 4 consume K-contiguous operands; the transpose
// re-lays a K-strided operand, and the execution graph uses it for weight transposes.
//
// Transpose mapping: a 256-lane block moves one 64x64 tile through LDS.  Reads are coalesced
// along the source row, writes along the destination row; the tile's LDS rows are padded by one
// element so the column-wise LDS reads of the write phase fall in different banks.
//
// bf16 with even extents takes a 128x128 tile of 2x2 element blocks instead: a lane loads two
// 4-byte pairs (rows r, r+1 at columns c, c+1), swaps them into the two destination pairs in
// registers, and the 32-bit pairs go through LDS as a 64x64 tile; every global access is then
// 4 bytes per lane (the 2-byte form runs at about a quarter of the copy bandwidth).  With
// extents that are multiples of 8 the same pairing runs on 16-byte loads and stores
// (transpose_bf16_vec).

#include "common.h"

namespace vdsl {

namespace {

template <typename T>
__global__ __launch_bounds__(256) void transpose_kernel(const T* __restrict__ src, T* __restrict__ dst, int64_t rows,
                                                        int64_t cols) {
  __shared__ T tile[64][65];
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 64, c0 = static_cast<int64_t>(blockIdx.x) * 64;
#pragma unroll
  for (int p = 0; p < 16; ++p) {
    const int64_t r = r0 + ty + 4 * p, c = c0 + tx;
    if (r < rows && c < cols) tile[ty + 4 * p][tx] = src[r * cols + c];
  }
  __syncthreads();
#pragma unroll
  for (int p = 0; p < 16; ++p) {
    const int64_t c = c0 + ty + 4 * p, r = r0 + tx;  // dst row c, column r
    if (r < rows && c < cols) dst[c * rows + r] = tile[tx][ty + 4 * p];
  }
}

// bf16, rows and cols even: block (bx, by) covers source rows 128*by.., cols 128*bx...
__global__ __launch_bounds__(256) void transpose_bf16_pairs(const uint32_t* __restrict__ src, uint32_t* __restrict__ dst,
                                                            int64_t rows, int64_t cols) {
  __shared__ uint32_t tile[128][65];  // [dst row within tile][dst column pair]
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 128, c0 = static_cast<int64_t>(blockIdx.x) * 128;
  const int64_t cp = cols / 2, rp = rows / 2;  // pairs per source row, per destination row
#pragma unroll 4
  for (int p = 0; p < 16; ++p) {
    const int q = ty + 4 * p;  // source row pair within the tile
    const int64_t r = r0 + 2 * q, c = c0 + 2 * tx;
    if (r < rows && c < cols) {
      const uint32_t a = src[r * cp + c / 2];        // (x[r][c], x[r][c+1])
      const uint32_t b = src[(r + 1) * cp + c / 2];  // (x[r+1][c], x[r+1][c+1])
      tile[2 * tx][q] = (a & 0xFFFFu) | (b << 16);            // dst row c:   (x[r][c], x[r+1][c])
      tile[2 * tx + 1][q] = (a >> 16) | (b & 0xFFFF0000u);    // dst row c+1: (x[r][c+1], x[r+1][c+1])
    }
  }
  __syncthreads();
#pragma unroll 4
  for (int p = 0; p < 32; ++p) {
    const int row = ty + 4 * p;  // destination row within the tile
    const int64_t c = c0 + row, r = r0 + 2 * tx;
    if (c < cols && r < rows) dst[c * rp + r / 2] = tile[row][tx];
  }
}

// bf16, rows % 8 == 0 and cols % 8 == 0: TPB 64x64 tiles per block; per tile lane u loads source rows
// r0 + 2q, r0 + 2q + 1 (q = u / 8) at columns c0 + 8t .. + 7 (t = u % 8) with two 16-byte loads,
// forms the 8 column pairs in registers and the tile leaves as 16-byte runs of the destination
// rows (store_pair_tile_transposed).
template <int TPB>
__global__ __launch_bounds__(256) void transpose_bf16_vec(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                                                          int64_t rows, int64_t cols) {
  // TPB 64x64 tiles stacked along the source rows per block: every tile's loads are issued before
  // any LDS write, so a thread has 2 TPB 16-byte loads in flight.
  __shared__ __align__(16) uint32_t tile[TPB][kPairTileWords];
  const int64_t rb = static_cast<int64_t>(blockIdx.y) * 64 * TPB, c0 = static_cast<int64_t>(blockIdx.x) * 64;
  const int q = static_cast<int>(threadIdx.x) >> 3, t = static_cast<int>(threadIdx.x) & 7;
  u32x4 a[TPB], b[TPB];
#pragma unroll
  for (int h = 0; h < TPB; ++h) {
    const int64_t r0 = rb + 64 * h;
    if (r0 + 2 * q < rows && c0 + 8 * t < cols) {
      const int64_t o = (r0 + 2 * q) * cols + c0 + 8 * t;
      a[h] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + o));
      b[h] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + o + cols));
    }
  }
#pragma unroll
  for (int h = 0; h < TPB; ++h) {
    if (rb + 64 * h + 2 * q < rows && c0 + 8 * t < cols) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        tile[h][pair_slot(8 * t + 2 * e, q)] = (a[h][e] & 0xFFFFu) | (b[h][e] << 16);
        tile[h][pair_slot(8 * t + 2 * e + 1, q)] = (a[h][e] >> 16) | (b[h][e] & 0xFFFF0000u);
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < TPB; ++h)
    if (rb + 64 * h < rows) store_pair_tile_transposed(tile[h], dst, rows, cols, rb + 64 * h, c0);
}

__global__ __launch_bounds__(256) void f32_to_bf16_kernel(const float* __restrict__ s, uint16_t* __restrict__ d, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256)
    d[i] = f32_to_bf16(s[i]);
}

__global__ __launch_bounds__(256) void bf16_to_f32_kernel(const uint16_t* __restrict__ s, float* __restrict__ d, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256)
    d[i] = bf16_to_f32(s[i]);
}

}  // namespace

int launch_transpose(const void* src, void* dst, int64_t rows, int64_t cols, int dtype, hipStream_t s) {
  if (rows == 0 || cols == 0) return VDSL_OK;
  if (dtype == VDSL_BF16 && rows % 8 == 0 && cols % 8 == 0) {
    const int64_t bx = (cols + 63) / 64, by = (rows + 127) / 128;
    if (bx > 0x7fffffff || by > 65535) return fail(VDSL_ERR_UNSUPPORTED, "transpose: tensor too large");
    hipLaunchKernelGGL(transpose_bf16_vec<2>, dim3(static_cast<unsigned>(bx), static_cast<unsigned>(by)), dim3(256), 0, s,
                       static_cast<const uint16_t*>(src), static_cast<uint16_t*>(dst), rows, cols);
    return check_launch("transpose_bf16_vec");
  }
  if (dtype == VDSL_BF16 && rows % 2 == 0 && cols % 2 == 0) {
    const int64_t bx = (cols + 127) / 128, by = (rows + 127) / 128;
    if (bx > 0x7fffffff || by > 65535) return fail(VDSL_ERR_UNSUPPORTED, "transpose: tensor too large");
    hipLaunchKernelGGL(transpose_bf16_pairs, dim3(static_cast<unsigned>(bx), static_cast<unsigned>(by)), dim3(256), 0, s,
                       static_cast<const uint32_t*>(src), static_cast<uint32_t*>(dst), rows, cols);
    return check_launch("transpose_bf16_pairs");
  }
  const int64_t gx = (cols + 63) / 64, gy = (rows + 63) / 64;
  if (gx > 0x7fffffff || gy > 65535) return fail(VDSL_ERR_UNSUPPORTED, "transpose: tensor too large");
  const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy));
  if (dtype == VDSL_F32)
    hipLaunchKernelGGL(transpose_kernel<float>, grid, dim3(256), 0, s, static_cast<const float*>(src), static_cast<float*>(dst), rows, cols);
  else
    hipLaunchKernelGGL(transpose_kernel<uint16_t>, grid, dim3(256), 0, s, static_cast<const uint16_t*>(src), static_cast<uint16_t*>(dst), rows, cols);
  return check_launch("transpose_kernel");
}

}  // namespace vdsl

using namespace vdsl;

extern "C" int vdsl_op_transpose(vdsl_queue q, int64_t rows, int64_t cols, int32_t dtype, vdsl_buffer src, vdsl_buffer dst) {
  VDSL_TRY(enter_queue(q));
  if (rows < 0 || cols < 0) return fail(VDSL_ERR_INVALID_ARG, "negative shape");
  if (dtype != VDSL_F32 && dtype != VDSL_BF16) return fail(VDSL_ERR_UNSUPPORTED, "transpose dtype must be f32 or bf16");
  const size_t n = nbytes(rows, cols, dtype_size(dtype));
  VDSL_TRY(check_buffer(q, src, n, "src", false));
  VDSL_TRY(check_buffer(q, dst, n, "dst", true));
  if (src == dst && n) return fail(VDSL_ERR_INVALID_ARG, "in-place transpose is not supported");
  return launch_transpose(src->ptr, dst->ptr, rows, cols, dtype, q->stream);
}

extern "C" int vdsl_op_cast(vdsl_queue q, int64_t n, int32_t src_dtype, vdsl_buffer src, int32_t dst_dtype, vdsl_buffer dst) {
  VDSL_TRY(enter_queue(q));
  if (n < 0) return fail(VDSL_ERR_INVALID_ARG, "negative element count");
  const bool ok = (src_dtype == VDSL_F32 || src_dtype == VDSL_BF16) && (dst_dtype == VDSL_F32 || dst_dtype == VDSL_BF16);
  if (!ok) return fail(VDSL_ERR_UNSUPPORTED, "cast supports f32 <-> bf16");
  VDSL_TRY(check_buffer(q, src, nbytes(n, dtype_size(src_dtype)), "src", false));
  VDSL_TRY(check_buffer(q, dst, nbytes(n, dtype_size(dst_dtype)), "dst", true));
  if (n == 0) return VDSL_OK;
  if (src_dtype == dst_dtype) return vdsl_buffer_copy(q, dst, 0, src, 0, static_cast<size_t>(n) * dtype_size(src_dtype));
  int64_t blocks = (n + 255) / 256;
  if (blocks > 16384) blocks = 16384;
  if (src_dtype == VDSL_F32)
    hipLaunchKernelGGL(f32_to_bf16_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, q->stream,
                       static_cast<const float*>(src->ptr), static_cast<uint16_t*>(dst->ptr), n);
  else
    hipLaunchKernelGGL(bf16_to_f32_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, q->stream,
                       static_cast<const uint16_t*>(src->ptr), static_cast<float*>(dst->ptr), n);
  return check_launch("cast_kernel");
}

// Batched vertex transform on gfx950: the MVP chain of the reference's test shader.
//
// color.mlir:10-39 (vertex_main) extends its vec3 position to vec4(pos, 1.0) (:15-21), multiplies
// it by the model, view and projection mat4 uniforms with three linalg.matvec (:29-36) and passes
// the position through as a varying (:39).  This file runs that program over n vertices, for mat4
// and for the dialect's other matrix types, mat2 and mat3 (source/README.md:34-37): one lane per
// four consecutive vertices, the matrices read once per lane from the uniform buffer (a
// wave-uniform address: scalar loads), positions and results moved as 16-byte vectors through LDS.
//
// Arithmetic (bit for bit the CPU oracle's orc_mat_transform): each matvec accumulates into a
// zero-initialised output in column order, out[i] = ((0 + M[i][0] v0) + M[i][1] v1) + ..., every
// product and sum rounded to f32 (linalg.matvec's mulf/addf; the library is built with
// -ffp-contract=off, so no multiply-add is fused).
//
// Roofline: HBM.  Per vertex 4 in_width bytes read, 4 dim written, plus the varying copy; at most
// 3 x 2 dim^2 = 96 f32 operations, below the 8 TB/s HBM rate's VALU budget for those bytes.

#include "common.h"

namespace vdsl {
namespace {

// out = M v for a D x D row-major matrix: out[i] = ((0 + M[i][0] v0) + M[i][1] v1) + ...
template <int D>
__device__ __forceinline__ void matvec(const float* __restrict__ m, const float (&v)[4], float (&o)[4]) {
#pragma unroll
  for (int i = 0; i < D; ++i) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < D; ++j) acc = acc + m[D * i + j] * v[j];
    o[i] = acc;
  }
}

// One block of 256 lanes transforms 1024 consecutive vertices.  Every global access instruction
// is contiguous across the wave (lane t moves 16-byte unit t + 256 k of the block's range), and the
// units are redistributed through LDS: a lane's four vertices are 4 IW floats in and 4 D floats out,
// which, moved by the lanes themselves at that stride, touched every cache line with several
// instructions and ran at a fifth of the HBM rate (measured for vec3 in, vec4 out).  The varying (a
// copy of pos) is stored straight from the coalesced loads.  LDS (16 KiB) holds the block's
// positions, then its results; reads of a lane's 4 IW floats (16-byte units IW t .. IW t + IW - 1)
// hit 16 distinct bank groups per 16 lanes for IW = 3, and mat4 results are written at unit
// 4t + (j ^ ((t >> 2) & 3)) so that both the writes (stride 4 units) and the contiguous reads back
// spread over all bank groups.
constexpr int kVerts = 1024;

__device__ __forceinline__ int out_slot(int s) { return (s & ~3) | ((s & 3) ^ ((s >> 4) & 3)); }

// D: matrix dimension (2..4, the output components); IW: components per input position (D - 1,
// extended by w = 1, or D); NM: matrices in the chain (1..3).
template <int D, int IW, int NM>
__global__ __launch_bounds__(256) void mat_transform_kernel(const float* __restrict__ pos, const float* __restrict__ mats,
                                                            float* __restrict__ out, float* __restrict__ varying, int64_t n) {
  __shared__ f32x4 stage[kVerts];  // 16 KiB: IW * 256 input units, then D * 256 result units
  float m[NM * D * D];
#pragma unroll
  for (int k = 0; k < NM * D * D; ++k) m[k] = mats[k];
  const int t = threadIdx.x;
  const int64_t v0 = static_cast<int64_t>(blockIdx.x) * kVerts;
  const bool whole = v0 + kVerts <= n;
  const int64_t fbase = v0 * IW;              // first float of the block's positions
  const int64_t fend = n * IW;                // floats of pos
  float* sf = reinterpret_cast<float*>(stage);
  // ---- positions in, varying out: units t + 256 k, k < IW ----
  if (whole) {
#pragma unroll
    for (int k = 0; k < IW; ++k) {
      const f32x4 u = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(pos + fbase) + t + 256 * k);
      stage[t + 256 * k] = u;
      if (varying) __builtin_nontemporal_store(u, reinterpret_cast<f32x4*>(varying + fbase) + t + 256 * k);
    }
  } else {
#pragma unroll 4
    for (int k = 0; k < 4 * IW; ++k) {
      const int64_t f = fbase + t + 256 * k;
      const float x = f < fend ? pos[f] : 0.0f;
      sf[t + 256 * k] = x;
      if (varying && f < fend) varying[f] = x;
    }
  }
  __syncthreads();
  float p[4 * IW];
#pragma unroll
  for (int k = 0; k < IW; ++k) {
    const f32x4 u = stage[IW * t + k];
    p[4 * k] = u[0]; p[4 * k + 1] = u[1]; p[4 * k + 2] = u[2]; p[4 * k + 3] = u[3];
  }
  __syncthreads();
  // ---- the four vertices 4t .. 4t+3 of the block ----
  float res[4 * D];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < IW; ++i) v[i] = p[IW * j + i];
    if constexpr (IW == D - 1) v[D - 1] = 1.0f;  // vec(pos, 1.0) (color.mlir:21)
#pragma unroll
    for (int r = 0; r < NM; ++r) {
      float o[4];
      matvec<D>(m + D * D * r, v, o);
#pragma unroll
      for (int i = 0; i < D; ++i) v[i] = o[i];
    }
#pragma unroll
    for (int i = 0; i < D; ++i) res[D * j + i] = v[i];
  }
  // the lane's 4 D results are units D t .. D t + D - 1 of the block's output
#pragma unroll
  for (int k = 0; k < D; ++k) {
    const f32x4 u = {res[4 * k], res[4 * k + 1], res[4 * k + 2], res[4 * k + 3]};
    stage[D == 4 ? out_slot(4 * t + k) : D * t + k] = u;
  }
  __syncthreads();
  // ---- results out: units t + 256 k, k < D ----
  if (whole) {
#pragma unroll
    for (int k = 0; k < D; ++k) {
      const int u = t + 256 * k;
      __builtin_nontemporal_store(stage[D == 4 ? out_slot(u) : u], reinterpret_cast<f32x4*>(out + v0 * D) + u);
    }
  } else {
    const int64_t oend = n * D;
#pragma unroll 4
    for (int k = 0; k < 4 * D; ++k) {
      const int f = t + 256 * k;  // float f of the block's results
      const int src = D == 4 ? 4 * out_slot(f >> 2) + (f & 3) : f;
      if (v0 * D + f < oend) out[v0 * D + f] = sf[src];
    }
  }
}

template <int D, int IW>
void launch_iw(int nm, const float* pos, const float* mats, float* out, float* varying, int64_t n, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((n + kVerts - 1) / kVerts)), block(256);
  if (nm == 1) hipLaunchKernelGGL((mat_transform_kernel<D, IW, 1>), grid, block, 0, s, pos, mats, out, varying, n);
  else if (nm == 2) hipLaunchKernelGGL((mat_transform_kernel<D, IW, 2>), grid, block, 0, s, pos, mats, out, varying, n);
  else hipLaunchKernelGGL((mat_transform_kernel<D, IW, 3>), grid, block, 0, s, pos, mats, out, varying, n);
}

template <int D>
void launch_dim(int in_width, int nm, const float* pos, const float* mats, float* out, float* varying, int64_t n, hipStream_t s) {
  if (in_width == D) launch_iw<D, D>(nm, pos, mats, out, varying, n, s);
  else launch_iw<D, D - 1>(nm, pos, mats, out, varying, n, s);
}

}  // namespace
}  // namespace vdsl

using namespace vdsl;

extern "C" int vdsl_op_mat_transform(vdsl_queue q, int64_t n, int32_t dim, int32_t in_width, vdsl_buffer pos, int32_t n_mats,
                                     vdsl_buffer mats, vdsl_buffer out, vdsl_buffer varying) {
  VDSL_TRY(enter_queue(q));
  if (n < 0) return fail(VDSL_ERR_INVALID_ARG, "negative vertex count");
  if (dim < 2 || dim > 4) return fail(VDSL_ERR_INVALID_ARG, "dim must be 2, 3 or 4 (mat2, mat3, mat4)");
  if (in_width != dim && in_width != dim - 1)
    return fail(VDSL_ERR_INVALID_ARG, "in_width must be dim, or dim - 1 (extended by w = 1)");
  if (n_mats < 1 || n_mats > 3) return fail(VDSL_ERR_INVALID_ARG, "n_mats must be 1, 2 or 3");
  VDSL_TRY(check_buffer(q, pos, nbytes(n, in_width, 4), "pos", false));
  VDSL_TRY(check_buffer(q, mats, nbytes(n_mats, static_cast<int64_t>(dim) * dim, 4), "mats", false));
  VDSL_TRY(check_buffer(q, out, nbytes(n, dim, 4), "out", true));
  if (varying) VDSL_TRY(check_buffer(q, varying, nbytes(n, in_width, 4), "varying", true));
  if (out == pos || varying == pos || (varying && varying == out))
    return fail(VDSL_ERR_INVALID_ARG, "out and varying must not alias pos or each other");
  if (n == 0) return VDSL_OK;
  if ((n + 1023) / 1024 > 0x7fffffff) return fail(VDSL_ERR_UNSUPPORTED, "mat_transform: too many vertices");
  const auto* p = static_cast<const float*>(pos->ptr);
  const auto* m = static_cast<const float*>(mats->ptr);
  auto* o = static_cast<float*>(out->ptr);
  float* vy = varying ? static_cast<float*>(varying->ptr) : nullptr;
  if (dim == 2) launch_dim<2>(in_width, n_mats, p, m, o, vy, n, q->stream);
  else if (dim == 3) launch_dim<3>(in_width, n_mats, p, m, o, vy, n, q->stream);
  else launch_dim<4>(in_width, n_mats, p, m, o, vy, n, q->stream);
  return check_launch("mat_transform_kernel");
}

extern "C" int vdsl_op_vec_transform(vdsl_queue q, int64_t n, int32_t in_width, vdsl_buffer pos, int32_t n_mats,
                                     vdsl_buffer mats, vdsl_buffer out, vdsl_buffer varying) {
  if (in_width != 3 && in_width != 4) {
    VDSL_TRY(enter_queue(q));
    return fail(VDSL_ERR_INVALID_ARG, "in_width must be 3 (vec3, extended by w = 1) or 4");
  }
  return vdsl_op_mat_transform(q, n, 4, in_width, pos, n_mats, mats, out, varying);
}

// Batched vertex transform on gfx950: the MVP chain of the reference's test shader.
//
// color.mlir:10-39 (vertex_main) extends its vec3 position to vec4(pos, 1.0) (:15-21), multiplies
// it by the model, view and projection mat4 uniforms with three linalg.matvec (:29-36) and passes
// the position through as a varying (:39).  This file runs that program over n vertices: one lane
// per four consecutive vertices, the matrices read once per lane from the uniform buffer (a
// wave-uniform address: scalar loads), positions and results moved as 16-byte vectors through LDS.
//
// Arithmetic (bit for bit the CPU oracle's orc_vec_transform): each matvec accumulates into a
// zero-initialised output in column order, out[i] = (((0 + M[i][0] v0) + M[i][1] v1) + M[i][2] v2)
// + M[i][3] v3, every product and sum rounded to f32 (linalg.matvec's mulf/addf; the library is
// built with -ffp-contract=off, so no multiply-add is fused).
//
// Roofline: HBM.  Per vertex 12 (vec3) or 16 (vec4) bytes read, 16 written, plus the varying copy;
// at most 3 x 32 = 96 f32 operations, below the 8 TB/s HBM rate's VALU budget for 28-40 bytes.

#include "common.h"

namespace vdsl {
namespace {

__device__ __forceinline__ void matvec4(const float* __restrict__ m, const float (&v)[4], float (&o)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = acc + m[4 * i + j] * v[j];
    o[i] = acc;
  }
}

// One block of 256 lanes transforms 1024 consecutive vertices.  Every global access instruction
// is contiguous across the wave (lane t moves 16-byte unit t + 256 k of the block's range), and the
// units are redistributed through LDS: a lane's four vertices are 48 (vec3) or 64 (vec4) bytes,
// which, moved by the lanes themselves as 16-byte pieces at that stride, touched every cache line
// with several instructions and ran at a fifth of the HBM rate.  The varying (a copy of pos) is
// stored straight from the coalesced loads.  LDS (16 KiB) holds the block's positions, then its
// results; reads of a lane's 48 bytes (16-byte units 3t..3t+2) hit 16 distinct bank groups per 16
// lanes, and results are written at unit 4t + (j ^ ((t >> 2) & 3)) so that both the writes
// (stride 4 units) and the contiguous reads back spread over all bank groups.
constexpr int kVerts = 1024;

__device__ __forceinline__ int out_slot(int s) { return (s & ~3) | ((s & 3) ^ ((s >> 4) & 3)); }

// IW: components per input position (3 or 4); NM: matrices in the chain (1..3).
template <int IW, int NM>
__global__ __launch_bounds__(256) void vec_transform_kernel(const float* __restrict__ pos, const float* __restrict__ mats,
                                                            float* __restrict__ out, float* __restrict__ varying, int64_t n) {
  __shared__ f32x4 stage[kVerts];  // 16 KiB: IW * 256 input units, then 1024 result units
  float m[NM * 16];
#pragma unroll
  for (int k = 0; k < NM * 16; ++k) m[k] = mats[k];
  const int t = threadIdx.x;
  const int64_t v0 = static_cast<int64_t>(blockIdx.x) * kVerts;
  const bool whole = v0 + kVerts <= n;
  const int64_t fbase = v0 * IW;              // first float of the block's positions
  const int64_t fend = n * IW;                // floats of pos
  // ---- positions in, varying out: units t + 256 k, k < IW ----
  if (whole) {
#pragma unroll
    for (int k = 0; k < IW; ++k) {
      const f32x4 u = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(pos + fbase) + t + 256 * k);
      stage[t + 256 * k] = u;
      if (varying) __builtin_nontemporal_store(u, reinterpret_cast<f32x4*>(varying + fbase) + t + 256 * k);
    }
  } else {
    float* sf = reinterpret_cast<float*>(stage);
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
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float v[4] = {p[IW * j], p[IW * j + 1], p[IW * j + 2], 1.0f};  // vec4(pos, 1.0) (color.mlir:21)
    if constexpr (IW == 4) v[3] = p[IW * j + 3];
#pragma unroll
    for (int r = 0; r < NM; ++r) {
      float o[4];
      matvec4(m + 16 * r, v, o);
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = o[i];
    }
    const f32x4 res = {v[0], v[1], v[2], v[3]};
    stage[out_slot(4 * t + j)] = res;
  }
  __syncthreads();
  // ---- results out: units t + 256 k, k < 4 ----
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int u = t + 256 * k;
    if (whole || v0 + u < n) __builtin_nontemporal_store(stage[out_slot(u)], reinterpret_cast<f32x4*>(out) + v0 + u);
  }
}

template <int IW>
void launch_iw(int nm, const float* pos, const float* mats, float* out, float* varying, int64_t n, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((n + kVerts - 1) / kVerts)), block(256);
  if (nm == 1) hipLaunchKernelGGL((vec_transform_kernel<IW, 1>), grid, block, 0, s, pos, mats, out, varying, n);
  else if (nm == 2) hipLaunchKernelGGL((vec_transform_kernel<IW, 2>), grid, block, 0, s, pos, mats, out, varying, n);
  else hipLaunchKernelGGL((vec_transform_kernel<IW, 3>), grid, block, 0, s, pos, mats, out, varying, n);
}

}  // namespace
}  // namespace vdsl

using namespace vdsl;

extern "C" int vdsl_op_vec_transform(vdsl_queue q, int64_t n, int32_t in_width, vdsl_buffer pos, int32_t n_mats,
                                     vdsl_buffer mats, vdsl_buffer out, vdsl_buffer varying) {
  VDSL_TRY(enter_queue(q));
  if (n < 0) return fail(VDSL_ERR_INVALID_ARG, "negative vertex count");
  if (in_width != 3 && in_width != 4) return fail(VDSL_ERR_INVALID_ARG, "in_width must be 3 (vec3, extended by w = 1) or 4");
  if (n_mats < 1 || n_mats > 3) return fail(VDSL_ERR_INVALID_ARG, "n_mats must be 1, 2 or 3");
  VDSL_TRY(check_buffer(q, pos, nbytes(n, in_width, 4), "pos", false));
  VDSL_TRY(check_buffer(q, mats, nbytes(n_mats, 16, 4), "mats", false));
  VDSL_TRY(check_buffer(q, out, nbytes(n, 4, 4), "out", true));
  if (varying) VDSL_TRY(check_buffer(q, varying, nbytes(n, in_width, 4), "varying", true));
  if (out == pos || varying == pos || (varying && varying == out))
    return fail(VDSL_ERR_INVALID_ARG, "out and varying must not alias pos or each other");
  if (n == 0) return VDSL_OK;
  if ((n + 1023) / 1024 > 0x7fffffff) return fail(VDSL_ERR_UNSUPPORTED, "vec_transform: too many vertices");
  const auto* p = static_cast<const float*>(pos->ptr);
  const auto* m = static_cast<const float*>(mats->ptr);
  auto* o = static_cast<float*>(out->ptr);
  float* vy = varying ? static_cast<float*>(varying->ptr) : nullptr;
  if (in_width == 3) launch_iw<3>(n_mats, p, m, o, vy, n, q->stream);
  else launch_iw<4>(n_mats, p, m, o, vy, n, q->stream);
  return check_launch("vec_transform_kernel");
}

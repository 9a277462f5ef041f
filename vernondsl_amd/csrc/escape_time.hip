// Op class 1: per-pixel escape-time iterative map on gfx950.
//
// Follows the Taichi program `paint(t)` in fractal.py:16-25:
//   - struct-for over the field (fractal.py:18) -> one lane per pixel (i, j);
//   - pixel -> complex map z = (i/n - 1, j/n - 0.5) * 2 (fractal.py:20) -> the affine map of
//     vdsl_escape_time_params, each step rounded in f32 (this file is built -ffp-contract=off);
//   - check-then-update loop `while |z| < 20 and it < 50: z = complex_sqr(z) + c; it += 1`
//     (fractal.py:22-24) with complex_sqr = (zr^2 - zi^2, zi*zr*2) (fractal.py:11-13);
//   - store `1 - it * 0.02` (fractal.py:25) or the raw int32 count.
//
// Mapping to the hardware: the work is VALU-bound with per-lane trip counts, so each wavefront
// takes an 8x8 pixel tile (spatially coherent lanes escape at similar iterations, which keeps
// more lanes of a wave live than a 1x64 strip does), and a wave leaves the loop as soon as all
// of its 64 lanes have escaped.  A 256-thread block holds 4 such tiles as a 16x16 patch.

#include <cmath>
#include <cstring>

#include "common.h"
#include "lanemask.h"

namespace vdsl {
namespace {

constexpr int kTile = 8;          // wave tile edge (8x8 = 64 lanes)
constexpr int kBlockEdge = 16;    // block patch edge: 2x2 wave tiles
// Trips per block of the deferred count (measured on the config-1 image: 8 -> 21.8 us, 16 -> 20.0,
// 32 -> 19.8; a block also bounds the trips a wave makes after its last lane escaped).
#ifndef VDSL_ESC_UNROLL
#define VDSL_ESC_UNROLL 16
#endif

__device__ __forceinline__ float pixel_coord(int idx, float den, float off, float scale, float post) {
  float v = static_cast<float>(idx) / den;  // correctly rounded f32 division
  v = v + off;
  v = v * scale;
  return v + post;
}

// Iteration count of pixel (i, j), run by one lane of a wave of in-grid pixels.
template <int FAMILY, int TEST, int ROUNDING>
__device__ __forceinline__ int escape_count(const vdsl_escape_time_params& p, int i, int j) {
  float zr, zi, cr, ci;
  {
    const float im = pixel_coord(j, p.im_den, p.im_off, p.im_scale, p.im_post);
    const float re = pixel_coord(i, p.re_den, p.re_off, p.re_scale, p.re_post);
    if (FAMILY == VDSL_ESC_MANDELBROT) {
      zr = 0.0f; zi = 0.0f; cr = re; ci = im;
    } else {
      zr = re; zi = im; cr = p.c_re; ci = p.c_im;
    }
  }
  // Escape test of this pixel's current z (mag = |z|^2): MAG2_GT continues while !(mag > bound);
  // NORM_GE continues while sqrtf(mag) < b, evaluated as mag < bound: for NORM_GE the launcher
  // replaces b by the f32 threshold with sqrtf(m) < b <=> m < threshold for every m.
  const float bound = p.bound;
  const int max_iter = p.max_iter;

  // Wave-uniform loop: every pixel steps z each trip; `live` (sticky: set until the first failed
  // escape test) marks the trips made while live, whose number is the count of updates of the
  // check-then-update loop.  An escaped pixel keeps stepping z but is no longer counted.  The live
  // set is a 64-bit lane mask held in scalar registers: each trip's escape test is a ballot (the
  // compare writes the mask directly) and one scalar AND keeps it sticky, so a trip costs the six
  // rounded operations of the update and one compare.  Counting is deferred to the end of each
  // block of kUnroll trips: when no lane died in the block, every live lane adds kUnroll (one
  // select); otherwise each lane adds the trips it was live for, whose bits follow from a binary
  // search over the block's sticky masks (scalar ops, then five selects).  The max_iter check is
  // made once per block (the tail block checks each trip), and the wave stops once no lane is live.
  constexpr int kUnroll = VDSL_ESC_UNROLL;
  static_assert(kUnroll == 16, "the bit-plane count covers 16-trip blocks");
  auto step = [&]() -> bool {  // one update of z; returns this trip's escape test (true: go on)
    float nzr, nzi, mag;
    if (ROUNDING == VDSL_ESC_ROUND_SEPARATE) {
      const float zr2 = zr * zr;
      const float zi2 = zi * zi;
      mag = zr2 + zi2;
      nzr = (zr2 - zi2) + cr;
      nzi = ((zi * zr) * 2.0f) + ci;
    } else {
      const float qq = zi * zi;
      mag = __builtin_fmaf(zr, zr, qq);
      nzr = __builtin_fmaf(zr, zr, -qq) + cr;
      nzi = __builtin_fmaf(zr + zr, zi, ci);
    }
    const bool pass = (TEST == VDSL_ESC_MAG2_GT) ? !(mag > bound) : (mag < bound);
    zr = nzr;
    zi = nzi;
    return pass;
  };
  uint64_t live = __builtin_amdgcn_ballot_w64(true);
  int it = 0;
  int k = 0;
  // Exact periodicity: z is saved (as bits) at the end of blocks 1, 2, 4, 8, ... and compared with
  // z at the end of every block.  A live lane whose z equals an earlier z of its own orbit repeats
  // the escape tests it has passed since then for ever, so its count is max_iter; it leaves the
  // live set at once instead of stepping on to max_iter.  Bitwise equality, so -0 != +0 and NaN
  // never matches: only a state that truly recurs is taken.
  uint32_t save_r = __float_as_uint(zr), save_i = __float_as_uint(zi);
  for (; k <= max_iter - kUnroll; k += kUnroll) {
    uint64_t m[kUnroll];
    uint64_t lk = live;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      lk &= __builtin_amdgcn_ballot_w64(step());
      m[u] = lk;
    }
    it += block_trips16(m, live);
    const uint32_t br = __float_as_uint(zr), bi = __float_as_uint(zi);
    const uint64_t per = lk & __builtin_amdgcn_ballot_w64(br == save_r) & __builtin_amdgcn_ballot_w64(bi == save_i);
    if (per) it = lane_select_keep(per, max_iter, it);
    live = lk & ~per;
    const int blocks_done = __builtin_amdgcn_readfirstlane(k) / kUnroll + 1;  // wave-uniform
    if ((blocks_done & (blocks_done - 1)) == 0) {
      save_r = br;
      save_i = bi;
    }
    if (live == 0) break;
  }
  if (k > max_iter - kUnroll && live != 0) {
    for (; k < max_iter; ++k) {
      live &= __builtin_amdgcn_ballot_w64(step());
      it += lane_select(live, 1, 0);
    }
  }
  return it;
}

template <int OUT>
__device__ __forceinline__ void escape_store(const vdsl_escape_time_params& p, void* out, int i, int j, int it) {
  const size_t o = static_cast<size_t>(i) * static_cast<size_t>(p.nj) + static_cast<size_t>(j);
  if (OUT == VDSL_ESC_OUT_I32_COUNT) {
    static_cast<int32_t*>(out)[o] = it;
  } else {
    const float f = static_cast<float>(it) * p.out_scale;
    static_cast<float*>(out)[o] = p.out_base + f;
  }
}

// One 8x8 tile per wave, 2x2 tiles per block, one block per 16x16 patch.
template <int FAMILY, int TEST, int ROUNDING, int OUT>
__global__ __launch_bounds__(256) void escape_time_kernel(vdsl_escape_time_params p, void* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int i = blockIdx.y * kBlockEdge + (wave >> 1) * kTile + (lane >> 3);
  const int j = blockIdx.x * kBlockEdge + (wave & 1) * kTile + (lane & 7);
  if (j >= p.nj || i >= p.ni) return;
  const int it = escape_count<FAMILY, TEST, ROUNDING>(p, i, j);
  escape_store<OUT>(p, out, i, j, it);
}

// Smallest f32 m >= 0 with sqrtf(m) >= b, so that for every f32 m (including +inf and NaN)
// sqrtf(m) < b  <=>  m < threshold.  Bisection over the ordered bit patterns of [0, +inf].
float norm_threshold(float b) {
  if (!(b > 0.0f)) return 0.0f;        // nothing is < b when b <= 0 (or NaN): m < 0 never holds
  uint32_t lo = 0, hi = 0x7F800000u;   // sqrtf(+0) = 0 < b;  sqrtf(+inf) = inf >= b
  while (hi - lo > 1) {
    const uint32_t mid = lo + (hi - lo) / 2;
    float m;
    std::memcpy(&m, &mid, 4);
    if (std::sqrt(m) >= b) hi = mid; else lo = mid;
  }
  float t;
  std::memcpy(&t, &hi, 4);
  return t;
}

// Unused dynamic LDS reserved per block to cap residency at 6 blocks (24 waves) per CU: 160 KiB
// of LDS / 24 KiB.  Left at the register limit (8 blocks per CU) the waves of set-interior tiles
// (256 trips) pile up to 8 deep on the SIMDs that took them first and finish last, at a fraction
// of the issue rate; fewer than ~4 waves per SIMD cannot hide the z update's dependence chain.
// Config 1: 6 blocks 18.6 us, 7 blocks 19.3, 8 (no cap) 19.9, 5 blocks 19.7, 3 or fewer 26.7.
constexpr unsigned kEscLdsBytes = 24u << 10;

template <int FAMILY, int TEST, int ROUNDING>
int launch_out(const vdsl_escape_time_params& p, void* out, hipStream_t s, dim3 grid) {
  if (p.out_kind == VDSL_ESC_OUT_I32_COUNT)
    hipLaunchKernelGGL((escape_time_kernel<FAMILY, TEST, ROUNDING, VDSL_ESC_OUT_I32_COUNT>), grid, dim3(256), kEscLdsBytes, s, p, out);
  else
    hipLaunchKernelGGL((escape_time_kernel<FAMILY, TEST, ROUNDING, VDSL_ESC_OUT_F32_AFFINE>), grid, dim3(256), kEscLdsBytes, s, p, out);
  return check_launch("escape_time_kernel");
}

template <int FAMILY, int TEST>
int launch_round(const vdsl_escape_time_params& p, void* out, hipStream_t s, dim3 grid) {
  if (p.rounding == VDSL_ESC_ROUND_SEPARATE) return launch_out<FAMILY, TEST, VDSL_ESC_ROUND_SEPARATE>(p, out, s, grid);
  return launch_out<FAMILY, TEST, VDSL_ESC_ROUND_FMA>(p, out, s, grid);
}

template <int FAMILY>
int launch_test(const vdsl_escape_time_params& p, void* out, hipStream_t s, dim3 grid) {
  if (p.escape_test == VDSL_ESC_MAG2_GT) return launch_round<FAMILY, VDSL_ESC_MAG2_GT>(p, out, s, grid);
  return launch_round<FAMILY, VDSL_ESC_NORM_GE>(p, out, s, grid);
}
}  // namespace
}  // namespace vdsl

using namespace vdsl;

extern "C" int vdsl_op_escape_time(vdsl_queue q, const vdsl_escape_time_params* p, vdsl_buffer out) {
  VDSL_TRY(enter_queue(q));
  if (!p) return fail(VDSL_ERR_INVALID_ARG, "params is null");
  if (p->ni < 0 || p->nj < 0) return fail(VDSL_ERR_INVALID_ARG, "negative grid extent");
  if (p->max_iter < 0) return fail(VDSL_ERR_INVALID_ARG, "max_iter < 0");
  if (p->family != VDSL_ESC_MANDELBROT && p->family != VDSL_ESC_JULIA)
    return fail(VDSL_ERR_INVALID_ARG, "unknown escape family");
  if (p->escape_test != VDSL_ESC_MAG2_GT && p->escape_test != VDSL_ESC_NORM_GE)
    return fail(VDSL_ERR_INVALID_ARG, "unknown escape test");
  if (p->rounding != VDSL_ESC_ROUND_SEPARATE && p->rounding != VDSL_ESC_ROUND_FMA)
    return fail(VDSL_ERR_INVALID_ARG, "unknown rounding form");
  if (p->out_kind != VDSL_ESC_OUT_I32_COUNT && p->out_kind != VDSL_ESC_OUT_F32_AFFINE)
    return fail(VDSL_ERR_INVALID_ARG, "unknown output kind");
  const size_t bytes = static_cast<size_t>(p->ni) * static_cast<size_t>(p->nj) * 4u;
  VDSL_TRY(check_buffer(q, out, bytes, "out", true));
  if (bytes == 0) return VDSL_OK;
  const dim3 grid((p->nj + kBlockEdge - 1) / kBlockEdge, (p->ni + kBlockEdge - 1) / kBlockEdge);
  if (grid.y > 65535u) return fail(VDSL_ERR_UNSUPPORTED, "ni too large");
  vdsl_escape_time_params kp = *p;
  if (kp.escape_test == VDSL_ESC_NORM_GE) kp.bound = norm_threshold(p->bound);
  if (kp.family == VDSL_ESC_MANDELBROT) return launch_test<VDSL_ESC_MANDELBROT>(kp, out->ptr, q->stream, grid);
  return launch_test<VDSL_ESC_JULIA>(kp, out->ptr, q->stream, grid);
}

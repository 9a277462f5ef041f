// Internal definitions shared by the runtime and the gfx950 kernels of libvdsl.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <string>

#include "fmath.h"
#include "vdsl.h"

// ---- handle objects ------------------------------------------------------------------------
enum : uint32_t {
  kMagicDevice = 0x56444556u,  // "VDEV"
  kMagicBuffer = 0x56425546u,  // "VBUF"
  kMagicQueue = 0x56515545u,   // "VQUE"
  kMagicGraph = 0x56475250u,   // "VGRP"
  kMagicEvent = 0x56455654u,   // "VEVT"
};

struct vdsl_device_s {
  uint32_t magic;
  int ordinal;
  hipDeviceProp_t props;
  std::atomic<int> live;  // buffers, queues, graphs and events that belong to this device
};

struct vdsl_buffer_s {
  uint32_t magic;
  vdsl_device dev;
  void* ptr;
  size_t bytes;
  int binding;
};

struct vdsl_queue_s {
  uint32_t magic;
  vdsl_device dev;
  hipStream_t stream;
  bool capturing;
};

struct vdsl_graph_s {
  uint32_t magic;
  vdsl_device dev;
  hipGraph_t graph;
  hipGraphExec_t exec;
};

struct vdsl_event_s {
  uint32_t magic;
  vdsl_device dev;
  hipEvent_t ev;
};

namespace vdsl {

// Records `msg` as this thread's last error and returns `status`.
int fail(int status, const std::string& msg);
// Fails with VDSL_ERR_DEVICE and the HIP error string if `e` is not hipSuccess.
int check_hip(hipError_t e, const char* what);
// Checks the launch that was just enqueued.
int check_launch(const char* kernel);

bool valid_device(vdsl_device d);
bool valid_buffer(vdsl_buffer b);
bool valid_queue(vdsl_queue q);

// Validates a queue and makes its device current.  Returns VDSL_OK or an error status.
int enter_queue(vdsl_queue q);
// Validates `b` (on the queue's device) and that it holds at least `bytes`.  `name` is used in
// the error message.  If `writable`, rejects UNIFORM_CONSTANT buffers.
int check_buffer(vdsl_queue q, vdsl_buffer b, size_t bytes, const char* name, bool writable);

size_t dtype_size(int dtype);

// Per-device set-up of the allocation-free int8 GEMM (gemm_w8a8.hip); called by vdsl_device_open
// with the device current.
void w8a8_noalloc_setup(int ordinal);

// Byte size a * b * c of a dense operand, or kSizeOverflow when a factor is negative or the
// product does not fit in size_t.  check_buffer rejects kSizeOverflow with VDSL_ERR_SHAPE, so an
// entry point that sizes every operand with nbytes() fails before it enqueues anything instead of
// accepting a wrapped (small) size and reading past an allocation.
constexpr size_t kSizeOverflow = ~static_cast<size_t>(0);
inline size_t nbytes(int64_t a, int64_t b, int64_t c = 1) {
  if (a < 0 || b < 0 || c < 0) return kSizeOverflow;
  size_t ab = 0, abc = 0;
  if (__builtin_mul_overflow(static_cast<size_t>(a), static_cast<size_t>(b), &ab) ||
      __builtin_mul_overflow(ab, static_cast<size_t>(c), &abc) || abc == kSizeOverflow)
    return kSizeOverflow;
  return abc;
}

}  // namespace vdsl

#define VDSL_TRY(expr)              \
  do {                              \
    int _st = (expr);               \
    if (_st != VDSL_OK) return _st; \
  } while (0)

// ---- device-side helpers -------------------------------------------------------------------
namespace vdsl {


__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round-to-nearest-even f32 -> bf16 with gfx950's v_cvt_pk_bf16_f32 (identical to the
// bit-level RNE of the CPU oracle for every non-NaN input; a NaN stays a quiet NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
// Two values converted by one v_cvt_pk_bf16_f32: lo in bits 0-15, hi in bits 16-31.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// Butterfly reductions across one 64-lane wavefront (every lane gets the result).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}
// erfc(x) by the Chebyshev-fitted form of Numerical Recipes (Press et al., 2nd ed., sec. 6.2,
// "erfcc"): erfc(|x|) = t exp(-x^2 + P(t)), t = 1 / (1 + |x|/2), P a degree-9 polynomial, with
// fractional error below 1.2e-7 for every x; erfc(-x) = 2 - erfc(x).  Branch-free (the library
// erfcf picks among argument ranges per lane), which matters in a GEMM epilogue that evaluates it
// on every output element.
__device__ __forceinline__ float erfc_cheb(float x) {
  const float z = fabsf(x);
  const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(0.5f, z, 1.0f));
  float p = 0.17087277f;
  p = __builtin_fmaf(p, t, -0.82215223f);
  p = __builtin_fmaf(p, t, 1.48851587f);
  p = __builtin_fmaf(p, t, -1.13520398f);
  p = __builtin_fmaf(p, t, 0.27886807f);
  p = __builtin_fmaf(p, t, -0.18628806f);
  p = __builtin_fmaf(p, t, 0.09678418f);
  p = __builtin_fmaf(p, t, 0.37409196f);
  p = __builtin_fmaf(p, t, 1.00002368f);
  p = __builtin_fmaf(p, t, -1.26551223f);
  const float r = t * __expf(__builtin_fmaf(-z, z, p));
  return x >= 0.0f ? r : 2.0f - r;
}

// 0.5 v (1 + erf(v / sqrt2)) written as 0.5 v erfc(-v / sqrt2): no cancellation for v < 0.
// Used where the result is rounded to bf16 (the GEMM epilogue): erfc_cheb rounds its exponent
// -x^2 + P once, an absolute error of up to ulp(x^2)/2, i.e. a relative error growing like
// x^2 2^-24 (4e-6 at |x| = 8.5), far below bf16 resolution.
__device__ __forceinline__ float gelu_f(float v) { return 0.5f * v * erfc_cheb(-v * 0.7071067811865476f); }

// GELU'(v), shared by the GELU backward kernels and the fused GEMM epilogue (one definition, so
// the fused and unfused paths agree bit for bit).
__device__ __forceinline__ float gelu_grad_f(float v) {
  // d/dv [0.5 v (1 + erf(v / sqrt2))] = Phi(v) + v phi(v), with Phi(v) = 0.5 erfc(-v / sqrt2)
  // (erfc keeps full relative accuracy where 1 + erf(.) would cancel, v < 0).  Branch-free:
  // erfc_cheb (fractional error < 1.2e-7) and exp_fast (< 2e-7 + 1 ulp); the result is rounded
  // to bf16, and near the zero of GELU' (v = -0.75) the absolute error stays below 2e-7 (1.2e-7
  // measured over config 4's 8.4 M pre-activations against the f64 formula).
  return 0.5f * erfc_cheb(-v * 0.7071067811865476f) + v * exp_fast(-0.5f * v * v) * 0.3989422804014327f;
}

// GELU for f32 results (the standalone elementwise op), relative accuracy ~1e-6 over the f32
// range.  With z = |v|/sqrt2 and erfc(z) = t exp(-z^2 + P(t)) as above, the exponent is the
// sensitive part (erfc's condition number is ~2 z^2), so it is never formed from a rounded z:
// z^2 = v^2 / 2 = (h + l) / 2 with h = fl(v v) and l = v v - h exact (one fma), and
// exp(-z^2 + P) = exp(-h/2) exp(P) (1 - l/2), both exponentials by exp_fast.  Only t, where
// the sensitivity is small, uses the rounded z.
__device__ __forceinline__ float gelu_f_acc(float v) {
  const float a = fabsf(v);
  const float z = a * 0.7071067811865476f;
  const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(0.5f, z, 1.0f));
  float p = 0.17087277f;
  p = __builtin_fmaf(p, t, -0.82215223f);
  p = __builtin_fmaf(p, t, 1.48851587f);
  p = __builtin_fmaf(p, t, -1.13520398f);
  p = __builtin_fmaf(p, t, 0.27886807f);
  p = __builtin_fmaf(p, t, -0.18628806f);
  p = __builtin_fmaf(p, t, 0.09678418f);
  p = __builtin_fmaf(p, t, 0.37409196f);
  p = __builtin_fmaf(p, t, 1.00002368f);
  p = __builtin_fmaf(p, t, -1.26551223f);
  const float h = a * a;
  const float l = __builtin_isfinite(h) ? __builtin_fmaf(a, a, -h) : 0.0f;  // inf - inf would be NaN
  const float c = (exp_fast(-0.5f * h) * exp_fast(p)) * t;
  const float e = __builtin_fmaf(c, -0.5f * l, c);  // erfc(|v| / sqrt2)
  return 0.5f * v * (v <= 0.0f ? e : 2.0f - e);     // erfc(-v / sqrt2)
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

// ---- transposed bf16 tiles through LDS as row pairs ------------------------------------------
// A 64x64 bf16 tile is held transposed in LDS as 32-bit pairs: the pair at (column c, p) holds
// the tile's elements (2p, c) and (2p + 1, c), i.e. two consecutive elements of transposed row c.
// A transposed row is 32 pairs (128 bytes); its groups of 4 pairs are XOR-swizzled by
// (c >> 2) & 7, which spreads the pair writes of lanes on neighbouring columns over the banks and
// keeps each group contiguous for one 16-byte read.
constexpr int kPairTileWords = 64 * 32;

__device__ __forceinline__ int pair_slot(int c, int p) { return c * 32 + (p ^ (((c >> 2) & 7) << 2)); }

// Writes the transposed tile (tile rows r0.., columns c0.. of a rows x cols source) to dst, whose
// row c0 + c holds source column c0 + c: 512 16-byte units (8 source rows of one column), two per
// lane of a 256-lane block, 8 lanes per transposed row.  Needs rows % 8 == 0 (16-byte aligned
// units, each wholly inside or outside the tensor); the caller has written every in-bounds pair
// and synchronised the block.
__device__ __forceinline__ void store_pair_tile_transposed(const uint32_t* __restrict__ tile, uint16_t* __restrict__ dst,
                                                           int64_t rows, int64_t cols, int64_t r0, int64_t c0) {
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int u = static_cast<int>(threadIdx.x) + 256 * k;
    const int c = u >> 3, g = u & 7;
    if (c0 + c < cols && r0 + 8 * g < rows) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(tile + pair_slot(c, 4 * g));
      *reinterpret_cast<u32x4*>(dst + (c0 + c) * rows + r0 + 8 * g) = v;
    }
  }
}

}  // namespace vdsl

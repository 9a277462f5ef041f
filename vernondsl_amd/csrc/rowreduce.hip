// Op class 3: row reductions (sum, max) + softmax, and column reductions, on gfx950.
//
// No reference code (the north-star op class).  Semantics, shared with the CPU oracle:
//   row_sum = sum_j x[j] accumulated in f64, rounded once to f32;
//   row_max = max_j x[j] (exact);
//   softmax[j] = e[j] / s,  e[j] = exp(x[j] - row_max) in f32,  s = f64 sum of e rounded to f32.
// (The register-resident kernels evaluate exp with the branch-free exp_fast of fmath.h, in its
// form for arguments <= 0, within a few ulp of the library expf that the generic kernel and the
// oracle use.)
// The register-resident kernels multiply by 1/s instead of dividing (within one ulp of e/s) and
// form their sums as f32 partials of 4 or 8 elements added into f64 accumulators (f32 rows) or,
// for bf16 rows, as f32 sums across the wave (DPP) added in f64 across waves: sums within a few
// ulp of the f64 accumulation, far inside the op's 1e-5 (f32) / 1e-2 (bf16) tolerances, for less
// VALU work per element, which bounds the bf16 kernels.
//
// Mapping: one 64-lane wavefront owns one row and keeps it in VGPRs, so x is read from HBM once
// and softmax written once (the HBM roofline's minimum traffic).  Lane l holds the 16-byte
// vectors v*64 + l, v < NV, so every load/store instruction of a wave covers 1 KiB contiguous.
// Reductions stay inside the wave (xor butterflies), so a 256-thread block is 4 independent
// rows and needs no LDS and no barrier.  Widths that are not one of the register-resident
// shapes use a 3-pass streaming kernel (max/sum, exp-sum, write) with the same arithmetic.

#include "common.h"

namespace vdsl {
namespace {

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// Wave reductions through DPP (no LDS round trip): a butterfly inside each row of 16 lanes
// (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror), then the four rows' values read
// as scalars and combined.  Every lane gets the result.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row_lane(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_f32<0xB1>(v);
  v += dpp_f32<0x4E>(v);
  v += dpp_f32<0x141>(v);
  v += dpp_f32<0x140>(v);
  return (row_lane(v, 0) + row_lane(v, 16)) + (row_lane(v, 32) + row_lane(v, 48));
}
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  v = fmaxf(v, dpp_f32<0x141>(v));
  v = fmaxf(v, dpp_f32<0x140>(v));
  return fmaxf(fmaxf(row_lane(v, 0), row_lane(v, 16)), fmaxf(row_lane(v, 32), row_lane(v, 48)));
}

// exp_fast for n <= 0 (softmax's x - max): 2^t cannot overflow there, so only a non-finite t
// (n = -inf or NaN) skips the correction.  The same value as exp_fast for every such n.
__device__ __forceinline__ float exp_nonpos(float n) {
  const float t = n * 1.4426950408889634f;
  float r = __builtin_fmaf(n, 1.4426950408889634f, -t);
  r = __builtin_fmaf(n, 1.92596299e-08f, r);  // log2(e) - fl(log2(e))
  const float e = __builtin_amdgcn_exp2f(t);
  const float c = __builtin_fmaf(e, r * 0.6931471805599453f, e);
  return __builtin_isfinite(t) ? c : e;
}

// A wave's partial sum: f64 butterflies for f32 rows; for bf16 rows (outputs with 8 significant
// bits, bound by VALU work rather than HBM) the lanes' f32 partials meet in f32 through DPP.
template <int DT>
__device__ __forceinline__ double wave_partial_sum(float lane_part, double lane_part64) {
  if constexpr (DT == VDSL_BF16) return static_cast<double>(wave_sum_dpp(lane_part));
  else return wave_sum_f64(lane_part64);
}
template <int DT>
__device__ __forceinline__ float wave_partial_max(float v) {
  if constexpr (DT == VDSL_BF16) return wave_max_dpp(v);
  else return wave_max(v);
}

template <int DT>
struct Elem;
template <>
struct Elem<VDSL_F32> {
  static constexpr int kPerVec = 4;  // elements per 16-byte vector
  __device__ static __forceinline__ void unpack(const uint4& v, float (&o)[4]) {
    o[0] = __uint_as_float(v.x); o[1] = __uint_as_float(v.y); o[2] = __uint_as_float(v.z); o[3] = __uint_as_float(v.w);
  }
  __device__ static __forceinline__ uint4 pack(const float (&o)[4]) {
    return make_uint4(__float_as_uint(o[0]), __float_as_uint(o[1]), __float_as_uint(o[2]), __float_as_uint(o[3]));
  }
  __device__ static __forceinline__ float load1(const void* p, int64_t i) { return static_cast<const float*>(p)[i]; }
  __device__ static __forceinline__ void store1(void* p, int64_t i, float v) { static_cast<float*>(p)[i] = v; }
};
template <>
struct Elem<VDSL_BF16> {
  static constexpr int kPerVec = 8;
  __device__ static __forceinline__ void unpack(const uint4& v, float (&o)[8]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      o[2 * k] = __uint_as_float(w[k] << 16);
      o[2 * k + 1] = __uint_as_float(w[k] & 0xFFFF0000u);
    }
  }
  __device__ static __forceinline__ uint4 pack(const float (&o)[8]) {
    return make_uint4(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]), pack_bf16x2(o[4], o[5]), pack_bf16x2(o[6], o[7]));
  }
  __device__ static __forceinline__ float load1(const void* p, int64_t i) {
    return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  }
  __device__ static __forceinline__ void store1(void* p, int64_t i, float v) { static_cast<uint16_t*>(p)[i] = f32_to_bf16(v); }
};

// Register-resident row: NV 16-byte vectors per lane, cols = 64 * NV * E::kPerVec.
template <int DT, int NV>
__global__ __launch_bounds__(256) void row_softmax_resident(const void* __restrict__ x, float* __restrict__ row_sum,
                                                            float* __restrict__ row_max, void* __restrict__ sm,
                                                            int64_t rows) {
  using E = Elem<DT>;
  constexpr int PV = E::kPerVec;
  constexpr int64_t cols = 64 * NV * PV;
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint4* src = reinterpret_cast<const uint4*>(static_cast<const char*>(x) + row * cols * (DT == VDSL_F32 ? 4 : 2));

  float v[NV][PV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const u32x4 r = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + k * 64 + lane));
    E::unpack(make_uint4(r[0], r[1], r[2], r[3]), v[k]);
  }
  double s = 0.0;
  float fs = 0.0f;
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    float part = 0.0f;
#pragma unroll
    for (int e = 0; e < PV; ++e) {
      part += v[k][e];
      m = fmaxf(m, v[k][e]);
    }
    s += static_cast<double>(part);
    fs += part;
  }
  s = wave_partial_sum<DT>(fs, s);
  m = wave_partial_max<DT>(m);
  if (lane == 0) {
    if (row_sum) row_sum[row] = static_cast<float>(s);
    if (row_max) row_max[row] = m;
  }
  if (!sm) return;
  double es = 0.0;
  float fes = 0.0f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    float part = 0.0f;
#pragma unroll
    for (int e = 0; e < PV; ++e) {
      v[k][e] = exp_nonpos(v[k][e] - m);
      part += v[k][e];
    }
    es += static_cast<double>(part);
    fes += part;
  }
  const float inv = 1.0f / static_cast<float>(wave_partial_sum<DT>(fes, es));
  uint4* dst = reinterpret_cast<uint4*>(static_cast<char*>(sm) + row * cols * (DT == VDSL_F32 ? 4 : 2));
#pragma unroll
  for (int k = 0; k < NV; ++k) {
#pragma unroll
    for (int e = 0; e < PV; ++e) v[k][e] = v[k][e] * inv;
    const uint4 w = E::pack(v[k]);
    const u32x4 wv = {w.x, w.y, w.z, w.w};
    __builtin_nontemporal_store(wv, reinterpret_cast<u32x4*>(dst + k * 64 + lane));
  }
}

// Wide rows, one block per row: cols = 64 * WPR * NV * PV, the row held in the registers of WPR
// waves (NV 16-byte vectors per lane, lane l of wave w holding vectors (w NV + k) 64 + l).  Each
// wave reduces its part; the WPR partial sums (f64) and maxima meet in LDS and every wave adds
// them in the same order.  Against one wave per row (all of a 4096-wide f32 row in one wave's
// registers, 88 VGPRs, 5 waves per SIMD) the smaller per-lane share runs at full occupancy and a
// row's load-reduce-store chain is 8 times shorter: [16384][4096] f32 84 us against 93-96 us.
template <int DT, int NV, int WPR>
__global__ __launch_bounds__(64 * WPR) void row_softmax_split(const void* __restrict__ x, float* __restrict__ row_sum,
                                                              float* __restrict__ row_max, void* __restrict__ sm,
                                                              int64_t rows) {
  using E = Elem<DT>;
  constexpr int PV = E::kPerVec;
  constexpr int64_t cols = 64 * WPR * NV * PV;
  __shared__ double part_sum[WPR];
  __shared__ float part_max[WPR];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t row = blockIdx.x;
  const uint4* src = reinterpret_cast<const uint4*>(static_cast<const char*>(x) + row * cols * (DT == VDSL_F32 ? 4 : 2)) +
                     wave * NV * 64 + lane;

  float v[NV][PV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const u32x4 r = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + k * 64));
    E::unpack(make_uint4(r[0], r[1], r[2], r[3]), v[k]);
  }
  double s = 0.0;
  float fs = 0.0f;
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    float part = 0.0f;
#pragma unroll
    for (int e = 0; e < PV; ++e) {
      part += v[k][e];
      m = fmaxf(m, v[k][e]);
    }
    s += static_cast<double>(part);
    fs += part;
  }
  s = wave_partial_sum<DT>(fs, s);
  m = wave_partial_max<DT>(m);
  if (lane == 0) {
    part_sum[wave] = s;
    part_max[wave] = m;
  }
  __syncthreads();
  s = 0.0;
  m = -INFINITY;
#pragma unroll
  for (int w = 0; w < WPR; ++w) {
    s += part_sum[w];
    m = fmaxf(m, part_max[w]);
  }
  if (threadIdx.x == 0) {
    if (row_sum) row_sum[row] = static_cast<float>(s);
    if (row_max) row_max[row] = m;
  }
  if (!sm) return;
  double es = 0.0;
  float fes = 0.0f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    float part = 0.0f;
#pragma unroll
    for (int e = 0; e < PV; ++e) {
      v[k][e] = exp_nonpos(v[k][e] - m);
      part += v[k][e];
    }
    es += static_cast<double>(part);
    fes += part;
  }
  es = wave_partial_sum<DT>(fes, es);
  __syncthreads();  // every wave has read part_sum
  if (lane == 0) part_sum[wave] = es;
  __syncthreads();
  es = 0.0;
#pragma unroll
  for (int w = 0; w < WPR; ++w) es += part_sum[w];
  const float inv = 1.0f / static_cast<float>(es);
  uint4* dst = reinterpret_cast<uint4*>(static_cast<char*>(sm) + row * cols * (DT == VDSL_F32 ? 4 : 2)) + wave * NV * 64 + lane;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
#pragma unroll
    for (int e = 0; e < PV; ++e) v[k][e] = v[k][e] * inv;
    const uint4 w = E::pack(v[k]);
    const u32x4 wv = {w.x, w.y, w.z, w.w};
    __builtin_nontemporal_store(wv, reinterpret_cast<u32x4*>(dst + k * 64));
  }
}

// Any width: three streaming passes over the row with the same arithmetic.
template <int DT>
__global__ __launch_bounds__(256) void row_softmax_generic(const void* __restrict__ x, float* __restrict__ row_sum,
                                                           float* __restrict__ row_max, void* __restrict__ sm,
                                                           int64_t rows, int64_t cols) {
  using E = Elem<DT>;
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = row * cols;
  double s = 0.0;
  float m = -INFINITY;
  for (int64_t c = lane; c < cols; c += 64) {
    const float v = E::load1(x, base + c);
    s += static_cast<double>(v);
    m = fmaxf(m, v);
  }
  s = wave_sum_f64(s);
  m = wave_max(m);
  if (lane == 0) {
    if (row_sum) row_sum[row] = static_cast<float>(s);
    if (row_max) row_max[row] = m;
  }
  if (!sm) return;
  double es = 0.0;
  for (int64_t c = lane; c < cols; c += 64) es += static_cast<double>(expf(E::load1(x, base + c) - m));
  const float esf = static_cast<float>(wave_sum_f64(es));
  for (int64_t c = lane; c < cols; c += 64) E::store1(sm, base + c, expf(E::load1(x, base + c) - m) / esf);
}

// Column reductions: a block owns 64 columns; 4 row groups accumulate in f64 and are combined in
// a fixed order, so results do not depend on scheduling.
template <int DT>
__global__ __launch_bounds__(256) void col_reduce_kernel(const void* __restrict__ x, float* __restrict__ col_sum,
                                                         float* __restrict__ col_max, int64_t rows, int64_t cols) {
  using E = Elem<DT>;
  __shared__ double ssum[4][64];
  __shared__ float smax[4][64];
  const int c_local = threadIdx.x & 63;
  const int g = threadIdx.x >> 6;
  const int64_t c = static_cast<int64_t>(blockIdx.x) * 64 + c_local;
  double s = 0.0;
  float m = -INFINITY;
  if (c < cols)
    for (int64_t r = g; r < rows; r += 4) {
      const float v = E::load1(x, r * cols + c);
      s += static_cast<double>(v);
      m = fmaxf(m, v);
    }
  ssum[g][c_local] = s;
  smax[g][c_local] = m;
  __syncthreads();
  if (g == 0 && c < cols) {
    const double t = ((ssum[0][c_local] + ssum[1][c_local]) + ssum[2][c_local]) + ssum[3][c_local];
    const float mm = fmaxf(fmaxf(smax[0][c_local], smax[1][c_local]), fmaxf(smax[2][c_local], smax[3][c_local]));
    if (col_sum) col_sum[c] = static_cast<float>(t);
    if (col_max) col_max[c] = mm;
  }
}

template <int DT>
int launch_rows(const void* x, float* rs, float* rm, void* sm, int64_t rows, int64_t cols, hipStream_t st) {
  constexpr int PV = Elem<DT>::kPerVec;
  // Rows of 8, 16 or 32 vectors per 64 lanes: one block per row.  f32: 4 waves of 2 vectors per
  // lane or 8 waves of 2 or 4; bf16 (VALU-bound): 4 vectors per lane in 2, 4 or 8 waves, which
  // halves the reductions per element at 4096 columns (42.9 us against 45.7 for 2 vectors in 4
  // waves on [16384][4096], with the DPP reductions).
  if (cols == 64 * 8 * PV || cols == 64 * 16 * PV || cols == 64 * 32 * PV) {
    if (rows > 0x7fffffff) return fail(VDSL_ERR_UNSUPPORTED, "too many rows");
    const dim3 g(static_cast<unsigned>(rows));
    if constexpr (DT == VDSL_BF16) {
      if (cols == 64 * 8 * PV) hipLaunchKernelGGL((row_softmax_split<DT, 4, 2>), g, dim3(128), 0, st, x, rs, rm, sm, rows);
      else if (cols == 64 * 16 * PV) hipLaunchKernelGGL((row_softmax_split<DT, 4, 4>), g, dim3(256), 0, st, x, rs, rm, sm, rows);
      else hipLaunchKernelGGL((row_softmax_split<DT, 4, 8>), g, dim3(512), 0, st, x, rs, rm, sm, rows);
    } else {
      if (cols == 64 * 8 * PV) hipLaunchKernelGGL((row_softmax_split<DT, 2, 4>), g, dim3(256), 0, st, x, rs, rm, sm, rows);
      else if (cols == 64 * 16 * PV) hipLaunchKernelGGL((row_softmax_split<DT, 2, 8>), g, dim3(512), 0, st, x, rs, rm, sm, rows);
      else hipLaunchKernelGGL((row_softmax_split<DT, 4, 8>), g, dim3(512), 0, st, x, rs, rm, sm, rows);
    }
    return check_launch("row_softmax_split");
  }
  const int64_t blocks = (rows + 3) / 4;
  if (blocks > 0x7fffffff) return fail(VDSL_ERR_UNSUPPORTED, "too many rows");
  const dim3 grid(static_cast<unsigned>(blocks)), block(256);
  switch (cols) {
#define VDSL_ROW_CASE(NV) \
  case 64 * NV * PV: hipLaunchKernelGGL((row_softmax_resident<DT, NV>), grid, block, 0, st, x, rs, rm, sm, rows); break;
    VDSL_ROW_CASE(1)
    VDSL_ROW_CASE(2)
    VDSL_ROW_CASE(4)
#undef VDSL_ROW_CASE
    default:
      hipLaunchKernelGGL((row_softmax_generic<DT>), grid, block, 0, st, x, rs, rm, sm, rows, cols);
  }
  return check_launch("row_softmax");
}

}  // namespace
}  // namespace vdsl

using namespace vdsl;

extern "C" int vdsl_op_row_reduce_softmax(vdsl_queue q, int64_t rows, int64_t cols, int32_t dtype, vdsl_buffer x,
                                          vdsl_buffer row_sum, vdsl_buffer row_max, vdsl_buffer softmax) {
  VDSL_TRY(enter_queue(q));
  if (rows < 0 || cols < 0) return fail(VDSL_ERR_INVALID_ARG, "negative shape");
  if (dtype != VDSL_F32 && dtype != VDSL_BF16) return fail(VDSL_ERR_UNSUPPORTED, "softmax dtype must be f32 or bf16");
  const size_t es = dtype_size(dtype);
  VDSL_TRY(check_buffer(q, x, nbytes(rows, cols, es), "x", false));
  if (row_sum) VDSL_TRY(check_buffer(q, row_sum, nbytes(rows, 4), "row_sum", true));
  if (row_max) VDSL_TRY(check_buffer(q, row_max, nbytes(rows, 4), "row_max", true));
  if (softmax) VDSL_TRY(check_buffer(q, softmax, nbytes(rows, cols, es), "softmax", true));
  if (rows == 0) return VDSL_OK;
  if (cols == 0) {
    // sum of an empty row is 0 and its max is -inf; nothing else to write
    if (row_sum) VDSL_TRY(vdsl_buffer_fill_u32(q, row_sum, 0, static_cast<size_t>(rows) * 4, 0u));
    if (row_max) VDSL_TRY(vdsl_buffer_fill_u32(q, row_max, 0, static_cast<size_t>(rows) * 4, 0xFF800000u));
    return VDSL_OK;
  }
  float* rs = row_sum ? static_cast<float*>(row_sum->ptr) : nullptr;
  float* rm = row_max ? static_cast<float*>(row_max->ptr) : nullptr;
  void* sm = softmax ? softmax->ptr : nullptr;
  if (dtype == VDSL_F32) return launch_rows<VDSL_F32>(x->ptr, rs, rm, sm, rows, cols, q->stream);
  return launch_rows<VDSL_BF16>(x->ptr, rs, rm, sm, rows, cols, q->stream);
}

extern "C" int vdsl_op_col_reduce(vdsl_queue q, int64_t rows, int64_t cols, int32_t dtype, vdsl_buffer x,
                                  vdsl_buffer col_sum, vdsl_buffer col_max) {
  VDSL_TRY(enter_queue(q));
  if (rows < 0 || cols < 0) return fail(VDSL_ERR_INVALID_ARG, "negative shape");
  if (dtype != VDSL_F32 && dtype != VDSL_BF16) return fail(VDSL_ERR_UNSUPPORTED, "col_reduce dtype must be f32 or bf16");
  VDSL_TRY(check_buffer(q, x, nbytes(rows, cols, dtype_size(dtype)), "x", false));
  if (col_sum) VDSL_TRY(check_buffer(q, col_sum, nbytes(cols, 4), "col_sum", true));
  if (col_max) VDSL_TRY(check_buffer(q, col_max, nbytes(cols, 4), "col_max", true));
  if (cols == 0) return VDSL_OK;
  const int64_t blocks = (cols + 63) / 64;
  float* cs = col_sum ? static_cast<float*>(col_sum->ptr) : nullptr;
  float* cm = col_max ? static_cast<float*>(col_max->ptr) : nullptr;
  if (dtype == VDSL_F32)
    hipLaunchKernelGGL((col_reduce_kernel<VDSL_F32>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, q->stream, x->ptr, cs, cm, rows, cols);
  else
    hipLaunchKernelGGL((col_reduce_kernel<VDSL_BF16>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, q->stream, x->ptr, cs, cm, rows, cols);
  return check_launch("col_reduce_kernel");
}

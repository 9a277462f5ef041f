// Op class 2: fused elementwise / broadcast map chains on gfx950.
//
// The reference has no elementwise code (the only compute is fractal.py:16-25); this op class
// comes from the north-star spec.  A chain is a straight-line register program
// (vdsl_map_instr, include/vdsl.h) evaluated once per output element, so a whole expression
// such as tanh(a*x + b) * exp(-x^2) + bias[col] costs one HBM read of each operand and one
// write of the result.
//
// Mapping: the tensor is [rows][cols] row-major.  A block of 256 lanes spans 256 float4 column
// slots (1024 columns) of R consecutive rows, so every wave reads 1 KiB contiguous per row with
// 16-byte loads, a row-broadcast operand (VDSL_BCAST_ROW, e.g. a bias) is loaded once per lane
// and reused for all R rows, and all R rows' loads are issued before any arithmetic.
//
// One interpreter serves two instantiations:
//   - generic: the program is a kernel argument, executed with a uniform (scalar-branch)
//     dispatch and uniform register indices;
//   - fixed: the program is a compile-time table (ProgTanhExpBias below); the same interpreter is
//     fully unrolled and constant-folded into straight-line code.  A runtime chain whose opcodes,
//     register indices and input broadcasts equal a table entry runs this version; its
//     immediates still come from the runtime program.

#include <type_traits>
#include <utility>

#include "common.h"

namespace vdsl {
namespace {

struct MapProg {
  vdsl_map_instr code[VDSL_MAP_MAX_INSTR];
  int32_t n;
  int32_t out_reg;
};

struct MapIn {
  const float* p[VDSL_MAP_MAX_INPUTS];
  int32_t bcast[VDSL_MAP_MAX_INPUTS];
  int32_t n;
};

// tanh in f32 without the argument-range branches of the library tanhf (which diverge per lane):
//   |u| < 0.4:  Taylor series u (1 + z (c1 + z (c2 + ... + z c5))), z = u^2, with the exact
//               coefficients c_k of tanh's expansion (-1/3, 2/15, -17/315, 62/2835, -1382/155925);
//               the first omitted term is below 1e-7 of the result there;
//   otherwise:  sign(u) (1 - 2 / (e^(2|u|) + 1)), whose cancellation costs at most a few ulp once
//               tanh(|u|) >= 0.38 (e^(2|u|) overflows to inf for large |u|, giving exactly 1).
// Both branches are evaluated and selected.  Relative error against tanh in f64: below 1.8e-7 in
// an f32 emulation of the same steps, plus the hardware exp2 / reciprocal (1 ulp each).
__device__ __forceinline__ float tanh_fast(float u) {
  const float a = fabsf(u);
  const float z = u * u;
  float p = -0.0088632358238101f;                  // -1382/155925
  p = __builtin_fmaf(p, z, 0.021869488060474396f);   // 62/2835
  p = __builtin_fmaf(p, z, -0.05396825447678566f);   // -17/315
  p = __builtin_fmaf(p, z, 0.13333334028720856f);    // 2/15
  p = __builtin_fmaf(p, z, -0.3333333432674408f);    // -1/3
  const float small = __builtin_fmaf(u * z, p, u);
  const float e = __builtin_amdgcn_exp2f(a * 2.8853900817779268f);  // e^(2|u|) = 2^(2|u| log2 e)
  const float big = __builtin_copysignf(__builtin_fmaf(-2.0f, __builtin_amdgcn_rcpf(e + 1.0f), 1.0f), u);
  return a < 0.4f ? small : big;
}

__device__ __forceinline__ float apply_op(int op, float a, float b, float c, float imm) {
  switch (op) {
    case VDSL_MAP_CONST: return imm;
    case VDSL_MAP_MOV: return a;
    case VDSL_MAP_NEG: return -a;
    case VDSL_MAP_ABS: return fabsf(a);
    case VDSL_MAP_SQUARE: return a * a;
    case VDSL_MAP_EXP: return exp_fast(a);
    case VDSL_MAP_LOG: return logf(a);
    case VDSL_MAP_TANH: return tanh_fast(a);
    case VDSL_MAP_SIGMOID: return 1.0f / (1.0f + exp_fast(-a));
    case VDSL_MAP_RELU: return a > 0.0f ? a : 0.0f;
    case VDSL_MAP_SQRT: return sqrtf(a);
    case VDSL_MAP_RECIP: return 1.0f / a;
    case VDSL_MAP_ADD: return a + b;
    case VDSL_MAP_SUB: return a - b;
    case VDSL_MAP_MUL: return a * b;
    case VDSL_MAP_DIV: return a / b;
    case VDSL_MAP_MAX: return fmaxf(a, b);
    case VDSL_MAP_MIN: return fminf(a, b);
    case VDSL_MAP_FMA: return __builtin_fmaf(a, b, c);
    case VDSL_MAP_MUL_IMM: return a * imm;
    case VDSL_MAP_ADD_IMM: return a + imm;
    default: return 0.0f;
  }
}

// Compile-time programs.  Each lists its opcodes/registers, input broadcasts and output register.
struct ProgTanhExpBias {
  // y = tanh(x * a + b) * exp(-(x * x)) + bias[col]   (input 0 = x: FULL, input 1 = bias: ROW),
  // register-allocated exactly as vernondsl_amd.mapchain.compile emits it.
  static constexpr int n = 10;
  static constexpr int n_inputs = 2;
  static constexpr int out_reg = 0;
  __host__ __device__ static constexpr int bcast_of(int k) { return k == 1 ? VDSL_BCAST_ROW : VDSL_BCAST_FULL; }
  static constexpr vdsl_map_instr code[VDSL_MAP_MAX_INSTR] = {
      {VDSL_MAP_LOAD, 0, 0, 0, 0, {0, 0, 0}, 0.f},     // r0 = x
      {VDSL_MAP_MUL_IMM, 1, 0, 0, 0, {0, 0, 0}, 0.f},  // r1 = r0 * a
      {VDSL_MAP_ADD_IMM, 1, 1, 0, 0, {0, 0, 0}, 0.f},  // r1 = r1 + b
      {VDSL_MAP_TANH, 1, 1, 0, 0, {0, 0, 0}, 0.f},     // r1 = tanh(r1)
      {VDSL_MAP_SQUARE, 0, 0, 0, 0, {0, 0, 0}, 0.f},   // r0 = r0 * r0
      {VDSL_MAP_NEG, 0, 0, 0, 0, {0, 0, 0}, 0.f},      // r0 = -r0
      {VDSL_MAP_EXP, 0, 0, 0, 0, {0, 0, 0}, 0.f},      // r0 = exp(r0)
      {VDSL_MAP_MUL, 0, 1, 0, 0, {0, 0, 0}, 0.f},      // r0 = r1 * r0
      {VDSL_MAP_LOAD, 1, 1, 0, 0, {0, 0, 0}, 0.f},     // r1 = bias[col]
      {VDSL_MAP_ADD, 0, 0, 1, 0, {0, 0, 0}, 0.f},      // r0 = r0 + r1
  };
};

struct GenericProgram {};  // marker: program comes from the kernel argument

template <int VEC>
struct Vec;
template <>
struct Vec<4> {
  using T = float4;
  __device__ static __forceinline__ void to(const T& v, float (&o)[4]) { o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w; }
  __device__ static __forceinline__ T from(const float (&o)[4]) { return make_float4(o[0], o[1], o[2], o[3]); }
};
template <>
struct Vec<1> {
  using T = float;
  __device__ static __forceinline__ void to(const T& v, float (&o)[1]) { o[0] = v; }
  __device__ static __forceinline__ T from(const float (&o)[1]) { return o[0]; }
};

// Loads input k for a VEC-wide element group at (row, col).  IDX is the index type of the launch
// (32-bit whenever every element offset fits, which saves the 64-bit address arithmetic).
template <int VEC, class IDX>
__device__ __forceinline__ void load_input(const float* __restrict__ p, int bcast, IDX row, IDX col, IDX cols,
                                           float (&o)[VEC]) {
  using V = Vec<VEC>;
  if (bcast == VDSL_BCAST_FULL) {
    // Streamed once: a nontemporal load keeps it from displacing reused data (the broadcast
    // operands) in the caches.
    if constexpr (VEC == 4) {
      const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p + row * cols + col));
      o[0] = v[0]; o[1] = v[1]; o[2] = v[2]; o[3] = v[3];
    } else {
      o[0] = __builtin_nontemporal_load(p + row * cols + col);
    }
  } else if (bcast == VDSL_BCAST_ROW) {
    V::to(*reinterpret_cast<const typename V::T*>(p + col), o);
  } else {
    const float s = (bcast == VDSL_BCAST_COL) ? p[row] : p[0];
#pragma unroll
    for (int k = 0; k < VEC; ++k) o[k] = s;
  }
}

// Inputs whose value does not depend on the row (broadcast along rows, or a scalar).
__device__ __forceinline__ bool row_invariant(int bcast) { return bcast == VDSL_BCAST_ROW || bcast == VDSL_BCAST_SCALAR; }

template <class P, int VEC, int PC>
__device__ __forceinline__ void fixed_step(const MapProg& rt, const float (&in)[VDSL_MAP_MAX_INPUTS][VEC],
                                           float (&r)[VDSL_MAP_MAX_REGS][VEC]) {
  constexpr vdsl_map_instr s = P::code[PC];
  if constexpr (s.op == VDSL_MAP_LOAD) {
#pragma unroll
    for (int k = 0; k < VEC; ++k) r[s.dst][k] = in[s.a][k];
  } else {
    const float imm = rt.code[PC].imm;
#pragma unroll
    for (int k = 0; k < VEC; ++k) r[s.dst][k] = apply_op(s.op, r[s.a][k], r[s.b][k], r[s.c][k], imm);
  }
}

template <class P, int VEC, int... PC>
__device__ __forceinline__ void run_fixed(const MapProg& rt, const float (&in)[VDSL_MAP_MAX_INPUTS][VEC],
                                          float (&r)[VDSL_MAP_MAX_REGS][VEC], std::integer_sequence<int, PC...>) {
  (fixed_step<P, VEC, PC>(rt, in, r), ...);
}

template <class P, int VEC>
__device__ __forceinline__ void run_program(const MapProg& rt, const float (&in)[VDSL_MAP_MAX_INPUTS][VEC],
                                            float (&r)[VDSL_MAP_MAX_REGS][VEC]) {
  if constexpr (!std::is_same<P, GenericProgram>::value) {
    run_fixed<P, VEC>(rt, in, r, std::make_integer_sequence<int, P::n>{});
  } else {
#pragma unroll 1
    for (int pc = 0; pc < rt.n; ++pc) {
      const vdsl_map_instr s = rt.code[pc];
      if (s.op == VDSL_MAP_LOAD) {
#pragma unroll
        for (int k = 0; k < VEC; ++k) r[s.dst][k] = in[s.a][k];
      } else {
        float t[VEC];
#pragma unroll
        for (int k = 0; k < VEC; ++k) t[k] = apply_op(s.op, r[s.a][k], r[s.b][k], r[s.c][k], s.imm);
#pragma unroll
        for (int k = 0; k < VEC; ++k) r[s.dst][k] = t[k];
      }
    }
  }
}

// Broadcast mode of input k: a compile-time constant for fixed programs.
template <class P>
__device__ __forceinline__ int input_bcast(const MapIn& in, int k) {
  if constexpr (std::is_same<P, GenericProgram>::value) return in.bcast[k];
  else return P::bcast_of(k);
}

// R rows of one thread's column group: every row's loads, then each row's program and store.
// GUARD: rows past `rows` are skipped (the last, partial group of a launch).
template <class P, int VEC, int R, bool GUARD, class IDX>
__device__ __forceinline__ void map_chain_rows(const MapProg& rt, const MapIn& in, float* __restrict__ out, IDX rows, IDX cols,
                                               IDX row0, IDX col, int n_in, int out_reg,
                                               const float (&vfix)[VDSL_MAP_MAX_INPUTS][VEC]) {
  float vin[R][VDSL_MAP_MAX_INPUTS][VEC];
#pragma unroll
  for (int u = 0; u < R; ++u) {
    const IDX row = row0 + u;
    if (!GUARD || row < rows) {
#pragma unroll
      for (int k = 0; k < VDSL_MAP_MAX_INPUTS; ++k) {
        if (k < n_in) {
          const int bc = input_bcast<P>(in, k);
          if (row_invariant(bc)) {
#pragma unroll
            for (int e = 0; e < VEC; ++e) vin[u][k][e] = vfix[k][e];
          } else {
            load_input<VEC, IDX>(in.p[k], bc, row, col, cols, vin[u][k]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int u = 0; u < R; ++u) {
    const IDX row = row0 + u;
    if (!GUARD || row < rows) {
      float r[VDSL_MAP_MAX_REGS][VEC];
#pragma unroll
      for (int g = 0; g < VDSL_MAP_MAX_REGS; ++g)
#pragma unroll
        for (int k = 0; k < VEC; ++k) r[g][k] = 0.0f;
      run_program<P, VEC>(rt, vin[u], r);
      if constexpr (VEC == 4) {
        const f32x4 v = {r[out_reg][0], r[out_reg][1], r[out_reg][2], r[out_reg][3]};
        __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(out + row * cols + col));
      } else {
        __builtin_nontemporal_store(r[out_reg][0], out + row * cols + col);
      }
    }
  }
}

// One thread per VEC-wide column group; the block's threads cover 256 VEC columns and step over R
// rows at a time (all R rows' loads issued before any compute).  Row-invariant inputs are loaded
// once per thread, not once per row.
template <class P, int VEC, int R, class IDX>
__global__ __launch_bounds__(256) void map_chain_kernel(MapProg rt, MapIn in, float* __restrict__ out, IDX rows, IDX cols) {
  const IDX col = (static_cast<IDX>(blockIdx.x) * 256 + static_cast<IDX>(threadIdx.x)) * VEC;
  if (col >= cols) return;
  int n_in, out_reg;
  if constexpr (std::is_same<P, GenericProgram>::value) {
    n_in = in.n;
    out_reg = rt.out_reg;
  } else {
    n_in = P::n_inputs;
    out_reg = P::out_reg;
  }
  float vfix[VDSL_MAP_MAX_INPUTS][VEC];
#pragma unroll
  for (int k = 0; k < VDSL_MAP_MAX_INPUTS; ++k) {
    if (k < n_in) {
      const int bc = input_bcast<P>(in, k);
      if (row_invariant(bc)) load_input<VEC, IDX>(in.p[k], bc, IDX(0), col, cols, vfix[k]);
    }
  }

  for (IDX row0 = static_cast<IDX>(blockIdx.y) * R; row0 < rows; row0 += static_cast<IDX>(gridDim.y) * R) {
    // A whole group of R rows takes the path without per-row guards: with them the compiler
    // waits for every row's loads before computing the first row.
    if (row0 + R <= rows) map_chain_rows<P, VEC, R, false>(rt, in, out, rows, cols, row0, col, n_in, out_reg, vfix);
    else map_chain_rows<P, VEC, R, true>(rt, in, out, rows, cols, row0, col, n_in, out_reg, vfix);
  }
}

template <class P>
bool matches(const MapProg& rt, const MapIn& in) {
  if (rt.n != P::n || in.n != P::n_inputs || rt.out_reg != P::out_reg) return false;
  for (int k = 0; k < P::n_inputs; ++k)
    if (in.bcast[k] != P::bcast_of(k)) return false;
  for (int pc = 0; pc < P::n; ++pc) {
    const vdsl_map_instr& a = rt.code[pc];
    const vdsl_map_instr& b = P::code[pc];
    if (a.op != b.op || a.dst != b.dst) return false;
    // Compare only the operand fields the opcode reads.
    switch (a.op) {
      case VDSL_MAP_CONST: break;
      case VDSL_MAP_LOAD:
      case VDSL_MAP_MOV: case VDSL_MAP_NEG: case VDSL_MAP_ABS: case VDSL_MAP_SQUARE: case VDSL_MAP_EXP:
      case VDSL_MAP_LOG: case VDSL_MAP_TANH: case VDSL_MAP_SIGMOID: case VDSL_MAP_RELU: case VDSL_MAP_SQRT:
      case VDSL_MAP_RECIP: case VDSL_MAP_MUL_IMM: case VDSL_MAP_ADD_IMM:
        if (a.a != b.a) return false;
        break;
      case VDSL_MAP_FMA:
        if (a.a != b.a || a.b != b.b || a.c != b.c) return false;
        break;
      default:
        if (a.a != b.a || a.b != b.b) return false;
    }
  }
  return true;
}

// 32-bit indices when every offset the kernel forms (row * cols + col, and row0 plus a grid's
// worth of rows) stays far below 2^31.
template <class P, int VEC, int R>
int launch(const MapProg& rt, const MapIn& in, float* out, int64_t rows, int64_t cols, hipStream_t s) {
  const int64_t slots = (cols + VEC - 1) / VEC;
  const int64_t gx = (slots + 255) / 256;
  int64_t gy = (rows + R - 1) / R;
  if (gy > 65535) gy = 65535;
  if (gx > 0x7fffffff) return fail(VDSL_ERR_UNSUPPORTED, "map chain: cols too large");
  const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy));
  if (rows * (cols + 256 * VEC) <= (int64_t{1} << 30) && rows <= (int64_t{1} << 30))
    hipLaunchKernelGGL((map_chain_kernel<P, VEC, R, int32_t>), grid, dim3(256), 0, s, rt, in, out, static_cast<int32_t>(rows),
                       static_cast<int32_t>(cols));
  else
    hipLaunchKernelGGL((map_chain_kernel<P, VEC, R, int64_t>), grid, dim3(256), 0, s, rt, in, out, rows, cols);
  return check_launch("map_chain_kernel");
}

}  // namespace
}  // namespace vdsl

using namespace vdsl;

extern "C" int vdsl_op_map_chain(vdsl_queue q, int64_t rows, int64_t cols, const vdsl_map_instr* code, int32_t n_instr,
                                 const vdsl_map_input* inputs, int32_t n_inputs, int32_t out_reg, vdsl_buffer out) {
  VDSL_TRY(enter_queue(q));
  if (rows < 0 || cols < 0) return fail(VDSL_ERR_INVALID_ARG, "negative shape");
  if (n_instr < 0 || n_instr > VDSL_MAP_MAX_INSTR) return fail(VDSL_ERR_INVALID_ARG, "n_instr out of range [0, 32]");
  if (n_inputs < 0 || n_inputs > VDSL_MAP_MAX_INPUTS) return fail(VDSL_ERR_INVALID_ARG, "n_inputs out of range [0, 4]");
  if (out_reg < 0 || out_reg >= VDSL_MAP_MAX_REGS) return fail(VDSL_ERR_INVALID_ARG, "out_reg out of range");
  if (n_instr && !code) return fail(VDSL_ERR_INVALID_ARG, "code is null");
  if (n_inputs && !inputs) return fail(VDSL_ERR_INVALID_ARG, "inputs is null");
  VDSL_TRY(check_buffer(q, out, nbytes(rows, cols, 4), "out", true));
  const int64_t n = rows * cols;  // no overflow: rows * cols * 4 fits size_t (checked above)

  MapProg rt{};
  rt.n = n_instr;
  rt.out_reg = out_reg;
  for (int pc = 0; pc < n_instr; ++pc) {
    const vdsl_map_instr& s = code[pc];
    if (s.op < VDSL_MAP_LOAD || s.op > VDSL_MAP_ADD_IMM)
      return fail(VDSL_ERR_INVALID_ARG, "instruction " + std::to_string(pc) + ": unknown opcode " + std::to_string(s.op));
    if (s.dst >= VDSL_MAP_MAX_REGS || s.b >= VDSL_MAP_MAX_REGS || s.c >= VDSL_MAP_MAX_REGS)
      return fail(VDSL_ERR_INVALID_ARG, "instruction " + std::to_string(pc) + ": register out of range");
    if (s.op == VDSL_MAP_LOAD ? s.a >= n_inputs : s.a >= VDSL_MAP_MAX_REGS)
      return fail(VDSL_ERR_INVALID_ARG, "instruction " + std::to_string(pc) + ": operand out of range");
    rt.code[pc] = s;
  }
  MapIn in{};
  in.n = n_inputs;
  for (int k = 0; k < n_inputs; ++k) {
    const vdsl_map_input& d = inputs[k];
    if (d.dtype != VDSL_F32) return fail(VDSL_ERR_UNSUPPORTED, "map chain inputs must be f32");
    if (d.bcast < VDSL_BCAST_FULL || d.bcast > VDSL_BCAST_SCALAR) return fail(VDSL_ERR_INVALID_ARG, "unknown broadcast");
    const int64_t need = d.bcast == VDSL_BCAST_FULL ? n : d.bcast == VDSL_BCAST_ROW ? cols : d.bcast == VDSL_BCAST_COL ? rows : 1;
    std::string name = "input" + std::to_string(k);
    VDSL_TRY(check_buffer(q, d.buf, nbytes(need, 4), name.c_str(), false));
    in.p[k] = static_cast<const float*>(d.buf->ptr);
    in.bcast[k] = d.bcast;
  }
  if (n == 0) return VDSL_OK;
  float* o = static_cast<float*>(out->ptr);
  // 16-byte vectors need cols % 4 == 0 and 16-byte aligned bases (hipMalloc gives 256).
  const bool vec4 = (cols % 4) == 0;
  if (vec4 && matches<ProgTanhExpBias>(rt, in)) return launch<ProgTanhExpBias, 4, 2>(rt, in, o, rows, cols, q->stream);
  if (vec4) return launch<GenericProgram, 4, 1>(rt, in, o, rows, cols, q->stream);
  return launch<GenericProgram, 1, 1>(rt, in, o, rows, cols, q->stream);
}

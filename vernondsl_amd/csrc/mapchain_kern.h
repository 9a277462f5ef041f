// Device side of op class 2 (fused elementwise / broadcast map chains), shared by the kernels
// compiled with the library (map_chain.hip) and the kernels map_chain.hip compiles at run time for
// one program (its text is embedded in the library and handed to hiprtc with vdsl.h and fmath.h),
// so both compile the same source: a program compiled at run time gives the results of the
// interpreter bit for bit.  Uses nothing from the C++ standard library.
//
// A chain is a straight-line register program (vdsl_map_instr, include/vdsl.h) evaluated once per
// output element.  One interpreter serves two kinds of program P:
//   - GenericProgram: the program is a kernel argument, executed with a uniform (scalar-branch)
//     dispatch and uniform register indices;
//   - a fixed program: a compile-time table (struct with n, n_inputs, code[], bcast_of(k) and, for
//     vector programs, width_of(k), out_width, out_regs[]); the same interpreter is fully unrolled
//     and constant-folded into straight-line code.  Its immediates still come from the runtime
//     program (MapProg), so one compiled kernel serves every set of constants.
#pragma once

#include "fmath.h"
#include "vdsl.h"

namespace vdsl {

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

struct GenericProgram {};  // marker: the program comes from the kernel argument

template <class A, class B>
struct SameType {
  static constexpr bool value = false;
};
template <class A>
struct SameType<A, A> {
  static constexpr bool value = true;
};
template <class P>
struct IsGeneric {
  static constexpr bool value = SameType<P, GenericProgram>::value;
};

template <int... I>
struct Seq {};
template <int N, int... I>
struct MakeSeq : MakeSeq<N - 1, N - 1, I...> {};
template <int... I>
struct MakeSeq<0, I...> {
  using type = Seq<I...>;
};

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

// ---- scalar operands: VEC consecutive columns per lane ---------------------------------------------
// Mapping: the tensor is [rows][cols] row-major.  A block of 256 lanes spans 256 VEC-wide column
// slots of R consecutive rows, so every wave reads 1 KiB contiguous per row with 16-byte loads
// (VEC = 4), a row-broadcast operand (VDSL_BCAST_ROW, e.g. a bias) is loaded once per lane and
// reused for all R rows, and all R rows' loads are issued before any arithmetic.

// Loads input k for a VEC-wide element group at (row, col).  IDX is the index type of the launch
// (32-bit whenever every element offset fits, which saves the 64-bit address arithmetic).
template <int VEC, class IDX>
__device__ __forceinline__ void load_input(const float* __restrict__ p, int bcast, IDX row, IDX col, IDX cols,
                                           float (&o)[VEC]) {
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
    if constexpr (VEC == 4) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(p + col);
      o[0] = v[0]; o[1] = v[1]; o[2] = v[2]; o[3] = v[3];
    } else {
      o[0] = p[col];
    }
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
                                          float (&r)[VDSL_MAP_MAX_REGS][VEC], Seq<PC...>) {
  (fixed_step<P, VEC, PC>(rt, in, r), ...);
}

template <class P, int VEC>
__device__ __forceinline__ void run_program(const MapProg& rt, const float (&in)[VDSL_MAP_MAX_INPUTS][VEC],
                                            float (&r)[VDSL_MAP_MAX_REGS][VEC]) {
  if constexpr (!IsGeneric<P>::value) {
    run_fixed<P, VEC>(rt, in, r, typename MakeSeq<P::n>::type{});
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
  if constexpr (IsGeneric<P>::value) return in.bcast[k];
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
__device__ __forceinline__ void map_chain_body(const MapProg& rt, const MapIn& in, float* __restrict__ out, IDX rows, IDX cols) {
  const IDX col = (static_cast<IDX>(blockIdx.x) * 256 + static_cast<IDX>(threadIdx.x)) * VEC;
  if (col >= cols) return;
  int n_in, out_reg;
  if constexpr (IsGeneric<P>::value) {
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

// ---- vector operands (vdsl_op_map_chain_v) ---------------------------------------------------------
// Inputs are AoS vectors of 1..4 f32 components; every LOAD names its component, the output is a
// vector of chosen registers.  One element per lane (a lane's record is one 4-, 8-, 12- or 16-byte
// access, consecutive lanes on consecutive records), R rows per lane with all of their loads issued
// before any arithmetic.
struct MapVIn {
  const float* p[VDSL_MAP_MAX_INPUTS];
  int32_t bcast[VDSL_MAP_MAX_INPUTS];
  int32_t width[VDSL_MAP_MAX_INPUTS];
  int32_t n;
};

struct MapVOut {
  int32_t regs[4];
  int32_t width;
};

// Record e (width components) of input p into o[0..width).  Streamed (FULL) records use
// nontemporal loads, as in the scalar kernel.
template <class IDX>
__device__ __forceinline__ void load_record(const float* __restrict__ p, bool streamed, int width, IDX e, float (&o)[4]) {
  const float* q = p + e * width;
  if (width == 4) {
    const f32x4 v = streamed ? __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(q))
                             : *reinterpret_cast<const f32x4*>(q);
    o[0] = v[0]; o[1] = v[1]; o[2] = v[2]; o[3] = v[3];
  } else if (width == 2) {
    const f32x2_t v = streamed ? __builtin_nontemporal_load(reinterpret_cast<const f32x2_t*>(q))
                               : *reinterpret_cast<const f32x2_t*>(q);
    o[0] = v[0]; o[1] = v[1];
  } else if (width == 3) {
    o[0] = streamed ? __builtin_nontemporal_load(q) : q[0];
    o[1] = streamed ? __builtin_nontemporal_load(q + 1) : q[1];
    o[2] = streamed ? __builtin_nontemporal_load(q + 2) : q[2];
  } else {
    o[0] = streamed ? __builtin_nontemporal_load(q) : q[0];
  }
}

template <class P, int PC>
__device__ __forceinline__ void fixed_vstep(const MapProg& rt, const float (&e)[4 * VDSL_MAP_MAX_INPUTS],
                                            float (&r)[VDSL_MAP_MAX_REGS]) {
  constexpr vdsl_map_instr s = P::code[PC];
  if constexpr (s.op == VDSL_MAP_LOAD) r[s.dst] = e[4 * s.a + s.c];
  else r[s.dst] = apply_op(s.op, r[s.a], r[s.b], r[s.c], rt.code[PC].imm);
}

template <class P, int... PC>
__device__ __forceinline__ void run_fixed_v(const MapProg& rt, const float (&e)[4 * VDSL_MAP_MAX_INPUTS],
                                            float (&r)[VDSL_MAP_MAX_REGS], Seq<PC...>) {
  (fixed_vstep<P, PC>(rt, e, r), ...);
}

template <class P, int R, class IDX>
__device__ __forceinline__ void map_chain_v_body(const MapProg& rt, const MapVIn& in, const MapVOut& vo, float* __restrict__ out,
                                                 IDX rows, IDX cols) {
  constexpr bool G = IsGeneric<P>::value;
  const IDX col = static_cast<IDX>(blockIdx.x) * 256 + static_cast<IDX>(threadIdx.x);
  if (col >= cols) return;
  int n_in, ow;
  if constexpr (G) {
    n_in = in.n;
    ow = vo.width;
  } else {
    n_in = P::n_inputs;
    ow = P::out_width;
  }
  for (IDX row0 = static_cast<IDX>(blockIdx.y) * R; row0 < rows; row0 += static_cast<IDX>(gridDim.y) * R) {
    float vin[R][VDSL_MAP_MAX_INPUTS][4];
#pragma unroll
    for (int u = 0; u < R; ++u) {
      const IDX row = row0 + u;
      if (row < rows) {
#pragma unroll
        for (int k = 0; k < VDSL_MAP_MAX_INPUTS; ++k) {
          if (k < n_in) {
            int bc, w;
            if constexpr (G) {
              bc = in.bcast[k];
              w = in.width[k];
            } else {
              bc = P::bcast_of(k);
              w = P::width_of(k);
            }
            const IDX e = bc == VDSL_BCAST_FULL ? row * cols + col : bc == VDSL_BCAST_ROW ? col : bc == VDSL_BCAST_COL ? row : IDX(0);
            load_record<IDX>(in.p[k], bc == VDSL_BCAST_FULL, w, e, vin[u][k]);
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < R; ++u) {
      const IDX row = row0 + u;
      if (row < rows) {
        // This row's components as one flat array: with a uniform index into 16 registers the
        // compiler keeps it in VGPRs (indexing vin[u][a][c] directly spilled all R rows to scratch).
        float e[4 * VDSL_MAP_MAX_INPUTS];
#pragma unroll
        for (int k = 0; k < VDSL_MAP_MAX_INPUTS; ++k)
#pragma unroll
          for (int c = 0; c < 4; ++c) e[4 * k + c] = vin[u][k][c];
        float r[VDSL_MAP_MAX_REGS];
#pragma unroll
        for (int g = 0; g < VDSL_MAP_MAX_REGS; ++g) r[g] = 0.0f;
        int regs[4];
        if constexpr (G) {
#pragma unroll 1
          for (int pc = 0; pc < rt.n; ++pc) {
            const vdsl_map_instr s = rt.code[pc];
            r[s.dst] = s.op == VDSL_MAP_LOAD ? e[4 * s.a + s.c] : apply_op(s.op, r[s.a], r[s.b], r[s.c], s.imm);
          }
#pragma unroll
          for (int k = 0; k < 4; ++k) regs[k] = vo.regs[k];
        } else {
          run_fixed_v<P>(rt, e, r, typename MakeSeq<P::n>::type{});
#pragma unroll
          for (int k = 0; k < 4; ++k) regs[k] = P::out_regs[k];
        }
        float* o = out + (row * cols + col) * ow;
        if (ow == 4) {
          const f32x4 v = {r[regs[0]], r[regs[1]], r[regs[2]], r[regs[3]]};
          __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(o));
        } else if (ow == 2) {
          const f32x2_t v = {r[regs[0]], r[regs[1]]};
          __builtin_nontemporal_store(v, reinterpret_cast<f32x2_t*>(o));
        } else {
          for (int k = 0; k < ow; ++k) __builtin_nontemporal_store(r[regs[k]], o + k);
        }
      }
    }
  }
}

}  // namespace vdsl

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

// ---- vector and matrix operands (vdsl_op_map_chain_v) -----------------------------------------------
// Inputs are AoS records of 1..4 f32 components (vectors) or 4, 9, 16 (mat2-4, row-major); every LOAD
// names its component, MATVEC / VECMAT multiply a matrix record by a vector held in registers, the
// output is a vector of chosen registers.  One element per lane (consecutive lanes on consecutive
// records), R rows per lane with all of their loads issued before any arithmetic.
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

// Matrix dimension of a record of w components (only matrix inputs reach the products: 4, 9, 16).
__host__ __device__ constexpr int mat_dim_of(int w) { return w == 16 ? 4 : w == 9 ? 3 : 2; }

// Record e (width components) of input p into o[0..width).  Streamed (FULL) records use
// nontemporal loads, as in the scalar kernel.  Records of 16 components (mat4) are four 16-byte
// loads (their bases are 64-byte aligned); 9-component records (mat3) are nine 4-byte loads.
template <class IDX, int S>
__device__ __forceinline__ void load_record(const float* __restrict__ p, bool streamed, int width, IDX e, float (&o)[S]) {
  const float* q = p + e * width;
  if (width == 4 || (S >= 16 && width == 16)) {
#pragma unroll
    for (int h = 0; h < (S >= 16 ? 4 : 1); ++h) {
      if (h * 4 < width) {
        const f32x4 v = streamed ? __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(q) + h)
                                 : reinterpret_cast<const f32x4*>(q)[h];
        o[4 * h] = v[0]; o[4 * h + 1] = v[1]; o[4 * h + 2] = v[2]; o[4 * h + 3] = v[3];
      }
    }
  } else if (width == 2) {
    const f32x2_t v = streamed ? __builtin_nontemporal_load(reinterpret_cast<const f32x2_t*>(q))
                               : *reinterpret_cast<const f32x2_t*>(q);
    o[0] = v[0]; o[1] = v[1];
  } else if (width == 3 || (S >= 9 && width == 9)) {
#pragma unroll
    for (int k = 0; k < (S >= 9 ? 9 : 3); ++k)
      if (k < width) o[k] = streamed ? __builtin_nontemporal_load(q + k) : q[k];
  } else {
    o[0] = streamed ? __builtin_nontemporal_load(q) : q[0];
  }
}

// Entry k (< 4) of a kernel-argument array, by compares: indexing the by-value argument struct with
// a run-time k copies it to scratch memory.
template <class T>
__device__ __forceinline__ T pick(const T (&a)[VDSL_MAP_MAX_INPUTS], int k) {
  return k == 0 ? a[0] : k == 1 ? a[1] : k == 2 ? a[2] : a[3];
}

// Element index of input k's record at (row, col) under its broadcast.
template <class IDX>
__device__ __forceinline__ IDX record_index(int bc, IDX row, IDX col, IDX cols) {
  return bc == VDSL_BCAST_FULL ? row * cols + col : bc == VDSL_BCAST_ROW ? col : bc == VDSL_BCAST_COL ? row : IDX(0);
}

// Components per input slot of the flat record array: 4 for vector-only programs, 16 when a
// program reads a mat3 or mat4 (a compile-time table fixes it; unused slots are dead code).
template <class P>
__host__ __device__ constexpr int slot_of() {
  int s = 4;
  for (int k = 0; k < P::n_inputs; ++k)
    if (P::width_of(k) > s) s = 16;
  return s;
}

template <class P, int S, int PC>
__device__ __forceinline__ void fixed_vstep(const MapProg& rt, const float (&e)[S * VDSL_MAP_MAX_INPUTS],
                                            float (&r)[VDSL_MAP_MAX_REGS]) {
  constexpr vdsl_map_instr s = P::code[PC];
  if constexpr (s.op == VDSL_MAP_LOAD) {
    r[s.dst] = e[S * s.a + s.c];
  } else if constexpr (s.op == VDSL_MAP_MATVEC || s.op == VDSL_MAP_VECMAT) {
    // linalg.matvec: ((0 + m0 v0) + m1 v1) + ..., each product and sum rounded (no contraction:
    // the library and run-time kernels are compiled with -ffp-contract=off)
    constexpr int n = mat_dim_of(P::width_of(s.a));
    constexpr int vr[4] = {s.b, s.ext[0], s.ext[1], s.ext[2]};
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < n; ++k) {
      const float m = e[S * s.a + (s.op == VDSL_MAP_MATVEC ? s.c * n + k : k * n + s.c)];
      acc = acc + m * r[vr[k]];
    }
    r[s.dst] = acc;
  } else {
    r[s.dst] = apply_op(s.op, r[s.a], r[s.b], r[s.c], rt.code[PC].imm);
  }
}

template <class P, int S, int... PC>
__device__ __forceinline__ void run_fixed_v(const MapProg& rt, const float (&e)[S * VDSL_MAP_MAX_INPUTS],
                                            float (&r)[VDSL_MAP_MAX_REGS], Seq<PC...>) {
  (fixed_vstep<P, S, PC>(rt, e, r), ...);
}

template <class P>
struct VSlot {
  static constexpr int value = slot_of<P>();
};
template <>
struct VSlot<GenericProgram> {
  static constexpr int value = 4;
};

// R rows' programs and stores for one lane's element (row0 + u, col), from the records in vin.
template <class P, int R, int S, class IDX>
__device__ __forceinline__ void map_chain_v_rows(const MapProg& rt, const MapVIn& in, const MapVOut& vo, float* __restrict__ out,
                                                 IDX rows, IDX cols, IDX row0, IDX col,
                                                 const float (&vin)[R][VDSL_MAP_MAX_INPUTS][S]) {
  constexpr bool G = IsGeneric<P>::value;
  int ow;
  if constexpr (G) ow = vo.width;
  else ow = P::out_width;
#pragma unroll
  for (int u = 0; u < R; ++u) {
    const IDX row = row0 + u;
    if (row < rows) {
      // This row's components as one flat array: with a uniform index into it the compiler keeps
      // it in VGPRs (indexing vin[u][a][c] directly spilled all R rows to scratch).
      float e[S * VDSL_MAP_MAX_INPUTS];
#pragma unroll
      for (int k = 0; k < VDSL_MAP_MAX_INPUTS; ++k)
#pragma unroll
        for (int c = 0; c < S; ++c) e[S * k + c] = vin[u][k][c];
      float r[VDSL_MAP_MAX_REGS];
#pragma unroll
      for (int g = 0; g < VDSL_MAP_MAX_REGS; ++g) r[g] = 0.0f;
      int regs[4];
      if constexpr (G) {
#pragma unroll 1
        for (int pc = 0; pc < rt.n; ++pc) {
          const vdsl_map_instr s = rt.code[pc];
          const bool mem = s.op == VDSL_MAP_MATVEC || s.op == VDSL_MAP_VECMAT || (s.op == VDSL_MAP_LOAD && pick(in.width, s.a) > S);
          if (s.op == VDSL_MAP_LOAD && !mem) {
            r[s.dst] = e[S * s.a + s.c];
          } else if (mem) {
            // components beyond the register-held slots, and matrix entries, come from memory (the
            // record is in the cache after its first use); a branch of its own keeps e in registers
            const int w = pick(in.width, s.a);
            const float* rec = pick(in.p, s.a) + record_index<IDX>(pick(in.bcast, s.a), row, col, cols) * w;
            if (s.op == VDSL_MAP_LOAD) {
              r[s.dst] = rec[s.c];
            } else {
              const int n = mat_dim_of(w);
              const int vr[4] = {s.b, s.ext[0], s.ext[1], s.ext[2]};
              float acc = 0.0f;
#pragma unroll
              for (int k = 0; k < 4; ++k) {
                if (k < n) {
                  const int ci = s.op == VDSL_MAP_MATVEC ? s.c * n + k : k * n + s.c;
                  acc = acc + rec[ci] * r[vr[k]];
                }
              }
              r[s.dst] = acc;
            }
          } else {
            r[s.dst] = apply_op(s.op, r[s.a], r[s.b], r[s.c], s.imm);
          }
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) regs[k] = vo.regs[k];
      } else {
        run_fixed_v<P, S>(rt, e, r, typename MakeSeq<P::n>::type{});
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

// ---- wide records through LDS -------------------------------------------------------------------------
// A FULL input of mat3 or mat4 records (36 or 64 bytes), loaded by each lane at its record's
// stride, makes every wave-wide load instruction touch 18-32 cache lines for 256-1024 useful
// bytes (the address unit coalesces only consecutive 16-byte accesses): measured 68% / 60% of the
// HBM rate for mat3 / mat4 times a vector.  A fixed program instead loads the block's 256 records
// of each such input per row as consecutive 16-byte units (unit t + 256 j by lane t: every
// instruction one contiguous 4 KiB), passes them through LDS and reads each lane's record from
// there.  mat4 records sit in LDS with their four 16-byte units permuted by (record >> 1) & 3, so
// that 8 consecutive lanes reading unit h of their records hit 8 distinct 16-byte bank groups;
// mat3 records (9 words, an odd stride) are conflict-free as they are.
template <class P>
__host__ __device__ constexpr bool staged_input(int k) {
  return k < P::n_inputs && P::bcast_of(k) == VDSL_BCAST_FULL && P::width_of(k) >= 9;
}

// Floats of one row's staged records (256 records of each staged input), and input k's offset.
template <class P>
__host__ __device__ constexpr int stage_offset(int k) {
  int f = 0;
  for (int j = 0; j < k; ++j)
    if (staged_input<P>(j)) f += 256 * P::width_of(j);
  return f;
}
template <class P>
__host__ __device__ constexpr int stage_floats() {
  return stage_offset<P>(VDSL_MAP_MAX_INPUTS);
}

// Rows per step of a program that stages records: four unless that needs more than 64 KiB of LDS.
template <class P>
__host__ __device__ constexpr int staged_rows(int r) {
  int n = r;
  while (n > 1 && n * stage_floats<P>() * 4 > 65536) --n;
  return n;
}

__device__ __forceinline__ int mat4_slot(int unit) {
  const int rec = unit >> 2;
  return (rec << 2) | ((unit & 3) ^ ((rec >> 1) & 3));
}

template <class P, int R, class IDX>
__device__ __forceinline__ void map_chain_v_staged(const MapProg& rt, const MapVIn& in, const MapVOut& vo, float* __restrict__ out,
                                                   IDX rows, IDX cols) {
  constexpr int S = VSlot<P>::value;
  constexpr int SF = stage_floats<P>();
  __shared__ f32x4 lds[R * SF / 4];
  const int t = threadIdx.x;
  const IDX col0 = static_cast<IDX>(blockIdx.x) * 256;
  const IDX col = col0 + t;
  for (IDX row0 = static_cast<IDX>(blockIdx.y) * R; row0 < rows; row0 += static_cast<IDX>(gridDim.y) * R) {
    float vin[R][VDSL_MAP_MAX_INPUTS][S];
    f32x4 unit[R][VDSL_MAP_MAX_INPUTS][4];
    // every row's loads first: staged inputs as contiguous units, the others per lane
#pragma unroll
    for (int u = 0; u < R; ++u) {
      const IDX row = row0 + u;
      if (row < rows) {
#pragma unroll
        for (int k = 0; k < VDSL_MAP_MAX_INPUTS; ++k) {
          if (k >= P::n_inputs) continue;
          const int w = P::width_of(k);
          if (staged_input<P>(k)) {
            const f32x4* src = reinterpret_cast<const f32x4*>(in.p[k] + (row * cols + col0) * w);
#pragma unroll
            for (int j = 0; j < 4; ++j)
              if (t + 256 * j < 64 * w) unit[u][k][j] = __builtin_nontemporal_load(src + t + 256 * j);
          } else {
            const int bc = P::bcast_of(k);
            load_record<IDX, S>(in.p[k], bc == VDSL_BCAST_FULL, w, record_index<IDX>(bc, row, col, cols), vin[u][k]);
          }
        }
      }
    }
    __syncthreads();  // the previous step's LDS reads are done
#pragma unroll
    for (int u = 0; u < R; ++u) {
      if (row0 + u < rows) {
#pragma unroll
        for (int k = 0; k < VDSL_MAP_MAX_INPUTS; ++k) {
          if (!staged_input<P>(k)) continue;
          const int w = P::width_of(k);
          f32x4* dst = lds + (u * SF + stage_offset<P>(k)) / 4;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int x = t + 256 * j;
            if (x < 64 * w) dst[w == 16 ? mat4_slot(x) : x] = unit[u][k][j];
          }
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < R; ++u) {
      if (row0 + u < rows) {
#pragma unroll
        for (int k = 0; k < VDSL_MAP_MAX_INPUTS; ++k) {
          if (!staged_input<P>(k)) continue;
          const int w = P::width_of(k);
          const f32x4* src = lds + (u * SF + stage_offset<P>(k)) / 4;
          if (w == 16) {
#pragma unroll
            for (int h = 0; h < 4; ++h) {
              const f32x4 v = src[mat4_slot(4 * t + h)];
              vin[u][k][4 * h] = v[0]; vin[u][k][4 * h + 1] = v[1]; vin[u][k][4 * h + 2] = v[2]; vin[u][k][4 * h + 3] = v[3];
            }
          } else {
            const float* f = reinterpret_cast<const float*>(src) + w * t;
#pragma unroll
            for (int c = 0; c < 9; ++c) vin[u][k][c] = f[c];
          }
        }
      }
    }
    map_chain_v_rows<P, R, S, IDX>(rt, in, vo, out, rows, cols, row0, col, vin);
  }
}

template <class P, int R, class IDX>
__device__ __forceinline__ void map_chain_v_body(const MapProg& rt, const MapVIn& in, const MapVOut& vo, float* __restrict__ out,
                                                 IDX rows, IDX cols) {
  constexpr bool G = IsGeneric<P>::value;
  // Slots per input of the per-row record array.  The interpreter keeps records of up to 4
  // components in registers and reads the components of wider records (mat3, mat4) from memory
  // when an instruction needs them.
  constexpr int S = VSlot<P>::value;
  if constexpr (!G) {
    if constexpr (stage_floats<P>() > 0) {
      // whole blocks whose staged rows start on 16-byte boundaries (mat4 rows always do; mat3
      // rows when cols is a multiple of 4) take the LDS path; the block's choice is uniform
      bool aligned = true;
      for (int k = 0; k < P::n_inputs; ++k)
        if (staged_input<P>(k) && P::width_of(k) % 4 != 0 && cols % 4 != 0) aligned = false;
      if (aligned && static_cast<IDX>(blockIdx.x) * 256 + 256 <= cols) {
        map_chain_v_staged<P, staged_rows<P>(R), IDX>(rt, in, vo, out, rows, cols);
        return;
      }
    }
  }
  const IDX col = static_cast<IDX>(blockIdx.x) * 256 + static_cast<IDX>(threadIdx.x);
  if (col >= cols) return;
  int n_in;
  if constexpr (G) n_in = in.n;
  else n_in = P::n_inputs;
  for (IDX row0 = static_cast<IDX>(blockIdx.y) * R; row0 < rows; row0 += static_cast<IDX>(gridDim.y) * R) {
    float vin[R][VDSL_MAP_MAX_INPUTS][S];
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
            if (w <= S) load_record<IDX, S>(in.p[k], bc == VDSL_BCAST_FULL, w, record_index<IDX>(bc, row, col, cols), vin[u][k]);
          }
        }
      }
    }
    map_chain_v_rows<P, R, S, IDX>(rt, in, vo, out, rows, cols, row0, col, vin);
  }
}

}  // namespace vdsl

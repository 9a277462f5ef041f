/*
 * vdsl_oracle.c - CPU restatement of every op class of include/vdsl.h.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker and the timed CPU baseline.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load liboracle.so, and
 * only to check or time it beside the HIP device; the product (libvdsl.so and the
 * vernondsl_amd package) never calls it and has no CPU fallback.
 *
 * Built with -ffp-contract=off: every f32 operation below rounds exactly where it is written;
 * fmaf() is used only where the spec asks for a single rounding.
 *
 * What pins each function (the checks live in tests/):
 *   orc_escape_time      fractal.py:11-25.  Pinned by an independent numpy evaluation (exactly
 *                        rounded; fma emulated by round-to-odd in f64), the known answers
 *                        sum = 49,860,131 and sha256 prefix 747b980a873b342e of the 1024^2
 *                        separately-rounded grid, the main-cardioid / period-2-bulb closed
 *                        forms, conjugate symmetry, and f64 brute force away from the boundary.
 *   orc_map_chain        no reference code.  Pinned against f64 numpy evaluation and the
 *                        special values x = 0 and |x| large.
 *   orc_pixel_program_rows
 *                        the general form of fractal.py:16-25 (a struct-for body with its check-
 *                        then-update loop).  Pinned by independent numpy restatements of whole
 *                        programs (Mandelbrot / Burning Ship / logistic maps, plain per-pixel
 *                        expressions, field reads, if / else and compound loop tests), by
 *                        equality with orc_escape_time on the programs both express, by closed
 *                        forms (a loop with no test runs max_iter times), and the comparison,
 *                        select, floor and trunc opcodes by numpy on every pair of special values;
 *                        asin, acos, atan, tan, atan2 and powf (the C library's float functions)
 *                        within 2 ulp of numpy's double-precision results, with atan2's signed-
 *                        zero quadrants and pow's IEEE special cases exactly; the bit operations
 *                        (and, or, xor, shifts) by numpy's int32 operations on every pair of a
 *                        set of values (negatives, fractions, NaN, past int32, counts past 31);
 *                        round (roundf) by an f64 restatement of halfway-away-from-zero rounding.
 *                        Scatter-adds (VDSL_PIX_ATOMIC_ADD, run pixel by pixel in row-major
 *                        order): by numpy's np.add.at over the same indices in the same order
 *                        (f32 bit for bit, int32 exactly with wrap-around) and by the drop rule
 *                        written out index by index over negative, fractional, too large,
 *                        infinite and NaN indices; histograms by np.bincount.
 *   orc_map_chain_v_rows vector operands (the vec2-4 / extract_component / swizzle vocabulary of
 *                        source/README.md:23-55).  Pinned by permutation closed forms: a swizzle
 *                        program equals numpy fancy indexing of the components, swizzles compose
 *                        as permutations, extract_component after a swizzle picks the permuted
 *                        component, and with width-1 operands it equals orc_map_chain.
 *                        Matrix operands (mat2-4, extract_component from a matrix, and the
 *                        MATVEC / VECMAT products of linalg.matvec, color.mlir:29-36): pinned by
 *                        identity, permutation and power-of-two matrices (exact), small-integer
 *                        matrices and vectors (exact integer arithmetic), numpy f64 within the
 *                        n-term rounding bound, VECMAT equal to MATVEC on the transposed matrix,
 *                        and an explicit numpy restatement of the accumulation order (signed zeros).
 *   orc_mat_transform / orc_vec_transform
 *                        the MVP chain of color.mlir:10-39 (vec(pos, 1) then linalg.matvec by up to
 *                        three matrices; vec_transform is the mat4 case).  Pinned by identity,
 *                        permutation, power-of-two scaling and translation matrices (exact in
 *                        f32), small-integer matrices and positions (exact integer arithmetic),
 *                        and numpy f64 within a rounding bound, for mat2, mat3 and mat4.
 *   orc_row_reduce_softmax / orc_col_reduce
 *                        no reference code.  Pinned by f64 sums, exact max, rows summing to 1,
 *                        constant row -> 1/cols, shift invariance, injected outlier argmax.
 *   orc_gemm_bf16        no reference code.  Pinned by exact integer-valued products (bf16
 *                        small integers), brute force in Python integers, and numpy f64.
 *   orc_gelu_fwd / orc_gelu_bwd / orc_gelu_grad / orc_mse_fwd_bwd
 *                        no reference code.  Pinned by central finite differences in f64.
 *   orc_relu_bwd / orc_add
 *                        no reference code.  Pinned by numpy's f32 select and f32 addition (an
 *                        IEEE addition has one correct result), bf16 operands widened exactly.
 *   orc_quantize_rows_i8 / orc_gemm_w8a8 / orc_w8a8_dequant
 *                        no reference code.  Pinned by int64 numpy dot products (exact) and a
 *                        numpy restatement of the f32 dequant sequence (orc_w8a8_dequant is the
 *                        GEMM's own epilogue code, checked against the same restatement).
 *   orc_transpose / orc_cast
 *                        pinned by numpy transpose / bit-level RNE.
 * The reference's own program (fractal.py) runs on third-party Taichi 1.7.4, which is not
 * importable here; its exact Taichi floating-point behaviour is parity unpinned.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "../include/vdsl.h"

#ifdef _OPENMP
#include <omp.h>
#endif

static inline float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

int orc_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void orc_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* ---- escape time: fractal.py:16-25 ------------------------------------------------------- */

static float pixel_coord(int idx, float den, float off, float scale, float post) {
  float v = (float)idx / den; /* fractal.py:20 `i / n` (true division in f32) */
  v = v + off;                /* `- 1` / `- 0.5` */
  v = v * scale;              /* `* 2` */
  return v + post;
}

/* Rows [i0, i1) of the grid.  Each pixel follows the check-then-update loop of
 * fractal.py:22-24 with complex_sqr (fractal.py:11-13). */
void orc_escape_time_rows(const vdsl_escape_time_params* p, void* out, int i0, int i1) {
#pragma omp parallel for schedule(dynamic, 4)
  for (int i = i0; i < i1; ++i) {
    for (int j = 0; j < p->nj; ++j) {
      const float re = pixel_coord(i, p->re_den, p->re_off, p->re_scale, p->re_post);
      const float im = pixel_coord(j, p->im_den, p->im_off, p->im_scale, p->im_post);
      float zr, zi, cr, ci;
      if (p->family == VDSL_ESC_MANDELBROT) {
        zr = 0.0f; zi = 0.0f; cr = re; ci = im;
      } else {
        zr = re; zi = im; cr = p->c_re; ci = p->c_im;
      }
      int it = 0;
      while (it < p->max_iter) {
        float mag, nzr, nzi;
        if (p->rounding == VDSL_ESC_ROUND_SEPARATE) {
          const float zr2 = zr * zr; /* z[0]**2 */
          const float zi2 = zi * zi; /* z[1]**2 */
          mag = zr2 + zi2;
          nzr = (zr2 - zi2) + cr;        /* z[0]**2 - z[1]**2, then + c */
          nzi = ((zi * zr) * 2.0f) + ci; /* z[1] * z[0] * 2, then + c */
        } else {
          const float q = zi * zi;
          mag = fmaf(zr, zr, q);
          nzr = fmaf(zr, zr, -q) + cr;
          nzi = fmaf(zr + zr, zi, ci);
        }
        int go_on = (p->escape_test == VDSL_ESC_MAG2_GT) ? !(mag > p->bound) : (sqrtf(mag) < p->bound);
        if (!go_on) break;
        zr = nzr;
        zi = nzi;
        ++it;
      }
      const size_t o = (size_t)i * (size_t)p->nj + (size_t)j;
      if (p->out_kind == VDSL_ESC_OUT_I32_COUNT) {
        ((int32_t*)out)[o] = it;
      } else {
        const float f = (float)it * p->out_scale; /* `iterations * 0.02` */
        ((float*)out)[o] = p->out_base + f;       /* `1 - ...` as 1 + (-0.02 * it) */
      }
    }
  }
}

void orc_escape_time(const vdsl_escape_time_params* p, void* out) { orc_escape_time_rows(p, out, 0, p->ni); }

/* ---- map chain --------------------------------------------------------------------------- */

static float map_apply(int op, float a, float b, float c, float imm) {
  switch (op) {
    case VDSL_MAP_CONST: return imm;
    case VDSL_MAP_MOV: return a;
    case VDSL_MAP_NEG: return -a;
    case VDSL_MAP_ABS: return fabsf(a);
    case VDSL_MAP_SQUARE: return a * a;
    case VDSL_MAP_EXP: return expf(a);
    case VDSL_MAP_LOG: return logf(a);
    case VDSL_MAP_TANH: return tanhf(a);
    case VDSL_MAP_SIGMOID: return 1.0f / (1.0f + expf(-a));
    case VDSL_MAP_RELU: return a > 0.0f ? a : 0.0f;
    case VDSL_MAP_SQRT: return sqrtf(a);
    case VDSL_MAP_RECIP: return 1.0f / a;
    case VDSL_MAP_ADD: return a + b;
    case VDSL_MAP_SUB: return a - b;
    case VDSL_MAP_MUL: return a * b;
    case VDSL_MAP_DIV: return a / b;
    case VDSL_MAP_MAX: return fmaxf(a, b);
    case VDSL_MAP_MIN: return fminf(a, b);
    case VDSL_MAP_FMA: return fmaf(a, b, c);
    case VDSL_MAP_MUL_IMM: return a * imm;
    case VDSL_MAP_ADD_IMM: return a + imm;
    default: return 0.0f;
  }
}

/* ---- general per-pixel programs (vdsl_pixel_program) -------------------------------------- */

/* Element e (pixel index), component comp of input a: f32 fields of in_widths[a] components, or
 * int32 fields read as float(v). */
static float pix_load(const vdsl_pixel_program* p, const void* const* inputs, int a, int64_t e, int comp) {
  if (p->in_dtypes[a] == VDSL_I32) return (float)((const int32_t*)inputs[a])[e];
  return ((const float*)inputs[a])[e * p->in_widths[a] + comp];
}

/* A field index from a register: 0 if !(x >= 0) (NaN included), else min((int)min(x, 2^30), n-1). */
static int64_t pix_index(float x, int64_t n) {
  if (!(x >= 0.0f)) return 0;
  const int64_t v = (int64_t)fminf(x, 1073741824.0f);
  return v < n - 1 ? v : n - 1;
}

/* A register stored to an int32 field: truncation toward zero, NaN -> 0, saturating. */
static int32_t pix_to_i32(float x) {
  if (x != x) return 0;
  if (x >= 2147483648.0f) return INT32_MAX;
  if (x < -2147483648.0f) return INT32_MIN;
  return (int32_t)x;
}

/* VDSL_PIX_RANDOM: Chris Wellons' lowbias32 hash of the seed, the draw and the pixel. */
static uint32_t pix_hash(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

static float pix_random(float seed, uint32_t draw, uint32_t pixel) {
  const uint32_t s = seed >= 0.0f && seed < 16777216.0f ? (uint32_t)seed : 0u;
  return (float)(pix_hash(pix_hash(pix_hash(s) ^ draw) ^ pixel) >> 8) * 0x1p-24f;
}

static float pix_apply(const vdsl_pixel_program* p, const vdsl_map_instr* s, const float* reg, const void* const* inputs,
                       int64_t o, int64_t i, int64_t j, int count, int64_t ni, int64_t nj) {
  switch (s->op) {
    case VDSL_MAP_LOAD: return pix_load(p, inputs, s->a, o, s->c);
    case VDSL_PIX_LOAD_AT: {  /* clamped to the input's own extents (the grid's unless in_rows/in_cols) */
      const int64_t rn = p->in_rows[s->a] ? p->in_rows[s->a] : ni, cn = p->in_cols[s->a] ? p->in_cols[s->a] : nj;
      return pix_load(p, inputs, s->a, pix_index(reg[s->b], rn) * cn + pix_index(reg[s->c], cn), (int)s->imm);
    }
    case VDSL_PIX_INDEX: return s->a == 0 ? (float)i : (float)j;
    case VDSL_PIX_COUNT: case VDSL_PIX_TRIP: return (float)count;  /* the trip, in the loop's sections */
    case VDSL_PIX_ATAN2: return atan2f(reg[s->a], reg[s->b]);
    case VDSL_PIX_ASIN: return asinf(reg[s->a]);
    case VDSL_PIX_ACOS: return acosf(reg[s->a]);
    case VDSL_PIX_ATAN: return atanf(reg[s->a]);
    case VDSL_PIX_TAN: return tanf(reg[s->a]);
    case VDSL_PIX_POWF: return powf(reg[s->a], reg[s->b]);
    case VDSL_PIX_ROUND: return roundf(reg[s->a]);
    case VDSL_PIX_BAND: return (float)(pix_to_i32(reg[s->a]) & pix_to_i32(reg[s->b]));
    case VDSL_PIX_BOR: return (float)(pix_to_i32(reg[s->a]) | pix_to_i32(reg[s->b]));
    case VDSL_PIX_BXOR: return (float)(pix_to_i32(reg[s->a]) ^ pix_to_i32(reg[s->b]));
    case VDSL_PIX_SHL: return (float)(int32_t)((uint32_t)pix_to_i32(reg[s->a]) << (pix_to_i32(reg[s->b]) & 31));
    case VDSL_PIX_SHR: return (float)(pix_to_i32(reg[s->a]) >> (pix_to_i32(reg[s->b]) & 31));
    case VDSL_PIX_COS: return cosf(reg[s->a]);
    case VDSL_PIX_SIN: return sinf(reg[s->a]);
    case VDSL_PIX_LT: return reg[s->a] < reg[s->b] ? 1.0f : 0.0f;
    case VDSL_PIX_LE: return reg[s->a] <= reg[s->b] ? 1.0f : 0.0f;
    case VDSL_PIX_EQ: return reg[s->a] == reg[s->b] ? 1.0f : 0.0f;
    case VDSL_PIX_NE: return reg[s->a] != reg[s->b] ? 1.0f : 0.0f;
    case VDSL_PIX_SELECT: return reg[s->a] != 0.0f ? reg[s->b] : reg[s->c];
    case VDSL_PIX_FLOOR: return floorf(reg[s->a]);
    case VDSL_PIX_RANDOM: return pix_random(reg[s->a], (uint32_t)s->imm, (uint32_t)(i * nj + j));
    case VDSL_PIX_TRUNC: return truncf(reg[s->a]);
    default: return map_apply(s->op, reg[s->a], reg[s->b], reg[s->c], s->imm);
  }
}

static int pix_test(int test, float a, float b) {
  switch (test) {
    case VDSL_PIX_TEST_LT: return a < b;
    case VDSL_PIX_TEST_LE: return a <= b;
    case VDSL_PIX_TEST_GT: return a > b;
    case VDSL_PIX_TEST_GE: return a >= b;
    default: return 1;
  }
}

/* VDSL_PIX_ATOMIC_ADD / MAX / MIN / STORE_AT: component imm of input a at [(int)r[b]][(int)r[c]]
 * += r[dst] (or becomes the max / min of it and r[dst], or r[dst]) when 0 <= r[b] < rows and 0 <= r[c] < cols of
 * input a, else nothing.  f32: one f32 addition, fmaxf, fminf; int32: the value converted as an
 * int32 store converts it, added modulo 2^32, or compared. */
static void pix_scatter_add(const vdsl_pixel_program* p, const vdsl_map_instr* s, const float* reg, const void* const* inputs,
                            int64_t ni, int64_t nj) {
  const int64_t rn = p->in_rows[s->a] ? p->in_rows[s->a] : ni, cn = p->in_cols[s->a] ? p->in_cols[s->a] : nj;
  const float x = reg[s->b], y = reg[s->c];
  if (!(x >= 0.0f && y >= 0.0f && x < 1073741824.0f && y < 1073741824.0f)) return;
  const int64_t xi = (int64_t)x, yi = (int64_t)y;
  if (xi >= rn || yi >= cn) return;
  const int64_t e = xi * cn + yi;
  if (p->in_dtypes[s->a] == VDSL_I32) {
    int32_t* t = (int32_t*)inputs[s->a] + e;
    const int32_t v = pix_to_i32(reg[s->dst]);
    if (s->op == VDSL_PIX_STORE_AT) *t = v;
    else if (s->op == VDSL_PIX_ATOMIC_ADD) *t = (int32_t)((uint32_t)*t + (uint32_t)v);
    else if (s->op == VDSL_PIX_ATOMIC_MAX) *t = v > *t ? v : *t;
    else *t = v < *t ? v : *t;
  } else {
    float* t = (float*)inputs[s->a] + e * p->in_widths[s->a] + (int)s->imm;
    if (s->op == VDSL_PIX_STORE_AT) *t = reg[s->dst];
    else if (s->op == VDSL_PIX_ATOMIC_ADD) *t = *t + reg[s->dst];
    else if (s->op == VDSL_PIX_ATOMIC_MAX) *t = fmaxf(*t, reg[s->dst]);
    else *t = fminf(*t, reg[s->dst]);
  }
}

static int pix_scatter_op(int op) {  /* the instructions with an effect: scatter add / max / min, store at */
  return op == VDSL_PIX_ATOMIC_ADD || op == VDSL_PIX_ATOMIC_MAX || op == VDSL_PIX_ATOMIC_MIN || op == VDSL_PIX_STORE_AT;
}

/* One instruction: its register, or a scatter-add's effect. */
static void pix_exec(const vdsl_pixel_program* p, int pc, float* reg, const void* const* inputs, int64_t o, int64_t i,
                     int64_t j, int count, int64_t ni, int64_t nj) {
  const vdsl_map_instr* s = &p->code[pc];
  if (pix_scatter_op(s->op)) pix_scatter_add(p, s, reg, inputs, ni, nj);
  else reg[s->dst] = pix_apply(p, s, reg, inputs, o, i, j, count, ni, nj);
}

/* Rows [r0, r1) of vdsl_op_pixel_program: per pixel, VDSL_PIX_MAX_REGS registers at 0, the pre section, the
 * check-then-update loop (fractal.py:22-24: test, stop unless it holds and fewer than max_iter
 * updates were made, body, count), the post section, then out[i][j][k] = r[out_regs[k]] (f32,
 * out_width components) or the count (int32), nothing for VDSL_PIX_OUT_NONE.  A LOAD reads
 * component c of input a's pixel (in_widths[a] components each).  A program with scatter-adds
 * runs its pixels one after another in row-major order (so an f32 target gets its adds in that
 * order); others run rows in parallel.  The program is taken as validated by the caller. */
void orc_pixel_program_rows(const vdsl_pixel_program* p, int64_t ni, int64_t nj, const void* const* inputs, void* out,
                            int64_t r0, int64_t r1) {
  const int t0 = p->n_pre, b0 = t0 + p->n_test, q0 = b0 + p->n_body, end = q0 + p->n_post;
  int scatters = 0;
  for (int pc = 0; pc < end; ++pc) scatters |= pix_scatter_op(p->code[pc].op);
#pragma omp parallel for schedule(dynamic, 4) if (!scatters)
  for (int64_t i = r0; i < r1; ++i)
    for (int64_t j = 0; j < nj; ++j) {
      const int64_t o = i * nj + j;
      float reg[VDSL_PIX_MAX_REGS];
      for (int k = 0; k < VDSL_PIX_MAX_REGS; ++k) reg[k] = 0.0f;
      int count = 0;
      for (int pc = 0; pc < t0; ++pc) pix_exec(p, pc, reg, inputs, o, i, j, 0, ni, nj);
      if (p->loop) {
        while (count < p->max_iter) {
          for (int pc = t0; pc < b0; ++pc) pix_exec(p, pc, reg, inputs, o, i, j, count, ni, nj);
          if (!pix_test(p->test, reg[p->test_a], reg[p->test_b])) break;
          for (int pc = b0; pc < q0; ++pc) pix_exec(p, pc, reg, inputs, o, i, j, count, ni, nj);
          ++count;
        }
      }
      for (int pc = q0; pc < end; ++pc) pix_exec(p, pc, reg, inputs, o, i, j, count, ni, nj);
      if (p->out_kind == VDSL_PIX_OUT_NONE) {
        continue;
      } else if (p->out_kind == VDSL_PIX_OUT_COUNT) {
        ((int32_t*)out)[o - r0 * nj] = count;
      } else if (p->out_kind == VDSL_PIX_OUT_I32) {
        ((int32_t*)out)[o - r0 * nj] = pix_to_i32(reg[p->out_regs[0]]);
      } else {
        for (int k = 0; k < p->out_width; ++k) ((float*)out)[(o - r0 * nj) * p->out_width + k] = reg[p->out_regs[k]];
      }
    }
}

/* Rows [r0, r1). in_ptrs[k] holds input k per bcast[k] (vdsl_broadcast). */
void orc_map_chain_rows(int64_t rows, int64_t cols, const vdsl_map_instr* code, int n_instr,
                        const float* const* in_ptrs, const int* bcast, int n_inputs, int out_reg, float* out,
                        int64_t r0, int64_t r1) {
  (void)rows;
  (void)n_inputs;
#pragma omp parallel for schedule(static)
  for (int64_t r = r0; r < r1; ++r) {
    for (int64_t c = 0; c < cols; ++c) {
      float reg[VDSL_MAP_MAX_REGS] = {0};
      for (int pc = 0; pc < n_instr; ++pc) {
        const vdsl_map_instr* s = &code[pc];
        if (s->op == VDSL_MAP_LOAD) {
          const float* p = in_ptrs[s->a];
          const int bc = bcast[s->a];
          reg[s->dst] = bc == VDSL_BCAST_FULL ? p[r * cols + c] : bc == VDSL_BCAST_ROW ? p[c] : bc == VDSL_BCAST_COL ? p[r] : p[0];
        } else {
          reg[s->dst] = map_apply(s->op, reg[s->a], reg[s->b], reg[s->c], s->imm);
        }
      }
      out[r * cols + c] = reg[out_reg];
    }
  }
}

void orc_map_chain(int64_t rows, int64_t cols, const vdsl_map_instr* code, int n_instr, const float* const* in_ptrs,
                   const int* bcast, int n_inputs, int out_reg, float* out) {
  orc_map_chain_rows(rows, cols, code, n_instr, in_ptrs, bcast, n_inputs, out_reg, out, 0, rows);
}

/* Vector operands (vdsl_op_map_chain_v): input k holds elements of widths[k] components (AoS);
 * a LOAD reads component `c` of its input's element; output element (r, c) is the out_width
 * registers out_regs[0..out_width) in that order. */
void orc_map_chain_v_rows(int64_t rows, int64_t cols, const vdsl_map_instr* code, int n_instr,
                          const float* const* in_ptrs, const int* bcast, const int* widths, int n_inputs,
                          const int* out_regs, int out_width, float* out, int64_t r0, int64_t r1) {
  (void)rows;
  (void)n_inputs;
#pragma omp parallel for schedule(static)
  for (int64_t r = r0; r < r1; ++r) {
    for (int64_t c = 0; c < cols; ++c) {
      float reg[VDSL_MAP_MAX_REGS] = {0};
      for (int pc = 0; pc < n_instr; ++pc) {
        const vdsl_map_instr* s = &code[pc];
        if (s->op == VDSL_MAP_LOAD || s->op == VDSL_MAP_MATVEC || s->op == VDSL_MAP_VECMAT) {
          const int bc = bcast[s->a], w = widths[s->a];
          const int64_t e = bc == VDSL_BCAST_FULL ? r * cols + c : bc == VDSL_BCAST_ROW ? c : bc == VDSL_BCAST_COL ? r : 0;
          const float* rec = in_ptrs[s->a] + e * w;
          if (s->op == VDSL_MAP_LOAD) {
            reg[s->dst] = rec[s->c];
          } else {
            /* a matrix input: w = n * n */
            const int n = w == 16 ? 4 : w == 9 ? 3 : 2;
            const int vr[4] = {s->b, s->ext[0], s->ext[1], s->ext[2]};
            float acc = 0.0f;
            for (int k = 0; k < n; ++k) {
              const float m = s->op == VDSL_MAP_MATVEC ? rec[s->c * n + k] : rec[k * n + s->c];
              const float prod = m * reg[vr[k]];
              acc = acc + prod;
            }
            reg[s->dst] = acc;
          }
        } else {
          reg[s->dst] = map_apply(s->op, reg[s->a], reg[s->b], reg[s->c], s->imm);
        }
      }
      for (int k = 0; k < out_width; ++k) out[(r * cols + c) * out_width + k] = reg[out_regs[k]];
    }
  }
}

/* The MVP chain of color.mlir:10-39 over n vertices, for dim x dim matrices (dim 2..4):
 * v = vec(pos, 1) for in_width dim - 1 (color.mlir:15-21 for dim 4), pos itself for in_width dim;
 * then for each of the n_mats row-major matrices in order, v <- M v with
 * out[i] = ((0 + M[i][0] v0) + M[i][1] v1) + ... (f32 products and sums, the mulf/addf
 * accumulation of linalg.matvec into a zero-initialised output, color.mlir:29-36). */
void orc_mat_transform(int64_t n, int dim, int in_width, const float* pos, int n_mats, const float* mats, float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t e = 0; e < n; ++e) {
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int i = 0; i < in_width; ++i) v[i] = pos[e * in_width + i];
    if (in_width == dim - 1) v[dim - 1] = 1.0f;
    for (int t = 0; t < n_mats; ++t) {
      const float* m = mats + dim * dim * t;
      float o[4];
      for (int i = 0; i < dim; ++i) {
        float acc = 0.0f;
        for (int j = 0; j < dim; ++j) {
          const float prod = m[dim * i + j] * v[j];
          acc = acc + prod;
        }
        o[i] = acc;
      }
      for (int i = 0; i < dim; ++i) v[i] = o[i];
    }
    for (int i = 0; i < dim; ++i) out[e * dim + i] = v[i];
  }
}

void orc_vec_transform(int64_t n, int in_width, const float* pos, int n_mats, const float* mats, float* out) {
  orc_mat_transform(n, 4, in_width, pos, n_mats, mats, out);
}

/* ---- row reduce + softmax ---------------------------------------------------------------- */

static inline float load_elem(const void* x, int dtype, int64_t idx) {
  return dtype == VDSL_BF16 ? bf16_to_f32(((const uint16_t*)x)[idx]) : ((const float*)x)[idx];
}

/* Rows [r0, r1).  sum: f64 accumulation rounded once to f32.  max: exact.  softmax:
 * e = expf(x - max) in f32, s = f64 sum of e rounded to f32, out = e / s (f32), then RNE to bf16
 * for bf16 tensors. */
void orc_row_reduce_softmax_rows(int64_t rows, int64_t cols, int dtype, const void* x, float* row_sum,
                                 float* row_max, void* softmax, int64_t r0, int64_t r1) {
  (void)rows;
#pragma omp parallel
  {
    float* e = (float*)malloc(sizeof(float) * (size_t)(cols > 0 ? cols : 1));
#pragma omp for schedule(static)
    for (int64_t r = r0; r < r1; ++r) {
      const int64_t base = r * cols;
      double s = 0.0;
      float m = -INFINITY;
      for (int64_t c = 0; c < cols; ++c) {
        const float v = load_elem(x, dtype, base + c);
        s += v;
        m = fmaxf(m, v);
      }
      if (row_sum) row_sum[r] = (float)s;
      if (row_max) row_max[r] = m;
      if (softmax) {
        double es = 0.0;
        for (int64_t c = 0; c < cols; ++c) {
          e[c] = expf(load_elem(x, dtype, base + c) - m);
          es += e[c];
        }
        const float esf = (float)es;
        for (int64_t c = 0; c < cols; ++c) {
          const float v = e[c] / esf;
          if (dtype == VDSL_BF16) ((uint16_t*)softmax)[base + c] = f32_to_bf16(v);
          else ((float*)softmax)[base + c] = v;
        }
      }
    }
    free(e);
  }
}

void orc_row_reduce_softmax(int64_t rows, int64_t cols, int dtype, const void* x, float* row_sum, float* row_max,
                            void* softmax) {
  orc_row_reduce_softmax_rows(rows, cols, dtype, x, row_sum, row_max, softmax, 0, rows);
}

void orc_col_reduce(int64_t rows, int64_t cols, int dtype, const void* x, float* col_sum, float* col_max) {
#pragma omp parallel for schedule(static)
  for (int64_t c = 0; c < cols; ++c) {
    double s = 0.0;
    float m = -INFINITY;
    for (int64_t r = 0; r < rows; ++r) {
      const float v = load_elem(x, dtype, r * cols + c);
      s += v;
      m = fmaxf(m, v);
    }
    if (col_sum) col_sum[c] = (float)s;
    if (col_max) col_max[c] = m;
  }
}

/* ---- bf16 GEMM, transpose, cast ---------------------------------------------------------- */

/* 0.5 v (1 + erf(v / sqrt2)) = 0.5 v erfc(-v / sqrt2) (no cancellation for v < 0). */
static double gelu_d(double v) { return 0.5 * v * erfc(-v * 0.70710678118654752440); }

static void store_out(void* C, int c_dtype, int64_t idx, float v) {
  if (c_dtype == VDSL_BF16) ((uint16_t*)C)[idx] = f32_to_bf16(v);
  else ((float*)C)[idx] = v;
}

/* Rows [m0, m1) of C = epilogue(op(A) op(B)); products and sums in f64 (exact products of bf16
 * values; the f64 sum is then rounded once to f32). */
void orc_gemm_bf16_rows(int ta, int tb, int64_t M, int64_t N, int64_t K, const uint16_t* A, const uint16_t* B,
                        void* C, int c_dtype, int epilogue, float* pre_act, int64_t m0, int64_t m1) {
#pragma omp parallel
  {
    double* acc = (double*)malloc(sizeof(double) * (size_t)(N > 0 ? N : 1));
#pragma omp for schedule(static)
    for (int64_t m = m0; m < m1; ++m) {
      for (int64_t n = 0; n < N; ++n) acc[n] = 0.0;
      for (int64_t k = 0; k < K; ++k) {
        const double a = bf16_to_f32(ta ? A[k * M + m] : A[m * K + k]);
        if (a == 0.0) continue;
        if (!tb) {
          const uint16_t* brow = B + k * N;
          for (int64_t n = 0; n < N; ++n) acc[n] += a * (double)bf16_to_f32(brow[n]);
        } else {
          for (int64_t n = 0; n < N; ++n) acc[n] += a * (double)bf16_to_f32(B[n * K + k]);
        }
      }
      for (int64_t n = 0; n < N; ++n) {
        const float v = (float)acc[n];
        if (pre_act) pre_act[m * N + n] = v;
        float o = v;
        if (epilogue == VDSL_EPI_GELU) o = (float)gelu_d((double)v);
        else if (epilogue == VDSL_EPI_RELU) o = v > 0.0f ? v : 0.0f;
        store_out(C, c_dtype, m * N + n, o);
      }
    }
    free(acc);
  }
  (void)M;
}

void orc_gemm_bf16(int ta, int tb, int64_t M, int64_t N, int64_t K, const uint16_t* A, const uint16_t* B, void* C,
                   int c_dtype, int epilogue, float* pre_act) {
  orc_gemm_bf16_rows(ta, tb, M, N, K, A, B, C, c_dtype, epilogue, pre_act, 0, M);
}

void orc_transpose(int64_t rows, int64_t cols, int dtype, const void* src, void* dst) {
  const size_t es = dtype == VDSL_BF16 ? 2 : 4;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c)
      memcpy((char*)dst + ((size_t)c * (size_t)rows + (size_t)r) * es, (const char*)src + ((size_t)r * (size_t)cols + (size_t)c) * es, es);
}

void orc_cast(int64_t n, int src_dtype, const void* src, int dst_dtype, void* dst) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) store_out(dst, dst_dtype, i, load_elem(src, src_dtype, i));
}

/* ---- autodiff blocks --------------------------------------------------------------------- */

/* Elementwise GELU (x_dtype, y_dtype: 0 = f32, 1 = bf16): f64 evaluation of the exact-erf form,
 * rounded once to f32 (then RNE to bf16 when y is bf16). */
void orc_gelu_fwd(int64_t n, int x_dtype, const void* x, int y_dtype, void* y) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    const float v = x_dtype == 0 ? ((const float*)x)[i] : bf16_to_f32(((const uint16_t*)x)[i]);
    const float g = (float)gelu_d((double)v);
    if (y_dtype == 0) ((float*)y)[i] = g;
    else ((uint16_t*)y)[i] = f32_to_bf16(g);
  }
}

/* d/dv GELU(v) = Phi(v) + v phi(v) = 0.5 erfc(-v/sqrt2) + v exp(-v^2/2) / sqrt(2 pi), in f64. */
static double gelu_grad_d(double v) {
  return 0.5 * erfc(-v * 0.70710678118654752440) + v * exp(-0.5 * v * v) * 0.39894228040143267794;
}

/* GELU'(x) elementwise in f32 (the f64 formula above, rounded once): the local derivative the
 * forward epilogue VDSL_EPI_GELU_DERIV stores for the backward pass. */
void orc_gelu_grad(int64_t n, const float* x, float* y) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) y[i] = (float)gelu_grad_d((double)x[i]);
}

void orc_gelu_bwd(int64_t rows, int64_t cols, const float* dh, const float* pre, uint16_t* da, uint16_t* da_t) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c) {
      const float g = (float)((double)dh[r * cols + c] * gelu_grad_d((double)pre[r * cols + c]));
      const uint16_t h = f32_to_bf16(g);
      if (da) da[r * cols + c] = h;
      if (da_t) da_t[c * rows + r] = h;
    }
}

/* ReLU backward: da = dh where pre > 0, else +0 (NaN pre included), RNE to bf16. */
void orc_relu_bwd(int64_t rows, int64_t cols, const float* dh, const float* pre, uint16_t* da, uint16_t* da_t) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c) {
      const float p = pre[r * cols + c];
      const uint16_t h = f32_to_bf16(p > 0.0f ? dh[r * cols + c] : 0.0f);
      if (da) da[r * cols + c] = h;
      if (da_t) da_t[c * rows + r] = h;
    }
}

/* out = a + b: operands widened to f32, one f32 addition, rounded to out's dtype. */
void orc_add(int64_t n, int a_dtype, const void* a, int b_dtype, const void* b, int out_dtype, void* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) store_out(out, out_dtype, i, load_elem(a, a_dtype, i) + load_elem(b, b_dtype, i));
}

/* loss = mean((y - t)^2) (f64 sum, rounded once); dy = (y - t) * (2 / n) in f32, RNE to bf16. */
void orc_mse_fwd_bwd(int64_t rows, int64_t cols, const float* y, const float* t, float* loss, uint16_t* dy,
                     uint16_t* dy_t) {
  const int64_t n = rows * cols;
  const float scale = 2.0f / (float)n;
  double s = 0.0;
#pragma omp parallel for schedule(static) reduction(+ : s)
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t c = 0; c < cols; ++c) {
      const float d = y[r * cols + c] - t[r * cols + c];
      s += (double)d * (double)d;
      const uint16_t h = f32_to_bf16(d * scale);
      if (dy) dy[r * cols + c] = h;
      if (dy_t) dy_t[c * rows + r] = h;
    }
  }
  if (loss) *loss = (float)(s / (double)n);
}

/* ---- int8 W8A8 --------------------------------------------------------------------------- */

/* s = max|x| / 127; q = clamp(rint(x / s), -127, 127); an all-zero (or underflowing) row gives
 * s = 0 and q = 0. */
void orc_quantize_rows_i8(int64_t rows, int64_t cols, int x_dtype, const void* x, int8_t* q, float* scale) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    float amax = 0.0f;
    for (int64_t c = 0; c < cols; ++c) amax = fmaxf(amax, fabsf(load_elem(x, x_dtype, r * cols + c)));
    const float s = amax / 127.0f;
    scale[r] = s;
    for (int64_t c = 0; c < cols; ++c) {
      int v = 0;
      if (s > 0.0f) {
        float t = rintf(load_elem(x, x_dtype, r * cols + c) / s);
        if (t > 127.0f) t = 127.0f;
        if (t < -127.0f) t = -127.0f;
        v = (int)t;
      }
      q[r * cols + c] = (int8_t)v;
    }
  }
}

/* The dequant epilogue of one accumulator: relu?((float(acc) * xs) * ws), each product rounded. */
static inline float w8a8_dequant_one(int32_t acc, float xs, float ws, int relu) {
  float v = (float)acc * xs;
  v = v * ws;
  if (relu && !(v > 0.0f)) v = 0.0f;
  return v;
}

/* Rows [m0, m1): acc = sum_k xq[m][k] w[n][k] (exact, int64 then int32);
 * y = relu?((float(acc) * xs[m]) * ws[n]) in f32, stored as out_dtype. */
void orc_gemm_w8a8_rows(int64_t M, int64_t N, int64_t K, const int8_t* xq, const float* xs, const int8_t* w,
                        const float* ws, void* y, int out_dtype, int relu, int32_t* acc_out, int64_t m0, int64_t m1) {
  (void)M;
#pragma omp parallel for schedule(static)
  for (int64_t m = m0; m < m1; ++m) {
    const int8_t* xr = xq + m * K;
    for (int64_t n = 0; n < N; ++n) {
      const int8_t* wr = w + n * K;
      int64_t acc = 0;
      for (int64_t k = 0; k < K; ++k) acc += (int64_t)xr[k] * (int64_t)wr[k];
      const int32_t a32 = (int32_t)acc;
      if (acc_out) acc_out[m * N + n] = a32;
      store_out(y, out_dtype, m * N + n, w8a8_dequant_one(a32, xs[m], ws[n], relu));
    }
  }
}

/* The epilogue of orc_gemm_w8a8 alone, on given int32 accumulators acc [M][N] (the same code, so
 * it is pinned with orc_gemm_w8a8): lets a full-size check take exact accumulators from another
 * source (an f64 matrix product of the int8 operands is exact at these sizes). */
void orc_w8a8_dequant(int64_t M, int64_t N, const int32_t* acc, const float* xs, const float* ws, void* y, int out_dtype,
                      int relu) {
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) store_out(y, out_dtype, m * N + n, w8a8_dequant_one(acc[m * N + n], xs[m], ws[n], relu));
}

void orc_gemm_w8a8(int64_t M, int64_t N, int64_t K, const int8_t* xq, const float* xs, const int8_t* w,
                   const float* ws, void* y, int out_dtype, int relu, int32_t* acc_out) {
  orc_gemm_w8a8_rows(M, N, K, xq, xs, w, ws, y, out_dtype, relu, acc_out, 0, M);
}

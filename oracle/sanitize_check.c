/*
 * sanitize_check.c - runs every routine of the CPU oracle (vdsl_oracle.c, test infrastructure) on
 * small, empty and ragged shapes, for a build with AddressSanitizer and UndefinedBehaviorSanitizer
 * (`make -C oracle sanitize`, run by tests/test_oracle_sanitize.py).  It checks memory safety and
 * defined behaviour of the oracle's indexing, not its numbers (the other oracle tests pin those):
 * every buffer is allocated at exactly the size the routine's contract names, so a read or write
 * one element past it is reported.  Exit status 0 and "sanitize_check: ok" on success.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../include/vdsl.h"

void orc_escape_time_rows(const vdsl_escape_time_params* p, void* out, int i0, int i1);
void orc_map_chain_rows(int64_t rows, int64_t cols, const vdsl_map_instr* code, int n_instr, const float* const* in_ptrs,
                        const int* bcast, int n_inputs, int out_reg, float* out, int64_t r0, int64_t r1);
void orc_map_chain_v_rows(int64_t rows, int64_t cols, const vdsl_map_instr* code, int n_instr, const float* const* in_ptrs,
                          const int* bcast, const int* widths, int n_inputs, const int* out_regs, int out_width, float* out,
                          int64_t r0, int64_t r1);
void orc_vec_transform(int64_t n, int in_width, const float* pos, int n_mats, const float* mats, float* out);
void orc_mat_transform(int64_t n, int dim, int in_width, const float* pos, int n_mats, const float* mats, float* out);
void orc_row_reduce_softmax_rows(int64_t rows, int64_t cols, int dtype, const void* x, float* row_sum, float* row_max,
                                 void* softmax, int64_t r0, int64_t r1);
void orc_col_reduce(int64_t rows, int64_t cols, int dtype, const void* x, float* col_sum, float* col_max);
void orc_gemm_bf16_rows(int ta, int tb, int64_t M, int64_t N, int64_t K, const uint16_t* A, const uint16_t* B, void* C,
                        int c_dtype, int epilogue, float* pre_act, int64_t m0, int64_t m1);
void orc_transpose(int64_t rows, int64_t cols, int dtype, const void* src, void* dst);
void orc_cast(int64_t n, int src_dtype, const void* src, int dst_dtype, void* dst);
void orc_gelu_fwd(int64_t n, int x_dtype, const void* x, int y_dtype, void* y);
void orc_gelu_bwd(int64_t rows, int64_t cols, const float* dh, const float* pre, uint16_t* da, uint16_t* da_t);
void orc_mse_fwd_bwd(int64_t rows, int64_t cols, const float* y, const float* t, float* loss, uint16_t* dy, uint16_t* dy_t);
void orc_quantize_rows_i8(int64_t rows, int64_t cols, int x_dtype, const void* x, int8_t* q, float* scale);
void orc_pixel_program_rows(const vdsl_pixel_program* p, int64_t ni, int64_t nj, const void* const* inputs, void* out,
                            int64_t r0, int64_t r1);
void orc_gemm_w8a8_rows(int64_t M, int64_t N, int64_t K, const int8_t* xq, const float* xs, const int8_t* w, const float* ws,
                        void* y, int out_dtype, int relu, int32_t* acc_out, int64_t m0, int64_t m1);

static uint64_t g_state = 0x5EED0009u;
static float frand(void) {  /* splitmix64, top 24 bits -> [-2, 2) */
  uint64_t z = (g_state += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z ^= z >> 31;
  return (float)(z >> 40) * (4.0f / 16777216.0f) - 2.0f;
}

/* Exactly n bytes (at least 1, so malloc(0) is never the question), filled with random floats or
 * bytes: reading a byte past the end is an ASan report. */
static void* buf(size_t n, int fill_floats) {
  void* p = malloc(n ? n : 1);
  if (!p) { fprintf(stderr, "out of memory\n"); exit(2); }
  if (fill_floats) for (size_t i = 0; i + 4 <= n; i += 4) { float f = frand(); memcpy((char*)p + i, &f, 4); }
  else for (size_t i = 0; i < n; ++i) ((unsigned char*)p)[i] = (unsigned char)(frand() * 60.0f);
  return p;
}

static void escape_time(void) {
  const int shapes[][2] = {{1, 1}, {7, 13}, {0, 5}, {5, 0}, {33, 17}};
  for (int s = 0; s < 5; ++s) {
    for (int out_kind = 0; out_kind < 2; ++out_kind) {
      vdsl_escape_time_params p;
      memset(&p, 0, sizeof p);
      p.ni = shapes[s][0]; p.nj = shapes[s][1];
      p.family = s & 1; p.escape_test = (s >> 1) & 1; p.rounding = out_kind; p.out_kind = out_kind;
      p.max_iter = 40; p.bound = 4.0f;
      p.re_den = 16.0f; p.re_off = -1.0f; p.re_scale = 2.0f; p.im_den = 16.0f; p.im_off = -0.5f; p.im_scale = 2.0f;
      p.c_re = -0.8f; p.c_im = 0.156f; p.out_base = 1.0f; p.out_scale = -0.02f;
      void* out = buf((size_t)p.ni * p.nj * 4, 0);
      orc_escape_time_rows(&p, out, 0, p.ni);
      free(out);
    }
  }
}

static void map_chains(void) {
  const int64_t shapes[][2] = {{1, 1}, {3, 5}, {0, 4}, {4, 0}, {9, 31}};
  for (int s = 0; s < 5; ++s) {
    const int64_t rows = shapes[s][0], cols = shapes[s][1];
    for (int bc = 0; bc < 4; ++bc) {
      const int64_t n_in = bc == VDSL_BCAST_FULL ? rows * cols : bc == VDSL_BCAST_ROW ? cols : bc == VDSL_BCAST_COL ? rows : 1;
      for (int w = 1; w <= 4; ++w) {
        float* in0 = buf((size_t)(rows * cols) * 4 * w, 1);
        float* in1 = buf((size_t)n_in * 4 * w, 1);
        const float* ptrs[2] = {in0, in1};
        const int bcast[2] = {VDSL_BCAST_FULL, bc}, widths[2] = {w, w};
        vdsl_map_instr code[6];
        memset(code, 0, sizeof code);
        code[0].op = VDSL_MAP_LOAD; code[0].dst = 0; code[0].a = 0; code[0].c = (uint8_t)(w - 1);
        code[1].op = VDSL_MAP_LOAD; code[1].dst = 1; code[1].a = 1; code[1].c = 0;
        code[2].op = VDSL_MAP_TANH; code[2].dst = 2; code[2].a = 0;
        code[3].op = VDSL_MAP_FMA; code[3].dst = 3; code[3].a = 2; code[3].b = 1; code[3].c = 0;
        code[4].op = VDSL_MAP_EXP; code[4].dst = 4; code[4].a = 3;
        code[5].op = VDSL_MAP_ADD_IMM; code[5].dst = 5; code[5].a = 4; code[5].imm = 0.5f;
        const int regs[4] = {5, 0, 3, 1};
        for (int ow = 1; ow <= 4; ++ow) {
          float* out = buf((size_t)(rows * cols) * 4 * ow, 0);
          orc_map_chain_v_rows(rows, cols, code, 6, ptrs, bcast, widths, 2, regs, ow, out, 0, rows);
          free(out);
        }
        if (w == 1) {
          float* out = buf((size_t)(rows * cols) * 4, 0);
          orc_map_chain_rows(rows, cols, code, 6, ptrs, bcast, 2, 5, out, 0, rows);
          free(out);
        }
        free(in0);
        free(in1);
      }
    }
  }
}

static void vec_transform(void) {
  const int64_t ns[] = {0, 1, 5, 1023};
  for (int s = 0; s < 4; ++s)
    for (int w = 3; w <= 4; ++w)
      for (int k = 1; k <= 3; ++k) {
        float* pos = buf((size_t)ns[s] * w * 4, 1);
        float* mats = buf((size_t)k * 64, 1);
        float* out = buf((size_t)ns[s] * 16, 0);
        orc_vec_transform(ns[s], w, pos, k, mats, out);
        free(pos); free(mats); free(out);
      }
  for (int s = 0; s < 4; ++s)
    for (int d = 2; d <= 4; ++d)
      for (int w = d - 1; w <= d; ++w)
        for (int k = 1; k <= 3; ++k) {
          float* pos = buf((size_t)ns[s] * w * 4, 1);
          float* mats = buf((size_t)k * d * d * 4, 1);
          float* out = buf((size_t)ns[s] * d * 4, 0);
          orc_mat_transform(ns[s], d, w, pos, k, mats, out);
          free(pos); free(mats); free(out);
        }
}

/* Matrix operands of the vector chain: every matrix size and broadcast, both products, and a load
 * of the last matrix component, each operand buffer at exactly its contract's size. */
static void map_chain_mat(void) {
  const int64_t shapes[][2] = {{1, 1}, {3, 5}, {0, 4}, {2, 0}};
  for (int s = 0; s < 4; ++s) {
    const int64_t rows = shapes[s][0], cols = shapes[s][1];
    for (int bc = 0; bc < 4; ++bc)
      for (int d = 2; d <= 4; ++d) {
        const int64_t n_in = bc == VDSL_BCAST_FULL ? rows * cols : bc == VDSL_BCAST_ROW ? cols : bc == VDSL_BCAST_COL ? rows : 1;
        float* vec = buf((size_t)(rows * cols) * 4 * d, 1);
        float* mat = buf((size_t)n_in * 4 * d * d, 1);
        const float* ptrs[2] = {vec, mat};
        const int bcast[2] = {VDSL_BCAST_FULL, bc}, widths[2] = {d, d * d};
        vdsl_map_instr code[8];
        memset(code, 0, sizeof code);
        for (int k = 0; k < d; ++k) {
          code[k].op = VDSL_MAP_LOAD; code[k].dst = (uint8_t)k; code[k].a = 0; code[k].c = (uint8_t)k;
        }
        code[d].op = VDSL_MAP_MATVEC; code[d].dst = 4; code[d].a = 1; code[d].b = 0; code[d].c = (uint8_t)(d - 1);
        code[d + 1].op = VDSL_MAP_VECMAT; code[d + 1].dst = 5; code[d + 1].a = 1; code[d + 1].b = 0; code[d + 1].c = (uint8_t)(d - 1);
        for (int k = 1; k < d; ++k) code[d].ext[k - 1] = code[d + 1].ext[k - 1] = (uint8_t)k;
        code[d + 2].op = VDSL_MAP_LOAD; code[d + 2].dst = 6; code[d + 2].a = 1; code[d + 2].c = (uint8_t)(d * d - 1);
        const int regs[4] = {4, 5, 6, 0};
        float* out = buf((size_t)(rows * cols) * 4 * 3, 0);
        orc_map_chain_v_rows(rows, cols, code, d + 3, ptrs, bcast, widths, 2, regs, 3, out, 0, rows);
        free(out);
        free(vec);
        free(mat);
      }
  }
}

static void reductions(void) {
  const int64_t shapes[][2] = {{1, 1}, {3, 300}, {5, 0}, {0, 7}, {17, 4096}};
  for (int s = 0; s < 5; ++s)
    for (int dt = 0; dt < 2; ++dt) {
      const int64_t rows = shapes[s][0], cols = shapes[s][1];
      const size_t es = dt == VDSL_F32 ? 4 : 2;
      void* x = buf((size_t)(rows * cols) * es, dt == VDSL_F32);
      float* rs = buf((size_t)rows * 4, 0);
      float* rm = buf((size_t)rows * 4, 0);
      void* sm = buf((size_t)(rows * cols) * es, 0);
      float* cs = buf((size_t)cols * 4, 0);
      float* cm = buf((size_t)cols * 4, 0);
      orc_row_reduce_softmax_rows(rows, cols, dt, x, rs, rm, sm, 0, rows);
      orc_col_reduce(rows, cols, dt, x, cs, cm);
      free(x); free(rs); free(rm); free(sm); free(cs); free(cm);
    }
}

static void gemms(void) {
  const int64_t shapes[][3] = {{1, 1, 1}, {3, 5, 7}, {0, 4, 4}, {4, 0, 4}, {4, 4, 0}, {33, 17, 40}};
  for (int s = 0; s < 6; ++s) {
    const int64_t M = shapes[s][0], N = shapes[s][1], K = shapes[s][2];
    for (int ta = 0; ta < 2; ++ta)
      for (int tb = 0; tb < 2; ++tb)
        for (int epi = 0; epi <= 2; ++epi) {
          uint16_t* A = buf((size_t)(M * K) * 2, 0);
          uint16_t* B = buf((size_t)(N * K) * 2, 0);
          const int cdt = epi == 0 ? VDSL_F32 : VDSL_BF16;
          void* C = buf((size_t)(M * N) * (cdt == VDSL_F32 ? 4 : 2), 0);
          float* pre = buf((size_t)(M * N) * 4, 0);
          orc_gemm_bf16_rows(ta, tb, M, N, K, A, B, C, cdt, epi, pre, 0, M);
          free(A); free(B); free(C); free(pre);
        }
    int8_t* xq = buf((size_t)(M * K), 0);
    int8_t* w = buf((size_t)(N * K), 0);
    float* xs = buf((size_t)M * 4, 1);
    float* ws = buf((size_t)N * 4, 1);
    void* y = buf((size_t)(M * N) * 4, 0);
    int32_t* acc = buf((size_t)(M * N) * 4, 0);
    orc_gemm_w8a8_rows(M, N, K, xq, xs, w, ws, y, VDSL_F32, 1, acc, 0, M);
    orc_gemm_w8a8_rows(M, N, K, xq, xs, w, ws, y, VDSL_BF16, 0, NULL, 0, M);
    free(xq); free(w); free(xs); free(ws); free(y); free(acc);
  }
}

static void elementwise(void) {
  const int64_t shapes[][2] = {{1, 1}, {3, 5}, {0, 3}, {8, 64}, {7, 33}};
  for (int s = 0; s < 5; ++s) {
    const int64_t rows = shapes[s][0], cols = shapes[s][1], n = rows * cols;
    for (int a = 0; a < 2; ++a)
      for (int b = 0; b < 2; ++b) {
        void* x = buf((size_t)n * (a == VDSL_F32 ? 4 : 2), a == VDSL_F32);
        void* y = buf((size_t)n * (b == VDSL_F32 ? 4 : 2), 0);
        void* xt = buf((size_t)n * (a == VDSL_F32 ? 4 : 2), 0);
        orc_cast(n, a, x, b, y);
        orc_gelu_fwd(n, a, x, b, y);
        orc_transpose(rows, cols, a, x, xt);
        free(x); free(y); free(xt);
      }
    float* dh = buf((size_t)n * 4, 1);
    float* pre = buf((size_t)n * 4, 1);
    uint16_t* da = buf((size_t)n * 2, 0);
    uint16_t* dat = buf((size_t)n * 2, 0);
    orc_gelu_bwd(rows, cols, dh, pre, da, dat);
    float* loss = buf(4, 0);
    if (n > 0) orc_mse_fwd_bwd(rows, cols, dh, pre, loss, da, dat);
    for (int dt = 0; dt < 2; ++dt) {
      int8_t* q = buf((size_t)n, 0);
      float* sc = buf((size_t)rows * 4, 0);
      orc_quantize_rows_i8(rows, cols, dt, dh, q, sc);
      free(q); free(sc);
    }
    free(dh); free(pre); free(da); free(dat); free(loss);
  }
}

/* Per-pixel programs: an escape loop over two input fields with a count and state read after the
 * loop, every pixel-only opcode, ragged and empty grids, a loop of no trips. */
static void pixel_programs(void) {
  static const vdsl_map_instr code[] = {
      /* pre: r2 = in0 (component 1 of 2), r3 = in1, r4 = 4, r0 = i / 16, r1 = j / 16 */
      {VDSL_MAP_LOAD, 2, 0, 0, 1, {0}, 0.f}, {VDSL_MAP_LOAD, 3, 1, 0, 0, {0}, 0.f}, {VDSL_MAP_CONST, 4, 0, 0, 0, {0}, 4.f},
      {VDSL_PIX_INDEX, 0, 0, 0, 0, {0}, 0.f}, {VDSL_MAP_MUL_IMM, 0, 0, 0, 0, {0}, 0.0625f},
      {VDSL_PIX_INDEX, 1, 1, 0, 0, {0}, 0.f}, {VDSL_MAP_MUL_IMM, 1, 1, 0, 0, {0}, 0.0625f},
      /* test: r5 = r0^2 + r1^2 < r4 */
      {VDSL_MAP_SQUARE, 5, 0, 0, 0, {0}, 0.f}, {VDSL_MAP_SQUARE, 6, 1, 0, 0, {0}, 0.f}, {VDSL_MAP_ADD, 5, 5, 6, 0, {0}, 0.f},
      /* body: (r0, r1) <- (r0^2 - r1^2 + r2, 2 r0 r1 + r3), through selects and floors */
      {VDSL_MAP_SQUARE, 6, 0, 0, 0, {0}, 0.f}, {VDSL_MAP_SQUARE, 7, 1, 0, 0, {0}, 0.f}, {VDSL_MAP_SUB, 6, 6, 7, 0, {0}, 0.f},
      {VDSL_MAP_ADD, 6, 6, 2, 0, {0}, 0.f}, {VDSL_MAP_MUL, 7, 0, 1, 0, {0}, 0.f}, {VDSL_MAP_MUL_IMM, 7, 7, 0, 0, {0}, 2.f},
      {VDSL_MAP_ADD, 7, 7, 3, 0, {0}, 0.f}, {VDSL_PIX_LT, 8, 6, 7, 0, {0}, 0.f},
      {VDSL_PIX_SELECT, 9, 8, 6, 7, {0}, 0.f}, {VDSL_PIX_FLOOR, 10, 9, 0, 0, {0}, 0.f},
      {VDSL_MAP_MOV, 0, 6, 0, 0, {0}, 0.f}, {VDSL_MAP_MOV, 1, 7, 0, 0, {0}, 0.f},
      /* post: r11 = count + cos(r0) + sin(r1) + (r0 == r1) + (r0 != r1) + (r0 <= r1) + r10 */
      {VDSL_PIX_COUNT, 11, 0, 0, 0, {0}, 0.f}, {VDSL_PIX_COS, 12, 0, 0, 0, {0}, 0.f}, {VDSL_MAP_ADD, 11, 11, 12, 0, {0}, 0.f},
      {VDSL_PIX_SIN, 12, 1, 0, 0, {0}, 0.f}, {VDSL_MAP_ADD, 11, 11, 12, 0, {0}, 0.f},
      {VDSL_PIX_EQ, 12, 0, 1, 0, {0}, 0.f}, {VDSL_MAP_ADD, 11, 11, 12, 0, {0}, 0.f},
      {VDSL_PIX_NE, 12, 0, 1, 0, {0}, 0.f}, {VDSL_MAP_ADD, 11, 11, 12, 0, {0}, 0.f},
      {VDSL_PIX_LE, 12, 0, 1, 0, {0}, 0.f}, {VDSL_MAP_ADD, 11, 11, 12, 0, {0}, 0.f}, {VDSL_MAP_ADD, 11, 11, 10, 0, {0}, 0.f},
  };
  vdsl_pixel_program p;
  memset(&p, 0, sizeof p);
  p.n_pre = 7; p.n_test = 3; p.n_body = 12; p.n_post = (int)(sizeof code / sizeof code[0]) - 22;
  p.loop = 1; p.test = VDSL_PIX_TEST_LT; p.test_a = 5; p.test_b = 4;
  p.in_widths[0] = 2; p.in_widths[1] = 1;
  memcpy(p.code, code, sizeof code);
  const int shapes[][2] = {{1, 1}, {7, 13}, {0, 5}, {5, 0}, {33, 17}};
  for (int s = 0; s < 5; ++s) {
    const int64_t ni = shapes[s][0], nj = shapes[s][1];
    for (int variant = 0; variant < 3; ++variant) {
      p.max_iter = variant == 0 ? 0 : 30;
      p.out_kind = variant == 2 ? VDSL_PIX_OUT_COUNT : VDSL_PIX_OUT_REG;
      p.out_width = variant == 1 ? 3 : 1; /* a vec3 field, or scalars */
      p.out_regs[0] = 11; p.out_regs[1] = 0; p.out_regs[2] = 1;
      float* in0 = buf((size_t)(ni * nj) * 8, 1);
      float* in1 = buf((size_t)(ni * nj) * 4, 1);
      const void* ins[2] = {in0, in1};
      void* out = buf((size_t)(ni * nj) * 4 * p.out_width, 0);
      orc_pixel_program_rows(&p, ni, nj, ins, out, 0, ni);
      free(in0); free(in1); free(out);
    }
  }
}

int main(void) {
  escape_time();
  pixel_programs();
  map_chains();
  vec_transform();
  map_chain_mat();
  reductions();
  gemms();
  elementwise();
  printf("sanitize_check: ok\n");
  return 0;
}

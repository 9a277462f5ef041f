/* Test driver, not part of libvdsl.so: the library's host code built under AddressSanitizer and
 * UndefinedBehaviorSanitizer (`make -C vernondsl_amd/csrc sanitize`, device code as usual) and
 * driven through its C ABI.  Every entry point is called with handles, shapes and buffers it must
 * refuse (null and foreign handles, sizes whose byte counts overflow, buffers one element short,
 * bad offsets, graph misuse) and with a small valid workload; every handle is released at the
 * end, so LeakSanitizer sees the library's own allocations.  Prints "abi_check: ok" and exits 0
 * when every call behaved as documented. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "vdsl.h"

static int g_fails = 0;

#define EXPECT_OK(call)                                                                              \
  do {                                                                                               \
    int st_ = (call);                                                                                \
    if (st_ != VDSL_OK) {                                                                            \
      printf("FAIL line %d: %s -> %d (%s)\n", __LINE__, #call, st_, vdsl_last_error());              \
      ++g_fails;                                                                                     \
    }                                                                                                \
  } while (0)

#define EXPECT_ERR(call)                                                                             \
  do {                                                                                               \
    int st_ = (call);                                                                                \
    if (st_ == VDSL_OK) {                                                                            \
      printf("FAIL line %d: %s was accepted\n", __LINE__, #call);                                    \
      ++g_fails;                                                                                     \
    } else if (vdsl_last_error() == NULL || vdsl_last_error()[0] == 0) {                             \
      printf("FAIL line %d: %s failed without a message\n", __LINE__, #call);                        \
      ++g_fails;                                                                                     \
    }                                                                                                \
  } while (0)

static const int64_t kHuge = (int64_t)1 << 62; /* rows * cols * bytes overflows 64 bits */

static vdsl_buffer alloc(vdsl_device d, size_t bytes) {
  vdsl_buffer b = NULL;
  EXPECT_OK(vdsl_buffer_alloc(d, bytes, VDSL_BIND_STORAGE_BUFFER, &b));
  return b;
}

static void fill_f32(vdsl_queue q, vdsl_buffer b, size_t n, float scale) {
  float* h = (float*)malloc(n * 4);
  for (size_t i = 0; i < n; ++i) h[i] = scale * (float)((int)(i % 17) - 8);
  EXPECT_OK(vdsl_buffer_write(q, b, 0, h, n * 4));
  free(h);
}

static void fill_bf16(vdsl_queue q, vdsl_buffer b, size_t n) {
  uint16_t* h = (uint16_t*)malloc(n * 2);
  for (size_t i = 0; i < n; ++i) h[i] = (uint16_t)(0x3F80u + (i % 7)); /* values near 1 */
  EXPECT_OK(vdsl_buffer_write(q, b, 0, h, n * 2));
  free(h);
}

int main(void) {
  setvbuf(stdout, NULL, _IONBF, 0); /* reports reach the log even if a sanitizer ends the run */
  vdsl_device d = NULL;
  vdsl_queue q = NULL;
  int count = 0;

  /* ---- before any device ---- */
  EXPECT_ERR(vdsl_device_open(VDSL_DEVICE_HIP, -1, &d));
  EXPECT_ERR(vdsl_device_open(VDSL_DEVICE_HIP, 0, NULL));
  EXPECT_ERR(vdsl_buffer_free(NULL));
  EXPECT_ERR(vdsl_queue_sync(NULL));
  EXPECT_ERR(vdsl_graph_destroy(NULL));
  EXPECT_ERR(vdsl_op_escape_time(NULL, NULL, NULL));
  EXPECT_OK(vdsl_device_count(VDSL_DEVICE_HIP, &count));
  if (count < 1) {
    printf("abi_check: no device\n");
    return 2;
  }
  EXPECT_OK(vdsl_device_open(VDSL_DEVICE_HIP, 0, &d));
  vdsl_device_info info;
  EXPECT_OK(vdsl_device_get_info(d, &info));
  EXPECT_OK(vdsl_queue_create(d, &q));
  EXPECT_ERR(vdsl_device_get_info((vdsl_device)q, &info)); /* a queue is not a device */
  EXPECT_ERR(vdsl_queue_sync((vdsl_queue)d));

  /* ---- buffers ---- */
  vdsl_buffer a = alloc(d, 4096), b = alloc(d, 4096), c = alloc(d, 4096);
  size_t sz = 0;
  EXPECT_OK(vdsl_buffer_size(a, &sz));
  if (sz != 4096) { printf("FAIL buffer size %zu\n", sz); ++g_fails; }
  vdsl_buffer refused = NULL;
  EXPECT_ERR(vdsl_buffer_alloc(d, (size_t)1 << 62, VDSL_BIND_STORAGE_BUFFER, &refused)); /* out of memory */
  EXPECT_ERR(vdsl_buffer_alloc(d, 16, 99, &refused));                                     /* binding kind */
  if (refused != NULL) { printf("FAIL refused allocation returned a handle\n"); ++g_fails; }
  char host[64] = {0};
  EXPECT_ERR(vdsl_buffer_write(q, a, 4090, host, 16));          /* past the end */
  EXPECT_ERR(vdsl_buffer_write(q, a, SIZE_MAX - 4, host, 16));  /* offset + bytes overflows */
  EXPECT_ERR(vdsl_buffer_read(q, a, 4096, host, 1));
  EXPECT_ERR(vdsl_buffer_fill_u32(q, a, 2, 8, 0u));             /* unaligned */
  EXPECT_ERR(vdsl_buffer_copy(q, b, 0, a, 1, 4096));
  EXPECT_OK(vdsl_buffer_fill_u32(q, a, 0, 4096, 0x3F800000u));
  EXPECT_OK(vdsl_buffer_copy(q, b, 0, a, 0, 4096));
  EXPECT_OK(vdsl_buffer_read(q, b, 4092, host, 4));
  EXPECT_OK(vdsl_queue_sync(q));
  float one = 0.0f;
  memcpy(&one, host, 4);
  if (one != 1.0f) { printf("FAIL copy read back %g\n", one); ++g_fails; }

  /* ---- op class 1: escape time and per-pixel programs ---- */
  vdsl_escape_time_params p;
  memset(&p, 0, sizeof p);
  p.ni = 7; p.nj = 13; p.family = VDSL_ESC_JULIA; p.escape_test = VDSL_ESC_NORM_GE; p.out_kind = VDSL_ESC_OUT_F32_AFFINE;
  p.max_iter = 50; p.bound = 20.0f; p.re_den = 7.0f; p.re_off = -1.0f; p.re_scale = 2.0f; p.im_den = 7.0f;
  p.im_off = -0.5f; p.im_scale = 2.0f; p.c_re = -0.8f; p.c_im = 0.2f; p.out_base = 1.0f; p.out_scale = -0.02f;
  EXPECT_OK(vdsl_op_escape_time(q, &p, a));
  p.ni = 100; p.nj = 100; /* 40000 bytes > 4096 */
  EXPECT_ERR(vdsl_op_escape_time(q, &p, a));
  p.ni = 7; p.max_iter = -1;
  EXPECT_ERR(vdsl_op_escape_time(q, &p, a));

  vdsl_pixel_program pp;
  memset(&pp, 0, sizeof pp);
  pp.n_pre = 2; pp.n_post = 1; pp.out_width = 1; pp.out_regs[0] = 2;
  pp.code[0].op = VDSL_PIX_INDEX; pp.code[0].dst = 0; pp.code[0].a = 0;
  pp.code[1].op = VDSL_PIX_INDEX; pp.code[1].dst = 1; pp.code[1].a = 1;
  pp.code[2].op = VDSL_PIX_SELECT; pp.code[2].dst = 2; pp.code[2].a = 0; pp.code[2].b = 1; pp.code[2].c = 0;
  EXPECT_OK(vdsl_op_pixel_program(q, 8, 16, &pp, NULL, 0, a));
  EXPECT_ERR(vdsl_op_pixel_program(q, 64, 64, &pp, NULL, 0, a)); /* out too small */
  EXPECT_ERR(vdsl_op_pixel_program(q, 8, 16, &pp, NULL, VDSL_PIX_MAX_INPUTS + 1, a));  /* too many inputs */
  pp.out_width = 5;
  EXPECT_ERR(vdsl_op_pixel_program(q, 8, 16, &pp, NULL, 0, a));  /* at most 4 components */
  pp.out_width = 4;
  EXPECT_OK(vdsl_op_pixel_program(q, 8, 16, &pp, NULL, 0, a));   /* a vec4 field: 2048 bytes */
  EXPECT_ERR(vdsl_op_pixel_program(q, 32, 16, &pp, NULL, 0, a)); /* 8192 bytes > 4096 */
  pp.out_width = 1;
  pp.code[2].c = VDSL_PIX_MAX_REGS;
  EXPECT_ERR(vdsl_op_pixel_program(q, 8, 16, &pp, NULL, 0, a));  /* register out of range */

  /* scatter-adds: total[0][0] += j for every pixel, into an f32 [1][1] input; no output */
  vdsl_pixel_program sp;
  memset(&sp, 0, sizeof sp);
  sp.n_post = 2; sp.out_kind = VDSL_PIX_OUT_NONE; sp.out_width = 1;
  sp.in_widths[0] = 1; sp.in_dtypes[0] = VDSL_F32; sp.in_rows[0] = 1; sp.in_cols[0] = 1;
  sp.code[0].op = VDSL_PIX_INDEX; sp.code[0].dst = 1; sp.code[0].a = 1;
  sp.code[1].op = VDSL_PIX_ATOMIC_ADD; sp.code[1].dst = 1; sp.code[1].a = 0; sp.code[1].b = 0; sp.code[1].c = 0;
  vdsl_buffer tot = alloc(d, 4);
  fill_f32(q, tot, 1, 0.0f);
  EXPECT_OK(vdsl_op_pixel_program(q, 8, 16, &sp, &tot, 1, NULL));
  sp.code[1].imm = 1.0f;  /* component 1 of a field of scalars */
  EXPECT_ERR(vdsl_op_pixel_program(q, 8, 16, &sp, &tot, 1, NULL));
  sp.code[1].imm = 0.0f;
  EXPECT_ERR(vdsl_op_pixel_program(q, 8, 16, &sp, &tot, 0, NULL));  /* no input 0 */
  sp.out_kind = VDSL_PIX_OUT_REG;
  EXPECT_ERR(vdsl_op_pixel_program(q, 8, 16, &sp, &tot, 1, NULL));  /* a stored output needs its buffer */
  EXPECT_OK(vdsl_buffer_free(tot));

  /* ---- op class 2: map chains ---- */
  vdsl_map_instr code[3];
  memset(code, 0, sizeof code);
  code[0].op = VDSL_MAP_LOAD; code[0].dst = 0; code[0].a = 0;
  code[1].op = VDSL_MAP_TANH; code[1].dst = 1; code[1].a = 0;
  code[2].op = VDSL_MAP_ADD_IMM; code[2].dst = 2; code[2].a = 1; code[2].imm = 0.5f;
  vdsl_map_input in = {b, VDSL_BCAST_FULL, VDSL_F32};
  fill_f32(q, b, 1024, 0.25f);
  EXPECT_OK(vdsl_op_map_chain(q, 8, 128, code, 3, &in, 1, 2, c));
  EXPECT_ERR(vdsl_op_map_chain(q, 1, kHuge, code, 3, &in, 1, 2, c)); /* byte count overflows */
  EXPECT_ERR(vdsl_op_map_chain(q, 8, 129, code, 3, &in, 1, 2, c));   /* one element short */
  EXPECT_ERR(vdsl_op_map_chain(q, 8, 128, code, 3, &in, 1, 9, c));   /* out_reg */
  vdsl_map_vinput vin = {b, VDSL_BCAST_FULL, VDSL_F32, 4, 0};
  const int32_t regs[4] = {2, 1, 0, 0};
  vdsl_map_instr vcode[3];
  memset(vcode, 0, sizeof vcode);
  for (int k = 0; k < 3; ++k) { vcode[k].op = VDSL_MAP_LOAD; vcode[k].dst = (uint8_t)k; vcode[k].a = 0; vcode[k].c = (uint8_t)k; }
  EXPECT_OK(vdsl_op_map_chain_v(q, 2, 128, vcode, 3, &vin, 1, regs, 4, c));
  EXPECT_ERR(vdsl_op_map_chain_v(q, 2, 128, vcode, 3, &vin, 1, regs, 5, c));
  EXPECT_ERR(vdsl_op_map_chain_v(q, kHuge, kHuge, vcode, 3, &vin, 1, regs, 4, c));

  /* vec transform: 16 vec3 positions, one mat4 */
  vdsl_buffer mats = alloc(d, 3 * 64);
  fill_f32(q, mats, 48, 0.125f);
  EXPECT_OK(vdsl_op_vec_transform(q, 16, 3, b, 1, mats, c, NULL));
  EXPECT_ERR(vdsl_op_vec_transform(q, 16, 3, b, 4, mats, c, NULL));      /* at most 3 matrices */
  EXPECT_ERR(vdsl_op_vec_transform(q, kHuge, 3, b, 1, mats, c, NULL));

  /* ---- op class 3: reductions ---- */
  vdsl_buffer rs = alloc(d, 64), rm = alloc(d, 64);
  EXPECT_OK(vdsl_op_row_reduce_softmax(q, 4, 256, VDSL_F32, b, rs, rm, c));
  EXPECT_OK(vdsl_op_row_reduce_softmax(q, 3, 100, VDSL_F32, b, rs, rm, c)); /* generic width */
  EXPECT_ERR(vdsl_op_row_reduce_softmax(q, 1, kHuge, VDSL_F32, b, rs, rm, c));
  EXPECT_ERR(vdsl_op_row_reduce_softmax(q, 17, 64, VDSL_F32, b, rs, rm, c)); /* row_sum holds 16 */
  EXPECT_ERR(vdsl_op_row_reduce_softmax(q, 4, 256, 99, b, rs, rm, c));
  EXPECT_OK(vdsl_op_col_reduce(q, 64, 16, VDSL_F32, b, rs, rm));
  EXPECT_ERR(vdsl_op_col_reduce(q, kHuge, 16, VDSL_F32, b, rs, rm));

  /* ---- layout and elementwise ---- */
  EXPECT_OK(vdsl_op_transpose(q, 16, 32, VDSL_BF16, b, c));
  EXPECT_ERR(vdsl_op_transpose(q, kHuge, 4, VDSL_BF16, b, c));
  EXPECT_OK(vdsl_op_cast(q, 512, VDSL_F32, b, VDSL_BF16, c));
  EXPECT_ERR(vdsl_op_cast(q, 2048, VDSL_F32, b, VDSL_BF16, c));
  EXPECT_OK(vdsl_op_gelu_fwd(q, 1024, VDSL_F32, b, VDSL_F32, c));
  EXPECT_ERR(vdsl_op_gelu_fwd(q, kHuge, VDSL_F32, b, VDSL_F32, c));

  /* ---- op class 4: bf16 GEMM, autodiff pieces ---- */
  {
    const int64_t M = 32, N = 32, K = 64;
    vdsl_buffer A = alloc(d, (size_t)(M * K * 2)), B = alloc(d, (size_t)(N * K * 2));
    vdsl_buffer C = alloc(d, (size_t)(M * N * 4)), pre = alloc(d, (size_t)(M * N * 4));
    fill_bf16(q, A, (size_t)(M * K));
    fill_bf16(q, B, (size_t)(N * K));
    size_t ws = 0;
    EXPECT_OK(vdsl_gemm_bf16_workspace_bytes(1, 0, M, N, K, &ws));
    vdsl_buffer W = alloc(d, ws ? ws : 16);
    EXPECT_OK(vdsl_op_gemm_bf16(q, 0, 1, M, N, K, A, B, C, VDSL_F32, VDSL_EPI_NONE, NULL, W));
    EXPECT_OK(vdsl_op_gemm_bf16(q, 0, 1, M, N, K, A, B, C, VDSL_BF16, VDSL_EPI_GELU, pre, W));
    EXPECT_OK(vdsl_op_gemm_bf16(q, 1, 0, M, N, K, A, B, C, VDSL_F32, VDSL_EPI_RELU, NULL, W));
    EXPECT_ERR(vdsl_op_gemm_bf16(q, 0, 1, M, N, K + 64, A, B, C, VDSL_F32, VDSL_EPI_NONE, NULL, W));
    EXPECT_ERR(vdsl_op_gemm_bf16(q, 0, 1, kHuge, kHuge, K, A, B, C, VDSL_F32, VDSL_EPI_NONE, NULL, W));
    EXPECT_ERR(vdsl_op_gemm_bf16(q, 0, 1, M, N, K, A, B, C, VDSL_F32, 42, NULL, W));
    vdsl_buffer da = alloc(d, (size_t)(M * N * 2)), dat = alloc(d, (size_t)(M * N * 2));
    EXPECT_OK(vdsl_op_gelu_bwd(q, M, N, C, pre, da, dat));
    EXPECT_ERR(vdsl_op_gelu_bwd(q, M, 2 * N, C, pre, da, dat));
    EXPECT_OK(vdsl_op_relu_bwd(q, M, N, C, pre, da, NULL));
    EXPECT_ERR(vdsl_op_relu_bwd(q, kHuge, N, C, pre, da, dat));
    EXPECT_OK(vdsl_op_add(q, M * N, VDSL_F32, C, VDSL_F32, pre, VDSL_F32, C));
    EXPECT_OK(vdsl_op_add(q, M * N - 3, VDSL_BF16, da, VDSL_F32, pre, VDSL_BF16, dat));
    EXPECT_ERR(vdsl_op_add(q, M * N, VDSL_F32, C, VDSL_F32, pre, VDSL_BF16, C));
    EXPECT_ERR(vdsl_op_add(q, 2 * M * N, VDSL_F32, C, VDSL_F32, pre, VDSL_F32, C));
    EXPECT_ERR(vdsl_op_add(q, M * N, VDSL_I8, C, VDSL_F32, pre, VDSL_F32, C));
    const int64_t parts = vdsl_mse_partials_count(M, N);
    vdsl_buffer loss = alloc(d, 4), part = alloc(d, (size_t)(parts > 0 ? parts : 1) * 8);
    EXPECT_OK(vdsl_op_mse_fwd_bwd(q, M, N, C, pre, loss, da, dat, part));
    EXPECT_ERR(vdsl_op_mse_fwd_bwd(q, kHuge, N, C, pre, loss, da, dat, part));
    /* int8: quantise A's rows, W8A8 GEMM against B's bytes */
    vdsl_buffer xq = alloc(d, (size_t)(M * K)), xs = alloc(d, (size_t)M * 4), wq = alloc(d, (size_t)(N * K));
    vdsl_buffer wsc = alloc(d, (size_t)N * 4), y = alloc(d, (size_t)(M * N * 4));
    EXPECT_OK(vdsl_op_quantize_rows_i8(q, M, K, VDSL_BF16, A, xq, xs));
    EXPECT_ERR(vdsl_op_quantize_rows_i8(q, kHuge, K, VDSL_BF16, A, xq, xs));
    EXPECT_OK(vdsl_op_quantize_rows_i8(q, N, K, VDSL_BF16, B, wq, wsc));
    size_t ws8 = 0;
    EXPECT_OK(vdsl_gemm_w8a8_workspace_bytes(M, N, K, &ws8));
    vdsl_buffer W8 = alloc(d, ws8 ? ws8 : 16);
    EXPECT_OK(vdsl_op_gemm_w8a8(q, M, N, K, xq, xs, wq, wsc, y, VDSL_F32, 1, NULL, W8));
    EXPECT_ERR(vdsl_op_gemm_w8a8(q, M, N, 2 * K, xq, xs, wq, wsc, y, VDSL_F32, 1, NULL, W8));
    EXPECT_ERR(vdsl_op_gemm_w8a8_packed_noalloc(q, kHuge, N, K, xq, xs, wq, wsc, y, VDSL_F32, 1, NULL));
    EXPECT_OK(vdsl_queue_sync(q));
    float out[4] = {0};
    EXPECT_OK(vdsl_buffer_read(q, y, 0, out, sizeof out));
    EXPECT_OK(vdsl_queue_sync(q));
    for (int k = 0; k < 4; ++k)
      if (!isfinite(out[k])) { printf("FAIL w8a8 output %g\n", out[k]); ++g_fails; }
    vdsl_buffer bufs[] = {A, B, C, pre, W, da, dat, loss, part, xq, xs, wq, wsc, y, W8};
    for (size_t k = 0; k < sizeof bufs / sizeof bufs[0]; ++k) EXPECT_OK(vdsl_buffer_free(bufs[k]));
  }

  /* ---- graphs and events ---- */
  vdsl_graph g = NULL;
  EXPECT_ERR(vdsl_graph_end(q, &g)); /* not recording */
  EXPECT_OK(vdsl_graph_begin(q));
  EXPECT_ERR(vdsl_graph_begin(q));   /* already recording */
  EXPECT_ERR(vdsl_queue_sync(q));    /* no synchronisation while recording */
  EXPECT_OK(vdsl_op_map_chain(q, 8, 128, code, 3, &in, 1, 2, c));
  EXPECT_OK(vdsl_graph_end(q, &g));
  vdsl_event e0 = NULL, e1 = NULL;
  EXPECT_OK(vdsl_event_create(d, &e0));
  EXPECT_OK(vdsl_event_create(d, &e1));
  EXPECT_OK(vdsl_event_record(e0, q));
  EXPECT_OK(vdsl_graph_launch(g, q));
  EXPECT_OK(vdsl_graph_launch(g, q));
  EXPECT_OK(vdsl_event_record(e1, q));
  float ms = -1.0f;
  EXPECT_OK(vdsl_event_elapsed_ms(e0, e1, &ms));
  if (!(ms >= 0.0f)) { printf("FAIL elapsed %g\n", ms); ++g_fails; }
  EXPECT_ERR(vdsl_event_elapsed_ms(e0, NULL, &ms));
  EXPECT_OK(vdsl_queue_sync(q));
  EXPECT_OK(vdsl_graph_destroy(g));
  EXPECT_OK(vdsl_event_destroy(e0));
  EXPECT_OK(vdsl_event_destroy(e1));

  /* ---- release everything: the device refuses to close while handles are live ---- */
  EXPECT_ERR(vdsl_device_close(d));
  vdsl_buffer rest[] = {a, b, c, mats, rs, rm};
  for (size_t k = 0; k < sizeof rest / sizeof rest[0]; ++k) EXPECT_OK(vdsl_buffer_free(rest[k]));
  EXPECT_OK(vdsl_queue_destroy(q));
  EXPECT_OK(vdsl_device_close(d));
  if (g_fails) {
    printf("abi_check: %d failures\n", g_fails);
    return 1;
  }
  printf("abi_check: ok\n");
  return 0;
}

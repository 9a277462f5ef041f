/*
 * vdsl.h - C ABI of the MI355X (gfx950) HIP device for VernonDSL's tensor-op hot path.
 *
 * The reference (morphling666/VernonDSL) has no C ABI, FFI or runtime: its only backend
 * seam is the MLIR pass plugin
 *     std::unique_ptr<mlir::Pass> mlir::vernon::createVernonToSPIRVPass();   VernonToSpirv.h:7-9
 *     void mlir::vernon::registerVernonToSPIRVPass();                        VernonToSpirv.cpp:71-75
 * and its only executing program is the Taichi kernel `paint` in fractal.py:16-25, which runs
 * inside third-party Taichi 1.7.4 (`ti.init(arch=...)`, fractal.py:5, selects the backend).
 * This header is the boundary that replaces both: a front end (the Python package
 * `vernondsl_amd`, or any ctypes/cffi/C++ caller) lowers a DSL program to the op classes below
 * and drives them through opaque handles.  Each declaration names the reference item it stands
 * in for.
 *
 * Conventions
 *  - Every function returns int: 0 (VDSL_OK) or a negative vdsl_status.  On failure
 *    vdsl_last_error() returns a thread-local message.  Nothing aborts the process.
 *  - Handles are opaque and owned by the caller; each is released by its *_destroy/_free/_close.
 *    A buffer belongs to the device it was allocated on.
 *  - Op calls are asynchronous: they enqueue work on the queue (one hipStream_t) and return.
 *    vdsl_buffer_read and vdsl_queue_sync block.
 *  - A queue is used by one host thread at a time; different queues may be used concurrently.
 *  - Between vdsl_graph_begin(q) and vdsl_graph_end(q, &g) op calls on q are recorded, not run;
 *    vdsl_graph_launch replays the whole recording as one hipGraph.  Host<->device transfers
 *    (vdsl_buffer_write/read) are rejected while a queue is capturing.
 *  - Tensors are dense and row-major.  "rows x cols" means cols is the contiguous axis.
 *  - bf16 is stored as uint16 (the upper half of an IEEE binary32); conversions round to
 *    nearest-even.
 */
#ifndef VDSL_H
#define VDSL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 3: vdsl_map_instr.ext and vdsl_map_vinput.mat_dim (matrix operands); 4: VDSL_PIX_TRIP,
 * vdsl_op_relu_bwd, vdsl_op_add (struct layouts unchanged since 3); 5: vdsl_pixel_program.in_rows
 * and in_cols (inputs of another shape than the grid); 6: VDSL_PIX_ATOMIC_ADD,
 * VDSL_PIX_OUT_NONE (scatter-adds) and VDSL_PIX_TRUNC (struct layouts unchanged since 5); 7:
 * VDSL_PIX_MAX_INSTR 256 and VDSL_PIX_MAX_INPUTS 8 (vdsl_pixel_program's arrays grow),
 * VDSL_PIX_ATOMIC_MAX / MIN, VDSL_PIX_STORE_AT, VDSL_PIX_RANDOM, VDSL_PIX_ATAN2 ... POWF and
 * the bit operations VDSL_PIX_BAND ... SHR, VDSL_PIX_ROUND. */
#define VDSL_ABI_VERSION 7

typedef enum vdsl_status {
  VDSL_OK = 0,
  VDSL_ERR_INVALID_ARG = -1,     /* bad enum, null pointer, negative size, ... */
  VDSL_ERR_INVALID_HANDLE = -2,  /* null or already-released handle */
  VDSL_ERR_OUT_OF_MEMORY = -3,   /* device allocation failed (real or injected) */
  VDSL_ERR_DEVICE = -4,          /* a HIP runtime call failed; message has the HIP error */
  VDSL_ERR_UNSUPPORTED = -5,     /* valid request this build does not implement */
  VDSL_ERR_CAPTURE = -6,         /* graph-capture misuse (nested begin, end without begin, ...) */
  VDSL_ERR_SHAPE = -7,           /* operand shape / buffer size mismatch */
  VDSL_ERR_NO_DEVICE = -8        /* no HIP device with that ordinal */
} vdsl_status;

typedef enum vdsl_device_kind {
  /* `arch=ti.hip` in the front end; ti.init(arch=...) at fractal.py:5 is the reference's
   * backend switch.  The CPU executor is test infrastructure (oracle/) and is not a device of
   * this library. */
  VDSL_DEVICE_HIP = 1
} vdsl_device_kind;

/* Buffer binding kinds: the vocabulary of the `vernon.semantic` argument attribute that
 * VernonToSPIRVPass maps to SPIR-V storage classes (VernonToSpirv.cpp:43-56; used in
 * color.mlir:4-9,43-45).  Ops may read any kind; UNIFORM_CONSTANT buffers are read-only on the
 * device, and an op that would write one fails with VDSL_ERR_INVALID_ARG.  An OUTPUT buffer holds
 * a result for the host: a bf16 GEMM storing a plain f32 result into one (vdsl_op_gemm_bf16,
 * vdsl_op_gemm_bf16_packed) uses streaming (non-temporal) stores, so later device work that
 * reads it right away may run slower than from a STORAGE_BUFFER; the values are the same. */
typedef enum vdsl_binding {
  VDSL_BIND_STORAGE_BUFFER = 0,  /* "storage_buffer": read-write (default) */
  VDSL_BIND_INPUT = 1,           /* "input" */
  VDSL_BIND_OUTPUT = 2,          /* "output" */
  VDSL_BIND_UNIFORM = 3,         /* "uniform" */
  VDSL_BIND_UNIFORM_CONSTANT = 4,/* "uniform_constant": device read-only */
  VDSL_BIND_IMAGE = 5,           /* "image" (the pass maps it to the Input class) */
  VDSL_BIND_VARYING = 6          /* "varying" (color.mlir:9,44; unmapped by the pass) */
} vdsl_binding;

typedef enum vdsl_dtype {
  VDSL_F32 = 0,
  VDSL_BF16 = 1,
  VDSL_I8 = 2,
  VDSL_I32 = 3
} vdsl_dtype;

typedef struct vdsl_device_s* vdsl_device;
typedef struct vdsl_buffer_s* vdsl_buffer;
typedef struct vdsl_queue_s* vdsl_queue;
typedef struct vdsl_graph_s* vdsl_graph;
typedef struct vdsl_event_s* vdsl_event;

typedef struct vdsl_device_info {
  char name[64];          /* marketing name, e.g. "AMD Instinct MI355X" */
  char arch[32];          /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
  int32_t compute_units;
  int32_t clock_khz;
  int32_t wavefront_size;
  int32_t lds_bytes_per_block;
  uint64_t hbm_bytes;
} vdsl_device_info;

/* ---- errors / version -------------------------------------------------------------------- */
const char* vdsl_last_error(void);
int vdsl_abi_version(void);

/* ---- device (replaces ti.init(arch=...), fractal.py:5) ------------------------------------ */
int vdsl_device_count(int kind, int* count);
int vdsl_device_open(int kind, int ordinal, vdsl_device* out);
int vdsl_device_close(vdsl_device dev);
int vdsl_device_get_info(vdsl_device dev, vdsl_device_info* info);

/* ---- buffers (replaces ti.field storage, fractal.py:8; binding kinds VernonToSpirv.cpp:43-56) */
int vdsl_buffer_alloc(vdsl_device dev, size_t bytes, int binding, vdsl_buffer* out);
int vdsl_buffer_free(vdsl_buffer buf);
int vdsl_buffer_size(vdsl_buffer buf, size_t* bytes);
int vdsl_buffer_binding(vdsl_buffer buf, int* binding);
/* Device address of the allocation, for interop with other HIP code in the same process. */
int vdsl_buffer_device_address(vdsl_buffer buf, uint64_t* address);
/* Host -> device.  Returns once `src` may be reused. */
int vdsl_buffer_write(vdsl_queue q, vdsl_buffer buf, size_t offset, const void* src, size_t bytes);
/* Device -> host.  Blocks until `dst` holds the data (replaces gui.set_image's read-back,
 * fractal.py:32). */
int vdsl_buffer_read(vdsl_queue q, vdsl_buffer buf, size_t offset, void* dst, size_t bytes);
/* Fill with a repeated 32-bit pattern using a kernel (safe to record into a graph).
 * offset and bytes must be multiples of 4. */
int vdsl_buffer_fill_u32(vdsl_queue q, vdsl_buffer buf, size_t offset, size_t bytes, uint32_t pattern);
int vdsl_buffer_copy(vdsl_queue q, vdsl_buffer dst, size_t dst_offset, vdsl_buffer src,
                     size_t src_offset, size_t bytes);

/* ---- queues ------------------------------------------------------------------------------ */
int vdsl_queue_create(vdsl_device dev, vdsl_queue* out);
int vdsl_queue_destroy(vdsl_queue q);
int vdsl_queue_sync(vdsl_queue q);

/* ---- execution-graph replay (one hipGraph per recorded op sequence) ------------------------ */
int vdsl_graph_begin(vdsl_queue q);
int vdsl_graph_end(vdsl_queue q, vdsl_graph* out);
int vdsl_graph_launch(vdsl_graph g, vdsl_queue q);
int vdsl_graph_destroy(vdsl_graph g);

/* ---- timing (hipEvents on the queue's own stream) ----------------------------------------- */
int vdsl_event_create(vdsl_device dev, vdsl_event* out);
int vdsl_event_record(vdsl_event ev, vdsl_queue q);
/* Waits for `end`, then returns the elapsed milliseconds between the two records. */
int vdsl_event_elapsed_ms(vdsl_event start, vdsl_event end, float* ms);
int vdsl_event_destroy(vdsl_event ev);

/* ========================================================================================== */
/* Op class 1: per-pixel escape-time iterative map.                                           */
/* Replaces the body of `paint(t)` (fractal.py:16-25): struct-for over the field (:18), the   */
/* pixel -> complex map (:20), the check-then-update loop (:22-24) built on complex_sqr        */
/* (:11-13), and the store (:25).                                                             */
/* ========================================================================================== */
typedef enum vdsl_escape_family {
  VDSL_ESC_MANDELBROT = 0,  /* z0 = 0, c = pixel coordinate */
  VDSL_ESC_JULIA = 1        /* z0 = pixel coordinate, c = (c_re, c_im)  (fractal.py:19-20) */
} vdsl_escape_family;

typedef enum vdsl_escape_test {
  VDSL_ESC_MAG2_GT = 0,     /* stop when zr*zr + zi*zi > bound  (config-1 form, bound = 4) */
  VDSL_ESC_NORM_GE = 1      /* continue while sqrt(zr*zr + zi*zi) < bound (fractal.py:22) */
} vdsl_escape_test;

typedef enum vdsl_escape_rounding {
  /* every product and sum rounded separately, in the order of complex_sqr (fractal.py:13):
   *   m = zr*zr + zi*zi;  zr' = (zr*zr - zi*zi) + cr;  zi' = ((zi*zr)*2) + ci               */
  VDSL_ESC_ROUND_SEPARATE = 0,
  /* fused multiply-add form (one rounding per fma):
   *   q = zi*zi;  m = fma(zr,zr,q);  zr' = fma(zr,zr,-q) + cr;  zi' = fma(zr+zr, zi, ci)      */
  VDSL_ESC_ROUND_FMA = 1
} vdsl_escape_rounding;

typedef enum vdsl_escape_output {
  VDSL_ESC_OUT_I32_COUNT = 0,   /* int32 iteration count */
  VDSL_ESC_OUT_F32_AFFINE = 1   /* f32 out_base + float(count) * out_scale (fractal.py:25) */
} vdsl_escape_output;

typedef struct vdsl_escape_time_params {
  int32_t ni;          /* extent of the outer axis i (real part); rows of the output */
  int32_t nj;          /* extent of the inner axis j (imaginary part); contiguous */
  int32_t family;      /* vdsl_escape_family */
  int32_t escape_test; /* vdsl_escape_test */
  int32_t rounding;    /* vdsl_escape_rounding */
  int32_t out_kind;    /* vdsl_escape_output */
  int32_t max_iter;    /* >= 0 */
  float bound;
  /* coordinate map, every step rounded in f32:  re = ((float(i) / re_den) + re_off) * re_scale + re_post
   * fractal.py:20 is (i/n - 1) * 2; the config-1 window is (i/1024) * 3 + (-2). */
  float re_den, re_off, re_scale, re_post;
  float im_den, im_off, im_scale, im_post;
  float c_re, c_im;    /* Julia constant (fractal.py:19) */
  float out_base, out_scale;
} vdsl_escape_time_params;

/* out: int32 or f32 [ni][nj] per out_kind. */
int vdsl_op_escape_time(vdsl_queue q, const vdsl_escape_time_params* p, vdsl_buffer out);

/* ========================================================================================== */
/* Op class 2: fused elementwise / broadcast map chain (no reference code; north-star op      */
/* class).  A chain is a straight-line register program evaluated per output element.         */
/* ========================================================================================== */
#define VDSL_MAP_MAX_INSTR 32
#define VDSL_MAP_MAX_REGS 8
#define VDSL_MAP_MAX_INPUTS 4

typedef enum vdsl_map_opcode {
  VDSL_MAP_LOAD = 1,    /* r[dst] = input[a] at this element (per the input's broadcast) */
  VDSL_MAP_CONST = 2,   /* r[dst] = imm */
  VDSL_MAP_MOV = 3,     /* r[dst] = r[a] */
  VDSL_MAP_NEG = 4,
  VDSL_MAP_ABS = 5,
  VDSL_MAP_SQUARE = 6,  /* r[a] * r[a] */
  VDSL_MAP_EXP = 7,
  VDSL_MAP_LOG = 8,
  VDSL_MAP_TANH = 9,
  VDSL_MAP_SIGMOID = 10,/* 1 / (1 + exp(-r[a])) */
  VDSL_MAP_RELU = 11,   /* max(r[a], 0) */
  VDSL_MAP_SQRT = 12,
  VDSL_MAP_RECIP = 13,  /* 1 / r[a] */
  VDSL_MAP_ADD = 14,    /* r[a] + r[b] */
  VDSL_MAP_SUB = 15,
  VDSL_MAP_MUL = 16,
  VDSL_MAP_DIV = 17,
  VDSL_MAP_MAX = 18,
  VDSL_MAP_MIN = 19,
  VDSL_MAP_FMA = 20,    /* fma(r[a], r[b], r[c]), one rounding */
  VDSL_MAP_MUL_IMM = 21,/* r[a] * imm */
  VDSL_MAP_ADD_IMM = 22,/* r[a] + imm */
  /* Matrix-vector products (vdsl_op_map_chain_v only; input a must be a matrix input, n = its
   * mat_dim): the vector is v = (r[b], r[ext[0]], r[ext[1]], r[ext[2]]) cut to n components and
   * c selects the output component.  linalg.matvec's accumulation into a zero-initialised
   * output (color.mlir:29-36), every product and sum rounded to f32, no fused multiply-add:
   *   MATVEC: r[dst] = ((0 + M[c][0] v0) + M[c][1] v1) + ...   (row c of M times v: M v)
   *   VECMAT: r[dst] = ((0 + v0 M[0][c]) + v1 M[1][c]) + ...   (v times column c: v^T M)
   * Every operand register is read before r[dst] is written, so dst may be one of them. */
  VDSL_MAP_MATVEC = 23,
  VDSL_MAP_VECMAT = 24
} vdsl_map_opcode;

typedef struct vdsl_map_instr {
  uint8_t op, dst, a, b, c;
  uint8_t ext[3];       /* VDSL_MAP_MATVEC / VECMAT: registers of vector components 1..3; else 0 */
  float imm;
} vdsl_map_instr;

typedef enum vdsl_broadcast {
  VDSL_BCAST_FULL = 0,   /* [rows][cols] */
  VDSL_BCAST_ROW = 1,    /* [cols]: one value per column, shared by every row (a row bias) */
  VDSL_BCAST_COL = 2,    /* [rows]: one value per row */
  VDSL_BCAST_SCALAR = 3  /* [1] */
} vdsl_broadcast;

typedef struct vdsl_map_input {
  vdsl_buffer buf;
  int32_t bcast;        /* vdsl_broadcast */
  int32_t dtype;        /* VDSL_F32 */
} vdsl_map_input;

/* out (f32 [rows][cols]) = r[out_reg] after running `code` for each element.  A LOAD's `c` field
 * must be 0 here (scalar inputs). */
int vdsl_op_map_chain(vdsl_queue q, int64_t rows, int64_t cols, const vdsl_map_instr* code,
                      int32_t n_instr, const vdsl_map_input* inputs, int32_t n_inputs,
                      int32_t out_reg, vdsl_buffer out);

/* ---- vector and matrix operands: the vernon dialect's vec2-4 / mat2-4 vocabulary ------------ */
/* (source/README.md:23-55.)  A map-chain input whose elements are f32 vectors of `width` (1..4)
 * components (!vernon.vec2-4 element types, mat_dim 0) or f32 mat2 / mat3 / mat4 matrices
 * (!vernon.mat2-4, mat_dim 2..4, width = mat_dim * mat_dim), stored AoS: element e of a FULL input
 * is the floats [e*width, e*width+width), a matrix row-major (component r * mat_dim + c is M[r][c]);
 * a ROW input holds [cols][width], a COL input [rows][width], a SCALAR input [width] (a uniform,
 * such as the mat4 uniforms of color.mlir:5-7). */
typedef struct vdsl_map_vinput {
  vdsl_buffer buf;
  int32_t bcast;        /* vdsl_broadcast (a vector or matrix counts as one element) */
  int32_t dtype;        /* VDSL_F32 */
  int32_t width;        /* components per element: 1..4 for a vector, mat_dim^2 for a matrix */
  int32_t mat_dim;      /* 0: a vector; 2, 3, 4: a mat2, mat3, mat4 */
} vdsl_map_vinput;

/* The map chain over vector and matrix operands.  A LOAD (op = VDSL_MAP_LOAD, a = input, c =
 * component) reads one component of its input's element: ExtractComponentOp (README.md:41-45)
 * fused into the load, for a matrix component c = row * mat_dim + col; a swizzle (SwizzleOp,
 * README.md:47-52) is several such loads, or the order of out_regs.  VDSL_MAP_MATVEC / VECMAT
 * multiply a matrix input's element by a vector held in registers (linalg.matvec of
 * color.mlir:29-36), one output component per instruction.
 * out: f32 [rows][cols][out_width] (AoS, out_width 1..4); component k of each element is
 * r[out_regs[k]] (tensor.from_elements of color.mlir:21,55).  Components are moved, never
 * rounded: a chain of loads and stores only is an exact permutation. */
int vdsl_op_map_chain_v(vdsl_queue q, int64_t rows, int64_t cols, const vdsl_map_instr* code,
                        int32_t n_instr, const vdsl_map_vinput* inputs, int32_t n_inputs,
                        const int32_t* out_regs, int32_t out_width, vdsl_buffer out);

/* ---- general per-pixel programs: the body of a struct-for over a 2-D field ------------------ */
/* The general form of op class 1 (fractal.py:16-25): what a Taichi @ti.kernel `for i, j in F:`
 * body computes per pixel, as a register program of four sections run in order on 32 f32
 * registers (all 0 at the start):
 *   pre  (code[0, n_pre)):            per-pixel set-up (index maps, field reads, constants);
 *   loop (code[n_pre, +n_test) test, code[.., +n_body) body): when `loop` is set, the
 *        check-then-update loop of fractal.py:22-24: run the test section; stop unless
 *        r[test_a] <test> r[test_b] holds (VDSL_PIX_TEST_NONE: always holds) and fewer than
 *        max_iter updates were made; run the body section; count one update; repeat;
 *   post (the last n_post instructions): the stored value, which may read the count.
 * out[i][j][k] = r[out_regs[k]] for k < out_width (an f32 field of scalars or vec2-4) or the
 * count (VDSL_PIX_OUT_COUNT: an int32 field of scalars).
 * Instructions are vdsl_map_instr with the map-chain opcodes (VDSL_MAP_LOAD: a = input field,
 * c = component, read at [i][j]) plus the ones below; every operation rounds once, in f32, where it is written
 * (an fma only for VDSL_MAP_FMA).  Compiled at run time for each program (once per device): a
 * program first seen while a queue records a graph is refused, so run it once before
 * recording.  No counterpart in the reference beyond the program surface it runs; the caller is
 * the Taichi-subset front end for kernel bodies other than the escape-time form of
 * vdsl_op_escape_time. */
#define VDSL_PIX_MAX_INSTR 256
#define VDSL_PIX_MAX_REGS 32
#define VDSL_PIX_MAX_INPUTS 8

typedef enum vdsl_pix_opcode {
  VDSL_PIX_INDEX = 32,  /* r[dst] = float(i) (a = 0, the outer axis) or float(j) (a = 1) */
  VDSL_PIX_COS = 33,    /* cosf(r[a]) */
  VDSL_PIX_SIN = 34,    /* sinf(r[a]) */
  VDSL_PIX_COUNT = 35,  /* r[dst] = float(count of loop updates); post section only */
  VDSL_PIX_LT = 36,     /* r[dst] = r[a] < r[b] ? 1 : 0 (a NaN operand gives 0) */
  VDSL_PIX_LE = 37,     /* r[a] <= r[b] ? 1 : 0 */
  VDSL_PIX_EQ = 38,     /* r[a] == r[b] ? 1 : 0 */
  VDSL_PIX_NE = 39,     /* r[a] != r[b] ? 1 : 0 (a NaN operand gives 1) */
  VDSL_PIX_SELECT = 40, /* r[a] != 0 ? r[b] : r[c] (NaN counts as true) */
  VDSL_PIX_FLOOR = 41,  /* floorf(r[a]) */
  /* Component (int)imm of input a's pixel [row][col], row = index(r[b], ni), col = index(r[c], nj)
   * with index(x, n) = 0 if !(x >= 0), n - 1 if x >= n - 1, else (int)x: a stencil or gather read,
   * clamped to the field (Taichi leaves reads outside a field undefined). */
  VDSL_PIX_LOAD_AT = 42,
  /* r[dst] = float(the loop's trip: the updates made before it, 0 on the first), test and body
   * sections only.  Every lane still in the loop is on the same trip, so this is the loop
   * variable of `for k in range(N)` and the counter of a while loop (an index: gathers at it
   * read one element per wave). */
  VDSL_PIX_TRIP = 43,
  /* Scatter-add (Taichi's `f[idx] += v` at an index other than the pixel's, an atomic add):
   * component (int)imm of input a at [(int)r[b]][(int)r[c]] += r[dst], when 0 <= r[b] < rows
   * and 0 <= r[c] < cols of input a (its own extents or the grid's).  Otherwise (an index
   * negative, NaN or too large: nothing is clamped) the add is dropped, as it is on lanes past
   * the grid.  r[dst] is read, no register is written.  Pre and post sections only.  Input a is
   * then written: its buffer must be writable, must not be `out`, and no LOAD / LOAD_AT of the
   * program may read it.  An int32 input adds r[dst] converted as VDSL_PIX_OUT_I32 stores it,
   * wrapping on overflow: exact in any order.  An f32 input adds in f32 with the hardware's
   * atomic float add; the adds of one launch to one element happen in no fixed order, and
   * several may be summed before they reach it (per wave or per block where the indices are
   * the same on every lane or constant, and in a per-block copy of a target of at most 8192
   * elements), so the sum's rounding may differ between runs (as Taichi's atomic adds). */
  VDSL_PIX_ATOMIC_ADD = 44,
  VDSL_PIX_TRUNC = 45,  /* truncf(r[a]): toward zero (Taichi's float -> int conversion, kept in f32) */
  /* Taichi's atomic_max / atomic_min: as VDSL_PIX_ATOMIC_ADD (operands, extents, drops,
   * refusals), the element becoming max / min(element, r[dst]): int32 exactly (the value
   * converted as VDSL_PIX_OUT_I32 stores it); f32 as fmaxf / fminf (a NaN operand is ignored), in
   * any order the same value except that the sign of a zero result may depend on the order. */
  VDSL_PIX_ATOMIC_MAX = 46,
  VDSL_PIX_ATOMIC_MIN = 47,
  /* Taichi's `F[idx] = v` at an index other than the pixel's: a plain store of r[dst] (int32:
   * converted as VDSL_PIX_OUT_I32 stores it) with the operands, extents, drops and refusals of
   * VDSL_PIX_ATOMIC_ADD; where several pixels store to one element, one of them wins, in no fixed
   * order (a race in Taichi too). */
  VDSL_PIX_STORE_AT = 48,
  /* r[dst] = a uniform number in [0, 1) (Taichi's ti.random()): h = H(H(H(s) ^ d) ^ (i nj + j)), with
   * s = (uint32)r[a] (a seed, an integer below 2^24 held as a float), d = (uint32)imm (which
   * draw of the pixel), H Chris Wellons' lowbias32 integer hash (x ^= x >> 16; x *= 0x7feb352d;
   * x ^= x >> 15; x *= 0x846ca68b; x ^= x >> 16), and the result (h >> 8) * 2^-24, exact in f32. */
  VDSL_PIX_RANDOM = 49,
  /* the device math library's float functions (a few ulp from the correctly rounded value):
   * atan2f(r[a], r[b]), asinf, acosf, atanf, tanf of r[a], powf(r[a], r[b]) */
  VDSL_PIX_ATAN2 = 50,
  VDSL_PIX_ASIN = 51,
  VDSL_PIX_ACOS = 52,
  VDSL_PIX_ATAN = 53,
  VDSL_PIX_TAN = 54,
  VDSL_PIX_POWF = 55,
  /* integer bit operations: both registers converted to int32 as VDSL_PIX_OUT_I32 stores them
   * (toward zero, NaN -> 0, saturating), the int32 operation, the result back to f32 (exact
   * below 2^24 in magnitude): r[a] & r[b], |, ^, r[a] << (r[b] & 31), and r[a] >> (r[b] & 31)
   * arithmetic (the sign copied in) */
  VDSL_PIX_BAND = 56,
  VDSL_PIX_BOR = 57,
  VDSL_PIX_BXOR = 58,
  VDSL_PIX_SHL = 59,
  VDSL_PIX_SHR = 60,
  /* roundf(r[a]): to the nearest integer, halfway cases away from zero (exact) */
  VDSL_PIX_ROUND = 61
} vdsl_pix_opcode;

typedef enum vdsl_pix_test {
  VDSL_PIX_TEST_NONE = 0, VDSL_PIX_TEST_LT = 1, VDSL_PIX_TEST_LE = 2, VDSL_PIX_TEST_GT = 3,
  VDSL_PIX_TEST_GE = 4
} vdsl_pix_test;

typedef enum vdsl_pix_output {
  VDSL_PIX_OUT_REG = 0,    /* f32 field: r[out_regs[k]], k < out_width */
  VDSL_PIX_OUT_COUNT = 1,  /* int32 field: the count of loop updates (out_width 1) */
  /* int32 field: r[out_regs[0]] converted as a Taichi int field assignment does, truncating
   * toward zero (NaN gives 0, values beyond the int32 range saturate); out_width 1 */
  VDSL_PIX_OUT_I32 = 2,
  /* no per-pixel store: a program whose effects are its VDSL_PIX_ATOMIC_ADDs (out may be null;
   * out_width 1) */
  VDSL_PIX_OUT_NONE = 3
} vdsl_pix_output;

typedef struct vdsl_pixel_program {
  int32_t n_pre, n_test, n_body, n_post;   /* section lengths; their sum <= VDSL_PIX_MAX_INSTR */
  int32_t loop;                            /* 0: no loop (n_test = n_body = 0) */
  int32_t max_iter;                        /* at most this many loop updates (>= 0) */
  int32_t test;                            /* vdsl_pix_test */
  int32_t test_a, test_b;                  /* registers compared by the test */
  int32_t out_kind;                        /* vdsl_pix_output */
  int32_t out_width;                       /* components stored per pixel, 1..4 (ti.Vector.field) */
  int32_t out_regs[4];                     /* their registers, in component order */
  int32_t in_widths[VDSL_PIX_MAX_INPUTS];  /* components per pixel of input k, 1..4 */
  int32_t in_dtypes[VDSL_PIX_MAX_INPUTS];  /* VDSL_F32, or VDSL_I32 (one component, read as float(v)) */
  /* Extents [in_rows[k]][in_cols[k]] of input k when it is not of the program's grid (a field of
   * another shape, read only by VDSL_PIX_LOAD_AT, whose indices it clamps to these extents); both
   * 0: the grid's [ni][nj]. */
  int32_t in_rows[VDSL_PIX_MAX_INPUTS];
  int32_t in_cols[VDSL_PIX_MAX_INPUTS];
  vdsl_map_instr code[VDSL_PIX_MAX_INSTR];
} vdsl_pixel_program;

/* Runs `prog` for every pixel of an [ni][nj] grid.  inputs: f32 [ni][nj][in_widths[k]] or int32
 * [ni][nj] fields (n_inputs <= VDSL_PIX_MAX_INPUTS; [in_rows[k]][in_cols[k]] for an input of its own
 * extents); out: f32 [ni][nj][out_width] (VDSL_PIX_OUT_REG) or int32
 * [ni][nj] (VDSL_PIX_OUT_COUNT, VDSL_PIX_OUT_I32), unused for VDSL_PIX_OUT_NONE.  A program may read its output buffer as an
 * input: at [i][j] that is the pixel's value before the store; elsewhere (LOAD_AT) the result
 * depends on the order pixels run in, as for a Taichi kernel reading the field it writes. */
int vdsl_op_pixel_program(vdsl_queue q, int32_t ni, int32_t nj, const vdsl_pixel_program* prog,
                          const vdsl_buffer* inputs, int32_t n_inputs, vdsl_buffer out);

/* Batched vertex transform: the MVP chain of the reference's test shader (color.mlir:10-39:
 * vec4(pos, 1.0), then linalg.matvec by model, view and proj) over n vertices.
 *   pos:  f32 [n][in_width]; in_width 3 (extended to vec4(pos, 1.0), color.mlir:15-21) or 4;
 *   mats: f32 [n_mats][4][4] row-major mat4 uniforms (!vernon.mat4<f32>), n_mats 1..3, applied in
 *         order (model, view, proj): v <- M v with
 *         out[i] = (((0 + M[i][0] v[0]) + M[i][1] v[1]) + M[i][2] v[2]) + M[i][3] v[3],
 *         every product and sum rounded to f32 (linalg.matvec's mulf/addf accumulation into a
 *         zero-initialised output, no contraction);
 *   out:  f32 [n][4] (gl_Position);
 *   varying (optional): f32 [n][in_width] = pos (the pass-through result of color.mlir:39). */
int vdsl_op_vec_transform(vdsl_queue q, int64_t n, int32_t in_width, vdsl_buffer pos, int32_t n_mats,
                          vdsl_buffer mats, vdsl_buffer out, vdsl_buffer varying);

/* The same chain for any square matrix type (!vernon.mat2 / mat3 / mat4, source/README.md:34-37):
 * dim 2, 3 or 4; pos f32 [n][in_width] with in_width dim (used as is) or dim - 1 (extended to
 * vec(pos, 1.0): homogeneous coordinates, as color.mlir:15-21 does for dim 4); mats f32
 * [n_mats][dim][dim] row-major, n_mats 1..3, applied in order with the accumulation above cut to
 * dim terms; out f32 [n][dim]; varying (optional) f32 [n][in_width] = pos.
 * vdsl_op_vec_transform(q, n, w, ...) is vdsl_op_mat_transform(q, n, 4, w, ...). */
int vdsl_op_mat_transform(vdsl_queue q, int64_t n, int32_t dim, int32_t in_width, vdsl_buffer pos, int32_t n_mats,
                          vdsl_buffer mats, vdsl_buffer out, vdsl_buffer varying);

/* ========================================================================================== */
/* Op class 3: row reductions + softmax (no reference code; north-star op class).             */
/* ========================================================================================== */
/* x: dtype [rows][cols] (F32 or BF16).  Any output may be NULL.
 * row_sum, row_max: f32 [rows];  softmax: dtype [rows][cols] = exp(x - max) / sum(exp(x - max)). */
int vdsl_op_row_reduce_softmax(vdsl_queue q, int64_t rows, int64_t cols, int32_t dtype,
                               vdsl_buffer x, vdsl_buffer row_sum, vdsl_buffer row_max,
                               vdsl_buffer softmax);
/* Column reductions of an f32/bf16 [rows][cols] tensor: col_sum, col_max f32 [cols] (either NULL). */
int vdsl_op_col_reduce(vdsl_queue q, int64_t rows, int64_t cols, int32_t dtype, vdsl_buffer x,
                       vdsl_buffer col_sum, vdsl_buffer col_max);

/* ========================================================================================== */
/* Op class 4: dense bf16 matmul on MFMA, fp32 accumulate (no reference code; north star).    */
/* ========================================================================================== */
typedef enum vdsl_epilogue {
  VDSL_EPI_NONE = 0,
  VDSL_EPI_GELU = 1,    /* exact-erf GELU: 0.5 * v * (1 + erf(v / sqrt(2))) */
  VDSL_EPI_RELU = 2,
  /* GELU, with pre_act receiving GELU'(v) (f32) instead of v: what the backward pass multiplies
   * by (vdsl_op_gemm_bf16_mul_packed), formed while erfc(-v / sqrt 2) is at hand for GELU(v).
   * vdsl_op_gemm_bf16_packed only. */
  VDSL_EPI_GELU_DERIV = 3
} vdsl_epilogue;

/* C (c_dtype [M][N]) = epilogue(op(A) . op(B)).
 *   trans_a = 0: A is [M][K];  trans_a = 1: A is stored [K][M].
 *   trans_b = 0: B is [K][N];  trans_b = 1: B is stored [N][K].
 * pre_act: if not NULL, receives the f32 [M][N] accumulator before the epilogue (for autodiff).
 * workspace: device scratch for operand re-layout; vdsl_gemm_bf16_workspace_bytes() says how
 * much (0 for trans_a = 0, trans_b = 1), and it may be NULL when that is 0. */
int vdsl_gemm_bf16_workspace_bytes(int32_t trans_a, int32_t trans_b, int64_t M, int64_t N,
                                   int64_t K, size_t* bytes);
int vdsl_op_gemm_bf16(vdsl_queue q, int32_t trans_a, int32_t trans_b, int64_t M, int64_t N,
                      int64_t K, vdsl_buffer A, vdsl_buffer B, vdsl_buffer C, int32_t c_dtype,
                      int32_t epilogue, vdsl_buffer pre_act, vdsl_buffer workspace);
/* Weights in MFMA fragment order, for vdsl_op_gemm_bf16_packed (packed once when the weights are
 * written, not per call): w bf16 [N][K] (out x in) -> wp, same bytes, in the layout of
 * vdsl_op_pack_w8a8_weights on the K*2-byte rows.  N % 32 == 0, K % 16 == 0. */
int vdsl_op_pack_bf16_weights(vdsl_queue q, int64_t N, int64_t K, vdsl_buffer w, vdsl_buffer wp);
/* vdsl_op_gemm_bf16(trans_a = 0, trans_b = 1) with B packed by vdsl_op_pack_bf16_weights: the
 * same products in the same order, bit for bit.  N % 32 == 0, K % 256 == 0.  No workspace. */
int vdsl_op_gemm_bf16_packed(vdsl_queue q, int64_t M, int64_t N, int64_t K, vdsl_buffer A,
                             vdsl_buffer Bp, vdsl_buffer C, int32_t c_dtype, int32_t epilogue,
                             vdsl_buffer pre_act);

/* 2-D transpose: dst [cols][rows] = src [rows][cols]^T, dtype F32 or BF16. */
int vdsl_op_transpose(vdsl_queue q, int64_t rows, int64_t cols, int32_t dtype, vdsl_buffer src,
                      vdsl_buffer dst);
/* Elementwise conversion of n elements (F32 <-> BF16). */
int vdsl_op_cast(vdsl_queue q, int64_t n, int32_t src_dtype, vdsl_buffer src, int32_t dst_dtype,
                 vdsl_buffer dst);

/* Elementwise GELU, y = 0.5 x (1 + erf(x / sqrt 2)) (the exact-erf form; no reference code, north
 * star op class 4, which fuses it into the GEMM epilogue; this is the standalone op).  x: F32 or
 * BF16 [n];  y: F32 or BF16 [n];  in-place (x == y, same dtype) is allowed. */
int vdsl_op_gelu_fwd(vdsl_queue q, int64_t n, int32_t x_dtype, vdsl_buffer x, int32_t y_dtype, vdsl_buffer y);

/* Autodiff building blocks for the MLP graph (no reference code; north star). */
/* GELU backward: da (bf16 [rows][cols]) = dh (f32) * GELU'(pre) (f32);  da_t (optional, bf16
 * [cols][rows]) receives the transpose of da. */
int vdsl_op_gelu_bwd(vdsl_queue q, int64_t rows, int64_t cols, vdsl_buffer dh, vdsl_buffer pre,
                     vdsl_buffer da, vdsl_buffer da_t);
/* ReLU backward, as vdsl_op_gelu_bwd: da = dh where pre > 0, else +0 (pre <= 0 or NaN; a select,
 * so an infinite dh there gives 0), rounded to bf16; da_t optional. */
int vdsl_op_relu_bwd(vdsl_queue q, int64_t rows, int64_t cols, vdsl_buffer dh, vdsl_buffer pre,
                     vdsl_buffer da, vdsl_buffer da_t);
/* out = a + b elementwise over n elements: each operand F32 or BF16 (widened exactly), one f32
 * addition, rounded once (RNE) to out's dtype (F32 or BF16).  out may be a or b when it has that
 * operand's dtype.  The forward of a residual sum and the sum of the gradients of a value that
 * several ops read. */
int vdsl_op_add(vdsl_queue q, int64_t n, int32_t a_dtype, vdsl_buffer a, int32_t b_dtype, vdsl_buffer b,
                int32_t out_dtype, vdsl_buffer out);
/* The backward of y = GELU(pre) through the GEMM that forms dL/dy, fused: dh = A B^T (f32
 * accumulate, never written), da (bf16 [M][N]) = dh * GELU'(pre), da_t (optional, bf16 [N][M]) =
 * da^T.  A: bf16 [M][K]; B: bf16 [N][K] (the NT form); pre: f32 [M][N].  Bit-identical to
 * vdsl_op_gemm_bf16(trans_a = 0, trans_b = 1, f32 C) followed by vdsl_op_gelu_bwd.  No reference
 * counterpart (north-star op class: compiler-generated backward GEMMs). */
int vdsl_op_gemm_bf16_gelu_bwd(vdsl_queue q, int64_t M, int64_t N, int64_t K, vdsl_buffer A,
                               vdsl_buffer B, vdsl_buffer pre, vdsl_buffer da, vdsl_buffer da_t);
/* vdsl_op_gemm_bf16_gelu_bwd with B packed by vdsl_op_pack_bf16_weights (for a constant B, e.g. the
 * transposed weight of the layer above): same results bit for bit.  N % 32 == 0, K % 256 == 0. */
int vdsl_op_gemm_bf16_gelu_bwd_packed(vdsl_queue q, int64_t M, int64_t N, int64_t K, vdsl_buffer A,
                                      vdsl_buffer Bp, vdsl_buffer pre, vdsl_buffer da, vdsl_buffer da_t);
/* c = bf16((A Bp^T) * g) elementwise, c_t = c^T (optional): the GEMM forming dL/dh fused with the
 * multiply by a stored local derivative g (f32 [M][N]; for a GELU layer, GELU'(pre) from the
 * forward epilogue VDSL_EPI_GELU_DERIV), so with that g it equals vdsl_op_gemm_bf16_gelu_bwd_packed
 * bit for bit without evaluating GELU' in the backward pass.  Bp packed by
 * vdsl_op_pack_bf16_weights.  N % 32 == 0, K % 256 == 0.  No counterpart in the reference
 * (north-star op class: compiler-generated backward GEMMs). */
int vdsl_op_gemm_bf16_mul_packed(vdsl_queue q, int64_t M, int64_t N, int64_t K, vdsl_buffer A,
                                 vdsl_buffer Bp, vdsl_buffer g, vdsl_buffer c, vdsl_buffer c_t);
/* MSE: loss (f32 [1]) = mean((y - t)^2);  dy (bf16 [rows][cols]) = 2 (y - t) / (rows*cols);
 * dy_t (optional) = dy^T.  y, t: f32 [rows][cols].  partials: f32 scratch of
 * vdsl_mse_partials_count(rows, cols) elements (deterministic two-stage reduction). */
int64_t vdsl_mse_partials_count(int64_t rows, int64_t cols);
int vdsl_op_mse_fwd_bwd(vdsl_queue q, int64_t rows, int64_t cols, vdsl_buffer y, vdsl_buffer t,
                        vdsl_buffer loss, vdsl_buffer dy, vdsl_buffer dy_t, vdsl_buffer partials);

/* The output layer of a regression head fused with its MSE loss (no reference counterpart;
 * north-star op class: compiler-generated backward): y = A Bp^T (f32 accumulate, Bp packed by
 * vdsl_op_pack_bf16_weights), d = y - t, and in the GEMM's epilogue loss = mean(d^2) (per-wave f64
 * partial sums, added by a one-block kernel in a fixed order), dy = bf16(d * 2 / (M N)),
 * dy_t = dy^T (optional), y itself (optional; the gradient does not need it).  dy and dy_t equal
 * vdsl_op_gemm_bf16_packed (f32 C) followed by vdsl_op_mse_fwd_bwd bit for bit; the loss is the
 * same f64 sum taken in another order.  M % 128 == 0, N % 256 == 0, K % 256 == 0.  partials: f32
 * scratch of vdsl_mse_partials_count(M, N) elements, as for vdsl_op_mse_fwd_bwd. */
int vdsl_op_gemm_bf16_mse_packed(vdsl_queue q, int64_t M, int64_t N, int64_t K, vdsl_buffer A,
                                 vdsl_buffer Bp, vdsl_buffer t, vdsl_buffer y, vdsl_buffer loss,
                                 vdsl_buffer dy, vdsl_buffer dy_t, vdsl_buffer partials);

/* ========================================================================================== */
/* Op class 5: int8 W8A8 GEMM with fused dequant (no reference code; north star).             */
/* ========================================================================================== */
/* Per-row symmetric activation quantisation:  s = max|x_row| / 127 (f32);
 * q = clamp(rne(x / s), -127, 127) (int8), q = 0 for an all-zero row.
 * x: F32 or BF16 [rows][cols];  q: int8 [rows][cols];  scale: f32 [rows]. */
int vdsl_op_quantize_rows_i8(vdsl_queue q, int64_t rows, int64_t cols, int32_t x_dtype,
                             vdsl_buffer x, vdsl_buffer qx, vdsl_buffer scale);
/* y (out_dtype [M][N]) = relu?( (float(acc) * x_scale[m]) * w_scale[n] ),
 * acc = sum_k xq[m][k] * w[n][k] in int32 (exact).  xq int8 [M][K]; w int8 [N][K] (out x in,
 * per-output-channel scales w_scale f32 [N]).  acc_out (optional) receives int32 [M][N].
 * workspace: int32 split-K partials, vdsl_gemm_w8a8_workspace_bytes() bytes (may be 0). */
int vdsl_gemm_w8a8_workspace_bytes(int64_t M, int64_t N, int64_t K, size_t* bytes);
int vdsl_op_gemm_w8a8(vdsl_queue q, int64_t M, int64_t N, int64_t K, vdsl_buffer xq,
                      vdsl_buffer x_scale, vdsl_buffer w, vdsl_buffer w_scale, vdsl_buffer y,
                      int32_t out_dtype, int32_t relu, vdsl_buffer acc_out, vdsl_buffer workspace);
/* Weights in MFMA fragment order, for vdsl_op_gemm_w8a8_packed (a layout transform done once when
 * weights are loaded, not per call).  w: int8 [N][K] (out x in); wp: int8, N*K bytes, receives
 * 1 KiB units u = (nb, kb), nb = n / 32, kb = k / 32, at byte (nb * (K/32) + kb) * 1024, lane l's
 * 16 bytes at 16 l = w[32 nb + l % 32][32 kb + 16 (l / 32) .. +15].  N % 32 == 0, K % 32 == 0.
 * Same role as ti.field storage (fractal.py:8) for a weight operand: no reference counterpart. */
int vdsl_op_pack_w8a8_weights(vdsl_queue q, int64_t N, int64_t K, vdsl_buffer w, vdsl_buffer wp);
/* vdsl_op_gemm_w8a8 with packed weights wp (vdsl_op_pack_w8a8_weights): same arithmetic, bit for
 * bit.  N % 32 == 0, K % 512 == 0.  workspace: int32 split-K partials,
 * vdsl_gemm_w8a8_packed_workspace_bytes() bytes (0 when the launch does not split K; any
 * contents).  Two calls that overlap in time need two workspaces. */
int vdsl_gemm_w8a8_packed_workspace_bytes(int64_t M, int64_t N, int64_t K, size_t* bytes);
int vdsl_op_gemm_w8a8_packed(vdsl_queue q, int64_t M, int64_t N, int64_t K, vdsl_buffer xq,
                             vdsl_buffer x_scale, vdsl_buffer wp, vdsl_buffer w_scale, vdsl_buffer y,
                             int32_t out_dtype, int32_t relu, vdsl_buffer acc_out,
                             vdsl_buffer workspace);

/* Allocation-free form of vdsl_op_gemm_w8a8_packed.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code recorded under graph capture that may not call
 * hipMalloc, tight serving loops, harnesses that forbid allocation).  It takes no workspace: the
 * split-K partials live in a library-owned device array of VDSL_W8A8_NOALLOC_SCRATCH_BYTES per GPU
 * (resolved when the device is opened, held until the process ends), and the call allocates
 * nothing.  Same arguments and results, bit for bit, as vdsl_op_gemm_w8a8_packed.  A shape whose
 * launch plan needs more scratch than the array holds (vdsl_gemm_w8a8_packed_workspace_bytes()
 * says how much) fails with VDSL_ERR_UNSUPPORTED before anything is enqueued.  Every call on one
 * GPU shares the array: calls on one queue are ordered and safe, calls that overlap in time on one
 * GPU (several queues) race and give wrong results. */
#define VDSL_W8A8_NOALLOC_SCRATCH_BYTES (16u << 20)
int vdsl_op_gemm_w8a8_packed_noalloc(vdsl_queue q, int64_t M, int64_t N, int64_t K, vdsl_buffer xq,
                                     vdsl_buffer x_scale, vdsl_buffer wp, vdsl_buffer w_scale,
                                     vdsl_buffer y, int32_t out_dtype, int32_t relu,
                                     vdsl_buffer acc_out);

/* ---- failure injection (tests of error paths, host-side only) ----------------------------- */
/* After `n` more successful buffer allocations, the next one fails with VDSL_ERR_OUT_OF_MEMORY
 * (n < 0 disables).  Also settable with the environment variable VDSL_FAIL_ALLOC_AFTER. */
int vdsl_debug_fail_alloc_after(int64_t n);

/* ---- tuning hook (tests and sweeps, host-side only) ----------------------------------------- */
/* Forces the GEMM tile configuration `config` (an index into the library's table for both
 * vdsl_op_gemm_bf16 and vdsl_op_gemm_w8a8) for later calls on every thread; config < 0 restores
 * the per-shape choice.  A configuration that cannot run a given shape (an index past the table,
 * a direct-to-LDS configuration whose stage does not divide K) is ignored for that call.  Also
 * settable with the environment variable VDSL_GEMM_CONFIG.  Query workspace sizes after setting
 * it: the int8 split-K workspace depends on the configuration.  No counterpart in the reference
 * (which has no kernels); callers are tuning sweeps and the tests that cover every configuration. */
int vdsl_debug_gemm_config(int32_t config);
/* Forces the launch plan of vdsl_op_gemm_w8a8_packed (and of its _noalloc form): cfg 0 =
 * 128 x 256 blocks, 1 = 64 x 256, 2 = 64 x 256 with loads 7 stages ahead, 3 = 128 x 128,
 * 4 = 64 x 128, 5 = 32 x 64, 6 = 32 x 128; K split
 * `split` ways (1..255).  cfg < 0 restores the per-shape plan.  A plan whose stages do not split K
 * evenly (K % (128 * stages per loop trip * split) != 0) is ignored for that call.  Query the
 * workspace size after setting it.  No counterpart in the reference; callers are tuning sweeps and
 * the tests that cover every plan. */
int vdsl_debug_w8a8_packed_plan(int32_t cfg, int32_t split);

/* ---- map-chain forms (benchmarks and tests, host-side only) ---------------------------------- */
/* A map chain (vdsl_op_map_chain, vdsl_op_map_chain_v) runs as a kernel compiled at run time for
 * the chain (hiprtc, for the device's architecture; cached per chain and device, at most 512
 * programs per device, shared with the per-pixel programs' cache; the chain's immediates stay
 * arguments) or in the generic interpreter; both give the same bits.  mode 0 (default): the
 * compiled form for launches of at least 2^20 elements, the interpreter for smaller ones; 1: the
 * interpreter for every chain; 2: the compiled form for every chain.  Nothing is compiled while a
 * queue records a graph: a chain that needs its compiled form and was not run before the
 * recording started fails with VDSL_ERR_CAPTURE.  A failed compilation fails the op (VDSL_ERR_DEVICE,
 * with the compiler's log), as does a full cache (VDSL_ERR_UNSUPPORTED).  Also settable with the
 * environment variable VDSL_MAP_MODE.  No counterpart in the reference; callers are benchmarks
 * and the tests that compare the forms. */
int vdsl_debug_map_chain_mode(int32_t mode);
/* Counters since the library was loaded: launches in compiled form, compilations, failed
 * compilations (any pointer may be NULL). */
int vdsl_debug_map_chain_stats(int64_t* compiled_launches, int64_t* compiles, int64_t* failures);

#ifdef __cplusplus
}
#endif

#endif /* VDSL_H */

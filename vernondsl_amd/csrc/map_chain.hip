// Op class 2: fused elementwise / broadcast map chains on gfx950 (host side).
//
// The reference has no elementwise code (the only compute is fractal.py:16-25); this op class
// comes from the north-star spec.  A chain is a straight-line register program
// (vdsl_map_instr, include/vdsl.h) evaluated once per output element, so a whole expression
// such as tanh(a*x + b) * exp(-x^2) + bias[col] costs one HBM read of each operand and one
// write of the result.  The device code is mapchain_kern.h.
//
// A chain runs in one of two forms, from the same source and bit-identical:
//   - a kernel compiled at run time for the chain (hiprtc, for the device's architecture, with the
//     library's own compile flags): the chain becomes a compile-time table and the interpreter
//     unrolls into straight-line code.  Compiled once per distinct chain and device (the
//     immediates are kernel arguments, not part of the compiled code), for every launch of at
//     least kCompileMinElements elements;
//   - the generic interpreter, a kernel argument program with uniform dispatch, for smaller
//     launches (microseconds of work, against a fraction of a second to compile).
// Nothing is compiled while a queue records a graph: a large chain first met there fails with
// VDSL_ERR_CAPTURE (run it once before recording), and a failed compilation is an error, not a
// fallback to the interpreter.  vdsl_debug_map_chain_mode selects one form for every chain.

#include <cstdlib>
#include <string>

#include "common.h"
#include "jit.h"
#include "mapchain_kern.h"

namespace vdsl {
namespace {

// The kernels built into the library: thin wrappers around the shared bodies.
template <class P, int VEC, int R, class IDX>
__global__ __launch_bounds__(256) void map_chain_kernel(MapProg rt, MapIn in, float* __restrict__ out, IDX rows, IDX cols) {
  map_chain_body<P, VEC, R, IDX>(rt, in, out, rows, cols);
}

template <class P, int R, class IDX>
__global__ __launch_bounds__(256) void map_chain_v_kernel(MapProg rt, MapVIn in, MapVOut vo, float* __restrict__ out,
                                                          IDX rows, IDX cols) {
  map_chain_v_body<P, R, IDX>(rt, in, vo, out, rows, cols);
}

// Launch geometry: VEC columns per lane, 256 lanes per block, R rows per step, at most 65535
// blocks along the rows (the kernels stride over the rest).  32-bit indices when every offset the
// kernel forms (row * cols + col, and row0 plus a grid's worth of rows) stays far below 2^31.
struct Geometry {
  dim3 grid;
  bool idx32;
};

int geometry(int vec, int r, int comps, int64_t rows, int64_t cols, Geometry& g) {
  const int64_t slots = (cols + vec - 1) / vec;
  const int64_t gx = (slots + 255) / 256;
  int64_t gy = (rows + r - 1) / r;
  if (gy > 65535) gy = 65535;
  if (gx > 0x7fffffff) return fail(VDSL_ERR_UNSUPPORTED, "map chain: cols too large");
  g.grid = dim3(static_cast<unsigned>(gx), static_cast<unsigned>(gy));
  g.idx32 = rows * (cols + 256 * vec) * comps <= (int64_t{1} << 30) && rows <= (int64_t{1} << 28);
  return VDSL_OK;
}

template <class P, int VEC, int R>
int launch(const MapProg& rt, const MapIn& in, float* out, int64_t rows, int64_t cols, hipStream_t s) {
  Geometry g;
  VDSL_TRY(geometry(VEC, R, 1, rows, cols, g));
  if (g.idx32)
    hipLaunchKernelGGL((map_chain_kernel<P, VEC, R, int32_t>), g.grid, dim3(256), 0, s, rt, in, out, static_cast<int32_t>(rows),
                       static_cast<int32_t>(cols));
  else
    hipLaunchKernelGGL((map_chain_kernel<P, VEC, R, int64_t>), g.grid, dim3(256), 0, s, rt, in, out, rows, cols);
  return check_launch("map_chain_kernel");
}

constexpr int kRowsV = 4;  // rows per lane step of the vector kernels

int launch_v(const MapProg& rt, const MapVIn& in, const MapVOut& vo, float* out, int64_t rows, int64_t cols, int comps,
             hipStream_t s) {
  Geometry g;
  VDSL_TRY(geometry(1, kRowsV, comps, rows, cols, g));
  if (g.idx32)
    hipLaunchKernelGGL((map_chain_v_kernel<GenericProgram, kRowsV, int32_t>), g.grid, dim3(256), 0, s, rt, in, vo, out,
                       static_cast<int32_t>(rows), static_cast<int32_t>(cols));
  else
    hipLaunchKernelGGL((map_chain_v_kernel<GenericProgram, kRowsV, int64_t>), g.grid, dim3(256), 0, s, rt, in, vo, out, rows,
                       cols);
  return check_launch("map_chain_v_kernel");
}

// ---- mode switch -------------------------------------------------------------------------------------
enum { kModeAuto = 0, kModeInterpret = 1, kModeCompile = 2 };
std::atomic<int> g_mode{-1};  // -1: not yet read from VDSL_MAP_MODE

int map_mode() {
  int v = g_mode.load();
  if (v < 0) {
    const char* e = std::getenv("VDSL_MAP_MODE");
    int init = e ? std::atoi(e) : kModeAuto;
    if (init < kModeAuto || init > kModeCompile) init = kModeAuto;
    g_mode.compare_exchange_strong(v, init);
    v = g_mode.load();
  }
  return v;
}

// ---- chains compiled at run time --------------------------------------------------------------------
// Launches of fewer elements run the interpreter: they are over in microseconds, and compiling
// costs a fraction of a second once per chain.
constexpr int64_t kCompileMinElements = int64_t{1} << 20;

JitCounters g_jit;
std::atomic<int64_t> g_jit_launches{0};

// The fixed-program table of a chain, as C++ source; it names the kernel completely (with the entry
// points), so it is also the cache key.  vec: columns per lane of a scalar chain (4, or 1 when the
// column count is not a multiple of 4).
std::string program_source(const MapProg& rt, int n_inputs, const int32_t* bcast, const int32_t* widths,
                           const int32_t* out_regs, int out_width, bool vector, int vec) {
  std::string s = "#include \"mapchain_kern.h\"\nnamespace vdsl {\nstruct JitProg {\n";
  s += "  static constexpr int n = " + std::to_string(rt.n) + ";\n";
  s += "  static constexpr int n_inputs = " + std::to_string(n_inputs) + ";\n";
  s += "  static constexpr int out_reg = " + std::to_string(rt.out_reg) + ";\n";
  s += "  static constexpr int out_width = " + std::to_string(out_width) + ";\n";
  auto table = [&](const char* name, const int32_t* v, int cnt) {
    s += std::string("  static constexpr int ") + name + "[4] = {";
    for (int k = 0; k < 4; ++k) s += std::to_string(k < cnt ? v[k] : 0) + (k < 3 ? ", " : "};\n");
  };
  table("bcast_tab", bcast, n_inputs);
  table("width_tab", widths, n_inputs);
  table("out_regs", out_regs, out_width);
  s += "  __host__ __device__ static constexpr int bcast_of(int k) { return bcast_tab[k]; }\n";
  s += "  __host__ __device__ static constexpr int width_of(int k) { return width_tab[k]; }\n";
  s += "  static constexpr vdsl_map_instr code[VDSL_MAP_MAX_INSTR] = {\n";
  for (int pc = 0; pc < rt.n; ++pc) {
    const vdsl_map_instr& c = rt.code[pc];
    s += "    {" + std::to_string(c.op) + ", " + std::to_string(c.dst) + ", " + std::to_string(c.a) + ", " +
         std::to_string(c.b) + ", " + std::to_string(c.c) + ", {" + std::to_string(c.ext[0]) + ", " +
         std::to_string(c.ext[1]) + ", " + std::to_string(c.ext[2]) + "}, 0.f},\n";
  }
  s += "  };\n};\n}  // namespace vdsl\n";
  if (!vector) {
    const std::string V = std::to_string(vec);
    s += "extern \"C\" __global__ __launch_bounds__(256) void vdsl_map_jit32(vdsl::MapProg rt, vdsl::MapIn in, "
         "float* __restrict__ out, int rows, int cols) {\n"
         "  vdsl::map_chain_body<vdsl::JitProg, " + V + ", 2, int>(rt, in, out, rows, cols);\n}\n";
    s += "extern \"C\" __global__ __launch_bounds__(256) void vdsl_map_jit64(vdsl::MapProg rt, vdsl::MapIn in, "
         "float* __restrict__ out, long long rows, long long cols) {\n"
         "  vdsl::map_chain_body<vdsl::JitProg, " + V + ", 2, long long>(rt, in, out, rows, cols);\n}\n";
  } else {
    const std::string R = std::to_string(kRowsV);
    s += "extern \"C\" __global__ __launch_bounds__(256) void vdsl_map_jit32(vdsl::MapProg rt, vdsl::MapVIn in, "
         "vdsl::MapVOut vo, float* __restrict__ out, int rows, int cols) {\n"
         "  vdsl::map_chain_v_body<vdsl::JitProg, " + R + ", int>(rt, in, vo, out, rows, cols);\n}\n";
    s += "extern \"C\" __global__ __launch_bounds__(256) void vdsl_map_jit64(vdsl::MapProg rt, vdsl::MapVIn in, "
         "vdsl::MapVOut vo, float* __restrict__ out, long long rows, long long cols) {\n"
         "  vdsl::map_chain_v_body<vdsl::JitProg, " + R + ", long long>(rt, in, vo, out, rows, cols);\n}\n";
  }
  return s;
}

// Whether a launch of `elements` runs the chain's own (compiled) kernel.
bool want_compiled(int64_t elements) {
  const int m = map_mode();
  if (m == kModeInterpret) return false;
  return m == kModeCompile || elements >= kCompileMinElements;
}

// Runs a chain in its compiled form, compiling it first if needed (never while recording: a chain
// first met during a recording fails with VDSL_ERR_CAPTURE).  Compilation errors are returned.
int launch_compiled(vdsl_queue q, const std::string& src, bool vector, int vec, int comps, void* prog_arg, void* in_arg,
                    void* vo_arg, float* out, int64_t rows, int64_t cols) {
  // Entries with 32- and 64-bit indices.
  const char* const entries[] = {"vdsl_map_jit32", "vdsl_map_jit64"};
  const JitKernels* c = nullptr;
  const int st = jit_kernels(q->dev->ordinal, src, entries, 2, q->capturing, g_jit, "map chain", &c);
  if (st == VDSL_ERR_UNSUPPORTED && q->capturing && !c)
    return fail(VDSL_ERR_CAPTURE,
                "map chain: a chain of this size is compiled at run time and was first met while the queue records a "
                "graph (nothing is compiled during recording); run it once before recording");
  if (st != VDSL_OK) return st;
  Geometry g;
  VDSL_TRY(geometry(vec, vector ? kRowsV : 2, comps, rows, cols, g));
  int32_t r32 = static_cast<int32_t>(rows), c32 = static_cast<int32_t>(cols);
  int64_t r64 = rows, c64 = cols;
  void* a32v[] = {prog_arg, in_arg, vo_arg, &out, &r32, &c32};
  void* a64v[] = {prog_arg, in_arg, vo_arg, &out, &r64, &c64};
  void* a32s[] = {prog_arg, in_arg, &out, &r32, &c32};
  void* a64s[] = {prog_arg, in_arg, &out, &r64, &c64};
  void** args = vector ? (g.idx32 ? a32v : a64v) : (g.idx32 ? a32s : a64s);
  VDSL_TRY(check_hip(hipModuleLaunchKernel(g.idx32 ? c->fn[0] : c->fn[1], g.grid.x, g.grid.y, 1, 256, 1, 1, 0, q->stream, args,
                                           nullptr),
                     "hipModuleLaunchKernel(map chain)"));
  ++g_jit_launches;
  return VDSL_OK;
}

// Shared validation of a chain's instructions.  widths[k]: the component count of input k (1 for
// the scalar entry point), which bounds a LOAD's component field; dims[k]: its matrix dimension
// (0 for vectors), which the matrix products require.
int load_program(const vdsl_map_instr* code, int32_t n_instr, int32_t n_inputs, const int32_t* widths, const int32_t* dims,
                 MapProg& rt) {
  if (n_instr < 0 || n_instr > VDSL_MAP_MAX_INSTR) return fail(VDSL_ERR_INVALID_ARG, "n_instr out of range [0, 32]");
  if (n_instr && !code) return fail(VDSL_ERR_INVALID_ARG, "code is null");
  rt = MapProg{};
  rt.n = n_instr;
  for (int pc = 0; pc < n_instr; ++pc) {
    const vdsl_map_instr& s = code[pc];
    const std::string at = "instruction " + std::to_string(pc) + ": ";
    if (s.op < VDSL_MAP_LOAD || s.op > VDSL_MAP_VECMAT) return fail(VDSL_ERR_INVALID_ARG, at + "unknown opcode " + std::to_string(s.op));
    rt.code[pc] = s;
    if (s.op == VDSL_MAP_MATVEC || s.op == VDSL_MAP_VECMAT) {
      if (s.a >= n_inputs || dims[s.a] == 0)
        return fail(VDSL_ERR_INVALID_ARG, at + "a matrix product needs a matrix input (vdsl_map_vinput.mat_dim 2..4)");
      const int n = dims[s.a];
      if (s.dst >= VDSL_MAP_MAX_REGS || s.b >= VDSL_MAP_MAX_REGS || s.c >= n)
        return fail(VDSL_ERR_INVALID_ARG, at + "register or matrix row out of range");
      for (int k = 0; k + 1 < n; ++k)
        if (s.ext[k] >= VDSL_MAP_MAX_REGS) return fail(VDSL_ERR_INVALID_ARG, at + "vector register out of range");
      // components past the matrix dimension are not read: keep them 0 so that equal products
      // compile to one kernel
      for (int k = n - 1; k < 3; ++k) rt.code[pc].ext[k] = 0;
      continue;
    }
    // a LOAD's c is a component (up to 15 for a mat4), every other opcode's a register
    if (s.dst >= VDSL_MAP_MAX_REGS || s.b >= VDSL_MAP_MAX_REGS || (s.op != VDSL_MAP_LOAD && s.c >= VDSL_MAP_MAX_REGS))
      return fail(VDSL_ERR_INVALID_ARG, at + "register out of range");
    if (s.op == VDSL_MAP_LOAD ? (s.a >= n_inputs || s.c >= widths[s.a]) : s.a >= VDSL_MAP_MAX_REGS)
      return fail(VDSL_ERR_INVALID_ARG, at + "operand out of range");
    rt.code[pc].ext[0] = rt.code[pc].ext[1] = rt.code[pc].ext[2] = 0;
  }
  return VDSL_OK;
}

}  // namespace
}  // namespace vdsl

using namespace vdsl;

extern "C" int vdsl_op_map_chain(vdsl_queue q, int64_t rows, int64_t cols, const vdsl_map_instr* code, int32_t n_instr,
                                 const vdsl_map_input* inputs, int32_t n_inputs, int32_t out_reg, vdsl_buffer out) {
  VDSL_TRY(enter_queue(q));
  if (rows < 0 || cols < 0) return fail(VDSL_ERR_INVALID_ARG, "negative shape");
  if (n_inputs < 0 || n_inputs > VDSL_MAP_MAX_INPUTS) return fail(VDSL_ERR_INVALID_ARG, "n_inputs out of range [0, 4]");
  if (out_reg < 0 || out_reg >= VDSL_MAP_MAX_REGS) return fail(VDSL_ERR_INVALID_ARG, "out_reg out of range");
  if (n_inputs && !inputs) return fail(VDSL_ERR_INVALID_ARG, "inputs is null");
  VDSL_TRY(check_buffer(q, out, nbytes(rows, cols, 4), "out", true));
  const int64_t n = rows * cols;  // no overflow: rows * cols * 4 fits size_t (checked above)
  const int32_t ones[VDSL_MAP_MAX_INPUTS] = {1, 1, 1, 1}, no_dims[VDSL_MAP_MAX_INPUTS] = {0, 0, 0, 0};
  MapProg rt;
  VDSL_TRY(load_program(code, n_instr, n_inputs, ones, no_dims, rt));
  rt.out_reg = out_reg;
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
  if (want_compiled(n)) {
    const int32_t regs[4] = {out_reg, 0, 0, 0};
    const std::string src = program_source(rt, n_inputs, in.bcast, ones, regs, 1, false, vec4 ? 4 : 1);
    return launch_compiled(q, src, false, vec4 ? 4 : 1, 1, &rt, &in, nullptr, o, rows, cols);
  }
  if (vec4) return launch<GenericProgram, 4, 1>(rt, in, o, rows, cols, q->stream);
  return launch<GenericProgram, 1, 1>(rt, in, o, rows, cols, q->stream);
}

extern "C" int vdsl_debug_map_chain_mode(int32_t mode) {
  if (mode < kModeAuto || mode > kModeCompile) return fail(VDSL_ERR_INVALID_ARG, "map chain mode must be 0, 1 or 2");
  map_mode();
  g_mode.store(mode);
  return VDSL_OK;
}

extern "C" int vdsl_debug_map_chain_stats(int64_t* compiled_launches, int64_t* compiles, int64_t* failures) {
  if (compiled_launches) *compiled_launches = g_jit_launches.load();
  if (compiles) *compiles = g_jit.compiles.load();
  if (failures) *failures = g_jit.failures.load();
  return VDSL_OK;
}

extern "C" int vdsl_op_map_chain_v(vdsl_queue q, int64_t rows, int64_t cols, const vdsl_map_instr* code, int32_t n_instr,
                                   const vdsl_map_vinput* inputs, int32_t n_inputs, const int32_t* out_regs, int32_t out_width,
                                   vdsl_buffer out) {
  VDSL_TRY(enter_queue(q));
  if (rows < 0 || cols < 0) return fail(VDSL_ERR_INVALID_ARG, "negative shape");
  if (n_inputs < 0 || n_inputs > VDSL_MAP_MAX_INPUTS) return fail(VDSL_ERR_INVALID_ARG, "n_inputs out of range [0, 4]");
  if (n_inputs && !inputs) return fail(VDSL_ERR_INVALID_ARG, "inputs is null");
  if (out_width < 1 || out_width > 4) return fail(VDSL_ERR_INVALID_ARG, "out_width out of range [1, 4]");
  if (!out_regs) return fail(VDSL_ERR_INVALID_ARG, "out_regs is null");
  MapVOut vo{};
  vo.width = out_width;
  for (int k = 0; k < out_width; ++k) {
    if (out_regs[k] < 0 || out_regs[k] >= VDSL_MAP_MAX_REGS) return fail(VDSL_ERR_INVALID_ARG, "out_regs entry out of range");
    vo.regs[k] = out_regs[k];
  }
  VDSL_TRY(check_buffer(q, out, nbytes(rows, cols, 4 * static_cast<int64_t>(out_width)), "out", true));
  MapVIn in{};
  in.n = n_inputs;
  int32_t widths[VDSL_MAP_MAX_INPUTS] = {1, 1, 1, 1}, dims[VDSL_MAP_MAX_INPUTS] = {0, 0, 0, 0};
  int comps = out_width;  // the widest record, which bounds the kernel's element offsets
  for (int k = 0; k < n_inputs; ++k) {
    const vdsl_map_vinput& d = inputs[k];
    if (d.dtype != VDSL_F32) return fail(VDSL_ERR_UNSUPPORTED, "map chain inputs must be f32");
    if (d.bcast < VDSL_BCAST_FULL || d.bcast > VDSL_BCAST_SCALAR) return fail(VDSL_ERR_INVALID_ARG, "unknown broadcast");
    if (d.mat_dim == 0) {
      if (d.width < 1 || d.width > 4) return fail(VDSL_ERR_INVALID_ARG, "vector input width out of range [1, 4]");
    } else if (d.mat_dim < 2 || d.mat_dim > 4) {
      return fail(VDSL_ERR_INVALID_ARG, "mat_dim must be 0 (a vector), 2, 3 or 4");
    } else if (d.width != d.mat_dim * d.mat_dim) {
      return fail(VDSL_ERR_INVALID_ARG, "a matrix input's width must be mat_dim * mat_dim");
    }
    const size_t need = d.bcast == VDSL_BCAST_FULL ? nbytes(rows, cols, 4 * static_cast<int64_t>(d.width))
                        : d.bcast == VDSL_BCAST_ROW ? nbytes(cols, 4 * static_cast<int64_t>(d.width))
                        : d.bcast == VDSL_BCAST_COL ? nbytes(rows, 4 * static_cast<int64_t>(d.width))
                                                    : nbytes(1, 4 * static_cast<int64_t>(d.width));
    std::string name = "input" + std::to_string(k);
    VDSL_TRY(check_buffer(q, d.buf, need, name.c_str(), false));
    // 8- and 16-byte records (and mat4s, read as 16-byte pieces) need their alignment (hipMalloc
    // bases are 256-byte aligned)
    const int align = d.width == 2 ? 8 : (d.width == 4 || d.width == 16) ? 16 : 4;
    if (reinterpret_cast<uintptr_t>(d.buf->ptr) % align) return fail(VDSL_ERR_INVALID_ARG, name + ": base not aligned to its record size");
    in.p[k] = static_cast<const float*>(d.buf->ptr);
    in.bcast[k] = d.bcast;
    in.width[k] = d.width;
    widths[k] = d.width;
    dims[k] = d.mat_dim;
    if (d.width > comps) comps = d.width;
  }
  MapProg rt;
  VDSL_TRY(load_program(code, n_instr, n_inputs, widths, dims, rt));
  if (rows == 0 || cols == 0) return VDSL_OK;
  float* o = static_cast<float*>(out->ptr);
  if (want_compiled(rows * cols)) {
    const std::string src = program_source(rt, n_inputs, in.bcast, widths, vo.regs, out_width, true, 1);
    return launch_compiled(q, src, true, 1, comps, &rt, &in, &vo, o, rows, cols);
  }
  return launch_v(rt, in, vo, o, rows, cols, comps, q->stream);
}

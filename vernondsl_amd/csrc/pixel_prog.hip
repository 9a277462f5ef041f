// General per-pixel programs (vdsl_op_pixel_program), host side: validation, the program's
// source for run-time compilation, and the launch.  The device code is pixprog_kern.h.
//
// The reference's only computing program is a Taichi struct-for (fractal.py:16-25); its
// escape-time form has a hand-tuned kernel (escape_time.hip).  Any other body the Taichi-subset
// front end lowers (other iterated maps, plain per-pixel expressions, reads of other fields) runs
// here: the body is a register program (include/vdsl.h), compiled once per program and device into
// straight-line code around the same check-then-update loop.

#include <algorithm>
#include <cstddef>
#include <cstdlib>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "common.h"
#include "jit.h"
#include "pixprog_kern.h"

namespace vdsl {
namespace {

JitCounters g_pix_jit;

bool scatter_op(int op) {  // an instruction with an effect and no result register
  return op == VDSL_PIX_ATOMIC_ADD || op == VDSL_PIX_ATOMIC_MAX || op == VDSL_PIX_ATOMIC_MIN || op == VDSL_PIX_STORE_AT;
}

int check_program(const vdsl_pixel_program& p, int n_inputs) {
  const int64_t total = int64_t{p.n_pre} + p.n_test + p.n_body + p.n_post;
  if (p.n_pre < 0 || p.n_test < 0 || p.n_body < 0 || p.n_post < 0 || total > VDSL_PIX_MAX_INSTR)
    return fail(VDSL_ERR_INVALID_ARG, "pixel program: section lengths must be >= 0 and sum to at most " + std::to_string(VDSL_PIX_MAX_INSTR));
  if (p.loop != 0 && p.loop != 1) return fail(VDSL_ERR_INVALID_ARG, "pixel program: loop must be 0 or 1");
  if (!p.loop && (p.n_test || p.n_body)) return fail(VDSL_ERR_INVALID_ARG, "pixel program: test/body sections without a loop");
  if (p.max_iter < 0) return fail(VDSL_ERR_INVALID_ARG, "pixel program: max_iter < 0");
  if (p.test < VDSL_PIX_TEST_NONE || p.test > VDSL_PIX_TEST_GE) return fail(VDSL_ERR_INVALID_ARG, "pixel program: unknown test");
  if (p.test_a < 0 || p.test_a >= VDSL_PIX_MAX_REGS || p.test_b < 0 || p.test_b >= VDSL_PIX_MAX_REGS)
    return fail(VDSL_ERR_INVALID_ARG, "pixel program: test register out of range");
  if (p.out_kind != VDSL_PIX_OUT_REG && p.out_kind != VDSL_PIX_OUT_COUNT && p.out_kind != VDSL_PIX_OUT_I32 &&
      p.out_kind != VDSL_PIX_OUT_NONE)
    return fail(VDSL_ERR_INVALID_ARG, "pixel program: unknown out_kind");
  if (p.out_width < 1 || p.out_width > 4 || (p.out_kind != VDSL_PIX_OUT_REG && p.out_width != 1))
    return fail(VDSL_ERR_INVALID_ARG, "pixel program: out_width must be 1..4 (1 for an int32 field)");
  for (int k = 0; k < p.out_width; ++k)
    if (p.out_regs[k] < 0 || p.out_regs[k] >= VDSL_PIX_MAX_REGS)
      return fail(VDSL_ERR_INVALID_ARG, "pixel program: out_regs out of range");
  for (int k = 0; k < n_inputs; ++k) {
    if (p.in_widths[k] < 1 || p.in_widths[k] > 4) return fail(VDSL_ERR_INVALID_ARG, "pixel program: in_widths must be 1..4");
    if ((p.in_rows[k] == 0) != (p.in_cols[k] == 0) || p.in_rows[k] < 0 || p.in_cols[k] < 0)
      return fail(VDSL_ERR_INVALID_ARG, "pixel program: in_rows / in_cols must both be 0 or both positive");
    if (p.in_dtypes[k] != VDSL_F32 && !(p.in_dtypes[k] == VDSL_I32 && p.in_widths[k] == 1))
      return fail(VDSL_ERR_INVALID_ARG, "pixel program: in_dtypes must be VDSL_F32 or VDSL_I32 (one component)");
  }
  if (p.out_kind == VDSL_PIX_OUT_COUNT && !p.loop) return fail(VDSL_ERR_INVALID_ARG, "pixel program: a count needs a loop");
  const int post0 = p.n_pre + p.n_test + p.n_body;
  for (int pc = 0; pc < total; ++pc) {
    const vdsl_map_instr& s = p.code[pc];
    const std::string at = "pixel program: instruction " + std::to_string(pc);
    const bool map_op = s.op >= VDSL_MAP_LOAD && s.op <= VDSL_MAP_ADD_IMM;
    const bool pix_op = s.op >= VDSL_PIX_INDEX && s.op <= VDSL_PIX_ROUND;
    if (!map_op && !pix_op) return fail(VDSL_ERR_INVALID_ARG, at + ": unknown opcode " + std::to_string(s.op));
    if (s.dst >= VDSL_PIX_MAX_REGS || s.b >= VDSL_PIX_MAX_REGS || s.c >= VDSL_PIX_MAX_REGS)
      return fail(VDSL_ERR_INVALID_ARG, at + ": register out of range");
    if (s.op == VDSL_MAP_LOAD) {
      if (s.a >= n_inputs || s.c >= p.in_widths[s.a])
        return fail(VDSL_ERR_INVALID_ARG, at + ": LOAD of an input or component that is not there");
      if (p.in_rows[s.a] || p.in_cols[s.a])
        return fail(VDSL_ERR_INVALID_ARG, at + ": LOAD (at the pixel) of an input of its own extents; use LOAD_AT");
    } else if (s.op == VDSL_PIX_LOAD_AT) {
      const bool comp_ok = s.a < n_inputs && s.imm >= 0.0f && s.imm < static_cast<float>(p.in_widths[s.a]) &&
                           s.imm == static_cast<float>(static_cast<int>(s.imm));
      if (!comp_ok) return fail(VDSL_ERR_INVALID_ARG, at + ": LOAD_AT of an input or component that is not there");
    } else if (scatter_op(s.op)) {
      const bool comp_ok = s.a < n_inputs && s.imm >= 0.0f && s.imm < static_cast<float>(p.in_widths[s.a]) &&
                           s.imm == static_cast<float>(static_cast<int>(s.imm));
      if (!comp_ok) return fail(VDSL_ERR_INVALID_ARG, at + ": ATOMIC_ADD to an input or component that is not there");
      if (pc >= p.n_pre && pc < post0)
        return fail(VDSL_ERR_INVALID_ARG, at + ": ATOMIC_ADD in the loop's sections (pre and post only)");
      for (int q = 0; q < total; ++q) {
        const vdsl_map_instr& l = p.code[q];
        if ((l.op == VDSL_MAP_LOAD || l.op == VDSL_PIX_LOAD_AT) && l.a == s.a)
          return fail(VDSL_ERR_INVALID_ARG, at + ": ATOMIC_ADD to an input the program also reads (instruction " +
                                                std::to_string(q) + ")");
      }
    } else if (s.op == VDSL_PIX_INDEX) {
      if (s.a > 1) return fail(VDSL_ERR_INVALID_ARG, at + ": INDEX axis must be 0 (i) or 1 (j)");
    } else if (s.a >= VDSL_PIX_MAX_REGS) {
      return fail(VDSL_ERR_INVALID_ARG, at + ": register out of range");
    }
    if (s.op == VDSL_PIX_COUNT && pc < post0) return fail(VDSL_ERR_INVALID_ARG, at + ": COUNT outside the post section");
    if (s.op == VDSL_PIX_TRIP && (pc < p.n_pre || pc >= post0))
      return fail(VDSL_ERR_INVALID_ARG, at + ": TRIP outside the loop's test and body sections");
  }
  return VDSL_OK;
}

std::vector<char> row_uniform_gathers(const vdsl_pixel_program& p);

// Elements (x components) of input k when its scatter-adds go to a copy in LDS per block
// (pixprog_kern.h), else 0: a target of at most kPrivMax elements that some add reaches at
// per-pixel indices (a histogram), while the copies of the targets before it and its own take
// at most kPrivMax elements in all (32 KiB of a block's LDS).  Adds at constant indices are
// summed in registers instead.
constexpr int kPrivMax = 8192;
int privatized(const vdsl_pixel_program& p, const std::vector<char>& flags, int k, int ni, int nj) {
  const int total = p.n_pre + p.n_test + p.n_body + p.n_post;
  int64_t used = 0, own = 0;
  for (int t = 0; t <= k; ++t) {
    bool per_pixel = false, other = false;  // adds at per-pixel indices; a max or min into it
    for (int pc = 0; pc < total; ++pc) {
      if (p.code[pc].a != t) continue;
      per_pixel |= p.code[pc].op == VDSL_PIX_ATOMIC_ADD && !(flags[pc] & 4);
      other |= p.code[pc].op == VDSL_PIX_ATOMIC_MAX || p.code[pc].op == VDSL_PIX_ATOMIC_MIN ||
               p.code[pc].op == VDSL_PIX_STORE_AT;
    }
    per_pixel &= !other;
    const int64_t elems = static_cast<int64_t>(p.in_rows[t] ? p.in_rows[t] : ni) * (p.in_cols[t] ? p.in_cols[t] : nj) *
                          p.in_widths[t];
    own = per_pixel && used + elems <= kPrivMax ? elems : 0;
    used += own;
  }
  return static_cast<int>(own);
}

// Rows per block in the row mapping (each thread evaluates that many pixels of its column, then
// stores them).  Measured on 8192^2 f32 (graph replays, one box): y = 2x + 1 runs best with 4
// (88.2 us; 2, 6, 8, 12, 16 rows: 87-97% of that rate), the clamped five-point stencil of
// examples/heat.py with 8 (95.7 us; 6: 95.9, 10: 99.1, 12: 99.6-99.9, 4: 103.0, 16: 107.5).  A
// program that stores nothing and adds only at constant indices (a reduction such as
// `total[None] += x[i, j]`) adds once per block, and those adds to one element are serialised
// (~13 ns each): 64 rows (the sum of an 8192^2 field: 834 / 420 / 214 us with 4 / 8 / 16 rows);
// so does one whose other adds go to per-block copies in LDS (their flush is per block too).
// VDSL_PIX_ROWS=r (1..64) overrides the choice, for tuning sweeps.
int rows_per_block(const vdsl_pixel_program& p, const std::vector<char>& flags, const int32_t* priv) {
  if (const char* e = std::getenv("VDSL_PIX_ROWS")) {  // tuning sweeps: rows per block, 1..64
    const int r = std::atoi(e);
    if (r >= 1 && r <= 64) return r;
  }
  const int total = p.n_pre + p.n_test + p.n_body + p.n_post;
  bool gathers = false, reduction = p.out_kind == VDSL_PIX_OUT_NONE;
  for (int pc = 0; pc < total; ++pc) {
    gathers |= p.code[pc].op == VDSL_PIX_LOAD_AT;
    if (scatter_op(p.code[pc].op) && ((!(flags[pc] & 4) && !priv[p.code[pc].a]) || p.code[pc].op == VDSL_PIX_STORE_AT))
      reduction = false;
  }
  return reduction ? 64 : gathers ? 8 : 4;
}

// Blocks of rows_per_block rows x 256 pixels for programs whose pixels all do the same work (no
// escape loop), while the row count fits the grid's y extent; 16x16 patches otherwise.  0 for
// the patches.
int row_mapping(const vdsl_pixel_program& p, const std::vector<char>& flags, const int32_t* priv, int ni) {
  // never more rows per block than the grid has: a 1-D field is a grid of one row, whose blocks
  // would otherwise run their loops for rows that do not exist
  const int rows = std::min(rows_per_block(p, flags, priv), std::max(ni, 1));
  return !(p.loop && p.test != VDSL_PIX_TEST_NONE) && (ni + rows - 1) / rows <= 65535 ? rows : 0;
}

// Registers an instruction reads (a, b, c as the opcode uses them).
int reads(int op) {
  switch (op) {
    case VDSL_MAP_LOAD: case VDSL_MAP_CONST: case VDSL_PIX_INDEX: case VDSL_PIX_COUNT: case VDSL_PIX_TRIP: return 0;
    case VDSL_PIX_LOAD_AT: return 6;  // b, c
    case VDSL_MAP_ADD: case VDSL_MAP_SUB: case VDSL_MAP_MUL: case VDSL_MAP_DIV: case VDSL_MAP_MAX: case VDSL_MAP_MIN:
    case VDSL_PIX_LT: case VDSL_PIX_LE: case VDSL_PIX_EQ: case VDSL_PIX_NE: case VDSL_PIX_ATAN2: case VDSL_PIX_POWF:
    case VDSL_PIX_BAND: case VDSL_PIX_BOR: case VDSL_PIX_BXOR: case VDSL_PIX_SHL: case VDSL_PIX_SHR:
      return 3;  // a, b
    case VDSL_MAP_FMA: case VDSL_PIX_SELECT: return 7;  // a, b, c
    case VDSL_PIX_ATOMIC_ADD: case VDSL_PIX_ATOMIC_MAX: case VDSL_PIX_ATOMIC_MIN: case VDSL_PIX_STORE_AT:
      return 6;  // b, c (and the value r[dst]; no register written)
    default: return 1;  // a
  }
}

// Gathers (LOAD_AT) and scatter-adds (ATOMIC_ADD) whose row operand (bit 0 of the flag) or column operand (bit 1) is the same on
// every lane of a wave in the row mapping, where a wave covers 64 pixels of one row and every lane
// makes every trip of a loop (the mapping has no escape loops): registers computed only from the
// row index i (INDEX 0), the loop's trip, constants and immediates.  Their row offset is then formed once per wave on the scalar unit.
// A forward pass over the sections (the loop's to a fixed point, joined with the state before it);
// loads, the column index and the count make a register vary, conservatively.
//
// Bit 2 marks a scatter-add whose row and column are both constants (computed from constants and
// immediates alone, in the pre or post section), the same on every lane in any mapping.
std::vector<char> row_uniform_gathers(const vdsl_pixel_program& p) {
  const int total = p.n_pre + p.n_test + p.n_body + p.n_post;
  std::vector<char> flag(total, 0);
  bool uni[VDSL_PIX_MAX_REGS];
  for (bool& u : uni) u = true;  // registers start at 0
  bool cst[VDSL_PIX_MAX_REGS];     // constants, pre and post sections
  for (bool& c : cst) c = true;
  auto const_step = [&](int pc) {
    const vdsl_map_instr& s = p.code[pc];
    const int rd = reads(s.op);
    if (scatter_op(s.op)) {
      if (cst[s.b] && cst[s.c]) flag[pc] = static_cast<char>(flag[pc] | 4);
      return;
    }
    const bool in_cst = (!(rd & 1) || cst[s.a]) && (!(rd & 2) || cst[s.b]) && (!(rd & 4) || cst[s.c]);
    const bool var = s.op == VDSL_MAP_LOAD || s.op == VDSL_PIX_LOAD_AT || s.op == VDSL_PIX_INDEX ||
                     s.op == VDSL_PIX_COUNT || s.op == VDSL_PIX_TRIP || s.op == VDSL_PIX_RANDOM;
    cst[s.dst] = !var && in_cst;
  };
  auto step = [&](int pc, bool* st) {
    const vdsl_map_instr& s = p.code[pc];
    const int rd = reads(s.op);
    const bool in_uni = (!(rd & 1) || st[s.a]) && (!(rd & 2) || st[s.b]) && (!(rd & 4) || st[s.c]);
    if (s.op == VDSL_PIX_LOAD_AT || scatter_op(s.op))
      flag[pc] = static_cast<char>((st[s.b] ? 1 : 0) | (st[s.c] ? 2 : 0));
    if (scatter_op(s.op)) return;  // writes no register
    bool out;
    if (s.op == VDSL_MAP_CONST || s.op == VDSL_PIX_TRIP) out = true;  // the trip is the same on every lane
    else if (s.op == VDSL_PIX_INDEX) out = s.a == 0;
    else if (s.op == VDSL_MAP_LOAD || s.op == VDSL_PIX_LOAD_AT || s.op == VDSL_PIX_COUNT || s.op == VDSL_PIX_RANDOM) out = false;
    else out = in_uni;
    st[s.dst] = out;
  };
  for (int pc = 0; pc < p.n_pre; ++pc) step(pc, uni), const_step(pc);
  // after the loop, a register it writes is no constant
  for (int pc = p.n_pre; pc < p.n_pre + p.n_test + p.n_body; ++pc)
    if (!scatter_op(p.code[pc].op)) cst[p.code[pc].dst] = false;
  if (p.loop) {
    bool head[VDSL_PIX_MAX_REGS];
    for (int r = 0; r < VDSL_PIX_MAX_REGS; ++r) head[r] = uni[r];
    for (int it = 0; it < 2 * VDSL_PIX_MAX_REGS + 2; ++it) {  // each pass can only clear flags
      bool st[VDSL_PIX_MAX_REGS];
      for (int r = 0; r < VDSL_PIX_MAX_REGS; ++r) st[r] = head[r];
      for (int pc = p.n_pre; pc < p.n_pre + p.n_test + p.n_body; ++pc) step(pc, st);
      bool changed = false;
      for (int r = 0; r < VDSL_PIX_MAX_REGS; ++r)
        if (head[r] && !st[r]) head[r] = false, changed = true;
      if (!changed) break;
    }
    bool after_test[VDSL_PIX_MAX_REGS];
    for (int r = 0; r < VDSL_PIX_MAX_REGS; ++r) after_test[r] = head[r];
    for (int pc = p.n_pre; pc < p.n_pre + p.n_test; ++pc) step(pc, after_test);
    bool st[VDSL_PIX_MAX_REGS];
    for (int r = 0; r < VDSL_PIX_MAX_REGS; ++r) st[r] = head[r];
    for (int pc = p.n_pre; pc < p.n_pre + p.n_test + p.n_body; ++pc) step(pc, st);  // the loop's flags, at the fixed point
    for (int r = 0; r < VDSL_PIX_MAX_REGS; ++r) uni[r] = head[r] && after_test[r];  // the loop ends after a test, or at max_iter
  }
  for (int pc = p.n_pre + p.n_test + p.n_body; pc < total; ++pc) step(pc, uni), const_step(pc);
  return flag;
}

// What the launch of a program over an [ni][nj] grid is worked out to: the dataflow flags of its
// gathers and scatter-adds, the LDS copies of its small scatter targets, the rows per block.
struct Plan {
  std::vector<char> flags;
  int32_t priv[VDSL_PIX_MAX_INPUTS] = {}, priv_off[VDSL_PIX_MAX_INPUTS] = {};
  int32_t priv_total = 0;
  int rows = 0;
};

Plan make_plan(const vdsl_pixel_program& p, int n_inputs, int ni, int nj) {
  Plan pl;
  pl.flags = row_uniform_gathers(p);
  for (int k = 0; k < n_inputs; ++k) {
    pl.priv[k] = privatized(p, pl.flags, k, ni, nj);
    pl.priv_off[k] = pl.priv_total;
    pl.priv_total += pl.priv[k];
  }
  pl.rows = row_mapping(p, pl.flags, pl.priv, ni);
  return pl;
}

// The program's table as C++ source (opcodes and registers; immediates stay kernel arguments).
// It names the kernel completely, so it is also the cache key.
std::string program_source(const vdsl_pixel_program& p, const Plan& pl, int n_inputs, int ni, int nj) {
  std::string s = "#include \"pixprog_kern.h\"\nnamespace vdsl {\nstruct PixJit {\n";
  auto c = [&](const char* name, int v) { s += std::string("  static constexpr int ") + name + " = " + std::to_string(v) + ";\n"; };
  c("n_pre", p.n_pre);
  c("n_test", p.n_test);
  c("n_body", p.n_body);
  c("n_post", p.n_post);
  c("loop", p.loop);
  c("test", p.test);
  c("test_a", p.test_a);
  c("test_b", p.test_b);
  c("out_kind", p.out_kind);
  c("out_width", p.out_width);
  c("rows", pl.rows);
  // 32-bit element offsets when every field's byte offsets stay below 2^32
  int maxw = p.out_width;
  for (int k = 0; k < n_inputs; ++k) maxw = p.in_widths[k] > maxw ? p.in_widths[k] : maxw;
  int64_t elems = static_cast<int64_t>(ni) * nj;  // the largest field of the launch, in elements
  for (int k = 0; k < n_inputs; ++k)
    if (p.in_rows[k]) elems = std::max(elems, static_cast<int64_t>(p.in_rows[k]) * p.in_cols[k]);
  c("idx32", elems * maxw * 4 <= int64_t{0xffffffff} ? 1 : 0);
  // Entries past out_width / n_inputs are not used: written as 0 / 1, so they do not split the cache.
  auto list = [&](const char* name, const int32_t* v, int n, int fill, int size) {
    s += std::string("  static constexpr int ") + name + "[" + std::to_string(size) + "] = {";
    for (int k = 0; k < size; ++k) s += std::to_string(k < n ? v[k] : fill) + (k < size - 1 ? ", " : "};\n");
  };
  list("out_regs", p.out_regs, p.out_width, 0, 4);
  list("in_widths", p.in_widths, n_inputs, 1, VDSL_PIX_MAX_INPUTS);
  list("in_dtypes", p.in_dtypes, n_inputs, VDSL_F32, VDSL_PIX_MAX_INPUTS);
  // per-block LDS copies of small scatter targets: sizes and offsets in one array
  list("priv", pl.priv, n_inputs, 0, VDSL_PIX_MAX_INPUTS);
  list("priv_off", pl.priv_off, n_inputs, 0, VDSL_PIX_MAX_INPUTS);
  c("priv_total", pl.priv_total);
  // ext[0] / ext[1] of a gather or scatter-add: 1 when its row / column operand is wave-uniform in
  // the row mapping; ext[2] of a scatter-add: 1 when both are constants
  const std::vector<char>& ru = pl.flags;
  s += "  static constexpr vdsl_map_instr code[VDSL_PIX_MAX_INSTR] = {\n";
  const int total = p.n_pre + p.n_test + p.n_body + p.n_post;
  for (int pc = 0; pc < total; ++pc) {
    const vdsl_map_instr& k = p.code[pc];
    s += "    {" + std::to_string(k.op) + ", " + std::to_string(k.dst) + ", " + std::to_string(k.a) + ", " + std::to_string(k.b) +
         ", " + std::to_string(k.c) + ", {" + std::to_string(ru[pc] & 1) + ", " + std::to_string((ru[pc] >> 1) & 1) +
         ", " + std::to_string((ru[pc] >> 2) & 1) + "}, 0.f},\n";
  }
  s += "  };\n};\n}  // namespace vdsl\n";
  s += "extern \"C\" __global__ __launch_bounds__(256) void vdsl_pix_jit(vdsl::PixRt rt, vdsl::PixIn in, void* out, int ni, "
       "int nj) {\n  vdsl::pixel_body<vdsl::PixJit>(rt, in, out, ni, nj);\n}\n";
  return s;
}

// Launches already worked out, keyed by the program's bytes without its immediates and max_iter
// (everything its source depends on) with the device and the grid: the source, its dataflow
// analysis and the cache lookup by source text cost more host time than the kernels of small
// programs (MPM88's 12 programs per substep: 57 us each from Python before).  Entries point into
// the compiled-program cache, whose entries stay for the process.
struct Launch {
  const JitKernels* k = nullptr;
  int rows = 0;
};
std::mutex g_launch_mu;
std::unordered_map<std::string, Launch> g_launches;
constexpr size_t kMaxLaunches = 4096;

std::string launch_key(const vdsl_pixel_program& p, int ordinal, int n_inputs, int ni, int nj) {
  const int total = p.n_pre + p.n_test + p.n_body + p.n_post;
  vdsl_pixel_program head = p;  // the fields before the code, without max_iter
  head.max_iter = 0;
  const int32_t ext[4] = {ordinal, n_inputs, ni, nj};
  std::string key(reinterpret_cast<const char*>(ext), sizeof ext);
  key.append(reinterpret_cast<const char*>(&head), offsetof(vdsl_pixel_program, code));
  for (int pc = 0; pc < total; ++pc) {
    vdsl_map_instr s = p.code[pc];
    s.imm = 0.0f;
    key.append(reinterpret_cast<const char*>(&s), sizeof s);
  }
  if (const char* e = std::getenv("VDSL_PIX_ROWS")) key.append(e);  // a tuning override changes the plan
  return key;
}

bool find_launch(const std::string& key, Launch& out) {
  std::lock_guard<std::mutex> lk(g_launch_mu);
  const auto it = g_launches.find(key);
  if (it == g_launches.end()) return false;
  out = it->second;
  return true;
}

void keep_launch(const std::string& key, const Launch& ln) {
  std::lock_guard<std::mutex> lk(g_launch_mu);
  if (g_launches.size() >= kMaxLaunches) g_launches.clear();  // a bound; entries are cheap to work out again
  g_launches[key] = ln;
}

}  // namespace
}  // namespace vdsl

using namespace vdsl;

extern "C" int vdsl_op_pixel_program(vdsl_queue q, int32_t ni, int32_t nj, const vdsl_pixel_program* prog,
                                     const vdsl_buffer* inputs, int32_t n_inputs, vdsl_buffer out) {
  VDSL_TRY(enter_queue(q));
  if (!prog) return fail(VDSL_ERR_INVALID_ARG, "prog is null");
  if (ni < 0 || nj < 0) return fail(VDSL_ERR_INVALID_ARG, "negative grid extent");
  if (n_inputs < 0 || n_inputs > VDSL_PIX_MAX_INPUTS)
    return fail(VDSL_ERR_INVALID_ARG, "n_inputs out of range [0, " + std::to_string(VDSL_PIX_MAX_INPUTS) + "]");
  if (n_inputs && !inputs) return fail(VDSL_ERR_INVALID_ARG, "inputs is null");
  const vdsl_pixel_program& p = *prog;
  VDSL_TRY(check_program(p, n_inputs));
  if (p.out_kind != VDSL_PIX_OUT_NONE) VDSL_TRY(check_buffer(q, out, nbytes(ni, nj, 4 * p.out_width), "out", true));
  bool target[VDSL_PIX_MAX_INPUTS] = {};  // inputs the program scatter-adds into (written)
  const int total = p.n_pre + p.n_test + p.n_body + p.n_post;
  for (int pc = 0; pc < total; ++pc)
    if (scatter_op(p.code[pc].op)) target[p.code[pc].a] = true;
  PixIn in{};
  for (int k = 0; k < n_inputs; ++k) {
    const std::string name = "input" + std::to_string(k);
    in.rows[k] = p.in_rows[k] ? p.in_rows[k] : ni;
    in.cols[k] = p.in_cols[k] ? p.in_cols[k] : nj;
    VDSL_TRY(check_buffer(q, inputs[k], nbytes(in.rows[k], in.cols[k], 4 * p.in_widths[k]), name.c_str(), target[k]));
    if (target[k] && p.out_kind != VDSL_PIX_OUT_NONE && inputs[k] == out)
      return fail(VDSL_ERR_INVALID_ARG, "pixel program: " + name + " is scatter-added into and is also the output");
    in.p[k] = static_cast<const float*>(inputs[k]->ptr);
  }
  if (ni == 0 || nj == 0) return VDSL_OK;
  if ((ni + 15) / 16 > 65535) return fail(VDSL_ERR_UNSUPPORTED, "pixel program: ni too large");
  PixRt rt{};
  for (int pc = 0; pc < total; ++pc) rt.imm[pc] = p.code[pc].imm;
  rt.max_iter = p.max_iter;
  // The kernel and its rows per block, from the launches seen before when this program (but for
  // its immediates and max_iter, which are arguments) ran on a grid of these extents on this
  // device; else from its source (compiled on first use).
  const std::string key = launch_key(p, q->dev->ordinal, n_inputs, ni, nj);
  Launch ln;
  if (!find_launch(key, ln)) {
    const Plan pl = make_plan(p, n_inputs, ni, nj);
    const std::string src = program_source(p, pl, n_inputs, ni, nj);
    const char* const entries[] = {"vdsl_pix_jit"};
    const int st = jit_kernels(q->dev->ordinal, src, entries, 1, q->capturing, g_pix_jit, "pixel program", &ln.k);
    if (st == VDSL_ERR_UNSUPPORTED && q->capturing)
      return fail(VDSL_ERR_CAPTURE, "pixel program: not compiled yet; run it once before recording a graph");
    VDSL_TRY(st);
    ln.rows = pl.rows;
    keep_launch(key, ln);
  }
  const JitKernels* k = ln.k;
  void* o = p.out_kind == VDSL_PIX_OUT_NONE ? nullptr : out->ptr;
  void* args[] = {&rt, &in, &o, &ni, &nj};
  const int rows = ln.rows;
  const unsigned gx = rows ? static_cast<unsigned>((nj + 255) / 256) : static_cast<unsigned>((nj + 15) / 16);
  const unsigned gy = rows ? static_cast<unsigned>((ni + rows - 1) / rows) : static_cast<unsigned>((ni + 15) / 16);
  return check_hip(hipModuleLaunchKernel(k->fn[0], gx, gy, 1, 256, 1, 1, 0, q->stream, args, nullptr),
                   "hipModuleLaunchKernel(pixel program)");
}

// Device side of general per-pixel programs (vdsl_op_pixel_program): the struct-for body of a
// Taichi kernel over a 2-D field, with the check-then-update loop of fractal.py:22-24.  The host
// (pixel_prog.hip) compiles this header at run time with one program's opcode table, so the
// program unrolls into straight-line code; only immediates and max_iter stay kernel arguments.
// Shares apply_op with the map chains (mapchain_kern.h), so an opcode means the same arithmetic in
// both op classes.  Uses nothing from the C++ standard library (hiprtc has none).
//
// Mapping: one lane per pixel.  For a program with an escape loop each wave takes an 8x8 tile
// (lanes of a tile tend to leave the loop at similar trips) and a 256-lane block a 16x16 patch;
// any other program runs 256 consecutive pixels of a row per block (coalesced memory access).  The loop is the escape-time
// kernel's (escape_time.hip) made general: wave-uniform, in blocks of 16 trips, with the live set
// a sticky 64-bit lane mask (one ballot and one scalar AND per trip) and the count added per
// block from the block's masks (lanemask.h).  Every lane runs every trip of its wave; what a lane
// computes after its test failed is discarded, as follows.  The program's register sets are
// worked out at compile time from the opcode table: only the registers the post section (or the
// store) reads that the loop also writes need their values from the trip the lane left the loop,
// and only those are kept, by one select per trip each (none for count-only programs such as an
// escape count).  When none is needed, a lane whose loop-carried registers return to the bits
// they held at an earlier block end (saved at the ends of blocks 1, 2, 4, 8, ...) would pass its
// test for ever: its count is max_iter and it leaves the live set at once (exact periodicity).
#pragma once

#include "lanemask.h"
#include "mapchain_kern.h"

namespace vdsl {

struct PixRt {
  float imm[VDSL_PIX_MAX_INSTR];
  int32_t max_iter;
};

struct PixIn {
  const float* p[VDSL_PIX_MAX_INPUTS];
  int rows[VDSL_PIX_MAX_INPUTS], cols[VDSL_PIX_MAX_INPUTS];  // each input's extents (the grid's for most)
};

// Element offsets into the fields: 32-bit when every byte offset of the launch's fields is below
// 2^32 (the host sets P::idx32), so a load is a scalar base plus a 32-bit vector offset and needs
// no 64-bit address arithmetic; 64-bit otherwise.
template <bool B>
struct PixOffT {
  using type = unsigned long long;
};
template <>
struct PixOffT<true> {
  using type = unsigned;
};
template <class P>
using PixOff = typename PixOffT<P::idx32 != 0>::type;

// One instruction at program counter PC of the table P.
// Element e, component c of input a (an int32 input is read as float(v)).
template <class P, int A>
__device__ __forceinline__ float pix_load(const PixIn& in, PixOff<P> e, int c) {
  if constexpr (P::idx32) {
    // the byte offset formed in 32 bits (the host checked it fits), so the load takes the field's
    // base in scalar registers and a 32-bit offset
    const char* base = reinterpret_cast<const char*>(in.p[A]);
    if constexpr (P::in_dtypes[A] == VDSL_I32) return static_cast<float>(*reinterpret_cast<const int*>(base + e * 4u));
    else return *reinterpret_cast<const float*>(base + (e * P::in_widths[A] + static_cast<unsigned>(c)) * 4u);
  } else {
    if constexpr (P::in_dtypes[A] == VDSL_I32) return static_cast<float>(reinterpret_cast<const int*>(in.p[A])[e]);
    else return in.p[A][e * P::in_widths[A] + c];
  }
}

// A field index from a register: 0 if !(x >= 0) (NaN included), else min((int)min(x, 2^30), n-1).
// fmaxf(x, 0) is 0 for a NaN or negative x (and either zero for -0), so the conversion is always
// of a value in [0, 2^30].
__device__ __forceinline__ unsigned pix_index(float x, int n) {
  const int v = static_cast<int>(fminf(fmaxf(x, 0.0f), 1073741824.0f));
  return static_cast<unsigned>(v < n - 1 ? v : n - 1);
}


// Scatter-adds and their max / min forms, combined where indices agree; with the stores at
// computed indices, the instructions that have an effect and no result register.
__device__ constexpr bool pix_scatter_op(int op) {
  return op == VDSL_PIX_ATOMIC_ADD || op == VDSL_PIX_ATOMIC_MAX || op == VDSL_PIX_ATOMIC_MIN;
}
__device__ constexpr bool pix_effect_op(int op) { return pix_scatter_op(op) || op == VDSL_PIX_STORE_AT; }

// A register stored to an int32 field: truncation toward zero, NaN -> 0, saturating.
__device__ __forceinline__ int pix_to_i32(float x) {
  if (x != x) return 0;
  if (x >= 2147483648.0f) return 2147483647;
  if (x < -2147483648.0f) return -2147483647 - 1;
  return static_cast<int>(x);
}

// Wave sums for scatter-adds at wave-uniform indices (every lane of the wave takes part; lanes
// that add nothing hold 0).  Lane l adds lane l ^ m's value, m = 32, 16, ..., 1.
__device__ __forceinline__ int pix_lane() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

__device__ __forceinline__ float pix_wave_sum(float v) {
  const int lane = pix_lane();
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1)
    v += __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ m) << 2, __float_as_int(v)));
  return v;
}

__device__ __forceinline__ int pix_wave_sum(int v) {
  const int lane = pix_lane();
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1)  // wrapping, as the atomic adds themselves
    v = static_cast<int>(static_cast<unsigned>(v) + static_cast<unsigned>(__builtin_amdgcn_ds_bpermute((lane ^ m) << 2, v)));
  return v;
}

// Wave maximum / minimum (OP VDSL_PIX_ATOMIC_MAX / MIN) of v: f32 as fmaxf / fminf (a lane with
// nothing to give holds NaN, which they ignore), int32 exactly.
template <int OP>
__device__ __forceinline__ float pix_wave_ext(float v) {
  const int lane = pix_lane();
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float o = __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ m) << 2, __float_as_int(v)));
    v = OP == VDSL_PIX_ATOMIC_MAX ? fmaxf(v, o) : fminf(v, o);
  }
  return v;
}

template <int OP>
__device__ __forceinline__ int pix_wave_ext(int v) {
  const int lane = pix_lane();
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const int o = __builtin_amdgcn_ds_bpermute((lane ^ m) << 2, v);
    v = OP == VDSL_PIX_ATOMIC_MAX ? (o > v ? o : v) : (o < v ? o : v);
  }
  return v;
}

// The combination of two values by scatter op OP (sum, max, min), and its identity.
template <int OP>
__device__ __forceinline__ float pix_combine(float a, float b) {
  return OP == VDSL_PIX_ATOMIC_ADD ? a + b : OP == VDSL_PIX_ATOMIC_MAX ? fmaxf(a, b) : fminf(a, b);
}
template <int OP>
__device__ __forceinline__ int pix_combine(int a, int b) {
  if constexpr (OP == VDSL_PIX_ATOMIC_ADD) return static_cast<int>(static_cast<unsigned>(a) + static_cast<unsigned>(b));
  else if constexpr (OP == VDSL_PIX_ATOMIC_MAX) return a > b ? a : b;
  else return a < b ? a : b;
}
template <int OP>
__device__ __forceinline__ float pix_none_f() {
  return OP == VDSL_PIX_ATOMIC_ADD ? 0.0f : __int_as_float(0x7FC00000);  // NaN: ignored by fmaxf / fminf
}
template <int OP>
__device__ __forceinline__ int pix_none_i() {
  return OP == VDSL_PIX_ATOMIC_ADD ? 0 : OP == VDSL_PIX_ATOMIC_MAX ? -2147483647 - 1 : 2147483647;
}

// The element a scatter-add into input A at [x][y] reaches: ok is false where x or y is outside
// A's extents (NaN fails every comparison; below 2^30 the conversion is exact truncation, and the
// row and column are then checked as integers, since float(rows) may round above 2^24).
template <class P, int A>
__device__ __forceinline__ PixOff<P> pix_target(const PixIn& in, float x, float y, bool& ok) {
  const bool num = x >= 0.0f && x < 1073741824.0f && y >= 0.0f && y < 1073741824.0f;
  const int xi = num ? static_cast<int>(x) : 0, yi = num ? static_cast<int>(y) : 0;
  ok = num && xi < in.rows[A] && yi < in.cols[A];
  return static_cast<PixOff<P>>(static_cast<unsigned>(xi)) * static_cast<unsigned>(in.cols[A]) + static_cast<unsigned>(yi);
}

template <class P, int A, int OP = VDSL_PIX_ATOMIC_ADD>
__device__ __forceinline__ void pix_atomic(const PixIn& in, PixOff<P> e, int c, float vf, int vi) {
  char* base = const_cast<char*>(reinterpret_cast<const char*>(in.p[A]));
  if constexpr (P::in_dtypes[A] == VDSL_I32) {
    int* t = reinterpret_cast<int*>(base) + e;
    if constexpr (OP == VDSL_PIX_ATOMIC_ADD) atomicAdd(t, vi);
    else if constexpr (OP == VDSL_PIX_ATOMIC_MAX) atomicMax(t, vi);
    else atomicMin(t, vi);
  } else {
    float* t = reinterpret_cast<float*>(base) + (e * static_cast<PixOff<P>>(P::in_widths[A]) + static_cast<PixOff<P>>(c));
    if constexpr (OP == VDSL_PIX_ATOMIC_ADD) {
      unsafeAtomicAdd(t, vf);
    } else {
      // compare and swap until the element holds fmaxf / fminf(element, vf) (or already did)
      unsigned* u = reinterpret_cast<unsigned*>(t);
      unsigned old = __hip_atomic_load(u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      for (;;) {
        const unsigned want = __float_as_uint(pix_combine<OP>(__uint_as_float(old), vf));
        if (want == old) break;
        const unsigned seen = atomicCAS(u, old, want);
        if (seen == old) break;
        old = seen;
      }
    }
  }
}

// Scatter-adds at constant indices (ext[2]: the same element for every pixel, such as
// `total[None] += v`) are not added where they run: each thread sums its pixels' values
// (PixAcc), and at the end of the block the sums of its four waves are added once (pix_flush).
template <class P>
struct PixConstAdds {
  static constexpr int end = P::n_pre + P::n_test + P::n_body + P::n_post;
  static constexpr bool at(int pc) { return pix_scatter_op(P::code[pc].op) && P::code[pc].ext[2] != 0; }
  static constexpr int slot(int pc) {
    int n = 0;
    for (int q = 0; q < pc; ++q) n += at(q) ? 1 : 0;
    return n;
  }
  static constexpr int N = slot(end);
};


template <class P>
struct PixAcc {
  static constexpr int N = PixConstAdds<P>::N > 0 ? PixConstAdds<P>::N : 1;
  float f[N];        // f32 targets: this thread's sum
  int i[N];          // int32 targets: this thread's sum, wrapping
  int n[N];          // adds made (none: nothing to add)
  float x[N], y[N];  // the indices (constants)
  unsigned* sh[VDSL_PIX_MAX_INPUTS];  // the block's LDS copy of input k where P::priv[k] > 0
};

// An add into input A's element e, component c: into the block's LDS copy where A has one
// (P::priv[A] > 0), else into memory.
template <class P, int A>
__device__ __forceinline__ void pix_add(const PixIn& in, PixAcc<P>& acc, PixOff<P> e, int c, float vf, int vi) {
  if constexpr (P::priv[A] > 0) {
    const unsigned k = static_cast<unsigned>(e) * static_cast<unsigned>(P::in_widths[A]) + static_cast<unsigned>(c);
    if constexpr (P::in_dtypes[A] == VDSL_I32) atomicAdd(reinterpret_cast<int*>(acc.sh[A]) + k, vi);
    else atomicAdd(reinterpret_cast<float*>(acc.sh[A]) + k, vf);
  } else {
    pix_atomic<P, A>(in, e, c, vf, vi);
  }
}

// VDSL_PIX_ATOMIC_ADD into input A: component c of [x][y] += v on lanes with act set, where the
// element is in A.  UNI: x and y are the same on every lane of the wave (host dataflow, row
// mapping), so the wave's values are summed and one lane adds.
template <class P, int A, bool UNI, int OP>
__device__ __forceinline__ void pix_scatter_add(const PixIn& in, PixAcc<P>& acc, float x, float y, float v, int c, bool act) {
  bool in_a;
  const PixOff<P> e = pix_target<P, A>(in, x, y, in_a);
  const bool ok = act && in_a;
  constexpr bool i32 = P::in_dtypes[A] == VDSL_I32;
  float vf = ok && !i32 ? v : pix_none_f<OP>();
  int vi = ok && i32 ? pix_to_i32(v) : pix_none_i<OP>();
  if constexpr (UNI) {
    const uint64_t any = __builtin_amdgcn_ballot_w64(ok);
    if (any == 0ull) return;
    if constexpr (OP == VDSL_PIX_ATOMIC_ADD) {
      if constexpr (i32) vi = pix_wave_sum(vi);
      else vf = pix_wave_sum(vf);
    } else {
      if constexpr (i32) vi = pix_wave_ext<OP>(vi);
      else vf = pix_wave_ext<OP>(vf);
    }
    if (pix_lane() == __builtin_ctzll(any)) {
      if constexpr (OP == VDSL_PIX_ATOMIC_ADD) pix_add<P, A>(in, acc, e, c, vf, vi);
      else pix_atomic<P, A, OP>(in, e, c, vf, vi);
    }
  } else if (ok) {
    if constexpr (OP == VDSL_PIX_ATOMIC_ADD) pix_add<P, A>(in, acc, e, c, vf, vi);
    else pix_atomic<P, A, OP>(in, e, c, vf, vi);
  }
}

template <class P, int PC>
__device__ __forceinline__ void pix_accumulate(PixAcc<P>& acc, float x, float y, float v, bool act) {
  constexpr vdsl_map_instr s = P::code[PC];
  constexpr int k = PixConstAdds<P>::slot(PC);
  constexpr int OP = s.op;
  if (act) {
    // the first value as it is (the accumulators start at 0, which is no identity of max / min)
    if constexpr (P::in_dtypes[s.a] == VDSL_I32)
      acc.i[k] = acc.n[k] ? pix_combine<OP>(acc.i[k], pix_to_i32(v)) : pix_to_i32(v);
    else
      acc.f[k] = acc.n[k] ? pix_combine<OP>(acc.f[k], v) : v;
    acc.n[k] += 1;
  }
  acc.x[k] = x;
  acc.y[k] = y;
}

// Wave sums of every constant-index add into LDS, then thread k adds the block's sum of add k.
// Every thread of the 256-thread block (4 waves) calls this once, after all its pixels.
template <class P, int PC>
__device__ __forceinline__ void pix_flush_wave(PixAcc<P>& acc, float (*sf)[PixAcc<P>::N], int (*si)[PixAcc<P>::N],
                                               int (*sn)[PixAcc<P>::N]) {
  if constexpr (PixConstAdds<P>::at(PC)) {
    constexpr int k = PixConstAdds<P>::slot(PC);
    constexpr int OP = P::code[PC].op;
    // lanes without a value give the identity (0 for sums; for max / min NaN, or the extreme int)
    const float f0 = acc.n[k] ? acc.f[k] : pix_none_f<OP>();
    const int i0 = acc.n[k] ? acc.i[k] : pix_none_i<OP>();
    float f;
    int iv;
    if constexpr (OP == VDSL_PIX_ATOMIC_ADD) f = pix_wave_sum(f0), iv = pix_wave_sum(i0);
    else f = pix_wave_ext<OP>(f0), iv = pix_wave_ext<OP>(i0);
    const int n = pix_wave_sum(acc.n[k]);
    if (pix_lane() == 0) {
      sf[threadIdx.x >> 6][k] = f;
      si[threadIdx.x >> 6][k] = iv;
      sn[threadIdx.x >> 6][k] = n;
    }
  }
}

template <class P, int PC>
__device__ __forceinline__ void pix_flush_add(const PixRt& rt, const PixIn& in, const PixAcc<P>& acc,
                                              float (*sf)[PixAcc<P>::N], int (*si)[PixAcc<P>::N], int (*sn)[PixAcc<P>::N]) {
  if constexpr (PixConstAdds<P>::at(PC)) {
    constexpr vdsl_map_instr s = P::code[PC];
    constexpr int k = PixConstAdds<P>::slot(PC);
    if (threadIdx.x == k) {
      constexpr int OP = s.op;
      const float f = pix_combine<OP>(pix_combine<OP>(pix_combine<OP>(sf[0][k], sf[1][k]), sf[2][k]), sf[3][k]);
      const int iv = pix_combine<OP>(pix_combine<OP>(pix_combine<OP>(si[0][k], si[1][k]), si[2][k]), si[3][k]);
      bool ok;
      const PixOff<P> e = pix_target<P, s.a>(in, acc.x[k], acc.y[k], ok);
      if (ok && sn[0][k] + sn[1][k] + sn[2][k] + sn[3][k] > 0)
        pix_atomic<P, s.a, OP>(in, e, static_cast<int>(rt.imm[PC]), f, iv);
    }
  }
}

template <class P, int... K>
__device__ __forceinline__ void pix_flush(const PixRt& rt, const PixIn& in, PixAcc<P>& acc, Seq<K...>) {
  if constexpr (PixConstAdds<P>::N > 0) {
    constexpr int N = PixAcc<P>::N;
    __shared__ float sf[4][N];
    __shared__ int si[4][N], sn[4][N];
    (pix_flush_wave<P, K>(acc, sf, si, sn), ...);
    __syncthreads();
    (pix_flush_add<P, K>(rt, in, acc, sf, si, sn), ...);
  }
}

// Chris Wellons' lowbias32 integer hash (a published 32-bit mixer) and VDSL_PIX_RANDOM's number.
__device__ __forceinline__ unsigned pix_hash(unsigned x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

__device__ __forceinline__ float pix_random(float seed, unsigned draw, unsigned pixel) {
  const unsigned s = seed >= 0.0f && seed < 16777216.0f ? static_cast<unsigned>(seed) : 0u;
  const unsigned h = pix_hash(pix_hash(pix_hash(s) ^ draw) ^ pixel);
  return static_cast<float>(h >> 8) * 0x1p-24f;
}

template <class P, int PC>
__device__ __forceinline__ void pix_step(const PixRt& rt, const PixIn& in, float (&r)[VDSL_PIX_MAX_REGS], PixOff<P> o,
                                         float fi, float fj, float fcount, int ni, int nj, bool act, PixAcc<P>& acc) {
  constexpr vdsl_map_instr s = P::code[PC];
  if constexpr (s.op == VDSL_PIX_STORE_AT) {
    bool ok;
    const PixOff<P> e = pix_target<P, s.a>(in, r[s.b], r[s.c], ok);
    if (act && ok) {
      char* base = const_cast<char*>(reinterpret_cast<const char*>(in.p[s.a]));
      if constexpr (P::in_dtypes[s.a] == VDSL_I32)
        reinterpret_cast<int*>(base)[e] = pix_to_i32(r[s.dst]);
      else
        reinterpret_cast<float*>(base)[e * static_cast<PixOff<P>>(P::in_widths[s.a]) + static_cast<PixOff<P>>(rt.imm[PC])] = r[s.dst];
    }
  } else if constexpr (pix_scatter_op(s.op) && s.ext[2] != 0) {
    pix_accumulate<P, PC>(acc, r[s.b], r[s.c], r[s.dst], act);  // constant indices: combined per block
  } else if constexpr (pix_scatter_op(s.op)) {
    // one add (max, min) per wave where both indices are the same on every lane (found
    // wave-uniform by the host in the row mapping: ext[0], ext[1]), else one per lane
    constexpr bool uni = P::rows > 0 && s.ext[0] != 0 && s.ext[1] != 0;
    pix_scatter_add<P, s.a, uni, s.op>(in, acc, r[s.b], r[s.c], r[s.dst], static_cast<int>(rt.imm[PC]), act);
  } else if constexpr (s.op == VDSL_MAP_LOAD) {
    r[s.dst] = pix_load<P, s.a>(in, o, s.c);
  } else if constexpr (s.op == VDSL_PIX_LOAD_AT) {
    // indices clamped to the input's own extents (the grid's, unless it is a field of another shape)
    unsigned ri = pix_index(r[s.b], in.rows[s.a]), ci = pix_index(r[s.c], in.cols[s.a]);
    // a row / column operand the host found wave-uniform (ext[0] / ext[1]; the row mapping puts
    // one row in each wave and runs no escape loops): its index is taken once per wave, into a
    // scalar register
    if constexpr (P::rows > 0 && s.ext[0] != 0) ri = __builtin_amdgcn_readfirstlane(ri);
    if constexpr (P::rows > 0 && s.ext[1] != 0) ci = __builtin_amdgcn_readfirstlane(ci);
    const PixOff<P> e = static_cast<PixOff<P>>(ri) * static_cast<unsigned>(in.cols[s.a]) + ci;
    r[s.dst] = pix_load<P, s.a>(in, e, static_cast<int>(rt.imm[PC]));
  } else if constexpr (s.op == VDSL_PIX_INDEX) {
    r[s.dst] = s.a == 0 ? fi : fj;
  } else if constexpr (s.op == VDSL_PIX_COUNT || s.op == VDSL_PIX_TRIP) {
    r[s.dst] = fcount;  // the count in the post section, the trip in the loop's sections
  } else if constexpr (s.op == VDSL_PIX_ATAN2) {
    r[s.dst] = atan2f(r[s.a], r[s.b]);
  } else if constexpr (s.op == VDSL_PIX_ASIN) {
    r[s.dst] = asinf(r[s.a]);
  } else if constexpr (s.op == VDSL_PIX_ACOS) {
    r[s.dst] = acosf(r[s.a]);
  } else if constexpr (s.op == VDSL_PIX_ATAN) {
    r[s.dst] = atanf(r[s.a]);
  } else if constexpr (s.op == VDSL_PIX_TAN) {
    r[s.dst] = tanf(r[s.a]);
  } else if constexpr (s.op == VDSL_PIX_POWF) {
    r[s.dst] = powf(r[s.a], r[s.b]);
  } else if constexpr (s.op == VDSL_PIX_ROUND) {
    r[s.dst] = roundf(r[s.a]);
  } else if constexpr (s.op >= VDSL_PIX_BAND && s.op <= VDSL_PIX_SHR) {
    const int x = pix_to_i32(r[s.a]), y = pix_to_i32(r[s.b]);
    int v;
    if constexpr (s.op == VDSL_PIX_BAND) v = x & y;
    else if constexpr (s.op == VDSL_PIX_BOR) v = x | y;
    else if constexpr (s.op == VDSL_PIX_BXOR) v = x ^ y;
    else if constexpr (s.op == VDSL_PIX_SHL) v = static_cast<int>(static_cast<unsigned>(x) << (y & 31));
    else v = x >> (y & 31);
    r[s.dst] = static_cast<float>(v);
  } else if constexpr (s.op == VDSL_PIX_COS) {
    r[s.dst] = cosf(r[s.a]);
  } else if constexpr (s.op == VDSL_PIX_SIN) {
    r[s.dst] = sinf(r[s.a]);
  } else if constexpr (s.op == VDSL_PIX_LT) {
    r[s.dst] = r[s.a] < r[s.b] ? 1.0f : 0.0f;
  } else if constexpr (s.op == VDSL_PIX_LE) {
    r[s.dst] = r[s.a] <= r[s.b] ? 1.0f : 0.0f;
  } else if constexpr (s.op == VDSL_PIX_EQ) {
    r[s.dst] = r[s.a] == r[s.b] ? 1.0f : 0.0f;
  } else if constexpr (s.op == VDSL_PIX_NE) {
    r[s.dst] = r[s.a] != r[s.b] ? 1.0f : 0.0f;
  } else if constexpr (s.op == VDSL_PIX_SELECT) {
    r[s.dst] = r[s.a] != 0.0f ? r[s.b] : r[s.c];
  } else if constexpr (s.op == VDSL_PIX_RANDOM) {
    const unsigned pixel = static_cast<unsigned>(fi) * static_cast<unsigned>(nj) + static_cast<unsigned>(fj);
    r[s.dst] = pix_random(r[s.a], static_cast<unsigned>(rt.imm[PC]), pixel);
  } else if constexpr (s.op == VDSL_PIX_FLOOR) {
    r[s.dst] = floorf(r[s.a]);
  } else if constexpr (s.op == VDSL_PIX_TRUNC) {
    r[s.dst] = truncf(r[s.a]);
  } else {
    r[s.dst] = apply_op(s.op, r[s.a], r[s.b], r[s.c], rt.imm[PC]);
  }
}

template <class P, int BASE, int... K>
__device__ __forceinline__ void pix_section(const PixRt& rt, const PixIn& in, float (&r)[VDSL_PIX_MAX_REGS], PixOff<P> o,
                                            float fi, float fj, float fcount, int ni, int nj, bool act, PixAcc<P>& acc,
                                            Seq<K...>) {
  (pix_step<P, BASE + K>(rt, in, r, o, fi, fj, fcount, ni, nj, act, acc), ...);
}

template <int TEST>
__device__ __forceinline__ bool pix_test(float a, float b) {
  if constexpr (TEST == VDSL_PIX_TEST_LT) return a < b;
  else if constexpr (TEST == VDSL_PIX_TEST_LE) return a <= b;
  else if constexpr (TEST == VDSL_PIX_TEST_GT) return a > b;
  else if constexpr (TEST == VDSL_PIX_TEST_GE) return a >= b;
  else return true;
}

// Registers an instruction reads (a bit per register).
__device__ constexpr uint32_t pix_reads(const vdsl_map_instr& s) {
  switch (s.op) {
    case VDSL_MAP_LOAD: case VDSL_MAP_CONST: case VDSL_PIX_INDEX: case VDSL_PIX_COUNT: return 0u;
    case VDSL_MAP_ADD: case VDSL_MAP_SUB: case VDSL_MAP_MUL: case VDSL_MAP_DIV: case VDSL_MAP_MAX: case VDSL_MAP_MIN:
    case VDSL_PIX_LT: case VDSL_PIX_LE: case VDSL_PIX_EQ: case VDSL_PIX_NE: case VDSL_PIX_ATAN2: case VDSL_PIX_POWF:
    case VDSL_PIX_BAND: case VDSL_PIX_BOR: case VDSL_PIX_BXOR: case VDSL_PIX_SHL: case VDSL_PIX_SHR:
      return (1u << s.a) | (1u << s.b);
    case VDSL_PIX_LOAD_AT: return (1u << s.b) | (1u << s.c);
    case VDSL_MAP_FMA: case VDSL_PIX_SELECT: return (1u << s.a) | (1u << s.b) | (1u << s.c);
    case VDSL_PIX_ATOMIC_ADD: case VDSL_PIX_ATOMIC_MAX: case VDSL_PIX_ATOMIC_MIN: case VDSL_PIX_STORE_AT:
      return (1u << s.dst) | (1u << s.b) | (1u << s.c);  // the value is r[dst]
    default: return 1u << s.a;
  }
}

// Register an instruction writes (a bit); an effect (scatter-add, max, min, store) writes none.
__device__ constexpr uint32_t pix_writes(const vdsl_map_instr& s) {
  return pix_effect_op(s.op) ? 0u : 1u << s.dst;
}

// Register sets of program P (instructions [lo, hi) of its table): written, and read before
// written (read-before-write, i.e. the values the range takes from before it).
template <class P>
struct PixSets {
  static constexpr int t0 = P::n_pre, b0 = t0 + P::n_test, q0 = b0 + P::n_body, end = q0 + P::n_post;
  static constexpr uint32_t writes(int lo, int hi) {
    uint32_t w = 0u;
    for (int pc = lo; pc < hi; ++pc) w |= pix_writes(P::code[pc]);
    return w;
  }
  static constexpr uint32_t rbw(int lo, int hi) {
    uint32_t w = 0u, r = 0u;
    for (int pc = lo; pc < hi; ++pc) {
      r |= pix_reads(P::code[pc]) & ~w;
      w |= pix_writes(P::code[pc]);
    }
    return r;
  }
  static constexpr uint32_t test_w = writes(t0, b0);
  static constexpr uint32_t body_w = writes(b0, q0);
  static constexpr uint32_t loop_w = test_w | body_w;
  static constexpr uint32_t stored() {
    uint32_t m = 0u;
    if (P::out_kind != VDSL_PIX_OUT_COUNT && P::out_kind != VDSL_PIX_OUT_NONE)
      for (int k = 0; k < P::out_width; ++k) m |= 1u << P::out_regs[k];
    return m;
  }
  // What the post section and the store take from the loop.
  static constexpr uint32_t post_r = rbw(q0, end) | (stored() & ~writes(q0, end));
  static constexpr uint32_t keep_t = test_w & post_r;   // kept from the trip a lane's test failed
  static constexpr uint32_t keep_b = body_w & post_r;   // kept from the lane's last counted trip
  static constexpr bool free_running = (loop_w & post_r) == 0u;
  static constexpr uint32_t carried = rbw(t0, q0) & loop_w;  // the loop's state from trip to trip
  static constexpr bool reads_trip() {
    for (int pc = t0; pc < q0; ++pc)
      if (P::code[pc].op == VDSL_PIX_TRIP) return true;
    return false;
  }
  // a loop that reads its trip is not a function of its state alone: no periodicity exit
  static constexpr bool periodic = free_running && carried != 0u && !reads_trip();
};

// act: the pixel lies in the grid (its scatter-adds happen); acc: the thread's sums of its
// constant-index adds.
template <class P, int BASE, int N>
__device__ __forceinline__ void pix_run(const PixRt& rt, const PixIn& in, float (&r)[VDSL_PIX_MAX_REGS], PixOff<P> o,
                                        float fi, float fj, float fcount, int ni, int nj, bool act, PixAcc<P>& acc) {
  pix_section<P, BASE>(rt, in, r, o, fi, fj, fcount, ni, nj, act, acc, typename MakeSeq<N>::type{});
}

// The loop's sections, which hold no scatter-adds.
template <class P, int BASE, int N>
__device__ __forceinline__ void pix_run(const PixRt& rt, const PixIn& in, float (&r)[VDSL_PIX_MAX_REGS], PixOff<P> o,
                                        float fi, float fj, float fcount, int ni, int nj) {
  PixAcc<P> none;
  pix_section<P, BASE>(rt, in, r, o, fi, fj, fcount, ni, nj, false, none, typename MakeSeq<N>::type{});
}

// r[k] <- r[k] where the lane's bit of `mask` is set, else old[k], for the registers in KEEP.
template <uint32_t KEEP>
__device__ __forceinline__ void pix_keep(float (&r)[VDSL_PIX_MAX_REGS], const float (&old)[VDSL_PIX_MAX_REGS], uint64_t mask) {
#pragma unroll
  for (int k = 0; k < VDSL_PIX_MAX_REGS; ++k)
    if constexpr (KEEP != 0u)
      if ((KEEP >> k) & 1u) r[k] = lane_select_f(mask, r[k], old[k]);
}

// One trip: the test section, the lane's test into the sticky mask `lk`, the body.  Registers in
// the keep sets hold their values on lanes that are not live.
template <class P>
__device__ __forceinline__ void pix_trip(const PixRt& rt, const PixIn& in, float (&r)[VDSL_PIX_MAX_REGS], PixOff<P> o,
                                         float fi, float fj, int ni, int nj, uint64_t& lk, float trip) {
  using S = PixSets<P>;
  float old[VDSL_PIX_MAX_REGS];
  if constexpr (S::keep_t != 0u) {
#pragma unroll
    for (int k = 0; k < VDSL_PIX_MAX_REGS; ++k) old[k] = r[k];
  }
  const uint64_t start = lk;
  pix_run<P, S::t0, P::n_test>(rt, in, r, o, fi, fj, trip, ni, nj);
  pix_keep<S::keep_t>(r, old, start);
  lk &= __builtin_amdgcn_ballot_w64(pix_test<P::test>(r[P::test_a], r[P::test_b]));
  if constexpr (S::keep_b != 0u) {
#pragma unroll
    for (int k = 0; k < VDSL_PIX_MAX_REGS; ++k) old[k] = r[k];
  }
  pix_run<P, S::b0, P::n_body>(rt, in, r, o, fi, fj, trip, ni, nj);
  pix_keep<S::keep_b>(r, old, lk);
}

// Pixel (i, j) of program P (the program table: n_pre, n_test, n_body, n_post, loop, test, test_a,
// test_b, out_kind, out_width, out_regs[], in_widths[], code[]): its stored registers into res,
// its trip count into count.
template <class P>
__device__ __forceinline__ void pixel_eval(const PixRt& rt, const PixIn& in, int ni, int nj, int i, int j, float (&res)[4],
                                           int& count_out, PixAcc<P>& acc) {
  using S = PixSets<P>;
  const bool inside = i < ni && j < nj;
  // Lanes past the grid run the program on pixel (0, 0), are never live, and store nothing.
  const PixOff<P> o = inside ? static_cast<PixOff<P>>(i) * static_cast<unsigned>(nj) + static_cast<unsigned>(j) : PixOff<P>(0);
  const float fi = static_cast<float>(i), fj = static_cast<float>(j);
  float r[VDSL_PIX_MAX_REGS];
#pragma unroll
  for (int k = 0; k < VDSL_PIX_MAX_REGS; ++k) r[k] = 0.0f;
  pix_run<P, 0, P::n_pre>(rt, in, r, o, fi, fj, 0.0f, ni, nj, inside, acc);
  int count = 0;
  if constexpr (P::loop && P::test == VDSL_PIX_TEST_NONE) {
    // No test: every lane makes max_iter trips; they run only if something after the loop reads
    // what they compute.
    const int max_iter = rt.max_iter;
    if constexpr (!S::free_running) {
      // four trips per iteration: loads that depend only on the trip (gathers at it) can be
      // issued for all four before the arithmetic of the first
      int t = 0;
      for (; t + 4 <= max_iter; t += 4) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const float trip = static_cast<float>(t + u);
          pix_run<P, S::t0, P::n_test>(rt, in, r, o, fi, fj, trip, ni, nj);
          pix_run<P, S::b0, P::n_body>(rt, in, r, o, fi, fj, trip, ni, nj);
        }
      }
      for (; t < max_iter; ++t) {
        const float trip = static_cast<float>(t);
        pix_run<P, S::t0, P::n_test>(rt, in, r, o, fi, fj, trip, ni, nj);
        pix_run<P, S::b0, P::n_body>(rt, in, r, o, fi, fj, trip, ni, nj);
      }
    }
    count = max_iter;
  } else if constexpr (P::loop) {
    constexpr int kUnroll = 16;
    const int max_iter = rt.max_iter;
    uint64_t live = __builtin_amdgcn_ballot_w64(inside);
    float save[VDSL_PIX_MAX_REGS];
#pragma unroll
    for (int k = 0; k < VDSL_PIX_MAX_REGS; ++k) save[k] = r[k];
    int t = 0;
    for (; t <= max_iter - kUnroll; t += kUnroll) {
      uint64_t m[kUnroll];
      uint64_t lk = live;
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        pix_trip<P>(rt, in, r, o, fi, fj, ni, nj, lk, static_cast<float>(t + u));
        m[u] = lk;
      }
      count += block_trips16(m, live);
      live = lk;
      if constexpr (S::periodic) {
        uint64_t same = live;
#pragma unroll
        for (int k = 0; k < VDSL_PIX_MAX_REGS; ++k)
          if ((S::carried >> k) & 1u) same &= __builtin_amdgcn_ballot_w64(__float_as_uint(r[k]) == __float_as_uint(save[k]));
        if (same) count = lane_select_keep(same, max_iter, count);
        live &= ~same;
        const int blocks_done = __builtin_amdgcn_readfirstlane(t) / kUnroll + 1;  // wave-uniform
        if ((blocks_done & (blocks_done - 1)) == 0) {
#pragma unroll
          for (int k = 0; k < VDSL_PIX_MAX_REGS; ++k)
            if ((S::carried >> k) & 1u) save[k] = r[k];
        }
      }
      if (live == 0ull) break;
    }
    if (t > max_iter - kUnroll && live != 0ull) {
      for (; t < max_iter; ++t) {  // the last max_iter % 16 trips, counted one by one
        pix_trip<P>(rt, in, r, o, fi, fj, ni, nj, live, static_cast<float>(t));
        count += lane_select(live, 1, 0);
      }
    }
  }
  pix_run<P, S::q0, P::n_post>(rt, in, r, o, fi, fj, static_cast<float>(count), ni, nj, inside, acc);
#pragma unroll
  for (int k = 0; k < 4; ++k) res[k] = k < P::out_width ? r[P::out_regs[k]] : 0.0f;
  count_out = count;
}

// Stores what pixel_eval gave for pixel (i, j), if it lies in the grid.  out: f32
// [ni][nj][out_width] or int32 [ni][nj].
template <class P>
__device__ __forceinline__ void pixel_store(void* __restrict__ out, int ni, int nj, int i, int j, const float (&res)[4],
                                            int count) {
  if constexpr (P::out_kind == VDSL_PIX_OUT_NONE) return;
  if (i >= ni || j >= nj) return;
  const PixOff<P> o = static_cast<PixOff<P>>(i) * static_cast<unsigned>(nj) + static_cast<unsigned>(j);
  char* base = static_cast<char*>(out);
  if constexpr (P::out_kind == VDSL_PIX_OUT_COUNT) {
    *reinterpret_cast<int*>(base + o * 4u) = count;
  } else if constexpr (P::out_kind == VDSL_PIX_OUT_I32) {
    *reinterpret_cast<int*>(base + o * 4u) = pix_to_i32(res[0]);
  } else {
#pragma unroll
    for (int k = 0; k < P::out_width; ++k)
      *reinterpret_cast<float*>(base + (o * P::out_width + static_cast<PixOff<P>>(k)) * 4u) = res[k];
  }
}

// P::rows > 0: a block takes 256 consecutive pixels of P::rows rows (programs whose pixels all
// do the same work, where memory access is what counts: every load and store of a wave is 256
// contiguous bytes).  A thread evaluates its P::rows pixels before it stores any of them, so the
// loads of all of them are in flight together (a store between them would hold every later load
// back, since the output may be an input).  Pixels read their own inputs before anything is
// stored, and a read of another pixel's element that the same launch writes has no defined
// order in any mapping.  Otherwise 8x8 tiles per wave and a 16x16 patch per block (escape loops,
// whose lanes leave at different trips).
//
// Row blocks are renumbered so that each XCD walks one contiguous band of whole rows: the hardware
// sends block L (row-major over the grid) to XCD L % 8, so without this the 256-column blocks to
// the left and right of a block run on other XCDs, and a gather's neighbour columns (j - 1 of the
// first lane, j + 1 of the last) cost two more 128-byte lines per 1 KiB row in this XCD's L2:
// +25% of the input fetched for a five-point stencil.  Any bijection is correct; this one keeps
// neighbouring blocks in one L2.
// The block's sums in an LDS copy added to input A, element by element (only those not +0 /
// 0: adding them would change nothing, beyond turning a -0 target into +0).
template <class P, int A>
__device__ __forceinline__ void pix_priv_flush(const PixIn& in, const unsigned* sh) {
  if constexpr (P::priv[A] > 0) {
    char* base = const_cast<char*>(reinterpret_cast<const char*>(in.p[A]));
    for (int e = threadIdx.x; e < P::priv[A]; e += 256) {
      const unsigned v = sh[P::priv_off[A] + e];
      if (v == 0u) continue;
      if constexpr (P::in_dtypes[A] == VDSL_I32) atomicAdd(reinterpret_cast<int*>(base) + e, static_cast<int>(v));
      else unsafeAtomicAdd(reinterpret_cast<float*>(base) + e, __uint_as_float(v));
    }
  }
}

template <class P, int... A>
__device__ __forceinline__ void pix_priv_flush_all(const PixIn& in, const unsigned* sh, Seq<A...>) {
  (pix_priv_flush<P, A>(in, sh), ...);
}

__device__ __forceinline__ unsigned xcd_band(unsigned L, unsigned G) {
  const unsigned x = L % 8, k = L / 8, q = G / 8, r = G % 8;
  return x * q + (x < r ? x : r) + k;  // XCD x takes logical blocks [x q + min(x, r), + q + (x < r))
}

template <class P>
__device__ __forceinline__ void pixel_body(const PixRt& rt, const PixIn& in, void* __restrict__ out, int ni, int nj) {
  float res[P::rows > 0 ? P::rows : 1][4];
  int count[P::rows > 0 ? P::rows : 1];
  PixAcc<P> acc{};
  // per-block LDS copies of the small scatter targets (a histogram's bins), in one array at the
  // offsets the host chose, zeroed first
  __shared__ unsigned sh[P::priv_total > 0 ? P::priv_total : 1];
  constexpr bool priv = P::priv_total > 0;
  if constexpr (priv) {
#pragma unroll
    for (int k = 0; k < VDSL_PIX_MAX_INPUTS; ++k) acc.sh[k] = sh + P::priv_off[k];
    for (int e = threadIdx.x; e < P::priv_total; e += 256) sh[e] = 0u;
    __syncthreads();
  }
  if constexpr (P::rows > 0) {
    const unsigned T = xcd_band(blockIdx.y * gridDim.x + blockIdx.x, gridDim.x * gridDim.y);
    const int j = static_cast<int>((T % gridDim.x) * 256 + threadIdx.x);
    const int i0 = static_cast<int>(T / gridDim.x) * P::rows;
    if constexpr (P::out_kind == VDSL_PIX_OUT_NONE) {
      // nothing stored (a reduction into a few elements, whose blocks cover many rows so that
      // few adds reach memory): the rows in a loop, eight at a time
#pragma unroll 8
      for (int t = 0; t < P::rows; ++t) {
        if constexpr (P::loop)
          if (i0 + t >= ni) break;
        float unused[4];
        int unused_count;
        pixel_eval<P>(rt, in, ni, nj, i0 + t, j, unused, unused_count, acc);
      }
    } else {
#pragma unroll
      for (int t = 0; t < P::rows; ++t) {
        // a loop is not run for the last band's rows past the grid (the same for the whole
        // block); a program without one evaluates them unconditionally, so the loads of all its
        // rows are issued together (a branch between them would order them)
        if constexpr (P::loop)
          if (i0 + t >= ni) break;
        pixel_eval<P>(rt, in, ni, nj, i0 + t, j, res[t], count[t], acc);
      }
#pragma unroll
      for (int t = 0; t < P::rows; ++t) pixel_store<P>(out, ni, nj, i0 + t, j, res[t], count[t]);
    }
  } else {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int i = static_cast<int>(blockIdx.y * 16 + (wave >> 1) * 8 + (lane >> 3));
    const int j = static_cast<int>(blockIdx.x * 16 + (wave & 1) * 8 + (lane & 7));
    pixel_eval<P>(rt, in, ni, nj, i, j, res[0], count[0], acc);
    pixel_store<P>(out, ni, nj, i, j, res[0], count[0]);
  }
  pix_flush<P>(rt, in, acc, typename MakeSeq<PixConstAdds<P>::end>::type{});
  if constexpr (priv) {
    __syncthreads();
    pix_priv_flush_all<P>(in, sh, typename MakeSeq<VDSL_PIX_MAX_INPUTS>::type{});
  }
}

}  // namespace vdsl

// Branch-free f32 math and the clang vector types, shared by the kernels compiled with the library
// and by the map-chain kernels the library compiles at run time (map_chain.hip embeds this file's
// text for hiprtc).  Self-contained: no includes.
#pragma once

namespace vdsl {

// Clang vector types (what the nontemporal and MFMA builtins accept).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// exp in f32, Cody-Waite style: n log2(e) = t + r with t = fl(n * log2e) and r its rounding
// residual (exact through an fma, plus the low part of log2 e), then e^n = 2^t (1 + r ln 2) with
// the hardware exp2.  Where t is not finite (n = +-inf, NaN) or 2^t overflows, 2^t itself is the
// answer (inf, 0 or NaN) and the correction, which would form inf * 0, is skipped.  Relative
// error below 2e-7 in an f32 emulation of these steps (against exp in f64 over [-87, 88]), plus
// the hardware exp2's 1 ulp.
__device__ __forceinline__ float exp_fast(float n) {
  const float t = n * 1.4426950408889634f;
  float r = __builtin_fmaf(n, 1.4426950408889634f, -t);
  r = __builtin_fmaf(n, 1.92596299e-08f, r);  // log2(e) - fl(log2(e))
  const float e = __builtin_amdgcn_exp2f(t);
  const float c = __builtin_fmaf(e, r * 0.6931471805599453f, e);
  return (__builtin_isfinite(t) && e != __builtin_inff()) ? c : e;
}

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

}  // namespace vdsl

// Per-lane work on 64-bit lane masks held in scalar registers, for wave-uniform loops whose lanes
// drop out one by one (the escape-time kernel, escape_time.hip, and general per-pixel programs,
// pixprog_kern.h).  A loop keeps its live set as a sticky mask (one ballot and one scalar AND per
// trip) instead of branching per lane, and turns masks into per-lane values with selects whose
// condition operand is the mask itself, so a mask is never expanded into a vector of 0/1 first.
// Uses nothing from the C++ standard library (this header is also compiled at run time).
#pragma once

#include <stdint.h>

namespace vdsl {

// if_set where the lane's bit of `mask` is set, else if_clear.
__device__ __forceinline__ int lane_select(uint64_t mask, int if_set, int if_clear) {
  int r;
  asm("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(r) : "v"(if_clear), "v"(if_set), "s"(mask));
  return r;
}

__device__ __forceinline__ float lane_select_f(uint64_t mask, float if_set, float if_clear) {
  float r;
  asm("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(r) : "v"(if_clear), "v"(if_set), "s"(mask));
  return r;
}

// V where the lane's bit is set, else 0.  volatile, so a select meant for a rarely taken branch is
// not hoisted out of it.
template <int V>
__device__ __forceinline__ int lane_bit(uint64_t mask) {
  int r;
  asm volatile("v_cndmask_b32_e64 %0, 0, %1, %2" : "=v"(r) : "n"(V), "s"(mask));
  return r;
}

__device__ __forceinline__ int lane_select_keep(uint64_t mask, int if_set, int keep) {
  int r;
  asm volatile("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(r) : "v"(keep), "v"(if_set), "s"(mask));
  return r;
}

// Trips each lane was live for in a block of 16 trips: m[u] is the sticky live mask after trip u
// (m[0] >= m[1] >= ... as lane sets), `start` the mask before the block.  Per lane the count is
// c = #{u : bit set in m[u]} in [0, 16]: with no lane lost in the block every live lane adds 16
// (one select); otherwise the bits of c follow from a binary search over the masks (scalar ops),
// since c >= 8 iff m[7], then c >= 8 + 4 iff m[11] (or c >= 4 iff m[3] below 8), and so on, and
// c == 16 adds m[15] (five selects).
__device__ __forceinline__ int block_trips16(const uint64_t (&m)[16], uint64_t start) {
  if (m[15] == start) return lane_select(start, 16, 0);
  const uint64_t b3 = m[7];
  const uint64_t b2 = (m[7] & m[11]) | (~m[7] & m[3]);
  const uint64_t c00 = ~b3 & ~b2, c01 = ~b3 & b2, c10 = b3 & ~b2, c11 = b3 & b2;
  const uint64_t b1 = (c00 & m[1]) | (c01 & m[5]) | (c10 & m[9]) | (c11 & m[13]);
  const uint64_t b0 = (c00 & ~b1 & m[0]) | (c00 & b1 & m[2]) | (c01 & ~b1 & m[4]) | (c01 & b1 & m[6]) |
                      (c10 & ~b1 & m[8]) | (c10 & b1 & m[10]) | (c11 & ~b1 & m[12]) | (c11 & b1 & m[14]);
  return lane_bit<1>(b0) + lane_bit<2>(b1) + lane_bit<4>(b2) + lane_bit<8>(b3) + lane_bit<1>(m[15]);
}

}  // namespace vdsl

// dc_intdiv.hpp — C# int division by a constant through a multiply-high (host and device).
#pragma once

#ifndef __HIPCC_RTC__
#include <hip/hip_runtime.h>
#endif

#include <cstdint>

namespace dc {

// Signed int32 division by a constant d, 2 <= |d| <= 2^31, as a multiply-high and shifts
// (T. Granlund and P. Montgomery, "Division by invariant integers using multiplication", PLDI 1994;
// the magic-number construction of H. S. Warren, Hacker's Delight, 2nd ed., figure 10-1). The
// constant is a wave-uniform immediate, so the construction runs on uniform values once per
// instruction and each element pays a multiply-high, an add, two shifts and an add, where a
// general division costs a reciprocal sequence of some twenty instructions.
struct DivMagic {
  int32_t m;  // magic multiplier
  int32_t s;  // shift
  int32_t d;  // the divisor
};

// Out of line: it runs once per instruction on wave-uniform values, and inlined into every
// unrolled interpreter variant it would keep the compiler from unrolling their element loops.
__host__ __device__ __attribute__((noinline)) inline DivMagic div_magic(int32_t d) {
  const uint32_t two31 = 0x80000000u;
  const uint32_t ad = d < 0 ? 0u - (uint32_t)d : (uint32_t)d;
  const uint32_t t = two31 + ((uint32_t)d >> 31);
  const uint32_t anc = t - 1u - t % ad;  // |nc|
  int p = 31;
  uint32_t q1 = two31 / anc, r1 = two31 - q1 * anc;
  uint32_t q2 = two31 / ad, r2 = two31 - q2 * ad;
  uint32_t delta;
  do {
    ++p;
    q1 *= 2u;
    r1 *= 2u;
    if (r1 >= anc) { ++q1; r1 -= anc; }
    q2 *= 2u;
    r2 *= 2u;
    if (r2 >= ad) { ++q2; r2 -= ad; }
    delta = ad - r2;
  } while (q1 < delta || (q1 == delta && r1 == 0u));
  int32_t m = (int32_t)(q2 + 1u);
  if (d < 0) m = (int32_t)(0u - (uint32_t)m);
  return DivMagic{m, p - 32, d};
}

// n / d truncated toward zero (C#'s int division), for the d of div_magic.
__host__ __device__ inline int32_t div_by_magic(int32_t n, const DivMagic& g) {
  int32_t q = (int32_t)(((int64_t)g.m * (int64_t)n) >> 32);
  if (g.d > 0 && g.m < 0) q = (int32_t)((uint32_t)q + (uint32_t)n);
  if (g.d < 0 && g.m > 0) q = (int32_t)((uint32_t)q - (uint32_t)n);
  q >>= g.s;
  return (int32_t)((uint32_t)q + ((uint32_t)q >> 31));
}

}  // namespace dc

// dc_gen_support.hpp — device helpers of the kernels the generator translates from [Kernel] C#
// bodies (dotcompute_amd/generator): the launch block (dc_gen_launch, declared in
// include/dotcompute_hip.h), bounds-checked span loads, and the C# meaning of integer division,
// shifts, float -> integer casts and Math.Abs/Min/Max. Errors a C# body would throw are reported by
// storing the launch's epoch into one of its error words (plain stores: any thread that hits the
// error writes the same value), which the host turns into the exception after the launch.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <limits>
#include <type_traits>

#include "../../include/dotcompute_hip.h"

namespace dcg {

__device__ inline void raise(const dc_gen_launch& l, int which) { l.error[which] = l.epoch; }

// Span<T> indexer: an index outside [0, len) throws IndexOutOfRangeException in C#.
template <typename T>
__device__ inline T ld(const T* p, int64_t i, int64_t len, const dc_gen_launch& l) {
  if ((uint64_t)i < (uint64_t)len) return p[i];
  raise(l, DC_GEN_ERR_INDEX);
  return T();
}

// Integer division and remainder: DivideByZeroException for a zero divisor; MinValue / -1 (and
// % -1) overflow, which .NET on x64 reports as OverflowException.
template <typename T>
__device__ inline T idiv(T a, T b, const dc_gen_launch& l) {
  if (b == 0) {
    raise(l, DC_GEN_ERR_DIVIDE_BY_ZERO);
    return T();
  }
  if constexpr (std::is_signed<T>::value) {
    if (b == T(-1) && a == std::numeric_limits<T>::min()) {
      raise(l, DC_GEN_ERR_OVERFLOW);
      return T();
    }
  }
  return a / b;
}
template <typename T>
__device__ inline T irem(T a, T b, const dc_gen_launch& l) {
  if (b == 0) {
    raise(l, DC_GEN_ERR_DIVIDE_BY_ZERO);
    return T();
  }
  if constexpr (std::is_signed<T>::value) {
    if (b == T(-1) && a == std::numeric_limits<T>::min()) {
      raise(l, DC_GEN_ERR_OVERFLOW);
      return T();
    }
  }
  return a % b;
}

// Shifts: C# masks the count to the operand width (5 bits for 32-bit operands, 6 for 64-bit); the
// left shift is done on the unsigned representation (wrapping, no undefined behaviour).
template <typename T>
__device__ inline T shl(T a, int32_t n) {
  using U = typename std::make_unsigned<T>::type;
  return (T)((U)a << (n & (int32_t)(sizeof(T) * 8 - 1)));
}
template <typename T>
__device__ inline T shr(T a, int32_t n) {
  return (T)(a >> (n & (int32_t)(sizeof(T) * 8 - 1)));  // arithmetic for signed T, logical for unsigned
}

// Floating -> integer cast as .NET 9 and later perform it: truncation toward zero, saturating at
// the target's range, NaN -> 0.
template <typename T, typename F>
__device__ inline T f2i(F x) {
  static_assert(sizeof(T) >= 4, "only int, uint, long and ulong targets");
  if (x != x) return T(0);
  const F lo = (F)std::numeric_limits<T>::min();                // exact: 0 or -2^(bits-1)
  const F hi = (F)std::numeric_limits<T>::max() + (F)1;         // 2^bits or 2^(bits-1): rounds exactly
  if (x <= lo) return std::numeric_limits<T>::min();
  if (x >= hi) return std::numeric_limits<T>::max();
  return (T)x;
}

// Math.Abs(int/long): OverflowException for MinValue.
template <typename T>
__device__ inline T abs_checked(T x, const dc_gen_launch& l) {
  if (x == std::numeric_limits<T>::min()) {
    raise(l, DC_GEN_ERR_OVERFLOW);
    return T();
  }
  return x < 0 ? (T)-x : x;
}

template <typename T>
__device__ inline T imin(T a, T b) { return a <= b ? a : b; }
template <typename T>
__device__ inline T imax(T a, T b) { return a >= b ? a : b; }

// Math.Min/Max(float/double): IEEE 754-2019 minimum/maximum, the semantics .NET implements: a NaN
// operand wins, and -0 counts as smaller than +0.
template <typename T>
__device__ inline T fmin_net(T a, T b) {
  if (a != b) {
    if (a == a) return a < b ? a : b;  // b NaN: a < b is false, b is returned
    return a;
  }
  return signbit(a) ? a : b;
}
template <typename T>
__device__ inline T fmax_net(T a, T b) {
  if (a != b) {
    if (a == a) return b < a ? a : b;
    return a;
  }
  return signbit(b) ? a : b;
}

}  // namespace dcg

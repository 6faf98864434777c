// Host-side check of dc::div_magic / dc::div_by_magic (dotcompute_amd/csrc/dc_intdiv.hpp) against
// int64 truncating division: every divisor class the interpreter sends there (2 <= |d| <= 2^31,
// powers of two, int.MinValue, +-int.MaxValue) and random dividends, int.MinValue included.
// Built and run on the CPU by tests/test_intdiv.py.
#include <cstdio>
#include <random>

#include "../../dotcompute_amd/csrc/dc_intdiv.hpp"

int main() {
  std::mt19937_64 rng(1);
  const int32_t ds[] = {2, 3, -2, -3, 5, 6, 7, -7, 8, 16, 1024, 65536, 641, 1000, -1000, 2147483647, -2147483647,
                        INT32_MIN, 1 << 30, -(1 << 30), 3 << 20, 0x7ffffffe, 12345678};
  const int32_t ns[] = {0, 1, -1, 2, -2, 7, -7, 8, -8, 2147483647, INT32_MIN, -2147483647, 1000000, -1000000};
  long bad = 0, total = 0;
  auto check = [&](int32_t n, int32_t d) {
    const dc::DivMagic g = dc::div_magic(d);
    const int32_t q = dc::div_by_magic(n, g);
    const int64_t ref = (int64_t)n / (int64_t)d;
    if (q != (int32_t)ref) {
      if (bad < 10) std::printf("n=%d d=%d: %d, expected %lld\n", n, d, q, (long long)ref);
      ++bad;
    }
    ++total;
  };
  for (int32_t d : ds)
    for (int32_t n : ns) check(n, d);
  for (int i = 0; i < 3000000; ++i) {
    int32_t d = (int32_t)rng();
    if (i % 3 == 0) d = (int32_t)(rng() % 2000) - 1000;
    if (i % 7 == 0) d = (int32_t)(1u << (rng() % 32)) * ((rng() & 1) ? 1 : -1);
    if (d == 0 || d == 1 || d == -1) continue;
    int32_t n = (int32_t)rng();
    if (i % 5 == 0) n = (int32_t)(rng() % 20001) - 10000;
    check(n, d);
    if (i < 200000) {
      check(INT32_MIN, d);
      check(INT32_MAX, d);
      check(-INT32_MAX, d);
    }
  }
  std::printf("%ld of %ld quotients wrong\n", bad, total);
  return bad != 0;
}

// Minimal test harness for the C++ host-layer tests (run by tests/test_host_layer.py).
#pragma once
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

namespace dctest {
struct Case {
  std::string name;
  bool gpu;
  std::function<void()> fn;
};
inline std::vector<Case>& Registry() {
  static std::vector<Case> r;
  return r;
}
struct Register {
  Register(const char* n, bool gpu, std::function<void()> f) { Registry().push_back({n, gpu, std::move(f)}); }
};
struct Failure : std::runtime_error {
  using std::runtime_error::runtime_error;
};
}  // namespace dctest

#define DC_CAT2(a, b) a##b
#define DC_CAT(a, b) DC_CAT2(a, b)
#define TEST_CPU(name)                                                                 \
  static void name();                                                                  \
  static dctest::Register DC_CAT(reg_, name)(#name, false, name);                      \
  static void name()
#define TEST_GPU(name)                                                                 \
  static void name();                                                                  \
  static dctest::Register DC_CAT(reg_, name)(#name, true, name);                       \
  static void name()

#define CHECK(cond)                                                                    \
  do {                                                                                 \
    if (!(cond)) {                                                                     \
      std::ostringstream os_;                                                          \
      os_ << __FILE__ << ":" << __LINE__ << ": CHECK(" #cond ") failed";              \
      throw dctest::Failure(os_.str());                                                \
    }                                                                                  \
  } while (0)

#define CHECK_THROWS(ExcType, stmt)                                                    \
  do {                                                                                 \
    bool thrown_ = false;                                                              \
    try {                                                                              \
      stmt;                                                                            \
    } catch (const ExcType&) {                                                         \
      thrown_ = true;                                                                  \
    }                                                                                  \
    if (!thrown_) {                                                                    \
      std::ostringstream os_;                                                          \
      os_ << __FILE__ << ":" << __LINE__ << ": expected " #ExcType " from " #stmt;     \
      throw dctest::Failure(os_.str());                                                \
    }                                                                                  \
  } while (0)

inline int dctest_main(int argc, char** argv) {
  bool run_cpu = false, run_gpu = false;
  std::string only;
  for (int i = 1; i < argc; ++i) {
    if (!std::strcmp(argv[i], "--cpu")) run_cpu = true;
    else if (!std::strcmp(argv[i], "--gpu")) run_gpu = true;
    else if (!std::strcmp(argv[i], "--only") && i + 1 < argc) only = argv[++i];
  }
  if (!run_cpu && !run_gpu) run_cpu = true;
  int failed = 0, ran = 0;
  for (auto& c : dctest::Registry()) {
    if ((c.gpu && !run_gpu) || (!c.gpu && !run_cpu)) continue;
    if (!only.empty() && c.name != only) continue;
    std::printf("[ RUN  ] %s\n", c.name.c_str());
    std::fflush(stdout);
    ++ran;
    try {
      c.fn();
      std::printf("[  OK  ] %s\n", c.name.c_str());
    } catch (const std::exception& e) {
      ++failed;
      std::printf("[ FAIL ] %s: %s\n", c.name.c_str(), e.what());
    }
    std::fflush(stdout);
  }
  std::printf("%d test(s) ran, %d failed\n", ran, failed);
  return failed ? 1 : (ran ? 0 : 2);
}

// launch_latency_probe.cpp — measurement-only program (not linked into any library): what one
// kernel launch plus one wait costs on MI355X through HIP itself, the floor under every
// synchronous call of the orchestrator. A 100,000-float add and an empty kernel, launched on one
// stream and waited for with hipStreamSynchronize, hipEventSynchronize or an hipEventQuery spin;
// medians over 2000 calls. Argument: "spin" or "yield" sets that device schedule first.
// Build and run:
//   hipcc --offload-arch=gfx950 -O3 dotcompute_amd/probes/launch_latency_probe.cpp -o /tmp/launch_latency_probe && \
//     /tmp/launch_latency_probe && /tmp/launch_latency_probe spin && /tmp/launch_latency_probe yield
#include <hip/hip_runtime.h>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>
#include <algorithm>
#define CK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { printf("HIP %s at %d\n", hipGetErrorString(e_), __LINE__); exit(1); } } while (0)
using Clock = std::chrono::steady_clock;
__global__ void vadd(const float* a, const float* b, float* c, int n) {
  int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) c[i] = a[i] + b[i];
}
__global__ void empty_k() {}
template <class F> double med(F&& f, int it = 2000) {
  for (int i = 0; i < 100; ++i) f();
  std::vector<double> us(it);
  for (int i = 0; i < it; ++i) { auto t0 = Clock::now(); f(); us[i] = std::chrono::duration<double, std::micro>(Clock::now() - t0).count(); }
  std::sort(us.begin(), us.end());
  return us[it / 2];
}
int main(int argc, char** argv) {
  const bool spin = argc > 1 && !strcmp(argv[1], "spin");
  const bool yield = argc > 1 && !strcmp(argv[1], "yield");
  if (spin) CK(hipSetDeviceFlags(hipDeviceScheduleSpin));
  if (yield) CK(hipSetDeviceFlags(hipDeviceScheduleYield));
  const int n = 100000;
  float *a, *b, *c;
  CK(hipMalloc(&a, n * 4)); CK(hipMalloc(&b, n * 4)); CK(hipMalloc(&c, n * 4));
  hipStream_t s; CK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  hipEvent_t ev; CK(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
  hipEvent_t e0, e1; CK(hipEventCreate(&e0)); CK(hipEventCreate(&e1));
  const unsigned g = (n + 255) / 256;
  printf("mode %s\n", spin ? "spin" : yield ? "yield" : "default");
  printf("vadd launch+streamsync   %.2f us\n", med([&] { vadd<<<g, 256, 0, s>>>(a, b, c, n); CK(hipStreamSynchronize(s)); }));
  printf("empty launch+streamsync  %.2f us\n", med([&] { empty_k<<<1, 64, 0, s>>>(); CK(hipStreamSynchronize(s)); }));
  printf("vadd launch+event poll   %.2f us\n", med([&] { vadd<<<g, 256, 0, s>>>(a, b, c, n); CK(hipEventRecord(ev, s)); while (hipEventQuery(ev) == hipErrorNotReady) {} }));
  printf("vadd launch+eventsync    %.2f us\n", med([&] { vadd<<<g, 256, 0, s>>>(a, b, c, n); CK(hipEventRecord(ev, s)); CK(hipEventSynchronize(ev)); }));
  printf("vadd launch only (x100 then sync)/100 %.2f us\n", med([&] { for (int i = 0; i < 100; ++i) vadd<<<g, 256, 0, s>>>(a, b, c, n); CK(hipStreamSynchronize(s)); }, 50) / 100);
  // kernel duration by events
  float ms = 0; CK(hipEventRecord(e0, s)); for (int i = 0; i < 1000; ++i) vadd<<<g, 256, 0, s>>>(a, b, c, n); CK(hipEventRecord(e1, s)); CK(hipEventSynchronize(e1)); CK(hipEventElapsedTime(&ms, e0, e1));
  printf("vadd back-to-back per launch (events) %.2f us\n", ms);
  // host-side launch call cost only
  printf("vadd launch call (host, no wait)  %.2f us\n", med([&] { vadd<<<g, 256, 0, s>>>(a, b, c, n); }, 1000));
  CK(hipStreamSynchronize(s));
  return 0;
}

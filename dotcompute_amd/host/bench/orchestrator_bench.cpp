// orchestrator_bench.cpp — end-to-end cost of the README quick start through the orchestrator:
// `orchestrator.ExecuteAsync<float[]>("VectorAdd", "HIP", a, b, result)` with host arrays (copy in,
// launch, copy back, what the managed API implies), and ExecuteWithBuffersAsync on device-resident
// buffers (launch and synchronise only). Beside them, the floor of the device-resident call: the
// same compiled kernel launched directly (its argument block built once) and waited for, and a
// wait on the idle stream. Prints one JSON object; bench.py reports it.
// Usage: dc_orchestrator_bench [n] [iterations]
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "DotCompute/Backends/Hip.hpp"
#include "DotCompute/Runtime.hpp"

using namespace DotCompute;
using Clock = std::chrono::steady_clock;

namespace {

struct Stats {
  double median_us, p10_us, p90_us;
};

template <typename F>
Stats Time(F&& f, int iterations, int warmup) {
  for (int i = 0; i < warmup; ++i) f();
  std::vector<double> us(iterations);
  for (int i = 0; i < iterations; ++i) {
    const auto t0 = Clock::now();
    f();
    us[i] = std::chrono::duration<double, std::micro>(Clock::now() - t0).count();
  }
  std::sort(us.begin(), us.end());
  return {us[us.size() / 2], us[us.size() / 10], us[us.size() * 9 / 10]};
}

}  // namespace

int main(int argc, char** argv) {
  const size_t n = argc > 1 ? (size_t)std::atoll(argv[1]) : 100000;
  const int iterations = argc > 2 ? std::atoi(argv[2]) : 300;
  ServiceCollection services;
  services.AddDotComputeRuntime().AddHipBackend();
  auto sp = services.BuildServiceProvider();
  auto orch = sp->GetRequiredOrchestrator();
  sp->Runtime()->Initialize();
  if (sp->Runtime()->GetAccelerators().empty()) {
    std::fprintf(stderr, "no HIP accelerator: %s\n", Backends::Hip::LastAcceleratorCreationError().c_str());
    return 2;
  }
  auto& acc = *sp->Runtime()->GetAccelerators()[0];
  std::vector<float> a(n), b(n), r(n);
  dc_gen_uniform_f32(a.data(), (int64_t)n, 42, 0, 0);
  dc_gen_uniform_f32(b.data(), (int64_t)n, 42, 1, 0);

  const Stats e2e = Time([&] { orch->ExecuteAsync("VectorAdd", "HIP", {Arg(a), Arg(b), Arg(r)}).get(); },
                         iterations, 30);
  size_t bad = 0;
  for (size_t i = 0; i < n; ++i) bad += r[i] != a[i] + b[i];

  auto da = acc.Memory().AllocateRaw(n, ElementType::Float32), db = acc.Memory().AllocateRaw(n, ElementType::Float32),
       dr = acc.Memory().AllocateRaw(n, ElementType::Float32);
  da->CopyFromHost(a.data(), n * sizeof(float));
  db->CopyFromHost(b.data(), n * sizeof(float));
  const Stats resident = Time([&] { orch->ExecuteWithBuffersAsync("VectorAdd", {da.get(), db.get(), dr.get()}, {}).get(); },
                              iterations, 30);
  // The floor under ExecuteWithBuffersAsync: the registry's VectorAdd kernel launched through its
  // compiled handle with a prebuilt argument block, then one wait (no lookup, no validation).
  auto* hip = dynamic_cast<Backends::Hip::HipAccelerator*>(&acc);
  std::string entry;
  for (const auto& k : Generated::KernelRegistry::GetAllKernels())
    if (k.Name == "VectorAdd") entry = k.HipEntryPoint;
  KernelDefinition def;
  def.Name = "VectorAdd";
  def.EntryPoint = entry;
  def.Language = KernelLanguage::HIP;
  auto compiled = acc.CompileKernelAsync(def).get();
  dc_gen_launch launch{};
  launch.work = (int64_t)n;
  launch.error = hip->GeneratedErrorWordsDevice();
  for (int k = 0; k < 3; ++k) launch.len[k] = (int64_t)n;
  KernelArguments kargs;
  kargs.AddBuffer(da.get());
  kargs.AddBuffer(db.get());
  kargs.AddBuffer(dr.get());
  RawArgument block;
  block.Bytes.resize(sizeof(launch));
  kargs.LaunchConfiguration.BlockSize = {DC_GEN_BLOCK, 1, 1};
  kargs.LaunchConfiguration.GridSize = {(uint32_t)((n + DC_GEN_BLOCK - 1) / DC_GEN_BLOCK), 1, 1};
  const Stats floor = Time([&] {
    launch.epoch = hip->NextLaunchEpoch();
    std::memcpy(block.Bytes.data(), &launch, sizeof(launch));
    kargs.ScalarArguments.assign(1, block);
    compiled->ExecuteAsync(kargs).get();
    hip->Synchronize();
  }, iterations, 30);
  const Stats idle_sync = Time([&] { hip->Synchronize(); }, iterations, 10);
  // The pieces of the host-array path on their own: one host -> device copy of an input and one
  // device -> host copy of the result, each waited for.
  const Stats h2d = Time([&] { da->CopyFromHost(a.data(), n * sizeof(float)); }, iterations, 10);
  const Stats d2h = Time([&] { dr->CopyToHost(r.data(), n * sizeof(float)); }, iterations, 10);
  std::printf(
      "{\"n\": %zu, \"iterations\": %d, \"bit_exact\": %s, "
      "\"execute_async_us\": {\"median\": %.2f, \"p10\": %.2f, \"p90\": %.2f}, "
      "\"execute_with_buffers_us\": {\"median\": %.2f, \"p10\": %.2f, \"p90\": %.2f}, "
      "\"launch_and_wait_us\": {\"median\": %.2f, \"p10\": %.2f, \"p90\": %.2f}, \"idle_wait_us\": %.2f, "
      "\"h2d_input_us\": %.2f, \"d2h_result_us\": %.2f}\n",
      n, iterations, bad == 0 ? "true" : "false", e2e.median_us, e2e.p10_us, e2e.p90_us, resident.median_us,
      resident.p10_us, resident.p90_us, floor.median_us, floor.p10_us, floor.p90_us, idle_sync.median_us, h2d.median_us,
      d2h.median_us);
  return bad == 0 ? 0 : 1;
}

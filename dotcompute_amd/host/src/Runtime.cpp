// Runtime.cpp — registry, discovery, DI and the orchestrator for the HIP backend.
#include "DotCompute/Runtime.hpp"

#include <algorithm>
#include <cctype>

namespace DotCompute {

namespace {
std::string Upper(std::string s) {
  std::transform(s.begin(), s.end(), s.begin(), [](unsigned char c) { return (char)std::toupper(c); });
  return s;
}
bool EqualsIgnoreCase(const std::string& a, const std::string& b) { return Upper(a) == Upper(b); }
}  // namespace

// ---- generated registry -------------------------------------------------------------------------

std::vector<KernelRegistrationInfo> Generated::KernelRegistry::GetAllKernels() {
  // [Kernel] public static void VectorAdd(ReadOnlySpan<float> a, ReadOnlySpan<float> b,
  //                                       Span<float> result)  — README.md quick start.
  KernelRegistrationInfo vadd;
  vadd.Name = "VectorAdd";
  vadd.FullName = "Kernels.VectorAdd";
  vadd.SupportedBackends = {"CPU"};  // the [Kernel] default (KernelAttribute.cs:36)
  vadd.Parameters = {{"a", ElementType::Float32, true, true},
                     {"b", ElementType::Float32, true, true},
                     {"result", ElementType::Float32, true, false}};
  vadd.Dimensions = 1;
  vadd.HipEntryPoint = "VectorAdd";  // dc_kernels_gfx950.hsaco: (a, b, result, __length)
  vadd.HipNeedsLength = true;
  vadd.HipBuiltin = HipOp::VectorAddF32;
  return {vadd};
}

// ---- discovery / DI -----------------------------------------------------------------------------

void AcceleratorRuntime::Initialize() {
  if (initialized_) return;
  for (auto& f : factories_) {
    std::shared_ptr<IAccelerator> acc = f ? f() : nullptr;
    if (acc) accelerators_.push_back(std::move(acc));
  }
  initialized_ = true;
}

ServiceCollection& ServiceCollection::AddDotComputeRuntime() {
  runtime_added_ = true;
  return *this;
}

ServiceCollection& ServiceCollection::AddHipBackend(Backends::Hip::HipBackendOptions options) {
  factories_.push_back([options]() -> std::shared_ptr<IAccelerator> { return Backends::Hip::TryCreateAccelerator(options); });
  return *this;
}

ServiceCollection& ServiceCollection::AddAccelerator(std::function<std::shared_ptr<IAccelerator>()> factory) {
  factories_.push_back(std::move(factory));
  return *this;
}

std::shared_ptr<ServiceProvider> ServiceCollection::BuildServiceProvider() const {
  auto sp = std::make_shared<ServiceProvider>();
  sp->runtime_ = std::make_shared<AcceleratorRuntime>(factories_);
  if (runtime_added_) sp->orchestrator_ = std::make_shared<KernelExecutionService>(sp->runtime_);
  return sp;
}

std::shared_ptr<IComputeOrchestrator> ServiceProvider::GetRequiredOrchestrator() const {
  if (!orchestrator_)
    throw InvalidOperationException("No service for type 'IComputeOrchestrator' has been registered: call AddDotComputeRuntime().");
  return orchestrator_;
}

// ---- orchestrator -------------------------------------------------------------------------------

KernelExecutionService::KernelExecutionService(std::shared_ptr<AcceleratorRuntime> runtime) : runtime_(std::move(runtime)) {}

void KernelExecutionService::EnsureInitialized() {
  std::lock_guard<std::mutex> lock(mu_);
  if (initialized_) return;
  runtime_->Initialize();
  // GeneratedKernelDiscoveryService.DiscoverAndRegisterKernelsAsync: the generated registry.
  for (const auto& k : Generated::KernelRegistry::GetAllKernels()) {
    registry_[k.FullName] = k;
    registry_.emplace(k.Name, k);
  }
  initialized_ = true;
}

void KernelExecutionService::RegisterKernels(const std::vector<KernelRegistrationInfo>& kernels) {
  EnsureInitialized();
  std::lock_guard<std::mutex> lock(mu_);
  for (const auto& k : kernels) {
    registry_[k.FullName] = k;
    registry_[k.Name] = k;  // short-name index (KernelExecutionService.cs:170-193)
  }
}

std::optional<KernelRegistrationInfo> KernelExecutionService::TryResolveKernel(const std::string& name) const {
  std::lock_guard<std::mutex> lock(mu_);
  auto it = registry_.find(name);
  if (it == registry_.end()) return std::nullopt;
  return it->second;
}

std::string KernelExecutionService::MapDeviceTypeToBackend(const std::string& deviceType) {
  const std::string u = Upper(deviceType);
  if (u == "CUDA") return "CUDA";
  if (u == "CPU") return "CPU";
  if (u == "METAL") return "Metal";
  if (u == "OPENCL") return "OpenCL";
  if (u == "HIP" || u == "ROCM") return "HIP";
  return deviceType;
}

int KernelExecutionService::GetBackendPriority(const std::string& deviceType) {
  const std::string u = Upper(deviceType);
  if (u == "CUDA" || u == "HIP") return 1;
  if (u == "METAL") return 2;
  if (u == "OPENCL") return 3;
  if (u == "CPU") return 4;
  return 999;
}

size_t KernelExecutionService::DeriveWorkSize(const KernelRegistrationInfo& reg, const std::vector<KernelArg>& args) {
  // First writable buffer parameter's array length, else the largest array argument.
  for (size_t i = 0; i < args.size() && i < reg.Parameters.size(); ++i) {
    const auto& p = reg.Parameters[i];
    if (p.IsBuffer && !p.IsReadOnly) {
      if (auto* h = std::get_if<HostArray>(&args[i])) return h->Length;
      if (auto* b = std::get_if<IUnifiedMemoryBuffer*>(&args[i])) return (*b)->Length();
    }
  }
  size_t mx = 0;
  for (const auto& a : args) {
    if (auto* h = std::get_if<HostArray>(&a)) mx = std::max(mx, h->Length);
    if (auto* b = std::get_if<IUnifiedMemoryBuffer*>(&a)) mx = std::max(mx, (*b)->Length());
  }
  return mx;
}

KernelLaunchConfiguration KernelExecutionService::DeriveLaunch(const KernelRegistrationInfo& reg,
                                                               const std::vector<KernelArg>& args, size_t totalWork) {
  const int d = std::clamp(reg.Dimensions, 1, 3);
  KernelLaunchConfiguration lc;
  auto ceil_div = [](int64_t extent, uint32_t block) {
    return (uint32_t)std::max<int64_t>(1, (extent + block - 1) / (int64_t)block);
  };
  if (d == 1) {
    lc.BlockSize = {256, 1, 1};
    lc.GridSize = {ceil_div((int64_t)totalWork, 256), 1, 1};
    return lc;
  }
  // Trailing integer scalars are the extents: last -> X, then Y, then Z.
  std::vector<int64_t> ext;
  for (auto it = args.rbegin(); it != args.rend() && (int)ext.size() < d; ++it)
    if (auto* v = std::get_if<int32_t>(&*it)) ext.push_back(*v);
  const int64_t x = !ext.empty() ? ext[0] : std::max<int64_t>(1, (int64_t)totalWork);
  const int64_t y = ext.size() > 1 ? ext[1] : 1;
  const int64_t z = ext.size() > 2 ? ext[2] : 1;
  lc.BlockSize = d == 2 ? Dim3{16, 16, 1} : Dim3{8, 8, 4};
  lc.GridSize = {ceil_div(x, lc.BlockSize.X), ceil_div(y, lc.BlockSize.Y), ceil_div(z, lc.BlockSize.Z)};
  return lc;
}

bool KernelExecutionService::ValidateKernelArgsAsync(const std::string& kernelName, const std::vector<KernelArg>& args) {
  EnsureInitialized();
  auto reg = TryResolveKernel(kernelName);
  if (!reg) return false;
  if (args.size() < reg->Parameters.size()) return false;
  for (size_t i = 0; i < reg->Parameters.size(); ++i) {
    const auto& p = reg->Parameters[i];
    if (p.IsBuffer) {
      if (auto* h = std::get_if<HostArray>(&args[i])) {
        if (h->Type != p.Type || (h->Length > 0 && !h->Data)) return false;
      } else if (auto* b = std::get_if<IUnifiedMemoryBuffer*>(&args[i])) {
        if (!*b || (*b)->Type() != p.Type) return false;
      } else {
        return false;
      }
    } else if (std::holds_alternative<HostArray>(args[i]) || std::holds_alternative<IUnifiedMemoryBuffer*>(args[i])) {
      return false;
    }
  }
  return true;
}

std::vector<std::shared_ptr<IAccelerator>> KernelExecutionService::GetSupportedAcceleratorsAsync(const std::string& kernelName) {
  EnsureInitialized();
  auto reg = TryResolveKernel(kernelName);
  std::vector<std::shared_ptr<IAccelerator>> out;
  if (!reg) return out;
  for (const auto& acc : runtime_->GetAccelerators()) {
    const std::string backend = MapDeviceTypeToBackend(acc->Info().DeviceType);
    bool ok = std::any_of(reg->SupportedBackends.begin(), reg->SupportedBackends.end(),
                          [&](const std::string& b) { return EqualsIgnoreCase(b, backend); });
    // A registry kernel with a prebuilt HIP entry point runs on HIP regardless of [Kernel(Backends)].
    if (backend == "HIP" && (!reg->HipEntryPoint.empty() || reg->HipBuiltin != HipOp::None)) ok = true;
    if (ok) out.push_back(acc);
  }
  return out;
}

std::shared_ptr<IAccelerator> KernelExecutionService::GetOptimalAcceleratorAsync(const std::string& kernelName) {
  auto supported = GetSupportedAcceleratorsAsync(kernelName);
  if (supported.empty()) return nullptr;
  return *std::min_element(supported.begin(), supported.end(), [](const auto& a, const auto& b) {
    return GetBackendPriority(a->Info().DeviceType) < GetBackendPriority(b->Info().DeviceType);
  });
}

std::future<std::vector<float>> KernelExecutionService::ExecuteAsync(const std::string& kernelName,
                                                                     std::vector<KernelArg> args) {
  EnsureInitialized();
  auto reg = TryResolveKernel(kernelName);
  if (!reg)
    throw ArgumentException("Kernel '" + kernelName + "' is not registered. Ensure the kernel's registry is "
                            "discovered, pass the fully-qualified or short name, or register it via RegisterKernels().");
  auto acc = GetOptimalAcceleratorAsync(kernelName);
  if (!acc) {
    if (runtime_->GetAccelerators().empty())
      throw InvalidOperationException("No accelerators are registered with the runtime, so kernel '" + kernelName +
                                      "' cannot run. Register a backend (services.AddHipBackend()) before executing kernels.");
    throw InvalidOperationException("Kernel '" + kernelName + "' is registered but none of the available accelerators "
                                    "support its backends.");
  }
  return ExecuteAsync(kernelName, *acc, std::move(args));
}

std::future<std::vector<float>> KernelExecutionService::ExecuteAsync(const std::string& kernelName,
                                                                     const std::string& preferredBackend,
                                                                     std::vector<KernelArg> args) {
  EnsureInitialized();
  std::shared_ptr<IAccelerator> chosen;
  for (const auto& acc : runtime_->GetAccelerators())
    if (EqualsIgnoreCase(acc->Info().DeviceType, preferredBackend)) {
      chosen = acc;
      break;
    }
  // No accelerator of the preferred type: fall back to the optimal one (KernelExecutionService.cs:238-242).
  if (!chosen) return ExecuteAsync(kernelName, std::move(args));
  return ExecuteAsync(kernelName, *chosen, std::move(args));
}

std::future<std::vector<float>> KernelExecutionService::ExecuteAsync(const std::string& kernelName,
                                                                     IAccelerator& accelerator,
                                                                     std::vector<KernelArg> args) {
  EnsureInitialized();
  auto reg = TryResolveKernel(kernelName);
  if (!reg)
    throw ArgumentException("Kernel '" + kernelName + "' is not registered. Add the kernel via RegisterKernels() "
                            "before executing, or check for typos.");
  if (!ValidateKernelArgsAsync(kernelName, args))
    throw ArgumentException("Kernel argument validation failed for kernel '" + kernelName + "' (received " +
                            std::to_string(args.size()) + " arguments). Verify argument count, types, and ordering.");
  std::vector<float> result = ExecuteOn(*reg, accelerator, args);
  std::promise<std::vector<float>> p;
  p.set_value(std::move(result));
  return p.get_future();
}

std::shared_ptr<ICompiledKernel> KernelExecutionService::GetCompiled(const KernelRegistrationInfo& reg,
                                                                     IAccelerator& accelerator) {
  const std::string key = accelerator.Info().Id + "/" + reg.FullName;
  {
    std::lock_guard<std::mutex> lock(mu_);
    auto it = cache_.find(key);
    if (it != cache_.end()) return it->second;
  }
  if (reg.HipEntryPoint.empty())
    throw NotSupportedException("Kernel '" + reg.Name + "' has no prebuilt HIP entry point for gfx950.");
  KernelDefinition def;
  def.Name = reg.Name;
  def.EntryPoint = reg.HipEntryPoint;
  def.Language = KernelLanguage::HIP;
  auto compiled = accelerator.CompileKernelAsync(def).get();
  std::lock_guard<std::mutex> lock(mu_);
  cache_[key] = compiled;
  return compiled;
}

void KernelExecutionService::PrecompileKernelAsync(const std::string& kernelName, IAccelerator* accelerator) {
  EnsureInitialized();
  auto reg = TryResolveKernel(kernelName);
  if (!reg) throw ArgumentException("Kernel '" + kernelName + "' is not registered.");
  std::shared_ptr<IAccelerator> acc;
  if (!accelerator) {
    acc = GetOptimalAcceleratorAsync(kernelName);
    if (!acc) throw InvalidOperationException("no accelerator supports kernel '" + kernelName + "'");
    accelerator = acc.get();
  }
  if (MapDeviceTypeToBackend(accelerator->Info().DeviceType) == "HIP" && !reg->HipEntryPoint.empty())
    GetCompiled(*reg, *accelerator);
}

std::vector<float> KernelExecutionService::ExecuteOn(const KernelRegistrationInfo& reg, IAccelerator& accelerator,
                                                     std::vector<KernelArg>& args) {
  const std::string backend = MapDeviceTypeToBackend(accelerator.Info().DeviceType);
  if (backend != "HIP")
    throw NotSupportedException("this build drives HIP accelerators only (got device type '" +
                                accelerator.Info().DeviceType + "')");
  const size_t totalWork = DeriveWorkSize(reg, args);

  // Marshal: a device buffer per host array, copied in (the reference copies every array,
  // including outputs, KernelExecutionService.cs:409-443); device buffers pass through.
  struct CopyBack {
    std::shared_ptr<IUnifiedMemoryBuffer> Buffer;
    HostArray Host;
  };
  std::vector<std::shared_ptr<IUnifiedMemoryBuffer>> owned;
  std::vector<CopyBack> copyBacks;
  KernelArguments kargs;
  std::vector<IUnifiedMemoryBuffer*> bufferArgs;
  for (size_t i = 0; i < args.size(); ++i) {
    const KernelParameterInfo* p = i < reg.Parameters.size() ? &reg.Parameters[i] : nullptr;
    if (auto* h = std::get_if<HostArray>(&args[i])) {
      auto buf = accelerator.Memory().AllocateRaw(h->Length, h->Type);
      buf->CopyFromHost(h->Data, h->Length * ElementSize(h->Type));
      kargs.AddBuffer(buf.get());
      bufferArgs.push_back(buf.get());
      if (p && p->IsBuffer && !p->IsReadOnly) copyBacks.push_back({buf, *h});
      owned.push_back(std::move(buf));
    } else if (auto* b = std::get_if<IUnifiedMemoryBuffer*>(&args[i])) {
      kargs.AddBuffer(*b);
      bufferArgs.push_back(*b);
    } else {
      std::visit(
          [&](auto v) {
            using V = decltype(v);
            if constexpr (!std::is_same_v<V, HostArray> && !std::is_same_v<V, IUnifiedMemoryBuffer*>) kargs.AddScalar(v);
          },
          args[i]);
    }
  }

  // An elementwise kernel indexes every buffer with the work-item index, so a buffer shorter than
  // the work size would be read or written past its end: the CPU invoker throws
  // IndexOutOfRangeException at the first such index; here the launch is refused instead.
  if (reg.HipNeedsLength || reg.HipBuiltin != HipOp::None)
    for (IUnifiedMemoryBuffer* b : bufferArgs)
      if (b->Length() < totalWork)
        throw IndexOutOfRangeException("Index was outside the bounds of the array: kernel '" + reg.Name +
                                       "' runs " + std::to_string(totalWork) + " work items but a buffer argument holds " +
                                       std::to_string(b->Length()) + " elements.");

  auto* hip = dynamic_cast<Backends::Hip::HipAccelerator*>(&accelerator);
  if (reg.HipBuiltin == HipOp::VectorAddF32 && hip && bufferArgs.size() == 3) {
    // Tuned library entry point (16-byte vector loads) for the registry's VectorAdd.
    Backends::Hip::Check(dc_hip_vector_add_f32(hip->Context(), static_cast<const float*>(bufferArgs[0]->DevicePointer()),
                                               static_cast<const float*>(bufferArgs[1]->DevicePointer()),
                                               static_cast<float*>(bufferArgs[2]->DevicePointer()),
                                               (int64_t)totalWork),
                         "dc_hip_vector_add_f32");
  } else {
    auto compiled = GetCompiled(reg, accelerator);
    if (reg.HipNeedsLength) kargs.AddScalar((uint32_t)totalWork);  // the implicit __length (:312-315)
    kargs.LaunchConfiguration = DeriveLaunch(reg, args, totalWork);
    compiled->ExecuteAsync(kargs).get();
  }
  accelerator.SynchronizeAsync().get();

  std::vector<float> first;
  bool have_first = false;
  for (auto& cb : copyBacks) {
    cb.Buffer->CopyToHost(cb.Host.Data, cb.Host.Length * ElementSize(cb.Host.Type));
    if (!have_first && cb.Host.Type == ElementType::Float32) {
      const float* f = static_cast<const float*>(cb.Host.Data);
      first.assign(f, f + cb.Host.Length);
      have_first = true;
    }
  }
  return first;
}

std::future<void> KernelExecutionService::ExecuteWithBuffersAsync(const std::string& kernelName,
                                                                  std::vector<IUnifiedMemoryBuffer*> buffers,
                                                                  std::vector<ScalarValue> scalarArgs) {
  EnsureInitialized();
  auto reg = TryResolveKernel(kernelName);
  if (!reg) throw ArgumentException("Kernel '" + kernelName + "' is not registered.");
  auto acc = GetOptimalAcceleratorAsync(kernelName);
  if (!acc) throw InvalidOperationException("no accelerator supports kernel '" + kernelName + "'");
  std::vector<KernelArg> args;
  for (auto* b : buffers) args.push_back(b);
  for (auto& s : scalarArgs) std::visit([&](auto v) { args.push_back(v); }, s);
  if (!ValidateKernelArgsAsync(kernelName, args)) throw ArgumentException("buffer/scalar arguments do not match the kernel");
  ExecuteOn(*reg, *acc, args);
  std::promise<void> p;
  p.set_value();
  return p.get_future();
}

}  // namespace DotCompute

// Runtime.cpp — registry, discovery, DI and the orchestrator for the HIP backend.
#include "DotCompute/Runtime.hpp"

#include <algorithm>
#include <cctype>
#include <climits>
#include <cstring>

namespace DotCompute {

namespace {
std::string Upper(std::string s) {
  std::transform(s.begin(), s.end(), s.begin(), [](unsigned char c) { return (char)std::toupper(c); });
  return s;
}
bool EqualsIgnoreCase(const std::string& a, const std::string& b) { return Upper(a) == Upper(b); }
}  // namespace

// ---- registry helpers ----------------------------------------------------------------------------

std::vector<std::string> BackendNames(int32_t flags) {
  std::vector<std::string> out;
  const std::pair<KernelBackends, const char*> names[] = {{KernelBackends::CPU, "CPU"}, {KernelBackends::CUDA, "CUDA"},
                                                          {KernelBackends::Metal, "Metal"}, {KernelBackends::OpenCL, "OpenCL"},
                                                          {KernelBackends::HIP, "HIP"}};
  for (const auto& [f, n] : names)
    if (flags & (int32_t)f) out.push_back(n);
  return out;
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
  if (initialized_.load(std::memory_order_acquire)) return;
  std::lock_guard<std::mutex> lock(mu_);
  if (initialized_.load(std::memory_order_relaxed)) return;
  runtime_->Initialize();
  // GeneratedKernelDiscoveryService.DiscoverAndRegisterKernelsAsync: the generated registry.
  for (const auto& k : Generated::KernelRegistry::GetAllKernels()) {
    auto rec = std::make_shared<const KernelRegistrationInfo>(k);
    registry_[k.FullName] = rec;
    registry_.emplace(k.Name, rec);
  }
  initialized_.store(true, std::memory_order_release);
}

void KernelExecutionService::RegisterKernels(const std::vector<KernelRegistrationInfo>& kernels) {
  EnsureInitialized();
  std::lock_guard<std::mutex> lock(mu_);
  for (const auto& k : kernels) {
    auto rec = std::make_shared<const KernelRegistrationInfo>(k);
    registry_[k.FullName] = rec;
    registry_[k.Name] = rec;  // short-name index (KernelExecutionService.cs:170-193)
  }
  // Cached choices belong to replaced records; a freed record's address may be reused.
  optimal_.clear();
  cache_.clear();
}

KernelExecutionService::Registration KernelExecutionService::Resolve(const std::string& name) const {
  std::lock_guard<std::mutex> lock(mu_);
  auto it = registry_.find(name);
  return it == registry_.end() ? nullptr : it->second;
}

std::optional<KernelRegistrationInfo> KernelExecutionService::TryResolveKernel(const std::string& name) const {
  Registration r = Resolve(name);
  if (!r) return std::nullopt;
  return *r;
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

bool KernelExecutionService::ArgumentsMatch(const KernelRegistrationInfo& reg, const std::vector<KernelArg>& args) {
  if (args.size() < reg.Parameters.size()) return false;
  for (size_t i = 0; i < reg.Parameters.size(); ++i) {
    const auto& p = reg.Parameters[i];
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

bool KernelExecutionService::ValidateKernelArgsAsync(const std::string& kernelName, const std::vector<KernelArg>& args) {
  EnsureInitialized();
  Registration reg = Resolve(kernelName);
  return reg && ArgumentsMatch(*reg, args);
}

std::vector<std::shared_ptr<IAccelerator>> KernelExecutionService::SupportedOn(const KernelRegistrationInfo& reg) const {
  std::vector<std::shared_ptr<IAccelerator>> out;
  for (const auto& acc : runtime_->GetAccelerators()) {
    const std::string backend = MapDeviceTypeToBackend(acc->Info().DeviceType);
    bool ok = std::any_of(reg.SupportedBackends.begin(), reg.SupportedBackends.end(),
                          [&](const std::string& b) { return EqualsIgnoreCase(b, backend); });
    // A registry kernel with a HIP entry point runs on HIP whether or not [Kernel(Backends)] names
    // HIP, as ExecuteAsync(name, "CUDA", ...) runs a CPU-only [Kernel] on CUDA (:230-246).
    if (backend == "HIP" && !reg.HipEntryPoint.empty()) ok = true;
    if (ok) out.push_back(acc);
  }
  return out;
}

std::vector<std::shared_ptr<IAccelerator>> KernelExecutionService::GetSupportedAcceleratorsAsync(const std::string& kernelName) {
  EnsureInitialized();
  Registration reg = Resolve(kernelName);
  if (!reg) return {};
  return SupportedOn(*reg);
}

// The accelerator of the best backend priority among those that support the kernel, chosen once
// per registration record (the runtime's accelerators are fixed once it is initialised).
std::shared_ptr<IAccelerator> KernelExecutionService::OptimalFor(const Registration& reg) {
  {
    std::lock_guard<std::mutex> lock(mu_);
    auto it = optimal_.find(reg.get());
    if (it != optimal_.end()) return it->second;
  }
  auto supported = SupportedOn(*reg);
  std::shared_ptr<IAccelerator> best;
  if (!supported.empty())
    best = *std::min_element(supported.begin(), supported.end(), [](const auto& a, const auto& b) {
      return GetBackendPriority(a->Info().DeviceType) < GetBackendPriority(b->Info().DeviceType);
    });
  std::lock_guard<std::mutex> lock(mu_);
  auto cur = registry_.find(reg->FullName);
  if (best && cur != registry_.end() && cur->second == reg) optimal_[reg.get()] = best;  // still published
  return best;
}

std::shared_ptr<IAccelerator> KernelExecutionService::GetOptimalAcceleratorAsync(const std::string& kernelName) {
  EnsureInitialized();
  Registration reg = Resolve(kernelName);
  if (!reg) return nullptr;
  return OptimalFor(reg);
}

std::future<std::vector<float>> KernelExecutionService::ExecuteAsync(const std::string& kernelName,
                                                                     std::vector<KernelArg> args) {
  EnsureInitialized();
  Registration reg = Resolve(kernelName);
  if (!reg)
    throw ArgumentException("Kernel '" + kernelName + "' is not registered. Ensure the kernel's registry is "
                            "discovered, pass the fully-qualified or short name, or register it via RegisterKernels().");
  auto acc = OptimalFor(reg);
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
  Registration reg = Resolve(kernelName);
  if (!reg)
    throw ArgumentException("Kernel '" + kernelName + "' is not registered. Add the kernel via RegisterKernels() "
                            "before executing, or check for typos.");
  if (!ArgumentsMatch(*reg, args))
    throw ArgumentException("Kernel argument validation failed for kernel '" + kernelName + "' (received " +
                            std::to_string(args.size()) + " arguments). Verify argument count, types, and ordering.");
  std::vector<float> result = ExecuteOn(*reg, accelerator, args);
  std::promise<std::vector<float>> p;
  p.set_value(std::move(result));
  return p.get_future();
}

std::shared_ptr<ICompiledKernel> KernelExecutionService::GetCompiled(const KernelRegistrationInfo& reg,
                                                                     IAccelerator& accelerator) {
  const auto key = std::make_pair(static_cast<const IAccelerator*>(&accelerator), &reg);
  {
    std::lock_guard<std::mutex> lock(mu_);
    auto it = cache_.find(key);
    if (it != cache_.end()) return it->second;
  }
  if (reg.HipEntryPoint.empty())
    throw NotSupportedException("Kernel '" + reg.Name + "' has no HIP translation for gfx950" +
                                (reg.HipDiagnostic.empty() ? std::string(".") : ": " + reg.HipDiagnostic));
  KernelDefinition def;
  def.Name = reg.Name;
  def.EntryPoint = reg.HipEntryPoint;
  def.Language = KernelLanguage::HIP;
  auto compiled = accelerator.CompileKernelAsync(def).get();
  std::lock_guard<std::mutex> lock(mu_);
  auto cur = registry_.find(reg.FullName);
  if (cur != registry_.end() && cur->second.get() == &reg) cache_[key] = compiled;  // a published record only
  return compiled;
}

void KernelExecutionService::PrecompileKernelAsync(const std::string& kernelName, IAccelerator* accelerator) {
  EnsureInitialized();
  Registration reg = Resolve(kernelName);
  if (!reg) throw ArgumentException("Kernel '" + kernelName + "' is not registered.");
  std::shared_ptr<IAccelerator> acc;
  if (!accelerator) {
    acc = OptimalFor(reg);
    if (!acc) throw InvalidOperationException("no accelerator supports kernel '" + kernelName + "'");
    accelerator = acc.get();
  }
  if (MapDeviceTypeToBackend(accelerator->Info().DeviceType) == "HIP" && !reg->HipEntryPoint.empty())
    GetCompiled(*reg, *accelerator);
}

namespace {
// The first writable float array, copied back (ExtractHostResult, KernelExecutionService.cs:475-501).
struct CopyBack {
  std::shared_ptr<IUnifiedMemoryBuffer> Buffer;
  HostArray Host;
};
std::vector<float> FirstFloatResult(const std::vector<CopyBack>& copyBacks) {
  for (const auto& cb : copyBacks)
    if (cb.Host.Type == ElementType::Float32) {
      const float* f = static_cast<const float*>(cb.Host.Data);
      return std::vector<float>(f, f + cb.Host.Length);
    }
  return {};
}

// A scalar argument converted to the parameter's declared type (the C# invoker unboxes
// `(T)args[i]`). Small types travel in a 32-bit slot; the kernel reads its low bytes.
ScalarValue ToParameterType(const KernelArg& a, ElementType t) {
  double d = 0;
  int64_t i = 0;
  uint64_t u = 0;
  bool is_float = false, is_unsigned = false;
  std::visit(
      [&](auto v) {
        using V = decltype(v);
        if constexpr (std::is_same_v<V, float> || std::is_same_v<V, double>) {
          d = (double)v;
          is_float = true;
        } else if constexpr (std::is_same_v<V, uint64_t> || std::is_same_v<V, uint32_t>) {
          u = (uint64_t)v;
          is_unsigned = true;
        } else if constexpr (std::is_integral_v<V>) {
          i = (int64_t)v;
        }
      },
      a);
  if (is_float && t != ElementType::Float32 && t != ElementType::Float64)
    throw ArgumentException("a floating-point argument was passed for an integer parameter");
  const int64_t iv = is_unsigned ? (int64_t)u : i;
  switch (t) {
    case ElementType::Float32: return is_float ? (float)d : is_unsigned ? (float)u : (float)i;
    case ElementType::Float64: return is_float ? d : is_unsigned ? (double)u : (double)i;
    case ElementType::Int64: return iv;
    case ElementType::UInt64: return is_unsigned ? u : (uint64_t)i;
    case ElementType::UInt32: return (uint32_t)iv;
    default: return (int32_t)iv;  // int, short, ushort, byte, sbyte, bool
  }
}
}  // namespace

std::vector<float> KernelExecutionService::ExecuteOn(const KernelRegistrationInfo& reg, IAccelerator& accelerator,
                                                     std::vector<KernelArg>& args) {
  const std::string backend = MapDeviceTypeToBackend(accelerator.Info().DeviceType);
  if (backend != "HIP")
    throw NotSupportedException("this build drives HIP accelerators only (got device type '" +
                                accelerator.Info().DeviceType + "')");
  auto* hip = dynamic_cast<Backends::Hip::HipAccelerator*>(&accelerator);
  if (reg.HipAbi == HipKernelAbi::Generated && hip) return ExecuteGenerated(reg, *hip, args);
  const size_t totalWork = DeriveWorkSize(reg, args);
  auto compiled = GetCompiled(reg, accelerator);  // throws NotSupportedException without a HIP slot

  // Plain entry points (kernels registered by hand against a code object): the reference's
  // marshalling — a device buffer per host array, every array copied in, including outputs
  // (KernelExecutionService.cs:409-443); device buffers pass through.
  std::vector<std::shared_ptr<IUnifiedMemoryBuffer>> owned;
  std::vector<CopyBack> copyBacks;
  KernelArguments kargs;
  std::vector<IUnifiedMemoryBuffer*> bufferArgs;
  for (size_t i = 0; i < args.size(); ++i) {
    const KernelParameterInfo* p = i < reg.Parameters.size() ? &reg.Parameters[i] : nullptr;
    if (auto* h = std::get_if<HostArray>(&args[i])) {
      auto buf = accelerator.Memory().AllocateRaw(h->Length, h->Type);
      buf->EnqueueCopyFromHost(h->Data, h->Length * ElementSize(h->Type));
      kargs.AddBuffer(buf.get());
      bufferArgs.push_back(buf.get());
      if (p && p->IsBuffer && !p->IsReadOnly) copyBacks.push_back({buf, *h});
      owned.push_back(std::move(buf));
    } else if (auto* b = std::get_if<IUnifiedMemoryBuffer*>(&args[i])) {
      kargs.AddBuffer(*b);
      bufferArgs.push_back(*b);
    } else {
      kargs.AddScalar(ToParameterType(args[i], p ? p->Type : ElementType::Int32));
    }
  }
  // An elementwise kernel indexes every buffer with the work-item index: a buffer shorter than
  // the work size would be read or written past its end (the CPU invoker throws
  // IndexOutOfRangeException at the first such index); the launch is refused instead.
  if (reg.HipNeedsLength)
    for (IUnifiedMemoryBuffer* b : bufferArgs)
      if (b->Length() < totalWork)
        throw IndexOutOfRangeException("Index was outside the bounds of the array: kernel '" + reg.Name +
                                       "' runs " + std::to_string(totalWork) + " work items but a buffer argument holds " +
                                       std::to_string(b->Length()) + " elements.");
  if (reg.HipNeedsLength) kargs.AddScalar((uint32_t)totalWork);  // the implicit __length (:312-315)
  kargs.LaunchConfiguration = DeriveLaunch(reg, args, totalWork);
  compiled->ExecuteAsync(kargs).get();
  for (auto& cb : copyBacks) cb.Buffer->EnqueueCopyToHost(cb.Host.Data, cb.Host.Length * ElementSize(cb.Host.Type));
  accelerator.SynchronizeAsync().get();
  return FirstFloatResult(copyBacks);
}

std::vector<float> KernelExecutionService::ExecuteGenerated(const KernelRegistrationInfo& reg,
                                                            Backends::Hip::HipAccelerator& accelerator,
                                                            std::vector<KernelArg>& args) {
  const size_t totalWork = DeriveWorkSize(reg, args);
  if (totalWork > (size_t)INT32_MAX)
    throw ArgumentException("kernel '" + reg.Name + "': more than 2^31 - 1 work items (C# spans hold int lengths)");
  // The coordinates of a 2-D / 3-D work item divide by the trailing integer extents, as the CPU
  // invoker does (KernelExecutionMetadataEmitter.cs:203-245): a zero extent throws there.
  std::vector<int64_t> ints;
  for (size_t i = 0; i < reg.Parameters.size(); ++i) {
    const auto& p = reg.Parameters[i];
    if (!p.IsBuffer && p.Type != ElementType::Float32 && p.Type != ElementType::Float64 && p.Type != ElementType::Bool)
      std::visit([&](auto v) {
        using V = decltype(v);
        if constexpr (std::is_arithmetic_v<V>) ints.push_back((int64_t)v);
      }, args[i]);
  }
  if (totalWork > 0 && reg.Dimensions >= 2 && ints.size() >= 2) {
    const int32_t x = (int32_t)ints[ints.size() - 1], y = (int32_t)ints[ints.size() - 2];
    const bool three = reg.Dimensions >= 3 && ints.size() >= 3;
    if (x == 0 || (three && y == 0) || (three && (int32_t)((uint32_t)x * (uint32_t)y) == 0))
      throw DivideByZeroException("Attempted to divide by zero. (kernel '" + reg.Name + "': a zero extent)");
  }

  // The accelerator's error words serve one generated launch at a time (see GeneratedLaunchMutex).
  std::lock_guard<std::mutex> serial(accelerator.GeneratedLaunchMutex());
  dc_gen_launch launch{};
  launch.work = (int64_t)totalWork;
  launch.epoch = accelerator.NextLaunchEpoch();
  launch.error = accelerator.GeneratedErrorWordsDevice();
  std::vector<std::shared_ptr<IUnifiedMemoryBuffer>> owned;
  std::vector<CopyBack> copyBacks;
  KernelArguments kargs;
  int nbuf = 0;
  for (size_t i = 0; i < reg.Parameters.size(); ++i) {
    const KernelParameterInfo& p = reg.Parameters[i];
    if (p.IsBuffer) {
      if (nbuf >= DC_GEN_MAX_BUFFERS) throw NotSupportedException("more than 16 buffer parameters");
      IUnifiedMemoryBuffer* dev = nullptr;
      if (auto* h = std::get_if<HostArray>(&args[i])) {
        // Every array goes in (as the reference copies them, KernelExecutionService.cs:755-763),
        // except one the body overwrites in full without reading it: the pool recycles device
        // blocks without clearing them, so an element the kernel leaves alone must arrive from the
        // host. Only what the body writes comes back. The memory comes from the accelerator's pool
        // (no device allocation once the sizes have been seen).
        auto buf = accelerator.Memory().AllocateRaw(h->Length, h->Type);
        if (p.IsRead || !p.IsCovered) buf->EnqueueCopyFromHost(h->Data, h->Length * ElementSize(h->Type));
        if (p.IsWritten) copyBacks.push_back({buf, *h});
        dev = buf.get();
        owned.push_back(std::move(buf));
      } else {
        dev = std::get<IUnifiedMemoryBuffer*>(args[i]);
      }
      launch.len[nbuf++] = (int64_t)dev->Length();
      kargs.AddBuffer(dev);
    } else {
      kargs.AddScalar(ToParameterType(args[i], p.Type));
    }
  }
  RawArgument block;
  block.Bytes.resize(sizeof(launch));
  std::memcpy(block.Bytes.data(), &launch, sizeof(launch));
  kargs.AddScalar(std::move(block));
  kargs.LaunchConfiguration.BlockSize = {DC_GEN_BLOCK, 1, 1};
  kargs.LaunchConfiguration.GridSize = {(uint32_t)((totalWork + DC_GEN_BLOCK - 1) / DC_GEN_BLOCK), 1, 1};
  if (totalWork > 0) GetCompiled(reg, accelerator)->ExecuteAsync(kargs).get();
  for (auto& cb : copyBacks) cb.Buffer->EnqueueCopyToHost(cb.Host.Data, cb.Host.Length * ElementSize(cb.Host.Type));
  accelerator.Synchronize();
  accelerator.ThrowIfGeneratedKernelFailed(launch.epoch, reg.Name);
  return FirstFloatResult(copyBacks);
}

std::future<void> KernelExecutionService::ExecuteWithBuffersAsync(const std::string& kernelName,
                                                                  std::vector<IUnifiedMemoryBuffer*> buffers,
                                                                  std::vector<ScalarValue> scalarArgs) {
  EnsureInitialized();
  Registration reg = Resolve(kernelName);
  if (!reg) throw ArgumentException("Kernel '" + kernelName + "' is not registered.");
  auto acc = OptimalFor(reg);
  if (!acc) throw InvalidOperationException("no accelerator supports kernel '" + kernelName + "'");
  std::vector<KernelArg> args;
  args.reserve(buffers.size() + scalarArgs.size());
  for (auto* b : buffers) args.push_back(b);
  for (auto& s : scalarArgs)
    std::visit(
        [&](const auto& v) {
          if constexpr (std::is_same_v<std::decay_t<decltype(v)>, RawArgument>)
            throw ArgumentException("raw struct arguments are not kernel parameters");
          else
            args.push_back(v);
        },
        s);
  if (!ArgumentsMatch(*reg, args)) throw ArgumentException("buffer/scalar arguments do not match the kernel");
  ExecuteOn(*reg, *acc, args);
  std::promise<void> p;
  p.set_value();
  return p.get_future();
}

}  // namespace DotCompute

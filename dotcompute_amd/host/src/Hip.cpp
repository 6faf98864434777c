// Hip.cpp — HipAccelerator, HipMemoryManager, HipBuffer, HipCompiledKernel.
#include "DotCompute/Backends/Hip.hpp"

#include <cstring>

namespace DotCompute {

const char* ToString(AcceleratorType t) {
  switch (t) {
    case AcceleratorType::Auto: return "Auto";
    case AcceleratorType::None: return "None";
    case AcceleratorType::CPU: return "CPU";
    case AcceleratorType::CUDA: return "CUDA";
    case AcceleratorType::ROCm: return "ROCm";
    case AcceleratorType::OneAPI: return "OneAPI";
    case AcceleratorType::Metal: return "Metal";
    case AcceleratorType::OpenCL: return "OpenCL";
    case AcceleratorType::DirectML: return "DirectML";
    case AcceleratorType::DirectCompute: return "DirectCompute";
  }
  return "Unknown";
}

size_t ElementSize(ElementType t) {
  switch (t) {
    case ElementType::Float32:
    case ElementType::Int32:
    case ElementType::UInt32: return 4;
    case ElementType::Int64:
    case ElementType::Float64: return 8;
    case ElementType::UInt16: return 2;
  }
  return 1;
}

}  // namespace DotCompute

namespace DotCompute::Backends::Hip {

void Check(int32_t status, const char* what) {
  if (status == DC_OK) return;
  std::string msg = std::string(what) + ": " + dc_hip_error_string(status);
  switch (status) {
    case DC_ERR_INVALID_ARGUMENT:
    case DC_ERR_DIMENSION: throw ArgumentException(msg);
    case DC_ERR_UNSUPPORTED: throw NotSupportedException(msg);
    case DC_ERR_OVERFLOW: throw OverflowException(msg);
    default: throw HipException(status, msg);
  }
}

// ---- HipAllocation -----------------------------------------------------------------------------

HipAllocation::HipAllocation(std::shared_ptr<dc_hip_ctx> ctx, size_t bytes) : ctx_(std::move(ctx)), bytes_(bytes) {
  if (bytes_ > 0) Check(dc_hip_malloc(ctx_.get(), bytes_, &ptr_), "dc_hip_malloc");
}

HipAllocation::~HipAllocation() {
  if (ptr_) dc_hip_free(ctx_.get(), ptr_);
}

void HipAllocation::Dispose() {
  if (ptr_) Check(dc_hip_free(ctx_.get(), ptr_), "dc_hip_free");
  ptr_ = nullptr;
  disposed_ = true;
}

void HipAllocation::CopyFromHost(const void* src, size_t bytes, size_t offset_bytes) {
  if (disposed_) throw InvalidOperationException("buffer has been disposed");
  if (offset_bytes + bytes > bytes_) throw ArgumentException("copy exceeds the buffer size");
  if (bytes == 0) return;
  if (!src) throw ArgumentNullException("source");
  Check(dc_hip_memcpy_h2d_async(ctx_.get(), static_cast<char*>(ptr_) + offset_bytes, src, bytes), "h2d");
  Check(dc_hip_synchronize(ctx_.get()), "dc_hip_synchronize");
}

void HipAllocation::CopyToHost(void* dst, size_t bytes, size_t offset_bytes) const {
  if (disposed_) throw InvalidOperationException("buffer has been disposed");
  if (offset_bytes + bytes > bytes_) throw ArgumentException("copy exceeds the buffer size");
  if (bytes == 0) return;
  if (!dst) throw ArgumentNullException("destination");
  Check(dc_hip_memcpy_d2h_async(ctx_.get(), dst, static_cast<const char*>(ptr_) + offset_bytes, bytes), "d2h");
  Check(dc_hip_synchronize(ctx_.get()), "dc_hip_synchronize");
}

// ---- HipMemoryManager -------------------------------------------------------------------------

std::shared_ptr<IUnifiedMemoryBuffer> HipMemoryManager::AllocateRaw(size_t count, ElementType type) {
  switch (type) {
    case ElementType::Float32: return std::make_shared<HipBuffer<float>>(ctx_, count);
    case ElementType::Int32: return std::make_shared<HipBuffer<int32_t>>(ctx_, count);
    case ElementType::UInt32: return std::make_shared<HipBuffer<uint32_t>>(ctx_, count);
    case ElementType::Int64: return std::make_shared<HipBuffer<int64_t>>(ctx_, count);
    case ElementType::Float64: return std::make_shared<HipBuffer<double>>(ctx_, count);
    case ElementType::UInt16: return std::make_shared<HipBuffer<uint16_t>>(ctx_, count);
  }
  throw ArgumentException("unknown element type");
}

size_t HipMemoryManager::TotalAvailableMemory() const {
  size_t free_b = 0, total_b = 0;
  Check(dc_hip_mem_info(ctx_.get(), &free_b, &total_b), "dc_hip_mem_info");
  return free_b;
}

// ---- HipCompiledKernel ------------------------------------------------------------------------

HipCompiledKernel::HipCompiledKernel(std::string name, std::shared_ptr<dc_hip_ctx> ctx,
                                     std::shared_ptr<dc_hip_module> module, void* function)
    : name_(std::move(name)), ctx_(std::move(ctx)), module_(std::move(module)), function_(function) {}

std::future<void> HipCompiledKernel::ExecuteAsync(const KernelArguments& arguments) {
  // One storage slot per argument, pointers to the slots in parameter order (as
  // CudaKernelLauncher pins a void*[] of argument slots, CudaKernelLauncher.cs:226-313).
  const size_t n = arguments.Buffers.size() + arguments.ScalarArguments.size();
  std::vector<uint64_t> storage(n, 0);
  std::vector<void*> slots(n, nullptr);
  size_t i = 0;
  for (IUnifiedMemoryBuffer* b : arguments.Buffers) {
    if (!b) throw ArgumentNullException("null buffer argument");
    void* p = b->DevicePointer();
    std::memcpy(&storage[i], &p, sizeof(p));
    slots[i] = &storage[i];
    ++i;
  }
  for (const ScalarValue& s : arguments.ScalarArguments) {
    std::visit([&](auto v) { std::memcpy(&storage[i], &v, sizeof(v)); }, s);
    slots[i] = &storage[i];
    ++i;
  }
  const KernelLaunchConfiguration& lc = arguments.LaunchConfiguration;
  Check(dc_hip_launch_kernel(ctx_.get(), function_, lc.GridSize.X, lc.GridSize.Y, lc.GridSize.Z, lc.BlockSize.X,
                             lc.BlockSize.Y, lc.BlockSize.Z, lc.SharedMemoryBytes, slots.data()),
        "dc_hip_launch_kernel");
  std::promise<void> p;
  p.set_value();
  return p.get_future();
}

// ---- HipAccelerator ---------------------------------------------------------------------------

namespace {
std::shared_ptr<dc_hip_ctx> MakeContext(int32_t device) {
  dc_hip_ctx* raw = nullptr;
  Check(dc_hip_ctx_create(device, &raw), "dc_hip_ctx_create");
  return std::shared_ptr<dc_hip_ctx>(raw, [](dc_hip_ctx* c) { dc_hip_ctx_destroy(c); });
}
}  // namespace

HipAccelerator::HipAccelerator(const HipBackendOptions& options)
    : ctx_(MakeContext(options.DeviceId)), memory_(ctx_), options_(options) {
  dc_hip_device_info d;
  Check(dc_hip_device_info_get(options.DeviceId, &d), "dc_hip_device_info_get");
  info_.Id = "HIP:" + std::to_string(options.DeviceId);
  info_.Name = d.name;
  info_.DeviceType = "HIP";
  info_.Vendor = "AMD";
  info_.Architecture = d.gcn_arch_name;
  info_.ComputeUnits = d.compute_units;
  info_.GlobalMemorySize = d.total_global_mem;
  info_.LocalMemorySize = d.lds_per_block;
  info_.MaxThreadsPerBlock = d.max_threads_per_block;
  info_.ClockRateKHz = d.clock_khz;
  info_.WarpSize = d.wave_size;
}

int32_t HipAccelerator::DeviceCount() {
  int32_t n = 0;
  if (dc_hip_device_count(&n) != DC_OK) return 0;
  return n;
}

void HipAccelerator::Synchronize() { Check(dc_hip_synchronize(ctx_.get()), "dc_hip_synchronize"); }

std::future<void> HipAccelerator::SynchronizeAsync() {
  Synchronize();
  std::promise<void> p;
  p.set_value();
  return p.get_future();
}

std::future<std::shared_ptr<ICompiledKernel>> HipAccelerator::CompileKernelAsync(const KernelDefinition& definition,
                                                                                 const CompilationOptions&) {
  // "Compilation" of a HIP kernel is a lookup: every kernel is prebuilt offline for gfx950.
  if (definition.Language != KernelLanguage::HIP && definition.Language != KernelLanguage::Binary)
    throw NotSupportedException("the HIP backend runs prebuilt gfx950 kernels; source language " +
                                std::to_string((int)definition.Language) + " is not compiled at run time");
  std::string path = !definition.Code.empty() ? definition.Code
                     : !options_.KernelObjectPath.empty() ? options_.KernelObjectPath
                                                          : std::string(dc_hip_default_module_path());
  if (path.empty()) throw InvalidOperationException("no gfx950 code object found next to libdotcompute_hip.so");
  std::shared_ptr<dc_hip_module> module;
  {
    std::lock_guard<std::mutex> lock(module_mu_);
    auto it = modules_.find(path);
    if (it == modules_.end()) {
      dc_hip_module* m = nullptr;
      Check(dc_hip_module_load(ctx_.get(), path.c_str(), &m), "dc_hip_module_load");
      module = std::shared_ptr<dc_hip_module>(m, [](dc_hip_module* mm) { dc_hip_module_unload(mm); });
      modules_[path] = module;
    } else {
      module = it->second;
    }
  }
  const std::string entry = definition.EntryPoint.empty() ? definition.Name : definition.EntryPoint;
  void* fn = nullptr;
  int32_t st = dc_hip_module_get_function(module.get(), entry.c_str(), &fn);
  if (st == DC_ERR_NOT_FOUND)
    throw ArgumentException("kernel entry point '" + entry + "' is not in " + path);
  Check(st, "dc_hip_module_get_function");
  std::promise<std::shared_ptr<ICompiledKernel>> p;
  p.set_value(std::make_shared<HipCompiledKernel>(definition.Name, ctx_, module, fn));
  return p.get_future();
}

std::shared_ptr<HipAccelerator> TryCreateAccelerator(const HipBackendOptions& options) {
  try {
    if (HipAccelerator::DeviceCount() <= options.DeviceId) return nullptr;
    return std::make_shared<HipAccelerator>(options);
  } catch (const std::exception&) {
    return nullptr;  // no usable gfx950 device: discovery skips this backend
  }
}

}  // namespace DotCompute::Backends::Hip

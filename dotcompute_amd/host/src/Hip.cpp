// Hip.cpp — HipAccelerator, HipMemoryManager, HipBuffer, HipCompiledKernel.
#include "DotCompute/Backends/Hip.hpp"

#include <algorithm>
#include <cstring>
#include <type_traits>

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
    case ElementType::UInt64:
    case ElementType::Float64: return 8;
    case ElementType::UInt16:
    case ElementType::Int16: return 2;
    case ElementType::UInt8:
    case ElementType::Int8:
    case ElementType::Bool: return 1;
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

// ---- DevicePool --------------------------------------------------------------------------------

size_t DevicePool::RoundedSize(size_t bytes) {
  // 256 B granules below 64 KiB, 4 KiB granules above: the same request always maps to one class.
  const size_t g = bytes < (64u << 10) ? 256 : 4096;
  return (std::max<size_t>(bytes, 1) + g - 1) / g * g;
}

void* DevicePool::Acquire(size_t bytes) {
  const size_t r = RoundedSize(bytes);
  {
    std::lock_guard<std::mutex> lock(mu_);
    auto it = free_.find(r);
    if (it != free_.end() && !it->second.empty()) {
      void* p = it->second.back();
      it->second.pop_back();
      cached_ -= r;
      ++hits_;
      return p;
    }
  }
  void* p = nullptr;
  int32_t st = dc_hip_malloc(ctx_.get(), r, &p);
  if (st != DC_OK) {
    // Out of memory with blocks parked here: return them to the device and try once more.
    std::map<size_t, std::vector<void*>> parked;
    {
      std::lock_guard<std::mutex> lock(mu_);
      parked.swap(free_);
      cached_ = 0;
    }
    for (auto& [sz, v] : parked)
      for (void* q : v) dc_hip_free(ctx_.get(), q);
    Check(dc_hip_malloc(ctx_.get(), r, &p), "dc_hip_malloc");
  }
  return p;
}

void DevicePool::Release(void* ptr, size_t bytes) {
  if (!ptr) return;
  const size_t r = RoundedSize(bytes);
  {
    std::lock_guard<std::mutex> lock(mu_);
    if (cached_ + r <= kMaxCachedBytes) {
      free_[r].push_back(ptr);
      cached_ += r;
      return;
    }
  }
  dc_hip_free(ctx_.get(), ptr);
}

size_t DevicePool::CachedBytes() const {
  std::lock_guard<std::mutex> lock(mu_);
  return cached_;
}

DevicePool::~DevicePool() {
  for (auto& [sz, v] : free_)
    for (void* q : v) dc_hip_free(ctx_.get(), q);
}

// ---- HipAllocation -----------------------------------------------------------------------------

HipAllocation::HipAllocation(std::shared_ptr<dc_hip_ctx> ctx, std::shared_ptr<DevicePool> pool, size_t bytes)
    : ctx_(std::move(ctx)), pool_(std::move(pool)), bytes_(bytes) {
  if (bytes_ > 0) ptr_ = pool_->Acquire(bytes_);
}

HipAllocation::~HipAllocation() {
  if (ptr_) pool_->Release(ptr_, bytes_);
}

void HipAllocation::Dispose() {
  if (ptr_) pool_->Release(ptr_, bytes_);
  ptr_ = nullptr;
  disposed_ = true;
}

void HipAllocation::CopyFromHost(const void* src, size_t bytes, size_t offset_bytes, bool wait) {
  if (disposed_) throw InvalidOperationException("buffer has been disposed");
  if (offset_bytes + bytes > bytes_) throw ArgumentException("copy exceeds the buffer size");
  if (bytes == 0) return;
  if (!src) throw ArgumentNullException("source");
  Check(dc_hip_memcpy_h2d_async(ctx_.get(), static_cast<char*>(ptr_) + offset_bytes, src, bytes), "h2d");
  if (wait) Check(dc_hip_synchronize(ctx_.get()), "dc_hip_synchronize");
}

void HipAllocation::CopyToHost(void* dst, size_t bytes, size_t offset_bytes, bool wait) const {
  if (disposed_) throw InvalidOperationException("buffer has been disposed");
  if (offset_bytes + bytes > bytes_) throw ArgumentException("copy exceeds the buffer size");
  if (bytes == 0) return;
  if (!dst) throw ArgumentNullException("destination");
  Check(dc_hip_memcpy_d2h_async(ctx_.get(), dst, static_cast<const char*>(ptr_) + offset_bytes, bytes), "d2h");
  if (wait) Check(dc_hip_synchronize(ctx_.get()), "dc_hip_synchronize");
}

// ---- HipMemoryManager -------------------------------------------------------------------------

std::shared_ptr<IUnifiedMemoryBuffer> HipMemoryManager::AllocateRaw(size_t count, ElementType type) {
  switch (type) {
    case ElementType::Float32: return std::make_shared<HipBuffer<float>>(ctx_, pool_, count);
    case ElementType::Int32: return std::make_shared<HipBuffer<int32_t>>(ctx_, pool_, count);
    case ElementType::UInt32: return std::make_shared<HipBuffer<uint32_t>>(ctx_, pool_, count);
    case ElementType::Int64: return std::make_shared<HipBuffer<int64_t>>(ctx_, pool_, count);
    case ElementType::Float64: return std::make_shared<HipBuffer<double>>(ctx_, pool_, count);
    case ElementType::UInt16: return std::make_shared<HipBuffer<uint16_t>>(ctx_, pool_, count);
    case ElementType::UInt64: return std::make_shared<HipBuffer<uint64_t>>(ctx_, pool_, count);
    case ElementType::Int16: return std::make_shared<HipBuffer<int16_t>>(ctx_, pool_, count);
    case ElementType::UInt8: return std::make_shared<HipBuffer<uint8_t>>(ctx_, pool_, count);
    case ElementType::Int8: return std::make_shared<HipBuffer<int8_t>>(ctx_, pool_, count);
    case ElementType::Bool: return std::make_shared<HipBuffer<uint8_t>>(ctx_, pool_, count);
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
  // A struct argument (RawArgument) points at its own bytes.
  const size_t n = arguments.Buffers.size() + arguments.ScalarArguments.size();
  // Slots on the stack for the usual argument counts (no allocation per launch).
  constexpr size_t kInline = 32;
  uint64_t storage_inline[kInline] = {};
  void* slots_inline[kInline] = {};
  std::vector<uint64_t> storage_heap;
  std::vector<void*> slots_heap;
  uint64_t* storage = storage_inline;
  void** slots = slots_inline;
  if (n > kInline) {
    storage_heap.assign(n, 0);
    slots_heap.assign(n, nullptr);
    storage = storage_heap.data();
    slots = slots_heap.data();
  }
  size_t i = 0;
  for (IUnifiedMemoryBuffer* b : arguments.Buffers) {
    if (!b) throw ArgumentNullException("null buffer argument");
    void* p = b->DevicePointer();
    std::memcpy(&storage[i], &p, sizeof(p));
    slots[i] = &storage[i];
    ++i;
  }
  for (const ScalarValue& s : arguments.ScalarArguments) {
    if (auto* raw = std::get_if<RawArgument>(&s)) {
      slots[i] = const_cast<uint8_t*>(raw->Bytes.data());
    } else {
      std::visit(
          [&](const auto& v) {
            if constexpr (!std::is_same_v<std::decay_t<decltype(v)>, RawArgument>) std::memcpy(&storage[i], &v, sizeof(v));
          },
          s);
      slots[i] = &storage[i];
    }
    ++i;
  }
  const KernelLaunchConfiguration& lc = arguments.LaunchConfiguration;
  Check(dc_hip_launch_kernel(ctx_.get(), function_, lc.GridSize.X, lc.GridSize.Y, lc.GridSize.Z, lc.BlockSize.X,
                             lc.BlockSize.Y, lc.BlockSize.Z, lc.SharedMemoryBytes, slots),
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
  void* h = nullptr;
  Check(dc_hip_malloc_host(ctx_.get(), 4 * sizeof(uint32_t), &h), "dc_hip_malloc_host");
  err_host_ = static_cast<uint32_t*>(h);
  std::memset(err_host_, 0, 4 * sizeof(uint32_t));
  void* dptr = nullptr;
  Check(dc_hip_host_device_pointer(ctx_.get(), h, &dptr), "dc_hip_host_device_pointer");
  err_device_ = static_cast<uint32_t*>(dptr);
}

HipAccelerator::~HipAccelerator() {
  if (err_host_) dc_hip_free_host(ctx_.get(), err_host_);
}

uint32_t HipAccelerator::NextLaunchEpoch() {
  std::lock_guard<std::mutex> lock(module_mu_);
  if (++epoch_ == 0) {  // wrapped: clear the words so no stale epoch can match
    std::memset(err_host_, 0, 4 * sizeof(uint32_t));
    epoch_ = 1;
  }
  return epoch_;
}

void HipAccelerator::ThrowIfGeneratedKernelFailed(uint32_t epoch, const std::string& kernel) const {
  auto word = [&](int k) { return __atomic_load_n(&err_host_[k], __ATOMIC_ACQUIRE); };
  if (word(DC_GEN_ERR_INDEX) == epoch)
    throw IndexOutOfRangeException("Index was outside the bounds of the array. (kernel '" + kernel + "')");
  if (word(DC_GEN_ERR_DIVIDE_BY_ZERO) == epoch)
    throw DivideByZeroException("Attempted to divide by zero. (kernel '" + kernel + "')");
  if (word(DC_GEN_ERR_OVERFLOW) == epoch)
    throw OverflowException("Arithmetic operation resulted in an overflow. (kernel '" + kernel + "')");
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

namespace {
std::mutex g_create_mu;
std::string g_create_error;
}  // namespace

std::string LastAcceleratorCreationError() {
  std::lock_guard<std::mutex> lock(g_create_mu);
  return g_create_error;
}

std::shared_ptr<HipAccelerator> TryCreateAccelerator(const HipBackendOptions& options) {
  try {
    if (HipAccelerator::DeviceCount() <= options.DeviceId) {
      std::lock_guard<std::mutex> lock(g_create_mu);
      g_create_error = "no HIP device " + std::to_string(options.DeviceId);
      return nullptr;
    }
    return std::make_shared<HipAccelerator>(options);
  } catch (const std::exception& e) {
    std::lock_guard<std::mutex> lock(g_create_mu);
    g_create_error = e.what();
    return nullptr;  // no usable gfx950 device: discovery skips this backend
  }
}

}  // namespace DotCompute::Backends::Hip

// Hip.hpp — DotCompute.Backends.HIP: the MI355X accelerator, its memory manager, compiled kernels
// and the registration entry point, all driving libdotcompute_hip.so through its C ABI.
//
// Mirrors the CUDA backend's public shape: CudaAccelerator (src/Backends/DotCompute.Backends.CUDA/
// CudaAccelerator.cs:59-232), CudaMemoryManager/CudaMemoryBuffer (Memory/CudaMemoryManager.cs:51,
// Memory/CudaMemoryBuffer.cs:22,229), CudaCompiledKernel + CudaKernelLauncher
// (Kernels/CudaCompiledKernel.cs, Kernels/CudaKernelLauncher.cs:205-349) and AddCudaBackend
// (CudaBackendPlugin.cs:311-380), which returns no accelerator instead of throwing when no
// device is present.
#pragma once

#include <map>
#include <mutex>
#include <vector>

#include "../Abstractions.hpp"
#include "dotcompute_hip.h"

namespace DotCompute::Backends::Hip {

// Throws HipException for a non-zero status of the C ABI.
void Check(int32_t status, const char* what);

class HipAccelerator;

// Device memory recycled per accelerator: a released block goes back to a free list keyed by its
// rounded size and the next allocation of that size takes it without calling dc_hip_malloc (the
// orchestrator allocates the same sizes on every call). Safe because every use of the memory is
// ordered on the context's one in-order stream: work enqueued after a release runs after the work
// that used the block before. Holds at most kMaxCachedBytes; larger surpluses are freed.
class DevicePool {
 public:
  explicit DevicePool(std::shared_ptr<dc_hip_ctx> ctx) : ctx_(std::move(ctx)) {}
  ~DevicePool();
  DevicePool(const DevicePool&) = delete;
  DevicePool& operator=(const DevicePool&) = delete;
  // Returns a block of at least `bytes` (rounded up to RoundedSize(bytes)).
  void* Acquire(size_t bytes);
  void Release(void* ptr, size_t bytes);
  static size_t RoundedSize(size_t bytes);
  size_t CachedBytes() const;
  size_t Hits() const { return hits_; }
  static constexpr size_t kMaxCachedBytes = (size_t)2 << 30;

 private:
  std::shared_ptr<dc_hip_ctx> ctx_;
  mutable std::mutex mu_;
  std::map<size_t, std::vector<void*>> free_;
  size_t cached_ = 0;
  size_t hits_ = 0;
};

// Device allocation owned by exactly one object; returned to its pool once, by Dispose() or the
// destructor.
class HipAllocation {
 public:
  HipAllocation(std::shared_ptr<dc_hip_ctx> ctx, std::shared_ptr<DevicePool> pool, size_t bytes);
  ~HipAllocation();
  HipAllocation(const HipAllocation&) = delete;
  HipAllocation& operator=(const HipAllocation&) = delete;
  void* Pointer() const { return ptr_; }
  size_t Bytes() const { return bytes_; }
  bool Disposed() const { return disposed_; }
  void CopyFromHost(const void* src, size_t bytes, size_t offset_bytes, bool wait = true);
  void CopyToHost(void* dst, size_t bytes, size_t offset_bytes, bool wait = true) const;
  void Dispose();

 private:
  std::shared_ptr<dc_hip_ctx> ctx_;
  std::shared_ptr<DevicePool> pool_;
  void* ptr_ = nullptr;
  size_t bytes_ = 0;
  bool disposed_ = false;
};

template <typename T>
class HipBuffer final : public IUnifiedMemoryBufferT<T> {
 public:
  HipBuffer(std::shared_ptr<dc_hip_ctx> ctx, std::shared_ptr<DevicePool> pool, size_t count)
      : alloc_(std::move(ctx), std::move(pool), count * sizeof(T)), count_(count) {}
  size_t SizeInBytes() const override { return alloc_.Bytes(); }
  size_t Length() const override { return count_; }
  ElementType Type() const override { return ElementTypeOf<T>::value; }
  void* DevicePointer() const override { return alloc_.Pointer(); }
  bool IsDisposed() const override { return alloc_.Disposed(); }
  void CopyFromHost(const void* src, size_t bytes, size_t offset_bytes = 0) override {
    alloc_.CopyFromHost(src, bytes, offset_bytes);
  }
  void CopyToHost(void* dst, size_t bytes, size_t offset_bytes = 0) const override {
    alloc_.CopyToHost(dst, bytes, offset_bytes);
  }
  void EnqueueCopyFromHost(const void* src, size_t bytes) override { alloc_.CopyFromHost(src, bytes, 0, false); }
  void EnqueueCopyToHost(void* dst, size_t bytes) const override { alloc_.CopyToHost(dst, bytes, 0, false); }
  void Dispose() override { alloc_.Dispose(); }

 private:
  HipAllocation alloc_;
  size_t count_;
};

class HipMemoryManager final : public IUnifiedMemoryManager {
 public:
  explicit HipMemoryManager(std::shared_ptr<dc_hip_ctx> ctx)
      : ctx_(ctx), pool_(std::make_shared<DevicePool>(std::move(ctx))) {}
  std::shared_ptr<IUnifiedMemoryBuffer> AllocateRaw(size_t count, ElementType type) override;
  size_t TotalAvailableMemory() const override;
  const DevicePool& Pool() const { return *pool_; }

 private:
  std::shared_ptr<dc_hip_ctx> ctx_;
  std::shared_ptr<DevicePool> pool_;
};

// A prebuilt gfx950 kernel resolved from a code object by entry-point name; launched with the
// arguments packed as the reference packs them (buffers then scalars, one pointer per slot).
class HipCompiledKernel final : public ICompiledKernel {
 public:
  HipCompiledKernel(std::string name, std::shared_ptr<dc_hip_ctx> ctx, std::shared_ptr<dc_hip_module> module,
                    void* function);
  const std::string& Name() const override { return name_; }
  std::future<void> ExecuteAsync(const KernelArguments& arguments) override;

 private:
  std::string name_;
  std::shared_ptr<dc_hip_ctx> ctx_;
  std::shared_ptr<dc_hip_module> module_;
  void* function_;
};

struct HipBackendOptions {
  int32_t DeviceId = 0;
  std::string KernelObjectPath;  // empty: dc_kernels_gfx950.hsaco next to libdotcompute_hip.so
};

class HipAccelerator final : public IAccelerator {
 public:
  explicit HipAccelerator(const HipBackendOptions& options = {});
  const AcceleratorInfo& Info() const override { return info_; }
  AcceleratorType Type() const override { return AcceleratorType::ROCm; }
  IUnifiedMemoryManager& Memory() override { return memory_; }
  std::future<std::shared_ptr<ICompiledKernel>> CompileKernelAsync(const KernelDefinition& definition,
                                                                   const CompilationOptions& options = {}) override;
  std::future<void> SynchronizeAsync() override;

  // Native handle for the op entry points (dc_hip_linq_*, dc_hip_gemm_*, dc_hip_spmv_*).
  dc_hip_ctx* Context() const { return ctx_.get(); }
  std::shared_ptr<dc_hip_ctx> SharedContext() const { return ctx_; }
  void Synchronize();

  // Error words of generated kernels (dc_gen_launch.error): pinned host memory the device writes
  // directly. NextLaunchEpoch() tags one launch; after it completes, ThrowIfGeneratedKernelFailed
  // raises the C# exception a word carrying that epoch stands for. The words are shared by every
  // generated launch on this accelerator, so a caller holds GeneratedLaunchMutex() from
  // NextLaunchEpoch() until ThrowIfGeneratedKernelFailed() returns: a second launch cannot then
  // overwrite a word before the first launch's caller has read it, and the words are only cleared
  // (when the epoch counter wraps) while no generated kernel runs.
  uint32_t* GeneratedErrorWordsDevice() const { return err_device_; }
  std::mutex& GeneratedLaunchMutex() { return gen_mu_; }
  uint32_t NextLaunchEpoch();
  void ThrowIfGeneratedKernelFailed(uint32_t epoch, const std::string& kernel) const;

  static int32_t DeviceCount();
  ~HipAccelerator() override;

 private:
  std::shared_ptr<dc_hip_ctx> ctx_;
  uint32_t* err_host_ = nullptr;
  uint32_t* err_device_ = nullptr;
  uint32_t epoch_ = 0;
  AcceleratorInfo info_;
  HipMemoryManager memory_;
  HipBackendOptions options_;
  std::mutex module_mu_;
  std::mutex gen_mu_;  // one generated launch at a time, from its epoch to its error check
  std::map<std::string, std::shared_ptr<dc_hip_module>> modules_;  // loaded code objects by path
};

// Creates the accelerator, or returns nullptr when no usable gfx950 device is present (the
// reference's plugin factories return null rather than throw, CudaBackendPlugin.cs:325-351).
std::shared_ptr<HipAccelerator> TryCreateAccelerator(const HipBackendOptions& options = {});
// Why the last TryCreateAccelerator call returned nullptr (diagnostics; the reference logs it).
std::string LastAcceleratorCreationError();

}  // namespace DotCompute::Backends::Hip

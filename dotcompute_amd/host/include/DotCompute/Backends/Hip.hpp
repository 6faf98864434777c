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

#include "../Abstractions.hpp"
#include "dotcompute_hip.h"

namespace DotCompute::Backends::Hip {

// Throws HipException for a non-zero status of the C ABI.
void Check(int32_t status, const char* what);

class HipAccelerator;

// Device allocation owned by exactly one object; freed once, by Dispose() or the destructor.
class HipAllocation {
 public:
  HipAllocation(std::shared_ptr<dc_hip_ctx> ctx, size_t bytes);
  ~HipAllocation();
  HipAllocation(const HipAllocation&) = delete;
  HipAllocation& operator=(const HipAllocation&) = delete;
  void* Pointer() const { return ptr_; }
  size_t Bytes() const { return bytes_; }
  bool Disposed() const { return disposed_; }
  void CopyFromHost(const void* src, size_t bytes, size_t offset_bytes);
  void CopyToHost(void* dst, size_t bytes, size_t offset_bytes) const;
  void Dispose();

 private:
  std::shared_ptr<dc_hip_ctx> ctx_;
  void* ptr_ = nullptr;
  size_t bytes_ = 0;
  bool disposed_ = false;
};

template <typename T>
class HipBuffer final : public IUnifiedMemoryBufferT<T> {
 public:
  HipBuffer(std::shared_ptr<dc_hip_ctx> ctx, size_t count) : alloc_(std::move(ctx), count * sizeof(T)), count_(count) {}
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
  void Dispose() override { alloc_.Dispose(); }

 private:
  HipAllocation alloc_;
  size_t count_;
};

class HipMemoryManager final : public IUnifiedMemoryManager {
 public:
  explicit HipMemoryManager(std::shared_ptr<dc_hip_ctx> ctx) : ctx_(std::move(ctx)) {}
  std::shared_ptr<IUnifiedMemoryBuffer> AllocateRaw(size_t count, ElementType type) override;
  size_t TotalAvailableMemory() const override;

 private:
  std::shared_ptr<dc_hip_ctx> ctx_;
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

  static int32_t DeviceCount();

 private:
  std::shared_ptr<dc_hip_ctx> ctx_;
  AcceleratorInfo info_;
  HipMemoryManager memory_;
  HipBackendOptions options_;
  std::mutex module_mu_;
  std::map<std::string, std::shared_ptr<dc_hip_module>> modules_;  // loaded code objects by path
};

// Creates the accelerator, or returns nullptr when no usable gfx950 device is present (the
// reference's plugin factories return null rather than throw, CudaBackendPlugin.cs:325-351).
std::shared_ptr<HipAccelerator> TryCreateAccelerator(const HipBackendOptions& options = {});

}  // namespace DotCompute::Backends::Hip

// Abstractions.hpp — the public contracts the HIP backend implements, restated in C++ with the
// reference's names and argument meanings.
//
// Reference: src/Core/DotCompute.Abstractions (IAccelerator.cs:17-205, ICompiledKernel
// IAccelerator.cs:674-686, Interfaces/IUnifiedMemoryManager.cs:12-160,
// Interfaces/IUnifiedMemoryBuffer.cs:13-246, Kernels/KernelArguments.cs:11-38,
// Kernels/KernelDefinition.cs:12-82, Types/AcceleratorType.cs:15-60).
// C# exceptions map to C++ exception types of the same name (ArgumentException,
// InvalidOperationException, NotSupportedException, OverflowException).
#pragma once

#include <cstddef>
#include <cstdint>
#include <future>
#include <memory>
#include <stdexcept>
#include <string>
#include <variant>
#include <vector>

namespace DotCompute {

// ---- exceptions (System.*) ------------------------------------------------------------------
struct ArgumentException : std::invalid_argument {
  using std::invalid_argument::invalid_argument;
};
struct ArgumentNullException : ArgumentException {
  using ArgumentException::ArgumentException;
};
struct InvalidOperationException : std::logic_error {
  using std::logic_error::logic_error;
};
struct NotSupportedException : std::logic_error {
  using std::logic_error::logic_error;
};
struct OverflowException : std::overflow_error {
  using std::overflow_error::overflow_error;
};
struct IndexOutOfRangeException : std::out_of_range {
  using std::out_of_range::out_of_range;
};
struct DivideByZeroException : std::domain_error {
  using std::domain_error::domain_error;
};
// A failed HIP runtime / library call (the reference raises CudaException with the CudaError).
struct HipException : std::runtime_error {
  int32_t Status;
  HipException(int32_t status, const std::string& what) : std::runtime_error(what), Status(status) {}
};

// ---- AcceleratorType (Types/AcceleratorType.cs:15-60) -----------------------------------------
enum class AcceleratorType : int32_t {
  Auto = -1,
  None = 0,
  CPU = 1,
  CUDA = 2,
  ROCm = 3,
  OneAPI = 4,
  Metal = 5,
  OpenCL = 6,
  DirectML = 7,
  DirectCompute = 8,
};
const char* ToString(AcceleratorType t);

// ---- AcceleratorInfo (IAccelerator.cs:567-586 for WarpSize) -----------------------------------
struct AcceleratorInfo {
  std::string Id;
  std::string Name;
  std::string DeviceType;        // "HIP": what the orchestrator matches a preferred backend against
  std::string Vendor;            // "AMD"
  std::string Architecture;      // gcnArchName, e.g. "gfx950:sramecc+:xnack-"
  int32_t ComputeUnits = 0;
  int64_t GlobalMemorySize = 0;
  int64_t LocalMemorySize = 0;   // LDS per workgroup
  int32_t MaxThreadsPerBlock = 0;
  int32_t ClockRateKHz = 0;
  int32_t WarpSize = 64;         // wavefront size on CDNA
};

// ---- memory (IUnifiedMemoryBuffer / IUnifiedMemoryManager) ------------------------------------
enum class ElementType : int32_t { Float32, Int32, UInt32, Int64, Float64, UInt16, UInt64, Int16, UInt8, Int8, Bool };
size_t ElementSize(ElementType t);

template <typename T>
struct ElementTypeOf;
template <> struct ElementTypeOf<float> { static constexpr ElementType value = ElementType::Float32; };
template <> struct ElementTypeOf<int32_t> { static constexpr ElementType value = ElementType::Int32; };
template <> struct ElementTypeOf<uint32_t> { static constexpr ElementType value = ElementType::UInt32; };
template <> struct ElementTypeOf<int64_t> { static constexpr ElementType value = ElementType::Int64; };
template <> struct ElementTypeOf<double> { static constexpr ElementType value = ElementType::Float64; };
template <> struct ElementTypeOf<uint16_t> { static constexpr ElementType value = ElementType::UInt16; };
template <> struct ElementTypeOf<uint64_t> { static constexpr ElementType value = ElementType::UInt64; };
template <> struct ElementTypeOf<int16_t> { static constexpr ElementType value = ElementType::Int16; };
template <> struct ElementTypeOf<uint8_t> { static constexpr ElementType value = ElementType::UInt8; };
template <> struct ElementTypeOf<int8_t> { static constexpr ElementType value = ElementType::Int8; };

// Untyped device buffer (IUnifiedMemoryBuffer). CopyFromAsync/CopyToAsync move host <-> device
// (IUnifiedMemoryBuffer.cs:236,246); both complete before the returned future is ready.
class IUnifiedMemoryBuffer {
 public:
  virtual ~IUnifiedMemoryBuffer() = default;
  virtual size_t SizeInBytes() const = 0;
  virtual size_t Length() const = 0;              // elements
  virtual ElementType Type() const = 0;
  virtual void* DevicePointer() const = 0;
  virtual bool IsDisposed() const = 0;
  virtual void CopyFromHost(const void* src, size_t bytes, size_t offset_bytes = 0) = 0;
  virtual void CopyToHost(void* dst, size_t bytes, size_t offset_bytes = 0) const = 0;
  // Enqueue the copy on the accelerator's stream without waiting; it has completed once the
  // accelerator synchronises. The host memory must stay valid until then.
  virtual void EnqueueCopyFromHost(const void* src, size_t bytes) { CopyFromHost(src, bytes); }
  virtual void EnqueueCopyToHost(void* dst, size_t bytes) const { CopyToHost(dst, bytes); }
  virtual void Dispose() = 0;
};

// Typed view (IUnifiedMemoryBuffer<T>, IUnifiedMemoryBuffer.cs:151,156).
template <typename T>
class IUnifiedMemoryBufferT : public IUnifiedMemoryBuffer {
 public:
  std::future<void> CopyFromAsync(const std::vector<T>& src) {
    CopyFromHost(src.data(), src.size() * sizeof(T));
    std::promise<void> p;
    p.set_value();
    return p.get_future();
  }
  std::future<void> CopyToAsync(std::vector<T>& dst) const {
    CopyToHost(dst.data(), dst.size() * sizeof(T));
    std::promise<void> p;
    p.set_value();
    return p.get_future();
  }
  T* Data() const { return static_cast<T*>(DevicePointer()); }
};

class IUnifiedMemoryManager {
 public:
  virtual ~IUnifiedMemoryManager() = default;
  // AllocateAsync<T>(count) (IUnifiedMemoryManager.cs:47)
  virtual std::shared_ptr<IUnifiedMemoryBuffer> AllocateRaw(size_t count, ElementType type) = 0;
  template <typename T>
  std::shared_ptr<IUnifiedMemoryBufferT<T>> AllocateAsync(size_t count) {
    return std::static_pointer_cast<IUnifiedMemoryBufferT<T>>(AllocateRaw(count, ElementTypeOf<T>::value));
  }
  // CopyToDeviceAsync / CopyFromDeviceAsync (:130, :143)
  template <typename T>
  void CopyToDeviceAsync(const std::vector<T>& src, IUnifiedMemoryBuffer& dst) {
    dst.CopyFromHost(src.data(), src.size() * sizeof(T));
  }
  template <typename T>
  void CopyFromDeviceAsync(const IUnifiedMemoryBuffer& src, std::vector<T>& dst) {
    src.CopyToHost(dst.data(), dst.size() * sizeof(T));
  }
  // FreeAsync (:160)
  virtual void FreeAsync(IUnifiedMemoryBuffer& buffer) { buffer.Dispose(); }
  virtual size_t TotalAvailableMemory() const = 0;
};

// ---- kernels (KernelArguments / KernelLaunchConfiguration / KernelDefinition) -----------------
struct Dim3 {
  uint32_t X = 1, Y = 1, Z = 1;
};

struct KernelLaunchConfiguration {
  Dim3 GridSize;
  Dim3 BlockSize{256, 1, 1};
  uint32_t SharedMemoryBytes = 0;
};

// A by-value struct argument passed as raw bytes (the launch block of generated kernels).
struct RawArgument {
  std::vector<uint8_t> Bytes;
};
using ScalarValue = std::variant<int32_t, uint32_t, int64_t, uint64_t, float, double, RawArgument>;

// Buffers first, then scalars, in parameter order (KernelArguments.cs:11-38; the orchestrator
// builds them in that order, KernelExecutionService.cs:409-443).
struct KernelArguments {
  std::vector<IUnifiedMemoryBuffer*> Buffers;
  std::vector<ScalarValue> ScalarArguments;
  KernelLaunchConfiguration LaunchConfiguration;
  void AddBuffer(IUnifiedMemoryBuffer* b) { Buffers.push_back(b); }
  void AddScalar(ScalarValue v) { ScalarArguments.push_back(v); }
};

enum class KernelLanguage : int32_t { CSharp, CUDA, OpenCL, HLSL, Metal, HIP, SPIRV, Binary };

struct KernelDefinition {
  std::string Name;
  std::string Code;        // HIP: path of a gfx950 code object; empty = the library's default module
  std::string EntryPoint;  // function name inside the code object
  KernelLanguage Language = KernelLanguage::HIP;
};

struct CompilationOptions {
  bool EnableDebugInfo = false;
};

// ICompiledKernel (IAccelerator.cs:674-686).
class ICompiledKernel {
 public:
  virtual ~ICompiledKernel() = default;
  virtual const std::string& Name() const = 0;
  virtual std::future<void> ExecuteAsync(const KernelArguments& arguments) = 0;
};

// IAccelerator (IAccelerator.cs:17-205; the members this path uses).
class IAccelerator {
 public:
  virtual ~IAccelerator() = default;
  virtual const AcceleratorInfo& Info() const = 0;
  virtual AcceleratorType Type() const = 0;
  // BaseAccelerator.DeviceType => Type.ToString() (src/Core/DotCompute.Core/BaseAccelerator.cs:81)
  std::string DeviceType() const { return ToString(Type()); }
  virtual IUnifiedMemoryManager& Memory() = 0;
  virtual std::future<std::shared_ptr<ICompiledKernel>> CompileKernelAsync(const KernelDefinition& definition,
                                                                           const CompilationOptions& options = {}) = 0;
  virtual std::future<void> SynchronizeAsync() = 0;
};

}  // namespace DotCompute

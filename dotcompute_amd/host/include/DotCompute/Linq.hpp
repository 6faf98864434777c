// Linq.hpp — the LINQ provider for the HIP backend: expression trees for float and int lambdas, the
// operation graph, the fusion planner that lowers a Where/Select(/Sum) chain to ONE prebuilt
// gfx950 kernel (a dc_linq_chain register program), and the queryable front end.
//
// Reference: AsComputeQueryable / ComputeQueryProvider / ComputeQueryable<T>
// (src/Extensions/DotCompute.Linq/ComputeQueryableExtensions.cs:19-68,74-646),
// ExpressionTreeVisitor (Compilation/ExpressionTreeVisitor.cs:38-159,234-272), OperationGraph /
// Operation / OperationType (Optimization/OperationGraph.cs:14-80, Optimization/OperationType.cs:12),
// the fusion rules of CudaKernelGenerator (CodeGeneration/CudaKernelGenerator.cs:1163-1226),
// BackendSelector + ComputeBackend (CodeGeneration/BackendSelector.cs:27-326, ComputeBackend.cs:9-28)
// and RuntimeExecutor (CodeGeneration/RuntimeExecutor.cs:148-179,245-312).
//
// Lambdas are written with a small expression DSL, e.g.
//   auto x = Linq::Param();
//   AsComputeQueryable(src).Where(x > 0.0f).Select(x * 2.0f + 1.0f).ToArray();
// which builds the same tree C# builds for `x => x > 0f` and `x => x * 2f + 1f`. The parameter takes
// the element type of the query (float or int, ComputeQueryable<T>); constants keep their own type
// (2 is an int, 2.0f a float), and an int constant in a float lambda is converted as C# converts it.
#pragma once

#include <functional>
#include <optional>
#include <type_traits>

#include "Abstractions.hpp"
#include "Backends/Hip.hpp"

namespace DotCompute::Linq {

// ---- expression trees ---------------------------------------------------------------------------
enum class ExprKind {
  Parameter, Constant,
  Negate, Abs, Sqrt, Floor, Ceiling, Round,
  Add, Subtract, Multiply, Divide, Modulo, Min, Max, Pow,
  GreaterThan, GreaterThanOrEqual, LessThan, LessThanOrEqual, Equal, NotEqual,
  AndAlso, OrElse, Not
};

struct ExprNode {
  ExprKind Kind;
  float Value = 0.0f;     // float Constant
  int32_t IValue = 0;     // int Constant
  bool IsInt = false;     // Constant: an int literal
  std::shared_ptr<const ExprNode> Left, Right;
};

class Expr {
 public:
  Expr(float constant);    // implicit: a float literal in a lambda body (2f)
  Expr(double constant);   // implicit: taken as the float literal it is rounded to
  Expr(int32_t constant);  // implicit: an int literal (2)
  explicit Expr(std::shared_ptr<const ExprNode> n) : node_(std::move(n)) {}
  // Lambda parameter `index`: 0 is the element (x => ...); Aggregate's (acc, x) => ... names the
  // accumulator 0 and the element 1.
  static Expr Parameter(int index = 0);
  const ExprNode& Node() const { return *node_; }
  std::shared_ptr<const ExprNode> Ptr() const { return node_; }
  bool IsPredicate() const;  // comparison or logical node
  std::string ToString() const;

 private:
  std::shared_ptr<const ExprNode> node_;
};

inline Expr Param(int index = 0) { return Expr::Parameter(index); }
Expr operator+(const Expr& a, const Expr& b);
Expr operator-(const Expr& a, const Expr& b);
Expr operator*(const Expr& a, const Expr& b);
Expr operator/(const Expr& a, const Expr& b);
Expr operator%(const Expr& a, const Expr& b);
Expr operator-(const Expr& a);
Expr operator>(const Expr& a, const Expr& b);
Expr operator>=(const Expr& a, const Expr& b);
Expr operator<(const Expr& a, const Expr& b);
Expr operator<=(const Expr& a, const Expr& b);
Expr operator==(const Expr& a, const Expr& b);
Expr operator!=(const Expr& a, const Expr& b);
Expr operator&&(const Expr& a, const Expr& b);
Expr operator||(const Expr& a, const Expr& b);
Expr operator!(const Expr& a);

namespace MathF {  // System.MathF members usable in lambdas
Expr Abs(const Expr& a);
Expr Sqrt(const Expr& a);
Expr Floor(const Expr& a);
Expr Ceiling(const Expr& a);
Expr Round(const Expr& a);  // MidpointRounding.ToEven
Expr Min(const Expr& a, const Expr& b);
Expr Max(const Expr& a, const Expr& b);
Expr Pow(const Expr& a, const Expr& b);  // the C runtime's powf, as .NET's MathF.Pow
}  // namespace MathF
namespace Math {  // System.Math members over int (Math.Abs(int.MinValue) throws OverflowException)
Expr Abs(const Expr& a);
Expr Min(const Expr& a, const Expr& b);
Expr Max(const Expr& a, const Expr& b);
}  // namespace Math

// ---- query representation: the Queryable.* method-call chain -------------------------------------
struct MethodCall {
  std::string Method;          // "Where", "Select", "Sum", "Count", "OrderBy", ...
  std::optional<Expr> Lambda;  // absent for parameterless operators (Sum(), Count())
  std::optional<int64_t> Count = std::nullopt;  // Take(n) / Skip(n)
  std::optional<Expr> Seed = std::nullopt;      // Aggregate(seed, func)
};

// ---- operation graph ------------------------------------------------------------------------------
enum class OperationType { Map = 0, Filter = 1, Reduce = 2, Scan = 3, Join = 4, GroupBy = 5, OrderBy = 6, Aggregate = 7 };

struct Operation {
  std::string Id;                       // "op_0", "op_1", ...
  OperationType Type = OperationType::Map;
  std::vector<std::string> Dependencies;
  std::string Method;                   // the LINQ method it came from
  std::optional<Expr> Lambda;           // Metadata["Lambda"]
};

struct OperationGraph {
  std::vector<Operation> Operations;
  const Operation* Root() const { return Operations.empty() ? nullptr : &Operations.back(); }
};

class ExpressionTreeVisitor {
 public:
  OperationGraph Visit(const std::vector<MethodCall>& chain) const;
  // ExpressionTreeVisitor.cs:234-272; nullopt for unsupported methods.
  static std::optional<OperationType> MapMethodToOperationType(const std::string& method);
};

// ---- backend selection ---------------------------------------------------------------------------
enum class ComputeBackend { CpuSimd = 0, Cuda = 1, Metal = 2, Hip = 3 };

struct WorkloadCharacteristics {
  size_t DataSize = 0;
  int OperationCount = 0;
  bool HasReduction = false;
};

class BackendSelector {
 public:
  static constexpr size_t MinGpuDataSize = 10'000;  // BackendSelector.cs:27
  explicit BackendSelector(bool hipAvailable) : hip_available_(hipAvailable) {}
  // This build has exactly one compute backend. Without a HIP device it throws instead of
  // returning CpuSimd: the queries must never silently run on the host.
  ComputeBackend SelectBackend(const WorkloadCharacteristics& workload) const;

 private:
  bool hip_available_;
};

// ---- fusion planner / HIP kernel generator -------------------------------------------------------
enum class Terminal {
  ToArray, Sum, Count, LongCount, Average, Min, Max,
  First, FirstOrDefault, Last, LastOrDefault, Single, SingleOrDefault, Aggregate
};

// Aggregate folds the HIP kernels run exactly: int (acc, x) => acc + x (unchecked, so the fold is
// the exact total wrapped to 32 bits, whatever the order), Math.Min / Math.Max over int, and
// MathF.Min / MathF.Max over float (IEEE minimum / maximum: associative).
enum class AggregateKind { None, Add, Min, Max };

struct FusedKernelPlan {
  dc_linq_chain Program{};                // one fused program for all Filter/Map stages
  Terminal Term = Terminal::ToArray;
  ElementType Element = ElementType::Float32;  // the chain's element type (float32 or int32 kernels)
  bool BareSource = true;                 // no Where/Select: the terminal runs on the source array itself
  bool CanFault = false;                  // an int32 program that can throw (DivideByZero / Overflow)
  AggregateKind Fold = AggregateKind::None;  // Terminal::Aggregate
  std::optional<int32_t> Seed;            // Aggregate(seed, func) over int
  std::vector<std::string> FusedOperationIds;
  std::string Listing() const;            // human-readable program
};

class HipKernelGenerator {
 public:
  // Lowers the graph to one fused kernel: all Filter/Map stages (CanBeFused chains) plus an
  // optional terminal Reduce that selects the Sum/Count or Min/Max kernel. `element` is the
  // query's element type. Throws NotSupportedException for graphs the prebuilt kernels cannot run
  // (OrderBy, GroupBy, Join, lambdas that change the element type, expressions needing more than
  // two saved registers, an int division or remainder or Math.Abs in the right operand of && / ||).
  FusedKernelPlan GenerateHipKernel(const OperationGraph& graph, ElementType element = ElementType::Float32) const;
  // CudaKernelGenerator.cs:1163-1226: consecutive Map/Filter operations form one group.
  static std::vector<const Operation*> IdentifyFusableOperations(const OperationGraph& graph);
  static bool CanBeFused(const Operation& op);
  // Appends the register program of one lambda: a value (ends in v) or a predicate (ends in p).
  static void CompileLambda(const Expr& lambda, bool predicate, std::vector<dc_linq_instr>& code,
                            ElementType element = ElementType::Float32);
};

// ---- execution -------------------------------------------------------------------------------------
template <typename T>
struct QueryResult {
  std::vector<T> Values;      // ToArray; First / Last / Single: the element, when Count > 0
  double Sum = 0.0;           // float sources: Sum / Average (float64 accumulator)
  int64_t IntSum = 0;         // int32 sources: the exact total
  bool SumOverflowed = false; // int32 sources: the checked int32 Sum throws OverflowException
  T Extreme{};                // Min / Max
  int64_t Count = 0;
};

// Element types the HIP LINQ kernels take (the reference's provider accepts any unmanaged T,
// ComputeQueryableExtensions.cs:249-259; the kernels here exist for float and int).
template <typename T>
inline constexpr bool IsLinqElement = std::is_same<T, float>::value || std::is_same<T, int32_t>::value;

class RuntimeExecutor {
 public:
  explicit RuntimeExecutor(std::shared_ptr<Backends::Hip::HipAccelerator> accelerator) : acc_(std::move(accelerator)) {}
  // Host source: allocate, copy in, launch, copy back only the compacted result. An int32 program
  // that throws for some element raises the exception LINQ-to-objects raises first
  // (DivideByZeroException / OverflowException).
  template <typename T>
  QueryResult<T> Execute(const FusedKernelPlan& plan, const T* data, size_t n);
  // Device-resident source (no host round trip for the input).
  template <typename T>
  QueryResult<T> Execute(const FusedKernelPlan& plan, const IUnifiedMemoryBuffer& source, size_t n);
  Backends::Hip::HipAccelerator& Accelerator() { return *acc_; }

  // Interprets the count the compaction kernel wrote. k >= 0 is the kept count. k == -1 means the
  // resident grid's bounded wait for a tile count gave up (the device did not run every workgroup
  // of the grid at once, e.g. because another process held CUs): the chain is then run once more
  // through `rerunOrdered`, which uses the ticket-ordered lookback grid (it cannot stall), and
  // that count is returned. Anything else, or a second -1, throws InvalidOperationException.
  static int64_t ResolveCompactedCount(int64_t k, const std::function<int64_t()>& rerunOrdered);
  // Throws the exception of an int32 fault word (4 * index + kind); returns for -1.
  static void ThrowIfFaulted(int64_t fault);

 private:
  QueryResult<float> Run(const FusedKernelPlan& plan, const float* device_in, size_t n);
  QueryResult<int32_t> Run(const FusedKernelPlan& plan, const int32_t* device_in, size_t n);
 public:
  // A chain cut by Take/Skip: `segments` are the fused Where/Select programs between the cuts,
  // cuts[i] the Take(k) or Skip(k) after segment i (one fewer than the segments), the last plan
  // carries the terminal. Each cut segment is compacted on the device and the cut applied to the
  // compacted range; nothing comes back to the host but the terminal's result.
  template <typename T>
  QueryResult<T> RunSegments(const std::vector<FusedKernelPlan>& segments, const std::vector<MethodCall>& cuts,
                             const T* device_in, size_t n);

 private:
  // Compaction of one program over [device_in, +n) into `out`: the kept count. With `limit`, the
  // consumer stops pulling after `limit` kept elements (Take, First, Single), so an element that
  // throws after them is never evaluated in C#: the count is then that of the elements before it.
  template <typename T>
  int64_t ToArrayLimited(const FusedKernelPlan& plan, const T* device_in, size_t n, T* out,
                         std::optional<int64_t> limit);
  std::shared_ptr<Backends::Hip::HipAccelerator> acc_;
};

class ComputeQueryProvider {
 public:
  // Default: the HIP accelerator of device 0 (the reference's provider probes a CudaAccelerator,
  // ComputeQueryableExtensions.cs:125-179). May hold no accelerator; executing then throws.
  ComputeQueryProvider();
  explicit ComputeQueryProvider(std::shared_ptr<Backends::Hip::HipAccelerator> accelerator);
  static std::shared_ptr<ComputeQueryProvider> Default();

  bool HasAccelerator() const { return executor_ != nullptr; }
  // Stages of ExecuteTyped (ComputeQueryableExtensions.cs:329-443): visit -> select backend ->
  // generate the fused kernel -> run it.
  template <typename T>
  QueryResult<T> Execute(const std::vector<MethodCall>& chain, Terminal terminal, const T* host, size_t n,
                         const IUnifiedMemoryBuffer* device);
  FusedKernelPlan Plan(const std::vector<MethodCall>& chain, Terminal terminal, size_t n,
                       ElementType element = ElementType::Float32) const;

 private:
  std::unique_ptr<RuntimeExecutor> executor_;
};

// ComputeQueryable<T> (ComputeQueryableExtensions.cs:74-118) for T = float or int.
template <typename T>
class ComputeQueryable {
  static_assert(IsLinqElement<T>, "the HIP LINQ kernels take float or int sources");

 public:
  // Enumerable.Average returns float for float sources and double for int sources.
  using AverageType = std::conditional_t<std::is_same<T, int32_t>::value, double, float>;

  ComputeQueryable(const T* data, size_t n, std::shared_ptr<ComputeQueryProvider> provider);
  ComputeQueryable(const IUnifiedMemoryBuffer& device, std::shared_ptr<ComputeQueryProvider> provider);

  ComputeQueryable Where(const Expr& predicate) const;
  ComputeQueryable Select(const Expr& selector) const;
  ComputeQueryable ComputeWhere(const Expr& predicate) const { return Where(predicate); }
  ComputeQueryable ComputeSelect(const Expr& selector) const { return Select(selector); }
  // Operators the HIP kernels do not implement: accepted into the chain, rejected at execution
  // with NotSupportedException (as the reference's generators reject them).
  ComputeQueryable OrderBy(const Expr& key) const;
  // Take / Skip (mapped to Filter operations by the reference, ExpressionTreeVisitor.cs:263-265):
  // the first n elements of the sequence at that point, or all but them. n <= 0: Take gives an
  // empty sequence, Skip the whole one (Enumerable semantics).
  ComputeQueryable Take(int64_t count) const;
  ComputeQueryable Skip(int64_t count) const;

  std::vector<T> ToArray() const;
  // Element operators (ExpressionTreeVisitor.cs:264-265), with Enumerable's exceptions:
  // InvalidOperationException "Sequence contains no elements" / "... more than one element".
  T First() const;
  T First(const Expr& predicate) const { return Where(predicate).First(); }
  T FirstOrDefault() const;   // default(T) = 0 on an empty sequence
  T Last() const;
  T LastOrDefault() const;
  T Single() const;
  T SingleOrDefault() const;  // 0 when empty; more than one element still throws
  // Aggregate((acc, x) => ...) and Aggregate(seed, (acc, x) => ...): the folds AggregateKind names,
  // with Param(0) the accumulator and Param(1) the element (over float: MathF.Min / MathF.Max);
  // other folds (float + and * depend on the order of their roundings) throw NotSupportedException.
  T Aggregate(const Expr& func) const;
  T Aggregate(T seed, const Expr& func) const;
  std::vector<T> ToComputeArray() const { return ToArray(); }
  // float: float64 accumulator, cast to float (Enumerable.Sum(IEnumerable<float>)). int: checked
  // int32 total, OverflowException by the BCL's rule for the source: its vectorised lane rule over a
  // bare array, the element-by-element running total after Where/Select.
  T Sum() const;
  int32_t Count() const;      // throws OverflowException above int.MaxValue
  int64_t LongCount() const;
  AverageType Average() const;  // throws InvalidOperationException on an empty sequence
  T Min() const;              // throws InvalidOperationException on an empty sequence
  T Max() const;              // throws InvalidOperationException on an empty sequence
  // Any / All (Reduce operators, ExpressionTreeVisitor.cs:244-245) on the count kernel: Any(p) is
  // "Where(p) keeps something", All(p) is "Where(!p) keeps nothing" (a NaN fails any comparison,
  // so !p keeps it and All is false, as Enumerable.All evaluates p per element).
  bool Any() const;
  bool Any(const Expr& predicate) const;
  bool All(const Expr& predicate) const;

  const std::vector<MethodCall>& Chain() const { return chain_; }
  FusedKernelPlan Explain(Terminal terminal = Terminal::ToArray) const;

 private:
  QueryResult<T> Run(Terminal t, const std::vector<MethodCall>* chain = nullptr) const;
  const T* host_ = nullptr;
  const IUnifiedMemoryBuffer* device_ = nullptr;
  size_t n_ = 0;
  std::shared_ptr<ComputeQueryProvider> provider_;
  std::vector<MethodCall> chain_;
};

extern template class ComputeQueryable<float>;
extern template class ComputeQueryable<int32_t>;

// AsComputeQueryable (ComputeQueryableExtensions.cs:19-23). The source must outlive the query.
ComputeQueryable<float> AsComputeQueryable(const std::vector<float>& source,
                                           std::shared_ptr<ComputeQueryProvider> provider = nullptr);
ComputeQueryable<float> AsComputeQueryable(const float* data, size_t n,
                                           std::shared_ptr<ComputeQueryProvider> provider = nullptr);
ComputeQueryable<int32_t> AsComputeQueryable(const std::vector<int32_t>& source,
                                             std::shared_ptr<ComputeQueryProvider> provider = nullptr);
ComputeQueryable<int32_t> AsComputeQueryable(const int32_t* data, size_t n,
                                             std::shared_ptr<ComputeQueryProvider> provider = nullptr);
// Device-resident source of element type T (the buffer's type must match: checked at execution).
template <typename T = float>
ComputeQueryable<T> AsComputeQueryable(const IUnifiedMemoryBuffer& device,
                                       std::shared_ptr<ComputeQueryProvider> provider = nullptr);

}  // namespace DotCompute::Linq

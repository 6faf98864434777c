// C++ tests of the host layer (orchestrator, LINQ provider + fusion planner, algorithms), mirroring
// the reference's own tests. CPU cases (--cpu) touch no device; GPU cases (--gpu) run on gfx950 and
// are checked against the CPU oracle (oracle/liboracle.so), which this test binary links as the
// checker only.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <thread>
#include <cstring>
#include <random>

#include "DotCompute/Algorithms.hpp"
#include "DotCompute/Linq.hpp"
#include "DotCompute/Runtime.hpp"
#include "test_framework.hpp"

extern "C" {
#include "../../oracle/oracle.h"
}

using namespace DotCompute;
using namespace DotCompute::Linq;
using DotCompute::Algorithms::CsrMatrix;
using DotCompute::Algorithms::Matrix;
using DotCompute::Algorithms::MatrixOperations;
using DotCompute::Algorithms::SparseOps;

namespace {

std::vector<float> Uniform(size_t n, uint64_t seed, uint32_t stream = 0, int unit = 0) {
  std::vector<float> v(n);
  oracle_gen_uniform_f32(v.data(), (int64_t)n, seed, stream, unit);
  return v;
}

bool BitsEqual(const std::vector<float>& a, const std::vector<float>& b) {
  return a.size() == b.size() && (a.empty() || std::memcmp(a.data(), b.data(), a.size() * sizeof(float)) == 0);
}

std::string Listing(const Expr& where, const Expr& select) {
  auto q = ComputeQueryable<float>(nullptr, 0, std::make_shared<ComputeQueryProvider>(nullptr)).Where(where).Select(select);
  return q.Explain().Listing();
}

// Evaluates a lambda tree exactly as C# evaluates it (one float rounding per operation); used to
// check the generated register program against the tree it came from.
float EvalValue(const ExprNode& n, float x) {
  switch (n.Kind) {
    case ExprKind::Parameter: return x;
    case ExprKind::Constant: return n.Value;
    case ExprKind::Negate: return -EvalValue(*n.Left, x);
    case ExprKind::Abs: return std::fabs(EvalValue(*n.Left, x));
    case ExprKind::Sqrt: return std::sqrt(EvalValue(*n.Left, x));
    case ExprKind::Add: return EvalValue(*n.Left, x) + EvalValue(*n.Right, x);
    case ExprKind::Subtract: return EvalValue(*n.Left, x) - EvalValue(*n.Right, x);
    case ExprKind::Multiply: return EvalValue(*n.Left, x) * EvalValue(*n.Right, x);
    case ExprKind::Divide: return EvalValue(*n.Left, x) / EvalValue(*n.Right, x);
    case ExprKind::Pow: return std::pow(EvalValue(*n.Left, x), EvalValue(*n.Right, x));  // float powf
    case ExprKind::Min: {
      float a = EvalValue(*n.Left, x), b = EvalValue(*n.Right, x);
      if (std::isnan(a) || std::isnan(b)) return NAN;
      if (a == b) return std::signbit(a) ? a : b;
      return a < b ? a : b;
    }
    case ExprKind::Max: {
      float a = EvalValue(*n.Left, x), b = EvalValue(*n.Right, x);
      if (std::isnan(a) || std::isnan(b)) return NAN;
      if (a == b) return std::signbit(a) ? b : a;
      return a > b ? a : b;
    }
    default: throw std::logic_error("not a value");
  }
}

bool EvalPred(const ExprNode& n, float x) {
  switch (n.Kind) {
    case ExprKind::GreaterThan: return EvalValue(*n.Left, x) > EvalValue(*n.Right, x);
    case ExprKind::GreaterThanOrEqual: return EvalValue(*n.Left, x) >= EvalValue(*n.Right, x);
    case ExprKind::LessThan: return EvalValue(*n.Left, x) < EvalValue(*n.Right, x);
    case ExprKind::LessThanOrEqual: return EvalValue(*n.Left, x) <= EvalValue(*n.Right, x);
    case ExprKind::Equal: return EvalValue(*n.Left, x) == EvalValue(*n.Right, x);
    case ExprKind::NotEqual: return EvalValue(*n.Left, x) != EvalValue(*n.Right, x);
    case ExprKind::AndAlso: return EvalPred(*n.Left, x) && EvalPred(*n.Right, x);
    case ExprKind::OrElse: return EvalPred(*n.Left, x) || EvalPred(*n.Right, x);
    case ExprKind::Not: return !EvalPred(*n.Left, x);
    default: throw std::logic_error("not a predicate");
  }
}

// Planner output for a Where(pred).Select(sel) chain, run by the oracle's interpreter, must equal
// the direct evaluation of the two trees on every input.
void CheckProgramAgainstTree(const Expr& pred, const Expr& sel, const std::vector<float>& xs) {
  auto q = ComputeQueryable<float>(nullptr, 0, std::make_shared<ComputeQueryProvider>(nullptr)).Where(pred).Select(sel);
  FusedKernelPlan plan = q.Explain();
  for (float x : xs) {
    float y = 0.0f;
    int32_t keep = oracle_linq_eval(&plan.Program, x, &y);
    CHECK(keep >= 0);
    const bool want = EvalPred(pred.Node(), x);
    CHECK((keep == 1) == want);
    if (want) {
      const float ref = EvalValue(sel.Node(), x);
      CHECK((std::isnan(ref) && std::isnan(y)) || std::memcmp(&ref, &y, 4) == 0);
    }
  }
}

// C# `int` evaluation of a lambda tree (unchecked + - *, / and % truncating, throwing
// DivideByZeroException / OverflowException, Math.Abs throwing for int.MinValue, operands left to
// right, && and || short-circuiting). Returns the fault kind (0 none) through `fault`.
struct IntEval {
  int fault = 0;
  int32_t Value(const ExprNode& n, int32_t x) {
    if (fault) return 0;
    switch (n.Kind) {
      case ExprKind::Parameter: return x;
      case ExprKind::Constant: return n.IValue;
      case ExprKind::Negate: return (int32_t)(0u - (uint32_t)Value(*n.Left, x));
      case ExprKind::Abs: {
        const int32_t v = Value(*n.Left, x);
        if (!fault && v == INT32_MIN) fault = DC_LINQ_FAULT_OVERFLOW;
        return v < 0 ? -v : v;
      }
      default: break;
    }
    const int32_t a = Value(*n.Left, x);
    const int32_t b = Value(*n.Right, x);
    if (fault) return 0;
    switch (n.Kind) {
      case ExprKind::Add: return (int32_t)((uint32_t)a + (uint32_t)b);
      case ExprKind::Subtract: return (int32_t)((uint32_t)a - (uint32_t)b);
      case ExprKind::Multiply: return (int32_t)((uint32_t)a * (uint32_t)b);
      case ExprKind::Divide:
      case ExprKind::Modulo:
        if (b == 0) { fault = DC_LINQ_FAULT_DIVIDE_BY_ZERO; return 0; }
        if (b == -1 && a == INT32_MIN) { fault = DC_LINQ_FAULT_OVERFLOW; return 0; }
        return n.Kind == ExprKind::Divide ? a / b : a % b;
      case ExprKind::Min: return std::min(a, b);
      case ExprKind::Max: return std::max(a, b);
      default: throw std::logic_error("not an int value");
    }
  }
  bool Pred(const ExprNode& n, int32_t x) {
    if (fault) return false;
    switch (n.Kind) {
      case ExprKind::AndAlso: return Pred(*n.Left, x) && Pred(*n.Right, x);
      case ExprKind::OrElse: return Pred(*n.Left, x) || Pred(*n.Right, x);
      case ExprKind::Not: return !Pred(*n.Left, x);
      default: break;
    }
    const int32_t a = Value(*n.Left, x), b = Value(*n.Right, x);
    switch (n.Kind) {
      case ExprKind::GreaterThan: return a > b;
      case ExprKind::GreaterThanOrEqual: return a >= b;
      case ExprKind::LessThan: return a < b;
      case ExprKind::LessThanOrEqual: return a <= b;
      case ExprKind::Equal: return a == b;
      case ExprKind::NotEqual: return a != b;
      default: throw std::logic_error("not a predicate");
    }
  }
};

FusedKernelPlan PlanI32(const Expr& pred, const Expr& sel) {
  return ComputeQueryable<int32_t>(nullptr, 0, std::make_shared<ComputeQueryProvider>(nullptr)).Where(pred).Select(sel)
      .Explain();
}

// The int32 program of Where(pred).Select(sel), run by the oracle's interpreter, must keep, map
// and throw exactly as the C# evaluation of the two trees does, element by element.
void CheckProgramAgainstTreeI32(const Expr& pred, const Expr& sel, const std::vector<int32_t>& xs) {
  FusedKernelPlan plan = PlanI32(pred, sel);
  CHECK(plan.Element == ElementType::Int32);
  for (int32_t x : xs) {
    int32_t y = 0, kind = 0;
    const int32_t keep = oracle_linq_eval_i32(&plan.Program, x, &y, &kind);
    CHECK(keep >= 0);
    IntEval ev;
    const bool want = ev.Pred(pred.Node(), x);
    int32_t ref = 0;
    if (!ev.fault && want) ref = ev.Value(sel.Node(), x);
    CHECK(kind == ev.fault);
    if (!ev.fault) {
      CHECK((keep == 1) == want);
      if (want) CHECK(y == ref);
    }
  }
}

std::vector<int32_t> IntSamples(size_t n, uint64_t seed) {
  std::vector<int32_t> v(n);
  oracle_gen_uniform_i32(v.data(), (int64_t)n, seed, 1, -1000, 1000);
  for (int32_t e : {0, 1, -1, 2, -2, 46341, -46341, INT32_MAX, INT32_MIN, INT32_MIN + 1}) v.push_back(e);
  return v;
}

std::vector<int32_t> Range(int32_t start, int32_t count) {  // Enumerable.Range
  std::vector<int32_t> v((size_t)count);
  for (int32_t i = 0; i < count; ++i) v[(size_t)i] = start + i;
  return v;
}

std::shared_ptr<Backends::Hip::HipAccelerator> Gpu() {
  static auto acc = Backends::Hip::TryCreateAccelerator();
  if (!acc) throw std::runtime_error("no gfx950 device");
  return acc;
}

}  // namespace

// ============================== CPU: fusion planner ==============================================

TEST_CPU(planner_emits_the_benchmark_chain) {
  auto x = Param();
  const std::string l = Listing(x > 0.0f, x * 2.0f + 1.0f);
  CHECK(l == "terminal ToArray (float32)\n0: LOAD e\n1: CMP_GT 0\n2: FILTER\n3: LOAD e\n4: MUL 2\n5: ADD 1\n6: MAP\n");
}

TEST_CPU(planner_swaps_constant_on_the_left) {
  auto x = Param();
  CHECK(Listing(0.5f < x, 2.0f - x) == "terminal ToArray (float32)\n0: LOAD e\n1: CMP_GT 0.5\n2: FILTER\n3: LOAD e\n4: RSUB 2\n5: MAP\n");
  CHECK(Listing(1.0f >= x, 3.0f / x) == "terminal ToArray (float32)\n0: LOAD e\n1: CMP_LE 1\n2: FILTER\n3: LOAD e\n4: RDIV 3\n5: MAP\n");
}

TEST_CPU(planner_folds_constants_like_csharp) {
  auto x = Param();
  CHECK(Listing(x > (1.0f - 1.0f), x * (2.0f + 1.0f)) ==
        "terminal ToArray (float32)\n0: LOAD e\n1: CMP_GT 0\n2: FILTER\n3: LOAD e\n4: MUL 3\n5: MAP\n");
}

TEST_CPU(planner_uses_save_registers_for_two_subtrees) {
  auto x = Param();
  const std::string l = Listing(x != 0.0f, (x + 1.0f) * (x - 1.0f));
  CHECK(l.find("STORE_S0") != std::string::npos);
  CHECK(l.find("MUL s0") != std::string::npos);
  std::vector<float> xs = Uniform(2000, 3);
  CheckProgramAgainstTree(x != 0.0f, (x + 1.0f) * (x - 1.0f), xs);
  CheckProgramAgainstTree(x > -0.5f, ((x + 1.0f) * (x - 1.0f)) / ((x * x) + (x - 3.0f)), xs);
}

TEST_CPU(planner_rejects_too_deep_expressions) {
  auto x = Param();
  // Needs two saved values for the right operand and two more while computing the left one.
  Expr p1 = ((x + 1.0f) * (x - 1.0f)) + ((x + 2.0f) * (x - 2.0f));
  Expr p2 = ((x + 3.0f) * (x - 3.0f)) + ((x + 4.0f) * (x - 4.0f));
  CHECK_THROWS(NotSupportedException, Listing(x > 0.0f, p1 / p2));
  // Sethi-Ullman order keeps this one within the two saved registers.
  Expr ok = ((x + 1.0f) * (x - 1.0f)) / (((x + 2.0f) * (x - 2.0f)) + ((x + 3.0f) * (x - 3.0f)));
  CheckProgramAgainstTree(x > 0.0f, ok, Uniform(3000, 8));
}

TEST_CPU(planner_compound_predicates_match_tree_evaluation) {
  auto x = Param();
  std::vector<float> xs = Uniform(5000, 11);
  xs.push_back(0.0f);
  xs.push_back(-0.0f);
  xs.push_back(NAN);
  CheckProgramAgainstTree(x > 0.0f && x < 0.5f, x * 2.0f + 1.0f, xs);
  CheckProgramAgainstTree(x < -0.5f || x > 0.5f, MathF::Abs(x), xs);
  CheckProgramAgainstTree((x < -0.5f || x > 0.5f) && (x != 0.75f || x * x > 0.9f), x - 0.25f, xs);
  CheckProgramAgainstTree(!(x >= 0.0f), MathF::Sqrt(-x), xs);
  CheckProgramAgainstTree(x * x + x > 0.1f, MathF::Min(x, 0.25f) + MathF::Max(x * 3.0f, -1.0f), xs);
  CheckProgramAgainstTree(x > 0.0f && x < 0.9f && x != 0.5f, 1.0f / (x + 1.0f), xs);
}

TEST_CPU(planner_rejects_three_composite_terms) {
  auto x = Param();
  Expr p = ((x < 0.0f || x > 1.0f) && (x != 2.0f || x != 3.0f)) || ((x < 5.0f || x > 6.0f) && (x != 7.0f || x != 8.0f));
  CHECK_THROWS(NotSupportedException, Listing(p, x));
}

TEST_CPU(planner_where_needs_a_predicate_and_select_a_value) {
  auto x = Param();
  CHECK_THROWS(NotSupportedException, Listing(x + 1.0f, x));
  CHECK_THROWS(NotSupportedException, Listing(x > 0.0f, x > 1.0f));
}

TEST_CPU(visitor_maps_methods_like_the_reference) {
  CHECK(*ExpressionTreeVisitor::MapMethodToOperationType("Select") == OperationType::Map);
  CHECK(*ExpressionTreeVisitor::MapMethodToOperationType("Where") == OperationType::Filter);
  CHECK(*ExpressionTreeVisitor::MapMethodToOperationType("Sum") == OperationType::Reduce);
  CHECK(*ExpressionTreeVisitor::MapMethodToOperationType("OrderBy") == OperationType::OrderBy);
  CHECK(*ExpressionTreeVisitor::MapMethodToOperationType("GroupBy") == OperationType::GroupBy);
  CHECK(!ExpressionTreeVisitor::MapMethodToOperationType("Zip").has_value());
  auto x = Param();
  OperationGraph g = ExpressionTreeVisitor().Visit({{"Where", x > 0.0f}, {"Select", x * 2.0f}, {"Sum", std::nullopt}});
  CHECK(g.Operations.size() == 3);
  CHECK(g.Operations[1].Dependencies.size() == 1 && g.Operations[1].Dependencies[0] == "op_0");
  CHECK(HipKernelGenerator::IdentifyFusableOperations(g).size() == 2);
  CHECK(g.Root()->Type == OperationType::Reduce);
}

TEST_CPU(planner_terminals_and_unsupported_operators) {
  auto x = Param();
  auto p = std::make_shared<ComputeQueryProvider>(nullptr);
  auto q = ComputeQueryable<float>(nullptr, 0, p).Where(x > 0.0f).Select(x * 2.0f + 1.0f);
  CHECK(q.Explain(Terminal::Sum).Term == Terminal::Sum);
  CHECK(q.Explain(Terminal::Average).Term == Terminal::Average);
  CHECK(q.Explain(Terminal::Count).FusedOperationIds.size() == 3);
  CHECK(q.Explain(Terminal::Min).Term == Terminal::Min);
  CHECK(q.Explain(Terminal::Max).Term == Terminal::Max);
  CHECK_THROWS(NotSupportedException, q.OrderBy(x).Explain());
  CHECK_THROWS(InvalidOperationException, q.Min());  // no HIP device behind this provider
}

TEST_CPU(planner_int_chains_follow_csharp_int_semantics) {
  auto x = Param();
  // Range(1, 100).Where(x => x % 2 == 0).Select(x => x * x) (LinqBackendIntegrationTests.cs:309-325)
  CHECK(PlanI32(x % 2 == 0, x * x).Listing() ==
        "terminal ToArray (int32)\n0: LOAD e\n1: REM 2\n2: CMP_EQ 0\n3: FILTER\n4: LOAD e\n5: MUL e\n6: MAP\n");
  CHECK(!PlanI32(x % 2 == 0, x * x).CanFault);
  CHECK(PlanI32(x != 0, 100 / x).CanFault);
  CHECK(PlanI32(x > 0, x / -1).CanFault);  // int.MinValue / -1
  CHECK(PlanI32(x > 0, Math::Abs(x)).CanFault);
  const auto xs = IntSamples(4000, 5);
  CheckProgramAgainstTreeI32(x % 2 == 0, x * x, xs);
  CheckProgramAgainstTreeI32(x > 2, x * 2, xs);
  CheckProgramAgainstTreeI32(x % 7 != 3 && x < 500, (x + 1) * (x - 1) - x % 5, xs);
  CheckProgramAgainstTreeI32(x != 0, 1000 / x + 1000 % x, xs);
  CheckProgramAgainstTreeI32(x > -5, 100 / x, xs);        // throws for x == 0
  CheckProgramAgainstTreeI32(x < 0 || x > 10, -x * 3, xs);  // wraps for int.MinValue
  CheckProgramAgainstTreeI32(x >= INT32_MIN, Math::Abs(x) % 1000, xs);
  CheckProgramAgainstTreeI32(x * x > 100, Math::Min(x, 7) + Math::Max(x * 3, -9), xs);
  CheckProgramAgainstTreeI32(x != 1, (x / (x - 1)) + (x % (x + 1)), xs);  // both operands throw
  CheckProgramAgainstTreeI32(!(x > 0), x / -1, xs);       // OverflowException for int.MinValue
}

TEST_CPU(planner_int_chains_reject_type_changes_and_conditional_throws) {
  auto x = Param();
  CHECK_THROWS(NotSupportedException, PlanI32(x > 0.5f, x));          // x > 0.5f is a float comparison
  CHECK_THROWS(NotSupportedException, PlanI32(x > 0, x * 2.0f));      // Select to float
  CHECK_THROWS(NotSupportedException, PlanI32(x > 0, MathF::Sqrt(x)));
  CHECK_THROWS(NotSupportedException, PlanI32(x != 0 && 10 / x > 1, x));  // evaluated only when x != 0
  CHECK_THROWS(NotSupportedException, PlanI32(x == 0 || 10 % x > 1, x));
  PlanI32(10 / x > 1 && x != 0, x);  // a throwing left operand is always evaluated: fine
  // C# constant folding is checked
  CHECK_THROWS(OverflowException, Expr(INT32_MAX) + Expr(1));
  CHECK_THROWS(DivideByZeroException, Expr(1) / Expr(0));
  CHECK(((Expr(7) + Expr(5)) % Expr(5)).Node().IValue == 2);
  // an int literal in a float lambda is converted to float (x > 0 means x > 0f)
  CHECK(Listing(x > 0, x * 2 + 1) == Listing(x > 0.0f, x * 2.0f + 1.0f));
}

TEST_CPU(planner_float_remainder_and_rounding_match_tree_evaluation) {
  auto x = Param();
  auto q = ComputeQueryable<float>(nullptr, 0, std::make_shared<ComputeQueryProvider>(nullptr));
  const FusedKernelPlan plan = q.Where(x % 0.25f != 0.0f).Select(MathF::Floor(x * 8.0f) + MathF::Ceiling(x) +
                                                                 MathF::Round(x * 3.0f)).Explain();
  for (float v : Uniform(5000, 21)) {
    float y = 0.0f;
    const int32_t keep = oracle_linq_eval(&plan.Program, v, &y);
    CHECK((keep == 1) == (std::fmod(v, 0.25f) != 0.0f));
    if (keep == 1) {
      const float ref = (std::floor(v * 8.0f) + std::ceil(v)) + std::nearbyint(v * 3.0f);
      CHECK(std::memcmp(&ref, &y, 4) == 0);
    }
  }
}

TEST_CPU(planner_pow_operand_order_and_element_type) {
  auto x = Param();
  // Pow(x, c) keeps c as the operand; Pow(c, x) takes the swapped form; Pow of two computed operands
  // saves the exponent first.
  CHECK(Listing(x > 0.0f, MathF::Pow(x, 2.5f)).find("1: CMP_GT 0\n2: FILTER\n3: LOAD e\n4: POW 2.5\n5: MAP") !=
        std::string::npos);
  CHECK(Listing(x > 0.0f, MathF::Pow(2.0f, x)).find("4: RPOW 2\n") != std::string::npos);
  CHECK(Listing(x > 0.0f, MathF::Pow(x + 1.0f, x * 0.5f)).find("POW s0") != std::string::npos);
  std::vector<float> xs = Uniform(4000, 23);
  xs.push_back(0.0f);
  xs.push_back(-0.0f);
  xs.push_back(NAN);
  xs.push_back(INFINITY);
  CheckProgramAgainstTree(MathF::Pow(x, 2.0f) > 0.25f, MathF::Pow(x, 0.5f) + MathF::Pow(3.0f, x), xs);
  CheckProgramAgainstTree(x != 0.0f, MathF::Pow(x + 1.0f, x * 0.5f) - MathF::Pow(x, x), xs);
  CHECK(MathF::Pow(x, 2.0f).ToString() == "MathF.Pow(x, 2f)");
  // MathF.Pow over an int converts to float: another element type than the chain's.
  auto i = Param();
  CHECK_THROWS(NotSupportedException, PlanI32(i > 0, MathF::Pow(i, 2)));
}

// ============================== CPU: runtime, registry, no-device behaviour =======================

TEST_CPU(orchestrator_backend_mapping_and_priority) {
  CHECK(KernelExecutionService::MapDeviceTypeToBackend("hip") == "HIP");
  CHECK(KernelExecutionService::MapDeviceTypeToBackend("ROCm") == "HIP");
  CHECK(KernelExecutionService::MapDeviceTypeToBackend("cuda") == "CUDA");
  CHECK(KernelExecutionService::GetBackendPriority("HIP") < KernelExecutionService::GetBackendPriority("CPU"));
  CHECK(KernelExecutionService::GetBackendPriority("Vulkan") == 999);
}

const KernelRegistrationInfo& Registered(const std::vector<KernelRegistrationInfo>& regs, const std::string& name) {
  for (const auto& r : regs)
    if (r.Name == name) return r;
  throw std::runtime_error("kernel not in the generated registry: " + name);
}

TEST_CPU(orchestrator_work_size_and_launch) {
  auto regs = Generated::KernelRegistry::GetAllKernels();
  const auto& vadd = Registered(regs, "VectorAdd");
  CHECK(vadd.FullName == "Kernels.VectorAdd" && vadd.HipNeedsLength && vadd.HipAbi == HipKernelAbi::Generated);
  std::vector<float> a(1000), b(1000), r(1000);
  std::vector<KernelArg> args{Arg(a), Arg(b), Arg(r)};
  CHECK(KernelExecutionService::DeriveWorkSize(vadd, args) == 1000);
  KernelLaunchConfiguration lc = KernelExecutionService::DeriveLaunch(vadd, args, 1000);
  CHECK(lc.BlockSize.X == 256 && lc.GridSize.X == 4 && lc.GridSize.Y == 1);
}

TEST_CPU(generated_registry_describes_every_kernel) {
  // KernelExecutionMetadataTests' checks, on this build's generated registry: dimensionality,
  // parameter descriptors, the HIP slot, and CPU-only registration when a body has no translation.
  auto regs = Generated::KernelRegistry::GetAllKernels();
  CHECK(regs.size() == 12);
  const auto& t = Registered(regs, "Transpose");
  CHECK(t.Dimensions == 2 && t.FullName == "DotCompute.Samples.Grids.Transpose");
  CHECK((t.SupportedBackends == std::vector<std::string>{"CPU", "HIP"}));
  CHECK(t.Parameters.size() == 4 && t.Parameters[0].IsBuffer && t.Parameters[0].IsReadOnly &&
        !t.Parameters[1].IsReadOnly && !t.Parameters[2].IsBuffer && t.Parameters[2].Type == ElementType::Int32);
  CHECK(t.HipSource.find("__x = __ii % __xext, __y = __ii / __xext") != std::string::npos);
  CHECK(Registered(regs, "Stencil3D").Dimensions == 3);
  const auto& saxpy = Registered(regs, "Saxpy");  // reads and writes y; only reads x
  CHECK(saxpy.Parameters[0].IsRead && !saxpy.Parameters[0].IsWritten);
  CHECK(saxpy.Parameters[1].IsRead && saxpy.Parameters[1].IsWritten);
  const auto& vadd = Registered(regs, "VectorAdd");  // the output is written in full, never read: not copied in
  CHECK(!vadd.Parameters[2].IsRead && vadd.Parameters[2].IsWritten && vadd.Parameters[2].IsCovered);
  // Outputs written under a condition (or in two branches) are copied in: elements the body leaves
  // alone must come back as the caller's values.
  CHECK(!Registered(regs, "CopyPositive").Parameters[1].IsCovered);
  CHECK(!Registered(regs, "ScaleClamp").Parameters[1].IsCovered);
  CHECK(Registered(regs, "HashMix").Parameters[1].IsCovered);
  CHECK((vadd.SupportedBackends == std::vector<std::string>{"CPU"}));
  const auto& soft = Registered(regs, "Softplus");
  CHECK(soft.HipEntryPoint.empty() && soft.HipDiagnostic.find("MathF.Log") != std::string::npos);
  CHECK((BackendNames((int32_t)KernelBackends::All) == std::vector<std::string>{"CPU", "CUDA", "Metal", "OpenCL", "HIP"}));
}

TEST_CPU(orchestrator_without_accelerators_throws) {
  ServiceCollection services;
  services.AddDotComputeRuntime();
  auto sp = services.BuildServiceProvider();
  auto orch = sp->GetRequiredOrchestrator();
  std::vector<float> a{1, 2}, b{3, 4}, r(2);
  CHECK_THROWS(InvalidOperationException, orch->ExecuteAsync("VectorAdd", {Arg(a), Arg(b), Arg(r)}).get());
  CHECK_THROWS(ArgumentException, orch->ExecuteAsync("NoSuchKernel", {Arg(a)}).get());
  CHECK(!orch->ValidateKernelArgsAsync("VectorAdd", {Arg(a), Arg(b)}));   // too few arguments
  CHECK(!orch->ValidateKernelArgsAsync("VectorAdd", {Arg(a), Arg(b), Arg(1.0f)}));  // scalar for a buffer
}

TEST_CPU(service_provider_requires_runtime) {
  ServiceCollection services;
  CHECK_THROWS(InvalidOperationException, services.BuildServiceProvider()->GetRequiredOrchestrator());
}

TEST_CPU(hip_backend_registration_skips_missing_device) {
  if (Backends::Hip::HipAccelerator::DeviceCount() > 0) return;  // only meaningful without a GPU
  ServiceCollection services;
  services.AddDotComputeRuntime().AddHipBackend();
  auto sp = services.BuildServiceProvider();
  sp->Runtime()->Initialize();
  CHECK(sp->Runtime()->GetAccelerators().empty());
  CHECK(Backends::Hip::TryCreateAccelerator() == nullptr);
  // The LINQ provider refuses to run instead of falling back to the host.
  auto x = Param();
  std::vector<float> src{1, 2, 3};
  auto q = AsComputeQueryable(src, std::make_shared<ComputeQueryProvider>(nullptr)).Where(x > 1.0f);
  CHECK_THROWS(InvalidOperationException, q.ToArray());
}

TEST_CPU(compaction_give_up_is_retried_on_the_ordered_grid) {
  // A resident grid that gave up reports count -1: the executor re-runs the chain once on the
  // ticket-ordered grid and returns that count; a second failure or any other negative count throws.
  int reruns = 0;
  CHECK(RuntimeExecutor::ResolveCompactedCount(12, [&] { ++reruns; return int64_t(0); }) == 12);
  CHECK(reruns == 0);
  CHECK(RuntimeExecutor::ResolveCompactedCount(-1, [&] { ++reruns; return int64_t(7); }) == 7);
  CHECK(reruns == 1);
  CHECK_THROWS(InvalidOperationException,
               RuntimeExecutor::ResolveCompactedCount(-1, [&] { ++reruns; return int64_t(-1); }));
  CHECK(reruns == 2);
  CHECK_THROWS(InvalidOperationException,
               RuntimeExecutor::ResolveCompactedCount(-5, [&] { ++reruns; return int64_t(3); }));
  CHECK(reruns == 2);  // only -1 (the documented give-up value) is retried
}

TEST_CPU(csr_matrix_validation_matches_reference) {
  CHECK_THROWS(ArgumentException, CsrMatrix<float>(2, 2, {1.0f}, {0}, {0, 1}));          // rowPointers != rows+1
  CHECK_THROWS(ArgumentException, CsrMatrix<float>(1, 2, {1.0f, 2.0f}, {0}, {0, 2}));   // values vs columns
  CsrMatrix<float> ok(1, 2, {1.0f, 2.0f}, {0, 1}, {0, 2});
  CHECK(ok.NonZeroCount() == 2);
  CHECK_THROWS(ArgumentException, Matrix(2, 2, std::vector<float>(3)));
}

// ============================== GPU: orchestrator ==================================================

TEST_GPU(readme_quick_start_vector_add_on_hip) {
  ServiceCollection services;
  services.AddDotComputeRuntime().AddHipBackend();
  auto orch = services.BuildServiceProvider()->GetRequiredOrchestrator();
  std::vector<float> a{1, 2, 3, 4, 5}, b{10, 20, 30, 40, 50}, result(5);
  std::vector<float> out = orch->ExecuteAsync("VectorAdd", "HIP", {Arg(a), Arg(b), Arg(result)}).get();
  CHECK((result == std::vector<float>{11, 22, 33, 44, 55}));
  CHECK(out == result);
}

TEST_GPU(vector_add_100k_bit_exact_and_unknown_backend_falls_back) {
  ServiceCollection services;
  services.AddDotComputeRuntime().AddHipBackend();
  auto orch = services.BuildServiceProvider()->GetRequiredOrchestrator();
  auto a = Uniform(100000, 42, 0), b = Uniform(100000, 42, 1);
  std::vector<float> r(100000), ref(100000);
  oracle_vector_add_f32(a.data(), b.data(), ref.data(), 100000);
  orch->ExecuteAsync("VectorAdd", "HIP", {Arg(a), Arg(b), Arg(r)}).get();
  CHECK(BitsEqual(r, ref));
  std::fill(r.begin(), r.end(), 0.0f);
  orch->ExecuteAsync("VectorAdd", "Vulkan", {Arg(a), Arg(b), Arg(r)}).get();  // -> optimal accelerator
  CHECK(BitsEqual(r, ref));
  std::fill(r.begin(), r.end(), 0.0f);
  orch->ExecuteAsync("Kernels.VectorAdd", {Arg(a), Arg(b), Arg(r)}).get();     // full name, no backend
  CHECK(BitsEqual(r, ref));
}

TEST_GPU(compiled_kernel_from_code_object_matches) {
  // The generated VectorAdd through ICompiledKernel, packed the way a managed caller packs it:
  // buffers, then the dc_gen_launch block as a by-value struct argument.
  auto acc = Gpu();
  KernelDefinition def;
  def.Name = "VectorAdd";
  def.EntryPoint = "VectorAdd";
  auto kernel = acc->CompileKernelAsync(def).get();
  const size_t n = 70001;
  auto a = Uniform(n, 5, 0), b = Uniform(n, 5, 1);
  auto da = acc->Memory().AllocateAsync<float>(n), db = acc->Memory().AllocateAsync<float>(n),
       dr = acc->Memory().AllocateAsync<float>(n);
  da->CopyFromAsync(a).get();
  db->CopyFromAsync(b).get();
  dc_gen_launch launch{};
  launch.work = (int64_t)n;
  launch.epoch = acc->NextLaunchEpoch();
  launch.error = acc->GeneratedErrorWordsDevice();
  launch.len[0] = launch.len[1] = launch.len[2] = (int64_t)n;
  RawArgument block;
  block.Bytes.resize(sizeof(launch));
  std::memcpy(block.Bytes.data(), &launch, sizeof(launch));
  KernelArguments args;
  args.AddBuffer(da.get());
  args.AddBuffer(db.get());
  args.AddBuffer(dr.get());
  args.AddScalar(block);
  args.LaunchConfiguration.GridSize = {(uint32_t)((n + 255) / 256), 1, 1};
  kernel->ExecuteAsync(args).get();
  acc->SynchronizeAsync().get();
  acc->ThrowIfGeneratedKernelFailed(launch.epoch, "VectorAdd");
  std::vector<float> r(n), ref(n);
  dr->CopyToAsync(r).get();
  oracle_vector_add_f32(a.data(), b.data(), ref.data(), (int64_t)n);
  CHECK(BitsEqual(r, ref));
  def.EntryPoint = "NoSuchKernel";
  CHECK_THROWS(ArgumentException, acc->CompileKernelAsync(def).get());
}

TEST_GPU(orchestrator_execute_with_device_buffers) {
  // ExecuteWithBuffersAsync (IComputeOrchestrator.cs:51): device-resident buffers pass straight to
  // the kernel; nothing is copied in or out.
  ServiceCollection services;
  services.AddDotComputeRuntime().AddHipBackend();
  auto sp = services.BuildServiceProvider();
  auto orch = sp->GetRequiredOrchestrator();
  sp->Runtime()->Initialize();
  if (sp->Runtime()->GetAccelerators().empty())
    throw std::runtime_error("no accelerator: " + Backends::Hip::LastAcceleratorCreationError());
  auto& acc = *sp->Runtime()->GetAccelerators().at(0);
  const size_t n = 250007;
  auto a = Uniform(n, 11, 0), b = Uniform(n, 11, 1);
  std::vector<float> ref(n), r(n);
  oracle_vector_add_f32(a.data(), b.data(), ref.data(), (int64_t)n);
  auto da = acc.Memory().AllocateRaw(n, ElementType::Float32), db = acc.Memory().AllocateRaw(n, ElementType::Float32),
       dr = acc.Memory().AllocateRaw(n, ElementType::Float32);
  da->CopyFromHost(a.data(), n * sizeof(float));
  db->CopyFromHost(b.data(), n * sizeof(float));
  orch->ExecuteWithBuffersAsync("VectorAdd", {da.get(), db.get(), dr.get()}, {}).get();
  dr->CopyToHost(r.data(), n * sizeof(float));
  CHECK(BitsEqual(r, ref));
  // A shorter input buffer is refused before any launch (the CPU invoker throws
  // IndexOutOfRangeException at the first index past its end).
  auto shortB = acc.Memory().AllocateRaw(n - 1, ElementType::Float32);
  CHECK_THROWS(IndexOutOfRangeException,
               orch->ExecuteWithBuffersAsync("VectorAdd", {da.get(), shortB.get(), dr.get()}, {}).get());
  std::vector<float> ha(n - 1);
  CHECK_THROWS(IndexOutOfRangeException, orch->ExecuteAsync("VectorAdd", "HIP", {Arg(ha), Arg(b), Arg(r)}).get());
}

TEST_GPU(csr_spmv_code_object_kernel_matches_oracle) {
  // The code-object kernel with SparseMatrixKernels.CUDASparseMatrixKernel's parameter list
  // (values, col_indices, row_pointers, x, y, num_rows), launched through HipCompiledKernel with
  // one wavefront per row, against float64 row sums.
  auto acc = Gpu();
  KernelDefinition def;
  def.Name = "csr_spmv";
  def.EntryPoint = "csr_spmv";
  auto kernel = acc->CompileKernelAsync(def).get();
  const int64_t rows = 1000000;
  std::vector<int32_t> rp(rows + 1);
  const int64_t nnz = oracle_gen_zipf_rowptr(rows, 2.0, 4096, 42, rp.data());
  std::vector<int32_t> col((size_t)nnz);
  std::vector<float> val((size_t)nnz);
  oracle_gen_zipf_fill(rows, rows, 42, rp.data(), col.data(), val.data());
  auto x = Uniform((size_t)rows, 42, 5, 1);
  auto dval = acc->Memory().AllocateAsync<float>((size_t)nnz);
  auto dcol = acc->Memory().AllocateAsync<int32_t>((size_t)nnz);
  auto drp = acc->Memory().AllocateAsync<int32_t>((size_t)rows + 1);
  auto dx = acc->Memory().AllocateAsync<float>((size_t)rows), dy = acc->Memory().AllocateAsync<float>((size_t)rows);
  dval->CopyFromAsync(val).get();
  dcol->CopyFromAsync(col).get();
  drp->CopyFromAsync(rp).get();
  dx->CopyFromAsync(x).get();
  KernelArguments args;
  args.AddBuffer(dval.get());
  args.AddBuffer(dcol.get());
  args.AddBuffer(drp.get());
  args.AddBuffer(dx.get());
  args.AddBuffer(dy.get());
  args.AddScalar((int32_t)rows);
  args.LaunchConfiguration.BlockSize = {256, 1, 1};
  args.LaunchConfiguration.GridSize = {(uint32_t)((rows + 3) / 4), 1, 1};  // 4 rows (waves) per block
  kernel->ExecuteAsync(args).get();
  acc->SynchronizeAsync().get();
  std::vector<float> y((size_t)rows);
  dy->CopyToAsync(y).get();
  std::vector<double> x64(x.begin(), x.end()), y64((size_t)rows), scale((size_t)rows), xabs((size_t)rows);
  std::vector<float> vabs(val.size());
  for (size_t i = 0; i < val.size(); ++i) vabs[i] = std::fabs(val[i]);
  for (int64_t i = 0; i < rows; ++i) xabs[i] = std::fabs(x64[i]);
  oracle_spmv_csr_f64(rp.data(), col.data(), val.data(), x64.data(), y64.data(), rows);
  oracle_spmv_csr_f64(rp.data(), col.data(), vabs.data(), xabs.data(), scale.data(), rows);
  int64_t bad = 0;
  for (int64_t r = 0; r < rows; ++r) bad += std::fabs(y[r] - y64[r]) > 1e-4 * scale[r] + 1e-30;
  CHECK(bad == 0);
}

// ============================== GPU: generated [Kernel] samples through the orchestrator ==========

std::shared_ptr<IComputeOrchestrator> HipOrchestrator() {
  ServiceCollection services;
  services.AddDotComputeRuntime().AddHipBackend();
  return services.BuildServiceProvider()->GetRequiredOrchestrator();
}

template <typename T>
std::vector<T> Ints(size_t n, uint64_t seed, int32_t lo, int32_t hi) {
  std::vector<int32_t> v(n);
  oracle_gen_uniform_i32(v.data(), (int64_t)n, seed, 1, lo, hi);
  return std::vector<T>(v.begin(), v.end());
}

template <typename T>
bool SameBits(const std::vector<T>& a, const std::vector<T>& b) {
  return a.size() == b.size() && (a.empty() || std::memcmp(a.data(), b.data(), a.size() * sizeof(T)) == 0);
}

TEST_GPU(generated_elementwise_kernels_match_oracle) {
  auto orch = HipOrchestrator();
  const size_t n = 1000003;
  {  // Saxpy: y is read and written
    auto x = Uniform(n, 70, 0), y = Uniform(n, 70, 1), ref = y;
    CHECK(oracle_kernel_saxpy(x.data(), (int64_t)n, ref.data(), (int64_t)n, 1.75f) == 0);
    std::vector<float> out = orch->ExecuteAsync("Saxpy", "HIP", {Arg(x), Arg(y), Arg(1.75f)}).get();
    CHECK(BitsEqual(y, ref) && BitsEqual(out, ref));
  }
  {  // ScaleClamp with NaN, infinities and signed zeros among the inputs
    auto in = Uniform(n, 71, 0);
    const float specials[] = {NAN, -NAN, INFINITY, -INFINITY, 0.0f, -0.0f, 1e-40f, -1e-40f, 0.25f, -0.5f};
    for (size_t i = 0; i < 10; ++i) in[i * 997] = specials[i];
    std::vector<float> out(n), ref(n);
    CHECK(oracle_kernel_scale_clamp(in.data(), (int64_t)n, ref.data(), (int64_t)n, 3.0f, -1.5f, 2.0f) == 0);
    orch->ExecuteAsync("ScaleClamp", "HIP", {Arg(in), Arg(out), Arg(3.0f), Arg(-1.5f), Arg(2.0f)}).get();
    CHECK(BitsEqual(out, ref));
  }
  {  // HashMix: wrapping uint multiplies and shifts
    auto keys = Ints<uint32_t>(n, 72, -2000000000, 2000000000);
    std::vector<uint32_t> out(n), ref(n);
    CHECK(oracle_kernel_hash_mix(keys.data(), (int64_t)n, ref.data(), (int64_t)n, 0x9E3779B9u) == 0);
    orch->ExecuteAsync("HashMix", "HIP", {Arg(keys), Arg(out), Arg((uint32_t)0x9E3779B9u)}).get();
    CHECK(SameBits(out, ref));
  }
  {  // LongMix: shift count 65 masked to 1, float -> long saturation, wrapping sums
    auto a = Ints<int64_t>(n, 73, -2000000000, 2000000000);
    for (size_t i = 0; i < n; i += 3) a[i] = a[i] * 4294967296LL + 12345;
    auto f = Uniform(n, 73, 2);
    for (size_t i = 0; i < n; i += 5) f[i] *= 8.0f;  // |f * 3e18| up to 2.4e19: saturates
    f[1] = NAN;
    std::vector<int64_t> out(n), ref(n);
    CHECK(oracle_kernel_long_mix(a.data(), (int64_t)n, f.data(), (int64_t)n, ref.data(), (int64_t)n, 65) == 0);
    orch->ExecuteAsync("LongMix", "HIP", {Arg(a), Arg(f), Arg(out), Arg(65)}).get();
    CHECK(SameBits(out, ref));
  }
  {  // Gather with valid indices
    auto src = Uniform(5000, 74, 0);
    auto idx = Ints<int32_t>(n, 74, 0, 4999);
    std::vector<float> out(n), ref(n);
    CHECK(oracle_kernel_gather(src.data(), 5000, idx.data(), (int64_t)n, ref.data(), (int64_t)n) == 0);
    orch->ExecuteAsync("Gather", "HIP", {Arg(src), Arg(idx), Arg(out)}).get();
    CHECK(BitsEqual(out, ref));
  }
  {  // IntDivide, divisors without zero
    auto a = Ints<int32_t>(n, 75, -2147483647, 2147483647);
    auto b = Ints<int32_t>(n, 76, 1, 100000);
    for (size_t i = 0; i < n; i += 2) b[i] = -b[i];
    std::vector<int32_t> out(n), ref(n);
    CHECK(oracle_kernel_int_divide(a.data(), (int64_t)n, b.data(), (int64_t)n, ref.data(), (int64_t)n) == 0);
    orch->ExecuteAsync("IntDivide", "HIP", {Arg(a), Arg(b), Arg(out)}).get();
    CHECK(SameBits(out, ref));
  }
}

TEST_GPU(generated_partial_writes_keep_the_callers_elements) {
  // A kernel that writes only some elements of its output must hand back the caller's values for
  // the rest, even when the device block it runs in last held another launch's data.
  auto orch = HipOrchestrator();
  const size_t n = 300001;
  std::vector<float> a(n, 7.0f), b(n, 8.0f), r(n, 0.0f);
  orch->ExecuteAsync("VectorAdd", "HIP", {Arg(a), Arg(b), Arg(r)}).get();  // leaves 15.0f in a pooled block
  auto in = Uniform(n, 81, 0);
  for (int round = 0; round < 2; ++round) {
    std::vector<float> out(n, -5.0f), ref(n);
    for (size_t i = 0; i < n; ++i) ref[i] = in[i] > 0.0f ? in[i] : -5.0f;
    std::vector<float> res = orch->ExecuteAsync("CopyPositive", "HIP", {Arg(in), Arg(out)}).get();
    CHECK(BitsEqual(out, ref) && BitsEqual(res, ref));
  }
}

TEST_GPU(generated_kernel_exceptions_are_not_lost_between_threads) {
  // Two threads launch generated kernels on one accelerator at the same time; every launch that
  // divides by zero must raise its exception, whatever the other thread's launch reported.
  auto orch = HipOrchestrator();
  std::atomic<int> thrown{0}, wrong{0};
  auto worker = [&](bool faulting) {
    for (int it = 0; it < 20; ++it) {
      std::vector<int32_t> a(50000, 7), b(50000, 1), q(50000);
      if (faulting) b[12345] = 0;
      try {
        orch->ExecuteAsync("IntDivide", "HIP", {Arg(a), Arg(b), Arg(q)}).get();
        if (faulting) ++wrong;
      } catch (const DivideByZeroException&) {
        if (faulting) ++thrown;
        else ++wrong;
      }
    }
  };
  std::thread t1(worker, true), t2(worker, false), t3(worker, true);
  t1.join();
  t2.join();
  t3.join();
  CHECK(thrown.load() == 40 && wrong.load() == 0);
}

TEST_GPU(generated_grid_kernels_match_oracle) {
  auto orch = HipOrchestrator();
  {  // 2-D transpose, rows x cols not a multiple of anything
    const int32_t rows = 1001, cols = 777;
    auto in = Uniform((size_t)rows * cols, 77, 0);
    std::vector<float> out((size_t)rows * cols), ref(out.size());
    CHECK(oracle_kernel_transpose(in.data(), (int64_t)in.size(), ref.data(), (int64_t)ref.size(), rows, cols) == 0);
    orch->ExecuteAsync("Transpose", "HIP", {Arg(in), Arg(out), Arg(rows), Arg(cols)}).get();
    CHECK(BitsEqual(out, ref));
  }
  {  // 2-D with a loop: the inner product in order, bit-identical to the sequential oracle
    const int32_t m = 300, k = 211, n = 257;
    auto a = Uniform((size_t)m * k, 78, 0), b = Uniform((size_t)k * n, 78, 1);
    std::vector<float> c((size_t)m * n), ref(c.size());
    CHECK(oracle_kernel_matmul_naive(a.data(), (int64_t)a.size(), b.data(), (int64_t)b.size(), ref.data(),
                                     (int64_t)ref.size(), k, m, n) == 0);
    std::vector<float> out = orch->ExecuteAsync("MatMulNaive", "HIP", {Arg(a), Arg(b), Arg(c), Arg(k), Arg(m), Arg(n)}).get();
    CHECK(BitsEqual(c, ref) && BitsEqual(out, ref));
  }
  {  // 3-D stencil
    const int32_t d = 21, h = 33, w = 45;
    auto src = Uniform((size_t)d * h * w, 79, 0);
    std::vector<float> dst(src.size()), ref(src.size());
    CHECK(oracle_kernel_stencil3d(src.data(), (int64_t)src.size(), ref.data(), (int64_t)ref.size(), d, h, w) == 0);
    orch->ExecuteAsync("Stencil3D", "HIP", {Arg(src), Arg(dst), Arg(d), Arg(h), Arg(w)}).get();
    CHECK(BitsEqual(dst, ref));
  }
}

TEST_GPU(generated_kernels_raise_csharp_exceptions) {
  auto orch = HipOrchestrator();
  // Index outside the source span: IndexOutOfRangeException (the oracle's CPU loop throws too).
  auto src = Uniform(100, 80, 0);
  std::vector<int32_t> idx{0, 5, 99, 100, 7};
  std::vector<float> out(5);
  CHECK(oracle_kernel_gather(src.data(), 100, idx.data(), 5, out.data(), 5) == 1);
  CHECK_THROWS(IndexOutOfRangeException, orch->ExecuteAsync("Gather", "HIP", {Arg(src), Arg(idx), Arg(out)}).get());
  idx[3] = -1;
  CHECK_THROWS(IndexOutOfRangeException, orch->ExecuteAsync("Gather", "HIP", {Arg(src), Arg(idx), Arg(out)}).get());
  idx[3] = 3;  // and the next launch on the same accelerator is clean
  orch->ExecuteAsync("Gather", "HIP", {Arg(src), Arg(idx), Arg(out)}).get();
  CHECK(out[3] == src[3]);
  // Integer division by zero and int.MinValue / -1.
  std::vector<int32_t> a{10, 20, 30}, b{1, 0, 3}, q(3);
  CHECK_THROWS(DivideByZeroException, orch->ExecuteAsync("IntDivide", "HIP", {Arg(a), Arg(b), Arg(q)}).get());
  a = {INT32_MIN, 1, 2};
  b = {-1, 1, 1};
  CHECK_THROWS(OverflowException, orch->ExecuteAsync("IntDivide", "HIP", {Arg(a), Arg(b), Arg(q)}).get());
  // A shorter input than the work size (VectorAdd reads b[i] for every i < result.Length).
  std::vector<float> x(1000, 1.0f), y(999, 2.0f), r(1000);
  CHECK_THROWS(IndexOutOfRangeException, orch->ExecuteAsync("VectorAdd", "HIP", {Arg(x), Arg(y), Arg(r)}).get());
  // A zero extent divides by zero in the coordinate reconstruction.
  std::vector<float> in(6), tout(6);
  CHECK_THROWS(DivideByZeroException, orch->ExecuteAsync("Transpose", "HIP", {Arg(in), Arg(tout), Arg(2), Arg(0)}).get());
  // No HIP translation: the orchestrator says so instead of running anything.
  std::vector<float> sx(10), sy(10);
  CHECK_THROWS(NotSupportedException, orch->ExecuteAsync("Softplus", "HIP", {Arg(sx), Arg(sy)}).get());
}

// ============================== GPU: LINQ provider =================================================

TEST_GPU(linq_reference_golden_vectors) {
  auto x = Param();
  auto p = std::make_shared<ComputeQueryProvider>(Gpu());
  // ComputeQueryProviderTests.cs:341-365, :602-612
  std::vector<float> s15{1, 2, 3, 4, 5};
  CHECK((AsComputeQueryable(s15, p).Where(x > 3.0f).ToArray() == std::vector<float>{4, 5}));
  std::vector<float> s3{1, 2, 3};
  CHECK((AsComputeQueryable(s3, p).Select(x * 2.0f).ToArray() == std::vector<float>{2, 4, 6}));
  CHECK(AsComputeQueryable(s15, p).Sum() == 15.0f);
  // LinqBackendIntegrationTests.cs:51-66, :139-176
  CHECK((AsComputeQueryable(s15, p).Where(x > 2.0f).Select(x * 2.0f).ToArray() == std::vector<float>{6, 8, 10}));
  std::vector<float> s10(10);
  for (int i = 0; i < 10; ++i) s10[i] = (float)(i + 1);
  CHECK((AsComputeQueryable(s10, p).Where(x > 3.0f).Select(x * 3.0f).ToArray() ==
         std::vector<float>{12, 15, 18, 21, 24, 27, 30}));
  std::vector<float> s1000(1000);
  for (int i = 0; i < 1000; ++i) s1000[i] = (float)(i + 1);
  CHECK(AsComputeQueryable(s1000, p).Sum() == 500500.0f);
  CHECK(AsComputeQueryable(s10, p).Where(x > 5.0f).Count() == 5);
  CHECK(AsComputeQueryable(s10, p).Average() == 5.5f);
  std::vector<float> empty;
  CHECK_THROWS(InvalidOperationException, AsComputeQueryable(empty, p).Average());
  CHECK(AsComputeQueryable(empty, p).Sum() == 0.0f);
  // FutureExpansionTests.cs:553-570: Range(1, 100) -> Sum 5050, Count 100, Max 100
  std::vector<float> s100(100);
  for (int i = 0; i < 100; ++i) s100[i] = (float)(i + 1);
  CHECK(AsComputeQueryable(s100, p).Sum() == 5050.0f);
  CHECK(AsComputeQueryable(s100, p).Count() == 100);
  CHECK(AsComputeQueryable(s100, p).Max() == 100.0f);
  // ExpressionTreeVisitorTests.cs:113-147: Min / Max of {5, 2, 8, 1}
  std::vector<float> s4{5, 2, 8, 1};
  CHECK(AsComputeQueryable(s4, p).Min() == 1.0f);
  CHECK(AsComputeQueryable(s4, p).Max() == 8.0f);
  CHECK_THROWS(InvalidOperationException, AsComputeQueryable(empty, p).Min());
  CHECK_THROWS(InvalidOperationException, AsComputeQueryable(s4, p).Where(x > 9.0f).Max());
  // ComputeQueryProviderTests.cs:573-597: {1,2,3}.Any(x > 2) and .All(x > 0) are true
  CHECK(AsComputeQueryable(s3, p).Any(x > 2.0f));
  CHECK(AsComputeQueryable(s3, p).All(x > 0.0f));
  CHECK(!AsComputeQueryable(s3, p).Any(x > 3.0f));
  CHECK(!AsComputeQueryable(s3, p).All(x > 1.0f));
  CHECK(!AsComputeQueryable(empty, p).Any() && AsComputeQueryable(empty, p).All(x > 0.0f));
  std::vector<float> with_nan{1.0f, NAN, 2.0f};
  CHECK(!AsComputeQueryable(with_nan, p).All(x > 0.0f));  // NaN > 0 is false
  CHECK(AsComputeQueryable(with_nan, p).Any(x != x));     // and NaN != NaN is true
}

TEST_GPU(linq_reference_golden_vectors_on_int_sources) {
  // The reference's LINQ known answers, as written: int sources and int lambdas.
  auto x = Param();
  auto p = std::make_shared<ComputeQueryProvider>(Gpu());
  // ComputeQueryProviderTests.cs:341-365: {1..5}.Where(x > 3) -> {4, 5}; {1,2,3}.Select(x * 2) -> {2, 4, 6}
  std::vector<int32_t> s15{1, 2, 3, 4, 5}, s3{1, 2, 3};
  CHECK((AsComputeQueryable(s15, p).Where(x > 3).ToArray() == std::vector<int32_t>{4, 5}));
  CHECK((AsComputeQueryable(s3, p).Select(x * 2).ToArray() == std::vector<int32_t>{2, 4, 6}));
  // :602-612: Sum of {1..5} = 15
  CHECK(AsComputeQueryable(s15, p).Sum() == 15);
  // LinqBackendIntegrationTests.cs:51-66: Where(x > 2).Select(x * 2) -> {6, 8, 10}
  CHECK((AsComputeQueryable(s15, p).Where(x > 2).Select(x * 2).ToArray() == std::vector<int32_t>{6, 8, 10}));
  // :139-161: {1..10}.Where(x > 3).Select(x * 3) -> {12, ..., 30}
  CHECK((AsComputeQueryable(Range(1, 10), p).Where(x > 3).Select(x * 3).ToArray() ==
         std::vector<int32_t>{12, 15, 18, 21, 24, 27, 30}));
  // :164-176: Enumerable.Range(1, 1000).Sum() == 500500
  const auto r1000 = Range(1, 1000);
  CHECK(AsComputeQueryable(r1000, p).Sum() == 500500);
  // :309-325: Range(1, 100).Where(x % 2 == 0).Select(x * x): 50 elements, first 4, last 10000
  const auto r100 = Range(1, 100);
  const auto sq = AsComputeQueryable(r100, p).Where(x % 2 == 0).Select(x * x).ToArray();
  CHECK(sq.size() == 50 && sq.front() == 4 && sq.back() == 10000);
  CHECK(AsComputeQueryable(r100, p).Where(x % 2 == 0).Select(x * x).Sum() == 171700);  // 4 * (1^2 + ... + 50^2)
  CHECK(AsComputeQueryable(r100, p).Where(x % 2 == 0).Count() == 50);
  CHECK(AsComputeQueryable(r100, p).Average() == 50.5);
  CHECK(AsComputeQueryable(r100, p).Where(x > 10).Min() == 11 && AsComputeQueryable(r100, p).Max() == 100);
  std::vector<int32_t> empty;
  CHECK(AsComputeQueryable(empty, p).Sum() == 0);
  CHECK_THROWS(InvalidOperationException, AsComputeQueryable(empty, p).Max());
  CHECK_THROWS(InvalidOperationException, AsComputeQueryable(s15, p).Where(x > 9).Average());
}

TEST_GPU(linq_int_exceptions_follow_linq_to_objects) {
  auto x = Param();
  auto p = std::make_shared<ComputeQueryProvider>(Gpu());
  std::vector<int32_t> z{5, 0, 7};
  CHECK_THROWS(DivideByZeroException, AsComputeQueryable(z, p).Select(100 / x).ToArray());
  CHECK_THROWS(DivideByZeroException, AsComputeQueryable(z, p).Select(100 % x).Sum());
  // a Where that drops the zero keeps the Select from ever dividing by it
  CHECK((AsComputeQueryable(z, p).Where(x != 0).Select(100 / x).ToArray() == std::vector<int32_t>{20, 14}));
  std::vector<int32_t> m{3, INT32_MIN};
  CHECK_THROWS(OverflowException, AsComputeQueryable(m, p).Select(x / -1).ToArray());
  CHECK_THROWS(OverflowException, AsComputeQueryable(m, p).Select(Math::Abs(x)).Max());
  CHECK(AsComputeQueryable(m, p).Select(-x).Min() == INT32_MIN);  // unchecked negation wraps
  // Sum: which comes first, the overflow of the running total or the throwing element
  std::vector<int32_t> a{INT32_MAX, 1, 0};  // x + 1000 / x: MaxValue, 1001 (the total overflows), then / 0
  CHECK_THROWS(OverflowException, AsComputeQueryable(a, p).Select(x + 1000 / x).Sum());
  CHECK_THROWS(DivideByZeroException, AsComputeQueryable(a, p).Select(x + 1000 / x).Count());
  std::vector<int32_t> b{INT32_MAX, 0, 1};
  CHECK_THROWS(DivideByZeroException, AsComputeQueryable(b, p).Select(x / x).Sum());
  // The two overflow rules of Enumerable.Sum(int): a bare array (span, 8 lanes) against the
  // element-by-element running total after Select. [int.MaxValue, 1, -1]: both throw.
  std::vector<int32_t> c{INT32_MAX, 1, -1};
  CHECK_THROWS(OverflowException, AsComputeQueryable(c, p).Sum());
  CHECK_THROWS(OverflowException, AsComputeQueryable(c, p).Select(x).Sum());
  // 32 elements, x0 = int.MaxValue, x1 = 1, x8 = -1: lane 0 holds MaxValue - 1, lane 1 holds 1, and
  // the lane totals add to MaxValue: no exception over the array; the running total overflows at x1.
  std::vector<int32_t> d(32, 0);
  d[0] = INT32_MAX;
  d[1] = 1;
  d[8] = -1;
  CHECK(AsComputeQueryable(d, p).Sum() == INT32_MAX);
  CHECK_THROWS(OverflowException, AsComputeQueryable(d, p).Select(x).Sum());
  CHECK(AsComputeQueryable(d, p).Select(x).Average() == (double)INT32_MAX / 32.0);  // a long sum: no overflow
}

TEST_GPU(linq_int_chains_match_oracle_at_1m) {
  auto x = Param();
  auto p = std::make_shared<ComputeQueryProvider>(Gpu());
  std::vector<int32_t> src(1 << 20);
  oracle_gen_uniform_i32(src.data(), (int64_t)src.size(), 45, 1, -1000, 1000);
  auto q = AsComputeQueryable(src, p).Where(x % 3 != 0).Select(x * x - 7 * x);
  const FusedKernelPlan plan = q.Explain();
  std::vector<int32_t> ref(src.size());
  int64_t fault = 0;
  const int64_t k = oracle_linq_where_select_i32(&plan.Program, src.data(), (int64_t)src.size(), ref.data(), &fault);
  ref.resize((size_t)k);
  CHECK(fault == DC_LINQ_FAULT_NONE && q.ToArray() == ref);
  int64_t total = 0;
  int32_t ovf = 0;
  const FusedKernelPlan ps = q.Explain(Terminal::Sum);
  CHECK(oracle_linq_where_select_sum_i32(&ps.Program, src.data(), (int64_t)src.size(), &total, &ovf, &fault) == k);
  CHECK(ovf == 1);  // about 700k values of ~3e5 each: the running total leaves int32
  CHECK_THROWS(OverflowException, q.Sum());
  CHECK(q.LongCount() == k);
  CHECK(q.Average() == (double)total / (double)k);
  int32_t mn = 0, mx = 0;
  const FusedKernelPlan pm = q.Explain(Terminal::Min);
  oracle_linq_where_select_minmax_i32(&pm.Program, src.data(), (int64_t)src.size(), 0, &mn, &fault);
  oracle_linq_where_select_minmax_i32(&pm.Program, src.data(), (int64_t)src.size(), 1, &mx, &fault);
  CHECK(q.Min() == mn && q.Max() == mx);
  auto q2 = AsComputeQueryable(src, p).Where(x > 0).Select(x - 500);  // small values: no overflow
  CHECK(q2.Sum() == (int32_t)[&] {
    int64_t s = 0;
    for (int32_t v : src) s += v > 0 ? v - 500 : 0;
    return s;
  }());
}

TEST_GPU(linq_take_skip_and_element_operators) {
  // Take/Skip/First/Last/Single (the reference maps them to Filter operations,
  // ExpressionTreeVisitor.cs:263-265) with Enumerable's results and exceptions.
  auto x = Param();
  auto p = std::make_shared<ComputeQueryProvider>(Gpu());
  const auto r100 = Range(1, 100);
  CHECK((AsComputeQueryable(r100, p).Where(x % 2 == 0).Skip(5).Take(10).ToArray() ==
         std::vector<int32_t>{12, 14, 16, 18, 20, 22, 24, 26, 28, 30}));
  CHECK((AsComputeQueryable(r100, p).Take(3).Select(x * 10).ToArray() == std::vector<int32_t>{10, 20, 30}));
  CHECK((AsComputeQueryable(r100, p).Skip(97).ToArray() == std::vector<int32_t>{98, 99, 100}));
  CHECK(AsComputeQueryable(r100, p).Skip(200).ToArray().empty() && AsComputeQueryable(r100, p).Take(-1).ToArray().empty());
  CHECK(AsComputeQueryable(r100, p).Where(x > 10).Take(5).Sum() == 11 + 12 + 13 + 14 + 15);
  CHECK(AsComputeQueryable(r100, p).Skip(90).Count() == 10);
  CHECK(AsComputeQueryable(r100, p).First() == 1 && AsComputeQueryable(r100, p).Last() == 100);
  CHECK(AsComputeQueryable(r100, p).First(x > 41) == 42);
  CHECK(AsComputeQueryable(r100, p).Where(x % 7 == 0).Last() == 98);
  CHECK(AsComputeQueryable(r100, p).Where(x > 99).Single() == 100);
  CHECK(AsComputeQueryable(r100, p).Where(x > 100).FirstOrDefault() == 0);
  CHECK(AsComputeQueryable(r100, p).Where(x > 100).LastOrDefault() == 0);
  CHECK(AsComputeQueryable(r100, p).Where(x > 100).SingleOrDefault() == 0);
  CHECK_THROWS(InvalidOperationException, AsComputeQueryable(r100, p).Where(x > 100).First());
  CHECK_THROWS(InvalidOperationException, AsComputeQueryable(r100, p).Where(x > 98).Single());
  CHECK_THROWS(InvalidOperationException, AsComputeQueryable(r100, p).Where(x > 98).SingleOrDefault());
  std::vector<float> f{0.5f, -1.0f, 2.5f, 4.0f};
  CHECK(AsComputeQueryable(f, p).Where(x < 0.0f).Single() == -1.0f);
  CHECK((AsComputeQueryable(f, p).Skip(1).Take(2).Select(x * 2.0f).ToArray() == std::vector<float>{-2.0f, 5.0f}));
  // Pull semantics: Take and First stop before an element that would throw; Last and Skip do not.
  std::vector<int32_t> z{1, 2, 3, 0, 5};
  CHECK((AsComputeQueryable(z, p).Select(100 / x).Take(3).ToArray() == std::vector<int32_t>{100, 50, 33}));
  CHECK_THROWS(DivideByZeroException, AsComputeQueryable(z, p).Select(100 / x).Take(4).ToArray());
  CHECK(AsComputeQueryable(z, p).Select(100 / x).First() == 100);
  CHECK_THROWS(DivideByZeroException, AsComputeQueryable(z, p).Select(100 / x).Last());
  CHECK_THROWS(DivideByZeroException, AsComputeQueryable(z, p).Select(100 / x).Skip(4).ToArray());
  CHECK_THROWS(InvalidOperationException, AsComputeQueryable(z, p).Select(100 / x).Single());  // 2 elements first
  // at 1M elements against the same chain evaluated on the host
  std::vector<int32_t> big(1 << 20);
  oracle_gen_uniform_i32(big.data(), (int64_t)big.size(), 58, 1, -1000, 1000);
  std::vector<int32_t> ref;
  for (int32_t v : big)
    if (v % 3 == 0) ref.push_back(v * 2);
  std::vector<int32_t> mid(ref.begin() + 1000, ref.begin() + 6000);
  CHECK(AsComputeQueryable(big, p).Where(x % 3 == 0).Select(x * 2).Skip(1000).Take(5000).ToArray() == mid);
  CHECK(AsComputeQueryable(big, p).Where(x % 3 == 0).Select(x * 2).Last() == ref.back());
}

TEST_GPU(linq_aggregate_folds) {
  auto acc = Param(0), x = Param(1), e = Param();
  auto p = std::make_shared<ComputeQueryProvider>(Gpu());
  const auto r100 = Range(1, 100);
  CHECK(AsComputeQueryable(r100, p).Aggregate(acc + x) == 5050);
  CHECK(AsComputeQueryable(r100, p).Aggregate(x + acc) == 5050);
  CHECK(AsComputeQueryable(r100, p).Aggregate(1000, acc + x) == 6050);
  CHECK(AsComputeQueryable(r100, p).Where(e % 2 == 1).Aggregate(Math::Max(acc, x)) == 99);
  CHECK(AsComputeQueryable(r100, p).Aggregate(-5, Math::Min(acc, x)) == -5);
  std::vector<int32_t> w{INT32_MAX, 1};
  CHECK(AsComputeQueryable(w, p).Aggregate(acc + x) == INT32_MIN);  // unchecked: wraps, no exception
  std::vector<int32_t> none;
  CHECK_THROWS(InvalidOperationException, AsComputeQueryable(none, p).Aggregate(acc + x));
  CHECK(AsComputeQueryable(none, p).Aggregate(7, acc + x) == 7);
  std::vector<float> f{1.0f, 2.0f};
  CHECK_THROWS(NotSupportedException, AsComputeQueryable(f, p).Aggregate(acc + x));  // order of float roundings
  CHECK_THROWS(NotSupportedException, AsComputeQueryable(r100, p).Aggregate(acc * x));
}

TEST_GPU(linq_float_aggregate_min_max_folds) {
  // Aggregate((acc, x) => MathF.Min(acc, x)) / MathF.Max: NaN if any element is NaN, -0 below +0
  // (unlike Enumerable.Min/Max, which skip NaNs in Max and take the first of equal zeros).
  auto acc = Param(0), x = Param(1), e = Param();
  auto p = std::make_shared<ComputeQueryProvider>(Gpu());
  auto bits = [](float v) {
    uint32_t b;
    std::memcpy(&b, &v, 4);
    return b;
  };
  std::vector<float> z{0.0f, 3.0f, -0.0f, 2.0f};
  CHECK(bits(AsComputeQueryable(z, p).Aggregate(MathF::Min(acc, x))) == bits(-0.0f));
  CHECK(bits(AsComputeQueryable(z, p).Where(e < 1.0f).Aggregate(MathF::Max(x, acc))) == bits(0.0f));
  CHECK(bits(AsComputeQueryable(z, p).Where(e < 1.0f).Max()) == bits(0.0f));  // the first of the zeros
  CHECK(bits(AsComputeQueryable(z, p).Where(e < 1.0f).Min()) == bits(0.0f));
  std::vector<float> n{1.0f, NAN, 5.0f};
  CHECK(std::isnan(AsComputeQueryable(n, p).Aggregate(MathF::Max(acc, x))));
  CHECK(AsComputeQueryable(n, p).Max() == 5.0f);  // Enumerable.Max skips the NaN
  CHECK(std::isnan(AsComputeQueryable(n, p).Aggregate(-7.0f, MathF::Min(acc, x))));  // the seed does not hide it
  std::vector<float> v = Uniform(500000, 31, 0);
  float mn = v[0], mx = v[0];
  for (float t : v) {
    mn = std::min(mn, t);
    mx = std::max(mx, t);
  }
  CHECK(AsComputeQueryable(v, p).Aggregate(MathF::Min(acc, x)) == mn);
  CHECK(AsComputeQueryable(v, p).Aggregate(MathF::Max(acc, x)) == mx);
  CHECK(AsComputeQueryable(v, p).Aggregate(100.0f, MathF::Min(acc, x)) == mn);
  CHECK(AsComputeQueryable(v, p).Aggregate(100.0f, MathF::Max(acc, x)) == 100.0f);
  std::vector<float> none;
  CHECK_THROWS(InvalidOperationException, AsComputeQueryable(none, p).Aggregate(MathF::Min(acc, x)));
  CHECK(AsComputeQueryable(none, p).Aggregate(2.5f, MathF::Max(acc, x)) == 2.5f);
  CHECK_THROWS(NotSupportedException, AsComputeQueryable(v, p).Aggregate(acc * x));
}

TEST_GPU(linq_min_max_match_enumerable) {
  auto x = Param();
  auto p = std::make_shared<ComputeQueryProvider>(Gpu());
  auto src = Uniform(500000, 31, 0);
  src[1234] = -0.0f;  // ties between signed zeros go to the earlier element
  src[4321] = 0.0f;
  auto q = AsComputeQueryable(src, p).Where(x < 0.75f).Select(x * 2.0f + 1.0f);
  float mn = 0, mx = 0;
  const FusedKernelPlan pmin = q.Explain(Terminal::Min), pmax = q.Explain(Terminal::Max);
  CHECK(oracle_linq_where_select_min(&pmin.Program, src.data(), (int64_t)src.size(), &mn) > 0);
  CHECK(oracle_linq_where_select_max(&pmax.Program, src.data(), (int64_t)src.size(), &mx) > 0);
  const float gmn = q.Min(), gmx = q.Max();
  CHECK(std::memcmp(&gmn, &mn, 4) == 0 && std::memcmp(&gmx, &mx, 4) == 0);
  std::vector<float> with_nan = src;
  with_nan[77777] = NAN;
  auto qn = AsComputeQueryable(with_nan, p).Select(x * 1.0f);
  CHECK(std::isnan(qn.Min()));   // Enumerable.Min: NaN is the smallest value
  CHECK(!std::isnan(qn.Max()));  // Enumerable.Max: NaNs are skipped
}

TEST_GPU(linq_benchmark_chain_bit_exact_vs_linq_to_objects) {
  auto x = Param();
  auto p = std::make_shared<ComputeQueryProvider>(Gpu());
  const size_t n = 1 << 20;
  auto src = Uniform(n, 44, 0);
  std::vector<float> ref(n);
  ref.resize((size_t)oracle_where_gt0_select_2x_plus_1(src.data(), (int64_t)n, ref.data()));
  auto q = AsComputeQueryable(src, p).Where(x > 0.0f).Select(x * 2.0f + 1.0f);
  CHECK(BitsEqual(q.ToArray(), ref));
  int64_t cnt = 0;
  double seq = 0.0;
  float fref = oracle_where_gt0_select_2x_plus_1_sum(src.data(), (int64_t)n, &cnt, &seq);
  const float got = q.Sum();
  CHECK(std::fabs(got - fref) <= 1e-5 * 20 * std::fabs(seq));
  CHECK(q.LongCount() == cnt);
}

TEST_GPU(linq_device_resident_source) {
  auto x = Param();
  auto acc = Gpu();
  auto p = std::make_shared<ComputeQueryProvider>(acc);
  auto src = Uniform(300000, 9, 0);
  auto dsrc = acc->Memory().AllocateAsync<float>(src.size());
  dsrc->CopyFromAsync(src).get();
  std::vector<float> ref(src.size());
  ref.resize((size_t)oracle_where_gt0_select_2x_plus_1(src.data(), (int64_t)src.size(), ref.data()));
  CHECK(BitsEqual(AsComputeQueryable(*dsrc, p).Where(x > 0.0f).Select(x * 2.0f + 1.0f).ToArray(), ref));
}

TEST_GPU(linq_general_lambdas_match_tree_evaluation) {
  auto x = Param();
  auto p = std::make_shared<ComputeQueryProvider>(Gpu());
  auto src = Uniform(200000, 21, 0);
  struct Case {
    Expr w, s;
  };
  std::vector<Case> cases = {
      {x > 0.0f && x < 0.5f, (x + 1.0f) * (x - 1.0f)},
      {(x < -0.5f || x > 0.5f) && (x != 0.75f || x * x > 0.9f), MathF::Abs(x) - 0.25f},
      {!(x >= 0.0f), MathF::Sqrt(-x) / (x - 2.0f)},
      {x * x + x > 0.1f, MathF::Min(x, 0.25f) + MathF::Max(x * 3.0f, -1.0f)},
  };
  for (const Case& c : cases) {
    std::vector<float> ref;
    for (float v : src)
      if (EvalPred(c.w.Node(), v)) ref.push_back(EvalValue(c.s.Node(), v));
    CHECK(BitsEqual(AsComputeQueryable(src, p).Where(c.w).Select(c.s).ToArray(), ref));
  }
}

TEST_GPU(linq_pow_lambdas_within_two_ulp) {
  // MathF.Pow is the C runtime's powf on the CPU and the device library's on the GPU, each within
  // 1 ulp of the exact value: same kept elements (the predicate has no Pow), values within 2 ulp.
  auto x = Param();
  auto p = std::make_shared<ComputeQueryProvider>(Gpu());
  auto src = Uniform(300000, 25, 0);
  // (x + 2)^x (both operands computed: the exponent goes through a save register) and 0.5^x: one
  // Pow each, all results positive, so the ulp distance is the difference of the bit patterns.
  for (const Expr& sel : {MathF::Pow(x + 2.0f, x), MathF::Pow(0.5f, x)}) {
    std::vector<float> ref;
    for (float v : src)
      if (v > -0.75f) ref.push_back(EvalValue(sel.Node(), v));
    const std::vector<float> got = AsComputeQueryable(src, p).Where(x > -0.75f).Select(sel).ToArray();
    CHECK(got.size() == ref.size());
    int64_t worst = 0;
    for (size_t k = 0; k < std::min(got.size(), ref.size()); ++k) {
      int32_t a, b;
      std::memcpy(&a, &got[k], 4);
      std::memcpy(&b, &ref[k], 4);
      worst = std::max<int64_t>(worst, std::llabs((int64_t)a - (int64_t)b));
    }
    CHECK(worst <= 2);
    const double sum = AsComputeQueryable(src, p).Where(x > -0.75f).Select(sel).Sum();
    double ref_sum = 0.0;
    for (float v : ref) ref_sum += v;
    CHECK(std::fabs(sum - ref_sum) <= 1e-5 * std::fabs(ref_sum));
  }
}

// ============================== GPU: algorithms ====================================================

TEST_GPU(matrix_multiply_matches_float64_reference) {
  auto acc = Gpu();
  const int m = 512, k = 384, n = 768;
  Matrix a(m, k, Uniform((size_t)m * k, 42)), b(k, n, Uniform((size_t)k * n, 43));
  Matrix c = MatrixOperations::MultiplyAsync(a, b, *acc).get();
  std::vector<int64_t> rows(m);
  for (int i = 0; i < m; ++i) rows[i] = i;
  std::vector<double> ref((size_t)m * n), absref((size_t)m * n);
  oracle_gemm_f64_rows(a.Data().data(), b.Data().data(), ref.data(), absref.data(), m, n, k, rows.data(), m, 8);
  for (size_t i = 0; i < ref.size(); ++i) CHECK(std::fabs(c.Data()[i] - ref[i]) <= 1e-4 * absref[i]);
  Matrix bad(k + 1, n);
  CHECK_THROWS(ArgumentException, MatrixOperations::MultiplyAsync(a, bad, *acc).get());
  Matrix cb = MatrixOperations::MultiplyAsync(a, b, *acc, Algorithms::MatMulPrecision::BFloat16).get();
  double num = 0, den = 0;
  for (size_t i = 0; i < ref.size(); ++i) {
    num += (cb.Data()[i] - ref[i]) * (cb.Data()[i] - ref[i]);
    den += ref[i] * ref[i];
  }
  CHECK(std::sqrt(num / den) < 1e-2);  // bf16 inputs vs fp32 inputs: ~2^-9 relative input rounding
}

TEST_GPU(sparse_spmv_and_power_iteration) {
  auto acc = Gpu();
  const int64_t rows = 200000;
  std::vector<int32_t> rp(rows + 1);
  int64_t nnz = oracle_gen_zipf_rowptr(rows, 2.0, 4096, 42, rp.data());
  std::vector<int32_t> col((size_t)nnz);
  std::vector<float> val((size_t)nnz);
  oracle_gen_zipf_fill(rows, rows, 42, rp.data(), col.data(), val.data());
  CsrMatrix<float> A((int32_t)rows, (int32_t)rows, val, col, rp);
  auto x = Uniform((size_t)rows, 42, 5, 1);
  std::vector<float> y = SparseOps::SpMV(A, x, *acc);
  std::vector<double> x64(x.begin(), x.end()), y64((size_t)rows), scale((size_t)rows);
  oracle_spmv_csr_f64(rp.data(), col.data(), val.data(), x64.data(), y64.data(), rows);
  for (int64_t r = 0; r < rows; ++r) CHECK(std::fabs(y[r] - y64[r]) <= 1e-4 * std::fabs(y64[r]) + 1e-30);
  std::vector<float> wrong((size_t)rows + 1);
  CHECK_THROWS(ArgumentException, SparseOps::SpMV(A, wrong, *acc));
  double s = 0.0;
  std::vector<float> xp = SparseOps::PowerIterate(A, x, 20, *acc, &s);
  std::vector<float> xo = x, yo((size_t)rows);
  double so = 0.0;
  oracle_spmv_power_f32(rp.data(), col.data(), val.data(), xo.data(), yo.data(), rows, 20, &so);
  CHECK(std::fabs(s - so) <= 1e-4 * std::fabs(so));
  for (int64_t r = 0; r < rows; ++r) CHECK(std::fabs(xp[r] - xo[r]) <= 1e-4 * std::fabs(xo[r]) + 1e-12);
}

TEST_GPU(sparse_spmv_double_and_int) {
  auto acc = Gpu();
  const int64_t rows = 50000;
  std::vector<int32_t> rp(rows + 1);
  int64_t nnz = oracle_gen_zipf_rowptr(rows, 2.0, 4096, 43, rp.data());
  std::vector<int32_t> col((size_t)nnz);
  std::vector<float> valf((size_t)nnz);
  oracle_gen_zipf_fill(rows, rows, 43, rp.data(), col.data(), valf.data());
  // double: rows up to 512 nonzeros are summed in index order, longer ones by a fixed tree
  std::vector<double> vd((size_t)nnz), xd((size_t)rows), yd((size_t)rows), sd((size_t)rows);
  for (int64_t i = 0; i < nnz; ++i) vd[(size_t)i] = (double)valf[(size_t)i] * 3.0 - 0.5;
  for (int64_t r = 0; r < rows; ++r) xd[(size_t)r] = 1.0 / (double)(r + 3);
  CsrMatrix<double> Ad((int32_t)rows, (int32_t)rows, vd, col, rp);
  std::vector<double> got_d = SparseOps::SpMV(Ad, xd, *acc);
  CHECK(oracle_spmv_csr_f64d(rp.data(), col.data(), vd.data(), xd.data(), yd.data(), rows, rows, rows) == 0);
  std::vector<double> avd(vd.size());
  for (size_t i = 0; i < vd.size(); ++i) avd[i] = std::fabs(vd[i]);
  CHECK(oracle_spmv_csr_f64d(rp.data(), col.data(), avd.data(), xd.data(), sd.data(), rows, rows, rows) == 0);
  for (int64_t r = 0; r < rows; ++r) {
    if (rp[r + 1] - rp[r] <= 512)
      CHECK(got_d[(size_t)r] == yd[(size_t)r]);
    else
      CHECK(std::fabs(got_d[(size_t)r] - yd[(size_t)r]) <= 1e-12 * sd[(size_t)r]);
  }
  // int: wrapping products and sums, bit-identical on every row
  std::vector<int32_t> vi((size_t)nnz), xi((size_t)rows), yi((size_t)rows);
  for (int64_t i = 0; i < nnz; ++i) vi[(size_t)i] = (int32_t)(0x9E3779B1u * (uint32_t)(i + 1));
  for (int64_t r = 0; r < rows; ++r) xi[(size_t)r] = (int32_t)(r % 70001) - 35000;
  CsrMatrix<int32_t> Ai((int32_t)rows, (int32_t)rows, vi, col, rp);
  std::vector<int32_t> got_i = SparseOps::SpMV(Ai, xi, *acc);
  CHECK(oracle_spmv_csr_i32(rp.data(), col.data(), vi.data(), xi.data(), yi.data(), rows, rows, rows) == 0);
  CHECK(got_i == yi);
  std::vector<int32_t> wrong((size_t)rows - 1);
  CHECK_THROWS(ArgumentException, SparseOps::SpMV(Ai, wrong, *acc));
}

int main(int argc, char** argv) { return dctest_main(argc, argv); }

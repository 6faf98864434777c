// Linq.cpp — expression DSL, visitor, fusion planner (register-program code generator), executor
// and queryable of the HIP LINQ provider.
#include "DotCompute/Linq.hpp"

#include <limits>
#include <mutex>
#include <sstream>

namespace DotCompute::Linq {

using Backends::Hip::Check;

// ---- expression DSL -------------------------------------------------------------------------------

namespace {
std::shared_ptr<const ExprNode> MakeNode(ExprKind k, std::shared_ptr<const ExprNode> l = nullptr,
                                     std::shared_ptr<const ExprNode> r = nullptr, float v = 0.0f) {
  auto n = std::make_shared<ExprNode>();
  n->Kind = k;
  n->Value = v;
  n->Left = std::move(l);
  n->Right = std::move(r);
  return n;
}
bool IsConst(const Expr& e) { return e.Node().Kind == ExprKind::Constant; }

// Binary arithmetic with constant folding of constant operands (the C# compiler folds constant
// sub-expressions of a lambda before building its expression tree), each fold rounding to float.
Expr Arith(ExprKind k, const Expr& a, const Expr& b) {
  if (IsConst(a) && IsConst(b)) {
    const float x = a.Node().Value, y = b.Node().Value;
    switch (k) {
      case ExprKind::Add: return Expr(x + y);
      case ExprKind::Subtract: return Expr(x - y);
      case ExprKind::Multiply: return Expr(x * y);
      case ExprKind::Divide: return Expr(x / y);
      default: break;
    }
  }
  return Expr(MakeNode(k, a.Ptr(), b.Ptr()));
}
bool IsCompareKind(ExprKind k) { return k >= ExprKind::GreaterThan && k <= ExprKind::NotEqual; }
bool IsPredicateKind(ExprKind k) { return IsCompareKind(k) || k == ExprKind::AndAlso || k == ExprKind::OrElse || k == ExprKind::Not; }
}  // namespace

Expr::Expr(float constant) : node_(MakeNode(ExprKind::Constant, nullptr, nullptr, constant)) {}
Expr Expr::Parameter() { return Expr(MakeNode(ExprKind::Parameter)); }
bool Expr::IsPredicate() const { return IsPredicateKind(node_->Kind); }

std::string Expr::ToString() const {
  const ExprNode& n = *node_;
  auto L = [&] { return Expr(n.Left).ToString(); };
  auto R = [&] { return Expr(n.Right).ToString(); };
  std::ostringstream os;
  switch (n.Kind) {
    case ExprKind::Parameter: return "x";
    case ExprKind::Constant: os << n.Value << "f"; return os.str();
    case ExprKind::Negate: return "-(" + L() + ")";
    case ExprKind::Abs: return "MathF.Abs(" + L() + ")";
    case ExprKind::Sqrt: return "MathF.Sqrt(" + L() + ")";
    case ExprKind::Add: return "(" + L() + " + " + R() + ")";
    case ExprKind::Subtract: return "(" + L() + " - " + R() + ")";
    case ExprKind::Multiply: return "(" + L() + " * " + R() + ")";
    case ExprKind::Divide: return "(" + L() + " / " + R() + ")";
    case ExprKind::Min: return "MathF.Min(" + L() + ", " + R() + ")";
    case ExprKind::Max: return "MathF.Max(" + L() + ", " + R() + ")";
    case ExprKind::GreaterThan: return "(" + L() + " > " + R() + ")";
    case ExprKind::GreaterThanOrEqual: return "(" + L() + " >= " + R() + ")";
    case ExprKind::LessThan: return "(" + L() + " < " + R() + ")";
    case ExprKind::LessThanOrEqual: return "(" + L() + " <= " + R() + ")";
    case ExprKind::Equal: return "(" + L() + " == " + R() + ")";
    case ExprKind::NotEqual: return "(" + L() + " != " + R() + ")";
    case ExprKind::AndAlso: return "(" + L() + " && " + R() + ")";
    case ExprKind::OrElse: return "(" + L() + " || " + R() + ")";
    case ExprKind::Not: return "!(" + L() + ")";
  }
  return "?";
}

Expr operator+(const Expr& a, const Expr& b) { return Arith(ExprKind::Add, a, b); }
Expr operator-(const Expr& a, const Expr& b) { return Arith(ExprKind::Subtract, a, b); }
Expr operator*(const Expr& a, const Expr& b) { return Arith(ExprKind::Multiply, a, b); }
Expr operator/(const Expr& a, const Expr& b) { return Arith(ExprKind::Divide, a, b); }
Expr operator-(const Expr& a) { return IsConst(a) ? Expr(-a.Node().Value) : Expr(MakeNode(ExprKind::Negate, a.Ptr())); }
Expr operator>(const Expr& a, const Expr& b) { return Expr(MakeNode(ExprKind::GreaterThan, a.Ptr(), b.Ptr())); }
Expr operator>=(const Expr& a, const Expr& b) { return Expr(MakeNode(ExprKind::GreaterThanOrEqual, a.Ptr(), b.Ptr())); }
Expr operator<(const Expr& a, const Expr& b) { return Expr(MakeNode(ExprKind::LessThan, a.Ptr(), b.Ptr())); }
Expr operator<=(const Expr& a, const Expr& b) { return Expr(MakeNode(ExprKind::LessThanOrEqual, a.Ptr(), b.Ptr())); }
Expr operator==(const Expr& a, const Expr& b) { return Expr(MakeNode(ExprKind::Equal, a.Ptr(), b.Ptr())); }
Expr operator!=(const Expr& a, const Expr& b) { return Expr(MakeNode(ExprKind::NotEqual, a.Ptr(), b.Ptr())); }
Expr operator&&(const Expr& a, const Expr& b) { return Expr(MakeNode(ExprKind::AndAlso, a.Ptr(), b.Ptr())); }
Expr operator||(const Expr& a, const Expr& b) { return Expr(MakeNode(ExprKind::OrElse, a.Ptr(), b.Ptr())); }
Expr operator!(const Expr& a) { return Expr(MakeNode(ExprKind::Not, a.Ptr())); }

namespace MathF {
Expr Abs(const Expr& a) { return Expr(MakeNode(ExprKind::Abs, a.Ptr())); }
Expr Sqrt(const Expr& a) { return Expr(MakeNode(ExprKind::Sqrt, a.Ptr())); }
Expr Min(const Expr& a, const Expr& b) { return Expr(MakeNode(ExprKind::Min, a.Ptr(), b.Ptr())); }
Expr Max(const Expr& a, const Expr& b) { return Expr(MakeNode(ExprKind::Max, a.Ptr(), b.Ptr())); }
}  // namespace MathF

// ---- visitor ---------------------------------------------------------------------------------------

std::optional<OperationType> ExpressionTreeVisitor::MapMethodToOperationType(const std::string& m) {
  if (m == "Select" || m == "Cast") return OperationType::Map;
  if (m == "Where" || m == "OfType" || m == "Take" || m == "Skip" || m == "First" || m == "FirstOrDefault" ||
      m == "Last" || m == "LastOrDefault" || m == "Single" || m == "SingleOrDefault")
    return OperationType::Filter;
  if (m == "Aggregate" || m == "Sum" || m == "Count" || m == "LongCount" || m == "Average" || m == "Min" || m == "Max" ||
      m == "Any" || m == "All")
    return OperationType::Reduce;
  if (m == "TakeWhile" || m == "SkipWhile") return OperationType::Scan;
  if (m == "Join" || m == "GroupJoin") return OperationType::Join;
  if (m == "GroupBy") return OperationType::GroupBy;
  if (m == "OrderBy" || m == "OrderByDescending" || m == "ThenBy" || m == "ThenByDescending") return OperationType::OrderBy;
  if (m == "Distinct" || m == "Union" || m == "Intersect" || m == "Except") return OperationType::Aggregate;
  return std::nullopt;
}

OperationGraph ExpressionTreeVisitor::Visit(const std::vector<MethodCall>& chain) const {
  OperationGraph g;
  for (size_t i = 0; i < chain.size(); ++i) {
    auto t = MapMethodToOperationType(chain[i].Method);
    if (!t) throw NotSupportedException("LINQ method '" + chain[i].Method + "' is not supported by the compute provider");
    Operation op;
    op.Id = "op_" + std::to_string(i);
    op.Type = *t;
    op.Method = chain[i].Method;
    op.Lambda = chain[i].Lambda;
    if (i > 0) op.Dependencies.push_back("op_" + std::to_string(i - 1));
    g.Operations.push_back(std::move(op));
  }
  return g;
}

// ---- backend selection -----------------------------------------------------------------------------

ComputeBackend BackendSelector::SelectBackend(const WorkloadCharacteristics&) const {
  if (!hip_available_)
    throw InvalidOperationException("No HIP accelerator is available for the compute query (the HIP backend needs a "
                                    "gfx950 device; this build has no host fallback).");
  return ComputeBackend::Hip;
}

// ---- fusion planner / code generator ---------------------------------------------------------------

namespace {

constexpr int kSaveRegisters = 2;

dc_linq_instr Instr(uint8_t op, uint8_t src = DC_LQ_SRC_IMM, float imm = 0.0f, uint8_t mode = DC_LQ_CMP_SET) {
  dc_linq_instr i;
  i.op = op;
  i.src = src;
  i.mode = mode;
  i.pad = 0;
  i.imm = imm;
  return i;
}

bool IsLeaf(const ExprNode& n) { return n.Kind == ExprKind::Parameter || n.Kind == ExprKind::Constant; }

// Whether `op(left, right)` should be emitted as "compute left; op right": yes when the right side
// is a leaf, unless it is the parameter and the left side a constant — then the swapped form
// keeps the constant as the immediate (`0.5f < x` -> CMP_GT 0.5, `2f - x` -> RSUB 2).
bool RightIsOperand(const ExprNode& n) {
  if (!IsLeaf(*n.Right)) return false;
  return !(n.Right->Kind == ExprKind::Parameter && n.Left->Kind == ExprKind::Constant);
}

// Operand source for a leaf: the element itself, or an immediate.
std::pair<uint8_t, float> LeafSource(const ExprNode& n) {
  return n.Kind == ExprKind::Parameter ? std::make_pair((uint8_t)DC_LQ_SRC_ELEM, 0.0f)
                                       : std::make_pair((uint8_t)DC_LQ_SRC_IMM, n.Value);
}

uint8_t ArithOp(ExprKind k) {
  switch (k) {
    case ExprKind::Add: return DC_LQ_ADD;
    case ExprKind::Subtract: return DC_LQ_SUB;
    case ExprKind::Multiply: return DC_LQ_MUL;
    case ExprKind::Divide: return DC_LQ_DIV;
    case ExprKind::Min: return DC_LQ_MIN;
    case ExprKind::Max: return DC_LQ_MAX;
    default: throw NotSupportedException("not an arithmetic node");
  }
}

// Operation with its operands swapped (v = operand OP v): exact for +, *, min, max (IEEE + and *
// commute; MathF.Min/Max are symmetric), and via RSUB/RDIV for - and /.
uint8_t ReversedArithOp(ExprKind k) {
  switch (k) {
    case ExprKind::Add: return DC_LQ_ADD;
    case ExprKind::Multiply: return DC_LQ_MUL;
    case ExprKind::Min: return DC_LQ_MIN;
    case ExprKind::Max: return DC_LQ_MAX;
    case ExprKind::Subtract: return DC_LQ_RSUB;
    case ExprKind::Divide: return DC_LQ_RDIV;
    default: throw NotSupportedException("not an arithmetic node");
  }
}

uint8_t CompareOp(ExprKind k, bool swapped) {
  switch (k) {
    case ExprKind::GreaterThan: return swapped ? DC_LQ_CMP_LT : DC_LQ_CMP_GT;
    case ExprKind::GreaterThanOrEqual: return swapped ? DC_LQ_CMP_LE : DC_LQ_CMP_GE;
    case ExprKind::LessThan: return swapped ? DC_LQ_CMP_GT : DC_LQ_CMP_LT;
    case ExprKind::LessThanOrEqual: return swapped ? DC_LQ_CMP_GE : DC_LQ_CMP_LE;
    case ExprKind::Equal: return DC_LQ_CMP_EQ;
    case ExprKind::NotEqual: return DC_LQ_CMP_NE;
    default: throw NotSupportedException("not a comparison node");
  }
}

struct Compiler {
  std::vector<dc_linq_instr>& code;

  void Emit(const dc_linq_instr& i) {
    if (code.size() >= (size_t)DC_LINQ_MAX_INSTR)
      throw NotSupportedException("the fused chain needs more than " + std::to_string(DC_LINQ_MAX_INSTR) +
                                  " instructions");
    code.push_back(i);
  }

  // Leaves the value of `n` in v. Saved registers with index >= `free_save` may be used.
  void Value(const ExprNode& n, int free_save) {
    switch (n.Kind) {
      case ExprKind::Parameter: Emit(Instr(DC_LQ_LOAD, DC_LQ_SRC_ELEM)); return;
      case ExprKind::Constant: Emit(Instr(DC_LQ_LOAD, DC_LQ_SRC_IMM, n.Value)); return;
      case ExprKind::Negate: Value(*n.Left, free_save); Emit(Instr(DC_LQ_NEG)); return;
      case ExprKind::Abs: Value(*n.Left, free_save); Emit(Instr(DC_LQ_ABS)); return;
      case ExprKind::Sqrt: Value(*n.Left, free_save); Emit(Instr(DC_LQ_SQRT)); return;
      case ExprKind::Add:
      case ExprKind::Subtract:
      case ExprKind::Multiply:
      case ExprKind::Divide:
      case ExprKind::Min:
      case ExprKind::Max: {
        if (RightIsOperand(n)) {
          Value(*n.Left, free_save);
          auto [src, imm] = LeafSource(*n.Right);
          Emit(Instr(ArithOp(n.Kind), src, imm));
        } else if (IsLeaf(*n.Left)) {
          Value(*n.Right, free_save);
          auto [src, imm] = LeafSource(*n.Left);
          Emit(Instr(ReversedArithOp(n.Kind), src, imm));
        } else {
          const int s = Save(free_save);
          Value(*n.Right, free_save);
          Emit(Instr(s == 0 ? DC_LQ_STORE_S0 : DC_LQ_STORE_S1));
          Value(*n.Left, free_save + 1);
          Emit(Instr(ArithOp(n.Kind), s == 0 ? DC_LQ_SRC_S0 : DC_LQ_SRC_S1));
        }
        return;
      }
      default:
        throw NotSupportedException("a boolean expression cannot be used as a float value in the HIP kernels");
    }
  }

  int Save(int free_save) {
    if (free_save >= kSaveRegisters)
      throw NotSupportedException("lambda is too deeply nested for the fused HIP kernel (more than " +
                                  std::to_string(kSaveRegisters) + " intermediate values)");
    return free_save;
  }

  static bool UsesQ(const ExprNode& n) {
    if (n.Kind == ExprKind::Not) return UsesQ(*n.Left);
    if (n.Kind != ExprKind::AndAlso && n.Kind != ExprKind::OrElse) return false;
    const bool ls = IsCompareKind(n.Left->Kind), rs = IsCompareKind(n.Right->Kind);
    if (ls || rs) return UsesQ(ls ? *n.Right : *n.Left);
    return true;
  }

  // Leaves the predicate in p, combined with the incoming p by `mode` (SET / AND / OR). Only
  // comparisons are emitted with AND/OR; composite predicates always start with SET.
  void Predicate(const ExprNode& n, uint8_t mode, bool q_busy) {
    if (IsCompareKind(n.Kind)) {
      if (RightIsOperand(n)) {
        Value(*n.Left, 0);
        auto [src, imm] = LeafSource(*n.Right);
        Emit(Instr(CompareOp(n.Kind, false), src, imm, mode));
      } else if (IsLeaf(*n.Left)) {
        Value(*n.Right, 0);
        auto [src, imm] = LeafSource(*n.Left);
        Emit(Instr(CompareOp(n.Kind, true), src, imm, mode));
      } else {
        Value(*n.Right, 0);
        Emit(Instr(DC_LQ_STORE_S0));
        Value(*n.Left, 1);
        Emit(Instr(CompareOp(n.Kind, false), DC_LQ_SRC_S0, 0.0f, mode));
      }
      return;
    }
    if (mode != DC_LQ_CMP_SET) throw NotSupportedException("internal: composite predicate combined with a mode");
    switch (n.Kind) {
      case ExprKind::Not:
        Predicate(*n.Left, DC_LQ_CMP_SET, q_busy);
        Emit(Instr(DC_LQ_PNOT));
        return;
      case ExprKind::AndAlso:
      case ExprKind::OrElse: {
        const uint8_t combine = n.Kind == ExprKind::AndAlso ? DC_LQ_CMP_AND : DC_LQ_CMP_OR;
        // Both sides are side-effect free, so they may be evaluated in either order.
        if (IsCompareKind(n.Right->Kind)) {
          Predicate(*n.Left, DC_LQ_CMP_SET, q_busy);
          Predicate(*n.Right, combine, q_busy);
        } else if (IsCompareKind(n.Left->Kind)) {
          Predicate(*n.Right, DC_LQ_CMP_SET, q_busy);
          Predicate(*n.Left, combine, q_busy);
        } else {
          if (q_busy || UsesQ(*n.Right))
            throw NotSupportedException("predicate combines too many composite conditions for the fused HIP kernel");
          Predicate(*n.Left, DC_LQ_CMP_SET, q_busy);
          Emit(Instr(DC_LQ_PSTORE));
          Predicate(*n.Right, DC_LQ_CMP_SET, true);
          Emit(Instr(n.Kind == ExprKind::AndAlso ? DC_LQ_PAND_Q : DC_LQ_POR_Q));
        }
        return;
      }
      default:
        throw NotSupportedException("Where() needs a boolean lambda");
    }
  }
};

const char* OpName(uint8_t op) {
  switch (op) {
    case DC_LQ_NOP: return "NOP";
    case DC_LQ_LOAD: return "LOAD";
    case DC_LQ_ADD: return "ADD";
    case DC_LQ_SUB: return "SUB";
    case DC_LQ_RSUB: return "RSUB";
    case DC_LQ_MUL: return "MUL";
    case DC_LQ_DIV: return "DIV";
    case DC_LQ_RDIV: return "RDIV";
    case DC_LQ_MIN: return "MIN";
    case DC_LQ_MAX: return "MAX";
    case DC_LQ_NEG: return "NEG";
    case DC_LQ_ABS: return "ABS";
    case DC_LQ_SQRT: return "SQRT";
    case DC_LQ_STORE_S0: return "STORE_S0";
    case DC_LQ_STORE_S1: return "STORE_S1";
    case DC_LQ_CMP_GT: return "CMP_GT";
    case DC_LQ_CMP_GE: return "CMP_GE";
    case DC_LQ_CMP_LT: return "CMP_LT";
    case DC_LQ_CMP_LE: return "CMP_LE";
    case DC_LQ_CMP_EQ: return "CMP_EQ";
    case DC_LQ_CMP_NE: return "CMP_NE";
    case DC_LQ_PNOT: return "PNOT";
    case DC_LQ_PSTORE: return "PSTORE";
    case DC_LQ_PAND_Q: return "PAND_Q";
    case DC_LQ_POR_Q: return "POR_Q";
    case DC_LQ_FILTER: return "FILTER";
    case DC_LQ_MAP: return "MAP";
  }
  return "?";
}

}  // namespace

void HipKernelGenerator::CompileLambda(const Expr& lambda, bool predicate, std::vector<dc_linq_instr>& code) {
  Compiler c{code};
  if (predicate) {
    if (!lambda.IsPredicate()) throw NotSupportedException("Where() needs a boolean lambda");
    c.Predicate(lambda.Node(), DC_LQ_CMP_SET, false);
  } else {
    if (lambda.IsPredicate()) throw NotSupportedException("Select() to bool is not supported by the float32 HIP kernels");
    c.Value(lambda.Node(), 0);
  }
}

bool HipKernelGenerator::CanBeFused(const Operation& op) {
  return op.Type == OperationType::Map || op.Type == OperationType::Filter;
}

std::vector<const Operation*> HipKernelGenerator::IdentifyFusableOperations(const OperationGraph& graph) {
  std::vector<const Operation*> out;
  for (const Operation& op : graph.Operations) {
    if (!CanBeFused(op)) break;  // Map->Map, Map->Filter, Filter->Map, Filter->Filter fuse
    out.push_back(&op);
  }
  return out;
}

FusedKernelPlan HipKernelGenerator::GenerateHipKernel(const OperationGraph& graph) const {
  FusedKernelPlan plan;
  const auto fused = IdentifyFusableOperations(graph);
  std::vector<dc_linq_instr> code;
  for (const Operation* op : fused) {
    if (op->Method != "Where" && op->Method != "Select")
      throw NotSupportedException("LINQ method '" + op->Method + "' has no HIP kernel");
    if (!op->Lambda) throw ArgumentNullException(op->Method + " needs a lambda");
    const bool is_filter = op->Type == OperationType::Filter;
    CompileLambda(*op->Lambda, is_filter, code);
    if (code.size() >= (size_t)DC_LINQ_MAX_INSTR) throw NotSupportedException("fused chain too long");
    code.push_back(Instr(is_filter ? DC_LQ_FILTER : DC_LQ_MAP));
    plan.FusedOperationIds.push_back(op->Id);
  }
  const size_t rest = graph.Operations.size() - fused.size();
  if (rest > 1) throw NotSupportedException("only one terminal operator may follow the fused Where/Select chain");
  if (rest == 1) {
    const Operation& term = graph.Operations.back();
    if (term.Type != OperationType::Reduce)
      throw NotSupportedException("LINQ method '" + term.Method + "' (" + std::to_string((int)term.Type) +
                                  ") breaks fusion and has no HIP kernel");
    if (term.Lambda) throw NotSupportedException(term.Method + "(selector) is not supported; use Select(...)." + term.Method + "()");
    if (term.Method == "Sum") plan.Term = Terminal::Sum;
    else if (term.Method == "Count") plan.Term = Terminal::Count;
    else if (term.Method == "LongCount") plan.Term = Terminal::LongCount;
    else if (term.Method == "Average") plan.Term = Terminal::Average;
    else if (term.Method == "Min") plan.Term = Terminal::Min;
    else if (term.Method == "Max") plan.Term = Terminal::Max;
    else throw NotSupportedException("reduction '" + term.Method + "' has no HIP kernel");
    plan.FusedOperationIds.push_back(term.Id);
  }
  plan.Program.n_instr = (int32_t)code.size();
  plan.Program.flags = 0;
  for (size_t i = 0; i < code.size(); ++i) plan.Program.code[i] = code[i];
  Check(dc_linq_chain_validate(&plan.Program), "dc_linq_chain_validate");
  return plan;
}

std::string FusedKernelPlan::Listing() const {
  std::ostringstream os;
  const char* term = Term == Terminal::ToArray ? "ToArray" : Term == Terminal::Sum ? "Sum"
                     : Term == Terminal::Average ? "Average" : Term == Terminal::Min ? "Min"
                     : Term == Terminal::Max ? "Max" : "Count";
  os << "terminal " << term << "\n";
  for (int i = 0; i < Program.n_instr; ++i) {
    const dc_linq_instr& in = Program.code[i];
    os << i << ": " << OpName(in.op);
    if (in.op != DC_LQ_NEG && in.op != DC_LQ_ABS && in.op != DC_LQ_SQRT && in.op != DC_LQ_FILTER && in.op != DC_LQ_MAP &&
        in.op < DC_LQ_PNOT && in.op != DC_LQ_STORE_S0 && in.op != DC_LQ_STORE_S1) {
      if (in.src == DC_LQ_SRC_IMM) os << " " << in.imm;
      else os << (in.src == DC_LQ_SRC_ELEM ? " e" : in.src == DC_LQ_SRC_S0 ? " s0" : " s1");
      if (in.op >= DC_LQ_CMP_GT && in.op <= DC_LQ_CMP_NE && in.mode != DC_LQ_CMP_SET)
        os << (in.mode == DC_LQ_CMP_AND ? " (and)" : " (or)");
    }
    os << "\n";
  }
  return os.str();
}

// ---- executor ----------------------------------------------------------------------------------------

int64_t RuntimeExecutor::ResolveCompactedCount(int64_t k, const std::function<int64_t()>& rerunOrdered) {
  if (k >= 0) return k;
  if (k == -1) {
    const int64_t k2 = rerunOrdered();
    if (k2 >= 0) return k2;
  }
  throw InvalidOperationException(
      "The HIP compaction kernel did not complete: its resident grid could not run all of its workgroups at "
      "once, and the re-run on the ticket-ordered grid reported count " + std::to_string(k) + ".");
}

QueryResult RuntimeExecutor::Run(const FusedKernelPlan& plan, const float* device_in, size_t n) {
  dc_hip_ctx* ctx = acc_->Context();
  QueryResult r;
  auto& mem = acc_->Memory();
  if (plan.Term == Terminal::ToArray) {
    auto out = mem.AllocateAsync<float>(std::max<size_t>(n, 1));
    auto cnt = mem.AllocateAsync<int64_t>(1);
    Check(dc_hip_linq_where_select_f32(ctx, &plan.Program, device_in, (int64_t)n, out->Data(), cnt->Data()),
          "dc_hip_linq_where_select_f32");
    acc_->Synchronize();
    int64_t k = 0;
    cnt->CopyToHost(&k, sizeof(k));
    k = ResolveCompactedCount(k, [&]() {
      dc_linq_chain ordered = plan.Program;
      ordered.flags |= DC_LINQ_FLAG_ORDERED_GRID;
      Check(dc_hip_linq_where_select_f32(ctx, &ordered, device_in, (int64_t)n, out->Data(), cnt->Data()),
            "dc_hip_linq_where_select_f32");
      acc_->Synchronize();
      int64_t k2 = 0;
      cnt->CopyToHost(&k2, sizeof(k2));
      return k2;
    });
    r.Count = k;
    r.Values.resize((size_t)k);
    out->CopyToHost(r.Values.data(), (size_t)k * sizeof(float));  // only the compacted prefix comes back
  } else if (plan.Term == Terminal::Min || plan.Term == Terminal::Max) {
    auto val = mem.AllocateAsync<float>(1);
    auto cnt = mem.AllocateAsync<int64_t>(1);
    Check(dc_hip_linq_where_select_minmax_f32(ctx, &plan.Program, device_in, (int64_t)n,
                                              plan.Term == Terminal::Min ? DC_LINQ_MIN : DC_LINQ_MAX, val->Data(),
                                              cnt->Data()),
          "dc_hip_linq_where_select_minmax_f32");
    acc_->Synchronize();
    val->CopyToHost(&r.Extreme, sizeof(float));
    cnt->CopyToHost(&r.Count, sizeof(int64_t));
  } else {
    auto sum = mem.AllocateAsync<double>(1);
    auto cnt = mem.AllocateAsync<int64_t>(1);
    Check(dc_hip_linq_where_select_sum_f32(ctx, &plan.Program, device_in, (int64_t)n, sum->Data(), cnt->Data()),
          "dc_hip_linq_where_select_sum_f32");
    acc_->Synchronize();
    sum->CopyToHost(&r.Sum, sizeof(double));
    cnt->CopyToHost(&r.Count, sizeof(int64_t));
  }
  return r;
}

QueryResult RuntimeExecutor::Execute(const FusedKernelPlan& plan, const float* data, size_t n) {
  auto in = acc_->Memory().AllocateAsync<float>(std::max<size_t>(n, 1));
  if (n) in->CopyFromHost(data, n * sizeof(float));
  return Run(plan, in->Data(), n);
}

QueryResult RuntimeExecutor::Execute(const FusedKernelPlan& plan, const IUnifiedMemoryBuffer& source, size_t n) {
  if (source.Type() != ElementType::Float32) throw NotSupportedException("the HIP LINQ kernels take float32 sources");
  return Run(plan, static_cast<const float*>(source.DevicePointer()), n);
}

// ---- provider ----------------------------------------------------------------------------------------

ComputeQueryProvider::ComputeQueryProvider() {
  auto acc = Backends::Hip::TryCreateAccelerator();
  if (acc) executor_ = std::make_unique<RuntimeExecutor>(std::move(acc));
}

ComputeQueryProvider::ComputeQueryProvider(std::shared_ptr<Backends::Hip::HipAccelerator> accelerator) {
  if (accelerator) executor_ = std::make_unique<RuntimeExecutor>(std::move(accelerator));
}

std::shared_ptr<ComputeQueryProvider> ComputeQueryProvider::Default() {
  static std::once_flag once;
  static std::shared_ptr<ComputeQueryProvider> provider;
  std::call_once(once, [] { provider = std::make_shared<ComputeQueryProvider>(); });
  return provider;
}

FusedKernelPlan ComputeQueryProvider::Plan(const std::vector<MethodCall>& chain, Terminal terminal, size_t n) const {
  std::vector<MethodCall> full = chain;
  switch (terminal) {
    case Terminal::Sum: full.push_back({"Sum", std::nullopt}); break;
    case Terminal::Count: full.push_back({"Count", std::nullopt}); break;
    case Terminal::LongCount: full.push_back({"LongCount", std::nullopt}); break;
    case Terminal::Average: full.push_back({"Average", std::nullopt}); break;
    case Terminal::Min: full.push_back({"Min", std::nullopt}); break;
    case Terminal::Max: full.push_back({"Max", std::nullopt}); break;
    case Terminal::ToArray: break;
  }
  // Stage 1: expression tree -> operation graph.
  OperationGraph graph = ExpressionTreeVisitor().Visit(full);
  // Stage 2: fused kernel for the graph.
  (void)n;
  return HipKernelGenerator().GenerateHipKernel(graph);
}

QueryResult ComputeQueryProvider::Execute(const std::vector<MethodCall>& chain, Terminal terminal, const float* host,
                                          size_t n, const IUnifiedMemoryBuffer* device) {
  FusedKernelPlan plan = Plan(chain, terminal, n);
  WorkloadCharacteristics w;
  w.DataSize = n;
  w.OperationCount = (int)plan.FusedOperationIds.size();
  w.HasReduction = terminal != Terminal::ToArray;
  BackendSelector(HasAccelerator()).SelectBackend(w);  // throws without a HIP device
  return device ? executor_->Execute(plan, *device, n) : executor_->Execute(plan, host, n);
}

// ---- queryable ----------------------------------------------------------------------------------------

ComputeQueryable::ComputeQueryable(const float* data, size_t n, std::shared_ptr<ComputeQueryProvider> provider)
    : host_(data), n_(n), provider_(std::move(provider)) {
  if (!data && n) throw ArgumentNullException("source");
}

ComputeQueryable::ComputeQueryable(const IUnifiedMemoryBuffer& device, std::shared_ptr<ComputeQueryProvider> provider)
    : device_(&device), n_(device.Length()), provider_(std::move(provider)) {}

ComputeQueryable ComputeQueryable::Where(const Expr& predicate) const {
  ComputeQueryable q = *this;
  q.chain_.push_back({"Where", predicate});
  return q;
}

ComputeQueryable ComputeQueryable::Select(const Expr& selector) const {
  ComputeQueryable q = *this;
  q.chain_.push_back({"Select", selector});
  return q;
}

ComputeQueryable ComputeQueryable::OrderBy(const Expr& key) const {
  ComputeQueryable q = *this;
  q.chain_.push_back({"OrderBy", key});
  return q;
}

QueryResult ComputeQueryable::Run(Terminal t) const { return provider_->Execute(chain_, t, host_, n_, device_); }

FusedKernelPlan ComputeQueryable::Explain(Terminal terminal) const { return provider_->Plan(chain_, terminal, n_); }

std::vector<float> ComputeQueryable::ToArray() const { return Run(Terminal::ToArray).Values; }

float ComputeQueryable::Sum() const { return (float)Run(Terminal::Sum).Sum; }

int64_t ComputeQueryable::LongCount() const { return Run(Terminal::LongCount).Count; }

int32_t ComputeQueryable::Count() const {
  const int64_t c = Run(Terminal::Count).Count;
  if (c > std::numeric_limits<int32_t>::max()) throw OverflowException("Arithmetic operation resulted in an overflow.");
  return (int32_t)c;
}

float ComputeQueryable::Average() const {
  QueryResult r = Run(Terminal::Average);
  if (r.Count == 0) throw InvalidOperationException("Sequence contains no elements");
  return (float)(r.Sum / (double)r.Count);
}

// BCL Enumerable.Min/Max(IEnumerable<float>) semantics (the reference runs these as LINQ-to-objects):
// the device reduction returns the same element bit for bit; an empty sequence throws.
float ComputeQueryable::Min() const {
  QueryResult r = Run(Terminal::Min);
  if (r.Count == 0) throw InvalidOperationException("Sequence contains no elements");
  return r.Extreme;
}

float ComputeQueryable::Max() const {
  QueryResult r = Run(Terminal::Max);
  if (r.Count == 0) throw InvalidOperationException("Sequence contains no elements");
  return r.Extreme;
}

bool ComputeQueryable::Any() const { return LongCount() > 0; }

bool ComputeQueryable::Any(const Expr& predicate) const { return Where(predicate).LongCount() > 0; }

bool ComputeQueryable::All(const Expr& predicate) const { return Where(!predicate).LongCount() == 0; }

ComputeQueryable AsComputeQueryable(const std::vector<float>& source, std::shared_ptr<ComputeQueryProvider> provider) {
  return ComputeQueryable(source.data(), source.size(), provider ? provider : ComputeQueryProvider::Default());
}

ComputeQueryable AsComputeQueryable(const float* data, size_t n, std::shared_ptr<ComputeQueryProvider> provider) {
  return ComputeQueryable(data, n, provider ? provider : ComputeQueryProvider::Default());
}

ComputeQueryable AsComputeQueryable(const IUnifiedMemoryBuffer& device, std::shared_ptr<ComputeQueryProvider> provider) {
  return ComputeQueryable(device, provider ? provider : ComputeQueryProvider::Default());
}

}  // namespace DotCompute::Linq

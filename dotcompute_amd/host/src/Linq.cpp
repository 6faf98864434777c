// Linq.cpp — expression DSL, visitor, fusion planner (register-program code generator), executor
// and queryable of the HIP LINQ provider.
#include "DotCompute/Linq.hpp"

#include <cmath>
#include <cstring>
#include <limits>
#include <mutex>
#include <sstream>

namespace DotCompute::Linq {

using Backends::Hip::Check;

// ---- expression DSL -------------------------------------------------------------------------------

namespace {
std::shared_ptr<const ExprNode> MakeNode(ExprKind k, std::shared_ptr<const ExprNode> l = nullptr,
                                     std::shared_ptr<const ExprNode> r = nullptr) {
  auto n = std::make_shared<ExprNode>();
  n->Kind = k;
  n->Left = std::move(l);
  n->Right = std::move(r);
  return n;
}
bool IsConst(const Expr& e) { return e.Node().Kind == ExprKind::Constant; }
// The value of a constant as a float (an int constant converted as C#'s implicit int -> float).
float AsFloat(const ExprNode& n) { return n.IsInt ? (float)n.IValue : n.Value; }

// C# constant folding of int operands: constant expressions are evaluated in a checked context,
// where an overflow or a division by constant zero is a compile-time error (CS0220, CS0020).
int32_t FoldInt(ExprKind k, int32_t x, int32_t y) {
  int64_t r = 0;
  switch (k) {
    case ExprKind::Add: r = (int64_t)x + y; break;
    case ExprKind::Subtract: r = (int64_t)x - y; break;
    case ExprKind::Multiply: r = (int64_t)x * y; break;
    case ExprKind::Divide:
    case ExprKind::Modulo:
      if (y == 0) throw DivideByZeroException("Division by constant zero");
      if (x == std::numeric_limits<int32_t>::min() && y == -1)
        throw OverflowException("The operation overflows at compile time in checked mode");
      r = k == ExprKind::Divide ? x / y : x % y;
      break;
    default: throw NotSupportedException("not a foldable operation");
  }
  if (r < std::numeric_limits<int32_t>::min() || r > std::numeric_limits<int32_t>::max())
    throw OverflowException("The operation overflows at compile time in checked mode");
  return (int32_t)r;
}

// Binary arithmetic with constant folding of constant operands (the C# compiler folds constant
// sub-expressions of a lambda before building its expression tree): int with int folds as int,
// otherwise as float (the int operand converted), each float fold rounding to float.
Expr Arith(ExprKind k, const Expr& a, const Expr& b) {
  if (IsConst(a) && IsConst(b)) {
    if (a.Node().IsInt && b.Node().IsInt) return Expr(FoldInt(k, a.Node().IValue, b.Node().IValue));
    const float x = AsFloat(a.Node()), y = AsFloat(b.Node());
    switch (k) {
      case ExprKind::Add: return Expr(x + y);
      case ExprKind::Subtract: return Expr(x - y);
      case ExprKind::Multiply: return Expr(x * y);
      case ExprKind::Divide: return Expr(x / y);
      case ExprKind::Modulo: return Expr(std::fmod(x, y));
      default: break;
    }
  }
  return Expr(MakeNode(k, a.Ptr(), b.Ptr()));
}
bool IsCompareKind(ExprKind k) { return k >= ExprKind::GreaterThan && k <= ExprKind::NotEqual; }
bool IsPredicateKind(ExprKind k) { return IsCompareKind(k) || k == ExprKind::AndAlso || k == ExprKind::OrElse || k == ExprKind::Not; }
}  // namespace

Expr::Expr(float constant) {
  auto n = std::make_shared<ExprNode>();
  n->Kind = ExprKind::Constant;
  n->Value = constant;
  node_ = std::move(n);
}
Expr::Expr(double constant) : Expr((float)constant) {}
Expr::Expr(int32_t constant) {
  auto n = std::make_shared<ExprNode>();
  n->Kind = ExprKind::Constant;
  n->IValue = constant;
  n->IsInt = true;
  node_ = std::move(n);
}
Expr Expr::Parameter(int index) {
  auto n = std::make_shared<ExprNode>();
  n->Kind = ExprKind::Parameter;
  n->IValue = index;
  return Expr(std::move(n));
}
bool Expr::IsPredicate() const { return IsPredicateKind(node_->Kind); }

std::string Expr::ToString() const {
  const ExprNode& n = *node_;
  auto L = [&] { return Expr(n.Left).ToString(); };
  auto R = [&] { return Expr(n.Right).ToString(); };
  std::ostringstream os;
  switch (n.Kind) {
    case ExprKind::Parameter: return n.IValue == 0 ? "x" : "x" + std::to_string(n.IValue);
    case ExprKind::Constant:
      if (n.IsInt) os << n.IValue;
      else os << n.Value << "f";
      return os.str();
    case ExprKind::Negate: return "-(" + L() + ")";
    case ExprKind::Abs: return "Abs(" + L() + ")";
    case ExprKind::Sqrt: return "MathF.Sqrt(" + L() + ")";
    case ExprKind::Floor: return "MathF.Floor(" + L() + ")";
    case ExprKind::Ceiling: return "MathF.Ceiling(" + L() + ")";
    case ExprKind::Round: return "MathF.Round(" + L() + ")";
    case ExprKind::Add: return "(" + L() + " + " + R() + ")";
    case ExprKind::Subtract: return "(" + L() + " - " + R() + ")";
    case ExprKind::Multiply: return "(" + L() + " * " + R() + ")";
    case ExprKind::Divide: return "(" + L() + " / " + R() + ")";
    case ExprKind::Modulo: return "(" + L() + " % " + R() + ")";
    case ExprKind::Min: return "Min(" + L() + ", " + R() + ")";
    case ExprKind::Max: return "Max(" + L() + ", " + R() + ")";
    case ExprKind::Pow: return "MathF.Pow(" + L() + ", " + R() + ")";
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
Expr operator%(const Expr& a, const Expr& b) { return Arith(ExprKind::Modulo, a, b); }
Expr operator-(const Expr& a) {
  if (!IsConst(a)) return Expr(MakeNode(ExprKind::Negate, a.Ptr()));
  if (!a.Node().IsInt) return Expr(-a.Node().Value);
  return Expr(FoldInt(ExprKind::Subtract, 0, a.Node().IValue));  // -int.MinValue does not fold
}
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
Expr Floor(const Expr& a) { return Expr(MakeNode(ExprKind::Floor, a.Ptr())); }
Expr Ceiling(const Expr& a) { return Expr(MakeNode(ExprKind::Ceiling, a.Ptr())); }
Expr Round(const Expr& a) { return Expr(MakeNode(ExprKind::Round, a.Ptr())); }
Expr Min(const Expr& a, const Expr& b) { return Expr(MakeNode(ExprKind::Min, a.Ptr(), b.Ptr())); }
Expr Max(const Expr& a, const Expr& b) { return Expr(MakeNode(ExprKind::Max, a.Ptr(), b.Ptr())); }
Expr Pow(const Expr& a, const Expr& b) { return Expr(MakeNode(ExprKind::Pow, a.Ptr(), b.Ptr())); }
}  // namespace MathF

namespace Math {
Expr Abs(const Expr& a) { return MathF::Abs(a); }
Expr Min(const Expr& a, const Expr& b) { return MathF::Min(a, b); }
Expr Max(const Expr& a, const Expr& b) { return MathF::Max(a, b); }
}  // namespace Math

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

dc_linq_instr Instr(uint8_t op, uint8_t src = DC_LQ_SRC_IMM, uint32_t imm_bits = 0, uint8_t mode = DC_LQ_CMP_SET) {
  dc_linq_instr i;
  i.op = op;
  i.src = src;
  i.mode = mode;
  i.pad = 0;
  i.imm_i32 = (int32_t)imm_bits;
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

uint8_t ArithOp(ExprKind k) {
  switch (k) {
    case ExprKind::Add: return DC_LQ_ADD;
    case ExprKind::Subtract: return DC_LQ_SUB;
    case ExprKind::Multiply: return DC_LQ_MUL;
    case ExprKind::Divide: return DC_LQ_DIV;
    case ExprKind::Modulo: return DC_LQ_REM;
    case ExprKind::Min: return DC_LQ_MIN;
    case ExprKind::Max: return DC_LQ_MAX;
    case ExprKind::Pow: return DC_LQ_POW;
    default: throw NotSupportedException("not an arithmetic node");
  }
}

// Operation with its operands swapped (v = operand OP v): exact for +, *, min, max (IEEE + and *
// commute, as do wrapping int + and *; Min/Max are symmetric), and via RSUB/RDIV/RREM/RPOW for -, /,
// % and Pow.
uint8_t ReversedArithOp(ExprKind k) {
  switch (k) {
    case ExprKind::Add: return DC_LQ_ADD;
    case ExprKind::Multiply: return DC_LQ_MUL;
    case ExprKind::Min: return DC_LQ_MIN;
    case ExprKind::Max: return DC_LQ_MAX;
    case ExprKind::Subtract: return DC_LQ_RSUB;
    case ExprKind::Divide: return DC_LQ_RDIV;
    case ExprKind::Modulo: return DC_LQ_RREM;
    case ExprKind::Pow: return DC_LQ_RPOW;
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

bool IsBinaryArith(ExprKind k) {
  return k == ExprKind::Add || k == ExprKind::Subtract || k == ExprKind::Multiply || k == ExprKind::Divide ||
         k == ExprKind::Modulo || k == ExprKind::Min || k == ExprKind::Max || k == ExprKind::Pow;
}

struct Compiler {
  std::vector<dc_linq_instr>& code;
  bool is_int;  // the element type: int32 (C# int semantics) or float32

  void Emit(const dc_linq_instr& i) {
    if (code.size() >= (size_t)DC_LINQ_MAX_INSTR)
      throw NotSupportedException("the fused chain needs more than " + std::to_string(DC_LINQ_MAX_INSTR) +
                                  " instructions");
    code.push_back(i);
  }

  // Whether evaluating `n` can throw for some element (int: / and % by anything but a constant
  // other than 0 and -1, and Math.Abs); float arithmetic never throws.
  bool CanThrow(const ExprNode& n) const {
    if (!is_int || IsLeaf(n)) return false;
    if (n.Kind == ExprKind::Abs) return true;
    if (n.Kind == ExprKind::Divide || n.Kind == ExprKind::Modulo) {
      const ExprNode& d = *n.Right;
      if (d.Kind != ExprKind::Constant || d.IValue == 0 || d.IValue == -1) return true;
    }
    return (n.Left && CanThrow(*n.Left)) || (n.Right && CanThrow(*n.Right));
  }

  // The immediate bits of a constant in the program's element type. An int constant in a float
  // lambda is converted as C# converts it; a float constant in an int lambda would make the lambda
  // float-typed (a different element type), which one fused kernel cannot change to.
  uint32_t ImmBits(const ExprNode& n) const {
    if (is_int) {
      if (!n.IsInt)
        throw NotSupportedException("a float constant in a lambda over int elements changes the element type; the "
                                    "fused HIP kernels keep one element type per chain");
      return (uint32_t)n.IValue;
    }
    const float f = AsFloat(n);
    uint32_t b;
    std::memcpy(&b, &f, sizeof(b));
    return b;
  }

  // Operand source for a leaf: the element itself, or an immediate.
  std::pair<uint8_t, uint32_t> LeafSource(const ExprNode& n) const {
    if (n.Kind == ExprKind::Parameter && n.IValue != 0)
      throw NotSupportedException("Where/Select lambdas take one parameter");
    return n.Kind == ExprKind::Parameter ? std::make_pair((uint8_t)DC_LQ_SRC_ELEM, 0u)
                                         : std::make_pair((uint8_t)DC_LQ_SRC_IMM, ImmBits(n));
  }

  // Leaves the value of `n` in v. Saved registers with index >= `free_save` may be used. Operands
  // are evaluated left before right wherever the left one can throw, so an element that throws in
  // both raises the left one's exception, as C# evaluates operands left to right.
  void Value(const ExprNode& n, int free_save) {
    switch (n.Kind) {
      case ExprKind::Parameter:
        if (n.IValue != 0) throw NotSupportedException("Where/Select lambdas take one parameter");
        Emit(Instr(DC_LQ_LOAD, DC_LQ_SRC_ELEM));
        return;
      case ExprKind::Constant: Emit(Instr(DC_LQ_LOAD, DC_LQ_SRC_IMM, ImmBits(n))); return;
      case ExprKind::Negate: Value(*n.Left, free_save); Emit(Instr(DC_LQ_NEG)); return;
      case ExprKind::Abs: Value(*n.Left, free_save); Emit(Instr(DC_LQ_ABS)); return;
      case ExprKind::Sqrt:
      case ExprKind::Floor:
      case ExprKind::Ceiling:
      case ExprKind::Round: {
        if (is_int)
          throw NotSupportedException("Math.Sqrt/Floor/Ceiling/Round of an int yields a double; the fused HIP "
                                      "kernels keep one element type per chain");
        Value(*n.Left, free_save);
        const uint8_t op = n.Kind == ExprKind::Sqrt ? DC_LQ_SQRT : n.Kind == ExprKind::Floor ? DC_LQ_FLOOR
                           : n.Kind == ExprKind::Ceiling ? DC_LQ_CEIL : DC_LQ_ROUND;
        Emit(Instr(op));
        return;
      }
      default:
        break;
    }
    if (!IsBinaryArith(n.Kind))
      throw NotSupportedException("a boolean expression cannot be used as a value in the HIP kernels");
    if (is_int && n.Kind == ExprKind::Pow)
      throw NotSupportedException("MathF.Pow of an int converts it to float; the fused HIP kernels keep one "
                                  "element type per chain");
    if (RightIsOperand(n)) {
      Value(*n.Left, free_save);
      auto [src, imm] = LeafSource(*n.Right);
      Emit(Instr(ArithOp(n.Kind), src, imm));
    } else if (IsLeaf(*n.Left)) {
      Value(*n.Right, free_save);
      auto [src, imm] = LeafSource(*n.Left);
      Emit(Instr(ReversedArithOp(n.Kind), src, imm));
    } else if (CanThrow(*n.Left)) {
      const int s = Save(free_save);
      Value(*n.Left, free_save);
      Emit(Instr(s == 0 ? DC_LQ_STORE_S0 : DC_LQ_STORE_S1));
      Value(*n.Right, free_save + 1);
      Emit(Instr(ReversedArithOp(n.Kind), s == 0 ? DC_LQ_SRC_S0 : DC_LQ_SRC_S1));
    } else {
      const int s = Save(free_save);
      Value(*n.Right, free_save);
      Emit(Instr(s == 0 ? DC_LQ_STORE_S0 : DC_LQ_STORE_S1));
      Value(*n.Left, free_save + 1);
      Emit(Instr(ArithOp(n.Kind), s == 0 ? DC_LQ_SRC_S0 : DC_LQ_SRC_S1));
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
      } else if (CanThrow(*n.Left)) {
        Value(*n.Left, 0);
        Emit(Instr(DC_LQ_STORE_S0));
        Value(*n.Right, 1);
        Emit(Instr(CompareOp(n.Kind, true), DC_LQ_SRC_S0, 0, mode));
      } else {
        Value(*n.Right, 0);
        Emit(Instr(DC_LQ_STORE_S0));
        Value(*n.Left, 1);
        Emit(Instr(CompareOp(n.Kind, false), DC_LQ_SRC_S0, 0, mode));
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
        // C# evaluates the right operand only when the left one does not decide: the program
        // evaluates both, which is the same as long as the right one cannot throw.
        if (CanThrow(*n.Right))
          throw NotSupportedException("an int division, remainder or Math.Abs in the right operand of && or || is "
                                      "evaluated conditionally in C#; the fused HIP kernel evaluates both operands");
        const uint8_t combine = n.Kind == ExprKind::AndAlso ? DC_LQ_CMP_AND : DC_LQ_CMP_OR;
        // Neither side has an effect an element could observe, so they may run in either order.
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
    case DC_LQ_REM: return "REM";
    case DC_LQ_RREM: return "RREM";
    case DC_LQ_MIN: return "MIN";
    case DC_LQ_MAX: return "MAX";
    case DC_LQ_NEG: return "NEG";
    case DC_LQ_ABS: return "ABS";
    case DC_LQ_SQRT: return "SQRT";
    case DC_LQ_FLOOR: return "FLOOR";
    case DC_LQ_CEIL: return "CEIL";
    case DC_LQ_ROUND: return "ROUND";
    case DC_LQ_POW: return "POW";
    case DC_LQ_RPOW: return "RPOW";
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

bool HasOperand(uint8_t op) {
  return op == DC_LQ_LOAD || (op >= DC_LQ_ADD && op <= DC_LQ_MAX) || op == DC_LQ_REM || op == DC_LQ_RREM ||
         (op >= DC_LQ_CMP_GT && op <= DC_LQ_CMP_NE) || op == DC_LQ_POW || op == DC_LQ_RPOW;
}

}  // namespace

void HipKernelGenerator::CompileLambda(const Expr& lambda, bool predicate, std::vector<dc_linq_instr>& code,
                                       ElementType element) {
  if (element != ElementType::Float32 && element != ElementType::Int32)
    throw NotSupportedException("the HIP LINQ kernels take float or int elements");
  Compiler c{code, element == ElementType::Int32};
  if (predicate) {
    if (!lambda.IsPredicate()) throw NotSupportedException("Where() needs a boolean lambda");
    c.Predicate(lambda.Node(), DC_LQ_CMP_SET, false);
  } else {
    if (lambda.IsPredicate()) throw NotSupportedException("Select() to bool is not supported by the HIP kernels");
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

FusedKernelPlan HipKernelGenerator::GenerateHipKernel(const OperationGraph& graph, ElementType element) const {
  FusedKernelPlan plan;
  plan.Element = element;
  const auto fused = IdentifyFusableOperations(graph);
  std::vector<dc_linq_instr> code;
  for (const Operation* op : fused) {
    if (op->Method != "Where" && op->Method != "Select")
      throw NotSupportedException("LINQ method '" + op->Method + "' has no HIP kernel");
    if (!op->Lambda) throw ArgumentNullException(op->Method + " needs a lambda");
    const bool is_filter = op->Type == OperationType::Filter;
    CompileLambda(*op->Lambda, is_filter, code, element);
    if (code.size() >= (size_t)DC_LINQ_MAX_INSTR) throw NotSupportedException("fused chain too long");
    code.push_back(Instr(is_filter ? DC_LQ_FILTER : DC_LQ_MAP));
    plan.FusedOperationIds.push_back(op->Id);
  }
  plan.BareSource = fused.empty();
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
  if (element == ElementType::Int32) {
    int32_t can = 0;
    Check(dc_linq_chain_can_fault_i32(&plan.Program, &can), "dc_linq_chain_can_fault_i32");
    plan.CanFault = can != 0;
  }
  return plan;
}

std::string FusedKernelPlan::Listing() const {
  std::ostringstream os;
  const char* term = Term == Terminal::ToArray ? "ToArray" : Term == Terminal::Sum ? "Sum"
                     : Term == Terminal::Average ? "Average" : Term == Terminal::Min ? "Min"
                     : Term == Terminal::Max ? "Max" : "Count";
  os << "terminal " << term << (Element == ElementType::Int32 ? " (int32)" : " (float32)") << "\n";
  for (int i = 0; i < Program.n_instr; ++i) {
    const dc_linq_instr& in = Program.code[i];
    os << i << ": " << OpName(in.op);
    if (HasOperand(in.op)) {
      if (in.src == DC_LQ_SRC_IMM) {
        if (Element == ElementType::Int32) os << " " << in.imm_i32;
        else os << " " << in.imm;
      } else {
        os << (in.src == DC_LQ_SRC_ELEM ? " e" : in.src == DC_LQ_SRC_S0 ? " s0" : " s1");
      }
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
      "once, and the re-run on the ordered grid reported count " + std::to_string(k) + ".");
}

void RuntimeExecutor::ThrowIfFaulted(int64_t fault) {
  if (fault < 0) return;
  if ((fault & 3) == DC_LINQ_FAULT_DIVIDE_BY_ZERO) throw DivideByZeroException("Attempted to divide by zero.");
  throw OverflowException("Arithmetic operation resulted in an overflow.");
}

QueryResult<float> RuntimeExecutor::Run(const FusedKernelPlan& plan, const float* device_in, size_t n) {
  dc_hip_ctx* ctx = acc_->Context();
  QueryResult<float> r;
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
  } else if (plan.Term == Terminal::Min || plan.Term == Terminal::Max || plan.Term == Terminal::Aggregate) {
    if (plan.Term == Terminal::Aggregate && plan.Fold != AggregateKind::Min && plan.Fold != AggregateKind::Max)
      throw NotSupportedException("internal: a float Aggregate other than MathF.Min / MathF.Max");
    const int32_t op = plan.Term == Terminal::Min   ? DC_LINQ_MIN
                       : plan.Term == Terminal::Max ? DC_LINQ_MAX
                       : plan.Fold == AggregateKind::Min ? DC_LINQ_FOLD_MIN
                                                         : DC_LINQ_FOLD_MAX;
    auto val = mem.AllocateAsync<float>(1);
    auto cnt = mem.AllocateAsync<int64_t>(1);
    Check(dc_hip_linq_where_select_minmax_f32(ctx, &plan.Program, device_in, (int64_t)n, op, val->Data(),
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

// int32 chains. A program that can throw brings a fault word; the first throwing element's
// exception is raised instead of a result, unless (Sum) the checked running total already
// overflowed before that element, which LINQ-to-objects would have raised first.
QueryResult<int32_t> RuntimeExecutor::Run(const FusedKernelPlan& plan, const int32_t* device_in, size_t n) {
  dc_hip_ctx* ctx = acc_->Context();
  QueryResult<int32_t> r;
  auto& mem = acc_->Memory();
  std::shared_ptr<IUnifiedMemoryBufferT<int64_t>> fault;
  if (plan.CanFault) fault = mem.AllocateAsync<int64_t>(1);
  int64_t* fault_ptr = fault ? fault->Data() : nullptr;
  auto read_fault = [&]() {
    int64_t f = DC_LINQ_FAULT_NONE;
    if (fault) fault->CopyToHost(&f, sizeof(f));
    return f;
  };
  if (plan.Term == Terminal::ToArray) {
    auto out = mem.AllocateAsync<int32_t>(std::max<size_t>(n, 1));
    auto cnt = mem.AllocateAsync<int64_t>(1);
    auto run = [&](const dc_linq_chain& prog) {
      Check(dc_hip_linq_where_select_i32(ctx, &prog, device_in, (int64_t)n, out->Data(), cnt->Data(), fault_ptr),
            "dc_hip_linq_where_select_i32");
      acc_->Synchronize();
      int64_t k = 0;
      cnt->CopyToHost(&k, sizeof(k));
      return k;
    };
    int64_t k = run(plan.Program);
    k = ResolveCompactedCount(k, [&]() {
      dc_linq_chain ordered = plan.Program;
      ordered.flags |= DC_LINQ_FLAG_ORDERED_GRID;
      return run(ordered);
    });
    ThrowIfFaulted(read_fault());
    r.Count = k;
    r.Values.resize((size_t)k);
    out->CopyToHost(r.Values.data(), (size_t)k * sizeof(int32_t));
  } else if (plan.Term == Terminal::Min || plan.Term == Terminal::Max) {
    auto val = mem.AllocateAsync<int32_t>(1);
    auto cnt = mem.AllocateAsync<int64_t>(1);
    Check(dc_hip_linq_where_select_minmax_i32(ctx, &plan.Program, device_in, (int64_t)n,
                                              plan.Term == Terminal::Min ? DC_LINQ_MIN : DC_LINQ_MAX, val->Data(),
                                              cnt->Data(), fault_ptr),
          "dc_hip_linq_where_select_minmax_i32");
    acc_->Synchronize();
    ThrowIfFaulted(read_fault());
    val->CopyToHost(&r.Extreme, sizeof(int32_t));
    cnt->CopyToHost(&r.Count, sizeof(int64_t));
  } else if (plan.Term == Terminal::Sum && plan.BareSource) {
    // Sum() of the array itself: the BCL's vectorised rule (Enumerable.Sum over a span).
    auto sum = mem.AllocateAsync<int64_t>(1);
    auto ovf = mem.AllocateAsync<int32_t>(1);
    Check(dc_hip_reduce_sum_i32(ctx, device_in, (int64_t)n, sum->Data(), ovf->Data()), "dc_hip_reduce_sum_i32");
    acc_->Synchronize();
    int32_t o = 0;
    sum->CopyToHost(&r.IntSum, sizeof(int64_t));
    ovf->CopyToHost(&o, sizeof(int32_t));
    r.SumOverflowed = o != 0;
    r.Count = (int64_t)n;
  } else {
    // Sum after Where/Select (the element-by-element checked total), Count, LongCount, Average.
    auto sum = mem.AllocateAsync<int64_t>(1);
    auto cnt = mem.AllocateAsync<int64_t>(1);
    auto ovf = mem.AllocateAsync<int32_t>(1);
    auto run = [&](size_t len) {
      Check(dc_hip_linq_where_select_sum_i32(ctx, &plan.Program, device_in, (int64_t)len, sum->Data(), cnt->Data(),
                                             ovf->Data(), fault_ptr),
            "dc_hip_linq_where_select_sum_i32");
      acc_->Synchronize();
      int32_t o = 0;
      ovf->CopyToHost(&o, sizeof(int32_t));
      return o != 0;
    };
    bool overflowed = run(n);
    const int64_t f = read_fault();
    if (f >= 0) {
      // Which exception comes first: the running total over the elements before the throwing one.
      if (plan.Term == Terminal::Sum && run((size_t)(f / 4)))
        throw OverflowException("Arithmetic operation resulted in an overflow.");
      ThrowIfFaulted(f);
    }
    sum->CopyToHost(&r.IntSum, sizeof(int64_t));
    cnt->CopyToHost(&r.Count, sizeof(int64_t));
    r.SumOverflowed = overflowed;
  }
  return r;
}

namespace {

bool IsCut(const MethodCall& m) { return m.Method == "Take" || m.Method == "Skip"; }

bool IsElementTerminal(Terminal t) {
  return t == Terminal::First || t == Terminal::FirstOrDefault || t == Terminal::Last || t == Terminal::LastOrDefault ||
         t == Terminal::Single || t == Terminal::SingleOrDefault;
}

int32_t LaunchToArray(dc_hip_ctx* ctx, const dc_linq_chain& prog, const float* in, int64_t n, float* out,
                      int64_t* cnt, int64_t*) {
  return dc_hip_linq_where_select_f32(ctx, &prog, in, n, out, cnt);
}
int32_t LaunchToArray(dc_hip_ctx* ctx, const dc_linq_chain& prog, const int32_t* in, int64_t n, int32_t* out,
                      int64_t* cnt, int64_t* fault) {
  return dc_hip_linq_where_select_i32(ctx, &prog, in, n, out, cnt, fault);
}

}  // namespace

template <typename T>
int64_t RuntimeExecutor::ToArrayLimited(const FusedKernelPlan& plan, const T* device_in, size_t n, T* out,
                                        std::optional<int64_t> limit) {
  dc_hip_ctx* ctx = acc_->Context();
  auto& mem = acc_->Memory();
  auto cnt = mem.AllocateAsync<int64_t>(1);
  std::shared_ptr<IUnifiedMemoryBufferT<int64_t>> fault;
  if (plan.CanFault) fault = mem.AllocateAsync<int64_t>(1);
  auto run = [&](size_t len) {
    auto once = [&](const dc_linq_chain& prog) {
      Check(LaunchToArray(ctx, prog, device_in, (int64_t)len, out, cnt->Data(), fault ? fault->Data() : nullptr),
            "dc_hip_linq_where_select");
      acc_->Synchronize();
      int64_t k = 0;
      cnt->CopyToHost(&k, sizeof(k));
      return k;
    };
    return ResolveCompactedCount(once(plan.Program), [&]() {
      dc_linq_chain ordered = plan.Program;
      ordered.flags |= DC_LINQ_FLAG_ORDERED_GRID;
      return once(ordered);
    });
  };
  const int64_t k = run(n);
  int64_t f = DC_LINQ_FAULT_NONE;
  if (fault) fault->CopyToHost(&f, sizeof(f));
  if (f < 0) return k;
  // Element f / 4 throws. The elements before it do not; if they already hold `limit` kept
  // elements, the consumer stopped pulling before it and LINQ-to-objects never evaluates it.
  if (limit) {
    const int64_t k_before = run((size_t)(f / 4));
    if (k_before >= *limit) return k_before;
  }
  ThrowIfFaulted(f);
  return k;
}

template <typename T>
QueryResult<T> RuntimeExecutor::RunSegments(const std::vector<FusedKernelPlan>& segments,
                                            const std::vector<MethodCall>& cuts, const T* device_in, size_t n) {
  auto& mem = acc_->Memory();
  const T* src = device_in;
  size_t len = n;
  std::vector<std::shared_ptr<IUnifiedMemoryBufferT<T>>> held;  // compacted segments still read
  for (size_t i = 0; i + 1 < segments.size(); ++i) {
    const bool take = cuts[i].Method == "Take";
    const size_t c = (size_t)std::max<int64_t>(0, *cuts[i].Count);
    if (segments[i].Program.n_instr > 0) {  // an empty segment leaves the sequence as it is
      auto out = mem.AllocateAsync<T>(std::max<size_t>(len, 1));
      const int64_t k = ToArrayLimited<T>(segments[i], src, len, out->Data(),
                                          take ? std::optional<int64_t>((int64_t)c) : std::nullopt);
      held.push_back(out);
      src = out->Data();
      len = (size_t)k;
    }
    if (take) {
      len = std::min(len, c);
    } else {
      const size_t skip = std::min(len, c);
      src += skip;
      len -= skip;
    }
  }
  const FusedKernelPlan& last = segments.back();
  if (IsElementTerminal(last.Term)) {
    // First stops pulling after one kept element, Single after two (the second one is already an
    // error), Last reads the whole sequence.
    const bool first = last.Term == Terminal::First || last.Term == Terminal::FirstOrDefault;
    const bool single = last.Term == Terminal::Single || last.Term == Terminal::SingleOrDefault;
    std::optional<int64_t> limit;
    if (first) limit = 1;
    if (single) limit = 2;
    const T* seq = src;
    int64_t k = (int64_t)len;
    std::shared_ptr<IUnifiedMemoryBufferT<T>> out;
    if (last.Program.n_instr > 0) {
      out = mem.AllocateAsync<T>(std::max<size_t>(len, 1));
      k = ToArrayLimited<T>(last, src, len, out->Data(), limit);
      seq = out->Data();
    }
    QueryResult<T> r;
    r.Count = k;
    if (k > 0) {
      const int64_t at = (first || single) ? 0 : k - 1;
      T v{};
      Check(dc_hip_memcpy_d2h_async(acc_->Context(), &v, seq + at, sizeof(T)), "dc_hip_memcpy_d2h_async");
      acc_->Synchronize();
      r.Values.push_back(v);
    }
    return r;
  }
  if (last.Term == Terminal::Aggregate) {
    // float: the MathF.Min / MathF.Max fold kernels. int: Add is the exact total (Count's kernel,
    // which has no overflow rule; the fold is unchecked and wraps); Min / Max are the Min / Max
    // kernels (over int, Math.Min / Math.Max fold to Enumerable.Min / Max).
    if constexpr (std::is_same<T, float>::value) return Run(last, src, len);
    FusedKernelPlan p = last;
    p.Term = last.Fold == AggregateKind::Add ? Terminal::Count
             : last.Fold == AggregateKind::Min ? Terminal::Min : Terminal::Max;
    p.BareSource = false;
    return Run(p, src, len);
  }
  return Run(last, src, len);
}

template int64_t RuntimeExecutor::ToArrayLimited<float>(const FusedKernelPlan&, const float*, size_t, float*,
                                                        std::optional<int64_t>);
template int64_t RuntimeExecutor::ToArrayLimited<int32_t>(const FusedKernelPlan&, const int32_t*, size_t, int32_t*,
                                                          std::optional<int64_t>);
template QueryResult<float> RuntimeExecutor::RunSegments<float>(const std::vector<FusedKernelPlan>&,
                                                                const std::vector<MethodCall>&, const float*, size_t);
template QueryResult<int32_t> RuntimeExecutor::RunSegments<int32_t>(const std::vector<FusedKernelPlan>&,
                                                                    const std::vector<MethodCall>&, const int32_t*,
                                                                    size_t);

template <typename T>
QueryResult<T> RuntimeExecutor::Execute(const FusedKernelPlan& plan, const T* data, size_t n) {
  auto in = acc_->Memory().AllocateAsync<T>(std::max<size_t>(n, 1));
  if (n) in->CopyFromHost(data, n * sizeof(T));
  return Run(plan, in->Data(), n);
}

template <typename T>
QueryResult<T> RuntimeExecutor::Execute(const FusedKernelPlan& plan, const IUnifiedMemoryBuffer& source, size_t n) {
  if (source.Type() != ElementTypeOf<T>::value)
    throw NotSupportedException("the device buffer's element type does not match the query's");
  return Run(plan, static_cast<const T*>(source.DevicePointer()), n);
}

template QueryResult<float> RuntimeExecutor::Execute<float>(const FusedKernelPlan&, const float*, size_t);
template QueryResult<int32_t> RuntimeExecutor::Execute<int32_t>(const FusedKernelPlan&, const int32_t*, size_t);
template QueryResult<float> RuntimeExecutor::Execute<float>(const FusedKernelPlan&, const IUnifiedMemoryBuffer&, size_t);
template QueryResult<int32_t> RuntimeExecutor::Execute<int32_t>(const FusedKernelPlan&, const IUnifiedMemoryBuffer&,
                                                                size_t);

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

namespace {

// The fold of an Aggregate lambda (acc, x) => ...: Add, Min or Max of the two parameters, in either
// order. int: all three. float: MathF.Min and MathF.Max (IEEE minimum / maximum, associative, on
// their own fold kernels); float + and * fold with one rounding per step in enumeration order,
// which a parallel reduction does not reproduce, so they are refused.
AggregateKind ParseFold(const Expr& func, ElementType element) {
  const ExprNode& n = func.Node();
  auto is_param = [](const std::shared_ptr<const ExprNode>& c, int i) {
    return c && c->Kind == ExprKind::Parameter && c->IValue == i;
  };
  const bool two_params = n.Left && n.Right && ((is_param(n.Left, 0) && is_param(n.Right, 1)) ||
                                                (is_param(n.Left, 1) && is_param(n.Right, 0)));
  const bool is_int = element == ElementType::Int32;
  if (two_params && n.Kind == ExprKind::Add && is_int) return AggregateKind::Add;
  if (two_params && n.Kind == ExprKind::Min) return AggregateKind::Min;
  if (two_params && n.Kind == ExprKind::Max) return AggregateKind::Max;
  throw NotSupportedException("Aggregate(" + func.ToString() + ") has no exact HIP kernel: the kernels fold int "
                              "(acc, x) => acc + x, Math.Min(acc, x) and Math.Max(acc, x), and float "
                              "MathF.Min(acc, x) and MathF.Max(acc, x)");
}

}  // namespace

// One segment (Where/Select operations only) with its terminal: the fused program, plus the
// element terminals and Aggregate, which run on the compacted sequence (the reference maps the
// element operators to Filter and Aggregate to Reduce, ExpressionTreeVisitor.cs:245,263-265).
FusedKernelPlan ComputeQueryProvider::Plan(const std::vector<MethodCall>& chain, Terminal terminal, size_t n,
                                           ElementType element) const {
  std::vector<MethodCall> full = chain;
  std::optional<MethodCall> fold;
  if (terminal == Terminal::Aggregate) {
    if (full.empty() || full.back().Method != "Aggregate" || !full.back().Lambda)
      throw ArgumentException("Aggregate needs its function as the last call of the chain");
    fold = full.back();
    full.pop_back();
  }
  switch (terminal) {
    case Terminal::Sum: full.push_back({"Sum", std::nullopt}); break;
    case Terminal::Count: full.push_back({"Count", std::nullopt}); break;
    case Terminal::LongCount: full.push_back({"LongCount", std::nullopt}); break;
    case Terminal::Average: full.push_back({"Average", std::nullopt}); break;
    case Terminal::Min: full.push_back({"Min", std::nullopt}); break;
    case Terminal::Max: full.push_back({"Max", std::nullopt}); break;
    default: break;  // ToArray, the element terminals and Aggregate: a Where/Select program alone
  }
  for (const MethodCall& m : full)
    if (IsCut(m)) throw NotSupportedException("internal: Take/Skip inside a fused segment");
  // Stage 1: expression tree -> operation graph.
  OperationGraph graph = ExpressionTreeVisitor().Visit(full);
  // Stage 2: fused kernel for the graph.
  (void)n;
  FusedKernelPlan plan = HipKernelGenerator().GenerateHipKernel(graph, element);
  if (IsElementTerminal(terminal)) plan.Term = terminal;
  if (fold) {
    plan.Term = Terminal::Aggregate;
    plan.Fold = ParseFold(*fold->Lambda, element);
    if (fold->Seed) {
      const ExprNode& sn = fold->Seed->Node();
      if (sn.Kind != ExprKind::Constant) throw ArgumentException("Aggregate's seed is a constant");
      if (element == ElementType::Int32) {
        if (!sn.IsInt) throw ArgumentException("Aggregate's seed over int is an int constant");
        plan.Seed = sn.IValue;
      }
    }
  }
  return plan;
}

template <typename T>
QueryResult<T> ComputeQueryProvider::Execute(const std::vector<MethodCall>& chain, Terminal terminal, const T* host,
                                             size_t n, const IUnifiedMemoryBuffer* device) {
  // Take/Skip cut the chain into segments of fused Where/Select operations; the terminal goes with
  // the last one (an Aggregate terminal brings its function as the chain's last call).
  std::vector<std::vector<MethodCall>> segs(1);
  std::vector<MethodCall> cuts;
  for (size_t i = 0; i < chain.size(); ++i) {
    const MethodCall& m = chain[i];
    if (IsCut(m)) {
      if (!m.Count) throw ArgumentNullException(m.Method + " needs a count");
      cuts.push_back(m);
      segs.emplace_back();
    } else {
      segs.back().push_back(m);
    }
  }
  std::vector<FusedKernelPlan> plans;
  for (size_t i = 0; i < segs.size(); ++i)
    plans.push_back(Plan(segs[i], i + 1 == segs.size() ? terminal : Terminal::ToArray, n, ElementTypeOf<T>::value));
  // After a Take/Skip the sequence is an iterator, not the source array (Enumerable.Sum's span rule).
  if (!cuts.empty()) plans.back().BareSource = false;
  WorkloadCharacteristics w;
  w.DataSize = n;
  w.OperationCount = (int)chain.size();
  w.HasReduction = terminal != Terminal::ToArray;
  BackendSelector(HasAccelerator()).SelectBackend(w);  // throws without a HIP device
  if (plans.size() == 1 && !IsElementTerminal(terminal) && terminal != Terminal::Aggregate)
    return device ? executor_->Execute<T>(plans[0], *device, n) : executor_->Execute<T>(plans[0], host, n);
  if (device) {
    if (device->Type() != ElementTypeOf<T>::value)
      throw NotSupportedException("the device buffer's element type does not match the query's");
    return executor_->RunSegments<T>(plans, cuts, static_cast<const T*>(device->DevicePointer()), n);
  }
  auto in = executor_->Accelerator().Memory().AllocateAsync<T>(std::max<size_t>(n, 1));
  if (n) in->CopyFromHost(host, n * sizeof(T));
  return executor_->RunSegments<T>(plans, cuts, in->Data(), n);
}

template QueryResult<float> ComputeQueryProvider::Execute<float>(const std::vector<MethodCall>&, Terminal,
                                                                 const float*, size_t, const IUnifiedMemoryBuffer*);
template QueryResult<int32_t> ComputeQueryProvider::Execute<int32_t>(const std::vector<MethodCall>&, Terminal,
                                                                     const int32_t*, size_t,
                                                                     const IUnifiedMemoryBuffer*);

// ---- queryable ----------------------------------------------------------------------------------------

template <typename T>
ComputeQueryable<T>::ComputeQueryable(const T* data, size_t n, std::shared_ptr<ComputeQueryProvider> provider)
    : host_(data), n_(n), provider_(std::move(provider)) {
  if (!data && n) throw ArgumentNullException("source");
}

template <typename T>
ComputeQueryable<T>::ComputeQueryable(const IUnifiedMemoryBuffer& device, std::shared_ptr<ComputeQueryProvider> provider)
    : device_(&device), n_(device.Length()), provider_(std::move(provider)) {}

template <typename T>
ComputeQueryable<T> ComputeQueryable<T>::Where(const Expr& predicate) const {
  ComputeQueryable q = *this;
  q.chain_.push_back({"Where", predicate});
  return q;
}

template <typename T>
ComputeQueryable<T> ComputeQueryable<T>::Select(const Expr& selector) const {
  ComputeQueryable q = *this;
  q.chain_.push_back({"Select", selector});
  return q;
}

template <typename T>
ComputeQueryable<T> ComputeQueryable<T>::OrderBy(const Expr& key) const {
  ComputeQueryable q = *this;
  q.chain_.push_back({"OrderBy", key});
  return q;
}

template <typename T>
QueryResult<T> ComputeQueryable<T>::Run(Terminal t, const std::vector<MethodCall>* chain) const {
  return provider_->Execute<T>(chain ? *chain : chain_, t, host_, n_, device_);
}

template <typename T>
ComputeQueryable<T> ComputeQueryable<T>::Take(int64_t count) const {
  ComputeQueryable q = *this;
  q.chain_.push_back({"Take", std::nullopt, count});
  return q;
}

template <typename T>
ComputeQueryable<T> ComputeQueryable<T>::Skip(int64_t count) const {
  ComputeQueryable q = *this;
  q.chain_.push_back({"Skip", std::nullopt, count});
  return q;
}

namespace {
[[noreturn]] void ThrowNoElements() { throw InvalidOperationException("Sequence contains no elements"); }
[[noreturn]] void ThrowMoreThanOne() { throw InvalidOperationException("Sequence contains more than one element"); }
}  // namespace

template <typename T>
T ComputeQueryable<T>::First() const {
  QueryResult<T> r = Run(Terminal::First);
  if (r.Count == 0) ThrowNoElements();
  return r.Values[0];
}

template <typename T>
T ComputeQueryable<T>::FirstOrDefault() const {
  QueryResult<T> r = Run(Terminal::FirstOrDefault);
  return r.Count == 0 ? T{} : r.Values[0];
}

template <typename T>
T ComputeQueryable<T>::Last() const {
  QueryResult<T> r = Run(Terminal::Last);
  if (r.Count == 0) ThrowNoElements();
  return r.Values[0];
}

template <typename T>
T ComputeQueryable<T>::LastOrDefault() const {
  QueryResult<T> r = Run(Terminal::LastOrDefault);
  return r.Count == 0 ? T{} : r.Values[0];
}

template <typename T>
T ComputeQueryable<T>::Single() const {
  QueryResult<T> r = Run(Terminal::Single);
  if (r.Count == 0) ThrowNoElements();
  if (r.Count > 1) ThrowMoreThanOne();
  return r.Values[0];
}

template <typename T>
T ComputeQueryable<T>::SingleOrDefault() const {
  QueryResult<T> r = Run(Terminal::SingleOrDefault);
  if (r.Count > 1) ThrowMoreThanOne();
  return r.Count == 0 ? T{} : r.Values[0];
}

namespace {

// MathF.Min / MathF.Max (.NET Core 3.0 and later): NaN if either operand is NaN, -0 below +0.
float NetMinF(float a, float b) {
  if (std::isnan(a)) return a;
  if (std::isnan(b)) return b;
  if (a == b) return std::signbit(a) ? a : b;
  return a < b ? a : b;
}
float NetMaxF(float a, float b) {
  if (std::isnan(a)) return a;
  if (std::isnan(b)) return b;
  if (a == b) return std::signbit(a) ? b : a;
  return a > b ? a : b;
}

}  // namespace

// Aggregate(func): the fold starts from the first element (an empty sequence throws);
// Aggregate(seed, func) from the seed. Add wraps as C#'s unchecked int +.
template <typename T>
T ComputeQueryable<T>::Aggregate(const Expr& func) const {
  std::vector<MethodCall> chain = chain_;
  chain.push_back({"Aggregate", func});
  QueryResult<T> r = Run(Terminal::Aggregate, &chain);
  if (r.Count == 0) ThrowNoElements();
  if constexpr (std::is_same<T, int32_t>::value) {
    return func.Node().Kind == ExprKind::Add ? (int32_t)(uint32_t)(uint64_t)r.IntSum : r.Extreme;
  } else {
    return r.Extreme;  // the MathF.Min / MathF.Max fold from the first element
  }
}

template <typename T>
T ComputeQueryable<T>::Aggregate(T seed, const Expr& func) const {
  std::vector<MethodCall> chain = chain_;
  chain.push_back({"Aggregate", func, std::nullopt, Expr(seed)});
  QueryResult<T> r = Run(Terminal::Aggregate, &chain);
  if constexpr (std::is_same<T, int32_t>::value) {
    const ExprKind k = func.Node().Kind;
    if (k == ExprKind::Add) return (int32_t)((uint32_t)seed + (uint32_t)(uint64_t)r.IntSum);
    if (r.Count == 0) return seed;
    return k == ExprKind::Min ? std::min(seed, r.Extreme) : std::max(seed, r.Extreme);
  } else {
    // MathF.Min / MathF.Max are associative: fold(seed, x1..xn) = f(seed, fold(x1..xn)).
    if (r.Count == 0) return seed;
    return func.Node().Kind == ExprKind::Min ? NetMinF(seed, r.Extreme) : NetMaxF(seed, r.Extreme);
  }
}

template <typename T>
FusedKernelPlan ComputeQueryable<T>::Explain(Terminal terminal) const {
  return provider_->Plan(chain_, terminal, n_, ElementTypeOf<T>::value);
}

template <typename T>
std::vector<T> ComputeQueryable<T>::ToArray() const { return Run(Terminal::ToArray).Values; }

template <typename T>
T ComputeQueryable<T>::Sum() const {
  QueryResult<T> r = Run(Terminal::Sum);
  if constexpr (std::is_same<T, int32_t>::value) {
    if (r.SumOverflowed) throw OverflowException("Arithmetic operation resulted in an overflow.");
    return (int32_t)r.IntSum;
  } else {
    return (float)r.Sum;
  }
}

template <typename T>
int64_t ComputeQueryable<T>::LongCount() const { return Run(Terminal::LongCount).Count; }

template <typename T>
int32_t ComputeQueryable<T>::Count() const {
  const int64_t c = Run(Terminal::Count).Count;
  if (c > std::numeric_limits<int32_t>::max()) throw OverflowException("Arithmetic operation resulted in an overflow.");
  return (int32_t)c;
}

// Enumerable.Average: float sources accumulate in float64 and return float; int sources sum in
// int64 and return double (the sum divided by the count).
template <typename T>
typename ComputeQueryable<T>::AverageType ComputeQueryable<T>::Average() const {
  QueryResult<T> r = Run(Terminal::Average);
  if (r.Count == 0) throw InvalidOperationException("Sequence contains no elements");
  if constexpr (std::is_same<T, int32_t>::value) return (double)r.IntSum / (double)r.Count;
  else return (float)(r.Sum / (double)r.Count);
}

// BCL Enumerable.Min/Max semantics (the reference runs these as LINQ-to-objects): the device
// reduction returns the same element bit for bit; an empty sequence throws.
template <typename T>
T ComputeQueryable<T>::Min() const {
  QueryResult<T> r = Run(Terminal::Min);
  if (r.Count == 0) throw InvalidOperationException("Sequence contains no elements");
  return r.Extreme;
}

template <typename T>
T ComputeQueryable<T>::Max() const {
  QueryResult<T> r = Run(Terminal::Max);
  if (r.Count == 0) throw InvalidOperationException("Sequence contains no elements");
  return r.Extreme;
}

template <typename T>
bool ComputeQueryable<T>::Any() const { return LongCount() > 0; }

template <typename T>
bool ComputeQueryable<T>::Any(const Expr& predicate) const { return Where(predicate).LongCount() > 0; }

template <typename T>
bool ComputeQueryable<T>::All(const Expr& predicate) const { return Where(!predicate).LongCount() == 0; }

template class ComputeQueryable<float>;
template class ComputeQueryable<int32_t>;

ComputeQueryable<float> AsComputeQueryable(const std::vector<float>& source,
                                           std::shared_ptr<ComputeQueryProvider> provider) {
  return ComputeQueryable<float>(source.data(), source.size(), provider ? provider : ComputeQueryProvider::Default());
}

ComputeQueryable<float> AsComputeQueryable(const float* data, size_t n, std::shared_ptr<ComputeQueryProvider> provider) {
  return ComputeQueryable<float>(data, n, provider ? provider : ComputeQueryProvider::Default());
}

ComputeQueryable<int32_t> AsComputeQueryable(const std::vector<int32_t>& source,
                                             std::shared_ptr<ComputeQueryProvider> provider) {
  return ComputeQueryable<int32_t>(source.data(), source.size(),
                                   provider ? provider : ComputeQueryProvider::Default());
}

ComputeQueryable<int32_t> AsComputeQueryable(const int32_t* data, size_t n,
                                             std::shared_ptr<ComputeQueryProvider> provider) {
  return ComputeQueryable<int32_t>(data, n, provider ? provider : ComputeQueryProvider::Default());
}

template <typename T>
ComputeQueryable<T> AsComputeQueryable(const IUnifiedMemoryBuffer& device, std::shared_ptr<ComputeQueryProvider> provider) {
  return ComputeQueryable<T>(device, provider ? provider : ComputeQueryProvider::Default());
}

template ComputeQueryable<float> AsComputeQueryable<float>(const IUnifiedMemoryBuffer&,
                                                           std::shared_ptr<ComputeQueryProvider>);
template ComputeQueryable<int32_t> AsComputeQueryable<int32_t>(const IUnifiedMemoryBuffer&,
                                                               std::shared_ptr<ComputeQueryProvider>);

}  // namespace DotCompute::Linq

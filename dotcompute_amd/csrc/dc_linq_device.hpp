// dc_linq_device.hpp — device side of the fused LINQ Where/Select kernels for gfx950: the
// register-program interpreter and its state, the affine and canonical fast paths, and the
// round-robin ToArray kernel body. Two users compile it: dc_linq.hip, whose prebuilt kernels run
// any program through the interpreter (or a fast path), and the run-time compiler
// (dc_linq_jit.hip), which instantiates the same kernel body for one program with every
// instruction a constant, so the compiled kernel computes exactly what the interpreter computes.
// Nothing here may need the HIP host runtime: under hipRTC (__HIPCC_RTC__) only the device
// builtins exist.
#pragma once

#ifndef __HIPCC_RTC__
#include <hip/hip_runtime.h>
#endif

#include <cstdint>
#include <type_traits>
#include <utility>

#ifdef __HIPCC_RTC__
#include "dotcompute_hip.h"
#else
#include "../../include/dotcompute_hip.h"
#endif
#include "dc_device.hpp"
#include "dc_intdiv.hpp"

namespace dclq {

// Calls f(std::integral_constant<int, U>) for U = 0, 1, ... in order: a compile-time unrolled loop, so
// the index into an array of register buffers is a constant whatever the size of the body (a
// `#pragma unroll` loop stays a loop when its unrolled body exceeds the compiler's size limit, and
// its register arrays then go to scratch memory).
template <typename F, int... U>
__device__ __attribute__((always_inline)) inline void for_each_index(F&& f, std::integer_sequence<int, U...>) {
  (f(std::integral_constant<int, U>{}), ...);
}

// ---- interpreter -------------------------------------------------------------------------------

// MathF.Min / MathF.Max semantics (NaN-propagating, -0 ordered below +0).
__device__ inline float net_min(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  if (a == b) return __builtin_signbit(a) ? a : b;
  return a < b ? a : b;
}
__device__ inline float net_max(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  if (a == b) return __builtin_signbit(a) ? b : a;
  return a > b ? a : b;
}

// One instruction, widened to dwords. gfx950 has no scalar byte load: reading the uint8 fields
// of dc_linq_instr directly compiles to a vector byte load per field, and the wait for it also
// waits for every outstanding streaming load of the thread. Two dword reads at a wave-uniform
// address stay scalar loads.
struct Instr {
  uint32_t op, src, mode, imm;  // imm: the constant's bits (float32 or int32 by program type)
};
// Internal opcode, never in a caller's chain: the multiply-high constants of the int32 DIV or REM
// by a constant that follows it (imm = m, mode = shift). The host inserts it (once per launch) so
// that the interpreter does not derive them again for every chunk of elements.
constexpr uint32_t kOpDivMagic = 0x40;
__device__ inline Instr fetch_instr(const dc_linq_chain& prog, int pc) {
  const uint32_t* w = reinterpret_cast<const uint32_t*>(&prog.code[pc]);
  const uint32_t w0 = w[0];
  return Instr{w0 & 0xFFu, (w0 >> 8) & 0xFFu, (w0 >> 16) & 0xFFu, w[1]};
}

// Exceptions of an int32 program, per element: bit j of `hit` is set once element j has thrown
// (at its first throwing operation; C# stops evaluating the element there), and bit j of `ovf`
// tells that this operation threw OverflowException (else DivideByZeroException).
struct Faults {
  uint32_t hit = 0, ovf = 0;
};

// Records the exceptions of one operation applied to element j: only elements still kept
// (`live`), and only their first exception.
__device__ __attribute__((always_inline)) inline void note_fault(Faults& f, int j, uint32_t live, bool dz, bool ov) {
  const uint32_t bit = ((dz || ov) && ((live >> j) & 1u)) ? ((1u << j) & ~f.hit) : 0u;
  f.hit |= bit;
  f.ovf |= ov ? bit : 0u;
}

// C# int arithmetic (unchecked context): + - * wrap; / and % throw for a zero divisor and
// overflow for int.MinValue / -1 (and % -1, as .NET on x64 does); the result of a throwing
// element is never used.
// C#'s float % (truncated remainder, exact). Kept out of line: a program with a remainder is rare,
// and fmodf inlined into every unrolled interpreter loop would bloat each kernel variant.
__device__ __attribute__((noinline)) float net_rem(float a, float b) { return ::fmodf(a, b); }
// MathF.Pow: the device library's powf (the C99 Annex F special values, as .NET Core's MathF.Pow),
// out of line for the same reason. Only the LIBM interpreter variant has it: its call sites change
// the register allocation of a kernel (a few reloads from scratch in the round-robin kernel's
// write-out), which the programs without it should not pay.
__device__ __attribute__((noinline)) float net_pow(float a, float b) { return ::powf(a, b); }

__device__ inline int32_t wrap_add(int32_t a, int32_t b) { return (int32_t)((uint32_t)a + (uint32_t)b); }
__device__ inline int32_t wrap_sub(int32_t a, int32_t b) { return (int32_t)((uint32_t)a - (uint32_t)b); }
__device__ inline int32_t wrap_mul(int32_t a, int32_t b) { return (int32_t)((uint32_t)a * (uint32_t)b); }
__device__ __attribute__((always_inline)) inline int32_t checked_div(int32_t a, int32_t b, int j, uint32_t live,
                                                                    Faults& f) {
  const bool dz = b == 0, ov = (b == -1) && (a == INT32_MIN);
  note_fault(f, j, live, dz, ov);
  return a / ((dz || ov) ? 1 : b);
}
__device__ __attribute__((always_inline)) inline int32_t checked_rem(int32_t a, int32_t b, int j, uint32_t live,
                                                                    Faults& f) {
  const bool dz = b == 0, ov = (b == -1) && (a == INT32_MIN);
  note_fault(f, j, live, dz, ov);
  return a % ((dz || ov) ? 1 : b);
}

// The interpreter's registers over the EPT elements of one thread: value v, save registers s0/s1,
// predicate p, saved predicate q, and the keep mask (bit j = element j), which starts as `live`
// (the elements that exist). T is the element type: float (no exceptions) or int32_t (C# int
// semantics, exceptions into `f`). exec() applies one instruction. The interpreter feeds it
// instructions fetched at run time; a kernel compiled at run time for one program feeds it
// constants, and the compiler then drops every branch on the instruction, so both compute the same.
// SAVES = false drops the s0/s1 registers for programs that never use them (the common case),
// which keeps the kernels at a higher occupancy. LIBM = true adds POW / RPOW (float32 only). Operands are read in place (an immediate stays a
// scalar operand of the vector instruction), so no per-element operand copy is materialised.
template <typename T, int EPT, bool SAVES, bool LIBM = false>
struct ProgramState {
  T v[EPT];
  T s0[SAVES ? EPT : 1], s1[SAVES ? EPT : 1];
  uint32_t p = 0, q = 0, keep;
  int32_t gm = 0, gs = 0;  // constants of the next DIV/REM by a constant (kOpDivMagic), if gv
  bool gv = false;

  __device__ __attribute__((always_inline)) explicit ProgramState(uint32_t live) : keep(live) {
#pragma unroll
    for (int j = 0; j < EPT; ++j) v[j] = T(0);
#pragma unroll
    for (int j = 0; j < (SAVES ? EPT : 1); ++j) {
      s0[j] = T(0);
      s1[j] = T(0);
    }
  }

  // int32 v / d (rem: v % d) for a constant divisor d outside {0, -1, 1}, which never throws, by a
  // multiply-high (g = dc::div_magic(d)).
  __device__ __attribute__((always_inline)) void div_const(const dc::DivMagic g, bool rem) {
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      const int32_t quo = dc::div_by_magic(v[j], g);
      v[j] = rem ? wrap_sub(v[j], wrap_mul(quo, g.d)) : quo;
    }
  }

  __device__ __attribute__((always_inline)) void exec(const Instr ins, T (&e)[EPT], Faults& f) {
    constexpr bool kInt = std::is_same<T, int32_t>::value;
    uint32_t c = 0;
    bool is_cmp = false;
// Applies `body` (which reads the operand as O) to every element, for the instruction's source.
#define DC_LQ_APPLY(body)                                                                   \
  do {                                                                                      \
    if (ins.src == DC_LQ_SRC_ELEM) {                                                        \
      _Pragma("unroll") for (int j = 0; j < EPT; ++j) { const T O = e[j]; body; }           \
    } else if (SAVES && ins.src == DC_LQ_SRC_S0) {                                          \
      _Pragma("unroll") for (int j = 0; j < EPT; ++j) { const T O = s0[SAVES ? j : 0]; body; } \
    } else if (SAVES && ins.src == DC_LQ_SRC_S1) {                                          \
      _Pragma("unroll") for (int j = 0; j < EPT; ++j) { const T O = s1[SAVES ? j : 0]; body; } \
    } else {                                                                                \
      const T O = __builtin_bit_cast(T, ins.imm);                                           \
      _Pragma("unroll") for (int j = 0; j < EPT; ++j) { body; }                             \
    }                                                                                       \
  } while (0)
    switch (ins.op) {
      case kOpDivMagic:
        gm = (int32_t)ins.imm;
        gs = (int32_t)ins.mode;
        gv = true;
        break;
      case DC_LQ_LOAD: DC_LQ_APPLY(v[j] = O); break;
      case DC_LQ_ADD:
        if constexpr (kInt) DC_LQ_APPLY(v[j] = wrap_add(v[j], O));
        else DC_LQ_APPLY(v[j] = v[j] + O);
        break;
      case DC_LQ_SUB:
        if constexpr (kInt) DC_LQ_APPLY(v[j] = wrap_sub(v[j], O));
        else DC_LQ_APPLY(v[j] = v[j] - O);
        break;
      case DC_LQ_RSUB:
        if constexpr (kInt) DC_LQ_APPLY(v[j] = wrap_sub(O, v[j]));
        else DC_LQ_APPLY(v[j] = O - v[j]);
        break;
      case DC_LQ_MUL:
        if constexpr (kInt) DC_LQ_APPLY(v[j] = wrap_mul(v[j], O));
        else DC_LQ_APPLY(v[j] = v[j] * O);
        break;
      case DC_LQ_DIV:
        if constexpr (kInt) {
          const int32_t d = (int32_t)ins.imm;
          if (ins.src == DC_LQ_SRC_IMM && d != 0 && d != -1 && d != 1) {  // never throws
            div_const(gv ? dc::DivMagic{gm, gs, d} : dc::div_magic(d), false);
            gv = false;
          } else {
            DC_LQ_APPLY(v[j] = checked_div(v[j], O, j, keep, f));
          }
        } else {
          DC_LQ_APPLY(v[j] = v[j] / O);
        }
        break;
      case DC_LQ_RDIV:
        if constexpr (kInt) DC_LQ_APPLY(v[j] = checked_div(O, v[j], j, keep, f));
        else DC_LQ_APPLY(v[j] = O / v[j]);
        break;
      case DC_LQ_REM:
        if constexpr (kInt) {
          const int32_t d = (int32_t)ins.imm;
          if (ins.src == DC_LQ_SRC_IMM && d != 0 && d != -1 && d != 1) {  // never throws
            div_const(gv ? dc::DivMagic{gm, gs, d} : dc::div_magic(d), true);
            gv = false;
          } else {
            DC_LQ_APPLY(v[j] = checked_rem(v[j], O, j, keep, f));
          }
        } else {
          DC_LQ_APPLY(v[j] = net_rem(v[j], O));
        }
        break;
      case DC_LQ_RREM:
        if constexpr (kInt) DC_LQ_APPLY(v[j] = checked_rem(O, v[j], j, keep, f));
        else DC_LQ_APPLY(v[j] = net_rem(O, v[j]));
        break;
      case DC_LQ_MIN:
        if constexpr (kInt) DC_LQ_APPLY(v[j] = min(v[j], O));
        else DC_LQ_APPLY(v[j] = net_min(v[j], O));
        break;
      case DC_LQ_MAX:
        if constexpr (kInt) DC_LQ_APPLY(v[j] = max(v[j], O));
        else DC_LQ_APPLY(v[j] = net_max(v[j], O));
        break;
      case DC_LQ_NEG:
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
          if constexpr (kInt) v[j] = wrap_sub(0, v[j]);
          else v[j] = -v[j];
        }
        break;
      case DC_LQ_ABS:
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
          if constexpr (kInt) {
            note_fault(f, j, keep, false, v[j] == INT32_MIN);  // Math.Abs(int.MinValue) throws
            v[j] = v[j] < 0 ? wrap_sub(0, v[j]) : v[j];
          } else {
            v[j] = __builtin_fabsf(v[j]);
          }
        }
        break;
      case DC_LQ_SQRT:
        if constexpr (!kInt) {
#pragma unroll
          for (int j = 0; j < EPT; ++j) v[j] = __builtin_sqrtf(v[j]);
        }
        break;
      case DC_LQ_FLOOR:
        if constexpr (!kInt) {
#pragma unroll
          for (int j = 0; j < EPT; ++j) v[j] = __builtin_floorf(v[j]);
        }
        break;
      case DC_LQ_CEIL:
        if constexpr (!kInt) {
#pragma unroll
          for (int j = 0; j < EPT; ++j) v[j] = __builtin_ceilf(v[j]);
        }
        break;
      case DC_LQ_ROUND:
        if constexpr (!kInt) {
#pragma unroll
          for (int j = 0; j < EPT; ++j) v[j] = __builtin_rintf(v[j]);  // ties to even, as MathF.Round
        }
        break;
      case DC_LQ_POW:
        if constexpr (!kInt && LIBM) DC_LQ_APPLY(v[j] = net_pow(v[j], O));
        break;
      case DC_LQ_RPOW:
        if constexpr (!kInt && LIBM) DC_LQ_APPLY(v[j] = net_pow(O, v[j]));
        break;
      case DC_LQ_STORE_S0:
        if (SAVES) {
#pragma unroll
          for (int j = 0; j < EPT; ++j) s0[SAVES ? j : 0] = v[j];
        }
        break;
      case DC_LQ_STORE_S1:
        if (SAVES) {
#pragma unroll
          for (int j = 0; j < EPT; ++j) s1[SAVES ? j : 0] = v[j];
        }
        break;
      case DC_LQ_CMP_GT: is_cmp = true; DC_LQ_APPLY(c |= (uint32_t)(v[j] > O) << j); break;
      case DC_LQ_CMP_GE: is_cmp = true; DC_LQ_APPLY(c |= (uint32_t)(v[j] >= O) << j); break;
      case DC_LQ_CMP_LT: is_cmp = true; DC_LQ_APPLY(c |= (uint32_t)(v[j] < O) << j); break;
      case DC_LQ_CMP_LE: is_cmp = true; DC_LQ_APPLY(c |= (uint32_t)(v[j] <= O) << j); break;
      case DC_LQ_CMP_EQ: is_cmp = true; DC_LQ_APPLY(c |= (uint32_t)(v[j] == O) << j); break;
      case DC_LQ_CMP_NE: is_cmp = true; DC_LQ_APPLY(c |= (uint32_t)(v[j] != O) << j); break;
      case DC_LQ_MAP:
#pragma unroll
        for (int j = 0; j < EPT; ++j) e[j] = v[j];
        break;
      case DC_LQ_PNOT: p = ~p; break;
      case DC_LQ_PSTORE: q = p; break;
      case DC_LQ_PAND_Q: p &= q; break;
      case DC_LQ_POR_Q: p |= q; break;
      case DC_LQ_FILTER: keep &= p; break;
      default: break;
    }
#undef DC_LQ_APPLY
    if (is_cmp) {
      if (ins.mode == DC_LQ_CMP_AND) p &= c;
      else if (ins.mode == DC_LQ_CMP_OR) p |= c;
      else p = c;
    }
  }
};

// Runs the program over the EPT elements of one thread; returns the keep mask.
template <typename T, int EPT, bool SAVES, bool LIBM = false>
__device__ __attribute__((always_inline)) inline uint32_t run_program(const dc_linq_chain& prog, T (&e)[EPT],
                                                                       uint32_t live, Faults& f) {
  ProgramState<T, EPT, SAVES, LIBM> st(live);
  const int n = prog.n_instr;
  // The next instruction's scalar load is issued before the current one runs, so its latency
  // overlaps the work of the current instruction instead of stalling the dispatch.
  Instr next = fetch_instr(prog, 0);
  for (int pc = 0; pc < n; ++pc) {
    const Instr ins = next;
    next = fetch_instr(prog, min(pc + 1, DC_LINQ_MAX_INSTR - 1));
    st.exec(ins, e, f);
  }
  return st.keep;
}

// Float programs (no exceptions), every element present.
template <int EPT, bool SAVES, bool LIBM = false>
__device__ __attribute__((always_inline)) inline uint32_t run_program_f32(const dc_linq_chain& prog, float (&e)[EPT]) {
  Faults none;
  return run_program<float, EPT, SAVES, LIBM>(prog, e, (EPT == 32) ? 0xFFFFFFFFu : ((1u << EPT) - 1u), none);
}

// An int32 program over elements held as float bit patterns (the kernels move 32-bit words and
// do not care for their type): converts in registers, runs, converts back.
template <int EPT, bool SAVES>
__device__ __attribute__((always_inline)) inline uint32_t run_program_i32(const dc_linq_chain& prog, float (&e)[EPT],
                                                                           uint32_t live, Faults& f) {
  int32_t x[EPT];
#pragma unroll
  for (int j = 0; j < EPT; ++j) x[j] = __builtin_bit_cast(int32_t, e[j]);
  const uint32_t keep = run_program<int32_t, EPT, SAVES>(prog, x, live, f);
#pragma unroll
  for (int j = 0; j < EPT; ++j) e[j] = __builtin_bit_cast(float, x[j]);
  return keep;
}

// Fault word of the int32 entry points (in ctx->counters, 0 between launches): the largest
// ~(4 * index + kind) over the throwing elements, i.e. the first element's code, complemented.
__device__ inline void publish_fault(uint64_t* word, int64_t index, bool overflow) {
  const uint64_t code = (uint64_t)index * 4u + (overflow ? DC_LINQ_FAULT_OVERFLOW : DC_LINQ_FAULT_DIVIDE_BY_ZERO);
  __hip_atomic_fetch_max(word, ~code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The first faulting element of a thread's group: its position j (lowest set bit; the callers lay
// elements out so that j increases with the sequence index) and kind.
__device__ inline int first_fault(const Faults& f, bool* overflow) {
  const int j = __builtin_ctz(f.hit);
  *overflow = ((f.ovf >> j) & 1u) != 0u;
  return j;
}

// ---- affine-chain fast path -------------------------------------------------------------------
// Chains whose every stage is `Where(x <cmp> c)` or `Select(x * a + b)` (also x*a, x+b, x-b) are
// lowered to a stage table and run without the interpreter's scratch registers, which lets more
// tiles be resident. Each stage rounds exactly as the interpreter does (x*a, then +b).
constexpr int kMaxAffineStages = 8;
enum AffineKind : uint8_t { kStageFilter = 0, kStageMap = 1 };
// Fields are 32-bit so the kernel reads them with scalar loads (no scalar byte loads on gfx950).
struct AffineChain {
  int32_t n_stages;
  uint32_t kind[kMaxAffineStages];
  uint32_t op[kMaxAffineStages];     // filter: DC_LQ_CMP_*; map: bit0 = has mul, bit1 = has add
  float c0[kMaxAffineStages];        // filter: constant; map: multiplier
  float c1[kMaxAffineStages];        // map: addend
};

template <int EPT>
__device__ inline uint64_t run_affine(const AffineChain& ch, float (&e)[EPT]) {
  uint64_t keep = (EPT == 64) ? ~0ull : ((1ull << EPT) - 1);
  // Unrolled over the stage slots: constant indices keep the table in scalar registers.
#pragma unroll
  for (int s = 0; s < kMaxAffineStages; ++s) {
    if (s >= ch.n_stages) break;
    const float c0 = ch.c0[s], c1 = ch.c1[s];
    if (ch.kind[s] == kStageFilter) {
      uint64_t c = 0;
      switch (ch.op[s]) {
#define DC_AFF_CMP(OPC, EXPR) \
  case OPC: _Pragma("unroll") for (int j = 0; j < EPT; ++j) c |= (uint64_t)(EXPR) << j; break
        DC_AFF_CMP(DC_LQ_CMP_GT, e[j] > c0);
        DC_AFF_CMP(DC_LQ_CMP_GE, e[j] >= c0);
        DC_AFF_CMP(DC_LQ_CMP_LT, e[j] < c0);
        DC_AFF_CMP(DC_LQ_CMP_LE, e[j] <= c0);
        DC_AFF_CMP(DC_LQ_CMP_EQ, e[j] == c0);
        default: DC_AFF_CMP(DC_LQ_CMP_NE, e[j] != c0);
#undef DC_AFF_CMP
      }
      keep &= c;
    } else {
      const uint32_t f = ch.op[s];
      if (f & 1) {
#pragma unroll
        for (int j = 0; j < EPT; ++j) e[j] = e[j] * c0;
      }
      if (f & 2) {
#pragma unroll
        for (int j = 0; j < EPT; ++j) e[j] = e[j] + c1;
      }
    }
  }
  return keep;
}

// kModeInterpLibm: the float interpreter with save registers and the library operations (POW).
enum ProgramMode : int { kModeInterp = 0, kModeInterpSaves = 1, kModeAffine = 2, kModeInterpI32 = 3, kModeInterpI32Saves = 4,
                         kModeInterpLibm = 5 };
constexpr bool mode_is_int(int m) { return m == kModeInterpI32 || m == kModeInterpI32Saves; }

// ---- one- and two-stage affine chains -------------------------------------------------------------
// A chain of one filter `x <cmp> t`, one map `x * a + b`, or one of each in either order is
// lowered to its shape and constants, and the kernels are instantiated per shape and comparison:
// a filter is then one compare per element (a lane mask, no per-element bit packing), a map two
// operations (a missing multiply is a = 1, a missing add b = -0: both exact, so the rounding is the
// interpreter's: x * a, then + b).
enum Shape2 : int { kShapeF = 0, kShapeM = 1, kShapeFM = 2, kShapeMF = 3 };

// Constants of a canonical chain.
struct RdConst {
  float t, a, b;
};

// Program variants of the streaming kernels (ToArray's resident grid, Sum, Min/Max): the
// interpreter (with or without save registers), any affine chain, and the one- and two-stage
// affine chains with the shape and comparison fixed at compile time. Canonical modes are
// kRdCanon + 8 * shape + (comparison - DC_LQ_CMP_GT).
// kRdInterpI32 / kRdInterpI32Saves: the int32 interpreter (programs over int32 elements).
// kRdInterpLibm: the float interpreter with save registers and the library operations (POW).
// kRdJit: the program compiled into the kernel at run time (dc_linq_jit.hip).
enum ReduceMode : int { kRdInterp = 0, kRdInterpSaves = 1, kRdAffine = 2, kRdInterpI32 = 3, kRdInterpI32Saves = 4,
                        kRdInterpLibm = 5, kRdJit = 8, kRdCanon = 16 };
constexpr bool rd_is_int(int rd) { return rd == kRdInterpI32 || rd == kRdInterpI32Saves; }
constexpr bool rd_is_float_interp(int rd) { return rd == kRdInterp || rd == kRdInterpSaves || rd == kRdInterpLibm; }
constexpr int rd_canon(int shape, int cmp) { return kRdCanon + 8 * shape + (cmp - DC_LQ_CMP_GT); }
constexpr bool rd_is_canon(int rd) { return rd >= kRdCanon; }
constexpr int rd_shape(int rd) { return (rd - kRdCanon) >> 3; }
constexpr int rd_cmp(int rd) { return DC_LQ_CMP_GT + ((rd - kRdCanon) & 7); }

template <int CMP>
__device__ __attribute__((always_inline)) inline bool rd_compare(float x, float t) {
  if constexpr (CMP == DC_LQ_CMP_GT) return x > t;
  else if constexpr (CMP == DC_LQ_CMP_GE) return x >= t;
  else if constexpr (CMP == DC_LQ_CMP_LT) return x < t;
  else if constexpr (CMP == DC_LQ_CMP_LE) return x <= t;
  else if constexpr (CMP == DC_LQ_CMP_EQ) return x == t;
  else return x != t;  // true for NaN, as in C#
}

// The program over EPT elements with one flag per element (kept). The canonical modes compute the
// flag with one compare, so it stays a lane mask.
template <int RD, int EPT>
__device__ __attribute__((always_inline)) inline void apply_reduce_flags(const dc_linq_chain& prog,
                                                                         const AffineChain& aff, const RdConst& k,
                                                                         float (&e)[EPT], bool (&kept)[EPT]) {
  if constexpr (rd_is_canon(RD)) {
    constexpr int SHAPE = rd_shape(RD), CMP = rd_cmp(RD);
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      if (SHAPE == kShapeM || SHAPE == kShapeMF) {
        e[j] = e[j] * k.a;
        e[j] = e[j] + k.b;
      }
      kept[j] = SHAPE == kShapeM ? true : rd_compare<CMP>(e[j], k.t);
      if (SHAPE == kShapeFM) {
        e[j] = e[j] * k.a;
        e[j] = e[j] + k.b;
      }
    }
  } else {
    uint32_t keep;
    if constexpr (RD == kRdAffine) keep = (uint32_t)run_affine<EPT>(aff, e);
    else keep = run_program_f32<EPT, RD == kRdInterpSaves || RD == kRdInterpLibm, RD == kRdInterpLibm>(prog, e);
#pragma unroll
    for (int j = 0; j < EPT; ++j) kept[j] = ((keep >> j) & 1u) != 0u;
  }
}

// apply_reduce_flags for every mode, the int32 ones included: elements outside `live` are not kept
// (int32 modes; the float modes are only called on present elements), and the exceptions of an
// int32 program go to `f`.
// The interpreters run over at most CHUNK elements at a time. The round-robin kernel passes all 16
// of a round's elements: each instruction's dispatch then covers twice the elements of 8-element
// chunks, measured at 256M as 737 -> 507 us for a general float program, 940 -> 700 us with save
// registers, 812 -> 694 us for the int32 Where(x % 2 == 0).Select(x * x). With 16 the save-register,
// library and int32 variants keep a few values in scratch (32-176 B per lane), and are still faster.
template <int RD, int EPT, int CHUNK = EPT>
__device__ __attribute__((always_inline)) inline void eval_flags(const dc_linq_chain& prog, const AffineChain& aff,
                                                                 const RdConst& k, float (&e)[EPT], bool (&kept)[EPT],
                                                                 uint32_t live, Faults& f) {
  constexpr bool kInterp = rd_is_int(RD) || rd_is_float_interp(RD);
  constexpr int kInterpChunk = CHUNK;
  if constexpr (kInterp && EPT > kInterpChunk) {
    static_assert(EPT % kInterpChunk == 0, "whole chunks");
    for_each_index([&](auto C) __attribute__((always_inline)) {
      constexpr int c = decltype(C)::value;
      float sub[kInterpChunk];
      bool ks[kInterpChunk];
#pragma unroll
      for (int i = 0; i < kInterpChunk; ++i) sub[i] = e[c * kInterpChunk + i];
      Faults fc;
      eval_flags<RD, kInterpChunk>(prog, aff, k, sub, ks, (live >> (c * kInterpChunk)) & ((1u << kInterpChunk) - 1u), fc);
#pragma unroll
      for (int i = 0; i < kInterpChunk; ++i) {
        e[c * kInterpChunk + i] = sub[i];
        kept[c * kInterpChunk + i] = ks[i];
      }
      f.hit |= fc.hit << (c * kInterpChunk);
      f.ovf |= fc.ovf << (c * kInterpChunk);
    }, std::make_integer_sequence<int, EPT / kInterpChunk>{});
  } else if constexpr (rd_is_int(RD)) {
    const uint32_t keep = run_program_i32<EPT, RD == kRdInterpI32Saves>(prog, e, live, f);
#pragma unroll
    for (int j = 0; j < EPT; ++j) kept[j] = ((keep >> j) & 1u) != 0u;
  } else {
    apply_reduce_flags<RD, EPT>(prog, aff, k, e, kept);
  }
}

// A program compiled into the kernel: Gen::run<EPT>(e, live, f) computes the keep mask of EPT
// elements (held as float bit patterns) exactly as the interpreter would, and Gen::kInt tells
// whether it is an int32 program. NoGen stands in where no program is compiled in.
struct NoGen {
  static constexpr bool kInt = false;
  template <int EPT>
  __device__ static uint32_t run(float (&)[EPT], uint32_t, Faults&) { return 0; }
};

template <int RD, class Gen>
constexpr bool prog_is_int() { return rd_is_int(RD) || (RD == kRdJit && Gen::kInt); }

// eval_flags, or the compiled-in program for RD = kRdJit (which needs no chunking: its straight-line
// code holds only the registers the program uses).
template <int RD, class Gen, int EPT, int CHUNK>
__device__ __attribute__((always_inline)) inline void eval_program(const dc_linq_chain& prog, const AffineChain& aff,
                                                                   const RdConst& k, float (&e)[EPT], bool (&kept)[EPT],
                                                                   uint32_t live, Faults& f) {
  if constexpr (RD == kRdJit) {
    const uint32_t keep = Gen::template run<EPT>(e, live, f);
#pragma unroll
    for (int j = 0; j < EPT; ++j) kept[j] = ((keep >> j) & 1u) != 0u;
  } else {
    eval_flags<RD, EPT, CHUNK>(prog, aff, k, e, kept, live, f);
  }
}

// ---- Where/Select -> ToArray, round-robin kernel for large inputs --------------------------------
// A resident grid of P workgroups (one per CU, all running at once). The workgroup at tile position w
// (w follows the XCDs: see the kernel) owns tile r*P + w of
// round r, so every round is a contiguous stretch of P tiles. Each tile publishes its kept count as
// one epoch-tagged word; the output offset of tile (r, w) is
//     base_r + sum_{w' < w} count(r, w'),   base_{r+1} = base_r + sum_{w'} count(r, w'),
// and every workgroup reads all P counts of a round itself, so no prefix ever has to travel from tile
// to tile (the serial front that limits a decoupled lookback). The loop is software-pipelined:
//   - loads run kRrAhead rounds ahead (kRrAhead + 1 register buffers per lane; 2 for the int32 interpreter);
//   - kept values of a tile wait in LDS for kRrDelay rounds before they are written, and the count
//     words of that round are read one round before the write, so they were published
//     kRrDelay - 2 full rounds earlier and are almost always already visible;
//   - the program is one of the compile-time variants (shape and comparison fixed for the one- and
//     two-stage affine chains): the kernel is bound by its instruction issue at this rate, so
//     the per-element work is kept to a compare, the map, and the ballot ranking.
// Roles inside the 576-thread workgroup: waves 0..7 each own a contiguous 1024-element chunk of every
// tile, rank their kept elements with ballot + mbcnt, stage them in a private LDS ring (in input
// order) and later write them as one contiguous run; wave 8 reads and checks the count words and
// broadcasts the output offset. The last wave to finish a tile (an LDS atomic) publishes its count.
// One workgroup barrier per round. Wave w runs on SIMD w mod 4 and a SIMD issues for its oldest
// ready wave first, so the control wave is the youngest: it shares SIMD 0 with workers 0 and 4
// without delaying them (as wave 0 it made worker 8 the slowest wave of every workgroup and
// every round waited for it: 274.6 against 267.5 us at 256M, 50 % kept).
// Geometry (measured at 256M, 50% kept: 8 workers x 4 vectors 290 us, 15 x 2 293 us, 12 x 3 297 us):
// fewer, wider worker waves spread the per-round fixed work (ranking tables, the barrier) over
// more elements.
constexpr int kRrBlock = 9 * dc::kWave;
constexpr int kRrWorkers = kRrBlock / dc::kWave - 1;     // 8 worker waves
constexpr int kRrVec = 4;                                // 16-byte loads per lane per tile
constexpr int kRrEpt = 4 * kRrVec;                       // 16 elements per lane
constexpr int kRrChunk = dc::kWave * kRrEpt;             // 1024 elements per worker wave
constexpr int64_t kRrTile = (int64_t)kRrWorkers * kRrChunk;  // 8192 elements = 32 KiB
constexpr int kRrAhead = 4;
constexpr int kRrDelay = 3;
constexpr int kRrRing = (kRrDelay + 1) * kRrChunk;       // floats per worker wave: 16 KiB, 130 KiB per workgroup
constexpr int kRrCountsPerLane = 4;
constexpr int kRrMaxGroups = dc::kWave * kRrCountsPerLane;  // P <= 256
constexpr uint32_t kRrSpinLimit = 1u << 22;              // ~seconds: a wait that never ends reports
static_assert((kRrDelay + 1) * kRrChunk <= kRrRing, "the ring holds every staged tile at 100% selectivity");
static_assert(kRrDelay < 8 && kRrDelay >= 2, "per-tile LDS tables are indexed modulo 8");


// Count words of `round` for workgroups q*64 + lane (q < 4): four coalesced 256-byte loads.
__device__ inline void rr_issue_counts(uint32_t (&c)[kRrCountsPerLane], const uint32_t* __restrict__ counts,
                                       uint32_t round, uint32_t P) {
  const uint32_t lane = threadIdx.x & 63;
#pragma unroll
  for (int q = 0; q < kRrCountsPerLane; ++q) {
    const uint32_t g = q * 64 + lane;
    c[q] = g < P ? dc::load_agent_u32(counts + (size_t)round * P + g) : 0u;
  }
}

// The control wave: re-reads until every count word of `round` carries this launch's epoch (bounded), then
// returns the sum of the counts of workgroups before `me` and the round total.
__device__ inline bool rr_resolve(uint32_t (&c)[kRrCountsPerLane], const uint32_t* __restrict__ counts, uint32_t round,
                                  uint32_t P, uint32_t epoch16, uint32_t me, uint32_t* pref, uint32_t* total) {
  const uint32_t lane = threadIdx.x & 63;
  for (uint32_t spin = 0;; ++spin) {
    bool missing = false;
#pragma unroll
    for (int q = 0; q < kRrCountsPerLane; ++q) missing |= (q * 64 + lane < P) && ((c[q] >> 16) != epoch16);
    if (!__ballot(missing)) break;
    if (spin == kRrSpinLimit) return false;
    __builtin_amdgcn_s_sleep(4);
    rr_issue_counts(c, counts, round, P);
  }
  uint32_t p = 0, t = 0;
#pragma unroll
  for (int q = 0; q < kRrCountsPerLane; ++q) {
    const uint32_t g = q * 64 + lane;
    const uint32_t v = g < P ? (c[q] & 0xFFFFu) : 0u;
    t += v;
    p += g < me ? v : 0u;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    t += __shfl_xor(t, off, 64);
    p += __shfl_xor(p, off, 64);
  }
  *pref = p;
  *total = t;
  return true;
}

// `head_in` holds the head_n (0..3) elements of a 4-byte aligned input that come before its first
// 16-byte boundary; `in` (16-byte aligned) holds the n elements after them. Every control wave
// evaluates the head itself (its kept count is the output offset of round 0) and workgroup 0 writes
// its kept elements first.
// RD = kRdJit: the program is compiled in (Gen::run, see NoGen); prog, aff and canon are unused.
// The kernels are thin wrappers around this body (the prebuilt where_select_rounds_kernel<RD> in
// dc_linq.hip, and the kernel compiled at run time for one program).
template <int RD, class Gen>
__device__ __attribute__((always_inline)) inline void rounds_body(
    const dc_linq_chain& prog, const AffineChain& aff, const RdConst& canon, const float* __restrict__ in, int64_t n,
    float* __restrict__ out,
    int64_t* __restrict__ count_out, uint32_t* __restrict__ counts, uint32_t epoch16, uint32_t P,
    uint32_t* __restrict__ done, uint64_t* __restrict__ fault, const float* __restrict__ head_in, int head_n) {
  constexpr bool kIntProg = prog_is_int<RD, Gen>();
  __shared__ float s_ring[kRrWorkers][kRrRing + dc::kWave];  // + a discard slot per lane
  // ring positions stay in [0, kRrRing); a position below 2 * kRrRing wraps with one unsigned min
  auto wrap = [](uint32_t q) __attribute__((always_inline)) {
    if constexpr ((kRrRing & (kRrRing - 1)) == 0) return q & (uint32_t)(kRrRing - 1);
    else return min(q, q - (uint32_t)kRrRing);
  };
  // Filter-then-map chains stage the raw value and map it when the run is written: only the
  // kept elements pay for the map.
  constexpr bool kLazyMap = rd_is_canon(RD) && rd_shape(RD) == kShapeFM;
  // int32 programs: the lane's first exception over every round, as ~(4 * index + kind) (0 = none),
  // published once at the end, so the round loop stays free of branches.
  uint64_t lane_fault = 0;
  // `first` = sequence index of element 0 of this lane's chunk of the tile; element 4j + k sits at
  // first + 256 j + k. `live` = the elements that exist.
  auto apply = [&](float (&e)[kRrEpt], bool (&kept)[kRrEpt], int64_t first, uint32_t live)
                   __attribute__((always_inline)) {
    if constexpr (kLazyMap) {
#pragma unroll
      for (int j = 0; j < kRrEpt; ++j) kept[j] = rd_compare<rd_cmp(RD)>(e[j], canon.t);
    } else if constexpr (kIntProg || rd_is_float_interp(RD) || RD == kRdJit) {
      Faults f;
      eval_program<RD, Gen, kRrEpt, kRrEpt>(prog, aff, canon, e, kept, live, f);
      if constexpr (kIntProg) {
        const int b = __builtin_ctz(f.hit | 0x80000000u);
        const uint64_t code = (uint64_t)(head_n + first + (b >> 2) * (4 * dc::kWave) + (b & 3)) * 4u +
                              (((f.ovf >> b) & 1u) ? DC_LINQ_FAULT_OVERFLOW : DC_LINQ_FAULT_DIVIDE_BY_ZERO);
        lane_fault = max(lane_fault, f.hit ? ~code : (uint64_t)0);
      }
    } else {
      apply_reduce_flags<RD, kRrEpt>(prog, aff, canon, e, kept);
    }
  };
  __shared__ uint32_t s_wcount[8][16];  // kept count of (tile slot, worker wave)
  __shared__ uint32_t s_acc[8];         // (waves finished << 24) | kept so far, per tile slot
  __shared__ int64_t s_off[2];          // output offset of the tile being written, by round parity
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // This workgroup's tile position in every round. Workgroups go to the XCDs round-robin, so
  // positions are dealt out XCD by XCD: consecutive tiles (and the partly written cache line
  // where one tile's output ends and the next one's begins) then share one XCD's L2, which merges
  // the two halves of that line before it is written back.
  const uint32_t w = (P % 8u == 0u) ? (blockIdx.x % 8u) * (P / 8u) + blockIdx.x / 8u : blockIdx.x;
  const int64_t num_tiles = (n + kRrTile - 1) / kRrTile;
  // Rounds in which every tile is full. A grid with one tile per workgroup (fewer tiles than CUs)
  // runs its only round as the tail round: no pipeline to fill and drain.
  const uint32_t R0 = (n / kRrTile) / P == 1 && num_tiles == P ? 0u : (uint32_t)((n / kRrTile) / P);
  const uint32_t rounds = R0 > 0 ? R0 + kRrDelay : 0;
  const bool tail_round = (int64_t)R0 * P < num_tiles;
  if (tid < 8) s_acc[tid] = 0;
  __syncthreads();

  if (wave == kRrWorkers) {
    // ---------------- control wave (the youngest wave: see the roles above)
    int64_t base = 0;
    if (head_n > 0) {  // the peeled head: lane l evaluates element l
      const bool present = lane < head_n;
      float e[1] = {present ? head_in[lane] : 0.0f};
      bool kept[1];
      Faults f;
      eval_program<RD, Gen, 1, 1>(prog, aff, canon, e, kept, present ? 1u : 0u, f);
      const bool k = kept[0] && present;
      const uint64_t b = __ballot(k);
      if (w == 0 && k)
        out[__builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u))] = e[0];
      if (kIntProg && f.hit) publish_fault(fault, lane, (f.ovf & 1u) != 0u);
      base = __builtin_popcountll(b);
    }
    uint32_t c[kRrCountsPerLane];
    bool ok = true;
    for (uint32_t r = 0; r < rounds; ++r) {
      if (r >= (uint32_t)kRrDelay) {
        uint32_t pf = 0, tt = 0;
        if (ok && !rr_resolve(c, counts, r - kRrDelay, P, epoch16, w, &pf, &tt)) ok = false;
        if (lane == 0) s_off[r & 1] = base + pf;
        base += tt;
      }
      if (r + 1 >= (uint32_t)kRrDelay && r + 1 - kRrDelay < R0) rr_issue_counts(c, counts, r + 1 - kRrDelay, P);
      if (lane == 0) s_acc[(r + 1) & 7] = 0;
      __syncthreads();
    }
    if (tail_round) {
      __syncthreads();  // the workers published the tail round's counts
      uint32_t pf = 0, tt = 0;
      rr_issue_counts(c, counts, R0, P);
      if (ok && !rr_resolve(c, counts, R0, P, epoch16, w, &pf, &tt)) ok = false;
      if (lane == 0) s_off[0] = base + pf;
      base += tt;
      __syncthreads();
    }
    if (lane == 0) {
      // Completion word: low 16 bits count finished workgroups, the rest counts failed ones. The last
      // workgroup writes the total (every workgroup holds the same base) or -1 if any wait gave up.
      // Relaxed: the last workgroup reads nothing the others wrote except this word (every
      // workgroup holds the same base), and an agent-scope release here would write back the
      // XCD's L2 once per workgroup.
      const uint32_t add = 1u | (ok ? 0u : (1u << 16));
      const uint32_t prev = __hip_atomic_fetch_add(done, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if ((prev & 0xFFFFu) == P - 1) {
        *count_out = ((prev >> 16) == 0 && ok) ? base : (int64_t)-1;
        dc::store_agent_u32(done, 0u);
      }
    }
    return;
  }

  // ---------------- worker waves
  const int ww = wave;
  float* ring = s_ring[ww];
  uint32_t head = 0, tail = 0;
  const int64_t chunk = (int64_t)ww * kRrChunk;

  auto load = [&](float (&e)[kRrEpt], uint32_t round) __attribute__((always_inline)) {
    const dc::f32x4* in4 = reinterpret_cast<const dc::f32x4*>(in + ((int64_t)round * P + w) * kRrTile + chunk);
#pragma unroll
    for (int j = 0; j < kRrVec; ++j) {
      const dc::f32x4 x = dc::load_stream(in4 + j * dc::kWave + lane);
      e[4 * j] = x.x; e[4 * j + 1] = x.y; e[4 * j + 2] = x.z; e[4 * j + 3] = x.w;
    }
  };
  // Ranks the kept elements of this wave's chunk (order: vector j, lane, slot k), appends them to the
  // ring, and publishes the tile count when this is the last worker wave to finish the tile.
  auto stage = [&](float (&e)[kRrEpt], const bool (&kept)[kRrEpt], uint32_t r) __attribute__((always_inline)) {
    uint32_t run = 0, pos[kRrVec];
#pragma unroll
    for (int j = 0; j < kRrVec; ++j) {
      uint32_t below = 0, total = 0;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint64_t b = __ballot(kept[4 * j + k]);
        below += __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
        total += (uint32_t)__builtin_popcountll(b);
      }
      pos[j] = run + below;
      run += total;
    }
#pragma unroll
    for (int j = 0; j < kRrVec; ++j) {
      uint32_t p = head + pos[j];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        // branch-free: a dropped element goes to the lane's discard slot past the ring
        const uint32_t q = kept[4 * j + k] ? wrap(p) : (uint32_t)(kRrRing + lane);
        ring[q] = e[4 * j + k];
        p += kept[4 * j + k] ? 1u : 0u;
      }
    }
    head = wrap(head + run);
    if (lane == 0) {
      s_wcount[r & 7][ww] = run;
      const uint32_t prev = atomicAdd(&s_acc[r & 7], (1u << 24) | run);
      if ((prev >> 24) == kRrWorkers - 1)
        dc::store_agent_u32(counts + (size_t)r * P + w, (epoch16 << 16) | ((prev & 0xFFFFFFu) + run));
    }
  };
  // Writes this wave's staged run of the tile of round q at its place in the output.
  auto write = [&](uint32_t q, uint32_t parity) __attribute__((always_inline)) {
    const uint32_t slot = q & 7;
    uint32_t cnt = 0, before = 0;
#pragma unroll
    for (int i = 0; i < kRrWorkers; ++i) {
      const uint32_t c = s_wcount[slot][i];
      before += i < ww ? c : 0u;
      cnt = i == ww ? c : cnt;
    }
    float* dst = out + s_off[parity] + before;
    for (uint32_t i = lane; i < cnt; i += dc::kWave) {
      float v = ring[wrap(tail + i)];
      if constexpr (kLazyMap) {
        v = v * canon.a;
        v = v + canon.b;
      }
      dst[i] = v;
    }
    tail = wrap(tail + cnt);
  };

  // Every load below is unconditional: rounds past the last one re-load round R0 - 1 (loaded one
  // round earlier, so mostly served by the cache). The compiler's memory-counter waits are
  // path-insensitive: on a path that skipped a later load, the wait for the round being staged
  // would have to cover every load still in flight, draining the pipeline.
  const uint32_t last = R0 > 0 ? R0 - 1 : 0;
  // Rounds of look-ahead: kRrAhead, or 2 for the interpreters: the int32 one's per-chunk state with
  // five buffers exceeded the 168 registers a lane may hold here and spilled to scratch, and the
  // float ones ran 3-33 % faster with two (149 -> 116 VGPRs without save registers, 165 -> 132 with
  // them, and no scratch for the library variant). Two rounds measured as fast as four on the
  // headline kernel, so the depth is not what bounds these kernels.
  constexpr int kAhead = (kIntProg || rd_is_float_interp(RD)) && RD != kRdJit ? 2 : kRrAhead;
  constexpr int kBufs = kAhead + 1;
  float e[kBufs][kRrEpt];  // register buffers: constant indices only, after full unrolling
  if (R0 > 0)
    for_each_index([&](auto U) __attribute__((always_inline)) { load(e[U.value], min((uint32_t)U.value, last)); },
                   std::make_integer_sequence<int, kAhead>{});
  uint32_t r = 0;
  // One round: issue the loads of round r + kAhead into buffer `en`, stage round r from `ec`,
  // write round r - kRrDelay. Unrolled kBufs ways so the buffers rotate without copies. The main
  // loop runs whole kBufs-round iterations with no early exit: a `break` between rounds becomes a
  // path back to the loop head after a partial iteration, and the waits at the head would then
  // assume fewer loads in flight than a full iteration leaves. The last R0 % kBufs rounds follow.
  auto round = [&](float (&ec)[kRrEpt], float (&en)[kRrEpt]) __attribute__((always_inline)) {
    load(en, min(r + kAhead, last));
    bool kept[kRrEpt];
    apply(ec, kept, ((int64_t)r * P + w) * kRrTile + chunk + 4 * lane, ~0u);
    stage(ec, kept, r);
    __syncthreads();
    if (r >= (uint32_t)kRrDelay) write(r - kRrDelay, r & 1);
    ++r;
  };
  for (uint32_t it = R0 / kBufs; it > 0; --it)
    for_each_index([&](auto U) __attribute__((always_inline)) { round(e[U.value], e[(U.value + kAhead) % kBufs]); },
                   std::make_integer_sequence<int, kBufs>{});
  for_each_index([&](auto U) __attribute__((always_inline)) { if (r < R0) round(e[U.value], e[(U.value + kAhead) % kBufs]); },
                 std::make_integer_sequence<int, kAhead>{});
  for (; r < rounds; ++r) {  // drain: the last kRrDelay staged tiles (fewer when R0 < kRrDelay)
    __syncthreads();
    if (r >= (uint32_t)kRrDelay) write(r - kRrDelay, r & 1);
  }
  if (tail_round) {  // tiles R0*P .. num_tiles-1 (full, partial or none), bounded loads
    const int64_t t = (int64_t)R0 * P + w;
    float e[kRrEpt];
    uint32_t valid = 0;
#pragma unroll
    for (int j = 0; j < kRrVec; ++j) {
      const int64_t at = t * kRrTile + chunk + j * 4 * dc::kWave + 4 * lane;
      const int64_t nv = t < num_tiles ? min(max(n - at, (int64_t)0), (int64_t)4) : 0;
      if (nv == 4) {  // a whole vector (in is 16-byte aligned)
        const dc::f32x4 v = dc::load_stream(reinterpret_cast<const dc::f32x4*>(in + at));
        e[4 * j] = v.x; e[4 * j + 1] = v.y; e[4 * j + 2] = v.z; e[4 * j + 3] = v.w;
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) e[4 * j + k] = k < nv ? in[at + k] : 0.0f;
      }
      valid |= ((1u << (uint32_t)nv) - 1u) << (4 * j);
    }
    bool kept[kRrEpt];
    apply(e, kept, t * kRrTile + chunk + 4 * lane, valid);
#pragma unroll
    for (int i = 0; i < kRrEpt; ++i) kept[i] = kept[i] && ((valid >> i) & 1u);
    stage(e, kept, R0);
    __syncthreads();
    __syncthreads();
    write(R0, 0);
  }
  if constexpr (kIntProg) {
    if (lane_fault) __hip_atomic_fetch_max(fault, lane_fault, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}


}  // namespace dclq

// dc_linq.hip — fused LINQ Where/Select(/Sum) kernels for gfx950.
//
// One prebuilt kernel per terminal (ToArray, Sum) interprets the register program that the host
// fusion planner builds from the chain's lambdas (dc_linq_chain, program model in
// include/dotcompute_hip.h). The program lives in the kernel arguments, so every instruction is
// wave-uniform: dispatch is scalar branching, and each instruction is applied to the 16 elements a
// thread holds in registers.
//
// ToArray (order-preserving stream compaction, one pass over the input), two kernels:
//  - large 16-byte aligned inputs: the round-robin kernel (where_select_rounds_kernel, described
//    at its definition): a resident grid, one workgroup per CU, tile counts published per round
//    and summed by every workgroup, so no prefix travels from tile to tile;
//  - everything else: a ticket-ordered grid with a decoupled lookback. tile = 512 threads x 32
//    elements = 16384 consecutive elements (64 KiB), claimed through an atomic ticket (so a tile
//    only ever waits on tiles that started before it); thread t loads 16-byte vectors j = 0..7 at
//    tile + j*2048 + t*4; for each vector j and slot k the wave takes ballot(keep) -> the element's
//    rank among the kept elements of (j, wave) is sum_k' mbcnt(ballot_k') + (kept slots k'' < k of
//    this thread); the 64 (j, wave) counts are scanned in LDS -> tile-local positions; the tile
//    aggregate is published for decoupled lookback and the tile's exclusive prefix is resolved by
//    wave 0 from the status words of up to 256 predecessors per round.
// Every float operation rounds once (the file is compiled with -ffp-contract=off), so the output
// equals LINQ-to-objects bit-for-bit.
#include <algorithm>
#include <map>
#include <mutex>

#include <utility>

#include "dc_device.hpp"
#include "dc_internal.hpp"

namespace {

constexpr int kBlock = 512;                        // compaction workgroup: 8 waves
constexpr int kWaves = kBlock / dc::kWave;
constexpr int kVecPerThread = 8;
constexpr int kElemPerThread = 4 * kVecPerThread;  // 32
constexpr int kTile = kBlock * kElemPerThread;     // 16384 elements = 64 KiB of input
constexpr int kChunk = 16;                         // elements interpreted per program pass
constexpr int kLookbackPerLane = 4;                // status words read per lane per lookback round
constexpr int kSumBlocksMax = 1024;

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
  uint32_t op, src, mode;
  float imm;
};
__device__ inline Instr fetch_instr(const dc_linq_chain& prog, int pc) {
  const uint32_t* w = reinterpret_cast<const uint32_t*>(&prog.code[pc]);
  const uint32_t w0 = w[0];
  return Instr{w0 & 0xFFu, (w0 >> 8) & 0xFFu, (w0 >> 16) & 0xFFu, __builtin_bit_cast(float, w[1])};
}

// Runs the program over the EPT elements of one thread. Returns the keep mask (bit j = element j).
// SAVES = false drops the s0/s1 registers for programs that never use them (the common case),
// which keeps the kernels at a higher occupancy. Operands are read in place (an immediate stays a
// scalar operand of the vector instruction), so no per-element operand copy is materialised.
template <int EPT, bool SAVES>
__device__ __attribute__((always_inline)) inline uint32_t run_program(const dc_linq_chain& prog, float (&e)[EPT]) {
  float v[EPT];
  float s0[SAVES ? EPT : 1], s1[SAVES ? EPT : 1];
#pragma unroll
  for (int j = 0; j < EPT; ++j) v[j] = 0.0f;
#pragma unroll
  for (int j = 0; j < (SAVES ? EPT : 1); ++j) { s0[j] = 0.0f; s1[j] = 0.0f; }
  uint32_t p = 0, q = 0, keep = (EPT == 32) ? 0xFFFFFFFFu : ((1u << EPT) - 1u);
  const int n = prog.n_instr;
  for (int pc = 0; pc < n; ++pc) {
    const Instr ins = fetch_instr(prog, pc);
    uint32_t c = 0;
    bool is_cmp = false;
// Applies `body` (which reads the operand as O) to every element, for the instruction's source.
#define DC_LQ_APPLY(body)                                                                   \
  do {                                                                                      \
    if (ins.src == DC_LQ_SRC_ELEM) {                                                        \
      _Pragma("unroll") for (int j = 0; j < EPT; ++j) { const float O = e[j]; body; }       \
    } else if (SAVES && ins.src == DC_LQ_SRC_S0) {                                          \
      _Pragma("unroll") for (int j = 0; j < EPT; ++j) { const float O = s0[SAVES ? j : 0]; body; } \
    } else if (SAVES && ins.src == DC_LQ_SRC_S1) {                                          \
      _Pragma("unroll") for (int j = 0; j < EPT; ++j) { const float O = s1[SAVES ? j : 0]; body; } \
    } else {                                                                                \
      const float O = ins.imm;                                                              \
      _Pragma("unroll") for (int j = 0; j < EPT; ++j) { body; }                             \
    }                                                                                       \
  } while (0)
    switch (ins.op) {
      case DC_LQ_LOAD: DC_LQ_APPLY(v[j] = O); break;
      case DC_LQ_ADD: DC_LQ_APPLY(v[j] = v[j] + O); break;
      case DC_LQ_SUB: DC_LQ_APPLY(v[j] = v[j] - O); break;
      case DC_LQ_RSUB: DC_LQ_APPLY(v[j] = O - v[j]); break;
      case DC_LQ_MUL: DC_LQ_APPLY(v[j] = v[j] * O); break;
      case DC_LQ_DIV: DC_LQ_APPLY(v[j] = v[j] / O); break;
      case DC_LQ_RDIV: DC_LQ_APPLY(v[j] = O / v[j]); break;
      case DC_LQ_MIN: DC_LQ_APPLY(v[j] = net_min(v[j], O)); break;
      case DC_LQ_MAX: DC_LQ_APPLY(v[j] = net_max(v[j], O)); break;
      case DC_LQ_NEG:
#pragma unroll
        for (int j = 0; j < EPT; ++j) v[j] = -v[j];
        break;
      case DC_LQ_ABS:
#pragma unroll
        for (int j = 0; j < EPT; ++j) v[j] = __builtin_fabsf(v[j]);
        break;
      case DC_LQ_SQRT:
#pragma unroll
        for (int j = 0; j < EPT; ++j) v[j] = __builtin_sqrtf(v[j]);
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
  return keep;
}

// True when the program reads or writes s0/s1 (selects the larger kernel variant).
inline bool program_uses_saves(const dc_linq_chain& prog) {
  for (int i = 0; i < prog.n_instr; ++i) {
    const dc_linq_instr& in = prog.code[i];
    if (in.op == DC_LQ_STORE_S0 || in.op == DC_LQ_STORE_S1) return true;
    if (in.src == DC_LQ_SRC_S0 || in.src == DC_LQ_SRC_S1) return true;
  }
  return false;
}

// ---- decoupled lookback -------------------------------------------------------------------------
// Status word: [63:62] flag (0 invalid, 1 aggregate, 2 inclusive prefix) | [61:40] epoch |
// [39:0] value. A word whose epoch differs from the launch's counts as invalid.
constexpr uint64_t kFlagAgg = 1ull << 62;
constexpr uint64_t kFlagInc = 2ull << 62;
constexpr uint64_t kValueMask = (1ull << 40) - 1;

__device__ inline uint64_t pack_status(uint64_t flag, uint32_t epoch, uint64_t value) {
  return flag | ((uint64_t)epoch << 40) | (value & kValueMask);
}

// Tile 0 publishes its inclusive prefix at once; every other tile first publishes its aggregate.
__device__ inline void publish_aggregate(uint64_t* __restrict__ status, int64_t tile, uint64_t aggregate,
                                         uint32_t epoch) {
  dc::store_agent_u64(status + tile, pack_status(tile == 0 ? kFlagInc : kFlagAgg, epoch, aggregate));
}

// Called by all 64 lanes of one wave after publish_aggregate. Returns the exclusive prefix of `tile`
// (valid in every lane) and publishes the tile's inclusive prefix. Each round reads the status of
// the 256 nearest unresolved predecessors (lane l: tiles end - 4l .. end - 4l - 3) and stops at
// the nearest inclusive prefix, adding the aggregates in between. Wide rounds matter: while the
// tiles in flight outrun the prefix front, every tile has to fold all aggregates between itself
// and the front, and each round costs one agent-scope round trip. A tile only waits on tiles with
// smaller tickets, which are all owned by running workgroups, so the wait always ends.
__device__ inline int64_t lookback(uint64_t* __restrict__ status, int64_t tile, uint64_t aggregate, uint32_t epoch) {
  if (tile == 0) return 0;
  constexpr int P = kLookbackPerLane;
  const int lane = threadIdx.x & 63;
  int64_t exclusive = 0;
  int64_t end = tile - 1;
  while (true) {
    uint64_t w[P];
#pragma unroll
    for (int q = 0; q < P; ++q) {
      const int64_t idx = end - (int64_t)(P * lane + q);
      w[q] = idx >= 0 ? dc::load_agent_u64(status + idx) : pack_status(kFlagInc, epoch, 0);
    }
    // Per lane: first inclusive slot (P if none), whether a not-yet-published slot precedes it,
    // and the sum of the values up to and including it.
    int first_inc = P;
    bool bad = false;
    int64_t part = 0;
#pragma unroll
    for (int q = P - 1; q >= 0; --q) {
      const uint32_t w_epoch = (uint32_t)((w[q] >> 40) & ((1u << 22) - 1));
      const uint64_t flag = w[q] & (3ull << 62);
      const bool valid = (flag != 0) && (w_epoch == epoch);
      if (valid && flag == kFlagInc) first_inc = q;
    }
#pragma unroll
    for (int q = 0; q < P; ++q) {
      if (q <= first_inc || first_inc == P) {
        const uint32_t w_epoch = (uint32_t)((w[q] >> 40) & ((1u << 22) - 1));
        const uint64_t flag = w[q] & (3ull << 62);
        const bool valid = (flag != 0) && (w_epoch == epoch);
        bad |= !valid && (q < first_inc || first_inc == P);
        part += (int64_t)(w[q] & kValueMask);
      }
    }
    const uint64_t inc_mask = __ballot(first_inc < P);
    const uint64_t bad_mask = __ballot(bad);
    const int limit = inc_mask ? __builtin_ctzll(inc_mask) : 63;  // lanes [0, limit] are needed
    const uint64_t need = (limit == 63) ? ~0ull : ((2ull << limit) - 1);
    if (bad_mask & need) {
      __builtin_amdgcn_s_sleep(1);
      continue;
    }
    exclusive += dc::wave_sum64<int64_t>(lane <= limit ? part : (int64_t)0);
    if (inc_mask) break;
    end -= 64 * P;
  }
  if (lane == 0) dc::store_agent_u64(status + tile, pack_status(kFlagInc, epoch, (uint64_t)exclusive + aggregate));
  return exclusive;
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

// Host-side lowering; returns false when the program is not an affine chain.
inline bool lower_affine(const dc_linq_chain& prog, AffineChain* out) {
  AffineChain a{};
  int pc = 0;
  while (pc < prog.n_instr) {
    if (a.n_stages == kMaxAffineStages) return false;
    const dc_linq_instr* c = &prog.code[pc];
    if (c->op != DC_LQ_LOAD || c->src != DC_LQ_SRC_ELEM) return false;
    ++pc;
    if (pc + 1 < prog.n_instr && prog.code[pc].op >= DC_LQ_CMP_GT && prog.code[pc].op <= DC_LQ_CMP_NE &&
        prog.code[pc].src == DC_LQ_SRC_IMM && prog.code[pc].mode == DC_LQ_CMP_SET && prog.code[pc + 1].op == DC_LQ_FILTER) {
      a.kind[a.n_stages] = kStageFilter;
      a.op[a.n_stages] = prog.code[pc].op;
      a.c0[a.n_stages] = prog.code[pc].imm;
      ++a.n_stages;
      pc += 2;
      continue;
    }
    uint8_t flags = 0;
    float mul = 1.0f, add = 0.0f;
    if (pc < prog.n_instr && prog.code[pc].op == DC_LQ_MUL && prog.code[pc].src == DC_LQ_SRC_IMM) {
      flags |= 1;
      mul = prog.code[pc].imm;
      ++pc;
    }
    if (pc < prog.n_instr && prog.code[pc].src == DC_LQ_SRC_IMM &&
        (prog.code[pc].op == DC_LQ_ADD || prog.code[pc].op == DC_LQ_SUB)) {
      flags |= 2;
      // x - b is computed as x + (-b): negating the constant is exact, so the rounding is the same.
      add = prog.code[pc].op == DC_LQ_ADD ? prog.code[pc].imm : -prog.code[pc].imm;
      ++pc;
    }
    if (pc >= prog.n_instr || prog.code[pc].op != DC_LQ_MAP) return false;
    ++pc;
    a.kind[a.n_stages] = kStageMap;
    a.op[a.n_stages] = flags;
    a.c0[a.n_stages] = mul;
    a.c1[a.n_stages] = add;
    ++a.n_stages;
  }
  *out = a;
  return true;
}

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

enum ProgramMode : int { kModeInterp = 0, kModeInterpSaves = 1, kModeAffine = 2 };

// Sets bit j of `mask` to p with one v_lshl_or_b32 (inline shift amount). Written as plain C the
// compiler turns each bit into a select between 0 and the literal 1 << j and hoists those literals
// into loop-invariant registers (a register per bit).
__device__ inline uint32_t insert_bit(uint32_t mask, bool p, int j) {
  uint32_t r;
  asm volatile("v_lshl_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"((uint32_t)p), "i"(j), "v"(mask));
  return r;
}

// ---- one- and two-stage affine chains in a branch-free canonical form ------------------------------
// Used by the round-robin kernel, whose software pipeline only keeps its loads in flight across
// rounds when the per-tile code has no branches (a branch makes the compiler's wait counts
// conservative and it then waits for every outstanding load once per unrolled loop).
//   filter:  y = x * sign;  keep = ((y >= c) & A) ^ ((y > c) & B) ^ C        (A, B, C in {0, 1})
//            x > t : sign  1, c  t, A 0 B 1 C 0      x >= t: sign  1, c  t, A 1 B 0 C 0
//            x < t : sign -1, c -t, A 0 B 1 C 0      x <= t: sign -1, c -t, A 1 B 0 C 0
//            x == t: sign  1, c  t, A 1 B 1 C 0      x != t: sign  1, c  t, A 1 B 1 C 1
//            (x * -1 and -t are exact, NaN compares false, and == is ge ^ gt, so every case
//            equals the direct comparison bit for bit, signed zeros and NaN included)
//   map:     x = x * a; x = x + b   (a missing multiply is a = 1, a missing add is b = -0: both exact)
enum Shape2 : int { kShapeF = 0, kShapeM = 1, kShapeFM = 2, kShapeMF = 3 };
struct Canon2 {
  float sign, c, a, b;
  uint32_t A, B, C;
};

inline bool lower_canon2(const AffineChain& ch, Canon2* out, int* shape) {
  const int n = ch.n_stages;
  if (n < 1 || n > 2 || (n == 2 && ch.kind[0] == ch.kind[1])) return false;
  Canon2 k{1.0f, 0.0f, 1.0f, -0.0f, 0u, 0u, 1u};
  for (int s = 0; s < n; ++s) {
    if (ch.kind[s] == kStageFilter) {
      const float t = ch.c0[s];
      switch (ch.op[s]) {
        case DC_LQ_CMP_GT: k.sign = 1.0f; k.A = 0; k.B = 1; k.C = 0; break;
        case DC_LQ_CMP_GE: k.sign = 1.0f; k.A = 1; k.B = 0; k.C = 0; break;
        case DC_LQ_CMP_LT: k.sign = -1.0f; k.A = 0; k.B = 1; k.C = 0; break;
        case DC_LQ_CMP_LE: k.sign = -1.0f; k.A = 1; k.B = 0; k.C = 0; break;
        case DC_LQ_CMP_EQ: k.sign = 1.0f; k.A = 1; k.B = 1; k.C = 0; break;
        case DC_LQ_CMP_NE: k.sign = 1.0f; k.A = 1; k.B = 1; k.C = 1; break;
        default: return false;
      }
      k.c = k.sign < 0.0f ? -t : t;
    } else {
      k.a = (ch.op[s] & 1u) ? ch.c0[s] : 1.0f;
      k.b = (ch.op[s] & 2u) ? ch.c1[s] : -0.0f;
    }
  }
  *shape = n == 1 ? (ch.kind[0] == kStageFilter ? kShapeF : kShapeM)
                  : (ch.kind[0] == kStageFilter ? kShapeFM : kShapeMF);
  *out = k;
  return true;
}

template <int SHAPE, int EPT>
__device__ inline uint32_t run_canon2(const Canon2& k, float (&e)[EPT]) {
  static_assert(EPT < 32, "keep mask");
  uint32_t keep = SHAPE == kShapeM ? ((1u << EPT) - 1u) : 0u;
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    if (SHAPE == kShapeM || SHAPE == kShapeMF) {
      e[j] = e[j] * k.a;
      e[j] = e[j] + k.b;
    }
    if (SHAPE != kShapeM) {
      const float y = e[j] * k.sign;
      const uint32_t ge = y >= k.c, gt = y > k.c;
      keep = insert_bit(keep, (((ge & k.A) ^ (gt & k.B) ^ k.C) & 1u) != 0u, j);
    }
    if (SHAPE == kShapeFM) {
      e[j] = e[j] * k.a;
      e[j] = e[j] + k.b;
    }
  }
  return keep;
}

// Round-robin kernel variants: the interpreter (with or without save registers) and the four
// canonical shapes.
enum RoundsMode : int { kRrInterp = 0, kRrInterpSaves = 1, kRrF = 2, kRrM = 3, kRrFM = 4, kRrMF = 5 };

template <int MODE, int EPT>
__device__ __attribute__((always_inline)) inline uint32_t apply_rounds(const dc_linq_chain& prog, const Canon2& k, float (&e)[EPT]) {
  if constexpr (MODE == kRrF) return run_canon2<kShapeF, EPT>(k, e);
  else if constexpr (MODE == kRrM) return run_canon2<kShapeM, EPT>(k, e);
  else if constexpr (MODE == kRrFM) return run_canon2<kShapeFM, EPT>(k, e);
  else if constexpr (MODE == kRrMF) return run_canon2<kShapeMF, EPT>(k, e);
  else return run_program<EPT, MODE == kRrInterpSaves>(prog, e);
}

// ---- Where/Select -> ToArray ------------------------------------------------------------------
// One tile per workgroup, claimed by ticket. Element order inside a tile is (vector j, wave, lane,
// slot k): thread t loads 16-byte vectors j = 0..7 at tile + 2048 j + 4 t. After the lookback each
// wave compacts the kept elements of one (j, wave) group through a 1 KiB LDS buffer and writes the
// group's contiguous output run with fully coalesced stores.
__device__ inline uint32_t take_ticket(uint32_t* __restrict__ ticket, uint32_t total_takes) {
  // Relaxed: the ticket only orders tile indices; no data is published through it.
  const uint32_t t = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (t == total_takes - 1) dc::store_agent_u32(ticket, 0u);
  return t;
}


template <int MODE>
__device__ inline uint64_t apply_program(const dc_linq_chain& prog, const AffineChain& aff,
                                         float (&e)[kElemPerThread]) {
  if constexpr (MODE == kModeAffine) {
    return run_affine<kElemPerThread>(aff, e);
  } else {
    uint64_t keep = 0;
#pragma unroll
    for (int c = 0; c < kElemPerThread / kChunk; ++c) {
      float sub[kChunk];
#pragma unroll
      for (int i = 0; i < kChunk; ++i) sub[i] = e[c * kChunk + i];
      keep |= (uint64_t)run_program<kChunk, MODE == kModeInterpSaves>(prog, sub) << (c * kChunk);
#pragma unroll
      for (int i = 0; i < kChunk; ++i) e[c * kChunk + i] = sub[i];
    }
    return keep;
  }
}

// Program over EPT <= 32 elements of one lane; bit j of the result = element j is kept.
template <int MODE, int EPT>
__device__ inline uint32_t apply_small(const dc_linq_chain& prog, const AffineChain& aff, float (&e)[EPT]) {
  if constexpr (MODE == kModeAffine) return (uint32_t)run_affine<EPT>(aff, e);
  else return run_program<EPT, MODE == kModeInterpSaves>(prog, e);
}

template <int MODE>
__global__ __launch_bounds__(kBlock) void where_select_kernel(const dc_linq_chain prog, const AffineChain aff,
                                                              const float* __restrict__ in, int64_t n,
                                                              float* __restrict__ out,
                                                              int64_t* __restrict__ count_out,
                                                              uint64_t* __restrict__ status,
                                                              uint32_t* __restrict__ ticket, uint32_t epoch,
                                                              uint32_t num_tiles, int vec_ok) {
  static_assert(kVecPerThread * kWaves == 64, "the group scan gives one (j, wave) group to each lane of wave 0");
  __shared__ uint32_t s_tile;
  __shared__ uint32_t s_offset[kVecPerThread][kWaves];
  __shared__ uint32_t s_aggregate;
  __shared__ int64_t s_exclusive;
  __shared__ float s_wbuf[kWaves][4 * dc::kWave];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  if (tid == 0) s_tile = take_ticket(ticket, num_tiles);
  __syncthreads();
  const uint32_t tile = s_tile;
  if (tile >= num_tiles) return;  // cannot happen while the ticket counter starts at zero
  const int64_t base = (int64_t)tile * kTile;

  float e[kElemPerThread];
  uint64_t valid;
  if (vec_ok && base + kTile <= n) {
    const dc::f32x4* in4 = reinterpret_cast<const dc::f32x4*>(in + base);
#pragma unroll
    for (int j = 0; j < kVecPerThread; ++j) {
      const dc::f32x4 x = dc::load_stream(in4 + j * kBlock + tid);
      e[4 * j + 0] = x.x;
      e[4 * j + 1] = x.y;
      e[4 * j + 2] = x.z;
      e[4 * j + 3] = x.w;
    }
    valid = ~0ull;
  } else {
    valid = 0;
#pragma unroll
    for (int j = 0; j < kVecPerThread; ++j)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int64_t idx = base + (int64_t)j * (4 * kBlock) + tid * 4 + k;
        const bool ok = idx < n;
        e[4 * j + k] = ok ? in[idx] : 0.0f;
        valid |= (uint64_t)ok << (4 * j + k);
      }
  }

  const uint64_t keep = apply_program<MODE>(prog, aff, e) & valid;

  // Kept count of every (j, wave) group, and this lane's rank inside it (ballot + mbcnt per slot).
  uint32_t below[kVecPerThread];
#pragma unroll
  for (int j = 0; j < kVecPerThread; ++j) {
    uint32_t total = 0, bl = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint64_t b = __ballot((keep >> (4 * j + k)) & 1u);
      bl += __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
      total += (uint32_t)__builtin_popcountll(b);
    }
    below[j] = bl;
    if (lane == 0) s_offset[j][wave] = total;
  }
  __syncthreads();
  if (wave == 0) {  // exclusive scan of the 64 group counts in output order, one group per lane
    uint32_t* flat = &s_offset[0][0];
    const uint32_t c = flat[lane];
    uint32_t incl = c;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t o = __shfl_up(incl, off, 64);
      if (lane >= off) incl += o;
    }
    flat[lane] = incl - c;
    if (lane == 63) {
      s_aggregate = incl;
      publish_aggregate(status, tile, incl, epoch);
    }
  }
  __syncthreads();
  const uint32_t aggregate = s_aggregate;
  if (wave == 0) {
    const int64_t excl = lookback(status, tile, aggregate, epoch);
    if (lane == 0) s_exclusive = excl;
  }
  __syncthreads();
  float* dst = out + s_exclusive;
#pragma unroll
  for (int j = 0; j < kVecPerThread; ++j) {
    const int g = j * kWaves + wave;  // flat group index; the run ends where the next group starts
    const uint32_t gbase = s_offset[j][wave];
    const uint32_t gend = (g == 63) ? aggregate : (&s_offset[0][0])[g + 1];
    uint32_t pos = below[j];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if ((keep >> (4 * j + k)) & 1u) s_wbuf[wave][pos++] = e[4 * j + k];
    __builtin_amdgcn_wave_barrier();
    float* gdst = dst + gbase;
    for (uint32_t i = lane; i < gend - gbase; i += dc::kWave) gdst[i] = s_wbuf[wave][i];
    __builtin_amdgcn_wave_barrier();
  }
  if (tid == 0 && tile == num_tiles - 1) *count_out = s_exclusive + (int64_t)aggregate;
}

// ---- Where/Select -> ToArray, round-robin kernel for large inputs --------------------------------
// A resident grid of P workgroups (one per CU, all running at once). Workgroup w owns tile r*P + w of
// round r, so every round is a contiguous stretch of P tiles. Each tile publishes its kept count as
// one epoch-tagged word; the output offset of tile (r, w) is
//     base_r + sum_{w' < w} count(r, w'),   base_{r+1} = base_r + sum_{w'} count(r, w'),
// and every workgroup reads all P counts of a round itself, so no prefix ever has to travel from tile
// to tile (the serial front that limits a decoupled lookback). The loop is software-pipelined:
//   - loads run kRrAhead rounds ahead (kRrAhead + 1 register buffers per lane);
//   - kept values of a tile wait in LDS for kRrDelay rounds before they are written, and the count
//     words of that round are read one round before the write, so they were published
//     kRrDelay - 2 full rounds earlier and are almost always already visible.
// Roles inside the 1024-thread workgroup: wave 0 reads and checks the count words and broadcasts the
// output offset; waves 1..15 each own a contiguous 512-element chunk of every tile, rank their kept
// elements with ballot + mbcnt, stage them in a private LDS ring (in input order) and later write
// them as one contiguous run. The last wave to finish a tile (an LDS atomic) publishes its count.
// One workgroup barrier per round.
constexpr int kRrBlock = 1024;
constexpr int kRrWorkers = kRrBlock / dc::kWave - 1;     // 15 worker waves
constexpr int kRrVec = 2;                                // 16-byte loads per lane per tile
constexpr int kRrEpt = 4 * kRrVec;                       // 8 elements per lane
constexpr int kRrChunk = dc::kWave * kRrEpt;             // 512 elements per worker wave
constexpr int64_t kRrTile = (int64_t)kRrWorkers * kRrChunk;  // 7680 elements = 30 KiB
constexpr int kRrAhead = 4;
constexpr int kRrDelay = 3;
constexpr int kRrRing = 2048;                            // floats per worker wave (power of two)
constexpr int kRrCountsPerLane = 4;
constexpr int kRrMaxGroups = dc::kWave * kRrCountsPerLane;  // P <= 256
constexpr uint32_t kRrSpinLimit = 1u << 22;              // ~seconds: a wait that never ends reports
constexpr int kRrMinRounds = 4;                          // below this the ticket kernel is used
static_assert((kRrDelay + 1) * kRrChunk <= kRrRing, "the ring holds every staged tile at 100% selectivity");
static_assert(kRrDelay < 8 && kRrDelay >= 2, "per-tile LDS tables are indexed modulo 8");

// Calls f(std::integral_constant<int, U>) for U = 0, 1, ... in order: a compile-time unrolled loop, so
// the index into an array of register buffers is a constant.
template <typename F, int... U>
__device__ __attribute__((always_inline)) inline void for_each_index(F&& f, std::integer_sequence<int, U...>) {
  (f(std::integral_constant<int, U>{}), ...);
}

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

// Wave 0: re-reads until every count word of `round` carries this launch's epoch (bounded), then
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

template <int MODE>
__global__ __launch_bounds__(kRrBlock) void where_select_rounds_kernel(
    const dc_linq_chain prog, const Canon2 canon, const float* __restrict__ in, int64_t n, float* __restrict__ out,
    int64_t* __restrict__ count_out, uint32_t* __restrict__ counts, uint32_t epoch16, uint32_t P,
    uint32_t* __restrict__ done) {
  constexpr uint32_t kMask = kRrRing - 1;
  __shared__ float s_ring[kRrWorkers][kRrRing];
  __shared__ uint32_t s_wcount[8][16];  // kept count of (tile slot, worker wave)
  __shared__ uint32_t s_acc[8];         // (waves finished << 24) | kept so far, per tile slot
  __shared__ int64_t s_off[2];          // output offset of the tile being written, by round parity
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t w = blockIdx.x;
  const int64_t num_tiles = (n + kRrTile - 1) / kRrTile;
  const uint32_t R0 = (uint32_t)((n / kRrTile) / P);  // rounds in which every tile is full
  const uint32_t rounds = R0 > 0 ? R0 + kRrDelay : 0;
  const bool tail_round = (int64_t)R0 * P < num_tiles;
  if (tid < 8) s_acc[tid] = 0;
  __syncthreads();

  if (wave == 0) {
    // ---------------- control wave
    int64_t base = 0;
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
      const uint32_t add = 1u | (ok ? 0u : (1u << 16));
      const uint32_t prev = __hip_atomic_fetch_add(done, add, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
      if ((prev & 0xFFFFu) == P - 1) {
        *count_out = ((prev >> 16) == 0 && ok) ? base : (int64_t)-1;
        dc::store_agent_u32(done, 0u);
      }
    }
    return;
  }

  // ---------------- worker waves
  const int ww = wave - 1;
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
  auto stage = [&](float (&e)[kRrEpt], uint32_t keep, uint32_t r) __attribute__((always_inline)) {
    uint32_t run = 0, pos[kRrVec];
#pragma unroll
    for (int j = 0; j < kRrVec; ++j) {
      uint32_t below = 0, total = 0;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint64_t b = __ballot((keep >> (4 * j + k)) & 1u);
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
      for (int k = 0; k < 4; ++k)
        if ((keep >> (4 * j + k)) & 1u) ring[(p++) & kMask] = e[4 * j + k];
    }
    head += run;
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
    for (uint32_t i = lane; i < cnt; i += dc::kWave) dst[i] = ring[(tail + i) & kMask];
    tail += cnt;
  };

  // Every load below is unconditional: rounds past the last one re-load round R0 - 1 (loaded one
  // round earlier, so mostly served by the cache). The compiler's memory-counter waits are
  // path-insensitive: on a path that skipped a later load, the wait for the round being staged
  // would have to cover every load still in flight, draining the pipeline.
  const uint32_t last = R0 > 0 ? R0 - 1 : 0;
  constexpr int kBufs = kRrAhead + 1;
  float e[kBufs][kRrEpt];  // register buffers: constant indices only, after full unrolling
  if (R0 > 0)
    for_each_index([&](auto U) __attribute__((always_inline)) { load(e[U.value], min((uint32_t)U.value, last)); },
                   std::make_integer_sequence<int, kRrAhead>{});
  uint32_t r = 0;
  // One round: issue the loads of round r + kRrAhead into buffer `en`, stage round r from `ec`,
  // write round r - kRrDelay. Unrolled kBufs ways so the buffers rotate without copies. The main
  // loop runs whole kBufs-round iterations with no early exit: a `break` between rounds becomes a
  // path back to the loop head after a partial iteration, and the waits at the head would then
  // assume fewer loads in flight than a full iteration leaves. The last R0 % kBufs rounds follow.
  auto round = [&](float (&ec)[kRrEpt], float (&en)[kRrEpt]) __attribute__((always_inline)) {
    load(en, min(r + kRrAhead, last));
    stage(ec, apply_rounds<MODE, kRrEpt>(prog, canon, ec), r);
    __syncthreads();
    if (r >= (uint32_t)kRrDelay) write(r - kRrDelay, r & 1);
    ++r;
  };
  for (uint32_t it = R0 / kBufs; it > 0; --it)
    for_each_index([&](auto U) __attribute__((always_inline)) { round(e[U.value], e[(U.value + kRrAhead) % kBufs]); },
                   std::make_integer_sequence<int, kBufs>{});
  for_each_index([&](auto U) __attribute__((always_inline)) { if (r < R0) round(e[U.value], e[(U.value + kRrAhead) % kBufs]); },
                 std::make_integer_sequence<int, kRrAhead>{});
  for (; r < rounds; ++r) {  // drain: the last kRrDelay staged tiles
    __syncthreads();
    write(r - kRrDelay, r & 1);
  }
  if (tail_round) {  // tiles R0*P .. num_tiles-1 (full, partial or none), bounded loads
    const int64_t t = (int64_t)R0 * P + w;
    float e[kRrEpt];
    uint32_t valid = 0;
#pragma unroll
    for (int j = 0; j < kRrVec; ++j) {
      const int64_t at = t * kRrTile + chunk + j * 4 * dc::kWave + 4 * lane;
#pragma unroll
      for (int k = 0; k < 4; ++k) e[4 * j + k] = (t < num_tiles && at + k < n) ? in[at + k] : 0.0f;
      const int64_t nv = t < num_tiles ? min(max(n - at, (int64_t)0), (int64_t)4) : 0;
      valid |= ((1u << (uint32_t)nv) - 1u) << (4 * j);
    }
    stage(e, apply_rounds<MODE, kRrEpt>(prog, canon, e) & valid, R0);
    __syncthreads();
    __syncthreads();
    write(R0, 0);
  }
}

// ---- Where/Select -> Sum / Count ----------------------------------------------------------------
// Pass 1: each block runs the program over one contiguous chunk (a thread takes 4 vectors, 16
// elements, per step) and writes its float64 sum and kept count; pass 2 sums the partials in block
// order (fixed tree, deterministic).
constexpr int kSumBlock = 512;


template <int MODE>
__global__ __launch_bounds__(kSumBlock) void where_select_sum_pass1(const dc_linq_chain prog, const AffineChain aff,
                                                                    const float* __restrict__ in, int64_t n,
                                                                    int vec_ok, double* __restrict__ psum,
                                                                    int64_t* __restrict__ pcnt) {
  __shared__ double lds_d[kSumBlock / dc::kWave];
  __shared__ int64_t lds_i[kSumBlock / dc::kWave];
  double acc = 0.0;
  int64_t cnt = 0;
  const int64_t n4 = vec_ok ? (n >> 2) : 0;
  const int64_t per = (n4 + gridDim.x - 1) / gridDim.x;
  const int64_t v0 = min(n4, (int64_t)blockIdx.x * per), v1 = min(n4, v0 + per);
  const dc::f32x4* in4 = reinterpret_cast<const dc::f32x4*>(in);
  int64_t i = v0 + threadIdx.x;
  for (; i + 3 * kSumBlock < v1; i += 4 * kSumBlock) {
    float e[16];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      dc::f32x4 x = dc::load_stream(in4 + i + j * kSumBlock);
      e[4 * j + 0] = x.x;
      e[4 * j + 1] = x.y;
      e[4 * j + 2] = x.z;
      e[4 * j + 3] = x.w;
    }
    const uint32_t keep = apply_small<MODE, 16>(prog, aff, e);
#pragma unroll
    for (int j = 0; j < 16; ++j) acc += ((keep >> j) & 1u) ? (double)e[j] : 0.0;
    cnt += __builtin_popcount(keep);
  }
  for (; i < v1; i += kSumBlock) {
    float e[4];
    dc::f32x4 x = dc::load_stream(in4 + i);
    e[0] = x.x; e[1] = x.y; e[2] = x.z; e[3] = x.w;
    const uint32_t keep = apply_small<MODE, 4>(prog, aff, e);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc += ((keep >> j) & 1u) ? (double)e[j] : 0.0;
    cnt += __builtin_popcount(keep);
  }
  if (blockIdx.x == gridDim.x - 1) {
    for (int64_t s = (n4 << 2) + threadIdx.x; s < n; s += kSumBlock) {
      float e[1] = {in[s]};
      if (apply_small<MODE, 1>(prog, aff, e) & 1u) {
        acc += (double)e[0];
        cnt += 1;
      }
    }
  }
  const double bsum = dc::block_sum64<kSumBlock>(acc, lds_d);
  const int64_t bcnt = dc::block_sum64<kSumBlock>(cnt, lds_i);
  if (threadIdx.x == 0) {
    psum[blockIdx.x] = bsum;
    pcnt[blockIdx.x] = bcnt;
  }
}

constexpr int kFinalBlock = 1024;

__global__ __launch_bounds__(kFinalBlock) void where_select_sum_pass2(const double* __restrict__ psum,
                                                                      const int64_t* __restrict__ pcnt, int count,
                                                                      double* __restrict__ sum_out,
                                                                      int64_t* __restrict__ count_out) {
  __shared__ double lds_d[kFinalBlock / dc::kWave];
  __shared__ int64_t lds_i[kFinalBlock / dc::kWave];
  double a = 0.0;
  int64_t c = 0;
  for (int b = threadIdx.x; b < count; b += kFinalBlock) {
    a += psum[b];
    c += pcnt[b];
  }
  const double total = dc::block_sum64<kFinalBlock>(a, lds_d);
  const int64_t total_cnt = dc::block_sum64<kFinalBlock>(c, lds_i);
  if (threadIdx.x == 0) {
    if (sum_out) *sum_out = total;
    if (count_out) *count_out = total_cnt;
  }
}

// Launches the two passes of Where/Select -> Sum with the partials in psum/pcnt (grid entries each).
int32_t launch_where_select_sum(dc_hip_ctx* ctx, const dc_linq_chain* chain, const float* input, int64_t n,
                                unsigned grid, double* psum, int64_t* pcnt, double* sum_out, int64_t* count_out) {
  AffineChain aff{};
  const bool affine = lower_affine(*chain, &aff);
  auto kernel = affine ? where_select_sum_pass1<kModeAffine>
                       : (program_uses_saves(*chain) ? where_select_sum_pass1<kModeInterpSaves>
                                                     : where_select_sum_pass1<kModeInterp>);
  kernel<<<grid, kSumBlock, 0, ctx->stream>>>(*chain, aff, input, n, dc::aligned16(input) ? 1 : 0, psum, pcnt);
  where_select_sum_pass2<<<1, kFinalBlock, 0, ctx->stream>>>(psum, pcnt, (int)grid, sum_out, count_out);
  return dc::last_launch_status();
}

unsigned where_select_sum_grid(int64_t n) {
  const int64_t per_block = (int64_t)kSumBlock * 16 * 4;  // elements per block-iteration x 4
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>((n + per_block - 1) / per_block, kSumBlocksMax));
}

// Scratch of dc_hip_linq_where_select_sum_f32_noalloc: one launch's per-workgroup partials (a
// float64 sum and an int64 count per workgroup, at most kSumBlocksMax workgroups), 16 KiB. One copy
// per GPU, held until the process ends; every call on a GPU uses it, so calls that overlap on one
// GPU race. Pass 1 writes every entry pass 2 reads, so nothing needs clearing between calls.
constexpr size_t kNoAllocScratchBytes = (size_t)kSumBlocksMax * (sizeof(double) + sizeof(int64_t));
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

}  // namespace

namespace dc {

// Resolves the device address of `scratch` for the context's device (the device is current):
// once per device, kept for every later context on it.
int32_t linq_noalloc_setup(dc_hip_ctx* ctx) {
  static std::mutex mu;
  static std::map<int, void*> per_device;
  std::lock_guard<std::mutex> lock(mu);
  auto it = per_device.find(ctx->device);
  if (it == per_device.end()) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return e != hipSuccess ? (int32_t)e : DC_ERR_NOT_FOUND;
    it = per_device.emplace(ctx->device, p).first;
  }
  ctx->noalloc_scratch = it->second;
  return DC_OK;
}

}  // namespace dc

namespace {

// ---- Where/Select -> Min / Max ------------------------------------------------------------------
// Same two-pass shape as the sum. The BCL's enumerator loops (Min: the first NaN, else the first
// smallest element; Max: NaNs skipped, the first largest, the last NaN when all are NaN) depend on
// the order only through ties, so every partial carries the sequence index of its candidate and the
// combination breaks ties by index. That combination is commutative and associative, so the grid's
// result is the enumerator's bit for bit (signed zeros and NaN payloads included), whatever the
// order in which lanes, waves and workgroups meet. An index of -1 marks "no element yet".
enum MinMaxOp : int { kOpMin = DC_LINQ_MIN, kOpMax = DC_LINQ_MAX };

template <int OP>
__device__ inline void mm_take(float& v, int64_t& i, float cv, int64_t ci) {
  if (ci < 0) return;
  bool take;
  if (i < 0) {
    take = true;
  } else {
    const bool vn = __builtin_isnan(v), cn = __builtin_isnan(cv);
    if (OP == kOpMin) {
      take = (vn || cn) ? (cn && (!vn || ci < i))           // the first NaN wins
                        : (cv < v || (cv == v && ci < i));  // else the first smallest
    } else {
      take = (vn || cn) ? (vn && (!cn || ci > i))           // a number beats NaN; all NaN: the last
                        : (cv > v || (cv == v && ci < i));  // else the first largest
    }
  }
  if (take) {
    v = cv;
    i = ci;
  }
}

// Wave-wide combination (butterfly: every lane ends with the wave's result).
template <int OP>
__device__ inline void mm_wave(float& v, int64_t& i, int64_t& c) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(v, off, 64);
    const int64_t oi = __shfl_xor(i, off, 64);
    c += __shfl_xor(c, off, 64);
    mm_take<OP>(v, i, ov, oi);
  }
}

// Block-wide combination; the result is valid in thread 0.
template <int OP, int BLOCK>
__device__ inline void mm_block(float& v, int64_t& i, int64_t& c) {
  __shared__ float sv[BLOCK / dc::kWave];
  __shared__ int64_t si[BLOCK / dc::kWave], sc[BLOCK / dc::kWave];
  mm_wave<OP>(v, i, c);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wave] = v;
    si[wave] = i;
    sc[wave] = c;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < BLOCK / dc::kWave; ++w) {
      mm_take<OP>(v, i, sv[w], si[w]);
      c += sc[w];
    }
  }
}

// In sequence order (every candidate comes after the current one) the enumerator's own rule
// applies and no index comparison is needed: Min takes x unless a NaN is held or x >= current;
// Max takes x when the current is NaN or x is larger.
template <int OP>
__device__ inline bool mm_in_order(bool have, float cur, float x) {
  if (OP == kOpMin) return !have || (!__builtin_isnan(cur) && !(x >= cur));
  return !have || __builtin_isnan(cur) || x > cur;
}

template <int MODE, int OP>
__global__ __launch_bounds__(kSumBlock) void where_select_minmax_pass1(const dc_linq_chain prog, const AffineChain aff,
                                                                       const float* __restrict__ in, int64_t n,
                                                                       int vec_ok, float* __restrict__ pv,
                                                                       int64_t* __restrict__ pi,
                                                                       int64_t* __restrict__ pcnt) {
  // A thread visits its elements in increasing sequence order (steps of 16 in index order, then
  // single vectors, then the scalar tail), so it keeps the enumerator's state directly.
  float bv = 0.0f;
  int64_t bi = -1, cnt = 0;
  auto fold = [&](float x, int64_t idx) __attribute__((always_inline)) {
    if (mm_in_order<OP>(bi >= 0, bv, x)) {
      bv = x;
      bi = idx;
    }
  };
  const int64_t n4 = vec_ok ? (n >> 2) : 0;
  const int64_t per = (n4 + gridDim.x - 1) / gridDim.x;
  const int64_t v0 = min(n4, (int64_t)blockIdx.x * per), v1 = min(n4, v0 + per);
  const dc::f32x4* in4 = reinterpret_cast<const dc::f32x4*>(in);
  int64_t i = v0 + threadIdx.x;
  for (; i + 3 * kSumBlock < v1; i += 4 * kSumBlock) {
    float e[16];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      dc::f32x4 x = dc::load_stream(in4 + i + j * kSumBlock);
      e[4 * j + 0] = x.x;
      e[4 * j + 1] = x.y;
      e[4 * j + 2] = x.z;
      e[4 * j + 3] = x.w;
    }
    const uint32_t keep = apply_small<MODE, 16>(prog, aff, e);
    // the step's own winner (its elements in order), then one fold into the running state
    float sv = 0.0f;
    int sj = -1;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const bool t = ((keep >> j) & 1u) && mm_in_order<OP>(sj >= 0, sv, e[j]);
      sv = t ? e[j] : sv;
      sj = t ? j : sj;
    }
    if (sj >= 0) fold(sv, 4 * (i + (int64_t)(sj >> 2) * kSumBlock) + (sj & 3));
    cnt += __builtin_popcount(keep);
  }
  for (; i < v1; i += kSumBlock) {
    float e[4];
    dc::f32x4 x = dc::load_stream(in4 + i);
    e[0] = x.x; e[1] = x.y; e[2] = x.z; e[3] = x.w;
    const uint32_t keep = apply_small<MODE, 4>(prog, aff, e);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if ((keep >> j) & 1u) fold(e[j], 4 * i + j);
    cnt += __builtin_popcount(keep);
  }
  if (blockIdx.x == gridDim.x - 1) {
    for (int64_t s = (n4 << 2) + threadIdx.x; s < n; s += kSumBlock) {
      float e[1] = {in[s]};
      if (apply_small<MODE, 1>(prog, aff, e) & 1u) {
        fold(e[0], s);
        cnt += 1;
      }
    }
  }
  mm_block<OP, kSumBlock>(bv, bi, cnt);
  if (threadIdx.x == 0) {
    pv[blockIdx.x] = bv;
    pi[blockIdx.x] = bi;
    pcnt[blockIdx.x] = cnt;
  }
}

template <int OP>
__global__ __launch_bounds__(kFinalBlock) void where_select_minmax_pass2(const float* __restrict__ pv,
                                                                         const int64_t* __restrict__ pi,
                                                                         const int64_t* __restrict__ pcnt, int count,
                                                                         float* __restrict__ value_out,
                                                                         int64_t* __restrict__ count_out) {
  float v = 0.0f;
  int64_t i = -1, c = 0;
  for (int b = threadIdx.x; b < count; b += kFinalBlock) {
    mm_take<OP>(v, i, pv[b], pi[b]);
    c += pcnt[b];
  }
  mm_block<OP, kFinalBlock>(v, i, c);
  if (threadIdx.x == 0) {
    if (value_out) *value_out = i >= 0 ? v : 0.0f;
    if (count_out) *count_out = c;
  }
}

// ---- strategy choice -----------------------------------------------------------------------------
const void* rounds_kernel(int mode) {
  switch (mode) {
    case kRrF: return reinterpret_cast<const void*>(&where_select_rounds_kernel<kRrF>);
    case kRrM: return reinterpret_cast<const void*>(&where_select_rounds_kernel<kRrM>);
    case kRrFM: return reinterpret_cast<const void*>(&where_select_rounds_kernel<kRrFM>);
    case kRrMF: return reinterpret_cast<const void*>(&where_select_rounds_kernel<kRrMF>);
    case kRrInterpSaves: return reinterpret_cast<const void*>(&where_select_rounds_kernel<kRrInterpSaves>);
    default: return reinterpret_cast<const void*>(&where_select_rounds_kernel<kRrInterp>);
  }
}

// Picks the round-robin variant for a program and fills its canonical constants.
int rounds_mode(const dc_linq_chain& prog, Canon2* canon) {
  AffineChain aff{};
  int shape = 0;
  if (lower_affine(prog, &aff) && lower_canon2(aff, canon, &shape)) {
    return shape == kShapeF ? kRrF : shape == kShapeM ? kRrM : shape == kShapeFM ? kRrFM : kRrMF;
  }
  *canon = Canon2{1.0f, 0.0f, 1.0f, -0.0f, 0u, 0u, 1u};
  return program_uses_saves(prog) ? kRrInterpSaves : kRrInterp;
}

uint32_t rounds_groups(const dc_hip_ctx* ctx) { return (uint32_t)std::min(ctx->cu_count, kRrMaxGroups); }

// The round-robin kernel needs a 16-byte aligned input of at least kRrMinRounds full rounds and
// room for one 1024-thread workgroup per CU (every program variant; asked once per context). The
// caller holds the context lock.
bool use_rounds(dc_hip_ctx* ctx, const float* input, int64_t n) {
  const uint32_t groups = rounds_groups(ctx);
  if (!dc::aligned16(input) || groups == 0 || n / kRrTile < (int64_t)kRrMinRounds * groups) return false;
  if (ctx->rounds_fit < 0) {
    bool fit = true;
    for (int mode : {kRrInterp, kRrInterpSaves, kRrF, kRrM, kRrFM, kRrMF}) {
      int per_cu = 0;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, rounds_kernel(mode), kRrBlock, 0) != hipSuccess ||
          per_cu < 1)
        fit = false;
    }
    ctx->rounds_fit = fit ? 1 : 0;
  }
  return ctx->rounds_fit == 1;
}

}  // namespace

extern "C" {

DC_HIP_API int32_t dc_linq_chain_validate(const dc_linq_chain* chain) {
  if (!chain) return DC_ERR_INVALID_ARGUMENT;
  if (chain->n_instr < 0 || chain->n_instr > DC_LINQ_MAX_INSTR ||
      (chain->flags & ~DC_LINQ_FLAG_ORDERED_GRID) != 0)
    return DC_ERR_INVALID_ARGUMENT;
  for (int i = 0; i < chain->n_instr; ++i) {
    const dc_linq_instr& in = chain->code[i];
    const bool op_ok = (in.op <= DC_LQ_STORE_S1) || (in.op >= DC_LQ_CMP_GT && in.op <= DC_LQ_MAP);
    if (!op_ok || in.src > DC_LQ_SRC_S1) return DC_ERR_UNSUPPORTED;
    if (in.op >= DC_LQ_CMP_GT && in.op <= DC_LQ_CMP_NE && in.mode > DC_LQ_CMP_OR) return DC_ERR_UNSUPPORTED;
  }
  return DC_OK;
}

DC_HIP_API int32_t dc_hip_linq_to_array_strategy(dc_hip_ctx* ctx, const float* input, int64_t n,
                                                 int32_t* strategy_out) {
  if (!ctx || !strategy_out || n < 0) return DC_ERR_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> lock(ctx->mu);
  *strategy_out = use_rounds(ctx, input, n) ? DC_LINQ_STRATEGY_ROUNDS : DC_LINQ_STRATEGY_LOOKBACK;
  return DC_OK;
}

DC_HIP_API int32_t dc_hip_linq_where_select_f32(dc_hip_ctx* ctx, const dc_linq_chain* chain, const float* input,
                                                int64_t n, float* output, int64_t* count_out) {
  if (n < 0 || !count_out || (n > 0 && (!input || !output))) return DC_ERR_INVALID_ARGUMENT;
  DC_RETURN_IF(dc_linq_chain_validate(chain));
  if (n >= (int64_t)1 << 40) return DC_ERR_INVALID_ARGUMENT;  // 40-bit counts in the status words
  DC_CTX_ENTER(ctx);
  if ((chain->flags & DC_LINQ_FLAG_ORDERED_GRID) == 0 && use_rounds(ctx, input, n)) {
    Canon2 canon{};
    const void* fn = rounds_kernel(rounds_mode(*chain, &canon));
    const uint32_t groups = rounds_groups(ctx);
    const int64_t tiles = (n + kRrTile - 1) / kRrTile;
    const size_t words = (size_t)((tiles + groups - 1) / groups + 1) * groups;
    uint32_t epoch16 = 0;
    DC_RETURN_IF(dc::ensure_round_counts(ctx, words, &epoch16));
    dc_linq_chain prog = *chain;
    const float* in_arg = input;
    int64_t n_arg = n;
    float* out_arg = output;
    int64_t* count_arg = count_out;
    uint32_t* counts_arg = ctx->round_counts;
    uint32_t groups_arg = groups;
    uint32_t* done_arg = ctx->counters + DC_SLOT_LINQ_DONE;
    void* args[] = {&prog, &canon, &in_arg, &n_arg, &out_arg, &count_arg, &counts_arg, &epoch16, &groups_arg, &done_arg};
    // One workgroup per CU, each needing most of a CU's LDS, on an otherwise idle device: every
    // workgroup is resident at once (an ordinary launch; measured faster than a cooperative one).
    DC_RETURN_IF(dc::resident_launch_begin(ctx));
    DC_RETURN_IF_HIP(hipLaunchKernel(fn, dim3(groups), dim3(kRrBlock), args, 0, ctx->stream));
    DC_RETURN_IF(dc::last_launch_status());
    return dc::resident_launch_end(ctx);
  }

  AffineChain aff{};
  const bool affine = lower_affine(*chain, &aff);
  const int mode = affine ? kModeAffine : (program_uses_saves(*chain) ? kModeInterpSaves : kModeInterp);
  const int64_t tiles = std::max<int64_t>(1, (n + kTile - 1) / kTile);
  if (tiles > 0x7FFFFFFFll) return DC_ERR_INVALID_ARGUMENT;
  uint32_t epoch = 0;
  DC_RETURN_IF(dc::ensure_status(ctx, (size_t)tiles, &epoch));
  auto kernel = mode == kModeAffine ? where_select_kernel<kModeAffine>
              : mode == kModeInterpSaves ? where_select_kernel<kModeInterpSaves>
                                         : where_select_kernel<kModeInterp>;
  kernel<<<(unsigned)tiles, kBlock, 0, ctx->stream>>>(*chain, aff, input, n, output, count_out, ctx->status,
                                                      ctx->counters + DC_SLOT_LINQ_TICKET, epoch, (uint32_t)tiles,
                                                      dc::aligned16(input) ? 1 : 0);
  return dc::last_launch_status();
}

DC_HIP_API int32_t dc_hip_linq_where_select_sum_f32(dc_hip_ctx* ctx, const dc_linq_chain* chain, const float* input,
                                                    int64_t n, double* sum_out, int64_t* count_out) {
  if (n < 0 || (n > 0 && !input)) return DC_ERR_INVALID_ARGUMENT;
  DC_RETURN_IF(dc_linq_chain_validate(chain));
  DC_CTX_ENTER(ctx);
  const unsigned grid = where_select_sum_grid(n);
  DC_RETURN_IF(dc::ensure_partials(ctx, (size_t)grid * 16));
  double* psum = static_cast<double*>(ctx->partials);
  int64_t* pcnt = reinterpret_cast<int64_t*>(psum + grid);
  return launch_where_select_sum(ctx, chain, input, n, grid, psum, pcnt, sum_out, count_out);
}

DC_HIP_API int32_t dc_hip_linq_where_select_sum_f32_noalloc(dc_hip_ctx* ctx, const dc_linq_chain* chain,
                                                            const float* input, int64_t n, double* sum_out,
                                                            int64_t* count_out) {
  if (n < 0 || (n > 0 && !input)) return DC_ERR_INVALID_ARGUMENT;
  DC_RETURN_IF(dc_linq_chain_validate(chain));
  DC_CTX_ENTER(ctx);
  if (ctx->noalloc_status != DC_OK) return ctx->noalloc_status;  // the symbol lookup at set-up failed
  const unsigned grid = where_select_sum_grid(n);
  // The grid is capped, so every n fits; the check keeps that invariant explicit.
  if ((size_t)grid * 16 > kNoAllocScratchBytes) return DC_ERR_OUT_OF_MEMORY;
  double* psum = static_cast<double*>(ctx->noalloc_scratch);  // never `scratch` itself: a host stand-in
  int64_t* pcnt = reinterpret_cast<int64_t*>(psum + grid);
  return launch_where_select_sum(ctx, chain, input, n, grid, psum, pcnt, sum_out, count_out);
}

DC_HIP_API int32_t dc_hip_linq_where_select_minmax_f32(dc_hip_ctx* ctx, const dc_linq_chain* chain,
                                                       const float* input, int64_t n, int32_t op, float* value_out,
                                                       int64_t* count_out) {
  if (n < 0 || (n > 0 && !input) || (op != DC_LINQ_MIN && op != DC_LINQ_MAX)) return DC_ERR_INVALID_ARGUMENT;
  DC_RETURN_IF(dc_linq_chain_validate(chain));
  DC_CTX_ENTER(ctx);
  const int64_t per_block = (int64_t)kSumBlock * 16 * 4;  // elements per block-iteration x 4
  const unsigned grid = (unsigned)std::max<int64_t>(1, std::min<int64_t>((n + per_block - 1) / per_block, kSumBlocksMax));
  DC_RETURN_IF(dc::ensure_partials(ctx, (size_t)grid * 24));
  int64_t* pi = static_cast<int64_t*>(ctx->partials);
  int64_t* pcnt = pi + grid;
  float* pv = reinterpret_cast<float*>(pcnt + grid);
  AffineChain aff{};
  const bool affine = lower_affine(*chain, &aff);
  const int mode = affine ? kModeAffine : (program_uses_saves(*chain) ? kModeInterpSaves : kModeInterp);
  const int vec_ok = dc::aligned16(input) ? 1 : 0;
#define DC_MINMAX(MODE, OP)                                                                                       \
  where_select_minmax_pass1<MODE, OP><<<grid, kSumBlock, 0, ctx->stream>>>(*chain, aff, input, n, vec_ok, pv, pi, pcnt); \
  where_select_minmax_pass2<OP><<<1, kFinalBlock, 0, ctx->stream>>>(pv, pi, pcnt, (int)grid, value_out, count_out)
  if (op == DC_LINQ_MIN) {
    if (mode == kModeAffine) { DC_MINMAX(kModeAffine, kOpMin); }
    else if (mode == kModeInterpSaves) { DC_MINMAX(kModeInterpSaves, kOpMin); }
    else { DC_MINMAX(kModeInterp, kOpMin); }
  } else {
    if (mode == kModeAffine) { DC_MINMAX(kModeAffine, kOpMax); }
    else if (mode == kModeInterpSaves) { DC_MINMAX(kModeInterpSaves, kOpMax); }
    else { DC_MINMAX(kModeInterp, kOpMax); }
  }
#undef DC_MINMAX
  return dc::last_launch_status();
}

}  // extern "C"

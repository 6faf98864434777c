// dc_linq.hip — fused LINQ Where/Select(/Sum) kernels for gfx950.
//
// One prebuilt kernel per terminal (ToArray, Sum) interprets the register program that the host
// fusion planner builds from the chain's lambdas (dc_linq_chain, program model in
// include/dotcompute_hip.h). The program lives in the kernel arguments, so every instruction is
// wave-uniform: dispatch is scalar branching, and each instruction is applied to the 16 elements a
// thread holds in registers.
//
// ToArray (order-preserving stream compaction, one pass over the input), two kernels:
//  - 4-byte aligned inputs of any size: the round-robin kernel (where_select_rounds_kernel,
//    described at its definition): a resident grid, one workgroup per CU (one per tile for inputs
//    of fewer tiles), tile counts published per round and summed by every workgroup, so no prefix
//    travels from tile to tile;
//  - inputs that are not 4-byte aligned, and the retry after a resident grid gave up
//    (DC_LINQ_FLAG_ORDERED_GRID): a ticket-ordered grid with a decoupled lookback. tile = 512 threads x 32
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

#include <type_traits>
#include <utility>
#include <vector>

#include "dc_device.hpp"
#include "dc_internal.hpp"
#include "dc_intdiv.hpp"
#include "dc_linq_device.hpp"

namespace {

using namespace dclq;

constexpr int kBlock = 512;                        // compaction workgroup: 8 waves
constexpr int kWaves = kBlock / dc::kWave;
constexpr int kVecPerThread = 8;
constexpr int kElemPerThread = 4 * kVecPerThread;  // 32
constexpr int kTile = kBlock * kElemPerThread;     // 16384 elements = 64 KiB of input
constexpr int kChunk = 16;                         // elements interpreted per program pass
constexpr int kLookbackPerLane = 4;                // status words read per lane per lookback round
constexpr int kSumBlocksMax = 1024;

__global__ void fault_finish_kernel(uint64_t* __restrict__ word, int64_t* __restrict__ fault_out) {
  const uint64_t w = *word;
  *fault_out = w ? (int64_t)~w : (int64_t)DC_LINQ_FAULT_NONE;
  *word = 0;
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

// True when the program calls a library operation (POW / RPOW: the LIBM interpreter variant).
inline bool program_uses_libm(const dc_linq_chain& prog) {
  for (int i = 0; i < prog.n_instr; ++i)
    if (prog.code[i].op == DC_LQ_POW || prog.code[i].op == DC_LQ_RPOW) return true;
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

inline bool lower_canon2(const AffineChain& ch, int* shape, int* cmp, RdConst* out) {
  const int n = ch.n_stages;
  if (n < 1 || n > 2 || (n == 2 && ch.kind[0] == ch.kind[1])) return false;
  RdConst k{0.0f, 1.0f, -0.0f};
  int c = DC_LQ_CMP_GT;
  for (int s = 0; s < n; ++s) {
    if (ch.kind[s] == kStageFilter) {
      if (ch.op[s] < DC_LQ_CMP_GT || ch.op[s] > DC_LQ_CMP_NE) return false;
      c = (int)ch.op[s];
      k.t = ch.c0[s];
    } else {
      k.a = (ch.op[s] & 1u) ? ch.c0[s] : 1.0f;
      k.b = (ch.op[s] & 2u) ? ch.c1[s] : -0.0f;
    }
  }
  *shape = n == 1 ? (ch.kind[0] == kStageFilter ? kShapeF : kShapeM)
                  : (ch.kind[0] == kStageFilter ? kShapeFM : kShapeMF);
  *cmp = c;
  *out = k;
  return true;
}

struct ReducePlan {
  int mode;
  AffineChain aff;
  RdConst k;
};

// Plan of an int32 program: the int32 interpreter, with or without save registers.
inline ReducePlan reduce_plan_i32(const dc_linq_chain& prog) {
  ReducePlan p{};
  p.k = RdConst{0.0f, 1.0f, -0.0f};
  p.mode = program_uses_saves(prog) ? kRdInterpI32Saves : kRdInterpI32;
  return p;
}

inline ReducePlan reduce_plan(const dc_linq_chain& prog) {
  ReducePlan p{};
  p.k = RdConst{0.0f, 1.0f, -0.0f};
  int shape = 0, cmp = DC_LQ_CMP_GT;
  if (!lower_affine(prog, &p.aff))
    p.mode = program_uses_libm(prog) ? kRdInterpLibm : program_uses_saves(prog) ? kRdInterpSaves : kRdInterp;
  else if (lower_canon2(p.aff, &shape, &cmp, &p.k)) p.mode = rd_canon(shape, cmp);
  else p.mode = kRdAffine;
  return p;
}

// Calls f(std::integral_constant<int, mode>{}) for a reduction mode chosen at run time.
#define DC_RD_CMP_MODES(X, SHAPE)                                                                        \
  X(rd_canon(SHAPE, DC_LQ_CMP_GT)) X(rd_canon(SHAPE, DC_LQ_CMP_GE)) X(rd_canon(SHAPE, DC_LQ_CMP_LT)) \
  X(rd_canon(SHAPE, DC_LQ_CMP_LE)) X(rd_canon(SHAPE, DC_LQ_CMP_EQ)) X(rd_canon(SHAPE, DC_LQ_CMP_NE))
template <class F>
void rd_dispatch(int mode, F&& f) {
  switch (mode) {
#define DC_RD_CASE(m)                   \
  case (m):                             \
    f(std::integral_constant<int, (m)>{}); \
    return;
    DC_RD_CASE(kRdInterpSaves)
    DC_RD_CASE(kRdInterpLibm)
    DC_RD_CASE(kRdAffine)
    DC_RD_CASE(rd_canon(kShapeM, DC_LQ_CMP_GT))
    DC_RD_CMP_MODES(DC_RD_CASE, kShapeF)
    DC_RD_CMP_MODES(DC_RD_CASE, kShapeFM)
    DC_RD_CMP_MODES(DC_RD_CASE, kShapeMF)
#undef DC_RD_CASE
    default:
      f(std::integral_constant<int, kRdInterp>{});
      return;
  }
}
#undef DC_RD_CMP_MODES

// rd_dispatch for the int32 modes.
template <class F>
void rd_dispatch_i32(int mode, F&& f) {
  if (mode == kRdInterpI32Saves) f(std::integral_constant<int, kRdInterpI32Saves>{});
  else f(std::integral_constant<int, kRdInterpI32>{});
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


// The program over a thread's 32 elements; `valid` marks the elements that exist. For the int32
// modes, bit b of *fhit / *fovf is element b's first exception and its kind (OverflowException).
template <int MODE>
__device__ inline uint64_t apply_program(const dc_linq_chain& prog, const AffineChain& aff,
                                         float (&e)[kElemPerThread], uint64_t valid, uint64_t* fhit,
                                         uint64_t* fovf) {
  if constexpr (MODE == kModeAffine) {
    return run_affine<kElemPerThread>(aff, e) & valid;
  } else if constexpr (mode_is_int(MODE)) {
    constexpr int C = kChunk;
    uint64_t keep = 0, hit = 0, ovf = 0;
    for_each_index([&](auto CI) __attribute__((always_inline)) {
      constexpr int c = decltype(CI)::value;
      float sub[C];
#pragma unroll
      for (int i = 0; i < C; ++i) sub[i] = e[c * C + i];
      Faults f;
      const uint32_t live = (uint32_t)(valid >> (c * C)) & ((1u << C) - 1u);
      keep |= (uint64_t)run_program_i32<C, MODE == kModeInterpI32Saves>(prog, sub, live, f) << (c * C);
      hit |= (uint64_t)f.hit << (c * C);
      ovf |= (uint64_t)f.ovf << (c * C);
#pragma unroll
      for (int i = 0; i < C; ++i) e[c * C + i] = sub[i];
    }, std::make_integer_sequence<int, kElemPerThread / C>{});
    *fhit = hit;
    *fovf = ovf;
    return keep;
  } else {
    uint64_t keep = 0;
#pragma unroll
    for (int c = 0; c < kElemPerThread / kChunk; ++c) {
      float sub[kChunk];
#pragma unroll
      for (int i = 0; i < kChunk; ++i) sub[i] = e[c * kChunk + i];
      keep |= (uint64_t)run_program_f32<kChunk, MODE == kModeInterpSaves || MODE == kModeInterpLibm,
                                        MODE == kModeInterpLibm>(prog, sub)
              << (c * kChunk);
#pragma unroll
      for (int i = 0; i < kChunk; ++i) e[c * kChunk + i] = sub[i];
    }
    return keep & valid;
  }
}


template <int MODE>
__global__ __launch_bounds__(kBlock) void where_select_kernel(const dc_linq_chain prog, const AffineChain aff,
                                                              const float* __restrict__ in, int64_t n,
                                                              float* __restrict__ out,
                                                              int64_t* __restrict__ count_out,
                                                              uint64_t* __restrict__ status,
                                                              uint32_t* __restrict__ ticket, uint32_t epoch,
                                                              uint32_t num_tiles, int vec_ok,
                                                              uint64_t* __restrict__ fault) {
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

  uint64_t fhit = 0, fovf = 0;
  const uint64_t keep = apply_program<MODE>(prog, aff, e, valid, &fhit, &fovf);
  if (mode_is_int(MODE) && fhit) {  // element 4j + k of this thread is tile element 2048 j + 4 t + k
    const int b = __builtin_ctzll(fhit);
    publish_fault(fault, base + (int64_t)(b >> 2) * (4 * kBlock) + tid * 4 + (b & 3), ((fovf >> b) & 1u) != 0u);
  }

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

// The prebuilt round-robin ToArray kernels, one per program mode (rounds_body in
// dc_linq_device.hpp; a run-time compiled kernel for one program has the same arguments).
template <int RD>
__global__ __launch_bounds__(kRrBlock) void where_select_rounds_kernel(
    const dc_linq_chain prog, const AffineChain aff, const RdConst canon, const float* __restrict__ in, int64_t n,
    float* __restrict__ out, int64_t* __restrict__ count_out, uint32_t* __restrict__ counts, uint32_t epoch16,
    uint32_t P, uint32_t* __restrict__ done, uint64_t* __restrict__ fault, const float* __restrict__ head_in,
    int head_n) {
  rounds_body<RD, NoGen>(prog, aff, canon, in, n, out, count_out, counts, epoch16, P, done, fault, head_in, head_n);
}

// ---- Where/Select -> Sum / Count / Min / Max: pass 1 ---------------------------------------------
// Each workgroup runs the program over one contiguous chunk of the 16-byte aligned region that
// starts h elements into the input: a thread loads 8 vectors (32 elements) per step and applies the
// program to each half of 16; the vectors after the chunk's last whole step are taken one per
// thread at a time. The elements before the aligned region (h < 4; h = n for an input that is not
// even 4-byte aligned) and after it (< 4) go to the last workgroup. Pass 2 combines the
// per-workgroup partials in a fixed tree (deterministic).
constexpr int kSumBlock = 512;
constexpr int kRdUnroll = 8;                                 // 16-byte vectors per thread per step
constexpr int64_t kRdStep = (int64_t)kRdUnroll * kSumBlock;  // vectors per workgroup per step

// Elements before the first 16-byte boundary (the whole input when it is not 4-byte aligned).
inline int64_t reduce_head(const float* in, int64_t n) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(in);
  if (a & 3) return n;
  return std::min<int64_t>(n, (int64_t)(((16 - (a & 15)) & 15) >> 2));
}

// Visits this workgroup's elements and returns this thread's share of the kept count.
// half(e, kept, base): 16 elements in sequence order, element j at vector base + (j >> 2) *
// kSumBlock of the aligned region, lane j & 3. single(x, kept, index): the remaining whole vectors,
// element by element, in sequence order after the halves. loose(x, kept, index): head and tail
// elements (last workgroup, out of order). The steps run a workgroup-uniform number of times, so
// their kept elements are counted per wave with ballots (scalar work) and credited to lane 0.
// int32 modes: *fault (per thread) becomes the largest ~(4 * index + kind) over the elements
// that throw, 0 if none.
template <int RD, class Half, class Single, class Loose>
__device__ __attribute__((always_inline)) inline int64_t visit_chunk(const dc_linq_chain& prog, const AffineChain& aff,
                                                                     const RdConst& canon, const float* __restrict__ in,
                                                                     int64_t n, int64_t h, Half&& half, Single&& single,
                                                                     Loose&& loose, uint64_t* fault = nullptr) {
  uint64_t lane_fault = 0;
  // Folds the first exception of a group of elements into lane_fault; index_of(b) = the
  // sequence index of the group's element b (increasing with b).
  auto note = [&](const Faults& f, auto index_of) __attribute__((always_inline)) {
    if constexpr (rd_is_int(RD)) {
      const int b = __builtin_ctz(f.hit | 0x80000000u);
      const uint64_t code = (uint64_t)index_of(b) * 4u +
                            (((f.ovf >> b) & 1u) ? DC_LINQ_FAULT_OVERFLOW : DC_LINQ_FAULT_DIVIDE_BY_ZERO);
      lane_fault = max(lane_fault, f.hit ? ~code : (uint64_t)0);
    }
  };
  const int64_t n4 = (n - h) >> 2;
  const int64_t per = (n4 + gridDim.x - 1) / gridDim.x;
  const int64_t v0 = min(n4, (int64_t)blockIdx.x * per), v1 = min(n4, v0 + per);
  const int64_t steps = (v1 - v0) / kRdStep;
  const dc::f32x4* xa = reinterpret_cast<const dc::f32x4*>(in + h);
  int64_t cnt = 0;
  uint64_t wave_cnt = 0;
  int64_t i = v0 + threadIdx.x;
  for (int64_t s = 0; s < steps; ++s, i += kRdStep) {
    dc::f32x4 v[kRdUnroll];
#pragma unroll
    for (int u = 0; u < kRdUnroll; ++u) v[u] = dc::load_stream(xa + i + u * kSumBlock);
    for_each_index([&](auto G) __attribute__((always_inline)) {
      constexpr int g = decltype(G)::value;
      float e[16];
      bool kept[16];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        e[4 * m + 0] = v[4 * g + m].x;
        e[4 * m + 1] = v[4 * g + m].y;
        e[4 * m + 2] = v[4 * g + m].z;
        e[4 * m + 3] = v[4 * g + m].w;
      }
      Faults f;
      eval_flags<RD, 16>(prog, aff, canon, e, kept, 0xFFFFu, f);
      const int64_t base = i + (int64_t)(4 * g) * kSumBlock;
      note(f, [&](int b) { return h + 4 * (base + (int64_t)(b >> 2) * kSumBlock) + (b & 3); });
#pragma unroll
      for (int j = 0; j < 16; ++j) wave_cnt += (uint64_t)__builtin_popcountll(__ballot(kept[j]));
      half(e, kept, base);
    }, std::make_integer_sequence<int, kRdUnroll / 4>{});
  }
  if ((threadIdx.x & (dc::kWave - 1)) == 0) cnt += (int64_t)wave_cnt;
  for (; i < v1; i += kSumBlock) {
    const dc::f32x4 x = dc::load_stream(xa + i);
    float e[4] = {x.x, x.y, x.z, x.w};
    bool kept[4];
    Faults f;
    eval_flags<RD, 4>(prog, aff, canon, e, kept, 0xFu, f);
    note(f, [&](int b) { return h + 4 * i + b; });
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      single(e[j], kept[j], h + 4 * i + j);
      cnt += kept[j] ? 1 : 0;
    }
  }
  if (blockIdx.x == gridDim.x - 1) {
    auto one = [&](int64_t s) __attribute__((always_inline)) {
      float e[1] = {in[s]};
      bool kept[1];
      Faults f;
      eval_flags<RD, 1>(prog, aff, canon, e, kept, 1u, f);
      note(f, [&](int) { return s; });
      loose(e[0], kept[0], s);
      cnt += kept[0] ? 1 : 0;
    };
    for (int64_t s = threadIdx.x; s < h; s += kSumBlock) one(s);
    for (int64_t s = h + 4 * n4 + threadIdx.x; s < n; s += kSumBlock) one(s);
  }
  if (fault) *fault = lane_fault;
  return cnt;
}

// Where/Select -> Sum / Count: float64 sum and kept count per workgroup.
// ONE (gridDim.x <= kSumBlock): the one-launch form. Every workgroup publishes its partials with
// agent-scope stores (written through its XCD's L2), waits for them to complete and takes a
// ticket; the workgroup with the last ticket adds the partials exactly as pass 2 does (its thread
// t holds 0 + partial t; the waves past the partials add +0 to pass 2's in-order sum of the wave
// totals), so both forms return the same bits. No fences: nothing else crosses workgroups.
template <int RD, bool ONE>
__global__ __launch_bounds__(kSumBlock) void where_select_sum_pass1(const dc_linq_chain prog, const AffineChain aff,
                                                                    const RdConst canon, const float* __restrict__ in,
                                                                    int64_t n, int64_t h, double* __restrict__ psum,
                                                                    int64_t* __restrict__ pcnt, uint32_t* __restrict__ done,
                                                                    double* __restrict__ sum_out,
                                                                    int64_t* __restrict__ count_out) {
  __shared__ double lds_d[kSumBlock / dc::kWave];
  __shared__ int64_t lds_i[kSumBlock / dc::kWave];
  __shared__ uint32_t s_last;
  // A dropped element adds +0.0, which leaves the float64 total unchanged (it starts at +0.0 and a
  // sum of +0.0 and -0.0 is +0.0), so the selection happens in float before the widening.
  double acc = 0.0;
  auto add = [&](float x, bool kept, int64_t) __attribute__((always_inline)) { acc += (double)(kept ? x : 0.0f); };
  const int64_t cnt = visit_chunk<RD>(
      prog, aff, canon, in, n, h,
      [&](const float (&e)[16], const bool (&kept)[16], int64_t) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 16; ++j) acc += (double)(kept[j] ? e[j] : 0.0f);
      },
      add, add);
  const double bsum = dc::block_sum64<kSumBlock>(acc, lds_d);
  const int64_t bcnt = dc::block_sum64<kSumBlock>(cnt, lds_i);
  if constexpr (!ONE) {
    if (threadIdx.x == 0) {
      psum[blockIdx.x] = bsum;
      pcnt[blockIdx.x] = bcnt;
    }
  } else {
    if (threadIdx.x == 0) {
      dc::store_agent_u64(reinterpret_cast<uint64_t*>(psum) + blockIdx.x, (uint64_t)__double_as_longlong(bsum));
      dc::store_agent_u64(reinterpret_cast<uint64_t*>(pcnt) + blockIdx.x, (uint64_t)bcnt);
      dc::wait_memory_ops();
      s_last = dc::fetch_add_relaxed_agent_u32(done, 1u) == gridDim.x - 1 ? 1u : 0u;
    }
    __syncthreads();
    if (!s_last) return;
    double a = 0.0;
    int64_t c = 0;
    if (threadIdx.x < gridDim.x) {
      a += __longlong_as_double((long long)dc::load_agent_u64(reinterpret_cast<const uint64_t*>(psum) + threadIdx.x));
      c += (int64_t)dc::load_agent_u64(reinterpret_cast<const uint64_t*>(pcnt) + threadIdx.x);
    }
    const double total = dc::block_sum64<kSumBlock>(a, lds_d);
    const int64_t total_cnt = dc::block_sum64<kSumBlock>(c, lds_i);
    if (threadIdx.x == 0) {
      if (sum_out) *sum_out = total;
      if (count_out) *count_out = total_cnt;
      dc::store_agent_u32(done, 0u);
    }
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

// Launches Where/Select -> Sum with the partials in psum/pcnt (grid entries each): one launch up
// to kSumOneLaunchMax elements, else pass 1 and pass 2.
constexpr int64_t kSumOneLaunchMax = (int64_t)1 << 21;
int32_t launch_where_select_sum(dc_hip_ctx* ctx, const dc_linq_chain* chain, const float* input, int64_t n,
                                unsigned grid, double* psum, int64_t* pcnt, double* sum_out, int64_t* count_out) {
  const ReducePlan p = reduce_plan(*chain);
  const int64_t h = reduce_head(input, n);
  uint32_t* done = ctx->counters + DC_SLOT_REDUCE_DONE;
  if (n <= kSumOneLaunchMax && grid <= (unsigned)kSumBlock) {
    rd_dispatch(p.mode, [&](auto mode) {
      where_select_sum_pass1<decltype(mode)::value, true>
          <<<grid, kSumBlock, 0, ctx->stream>>>(*chain, p.aff, p.k, input, n, h, psum, pcnt, done, sum_out, count_out);
    });
    return dc::last_launch_status();
  }
  rd_dispatch(p.mode, [&](auto mode) {
    where_select_sum_pass1<decltype(mode)::value, false>
        <<<grid, kSumBlock, 0, ctx->stream>>>(*chain, p.aff, p.k, input, n, h, psum, pcnt, nullptr, nullptr, nullptr);
  });
  where_select_sum_pass2<<<1, kFinalBlock, 0, ctx->stream>>>(psum, pcnt, (int)grid, sum_out, count_out);
  return dc::last_launch_status();
}

// One workgroup per CU (measured best: 8 waves per CU streaming one contiguous chunk each; more
// workgroups, or larger ones, are slower at every size from 16M elements up), fewer when the
// input gives a workgroup less than 8 vectors per thread.
unsigned where_select_sum_grid(const dc_hip_ctx* ctx, int64_t n) {
  const int64_t per_block = (int64_t)kSumBlock * 4 * 8;
  const int64_t cap = std::min<int64_t>(std::max(ctx->cu_count, 1), kSumBlocksMax);
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>((n + per_block - 1) / per_block, cap));
}


// ---- Where/Select -> Sum / Count over int32 ------------------------------------------------------
// After Where/Select the reference's Sum() runs Enumerable.Sum over an iterator, which adds element
// by element with checked int32 adds: OverflowException as soon as a prefix sum of the kept, mapped
// elements (in sequence order) leaves int32. Pass 1 gives each workgroup one contiguous chunk of the
// aligned region (as the float Sum does) and sums the chunk's positive parts and negative parts
// separately (exact and order-free); the loose head and tail elements form two more chunks, the
// first and last in sequence order. Every prefix inside a chunk lies in [S - neg, S + pos], S being
// the prefix before the chunk, and S + pos - neg is itself a prefix (the chunk's end). Pass 2 (one
// workgroup) scans the chunk sums in sequence order: a chunk end outside int32 is an overflow; a
// chunk whose bounds leave int32 while its end does not is re-checked exactly (its elements
// re-read and re-evaluated in sequence order, combining (sum, max prefix, min prefix) in order).
// The screen clears chunks whose running totals stay well inside int32 (the common case), so the
// exact check is the exception.
enum MinMaxOp : int { kOpMin = DC_LINQ_MIN, kOpMax = DC_LINQ_MAX };
constexpr int kI32Fields = 4;  // per chunk: pos, neg (a magnitude), kept count, ~first fault code

__device__ inline void add_parts(uint64_t& pos, uint64_t& neg, int32_t x) {
  pos += (uint32_t)max(x, 0);
  neg += 0u - (uint32_t)min(x, 0);  // |x| of a negative x, 2^31 for int.MinValue
}

template <int RD>
__global__ __launch_bounds__(kSumBlock) void where_select_sum_i32_pass1(const dc_linq_chain prog,
                                                                        const float* __restrict__ in, int64_t n,
                                                                        int64_t h, int64_t* __restrict__ part) {
  __shared__ int64_t lds[kSumBlock / dc::kWave];
  __shared__ unsigned long long s_fault;
  const int G = gridDim.x, C = G + 2;  // chunk c of workgroup c; G = head, G + 1 = tail
  uint64_t pos = 0, neg = 0, hpos = 0, hneg = 0, tpos = 0, tneg = 0, fault = 0;
  const AffineChain aff{};
  const RdConst canon{0.0f, 1.0f, -0.0f};
  const int64_t cnt = visit_chunk<RD>(
      prog, aff, canon, in, n, h,
      [&](const float (&e)[16], const bool (&kept)[16], int64_t) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 16; ++j) add_parts(pos, neg, kept[j] ? __builtin_bit_cast(int32_t, e[j]) : 0);
      },
      [&](float x, bool kept, int64_t) __attribute__((always_inline)) {
        add_parts(pos, neg, kept ? __builtin_bit_cast(int32_t, x) : 0);
      },
      [&](float x, bool kept, int64_t i) __attribute__((always_inline)) {
        const int32_t v = kept ? __builtin_bit_cast(int32_t, x) : 0;
        if (i < h) add_parts(hpos, hneg, v);
        else add_parts(tpos, tneg, v);
      },
      &fault);
  if (threadIdx.x == 0) s_fault = 0;
  const int64_t bpos = dc::block_sum64<kSumBlock>((int64_t)pos, lds);
  const int64_t bneg = dc::block_sum64<kSumBlock>((int64_t)neg, lds);
  const int64_t bcnt = dc::block_sum64<kSumBlock>(cnt, lds);
  if (fault) atomicMax(&s_fault, (unsigned long long)fault);
  const bool last = blockIdx.x == (unsigned)G - 1u;  // uniform: the block sums below are collective
  int64_t lp[4] = {0, 0, 0, 0};
  if (last) {
    lp[0] = dc::block_sum64<kSumBlock>((int64_t)hpos, lds);
    lp[1] = dc::block_sum64<kSumBlock>((int64_t)hneg, lds);
    lp[2] = dc::block_sum64<kSumBlock>((int64_t)tpos, lds);
    lp[3] = dc::block_sum64<kSumBlock>((int64_t)tneg, lds);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const int b = blockIdx.x;
    part[b] = bpos;
    part[C + b] = bneg;
    part[2 * C + b] = bcnt;  // the loose elements' kept count is in the last chunk's count
    part[3 * C + b] = (int64_t)s_fault;
    if (last) {
      part[G] = lp[0];
      part[C + G] = lp[1];
      part[G + 1] = lp[2];
      part[C + G + 1] = lp[3];
      part[2 * C + G] = part[2 * C + G + 1] = 0;
      part[3 * C + G] = part[3 * C + G + 1] = 0;
    }
  }
}

__device__ inline bool fits_i32(int64_t v) { return v >= (int64_t)INT32_MIN && v <= (int64_t)INT32_MAX; }

template <int RD>
__global__ __launch_bounds__(kFinalBlock) void where_select_sum_i32_pass2(
    const dc_linq_chain prog, const float* __restrict__ in, int64_t n, int64_t h, const int64_t* __restrict__ part,
    int G, int64_t* __restrict__ sum_out, int64_t* __restrict__ count_out, int32_t* __restrict__ overflow_out,
    int64_t* __restrict__ fault_out) {
  constexpr int W = kFinalBlock / dc::kWave;
  __shared__ int64_t lds[W];
  __shared__ int64_t wpre[W];
  __shared__ unsigned long long s_fault;
  __shared__ int s_ovf, s_nflag;
  __shared__ int s_flag[kFinalBlock];
  __shared__ int64_t s_start[kFinalBlock];
  __shared__ int64_t tr_s[kFinalBlock], tr_max[kFinalBlock], tr_min[kFinalBlock];
  const int C = G + 2;
  const int t = threadIdx.x, lane = t & (dc::kWave - 1), wave = t / dc::kWave;
  // sequence slot t: 0 = head, 1 .. G = chunk t - 1, G + 1 = tail
  const int c = t == 0 ? G : (t <= G ? t - 1 : (t == G + 1 ? G + 1 : -1));
  int64_t pos = 0, neg = 0, cnt = 0;
  uint64_t fault = 0;
  if (c >= 0) {
    pos = part[c];
    neg = part[C + c];
    cnt = part[2 * C + c];
    fault = (uint64_t)part[3 * C + c];
  }
  if (t == 0) {
    s_fault = 0;
    s_ovf = 0;
    s_nflag = 0;
  }
  const int64_t sum = pos - neg;
  // exclusive scan of the chunk sums in sequence order: within each wave, then over the wave totals
  const int64_t incl = dc::wave_inclusive_scan64(sum);
  if (lane == dc::kWave - 1) lds[wave] = incl;
  __syncthreads();
  if (t == 0) {
    int64_t run = 0;
    for (int w = 0; w < W; ++w) {
      wpre[w] = run;
      run += lds[w];
    }
  }
  __syncthreads();
  const int64_t S = wpre[wave] + incl - sum;
  if (fault) atomicMax(&s_fault, (unsigned long long)fault);
  bool flagged = false;
  if (c >= 0) {
    if (!fits_i32(S + sum)) atomicOr(&s_ovf, 1);
    else if (!fits_i32(S + pos) || !fits_i32(S - neg)) flagged = true;
  }
  const int64_t total = dc::block_sum64<kFinalBlock>(sum, lds);
  const int64_t total_cnt = dc::block_sum64<kFinalBlock>(cnt, lds);
  if (flagged) {
    const int k = atomicAdd(&s_nflag, 1);
    s_flag[k] = t;
    s_start[k] = S;
  }
  __syncthreads();
  const int64_t n4 = (n - h) >> 2;
  const int64_t per = (n4 + G - 1) / G;
  const AffineChain aff{};
  const RdConst canon{0.0f, 1.0f, -0.0f};
  // Exact check of the flagged chunks (none when a fault or an overflow is already known).
  for (int k = 0; k < s_nflag && s_fault == 0 && s_ovf == 0; ++k) {
    const int slot = s_flag[k];
    int64_t a, b;
    if (slot == 0) {
      a = 0;
      b = h;
    } else if (slot == G + 1) {
      a = h + 4 * n4;
      b = n;
    } else {
      const int64_t v0 = min(n4, (int64_t)(slot - 1) * per), v1 = min(n4, v0 + per);
      a = h + 4 * v0;
      b = h + 4 * v1;
    }
    const int64_t piece = (b - a + kFinalBlock - 1) / kFinalBlock;
    const int64_t i0 = min(b, a + t * piece), i1 = min(b, i0 + piece);
    int64_t rs = 0, mx = 0, mn = 0;  // prefix relative to the chunk start, its max and min (empty prefix included)
    for (int64_t i = i0; i < i1; ++i) {
      float e[1] = {in[i]};
      bool kept[1];
      Faults f;
      eval_flags<RD, 1>(prog, aff, canon, e, kept, 1u, f);
      rs += kept[0] ? (int64_t)__builtin_bit_cast(int32_t, e[0]) : 0;
      mx = max(mx, rs);
      mn = min(mn, rs);
    }
    tr_s[t] = rs;
    tr_max[t] = mx;
    tr_min[t] = mn;
    __syncthreads();
    for (int stride = 1; stride < kFinalBlock; stride <<= 1) {
      if ((t & (2 * stride - 1)) == 0) {  // (left = t, right = t + stride), in sequence order
        const int r = t + stride;
        const int64_t ls = tr_s[t];
        tr_max[t] = max(tr_max[t], ls + tr_max[r]);
        tr_min[t] = min(tr_min[t], ls + tr_min[r]);
        tr_s[t] = ls + tr_s[r];
      }
      __syncthreads();
    }
    if (t == 0 && (!fits_i32(s_start[k] + tr_max[0]) || !fits_i32(s_start[k] + tr_min[0]))) s_ovf = 1;
    __syncthreads();
  }
  if (t == 0) {
    if (sum_out) *sum_out = total;
    if (count_out) *count_out = total_cnt;
    if (overflow_out) *overflow_out = s_ovf;
    if (fault_out) *fault_out = s_fault ? (int64_t)~(uint64_t)s_fault : (int64_t)DC_LINQ_FAULT_NONE;
  }
}

// ---- Where/Select -> Min / Max over int32 --------------------------------------------------------
// Math.Min/Max over int32 has no ties to break (equal elements are the same value) and no NaN, so a
// plain min/max tree is the enumerator's result.
template <int OP>
__device__ inline int32_t pick(int32_t a, int32_t b) { return OP == kOpMin ? min(a, b) : max(a, b); }

template <int OP, int BLOCK>
__device__ inline int32_t block_pick(int32_t v, int32_t* scratch) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = pick<OP>(v, __shfl_xor(v, off, 64));
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  __syncthreads();
  v = scratch[0];
  for (int w = 1; w < BLOCK / dc::kWave; ++w) v = pick<OP>(v, scratch[w]);
  __syncthreads();
  return v;
}

template <int RD, int OP>
__global__ __launch_bounds__(kSumBlock) void where_select_minmax_i32_pass1(const dc_linq_chain prog,
                                                                           const float* __restrict__ in, int64_t n,
                                                                           int64_t h, int64_t* __restrict__ part) {
  __shared__ int64_t lds[kSumBlock / dc::kWave];
  __shared__ int32_t lds_v[kSumBlock / dc::kWave];
  __shared__ unsigned long long s_fault;
  const int G = gridDim.x;
  int32_t best = OP == kOpMin ? INT32_MAX : INT32_MIN;  // the identity: an empty chunk changes nothing
  uint64_t fault = 0;
  auto take = [&](float x, bool kept) __attribute__((always_inline)) {
    best = kept ? pick<OP>(best, __builtin_bit_cast(int32_t, x)) : best;
  };
  const AffineChain aff{};
  const RdConst canon{0.0f, 1.0f, -0.0f};
  const int64_t cnt = visit_chunk<RD>(
      prog, aff, canon, in, n, h,
      [&](const float (&e)[16], const bool (&kept)[16], int64_t) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 16; ++j) take(e[j], kept[j]);
      },
      [&](float x, bool kept, int64_t) __attribute__((always_inline)) { take(x, kept); },
      [&](float x, bool kept, int64_t) __attribute__((always_inline)) { take(x, kept); }, &fault);
  if (threadIdx.x == 0) s_fault = 0;
  const int32_t bbest = block_pick<OP, kSumBlock>(best, lds_v);
  const int64_t bcnt = dc::block_sum64<kSumBlock>(cnt, lds);
  if (fault) atomicMax(&s_fault, (unsigned long long)fault);
  __syncthreads();
  if (threadIdx.x == 0) {
    part[blockIdx.x] = bbest;
    part[G + blockIdx.x] = bcnt;
    part[2 * G + blockIdx.x] = (int64_t)s_fault;
  }
}

template <int OP>
__global__ __launch_bounds__(kFinalBlock) void where_select_minmax_i32_pass2(const int64_t* __restrict__ part, int G,
                                                                             int32_t* __restrict__ value_out,
                                                                             int64_t* __restrict__ count_out,
                                                                             int64_t* __restrict__ fault_out) {
  __shared__ int64_t lds[kFinalBlock / dc::kWave];
  __shared__ int32_t lds_v[kFinalBlock / dc::kWave];
  __shared__ unsigned long long s_fault;
  int32_t v = OP == kOpMin ? INT32_MAX : INT32_MIN;
  int64_t c = 0;
  uint64_t fault = 0;
  for (int b = threadIdx.x; b < G; b += kFinalBlock) {
    v = pick<OP>(v, (int32_t)part[b]);
    c += part[G + b];
    fault = max(fault, (uint64_t)part[2 * G + b]);
  }
  if (threadIdx.x == 0) s_fault = 0;
  const int32_t bv = block_pick<OP, kFinalBlock>(v, lds_v);
  const int64_t bc = dc::block_sum64<kFinalBlock>(c, lds);
  if (fault) atomicMax(&s_fault, (unsigned long long)fault);
  __syncthreads();
  if (threadIdx.x == 0) {
    if (value_out) *value_out = bv;
    if (count_out) *count_out = bc;
    if (fault_out) *fault_out = s_fault ? (int64_t)~(uint64_t)s_fault : (int64_t)DC_LINQ_FAULT_NONE;
  }
}


// Scratch of dc_hip_linq_where_select_sum_f32_noalloc: one launch's per-workgroup partials (a
// float64 sum and an int64 count per workgroup, at most kSumBlocksMax workgroups), 16 KiB. One copy
// per GPU, held until the process ends; every call on a GPU uses it, and the calls of this process
// on one GPU are ordered one after another (dc::ResidentLaunch, kind kOrderNoAlloc). Pass 1 writes
// every entry pass 2 reads, so nothing needs clearing between calls.
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

// Order keys of pass 1. Within a thread elements arrive in sequence order, where the enumerator's
// rule needs no index: Min replaces its value by a later one only if that is smaller, or if it is
// a NaN and no NaN is held; Max only if it is larger, or if only NaNs are held. Both follow from an
// integer key per element whose order is the comparison order with -0 and +0 one key (the
// magnitude, negated for a negative sign) and NaN one key: Min's below every number, Max's below
// every number but above "not kept". A strict key comparison is then the rule (with Max's
// NaN-after-NaN case added), and a run of elements reduces as a plain integer min/max tree.
// Only keys 0 (a zero of either sign) and NaN stand for more than one bit pattern; for every
// other key the winner's bits follow from the key, so the winner's position is looked up only
// when the key is one of those two.
template <int OP>
struct MmKey {
  static constexpr int32_t kAbsent = OP == kOpMin ? INT32_MAX : INT32_MIN;
  static constexpr int32_t kNan = OP == kOpMin ? INT32_MIN : INT32_MIN + 1;
};

template <int OP>
__device__ inline int32_t mm_key(float x, bool kept) {
  const int32_t b = __builtin_bit_cast(int32_t, x);
  const int32_t sgn = b >> 31;                         // 0 or -1
  const int32_t key = ((b & 0x7FFFFFFF) ^ sgn) - sgn;  // +-magnitude
  return !kept ? MmKey<OP>::kAbsent : (__builtin_isnan(x) ? MmKey<OP>::kNan : key);
}

__device__ inline uint32_t mm_key_bits(int32_t key) {  // inverse of mm_key for keys other than 0 / NaN
  const int32_t sgn = key >> 31;
  return (uint32_t)((key ^ sgn) - sgn) | ((uint32_t)sgn & 0x80000000u);
}

template <int OP>
__device__ inline bool mm_key_later_wins(int32_t cur, int32_t x) {
  if (OP == kOpMin) return x < cur;
  return x > cur || (x == MmKey<OP>::kNan && cur == MmKey<OP>::kNan);
}

template <int RD, int OP>
__global__ __launch_bounds__(kSumBlock) void where_select_minmax_pass1(const dc_linq_chain prog, const AffineChain aff,
                                                                       const RdConst canon, const float* __restrict__ in,
                                                                       int64_t n, int64_t h, float* __restrict__ pv,
                                                                       int64_t* __restrict__ pi,
                                                                       int64_t* __restrict__ pcnt) {
  // Thread state: the winner's key and bits and where it came from, as (vector base, position id
  // in its half); the sequence index is formed once, at the end (meaningful for keys 0 and NaN,
  // where it breaks ties between threads; any index of the same bits serves the other keys). The
  // loose head and tail elements are gathered apart with the index-ordered rule and joined after.
  int32_t rk = MmKey<OP>::kAbsent;
  uint32_t rbits = 0;
  int64_t rbase = 0;
  int rid = 0;
  float lv = 0.0f;
  int64_t li = -1;
  int64_t cnt = visit_chunk<RD>(
      prog, aff, canon, in, n, h,
      [&](const float (&e)[16], const bool (&kept)[16], int64_t base) __attribute__((always_inline)) {
        // Fast path: IEEE-754-2019 minimum/maximum (three operands per instruction) over the kept
        // values, the others replaced by the identity (+inf for Min, -inf for Max). It propagates
        // NaN and orders -0 below +0, so its result is the half's winner, bits included, unless
        // it is a NaN or a zero; those halves (and only those) take the exact key path.
        constexpr float kFill = OP == kOpMin ? __builtin_inff() : -__builtin_inff();
        float f[16];
        bool any = false;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          f[j] = kept[j] ? e[j] : kFill;
          any = any || kept[j];
        }
        auto mm3 = [](float x, float y, float z) __attribute__((always_inline)) {
          return OP == kOpMin ? __builtin_elementwise_minimum(__builtin_elementwise_minimum(x, y), z)
                              : __builtin_elementwise_maximum(__builtin_elementwise_maximum(x, y), z);
        };
        const float g0 = mm3(f[0], f[1], f[2]), g1 = mm3(f[3], f[4], f[5]), g2 = mm3(f[6], f[7], f[8]);
        const float g3 = mm3(f[9], f[10], f[11]), g4 = mm3(f[12], f[13], f[14]);
        const float m = mm3(mm3(g0, g1, g2), mm3(g3, g4, f[15]), kFill);
        int32_t hk = any ? mm_key<OP>(m, true) : MmKey<OP>::kAbsent;
        uint32_t bits = __builtin_bit_cast(uint32_t, m);
        int id = 0;
        if (any && (__builtin_isnan(m) || m == 0.0f)) {
          int32_t k[16];
#pragma unroll
          for (int j = 0; j < 16; ++j) k[j] = mm_key<OP>(e[j], kept[j]);
          hk = k[0];
#pragma unroll
          for (int j = 1; j < 16; ++j) hk = OP == kOpMin ? min(hk, k[j]) : max(hk, k[j]);
          // the enumerator's element among equal keys: the first, or for Max over NaNs the last
          const bool last = OP == kOpMax && hk == MmKey<OP>::kNan;
          bool found = false;
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const bool hit = k[j] == hk && (last || !found);
            bits = hit ? __builtin_bit_cast(uint32_t, e[j]) : bits;
            id = hit ? j : id;
            found = found || hit;
          }
        }
        if (mm_key_later_wins<OP>(rk, hk)) {
          rk = hk;
          rbits = bits;
          rbase = base;
          rid = id;
        }
      },
      [&](float x, bool kept, int64_t idx) __attribute__((always_inline)) {
        const int32_t xk = mm_key<OP>(x, kept);
        if (mm_key_later_wins<OP>(rk, xk)) {
          rk = xk;
          rbits = __builtin_bit_cast(uint32_t, x);
          rbase = (idx - h) >> 2;  // idx = h + 4 * vector + lane
          rid = (int)((idx - h) & 3);
        }
      },
      [&](float x, bool kept, int64_t idx) __attribute__((always_inline)) {
        if (kept) mm_take<OP>(lv, li, x, idx);
      });
  float bv = __builtin_bit_cast(float, rbits);
  int64_t bi = rk != MmKey<OP>::kAbsent ? h + 4 * (rbase + (int64_t)(rid >> 2) * kSumBlock) + (rid & 3) : -1;
  mm_take<OP>(bv, bi, lv, li);
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

// ---- Where/Select -> Aggregate((acc, x) => MathF.Min(acc, x)) / MathF.Max -----------------------
// MathF.Min and MathF.Max are IEEE 754-2019 minimum / maximum: a NaN operand gives NaN, and -0
// orders below +0. The fold is then associative and commutative (up to which NaN it returns, and
// .NET gives NaN payloads no meaning), so each partial is a plain value and the grid's result is the
// sequential fold's, whatever the order in which lanes, waves and workgroups meet. A dropped
// element contributes the identity (+inf for Min, -inf for Max), which changes no result. Every
// program variant of the other reductions runs it (the canonical shapes too).
template <int OP>
__device__ inline float fold_op(float a, float b) {
  return OP == kOpMin ? __builtin_elementwise_minimum(a, b) : __builtin_elementwise_maximum(a, b);
}

template <int OP>
constexpr float fold_identity() {
  return OP == kOpMin ? __builtin_inff() : -__builtin_inff();
}

// Block-wide fold; the result is valid in thread 0.
template <int OP, int BLOCK>
__device__ inline float fold_block(float v, float* scratch) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fold_op<OP>(v, __shfl_xor(v, off, 64));
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  __syncthreads();
  if (threadIdx.x == 0)
    for (int w = 1; w < BLOCK / dc::kWave; ++w) v = fold_op<OP>(v, scratch[w]);
  return v;
}

template <int RD, int OP>
__global__ __launch_bounds__(kSumBlock) void where_select_fold_pass1(const dc_linq_chain prog, const AffineChain aff,
                                                                     const RdConst canon, const float* __restrict__ in,
                                                                     int64_t n, int64_t h, float* __restrict__ pv,
                                                                     int64_t* __restrict__ pcnt) {
  __shared__ float lds_f[kSumBlock / dc::kWave];
  __shared__ int64_t lds_i[kSumBlock / dc::kWave];
  constexpr float kId = fold_identity<OP>();
  float acc = kId;
  auto one = [&](float x, bool kept, int64_t) __attribute__((always_inline)) { acc = fold_op<OP>(acc, kept ? x : kId); };
  const int64_t cnt = visit_chunk<RD>(
      prog, aff, canon, in, n, h,
      [&](const float (&e)[16], const bool (&kept)[16], int64_t) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 16; ++j) acc = fold_op<OP>(acc, kept[j] ? e[j] : kId);
      },
      one, one);
  const float bv = fold_block<OP, kSumBlock>(acc, lds_f);
  const int64_t bcnt = dc::block_sum64<kSumBlock>(cnt, lds_i);
  if (threadIdx.x == 0) {
    pv[blockIdx.x] = bv;
    pcnt[blockIdx.x] = bcnt;
  }
}

template <int OP>
__global__ __launch_bounds__(kFinalBlock) void where_select_fold_pass2(const float* __restrict__ pv,
                                                                       const int64_t* __restrict__ pcnt, int count,
                                                                       float* __restrict__ value_out,
                                                                       int64_t* __restrict__ count_out) {
  __shared__ float lds_f[kFinalBlock / dc::kWave];
  __shared__ int64_t lds_i[kFinalBlock / dc::kWave];
  float v = fold_identity<OP>();
  int64_t c = 0;
  for (int b = threadIdx.x; b < count; b += kFinalBlock) {
    v = fold_op<OP>(v, pv[b]);
    c += pcnt[b];
  }
  v = fold_block<OP, kFinalBlock>(v, lds_f);
  const int64_t total = dc::block_sum64<kFinalBlock>(c, lds_i);
  if (threadIdx.x == 0) {
    if (value_out) *value_out = total ? v : 0.0f;
    if (count_out) *count_out = total;
  }
}

// ---- strategy choice -----------------------------------------------------------------------------
const void* rounds_kernel(int mode) {
  const void* fn = nullptr;
  auto pick = [&](auto m) { fn = reinterpret_cast<const void*>(&where_select_rounds_kernel<decltype(m)::value>); };
  if (rd_is_int(mode)) rd_dispatch_i32(mode, pick);
  else rd_dispatch(mode, pick);
  return fn;
}

// Every program variant (rd_dispatch's and rd_dispatch_i32's cases).
std::vector<int> all_reduce_modes() {
  std::vector<int> m = {kRdInterp, kRdInterpSaves, kRdInterpLibm, kRdAffine, kRdInterpI32, kRdInterpI32Saves,
                        rd_canon(kShapeM, DC_LQ_CMP_GT)};
  for (int shape : {kShapeF, kShapeFM, kShapeMF})
    for (int cmp = DC_LQ_CMP_GT; cmp <= DC_LQ_CMP_NE; ++cmp) m.push_back(rd_canon(shape, cmp));
  return m;
}

// Workgroups of the round-robin grid over n (16-byte aligned) elements: one per CU, or one per
// tile when the input has fewer tiles than CUs (then each owns one tile of the only round).
uint32_t rounds_groups(const dc_hip_ctx* ctx, int64_t n) {
  const int64_t tiles = (n + kRrTile - 1) / kRrTile;
  return (uint32_t)std::max<int64_t>(1, std::min<int64_t>(tiles, std::min(ctx->cu_count, kRrMaxGroups)));
}

// Elements before the first 16-byte boundary of a 4-byte aligned input (0..3, at most n), or -1
// for an input that is not 4-byte aligned.
int64_t head16(const float* input, int64_t n) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(input);
  if (a & 3) return -1;
  return std::min<int64_t>(n, (int64_t)(((16 - (a & 15)) & 15) >> 2));
}

// The round-robin kernel takes every 4-byte aligned input (it peels the 0..3 head elements before
// the first 16-byte boundary) when one workgroup fits per CU (every program variant; asked once
// per context). Measured against the lookback kernel (50 % kept, cache-resident below 64M): 16K
// elements 5.1 against 6.7 us, 1M 7.2 against 10.1, 4M 10.0 against 15.1, 8M 14.7 against 24.1;
// at 3M, one full round plus a tail round, 13.5 against 13.1. The caller holds the context lock.
bool use_rounds(dc_hip_ctx* ctx, const float* input, int64_t n) {
  const int64_t h = head16(input, n);
  if (h < 0 || ctx->cu_count <= 0) return false;
  if (ctx->rounds_fit < 0) {
    bool fit = true;
    for (int mode : all_reduce_modes()) {
      int per_cu = 0;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, rounds_kernel(mode), kRrBlock, 0) != hipSuccess ||
          per_cu < 1)
        fit = false;
    }
    ctx->rounds_fit = fit ? 1 : 0;
  }
  return ctx->rounds_fit == 1;
}

// The chain the int32 interpreter kernels run: every DIV/REM by a constant outside {0, -1, 1}
// preceded by a kOpDivMagic instruction carrying its multiply-high constants, computed here once
// per launch (the original chain when the inserted instructions would not fit).
dc_linq_chain device_chain_i32(const dc_linq_chain& c) {
  auto const_div = [](const dc_linq_instr& in) {
    return (in.op == DC_LQ_DIV || in.op == DC_LQ_REM) && in.src == DC_LQ_SRC_IMM && in.imm_i32 != 0 &&
           in.imm_i32 != -1 && in.imm_i32 != 1;
  };
  int extra = 0;
  for (int i = 0; i < c.n_instr; ++i) extra += const_div(c.code[i]) ? 1 : 0;
  if (extra == 0 || c.n_instr + extra > DC_LINQ_MAX_INSTR) return c;
  dc_linq_chain out = c;
  int k = 0;
  for (int i = 0; i < c.n_instr; ++i) {
    if (const_div(c.code[i])) {
      const dc::DivMagic g = dc::div_magic(c.code[i].imm_i32);
      dc_linq_instr m{};
      m.op = (uint8_t)kOpDivMagic;
      m.src = DC_LQ_SRC_IMM;
      m.mode = (uint8_t)g.s;
      m.imm_i32 = g.m;
      out.code[k++] = m;
    }
    out.code[k++] = c.code[i];
  }
  out.n_instr = k;
  return out;
}

// Whether ToArray launches run-time compiled kernels (off; see launch_to_array).
constexpr bool kLaunchCompiled = false;

// ToArray for both element types (the caller holds the context lock and has validated the chain):
// the round-robin kernel for large aligned inputs, else the ticket-ordered lookback kernel. int32
// programs publish their exceptions into the context's fault word.
int32_t launch_to_array(dc_hip_ctx* ctx, const dc_linq_chain* chain, bool is_int, const float* input, int64_t n,
                        float* output, int64_t* count_out) {
  uint64_t* fault_word = reinterpret_cast<uint64_t*>(ctx->counters + DC_SLOT_LINQ_FAULT);
  if ((chain->flags & DC_LINQ_FLAG_ORDERED_GRID) == 0 && use_rounds(ctx, input, n)) {
    const ReducePlan plan = is_int ? reduce_plan_i32(*chain) : reduce_plan(*chain);
    const void* fn = rounds_kernel(plan.mode);
    // Programs the prebuilt kernels interpret can run on a kernel compiled for them
    // (dc::linq_jit_rounds). Switched off: a compiled kernel for a filtered division faulted the
    // device and its cause is not found yet, so every program runs on the interpreter.
    hipFunction_t jit = nullptr;
    const bool interpreted = is_int || rd_is_float_interp(plan.mode);
    if (kLaunchCompiled && interpreted && n >= DC_LINQ_COMPILE_MIN_ELEMENTS &&
        (chain->flags & DC_LINQ_FLAG_INTERPRET) == 0) {
      jit = dc::linq_jit_rounds(ctx, *chain, is_int);
      if (!jit) ++ctx->jit_failures;
    }
    AffineChain aff = plan.aff;
    RdConst canon = plan.k;
    const int head_n = (int)head16(input, n);  // 0..3: use_rounds accepted the input
    const uint32_t groups = rounds_groups(ctx, n - head_n);
    const int64_t tiles = (n - head_n + kRrTile - 1) / kRrTile;
    const size_t words = (size_t)((tiles + groups - 1) / groups + 1) * groups;
    uint32_t epoch16 = 0;
    DC_RETURN_IF(dc::ensure_round_counts(ctx, words, &epoch16));
    dc_linq_chain prog = is_int ? device_chain_i32(*chain) : *chain;
    const float* in_arg = input + head_n;
    int64_t n_arg = n - head_n;
    const float* head_arg = input;
    int head_arg_n = head_n;
    float* out_arg = output;
    int64_t* count_arg = count_out;
    uint32_t* counts_arg = ctx->round_counts;
    uint32_t groups_arg = groups;
    uint32_t* done_arg = ctx->counters + DC_SLOT_LINQ_DONE;
    uint64_t* fault_arg = fault_word;
    void* args[] = {&prog,       &aff,     &canon,      &in_arg,   &n_arg,     &out_arg,  &count_arg,
                    &counts_arg, &epoch16, &groups_arg, &done_arg, &fault_arg, &head_arg, &head_arg_n};
    // One workgroup per CU, each needing most of a CU's LDS, on an otherwise idle device: every
    // workgroup is resident at once (an ordinary launch; measured faster than a cooperative one).
    dc::ResidentLaunch resident(ctx);
    DC_RETURN_IF(resident.status());
    if (jit) {
      DC_RETURN_IF_HIP(hipModuleLaunchKernel(jit, groups, 1, 1, kRrBlock, 1, 1, 0, ctx->stream, args, nullptr));
      ++ctx->jit_launches;
    } else {
      DC_RETURN_IF_HIP(hipLaunchKernel(fn, dim3(groups), dim3(kRrBlock), args, 0, ctx->stream));
    }
    DC_RETURN_IF(dc::last_launch_status());
    resident.done();
    return DC_OK;
  }

  AffineChain aff{};
  const bool saves = program_uses_saves(*chain);
  const bool affine = !is_int && lower_affine(*chain, &aff);
  const int mode = is_int ? (saves ? kModeInterpI32Saves : kModeInterpI32)
                  : affine ? kModeAffine
                  : program_uses_libm(*chain) ? kModeInterpLibm
                                              : (saves ? kModeInterpSaves : kModeInterp);
  const int64_t tiles = std::max<int64_t>(1, (n + kTile - 1) / kTile);
  if (tiles > 0x7FFFFFFFll) return DC_ERR_INVALID_ARGUMENT;
  uint32_t epoch = 0;
  DC_RETURN_IF(dc::ensure_status(ctx, (size_t)tiles, &epoch));
  auto kernel = mode == kModeAffine            ? where_select_kernel<kModeAffine>
              : mode == kModeInterpSaves       ? where_select_kernel<kModeInterpSaves>
              : mode == kModeInterpLibm        ? where_select_kernel<kModeInterpLibm>
              : mode == kModeInterpI32         ? where_select_kernel<kModeInterpI32>
              : mode == kModeInterpI32Saves    ? where_select_kernel<kModeInterpI32Saves>
                                               : where_select_kernel<kModeInterp>;
  kernel<<<(unsigned)tiles, kBlock, 0, ctx->stream>>>(is_int ? device_chain_i32(*chain) : *chain, aff, input, n,
                                                     output, count_out, ctx->status,
                                                      ctx->counters + DC_SLOT_LINQ_TICKET, epoch, (uint32_t)tiles,
                                                      dc::aligned16(input) ? 1 : 0, fault_word);
  return dc::last_launch_status();
}

// Structural validation plus the int32 rule: no SQRT / FLOOR / CEIL / ROUND / POW (no int form).
int32_t validate_i32(const dc_linq_chain* chain) {
  DC_RETURN_IF(dc_linq_chain_validate(chain));
  for (int i = 0; i < chain->n_instr; ++i) {
    const uint8_t op = chain->code[i].op;
    if (op == DC_LQ_SQRT || op == DC_LQ_FLOOR || op == DC_LQ_CEIL || op == DC_LQ_ROUND || op == DC_LQ_POW ||
        op == DC_LQ_RPOW)
      return DC_ERR_UNSUPPORTED;
  }
  return DC_OK;
}

bool can_fault_i32(const dc_linq_chain& chain) {
  for (int i = 0; i < chain.n_instr; ++i) {
    const dc_linq_instr& in = chain.code[i];
    if (in.op == DC_LQ_ABS || in.op == DC_LQ_RDIV || in.op == DC_LQ_RREM) return true;
    if ((in.op == DC_LQ_DIV || in.op == DC_LQ_REM) &&
        (in.src != DC_LQ_SRC_IMM || in.imm_i32 == 0 || in.imm_i32 == -1))
      return true;
  }
  return false;
}

}  // namespace

extern "C" {

DC_HIP_API int32_t dc_linq_chain_validate(const dc_linq_chain* chain) {
  if (!chain) return DC_ERR_INVALID_ARGUMENT;
  if (chain->n_instr < 0 || chain->n_instr > DC_LINQ_MAX_INSTR ||
      (chain->flags & ~(DC_LINQ_FLAG_ORDERED_GRID | DC_LINQ_FLAG_INTERPRET)) != 0)
    return DC_ERR_INVALID_ARGUMENT;
  for (int i = 0; i < chain->n_instr; ++i) {
    const dc_linq_instr& in = chain->code[i];
    const bool op_ok = (in.op <= DC_LQ_ROUND) || (in.op >= DC_LQ_CMP_GT && in.op <= DC_LQ_RPOW);
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
  return launch_to_array(ctx, chain, false, input, n, output, count_out);
}

DC_HIP_API int32_t dc_linq_chain_validate_i32(const dc_linq_chain* chain) { return validate_i32(chain); }

DC_HIP_API int32_t dc_linq_chain_can_fault_i32(const dc_linq_chain* chain, int32_t* can_fault_out) {
  if (!can_fault_out) return DC_ERR_INVALID_ARGUMENT;
  DC_RETURN_IF(validate_i32(chain));
  *can_fault_out = can_fault_i32(*chain) ? 1 : 0;
  return DC_OK;
}

DC_HIP_API int32_t dc_hip_linq_where_select_i32(dc_hip_ctx* ctx, const dc_linq_chain* chain, const int32_t* input,
                                                int64_t n, int32_t* output, int64_t* count_out, int64_t* fault_out) {
  if (n < 0 || !count_out || (n > 0 && (!input || !output))) return DC_ERR_INVALID_ARGUMENT;
  DC_RETURN_IF(validate_i32(chain));
  if (!fault_out && can_fault_i32(*chain)) return DC_ERR_INVALID_ARGUMENT;
  if (n >= (int64_t)1 << 40) return DC_ERR_INVALID_ARGUMENT;  // 40-bit counts in the status words
  DC_CTX_ENTER(ctx);
  DC_RETURN_IF(launch_to_array(ctx, chain, true, reinterpret_cast<const float*>(input), n,
                               reinterpret_cast<float*>(output), count_out));
  if (fault_out) {
    fault_finish_kernel<<<1, 1, 0, ctx->stream>>>(reinterpret_cast<uint64_t*>(ctx->counters + DC_SLOT_LINQ_FAULT),
                                                  fault_out);
    DC_RETURN_IF(dc::last_launch_status());
  }
  return DC_OK;
}

DC_HIP_API int32_t dc_hip_linq_where_select_sum_i32(dc_hip_ctx* ctx, const dc_linq_chain* chain, const int32_t* input,
                                                    int64_t n, int64_t* sum_out, int64_t* count_out,
                                                    int32_t* overflow_out, int64_t* fault_out) {
  if (n < 0 || (n > 0 && !input)) return DC_ERR_INVALID_ARGUMENT;
  if (n >= ((int64_t)1 << 32)) return DC_ERR_INVALID_ARGUMENT;  // int64 partial sums stay exact below 2^32 elements
  DC_RETURN_IF(validate_i32(chain));
  if (!fault_out && can_fault_i32(*chain)) return DC_ERR_INVALID_ARGUMENT;
  DC_CTX_ENTER(ctx);
  const unsigned grid = std::min<unsigned>(where_select_sum_grid(ctx, n), kFinalBlock - 2);
  DC_RETURN_IF(dc::ensure_partials(ctx, (size_t)(grid + 2) * kI32Fields * sizeof(int64_t)));
  int64_t* part = static_cast<int64_t*>(ctx->partials);
  const float* in = reinterpret_cast<const float*>(input);
  const int64_t h = reduce_head(in, n);
  const dc_linq_chain dev = device_chain_i32(*chain);
  rd_dispatch_i32(reduce_plan_i32(*chain).mode, [&](auto mode) {
    constexpr int RD = decltype(mode)::value;
    where_select_sum_i32_pass1<RD><<<grid, kSumBlock, 0, ctx->stream>>>(dev, in, n, h, part);
    where_select_sum_i32_pass2<RD><<<1, kFinalBlock, 0, ctx->stream>>>(dev, in, n, h, part, (int)grid, sum_out,
                                                                      count_out, overflow_out, fault_out);
  });
  return dc::last_launch_status();
}

DC_HIP_API int32_t dc_hip_linq_where_select_minmax_i32(dc_hip_ctx* ctx, const dc_linq_chain* chain,
                                                       const int32_t* input, int64_t n, int32_t op, int32_t* value_out,
                                                       int64_t* count_out, int64_t* fault_out) {
  if (n < 0 || (n > 0 && !input) || (op != DC_LINQ_MIN && op != DC_LINQ_MAX)) return DC_ERR_INVALID_ARGUMENT;
  DC_RETURN_IF(validate_i32(chain));
  if (!fault_out && can_fault_i32(*chain)) return DC_ERR_INVALID_ARGUMENT;
  DC_CTX_ENTER(ctx);
  const unsigned grid = where_select_sum_grid(ctx, n);
  DC_RETURN_IF(dc::ensure_partials(ctx, (size_t)grid * 3 * sizeof(int64_t)));
  int64_t* part = static_cast<int64_t*>(ctx->partials);
  const float* in = reinterpret_cast<const float*>(input);
  const int64_t h = reduce_head(in, n);
  const dc_linq_chain dev = device_chain_i32(*chain);
  rd_dispatch_i32(reduce_plan_i32(*chain).mode, [&](auto mode) {
    constexpr int RD = decltype(mode)::value;
    if (op == DC_LINQ_MIN)
      where_select_minmax_i32_pass1<RD, kOpMin><<<grid, kSumBlock, 0, ctx->stream>>>(dev, in, n, h, part);
    else
      where_select_minmax_i32_pass1<RD, kOpMax><<<grid, kSumBlock, 0, ctx->stream>>>(dev, in, n, h, part);
  });
  if (op == DC_LINQ_MIN)
    where_select_minmax_i32_pass2<kOpMin><<<1, kFinalBlock, 0, ctx->stream>>>(part, (int)grid, value_out, count_out,
                                                                             fault_out);
  else
    where_select_minmax_i32_pass2<kOpMax><<<1, kFinalBlock, 0, ctx->stream>>>(part, (int)grid, value_out, count_out,
                                                                             fault_out);
  return dc::last_launch_status();
}

DC_HIP_API int32_t dc_hip_linq_where_select_sum_f32(dc_hip_ctx* ctx, const dc_linq_chain* chain, const float* input,
                                                    int64_t n, double* sum_out, int64_t* count_out) {
  if (n < 0 || (n > 0 && !input)) return DC_ERR_INVALID_ARGUMENT;
  DC_RETURN_IF(dc_linq_chain_validate(chain));
  DC_CTX_ENTER(ctx);
  const unsigned grid = where_select_sum_grid(ctx, n);
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
  const unsigned grid = where_select_sum_grid(ctx, n);
  // The grid is capped, so every n fits; the check keeps that invariant explicit.
  if ((size_t)grid * 16 > kNoAllocScratchBytes) return DC_ERR_OUT_OF_MEMORY;
  double* psum = static_cast<double*>(ctx->noalloc_scratch);  // never `scratch` itself: a host stand-in
  int64_t* pcnt = reinterpret_cast<int64_t*>(psum + grid);
  // Calls from different contexts on one device share the array: each is ordered behind the
  // previous one (an event recorded on that context's stream; nothing is allocated).
  dc::ResidentLaunch order(ctx, dc::kOrderNoAlloc);
  DC_RETURN_IF(order.status());
  DC_RETURN_IF(launch_where_select_sum(ctx, chain, input, n, grid, psum, pcnt, sum_out, count_out));
  order.done();
  return DC_OK;
}

DC_HIP_API int32_t dc_hip_linq_where_select_minmax_f32(dc_hip_ctx* ctx, const dc_linq_chain* chain,
                                                       const float* input, int64_t n, int32_t op, float* value_out,
                                                       int64_t* count_out) {
  if (n < 0 || (n > 0 && !input) || op < DC_LINQ_MIN || op > DC_LINQ_FOLD_MAX) return DC_ERR_INVALID_ARGUMENT;
  DC_RETURN_IF(dc_linq_chain_validate(chain));
  DC_CTX_ENTER(ctx);
  const unsigned grid = where_select_sum_grid(ctx, n);
  DC_RETURN_IF(dc::ensure_partials(ctx, (size_t)grid * 24));
  int64_t* pi = static_cast<int64_t*>(ctx->partials);
  int64_t* pcnt = pi + grid;
  float* pv = reinterpret_cast<float*>(pcnt + grid);
  const ReducePlan p = reduce_plan(*chain);
  const int64_t h = reduce_head(input, n);
  if (op == DC_LINQ_FOLD_MIN || op == DC_LINQ_FOLD_MAX) {
    rd_dispatch(p.mode, [&](auto mode) {
      constexpr int RD = decltype(mode)::value;
      if (op == DC_LINQ_FOLD_MIN)
        where_select_fold_pass1<RD, kOpMin><<<grid, kSumBlock, 0, ctx->stream>>>(*chain, p.aff, p.k, input, n, h, pv, pcnt);
      else
        where_select_fold_pass1<RD, kOpMax><<<grid, kSumBlock, 0, ctx->stream>>>(*chain, p.aff, p.k, input, n, h, pv, pcnt);
    });
    if (op == DC_LINQ_FOLD_MIN)
      where_select_fold_pass2<kOpMin><<<1, kFinalBlock, 0, ctx->stream>>>(pv, pcnt, (int)grid, value_out, count_out);
    else
      where_select_fold_pass2<kOpMax><<<1, kFinalBlock, 0, ctx->stream>>>(pv, pcnt, (int)grid, value_out, count_out);
    return dc::last_launch_status();
  }
  rd_dispatch(p.mode, [&](auto mode) {
    constexpr int RD = decltype(mode)::value;
    if (op == DC_LINQ_MIN)
      where_select_minmax_pass1<RD, kOpMin>
          <<<grid, kSumBlock, 0, ctx->stream>>>(*chain, p.aff, p.k, input, n, h, pv, pi, pcnt);
    else
      where_select_minmax_pass1<RD, kOpMax>
          <<<grid, kSumBlock, 0, ctx->stream>>>(*chain, p.aff, p.k, input, n, h, pv, pi, pcnt);
  });
  if (op == DC_LINQ_MIN)
    where_select_minmax_pass2<kOpMin><<<1, kFinalBlock, 0, ctx->stream>>>(pv, pi, pcnt, (int)grid, value_out, count_out);
  else
    where_select_minmax_pass2<kOpMax><<<1, kFinalBlock, 0, ctx->stream>>>(pv, pi, pcnt, (int)grid, value_out, count_out);
  return dc::last_launch_status();
}

}  // extern "C"

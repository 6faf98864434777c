// dc_linq.hip — fused LINQ Where/Select(/Sum) kernels for gfx950.
//
// One prebuilt kernel per terminal (ToArray, Sum) interprets the register program that the host
// fusion planner builds from the chain's lambdas (dc_linq_chain, program model in
// include/dotcompute_hip.h). The program lives in the kernel arguments, so every instruction is
// wave-uniform: dispatch is scalar branching, and each instruction is applied to the 16 elements a
// thread holds in registers.
//
// ToArray (order-preserving stream compaction, single pass):
//   tile = 256 threads x 16 elements = 4096 consecutive elements, claimed through an atomic
//   ticket (so a tile only ever waits on tiles that started before it);
//   thread t loads 16-byte vectors j = 0..3 at tile + j*1024 + t*4 (coalesced, non-temporal);
//   for each vector j and lane k the wave takes ballot(keep) -> the element's rank among the
//   kept elements of (j, wave) is sum_k' mbcnt(ballot_k') + (kept lanes k'' < k of this thread);
//   16 (j, wave) counts are scanned in LDS -> tile-local positions; the tile aggregate is
//   published for decoupled lookback and the tile's exclusive prefix is resolved by wave 0 from
//   the status words of up to 64 predecessors at once; kept values are staged in LDS in output
//   order and written out with coalesced stores.
// Every float operation rounds once (the file is compiled with -ffp-contract=off), so the output
// equals LINQ-to-objects bit-for-bit.
#include <algorithm>

#include "dc_device.hpp"
#include "dc_internal.hpp"

namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / dc::kWave;
constexpr int kVecPerThread = 4;
constexpr int kElemPerThread = 4 * kVecPerThread;  // 16
constexpr int kTile = kBlock * kElemPerThread;     // 4096
constexpr int kSumBlocksMax = 2048;

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

// Runs the program over the EPT elements of one thread. Returns the keep mask (bit j = element j).
// SAVES = false drops the s0/s1 registers for programs that never use them (the common case),
// which keeps the kernels at a higher occupancy. Operands are read in place (an immediate stays a
// scalar operand of the vector instruction), so no per-element operand copy is materialised.
template <int EPT, bool SAVES>
__device__ inline uint32_t run_program(const dc_linq_chain& prog, float (&e)[EPT]) {
  float v[EPT];
  float s0[SAVES ? EPT : 1], s1[SAVES ? EPT : 1];
#pragma unroll
  for (int j = 0; j < EPT; ++j) v[j] = 0.0f;
#pragma unroll
  for (int j = 0; j < (SAVES ? EPT : 1); ++j) { s0[j] = 0.0f; s1[j] = 0.0f; }
  uint32_t p = 0, q = 0, keep = (EPT == 32) ? 0xFFFFFFFFu : ((1u << EPT) - 1u);
  const int n = prog.n_instr;
  for (int pc = 0; pc < n; ++pc) {
    const dc_linq_instr ins = prog.code[pc];
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

// Called by all 64 lanes of wave 0. Returns the exclusive prefix of `tile` (valid in every lane).
__device__ inline int64_t lookback(uint64_t* __restrict__ status, int64_t tile, uint64_t aggregate,
                                   uint32_t epoch) {
  const int lane = threadIdx.x & 63;
  if (tile == 0) {
    if (lane == 0) dc::store_agent_u64(status, pack_status(kFlagInc, epoch, aggregate));
    return 0;
  }
  if (lane == 0) dc::store_agent_u64(status + tile, pack_status(kFlagAgg, epoch, aggregate));
  int64_t exclusive = 0;
  int64_t end = tile - 1;  // lane l inspects tile end - l
  while (true) {
    const int64_t idx = end - lane;
    bool valid = true, inc = true;
    uint64_t value = 0;
    if (idx >= 0) {
      uint64_t w = dc::load_agent_u64(status + idx);
      uint32_t w_epoch = (uint32_t)((w >> 40) & ((1u << 22) - 1));
      uint64_t flag = w & (3ull << 62);
      valid = (flag != 0) && (w_epoch == epoch);
      inc = valid && (flag == kFlagInc);
      value = w & kValueMask;
    }
    const uint64_t inc_mask = __ballot(inc);
    const uint64_t bad_mask = __ballot(!valid);
    const int limit = inc_mask ? __builtin_ctzll(inc_mask) : 63;  // lanes [0, limit] are needed
    const uint64_t need = (limit == 63) ? ~0ull : ((2ull << limit) - 1);
    if (bad_mask & need) {
      __builtin_amdgcn_s_sleep(1);
      continue;
    }
    int64_t contrib = (lane <= limit) ? (int64_t)value : 0;
    exclusive += dc::wave_sum64<int64_t>(contrib);
    if (inc_mask) break;
    end -= 64;
  }
  if (lane == 0) dc::store_agent_u64(status + tile, pack_status(kFlagInc, epoch, (uint64_t)exclusive + aggregate));
  return exclusive;
}

// ---- Where/Select -> ToArray ------------------------------------------------------------------
template <bool SAVES>
__global__ __launch_bounds__(kBlock) void where_select_kernel(const dc_linq_chain prog, const float* __restrict__ in,
                                                              int64_t n, float* __restrict__ out,
                                                              int64_t* __restrict__ count_out,
                                                              uint64_t* __restrict__ status,
                                                              uint32_t* __restrict__ ticket, uint32_t epoch,
                                                              int64_t num_tiles, int vec_ok) {
  __shared__ uint32_t s_tile;
  __shared__ uint32_t s_count[kVecPerThread][kWaves];
  __shared__ uint32_t s_offset[kVecPerThread][kWaves];
  __shared__ uint32_t s_aggregate;
  __shared__ int64_t s_exclusive;
  __shared__ float s_stage[kTile];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  if (tid == 0) {
    // Relaxed: the ticket only orders tile indices; no data is published through it.
    uint32_t t = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_tile = t;
    // Every ticket has been handed out once the last one is taken: reset for the next launch.
    if ((int64_t)t == num_tiles - 1) dc::store_agent_u32(ticket, 0u);
  }
  __syncthreads();
  const int64_t tile = s_tile;
  if (tile >= num_tiles) return;  // cannot happen while the ticket counter starts at zero
  const int64_t base = tile * kTile;

  float e[kElemPerThread];
  uint32_t valid;
  if (vec_ok && base + kTile <= n) {
    const dc::f32x4* in4 = reinterpret_cast<const dc::f32x4*>(in + base);
#pragma unroll
    for (int j = 0; j < kVecPerThread; ++j) {
      dc::f32x4 x = dc::load_stream(in4 + j * kBlock + tid);
      e[4 * j + 0] = x.x;
      e[4 * j + 1] = x.y;
      e[4 * j + 2] = x.z;
      e[4 * j + 3] = x.w;
    }
    valid = 0xFFFFu;
  } else {
    valid = 0;
#pragma unroll
    for (int j = 0; j < kVecPerThread; ++j)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int64_t idx = base + (int64_t)j * (4 * kBlock) + tid * 4 + k;
        const bool ok = idx < n;
        e[4 * j + k] = ok ? in[idx] : 0.0f;
        valid |= (uint32_t)ok << (4 * j + k);
      }
  }

  const uint32_t keep = run_program<kElemPerThread, SAVES>(prog, e) & valid;

  // Rank of this thread's first kept element of vector j inside its (j, wave) group: the kept
  // elements of lower lanes, counted with one ballot + mbcnt per element slot k.
  uint32_t below[kVecPerThread];
#pragma unroll
  for (int j = 0; j < kVecPerThread; ++j) {
    uint32_t bl = 0, total = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint64_t b = __ballot((keep >> (4 * j + k)) & 1u);
      bl += __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
      total += (uint32_t)__builtin_popcountll(b);
    }
    below[j] = bl;
    if (lane == 0) s_count[j][wave] = total;
  }
  __syncthreads();
  if (tid == 0) {
    uint32_t run = 0;
#pragma unroll
    for (int j = 0; j < kVecPerThread; ++j)
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        s_offset[j][w] = run;
        run += s_count[j][w];
      }
    s_aggregate = run;
  }
  __syncthreads();
  const uint32_t aggregate = s_aggregate;

  if (wave == 0) {
    int64_t excl = lookback(status, tile, aggregate, epoch);
    if (lane == 0) s_exclusive = excl;
  }
  // Stage kept elements in output order.
#pragma unroll
  for (int j = 0; j < kVecPerThread; ++j) {
    uint32_t pos = s_offset[j][wave] + below[j];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if ((keep >> (4 * j + k)) & 1u) s_stage[pos++] = e[4 * j + k];
  }
  __syncthreads();
  const int64_t exclusive = s_exclusive;
  float* dst = out + exclusive;
  for (uint32_t i = tid; i < aggregate; i += kBlock) __builtin_nontemporal_store(s_stage[i], dst + i);
  if (tid == 0 && tile == num_tiles - 1) *count_out = exclusive + (int64_t)aggregate;
}

// ---- Where/Select -> Sum / Count ----------------------------------------------------------------
// Pass 1: each block runs the program over one contiguous chunk (a thread takes 4 vectors, 16
// elements, per step) and writes its float64 sum and kept count; pass 2 sums the partials in block
// order (fixed tree, deterministic).
constexpr int kSumBlock = 512;

template <bool SAVES>
__global__ __launch_bounds__(kSumBlock) void where_select_sum_pass1(const dc_linq_chain prog,
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
    const uint32_t keep = run_program<16, SAVES>(prog, e);
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if ((keep >> j) & 1u) acc += (double)e[j];
    cnt += __builtin_popcount(keep);
  }
  for (; i < v1; i += kSumBlock) {
    float e[4];
    dc::f32x4 x = dc::load_stream(in4 + i);
    e[0] = x.x; e[1] = x.y; e[2] = x.z; e[3] = x.w;
    const uint32_t keep = run_program<4, SAVES>(prog, e);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if ((keep >> j) & 1u) acc += (double)e[j];
    cnt += __builtin_popcount(keep);
  }
  if (blockIdx.x == gridDim.x - 1) {
    for (int64_t s = (n4 << 2) + threadIdx.x; s < n; s += kSumBlock) {
      float e[1] = {in[s]};
      if (run_program<1, SAVES>(prog, e) & 1u) {
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

}  // namespace

extern "C" {

DC_HIP_API int32_t dc_linq_chain_validate(const dc_linq_chain* chain) {
  if (!chain) return DC_ERR_INVALID_ARGUMENT;
  if (chain->n_instr < 0 || chain->n_instr > DC_LINQ_MAX_INSTR || chain->flags != 0) return DC_ERR_INVALID_ARGUMENT;
  for (int i = 0; i < chain->n_instr; ++i) {
    const dc_linq_instr& in = chain->code[i];
    const bool op_ok = (in.op <= DC_LQ_STORE_S1) || (in.op >= DC_LQ_CMP_GT && in.op <= DC_LQ_MAP);
    if (!op_ok || in.src > DC_LQ_SRC_S1) return DC_ERR_UNSUPPORTED;
    if (in.op >= DC_LQ_CMP_GT && in.op <= DC_LQ_CMP_NE && in.mode > DC_LQ_CMP_OR) return DC_ERR_UNSUPPORTED;
  }
  return DC_OK;
}

DC_HIP_API int32_t dc_hip_linq_where_select_f32(dc_hip_ctx* ctx, const dc_linq_chain* chain, const float* input,
                                                int64_t n, float* output, int64_t* count_out) {
  if (n < 0 || !count_out || (n > 0 && (!input || !output))) return DC_ERR_INVALID_ARGUMENT;
  DC_RETURN_IF(dc_linq_chain_validate(chain));
  if (n >= (int64_t)1 << 40) return DC_ERR_INVALID_ARGUMENT;  // 40-bit counts in the status words
  DC_CTX_ENTER(ctx);
  const int64_t tiles = std::max<int64_t>(1, (n + kTile - 1) / kTile);
  if (tiles > 0xFFFFFFFFll) return DC_ERR_INVALID_ARGUMENT;
  uint32_t epoch = 0;
  DC_RETURN_IF(dc::ensure_status(ctx, (size_t)tiles, &epoch));
  auto kernel = program_uses_saves(*chain) ? where_select_kernel<true> : where_select_kernel<false>;
  kernel<<<(unsigned)tiles, kBlock, 0, ctx->stream>>>(*chain, input, n, output, count_out, ctx->status,
                                                      ctx->counters + DC_SLOT_LINQ_TICKET, epoch, tiles,
                                                      dc::aligned16(input) ? 1 : 0);
  return dc::last_launch_status();
}

DC_HIP_API int32_t dc_hip_linq_where_select_sum_f32(dc_hip_ctx* ctx, const dc_linq_chain* chain, const float* input,
                                                    int64_t n, double* sum_out, int64_t* count_out) {
  if (n < 0 || (n > 0 && !input)) return DC_ERR_INVALID_ARGUMENT;
  DC_RETURN_IF(dc_linq_chain_validate(chain));
  DC_CTX_ENTER(ctx);
  const int64_t per_block = (int64_t)kSumBlock * 16 * 4;  // elements per block-iteration x 4
  const unsigned grid = (unsigned)std::max<int64_t>(1, std::min<int64_t>((n + per_block - 1) / per_block, kSumBlocksMax));
  DC_RETURN_IF(dc::ensure_partials(ctx, (size_t)grid * 16));
  double* psum = static_cast<double*>(ctx->partials);
  int64_t* pcnt = reinterpret_cast<int64_t*>(psum + grid);
  auto kernel = program_uses_saves(*chain) ? where_select_sum_pass1<true> : where_select_sum_pass1<false>;
  kernel<<<grid, kSumBlock, 0, ctx->stream>>>(*chain, input, n, dc::aligned16(input) ? 1 : 0, psum, pcnt);
  where_select_sum_pass2<<<1, kFinalBlock, 0, ctx->stream>>>(psum, pcnt, (int)grid, sum_out, count_out);
  return dc::last_launch_status();
}

}  // extern "C"

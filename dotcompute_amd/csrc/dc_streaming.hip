// dc_streaming.hip — HBM-bound streaming kernels for gfx950: VectorAdd and the deterministic
// float64-accumulated / int64-exact sum reductions.
//
// Layout: inputs are contiguous 1-D arrays in HBM; every workgroup streams one contiguous chunk
// of 16-byte vectors (global_load_dwordx4), several loads in flight per thread.
// Reductions: per-thread accumulators in a fixed order -> DPP wave tree -> LDS block tree ->
// per-block partial -> a one-block pass sums the partials in block order. Fixed grid size for a
// given n, so the result is bit-reproducible run to run.
#include <algorithm>
#include <type_traits>

#include "dc_device.hpp"
#include "dc_internal.hpp"

namespace {

constexpr int kBlock = 256;

// ---------------------------------------------------------------------------------------------
// VectorAdd: result[i] = a[i] + b[i] (one rounding per element, bit-exact with any IEEE CPU).
// ---------------------------------------------------------------------------------------------
// 16-byte aligned operands: one vector pair per thread over a grid that covers the input
// (1024-thread workgroups), non-temporal loads and stores (the output is written in whole lines
// and not read again here); past HIP's 2^32 work-items per grid the threads stride. Measured at
// 256M (3.2 GB): 490 us (6.57 TB/s), against 499 us with 256-thread workgroups, 530 us with two
// pairs per thread, 535 us with cached loads, 563 us for one contiguous chunk per workgroup
// (four per CU, two pairs in flight) and 531 us for torch.add's kernel on the same machine.
constexpr int kVaBlock = 1024;
constexpr int64_t kVaMaxBlocks = 0xFFFFFFFFll / kVaBlock;
__global__ __launch_bounds__(kVaBlock) void vector_add_f32x4_kernel(const dc::f32x4* __restrict__ a,
                                                                    const dc::f32x4* __restrict__ b,
                                                                    dc::f32x4* __restrict__ r, int64_t n4,
                                                                    const float* __restrict__ a_tail,
                                                                    const float* __restrict__ b_tail,
                                                                    float* __restrict__ r_tail, int tail) {
  const int64_t stride = (int64_t)gridDim.x * kVaBlock;
  for (int64_t i = (int64_t)blockIdx.x * kVaBlock + threadIdx.x; i < n4; i += stride)
    __builtin_nontemporal_store(dc::load_stream(a + i) + dc::load_stream(b + i), r + i);
  if (blockIdx.x == 0 && threadIdx.x < tail) r_tail[threadIdx.x] = a_tail[threadIdx.x] + b_tail[threadIdx.x];
}

__global__ __launch_bounds__(kBlock) void vector_add_f32_kernel(const float* __restrict__ a,
                                                                const float* __restrict__ b,
                                                                float* __restrict__ r, int64_t n) {
  int64_t i = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (; i < n; i += stride) r[i] = a[i] + b[i];
}

// ---------------------------------------------------------------------------------------------
// Sum reductions: pass 1 — each block sums one contiguous chunk of the input (threads stride
// 16-byte vectors through it, kUnroll loads in flight) into a per-block partial; pass 2 — one
// block sums the partials in block order. Large inputs take two launches: a last-block combine
// with agent-scope release/acquire fences in every block (on gfx950 those write back and
// invalidate the XCD's L2) measured 195 us at 256M elements against 155 us for the two launches.
// Inputs up to kOneLaunchMax elements take one launch without fences: each block publishes its
// partial with an agent-scope store (written through its XCD's L2), waits for that store to
// complete, then takes a ticket; the block with the last ticket reads the partials with
// agent-scope loads and combines them in the same order as the second launch, so both
// strategies return the same bits.
// ---------------------------------------------------------------------------------------------
constexpr int kRedBlock = 512;
constexpr int kRedUnroll = 8;
// The f32 Sum keeps fewer loads in flight at scale: 4 vectors per thread (about 8 MB in flight
// over the chip, as much as the plain read streams that run fastest) took 149.8 us at 256M against
// 152.5 us with 8; the i32 kernel, with more work per element, needs its 8 (4: 183 us). The
// one-launch form takes its 8 vectors per thread at once (one memory round trip at 1M elements
// instead of two). A thread's k-th vector goes to accumulator k mod 2 whatever the unroll, so the
// result does not depend on it.
constexpr int kRedUnrollF32 = 4;
constexpr int kFinalBlock = 1024;
// One launch up to 2M elements (at most 128 workgroups; 1M: Sum f32 4.2 against 5.6 us, Sum i32
// 6.3 against 9.1 us). With 256 workgroups (4M elements) the 256 tickets taken one after another
// at one address cost more than the second launch (6.5 against 5.7 us).
constexpr int64_t kOneLaunchMax = (int64_t)1 << 21;  // elements

__device__ inline double add4(double acc, dc::f32x4 v) {
  acc += (double)v.x;
  acc += (double)v.y;
  acc += (double)v.z;
  acc += (double)v.w;
  return acc;
}
__device__ inline int64_t add4(int64_t acc, dc::i32x4 v) {
  return acc + (int64_t)v.x + (int64_t)v.y + (int64_t)v.z + (int64_t)v.w;
}

// Vectors [v0, v1) of this block's chunk of the 16-byte aligned part x[h, h + 4*n4); the scalar
// elements before it (h < 4, when x is not 16-byte aligned) and after it (< 4) go to the last block.
template <typename In4, typename In, typename Acc, int UNROLL>
__device__ inline Acc chunk_partial(const In* __restrict__ x, int64_t n, int h) {
  static_assert(UNROLL % 2 == 0, "vector k of a thread goes to accumulator k mod 2");
  Acc acc0 = 0, acc1 = 0;
  const int64_t n4 = (n - h) >> 2;
  const int64_t per = (n4 + gridDim.x - 1) / gridDim.x;
  const int64_t v0 = min(n4, (int64_t)blockIdx.x * per), v1 = min(n4, v0 + per);
  const In4* x4 = reinterpret_cast<const In4*>(x + h);
  int64_t i = v0 + threadIdx.x;
  for (; i + (UNROLL - 1) * kRedBlock < v1; i += UNROLL * kRedBlock) {
    In4 v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) v[u] = dc::load_stream(x4 + i + u * kRedBlock);
#pragma unroll
    for (int u = 0; u < UNROLL; u += 2) {
      acc0 = add4(acc0, v[u]);
      acc1 = add4(acc1, v[u + 1]);
    }
  }
  for (; i + kRedBlock < v1; i += 2 * kRedBlock) {  // the remaining pairs, then a last odd one
    const In4 a = dc::load_stream(x4 + i), b = dc::load_stream(x4 + i + kRedBlock);
    acc0 = add4(acc0, a);
    acc1 = add4(acc1, b);
  }
  if (i < v1) acc0 = add4(acc0, dc::load_stream(x4 + i));
  if (blockIdx.x == gridDim.x - 1 && threadIdx.x < 8) {
    const int64_t s = threadIdx.x < 4 ? threadIdx.x : h + (n4 << 2) + (threadIdx.x - 4);
    if ((threadIdx.x < 4 && s < h) || (threadIdx.x >= 4 && s < n)) acc1 += (Acc)x[s];
  }
  return acc0 + acc1;
}

__global__ __launch_bounds__(kRedBlock) void reduce_sum_f32_pass1(const float* __restrict__ x, int64_t n, int h,
                                                                  double* __restrict__ partials) {
  __shared__ double lds[kRedBlock / dc::kWave];
  double acc = chunk_partial<dc::f32x4, float, double, kRedUnrollF32>(x, n, h);
  double t = dc::block_sum64<kRedBlock>(acc, lds);
  if (threadIdx.x == 0) partials[blockIdx.x] = t;
}

// Pass 1 and the combine in one launch (gridDim.x <= kRedBlock). The last block's thread t holds
// 0 + partial t as the combine kernel's thread t does; the waves past the partials contribute +0
// there, which leaves its in-order sum of the wave totals unchanged.
__global__ __launch_bounds__(kRedBlock) void reduce_sum_f32_one(const float* __restrict__ x, int64_t n, int h,
                                                                uint64_t* __restrict__ partials,
                                                                uint32_t* __restrict__ done, double* __restrict__ sum_out) {
  __shared__ double lds[kRedBlock / dc::kWave];
  __shared__ uint32_t s_last;
  const double t = dc::block_sum64<kRedBlock>(chunk_partial<dc::f32x4, float, double, 8>(x, n, h), lds);
  if (threadIdx.x == 0) {
    dc::store_agent_u64(partials + blockIdx.x, (uint64_t)__double_as_longlong(t));
    dc::wait_memory_ops();
    s_last = dc::fetch_add_relaxed_agent_u32(done, 1u) == gridDim.x - 1 ? 1u : 0u;
  }
  __syncthreads();
  if (!s_last) return;
  double acc = 0;
  if (threadIdx.x < gridDim.x) acc += __longlong_as_double((long long)dc::load_agent_u64(partials + threadIdx.x));
  const double total = dc::block_sum64<kRedBlock>(acc, lds);
  if (threadIdx.x == 0) {
    *sum_out = total;
    dc::store_agent_u32(done, 0u);
  }
}

// ---------------------------------------------------------------------------------------------
// Checked int32 Sum with the overflow rule of the .NET 10 BCL's Enumerable.Sum(IEnumerable<int>)
// for array/list sources on x64 (System.Linq Sum.cs, SumSignedIntegersVectorized; reached from
// ComputeQueryableExtensions.cs:265-267). With W = Vector<int>.Count = 8 lanes:
//   n < 4W:  one checked running total: OverflowException as soon as a prefix sum leaves int32.
//   n >= 4W: the elements [0, V) are summed in W wrapping lanes (lane c takes the elements whose
//            index is c mod W, in order) and any lane add that overflows throws; then the lane
//            totals are added in lane order with checked adds, then the elements [V, n), checked.
//            V is where the BCL's vector loops stop (at most W elements before n; bcl_vector_end).
// So an OverflowException happens iff (a) a prefix of some lane's subsequence leaves int32, or
// (b) a prefix of (lane 0 total, lane 1 total, ...) leaves int32, or (c) that sum plus a prefix of
// the scalar tail does. The exact int64 total is reported either way.
//
// GPU design: pass 1 (every workgroup, one contiguous chunk of 16-byte vectors) computes per lane
// class c the chunk's class sum T_c (int64) and the chunk's largest and smallest element. Pass 2
// (one workgroup) scans the class sums over the chunks to get each chunk's starting class prefix
// S_c. A chunk holding k elements of class c cannot overflow that class if S_c + k*max(hi, 0) and
// S_c + k*min(lo, 0) both fit (every prefix inside the chunk lies between them). Chunks that fail
// that screen (inputs whose magnitudes reach about 2^31 / k, e.g. |x| >~ 6.5e4 at 256M elements)
// get an exact check: the chunk's elements are re-read and every class prefix inside it is
// bounded by an ordered (sum, max prefix, min prefix) combination. Rules (b) and (c) touch at most
// 8 + 8 values and run on one thread. Before all that, the one-launch form screens the whole
// input with one block reduction: when n * max(largest, 0) and n * min(smallest, 0) fit in int32,
// no prefix of any rule can leave int32 and the exact total is the answer (at 1M elements: every
// magnitude <= 2047).
// ---------------------------------------------------------------------------------------------
constexpr int kBclLanes = 8;  // Vector<int>.Count on x64 (256-bit Vector<T>)

__device__ inline int64_t parity_sum(int64_t v) {
#pragma unroll
  for (int off = 2; off < dc::kWave; off <<= 1) v += __shfl_xor(v, off, dc::kWave);
  return v;
}

// What the one-launch form of the i32 Sum passes to its combine.
struct BclArgs {
  const int32_t* x;
  int64_t n, V;
  int64_t* sum_out;
  int32_t* overflow_out;
  uint32_t* done;
};

__device__ inline bool fits_i32(int64_t v) { return v >= -2147483648LL && v <= 2147483647LL; }

constexpr int kBclFinalBlock = 1024;

// The combine of the class partials of G <= BLOCK chunks, run by one BLOCK-thread workgroup.
// AGENT: the partials were published by other workgroups of the same launch (agent-scope loads),
// the one-launch form for inputs of at most kOneLaunchMax elements, which also runs the
// whole-input screen (past 2M elements it passes only for magnitudes below 1024, and costs the
// two-launch form about 1.5 us when it fails).
template <int BLOCK, bool AGENT>
__device__ void bcl_combine(const int64_t* __restrict__ partials, int G, const int32_t* __restrict__ x, int64_t n,
                            int h, int64_t n4, int64_t V, int64_t per, int64_t* __restrict__ sum_out,
                            int32_t* __restrict__ overflow_out) {
  const int t = threadIdx.x, lane = t & (dc::kWave - 1), wave = t / dc::kWave;
  auto part = [&](size_t i) -> int64_t {
    if constexpr (AGENT) return (int64_t)dc::load_agent_u64(reinterpret_cast<const uint64_t*>(partials) + i);
    else return partials[i];
  };
  // The few scalar elements, loaded once by separate threads (all independent loads in flight):
  // n < 32: all of them; else the unaligned head [0, h), the elements [h + 4*n4, V) after the last
  // whole vector, and the tail [V, n) (at most 8).
  __shared__ int32_t elem[4 * kBclLanes];
  __shared__ int64_t wpre[BLOCK / dc::kWave + 1][kBclLanes];
  __shared__ int64_t lane_total[kBclLanes];
  __shared__ int64_t cur_start[kBclLanes];
  __shared__ int flag_list[BLOCK];
  __shared__ int flag_count, ovf_s;
  __shared__ int64_t tr_s[BLOCK], tr_max[BLOCK], tr_min[BLOCK];
  const int64_t mid0 = h + 4 * n4;
  // The partials first: their loads and the element loads below are then in flight together.
  int64_t T[kBclLanes], incl[kBclLanes];
#pragma unroll
  for (int c = 0; c < kBclLanes; ++c) T[c] = t < G ? part((size_t)c * G + t) : 0;
  // A chunk of nv vectors holds at most (nv + 1) / 2 elements of each class.
  const int64_t k_per_class = t < G ? (min(n4, (int64_t)(t + 1) * per) - min(n4, (int64_t)t * per) + 1) / 2 : 0;
  const int64_t hi_t = t < G ? part((size_t)8 * G + t) : 0, lo_t = t < G ? part((size_t)9 * G + t) : 0;
  const int64_t up = k_per_class * max(hi_t, (int64_t)0);
  const int64_t down = k_per_class * min(lo_t, (int64_t)0);
  int32_t ev = 0;  // this thread's scalar element (threads < 32)
  if (t < 4 * kBclLanes) {
    int64_t idx = -1;
    if (n < 4 * kBclLanes) idx = t < n ? t : -1;
    else if (t < 4) idx = t < h ? t : -1;
    else if (t < 8) idx = mid0 + (t - 4) < V ? mid0 + (t - 4) : -1;
    else if (t < 8 + 2 * kBclLanes) idx = V + (t - 8) < n ? V + (t - 8) : -1;
    ev = idx >= 0 ? x[idx] : 0;
    elem[t] = ev;
  }
  if (AGENT && n >= 4 * kBclLanes) {
    // Screen: every prefix the three rules look at is a sum of at most n input elements, so when
    // n * max(largest, 0) and n * min(smallest, 0) both fit in int32 nothing overflows and the
    // total is the answer (one block reduction instead of the class scans below).
    int64_t s = ev;
    int32_t mx = max(ev, 0), mn = min(ev, 0);
    if (t < G) {
#pragma unroll
      for (int c = 0; c < kBclLanes; ++c) s += T[c];
      mx = max(mx, (int32_t)hi_t);
      mn = min(mn, (int32_t)lo_t);
    }
    s = dc::wave_sum64(s);
#pragma unroll
    for (int off = 1; off < dc::kWave; off <<= 1) {
      mx = max(mx, __shfl_xor(mx, off, dc::kWave));
      mn = min(mn, __shfl_xor(mn, off, dc::kWave));
    }
    if (lane == 0) {
      tr_s[wave] = s;
      tr_max[wave] = mx;
      tr_min[wave] = mn;
    }
    __syncthreads();
    int64_t total = 0, big = 0, small = 0;
    for (int w = 0; w < (max(G, 4 * kBclLanes) + dc::kWave - 1) / dc::kWave; ++w) {  // waves holding values
      total += tr_s[w];
      big = max(big, tr_max[w]);
      small = min(small, tr_min[w]);
    }
    if (fits_i32(n * big) && fits_i32(n * small)) {
      if (t == 0) {
        *sum_out = total;
        if (overflow_out) *overflow_out = 0;
      }
      return;
    }
    __syncthreads();  // tr_* are reused by the exact check
  }
  if (n < 4 * kBclLanes) {  // the BCL's scalar checked loop
    __syncthreads();
    if (t == 0) {
      int64_t s = 0;
      int ovf = 0;
      for (int64_t i = 0; i < n; ++i) {
        s += elem[i];
        if (!fits_i32(s)) ovf = 1;
      }
      *sum_out = s;
      if (overflow_out) *overflow_out = ovf;
    }
    return;
  }

  // Inclusive scan of the class sums over chunks (thread t = chunk t): within each wave, then the
  // wave totals by one thread per class.
#pragma unroll
  for (int c = 0; c < kBclLanes; ++c) incl[c] = dc::wave_inclusive_scan64(T[c]);
  if (lane == dc::kWave - 1)
#pragma unroll
    for (int c = 0; c < kBclLanes; ++c) wpre[wave + 1][c] = incl[c];
  if (t == 0) {
    flag_count = 0;
    ovf_s = 0;
  }
  __syncthreads();
  if (t < kBclLanes) {  // exclusive prefix over the waves, starting from the head element of class t
    int64_t run = t < h ? (int64_t)elem[t] : 0;
    for (int w = 0; w < (G + dc::kWave - 1) / dc::kWave; ++w) {  // later waves hold no chunk
      const int64_t wt = wpre[w + 1][t];
      wpre[w][t] = run;
      run += wt;
    }
    lane_total[t] = run;
  }
  __syncthreads();
  bool flagged = false;
  int64_t start[kBclLanes];
#pragma unroll
  for (int c = 0; c < kBclLanes; ++c) {
    start[c] = wpre[wave][c] + incl[c] - T[c];
    if (t < G && (!fits_i32(start[c] + up) || !fits_i32(start[c] + down))) flagged = true;
  }
  if (flagged) flag_list[atomicAdd(&flag_count, 1)] = t;
  __syncthreads();
  const int nflag = flag_count;
  for (int k = 0; k < nflag; ++k) {
    const int f = flag_list[k];
    if (t == f)
      for (int c = 0; c < kBclLanes; ++c) cur_start[c] = start[c];
    __syncthreads();
    const int64_t e0 = h + 4 * min(n4, (int64_t)f * per), e1 = h + 4 * min(n4, (int64_t)(f + 1) * per);
    const int64_t piece = (e1 - e0 + BLOCK - 1) / BLOCK;
    const int64_t a = min(e1, e0 + t * piece), b = min(e1, a + piece);
    for (int c = 0; c < kBclLanes; ++c) {
      int64_t s = 0, mx = 0, mn = 0;  // relative prefix sum, its max and min (the empty prefix included)
      for (int64_t i = a + ((c - a) & (kBclLanes - 1)); i < b; i += kBclLanes) {
        s += x[i];
        mx = max(mx, s);
        mn = min(mn, s);
      }
      tr_s[t] = s;
      tr_max[t] = mx;
      tr_min[t] = mn;
      __syncthreads();
      for (int stride = 1; stride < BLOCK; stride <<= 1) {
        if ((t & (2 * stride - 1)) == 0) {  // (left = t, right = t + stride), in sequence order
          const int r = t + stride;
          const int64_t ls = tr_s[t];
          tr_max[t] = max(tr_max[t], ls + tr_max[r]);
          tr_min[t] = min(tr_min[t], ls + tr_min[r]);
          tr_s[t] = ls + tr_s[r];
        }
        __syncthreads();
      }
      if (t == 0 && (!fits_i32(cur_start[c] + tr_max[0]) || !fits_i32(cur_start[c] + tr_min[0]))) ovf_s = 1;
      __syncthreads();
    }
    if (ovf_s) break;
  }
  if (t == 0) {
    int ovf = ovf_s;
    // The scalar elements after the last whole vector but before V, then each class's final prefix.
    for (int64_t i = mid0; i < V; ++i) lane_total[i & (kBclLanes - 1)] += elem[4 + (i - mid0)];
    int64_t r = 0;
    for (int c = 0; c < kBclLanes; ++c) {
      if (!fits_i32(lane_total[c])) ovf = 1;
      r += lane_total[c];
      if (!fits_i32(r)) ovf = 1;  // the lane totals are added with checked int32 adds
    }
    for (int64_t i = V; i < n; ++i) {
      r += elem[8 + (i - V)];
      if (!fits_i32(r)) ovf = 1;  // the scalar tail, checked
    }
    *sum_out = r;
    if (overflow_out) *overflow_out = ovf;
  }
}

__global__ __launch_bounds__(kBclFinalBlock) void reduce_sum_i32_bcl_final(
    const int64_t* __restrict__ partials, int G, const int32_t* __restrict__ x, int64_t n, int h, int64_t n4,
    int64_t V, int64_t per, int64_t* __restrict__ sum_out, int32_t* __restrict__ overflow_out) {
  bcl_combine<kBclFinalBlock, false>(partials, G, x, n, h, n4, V, per, sum_out, overflow_out);
}

// xa = x + h is 16-byte aligned; the chunk of workgroup w is vectors [w*per, (w+1)*per) of xa's
// first n4 vectors (per is even, so a thread's vectors all have the parity of its lane).
// partials: [c*G + w] class sums (c = lane class 0..7), [8*G + w] the chunk's largest element,
// [9*G + w] its smallest.
// ONE: the one-launch form (gridDim.x <= kRedBlock), whose last block to finish runs the combine.
template <bool ONE>
__global__ __launch_bounds__(kRedBlock) void reduce_sum_i32_classes(const int32_t* __restrict__ xa, int64_t n4,
                                                                    int64_t per, int h, int64_t* __restrict__ partials,
                                                                    BclArgs fin) {
  // Class sums are accumulated with a bias of 2^31 per element (x ^ 0x80000000 is x + 2^31 as an
  // unsigned value): one 64-bit add of a zero-extended word, no sign extension; the bias is taken
  // off at the end from the number of vectors the thread read.
  uint64_t acc[4] = {0, 0, 0, 0};
  int32_t hi = INT32_MIN, lo = INT32_MAX;
  const int64_t v0 = min(n4, (int64_t)blockIdx.x * per), v1 = min(n4, v0 + per);
  const dc::i32x4* x4 = reinterpret_cast<const dc::i32x4*>(xa);
  auto accumulate = [&](dc::i32x4 v) {
    acc[0] += (uint32_t)v.x ^ 0x80000000u;
    acc[1] += (uint32_t)v.y ^ 0x80000000u;
    acc[2] += (uint32_t)v.z ^ 0x80000000u;
    acc[3] += (uint32_t)v.w ^ 0x80000000u;
    hi = max(hi, max(v.x, v.y));
    hi = max(hi, max(v.z, v.w));
    lo = min(lo, min(v.x, v.y));
    lo = min(lo, min(v.z, v.w));
  };
  int64_t i = v0 + threadIdx.x;
  for (; i + (kRedUnroll - 1) * kRedBlock < v1; i += kRedUnroll * kRedBlock) {
    dc::i32x4 v[kRedUnroll];
#pragma unroll
    for (int u = 0; u < kRedUnroll; ++u) v[u] = dc::load_stream(x4 + i + u * kRedBlock);
#pragma unroll
    for (int u = 0; u < kRedUnroll; ++u) accumulate(v[u]);
  }
  for (; i < v1; i += kRedBlock) accumulate(dc::load_stream(x4 + i));
  const int64_t mine = v1 > v0 + threadIdx.x ? (v1 - v0 - threadIdx.x + kRedBlock - 1) / kRedBlock : 0;
  int64_t cs[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) cs[j] = parity_sum((int64_t)(acc[j] - ((uint64_t)mine << 31)));
  __shared__ int64_t lds[kRedBlock / dc::kWave][2][4];
  __shared__ int32_t lds_hi[kRedBlock / dc::kWave], lds_lo[kRedBlock / dc::kWave];
  const int lane = threadIdx.x & (dc::kWave - 1), wave = threadIdx.x / dc::kWave;
#pragma unroll
  for (int off = 1; off < dc::kWave; off <<= 1) {
    hi = max(hi, __shfl_xor(hi, off, dc::kWave));
    lo = min(lo, __shfl_xor(lo, off, dc::kWave));
  }
  if (lane < 2)
#pragma unroll
    for (int j = 0; j < 4; ++j) lds[wave][lane][j] = cs[j];
  if (lane == 0) {
    lds_hi[wave] = hi;
    lds_lo[wave] = lo;
  }
  __syncthreads();
  const unsigned G = gridDim.x;
  auto publish = [](int64_t* at, int64_t v) {
    if constexpr (ONE) dc::store_agent_u64(reinterpret_cast<uint64_t*>(at), (uint64_t)v);
    else *at = v;
  };
  if (threadIdx.x < 8) {
    const int p = threadIdx.x >> 2, j = threadIdx.x & 3;
    int64_t t = 0;
#pragma unroll
    for (int w = 0; w < kRedBlock / dc::kWave; ++w) t += lds[w][p][j];
    // element h + 4*v + j has lane class (h + 4*(v & 1) + j) mod 8, and v & 1 == lane & 1 == p
    publish(partials + (size_t)((h + 4 * p + j) & (kBclLanes - 1)) * G + blockIdx.x, t);
  } else if (threadIdx.x == 8 || threadIdx.x == 9) {
    int32_t m = threadIdx.x == 8 ? INT32_MIN : INT32_MAX;
    for (int w = 0; w < kRedBlock / dc::kWave; ++w) m = threadIdx.x == 8 ? max(m, lds_hi[w]) : min(m, lds_lo[w]);
    publish(partials + (size_t)threadIdx.x * G + blockIdx.x, m);
  }
  if constexpr (ONE) {  // partials published as in reduce_sum_f32_one
    __shared__ uint32_t s_last;
    dc::wait_memory_ops();
    __syncthreads();
    if (threadIdx.x == 0) s_last = dc::fetch_add_relaxed_agent_u32(fin.done, 1u) == G - 1 ? 1u : 0u;
    __syncthreads();
    if (s_last) {
      bcl_combine<kRedBlock, true>(partials, (int)G, fin.x, fin.n, h, n4, fin.V, per, fin.sum_out, fin.overflow_out);
      if (threadIdx.x == 0) dc::store_agent_u32(fin.done, 0u);
    }
  }
}

// Sums partials[0..count) in a fixed order: thread t takes t, t+1024, ... then the block tree.
template <typename Acc>
__global__ __launch_bounds__(kFinalBlock) void reduce_partials(const Acc* __restrict__ partials, int count,
                                                               Acc* __restrict__ out) {
  __shared__ Acc lds[kFinalBlock / dc::kWave];
  Acc acc = 0;
  // Thread t adds partials t, t + 1024, t + 2048, ... in that order; eight loads go out together.
  for (int i0 = threadIdx.x; i0 < count; i0 += 8 * kFinalBlock) {
    Acc v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = i0 + k * kFinalBlock < count ? partials[i0 + k * kFinalBlock] : Acc(0);
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (i0 + k * kFinalBlock < count) acc += v[k];
  }
  Acc total = dc::block_sum64<kFinalBlock>(acc, lds);
  if (threadIdx.x == 0) *out = total;
}

// Grid for a reduction over n elements: a fixed function of n and of the device's CU count, so
// results are reproducible run to run on one device (and on devices with the same CU count); the
// partial order, and with it the last bits of a float64 sum, can differ between CU counts.
unsigned reduce_grid(const dc_hip_ctx* ctx, int64_t n) {
  const int64_t per_block = (int64_t)kRedBlock * 4 * kRedUnroll;  // elements per block-iteration
  const int64_t g = (n + per_block - 1) / per_block;
  // One workgroup per CU, each streaming one contiguous chunk: measured faster than 2-4 per CU
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>(g, std::max(ctx->cu_count, 1)));
}

// Elements before the first 16-byte boundary of x (0..3), capped at n.
template <typename T>
int head_to_aligned(const T* x, int64_t n) {
  const int h = (int)(((16 - (reinterpret_cast<uintptr_t>(x) & 15)) & 15) / sizeof(T));
  return (int)std::min<int64_t>(h, n);
}

// Where the BCL's vector loops in SumSignedIntegersVectorized stop for n >= 4W elements: a
// do-while over blocks of 4W while index < n - 4W, then (if index < n - W) a do-while over blocks
// of W while index < n - W. Closed form of those two loops.
int64_t bcl_vector_end(int64_t n) {
  const int64_t W = kBclLanes;
  const int64_t lim1 = n - 4 * W;
  int64_t index = 4 * W * std::max<int64_t>(1, (lim1 + 4 * W - 1) / (4 * W));
  const int64_t lim2 = n - W;
  if (index < lim2) index += W * ((lim2 - index + W - 1) / W);
  return index;
}

}  // namespace

namespace dc {

int32_t launch_reduce_sum_f32(dc_hip_ctx* ctx, const float* input, int64_t n, double* sum_out) {
  unsigned grid = reduce_grid(ctx, n);
  DC_RETURN_IF(dc::ensure_partials(ctx, grid * sizeof(double)));
  double* partials = static_cast<double*>(ctx->partials);
  const int h = head_to_aligned(input, n);
  if (n <= kOneLaunchMax && grid <= (unsigned)kRedBlock) {
    reduce_sum_f32_one<<<grid, kRedBlock, 0, ctx->stream>>>(input, n, h, reinterpret_cast<uint64_t*>(partials),
                                                           ctx->counters + DC_SLOT_REDUCE_DONE, sum_out);
    return dc::last_launch_status();
  }
  reduce_sum_f32_pass1<<<grid, kRedBlock, 0, ctx->stream>>>(input, n, h, partials);
  reduce_partials<double><<<1, kFinalBlock, 0, ctx->stream>>>(partials, (int)grid, sum_out);
  return dc::last_launch_status();
}

int32_t launch_reduce_partials_f64(dc_hip_ctx* ctx, const double* partials, int count, double* sum_out) {
  reduce_partials<double><<<1, kFinalBlock, 0, ctx->stream>>>(partials, count, sum_out);
  return dc::last_launch_status();
}

}  // namespace dc

extern "C" {

DC_HIP_API int32_t dc_hip_vector_add_f32(dc_hip_ctx* ctx, const float* a, const float* b, float* result, int64_t n) {
  if (n < 0 || (n > 0 && (!a || !b || !result))) return DC_ERR_INVALID_ARGUMENT;
  DC_CTX_ENTER(ctx);
  if (n == 0) return DC_OK;
  if (dc::aligned16(a) && dc::aligned16(b) && dc::aligned16(result)) {
    int64_t n4 = n >> 2;
    int tail = (int)(n & 3);
    const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>((n4 + kVaBlock - 1) / kVaBlock, kVaMaxBlocks));
    vector_add_f32x4_kernel<<<(unsigned)blocks, kVaBlock, 0, ctx->stream>>>(
        reinterpret_cast<const dc::f32x4*>(a), reinterpret_cast<const dc::f32x4*>(b),
        reinterpret_cast<dc::f32x4*>(result), n4, a + (n4 << 2), b + (n4 << 2), result + (n4 << 2), tail);
  } else {
    int64_t blocks = std::max<int64_t>(1, std::min<int64_t>((n + kBlock - 1) / kBlock, 8192));
    vector_add_f32_kernel<<<(unsigned)blocks, kBlock, 0, ctx->stream>>>(a, b, result, n);
  }
  return dc::last_launch_status();
}

DC_HIP_API int32_t dc_hip_reduce_sum_f32(dc_hip_ctx* ctx, const float* input, int64_t n, double* sum_out) {
  if (n < 0 || !sum_out || (n > 0 && !input)) return DC_ERR_INVALID_ARGUMENT;
  DC_CTX_ENTER(ctx);
  return dc::launch_reduce_sum_f32(ctx, input, n, sum_out);
}

DC_HIP_API int32_t dc_hip_reduce_sum_i32(dc_hip_ctx* ctx, const int32_t* input, int64_t n, int64_t* sum_out,
                                         int32_t* overflow_out) {
  if (n < 0 || !sum_out || (n > 0 && !input)) return DC_ERR_INVALID_ARGUMENT;
  if (n >= ((int64_t)1 << 32)) return DC_ERR_INVALID_ARGUMENT;  // int64 totals stay exact below 2^32 elements
  if ((reinterpret_cast<uintptr_t>(input) & 3) != 0) return DC_ERR_MISALIGNED;
  DC_CTX_ENTER(ctx);
  const unsigned grid = reduce_grid(ctx, n);
  DC_RETURN_IF(dc::ensure_partials(ctx, (size_t)grid * (kBclLanes + 2) * sizeof(int64_t)));
  int64_t* partials = static_cast<int64_t*>(ctx->partials);
  const int64_t V = n >= 4 * kBclLanes ? bcl_vector_end(n) : 0;
  const int h = head_to_aligned(input, V);
  const int64_t n4 = (V - h) >> 2;
  const int64_t per = (((n4 + grid - 1) / grid) + 1) & ~(int64_t)1;  // even: a lane's vectors share one parity
  if (n <= kOneLaunchMax && grid <= (unsigned)kRedBlock) {
    const BclArgs fin{input, n, V, sum_out, overflow_out, ctx->counters + DC_SLOT_REDUCE_DONE};
    reduce_sum_i32_classes<true><<<grid, kRedBlock, 0, ctx->stream>>>(input + h, n4, per, h, partials, fin);
    return dc::last_launch_status();
  }
  reduce_sum_i32_classes<false><<<grid, kRedBlock, 0, ctx->stream>>>(input + h, n4, per, h, partials, BclArgs{});
  reduce_sum_i32_bcl_final<<<1, kBclFinalBlock, 0, ctx->stream>>>(partials, (int)grid, input, n, h, n4, V, per,
                                                                  sum_out, overflow_out);
  return dc::last_launch_status();
}

}  // extern "C"

// dc_spmv.hip — CSR SpMV y = A·x (float32) for gfx950, and the normalised power iteration the
// SpMV benchmark runs (y = A·x; x = y / Σy, 20 times).
//
// Out-degrees follow a Zipf law: most rows hold 1-8 nonzeros, a thin tail holds up to 4096. A
// thread or a small lane group per row would leave most lanes idle and turn every row into a
// chain of dependent, uncoalesced loads, so the work is split by NONZEROS instead:
//   windows: the nonzero array is cut into windows of kWindow entries. Workgroup k owns the rows
//     whose first nonzero lies in window k (row_start[k] = lower_bound(row_pointers, k·kWindow),
//     found once by an analysis pass). It streams the products values[i]·x[col[i]] of those rows
//     into LDS with fully coalesced value/column loads (x is a gather, served mostly by L2 / the
//     256 MB MALL), then one thread per row adds its products in index order — the same order as
//     SparseOps.SpMV (SparseMatrix.cs:669-692), so short rows are bit-identical to the reference.
//   long rows (more than kLongRow nonzeros): listed by a classification pass and handled one
//     workgroup per row with a fixed-order block reduction (deterministic, not sequential order).
// A window's product span is at most kWindow + kLongRow entries (only its last row can run past
// the window, and it is short or excluded), which sizes the LDS buffer.
#include <algorithm>
#include <new>

#include "dc_device.hpp"
#include "dc_internal.hpp"

namespace {

constexpr int kBlock = 256;
constexpr int kWindow = 1024;   // nonzeros per window
constexpr int kLongRow = 512;   // rows longer than this go to the long-row pass
constexpr int kLongBlock = 256;

// row_start[k] = first row whose first nonzero index is >= k·kWindow, for k in [0, windows);
// row_start[windows] = rows.
__global__ __launch_bounds__(kBlock) void spmv_window_starts(const int32_t* __restrict__ rp, int64_t rows,
                                                             int32_t windows, int32_t* __restrict__ row_start) {
  const int64_t k = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  if (k > windows) return;
  if (k == windows) {
    row_start[k] = (int32_t)rows;
    return;
  }
  const int64_t target = k * (int64_t)kWindow;
  int64_t lo = 0, hi = rows;  // search rp[0..rows]
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if ((int64_t)rp[mid] < target) lo = mid + 1; else hi = mid;
  }
  row_start[k] = (int32_t)lo;
}

// Appends every row longer than kLongRow to `list`. One atomic per wave (ballot + mbcnt give each
// long row its slot), so the counter is not hammered once per long row.
__global__ __launch_bounds__(kBlock) void spmv_classify(const int32_t* __restrict__ rp, int64_t rows,
                                                        int32_t* __restrict__ list, uint32_t* __restrict__ count) {
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  const int lane = threadIdx.x & 63;
  // Every lane of a wave runs the same number of iterations (the bound is rounded up to whole
  // strides), so the ballot and the broadcast below always see the full wave.
  const int64_t iters = (rows + stride - 1) / stride;
  for (int64_t it = 0; it < iters; ++it) {
    const int64_t r = it * stride + blockIdx.x * (int64_t)kBlock + threadIdx.x;
    const bool is_long = r < rows && (rp[r + 1] - rp[r] > kLongRow);
    const uint64_t m = __ballot(is_long);
    if (m == 0) continue;
    uint32_t base = 0;
    if (lane == 0)
      base = __hip_atomic_fetch_add(count, (uint32_t)__builtin_popcountll(m), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    base = (uint32_t)__builtin_amdgcn_readfirstlane((int)base);
    if (is_long)
      list[base + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u))] = (int32_t)r;
  }
}

__global__ __launch_bounds__(kBlock) void spmv_windows_kernel(const int32_t* __restrict__ rp, const int32_t* __restrict__ col,
                                                              const float* __restrict__ val, const float* __restrict__ x,
                                                              float* __restrict__ y,
                                                              const int32_t* __restrict__ row_start) {
  __shared__ float s_prod[kWindow + kLongRow];
  const int32_t r0 = row_start[blockIdx.x], r1 = row_start[blockIdx.x + 1];
  if (r0 >= r1) return;  // uniform across the workgroup: no row starts in this window
  const int32_t b = rp[r0];
  const int32_t last_begin = rp[r1 - 1], last_end = rp[r1];
  // The last row may run past the window; if it is long it belongs to the long-row pass.
  int32_t e = (last_end - last_begin > kLongRow) ? last_begin : last_end;
  e = min(e, b + kWindow + kLongRow);  // a well-formed CSR never needs this clamp; it keeps LDS in bounds
  // All column/value loads of this thread's slots go out first, then all x gathers, so a window
  // costs two memory round trips instead of two per slot. Values and columns are streamed once
  // (non-temporal); x is what the caches are for.
  constexpr int kSlots = (kWindow + kLongRow) / kBlock;
  int32_t c[kSlots];
  float v[kSlots];
#pragma unroll
  for (int k = 0; k < kSlots; ++k) {
    const int32_t i = b + (int32_t)threadIdx.x + k * kBlock;
    c[k] = 0;
    v[k] = 0.0f;
    if (i < e) {
      c[k] = __builtin_nontemporal_load(col + i);
      v[k] = __builtin_nontemporal_load(val + i);
    }
  }
  float xv[kSlots];  // every gather in flight before the first product is stored (c = 0 past e)
#pragma unroll
  for (int k = 0; k < kSlots; ++k) xv[k] = x[c[k]];
#pragma unroll
  for (int k = 0; k < kSlots; ++k) {
    const int32_t i = b + (int32_t)threadIdx.x + k * kBlock;
    if (i < e) s_prod[i - b] = v[k] * xv[k];
  }
  __syncthreads();
  for (int32_t r = r0 + (int32_t)threadIdx.x; r < r1; r += kBlock) {
    const int32_t rb = rp[r], re = rp[r + 1];
    if (re - rb > kLongRow) continue;
    float sum = 0.0f;
    const int32_t i0 = max(rb - b, 0), i1 = min(re - b, e - b);
    for (int32_t i = i0; i < i1; ++i) sum += s_prod[i];
    __builtin_nontemporal_store(sum, y + r);
  }
}

__global__ __launch_bounds__(kLongBlock) void spmv_long_rows(const int32_t* __restrict__ rp, const int32_t* __restrict__ col,
                                                             const float* __restrict__ val, const float* __restrict__ x,
                                                             float* __restrict__ y, const int32_t* __restrict__ list,
                                                             const uint32_t* __restrict__ count) {
  __shared__ float lds[kLongBlock / dc::kWave];
  const uint32_t n_long = *count;
  for (uint32_t t = blockIdx.x; t < n_long; t += gridDim.x) {
    const int32_t row = list[t];
    const int32_t b = rp[row], e = rp[row + 1];
    float sum = 0.0f;
    // Four slots per pass: their loads and gathers are independent and overlap.
    for (int32_t i0 = b + (int32_t)threadIdx.x; i0 < e; i0 += 4 * kLongBlock) {
      int32_t c[4];
      float v[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int32_t i = i0 + k * kLongBlock;
        c[k] = 0;
        v[k] = 0.0f;
        if (i < e) {
          c[k] = __builtin_nontemporal_load(col + i);
          v[k] = __builtin_nontemporal_load(val + i);
        }
      }
      float xv[4], p[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) xv[k] = x[c[k]];  // c = 0 past e: gathered, then dropped below
#pragma unroll
      for (int k = 0; k < 4; ++k) p[k] = (i0 + k * kLongBlock < e) ? v[k] * xv[k] : 0.0f;
      sum += (p[0] + p[1]) + (p[2] + p[3]);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = sum;
    __syncthreads();
    if (threadIdx.x == 0) {
      float total = lds[0];
#pragma unroll
      for (int w = 1; w < kLongBlock / dc::kWave; ++w) total += lds[w];
      y[row] = total;
    }
    __syncthreads();
  }
}

// x[i] = (float)(y[i] / s), s = *sum (float64 division, one rounding to float).
__global__ __launch_bounds__(kBlock) void normalise_kernel(const float* y, float* x, int64_t n,
                                                           const double* __restrict__ sum) {
  const double s = *sum;
  int64_t i = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (; i < n; i += stride) x[i] = (float)((double)y[i] / s);
}

struct SpmvPlan {
  int32_t windows;
  size_t list_cap;
};

SpmvPlan make_plan(int64_t nnz) {
  SpmvPlan p;
  p.windows = (int32_t)(nnz / kWindow + 1);  // every first-nonzero index in [0, nnz] has a window
  p.list_cap = (size_t)(nnz / (kLongRow + 1) + 1);
  return p;
}

// Analysis: window starts and the long-row list (once per matrix in the power iteration).
int32_t launch_analysis(dc_hip_ctx* ctx, const SpmvPlan& plan, const int32_t* rp, int64_t rows) {
  DC_RETURN_IF(dc::ensure_spmv_rows(ctx, plan.list_cap));
  DC_RETURN_IF(dc::ensure_spmv_windows(ctx, (size_t)plan.windows + 1));
  uint32_t* count = ctx->counters + DC_SLOT_SPMV_LONG;
  DC_RETURN_IF(dc::zero_async(ctx, count, sizeof(uint32_t)));
  const unsigned wgrid = (unsigned)((plan.windows + 1 + kBlock - 1) / kBlock);
  spmv_window_starts<<<wgrid, kBlock, 0, ctx->stream>>>(rp, rows, plan.windows, ctx->spmv_windows);
  DC_RETURN_IF(dc::last_launch_status());
  const unsigned grid = (unsigned)std::max<int64_t>(1, std::min<int64_t>((rows + kBlock - 1) / kBlock, 16384));
  spmv_classify<<<grid, kBlock, 0, ctx->stream>>>(rp, rows, ctx->spmv_rows, count);
  return dc::last_launch_status();
}

int32_t launch_spmv(dc_hip_ctx* ctx, const SpmvPlan& plan, const int32_t* rp, const int32_t* col, const float* val,
                    const float* x, float* y) {
  spmv_windows_kernel<<<(unsigned)plan.windows, kBlock, 0, ctx->stream>>>(rp, col, val, x, y, ctx->spmv_windows);
  DC_RETURN_IF(dc::last_launch_status());
  const unsigned lgrid = (unsigned)std::max<size_t>(1, std::min<size_t>(plan.list_cap, 2048));
  spmv_long_rows<<<lgrid, kLongBlock, 0, ctx->stream>>>(rp, col, val, x, y, ctx->spmv_rows,
                                                        ctx->counters + DC_SLOT_SPMV_LONG);
  return dc::last_launch_status();
}

int32_t check_csr(const int32_t* rp, const int32_t* col, const float* val, int64_t rows, int64_t nnz) {
  if (rows < 0 || nnz < 0 || nnz > INT32_MAX - 2 * kWindow || rows >= INT32_MAX) return DC_ERR_INVALID_ARGUMENT;
  if (!rp || (nnz > 0 && (!col || !val))) return DC_ERR_INVALID_ARGUMENT;
  return DC_OK;
}

// =============================================================================================
// Column-sliced plan for repeated SpMV (the power iteration; any CsrMatrix multiplied many times).
//
// Random 4-byte gathers from a vector far larger than one XCD's 4 MB L2 miss in L2 and are served
// by the memory-side cache at ~60 G gathers/s on MI355X; gathers confined to a 4 MB range per XCD
// hit in L2 and run ~4x faster (measured with a standalone probe). The plan therefore cuts the
// columns into S slices of at most kSliceCols columns (4 MB of x) and rebuilds the matrix slice by
// slice: slice s holds the nonzeros of every row whose column falls in s, in row order, as
// "segments" (one segment per nonempty (row, slice) pair). Workgroup w runs on XCD w % 8 (the
// dispatcher's round-robin; correctness never depends on it), and XCD j only processes windows of
// the slices s with s % 8 == j (S >= 8), or its share of slice j % S (S < 8), so each XCD gathers
// from one 4 MB range at a time.
//   gather pass: one wave per window of kWW nonzeros; products into the wave's LDS, then one lane
//     per segment adds them in index order -> partial[segment].
//   combine pass: one thread per row adds its segments' partials in slice order (0.0f + p0 + p1
//     ...). With S == 1 every row is one segment and the result equals the sequential row sum.
// Segments longer than kLongSeg go to a workgroup-per-segment pass (fixed-order tree).
// The analysis (count, scan, scatter, window descriptors) runs on the device, once per plan.
// =============================================================================================
constexpr int kRB = 256;                  // rows per analysis / combine workgroup (a thread per row)
constexpr int kMaxSlices = 32;
constexpr int64_t kSliceCols = 1 << 20;   // columns per slice: 4 MB of x, one XCD's L2
constexpr int kWW = 512;                  // nonzeros per wave window
constexpr int kLongSeg = 256;             // longer segments go to the long-segment pass
constexpr int kSeqSeg = 32;               // longer segments are summed by the whole wave
constexpr int kSpan = kWW + kLongSeg;     // products a window can hold (its segments end before this)
constexpr int kXcds = 8;
constexpr int kGatherBlock = 256;         // 4 waves, each with its own windows
constexpr int kXcdWords = 8;              // per (phase, XCD): nranges, total, (start, count, stride)
constexpr int kMaxPhases = kMaxSlices / 8;
constexpr int kScanBlock = 1024;

__device__ inline uint32_t lane_rank(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

__device__ inline void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ inline int32_t wave_incl_scan(int32_t v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int32_t u = __shfl_up(v, off, 64);
    if (lane >= off) v += u;
  }
  return v;
}

// Column -> slice. Columns outside [0, cols) are clamped into range, so a malformed matrix can never
// index outside x or the slice tables (the managed CsrMatrix rejects such columns before this).
__device__ inline uint32_t clamp_col(int32_t c, uint32_t cols) { return (uint32_t)c < cols ? (uint32_t)c : cols - 1; }

// The nonzeros of 64 consecutive rows are contiguous in CSR order, so a wave streams them in
// coalesced chunks of 64. Lane l holds the first nonzero of row rw0 + l (clamped into the wave's
// range); the row of element i is the last lane whose start is <= i.
struct WaveRows {
  int32_t start;     // this lane's row start (nz1 for lanes past the last row)
  int32_t nz0, nz1;  // nonzero range of the wave's rows, clamped to [0, nnz]
};

__device__ inline WaveRows wave_rows(const int32_t* __restrict__ rp, int64_t rw0, int64_t rows, int32_t nnz) {
  const int lane = threadIdx.x & 63;
  const int64_t rw1 = min(rw0 + 64, rows);
  WaveRows w;
  w.nz0 = min(max(rp[rw0], 0), nnz);
  w.nz1 = min(max(rp[rw1], w.nz0), nnz);
  const int64_t r = rw0 + lane;
  w.start = r < rw1 ? min(max(rp[r], w.nz0), w.nz1) : w.nz1;
  return w;
}

// Lane (0..63) of the row holding element i: six shuffles over the lanes' row starts.
__device__ inline int wave_row_of(int32_t start, int32_t i) {
  int l = 0;
#pragma unroll
  for (int step = 32; step > 0; step >>= 1)
    if (__shfl(start, l + step, 64) <= i) l += step;
  return l;
}

// Counts the wave's rows into cnt[row][slice] (LDS adds without return). kChunks chunks of column
// loads go out together, so a wave waits one memory round trip per kChunks * 64 nonzeros.
constexpr int kChunks = 4;
template <int SMAX>
__device__ inline void wave_count(const int32_t* __restrict__ col, const WaveRows& w, uint32_t cols, uint32_t width,
                                  int32_t (*cnt)[SMAX + 1]) {
  const int lane = threadIdx.x & 63;
  for (int32_t base = w.nz0; base < w.nz1; base += 64 * kChunks) {
    int32_t c[kChunks];
#pragma unroll
    for (int u = 0; u < kChunks; ++u) c[u] = col[min(base + 64 * u + lane, w.nz1 - 1)];  // base < nz1
#pragma unroll
    for (int u = 0; u < kChunks; ++u) {
      const int32_t i = base + 64 * u + lane;
      const int l = wave_row_of(w.start, i);
      if (i < w.nz1) atomicAdd(&cnt[l][clamp_col(c[u], cols) / width], 1);
    }
  }
}

// Row blocks are handed to workgroups XCD by XCD: workgroup w (on XCD w % 8) takes block
// (w % 8) * per + w / 8, so each XCD works through one contiguous range of rows and the
// slice-major lines it writes are not shared with another XCD's L2. -1: no block for w.
__device__ inline int32_t xcd_block(int32_t nblocks) {
  const int32_t per = (nblocks + kXcds - 1) / kXcds;
  const int32_t b = (int32_t)(blockIdx.x % kXcds) * per + (int32_t)(blockIdx.x / kXcds);
  return b < nblocks ? b : -1;
}

// P1: per (slice, block of kRB rows), the number of nonzeros and of segments. SMAX >= S sizes the
// LDS table.
template <int SMAX>
__global__ __launch_bounds__(kRB) void plan_count(const int32_t* __restrict__ rp, const int32_t* __restrict__ col,
                                                  int64_t rows, int32_t nnz, int32_t S, uint32_t width, uint32_t cols,
                                                  int32_t* __restrict__ tn, int32_t* __restrict__ ts, int32_t ld,
                                                  int32_t nblocks) {
  __shared__ int32_t cnt[kRB][SMAX + 1];
  const int32_t blk = xcd_block(nblocks);
  if (blk < 0) return;  // whole workgroup
  const int t = threadIdx.x, wave = t >> 6;
  for (int s = 0; s < S; ++s) cnt[t][s] = 0;
  __syncthreads();
  const int64_t rw0 = (int64_t)blk * kRB + wave * 64;
  if (rw0 < rows) wave_count<SMAX>(col, wave_rows(rp, rw0, rows, nnz), cols, width, cnt + wave * 64);
  __syncthreads();
  // Column sums over the block's rows: thread t -> slice t / 8, rows (t % 8) * 32 .. + 31.
  const int s = t >> 3, part = t & 7;
  int32_t n = 0, g = 0;
  if (s < S) {
    for (int k = 0; k < 32; ++k) {
      const int32_t c = cnt[part * 32 + k][s];
      n += c;
      g += c > 0 ? 1 : 0;
    }
  }
#pragma unroll
  for (int off = 1; off < 8; off <<= 1) {
    n += __shfl_xor(n, off, 64);
    g += __shfl_xor(g, off, 64);
  }
  if (s < S && part == 0) {
    tn[(int64_t)s * ld + blk] = n;
    ts[(int64_t)s * ld + blk] = g;
  }
}

// P2: workgroup s turns row s of tn and ts (entries 0..nblocks-1, leading dimension ld) into
// exclusive prefix sums, with the slice total at entry nblocks; tot[s] / tot[S + s] = totals.
__global__ __launch_bounds__(kScanBlock) void plan_scan(int32_t* __restrict__ tn, int32_t* __restrict__ ts,
                                                        int32_t nblocks, int32_t ld, int32_t S,
                                                        int32_t* __restrict__ tot) {
  __shared__ int32_t wsum[2][kScanBlock / 64];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  int32_t* rn = tn + (int64_t)blockIdx.x * ld;
  int32_t* rs = ts + (int64_t)blockIdx.x * ld;
  int32_t carry_n = 0, carry_g = 0;
  for (int32_t base = 0; base < nblocks; base += 4 * kScanBlock) {
    int32_t vn[4], vg[4];
    int32_t sn = 0, sg = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int32_t i = base + 4 * t + k;
      vn[k] = i < nblocks ? rn[i] : 0;
      vg[k] = i < nblocks ? rs[i] : 0;
      sn += vn[k];
      sg += vg[k];
    }
    const int32_t in = wave_incl_scan(sn), ig = wave_incl_scan(sg);
    if (lane == 63) {
      wsum[0][wave] = in;
      wsum[1][wave] = ig;
    }
    __syncthreads();
    int32_t pn = carry_n, pg = carry_g, totn = 0, totg = 0;
    for (int w = 0; w < kScanBlock / 64; ++w) {
      if (w < wave) {
        pn += wsum[0][w];
        pg += wsum[1][w];
      }
      totn += wsum[0][w];
      totg += wsum[1][w];
    }
    pn += in - sn;
    pg += ig - sg;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int32_t i = base + 4 * t + k;
      if (i < nblocks) {
        rn[i] = pn;
        rs[i] = pg;
      }
      pn += vn[k];
      pg += vg[k];
    }
    carry_n += totn;
    carry_g += totg;
    __syncthreads();
  }
  if (t == 0) {
    rn[nblocks] = carry_n;
    rs[nblocks] = carry_g;
    tot[blockIdx.x] = carry_n;
    tot[S + blockIdx.x] = carry_g;
  }
}

// P3 (one thread): slice bases (nb = nonzero offsets, sb = segment offsets), the segment sentinel,
// the per-(phase, XCD) window ranges, and the long-segment counters.
__global__ void plan_bases(const int32_t* __restrict__ tot, int32_t S, int32_t* __restrict__ nb,
                           int32_t* __restrict__ sb, int32_t* __restrict__ seg_ptr, int32_t* __restrict__ xcd,
                           uint32_t* __restrict__ long_cnt) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  nb[0] = 0;
  sb[0] = 0;
  for (int s = 0; s < S; ++s) {
    nb[s + 1] = nb[s] + tot[s];
    sb[s + 1] = sb[s] + tot[S + s];
  }
  seg_ptr[sb[S]] = nb[S];
  // Phase p (one gather launch each) gives XCD j one window range: slice j + 8 p when S >= 8, so
  // an XCD never has two slices live in its L2; with S < 8 a single phase, XCD j taking every
  // (8 / S)-th window of slice j % S.
  const int phases = S >= kXcds ? S / kXcds : 1;
  for (int ph = 0; ph < phases; ++ph) {
    for (int j = 0; j < kXcds; ++j) {
      int32_t* xr = xcd + (ph * kXcds + j) * kXcdWords;
      const int s = S >= kXcds ? j + kXcds * ph : j % S;
      const int member = S >= kXcds ? 0 : j / S, members = S >= kXcds ? 1 : kXcds / S;
      const int32_t w0 = (nb[s] + kWW - 1) / kWW, w1 = (nb[s + 1] + kWW - 1) / kWW;
      const int32_t count = w1 - w0 > member ? (w1 - w0 - member + members - 1) / members : 0;
      xr[0] = 1;
      xr[1] = count;
      xr[2] = w0 + member;
      xr[3] = count;
      xr[4] = members;
    }
  }
  for (int j = 0; j < kXcds; ++j) long_cnt[j] = 0;
}

// P4: stable scatter of every row's nonzeros into the slice-major copy, plus per (row, slice)
// segment its first nonzero (seg_ptr) and its row within the block (seg_row). The per-row counts
// are recomputed exactly as plan_count computes them, so both passes agree.
template <int SMAX>
__global__ __launch_bounds__(kRB) void plan_scatter(const int32_t* __restrict__ rp, const int32_t* __restrict__ col,
                                                    const float* __restrict__ val, int64_t rows, int32_t nnz, int32_t S,
                                                    uint32_t width, uint32_t cols, const int32_t* __restrict__ tn,
                                                    const int32_t* __restrict__ ts, int32_t ld,
                                                    const int32_t* __restrict__ nb, const int32_t* __restrict__ sb,
                                                    int32_t* __restrict__ col_s, float* __restrict__ val_s,
                                                    int32_t* __restrict__ seg_ptr, uint8_t* __restrict__ seg_row,
                                                    int32_t* __restrict__ long_list, uint32_t* __restrict__ long_cnt,
                                                    int32_t long_cap, int32_t nblocks) {
  __shared__ int32_t cnt[kRB][SMAX + 1];
  __shared__ int32_t wn[kRB / 64][SMAX], wg[kRB / 64][SMAX];
  const int32_t blk = xcd_block(nblocks);
  if (blk < 0) return;  // whole workgroup
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  for (int s = 0; s < S; ++s) cnt[t][s] = 0;
  __syncthreads();
  const int64_t rw0 = (int64_t)blk * kRB + wave * 64;
  const bool active = rw0 < rows;  // wave-uniform
  WaveRows w{0, 0, 0};
  if (active) {
    w = wave_rows(rp, rw0, rows, nnz);
    wave_count<SMAX>(col, w, cols, width, cnt + wave * 64);
  }
  __syncthreads();
  for (int s = 0; s < S; ++s) {
    const int32_t c = cnt[t][s];
    const int32_t incl = wave_incl_scan(c);
    const uint64_t bal = __ballot(c > 0);
    if (lane == 63) wn[wave][s] = incl;
    if (lane == 0) wg[wave][s] = __builtin_popcountll(bal);
  }
  __syncthreads();
  for (int s = 0; s < S; ++s) {
    const int32_t c = cnt[t][s];
    const int32_t excl = wave_incl_scan(c) - c;
    const uint64_t bal = __ballot(c > 0);
    int32_t pn = 0, pg = 0;
    for (int v = 0; v < wave; ++v) {
      pn += wn[v][s];
      pg += wg[v][s];
    }
    if (c > 0) {
      const int64_t k = (int64_t)s * ld + blk;
      const int32_t p = nb[s] + tn[k] + pn + excl;
      const int32_t g = sb[s] + ts[k] + pg + (int32_t)lane_rank(bal);
      seg_ptr[g] = p;
      seg_row[g] = (uint8_t)t;
      if (c > kLongSeg) {
        // the XCD that gathers this slice; with S < 8 slices the XCDs sharing it take turns
        const int j = S >= kXcds ? (s & (kXcds - 1)) : s + S * (int)((uint32_t)g % (uint32_t)(kXcds / S));
        const uint32_t slot = atomicAdd(long_cnt + j, 1u);
        if (slot < (uint32_t)long_cap) long_list[(int64_t)j * long_cap + slot] = g;
      }
      cnt[t][s] = p;  // becomes this row's write cursor in slice s
    }
  }
  __syncthreads();
  if (!active) return;
  // Stream the wave's nonzeros again. Within a chunk, the lanes of one (row, slice) pair keep their
  // index order: rank = lanes below this one with the same slice, from the row's first lane on.
  int32_t (*cur)[SMAX + 1] = cnt + wave * 64;
  for (int32_t base0 = w.nz0; base0 < w.nz1; base0 += 64 * kChunks) {
    uint32_t cc[kChunks];
    float vv[kChunks];
    // Unconditional loads from a clamped index (base0 < nz1 here), so all of them go out together;
    // lanes past nz1 are dropped below.
#pragma unroll
    for (int u = 0; u < kChunks; ++u) {
      const int32_t i = min(base0 + 64 * u + lane, w.nz1 - 1);
      cc[u] = (uint32_t)col[i];
      vv[u] = val[i];
    }
#pragma unroll
    for (int u = 0; u < kChunks; ++u) cc[u] = clamp_col((int32_t)cc[u], cols);
#pragma unroll
    for (int u = 0; u < kChunks; ++u) {
      const int32_t base = base0 + 64 * u;
      const int32_t i = base + lane;
      const bool valid = i < w.nz1;
      const int l = wave_row_of(w.start, i);
      const int32_t s = valid ? (int32_t)(cc[u] / width) : S;
      const int first = max(__shfl(w.start, l, 64) - base, 0);
      uint64_t mine = 0;
      for (int q = 0; q < S; ++q) {
        const uint64_t m = __ballot(s == q);
        if (s == q) mine = m;
      }
      const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
      const int32_t rank = __builtin_popcountll(mine & below & (~0ull << first));
      if (valid) {
        const int32_t pos = cur[l][s] + rank;
        col_s[pos] = (int32_t)cc[u];
        val_s[pos] = vv[u];
      }
      wave_lds_sync();
      if (valid) atomicAdd(&cur[l][s], 1);
      wave_lds_sync();
    }
  }
}

// P5: window k covers nonzeros [k·kWW, (k+1)·kWW) of the slice-major copy; it owns the segments
// that start there, {g0, g1}, and loads the products [b, e) of those segments. A segment longer
// than kLongSeg can only be the window's last one (it reaches past the window), and is excluded.
__global__ __launch_bounds__(256) void plan_desc(const int32_t* __restrict__ seg_ptr, const int32_t* __restrict__ nb,
                                                 const int32_t* __restrict__ sb, int32_t S, int64_t nwin,
                                                 int4* __restrict__ desc) {
  const int64_t k = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (k >= nwin) return;
  const int32_t G = sb[S], Z = nb[S];
  const int64_t lo = k * kWW, hi = min(lo + kWW, (int64_t)Z);
  if (lo >= Z) {
    desc[k] = make_int4(G, G, Z, Z);
    return;
  }
  auto lower_bound = [&](int64_t target) {
    int32_t a = 0, z = G;
    while (a < z) {
      const int32_t mid = (a + z) >> 1;
      if ((int64_t)seg_ptr[mid] < target) a = mid + 1; else z = mid;
    }
    return a;
  };
  const int32_t g0 = lower_bound(lo), g1 = lower_bound(hi);
  const int32_t b = seg_ptr[g0];
  int32_t e = b;
  if (g1 > g0) {
    const int32_t lb = seg_ptr[g1 - 1], le = seg_ptr[g1];
    e = (le - lb > kLongSeg) ? lb : le;
  }
  e = min(e, b + kSpan);  // a consistent plan never needs this; it keeps the LDS span in bounds
  desc[k] = make_int4(g0, g1, b, e);
}


// Sequential sum of p[i0..i1) (index order), LDS reads four at a time.
__device__ inline float lds_seq_sum(const float* __restrict__ p, int32_t i0, int32_t i1) {
  float sum = 0.0f;
  int32_t i = i0;
  for (; i + 4 <= i1; i += 4) {
    const float a0 = p[i], a1 = p[i + 1], a2 = p[i + 2], a3 = p[i + 3];
    sum += a0;
    sum += a1;
    sum += a2;
    sum += a3;
  }
  for (; i < i1; ++i) sum += p[i];
  return sum;
}

// Buffer resources (dc::range_rsrc): loads past a range's end return 0 and stores past it are
// dropped by the hardware range check, so a window's loads and stores need no branches.
using dc::range_rsrc;
constexpr int kNt = dc::kBufNt;
constexpr uint32_t kDrop = 0x80000000u;  // a buffer offset past any range: the access is dropped
constexpr int kChunksW = kSpan / 256;    // 16-byte loads per lane covering a window's span
constexpr int kSegChunks = (kWW + 1 + 255) / 256;  // ... and its segment starts plus the end

// A window's loads, 16 bytes per lane: lane l holds elements 256 k + 4 l .. + 3 of chunk k.
struct WindowLoads {
  dc::i32x4 sp[kSegChunks];  // seg_ptr[g0 + ...]
  dc::i32x4 c[kChunksW];     // col_s[b + ...]
  dc::f32x4 v[kChunksW];     // val_s[b + ...]
};

// Ranges are rounded up to whole 16-byte groups (the arrays carry 16 bytes of slack), so a load is
// either wholly inside or wholly past the range; elements past e (or past g1) are ignored.
__device__ inline void window_issue(const int4 d, const int32_t* __restrict__ seg_ptr,
                                    const int32_t* __restrict__ col_s, const float* __restrict__ val_s,
                                    WindowLoads& w) {
  const uint32_t lane16 = (threadIdx.x & 63) * 16;
  const auto rs = range_rsrc(seg_ptr + d.x, ((d.y - d.x + 1 + 3) & ~3) * 4);
  const auto rc = range_rsrc(col_s + d.z, ((d.w - d.z + 3) & ~3) * 4);
  const auto rv = range_rsrc(val_s + d.z, ((d.w - d.z + 3) & ~3) * 4);
#pragma unroll
  for (int k = 0; k < kSegChunks; ++k)
    w.sp[k] = __builtin_bit_cast(dc::i32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, lane16 + 1024 * k, 0, kNt));
#pragma unroll
  for (int k = 0; k < kChunksW; ++k) {
    w.c[k] = __builtin_bit_cast(dc::i32x4, __builtin_amdgcn_raw_buffer_load_b128(rc, lane16 + 1024 * k, 0, kNt));
    w.v[k] = __builtin_bit_cast(dc::f32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, lane16 + 1024 * k, 0, kNt));
  }
}

__device__ inline int4 uniform_int4(int4 d) {
  return make_int4(__builtin_amdgcn_readfirstlane(d.x), __builtin_amdgcn_readfirstlane(d.y),
                   __builtin_amdgcn_readfirstlane(d.z), __builtin_amdgcn_readfirstlane(d.w));
}

// Float sum over the wave's 64 lanes in a fixed DPP tree order (result broadcast from lane 63).
__device__ inline float wave_sum_f32(float v) {
  auto step = [](float a, uint32_t b) { return a + __builtin_bit_cast(float, b); };
  v = step(v, dc::dpp_u32<0xB1, 0xF>(__builtin_bit_cast(uint32_t, v)));   // lanes xor 1
  v = step(v, dc::dpp_u32<0x4E, 0xF>(__builtin_bit_cast(uint32_t, v)));   // lanes xor 2
  v = step(v, dc::dpp_u32<0x141, 0xF>(__builtin_bit_cast(uint32_t, v)));  // half-row mirror
  v = step(v, dc::dpp_u32<0x140, 0xF>(__builtin_bit_cast(uint32_t, v)));  // row mirror
  v = step(v, dc::dpp_u32<0x142, 0xA>(__builtin_bit_cast(uint32_t, v)));  // row_bcast:15
  v = step(v, dc::dpp_u32<0x143, 0xC>(__builtin_bit_cast(uint32_t, v)));  // row_bcast:31
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ inline int32_t elem(const dc::i32x4& v, int j) { return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w; }


// Gather pass: persistent grid, XCD-affine; each wave walks its XCD's windows. Per window: one
// round trip for the 16-byte column/value/segment-start loads, one for the gathers (only the
// chunks that hold products), products to the wave's LDS (one 16-byte write per chunk), then the
// segment sums. The address unit is the limit here, so the number of memory instructions per
// window is what this layout minimises. Segment sums: up to kSeqSeg products, one lane adds them
// in index order; longer segments (up to kLongSeg) are summed by the whole wave: lane k adds
// products k, k + 64, ... in order, then a fixed DPP tree. Lane l owns segments 256 k + 4 l + j.
__global__ __launch_bounds__(kGatherBlock) void spmv_slice_windows(const int4* __restrict__ desc,
                                                                   const int32_t* __restrict__ seg_ptr,
                                                                   const int32_t* __restrict__ col_s,
                                                                   const float* __restrict__ val_s,
                                                                   const float* __restrict__ x,
                                                                   float* __restrict__ partial,
                                                                   const int32_t* __restrict__ xcd, int32_t cols,
                                                                   const double* __restrict__ sums_in, int32_t nsums,
                                                                   double* __restrict__ sum_out) {
  __shared__ dc::f32x4 prod[kGatherBlock / 64][kSpan / 4];
  if (sum_out && blockIdx.x == 0) {
    // The power iteration's previous L1 norm: workgroup 0 adds the previous SpMV's block sums in a
    // fixed order (thread t takes t, t + 256, ...; eight loads in flight), then its windows.
    __shared__ double red[kGatherBlock / 64];
    double a = 0.0;
    for (int32_t i0 = threadIdx.x; i0 < nsums; i0 += 8 * kGatherBlock) {
      double v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = i0 + k * kGatherBlock < nsums ? sums_in[i0 + k * kGatherBlock] : 0.0;
#pragma unroll
      for (int k = 0; k < 8; ++k) a += v[k];
    }
    const double total = dc::block_sum64<kGatherBlock>(a, red);
    if (threadIdx.x == 0) *sum_out = total;
  }
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = blockIdx.x & (kXcds - 1);
  const int32_t per_xcd_waves = (int32_t)(gridDim.x / kXcds) * (kGatherBlock / 64);
  const int32_t v = (int32_t)(blockIdx.x / kXcds) * (kGatherBlock / 64) + wave;
  const int32_t* xr = xcd + j * kXcdWords;
  const int32_t nr = xr[0], total = xr[1];
  if (v >= total) return;
  dc::f32x4* wp4 = prod[wave];
  const float* wp = reinterpret_cast<const float*>(prod[wave]);
  const auto rx = range_rsrc(x, (int32_t)((uint32_t)cols * 4u));  // x < 4 GB (checked at plan creation)
  auto window_desc = [&](int32_t l) {
    if (l >= total) return make_int4(0, 0, 0, 0);
    int32_t rem = l, k = 0;
    for (int q = 0; q < nr; ++q) {
      const int32_t cnt = xr[3 + 3 * q];
      if (rem < cnt) {
        k = xr[2 + 3 * q] + rem * xr[4 + 3 * q];
        break;
      }
      rem -= cnt;
    }
    return uniform_int4(desc[k]);
  };
  int4 d = window_desc(v);
  for (int32_t l = v; l < total; l += per_xcd_waves) {
    const int32_t g0 = d.x, g1 = d.y, b = d.z, e = d.w;
    WindowLoads w;
    window_issue(d, seg_ptr, col_s, val_s, w);
    const int4 dn = window_desc(l + per_xcd_waves);
    const int32_t span = e - b;
    // gathers: only chunks that hold products (a wave-uniform skip); x[0] for elements past e
    dc::f32x4 xv[kChunksW];
#pragma unroll
    for (int k = 0; k < kChunksW; ++k) {
      xv[k] = dc::f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      if (256 * k < span) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float g = __builtin_bit_cast(
              float, __builtin_amdgcn_raw_buffer_load_b32(rx, (uint32_t)elem(w.c[k], q) * 4u, 0, 0));
          if (q == 0) xv[k].x = g; else if (q == 1) xv[k].y = g; else if (q == 2) xv[k].z = g; else xv[k].w = g;
        }
      }
    }
#pragma unroll
    for (int k = 0; k < kChunksW; ++k)
      if (256 * k + 4 * lane < span) wp4[64 * k + lane] = w.v[k] * xv[k];  // products past e are never read
    wave_lds_sync();
    // segment sums: lane l, chunk k, element q -> segment s = 256 k + 4 l + q
    constexpr int kSumChunks = kWW / 256;  // a window owns at most kWW segments; the last chunk of
    constexpr int kSegSlots = kSumChunks * 4;  // starts only supplies the final segment's end
    float psum[kSegSlots];
    uint32_t off[kSegSlots];
    uint64_t wide[kSegSlots];
    const int32_t nseg = g1 - g0;
#pragma unroll
    for (int k = 0; k < kSumChunks; ++k) {
      const int32_t next_lane = __shfl(w.sp[k].x, (lane + 1) & 63, 64);  // lane l + 1's first start
      const int32_t next_chunk = __shfl(w.sp[k + 1].x, 0, 64);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int si = 4 * k + q;
        const int32_t sidx = 256 * k + 4 * lane + q;
        const int32_t rb = elem(w.sp[k], q);
        const int32_t re = q < 3 ? elem(w.sp[k], q + 1) : (lane < 63 ? next_lane : next_chunk);
        const bool in = sidx < nseg;
        const bool seq = in && re - rb <= kSeqSeg;
        wide[si] = __ballot(in && re - rb > kSeqSeg && re - rb <= kLongSeg);
        psum[si] = seq ? lds_seq_sum(wp, rb - b, min(re, e) - b) : 0.0f;
        off[si] = seq ? (uint32_t)sidx * 4u : kDrop;
      }
    }
#pragma unroll
    for (int si = 0; si < kSegSlots; ++si) {
      for (uint64_t m = wide[si]; m; m &= m - 1) {  // wave-uniform loop over this slot's wide segments
        const int L = __builtin_ctzll(m);
        const int k = si / 4, q = si % 4;
        const int32_t rb = __shfl(elem(w.sp[k], q), L, 64);
        int32_t re;
        if (q < 3) re = __shfl(elem(w.sp[k], q + 1), L, 64);
        else if (L < 63) re = __shfl(w.sp[k].x, L + 1, 64);
        else re = __shfl(w.sp[k + 1].x, 0, 64);
        float t = 0.0f;
        for (int32_t i = rb - b + lane; i < min(re, e) - b; i += 64) t += wp[i];
        const float tw = wave_sum_f32(t);
        if (lane == L) {
          psum[si] = tw;
          off[si] = (uint32_t)(256 * k + 4 * L + q) * 4u;
        }
      }
    }
    const auto rp = range_rsrc(partial + g0, nseg * 4);
#pragma unroll
    for (int k = 0; k < kSumChunks; ++k) {
      if (256 * k < nseg) {  // wave-uniform: groups holding no segment issue no store
#pragma unroll
        for (int q = 0; q < 4; ++q)
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int32_t, psum[4 * k + q]), rp, off[4 * k + q], 0, kNt);
      }
    }
    wave_lds_sync();
    d = dn;
  }
}

// Long segments (more than kLongSeg nonzeros in one slice): one wavefront per segment, on the XCD
// that owns its slice. A segment's cost is a chain of dependent round trips (its bounds, its
// columns and values, its gathers), so the pass is latency-bound: a wavefront per segment keeps as
// many segments in flight as the device holds waves, and kLongBatch loads per lane cover segments
// of up to kLongBatch * 64 nonzeros in one round trip each. Lane k adds products k, k + 64, ... in
// order, then a fixed DPP tree: deterministic.
constexpr int kLongWave = 64;
constexpr int kLongBatch = 32;
__global__ __launch_bounds__(kLongWave) void spmv_slice_long(const int32_t* __restrict__ seg_ptr,
                                                             const int32_t* __restrict__ col_s,
                                                             const float* __restrict__ val_s,
                                                             const float* __restrict__ x, float* __restrict__ partial,
                                                             const int32_t* __restrict__ long_list,
                                                             const uint32_t* __restrict__ long_cnt, int32_t long_cap) {
  const int j = blockIdx.x & (kXcds - 1);
  const int lane = threadIdx.x;
  const uint32_t n_long = min(long_cnt[j], (uint32_t)long_cap);
  for (uint32_t t = blockIdx.x / kXcds; t < n_long; t += gridDim.x / kXcds) {
    const int32_t g = long_list[(int64_t)j * long_cap + t];
    const int32_t b = seg_ptr[g], e = seg_ptr[g + 1];
    float sum = 0.0f;
    for (int32_t i0 = b + lane; i0 < e; i0 += kLongBatch * kLongWave) {
      int32_t c[kLongBatch];
      float v[kLongBatch], xv[kLongBatch];
#pragma unroll
      for (int k = 0; k < kLongBatch; ++k) {
        const int32_t i = i0 + k * kLongWave;
        c[k] = 0;
        v[k] = 0.0f;
        if (i < e) {
          c[k] = __builtin_nontemporal_load(col_s + i);
          v[k] = __builtin_nontemporal_load(val_s + i);
        }
      }
#pragma unroll
      for (int k = 0; k < kLongBatch; ++k) xv[k] = x[c[k]];  // c = 0 past e: gathered, then dropped below
#pragma unroll
      for (int k = 0; k < kLongBatch; ++k) sum += (i0 + k * kLongWave < e) ? v[k] * xv[k] : 0.0f;
    }
    const float total = wave_sum_f32(sum);
    if (lane == 0) partial[g] = total;
  }
}

// Combine pass, a workgroup per block of kRB rows: the block's segments of each slice are one
// contiguous run of the slice-major arrays; every thread takes runs' entries (kCombineBatch
// loads in flight) and drops each partial into tab[row][slice]; then thread r adds its row in
// slice order: y = 0.0f + tab[r][0] + tab[r][1] + ... (absent slices hold +0.0f, which leaves a
// sum that starts at +0.0f unchanged). With kSums, also the block's float64 sum of y (fixed
// order) for the power iteration. SMAX >= S sizes the LDS table.
constexpr int kCombineBatch = 4;
// With `scale` (the power iteration), y = (float)((double)row sum / *scale): the previous step's
// normalisation x = y / s applied to this step's product instead (A·(u / s) = (A·u) / s).
template <bool kSums, int SMAX>
__global__ __launch_bounds__(kRB) void spmv_slice_combine(const int32_t* __restrict__ ts, int32_t ld, int32_t S,
                                                          const int32_t* __restrict__ sb,
                                                          const uint8_t* __restrict__ seg_row,
                                                          const float* __restrict__ partial, float* __restrict__ y,
                                                          int64_t rows, double* __restrict__ block_sums,
                                                          const double* __restrict__ scale) {
  __shared__ float tab[kRB][SMAX + 1];
  __shared__ int32_t run_pre[SMAX + 1], run_base[SMAX];
  __shared__ double red[kRB / 64];
  const int t = threadIdx.x;
#pragma unroll
  for (int s = 0; s < SMAX; ++s) tab[t][s] = 0.0f;
  if (t < 64) {  // wave 0: run lengths and their prefix over slices
    int32_t n = 0;
    if (t < S) {
      const int64_t k = (int64_t)t * ld + blockIdx.x;
      const int32_t a = ts[k];
      n = ts[k + 1] - a;
      run_base[t] = sb[t] + a;
    }
    const int32_t incl = wave_incl_scan(n);
    if (t < S) run_pre[t] = incl - n;
    if (t == S - 1) run_pre[S] = incl;
  }
  __syncthreads();
  const int32_t total = run_pre[S];
  for (int32_t q0 = t; q0 < total; q0 += kCombineBatch * kRB) {
    int ss[kCombineBatch];
    uint32_t rr[kCombineBatch];
    float pv[kCombineBatch];
#pragma unroll
    for (int u = 0; u < kCombineBatch; ++u) {
      const int32_t q = q0 + u * kRB;
      int s = 0;  // last slice whose run starts at or before q
#pragma unroll
      for (int step = SMAX / 2; step > 0; step >>= 1)
        if (s + step < S && run_pre[s + step] <= q) s += step;
      ss[u] = s;
      rr[u] = 0;
      pv[u] = 0.0f;
      if (q < total) {
        const int32_t g = run_base[s] + (q - run_pre[s]);
        rr[u] = seg_row[g];
        pv[u] = __builtin_nontemporal_load(partial + g);
      }
    }
#pragma unroll
    for (int u = 0; u < kCombineBatch; ++u)
      if (q0 + u * kRB < total) tab[rr[u]][ss[u]] = pv[u];
  }
  __syncthreads();
  float acc = 0.0f;
#pragma unroll
  for (int s = 0; s < SMAX; ++s)
    if (s < S) acc += tab[t][s];
  if (scale) acc = (float)((double)acc / *scale);
  const int64_t r = (int64_t)blockIdx.x * kRB + t;
  if (r < rows) y[r] = acc;
  if constexpr (kSums) {
    const double tsum = dc::block_sum64<kRB>(r < rows ? (double)acc : 0.0, red);
    if (t == 0) block_sums[blockIdx.x] = tsum;
  }
}

template <bool kSums>
int32_t launch_combine(dc_hip_ctx* ctx, unsigned grid, const int32_t* ts, int32_t ld, int32_t S, const int32_t* sb,
                       const uint8_t* seg_row, const float* partial, float* y, int64_t rows, double* block_sums,
                       const double* scale) {
#define DC_COMBINE(SM)                                                                                          \
  spmv_slice_combine<kSums, SM><<<grid, kRB, 0, ctx->stream>>>(ts, ld, S, sb, seg_row, partial, y, rows, block_sums, \
                                                               scale)
  if (S <= 1) DC_COMBINE(1);
  else if (S <= 2) DC_COMBINE(2);
  else if (S <= 4) DC_COMBINE(4);
  else if (S <= 8) DC_COMBINE(8);
  else if (S <= 16) DC_COMBINE(16);
  else DC_COMBINE(32);
#undef DC_COMBINE
  return dc::last_launch_status();
}

}  // namespace

// Device memory of a plan, carved from one allocation.
struct dc_hip_spmv_plan {
  int device = 0;
  int64_t rows = 0, cols = 0, nnz = 0;
  int32_t slices = 1;
  int64_t slice_cols = 0;
  int32_t nblocks = 0;
  int64_t nwin = 0;
  int32_t long_cap = 1;
  bool owns_mem = false;
  void* mem = nullptr;
  size_t bytes = 0;
  int32_t *col_s = nullptr, *seg_ptr = nullptr, *tn = nullptr, *ts = nullptr, *tot = nullptr, *nb = nullptr,
          *sb = nullptr, *xcd = nullptr, *long_list = nullptr;
  uint8_t* seg_row = nullptr;
  uint32_t* long_cnt = nullptr;
  float *val_s = nullptr, *partial = nullptr;
  int4* desc = nullptr;
  double *block_sums = nullptr, *scalars = nullptr;
};

namespace {

// Walks the plan's memory layout: with mem == nullptr it only sizes it (p->bytes).
void plan_layout(dc_hip_spmv_plan* p, void* mem) {
  char* m = static_cast<char*>(mem);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* q = m ? m + off : nullptr;
    off += (bytes + 255) & ~(size_t)255;
    return q;
  };
  const size_t nz = (size_t)std::max<int64_t>(p->nnz, 1);
  const size_t tab = (size_t)p->slices * (p->nblocks + 1) * 4;
  // col_s, val_s and seg_ptr are read with 16-byte loads over ranges rounded up to whole groups:
  // 16 bytes of slack after each keeps those loads inside the allocation
  p->col_s = reinterpret_cast<int32_t*>(take(nz * 4 + 16));
  p->val_s = reinterpret_cast<float*>(take(nz * 4 + 16));
  p->seg_ptr = reinterpret_cast<int32_t*>(take((nz + 1) * 4 + 16));
  p->partial = reinterpret_cast<float*>(take(nz * 4));
  p->seg_row = reinterpret_cast<uint8_t*>(take(nz));
  p->tn = reinterpret_cast<int32_t*>(take(tab));
  p->ts = reinterpret_cast<int32_t*>(take(tab));
  p->tot = reinterpret_cast<int32_t*>(take(2 * kMaxSlices * 4));
  p->nb = reinterpret_cast<int32_t*>(take((kMaxSlices + 1) * 4));
  p->sb = reinterpret_cast<int32_t*>(take((kMaxSlices + 1) * 4));
  p->xcd = reinterpret_cast<int32_t*>(take(kMaxPhases * kXcds * kXcdWords * 4));
  p->desc = reinterpret_cast<int4*>(take((size_t)std::max<int64_t>(p->nwin, 1) * 16));
  p->long_cnt = reinterpret_cast<uint32_t*>(take(kXcds * 4));
  p->long_list = reinterpret_cast<int32_t*>(take((size_t)kXcds * p->long_cap * 4));
  p->block_sums = reinterpret_cast<double*>(take((size_t)p->nblocks * 8));
  p->scalars = reinterpret_cast<double*>(take(8 * 8));
  p->mem = mem;
  p->bytes = off;
}

// Shape of the plan (slices, sizes) and the bytes it needs.
void plan_shape(dc_hip_spmv_plan* p, int64_t rows, int64_t cols, int64_t nnz, int64_t slice_cols_max) {
  p->rows = rows;
  p->cols = cols;
  p->nnz = nnz;
  const int64_t wmax = slice_cols_max > 0 ? slice_cols_max : kSliceCols;
  int64_t S = 1;
  if (cols > wmax) {
    if (cols <= 2 * wmax) S = 2;
    else if (cols <= 4 * wmax) S = 4;
    else S = std::min<int64_t>(kMaxSlices, kXcds * ((cols + kXcds * wmax - 1) / (kXcds * wmax)));
  } else if (slice_cols_max == 0) {
    // x fits one slice, but every XCD gathering from all of it (with the nonzeros streaming
    // through the same L2) misses far more than an XCD holding a share of at most 512 KB: with
    // S < 8 slices, XCD j takes slice j % S. Measured at 1M rows: S = 1 58.8 us per SpMV, S = 2
    // 51.5, S = 4 48.5, S = 8 48.3, S = 16 56.7 (more segments than the cache saves).
    const int64_t xbytes = cols * 4;
    S = xbytes <= (int64_t{512} << 10) ? 1 : xbytes <= (int64_t{1} << 20) ? 2 : xbytes <= (int64_t{2} << 20) ? 4 : 8;
  }
  p->slices = (int32_t)S;
  p->slice_cols = std::max<int64_t>(1, (cols + S - 1) / S);
  p->nblocks = (int32_t)std::max<int64_t>(1, (rows + kRB - 1) / kRB);
  p->nwin = (nnz + kWW - 1) / kWW;
  p->long_cap = (int32_t)(nnz / (kLongSeg + 1) + 1);
  plan_layout(p, nullptr);
}

// The analysis kernels, on the context stream.
int32_t plan_build(dc_hip_ctx* ctx, dc_hip_spmv_plan* p, const int32_t* rp, const int32_t* col, const float* val) {
  const int32_t S = p->slices, ld = p->nblocks + 1;
  const uint32_t width = (uint32_t)p->slice_cols, cols = (uint32_t)std::max<int64_t>(p->cols, 1);
  const int32_t nnz = (int32_t)p->nnz;
  if (p->rows == 0) return DC_OK;
  const unsigned agrid = (unsigned)(kXcds * ((p->nblocks + kXcds - 1) / kXcds));
#define DC_PLAN_COUNT(SM)                                                                                      \
  plan_count<SM><<<agrid, kRB, 0, ctx->stream>>>(rp, col, p->rows, nnz, S, width, cols, p->tn, p->ts, ld, \
                                                 p->nblocks)
  if (S <= 1) DC_PLAN_COUNT(1);
  else if (S <= 2) DC_PLAN_COUNT(2);
  else if (S <= 4) DC_PLAN_COUNT(4);
  else if (S <= 8) DC_PLAN_COUNT(8);
  else if (S <= 16) DC_PLAN_COUNT(16);
  else DC_PLAN_COUNT(32);
#undef DC_PLAN_COUNT
  DC_RETURN_IF(dc::last_launch_status());
  plan_scan<<<(unsigned)S, kScanBlock, 0, ctx->stream>>>(p->tn, p->ts, p->nblocks, ld, S, p->tot);
  DC_RETURN_IF(dc::last_launch_status());
  plan_bases<<<1, 64, 0, ctx->stream>>>(p->tot, S, p->nb, p->sb, p->seg_ptr, p->xcd, p->long_cnt);
  DC_RETURN_IF(dc::last_launch_status());
#define DC_PLAN_SCATTER(SM)                                                                                 \
  plan_scatter<SM><<<agrid, kRB, 0, ctx->stream>>>(rp, col, val, p->rows, nnz, S, width, cols, p->tn, p->ts, ld, \
                                                   p->nb, p->sb, p->col_s, p->val_s, p->seg_ptr, p->seg_row,      \
                                                   p->long_list, p->long_cnt, p->long_cap, p->nblocks)
  if (S <= 1) DC_PLAN_SCATTER(1);
  else if (S <= 2) DC_PLAN_SCATTER(2);
  else if (S <= 4) DC_PLAN_SCATTER(4);
  else if (S <= 8) DC_PLAN_SCATTER(8);
  else if (S <= 16) DC_PLAN_SCATTER(16);
  else DC_PLAN_SCATTER(32);
#undef DC_PLAN_SCATTER
  DC_RETURN_IF(dc::last_launch_status());
  if (p->nwin > 0) {
    plan_desc<<<(unsigned)((p->nwin + 255) / 256), 256, 0, ctx->stream>>>(p->seg_ptr, p->nb, p->sb, S, p->nwin,
                                                                           p->desc);
    DC_RETURN_IF(dc::last_launch_status());
  }
  return DC_OK;
}

// One SpMV through the plan: y = A·x (with `sums`, also the per-block float64 sums of y). With
// `scale`, y = (A·x) / *scale (the power iteration's normalisation of x, applied to the product).
// With `prev_sum_out`, *prev_sum_out = the sum of the block sums as they stand (the previous
// SpMV's), computed before this SpMV's combine replaces them: by the first gather launch, so it
// costs no launch of its own.
int32_t plan_spmv(dc_hip_ctx* ctx, const dc_hip_spmv_plan* p, const float* x, float* y, bool sums = false,
                  const double* scale = nullptr, double* prev_sum_out = nullptr) {
  if (p->rows == 0) return DC_OK;
  const int ld = p->nblocks + 1;
  if (p->nwin > 0) {
    const int per_xcd_cus = std::max(1, ctx->cu_count / kXcds);
    const int phases = p->slices >= kXcds ? p->slices / kXcds : 1;
    // resident gather workgroups per CU (registers and LDS decide it), asked once per process
    static const int per_cu = [] {
      int n = 0;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, spmv_slice_windows, kGatherBlock, 0) != hipSuccess || n < 1)
        n = 4;
      return n;
    }();
    const int64_t want = (p->nwin / phases / kXcds + 3) / 4 + 1;  // workgroups per XCD, one window per wave
    const int64_t per_xcd = std::min<int64_t>(want, (int64_t)per_xcd_cus * per_cu);
    for (int ph = 0; ph < phases; ++ph) {
      spmv_slice_windows<<<(unsigned)(per_xcd * kXcds), kGatherBlock, 0, ctx->stream>>>(
          p->desc, p->seg_ptr, p->col_s, p->val_s, x, p->partial, p->xcd + ph * kXcds * kXcdWords,
          (int32_t)p->cols, p->block_sums, p->nblocks, ph == 0 ? prev_sum_out : nullptr);
      DC_RETURN_IF(dc::last_launch_status());
    }
    // A wavefront per long segment (up to 16 resident per CU); those past the device-side count
    // return at once.
    const int64_t lgrid = std::min<int64_t>((int64_t)p->long_cap, (int64_t)per_xcd_cus * 16);
    spmv_slice_long<<<(unsigned)(std::max<int64_t>(1, lgrid) * kXcds), kLongWave, 0, ctx->stream>>>(
        p->seg_ptr, p->col_s, p->val_s, x, p->partial, p->long_list, p->long_cnt, p->long_cap);
    DC_RETURN_IF(dc::last_launch_status());
  } else if (prev_sum_out) {
    DC_RETURN_IF(dc::launch_reduce_partials_f64(ctx, p->block_sums, p->nblocks, prev_sum_out));
  }
  if (sums)
    return launch_combine<true>(ctx, (unsigned)p->nblocks, p->ts, ld, p->slices, p->sb, p->seg_row, p->partial, y,
                                p->rows, p->block_sums, scale);
  return launch_combine<false>(ctx, (unsigned)p->nblocks, p->ts, ld, p->slices, p->sb, p->seg_row, p->partial, y,
                               p->rows, nullptr, scale);
}

// y_k = A·x_k; s_k = Σ y_k; x_{k+1} = y_k / s_k. The division moves into the next step's combine
// (y_{k+1} = (A·y_k) / s_k), so the unnormalised y_k is the next step's input as it stands and the
// buffers swap roles (x, y, x, ...); the last y is normalised into x once at the end. s_k is formed
// by step k + 1's first gather launch, from step k's block sums, before step k + 1's combine
// (which divides by it) overwrites them, so it costs no launch of its own.
int32_t plan_power_iterate(dc_hip_ctx* ctx, const dc_hip_spmv_plan* p, float* x, float* y, int32_t iterations,
                           double* last_sum_out) {
  if (p->rows == 0 || iterations == 0) return DC_OK;
  double* s = p->scalars;
  const unsigned ngrid = (unsigned)std::max<int64_t>(1, std::min<int64_t>((p->rows + kBlock - 1) / kBlock, 16384));
  const float* src = x;
  float* dst = y;
  for (int32_t it = 0; it < iterations; ++it) {
    DC_RETURN_IF(plan_spmv(ctx, p, src, dst, true, it == 0 ? nullptr : s, it == 0 ? nullptr : s));
    src = dst;
    dst = dst == y ? x : y;
  }
  DC_RETURN_IF(dc::launch_reduce_partials_f64(ctx, p->block_sums, p->nblocks, s));
  normalise_kernel<<<ngrid, kBlock, 0, ctx->stream>>>(src, x, p->rows, s);  // in place when src == x
  DC_RETURN_IF(dc::last_launch_status());
  if (last_sum_out) DC_RETURN_IF_HIP(hipMemcpyAsync(last_sum_out, s, sizeof(double), hipMemcpyDeviceToDevice, ctx->stream));
  return DC_OK;
}

int32_t check_plan_shape(int64_t rows, int64_t cols, int64_t nnz) {
  if (cols < 0 || (nnz > 0 && cols == 0)) return DC_ERR_INVALID_ARGUMENT;
  if (cols > (int64_t{1} << 30) - 1) return DC_ERR_UNSUPPORTED;  // x is addressed with 32-bit byte offsets
  (void)rows;
  return DC_OK;
}

}  // namespace

extern "C" {

DC_HIP_API int32_t dc_hip_spmv_csr_f32(dc_hip_ctx* ctx, const int32_t* row_pointers, const int32_t* col_indices,
                                       const float* values, const float* x, float* y, int64_t rows, int64_t cols,
                                       int64_t nnz) {
  DC_RETURN_IF(check_csr(row_pointers, col_indices, values, rows, nnz));
  if (cols < 0 || (rows > 0 && !y) || (cols > 0 && !x)) return DC_ERR_INVALID_ARGUMENT;
  DC_CTX_ENTER(ctx);
  if (rows == 0) return DC_OK;
  const SpmvPlan plan = make_plan(nnz);
  DC_RETURN_IF(launch_analysis(ctx, plan, row_pointers, rows));
  return launch_spmv(ctx, plan, row_pointers, col_indices, values, x, y);
}

DC_HIP_API int32_t dc_hip_spmv_plan_create(dc_hip_ctx* ctx, const int32_t* row_pointers, const int32_t* col_indices,
                                           const float* values, int64_t rows, int64_t cols, int64_t nnz,
                                           int64_t slice_cols_max, dc_hip_spmv_plan** plan_out) {
  if (!plan_out) return DC_ERR_INVALID_ARGUMENT;
  *plan_out = nullptr;
  DC_RETURN_IF(check_csr(row_pointers, col_indices, values, rows, nnz));
  DC_RETURN_IF(check_plan_shape(rows, cols, nnz));
  if (slice_cols_max < 0) return DC_ERR_INVALID_ARGUMENT;
  DC_CTX_ENTER(ctx);
  dc_hip_spmv_plan* p = new (std::nothrow) dc_hip_spmv_plan;
  if (!p) return DC_ERR_OUT_OF_MEMORY;
  p->device = ctx->device;
  plan_shape(p, rows, cols, nnz, slice_cols_max);
  void* mem = nullptr;
  if (hipMalloc(&mem, p->bytes) != hipSuccess) {
    delete p;
    return DC_ERR_OUT_OF_MEMORY;
  }
  p->owns_mem = true;
  plan_layout(p, mem);
  const int32_t st = plan_build(ctx, p, row_pointers, col_indices, values);
  if (st != DC_OK) {
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipFree(mem);
    delete p;
    return st;
  }
  *plan_out = p;
  return DC_OK;
}

DC_HIP_API int32_t dc_hip_spmv_plan_destroy(dc_hip_spmv_plan* plan) {
  if (!plan) return DC_ERR_INVALID_ARGUMENT;
  DC_RETURN_IF_HIP(hipSetDevice(plan->device));
  // Work queued on any stream may still read the plan: wait for the device before freeing.
  DC_RETURN_IF_HIP(hipDeviceSynchronize());
  if (plan->owns_mem && plan->mem) DC_RETURN_IF_HIP(hipFree(plan->mem));
  delete plan;
  return DC_OK;
}

DC_HIP_API int32_t dc_hip_spmv_plan_info(const dc_hip_spmv_plan* plan, int32_t* slices, int64_t* slice_cols,
                                         int64_t* device_bytes) {
  if (!plan) return DC_ERR_INVALID_ARGUMENT;
  if (slices) *slices = plan->slices;
  if (slice_cols) *slice_cols = plan->slice_cols;
  if (device_bytes) *device_bytes = (int64_t)plan->bytes;
  return DC_OK;
}

DC_HIP_API int32_t dc_hip_spmv_plan_execute_f32(dc_hip_ctx* ctx, const dc_hip_spmv_plan* plan, const float* x,
                                                float* y) {
  if (!plan || (plan->rows > 0 && !y) || (plan->cols > 0 && !x)) return DC_ERR_INVALID_ARGUMENT;
  DC_CTX_ENTER(ctx);
  if (plan->device != ctx->device) return DC_ERR_INVALID_ARGUMENT;
  return plan_spmv(ctx, plan, x, y);
}

DC_HIP_API int32_t dc_hip_spmv_plan_power_iterate_f32(dc_hip_ctx* ctx, const dc_hip_spmv_plan* plan, float* x,
                                                      float* y, int32_t iterations, double* last_sum_out) {
  if (!plan || iterations < 0 || (plan->rows > 0 && (!x || !y))) return DC_ERR_INVALID_ARGUMENT;
  if (plan->rows != plan->cols) return DC_ERR_DIMENSION;
  DC_CTX_ENTER(ctx);
  if (plan->device != ctx->device) return DC_ERR_INVALID_ARGUMENT;
  return plan_power_iterate(ctx, plan, x, y, iterations, last_sum_out);
}

DC_HIP_API int32_t dc_hip_spmv_power_iterate_f32(dc_hip_ctx* ctx, const int32_t* row_pointers,
                                                 const int32_t* col_indices, const float* values, float* x, float* y,
                                                 int64_t rows, int64_t nnz, int32_t iterations, double* last_sum_out) {
  DC_RETURN_IF(check_csr(row_pointers, col_indices, values, rows, nnz));
  if (iterations < 0 || (rows > 0 && (!x || !y))) return DC_ERR_INVALID_ARGUMENT;
  DC_RETURN_IF(check_plan_shape(rows, rows, nnz));
  DC_CTX_ENTER(ctx);
  if (rows == 0 || iterations == 0) return DC_OK;
  // The plan lives in context scratch (reused by the next call; calls on a context are ordered).
  dc_hip_spmv_plan p;
  p.device = ctx->device;
  plan_shape(&p, rows, rows, nnz, 0);
  DC_RETURN_IF(dc::ensure_spmv_plan_mem(ctx, p.bytes));
  plan_layout(&p, ctx->spmv_plan_mem);
  DC_RETURN_IF(plan_build(ctx, &p, row_pointers, col_indices, values));
  return plan_power_iterate(ctx, &p, x, y, iterations, last_sum_out);
}

}  // extern "C"

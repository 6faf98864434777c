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
//   long rows (more than kLongRow nonzeros): summed by the workgroup of the window in which they
//     start, after its short rows, with a fixed-order block reduction (deterministic, not
//     sequential order). At most two long rows start in one window (each holds kLongRow + 1 or
//     more nonzeros, so a third would start past the window).
// A window's product span is at most kWindow + kLongRow entries (only its last row can run past
// the window, and it is short or excluded), which sizes the LDS buffer.
#include <algorithm>
#include <new>

#include "dc_device.hpp"
#include "dc_internal.hpp"

namespace {

constexpr int kBlock = 256;
constexpr int kWindow = 1024;   // nonzeros per window
constexpr int kLongRow = 512;   // rows longer than this are summed by the whole workgroup
constexpr int kMaxLongPerWindow = 4;  // a well-formed CSR starts at most two long rows in a window

// row_start[k] = first row whose first nonzero index is >= k·kWindow, for k in [0, windows);
// row_start[windows] = rows. One thread per entry r of the row pointers (coalesced, no search):
// the windows k with rp[r - 1] < k·kWindow <= rp[r] start at row r (for r = 0, k = 0 only). With
// monotone row pointers every k is written exactly once.
__global__ __launch_bounds__(kBlock) void spmv_window_starts(const int32_t* __restrict__ rp, int64_t rows,
                                                             int32_t windows, int32_t* __restrict__ row_start) {
  const int64_t r = blockIdx.x * (int64_t)kBlock + threadIdx.x;
  if (r > rows) return;
  const int64_t cur = rp[r];
  const int64_t k_lo = r == 0 ? 0 : (int64_t)rp[r - 1] / kWindow + 1;  // first k with k·W > rp[r - 1]
  const int64_t k_hi = min(cur < 0 ? (int64_t)-1 : cur / kWindow, (int64_t)windows - 1);
  for (int64_t k = max(k_lo, (int64_t)0); k <= k_hi; ++k) row_start[k] = (int32_t)r;
  if (r == rows) row_start[windows] = (int32_t)rows;
}

// Element arithmetic of SparseOps.SpMV<T> (SparseMatrix.cs:669-692) for T = float, double or int:
// one rounding per product and per addition for the floating types; for int, C#'s unchecked
// wrapping multiply and add (so a long row's fixed-order tree gives the same bits as the
// sequential sum).
template <typename T>
__device__ inline T spmv_mul(T a, T b) { return a * b; }
template <typename T>
__device__ inline T spmv_add(T a, T b) { return a + b; }
template <>
__device__ inline int32_t spmv_mul(int32_t a, int32_t b) { return (int32_t)((uint32_t)a * (uint32_t)b); }
template <>
__device__ inline int32_t spmv_add(int32_t a, int32_t b) { return (int32_t)((uint32_t)a + (uint32_t)b); }

// Sum of the products of nonzeros [b, e) by the whole workgroup (kBlock threads) in a fixed order:
// thread t adds, pass by pass, the pairwise sum of its four slots t + k·kBlock; then a butterfly
// across each wave and the waves in index order. Called by every thread; returns the total to
// thread 0. `red` holds one value per wave.
template <typename T>
__device__ T long_row_sum(int32_t b, int32_t e, const int32_t* __restrict__ col, const T* __restrict__ val,
                          const T* __restrict__ x, T* red) {
  T sum = T(0);
  // Four slots per pass: their loads and gathers are independent and overlap.
  for (int32_t i0 = b + (int32_t)threadIdx.x; i0 < e; i0 += 4 * kBlock) {
    int32_t c[4];
    T v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int32_t i = i0 + k * kBlock;
      c[k] = 0;
      v[k] = T(0);
      if (i < e) {
        c[k] = __builtin_nontemporal_load(col + i);
        v[k] = __builtin_nontemporal_load(val + i);
      }
    }
    T xv[4], p[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) xv[k] = x[c[k]];  // c = 0 past e: gathered, then dropped below
#pragma unroll
    for (int k = 0; k < 4; ++k) p[k] = (i0 + k * kBlock < e) ? spmv_mul(v[k], xv[k]) : T(0);
    sum = spmv_add(sum, spmv_add(spmv_add(p[0], p[1]), spmv_add(p[2], p[3])));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) sum = spmv_add(sum, __shfl_xor(sum, off, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = sum;
  __syncthreads();
  T total = red[0];
#pragma unroll
  for (int w = 1; w < kBlock / dc::kWave; ++w) total = spmv_add(total, red[w]);
  __syncthreads();  // red is reused by the next call
  return total;
}

template <typename T>
__global__ __launch_bounds__(kBlock) void spmv_windows_kernel(const int32_t* __restrict__ rp, const int32_t* __restrict__ col,
                                                              const T* __restrict__ val, const T* __restrict__ x,
                                                              T* __restrict__ y,
                                                              const int32_t* __restrict__ row_start, int32_t rows) {
  __shared__ T s_prod[kWindow + kLongRow];
  __shared__ int32_t s_long[kMaxLongPerWindow];
  __shared__ uint32_t s_nlong;
  __shared__ T s_red[kBlock / dc::kWave];
  // (clamped: with row pointers that are not monotone an entry may be stale; the rows read stay
  // inside [0, rows])
  const int32_t r0 = min(max(row_start[blockIdx.x], 0), rows), r1 = min(max(row_start[blockIdx.x + 1], 0), rows);
  if (r0 >= r1) return;  // uniform across the workgroup: no row starts in this window
  if (threadIdx.x == 0) s_nlong = 0;
  const int32_t b = rp[r0];
  const int32_t last_begin = rp[r1 - 1], last_end = rp[r1];
  // The last row may run past the window; if it is long it is summed after the short rows.
  int32_t e = (last_end - last_begin > kLongRow) ? last_begin : last_end;
  e = min(e, b + kWindow + kLongRow);  // a well-formed CSR never needs this clamp; it keeps LDS in bounds
  // All column/value loads of this thread's slots go out first, then all x gathers, so a window
  // costs two memory round trips instead of two per slot. Values and columns are streamed once
  // (non-temporal); x is what the caches are for.
  constexpr int kSlots = (kWindow + kLongRow) / kBlock;
  int32_t c[kSlots];
  T v[kSlots];
#pragma unroll
  for (int k = 0; k < kSlots; ++k) {
    const int32_t i = b + (int32_t)threadIdx.x + k * kBlock;
    c[k] = 0;
    v[k] = T(0);
    if (i < e) {
      c[k] = __builtin_nontemporal_load(col + i);
      v[k] = __builtin_nontemporal_load(val + i);
    }
  }
  T xv[kSlots];  // every gather in flight before the first product is stored (c = 0 past e)
#pragma unroll
  for (int k = 0; k < kSlots; ++k) xv[k] = x[c[k]];
#pragma unroll
  for (int k = 0; k < kSlots; ++k) {
    const int32_t i = b + (int32_t)threadIdx.x + k * kBlock;
    if (i < e) s_prod[i - b] = spmv_mul(v[k], xv[k]);
  }
  __syncthreads();
  for (int32_t r = r0 + (int32_t)threadIdx.x; r < r1; r += kBlock) {
    const int32_t rb = rp[r], re = rp[r + 1];
    if (re - rb > kLongRow) {
      const uint32_t slot = atomicAdd(&s_nlong, 1u);
      if (slot < (uint32_t)kMaxLongPerWindow) s_long[slot] = r;  // more only with malformed row pointers
      continue;
    }
    T sum = T(0);
    const int32_t i0 = max(rb - b, 0), i1 = min(re - b, e - b);
    for (int32_t i = i0; i < i1; ++i) sum = spmv_add(sum, s_prod[i]);
    __builtin_nontemporal_store(sum, y + r);
  }
  __syncthreads();
  const uint32_t n_long = min(s_nlong, (uint32_t)kMaxLongPerWindow);  // uniform
  for (uint32_t t = 0; t < n_long; ++t) {
    const int32_t row = s_long[t];
    const T total = long_row_sum(rp[row], rp[row + 1], col, val, x, s_red);
    if (threadIdx.x == 0) y[row] = total;
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
};

SpmvPlan make_plan(int64_t nnz) {
  SpmvPlan p;
  p.windows = (int32_t)(nnz / kWindow + 1);  // every first-nonzero index in [0, nnz] has a window
  return p;
}

// Analysis: the window starts (one pass over the row pointers).
int32_t launch_analysis(dc_hip_ctx* ctx, const SpmvPlan& plan, const int32_t* rp, int64_t rows) {
  DC_RETURN_IF(dc::ensure_spmv_windows(ctx, (size_t)plan.windows + 1));
  const unsigned grid = (unsigned)((rows + 1 + kBlock - 1) / kBlock);
  spmv_window_starts<<<grid, kBlock, 0, ctx->stream>>>(rp, rows, plan.windows, ctx->spmv_windows);
  return dc::last_launch_status();
}

template <typename T>
int32_t launch_spmv(dc_hip_ctx* ctx, const SpmvPlan& plan, const int32_t* rp, const int32_t* col, const T* val,
                    const T* x, T* y, int64_t rows) {
  spmv_windows_kernel<T><<<(unsigned)plan.windows, kBlock, 0, ctx->stream>>>(rp, col, val, x, y, ctx->spmv_windows,
                                                                             (int32_t)rows);
  return dc::last_launch_status();
}

int32_t check_csr(const int32_t* rp, const int32_t* col, const void* val, int64_t rows, int64_t nnz) {
  if (rows < 0 || nnz < 0 || nnz > INT32_MAX - 2 * kWindow || rows >= INT32_MAX) return DC_ERR_INVALID_ARGUMENT;
  if (!rp || (nnz > 0 && (!col || !val))) return DC_ERR_INVALID_ARGUMENT;
  return DC_OK;
}

// =============================================================================================
// Tiled plan for repeated SpMV (the power iteration; any CsrMatrix multiplied many times).
//
// The cost of a CSR SpMV is its random 4-byte gathers from x. Served by L2 they are bound by the
// rate of L1-miss requests a CU keeps in flight (about 0.3 per cycle per CU on MI355X), served by
// the memory-side cache by far less. The plan moves every gather into LDS:
//   - columns are cut into slices of at most kTileCols columns (a 128 KB tile of x, one CU's LDS);
//   - rows are cut into blocks: row r is in block rp[r] / span + r / kBlockRows (span = 4096 or
//     8192 nonzeros, chosen per plan), so a block holds fewer than 2 span nonzeros unless it ends
//     with a giant row (more than span nonzeros; at most one per block, always its last row: the
//     next row starts past the block's span);
//   - the plan keeps a slice-major copy of the nonzeros: slice s holds, block after block, the
//     nonzeros of block b whose column falls in s (the run (b, s)), each with its column within
//     the slice (uint16), its value, and its position within the block's CSR range (uint16).
//     Giant rows are kept in CSR order in one more region (slice index S), their column split over
//     the two uint16 arrays.
// product pass: persistent workgroups split the slice-major entries evenly; a workgroup loads the
//   x tile of each slice its share touches into LDS and streams p = val · x_tile[col16] (16-byte
//   loads and stores).
// row pass: a workgroup per block (span / 8 threads) stages the block's products from its runs
//   into LDS at their CSR positions, then sums each row: rows of at most kSeqRow nonzeros one lane each, sequentially in
//   index order (0.0f + p_0 + p_1 + ...: the reference's float32 row sum bit for bit), longer rows
//   by the whole wave (lane k adds products k, k + 64, ... in order, then a fixed DPP tree); giant
//   rows the same way with their products formed from x directly.
// Both passes stream; only the LDS gathers are random. The analysis (block bounds, per-(slice,
// block) counts, their scans, the scatter) runs on the device, once per plan.
// =============================================================================================
constexpr int kTileCols = 32768;          // widest slice: a 128 KB x tile
constexpr int kMinTileCols = 4096;        // narrowest default slice
constexpr int kSpanBig = 8192;            // block span (nonzeros) of large matrices; small ones
constexpr int kSpanSmall = 4096;          // take half, with row-pass workgroups of half the size
constexpr int kBlockRows = 16384;
constexpr int kStage = 2 * kSpanBig;      // most products of a block's rows other than a giant one
constexpr int kSeqRow = 32;               // rows up to this length are summed by one lane
constexpr int kPass = 1024;               // threads per workgroup of the plan kernels
constexpr int kPassWaves = kPass / 64;
constexpr int kMaxSlices = 32768;         // (1 << 30) columns / kTileCols
constexpr int kPad = 8;                   // slice regions start at multiples of 8 entries
constexpr int kScatterRuns = 1024;            // below this many slices, the scatter stages through LDS
constexpr int kRowPre = 2;                // row pass: row steps whose bounds are loaded before staging
constexpr int kXcds = 8;

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
__device__ inline int32_t clamp_nz(int32_t v, int32_t nnz) { return min(max(v, 0), nnz); }

// Blocks are handed to workgroups XCD by XCD: workgroup w (on XCD w % 8) takes block
// (w % 8) * per + w / 8, so each XCD works through one contiguous range of blocks, and the cache
// lines that neighbouring blocks' runs share are fetched into one L2. -1: no block for w (the grid
// is 8 * per).
__device__ inline int32_t xcd_block(int32_t nblocks) {
  const int32_t per = (nblocks + kXcds - 1) / kXcds;
  const int32_t b = (int32_t)(blockIdx.x % kXcds) * per + (int32_t)(blockIdx.x / kXcds);
  return b < nblocks ? b : -1;
}

// Sequential sum of p[i0..i1) (index order), LDS reads eight, then four at a time.
__device__ inline float lds_seq_sum(const float* __restrict__ p, int32_t i0, int32_t i1) {
  float sum = 0.0f;
  int32_t i = i0;
  for (; i + 8 <= i1; i += 8) {
    float a[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) a[u] = p[i + u];
#pragma unroll
    for (int u = 0; u < 8; ++u) sum += a[u];
  }
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

// Exclusive prefix sum of a[0..n) in place (global or LDS) by one kPass-thread workgroup; returns
// the total to every thread. Called by every thread of the workgroup.
__device__ int32_t block_scan_inplace(int32_t* a, int32_t n, int32_t* wsum) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  int32_t carry = 0;
  for (int32_t base = 0; base < n; base += 4 * kPass) {
    int32_t v[4], sum = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int32_t i = base + 4 * t + k;
      v[k] = i < n ? a[i] : 0;
      sum += v[k];
    }
    const int32_t incl = wave_incl_scan(sum);
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int32_t pre = carry, tot = 0;
#pragma unroll
    for (int w = 0; w < kPassWaves; ++w) {
      const int32_t x = wsum[w];
      if (w < wave) pre += x;
      tot += x;
    }
    pre += incl - sum;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int32_t i = base + 4 * t + k;
      if (i < n) a[i] = pre;
      pre += v[k];
    }
    carry += tot;
    __syncthreads();
  }
  return carry;
}

__device__ inline int64_t block_of(int32_t start, int32_t nnz, int64_t r, int32_t span) {
  return (int64_t)clamp_nz(start, nnz) / span + r / kBlockRows;
}

// Rows [r0, r1) of block b; its nonzeros other than a giant row's are [j0, j1), the giant row's
// (if any) [j1, jg). A consistent matrix has j1 - j0 < 2 span; the clamp keeps a malformed one's
// positions inside the stage (its results are then meaningless, but every access stays in range).
// The plan keeps them per block (binfo: two int4 per block), so a pass reads them in one load.
struct BlockRange {
  int32_t r0, r1, j0, j1, jg;
};
__device__ inline BlockRange load_block(const int4* __restrict__ binfo, int32_t b) {
  const int4 a = binfo[2 * b], c = binfo[2 * b + 1];
  return BlockRange{a.x, a.y, a.z, a.w, c.x};
}

// A1: first row of each block (blk_row[nblocks] = rows): thread r compares row r's block with
// row r - 1's and writes the blocks that start at r (one thread per row, no search).
__global__ __launch_bounds__(256) void plan_blocks(const int32_t* __restrict__ rp, int64_t rows, int32_t nnz,
                                                   int32_t nblocks, int32_t span, int32_t* __restrict__ blk_row) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r > rows) return;
  const int64_t here = r < rows ? min(block_of(rp[r], nnz, r, span), (int64_t)nblocks - 1) : (int64_t)nblocks;
  const int64_t prev = r > 0 ? min(block_of(rp[r - 1], nnz, r - 1, span), (int64_t)nblocks - 1) : -1;
  for (int64_t k = max(prev, (int64_t)-1) + 1; k <= here; ++k) blk_row[k] = (int32_t)r;
}

// A1b: the bounds of each block (BlockRange) from blk_row and the row pointers.
// Row bounds are clamped into [0, rows]: with row pointers that are not monotone some blk_row
// entries are never written, and the passes must still stay in range.
__global__ __launch_bounds__(256) void plan_block_info(const int32_t* __restrict__ rp, int32_t rows, int32_t nnz,
                                                       const int32_t* __restrict__ blk_row, int32_t nblocks,
                                                       int32_t span, int4* __restrict__ binfo) {
  const int32_t b = (int32_t)(blockIdx.x * 256 + threadIdx.x);
  if (b >= nblocks) return;
  BlockRange g;
  g.r0 = min(max(blk_row[b], 0), rows);
  g.r1 = min(max(blk_row[b + 1], g.r0), rows);
  g.j0 = g.r0 < g.r1 ? clamp_nz(rp[g.r0], nnz) : 0;
  g.j1 = g.jg = g.j0;
  if (g.r0 < g.r1) {
    const int32_t last = max(clamp_nz(rp[g.r1 - 1], nnz), g.j0), end = max(clamp_nz(rp[g.r1], nnz), last);
    const bool giant = end - last > span;
    g.j1 = min(giant ? last : end, g.j0 + 2 * span);
    g.jg = giant ? end : g.j1;
  }
  binfo[2 * b] = make_int4(g.r0, g.r1, g.j0, g.j1);
  binfo[2 * b + 1] = make_int4(g.jg, 0, 0, 0);
}

// A2: tcnt[s][b] = nonzeros of block b in slice s (s < S), and of its giant row (s = S). SMAX >= S + 1
// sizes the LDS histogram.
template <int SMAX>
__global__ __launch_bounds__(kPass) void plan_tile_count(const int32_t* __restrict__ col,
                                                         const int4* __restrict__ binfo, int32_t nblocks, int32_t S,
                                                         uint32_t width, uint32_t cols, int32_t* __restrict__ tcnt) {
  __shared__ int32_t hist[SMAX];
  const int32_t b = xcd_block(nblocks);
  if (b < 0) return;  // whole workgroup
  const int t = threadIdx.x;
  for (int s = t; s <= S; s += kPass) hist[s] = 0;
  __syncthreads();
  const BlockRange g = load_block(binfo, b);
  for (int32_t j0 = g.j0 + t; j0 < g.j1; j0 += 4 * kPass) {
    int32_t c[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) c[u] = j0 + u * kPass < g.j1 ? col[j0 + u * kPass] : 0;
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (j0 + u * kPass < g.j1) atomicAdd(&hist[clamp_col(c[u], cols) / width], 1);
  }
  if (t == 0) hist[S] += g.jg - g.j1;
  __syncthreads();
  for (int s = t; s <= S; s += kPass) tcnt[(int64_t)s * nblocks + b] = hist[s];
}

// A3: workgroup s turns row s of tcnt into run offsets within the slice (exclusive prefix over
// blocks); tot[s] = the slice's total.
__global__ __launch_bounds__(kPass) void plan_tile_scan(int32_t* __restrict__ tcnt, int32_t nblocks,
                                                        int32_t* __restrict__ tot) {
  __shared__ int32_t wsum[kPassWaves];
  const int32_t total = block_scan_inplace(tcnt + (int64_t)blockIdx.x * nblocks, nblocks, wsum);
  if (threadIdx.x == 0) tot[blockIdx.x] = total;
}

// A4 (one workgroup): region starts sbase[0..S+1] (each slice region rounded up to whole groups of
// kPad entries; the giant region S last), the padding entries (column 0, value 0), and the share of
// each of the nwg product-pass workgroups: wrange[w] = {first entry, end, slice of the first entry}
// (equal shares of whole kPad-entry groups of the slice regions [0, sbase[S])).
__global__ __launch_bounds__(kPass) void plan_tile_bases(const int32_t* __restrict__ tot, int32_t S,
                                                         int32_t* __restrict__ sbase, uint16_t* __restrict__ col16,
                                                         uint16_t* __restrict__ dest16, float* __restrict__ val_s,
                                                         int32_t nwg, int4* __restrict__ wrange) {
  __shared__ int32_t wsum[kPassWaves];
  for (int s = threadIdx.x; s <= S; s += kPass) sbase[s] = (tot[s] + kPad - 1) & ~(kPad - 1);
  __syncthreads();
  const int32_t total = block_scan_inplace(sbase, S + 1, wsum);
  if (threadIdx.x == 0) sbase[S + 1] = total;
  __syncthreads();
  for (int s = threadIdx.x; s <= S; s += kPass)
    for (int32_t i = sbase[s] + tot[s]; i < sbase[s + 1]; ++i) {
      col16[i] = 0;
      dest16[i] = 0;
      val_s[i] = 0.0f;
    }
  const int32_t Z = sbase[S];
  const int64_t per = ((int64_t)(Z + nwg - 1) / nwg + kPad - 1) & ~(int64_t)(kPad - 1);
  for (int w = threadIdx.x; w < nwg; w += kPass) {
    const int32_t lo = (int32_t)min((int64_t)w * per, (int64_t)Z);
    const int32_t hi = (int32_t)min((int64_t)lo + per, (int64_t)Z);
    int32_t a = 0, z = S - 1;  // last slice whose region starts at or before lo
    while (a < z) {
      const int32_t m = (a + z + 1) >> 1;
      if (sbase[m] <= lo) a = m; else z = m - 1;
    }
    wrange[w] = make_int4(lo, hi, a, 0);
  }
}

// A5: the scatter. Run (b, s) starts at toff[b][s] = sbase[s] + its offset within the slice
// (toff[nblocks][s] = the slice's end). A giant row's entries go to region S in CSR order, column
// low half in col16 and high half in dest16. With kStaged (S < kScatterRuns), the block's entries are
// first sorted by slice in LDS (the order within a slice is that of LDS atomics, which the results
// do not depend on: every product is staged at its CSR position), then written out with the
// threads on consecutive local positions li: the run holding li is first_k[li / 64] plus the run
// starts in (64 (li / 64), li] (a bitmap of run starts), and nz_gb of that run maps li to its global
// position; otherwise each entry is written where its atomic cursor lands.
template <int SMAX, bool kStaged, int STAGE = kStage>
__global__ __launch_bounds__(kPass) void plan_tile_scatter(
    const int32_t* __restrict__ col, const float* __restrict__ val, const int4* __restrict__ binfo,
    int32_t nblocks, int32_t S, uint32_t width, uint32_t cols, const int32_t* __restrict__ tcnt,
    const int32_t* __restrict__ tot, const int32_t* __restrict__ sbase, int32_t* __restrict__ toff,
    uint16_t* __restrict__ col16, float* __restrict__ val_s, uint16_t* __restrict__ dest16) {
  __shared__ int32_t cur[SMAX];
  __shared__ int32_t nz_gb[kStaged ? SMAX : 1];              // k-th non-empty run: global base - local start
  __shared__ uint32_t starts[kStaged ? STAGE / 32 : 1];     // bit li: a non-empty run starts at li
  __shared__ int32_t first_k[kStaged ? STAGE / 64 : 1];     // the run holding local position 64c
  __shared__ uint32_t st_cd[kStaged ? STAGE : 1];
  __shared__ float st_v[kStaged ? STAGE : 1];
  __shared__ int32_t wsum[kPassWaves];
  __shared__ int32_t wcnt[kPassWaves];
  const int32_t b = xcd_block(nblocks);
  if (b < 0) return;  // whole workgroup
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int32_t S1 = S + 1;
  int32_t n = 0;  // kStaged: thread t's run length (t < S)
  if constexpr (kStaged)
    for (int i = t; i < STAGE / 32; i += kPass) starts[i] = 0;
  for (int s = t; s <= S; s += kPass) {
    const int32_t o = sbase[s] + tcnt[(int64_t)s * nblocks + b];
    const int32_t next = b + 1 < nblocks ? sbase[s] + tcnt[(int64_t)s * nblocks + b + 1] : sbase[s] + tot[s];
    cur[s] = o;
    toff[(int64_t)b * S1 + s] = o;
    if (b == nblocks - 1) toff[(int64_t)nblocks * S1 + s] = next;
    if (kStaged && s == t && s < S) n = next - o;
  }
  const BlockRange g = load_block(binfo, b);
  int32_t E = 0;
  if constexpr (kStaged) {
    // local slice-major numbering: thread t (run t) takes its first local position from a scan
    static_assert(SMAX <= kPass, "one thread per run");
    const int32_t incl = wave_incl_scan(n);
    const uint64_t ne = __ballot(n > 0);
    if (lane == 63) {
      wsum[wave] = incl;
      wcnt[wave] = __builtin_popcountll(ne);
    }
    __syncthreads();
    int32_t pre = incl - n;
    int32_t k = __builtin_popcountll(ne & ((1ull << lane) - 1));  // non-empty runs before run t
#pragma unroll
    for (int w = 0; w < kPassWaves; ++w) {
      const int32_t v = wsum[w];
      if (w < wave) {
        pre += v;
        k += wcnt[w];
      }
      E += v;
    }
    E = min(E, STAGE);
    if (t < S) {
      if (n > 0 && pre < STAGE) {
        nz_gb[k] = cur[t] - pre;  // local position li of run t goes to nz_gb[k] + li
        atomicOr(&starts[pre >> 5], 1u << (pre & 31));
        for (int32_t c = (pre + 63) >> 6; c < STAGE / 64 && (c << 6) < pre + n; ++c) first_k[c] = k;
      }
      cur[t] = pre;
    }
  }
  __syncthreads();
  for (int32_t j0 = g.j0 + t; j0 < g.j1; j0 += 4 * kPass) {
    int32_t c[4];
    float v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int32_t j = j0 + u * kPass;
      c[u] = j < g.j1 ? col[j] : 0;
      v[u] = j < g.j1 ? val[j] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int32_t j = j0 + u * kPass;
      if (j < g.j1) {
        const uint32_t cc = clamp_col(c[u], cols), s = cc / width;
        const int32_t pos = atomicAdd(&cur[s], 1);
        if constexpr (kStaged) {
          if (pos < STAGE) {
            st_cd[pos] = (cc - s * width) | ((uint32_t)(j - g.j0) << 16);
            st_v[pos] = v[u];
          }
        } else {
          col16[pos] = (uint16_t)(cc - s * width);
          val_s[pos] = v[u];
          dest16[pos] = (uint16_t)(j - g.j0);
        }
      }
    }
  }
  __syncthreads();
  if constexpr (kStaged) {
    for (int32_t li = t; li < E; li += kPass) {
      const int32_t c = li >> 6;
      const uint64_t word = (uint64_t)starts[2 * c] | ((uint64_t)starts[2 * c + 1] << 32);
      const uint64_t below = (2ull << lane) - 1;  // bits 0..lane (lane 63: all)
      const int32_t k = first_k[c] + __builtin_popcountll(word & below & ~1ull);
      const int32_t dst = nz_gb[k] + li;
      const uint32_t cd = st_cd[li];
      col16[dst] = (uint16_t)(cd & 0xFFFFu);
      dest16[dst] = (uint16_t)(cd >> 16);
      val_s[dst] = st_v[li];
    }
  }
  const int32_t gpos = cur[S];  // the giant row's run (no atomic moves cur[S])
  for (int32_t j = g.j1 + t; j < g.jg; j += kPass) {
    const uint32_t cc = clamp_col(col[j], cols);
    col16[gpos + (j - g.j1)] = (uint16_t)(cc & 0xFFFFu);
    dest16[gpos + (j - g.j1)] = (uint16_t)(cc >> 16);
    val_s[gpos + (j - g.j1)] = val[j];
  }
}

// A6 (table path of the row pass): per block, each run's local start (the block's runs numbered
// slice by slice; below 2 * span, so 16 bits) and the block's total in entry S.
__global__ __launch_bounds__(kPass) void plan_run_tables(const int32_t* __restrict__ toff, int32_t nblocks, int32_t S,
                                                         uint16_t* __restrict__ rpre) {
  __shared__ int32_t wsum[kPassWaves];
  const int32_t b = xcd_block(nblocks);
  if (b < 0) return;  // whole workgroup
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int32_t S1 = S + 1;
  int32_t o = 0, n = 0;
  if (t < S) {
    o = toff[(int64_t)b * S1 + t];
    n = toff[(int64_t)(b + 1) * S1 + t] - o;
  }
  const int32_t incl = wave_incl_scan(n);
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  int32_t pre = incl - n, E = 0;
#pragma unroll
  for (int w = 0; w < kPassWaves; ++w) {
    const int32_t v = wsum[w];
    if (w < wave) pre += v;
    E += v;
  }
  uint16_t* row = rpre + (int64_t)b * S1;
  if (t < S) row[t] = (uint16_t)min(pre, 65535);
  if (t == 0) row[S] = (uint16_t)min(E, 65535);
}

// Product pass: p[i] = val_s[i] * x_tile[col16[i]] over the slice regions [0, sbase[S]). Workgroup
// w takes the share wrange[w] (equal shares of whole kPad-entry groups); at each slice its share
// enters it loads that slice's x tile into LDS (16 waves, 8 loads in flight per lane). With
// sum_out, workgroup 0 first adds sums_in[0..nsums) in a fixed order (the power iteration's
// previous L1 norm).
__global__ __launch_bounds__(kPass) void spmv_tile_products(const uint16_t* __restrict__ col16,
                                                            const float* __restrict__ val_s,
                                                            const int32_t* __restrict__ sbase,
                                                            const int4* __restrict__ wrange, uint32_t width,
                                                            const float* __restrict__ x, uint32_t cols,
                                                            float* __restrict__ p, const double* __restrict__ sums_in,
                                                            int32_t nsums, double* __restrict__ sum_out) {
  __shared__ float xt[kTileCols];
  __shared__ double red[kPassWaves];
  const int t = threadIdx.x;
  if (sum_out && blockIdx.x == 0) {
    double a = 0.0;
    for (int32_t i0 = t; i0 < nsums; i0 += 8 * kPass) {
      double v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = i0 + k * kPass < nsums ? sums_in[i0 + k * kPass] : 0.0;
#pragma unroll
      for (int k = 0; k < 8; ++k) a += v[k];
    }
    const double total = dc::block_sum64<kPass>(a, red);
    if (t == 0) *sum_out = total;
  }
  const int4 wr = wrange[blockIdx.x];
  int32_t lo = wr.x, s = wr.z;
  const int32_t hi = wr.y;
  for (; lo < hi; ++s) {
    const int32_t e = min(hi, sbase[s + 1]);
    if (lo >= e) continue;  // workgroup-uniform
    __syncthreads();        // the previous tile's readers are done
    const uint32_t c0 = (uint32_t)s * width;
    const int32_t tw = (int32_t)min(width, cols - c0);
    const auto rx = dc::range_rsrc(x + c0, tw * 4);
    for (int32_t cb = 0; cb < tw; cb += 8 * kPass) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        v[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rx, (uint32_t)(cb + u * kPass + t) * 4u, 0, 0));
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (cb + u * kPass + t < kTileCols) xt[cb + u * kPass + t] = v[u];
    }
    __syncthreads();
    for (int32_t i = lo + kPad * t; i < e; i += 2 * kPad * kPass) {
      const int32_t i2 = i + kPad * kPass;
      const bool two = i2 < e;
      const dc::i32x4 c1 = __builtin_nontemporal_load(reinterpret_cast<const dc::i32x4*>(col16 + i));
      const dc::f32x4 a1 = __builtin_nontemporal_load(reinterpret_cast<const dc::f32x4*>(val_s + i));
      const dc::f32x4 b1 = __builtin_nontemporal_load(reinterpret_cast<const dc::f32x4*>(val_s + i + 4));
      dc::i32x4 c2 = {0, 0, 0, 0};
      dc::f32x4 a2 = {0.0f, 0.0f, 0.0f, 0.0f}, b2 = a2;
      if (two) {
        c2 = __builtin_nontemporal_load(reinterpret_cast<const dc::i32x4*>(col16 + i2));
        a2 = __builtin_nontemporal_load(reinterpret_cast<const dc::f32x4*>(val_s + i2));
        b2 = __builtin_nontemporal_load(reinterpret_cast<const dc::f32x4*>(val_s + i2 + 4));
      }
      auto lo16 = [](int32_t w) { return (uint32_t)w & 0xFFFFu; };
      auto hi16 = [](int32_t w) { return (uint32_t)w >> 16; };
      const dc::f32x4 p1a = {a1.x * xt[lo16(c1.x)], a1.y * xt[hi16(c1.x)], a1.z * xt[lo16(c1.y)], a1.w * xt[hi16(c1.y)]};
      const dc::f32x4 p1b = {b1.x * xt[lo16(c1.z)], b1.y * xt[hi16(c1.z)], b1.z * xt[lo16(c1.w)], b1.w * xt[hi16(c1.w)]};
      *reinterpret_cast<dc::f32x4*>(p + i) = p1a;
      *reinterpret_cast<dc::f32x4*>(p + i + 4) = p1b;
      if (two) {
        const dc::f32x4 p2a = {a2.x * xt[lo16(c2.x)], a2.y * xt[hi16(c2.x)], a2.z * xt[lo16(c2.y)], a2.w * xt[hi16(c2.y)]};
        const dc::f32x4 p2b = {b2.x * xt[lo16(c2.z)], b2.y * xt[hi16(c2.z)], b2.z * xt[lo16(c2.w)], b2.w * xt[hi16(c2.w)]};
        *reinterpret_cast<dc::f32x4*>(p + i2) = p2a;
        *reinterpret_cast<dc::f32x4*>(p + i2 + 4) = p2b;
      }
    }
    lo = e;
  }
}

// Row pass, a workgroup of SPAN / 8 threads per block (XCD-contiguous; 8 B of LDS per span
// nonzero: two workgroups per CU with span 8192, four with 4096). With kTable (S <= SPAN / 8)
// the staging is one round trip: the block's run lengths go to LDS, a prefix
// over them numbers its products in slice-major order, every product's run is written to a table
// (held in the stage buffer until the products arrive), and thread t loads products t, t + kPass,
// ... before writing any of them to their CSR positions. Without it (more slices), a wave stages
// whole runs. The bounds of the first kRowPre row steps are loaded before the staging. Then the
// rows, a lane per row, 64 consecutive rows per wave step. With `scale`, y = (float)((double)row
// sum / *scale) (the power iteration's previous normalisation moved onto this product); with
// block_sums, the block's float64 sum of y in a fixed order.
template <bool kTable, int SPAN>
__global__ __launch_bounds__(SPAN / 8) void spmv_tile_rows(
    const int32_t* __restrict__ rp, int32_t nnz, const int4* __restrict__ binfo, int32_t nblocks,
    const int32_t* __restrict__ toff, const uint16_t* __restrict__ rpre, int32_t S, const float* __restrict__ p,
    const uint16_t* __restrict__ dest16,
    const uint16_t* __restrict__ col16, const float* __restrict__ val_s, const float* __restrict__ x, uint32_t cols,
    float* __restrict__ y, double* __restrict__ block_sums, const double* __restrict__ scale, uint32_t pbytes) {
  constexpr int kThreads = SPAN / 8, kWaves = kThreads / 64, kSt = 2 * SPAN;  // kSt: stage entries
  __shared__ float stage[kSt];
  __shared__ int32_t run_base[kTable ? kThreads : 1];
  __shared__ double red[kWaves];
  const int32_t b = xcd_block(nblocks);
  if (b < 0) return;  // whole workgroup
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int32_t S1 = S + 1;
  const int32_t* t0 = toff + (int64_t)b * S1;
  const int32_t* t1 = t0 + S1;
  const BlockRange g = load_block(binfo, b);
  int32_t pb[kRowPre], pe[kRowPre];  // bounds of the rows of the first kRowPre row steps
#pragma unroll
  for (int k = 0; k < kRowPre; ++k) {
    const int32_t r = g.r0 + wave * 64 + lane + k * kThreads;
    pb[k] = r < g.r1 ? rp[r] : 0;
    pe[k] = r < g.r1 ? rp[r + 1] : 0;
  }
  if constexpr (kTable) {
    // thread t holds run t (S <= kThreads): its offsets from the two rows of run offsets it shares
    // with the neighbouring blocks, and its local start, precomputed once per plan by
    // plan_run_tables; it writes its products' entries of the run table
    const uint16_t* rt = rpre + (int64_t)b * S1;
    int32_t pre = 0, n = 0;
    if (t < S) {
      const int32_t o = t0[t];
      pre = rt[t];
      n = t1[t] - o;
      run_base[t] = o - pre;  // product li of run t is at run_base[t] + li
    }
    const int32_t E = min((int32_t)rt[S], kSt);
    int16_t* run_of = reinterpret_cast<int16_t*>(stage);  // kSt int16 fit in half the stage
    if (S <= kWaves) {
      // Few runs (a matrix of few columns, one or two x slices): one lane per run would write up
      // to E entries alone while the workgroup waits; the whole workgroup fills each run instead.
      for (int32_t s = 0; s < S; ++s) {
        const int32_t ps = rt[s], pe = min(ps + (t1[s] - t0[s]), E);
        for (int32_t li = ps + t; li < pe; li += kThreads) run_of[li] = (int16_t)s;
      }
    } else {
      for (int32_t li = pre; li < min(pre + n, E); ++li) run_of[li] = (int16_t)t;
    }
    __syncthreads();
    constexpr int kIt = kSt / kThreads;
    const int32_t nit = (E + kThreads - 1) / kThreads;
    float pv[kIt];
    uint32_t dv[kIt];
    // buffer loads: 32-bit offsets on a scalar base (the plan keeps p below 4 GiB for this path)
    const auto rp4 = dc::range_rsrc(p, (int32_t)(uint32_t)(pbytes));
    const auto rd2 = dc::range_rsrc(dest16, (int32_t)(uint32_t)(pbytes / 2));
#pragma unroll
    for (int k = 0; k < kIt; ++k) {
      pv[k] = 0.0f;
      dv[k] = kSt;
      const int32_t li = t + k * kThreads;
      if (k < nit && li < E) {
        const uint32_t at = (uint32_t)(run_base[run_of[li]] + li);
        pv[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rp4, at * 4u, 0, 0));
        dv[k] = __builtin_amdgcn_raw_buffer_load_b16(rd2, at * 2u, 0, 0);
      }
    }
    __syncthreads();  // every run_of read is done before the stage is overwritten
#pragma unroll
    for (int k = 0; k < kIt; ++k)
      if (k < nit && dv[k] < (uint32_t)kSt) stage[dv[k]] = pv[k];
  } else {
    for (int s = wave; s < S; s += kWaves) {
      const int32_t o = t0[s], n = t1[s] - o;
      for (int32_t k = lane; k < n; k += 64) {
        const uint32_t d = dest16[o + k];
        if (d < (uint32_t)kSt) stage[d] = p[o + k];
      }
    }
  }
  __syncthreads();
  const int32_t gpos = t0[S];  // the giant row's entries (region S, CSR order)
  double dsum = 0.0;
  int it = 0;
  for (int32_t rr = g.r0 + wave * 64; rr < g.r1; rr += kThreads, ++it) {  // wave-uniform
    const int32_t r = rr + lane;
    const bool in = r < g.r1;
    int32_t rb = 0, re = 0;
    if (in) {
      static_assert(kRowPre == 2, "the prefetched bounds are picked by two selects");
      const int32_t lb = it == 0 ? pb[0] : it == 1 ? pb[1] : rp[r];
      const int32_t le = it == 0 ? pe[0] : it == 1 ? pe[1] : rp[r + 1];
      rb = min(max(clamp_nz(lb, nnz), g.j0), g.jg);
      re = min(max(clamp_nz(le, nnz), rb), g.jg);
    }
    const int32_t d = re - rb;
    float acc = 0.0f;
    if (in && d <= kSeqRow) acc = lds_seq_sum(stage, rb - g.j0, min(re, g.j1) - g.j0);
    for (uint64_t m = __ballot(in && d > kSeqRow && re <= g.j1); m; m &= m - 1) {
      const int L = __builtin_ctzll(m);
      const int32_t lb = __builtin_amdgcn_readlane(rb, L) - g.j0, le = __builtin_amdgcn_readlane(re, L) - g.j0;
      float tt = 0.0f;
      for (int32_t i = lb + lane; i < le; i += 64) tt += stage[i];
      const float tw = wave_sum_f32(tt);
      if (lane == L) acc = tw;
    }
    for (uint64_t m = __ballot(in && d > kSeqRow && re > g.j1); m; m &= m - 1) {  // the giant row
      const int L = __builtin_ctzll(m);
      const int32_t gb = max(__builtin_amdgcn_readlane(rb, L) - g.j1, 0);
      const int32_t ge = __builtin_amdgcn_readlane(re, L) - g.j1;
      float tt = 0.0f;
      for (int32_t i = gb + lane; i < ge; i += 64) {
        const uint32_t c = (uint32_t)col16[gpos + i] | ((uint32_t)dest16[gpos + i] << 16);
        tt += __fmul_rn(val_s[gpos + i], x[min(c, cols - 1)]);
      }
      const float tw = wave_sum_f32(tt);
      if (lane == L) acc = tw;
    }
    if (scale) acc = (float)((double)acc / *scale);
    if (in) {
      y[r] = acc;
      dsum += (double)acc;
    }
  }
  if (block_sums) {
    const double tsum = dc::block_sum64<kThreads>(dsum, red);
    if (t == 0) block_sums[b] = tsum;
  }
}

}  // namespace

// Device memory of a plan, carved from one allocation.
struct dc_hip_spmv_plan {
  int device = 0;
  int64_t rows = 0, cols = 0, nnz = 0;
  int32_t slices = 1;
  int64_t slice_cols = 1;
  int32_t nblocks = 1;
  int64_t zcap = 0;
  bool owns_mem = false;
  void* mem = nullptr;
  size_t bytes = 0;
  uint16_t *col16 = nullptr, *dest16 = nullptr;
  float *val_s = nullptr, *p = nullptr;
  int32_t *rp = nullptr, *tcnt = nullptr, *toff = nullptr, *tot = nullptr, *sbase = nullptr, *blk_row = nullptr;
  int4 *binfo = nullptr, *wrange = nullptr;
  uint16_t* rpre = nullptr;  // per (block, run): the run's local start; run S: the block's total
  int32_t span = kSpanBig;  // block span in nonzeros
  int32_t nwg = 1;  // product-pass workgroups (one per CU)
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
  const size_t z = (size_t)p->zcap, S1 = (size_t)p->slices + 1, nb = (size_t)p->nblocks;
  p->col16 = reinterpret_cast<uint16_t*>(take(z * 2));
  p->dest16 = reinterpret_cast<uint16_t*>(take(z * 2));
  p->val_s = reinterpret_cast<float*>(take(z * 4));
  p->p = reinterpret_cast<float*>(take(z * 4));
  p->rp = reinterpret_cast<int32_t*>(take((size_t)(p->rows + 1) * 4));
  p->tcnt = reinterpret_cast<int32_t*>(take(S1 * nb * 4));
  p->toff = reinterpret_cast<int32_t*>(take(S1 * (nb + 1) * 4));
  p->tot = reinterpret_cast<int32_t*>(take(S1 * 4));
  p->sbase = reinterpret_cast<int32_t*>(take((S1 + 1) * 4));
  p->blk_row = reinterpret_cast<int32_t*>(take((nb + 1) * 4));
  p->binfo = reinterpret_cast<int4*>(take(nb * 32));
  p->rpre = reinterpret_cast<uint16_t*>(take(S1 * nb * 2));
  p->wrange = reinterpret_cast<int4*>(take((size_t)p->nwg * 16));
  p->block_sums = reinterpret_cast<double*>(take(nb * 8));
  p->scalars = reinterpret_cast<double*>(take(8 * 8));
  p->mem = mem;
  p->bytes = off;
}

// Shape of the plan (slices, blocks, sizes) and the bytes it needs.
int32_t plan_shape(dc_hip_spmv_plan* p, int64_t rows, int64_t cols, int64_t nnz, int64_t slice_cols_max,
                   int cu_count) {
  p->rows = rows;
  p->nwg = std::max(1, cu_count);
  p->cols = cols;
  p->nnz = nnz;
  // Blocks of 8192 nonzeros, or of 4096 when that still gives fewer than four blocks per CU:
  // row-pass workgroups of half the size, four per CU, hide more of each block's two round trips
  // (1M rows of 5.4 nonzeros: row pass 19.6 against 22.5 us; at 16M rows both spans take the same
  // time and the larger one halves the plan's per-block tables and scatter work).
  const int64_t rows_term = rows > 0 ? (rows - 1) / kBlockRows : 0;
  p->span = nnz / kSpanBig + rows_term + 1 < 4 * (int64_t)p->nwg ? kSpanSmall : kSpanBig;
  int64_t W;
  if (slice_cols_max > 0) {
    W = std::min<int64_t>(slice_cols_max, kTileCols);
  } else {
    // Default: every product-pass workgroup loads the x tile of each slice its share touches, so
    // the tiles cost about nwg * 4 W bytes per SpMV against 10 bytes per nonzero streamed. The
    // widest power of two up to kTileCols with W <= nnz / (2 nwg) keeps the tiles a small share
    // (at 1M rows of 5.4 nonzeros on 256 CUs: 8192 columns, 39.0 us per power step against 42.3
    // with 32768), but no narrower than kMinTileCols and wide enough for the row pass's LDS
    // tables (at most span / 8 slices) while that is possible.
    W = kMinTileCols;
    const int64_t want = nnz / (2 * (int64_t)p->nwg);
    while (W < kTileCols && (2 * W <= want || (cols + W - 1) / W > p->span / 8)) W *= 2;
  }
  if ((cols + W - 1) / W > kMaxSlices) W = (cols + kMaxSlices - 1) / kMaxSlices;
  const int64_t S = std::max<int64_t>(1, (cols + W - 1) / W);
  p->slices = (int32_t)S;
  p->slice_cols = W;
  p->nblocks = (int32_t)(nnz / p->span + rows_term + 1);
  p->zcap = nnz + (S + 1) * kPad + kPad;
  // positions are int32 and the (slice, block) tables are indexed with int32 products of their sides
  if (p->zcap > INT32_MAX || (S + 1) * (int64_t)(p->nblocks + 1) > (int64_t{1} << 29)) return DC_ERR_UNSUPPORTED;
  plan_layout(p, nullptr);
  return DC_OK;
}

// The analysis kernels, on the context stream.
int32_t plan_build(dc_hip_ctx* ctx, dc_hip_spmv_plan* p, const int32_t* rp, const int32_t* col, const float* val) {
  if (p->rows == 0) return DC_OK;
  const int32_t S = p->slices, nb = p->nblocks, nnz = (int32_t)p->nnz;
  const uint32_t width = (uint32_t)p->slice_cols, cols = (uint32_t)std::max<int64_t>(p->cols, 1);
  DC_RETURN_IF_HIP(hipMemcpyAsync(p->rp, rp, (size_t)(p->rows + 1) * 4, hipMemcpyDeviceToDevice, ctx->stream));
  plan_blocks<<<(unsigned)((p->rows + 1 + 255) / 256), 256, 0, ctx->stream>>>(p->rp, p->rows, nnz, nb, p->span,
                                                                               p->blk_row);
  DC_RETURN_IF(dc::last_launch_status());
  plan_block_info<<<(unsigned)((nb + 255) / 256), 256, 0, ctx->stream>>>(p->rp, (int32_t)p->rows, nnz, p->blk_row,
                                                                         nb, p->span, p->binfo);
  DC_RETURN_IF(dc::last_launch_status());
  const unsigned bgrid = (unsigned)(kXcds * ((nb + kXcds - 1) / kXcds));
#define DC_TILE_COUNT(SM)                                                                                   \
  plan_tile_count<SM><<<bgrid, kPass, 0, ctx->stream>>>(col, p->binfo, nb, S, width, cols, p->tcnt)
  if (S + 1 <= 1024) DC_TILE_COUNT(1024);
  else if (S + 1 <= 8192) DC_TILE_COUNT(8192);
  else DC_TILE_COUNT(kMaxSlices + 8);
#undef DC_TILE_COUNT
  DC_RETURN_IF(dc::last_launch_status());
  plan_tile_scan<<<(unsigned)(S + 1), kPass, 0, ctx->stream>>>(p->tcnt, nb, p->tot);
  DC_RETURN_IF(dc::last_launch_status());
  plan_tile_bases<<<1, kPass, 0, ctx->stream>>>(p->tot, S, p->sbase, p->col16, p->dest16, p->val_s, p->nwg,
                                                p->wrange);
  DC_RETURN_IF(dc::last_launch_status());
#define DC_TILE_SCATTER(SM, ST, STG)                                                                          \
  plan_tile_scatter<SM, ST, STG><<<bgrid, kPass, 0, ctx->stream>>>(col, val, p->binfo, nb, S, width, cols, p->tcnt,  \
                                                                   p->tot, p->sbase, p->toff, p->col16, p->val_s,  \
                                                                   p->dest16)
  // staging sized for the block span (a block holds fewer than 2 * span entries besides a giant
  // row): 4096-entry spans stage in half the LDS, so two workgroups fit per CU
  if (S < kScatterRuns && p->span == kSpanSmall) DC_TILE_SCATTER(kScatterRuns, true, 2 * kSpanSmall);
  else if (S < kScatterRuns) DC_TILE_SCATTER(kScatterRuns, true, kStage);
  else if (S + 1 <= 8192) DC_TILE_SCATTER(8192, false, kStage);
  else DC_TILE_SCATTER(kMaxSlices + 8, false, kStage);
#undef DC_TILE_SCATTER
  DC_RETURN_IF(dc::last_launch_status());
  if (S <= p->span / 8 && S <= kPass)  // the row pass's table path reads the run tables
    plan_run_tables<<<bgrid, kPass, 0, ctx->stream>>>(p->toff, nb, S, p->rpre);
  return dc::last_launch_status();
}

// One SpMV through the plan: y = A·x (with `sums`, also the per-block float64 sums of y). With
// `scale`, y = (A·x) / *scale. With `prev_sum_out`, *prev_sum_out = the sum of the block sums as
// they stand (the previous SpMV's), formed by the product pass before this SpMV's row pass
// replaces them, so it costs no launch of its own.
int32_t plan_spmv(dc_hip_ctx* ctx, const dc_hip_spmv_plan* p, const float* x, float* y, bool sums = false,
                  const double* scale = nullptr, double* prev_sum_out = nullptr) {
  if (p->rows == 0) return DC_OK;
  const uint32_t width = (uint32_t)p->slice_cols, cols = (uint32_t)std::max<int64_t>(p->cols, 1);
  spmv_tile_products<<<(unsigned)p->nwg, kPass, 0, ctx->stream>>>(
      p->col16, p->val_s, p->sbase, p->wrange, width, x, (uint32_t)p->cols, p->p, p->block_sums, p->nblocks,
      prev_sum_out);
  DC_RETURN_IF(dc::last_launch_status());
  const unsigned bgrid = (unsigned)(kXcds * ((p->nblocks + kXcds - 1) / kXcds));
  double* bs = sums ? p->block_sums : nullptr;
#define DC_TILE_ROWS(TABLE, SP)                                                                                 \
  spmv_tile_rows<TABLE, SP><<<bgrid, SP / 8, 0, ctx->stream>>>(p->rp, (int32_t)p->nnz, p->binfo, p->nblocks, p->toff, p->rpre, \
                                                               p->slices, p->p, p->dest16, p->col16, p->val_s, x,    \
                                                               cols, y, bs, scale, (uint32_t)(p->zcap * 4))
  // the table path addresses the products with 32-bit byte offsets
  const bool table = p->slices <= p->span / 8 && p->zcap * 4 <= (int64_t)UINT32_MAX;
  if (p->span == kSpanSmall) {
    if (table) DC_TILE_ROWS(true, kSpanSmall);
    else DC_TILE_ROWS(false, kSpanSmall);
  } else {
    if (table) DC_TILE_ROWS(true, kSpanBig);
    else DC_TILE_ROWS(false, kSpanBig);
  }
#undef DC_TILE_ROWS
  return dc::last_launch_status();
}

// y_k = A·x_k; s_k = Σ y_k; x_{k+1} = y_k / s_k. The division moves into the next step's row pass
// (y_{k+1} = (A·y_k) / s_k), so the unnormalised y_k is the next step's input as it stands and the
// buffers swap roles (x, y, x, ...); the last y is normalised into x once at the end. s_k is formed
// by step k + 1's product pass from step k's block sums, before step k + 1's row pass (which
// divides by it) overwrites them.
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

// One-shot y = A·x for any element type (the entry points dc_hip_spmv_csr_f32/_f64/_i32).
template <typename T>
int32_t spmv_csr(dc_hip_ctx* ctx, const int32_t* row_pointers, const int32_t* col_indices, const T* values, const T* x,
                 T* y, int64_t rows, int64_t cols, int64_t nnz) {
  DC_RETURN_IF(check_csr(row_pointers, col_indices, values, rows, nnz));
  if (cols < 0 || (rows > 0 && !y) || (cols > 0 && !x)) return DC_ERR_INVALID_ARGUMENT;
  DC_CTX_ENTER(ctx);
  if (rows == 0) return DC_OK;
  const SpmvPlan plan = make_plan(nnz);
  DC_RETURN_IF(launch_analysis(ctx, plan, row_pointers, rows));
  return launch_spmv(ctx, plan, row_pointers, col_indices, values, x, y, rows);
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
  return spmv_csr(ctx, row_pointers, col_indices, values, x, y, rows, cols, nnz);
}

DC_HIP_API int32_t dc_hip_spmv_csr_f64(dc_hip_ctx* ctx, const int32_t* row_pointers, const int32_t* col_indices,
                                       const double* values, const double* x, double* y, int64_t rows, int64_t cols,
                                       int64_t nnz) {
  return spmv_csr(ctx, row_pointers, col_indices, values, x, y, rows, cols, nnz);
}

DC_HIP_API int32_t dc_hip_spmv_csr_i32(dc_hip_ctx* ctx, const int32_t* row_pointers, const int32_t* col_indices,
                                       const int32_t* values, const int32_t* x, int32_t* y, int64_t rows, int64_t cols,
                                       int64_t nnz) {
  return spmv_csr(ctx, row_pointers, col_indices, values, x, y, rows, cols, nnz);
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
  const int32_t shape_st = plan_shape(p, rows, cols, nnz, slice_cols_max, ctx->cu_count);
  if (shape_st != DC_OK) {
    delete p;
    return shape_st;
  }
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
  DC_RETURN_IF(plan_shape(&p, rows, rows, nnz, 0, ctx->cu_count));
  DC_RETURN_IF(dc::ensure_spmv_plan_mem(ctx, p.bytes));
  plan_layout(&p, ctx->spmv_plan_mem);
  DC_RETURN_IF(plan_build(ctx, &p, row_pointers, col_indices, values));
  return plan_power_iterate(ctx, &p, x, y, iterations, last_sum_out);
}

}  // extern "C"

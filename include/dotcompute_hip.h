/*
 * dotcompute_hip.h — C ABI of libdotcompute_hip.so, the MI355X (gfx950) HIP backend of DotCompute.
 *
 * This is the boundary the managed backend (DotCompute.Backends.HIP, C#) binds with
 * [LibraryImport]; every other caller (the C++ host layer under dotcompute_amd/host, the Python
 * ctypes harness in dotcompute_amd/hip.py) goes through exactly the same symbols.
 *
 * Conventions
 *   - Every function returns int32_t: 0 (DC_OK) on success, a positive hipError_t value when a HIP
 *     runtime call failed, or one of the negative DC_ERR_* codes below. dc_hip_error_string()
 *     maps any of them to static text.
 *   - A context (dc_hip_ctx) is one device plus one in-order HIP stream plus the scratch memory the
 *     kernels need (lookback status words, tile tickets, partial sums). Calls on one context are
 *     serialised by a mutex inside the library; different contexts are independent.
 *   - Op entry points (dc_hip_vector_add_f32 … dc_hip_spmv_*) take DEVICE pointers, enqueue work on
 *     the context's stream and return without waiting (like cuLaunchKernel in the CUDA backend);
 *     their scalar results (sums, counts) are written to device memory. dc_hip_synchronize()
 *     waits for the stream, which is what the reference does after every launch.
 *   - Device memory is allocated by dc_hip_malloc and owned by the caller's buffer object, which
 *     must free it exactly once with dc_hip_free.
 *
 * Reference interfaces each group replaces are cited per declaration (paths relative to the
 * DotCompute repository root).
 */
#ifndef DOTCOMPUTE_HIP_H
#define DOTCOMPUTE_HIP_H

#ifndef __HIPCC_RTC__ /* the run-time compiler of LINQ programs provides these types itself */
#include <stddef.h>
#include <stdint.h>
#endif

#ifdef __cplusplus
extern "C" {
#endif

#if defined(_WIN32)
#define DC_HIP_API __declspec(dllexport)
#else
#define DC_HIP_API __attribute__((visibility("default")))
#endif

#define DC_HIP_ABI_VERSION 1

/* ---------------------------------------------------------------------------------------------
 * Status codes (replaces CudaError + CudaErrorClassification,
 * src/Backends/DotCompute.Backends.CUDA/ErrorHandling/CudaErrorClassification.cs:17)
 * ------------------------------------------------------------------------------------------- */
#define DC_OK 0
#define DC_ERR_INVALID_ARGUMENT (-1)  /* null pointer, negative size, bad shape                  */
#define DC_ERR_NO_DEVICE (-2)         /* no HIP device / device index out of range              */
#define DC_ERR_UNSUPPORTED (-3)       /* device is not gfx950, or a LINQ chain the kernels cannot run */
#define DC_ERR_OVERFLOW (-4)          /* checked int32 sum overflowed (System.OverflowException)  */
#define DC_ERR_MISALIGNED (-5)        /* pointer alignment the kernel requires was not met        */
#define DC_ERR_DIMENSION (-6)         /* matrix/vector dimension mismatch (ArgumentException)     */
#define DC_ERR_OUT_OF_MEMORY (-7)     /* scratch or host allocation failed                        */
#define DC_ERR_NOT_FOUND (-8)         /* module / function name not found                         */
#define DC_ERR_COMPILE (-9)           /* run-time compilation of a LINQ program failed              */

DC_HIP_API const char* dc_hip_error_string(int32_t status);
DC_HIP_API int32_t dc_hip_abi_version(void);

/* ---------------------------------------------------------------------------------------------
 * Devices and contexts
 * Replaces cudaGetDeviceCount / cudaGetDeviceProperties
 * (src/Backends/DotCompute.Backends.CUDA/Types/Native/CudaRuntime.cs:160) and the accelerator's
 * context/stream creation (src/Backends/DotCompute.Backends.CUDA/CudaAccelerator.cs:140-146).
 * ------------------------------------------------------------------------------------------- */
typedef struct dc_hip_device_info {
  char name[256];
  char gcn_arch_name[64];       /* e.g. "gfx950:sramecc+:xnack-" */
  int32_t device_id;
  int32_t compute_units;
  int32_t wave_size;            /* 64 on CDNA */
  int32_t max_threads_per_block;
  int32_t clock_khz;
  int32_t memory_clock_khz;
  int32_t memory_bus_width_bits;
  int32_t l2_cache_bytes;
  int64_t total_global_mem;
  int64_t lds_per_block;
  int32_t pci_bus_id;
  int32_t is_gfx950;            /* 1 when the kernels in this library can run on the device */
} dc_hip_device_info;

typedef struct dc_hip_ctx dc_hip_ctx;
typedef struct dc_hip_event dc_hip_event;
typedef struct dc_hip_module dc_hip_module;

DC_HIP_API int32_t dc_hip_device_count(int32_t* count);
DC_HIP_API int32_t dc_hip_device_info_get(int32_t device, dc_hip_device_info* info);
DC_HIP_API int32_t dc_hip_ctx_create(int32_t device, dc_hip_ctx** ctx);
DC_HIP_API int32_t dc_hip_ctx_destroy(dc_hip_ctx* ctx);
DC_HIP_API int32_t dc_hip_ctx_device(const dc_hip_ctx* ctx, int32_t* device);
/* Blocks until every operation enqueued on the context's stream has finished
 * (replaces cudaDeviceSynchronize, CudaAccelerator.cs:198-208). */
DC_HIP_API int32_t dc_hip_synchronize(dc_hip_ctx* ctx);

/* ---------------------------------------------------------------------------------------------
 * Memory (replaces cudaMalloc/cudaFree/cudaMemcpyAsync/cudaMemset,
 * src/Backends/DotCompute.Backends.CUDA/Types/Native/CudaRuntime.cs:243,247,278,291, used by
 * IUnifiedMemoryManager.AllocateAsync/CopyToDeviceAsync/CopyFromDeviceAsync/FreeAsync,
 * src/Core/DotCompute.Abstractions/Interfaces/IUnifiedMemoryManager.cs:47,130,143,160).
 * Copies are asynchronous on the context stream; host memory must stay valid (pinned, for
 * managed callers) until dc_hip_synchronize returns.
 * ------------------------------------------------------------------------------------------- */
DC_HIP_API int32_t dc_hip_malloc(dc_hip_ctx* ctx, size_t bytes, void** device_ptr);
DC_HIP_API int32_t dc_hip_free(dc_hip_ctx* ctx, void* device_ptr);
DC_HIP_API int32_t dc_hip_malloc_host(dc_hip_ctx* ctx, size_t bytes, void** host_ptr); /* pinned */
DC_HIP_API int32_t dc_hip_free_host(dc_hip_ctx* ctx, void* host_ptr);
DC_HIP_API int32_t dc_hip_memcpy_h2d_async(dc_hip_ctx* ctx, void* dst, const void* src, size_t bytes);
DC_HIP_API int32_t dc_hip_memcpy_d2h_async(dc_hip_ctx* ctx, void* dst, const void* src, size_t bytes);
DC_HIP_API int32_t dc_hip_memcpy_d2d_async(dc_hip_ctx* ctx, void* dst, const void* src, size_t bytes);
/* Fills `bytes` bytes with `value` (a kernel, not hipMemsetAsync, so it is safe under capture). */
DC_HIP_API int32_t dc_hip_memset_async(dc_hip_ctx* ctx, void* dst, int32_t value, size_t bytes);
DC_HIP_API int32_t dc_hip_mem_info(dc_hip_ctx* ctx, size_t* free_bytes, size_t* total_bytes);

/* ---------------------------------------------------------------------------------------------
 * Events on the context stream (the profiling hook; the reference times launches with
 * cudaEvent pairs, src/Backends/DotCompute.Backends.CUDA/Timing/CudaEventTimer.cs:219 and
 * src/Backends/DotCompute.Backends.CUDA/Types/Native/CudaRuntime.cs:524).
 * ------------------------------------------------------------------------------------------- */
DC_HIP_API int32_t dc_hip_event_create(dc_hip_ctx* ctx, dc_hip_event** event);
DC_HIP_API int32_t dc_hip_event_destroy(dc_hip_event* event);
DC_HIP_API int32_t dc_hip_event_record(dc_hip_ctx* ctx, dc_hip_event* event);
DC_HIP_API int32_t dc_hip_event_synchronize(dc_hip_event* event);
DC_HIP_API int32_t dc_hip_event_elapsed_ms(dc_hip_event* start, dc_hip_event* stop, float* ms);

/* ---------------------------------------------------------------------------------------------
 * Modules and generic launch: the ICompiledKernel path for prebuilt gfx950 code objects.
 * Replaces cuModuleLoadData / cuModuleGetFunction / cuLaunchKernel
 * (src/Backends/DotCompute.Backends.CUDA/Types/Native/CudaRuntime.cs:451,464,470) as driven by
 * CudaKernelLauncher.LaunchKernelInternalAsync (Kernels/CudaKernelLauncher.cs:205-349): `args` is
 * an array of pointers to the argument values, in parameter order.
 * ------------------------------------------------------------------------------------------- */
DC_HIP_API int32_t dc_hip_module_load(dc_hip_ctx* ctx, const char* path, dc_hip_module** module);
DC_HIP_API int32_t dc_hip_module_load_data(dc_hip_ctx* ctx, const void* image, dc_hip_module** module);
DC_HIP_API int32_t dc_hip_module_unload(dc_hip_module* module);
DC_HIP_API int32_t dc_hip_module_get_function(dc_hip_module* module, const char* name, void** function);
DC_HIP_API int32_t dc_hip_launch_kernel(dc_hip_ctx* ctx, void* function,
                                        uint32_t grid_x, uint32_t grid_y, uint32_t grid_z,
                                        uint32_t block_x, uint32_t block_y, uint32_t block_z,
                                        uint32_t shared_mem_bytes, void** args);
/* Path of the code object (dc_kernels_gfx950.hsaco) installed next to this library, or "" */
DC_HIP_API const char* dc_hip_default_module_path(void);

/* Launch block of the kernels generated from [Kernel] C# bodies (the HIP slot of the kernel
 * registry; the reference's generated CUDA kernels take (buffers..., scalars..., __length),
 * KernelExecutionMetadataEmitter.cs:65-105). A generated kernel takes its buffers and scalars in
 * declaration order, then this struct by value. It runs `work` work items, one per thread, in
 * workgroups of 256 (grid ceil(work / 256)); `len` holds each buffer parameter's element count
 * (Span<T>.Length), in buffer order. A work item that would throw in C# stores `epoch` into
 * error[DC_GEN_ERR_*]; the caller clears nothing, and compares the words with the epoch it passed
 * after the launch completes. `error` points to device-visible memory of 4 words. */
#define DC_GEN_MAX_BUFFERS 16
#define DC_GEN_BLOCK 256
#define DC_GEN_ERR_INDEX 0          /* IndexOutOfRangeException */
#define DC_GEN_ERR_DIVIDE_BY_ZERO 1 /* DivideByZeroException   */
#define DC_GEN_ERR_OVERFLOW 2       /* OverflowException       */
typedef struct dc_gen_launch {
  int64_t work;
  uint32_t epoch;
  uint32_t reserved;
  uint32_t* error;
  int64_t len[DC_GEN_MAX_BUFFERS];
} dc_gen_launch;

/* Device address of pinned host memory from dc_hip_malloc_host (replaces cudaHostGetDevicePointer),
 * for device-visible words such as dc_gen_launch.error. */
DC_HIP_API int32_t dc_hip_host_device_pointer(dc_hip_ctx* ctx, void* host_ptr, void** device_ptr);

/* ---------------------------------------------------------------------------------------------
 * Seeded, counter-based input generators (device side). Element i of stream s with seed k is
 * r = splitmix64(k ^ (s << 40) ^ i). Floats: [-1,1) -> (r >> 40) * 2^-23 - 1, [0,1) -> (r >> 40) *
 * 2^-24 (both exact in float32). Integers in [lo, hi]: lo + ((r >> 32) * (hi - lo + 1) >> 32).
 * dc_gen_* below reproduce the same streams bit-for-bit on the host.
 * ------------------------------------------------------------------------------------------- */
DC_HIP_API int32_t dc_hip_fill_uniform_f32(dc_hip_ctx* ctx, float* dst, int64_t n, uint64_t seed,
                                           uint32_t stream, int32_t unit_interval /* 0:[-1,1) 1:[0,1) */);
DC_HIP_API int32_t dc_hip_fill_uniform_i32(dc_hip_ctx* ctx, int32_t* dst, int64_t n, uint64_t seed,
                                           uint32_t stream, int32_t lo, int32_t hi);
DC_HIP_API int32_t dc_gen_uniform_f32(float* dst, int64_t n, uint64_t seed, uint32_t stream,
                                      int32_t unit_interval);
DC_HIP_API int32_t dc_gen_uniform_i32(int32_t* dst, int64_t n, uint64_t seed, uint32_t stream,
                                      int32_t lo, int32_t hi);
/* Synthetic PageRank-style CSR graph (host, multithreaded): out-degree of row r drawn from a
 * Zipf(alpha) law on [1, max_degree]; column indices uniform over [0, cols) without self-loops;
 * value = 1/out-degree. Call once with row_pointers only to learn nnz (row_pointers[rows]),
 * then again with col_indices/values sized nnz. */
DC_HIP_API int32_t dc_gen_zipf_csr_rowptr(int64_t rows, double alpha, int32_t max_degree,
                                          uint64_t seed, int32_t* row_pointers /* rows+1 */);
DC_HIP_API int32_t dc_gen_zipf_csr_fill(int64_t rows, int64_t cols, uint64_t seed,
                                        const int32_t* row_pointers, int32_t* col_indices,
                                        float* values);

/* ---------------------------------------------------------------------------------------------
 * VectorAdd — the README [Kernel] quick start, result[i] = a[i] + b[i]
 * Replaces the generated CUDA kernel launched by KernelExecutionService.ExecuteAsync
 * (src/Runtime/DotCompute.Runtime/Services/KernelExecutionService.cs:290-335; body emitted by
 * src/Runtime/DotCompute.Generators/Kernel/Generation/KernelExecutionMetadataEmitter.cs:65-105)
 * and OptimizedVectorAddKernel (src/Backends/DotCompute.Backends.CPU/Kernels/Optimized/
 * OptimizedVectorAddKernel.cs:81-111).
 * ------------------------------------------------------------------------------------------- */
DC_HIP_API int32_t dc_hip_vector_add_f32(dc_hip_ctx* ctx, const float* a, const float* b,
                                         float* result, int64_t n);

/* ---------------------------------------------------------------------------------------------
 * Sum reductions (deterministic: fixed per-thread order, fixed tree, last-block combine).
 * f32: accumulated in float64, result written as a double; the managed caller casts to float,
 *      as Enumerable.Sum(IEnumerable<float>) does (reached from
 *      src/Extensions/DotCompute.Linq/ComputeQueryableExtensions.cs:265-267) and as
 *      OptimizedReductionKernel does (src/Backends/DotCompute.Backends.CPU/Kernels/Optimized/
 *      OptimizedReductionKernel.cs:69-95).
 * i32: exact int64 total written to *sum_out; *overflow_out (device int32) is set to 1 when the
 *      total does not fit int32, which the managed caller raises as OverflowException
 *      (checked Enumerable.Sum(IEnumerable<int>)).
 * Replaces CudaKernelGenerator.GenerateReduceOperation
 * (src/Extensions/DotCompute.Linq/CodeGeneration/CudaKernelGenerator.cs:399-463).
 * ------------------------------------------------------------------------------------------- */
DC_HIP_API int32_t dc_hip_reduce_sum_f32(dc_hip_ctx* ctx, const float* input, int64_t n,
                                         double* sum_out);
DC_HIP_API int32_t dc_hip_reduce_sum_i32(dc_hip_ctx* ctx, const int32_t* input, int64_t n,
                                         int64_t* sum_out, int32_t* overflow_out);

/* ---------------------------------------------------------------------------------------------
 * Fused LINQ chains: Where / Select stages over float32, compiled by the host-side fusion planner
 * into a small register program (dc_linq_chain) that one prebuilt kernel interprets.
 * Replaces the per-chain CUDA-C that CudaKernelGenerator emits
 * (src/Extensions/DotCompute.Linq/CodeGeneration/CudaKernelGenerator.cs:81-125, fused
 * :1058-1134, filter :351-376) and the launch in RuntimeExecutor.ExecuteGpuKernelAsync
 * (src/Extensions/DotCompute.Linq/CodeGeneration/RuntimeExecutor.cs:245-312), with the
 * LINQ-to-objects semantics the provider falls back to today (ComputeQueryableExtensions.cs:628-633):
 * output is compacted and order-preserving.
 *
 * Program model. Per element the kernel holds: e (the pipeline element), v (accumulator), s0, s1
 * (saved values), p and q (predicate registers) and k (keep flag, initially true).
 * Each instruction: op, src (operand source), imm (constant operand).
 *   value ops   v = f(v, operand)         LOAD ADD SUB RSUB MUL DIV RDIV REM RREM MIN MAX POW RPOW
 *               v = f(v)                  NEG ABS SQRT FLOOR CEIL ROUND
 *   STORE_S0/1  s0/s1 = v
 *   CMP_*       c = (v <cmp> operand); p = c (mode SET), p && c (AND), p || c (OR)
 *   PNOT        p = !p;  PSTORE q = p;  PAND_Q p = p && q;  POR_Q p = p || q
 *   FILTER      k = k && p                 (ends a Where stage)
 *   MAP         e = v                      (ends a Select stage)
 * The element type is the entry point's (_f32 or _i32); `imm` is read as that type.
 * float32 programs: every operation rounds once to float32 (no contraction), matching .NET's
 *   scalar float arithmetic, so outputs are bit-identical to LINQ-to-objects for the same lambdas.
 *   REM is C#'s float `%` (truncated remainder, exact, the sign of the dividend); FLOOR, CEIL and
 *   ROUND are MathF.Floor, MathF.Ceiling and MathF.Round (ties to even). POW / RPOW are MathF.Pow
 *   (v = Pow(v, operand) / Pow(operand, v); the reference maps Pow to `pow`,
 *   CudaKernelGenerator.cs:1380): the device library's powf, within 1 ulp of the exact value as the
 *   C runtime's powf that .NET calls is, so results may differ from LINQ-to-objects by up to 2 ulp;
 *   special values (NaN, infinities, signed zeros) follow IEEE 754 / C99 Annex F, as .NET's.
 * int32 programs: C# `int` arithmetic in an unchecked context. + - * and NEG wrap; DIV/RDIV and
 *   REM/RREM truncate toward zero and throw on a zero divisor (DivideByZeroException) and on
 *   int.MinValue divided by -1 (OverflowException, as .NET on x64 also does for %); ABS is
 *   Math.Abs (OverflowException for int.MinValue); MIN/MAX are Math.Min/Max. SQRT, FLOOR, CEIL,
 *   ROUND, POW and RPOW have no int32 form (DC_ERR_UNSUPPORTED). A throwing operation is evaluated only for
 *   elements still kept at that point of the chain, as LINQ-to-objects evaluates a Select only for
 *   the elements its Where passed; the kernels report the first element (in sequence order) that
 *   throws through `fault_out` (below) instead of an output.
 * ------------------------------------------------------------------------------------------- */
#define DC_LINQ_MAX_INSTR 48

enum dc_linq_op {
  DC_LQ_NOP = 0,
  DC_LQ_LOAD = 1,
  DC_LQ_ADD = 2,
  DC_LQ_SUB = 3,
  DC_LQ_RSUB = 4,
  DC_LQ_MUL = 5,
  DC_LQ_DIV = 6,
  DC_LQ_RDIV = 7,
  DC_LQ_MIN = 8,
  DC_LQ_MAX = 9,
  DC_LQ_NEG = 10,
  DC_LQ_ABS = 11,
  DC_LQ_SQRT = 12,
  DC_LQ_STORE_S0 = 13,
  DC_LQ_STORE_S1 = 14,
  DC_LQ_REM = 15,   /* v = v % operand */
  DC_LQ_RREM = 16,  /* v = operand % v */
  DC_LQ_FLOOR = 17, /* float32 only */
  DC_LQ_CEIL = 18,  /* float32 only */
  DC_LQ_ROUND = 19, /* float32 only: ties to even */
  DC_LQ_CMP_GT = 20,
  DC_LQ_CMP_GE = 21,
  DC_LQ_CMP_LT = 22,
  DC_LQ_CMP_LE = 23,
  DC_LQ_CMP_EQ = 24,
  DC_LQ_CMP_NE = 25,
  DC_LQ_PNOT = 26,
  DC_LQ_PSTORE = 27,
  DC_LQ_PAND_Q = 28,
  DC_LQ_POR_Q = 29,
  DC_LQ_FILTER = 30,
  DC_LQ_MAP = 31,
  DC_LQ_POW = 32,  /* float32 only: v = MathF.Pow(v, operand) */
  DC_LQ_RPOW = 33  /* float32 only: v = MathF.Pow(operand, v) */
};

enum dc_linq_src {
  DC_LQ_SRC_IMM = 0,   /* the instruction's constant */
  DC_LQ_SRC_ELEM = 1,  /* e */
  DC_LQ_SRC_S0 = 2,
  DC_LQ_SRC_S1 = 3
};

enum dc_linq_cmp_mode { DC_LQ_CMP_SET = 0, DC_LQ_CMP_AND = 1, DC_LQ_CMP_OR = 2 };

typedef struct dc_linq_instr {
  uint8_t op;    /* enum dc_linq_op */
  uint8_t src;   /* enum dc_linq_src (value and CMP ops) */
  uint8_t mode;  /* enum dc_linq_cmp_mode (CMP ops) */
  uint8_t pad;
  union {
    float imm;        /* float32 programs */
    int32_t imm_i32;  /* int32 programs */
  };
} dc_linq_instr;

/* dc_linq_chain.flags bits. DC_LINQ_FLAG_ORDERED_GRID: run a ToArray on the ticket-ordered lookback
 * grid even where the resident grid would be chosen (the retry after a resident grid gave up).
 * DC_LINQ_FLAG_INTERPRET: never compile the program at run time (see dc_linq_chain_compile); run it
 * on the prebuilt interpreter kernels. */
#define DC_LINQ_FLAG_ORDERED_GRID 1
#define DC_LINQ_FLAG_INTERPRET 2

typedef struct dc_linq_chain {
  int32_t n_instr;
  int32_t flags;  /* DC_LINQ_FLAG_* bits; 0 by default */
  dc_linq_instr code[DC_LINQ_MAX_INSTR];
} dc_linq_chain;

/* Checks a program for structural validity (opcodes, operand sources, length). */
DC_HIP_API int32_t dc_linq_chain_validate(const dc_linq_chain* chain);
/* The same for an int32 program (which has no SQRT, FLOOR, CEIL, ROUND, POW or RPOW: DC_ERR_UNSUPPORTED). */
DC_HIP_API int32_t dc_linq_chain_validate_i32(const dc_linq_chain* chain);

/* Run-time compilation (replaces the NVRTC path of CudaRuntimeKernelCompiler.CompileAsync,
 * src/Extensions/DotCompute.Linq/Compilation/CudaRuntimeKernelCompiler.cs:80-138, and its cache by
 * source and options, :92-135). A program that is not an affine chain (those have prebuilt
 * kernels) can be compiled with hipRTC into a round-robin ToArray kernel of its own: the generated
 * source feeds the interpreter's own instruction semantics the program as constants. The library
 * builds and caches such kernels (once per process, device, element type and program) for inputs
 * of at least DC_LINQ_COMPILE_MIN_ELEMENTS, but the ToArray entry points do not launch them at
 * present: every program runs on the prebuilt interpreter kernels, and dc_hip_linq_compile_stats
 * reports no compiled launches. DC_LINQ_FLAG_INTERPRET (accepted on every chain) opts a chain
 * out of compilation. */
#define DC_LINQ_COMPILE_MIN_ELEMENTS (1 << 22)
enum dc_linq_element { DC_LINQ_ELEMENT_F32 = 0, DC_LINQ_ELEMENT_I32 = 1 };
/* Compiles a program's ToArray kernel for `arch` (e.g. "gfx950") without a device and reports its
 * code size: DC_ERR_COMPILE when hipRTC rejects the generated source (its log goes to stderr).
 * For tools and tests; the entry points compile on their own. */
DC_HIP_API int32_t dc_linq_chain_compile(const dc_linq_chain* chain, int32_t element_type, const char* arch,
                                         size_t* code_bytes_out);
/* Launches of run-time compiled kernels on this context so far, and compilations that failed. */
DC_HIP_API int32_t dc_hip_linq_compile_stats(dc_hip_ctx* ctx, int64_t* compiled_launches, int64_t* compile_failures);
/* Whether an int32 program can throw for some input (a DIV/RDIV/REM/RREM whose divisor is not an
 * immediate other than 0 and -1, or an ABS): *can_fault_out = 1 or 0. The int32 entry points need a
 * fault_out word for such programs and accept NULL for the others. */
DC_HIP_API int32_t dc_linq_chain_can_fault_i32(const dc_linq_chain* chain, int32_t* can_fault_out);

/* Where/Select → ToArray: writes the kept, mapped elements in input order to `output` (capacity n)
 * and their number to *count_out (device int64). One pass over the input. Large 16-byte aligned
 * inputs run on a resident grid (one workgroup per CU, per-round tile counts); the others, and
 * chains with DC_LINQ_FLAG_ORDERED_GRID, on a ticket-ordered grid with a decoupled lookback
 * (dc_hip_linq_to_array_strategy tells which). *count_out is -1 if the resident grid's bounded
 * wait for a tile count ever gave up (the device did not run every workgroup of the grid at once);
 * the output is then undefined and the caller re-runs the chain with DC_LINQ_FLAG_ORDERED_GRID,
 * whose waits always end. */
DC_HIP_API int32_t dc_hip_linq_where_select_f32(dc_hip_ctx* ctx, const dc_linq_chain* chain,
                                                const float* input, int64_t n, float* output,
                                                int64_t* count_out);
/* The kernel dc_hip_linq_where_select_f32 would use for this input (no device work). Diagnostic:
 * no counterpart in the reference, whose filter kernel has one shape (CudaKernelGenerator.cs:351-376). */
enum dc_linq_strategy { DC_LINQ_STRATEGY_LOOKBACK = 0, DC_LINQ_STRATEGY_ROUNDS = 1 };
DC_HIP_API int32_t dc_hip_linq_to_array_strategy(dc_hip_ctx* ctx, const float* input, int64_t n,
                                                 int32_t* strategy_out);
/* Where/Select → Sum (and Count): float64-accumulated sum of the kept, mapped elements to
 * *sum_out and their number to *count_out (either may be NULL). Deterministic. */
DC_HIP_API int32_t dc_hip_linq_where_select_sum_f32(dc_hip_ctx* ctx, const dc_linq_chain* chain,
                                                    const float* input, int64_t n,
                                                    double* sum_out, int64_t* count_out);
/* dc_hip_linq_where_select_sum_f32 that allocates nothing: for callers that cannot call
 * hipMalloc (code under HIP graph capture, tight serving loops, harnesses that forbid allocation).
 * No counterpart in the reference. Same kernels, same results bit for bit; the per-workgroup partials
 * live in a 16 KiB static device array (one per GPU, resolved at context creation) instead of
 * context scratch that grows on demand. Every n fits (the grid is capped at 1024 workgroups).
 * All calls of this process on one GPU share that array (another process loads its own copy): the
 * library orders them one after another, a call from another context waiting, on its stream, for
 * the previous call's stream position. */
DC_HIP_API int32_t dc_hip_linq_where_select_sum_f32_noalloc(dc_hip_ctx* ctx, const dc_linq_chain* chain,
                                                            const float* input, int64_t n,
                                                            double* sum_out, int64_t* count_out);
/* Where/Select → Min or Max of the kept, mapped elements: the result to *value_out (device float)
 * and the number of kept elements to *count_out (device int64; 0 = empty sequence, *value_out is
 * then unspecified and the managed layer throws InvalidOperationException). Replaces the reference's
 * Min/Max terminal operators (mapped to Reduce, src/Extensions/DotCompute.Linq/Compilation/
 * ExpressionTreeVisitor.cs:244-245; executed as LINQ-to-objects through the scalar branch,
 * ComputeQueryableExtensions.cs:265-267) and returns what the .NET 10 BCL Enumerable.Min/Max
 * (IEnumerable<float>) returns, bit for bit: Min the first NaN, else the first smallest element;
 * Max the first largest non-NaN element, or the last NaN when all are NaN. Deterministic.
 * DC_LINQ_FOLD_MIN / DC_LINQ_FOLD_MAX compute Aggregate((acc, x) => MathF.Min(acc, x)) / MathF.Max
 * instead (Aggregate maps to Reduce, ExpressionTreeVisitor.cs:263): IEEE 754-2019 minimum /
 * maximum, NaN if any kept element is NaN, -0 below +0; the fold without a seed. */
enum dc_linq_minmax { DC_LINQ_MIN = 0, DC_LINQ_MAX = 1, DC_LINQ_FOLD_MIN = 2, DC_LINQ_FOLD_MAX = 3 };
DC_HIP_API int32_t dc_hip_linq_where_select_minmax_f32(dc_hip_ctx* ctx, const dc_linq_chain* chain,
                                                       const float* input, int64_t n, int32_t op,
                                                       float* value_out, int64_t* count_out);

/* ---------------------------------------------------------------------------------------------
 * Fused LINQ chains over int32 sources (AsComputeQueryable over an int[]; the reference's provider
 * types any unmanaged T, src/Extensions/DotCompute.Linq/ComputeQueryableExtensions.cs:249-259,329,
 * and its generator maps int to CUDA `int` with the `%` operator, CodeGeneration/
 * CudaKernelGenerator.cs:1351,1399-1416). Same program model and kernels as the float32 entry
 * points, with C# int semantics (above).
 *
 * Faults. `fault_out` (device int64) receives -1 when no element throws, else 4 * i + kind for the
 * first element i (in sequence order) whose evaluation throws, kind DC_LINQ_FAULT_*: the exception
 * LINQ-to-objects would raise there. The other outputs are then unspecified. fault_out may be NULL
 * only for programs that cannot throw (dc_linq_chain_can_fault_i32); otherwise DC_ERR_INVALID_ARGUMENT.
 * ------------------------------------------------------------------------------------------- */
#define DC_LINQ_FAULT_NONE (-1)
#define DC_LINQ_FAULT_DIVIDE_BY_ZERO 1 /* System.DivideByZeroException */
#define DC_LINQ_FAULT_OVERFLOW 2       /* System.OverflowException     */

/* Where/Select -> ToArray over int32: as dc_hip_linq_where_select_f32 (order-preserving compaction,
 * *count_out -1 when the resident grid gave up and the chain must be re-run with
 * DC_LINQ_FLAG_ORDERED_GRID). */
DC_HIP_API int32_t dc_hip_linq_where_select_i32(dc_hip_ctx* ctx, const dc_linq_chain* chain,
                                                const int32_t* input, int64_t n, int32_t* output,
                                                int64_t* count_out, int64_t* fault_out);
/* Where/Select -> Sum / Count / Average over int32: the exact int64 total of the kept, mapped elements
 * to *sum_out and their number to *count_out (either may be NULL). *overflow_out (device int32, may
 * be NULL) is set to 1 when a checked int32 running total over those elements in sequence order
 * leaves the int32 range at some element, the rule of Enumerable.Sum(IEnumerable<int>) over an
 * iterator (a Where/Select result, which has no span, so the BCL adds element by element with
 * checked adds), else 0. Sum() over a bare int[] follows the BCL's vectorised rule instead:
 * dc_hip_reduce_sum_i32. Deterministic. */
DC_HIP_API int32_t dc_hip_linq_where_select_sum_i32(dc_hip_ctx* ctx, const dc_linq_chain* chain,
                                                    const int32_t* input, int64_t n, int64_t* sum_out,
                                                    int64_t* count_out, int32_t* overflow_out,
                                                    int64_t* fault_out);
/* Where/Select -> Min or Max over int32 (Math.Min/Max order; *value_out unspecified when
 * *count_out is 0, the empty sequence). */
DC_HIP_API int32_t dc_hip_linq_where_select_minmax_i32(dc_hip_ctx* ctx, const dc_linq_chain* chain,
                                                       const int32_t* input, int64_t n, int32_t op,
                                                       int32_t* value_out, int64_t* count_out,
                                                       int64_t* fault_out);

/* ---------------------------------------------------------------------------------------------
 * Dense GEMM, row-major: C[m×n] = A[m×k] · B[k×n].
 * Replaces OptimizedMatrixMultiplyKernel (src/Backends/DotCompute.Backends.CPU/Kernels/Optimized/
 * OptimizedMatrixMultiplyKernel.cs:72-96), MatrixOperations.MultiplyAsync / MultiplyOnGPUAsync
 * (src/Extensions/DotCompute.Algorithms/LinearAlgebra/Operations/MatrixOperations.cs:28-64,359-440)
 * and the 16×16 tiled string kernels (LinearAlgebra/MatrixKernels.cs:11-80).
 * f32: fp32 inputs, fp32 MFMA (v_mfma_f32_*_f32), fp32 accumulate.
 * bf16: bf16 inputs (uint16 bit patterns), bf16 MFMA, fp32 accumulate and output.
 * Leading dimensions equal the row lengths (k for A, n for B and C).
 * ------------------------------------------------------------------------------------------- */
DC_HIP_API int32_t dc_hip_gemm_f32(dc_hip_ctx* ctx, const float* a, const float* b, float* c,
                                   int64_t m, int64_t n, int64_t k);
DC_HIP_API int32_t dc_hip_gemm_bf16(dc_hip_ctx* ctx, const uint16_t* a, const uint16_t* b, float* c,
                                    int64_t m, int64_t n, int64_t k);
/* Round-to-nearest-even float32 → bfloat16 conversion (NaN stays NaN). */
DC_HIP_API int32_t dc_hip_convert_f32_to_bf16(dc_hip_ctx* ctx, const float* input, uint16_t* output,
                                              int64_t n);

/* ---------------------------------------------------------------------------------------------
 * CSR SpMV, y = A·x in float32 (CsrMatrix<T> + SparseOps.SpMV,
 * src/Extensions/DotCompute.Algorithms/Sparse/SparseMatrix.cs:68-272,669-692; the never-launched
 * CUDA string kernel Kernels/LinearAlgebra/SparseMatrixKernels.cs:47-75).
 * row_pointers has rows+1 entries (int32 offsets, as CsrMatrix<T>); x has cols entries.
 * The matrix must be a valid CSR: row_pointers non-decreasing from 0 to nnz and every column index
 * in [0, cols) (the host CsrMatrix checks both, as the reference's does its sizes); these one-shot
 * entry points read what the indices point at without checking them. The plan entry points below
 * clamp every index instead.
 * ------------------------------------------------------------------------------------------- */
DC_HIP_API int32_t dc_hip_spmv_csr_f32(dc_hip_ctx* ctx, const int32_t* row_pointers,
                                       const int32_t* col_indices, const float* values,
                                       const float* x, float* y, int64_t rows, int64_t cols,
                                       int64_t nnz);
/* The same for SparseOps.SpMV<double> and SpMV<int> (the reference's SpMV is generic over
 * INumber<T>, SparseMatrix.cs:669): per row T.Zero plus each product in index order for rows of
 * at most 512 nonzeros (bit-identical to the reference loop), a fixed-order tree for longer rows;
 * int multiplies and adds wrap (C#'s unchecked arithmetic, so every row is bit-identical). */
DC_HIP_API int32_t dc_hip_spmv_csr_f64(dc_hip_ctx* ctx, const int32_t* row_pointers,
                                       const int32_t* col_indices, const double* values,
                                       const double* x, double* y, int64_t rows, int64_t cols,
                                       int64_t nnz);
DC_HIP_API int32_t dc_hip_spmv_csr_i32(dc_hip_ctx* ctx, const int32_t* row_pointers,
                                       const int32_t* col_indices, const int32_t* values,
                                       const int32_t* x, int32_t* y, int64_t rows, int64_t cols,
                                       int64_t nnz);
/* Power iteration used by the SpMV benchmark: repeat `iterations` times
 *   y = A·x;  s = Σ y (float64);  x = y / s
 * leaving the normalised vector in x (rows == cols required). `y` is caller-provided scratch of
 * rows floats. The final L1 norm before the last normalisation is written to *last_sum_out
 * (device double, may be NULL). Builds a tiled plan (below) in context scratch first and runs
 * every iteration through it. */
DC_HIP_API int32_t dc_hip_spmv_power_iterate_f32(dc_hip_ctx* ctx, const int32_t* row_pointers,
                                                 const int32_t* col_indices, const float* values,
                                                 float* x, float* y, int64_t rows, int64_t nnz,
                                                 int32_t iterations, double* last_sum_out);

/* Tiled SpMV plan: an analysis of a CSR matrix, built once on the device, for matrices that are
 * multiplied many times (CsrMatrix<T> reused across SparseOps.SpMV calls,
 * src/Extensions/DotCompute.Algorithms/Sparse/SparseMatrix.cs:669-692; the power iteration).
 * The plan holds its own slice-major copy of the nonzeros and of the row pointers (device memory
 * owned by the plan), so the CSR arrays may be freed once the creating call's stream work has run.
 * Columns are cut into slices of at most `slice_cols_max` columns (at most 32768: a 128 KB tile
 * of x in one CU's LDS; 0 = the default, the widest power of two from 4096 to 32768 columns that
 * is at most nnz / (2 x the device's CU count), wide enough for at most 512 or 1024 slices (the
 * row pass's LDS tables, by matrix size) where 32768 allows; widened when more than 32768 slices
 * would be needed); every product val·x[col] is
 * formed once from an LDS tile, and each row is summed from its products in index order. Result: rows of at most 32 nonzeros equal the
 * sequential float32 row sum (0.0f + p_0 + p_1 + ...) bit for bit, whatever the slice count;
 * longer rows are summed in a fixed order (lane k of a wave adds products k, k + 64, ..., then a
 * fixed tree), within the fp32 tolerance. Column indices outside [0, cols) are clamped into range
 * on the device (they never fault); callers validate first. */
typedef struct dc_hip_spmv_plan dc_hip_spmv_plan;
DC_HIP_API int32_t dc_hip_spmv_plan_create(dc_hip_ctx* ctx, const int32_t* row_pointers,
                                           const int32_t* col_indices, const float* values,
                                           int64_t rows, int64_t cols, int64_t nnz,
                                           int64_t slice_cols_max, dc_hip_spmv_plan** plan_out);
/* y = A·x through the plan (asynchronous on the context stream). */
DC_HIP_API int32_t dc_hip_spmv_plan_execute_f32(dc_hip_ctx* ctx, const dc_hip_spmv_plan* plan,
                                                const float* x, float* y);
/* The power iteration above, through an existing plan (rows == cols). */
DC_HIP_API int32_t dc_hip_spmv_plan_power_iterate_f32(dc_hip_ctx* ctx, const dc_hip_spmv_plan* plan,
                                                      float* x, float* y, int32_t iterations,
                                                      double* last_sum_out);
/* Number of column slices, columns per slice, device bytes held. Any pointer may be NULL. */
DC_HIP_API int32_t dc_hip_spmv_plan_info(const dc_hip_spmv_plan* plan, int32_t* slices,
                                         int64_t* slice_cols, int64_t* device_bytes);
/* Waits for the device, then frees the plan. */
DC_HIP_API int32_t dc_hip_spmv_plan_destroy(dc_hip_spmv_plan* plan);

#ifdef __cplusplus
}
#endif

#endif /* DOTCOMPUTE_HIP_H */

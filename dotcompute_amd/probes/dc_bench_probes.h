/*
 * dc_bench_probes.h — measurement-only probes of libdotcompute_bench.so (bench.py's streaming
 * ceilings). Not part of the product ABI in include/dotcompute_hip.h and with no counterpart in the
 * reference: what plain streaming kernels reach on this device for a given read/write mix.
 *
 * One 16-byte vector per thread over a grid that covers the input (1024-thread workgroups),
 * non-temporal loads and stores, on the context's stream. `n` floats, a multiple of 8; `src` and
 * `dst` 16-byte aligned (DC_ERR_MISALIGNED otherwise).
 *   DC_PROBE_COPY:           dst[i] = src[i], i < n                    (reads 4n B, writes 4n B)
 *   DC_PROBE_READ2_WRITE1:   dst[i] = src[i] + src[n/2 + i], i < n/2   (reads 4n B, writes 2n B)
 *   DC_PROBE_READ:           reads src[0, n) and writes nothing (each value is compared with
 *                            a NaN passed at run time, which never compares equal)  (reads 4n B)
 */
#ifndef DC_BENCH_PROBES_H
#define DC_BENCH_PROBES_H

#include "../../include/dotcompute_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

#define DC_BENCH_API __attribute__((visibility("default")))

#define DC_PROBE_COPY 0
#define DC_PROBE_READ2_WRITE1 1
#define DC_PROBE_READ 2
DC_BENCH_API int32_t dc_bench_stream_probe(dc_hip_ctx* ctx, int32_t kind, const float* src, float* dst, int64_t n);

#ifdef __cplusplus
}
#endif

#endif /* DC_BENCH_PROBES_H */

// dc_spmv.hip — placeholder until the SpMV kernels land.
#include "dc_internal.hpp"
extern "C" {
DC_HIP_API int32_t dc_hip_spmv_csr_f32(dc_hip_ctx*, const int32_t*, const int32_t*, const float*, const float*, float*, int64_t, int64_t, int64_t) { return DC_ERR_UNSUPPORTED; }
DC_HIP_API int32_t dc_hip_spmv_power_iterate_f32(dc_hip_ctx*, const int32_t*, const int32_t*, const float*, float*, float*, int64_t, int64_t, int32_t, double*) { return DC_ERR_UNSUPPORTED; }
}

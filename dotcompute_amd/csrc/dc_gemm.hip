// dc_gemm.hip — placeholder until the MFMA GEMM lands.
#include "dc_internal.hpp"
extern "C" {
DC_HIP_API int32_t dc_hip_gemm_f32(dc_hip_ctx*, const float*, const float*, float*, int64_t, int64_t, int64_t) { return DC_ERR_UNSUPPORTED; }
DC_HIP_API int32_t dc_hip_gemm_bf16(dc_hip_ctx*, const uint16_t*, const uint16_t*, float*, int64_t, int64_t, int64_t) { return DC_ERR_UNSUPPORTED; }
DC_HIP_API int32_t dc_hip_convert_f32_to_bf16(dc_hip_ctx*, const float*, uint16_t*, int64_t) { return DC_ERR_UNSUPPORTED; }
}

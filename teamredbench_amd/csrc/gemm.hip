// GEMM dispatch: picks the kernel family for a (dtype, M, N, K) case and
// forwards the launch. Validation of dtype and sizes lives here.
#include "gemm_common.hpp"

namespace mb {

int gemm_plan(int dtype, int64_t M, int64_t N, int64_t K, const DeviceProps& props,
              GemmPlan* plan) {
    if (dtype != MB_DT_BFLOAT16 && dtype != MB_DT_FLOAT16 && !is_fp8(dtype) && dtype != MB_DT_FLOAT32 &&
        dtype != MB_DT_FLOAT64) {
        set_error("GEMM supports bfloat16, float16, float8_e4m3fn, float8_e5m2, float32 and float64 (got %s)",
                  dtype_name(dtype));
        return MB_ERR_UNSUPPORTED;
    }
    if (M < 1 || N < 1 || K < 1) {
        set_error("GEMM sizes must be >= 1 (M=%lld N=%lld K=%lld)", (long long)M, (long long)N,
                  (long long)K);
        return MB_ERR_INVALID_ARG;
    }
    if (dtype == MB_DT_FLOAT32 || dtype == MB_DT_FLOAT64) return gemm_highp_plan(dtype, M, N, K, props, plan);
    const bool generic_only = tuning(MB_TUNE_GEMM_FORCE_GENERIC) == 1;
    if (!generic_only && tuning(MB_TUNE_GEMM_NO_SMALL_M) != 1 &&
        gemm_gemv_plan(dtype, M, N, K, props, plan) == MB_OK)
        return MB_OK;
    const char* why = "forced by the gemm_force_generic override";
    if (!generic_only && gemm_tiled_plan(dtype, M, N, K, props, plan, &why) == MB_OK) return MB_OK;
    const int rc = gemm_generic_plan(dtype, M, N, K, plan);
    plan->fallback = why;
    return rc;
}

int gemm_launch(int dtype, const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
                float scale_a, float scale_b, void* workspace, const GemmPlan& plan,
                hipStream_t stream) {
    const float alpha = is_fp8(dtype) ? scale_a * scale_b : 1.0f;
    switch (plan.variant) {
        case kVariantGeneric:
            return gemm_generic_launch(dtype, A, B, C, M, N, K, alpha, stream);
        case kVariantTiled:
            return gemm_tiled_launch(dtype, A, B, C, M, N, K, alpha, workspace, plan, stream);
        case kVariantHighp:
            return gemm_highp_launch(dtype, A, B, C, M, N, K, plan, stream);
        case kVariantGemv:
            return gemm_gemv_launch(dtype, A, B, C, M, N, K, workspace, plan, stream);
        default:
            set_error("GEMM plan variant %d not available", plan.variant);
            return MB_ERR_UNSUPPORTED;
    }
}

}  // namespace mb

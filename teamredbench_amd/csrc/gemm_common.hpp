// Pieces shared by the GEMM kernel families: MFMA wrappers, output rounding,
// and the plan/launch entry points of each family.
#pragma once

#include "mb_common.hpp"

namespace mb {

enum GemmVariant {
    kVariantGeneric = 0,  // any shape, bounds-checked (gemm_generic.hip)
    kVariantTiled = 1,    // N % 256, LDS-DMA pipelined, optional split-K (gemm_tiled.hip)
    kVariantHighp = 2,    // fp32 / fp64 inputs, any shape (gemm_highp.hip)
    kVariantGemv = 3,     // bf16 / fp16 with M <= 4: streaming FMA kernel (gemm_gemv.hip)
};

constexpr bool is_fp8(int dtype) { return dtype == MB_DT_FLOAT8_E4M3FN || dtype == MB_DT_FLOAT8_E5M2; }

// One 16 x 16 MFMA step; operand fragments come from LDS (or registers)
// through byte pointers. bf16/f16: 8 elements (16 bytes) per lane, K = 32.
// fp8 (e4m3 or e5m2): 32 elements (32 bytes) per lane, K = 128, unit block scales.
template <int DT>
struct Mfma16;

template <>
struct Mfma16<MB_DT_BFLOAT16> {
    __device__ static inline f32x4 run(const void* pa, const void* pb, f32x4 c) {
        bf16x8 a = *static_cast<const bf16x8*>(pa);
        bf16x8 b = *static_cast<const bf16x8*>(pb);
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};

template <>
struct Mfma16<MB_DT_FLOAT16> {
    __device__ static inline f32x4 run(const void* pa, const void* pb, f32x4 c) {
        f16x8 a = *static_cast<const f16x8*>(pa);
        f16x8 b = *static_cast<const f16x8*>(pb);
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};

// E8M0 exponent 127 encodes a block scale of 1.0; operand format code 0
// selects fp8 e4m3, 1 selects bf8 e5m2 (for both operands).
template <>
struct Mfma16<MB_DT_FLOAT8_E4M3FN> {
    __device__ static inline f32x4 run(const void* pa, const void* pb, f32x4 c) {
        i32x8 a = *static_cast<const i32x8*>(pa);
        i32x8 b = *static_cast<const i32x8*>(pb);
        return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
    }
};

template <>
struct Mfma16<MB_DT_FLOAT8_E5M2> {
    __device__ static inline f32x4 run(const void* pa, const void* pb, f32x4 c) {
        i32x8 a = *static_cast<const i32x8*>(pa);
        i32x8 b = *static_cast<const i32x8*>(pb);
        return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 1, 1, 0, 127, 0, 127);
    }
};

// Output element type (16-bit kernels): bf16 for bf16 and fp8 inputs, fp16 for fp16.
template <int DT>
__device__ inline void store_out(void* C, int64_t idx, float v) {
    if (DT == MB_DT_FLOAT16) {
        static_cast<_Float16*>(C)[idx] = (_Float16)v;
    } else {
        static_cast<__bf16*>(C)[idx] = (__bf16)v;
    }
}

int gemm_generic_plan(int dtype, int64_t M, int64_t N, int64_t K, GemmPlan* plan);
// MB_ERR_SHAPE with *why naming the reason when no tiled configuration takes the shape.
int gemm_tiled_plan(int dtype, int64_t M, int64_t N, int64_t K, const DeviceProps& props,
                    GemmPlan* plan, const char** why);
int gemm_tiled_launch(int dtype, const void* A, const void* B, void* C, int64_t M, int64_t N,
                      int64_t K, float alpha, void* workspace, const GemmPlan& plan, hipStream_t stream);
int gemm_generic_launch(int dtype, const void* A, const void* B, void* C, int64_t M, int64_t N,
                        int64_t K, float alpha, hipStream_t stream);
int gemm_highp_plan(int dtype, int64_t M, int64_t N, int64_t K, const DeviceProps& props, GemmPlan* plan);
int gemm_gemv_plan(int dtype, int64_t M, int64_t N, int64_t K, const DeviceProps& props, GemmPlan* plan);
int gemm_gemv_launch(int dtype, const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
                     void* workspace, const GemmPlan& plan, hipStream_t stream);
int gemm_highp_launch(int dtype, const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
                      const GemmPlan& plan, hipStream_t stream);

}  // namespace mb

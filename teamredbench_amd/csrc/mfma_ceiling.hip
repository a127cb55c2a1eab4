// The sustained throughput of one MFMA instruction on this part, with no
// memory traffic: every wave issues independent MFMAs back to back on operand
// registers, alternating between two operand sets so that consecutive MFMAs
// of a chain see different data. Under the part's power limit the clock, and
// so the MFMA rate, settles well below the figure the peak assumes; this
// kernel measures what a GEMM's MFMA work can reach at most, next to the
// GEMM itself (mb_mfma_ceiling).
#include "mb_common.hpp"

namespace mb {
namespace {

constexpr int kCeilingThreads = 256;
constexpr int kChains = 8;   // independent accumulator chains per wave

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

template <int KIND>
struct CeilingOp;

template <>
struct CeilingOp<MB_MFMA_BF16_32X32X16> {
    typedef u32x4 Operand;
    typedef f32x16 Acc;
    __device__ static Acc run(const Operand& a, const Operand& b, Acc c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                        c, 0, 0, 0);
    }
};

template <>
struct CeilingOp<MB_MFMA_BF16_16X16X32> {
    typedef u32x4 Operand;
    typedef f32x4 Acc;
    __device__ static Acc run(const Operand& a, const Operand& b, Acc c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                        c, 0, 0, 0);
    }
};

template <>
struct CeilingOp<MB_MFMA_FP8_32X32X64> {
    typedef i32x8 Operand;
    typedef f32x16 Acc;
    __device__ static Acc run(const Operand& a, const Operand& b, Acc c) {
        return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
    }
};

template <>
struct CeilingOp<MB_MFMA_FP8_16X16X128> {
    typedef i32x8 Operand;
    typedef f32x4 Acc;
    __device__ static Acc run(const Operand& a, const Operand& b, Acc c) {
        return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
    }
};

template <>
struct CeilingOp<MB_MFMA_F32_32X32X2> {
    typedef float Operand;
    typedef f32x16 Acc;
    __device__ static Acc run(const Operand& a, const Operand& b, Acc c) {
        return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
    }
};

// Each lane loads its two operand sets from `operands` (random values of the
// instruction's type, 2 x 2 x 32 bytes per lane), runs `iterations` rounds of
// kChains independent MFMAs, and writes the sum of its accumulators to out
// (one float per thread), which keeps the work observable.
template <int KIND>
__global__ void __launch_bounds__(kCeilingThreads)
mfma_ceiling_kernel(const unsigned char* __restrict__ operands, float* __restrict__ out, int iterations) {
    typedef CeilingOp<KIND> Op;
    typedef typename Op::Operand Operand;
    typedef typename Op::Acc Acc;
    const int lane = threadIdx.x & 63;
    const unsigned char* mine = operands + lane * 4 * 32;
    Operand a[2], b[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        __builtin_memcpy(&a[s], mine + 64 * s, sizeof(Operand));
        __builtin_memcpy(&b[s], mine + 64 * s + 32, sizeof(Operand));
    }
    Acc acc[kChains];
#pragma unroll
    for (int c = 0; c < kChains; ++c)
#pragma unroll
        for (int r = 0; r < (int)(sizeof(Acc) / sizeof(float)); ++r) acc[c][r] = 0.f;
    for (int i = 0; i < iterations; i += 2) {
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int c = 0; c < kChains; ++c) acc[c] = Op::run(a[(s + c) & 1], b[(s + c) & 1], acc[c]);
    }
    float sum = 0.f;
#pragma unroll
    for (int c = 0; c < kChains; ++c)
#pragma unroll
        for (int r = 0; r < (int)(sizeof(Acc) / sizeof(float)); ++r) sum += acc[c][r];
    out[(int64_t)blockIdx.x * kCeilingThreads + threadIdx.x] = sum;
}

}  // namespace

int mfma_ceiling_launch(int kind, const void* operands, float* out, int blocks, int iterations, hipStream_t stream) {
    const auto* ops = static_cast<const unsigned char*>(operands);
    const dim3 grid(blocks), block(kCeilingThreads);
    switch (kind) {
        case MB_MFMA_BF16_32X32X16:
            hipLaunchKernelGGL(mfma_ceiling_kernel<MB_MFMA_BF16_32X32X16>, grid, block, 0, stream, ops, out, iterations);
            break;
        case MB_MFMA_BF16_16X16X32:
            hipLaunchKernelGGL(mfma_ceiling_kernel<MB_MFMA_BF16_16X16X32>, grid, block, 0, stream, ops, out, iterations);
            break;
        case MB_MFMA_FP8_32X32X64:
            hipLaunchKernelGGL(mfma_ceiling_kernel<MB_MFMA_FP8_32X32X64>, grid, block, 0, stream, ops, out, iterations);
            break;
        case MB_MFMA_FP8_16X16X128:
            hipLaunchKernelGGL(mfma_ceiling_kernel<MB_MFMA_FP8_16X16X128>, grid, block, 0, stream, ops, out, iterations);
            break;
        case MB_MFMA_F32_32X32X2:
            hipLaunchKernelGGL(mfma_ceiling_kernel<MB_MFMA_F32_32X32X2>, grid, block, 0, stream, ops, out, iterations);
            break;
        default:
            set_error("mfma ceiling: unknown instruction %d", kind);
            return MB_ERR_INVALID_ARG;
    }
    MB_HIP_TRY(hipGetLastError());
    return MB_OK;
}

}  // namespace mb

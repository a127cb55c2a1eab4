// General-shape GEMM for gfx950: C = A * B (row-major) with fp32 MFMA
// accumulation, for any M, N, K >= 1. Used for shapes the tiled fast path
// does not take (ragged edges, tiny problems). Correctness over speed: global
// loads are element-wise and bounds-checked, zero-padding the LDS tiles.
//
// Block: 256 threads = 4 waves in a 2x2 grid; block tile 64 x 64; each wave
// owns a 32 x 32 sub-tile as 2 x 2 MFMA fragments of 16 x 16.
// LDS keeps both operands K-contiguous (A as [m][k], B transposed to [n][k])
// so every lane reads its MFMA operand with one 16- or 32-byte LDS load.
#include "gemm_common.hpp"

namespace mb {
namespace {

constexpr int kGenTile = 64;
constexpr int kGenThreads = 256;

// bf16 / f16: v_mfma_f32_16x16x32_{bf16,f16}; lane l holds row (l % 16) and
// k-slots 8*(l/16) .. 8*(l/16)+7 of a 16 x 32 operand fragment.
// fp8 (e4m3 or e5m2): v_mfma_scale_f32_16x16x128_f8f6f4 with unit E8M0
// scales; lane l holds row (l % 16) and 32 k-slots starting at 32*(l/16).
template <int DT>
struct GenericTraits;

template <>
struct GenericTraits<MB_DT_BFLOAT16> {
    typedef uint16_t E;
    static constexpr int kBK = 32;
    static constexpr int kLaneK = 8;
};
template <>
struct GenericTraits<MB_DT_FLOAT16> {
    typedef uint16_t E;
    static constexpr int kBK = 32;
    static constexpr int kLaneK = 8;
};
template <>
struct GenericTraits<MB_DT_FLOAT8_E4M3FN> {
    typedef uint8_t E;
    static constexpr int kBK = 128;
    static constexpr int kLaneK = 32;
};
template <>
struct GenericTraits<MB_DT_FLOAT8_E5M2> : GenericTraits<MB_DT_FLOAT8_E4M3FN> {};

template <int DT>
__global__ void __launch_bounds__(kGenThreads)
gemm_generic_kernel(const void* __restrict__ Ap, const void* __restrict__ Bp, void* __restrict__ Cp,
                    int64_t M, int64_t N, int64_t K, float alpha) {
    typedef GenericTraits<DT> Tr;
    typedef typename Tr::E E;
    constexpr int BK = Tr::kBK;
    constexpr int LK = Tr::kLaneK;
    // K-contiguous tiles; rows padded by 16 bytes to spread LDS banks.
    constexpr int kRowBytes = BK * (int)sizeof(E) + 16;
    __shared__ __attribute__((aligned(16))) unsigned char lds_a[kGenTile * kRowBytes];
    __shared__ __attribute__((aligned(16))) unsigned char lds_b[kGenTile * kRowBytes];

    const E* A = static_cast<const E*>(Ap);
    const E* B = static_cast<const E*>(Bp);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int64_t m0 = (int64_t)blockIdx.y * kGenTile;
    const int64_t n0 = (int64_t)blockIdx.x * kGenTile;

    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

    for (int64_t k0 = 0; k0 < K; k0 += BK) {
        // A tile: element (r, kk) -> lds_a[r][kk]; B tile: (kk, c) -> lds_b[c][kk].
        for (int idx = tid; idx < kGenTile * BK; idx += kGenThreads) {
            const int r = idx / BK, kk = idx % BK;
            const int64_t gm = m0 + r, gk = k0 + kk;
            E v = 0;
            if (gm < M && gk < K) v = A[gm * K + gk];
            reinterpret_cast<E*>(lds_a + r * kRowBytes)[kk] = v;
        }
        for (int idx = tid; idx < kGenTile * BK; idx += kGenThreads) {
            const int kk = idx / kGenTile, c = idx % kGenTile;
            const int64_t gk = k0 + kk, gn = n0 + c;
            E v = 0;
            if (gk < K && gn < N) v = B[gk * N + gn];
            reinterpret_cast<E*>(lds_b + c * kRowBytes)[kk] = v;
        }
        __syncthreads();
        const int kslot = (lane >> 4) * LK * (int)sizeof(E);  // byte offset in the row
#pragma unroll
        for (int i = 0; i < 2; ++i) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int ar = wm * 32 + i * 16 + (lane & 15);
                const int bc = wn * 32 + j * 16 + (lane & 15);
                const unsigned char* pa = lds_a + ar * kRowBytes + kslot;
                const unsigned char* pb = lds_b + bc * kRowBytes + kslot;
                acc[i][j] = Mfma16<DT>::run(pa, pb, acc[i][j]);
            }
        }
        __syncthreads();
    }

    // Epilogue: 16x16 fragment layout, lane l reg r -> row 4*(l/16)+r, col l%16.
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t gm = m0 + wm * 32 + i * 16 + (lane >> 4) * 4 + r;
                const int64_t gn = n0 + wn * 32 + j * 16 + (lane & 15);
                if (gm < M && gn < N) store_out<DT>(Cp, gm * N + gn, acc[i][j][r] * alpha);
            }
        }
    }
}

}  // namespace

int gemm_generic_plan(int dtype, int64_t M, int64_t N, int64_t K, GemmPlan* plan) {
    (void)K;
    plan->implementation = "gfx950_mfma_generic";
    plan->threads = kGenThreads;
    const int64_t gx = (N + kGenTile - 1) / kGenTile, gy = (M + kGenTile - 1) / kGenTile;
    plan->grid = (int)(gx * gy);
    plan->tile_m = kGenTile;
    plan->tile_n = kGenTile;
    plan->tile_k = is_fp8(dtype) ? 128 : 32;
    plan->wave_grid_m = 2;
    plan->wave_grid_n = 2;
    plan->wave_tile_m = 2;
    plan->wave_tile_n = 2;
    plan->frag_m = 16;
    plan->frag_n = 16;
    plan->frag_k = is_fp8(dtype) ? 128 : 32;
    plan->k_stages = 1;
    plan->split_k = 1;
    plan->tile_group_m = 1;
    plan->workspace = 0;
    plan->variant = kVariantGeneric;
    if (gy > 65535) {
        set_error("generic GEMM: M=%lld too large", (long long)M);
        return MB_ERR_SHAPE;
    }
    return MB_OK;
}

int gemm_generic_launch(int dtype, const void* A, const void* B, void* C, int64_t M, int64_t N,
                        int64_t K, float alpha, hipStream_t stream) {
    const dim3 grid((unsigned)((N + kGenTile - 1) / kGenTile), (unsigned)((M + kGenTile - 1) / kGenTile));
    switch (dtype) {
        case MB_DT_BFLOAT16:
            hipLaunchKernelGGL(gemm_generic_kernel<MB_DT_BFLOAT16>, grid, dim3(kGenThreads), 0, stream,
                               A, B, C, M, N, K, alpha);
            break;
        case MB_DT_FLOAT16:
            hipLaunchKernelGGL(gemm_generic_kernel<MB_DT_FLOAT16>, grid, dim3(kGenThreads), 0, stream,
                               A, B, C, M, N, K, alpha);
            break;
        case MB_DT_FLOAT8_E4M3FN:
            hipLaunchKernelGGL(gemm_generic_kernel<MB_DT_FLOAT8_E4M3FN>, grid, dim3(kGenThreads), 0,
                               stream, A, B, C, M, N, K, alpha);
            break;
        case MB_DT_FLOAT8_E5M2:
            hipLaunchKernelGGL(gemm_generic_kernel<MB_DT_FLOAT8_E5M2>, grid, dim3(kGenThreads), 0,
                               stream, A, B, C, M, N, K, alpha);
            break;
        default:
            set_error("generic GEMM: unsupported dtype %d", dtype);
            return MB_ERR_UNSUPPORTED;
    }
    MB_HIP_TRY(hipGetLastError());
    return MB_OK;
}

}  // namespace mb

// General-shape GEMM for gfx950: C = alpha * A * B (row-major) with fp32
// MFMA accumulation, for any M, N, K >= 1. It takes the shapes the LDS-DMA
// kernels cannot: A or B rows not on 16 bytes (K or N not a multiple of 8, of
// 16 for fp8). Every global access is bounds-checked.
//
// Block: 256 threads = 4 waves in a 2 x 2 grid; block tile 128 x 128; each
// wave owns 64 x 64 of C as 2 x 2 fragments of 32 x 32
// (v_mfma_f32_32x32x16_{bf16,f16}, or v_mfma_scale_f32_32x32x64_f8f6f4 with
// unit scales for fp8). A stage is 64 bytes of K. Both operands sit in LDS
// K-contiguous -- A as [m][k], B transposed to [n][k] -- in rows padded to 80
// bytes, so each lane reads its operand with 16-byte LDS loads and the 8
// lanes of one LDS phase (8 consecutive rows) hit distinct banks. Two LDS
// buffers: while the MFMAs of stage k read one, the loads of stage k + 1 are
// in flight into registers (element loads unpacked until then), and they are
// written to the other buffer before the stage's single barrier.
//
// Global loads: a thread stages 32 bytes of A (row t / 2, half t % 2 of the
// stage) and 32 bytes of B (column t % 128, half t / 128 of the stage's K
// rows). A comes in two 16-byte loads when its rows are on 16 bytes (K * elem
// a multiple of 16; a 16-byte piece is then wholly inside K or wholly past
// it), element by element otherwise; B always element by element, adjacent
// lanes on adjacent columns. Out-of-range elements load as zero.
#include "gemm_common.hpp"

#include <type_traits>

namespace mb {
namespace {

constexpr int kGenTile = 128;
constexpr int kGenThreads = 256;
constexpr int kGenStageBytes = 64;                      // bytes of K per stage
constexpr int kGenRow = kGenStageBytes + 16;            // LDS row pitch
constexpr int kGenBuf = kGenTile * kGenRow;             // one operand, one stage

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

template <int DT>
struct GenFrag;

template <>
struct GenFrag<MB_DT_BFLOAT16> {
    typedef u32x4 T;
    static constexpr int kSub = 2;   // K substeps of 16 per stage
    __device__ static f32x16 mfma(const T& a, const T& b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                        c, 0, 0, 0);
    }
};
template <>
struct GenFrag<MB_DT_FLOAT16> : GenFrag<MB_DT_BFLOAT16> {
    __device__ static f32x16 mfma(const T& a, const T& b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b),
                                                       c, 0, 0, 0);
    }
};
// Format code 0 = e4m3, 1 = e5m2 (both operands); zero scale operands select
// the unscaled encoding.
template <>
struct GenFrag<MB_DT_FLOAT8_E4M3FN> {
    typedef i32x8 T;
    static constexpr int kSub = 1;   // one 64-deep MFMA per stage
    __device__ static f32x16 mfma(const T& a, const T& b, f32x16 c) {
        return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
    }
};
template <>
struct GenFrag<MB_DT_FLOAT8_E5M2> : GenFrag<MB_DT_FLOAT8_E4M3FN> {
    __device__ static f32x16 mfma(const T& a, const T& b, f32x16 c) {
        return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 1, 1, 0, 0, 0, 0);
    }
};

template <int DT, bool VEC_A>
__global__ void __launch_bounds__(kGenThreads)
gemm_generic_kernel(const unsigned char* __restrict__ A, const unsigned char* __restrict__ B, void* __restrict__ C,
                    int64_t M, int64_t N, int64_t K, float alpha) {
    typedef GenFrag<DT> Fr;
    constexpr int E = is_fp8(DT) ? 1 : 2;
    constexpr int BK = kGenStageBytes / E;       // K elements per stage
    constexpr int HALF = BK / 2;                 // elements a thread stages per operand
    __shared__ __attribute__((aligned(16))) unsigned char lds_a[2][kGenBuf];
    __shared__ __attribute__((aligned(16))) unsigned char lds_b[2][kGenBuf];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int64_t m0 = (int64_t)blockIdx.y * kGenTile;
    const int64_t n0 = (int64_t)blockIdx.x * kGenTile;

    // Staging assignment: A row ar, K half ah; B column bc, K half bh.
    const int ar = tid >> 1, ah = tid & 1;
    const int bc = tid & (kGenTile - 1), bh = tid >> 7;
    const int64_t a_row = m0 + ar, b_col = n0 + bc;

    // One element of A or B (zero-extended), and 32 bytes of them packed in order.
    auto elem = [](const unsigned char* p) __attribute__((always_inline)) -> unsigned {
        if constexpr (E == 1) return (unsigned)*p;
        else return (unsigned)*reinterpret_cast<const uint16_t*>(p);
    };
    auto pack = [](const unsigned* v, u32x4* st) __attribute__((always_inline)) {
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            unsigned word;
            if constexpr (E == 2) word = v[2 * w] | (v[2 * w + 1] << 16);
            else word = v[4 * w] | (v[4 * w + 1] << 8) | (v[4 * w + 2] << 16) | (v[4 * w + 3] << 24);
            st[w >> 2][w & 3] = word;
        }
    };
    // The next stage's loads land in these registers while the current
    // stage's MFMAs run; element loads stay unpacked until the LDS store, so
    // nothing waits for them before it.
    u32x4 sa[2];
    unsigned va[VEC_A ? 1 : HALF], vb[HALF];
    // FULL: the stage lies wholly inside K, so only the row / column bound is checked.
    auto load_stage = [&](int64_t k0, auto full) __attribute__((always_inline)) {
        constexpr bool FULL = decltype(full)::value;
        const int64_t ka = k0 + (int64_t)ah * HALF;
        if constexpr (VEC_A) {
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const int64_t k = ka + p * (16 / E);
                sa[p] = (a_row < M && (FULL || k < K)) ? *reinterpret_cast<const u32x4*>(A + (a_row * K + k) * E)
                                                       : (u32x4){0u, 0u, 0u, 0u};
            }
        } else {
            const unsigned char* pa = A + (a_row * K + ka) * E;
#pragma unroll 32
            for (int e = 0; e < HALF; ++e) va[e] = (a_row < M && (FULL || ka + e < K)) ? elem(pa + e * E) : 0u;
        }
        const int64_t kb = k0 + (int64_t)bh * HALF;
        const unsigned char* pb = B + (kb * N + b_col) * E;
        const int64_t ldb = N * E;
#pragma unroll 32
        for (int e = 0; e < HALF; ++e) vb[e] = (b_col < N && (FULL || kb + e < K)) ? elem(pb + e * ldb) : 0u;
    };
    auto load = [&](int64_t st) __attribute__((always_inline)) {
        if (st < K / BK) load_stage(st * BK, std::true_type{});
        else load_stage(st * BK, std::false_type{});
    };
    auto store_stage = [&](int buf) __attribute__((always_inline)) {
        if constexpr (!VEC_A) pack(va, sa);
        u32x4 sb[2];
        pack(vb, sb);
        unsigned char* pa = lds_a[buf] + ar * kGenRow + ah * 32;
        unsigned char* pb = lds_b[buf] + bc * kGenRow + bh * 32;
        *reinterpret_cast<u32x4*>(pa) = sa[0];
        *reinterpret_cast<u32x4*>(pa + 16) = sa[1];
        *reinterpret_cast<u32x4*>(pb) = sb[0];
        *reinterpret_cast<u32x4*>(pb + 16) = sb[1];
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // Lane l reads row (l % 32) of a fragment; its K bytes within the stage:
    // 16-bit substep s: 32 s + 16 (l / 32) .. +15; fp8: 32 (l / 32) .. +31.
    const int frow = lane & 31;
    const int fk = (lane >> 5) * (Fr::kSub == 2 ? 16 : 32);
    auto compute = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < Fr::kSub; ++s) {
            typename Fr::T fa[2], fb[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const unsigned char* p = lds_a[buf] + (wm * 64 + i * 32 + frow) * kGenRow + s * 32 + fk;
                const unsigned char* q = lds_b[buf] + (wn * 64 + i * 32 + frow) * kGenRow + s * 32 + fk;
                if constexpr (Fr::kSub == 2) {
                    fa[i] = *reinterpret_cast<const u32x4*>(p);
                    fb[i] = *reinterpret_cast<const u32x4*>(q);
                } else {
                    const u32x4 a0 = *reinterpret_cast<const u32x4*>(p), a1 = *reinterpret_cast<const u32x4*>(p + 16);
                    const u32x4 b0 = *reinterpret_cast<const u32x4*>(q), b1 = *reinterpret_cast<const u32x4*>(q + 16);
                    fa[i] = (i32x8){(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3],
                                    (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
                    fb[i] = (i32x8){(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3],
                                    (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
                }
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = Fr::mfma(fa[i], fb[j], acc[i][j]);
        }
    };

    const int64_t stages = (K + BK - 1) / BK;
    load(0);
    store_stage(0);
    __syncthreads();
    for (int64_t kt = 0; kt < stages; ++kt) {
        const bool more = kt + 1 < stages;
        if (more) load(kt + 1);
        compute((int)(kt & 1));
        if (more) store_stage((int)((kt + 1) & 1));
        __syncthreads();
    }

    // Epilogue: accumulator register r = 4g + q of fragment (i, j) holds
    // C[row 32 i + 8 g + 4 (l / 32) + q][column 32 j + l % 32] of the wave's
    // 64 x 64; lanes 0-31 of a store cover 32 consecutive columns of one row.
    const int64_t col_w = n0 + wn * 64 + (lane & 31);
    const int64_t row_w = m0 + wm * 64 + 4 * (lane >> 5);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = row_w + 32 * i + 8 * (r >> 2) + (r & 3);
                const int64_t col = col_w + 32 * j;
                if (row < M && col < N) store_out<DT>(C, row * N + col, acc[i][j][r] * alpha);
            }
}

template <int DT>
void launch_generic(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, float alpha,
                    dim3 grid, hipStream_t stream) {
    const auto* a = static_cast<const unsigned char*>(A);
    const auto* b = static_cast<const unsigned char*>(B);
    constexpr int E = is_fp8(DT) ? 1 : 2;
    if ((K * E) % 16 == 0)
        hipLaunchKernelGGL((gemm_generic_kernel<DT, true>), grid, dim3(kGenThreads), 0, stream, a, b, C, M, N, K,
                           alpha);
    else
        hipLaunchKernelGGL((gemm_generic_kernel<DT, false>), grid, dim3(kGenThreads), 0, stream, a, b, C, M, N, K,
                           alpha);
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
    plan->tile_k = is_fp8(dtype) ? 64 : 32;
    plan->wave_grid_m = 2;
    plan->wave_grid_n = 2;
    plan->wave_tile_m = 2;
    plan->wave_tile_n = 2;
    plan->frag_m = 32;
    plan->frag_n = 32;
    plan->frag_k = is_fp8(dtype) ? 64 : 16;
    plan->k_stages = 2;
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
        case MB_DT_BFLOAT16: launch_generic<MB_DT_BFLOAT16>(A, B, C, M, N, K, alpha, grid, stream); break;
        case MB_DT_FLOAT16: launch_generic<MB_DT_FLOAT16>(A, B, C, M, N, K, alpha, grid, stream); break;
        case MB_DT_FLOAT8_E4M3FN: launch_generic<MB_DT_FLOAT8_E4M3FN>(A, B, C, M, N, K, alpha, grid, stream); break;
        case MB_DT_FLOAT8_E5M2: launch_generic<MB_DT_FLOAT8_E5M2>(A, B, C, M, N, K, alpha, grid, stream); break;
        default:
            set_error("generic GEMM: unsupported dtype %d", dtype);
            return MB_ERR_UNSUPPORTED;
    }
    MB_HIP_TRY(hipGetLastError());
    return MB_OK;
}

}  // namespace mb

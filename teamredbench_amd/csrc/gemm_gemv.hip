// Small-M GEMM for gfx950 (M <= 4, bf16 / fp16): C (M x N) = A (M x K) * B
// (K x N), all row-major, fp32 accumulation, one rounding to the input type.
//
// With a handful of rows of A the work is a stream over B (2 * K * N bytes)
// and the matrix cores would multiply mostly padding, so this path keeps B
// out of LDS and off the MFMAs: every lane reads 16 bytes (8 columns) of a
// row of B per load and multiplies them by that row's A values with fp32
// FMAs. A block covers 256 columns; each of its 8 half-waves takes chunks of
// 8 consecutive K rows (8 B-row loads and one 16-byte load per row of A per
// chunk), several chunks in flight. The 8 partial sums of a column are added
// through LDS at the end. K is split over blocks until the
// grid covers the GPU twice; the splits' fp32 partials go to the caller's
// workspace and a second kernel adds them (gemm_gemv_reduce_kernel) and
// rounds once.
#include "gemm_common.hpp"

#include <algorithm>

namespace mb {
namespace {

constexpr int kGvThreads = 256;
constexpr int kGvCols = 256;         // 32 lanes x 8 columns
constexpr int kGvHalfWaves = 8;      // 4 waves x 2 half-waves, each on its own K chunks
constexpr int kGvChunk = 8;          // consecutive K rows per half-wave chunk (one 16-byte A load)
constexpr int kGvUnroll = 2;         // chunks in flight per lane
constexpr int kGvMaxM = 4;
constexpr int64_t kGvMaxSplits = 512;   // the reduction adds up to 512 planes in one trip

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

template <int DT>
__device__ __forceinline__ float elem(unsigned word, int hi) {
    if constexpr (DT == MB_DT_BFLOAT16) {
        return __uint_as_float(hi ? (word & 0xffff0000u) : (word << 16));
    } else {
        const unsigned short h = hi ? (unsigned short)(word >> 16) : (unsigned short)(word & 0xffffu);
        return (float)__builtin_bit_cast(_Float16, h);
    }
}

template <int DT>
__device__ __forceinline__ uint16_t round16(float v) {
    if constexpr (DT == MB_DT_BFLOAT16) return __builtin_bit_cast(uint16_t, (__bf16)v);
    else return __builtin_bit_cast(uint16_t, (_Float16)v);
}

template <int DT, int MR>
__global__ void __launch_bounds__(kGvThreads)
gemm_gemv_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, uint16_t* __restrict__ C,
                 int N, int K, int k_len, float* __restrict__ ws) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int hw = wave * 2 + (lane >> 5);                      // half-wave 0..7
    const int col0 = (int)blockIdx.x * kGvCols + 8 * (lane & 31);
    const bool in_cols = col0 < N;                               // N % 8 == 0: all 8 columns or none
    const int kb = (int)blockIdx.y * k_len;                      // k_len and K are multiples of 8
    const int ke = min(K, kb + k_len);

    float acc[MR][8];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[m][e] = 0.f;

    // Half-wave hw takes the chunks of 8 consecutive K rows numbered hw,
    // hw + 8, ...: 8 row loads of B (16 bytes each) and one 16-byte load of
    // A per row of A per chunk, kGvUnroll chunks in flight.
    for (int c0 = kb + kGvChunk * hw; c0 < ke; c0 += kGvChunk * kGvHalfWaves * kGvUnroll) {
        u32x4 bv[kGvUnroll][kGvChunk];
        u32x4 av[kGvUnroll][MR];
#pragma unroll
        for (int u = 0; u < kGvUnroll; ++u) {
            const int k = c0 + kGvChunk * kGvHalfWaves * u;
            const bool live = k < ke && in_cols;
#pragma unroll
            for (int r = 0; r < kGvChunk; ++r)
                bv[u][r] = live ? *reinterpret_cast<const u32x4*>(B + (int64_t)(k + r) * N + col0)
                                : (u32x4){0u, 0u, 0u, 0u};
#pragma unroll
            for (int m = 0; m < MR; ++m)
                av[u][m] = live ? *reinterpret_cast<const u32x4*>(A + (int64_t)m * K + k) : (u32x4){0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < kGvUnroll; ++u)
#pragma unroll
            for (int r = 0; r < kGvChunk; ++r)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float b = elem<DT>(bv[u][r][e >> 1], e & 1);
#pragma unroll
                    for (int m = 0; m < MR; ++m) acc[m][e] = fmaf(elem<DT>(av[u][m][r >> 1], r & 1), b, acc[m][e]);
                }
    }

    // Sum the 8 half-waves' partials: red[hw][m][column in block].
    __shared__ __attribute__((aligned(16))) float red[kGvHalfWaves][MR][kGvCols];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        *reinterpret_cast<f32x4*>(&red[hw][m][8 * (lane & 31)]) = (f32x4){acc[m][0], acc[m][1], acc[m][2], acc[m][3]};
        *reinterpret_cast<f32x4*>(&red[hw][m][8 * (lane & 31) + 4]) =
            (f32x4){acc[m][4], acc[m][5], acc[m][6], acc[m][7]};
    }
    __syncthreads();
    const int t = threadIdx.x;
    const int col = (int)blockIdx.x * kGvCols + t;
    if (col >= N) return;
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        float s = 0.f;
#pragma unroll
        for (int r = 0; r < kGvHalfWaves; ++r) s += red[r][m][t];
        if (ws != nullptr) {
            ws[((int64_t)blockIdx.y * MR + m) * N + col] = s;
        } else {
            C[(int64_t)m * N + col] = round16<DT>(s);
        }
    }
}

// C[i] = round(sum_s ws[s][i]) over `splits` partial planes of mn elements.
// A block of W waves takes 64 consecutive elements; its wave w adds planes
// w, w + W, ... with L loads in flight at once, so W * L splits cost one trip
// to memory (the planes were just written by the previous kernel: the pass is
// latency-bound), and the waves' sums meet in LDS and are added in wave order.
// Above 16 splits the launch takes 16 waves, each with the fewest loads that
// cover the split count in one trip: a wave with fewer loads in flight is
// done sooner, and on MI355X 16 waves of 8 loads added 128 splits of a
// 1 x 1024 partial 0.7 us sooner than 4 waves of 32 (7.9 vs 8.6 us for the
// whole 1 x 1024 x 8192 product).
constexpr int kGvReduceCols = 64;

template <int DT, int W, int L>
__global__ void __launch_bounds__(kGvReduceCols * W)
gemm_gemv_reduce_kernel(const float* __restrict__ ws, uint16_t* __restrict__ C, int64_t mn, int splits) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t i = (int64_t)blockIdx.x * kGvReduceCols + lane;
    float s = 0.f;
    for (int p0 = 0; p0 < splits; p0 += W * L) {
        float v[L];
#pragma unroll
        for (int j = 0; j < L; ++j) {
            const int p = p0 + wave + W * j;
            v[j] = (p < splits && i < mn) ? ws[(int64_t)p * mn + i] : 0.f;
        }
#pragma unroll
        for (int j = 0; j < L; ++j) s += v[j];
    }
    __shared__ float red[W][kGvReduceCols];
    red[wave][lane] = s;
    __syncthreads();
    if (wave != 0 || i >= mn) return;
    float t = red[0][lane];
#pragma unroll
    for (int w = 1; w < W; ++w) t += red[w][lane];
    C[i] = round16<DT>(t);
}

template <int DT>
int launch_reduce(const float* ws, uint16_t* C, int64_t mn, int splits, hipStream_t stream) {
    typedef void (*Reduce)(const float*, uint16_t*, int64_t, int);
    Reduce reduce = gemm_gemv_reduce_kernel<DT, 16, 32>;
    int waves = 16;
    if (splits <= 4) reduce = gemm_gemv_reduce_kernel<DT, 4, 1>, waves = 4;
    else if (splits <= 8) reduce = gemm_gemv_reduce_kernel<DT, 4, 2>, waves = 4;
    else if (splits <= 16) reduce = gemm_gemv_reduce_kernel<DT, 4, 4>, waves = 4;
    else if (splits <= 32) reduce = gemm_gemv_reduce_kernel<DT, 16, 2>;
    else if (splits <= 64) reduce = gemm_gemv_reduce_kernel<DT, 16, 4>;
    else if (splits <= 128) reduce = gemm_gemv_reduce_kernel<DT, 16, 8>;
    else if (splits <= 256) reduce = gemm_gemv_reduce_kernel<DT, 16, 16>;
    hipLaunchKernelGGL(reduce, dim3((unsigned)((mn + kGvReduceCols - 1) / kGvReduceCols)),
                       dim3(kGvReduceCols * waves), 0, stream, ws, C, mn, splits);
    MB_HIP_TRY(hipGetLastError());
    return MB_OK;
}

template <int DT, int MR>
int launch_m(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, const GemmPlan& plan,
             void* workspace, hipStream_t stream) {
    const int splits = plan.split_k;
    const int k_len = (int)((K / kGvChunk + splits - 1) / splits) * kGvChunk;   // whole chunks per split
    const dim3 grid((unsigned)((N + kGvCols - 1) / kGvCols), (unsigned)splits);
    float* ws = splits > 1 ? static_cast<float*>(workspace) : nullptr;
    hipLaunchKernelGGL((gemm_gemv_kernel<DT, MR>), grid, dim3(kGvThreads), 0, stream,
                       static_cast<const uint16_t*>(A), static_cast<const uint16_t*>(B), static_cast<uint16_t*>(C),
                       (int)N, (int)K, k_len, ws);
    MB_HIP_TRY(hipGetLastError());
    if (splits > 1) return launch_reduce<DT>(ws, static_cast<uint16_t*>(C), M * N, splits, stream);
    return MB_OK;
}

template <int DT>
int launch_dt(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, const GemmPlan& plan,
              void* workspace, hipStream_t stream) {
    switch (M) {
        case 1: return launch_m<DT, 1>(A, B, C, M, N, K, plan, workspace, stream);
        case 2: return launch_m<DT, 2>(A, B, C, M, N, K, plan, workspace, stream);
        case 3: return launch_m<DT, 3>(A, B, C, M, N, K, plan, workspace, stream);
        default: return launch_m<DT, 4>(A, B, C, M, N, K, plan, workspace, stream);
    }
}

}  // namespace

// Takes bf16/fp16 with 1 <= M <= 4, N % 8 == 0 and K % 8 == 0 (16-byte
// loads of B's rows and of A's 8-row chunks); other cases return
// MB_ERR_SHAPE and go to the MFMA kernels.
int gemm_gemv_plan(int dtype, int64_t M, int64_t N, int64_t K, const DeviceProps& props, GemmPlan* plan) {
    if ((dtype != MB_DT_BFLOAT16 && dtype != MB_DT_FLOAT16) || M < 1 || M > kGvMaxM || N % 8 != 0 || K % 8 != 0)
        return MB_ERR_SHAPE;
    // The kernel's K and column indices are 32-bit: split starts (at most
    // K + 8 x splits), the chunk loop's last step (128 rows past K) and the
    // last block's columns (up to 248 past N) stay below 2^31.
    if (K > (int64_t(1) << 31) - 8 * kGvMaxSplits - 256 || N > (int64_t(1) << 31) - 256) return MB_ERR_SHAPE;
    const int64_t cus = props.cu_count > 0 ? props.cu_count : 256;
    const int64_t groups = (N + kGvCols - 1) / kGvCols;
    // Split K until the grid holds 8 blocks per CU (the loads they keep in
    // flight are what streams B), keeping at least one chunk per half-wave in
    // each split, the fp32 partials (splits x M x N x 4 bytes) within 1/16 of
    // B's bytes (K x N x 2), since the reduction pass reads them back, and at
    // most 512 splits, which that pass adds in one trip to memory. On MI355X
    // with B from HBM, against 2 blocks per CU and no partials bound: 1 x 4096
    // x 4096 10.5 -> 9.9 us (32 -> 64 splits), 1 x 8192 x 8192 28.3 -> 26.3
    // (16 -> 64), 4 x 8192 x 8192 31.6 -> 29.3, 1 x 1024 x 8192 8.7 -> 7.9
    // (128, reduction as above), 2 x 28672 x 4096 44.4 -> 44.2 (4 -> 16).
    int64_t splits = 1;
    while (groups * splits * 2 <= 8 * cus && K / (splits * 2) >= kGvChunk * kGvHalfWaves &&
           splits * 2 * 32 * M <= K && splits < kGvMaxSplits)
        splits *= 2;
    const int64_t force_splits = tuning(MB_TUNE_GEMM_SPLITS);
    if (force_splits >= 1) splits = force_splits;
    plan->implementation = "gfx950_gemv_stream";
    plan->threads = kGvThreads;
    plan->grid = (int)(groups * splits);
    plan->tile_m = (int)M;
    plan->tile_n = kGvCols;
    plan->tile_k = kGvChunk * kGvHalfWaves;
    plan->wave_grid_m = 1;
    plan->wave_grid_n = 1;
    plan->wave_tile_m = 1;
    plan->wave_tile_n = 1;
    plan->frag_m = plan->frag_n = plan->frag_k = 0;   // no matrix-core fragments on this path
    plan->k_stages = kGvUnroll;
    plan->split_k = (int)splits;
    plan->tile_group_m = 1;
    plan->workspace = splits > 1 ? (size_t)splits * (size_t)M * (size_t)N * sizeof(float) : 0;
    plan->variant = kVariantGemv;
    return MB_OK;
}

int gemm_gemv_launch(int dtype, const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
                     void* workspace, const GemmPlan& plan, hipStream_t stream) {
    switch (dtype) {
        case MB_DT_BFLOAT16: return launch_dt<MB_DT_BFLOAT16>(A, B, C, M, N, K, plan, workspace, stream);
        case MB_DT_FLOAT16: return launch_dt<MB_DT_FLOAT16>(A, B, C, M, N, K, plan, workspace, stream);
        default:
            set_error("small-M GEMM: unsupported dtype %d", dtype);
            return MB_ERR_UNSUPPORTED;
    }
}

}  // namespace mb

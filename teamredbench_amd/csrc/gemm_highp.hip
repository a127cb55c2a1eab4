// fp32 and fp64 GEMM for gfx950 on the full-precision matrix cores:
// C = A * B, A (M x K), B (K x N), C (M x N) all row-major in the input type,
// accumulated in that type by the MFMAs (fp32: v_mfma_f32_32x32x2_f32; fp64:
// v_mfma_f64_16x16x4_f64), for any M, N, K >= 1.
//
// These MFMAs deliver 1/16 (fp32) and 1/32 (fp64) of the bf16 rate, so a
// 128 x 128 block tile with 64 bytes of K per stage already needs far less
// LDS and L2 bandwidth than the units can use; the kernel keeps the plain
// structure: operands come through registers into a double-buffered LDS tile
// (one barrier per stage), and the next stage's global loads are in flight
// while the current stage's MFMAs run.
//
// LDS layout per stage: A transposed to [BK][BM + pad] (the MFMA hands each
// lane one A row at a fixed k, so consecutive lanes read consecutive
// addresses) and B as [BK][BN + pad]. The threads that load A are laid out
// rows first, so the transposing stores of a wave also go to 64 consecutive
// rows of one k. The 128-byte pad puts the lanes that
// read the next k (fp32: lanes 32-63; fp64: every other group of 16) on the
// other half of the 64 banks, so operand reads are conflict-free. 4 waves in
// a 2 x 2 grid own 64 x 64 of C each.
//
// Global loads move 16 bytes per lane when the row pitches keep 16-byte
// alignment (K and N multiples of 16 / elem bytes); otherwise element-wise.
// Either way elements outside the matrices read as zero and stores outside C
// are skipped, so ragged edges need no separate kernel.
#include "gemm_common.hpp"

namespace mb {
namespace {

constexpr int kHpBM = 128, kHpBN = 128, kHpThreads = 256;

template <typename T>
struct HighpTraits;

// fp32: 32 x 32 fragments, K = 2 per MFMA; lane l supplies A[row l%32][k l/32]
// and B[k l/32][col l%32]; accumulator r = 4g + q holds row 8g + 4*(l/32) + q,
// col l%32.
template <>
struct HighpTraits<float> {
    static constexpr int kBK = 16;        // K elements per stage (64 bytes)
    static constexpr int kFrag = 32;
    static constexpr int kFragK = 2;
    static constexpr int kAcc = 16;
    typedef f32x16 Acc;
    __device__ static inline Acc mfma(float a, float b, Acc c) {
        return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
    }
    // Row (within the fragment) of accumulator register r for lane l.
    __device__ static inline int acc_row(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }
    __device__ static inline int lane_k(int lane) { return lane >> 5; }
    __device__ static inline int lane_mn(int lane) { return lane & 31; }
};

// fp64: 16 x 16 fragments, K = 4 per MFMA; lane l supplies A[row l%16][k l/16]
// and B[k l/16][col l%16]; accumulator r holds row 4r + l/16, col l%16 (each
// register is one group of 4 rows interleaved over the four 16-lane blocks,
// unlike the fp32 16x16 form, whose lane block owns 4 consecutive rows).
template <>
struct HighpTraits<double> {
    static constexpr int kBK = 8;         // K elements per stage (64 bytes)
    static constexpr int kFrag = 16;
    static constexpr int kFragK = 4;
    static constexpr int kAcc = 4;
    typedef f64x4 Acc;
    __device__ static inline Acc mfma(double a, double b, Acc c) {
        return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
    }
    __device__ static inline int acc_row(int r, int lane) { return 4 * r + (lane >> 4); }
    __device__ static inline int lane_k(int lane) { return lane >> 4; }
    __device__ static inline int lane_mn(int lane) { return lane & 15; }
};

template <typename T, bool VEC>
__global__ void __launch_bounds__(kHpThreads)
gemm_highp_kernel(const T* __restrict__ A, const T* __restrict__ B, T* __restrict__ C, int64_t M, int64_t N,
                  int64_t K) {
    typedef HighpTraits<T> Tr;
    typedef typename Tr::Acc Acc;
    constexpr int BK = Tr::kBK;
    constexpr int F = Tr::kFrag;
    constexpr int FR = 64 / F;                    // fragments per wave side (wave tile 64 x 64)
    constexpr int V = 16 / (int)sizeof(T);        // elements per 16-byte vector
    constexpr int PAD = 128 / (int)sizeof(T);     // 128 bytes: half the LDS banks
    constexpr int A_LD = kHpBM + PAD;             // padded row of the transposed A tile
    constexpr int B_LD = kHpBN + PAD;
    constexpr int A_VECS = kHpBM * BK / V;        // 16-byte pieces per stage
    constexpr int B_VECS = BK * kHpBN / V;
    constexpr int PER_A = A_VECS / kHpThreads, PER_B = B_VECS / kHpThreads;
    static_assert(A_VECS % kHpThreads == 0 && B_VECS % kHpThreads == 0, "stage must split over the threads");

    __shared__ T sa[2][BK][A_LD];
    __shared__ __attribute__((aligned(16))) T sb[2][BK][B_LD];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int64_t m0 = (int64_t)blockIdx.y * kHpBM, n0 = (int64_t)blockIdx.x * kHpBN;

    T ra[PER_A][V], rb[PER_B][V];
    // Global -> registers for the stage at k0; zero outside the matrices.
    auto load = [&](int64_t k0) {
#pragma unroll
        for (int q = 0; q < PER_A; ++q) {
            const int v = tid + q * kHpThreads;
            const int row = v % kHpBM, kv = (v / kHpBM) * V;
            const int64_t gm = m0 + row, gk = k0 + kv;
            if constexpr (VEC) {
                if (gm < M && gk < K) {
                    *reinterpret_cast<u32x4*>(ra[q]) = *reinterpret_cast<const u32x4*>(A + gm * K + gk);
                } else {
#pragma unroll
                    for (int e = 0; e < V; ++e) ra[q][e] = T(0);
                }
            } else {
#pragma unroll
                for (int e = 0; e < V; ++e) ra[q][e] = (gm < M && gk + e < K) ? A[gm * K + gk + e] : T(0);
            }
        }
#pragma unroll
        for (int q = 0; q < PER_B; ++q) {
            const int v = tid + q * kHpThreads;
            const int kr = v / (kHpBN / V), cv = (v % (kHpBN / V)) * V;
            const int64_t gk = k0 + kr, gn = n0 + cv;
            if constexpr (VEC) {
                if (gk < K && gn < N) {
                    *reinterpret_cast<u32x4*>(rb[q]) = *reinterpret_cast<const u32x4*>(B + gk * N + gn);
                } else {
#pragma unroll
                    for (int e = 0; e < V; ++e) rb[q][e] = T(0);
                }
            } else {
#pragma unroll
                for (int e = 0; e < V; ++e) rb[q][e] = (gk < K && gn + e < N) ? B[gk * N + gn + e] : T(0);
            }
        }
    };
    // Registers -> LDS buffer `buf` (A transposed).
    auto store = [&](int buf) {
#pragma unroll
        for (int q = 0; q < PER_A; ++q) {
            const int v = tid + q * kHpThreads;
            const int row = v % kHpBM, kv = (v / kHpBM) * V;
#pragma unroll
            for (int e = 0; e < V; ++e) sa[buf][kv + e][row] = ra[q][e];
        }
#pragma unroll
        for (int q = 0; q < PER_B; ++q) {
            const int v = tid + q * kHpThreads;
            const int kr = v / (kHpBN / V), cv = (v % (kHpBN / V)) * V;
            *reinterpret_cast<u32x4*>(&sb[buf][kr][cv]) = *reinterpret_cast<const u32x4*>(rb[q]);
        }
    };

    Acc acc[FR][FR];
#pragma unroll
    for (int i = 0; i < FR; ++i)
#pragma unroll
        for (int j = 0; j < FR; ++j)
#pragma unroll
            for (int r = 0; r < Tr::kAcc; ++r) acc[i][j][r] = T(0);

    const int lk = Tr::lane_k(lane), lmn = Tr::lane_mn(lane);
    const int64_t ksteps = (K + BK - 1) / BK;
    load(0);
    store(0);
    __syncthreads();
    for (int64_t kt = 0; kt < ksteps; ++kt) {
        const int buf = (int)(kt & 1);
        if (kt + 1 < ksteps) load((kt + 1) * BK);
#pragma unroll
        for (int kk = 0; kk < BK; kk += Tr::kFragK) {
            T a[FR], b[FR];
#pragma unroll
            for (int i = 0; i < FR; ++i) a[i] = sa[buf][kk + lk][wm * 64 + i * F + lmn];
#pragma unroll
            for (int j = 0; j < FR; ++j) b[j] = sb[buf][kk + lk][wn * 64 + j * F + lmn];
#pragma unroll
            for (int i = 0; i < FR; ++i)
#pragma unroll
                for (int j = 0; j < FR; ++j) acc[i][j] = Tr::mfma(a[i], b[j], acc[i][j]);
        }
        if (kt + 1 < ksteps) store(buf ^ 1);
        __syncthreads();
    }

    // Epilogue: a register index gives each lane one row; consecutive lanes
    // hold consecutive columns of it.
#pragma unroll
    for (int i = 0; i < FR; ++i) {
#pragma unroll
        for (int j = 0; j < FR; ++j) {
            const int64_t gn = n0 + wn * 64 + j * F + lmn;
#pragma unroll
            for (int r = 0; r < Tr::kAcc; ++r) {
                const int64_t gm = m0 + wm * 64 + i * F + Tr::acc_row(r, lane);
                if (gm < M && gn < N) C[gm * N + gn] = acc[i][j][r];
            }
        }
    }
}

template <typename T>
int launch_typed(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
    constexpr int V = 16 / (int)sizeof(T);
    const dim3 grid((unsigned)((N + kHpBN - 1) / kHpBN), (unsigned)((M + kHpBM - 1) / kHpBM));
    const T* a = static_cast<const T*>(A);
    const T* b = static_cast<const T*>(B);
    T* c = static_cast<T*>(C);
    if (K % V == 0 && N % V == 0) {
        hipLaunchKernelGGL((gemm_highp_kernel<T, true>), grid, dim3(kHpThreads), 0, stream, a, b, c, M, N, K);
    } else {
        hipLaunchKernelGGL((gemm_highp_kernel<T, false>), grid, dim3(kHpThreads), 0, stream, a, b, c, M, N, K);
    }
    MB_HIP_TRY(hipGetLastError());
    return MB_OK;
}

}  // namespace

int gemm_highp_plan(int dtype, int64_t M, int64_t N, int64_t K, GemmPlan* plan) {
    (void)K;
    const bool f64 = dtype == MB_DT_FLOAT64;
    const int64_t gx = (N + kHpBN - 1) / kHpBN, gy = (M + kHpBM - 1) / kHpBM;
    if (gy > 65535 || gx > INT32_MAX) {
        set_error("fp32/fp64 GEMM: M=%lld N=%lld too large", (long long)M, (long long)N);
        return MB_ERR_SHAPE;
    }
    plan->implementation = f64 ? "gfx950_mfma_f64_16x16x4" : "gfx950_mfma_f32_32x32x2";
    plan->threads = kHpThreads;
    plan->grid = (int)(gx * gy);
    plan->tile_m = kHpBM;
    plan->tile_n = kHpBN;
    plan->tile_k = f64 ? HighpTraits<double>::kBK : HighpTraits<float>::kBK;
    plan->wave_grid_m = 2;
    plan->wave_grid_n = 2;
    plan->frag_m = plan->frag_n = f64 ? 16 : 32;
    plan->frag_k = f64 ? 4 : 2;
    plan->wave_tile_m = plan->wave_tile_n = 64 / plan->frag_m;
    plan->k_stages = 2;
    plan->split_k = 1;
    plan->tile_group_m = 1;
    plan->workspace = 0;
    plan->variant = kVariantHighp;
    return MB_OK;
}

int gemm_highp_launch(int dtype, const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
                      hipStream_t stream) {
    switch (dtype) {
        case MB_DT_FLOAT32: return launch_typed<float>(A, B, C, M, N, K, stream);
        case MB_DT_FLOAT64: return launch_typed<double>(A, B, C, M, N, K, stream);
        default:
            set_error("fp32/fp64 GEMM: unsupported dtype %d", dtype);
            return MB_ERR_UNSUPPORTED;
    }
}

}  // namespace mb

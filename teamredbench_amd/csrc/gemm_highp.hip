// fp32 and fp64 GEMM for gfx950 on the full-precision matrix cores:
// C = A * B, A (M x K), B (K x N), C (M x N) all row-major in the input type,
// accumulated in that type by the MFMAs (fp32: v_mfma_f32_32x32x2_f32; fp64:
// v_mfma_f64_16x16x4_f64), for any M, N, K >= 1.
//
// Two kernels. Shapes whose A and B rows start on 16 bytes run on an LDS-DMA
// ring like the 16-bit pipelined kernel (gemm_f32_dma_kernel,
// gemm_f64_dma_kernel below: 95% and 93% of peak at 8192^3): fp64 on 128 x 128
// tiles, fp32 on 256 x 256 tiles where their rounds fill the CUs and on
// 128 x 128 tiles elsewhere (highp_dma_config). Every other shape runs the
// register-staged kernel that follows, which takes any shape and stays near
// 80% of peak:
//
// Register-staged kernel. Operands come through registers into a
// double-buffered LDS tile (one barrier per stage), and the next stage's
// global loads are in flight while the current stage's MFMAs run. A 128 x 128
// block tile with 64 bytes of K per stage, 4 waves in a 2 x 2 grid owning
// 64 x 64 of C each.
//
// LDS layout per stage: A transposed to [BK][BM + pad] (the MFMA hands each
// lane one A row at a fixed k, so consecutive lanes read consecutive
// addresses) and B as [BK][BN + pad]. The threads that load A are laid out
// rows first, so the transposing stores of a wave also go to 64 consecutive
// rows of one k. The 128-byte pad puts the lanes that
// read the next k (fp32: lanes 32-63; fp64: every other group of 16) on the
// other half of the 64 banks, so operand reads are conflict-free.
//
// Global loads move 16 bytes per lane when the row pitches keep 16-byte
// alignment (K and N multiples of 16 / elem bytes); otherwise element-wise.
// Either way elements outside the matrices read as zero and stores outside C
// are skipped, so ragged edges need no separate kernel.
#include "gemm_pipeline.hpp"

#include <cstdlib>
#include <utility>

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

// ---- fp32 on an LDS-DMA ring (256 x 256 and 128 x 128 tiles) ---------------
//
// The register-staged kernel above tops out near 80% of the fp32 peak: its
// load, LDS store and barrier phases leave the matrix pipe idle between MFMA
// groups. This one follows the 16-bit pipelined kernel instead: A and B go
// global -> LDS with buffer_load ... lds into a ring of 4 slots (one barrier
// per stage, loads of stage kt + 3 issued into the slot stage kt - 1 just
// vacated), and on 256 x 256 tiles each wave owns 128 x 128 of C as 4 x 4
// fragments of v_mfma_f32_32x32x2_f32, so a stage is 128 MFMAs (8192 cycles)
// against one barrier.
//
// K order inside a stage. The MFMA sums two K values, one from each lane
// half; here lane half h supplies K 8h + t at step t (t = 0..7), which is any
// fixed permutation of the stage's 16 K values and leaves the sum the same.
// So a lane's A operands for the whole stage are 8 consecutive floats of one
// row -- two ds_read_b128 per fragment from the [256 rows][64 B] A slot (the
// 16-bit kernel's layout and swizzle) -- and its B operand at step t is one
// float of row 8h + t, read with ds_read_b32. B keeps its HBM layout ([16
// rows][1024 B]); rows 8..15 have their 16-byte chunks XOR 8, so the two lane
// halves, which read rows 8 apart (8 KiB, the same banks), land 128 bytes
// apart and the read is conflict-free.
//
// The MFMA takes the B operand first, so a lane's 16 accumulators of a
// fragment hold one C row, 4 runs of 4 consecutive columns; the epilogue
// stores them as 16-byte pieces straight from registers (a tile computes for
// milliseconds; its 256 KiB of C do not need LDS staging).
constexpr int kF32Stages = 4, kF32StageK = 16, kF32GroupM = 4;

__device__ __forceinline__ int swz_b32(int row) { return ((row >> 3) & 1) << 3; }

template <int BM, int BN, bool RAGGED_K = false>
__global__ void __launch_bounds__(256)
gemm_f32_dma_kernel(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M, int N,
                    int K, int tiles_m, int tiles_n) {
    // Per-tile sizes: waves in a 2 x 2 grid, fragments of 32 x 32.
    constexpr int WTM = BM / 2, WTN = BN / 2, FM = WTM / 32, FN = WTN / 32;
    constexpr int ABytes = BM * 64, BRow = BN * 4, BBytes = kF32StageK * BRow, Slot = ABytes + BBytes;
    constexpr int AInstr = ABytes / 1024 / 4, BInstr = BBytes / 1024 / 4, Loads = AInstr + BInstr;
    static_assert(AInstr >= 1 && BInstr >= 1 && WTM % 32 == 0 && WTN % 32 == 0 && BRow >= 256, "tile shape");
    __shared__ __attribute__((aligned(1024))) unsigned char ring[kF32Stages][Slot];
    const int tid = threadIdx.x, lane = tid & 63, half = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    int tm, tn;
    tile_coords((int)blockIdx.x, tiles_m * tiles_n, tiles_m, tiles_n, kF32GroupM, &tm, &tn);
    const int lda = K * 4, ldb = N * 4;
    // Buffer ranges end at A's row M and at B's last byte: rows of a partial
    // last M tile, and B's rows past K, load zeros; the columns of a partial
    // last N tile load the start of B's next row and are not stored.
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(A) + (int64_t)tm * BM * K, (short)0, min(BM, M - tm * BM) * lda, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(B) + (int64_t)tn * BN, (short)0, K * ldb - tn * BN * 4, kBufferFlags);
    int a_voff[AInstr], a_kbyte[AInstr], b_voff[BInstr];
#pragma unroll
    for (int q = 0; q < AInstr; ++q) {
        const int lin = (wave * AInstr + q) * 1024 + lane * 16;
        const int row = lin / 64, pchunk = (lin % 64) >> 4;
        a_kbyte[q] = (pchunk ^ swz_a(row)) << 4;
        a_voff[q] = row * lda + a_kbyte[q];
    }
#pragma unroll
    for (int q = 0; q < BInstr; ++q) {
        const int lin = (wave * BInstr + q) * 1024 + lane * 16;
        const int row = lin / BRow, pchunk = (lin % BRow) >> 4;
        b_voff[q] = row * ldb + ((pchunk ^ swz_b32(row)) << 4);
    }
    // DMA instruction q of stage kt into `slot`: A pieces first, then B.
    // RAGGED_K (K not a multiple of the stage): A pieces at or past K load zeros.
    auto issue_one = [&](int kt, int slot, auto idx) {
        constexpr int q = decltype(idx)::value;
        const unsigned base = (unsigned)(uintptr_t)(MB_LDS unsigned char*)ring[slot];
        if constexpr (q < AInstr)
            lds_dma16(ra, base + (wave * AInstr + q) * 1024,
                      RAGGED_K && a_kbyte[q] >= K * 4 - kt * 64 ? (int)0x80000000u : a_voff[q], kt * 64);
        else
            lds_dma16(rb, base + ABytes + (wave * BInstr + q - AInstr) * 1024, b_voff[q - AInstr],
                      kt * kF32StageK * ldb);
    };
    auto issue = [&](int kt, int slot) {
        [&]<int... Q>(std::integer_sequence<int, Q...>) {
            (issue_one(kt, slot, std::integral_constant<int, Q>{}), ...);
        }(std::make_integer_sequence<int, Loads>{});
    };

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int ksteps = (K + kF32StageK - 1) / kF32StageK, last = ksteps - 1;
#pragma unroll
    for (int st = 0; st < kF32Stages - 1; ++st) issue(min(st, last), st);
    const int a_row = wm * WTM + (lane & 31);
    const int b_col = wn * WTN + (lane & 31);
    // A operands: a[i][t] is K 8h + t of fragment i's row. Steps 0-3 use the
    // first 16-byte chunk, steps 4-7 the second, so the next stage's first
    // chunk is read into the registers steps 0-3 are done with (after the
    // mid-stage barrier) and its second chunk at the stage boundary, four
    // steps before it is needed: one register set.
    float a[FM][8];
    float b[4][FN];     // B operands of steps t .. t + 3, read two steps ahead
    auto read_a = [&](int kt, int e) {
        const unsigned char* slot = ring[kt % kF32Stages];
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const int row = a_row + 32 * i;
            // Whole float vectors: __builtin_bit_cast of a single ext_vector
            // element (bit_cast(float, v[w]) on a u32x4) is miscompiled by this
            // clang -- it reuses element 0 and drops the other loads.
            const f32x4 v = *reinterpret_cast<const f32x4*>(slot + row * 64 + (((2 * half + e) ^ swz_a(row)) << 4));
#pragma unroll
            for (int w = 0; w < 4; ++w) a[i][4 * e + w] = v[w];
        }
    };
    auto read_b = [&](int kt, int t, int set) {
        const unsigned char* sb = ring[kt % kF32Stages] + ABytes;
        const int row = 8 * half + t;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int col = b_col + 32 * j;
            b[set][j] =
                *reinterpret_cast<const float*>(sb + row * BRow + (((col >> 2) ^ swz_b32(row)) << 4) + 4 * (col & 3));
        }
    };
    // One barrier per stage, at its middle: it certifies that stage kt + 1 has
    // landed for every wave and that every wave is done with stage kt - 1's
    // slot, which takes stage kt + 3's loads. Those loads are spread over the
    // stage's second half, evenly between its MFMAs (issued back to back after
    // the barrier, they held the wave's issue for longer than the one MFMA in
    // flight covers). The next stage's operands are read under this stage's
    // MFMAs (A's first chunk after the barrier, its first two B operands in
    // the last two steps, A's second chunk at the boundary), so a stage
    // boundary has no wait. B is read two steps (8 or 32 MFMAs) ahead of its
    // use: on 128 x 128 tiles one step (4 MFMAs) did not cover the LDS
    // latency when two blocks share a CU (3072 x 6144 x 4096 ran 17% faster
    // with two; other shapes within 0.7%). Past the last stage the loads
    // repeat it (in bounds, never used).
    constexpr int kSteps = kF32StageK / 2, kMid = kSteps / 2;
    static_assert(kSteps % 4 == 0 && kMid >= 2, "B sets cycle with the stage; next-stage reads follow the barrier");
    constexpr int kMfma = FM * FN;                               // MFMAs per step
    constexpr int kLoadSteps = kSteps - kMid;
    static_assert(Loads % kLoadSteps == 0 && kMfma % (Loads / kLoadSteps) == 0, "loads spread evenly");
    constexpr int kLoadsPerStep = Loads / kLoadSteps, kLoadGap = kMfma / kLoadsPerStep;
    wait_vmcnt_and_barrier<Loads * (kF32Stages - 2)>();
    read_a(0, 0);
    read_a(0, 1);
    read_b(0, 0, 0);
    read_b(0, 1, 1);
    for (int kt = 0; kt < ksteps; ++kt) {
        const int load_kt = min(kt + kF32Stages - 1, last), load_slot = (kt + kF32Stages - 1) % kF32Stages;
        [&]<int... T>(std::integer_sequence<int, T...>) {
            ([&] {
                constexpr int t = T;
                if (t == 0 && kt > 0) read_a(kt, 1);
                if constexpr (t == kMid) {
                    wait_vmcnt_and_barrier<Loads * (kF32Stages - 3)>();
                    read_a(kt + 1, 0);
                }
                // (t + 2) & 3 is also the set of step t + 2 - kSteps of the next stage: kSteps % 4 == 0
                if constexpr (t + 2 < kSteps) read_b(kt, t + 2, (t + 2) & 3);
                else read_b(kt + 1, t + 2 - kSteps, (t + 2) & 3);
                __builtin_amdgcn_sched_barrier(0);
                [&]<int... Q>(std::integer_sequence<int, Q...>) {
                    ([&] {
                        constexpr int m = Q, i = m / FN, j = m % FN;
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(b[t & 3][j], a[i][t], acc[i][j], 0, 0, 0);
                        if constexpr (t >= kMid && m % kLoadGap == 0)
                            issue_one(load_kt, load_slot,
                                      std::integral_constant<int, (t - kMid) * kLoadsPerStep + m / kLoadGap>{});
                        __builtin_amdgcn_sched_barrier(0);   // keeps each load where it is placed
                    }(), ...);
                }(std::make_integer_sequence<int, kMfma>{});
            }(), ...);
        }(std::make_integer_sequence<int, kSteps>{});
    }
    wait_vmcnt_and_barrier<0>();

    // Accumulator register 4g + q of lane l holds C[row 32i + l % 32]
    // [col 32j + 8g + 4 * (l / 32) + q] of the wave's tile.
    // Rows at or past M and 4-column groups at or past N (a multiple of 4) are not stored.
    const int col0 = tn * BN + wn * WTN + 4 * half;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        const int row = tm * BM + wm * WTM + 32 * i + (lane & 31);
        if (row >= M) continue;
        float* crow = C + (int64_t)row * N + col0;
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 v = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
                if (col0 + 32 * j + 8 * g < N) *reinterpret_cast<f32x4*>(crow + 32 * j + 8 * g) = v;
            }
    }
}

// ---- fp64 on the same LDS-DMA ring (128 x 128 tiles) -----------------------
//
// v_mfma_f64_16x16x4_f64 sums four K values, one from each 16-lane group g;
// here group g supplies K 2g + t at step t (t = 0, 1) of a stage's 8, so a
// lane's A operands for the stage are 2 consecutive doubles of one row -- one
// ds_read_b128 per fragment from the [128 rows][64 B] A slot -- and its B
// operand at step t is one double of row 2g + t (ds_read_b64). B keeps its HBM
// layout, [8 rows][128 doubles = 1024 B]; rows with bit 1 set have their
// 16-byte chunks XOR 8, so groups 0 and 1 (and 2 and 3), which read rows 2
// apart (the same banks), land 128 bytes apart. Waves own 64 x 64 of C as
// 4 x 4 fragments (64 accumulator registers); A is the MFMA's first operand,
// so accumulator r of lane l is C row 4r + l / 16, column l % 16, and a store
// instruction writes 4 rows x 128 bytes straight from registers. With 64 KiB
// of ring and under 200 registers per lane, two blocks fit a CU, one wave of
// each on every SIMD: on MI355X these tiles ran up to 21% faster than
// 256 x 128 tiles (one block per CU) on 12 shapes from 3072 x 6144 x 4096 to
// 10240^2 x 4096, 8192^3 included (73.3 against 72.1 TFLOP/s), and 0.5%
// slower on one (4608^3).
constexpr int kF64Stages = 4, kF64StageK = 8;

__device__ __forceinline__ int swz_b64(int row) { return ((row >> 1) & 1) << 3; }

template <int BM, int BN, bool RAGGED_K = false>
__global__ void __launch_bounds__(256)
gemm_f64_dma_kernel(const double* __restrict__ A, const double* __restrict__ B, double* __restrict__ C, int M,
                    int N, int K, int tiles_m, int tiles_n) {
    // Per-tile sizes: waves in a 2 x 2 grid, fragments of 16 x 16.
    constexpr int WTM = BM / 2, WTN = BN / 2, FM = WTM / 16, FN = WTN / 16;
    constexpr int ABytes = BM * 64, BRow = BN * 8, BBytes = kF64StageK * BRow, Slot = ABytes + BBytes;
    constexpr int AInstr = ABytes / 1024 / 4, BInstr = BBytes / 1024 / 4, Loads = AInstr + BInstr;
    static_assert(AInstr >= 1 && BInstr >= 1 && WTM % 16 == 0 && WTN % 16 == 0 && BRow >= 256, "tile shape");
    __shared__ __attribute__((aligned(1024))) unsigned char ring[kF64Stages][Slot];
    const int tid = threadIdx.x, lane = tid & 63, grp = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    int tm, tn;
    tile_coords((int)blockIdx.x, tiles_m * tiles_n, tiles_m, tiles_n, kF32GroupM, &tm, &tn);
    const int lda = K * 8, ldb = N * 8;
    // Buffer ranges as in gemm_f32_dma_kernel: partial last tiles and a ragged K.
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<double*>(A) + (int64_t)tm * BM * K, (short)0, min(BM, M - tm * BM) * lda, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<double*>(B) + (int64_t)tn * BN, (short)0, K * ldb - tn * BN * 8, kBufferFlags);
    int a_voff[AInstr], a_kbyte[AInstr], b_voff[BInstr];
#pragma unroll
    for (int q = 0; q < AInstr; ++q) {
        const int lin = (wave * AInstr + q) * 1024 + lane * 16;
        const int row = lin / 64, pchunk = (lin % 64) >> 4;
        a_kbyte[q] = (pchunk ^ swz_a(row)) << 4;
        a_voff[q] = row * lda + a_kbyte[q];
    }
#pragma unroll
    for (int q = 0; q < BInstr; ++q) {
        const int lin = (wave * BInstr + q) * 1024 + lane * 16;
        const int row = lin / BRow, pchunk = (lin % BRow) >> 4;
        b_voff[q] = row * ldb + ((pchunk ^ swz_b64(row)) << 4);
    }
    auto issue_one = [&](int kt, int slot, auto idx) {
        constexpr int q = decltype(idx)::value;
        const unsigned base = (unsigned)(uintptr_t)(MB_LDS unsigned char*)ring[slot];
        if constexpr (q < AInstr)
            lds_dma16(ra, base + (wave * AInstr + q) * 1024,
                      RAGGED_K && a_kbyte[q] >= K * 8 - kt * 64 ? (int)0x80000000u : a_voff[q], kt * 64);
        else
            lds_dma16(rb, base + ABytes + (wave * BInstr + q - AInstr) * 1024, b_voff[q - AInstr],
                      kt * kF64StageK * ldb);
    };
    auto issue = [&](int kt, int slot) {
        [&]<int... Q>(std::integer_sequence<int, Q...>) {
            (issue_one(kt, slot, std::integral_constant<int, Q>{}), ...);
        }(std::make_integer_sequence<int, Loads>{});
    };

    f64x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.0;

    const int ksteps = (K + kF64StageK - 1) / kF64StageK, last = ksteps - 1;
#pragma unroll
    for (int st = 0; st < kF64Stages - 1; ++st) issue(min(st, last), st);
    const int a_row = wm * WTM + (lane & 15);
    const int b_col = wn * WTN + (lane & 15);
    double a[2][FM][2];  // A operands of this stage and the next
    double b[2][FN];     // B operands of this step and the next
    auto read_a = [&](int kt, auto setc) {
        constexpr int set = decltype(setc)::value;
        const unsigned char* slot = ring[kt % kF64Stages];
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const int row = a_row + 16 * i;
            const f64x2 v = *reinterpret_cast<const f64x2*>(slot + row * 64 + ((grp ^ swz_a(row)) << 4));
            a[set][i][0] = v[0];
            a[set][i][1] = v[1];
        }
    };
    auto read_b = [&](int kt, int t, int set) {
        const unsigned char* sb = ring[kt % kF64Stages] + ABytes;
        const int row = 2 * grp + t;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int col = b_col + 16 * j;
            b[set][j] = *reinterpret_cast<const double*>(sb + row * BRow + (((col >> 1) ^ swz_b64(row)) << 4) +
                                                         8 * (col & 1));
        }
    };
    // The fp32 kernel's schedule: one barrier per stage, between its two
    // steps, after which stage kt + 1's A operands are read under the second
    // step's MFMAs and its first B operands at the end of the stage; stage
    // kt + 3's loads are spread evenly between the second step's MFMAs.
    constexpr int kMfma = FM * FN, kLoadGap = kMfma / Loads;
    static_assert(kLoadGap >= 1, "a load per MFMA at most");
    auto stage = [&](int kt, auto curc) {
        constexpr int cur = decltype(curc)::value;
        const int load_kt = min(kt + kF64Stages - 1, last), load_slot = (kt + kF64Stages - 1) % kF64Stages;
        [&]<int... T>(std::integer_sequence<int, T...>) {
            ([&] {
                constexpr int t = T;
                if constexpr (t == 1) {
                    wait_vmcnt_and_barrier<Loads * (kF64Stages - 3)>();
                    read_a(kt + 1, std::integral_constant<int, cur ^ 1>{});
                    read_b(kt + 1, 0, 0);
                } else {
                    read_b(kt, 1, 1);
                }
                __builtin_amdgcn_sched_barrier(0);
                [&]<int... Q>(std::integer_sequence<int, Q...>) {
                    ([&] {
                        constexpr int m = Q, i = m / FN, j = m % FN;
                        acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[cur][i][t], b[t][j], acc[i][j], 0, 0, 0);
                        if constexpr (t == 1 && m % kLoadGap == 0 && m / kLoadGap < Loads)
                            issue_one(load_kt, load_slot, std::integral_constant<int, m / kLoadGap>{});
                        __builtin_amdgcn_sched_barrier(0);   // keeps each load where it is placed
                    }(), ...);
                }(std::make_integer_sequence<int, kMfma>{});
            }(), ...);
        }(std::make_integer_sequence<int, 2>{});
    };
    wait_vmcnt_and_barrier<Loads * (kF64Stages - 2)>();
    read_a(0, std::integral_constant<int, 0>{});
    read_b(0, 0, 0);
    for (int kt = 0; kt < ksteps; kt += 2) {
        stage(kt, std::integral_constant<int, 0>{});
        if (kt + 1 < ksteps) stage(kt + 1, std::integral_constant<int, 1>{});
    }
    wait_vmcnt_and_barrier<0>();

    // Rows at or past M and columns at or past N are not stored.
    const int col0 = tn * BN + wn * WTN + (lane & 15);
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = tm * BM + wm * WTM + 16 * i + 4 * r + grp;
            if (row >= M) continue;
            double* crow = C + (int64_t)row * N + col0;
#pragma unroll
            for (int j = 0; j < FN; ++j)
                if (col0 + 16 * j < N) crow[16 * j] = acc[i][j][r];
        }
}

// Which LDS-DMA ring a shape takes: 1 = fp32 on 256 x 256 tiles, when they
// cover every CU and their rounds cost no more than 128 x 128 tiles' (rule
// below); 2 = 128 x 128 tiles, every other fp32 shape and every fp64 one,
// partial last tiles included. 0 = the register-staged kernel, with *why naming the
// reason: A's or B's rows not on 16 bytes, or buffer offsets (B's K x N bytes,
// a 256-row A panel) beyond 31 bits. A K that is not whole stages runs the
// RAGGED_K instantiations, whose A pieces past K load zeros.
int highp_dma_config(bool f64, int64_t M, int64_t N, int64_t K, int cus, const char** why) {
    if (tuning(MB_TUNE_GEMM_HIGHP_STAGED) == 1) {
        *why = "forced by the gemm_highp_staged override";
        return 0;
    }
    const int64_t e = f64 ? 8 : 4, stage_k = f64 ? kF64StageK : kF32StageK;
    // The DMA loads need A's and B's rows on 16 bytes.
    if ((K * e) % 16 != 0) {
        *why = f64 ? "K is not a multiple of 2" : "K is not a multiple of 4";
        return 0;
    }
    if ((N * e) % 16 != 0) {
        *why = f64 ? "N is not a multiple of 2" : "N is not a multiple of 4";
        return 0;
    }
    const int64_t k_pad = (K + stage_k - 1) / stage_k * stage_k;
    if ((k_pad * N + 256) * e >= (int64_t(1) << 31) || 256 * k_pad * e >= (int64_t(1) << 31)) {
        *why = "operand offsets exceed 32-bit buffer addressing (K*N or 256*K bytes >= 2 GiB)";
        return 0;
    }
    // The LDS-DMA kernels take M and N as int (row and column guards); the
    // register-staged kernel indexes with int64.
    if (M >= (int64_t(1) << 31) || N >= (int64_t(1) << 31)) {
        *why = "M or N >= 2^31 exceeds the 32-bit row and column indexes of the LDS-DMA kernels";
        return 0;
    }
    auto tiles = [&](int64_t tm, int64_t tn) { return ((M + tm - 1) / tm) * ((N + tn - 1) / tn); };
    auto rounds = [&](int64_t t) { return (t + cus - 1) / cus; };
    const int64_t small = tiles(128, 128), large = tiles(256, 256);
    if (small > INT32_MAX) {
        *why = "more than 2^31 tiles";
        return 0;
    }
    if (f64) return 2;   // 128 x 128 tiles: two blocks per CU (gemm_f64_dma_kernel)
    // fp32: 256 x 256 tiles run 2.5% faster per FLOP than 128 x 128 ones
    // (8192^3, whole rounds of either: 150.1 against 145.8 TFLOP/s on MI355X) but
    // come in rounds of four times the work, so they are taken only when their
    // rounds cost no more: rounds(256 x 256) <= rounds(128 x 128) / 4 / 0.975.
    // This picked the faster tile on all of 12 shapes measured: 256 x 256 at
    // 4096^3, 8192^3, 6144 x 8192 x 4096 and 5632^2 x 4096 (1.9 rounds, 2%);
    // 128 x 128 where the last 256 x 256 round is partly empty, 1.05-1.32x
    // faster there (6144^3 124.5 against 109.5 TFLOP/s, 3072 x 6144 x 4096
    // 109.3 against 83.9). Ragged M or N: partial last tiles on either.
    const bool large_pays = large >= cus && 4.0 * 0.975 * (double)rounds(large) <= (double)rounds(small);
    if (M % 256 == 0 && N % 256 == 0 && large_pays) return 1;
    if (M % 128 == 0 && N % 128 == 0) return 2;
    return large_pays ? 1 : 2;
}

void highp_dma_tile(int cfg, int* bm, int* bn) {
    *bm = *bn = cfg == 1 ? 256 : 128;
}

template <typename T, int BM, int BN>
int launch_dma(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
    const int tiles_m = (int)((M + BM - 1) / BM), tiles_n = (int)((N + BN - 1) / BN);
    const T* a = static_cast<const T*>(A);
    const T* b = static_cast<const T*>(B);
    T* c = static_cast<T*>(C);
    const dim3 grid(tiles_m * tiles_n);
    if constexpr (sizeof(T) == 4) {
        auto kernel = K % kF32StageK != 0 ? gemm_f32_dma_kernel<BM, BN, true> : gemm_f32_dma_kernel<BM, BN, false>;
        hipLaunchKernelGGL(kernel, grid, dim3(256), 0, stream, a, b, c, (int)M, (int)N, (int)K, tiles_m, tiles_n);
    } else {
        auto kernel = K % kF64StageK != 0 ? gemm_f64_dma_kernel<BM, BN, true> : gemm_f64_dma_kernel<BM, BN, false>;
        hipLaunchKernelGGL(kernel, grid, dim3(256), 0, stream, a, b, c, (int)M, (int)N, (int)K, tiles_m, tiles_n);
    }
    MB_HIP_TRY(hipGetLastError());
    return MB_OK;
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

int gemm_highp_plan(int dtype, int64_t M, int64_t N, int64_t K, const DeviceProps& props, GemmPlan* plan) {
    const bool f64 = dtype == MB_DT_FLOAT64;
    const char* why = "";
    const int cfg = highp_dma_config(f64, M, N, K, props.cu_count > 0 ? props.cu_count : 256, &why);
    if (cfg != 0) {
        int bm, bn;
        highp_dma_tile(cfg, &bm, &bn);
        plan->implementation = f64 ? "gfx950_mfma_f64_16x16x4_lds_dma" : "gfx950_mfma_f32_32x32x2_lds_dma";
        plan->threads = 256;
        plan->grid = (int)(((M + bm - 1) / bm) * ((N + bn - 1) / bn));
        plan->tile_m = bm;
        plan->tile_n = bn;
        plan->tile_k = f64 ? kF64StageK : kF32StageK;
        plan->wave_grid_m = plan->wave_grid_n = 2;
        plan->frag_m = plan->frag_n = f64 ? 16 : 32;
        plan->frag_k = f64 ? 4 : 2;
        plan->wave_tile_m = bm / 2 / plan->frag_m;
        plan->wave_tile_n = bn / 2 / plan->frag_n;
        plan->k_stages = f64 ? kF64Stages : kF32Stages;
        plan->split_k = 1;
        plan->tile_group_m = kF32GroupM;
        plan->workspace = 0;
        plan->variant = kVariantHighp;
        plan->config = cfg;
        return MB_OK;
    }
    const int64_t gx = (N + kHpBN - 1) / kHpBN, gy = (M + kHpBM - 1) / kHpBM;
    if (gy > 65535 || gx > INT32_MAX) {
        set_error("fp32/fp64 GEMM: M=%lld N=%lld too large for the register-staged kernel's grid (%s)",
                  (long long)M, (long long)N, why);
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
    plan->fallback = why;
    plan->variant = kVariantHighp;
    return MB_OK;
}

int gemm_highp_launch(int dtype, const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
                      const GemmPlan& plan, hipStream_t stream) {
    switch (dtype) {
        case MB_DT_FLOAT32:
            if (plan.config == 1) return launch_dma<float, 256, 256>(A, B, C, M, N, K, stream);
            if (plan.config == 2) return launch_dma<float, 128, 128>(A, B, C, M, N, K, stream);
            return launch_typed<float>(A, B, C, M, N, K, stream);
        case MB_DT_FLOAT64:
            if (plan.config == 2) return launch_dma<double, 128, 128>(A, B, C, M, N, K, stream);
            return launch_typed<double>(A, B, C, M, N, K, stream);
        default:
            set_error("fp32/fp64 GEMM: unsupported dtype %d", dtype);
            return MB_ERR_UNSUPPORTED;
    }
}

}  // namespace mb

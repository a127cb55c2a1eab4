// LDS-pipelined MFMA GEMM for gfx950: C = alpha * (A * B), A (M x K) and
// B (K x N) row-major, fp32 accumulation, output bf16 (bf16 and fp8 e4m3 /
// e5m2 inputs) or fp16 (fp16 inputs). Tiles of 256 x 256, 128 x 256,
// 128 x 128, 64 x 128 or 64 x 64. Takes shapes with A's and B's rows on 16 bytes (K
// and N multiples of 8, of 16 for fp8), any M: the rows of a partial last M
// tile read as zeros, and the columns of a partial last N tile read the start
// of B's next row (zeros past B's end); neither is stored. A K that is not a
// multiple of the stage depth runs whole stages, its A pieces past K loaded as
// zeros (the RAGGED_K instantiations) and B's rows past K lying past B's end.
// Everything else goes to the bounds-checked kernel.
//
// Data path. A stage is 64 bytes of K per row. A is held two stages at a
// time, as [BM rows][128 B] pair slots; B one stage at a time, as
// [K rows][BN * elem bytes] -- B keeps its HBM layout (N-contiguous). Both
// arrive with buffer_load_dwordx4 ... lds (HBM/L2 -> LDS, no register
// staging): one wave instruction fills 1 KiB of LDS in lane order, and each
// lane picks the global 16 bytes that belong at its slot of the swizzled
// layout. An A instruction covers 8 rows x 128 bytes, whole cache lines:
// loading A one 64-byte stage at a time made two L2 requests per line and
// ran 2-13% slower. The MFMA operands come out of LDS with ds_read_b128 for
// A and the gfx950 transposing reads (ds_read_b64_tr_b16 for 16-bit B,
// ds_read_b64_tr_b8 for fp8 B), which hand each lane 4 (8) consecutive K
// values of one B column -- the MFMA operand layout -- with no transpose pass
// anywhere.
//
// LDS swizzles (16-byte chunk c of a row is stored at chunk c ^ f(row)):
//   A rows (8 chunks):          f = ((r >> 1) & 7) ^ ((r & 1) << 2)
//   16-bit B rows (32 chunks):  f = ((k << 2) ^ (k << 1)) & 15, k = row & 3
//   16-bit B rows (8 chunks):   f = 2k,                         k = row & 3
//   fp8 B rows (16 chunks):     f = (2k) ^ (k >> 2),            k = row & 7
//   fp8 B rows (8 chunks):      f = k,                          k = row & 7
//   fp8 B rows (4 chunks):      f = (k >> 1) & 3,               k = row & 7
// Each keeps every operand read of a wave free of bank conflicts for both 8-
// and 16-lane LDS phases (checked exhaustively on the host).
//
// Pipeline. NA A pair slots and NB B stage slots, one barrier per stage.
// While the MFMAs of stage k run from registers, every operand of stage
// k + 1 is read from LDS into a second register set, B stage k + NB is
// loaded into the slot stage k has just vacated and, on odd k, A pair
// (k - 1) / 2 + NA into the pair slot whose second stage was k; all spread
// evenly between the MFMAs. The barrier is a bare s_barrier preceded by an
// explicit vmcnt wait for the loads of stage k + 1 only, derived at compile
// time from the issue order (load_schedule) -- a full __syncthreads() would
// wait for all of them. Each step's first two MFMAs go out ahead of its
// barrier, from operands already in registers, so the MFMA pipe stays busy
// while the wave waits there.
//
// Waves form a WGM x WGN grid; each wave owns (BM/WGM) x (BN/WGN) of C as
// 32 x 32 fragments: v_mfma_f32_32x32x16_{bf16,f16} (two per stage), or for
// fp8 v_mfma_f32_32x32x64_f8f6f4 (one per stage). fp8 on 256- and 128-row x
// 256-column tiles runs gemm_fp8_mi16_kernel below instead: 16 x 16 fragments
// on v_mfma_scale_f32_16x16x128_f8f6f4, one MFMA spanning a pair of stages. The MFMA takes the B
// fragment as its first operand, so a lane's 16 accumulators are 4 runs of 4
// consecutive C columns in one C row. The epilogue rounds them to 16 bits
// through LDS so that the stores to C are whole 256-byte row segments.
//
// Tile order: blocks are dispatched round-robin over the 8 XCDs (block b on
// XCD b % 8); each XCD gets a contiguous range of tiles in an order grouped
// by `group_m` tile rows, i.e. a compact group_m x (range / group_m) patch of
// C whose A row panels and B column panels its L2 shares.
#include "gemm_pipeline.hpp"

#include <cmath>
#include <cstdlib>
#include <numeric>
#include <utility>

namespace mb {
namespace {

constexpr int kStageK = 64;                  // bytes of K per row per stage
// MFMAs of a step issued ahead of its barrier. They take operands already in
// registers, and the MFMA pipe works through them while the wave waits at the
// barrier (one wave per SIMD: nothing else would keep it busy). Two measured
// best: against one, fp8 8192^3 +1.0%, 8192 x 1024 x 8192 +1.9%, 16-bit
// shapes +0.3-0.5%; three and four lose on 128-row tiles.
constexpr int kPreBarrierMfma = 2;

__device__ __forceinline__ int swz_b16(int k) { return ((k << 2) ^ (k << 1)) & 15; }
// 16-bit B rows of 128 bytes (64 columns, 8 chunks).
__device__ __forceinline__ int swz_b16_128(int k) { return 2 * k; }
// fp8 B rows of 256 bytes (256 columns), of 128 bytes (128 columns) and of 64 bytes (64 columns).
__device__ __forceinline__ int swz_b8(int k) { return (2 * k) ^ (k >> 2); }
__device__ __forceinline__ int swz_b8_128(int k) { return k; }
__device__ __forceinline__ int swz_b8_64(int k) { return (k >> 1) & 3; }

// The B-row swizzle of a tile's row width (bytes) and element size: chunk c of
// B row k sits at chunk c ^ b_swizzle(k).
template <int E, int ROW>
__device__ __forceinline__ int b_swizzle(int k) {
    if constexpr (E == 2) return ROW == 128 ? swz_b16_128(k & 3) : swz_b16(k & 3);
    else return ROW == 256 ? swz_b8(k & 7) : ROW == 128 ? swz_b8_128(k & 7) : swz_b8_64(k & 7);
}

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4_t __attribute__((__vector_size__(4 * sizeof(__bf16))));
typedef int i32x2_t __attribute__((__vector_size__(2 * sizeof(int))));

template <int DT>
struct Traits;

template <>
struct Traits<MB_DT_BFLOAT16> {
    static constexpr int kElem = 2;
    typedef u32x4 Frag;
    __device__ static __forceinline__ f32x16 mfma(const Frag& a, const Frag& b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                        __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    }
};

template <>
struct Traits<MB_DT_FLOAT16> : Traits<MB_DT_BFLOAT16> {
    __device__ static __forceinline__ f32x16 mfma(const Frag& a, const Frag& b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                       __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
};

template <>
struct Traits<MB_DT_FLOAT8_E4M3FN> {
    static constexpr int kElem = 1;
    typedef i32x8 Frag;
    // Format code 0 = e4m3 for both operands; zero scale operands select the
    // unscaled encoding of the instruction.
    __device__ static __forceinline__ f32x16 mfma(const Frag& a, const Frag& b, f32x16 c) {
        return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
    }
};

// Format code 1 = bf8 e5m2 for both operands.
template <>
struct Traits<MB_DT_FLOAT8_E5M2> : Traits<MB_DT_FLOAT8_E4M3FN> {
    __device__ static __forceinline__ f32x16 mfma(const Frag& a, const Frag& b, f32x16 c) {
        return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 1, 1, 0, 0, 0, 0);
    }
};

// A is held two stages at a time: rows of 128 bytes (stage 2p in chunks 0-3,
// stage 2p + 1 in chunks 4-7), chunk c of row r stored at chunk c ^ swz_a2(r).
// For the operand reads (32 consecutive rows, one logical chunk per half
// wave) every 8 consecutive rows land on 8 distinct 16-byte bank groups and
// every 16 on 16 distinct (row parity, chunk) pairs: no bank conflicts for 8-
// or 16-lane LDS phases.
__device__ __forceinline__ int swz_a2(int r) { return ((r >> 1) & 7) ^ ((r & 1) << 2); }

// One 16-byte piece of this lane's A operand: row `row` of the pair slot,
// 16-byte K chunk `chunk` (0..7: 4 * stage parity + chunk within the stage;
// 16-bit: chunk 2s + lane/32 of substep s; fp8: chunks 2*(lane/32) and +1
// form the 32-byte operand).
__device__ __forceinline__ u32x4 read_a_piece(const unsigned char* slot, int row, int chunk) {
    return *reinterpret_cast<const u32x4*>(slot + row * 2 * kStageK + ((chunk ^ swz_a2(row)) << 4));
}

// Issue order of the LDS-DMA loads and the vmcnt waits it allows. Loop step j
// issues, in this order, the A pair (j - 1) / 2 + NA when j is odd (AI loads
// per wave) and B stage j + NB (BI loads). The prologue issues A pairs
// 0..NA-1 and B stages 0..NB-1 in the order the same rule gives for the
// steps -V..-1 that precede step 0. Before step j the pipeline needs stage
// j + 1: B stage j + 1 and A pair (j + 1) / 2; wait(j) is the number of loads
// issued after the later of the two, i.e. the vmcnt at which both have
// landed. Loads complete in issue order. The loop uses, per step parity, the
// smallest wait over the first steps and the steady state, so every step's
// wait is exact or stricter; `prologue` is the wait before stage 0 is read.
struct LoadSchedule {
    int odd_wait, even_wait, prologue;
};

constexpr LoadSchedule load_schedule(int NA, int NB, int AI, int BI) {
    constexpr int kSteps = 64;
    // end[kind][index]: loads issued up to and including that pair (kind 0)
    // or stage (kind 1); issued_before[j]: loads issued before step j.
    int end_a[2 * kSteps] = {}, end_b[2 * kSteps] = {}, issued_before[kSteps] = {};
    int total = 0;
    const int V = 2 * NA - 1 > NB ? 2 * NA - 1 : NB;
    for (int v = -V; v < kSteps; ++v) {
        if (v >= 0) issued_before[v] = total;
        if ((v & 1) != 0) {
            const int pair = (v - 1 >= 0 ? (v - 1) / 2 : -((1 - v) / 2)) + NA;
            if (pair >= 0 && pair < 2 * kSteps) end_a[pair] = (total += AI);
        }
        if (v + NB >= 0 && v + NB < 2 * kSteps) end_b[v + NB] = (total += BI);
    }
    LoadSchedule r{1 << 20, 1 << 20, 0};
    const int p0 = end_a[0] > end_b[0] ? end_a[0] : end_b[0];
    r.prologue = issued_before[0] - p0;
    for (int j = 0; j + 1 < kSteps; ++j) {
        const int need = end_a[(j + 1) / 2] > end_b[j + 1] ? end_a[(j + 1) / 2] : end_b[j + 1];
        const int w = issued_before[j] - need;
        if (j & 1) r.odd_wait = w < r.odd_wait ? w : r.odd_wait;
        else r.even_wait = w < r.even_wait ? w : r.even_wait;
    }
    return r;
}

// Issue order and vmcnt waits of the fp8 16x16x128 kernel's ring. B stage S
// is read into registers during step S - 2 (stages 0 and 1 before step 0)
// and A pair P during steps 2P - 1 .. 2P + 1. Step k issues, in this order,
// A pair k / 2 + NA - 1 when k is even (AI loads per wave) and B stage
// k + 1 + NB (BI loads); the prologue issues pairs 0..NA-2 and stages
// 0..NB-1 by the same rule over the steps before step 0, then, once stages
// 0 and 1 are read and a barrier has freed stage 0's slot, stage NB. Before
// step j the pipeline needs B stage j + 2 and A pair (j + 1) / 2.
constexpr int floor_half(int v) { return v >= 0 ? v / 2 : -((1 - v) / 2); }

constexpr LoadSchedule load_schedule_mi16(int NA, int NB, int AI, int BI, bool split_a) {
    constexpr int kSteps = 64;
    int end_a[kSteps + 16] = {}, end_b[kSteps + 16] = {}, issued_before[kSteps] = {};
    int total = 0;
    // A loads of step (or virtual step) v: all AI of pair v / 2 + NA - 1 on
    // even v, or, split, AI / 2 of pair floor(v / 2) + NA - 1 on every v.
    auto a_step = [&](int v) {
        const int pair = floor_half(v) + NA - 1;
        if (pair < 0 || pair >= kSteps + 16) return;
        if (split_a) total += AI / 2;
        else if ((v & 1) == 0) total += AI;
        else return;
        end_a[pair] = total;
    };
    const int V = NB + 1 > 2 * NA - 2 ? NB + 1 : 2 * NA - 2;
    for (int v = -V; v < 0; ++v) {
        a_step(v);
        if (v + 1 + NB >= 0 && v + 1 + NB < NB) end_b[v + 1 + NB] = (total += BI);
    }
    LoadSchedule r{1 << 20, 1 << 20, 0};
    int p0 = end_a[0] > end_b[0] ? end_a[0] : end_b[0];
    p0 = p0 > end_b[1] ? p0 : end_b[1];
    r.prologue = total - p0;
    end_b[NB] = (total += BI);
    for (int k = 0; k < kSteps; ++k) {
        issued_before[k] = total;
        a_step(k);
        if (k + 1 + NB < kSteps + 16) end_b[k + 1 + NB] = (total += BI);
    }
    for (int j = 0; j + 2 < kSteps; ++j) {
        const int need = end_a[(j + 1) / 2] > end_b[j + 2] ? end_a[(j + 1) / 2] : end_b[j + 2];
        const int w = issued_before[j] - need;
        if (j & 1) r.odd_wait = w < r.odd_wait ? w : r.odd_wait;
        else r.even_wait = w < r.even_wait ? w : r.even_wait;
    }
    return r;
}

// One transposing read of this lane's B operand (column nb + lane % 32).
// 16-bit: 4 K-rows x 16 columns per 16-lane group, part t (0..1) of substep s
// gives K 16s + 8*(lane/32) + 4t .. +3. fp8: 8 K-rows x 16 columns, part t
// (0..3) gives K 32*(lane/32) + 8t .. +7. `st` is the B part of the stage.
template <int DT, int BN>
__device__ __forceinline__ u32x2 read_b_piece(const unsigned char* st, int nb, int s, int t, int lane) {
    const int g = lane >> 4, i = lane & 15;
    if constexpr (Traits<DT>::kElem == 2) {
        constexpr int row_bytes = BN * 2;
        const int k = 16 * s + 8 * (g >> 1) + 4 * t + (i >> 2);
        const int n = nb + 16 * (g & 1) + 4 * (i & 3);
        const int off = k * row_bytes + (((n >> 3) ^ b_swizzle<2, row_bytes>(k)) << 4) + 8 * (i & 1);
        const bf16x4_t v =
            __builtin_amdgcn_ds_read_tr16_b64_v4bf16((MB_LDS bf16x4_t*)((MB_LDS unsigned char*)st + off));
        return __builtin_bit_cast(u32x2, v);
    } else {
        constexpr int row_bytes = BN;
        const int k = 32 * (g >> 1) + 8 * t + (i >> 1);
        const int n = nb + 16 * (g & 1) + 8 * (i & 1);
        const int f = b_swizzle<1, row_bytes>(k);
        const int off = k * row_bytes + (((n >> 4) ^ f) << 4) + 8 * (i & 1);
        const i32x2_t v = __builtin_amdgcn_ds_read_tr8_b64_v2i32((MB_LDS i32x2_t*)((MB_LDS unsigned char*)st + off));
        return __builtin_bit_cast(u32x2, v);
    }
}

// Output: 4 consecutive columns, rounded once from fp32.
template <int DT>
__device__ __forceinline__ u32x2 pack4(float a, float b, float c, float d) {
    if constexpr (DT == MB_DT_FLOAT16) {
        f16x4 h = {(_Float16)a, (_Float16)b, (_Float16)c, (_Float16)d};
        return __builtin_bit_cast(u32x2, h);
    } else {
        bf16x4 h = {(__bf16)a, (__bf16)b, (__bf16)c, (__bf16)d};
        return __builtin_bit_cast(u32x2, h);
    }
}

// Second half of the epilogue: a wave's (WTM x ROW_BYTES / 2) tile, staged in
// LDS as 16-bit values (chunk c of row r at chunk c ^ (r % chunks)), read back
// row by row and stored so that 16 (8, 4) lanes write one 256-byte (128-,
// 64-byte) C row segment: whole cache lines, half lines for 64 bytes. Read-backs go out in batches of BATCH
// before their stores, so no store waits on the LDS read just before it.
// The stores are nontemporal: nothing in the kernel reads C back, and every
// CU stores its tile at about the same moment, so keeping those lines out of
// L2 lets the burst drain faster (measured +0.6% at 8192^3, +1.8% at 4096^3,
// +2.6% at fp8 8192 x 1024 x 8192). Rows at or past M (a partial last tile)
// and 8-column chunks at or past N (a partial last tile of a ragged N, which
// is a multiple of 8) are not stored.
template <int WTM, int ROW_BYTES>
__device__ __forceinline__ void store_staged_tile(const unsigned char* stage, unsigned char* C, int M, int N,
                                                  int row_base, int64_t col_base, int lane) {
    constexpr int ROW_CHUNKS = ROW_BYTES / 16;
    const int64_t ldc = (int64_t)N * 2;  // bytes per C row (16-bit output)
    constexpr int ROWS_PER_STORE = 64 / ROW_CHUNKS;
    constexpr int STORES = WTM / ROWS_PER_STORE;
    constexpr int BATCH = STORES < 8 ? STORES : 8;
    static_assert(STORES % BATCH == 0, "stores split into batches");
    const int c = lane % ROW_CHUNKS;
    const int r0 = lane / ROW_CHUNKS;
    const bool col_in = col_base + 8 * c < N;
    int grow = row_base + r0;
    unsigned char* cptr = C + (int64_t)grow * ldc + col_base * 2 + c * 16;
#pragma unroll
    for (int p0 = 0; p0 < STORES; p0 += BATCH) {
        u32x4 rows[BATCH];
#pragma unroll
        for (int p = 0; p < BATCH; ++p) {
            const int r = ROWS_PER_STORE * (p0 + p) + r0;
            rows[p] = *reinterpret_cast<const u32x4*>(stage + r * ROW_BYTES + ((c ^ (r % ROW_CHUNKS)) << 4));
        }
#pragma unroll
        for (int p = 0; p < BATCH; ++p) {
            if (grow < M && col_in) __builtin_nontemporal_store(rows[p], reinterpret_cast<u32x4*>(cptr));
            grow += ROWS_PER_STORE;
            cptr += ROWS_PER_STORE * ldc;
        }
    }
}

template <int DT, int BM, int BN, int WGM, int WGN, int NA, int NB, bool SCALED, bool RAGGED_K = false>
__global__ void __launch_bounds__(64 * WGM * WGN)
gemm_tiled_kernel(const unsigned char* __restrict__ A, const unsigned char* __restrict__ B,
                  unsigned char* __restrict__ C, int M, int N, int K, float alpha, int tiles_m,
                  int tiles_n, int group_m, int splits, int k_len, float* __restrict__ ws) {
    typedef Traits<DT> Tr;
    typedef typename Tr::Frag Frag;
    constexpr int W = WGM * WGN;
    constexpr int E = Tr::kElem;
    constexpr int WTM = BM / WGM, WTN = BN / WGN;
    constexpr int FM = WTM / 32, FN = WTN / 32;
    constexpr int K_ROWS = kStageK / E;                 // K elements per stage = B rows per stage
    constexpr int PAIR = 2 * BM * kStageK;              // A slot: two stages, [BM][128 B]
    constexpr int B_ROW = BN * E;                       // bytes per B row in LDS
    constexpr int B_BYTES = K_ROWS * B_ROW;             // B slot: one stage
    constexpr int A_INSTR = PAIR / 1024 / W;            // LDS-DMA instructions per wave per A pair
    constexpr int B_INSTR = B_BYTES / 1024 / W;         // ... per B stage
    constexpr int LDS_BYTES = NA * PAIR + NB * B_BYTES;
    static_assert(PAIR % (1024 * W) == 0 && B_BYTES % (1024 * W) == 0, "stage must split over the waves");
    static_assert(A_INSTR % 2 == 0, "A offsets assume an even number of pair loads per wave");
    static_assert(E == 2 ? (B_ROW == 512 || B_ROW == 256 || B_ROW == 128) : (B_ROW == 256 || B_ROW == 128 || B_ROW == 64),
                  "B swizzles cover 16-bit rows of 512 / 256 / 128 bytes and fp8 rows of 256 / 128 / 64 bytes");
    static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be 32-aligned");
    static_assert(NA >= 2 && NB >= 3 && LDS_BYTES <= 160 * 1024, "LDS ring does not fit");
    constexpr LoadSchedule kSched = load_schedule(NA, NB, A_INSTR, B_INSTR);
    static_assert(kSched.prologue >= 0 && kSched.odd_wait >= 0 && kSched.even_wait >= 0 &&
                  kSched.prologue < 64 && kSched.odd_wait < 64 && kSched.even_wait < 64,
                  "load schedule leaves a needed stage unissued or overflows vmcnt");

    // One LDS array: NA A pair slots, then NB B stage slots; every slot
    // address is a compile-time offset.
    __shared__ __attribute__((aligned(1024))) unsigned char lds[LDS_BYTES];
    auto a_slot = [&](auto idx) -> unsigned char* {
        static_assert(decltype(idx)::value < NA, "A slot out of range");
        return lds + decltype(idx)::value * PAIR;
    };
    auto b_slot = [&](auto idx) -> unsigned char* {
        static_assert(decltype(idx)::value < NB, "B slot out of range");
        return lds + NA * PAIR + decltype(idx)::value * B_BYTES;
    };

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WGN, wn = wave % WGN;
    // Block -> (tile, K split). With one split the tile index is the block
    // index (XCD-grouped); with several, the splits of a tile are adjacent.
    const int split = splits > 1 ? (int)blockIdx.x % splits : 0;
    const int tile = splits > 1 ? (int)blockIdx.x / splits : (int)blockIdx.x;
    int tm, tn;
    tile_coords(tile, tiles_m * tiles_n, tiles_m, tiles_n, group_m, &tm, &tn);
    const int lda = K * E;   // bytes per A row
    const int ldb = N * E;   // bytes per B row
    const int k0 = split * k_len;  // first K element of this block

    // Buffer resources over this block's A row panel and B column panel. The A
    // range stops at row M, so the rows of a last, partial tile read as zeros.
    // The B range stops at B's last byte: in a partial last N tile (ragged N)
    // the columns at or past N of a row read the start of the next row, which
    // only reaches C columns that are not stored, and past the last row they
    // read as zeros.
    const int a_rows = min(BM, M - tm * BM);
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<unsigned char*>(A) + (int64_t)tm * BM * lda, (short)0, a_rows * lda, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<unsigned char*>(B) + (int64_t)tn * BN * E, (short)0, K * ldb - tn * BN * E, kBufferFlags);

    // Global byte offsets of this lane's 16-byte pieces (pair 0 / stage 0);
    // a pair advances A by 2 * kStageK bytes, a stage advances B by K_ROWS
    // rows. A load q of a wave fills rows 8 * (wave * A_INSTR + q) .. +7 with
    // whole 128-byte lines; the swizzle of those rows depends on q only
    // through its parity, so two vector offsets serve all q and the rest,
    // 16 * (q / 2) rows, is a uniform offset.
    int a_voff[2], a_kbyte[2], b_voff[B_INSTR];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int lin = (wave * A_INSTR + q) * 1024 + lane * 16;   // LDS byte in the pair slot
        const int row = lin / (2 * kStageK), pchunk = (lin % (2 * kStageK)) >> 4;
        a_kbyte[q] = (pchunk ^ swz_a2(row)) << 4;                  // K byte of the piece within its pair
        a_voff[q] = row * lda + a_kbyte[q];
    }
#pragma unroll
    for (int q = 0; q < B_INSTR; ++q) {
        const int lin = (wave * B_INSTR + q) * 1024 + lane * 16;   // LDS byte in the B part
        const int row = lin / B_ROW, pchunk = (lin % B_ROW) >> 4;
        const int f = b_swizzle<E, B_ROW>(row);
        b_voff[q] = row * ldb + ((pchunk ^ f) << 4);
    }

    // DMA instruction q of A pair `pair` into `slot`, and of B stage `kt`.
    // RAGGED_K (K not a multiple of the stage): the A pieces at or past K load
    // zeros (an offset past the buffer range), so the stages that run past K
    // add nothing; B's rows past K lie past B's end and load zeros too.
    auto issue_a = [&](int pair, unsigned char* slot, auto idx) {
        constexpr int q = decltype(idx)::value;
        const unsigned base = (unsigned)(uintptr_t)(MB_LDS unsigned char*)slot;
        const int kb = k0 * E + pair * 2 * kStageK;
        int voff = a_voff[q & 1];
        if constexpr (RAGGED_K) voff = a_kbyte[q & 1] < K * E - kb ? voff : (int)0x80000000u;
        lds_dma16(ra, base + (wave * A_INSTR + q) * 1024, voff, kb + 16 * (q >> 1) * lda);
    };
    auto issue_b = [&](int kt, unsigned char* slot, auto idx) {
        constexpr int q = decltype(idx)::value;
        const unsigned base = (unsigned)(uintptr_t)(MB_LDS unsigned char*)slot;
        lds_dma16(rb, base + (wave * B_INSTR + q) * 1024, b_voff[q], (k0 + kt * K_ROWS) * ldb);
    };

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int half = lane >> 5;
    const int a_row = wm * WTM + (lane & 31);
    const int b_col = wn * WTN;

    // The operands of one stage. 16-bit: two K substeps of 16 (one MFMA per
    // fragment pair each), one 16-byte A read and two transposing B reads per
    // fragment and substep. fp8: one substep of 64, two A reads and four B
    // reads per fragment.
    constexpr bool kWide = Tr::kElem == 1;             // fp8: 32-byte operands
    constexpr int SUBS = kWide ? 1 : 2;                 // K substeps per stage
    constexpr int B_PIECES = kWide ? 4 : 2;             // transposing reads per B fragment
    constexpr int A_PIECES = kWide ? 2 : 1;             // 16-byte reads per A fragment
    constexpr int PER_SUB = FM * A_PIECES + FN * B_PIECES;
    constexpr int N_READS = SUBS * PER_SUB;
    constexpr int N_MFMA = SUBS * FM * FN;
    struct StageOps {
        Frag a[SUBS][FM];
        Frag b[SUBS][FN];
    };

    // Read number r of a stage, in the order the MFMAs consume operands: per
    // substep A fragment 0, then the B fragments, then A fragments 1..FM-1.
    // `aslot` is the stage's A pair slot and P its half (the stage's parity).
    auto read_op = [&](const unsigned char* aslot, const unsigned char* bslot, auto par, auto idx, StageOps& o) {
        constexpr int P = decltype(par)::value;
        constexpr int r = decltype(idx)::value;
        constexpr int s = r / PER_SUB, u = r % PER_SUB;
        if constexpr (u >= A_PIECES && u < A_PIECES + FN * B_PIECES) {
            constexpr int j = (u - A_PIECES) / B_PIECES, t = (u - A_PIECES) % B_PIECES;
            const u32x2 v = read_b_piece<DT, BN>(bslot, b_col + 32 * j, s, t, lane);
            o.b[s][j][2 * t] = v[0];
            o.b[s][j][2 * t + 1] = v[1];
        } else {
            constexpr int q = u < A_PIECES ? u : u - FN * B_PIECES;
            constexpr int i = q / A_PIECES, e = q % A_PIECES;
            const int chunk = 4 * P + (kWide ? 2 * half + e : 2 * s + half);
            const u32x4 v = read_a_piece(aslot, a_row + 32 * i, chunk);
#pragma unroll
            for (int w = 0; w < 4; ++w) o.a[s][i][4 * e + w] = v[w];
        }
    };
    auto mfma_op = [&](auto idx, const StageOps& o) {
        constexpr int q = decltype(idx)::value;
        constexpr int s = q / (FM * FN), i = (q / FN) % FM, j = q % FN;
        acc[i][j] = Tr::mfma(o.b[s][j], o.a[s][i], acc[i][j]);
    };

    // Software pipeline, one barrier per stage. A sits in NA pair slots (two
    // stages each, loaded as whole 128-byte lines of every row), B in NB stage
    // slots. Step kt (stage kt's operands already in registers):
    //   wait until stage kt+1 has landed and this wave's LDS reads are done,
    //   barrier; then the stage's MFMAs, with every LDS read of stage kt+1
    //   (into the other register set) and this step's loads spread evenly
    //   between them: B stage kt+NB into the B slot stage kt vacated, and, on
    //   odd steps, A pair (kt-1)/2+NA into the pair slot whose second stage
    //   (kt) has just been read.
    // The barrier certifies stage kt+1 for every wave, and that every wave
    // has finished reading stage kt (those reads went out during step kt-1).
    // Loads past the last stage (pair) re-read the last one (in bounds, never
    // consumed), so every step issues a fixed number of loads and the vmcnt
    // waits (load_schedule) hold at the tail too.
    // sched_barrier(0) after each MFMA and its memory instructions pins the
    // interleaving, so the MFMA pipe never waits behind a burst of issues.
    const int ksteps = k_len / K_ROWS;
    const int last = ksteps - 1;
    const int last_pair = last / 2;
    constexpr int V = 2 * NA - 1 > NB ? 2 * NA - 1 : NB;
    [&]<int... U>(std::integer_sequence<int, U...>) {
        ([&] {
            constexpr int v = U - V;
            if constexpr ((v & 1) != 0 && (v - 1) / 2 + NA >= 0) {
                constexpr int pair = (v - 1) / 2 + NA;  // v - 1 is even: exact
                [&]<int... Q>(std::integer_sequence<int, Q...>) {
                    (issue_a(min(pair, last_pair), a_slot(std::integral_constant<int, pair>{}),
                             std::integral_constant<int, Q>{}), ...);
                }(std::make_integer_sequence<int, A_INSTR>{});
            }
            if constexpr (v + NB >= 0) {
                [&]<int... Q>(std::integer_sequence<int, Q...>) {
                    (issue_b(min(v + NB, last), b_slot(std::integral_constant<int, v + NB>{}),
                             std::integral_constant<int, Q>{}), ...);
                }(std::make_integer_sequence<int, B_INSTR>{});
            }
        }(), ...);
    }(std::make_integer_sequence<int, V>{});
    // Two operand sets, used alternately (step I computes from set I % 2 and
    // reads into the other); the loop is unrolled to a multiple of 2 * NA and
    // of NB steps, so every slot is a compile-time choice and the sets are
    // never copied.
    StageOps ops[2];
    wait_vmcnt_and_barrier<kSched.prologue>();
    [&]<int... R>(std::integer_sequence<int, R...>) {
        (read_op(a_slot(std::integral_constant<int, 0>{}), b_slot(std::integral_constant<int, 0>{}),
                 std::integral_constant<int, 0>{}, std::integral_constant<int, R>{}, ops[0]), ...);
    }(std::make_integer_sequence<int, N_READS>{});

    auto step = [&](auto idx, int kt) {
        constexpr int I = decltype(idx)::value;
        constexpr bool ODD = (I & 1) != 0;
        constexpr int A_LOADS = ODD ? A_INSTR : 0;
        constexpr int LOADS = A_LOADS + B_INSTR;
        constexpr int N_MEM = N_READS + LOADS;              // memory instructions this step
        constexpr int PRE = N_MFMA >= 16 ? kPreBarrierMfma : 0;   // MFMAs before the barrier (long steps)
        static_assert(PRE >= 0 && PRE < N_MFMA, "pre-barrier MFMAs must leave slots for the memory instructions");
        constexpr int PER = (N_MEM + N_MFMA - PRE - 1) / (N_MFMA - PRE);  // ... issued after each later MFMA
        // Memory instruction m is a load when m + 1 is one of the first LOADS
        // multiples of kStride, otherwise the next operand read: the loads
        // sit evenly among the reads (A pair loads first, then B).
        constexpr int kStride = N_MEM / LOADS;
        constexpr auto kIsLoad = [](int m) { return (m + 1) % kStride == 0 && (m + 1) / kStride <= LOADS; };
        const unsigned char* next_a = a_slot(std::integral_constant<int, ((I + 1) / 2) % NA>{});
        const unsigned char* next_b = b_slot(std::integral_constant<int, (I + 1) % NB>{});
        unsigned char* load_a = a_slot(std::integral_constant<int, ((I + 2 * NA - 1) / 2) % NA>{});
        unsigned char* load_b = b_slot(std::integral_constant<int, I % NB>{});
        const StageOps& cur = ops[I % 2];
        StageOps& nxt = ops[(I + 1) % 2];
        const int bload = min(kt + NB, last);
        const int aload = min((kt - 1) / 2 + NA, last_pair);
        [&]<int... Q>(std::integer_sequence<int, Q...>) {
            ([&] {
                if constexpr (Q == PRE) {
                    wait_vmcnt_and_barrier<ODD ? kSched.odd_wait : kSched.even_wait>();
                    __builtin_amdgcn_sched_barrier(0);   // the scheduler would hoist the next MFMA above it
                }
                mfma_op(std::integral_constant<int, Q>{}, cur);
                constexpr int S = Q < PRE ? 0 : (Q - PRE) * PER;
                constexpr int lo = Q < PRE ? 0 : S < N_MEM ? S : N_MEM;
                constexpr int hi = Q < PRE ? 0 : S + PER < N_MEM ? S + PER : N_MEM;
                [&]<int... R>(std::integer_sequence<int, R...>) {
                    ([&] {
                        constexpr int m = lo + R;
                        if constexpr (kIsLoad(m)) {
                            constexpr int l = (m + 1) / kStride - 1;
                            if constexpr (l < A_LOADS)
                                issue_a(aload, load_a, std::integral_constant<int, l>{});
                            else
                                issue_b(bload, load_b, std::integral_constant<int, l - A_LOADS>{});
                        } else {
                            constexpr int loads_before = m / kStride < LOADS ? m / kStride : LOADS;
                            read_op(next_a, next_b, std::integral_constant<int, (I + 1) & 1>{},
                                    std::integral_constant<int, m - loads_before>{}, nxt);
                        }
                    }(), ...);
                }(std::make_integer_sequence<int, hi - lo>{});
                __builtin_amdgcn_sched_barrier(0);
            }(), ...);
        }(std::make_integer_sequence<int, N_MFMA>{});
    };
    constexpr int UNROLL = std::lcm(2 * NA, NB);
    for (int kt = 0; kt < ksteps; kt += UNROLL) {
        [&]<int... I>(std::integer_sequence<int, I...>) {
            ((kt + I < ksteps ? step(std::integral_constant<int, I>{}, kt + I) : void()), ...);
        }(std::make_integer_sequence<int, UNROLL>{});
    }
    wait_vmcnt_and_barrier<0>();

    // Epilogue. Accumulator register r = 4g + q of lane l holds
    // C[row = 32*i + l % 32][col = 32*j + 8g + 4*(l / 32) + q]: stored straight
    // from registers, every store instruction would put 16 bytes into each of
    // 32 rows. Instead each wave rounds its (WTM x WTN) tile to 16 bits into
    // its own region of the LDS ring (all of it is free after the final wait
    // and barrier), 32 rows at a time for 128-row wave tiles, and reads them
    // back row by row so that 16 (8, 4) lanes
    // store one 256-byte (128-, 64-byte) row segment of a 128- (64-, 32-)
    // column wave tile: whole cache lines (half lines for 32 columns), half
    // the store instructions. Staged rows are 16 (8, 4) chunks of 16 bytes;
    // chunk c of row r sits at chunk c ^ (r % chunks),
    // which keeps the reads (all chunks of a few rows) free of bank conflicts;
    // the writes (one chunk of 32 rows) conflict 2-way, since each half wave
    // fills only one 8-byte half of every chunk. Rows at or past M (a
    // partial last tile) are not stored. With K splits the block writes its
    // unscaled fp32 partial to ws[split][row][col] directly; a second kernel
    // sums the splits. Plans split only tiles of at most 128 rows, so the
    // 256-row kernels leave that path out (its registers spilled there).
    const int row0 = tm * BM + wm * WTM + (lane & 31);
    const int64_t col0 = (int64_t)tn * BN + wn * WTN + 4 * half;
    if (BM > 128 || ws == nullptr) {
        constexpr int ROW_BYTES = WTN * 2;
        constexpr int ROW_CHUNKS = ROW_BYTES / 16;
        static_assert(ROW_CHUNKS == 16 || ROW_CHUNKS == 8 || ROW_CHUNKS == 4,
                      "staging covers wave tiles 128, 64 or 32 columns wide");
        static_assert(W * WTM * ROW_BYTES <= LDS_BYTES, "the waves' tiles must fit the LDS ring");
        unsigned char* stage = lds + wave * WTM * ROW_BYTES;
        // alpha is 1 except for scaled fp8: the unscaled instantiation skips
        // the multiply, a VALU op per accumulator. Waves of 128 rows stage and
        // store 32 rows at a time, so a group's stores go out while the next
        // group is rounded; shorter wave tiles in one group (smaller groups
        // shorten their read-back batches, which cost 2-4% there).
        constexpr int GROUP = WTM >= 128 ? 32 : WTM;          // C rows per staged group
        auto stage_row = [&](auto irow) {
            constexpr int i = decltype(irow)::value;
            const int r = 32 * i + (lane & 31);
#pragma unroll
            for (int j = 0; j < FN; ++j) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const f32x16& v = acc[i][j];
                    u32x2 packed;
                    if constexpr (SCALED) {
                        packed = pack4<DT>(v[4 * g] * alpha, v[4 * g + 1] * alpha, v[4 * g + 2] * alpha,
                                           v[4 * g + 3] * alpha);
                    } else {
                        packed = pack4<DT>(v[4 * g], v[4 * g + 1], v[4 * g + 2], v[4 * g + 3]);
                    }
                    const int chunk = (4 * j + g) ^ (r % ROW_CHUNKS);
                    *reinterpret_cast<u32x2*>(stage + r * ROW_BYTES + chunk * 16 + 8 * half) = packed;
                }
            }
        };
        // Groups start on multiples of 32 rows, which keeps the staging swizzle (row % ROW_CHUNKS, ROW_CHUNKS <= 16).
        [&]<int... G>(std::integer_sequence<int, G...>) {
            ([&] {
                constexpr int grp = G;
                [&]<int... I>(std::integer_sequence<int, I...>) {
                    (stage_row(std::integral_constant<int, grp * (GROUP / 32) + I>{}), ...);
                }(std::make_integer_sequence<int, GROUP / 32>{});
                store_staged_tile<GROUP, ROW_BYTES>(stage + GROUP * grp * ROW_BYTES, C, M, N,
                                                    tm * BM + wm * WTM + GROUP * grp, (int64_t)tn * BN + wn * WTN, lane);
            }(), ...);
        }(std::make_integer_sequence<int, WTM / GROUP>{});
    } else if constexpr (BM <= 128) {
        float* part = ws + (int64_t)split * M * N;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            if (row0 + 32 * i >= M) continue;
            float* prow = part + (int64_t)(row0 + 32 * i) * N;
#pragma unroll
            for (int j = 0; j < FN; ++j) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const f32x16& v = acc[i][j];
                    const f32x4 q = {v[4 * g], v[4 * g + 1], v[4 * g + 2], v[4 * g + 3]};
                    // N is a multiple of 8: the 4 columns are all in C or all past it
                    if (col0 + 32 * j + 8 * g < N) *reinterpret_cast<f32x4*>(prow + col0 + 32 * j + 8 * g) = q;
                }
            }
        }
    }
}

// fp8 (e4m3 / e5m2) on v_mfma_scale_f32_16x16x128_f8f6f4, which sustains 7-8%
// more than the 32x32x64 form under the part's power limit. Same LDS ring,
// DMA loads, A pair layout and XCD tile order as gemm_tiled_kernel; what
// differs:
//  - Operand K layout. The instruction pairs byte b of lane l of one operand
//    with byte b of lane l of the other (both hold K in the same places), so
//    any K order shared by A and B gives the same dot product. Here lane l,
//    g = l / 16, holds K 16g .. 16g + 15 in bytes 0-15 and K 64 + 16g ..
//    64 + 16g + 15 in bytes 16-31: bytes 0-15 come from the first stage of a
//    pair and bytes 16-31 from the second, so B is still read one stage at a
//    time. A: two 16-byte reads (chunks g and 4 + g of the pair row). B: per
//    stage two transposing reads (8 K rows x 16 columns per 16-lane group).
//  - Steps. One MFMA consumes a whole pair (128 K), so the two steps of pair p
//    share its MFMAs: step 2p does fragment rows 0 .. FM/2 - 1, step 2p + 1
//    the rest. B fragments of pair p + 1 are read during pair p's steps (stage
//    k + 2 during step k, into the other of two B register sets); A fragment
//    rows stream one row ahead (row i + 1 is read after the first MFMA of row
//    i, row 0 of the next pair during the last row).
//  - Ring. B stage S lives in slot S % NB and is read during step S - 2; A
//    pair P in slot P % NA, read during steps 2P - 1 .. 2P + 1. Step k loads
//    A pair k / 2 + NA - 1 (even k) into the slot pair k / 2 - 1 vacated, and
//    B stage k + 1 + NB into the slot of stage k + 1; waits from
//    load_schedule_mi16.
//  - fp8 B rows: chunk c of row k stored at c ^ f(k), f = swz_b8(k & 7) ^ bit 4
//    of k (256-byte rows) or (k & 7) ^ bit 4 of k (128-byte rows): the two
//    16-lane groups of a 32-lane LDS phase read rows 16 apart.
// Requires an even number of stages per split.
constexpr int kMi16AAhead = 1;              // A fragment rows read this far ahead
constexpr bool kMi16SpreadLoads = true;     // DMA loads spread over the step, or first
constexpr bool kMi16SplitA = false;         // an A pair's loads over both steps of a pair, or the even one

__device__ __forceinline__ int swz_b8_mi16(int k, int row_bytes) {
    return (row_bytes == 256 ? swz_b8(k & 7) : (k & 7)) ^ ((k >> 4) & 1);
}

template <int DT>
__device__ __forceinline__ f32x4 mfma16_fp8(const i32x8& a, const i32x8& b, f32x4 c) {
    constexpr int fmt = DT == MB_DT_FLOAT8_E5M2 ? 1 : 0;  // 0 = e4m3, 1 = bf8 e5m2
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, fmt, fmt, 0, 0, 0, 0);
}

template <int DT, int BM, int BN, int WGM, int WGN, int NA, int NB, bool SCALED, bool RAGGED_K = false>
__global__ void __launch_bounds__(64 * WGM * WGN)
gemm_fp8_mi16_kernel(const unsigned char* __restrict__ A, const unsigned char* __restrict__ B,
                     unsigned char* __restrict__ C, int M, int N, int K, float alpha, int tiles_m, int tiles_n,
                     int group_m, int splits, int k_len, float* __restrict__ ws) {
    constexpr int W = WGM * WGN;
    constexpr int WTM = BM / WGM, WTN = BN / WGN;
    constexpr int FM = WTM / 16, FN = WTN / 16;
    constexpr int HALF_ROWS = FM / 2;                   // fragment rows per step
    constexpr int PAIR = 2 * BM * kStageK;              // A slot: two stages, [BM][128 B]
    constexpr int B_ROW = BN;                           // bytes per B row (fp8)
    constexpr int B_BYTES = kStageK * B_ROW;            // B slot: one stage, 64 K rows
    constexpr int A_INSTR = PAIR / 1024 / W;
    constexpr int B_INSTR = B_BYTES / 1024 / W;
    constexpr int RPI = 1024 / B_ROW;                   // B rows per DMA instruction
    constexpr int LDS_BYTES = NA * PAIR + NB * B_BYTES;
    static_assert(W == 4 && FM % 2 == 0 && FN >= 2, "four waves, an even number of fragment rows");
    static_assert(B_ROW == 256 || B_ROW == 128, "fp8 B rows of 256 or 128 bytes");
    static_assert(A_INSTR % 2 == 0 && B_INSTR % 2 == 0 && B_INSTR * RPI * W == kStageK,
                  "A and B offsets assume two vector offsets per wave");
    static_assert(NA >= 2 && NB >= 3 && LDS_BYTES <= 160 * 1024, "LDS ring does not fit");
    constexpr LoadSchedule kSched = load_schedule_mi16(NA, NB, A_INSTR, B_INSTR, kMi16SplitA);
    static_assert(kSched.prologue >= 0 && kSched.odd_wait >= 0 && kSched.even_wait >= 0 &&
                  kSched.prologue < 64 && kSched.odd_wait < 64 && kSched.even_wait < 64,
                  "load schedule leaves a needed stage unissued or overflows vmcnt");

    __shared__ __attribute__((aligned(1024))) unsigned char lds[LDS_BYTES];
    auto a_slot = [&](auto idx) -> unsigned char* {
        static_assert(decltype(idx)::value < NA, "A slot out of range");
        return lds + decltype(idx)::value * PAIR;
    };
    auto b_slot = [&](auto idx) -> unsigned char* {
        static_assert(decltype(idx)::value < NB, "B slot out of range");
        return lds + NA * PAIR + decltype(idx)::value * B_BYTES;
    };

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int g = lane >> 4, l16 = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WGN, wn = wave % WGN;
    const int split = splits > 1 ? (int)blockIdx.x % splits : 0;
    const int tile = splits > 1 ? (int)blockIdx.x / splits : (int)blockIdx.x;
    int tm, tn;
    tile_coords(tile, tiles_m * tiles_n, tiles_m, tiles_n, group_m, &tm, &tn);
    const int lda = K, ldb = N;
    const int k0 = split * k_len;

    const int a_rows = min(BM, M - tm * BM);
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<unsigned char*>(A) + (int64_t)tm * BM * lda, (short)0, a_rows * lda, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<unsigned char*>(B) + (int64_t)tn * BN, (short)0, K * ldb - tn * BN, kBufferFlags);

    // DMA offsets: instruction q of a wave covers A rows 8 * (wave * A_INSTR
    // + q) .. +7 (whole 128-byte pair rows) and B rows RPI * (wave * B_INSTR +
    // q) .. +RPI-1 of the stage. Both swizzles depend on q only through its
    // parity (the B rows of a wave share bit 4), so two vector offsets per
    // operand serve every q; the rest is a uniform offset.
    int a_voff[2], a_kbyte[2], b_voff[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int lin = (wave * A_INSTR + q) * 1024 + lane * 16;
        const int row = lin / (2 * kStageK), pchunk = (lin % (2 * kStageK)) >> 4;
        a_kbyte[q] = (pchunk ^ swz_a2(row)) << 4;
        a_voff[q] = row * lda + a_kbyte[q];
        const int blin = (wave * B_INSTR + q) * 1024 + lane * 16;
        const int brow = blin / B_ROW, bchunk = (blin % B_ROW) >> 4;
        b_voff[q] = brow * ldb + ((bchunk ^ swz_b8_mi16(brow, B_ROW)) << 4);
    }
    // RAGGED_K: A pieces at or past K load zeros, as in gemm_tiled_kernel.
    auto issue_a = [&](int pair, unsigned char* slot, auto idx) {
        constexpr int q = decltype(idx)::value;
        const unsigned base = (unsigned)(uintptr_t)(MB_LDS unsigned char*)slot;
        const int kb = k0 + pair * 2 * kStageK;
        int voff = a_voff[q & 1];
        if constexpr (RAGGED_K) voff = a_kbyte[q & 1] < K - kb ? voff : (int)0x80000000u;
        lds_dma16(ra, base + (wave * A_INSTR + q) * 1024, voff, kb + 16 * (q >> 1) * lda);
    };
    auto issue_b = [&](int kt, unsigned char* slot, auto idx) {
        constexpr int q = decltype(idx)::value;
        const unsigned base = (unsigned)(uintptr_t)(MB_LDS unsigned char*)slot;
        lds_dma16(rb, base + (wave * B_INSTR + q) * 1024, b_voff[q & 1],
                  (k0 + kt * kStageK + 2 * RPI * (q >> 1)) * ldb);
    };

    // Operand reads. A fragment row i (16 rows): chunks g and 4 + g of the
    // pair row. B fragment j, stage half h, part t: 8 K rows 16g + 8t .. +7
    // of the stage, columns b_col + 16j .. +15, into bytes 16h + 8t .. +7.
    // Per-lane byte offsets within a slot: the A swizzle of row a_row + 16i
    // equals that of l16 (wm * WTM and 16i leave bits 0-3 alone), and the B
    // swizzle of row 16g + 8t + l16 / 2 does not depend on t, so two A offsets
    // and one B offset per fragment column serve every read; rows and parts
    // are immediates.
    const int a_row = wm * WTM + l16;
    const int b_col = wn * WTN;
    const int sa = swz_a2(l16);
    int a_off[2] = {a_row * 2 * kStageK + ((g ^ sa) << 4), a_row * 2 * kStageK + (((4 + g) ^ sa) << 4)};
    const int kb = 16 * g + (l16 >> 1);
    int b_off[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j)
        b_off[j] = kb * B_ROW + ((((b_col >> 4) + j) ^ swz_b8_mi16(kb, B_ROW)) << 4) + 8 * (l16 & 1);
    // Slot bases past 64 KiB do not fit the LDS instructions' offset field;
    // redefining the offsets once per step (an empty asm) keeps the compiler
    // from hoisting a register per (slot, offset) out of the loop.
    auto launder_offsets = [&] {
        asm volatile("" : "+v"(a_off[0]), "+v"(a_off[1]));
#pragma unroll
        for (int j = 0; j < FN; ++j) asm volatile("" : "+v"(b_off[j]));
    };
    auto read_a = [&](const unsigned char* slot, int i, i32x8& dst) {
        const u32x4 lo = *reinterpret_cast<const u32x4*>(slot + a_off[0] + i * 16 * 2 * kStageK);
        const u32x4 hi = *reinterpret_cast<const u32x4*>(slot + a_off[1] + i * 16 * 2 * kStageK);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            dst[w] = (int)lo[w];
            dst[4 + w] = (int)hi[w];
        }
    };
    auto read_b = [&](const unsigned char* st, int j, int h, int t, i32x8& dst) {
        const i32x2_t v = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            (MB_LDS i32x2_t*)((MB_LDS unsigned char*)st + b_off[j] + t * 8 * B_ROW));
        dst[4 * h + 2 * t] = v[0];
        dst[4 * h + 2 * t + 1] = v[1];
    };

    f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    // A fragment rows are read A_AHEAD rows before their MFMAs, into a ring
    // of A_AHEAD + 1 registers sets indexed by the row's position in the
    // unrolled loop (pair * FM + row).
    constexpr int A_AHEAD = kMi16AAhead;
    i32x8 bop[2][FN];              // B fragments of the current and the next pair
    i32x8 aop[A_AHEAD + 1];

    const int ksteps = k_len / kStageK;  // even
    const int last = ksteps - 1;
    const int last_pair = last / 2;
    // Prologue: virtual steps -V..-1 issue A pairs 0..NA-2 and B stages 0..NB-1.
    constexpr int V = NB + 1 > 2 * NA - 2 ? NB + 1 : 2 * NA - 2;
    [&]<int... U>(std::integer_sequence<int, U...>) {
        ([&] {
            constexpr int v = U - V;
            constexpr int pair = floor_half(v) + NA - 1;
            if constexpr (pair >= 0 && (kMi16SplitA || (v & 1) == 0)) {
                constexpr int q0 = kMi16SplitA && (v & 1) != 0 ? A_INSTR / 2 : 0;
                constexpr int nq = kMi16SplitA ? A_INSTR / 2 : A_INSTR;
                [&]<int... Q>(std::integer_sequence<int, Q...>) {
                    (issue_a(min(pair, last_pair), a_slot(std::integral_constant<int, pair>{}),
                             std::integral_constant<int, q0 + Q>{}), ...);
                }(std::make_integer_sequence<int, nq>{});
            }
            if constexpr (v + 1 + NB >= 0 && v + 1 + NB < NB) {
                constexpr int st = v + 1 + NB;
                [&]<int... Q>(std::integer_sequence<int, Q...>) {
                    (issue_b(min(st, last), b_slot(std::integral_constant<int, st>{}),
                             std::integral_constant<int, Q>{}), ...);
                }(std::make_integer_sequence<int, B_INSTR>{});
            }
        }(), ...);
    }(std::make_integer_sequence<int, V>{});
    wait_vmcnt_and_barrier<kSched.prologue>();
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            read_b(b_slot(std::integral_constant<int, 0>{}), j, 0, t, bop[0][j]);
            read_b(b_slot(std::integral_constant<int, 1>{}), j, 1, t, bop[0][j]);
        }
#pragma unroll
    for (int i = 0; i < A_AHEAD; ++i) read_a(a_slot(std::integral_constant<int, 0>{}), i, aop[i]);
    // Every wave has read stage 0: its slot takes stage NB.
    wait_vmcnt_and_barrier<63>();
    [&]<int... Q>(std::integer_sequence<int, Q...>) {
        (issue_b(min(NB, last), b_slot(std::integral_constant<int, 0>{}), std::integral_constant<int, Q>{}), ...);
    }(std::make_integer_sequence<int, B_INSTR>{});

    auto step = [&](auto idx, int kt) {
        constexpr int I = decltype(idx)::value;
        constexpr int H = I & 1;                  // which half of the pair's fragment rows
        constexpr int CUR = (I / 2) & 1;          // B register set of this pair
        constexpr int A_LOADS = kMi16SplitA ? A_INSTR / 2 : H == 0 ? A_INSTR : 0;
        constexpr int A_Q0 = kMi16SplitA && H == 1 ? A_INSTR / 2 : 0;   // first A instruction of this step
        constexpr int LOADS = A_LOADS + B_INSTR;
        constexpr int N_MFMA = HALF_ROWS * FN;
        constexpr int N_OTHER = LOADS + 2 * FN;   // loads first, then this stage's next-pair B reads
        constexpr int PRE = kPreBarrierMfma < FN ? kPreBarrierMfma : FN - 1;   // MFMAs before the barrier,
        static_assert(PRE >= 0, "within the step's first fragment row");
        constexpr int PER = (N_OTHER + N_MFMA - PRE - 1) / (N_MFMA - PRE);
        const unsigned char* a_cur = a_slot(std::integral_constant<int, (I / 2) % NA>{});
        const unsigned char* a_next = a_slot(std::integral_constant<int, (I / 2 + 1) % NA>{});
        const unsigned char* b_read = b_slot(std::integral_constant<int, (I + 2) % NB>{});
        unsigned char* a_load = a_slot(std::integral_constant<int, (I / 2 + NA - 1) % NA>{});
        unsigned char* b_load = b_slot(std::integral_constant<int, (I + 1) % NB>{});
        const int aload = min((kt >> 1) + NA - 1, last_pair);
        const int bload = min(kt + 1 + NB, last);
        // Other memory instruction m is a load when m + 1 is one of the first
        // LOADS multiples of kStride (spread evenly), otherwise the next B read.
        constexpr int kStride = kMi16SpreadLoads ? N_OTHER / LOADS : 1;
        constexpr auto kIsLoad = [](int m) { return (m + 1) % kStride == 0 && (m + 1) / kStride <= LOADS; };
        [&]<int... Q>(std::integer_sequence<int, Q...>) {
            ([&] {
                constexpr int i = H * HALF_ROWS + Q / FN, j = Q % FN;
                constexpr int row_pos = (I / 2) * FM + i;   // position in the unrolled loop
                if constexpr (Q == PRE) {
                    wait_vmcnt_and_barrier<H ? kSched.odd_wait : kSched.even_wait>();
                    __builtin_amdgcn_sched_barrier(0);   // the scheduler would hoist the next MFMA above it
                    launder_offsets();
                }
                acc[i][j] = mfma16_fp8<DT>(bop[CUR][j], aop[row_pos % (A_AHEAD + 1)], acc[i][j]);
                // The next fragment row's A read follows the row's first MFMA, or for the step's first
                // row the barrier (a read before it would hold the barrier's LDS wait).
                if constexpr (Q / FN == 0 ? Q == PRE : j == 0) {
                    constexpr int ahead = (row_pos + A_AHEAD) % (A_AHEAD + 1);
                    if constexpr (i + A_AHEAD < FM) read_a(a_cur, i + A_AHEAD, aop[ahead]);
                    else read_a(a_next, i + A_AHEAD - FM, aop[ahead]);
                }
                constexpr int S = Q < PRE ? 0 : (Q - PRE) * PER;
                constexpr int lo = Q < PRE ? 0 : S < N_OTHER ? S : N_OTHER;
                constexpr int hi = Q < PRE ? 0 : S + PER < N_OTHER ? S + PER : N_OTHER;
                [&]<int... R>(std::integer_sequence<int, R...>) {
                    ([&] {
                        constexpr int m = lo + R;
                        if constexpr (kIsLoad(m)) {
                            constexpr int l = (m + 1) / kStride - 1;
                            if constexpr (l < A_LOADS) issue_a(aload, a_load, std::integral_constant<int, A_Q0 + l>{});
                            else issue_b(bload, b_load, std::integral_constant<int, l - A_LOADS>{});
                        } else {
                            constexpr int loads_before = m / kStride < LOADS ? m / kStride : LOADS;
                            constexpr int r = m - loads_before;
                            read_b(b_read, r / 2, H, r % 2, bop[CUR ^ 1][r / 2]);
                        }
                    }(), ...);
                }(std::make_integer_sequence<int, hi - lo>{});
                __builtin_amdgcn_sched_barrier(0);
            }(), ...);
        }(std::make_integer_sequence<int, N_MFMA>{});
    };
    // The stage count is even: both steps of a pair run or neither, so every
    // register set is whole wherever control flow joins.
    constexpr int UNROLL = std::lcm(std::lcm(2 * NA, NB), 4);
    static_assert((UNROLL / 2) * FM % (A_AHEAD + 1) == 0, "A register ring must wrap with the unrolled loop");
    for (int kt = 0; kt < ksteps; kt += UNROLL) {
        [&]<int... P>(std::integer_sequence<int, P...>) {
            ((kt + 2 * P < ksteps ? (step(std::integral_constant<int, 2 * P>{}, kt + 2 * P),
                                     step(std::integral_constant<int, 2 * P + 1>{}, kt + 2 * P + 1))
                                  : void()), ...);
        }(std::make_integer_sequence<int, UNROLL / 2>{});
    }
    wait_vmcnt_and_barrier<0>();

    // Epilogue. Accumulator register r of fragment (i, j) of lane l holds
    // C[16i + l % 16][16j + 4(l / 16) + r]: four consecutive columns of one
    // row, rounded to 16 bits into the wave's LDS staging rows and stored as
    // whole row segments (store_staged_tile). With K splits the block writes
    // its unscaled fp32 partial to ws[split][row][col] instead (tiles of at
    // most 128 rows only).
    if (BM > 128 || ws == nullptr) {
        constexpr int ROW_BYTES = WTN * 2;
        constexpr int ROW_CHUNKS = ROW_BYTES / 16;
        static_assert(ROW_CHUNKS == 16 || ROW_CHUNKS == 8, "staging covers wave tiles 128 or 64 columns wide");
        static_assert(W * WTM * ROW_BYTES <= LDS_BYTES, "the waves' tiles must fit the LDS ring");
        unsigned char* stage = lds + wave * WTM * ROW_BYTES;
        // Waves of 128 rows in groups of 32 (two fragment rows), as in
        // gemm_tiled_kernel: a group's stores go out while the next is
        // rounded; groups start on multiples of 32 rows, which keeps the
        // staging swizzle. Shorter wave tiles in one group.
        constexpr int GROUP = WTM >= 128 ? 32 : WTM;          // C rows per staged group
        static_assert(GROUP % 16 == 0 && WTM % GROUP == 0, "groups of whole fragment rows");
        [&]<int... P>(std::integer_sequence<int, P...>) {
            ([&] {
                constexpr int p = P;
#pragma unroll
                for (int i = p * (GROUP / 16); i < (p + 1) * (GROUP / 16); ++i) {
                    const int r = 16 * i + l16;
#pragma unroll
                    for (int j = 0; j < FN; ++j) {
                        const f32x4& v = acc[i][j];
                        u32x2 packed;
                        if constexpr (SCALED) packed = pack4<DT>(v[0] * alpha, v[1] * alpha, v[2] * alpha, v[3] * alpha);
                        else packed = pack4<DT>(v[0], v[1], v[2], v[3]);
                        const int chunk = (2 * j + (g >> 1)) ^ (r % ROW_CHUNKS);
                        *reinterpret_cast<u32x2*>(stage + r * ROW_BYTES + chunk * 16 + 8 * (g & 1)) = packed;
                    }
                }
                store_staged_tile<GROUP, ROW_BYTES>(stage + GROUP * p * ROW_BYTES, C, M, N, tm * BM + wm * WTM + GROUP * p,
                                                    (int64_t)tn * BN + wn * WTN, lane);
            }(), ...);
        }(std::make_integer_sequence<int, WTM / GROUP>{});
    } else if constexpr (BM <= 128) {
        float* part = ws + (int64_t)split * M * N;
        const int row0 = tm * BM + wm * WTM + l16;
        const int64_t col0 = (int64_t)tn * BN + wn * WTN + 4 * g;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            if (row0 + 16 * i >= M) continue;
            float* prow = part + (int64_t)(row0 + 16 * i) * N;
#pragma unroll
            for (int j = 0; j < FN; ++j)
                if (col0 + 16 * j < N) *reinterpret_cast<f32x4*>(prow + col0 + 16 * j) = acc[i][j];
        }
    }
}

// Sum of the K-split partials: C[m][n] = alpha * sum_s ws[s][m][n], rounded
// once to the output type. Each thread handles 4 consecutive columns and has
// L splits' loads in flight at once, L the split count rounded up to a power
// of two (at most 32): the planes were just written by the GEMM kernel, so
// the pass is latency-bound. The adds keep split order.
template <int DT, int L>
__global__ void __launch_bounds__(256)
gemm_splitk_reduce_kernel(const float* __restrict__ ws, unsigned char* __restrict__ C, int64_t quads,
                          int64_t plane, int splits, float alpha) {
    constexpr int kLoads = L;
    const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= quads) return;
    f32x4 sum = {-0.f, -0.f, -0.f, -0.f};   // -0 + x == x for every x, so the sum starts exactly at split 0
    for (int s0 = 0; s0 < splits; s0 += kLoads) {
        f32x4 v[kLoads];
#pragma unroll
        for (int u = 0; u < kLoads; ++u)
            v[u] = s0 + u < splits ? *reinterpret_cast<const f32x4*>(ws + (s0 + u) * plane + 4 * q)
                                   : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < kLoads; ++u)
            if (s0 + u < splits) sum += v[u];
    }
    *reinterpret_cast<u32x2*>(C + 8 * q) = pack4<DT>(sum[0] * alpha, sum[1] * alpha, sum[2] * alpha, sum[3] * alpha);
}

struct TiledConfig {
    int bm, bn, wgm, wgn, na, nb, group_m;  // na A pair slots, nb B stage slots
};

constexpr TiledConfig kConfigs[] = {
    {256, 256, 2, 2, 3, 4, 4},  // 0: large problems, 128 x 128 per wave; 3 x 32 + 4 x 16 KiB
    {128, 256, 2, 2, 3, 6, 8},  // 1: mid-size problems, 64 x 128 per wave; 3 x 16 + 6 x 16 KiB
    {128, 128, 2, 2, 3, 6, 4},  // 2: few tiles, N % 256 != 0: 64 x 64 per wave; 3 x 16 + 6 x 8 KiB
    {64, 128, 2, 2, 3, 6, 4},   // 3: small and skinny problems: 32 x 64 per wave; 3 x 8 + 6 x 8 KiB
    {64, 64, 2, 2, 3, 6, 4},    // 4: one-round problems of up to 256 such tiles: 32 x 32 per wave; 3 x 8 + 6 x 4 KiB
};

template <int DT, int CFG>
int launch_cfg(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, float alpha,
               const GemmPlan& plan, void* workspace, hipStream_t stream) {
    constexpr TiledConfig c = kConfigs[CFG];
    const int tiles_m = (int)((M + c.bm - 1) / c.bm), tiles_n = (int)((N + c.bn - 1) / c.bn);
    const int splits = plan.split_k;
    float* ws = splits > 1 ? static_cast<float*>(workspace) : nullptr;
    const dim3 grid(tiles_m * tiles_n * splits), block(64 * c.wgm * c.wgn);
    const auto* a = static_cast<const unsigned char*>(A);
    const auto* b = static_cast<const unsigned char*>(B);
    auto* cp = static_cast<unsigned char*>(C);
    // Only fp8 carries a scale; the split-K partials are scaled by the reduction.
    // fp8 runs the 16x16x128 kernel when the plan says so (frag_m 16).
    typedef void (*Kernel)(const unsigned char*, const unsigned char*, unsigned char*, int, int, int, float, int,
                           int, int, int, int, float*);
    const bool scaled = is_fp8(DT) && alpha != 1.0f && splits == 1;
    // K not a multiple of splits x stage: every split runs k_len (whole
    // stages), and the instantiations with RAGGED_K zero the A pieces past K.
    const int64_t stage_k = kStageK / Traits<DT>::kElem;
    const int64_t stages = (K + stage_k - 1) / stage_k;
    const int64_t k_len = (stages + splits - 1) / splits * stage_k;   // the plan's split_k_len
    const bool ragged_k = k_len * splits != K;
    auto pick = [&](auto rk) -> Kernel {
        constexpr bool RK = decltype(rk)::value;
        if constexpr (is_fp8(DT)) {
            if constexpr (c.bn >= 128) {   // the 16x16x128 kernel's B swizzles cover rows of 128 bytes or more
                if (plan.frag_m == 16)
                    return scaled ? gemm_fp8_mi16_kernel<DT, c.bm, c.bn, c.wgm, c.wgn, c.na, c.nb, true, RK>
                                  : gemm_fp8_mi16_kernel<DT, c.bm, c.bn, c.wgm, c.wgn, c.na, c.nb, false, RK>;
            }
            if (scaled) return gemm_tiled_kernel<DT, c.bm, c.bn, c.wgm, c.wgn, c.na, c.nb, true, RK>;
        }
        return gemm_tiled_kernel<DT, c.bm, c.bn, c.wgm, c.wgn, c.na, c.nb, false, RK>;
    };
    const Kernel kernel = ragged_k ? pick(std::true_type{}) : pick(std::false_type{});
    hipLaunchKernelGGL(kernel, grid, block, 0, stream, a, b, cp, (int)M, (int)N, (int)K, scaled ? alpha : 1.0f,
                       tiles_m, tiles_n, c.group_m, splits, (int)k_len, ws);
    MB_HIP_TRY(hipGetLastError());
    if (splits > 1) {
        const int64_t quads = M * N / 4;
        auto reduce = splits <= 4 ? gemm_splitk_reduce_kernel<DT, 4>
                    : splits <= 8 ? gemm_splitk_reduce_kernel<DT, 8>
                    : splits <= 16 ? gemm_splitk_reduce_kernel<DT, 16> : gemm_splitk_reduce_kernel<DT, 32>;
        hipLaunchKernelGGL(reduce, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, stream,
                           static_cast<const float*>(ws), static_cast<unsigned char*>(C), quads, M * N, splits, alpha);
        MB_HIP_TRY(hipGetLastError());
    }
    return MB_OK;
}

template <int DT>
int launch_dtype(const GemmPlan& plan, const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
                 float alpha, void* workspace, hipStream_t stream) {
    if (plan.config == 0) return launch_cfg<DT, 0>(A, B, C, M, N, K, alpha, plan, workspace, stream);
    if (plan.config == 2) return launch_cfg<DT, 2>(A, B, C, M, N, K, alpha, plan, workspace, stream);
    if (plan.config == 3) return launch_cfg<DT, 3>(A, B, C, M, N, K, alpha, plan, workspace, stream);
    if (plan.config == 4) return launch_cfg<DT, 4>(A, B, C, M, N, K, alpha, plan, workspace, stream);
    return launch_cfg<DT, 1>(A, B, C, M, N, K, alpha, plan, workspace, stream);
}

}  // namespace

// Picks the tiled configuration for a shape, or returns MB_ERR_SHAPE with
// *why set when the shape does not divide into any of them (or its buffers
// need offsets beyond the 32-bit range of buffer addressing).
int gemm_tiled_plan(int dtype, int64_t M, int64_t N, int64_t K, const DeviceProps& props,
                    GemmPlan* plan, const char** why) {
    const int64_t e = is_fp8(dtype) ? 1 : 2;
    const int64_t stage_k = kStageK / e;
    // B's rows must start on 16 bytes (N a multiple of 8, or of 16 for fp8)
    // for the 16-byte DMA loads. N a multiple of 256 takes any tile width; a
    // multiple of 128 only the 128-column tiles (configurations 2 and 3),
    // which then cover N exactly. Any other N (ragged) takes any tile width,
    // with a partial last column of tiles: its columns past N load the start
    // of B's next row (or zeros past B's end) and are not stored.
    if ((N * e) % 16 != 0) {
        *why = e == 1 ? "N is not a multiple of 16" : "N is not a multiple of 8";
        return MB_ERR_SHAPE;
    }
    const bool ragged_n = N % 128 != 0;
    const bool n128_only = !ragged_n && N % 256 != 0;
    // A's rows must start on 16 bytes too. K that is not a multiple of the
    // stage (ragged) runs over k_pad, K rounded up to whole stages: the A
    // pieces past K load zeros, and B's rows past K lie past B's end.
    if ((K * e) % 16 != 0) {
        *why = e == 1 ? "K is not a multiple of 16" : "K is not a multiple of 8";
        return MB_ERR_SHAPE;
    }
    const int64_t k_pad = (K + stage_k - 1) / stage_k * stage_k;
    // 32-bit buffer offsets: B's rows up to k_pad (plus a partial tile's 256
    // columns past the last), a 256-row A panel, and the C / partial planes.
    if ((k_pad * N + 256) * e >= (int64_t(1) << 31) || 256 * k_pad * e >= (int64_t(1) << 31) ||
        M >= (int64_t(1) << 31) || M * N >= (int64_t(1) << 31)) {
        *why = "operand offsets exceed 32-bit buffer addressing (K*N or 256*K bytes, or M*N, >= 2^31)";
        return MB_ERR_SHAPE;
    }
    // K splits. A whole-stage K splits into s parts of K / s when they are
    // whole stages. A ragged K splits into ceil(stages / s) stages each, the
    // last split running furthest past K, for any s up to the stage count
    // whose rows stay within 32-bit offsets.
    const bool ragged_k = k_pad != K;
    const int64_t stages = k_pad / stage_k;
    auto split_ok = [&](int64_t sp) {
        if (!ragged_k) return K % (stage_k * sp) == 0;
        return sp <= stages && ((stages + sp - 1) / sp * sp * stage_k * N + 256) * e < (int64_t(1) << 31);
    };
    auto split_k_len = [&](int64_t sp) { return (stages + sp - 1) / sp * stage_k; };
    const int64_t cus = props.cu_count > 0 ? props.cu_count : 256;
    auto tiles = [&](int i) {
        return ((M + kConfigs[i].bm - 1) / kConfigs[i].bm) * ((N + kConfigs[i].bn - 1) / kConfigs[i].bn);
    };
    const int forced_cfg = (int)tuning(MB_TUNE_GEMM_TILED_CONFIG);  // -1 unless forced
    const int pinned = forced_cfg >= 0 && n128_only && forced_cfg < 2 ? 2 : forced_cfg;
    // 256 x 256 tiles once they occupy more than half the CUs. Short of a
    // full round they still beat the smaller tiles, whose twice-as-many
    // blocks need a second round: on MI355X, with A and B cycled through
    // copies that exceed the Infinity Cache, 16 shapes with 132 to 240 such
    // tiles (M 1536..4096, N 3072..8192, K 512..8192) ran 1.12-1.64x faster on
    // them than on the cost model's pick, 1.29x in geometric mean over bf16
    // and fp8 e4m3 (bf16 3072 x 3072 x 4096 74.8 against 104.6 us on 128 x 256
    // tiles at 2 splits, fp8 4096 x 3072 x 8192 74.5 against 122.4 on 128 x
    // 128), while at 128 or 64 of them (1024 x 8192, 2048 x 4096, 2048^2) they
    // ran 27-125% slower.
    int cfg = pinned >= 0 ? pinned : (!n128_only && 2 * tiles(0) > cus && M % kConfigs[0].bm == 0) ? 0 : -1;
    // Last-round fill. 128 x 256 tiles run 7-14% below 256 x 256 per FLOP on
    // MI355X, and a partly filled last round costs less than a full one (the
    // busy CUs clock up under the power limit), so the smaller tile pays only
    // when the last 256 x 256 round is at most a quarter full and there are
    // few rounds: 2560 x 8192 x 8192 ran 11-14% faster on 128 x 256 tiles,
    // 6144^3 1-5%, while 2.5- and 3.5-round shapes ran 3-15% slower.
    // Such shapes have at least one tile per CU: no K split.
    bool fill_rule = false;
    if (pinned < 0 && cfg == 0) {
        const int64_t full = tiles(0) / cus, rest = tiles(0) % cus;
        fill_rule = full <= 2 && rest > 0 && 4 * rest <= cus;
        if (fill_rule) cfg = 1;
    }
    // Problems with too few 256 x 256 tiles to fill half the GPU: the tile
    // configuration (128 x 256, 128 x 128 or 64 x 128) and the K split count s
    // (1, 2, 4 .. 32, whole stages per split) that a cost model rates fastest:
    //   blocks  = tiles * s, in ceil(blocks / CUs) rounds;
    //   MFMA    = rounds x one block's 2 * BM * BN * K / s FLOP at a per-CU
    //             rate of the configuration (3.70 / 2.87 / 1.99 TFLOP/s for
    //             16-bit inputs, twice that for fp8);
    //   stream  = the A and B bytes at 6.26 TB/s times the fraction of the
    //             CUs the blocks occupy (each block keeps a fixed number of
    //             loads in flight, so too few blocks leave HBM idle);
    //   partials (s > 1): the fp32 partials written and read back at the
    //             same rate, plus 4.72 us for the reduction pass;
    //   time    = max(MFMA, stream) + rounds x 2.71 us (prologue, epilogue)
    //             + partials.
    // The constants minimise the measured cost of the model's pick, not its
    // timing error (they are effective figures, not the part's rates), over
    // 906 timings on MI355X (bf16, fp16, fp8 e4m3; 61 shapes, M = 8..4096,
    // N = 256..16384, K = 768..16384; every configuration x split 1..16),
    // with B cycled through copies that exceed the 256 MB Infinity Cache:
    // the pick is within 0.65% of the measured best in geometric mean (11%
    // at worst), against 1.8% (24%) for constants fitted to the timings
    // themselves. On 48 further shapes where the two sets pick differently
    // (splits up to 32), these picks ran 7.6% faster in geometric mean
    // (0.89x - 1.39x): fp8 128 x 14336 x 8192 37.7 us on 128 x 128 tiles at
    // 2 splits against 43.5 on 64 x 128 at 1, fp8 8 x 1024 x 2048 7.9 us at 32
    // splits against 11.0 at 1, bf16 32 x 14336 x 8192 55.5 us at 4 splits
    // against 49.4 at 2.
    int splits = 1;
    if (!fill_rule && (cfg < 0 || kConfigs[cfg].bm <= 128)) {
        // kRate[4] (64 x 64 tiles) only prices the split count when that configuration is forced.
        constexpr double kRate[5] = {0.0, 3.70e12, 2.87e12, 1.99e12, 1.20e12}, kBw = 6.26e12, kRound = 2.71e-6,
                         kReduce = 4.72e-6;
        int cands[3] = {1, 2, 3}, n_cands = 3, first = 0;
        if (cfg >= 0) cands[0] = cfg, n_cands = 1;
        else if (n128_only) first = 1;
        double best = -1.0;
        for (int ci = first; ci < n_cands; ++ci) {
            const int c = cands[ci];
            const double bm = kConfigs[c].bm, bn = kConfigs[c].bn;
            const double rate = kRate[c] * (e == 1 ? 2.0 : 1.0);
            for (int64_t sp = 1; sp <= 32; sp *= 2) {
                if (!split_ok(sp)) continue;
                const double blocks = (double)(tiles(c) * sp);
                const double rounds = std::ceil(blocks / (double)cus);
                const double mfma = rounds * 2.0 * bm * bn * (double)split_k_len(sp) / rate;
                const double occupancy = blocks < (double)cus ? blocks / (double)cus : 1.0;
                const double stream = (double)((K * N + M * K) * e) / (kBw * occupancy);
                const double partials = sp > 1 ? 2.0 * (double)sp * (double)M * (double)N * 4.0 / kBw + kReduce : 0.0;
                const double t = (mfma > stream ? mfma : stream) + rounds * kRound + partials;
                if (best < 0.0 || t < best) {
                    best = t;
                    cfg = c;
                    splits = (int)sp;
                }
            }
        }
    }
    // 64 x 64 tiles for narrow problems: a plan of 64 x 128 tiles with N at
    // most 2048 takes them with half its K splits (the same block count, each
    // block half the columns over twice the K: one reduction pass less, or
    // none), or, unsplit, when twice its blocks still fit one round. On
    // MI355X, B from HBM, 61 such shapes (M 8..1024, N 256..2048, K
    // 512..16384, bf16 and fp8 e4m3) ran 1.128x faster in geometric mean
    // (0.96x - 1.33x): 1024^3 bf16 6.3 against 7.6 us, 1024 x 1024 x 2048 7.8
    // against 14.0 (no split instead of two), 128 x 1024 x 8192 12.8 against
    // 14.6. Wider N keeps 64 x 128 tiles: their 256-byte B rows stream HBM
    // better (16 x 8192 x 8192 fp8 19.7 against 22.1 us on 64 x 64).
    if (pinned < 0 && cfg == 3 && N <= 2048) {
        const int s4 = splits > 1 ? splits / 2 : 1;
        if (splits > 1 || tiles(4) <= cus) {
            cfg = 4;
            splits = s4;
        }
    }
    const int64_t force_splits = tuning(MB_TUNE_GEMM_SPLITS);
    if (force_splits >= 1 && split_ok(force_splits)) splits = (int)force_splits;
    if (kConfigs[cfg].bm > 128) splits = 1;   // the 256-row kernels carry no split path
    if (tiles(cfg) * splits > INT32_MAX) {
        *why = "more than 2^31 tiles";
        return MB_ERR_SHAPE;
    }
    const TiledConfig& c = kConfigs[cfg];
    // fp8 takes v_mfma_scale_f32_16x16x128_f8f6f4 on tiles of 128 rows or
    // more when every split holds an even number of stages (one MFMA spans
    // two): on MI355X 2.3-4.2% faster than the 32x32x64 kernel at 4096^3 -
    // 16384^3 (256 x 256), 2.6-3.9% on 128 x 256 tiles, and on 128 x 128 tiles
    // 2-5.5% faster on 8 of 10 shapes (2048^3 13.5 against 14.3 us, e4m3 and
    // e5m2 alike), equal at 128 x 8192 x 8192 and 1% slower at 1024 x 1024 x
    // 4096. The 64 x 128 tiles (two fragment rows per wave) keep 32x32x64:
    // within 0.6% either way there. The gemm_fp8_mfma override (16 or 32)
    // forces either.
    const int64_t mfma_force = tuning(MB_TUNE_GEMM_FP8_MFMA);
    const bool mi16 = e == 1 && (split_k_len(splits) / stage_k) % 2 == 0 && c.bn >= 128 &&
                      (mfma_force == 16 || (mfma_force != 32 && c.bm >= 128));
    const int frag = mi16 ? 16 : 32;
    plan->implementation = mi16 ? "gfx950_mfma16_lds_dma" : "gfx950_mfma32_lds_dma";
    plan->threads = 64 * c.wgm * c.wgn;
    plan->grid = (int)(tiles(cfg) * splits);
    plan->tile_m = c.bm;
    plan->tile_n = c.bn;
    plan->tile_k = (int)stage_k;
    plan->wave_grid_m = c.wgm;
    plan->wave_grid_n = c.wgn;
    plan->wave_tile_m = c.bm / c.wgm / frag;
    plan->wave_tile_n = c.bn / c.wgn / frag;
    plan->frag_m = frag;
    plan->frag_n = frag;
    plan->frag_k = mi16 ? 128 : is_fp8(dtype) ? 64 : 16;
    plan->k_stages = c.nb;
    plan->split_k = splits;
    plan->tile_group_m = c.group_m;
    plan->workspace = splits > 1 ? (size_t)splits * (size_t)M * (size_t)N * sizeof(float) : 0;
    plan->variant = kVariantTiled;
    plan->config = cfg;
    return MB_OK;
}

int gemm_tiled_launch(int dtype, const void* A, const void* B, void* C, int64_t M, int64_t N,
                      int64_t K, float alpha, void* workspace, const GemmPlan& plan, hipStream_t stream) {
    switch (dtype) {
        case MB_DT_BFLOAT16:
            return launch_dtype<MB_DT_BFLOAT16>(plan, A, B, C, M, N, K, alpha, workspace, stream);
        case MB_DT_FLOAT16:
            return launch_dtype<MB_DT_FLOAT16>(plan, A, B, C, M, N, K, alpha, workspace, stream);
        case MB_DT_FLOAT8_E4M3FN:
            return launch_dtype<MB_DT_FLOAT8_E4M3FN>(plan, A, B, C, M, N, K, alpha, workspace, stream);
        case MB_DT_FLOAT8_E5M2:
            return launch_dtype<MB_DT_FLOAT8_E5M2>(plan, A, B, C, M, N, K, alpha, workspace, stream);
        default:
            set_error("tiled GEMM: unsupported dtype %d", dtype);
            return MB_ERR_UNSUPPORTED;
    }
}

}  // namespace mb

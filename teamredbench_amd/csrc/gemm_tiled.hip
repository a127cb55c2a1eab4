// LDS-tiled MFMA GEMM for gfx950: C = alpha * (A * B), A (M x K) and B (K x N)
// row-major, fp32 accumulation, output bf16 (bf16 and fp8 e4m3 inputs) or
// fp16 (fp16 inputs). Takes shapes with M % BM == 0, N % BN == 0 and
// K % BK == 0; everything else goes to the generic kernel.
//
// Block tile BM x BN, K step of 128 bytes per row (BK = 64 for 16-bit
// inputs, 128 for fp8). Both operands live in LDS K-contiguous -- A as
// [m][128 B], B as [n][128 B] -- so every lane fetches its MFMA operand with
// one (16-bit) or two (fp8) 16-byte LDS reads. B arrives N-contiguous from
// HBM: each thread loads an 8-column strip of 8 (16-bit) or 16 (fp8) K-rows
// and transposes it in registers before the LDS write, so no re-layout pass
// over B runs outside the kernel. 16-byte chunks are XOR-swizzled by row
// (chunk ^ ((row ^ row >> 3) & 7)), which keeps the MFMA operand reads and
// the A writes free of bank conflicts.
//
// Two LDS buffers: while the waves run the MFMAs of step k out of one
// buffer, the buffer loads of step k+1 are in flight into registers; they go
// to the other buffer after the MFMAs, and one barrier per step orders both.
// The K loop is unrolled by two so every LDS address is a loop-invariant
// register plus an immediate.
//
// Waves form a WGM x WGN grid; each wave owns a (BM/WGM) x (BN/WGN) block of
// 32 x 32 fragments: v_mfma_f32_32x32x16_{bf16,f16}, or for fp8
// v_mfma_f32_32x32x64_f8f6f4 (e4m3 operands). The MFMA takes the B fragment
// as its first operand, so a lane's 16 accumulators are 4 runs of 4
// consecutive C columns in one C row: the epilogue stores 8 bytes at a time.
//
// Tile order: blocks are dispatched round-robin over the 8 XCDs, so block b
// runs on XCD b % 8; the kernel hands each XCD a contiguous range of tiles,
// walked in groups of `group_m` tile rows so the blocks sharing an XCD's L2
// also share A row panels and B column panels.
#include "gemm_common.hpp"

#include <cstdlib>

namespace mb {
namespace {

constexpr int kRowBytes = 128;  // bytes of K per LDS row (8 chunks of 16 B)
constexpr int kBufferFlags = 0x00020000;  // raw buffer resource word 3 on gfx9

__device__ __forceinline__ int swz(int row) { return (row ^ (row >> 3)) & 7; }
__device__ __forceinline__ int lds_off(int row, int chunk) {
    return row * kRowBytes + ((chunk ^ swz(row)) << 4);
}

typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));
typedef unsigned char u8x8 __attribute__((ext_vector_type(8)));
typedef unsigned char u8x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// ---- per-dtype pieces -------------------------------------------------------

template <int DT>
struct Traits;

template <>
struct Traits<MB_DT_BFLOAT16> {
    static constexpr int kElem = 2;
    static constexpr int kBK = 64;          // K elements per step
    static constexpr int kStripRows = 8;    // K rows per B strip (16-byte row loads)
    static constexpr int kSub = 4;          // MFMA K substeps per step
    typedef u32x4 Frag;                     // one lane's operand: 8 bf16
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
    static constexpr int kBK = 128;
    static constexpr int kStripRows = 16;   // 8-byte row loads
    static constexpr int kSub = 2;
    typedef i32x8 Frag;                     // one lane's operand: 32 e4m3
    // Format code 0 = e4m3 for both operands; zero scale operands select the
    // unscaled encoding of the instruction.
    __device__ static __forceinline__ f32x16 mfma(const Frag& a, const Frag& b, f32x16 c) {
        return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
    }
};

// Registers of one B strip: kStripRows row loads of 8 columns.
template <int DT>
struct Strip;

template <>
struct Strip<MB_DT_BFLOAT16> {
    u32x4 r[8];
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rsrc, int voff, int soff, int ldb) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            r[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, voff, soff + i * ldb, 0));
    }
    // Column j (0..7) as 8 consecutive K values: 16 bytes.
    __device__ __forceinline__ u32x4 column(int j) const {
        u16x8 out;
#pragma unroll
        for (int i = 0; i < 8; ++i) out[i] = __builtin_bit_cast(u16x8, r[i])[j];
        return __builtin_bit_cast(u32x4, out);
    }
};
template <>
struct Strip<MB_DT_FLOAT16> : Strip<MB_DT_BFLOAT16> {};

template <>
struct Strip<MB_DT_FLOAT8_E4M3FN> {
    u32x2 r[16];
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rsrc, int voff, int soff, int ldb) {
#pragma unroll
        for (int i = 0; i < 16; ++i)
            r[i] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rsrc, voff, soff + i * ldb, 0));
    }
    // Column j (0..7) as 16 consecutive K values: 16 bytes.
    __device__ __forceinline__ u32x4 column(int j) const {
        u8x16 out;
#pragma unroll
        for (int i = 0; i < 16; ++i) out[i] = __builtin_bit_cast(u8x8, r[i])[j];
        return __builtin_bit_cast(u32x4, out);
    }
};

// Operand fragment of a 32-row slab at `row0`, K substep `s`.
template <int DT>
__device__ __forceinline__ typename Traits<DT>::Frag load_frag(const unsigned char* lds, int row, int s,
                                                               int half) {
    if constexpr (Traits<DT>::kElem == 2) {
        // 32x32x16: lane holds K 8*half .. 8*half+7 of substep s -> chunk 2s + half.
        return *reinterpret_cast<const u32x4*>(lds + lds_off(row, 2 * s + half));
    } else {
        // 32x32x64: lane holds K 32*half .. 32*half+31 of substep s -> chunks 4s+2half, +1.
        const u32x4 lo = *reinterpret_cast<const u32x4*>(lds + lds_off(row, 4 * s + 2 * half));
        const u32x4 hi = *reinterpret_cast<const u32x4*>(lds + lds_off(row, 4 * s + 2 * half + 1));
        return __builtin_bit_cast(i32x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
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

// Tile index -> (tile row, tile column), XCD-contiguous and grouped by rows.
__device__ __forceinline__ void tile_coords(int b, int nblocks, int tiles_m, int tiles_n, int group_m,
                                            int* tm, int* tn) {
    int t = b;
    if ((nblocks & 7) == 0) t = (b & 7) * (nblocks >> 3) + (b >> 3);
    const int per_group = group_m * tiles_n;
    const int g = t / per_group;
    const int first_m = g * group_m;
    const int rows = min(tiles_m - first_m, group_m);
    const int r = t - g * per_group;
    *tm = first_m + r % rows;
    *tn = r / rows;
}

template <int DT, int BM, int BN, int WGM, int WGN>
__global__ void __launch_bounds__(64 * WGM * WGN)
gemm_tiled_kernel(const unsigned char* __restrict__ A, const unsigned char* __restrict__ B,
                  unsigned char* __restrict__ C, int M, int N, int K, float alpha, int tiles_m,
                  int tiles_n, int group_m) {
    typedef Traits<DT> Tr;
    typedef typename Tr::Frag Frag;
    constexpr int T = 64 * WGM * WGN;
    constexpr int E = Tr::kElem;
    constexpr int WTM = BM / WGM, WTN = BN / WGN;
    constexpr int FM = WTM / 32, FN = WTN / 32;
    constexpr int A_CHUNKS = BM * 8 / T;          // 16-byte A chunks per thread per step
    constexpr int B_STRIPS = (BN + T - 1) / T;    // B strips per thread per step
    constexpr int A_BYTES = BM * kRowBytes, B_BYTES = BN * kRowBytes;
    static_assert(BM * 8 % T == 0, "A tile must split evenly over the block");
    static_assert(FM >= 1 && FN >= 1 && WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be 32-aligned");

    __shared__ __attribute__((aligned(16))) unsigned char lds[2 * (A_BYTES + B_BYTES)];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    int tm, tn;
    tile_coords(blockIdx.x, gridDim.x, tiles_m, tiles_n, group_m, &tm, &tn);
    const int lda = K * E;   // bytes per A row
    const int ldb = N * E;   // bytes per B row

    // Buffer resources over this block's A row panel and B column panel.
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<unsigned char*>(A) + (int64_t)tm * BM * lda, (short)0, BM * lda, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<unsigned char*>(B) + (int64_t)tn * BN * E, (short)0, K * ldb, kBufferFlags);

    // A: thread t moves chunk (t % 8) of rows t/8 + i*(T/8).
    const int a_row0 = tid >> 3, a_chunk = tid & 7;
    const int a_voff = a_row0 * lda + a_chunk * 16;
    // B: strip sb = t + i*T covers columns 8*(sb % (BN/8)) .. +7 and K chunk sb / (BN/8).
    int b_voff[B_STRIPS], b_ng[B_STRIPS], b_kg[B_STRIPS];
#pragma unroll
    for (int i = 0; i < B_STRIPS; ++i) {
        const int sb = tid + i * T;
        b_ng[i] = sb % (BN / 8);
        b_kg[i] = sb / (BN / 8);
        b_voff[i] = b_kg[i] * Tr::kStripRows * ldb + b_ng[i] * 8 * E;
    }

    u32x4 a_reg[A_CHUNKS];
    Strip<DT> b_reg[B_STRIPS];

    auto load_step = [&](int kt) {
        const int a_soff = kt * kRowBytes;
#pragma unroll
        for (int i = 0; i < A_CHUNKS; ++i)
            a_reg[i] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, a_voff, a_soff + i * (T / 8) * lda, 0));
        const int b_soff = kt * Tr::kBK * ldb;
#pragma unroll
        for (int i = 0; i < B_STRIPS; ++i)
            if (BN % T == 0 || tid + i * T < BN) b_reg[i].load(rb, b_voff[i], b_soff, ldb);
    };
    auto store_step = [&](int buf) {
        unsigned char* la = lds + buf * (A_BYTES + B_BYTES);
        unsigned char* lb = la + A_BYTES;
#pragma unroll
        for (int i = 0; i < A_CHUNKS; ++i)
            *reinterpret_cast<u32x4*>(la + lds_off(a_row0 + i * (T / 8), a_chunk)) = a_reg[i];
#pragma unroll
        for (int i = 0; i < B_STRIPS; ++i) {
            if (!(BN % T == 0 || tid + i * T < BN)) continue;
#pragma unroll
            for (int j = 0; j < 8; ++j)
                *reinterpret_cast<u32x4*>(lb + lds_off(b_ng[i] * 8 + j, b_kg[i])) = b_reg[i].column(j);
        }
    };

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int half = lane >> 5;
    const int ra_row = wm * WTM + (lane & 31);
    const int rb_row = wn * WTN + (lane & 31);

    auto compute_step = [&](int buf) {
        const unsigned char* la = lds + buf * (A_BYTES + B_BYTES);
        const unsigned char* lb = la + A_BYTES;
        Frag fa[2][FM], fb[2][FN];
#pragma unroll
        for (int i = 0; i < FM; ++i) fa[0][i] = load_frag<DT>(la, ra_row + 32 * i, 0, half);
#pragma unroll
        for (int j = 0; j < FN; ++j) fb[0][j] = load_frag<DT>(lb, rb_row + 32 * j, 0, half);
#pragma unroll
        for (int s = 0; s < Tr::kSub; ++s) {
            const int cur = s & 1;
            if (s + 1 < Tr::kSub) {
#pragma unroll
                for (int i = 0; i < FM; ++i) fa[cur ^ 1][i] = load_frag<DT>(la, ra_row + 32 * i, s + 1, half);
#pragma unroll
                for (int j = 0; j < FN; ++j) fb[cur ^ 1][j] = load_frag<DT>(lb, rb_row + 32 * j, s + 1, half);
            }
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) acc[i][j] = Tr::mfma(fb[cur][j], fa[cur][i], acc[i][j]);
        }
    };

    const int ksteps = K / Tr::kBK;
    load_step(0);
    store_step(0);
    __syncthreads();
    int kt = 0;
    for (; kt + 2 <= ksteps; kt += 2) {
        if (kt + 1 < ksteps) load_step(kt + 1);
        compute_step(0);
        if (kt + 1 < ksteps) store_step(1);
        __syncthreads();
        if (kt + 2 < ksteps) load_step(kt + 2);
        compute_step(1);
        if (kt + 2 < ksteps) store_step(0);
        __syncthreads();
    }
    if (kt < ksteps) compute_step(0);

    // Epilogue. Accumulator register r = 4g + q of lane l holds
    // C[row = 32*i + l % 32][col = 32*j + 8g + 4*(l / 32) + q].
    const int64_t ldc = (int64_t)N * 2;  // bytes per C row (16-bit output)
    unsigned char* crow = C + ((int64_t)tm * BM + wm * WTM + (lane & 31)) * ldc;
    const int64_t ccol = (int64_t)tn * BN + wn * WTN + 4 * half;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x16& v = acc[i][j];
                const u32x2 packed = pack4<DT>(v[4 * g] * alpha, v[4 * g + 1] * alpha, v[4 * g + 2] * alpha,
                                               v[4 * g + 3] * alpha);
                *reinterpret_cast<u32x2*>(crow + 32 * i * ldc + (ccol + 32 * j + 8 * g) * 2) = packed;
            }
        }
    }
}

struct TiledConfig {
    int bm, bn, wgm, wgn;
};

constexpr TiledConfig kConfigs[] = {
    {256, 256, 2, 2},  // 0: large square-ish problems, 128 x 128 per wave
    {128, 128, 2, 2},  // 1: mid-size problems, 64 x 64 per wave
};

template <int DT, int CFG>
int launch_cfg(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, float alpha,
               int group_m, hipStream_t stream) {
    constexpr TiledConfig c = kConfigs[CFG];
    const int tiles_m = (int)(M / c.bm), tiles_n = (int)(N / c.bn);
    hipLaunchKernelGGL((gemm_tiled_kernel<DT, c.bm, c.bn, c.wgm, c.wgn>), dim3(tiles_m * tiles_n),
                       dim3(64 * c.wgm * c.wgn), 0, stream, static_cast<const unsigned char*>(A),
                       static_cast<const unsigned char*>(B), static_cast<unsigned char*>(C), (int)M,
                       (int)N, (int)K, alpha, tiles_m, tiles_n, group_m);
    MB_HIP_TRY(hipGetLastError());
    return MB_OK;
}

template <int DT>
int launch_dtype(int cfg, const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
                 float alpha, int group_m, hipStream_t stream) {
    if (cfg == 0) return launch_cfg<DT, 0>(A, B, C, M, N, K, alpha, group_m, stream);
    return launch_cfg<DT, 1>(A, B, C, M, N, K, alpha, group_m, stream);
}

}  // namespace

// Picks the tiled configuration for a shape, or returns MB_ERR_SHAPE when the
// shape does not divide into any of them (or its buffers need offsets beyond
// the 32-bit range of buffer addressing).
int gemm_tiled_plan(int dtype, int64_t M, int64_t N, int64_t K, const DeviceProps& props,
                    GemmPlan* plan) {
    const int64_t e = dtype == MB_DT_FLOAT8_E4M3FN ? 1 : 2;
    const int64_t bk = 128 / e;
    if (K % bk != 0) return MB_ERR_SHAPE;
    if (K * N * e >= (int64_t(1) << 31) || 256 * K * e >= (int64_t(1) << 31) || M >= (int64_t(1) << 31))
        return MB_ERR_SHAPE;
    const int64_t cus = props.cu_count > 0 ? props.cu_count : 256;
    auto fits = [&](int i) { return M % kConfigs[i].bm == 0 && N % kConfigs[i].bn == 0; };
    auto tiles = [&](int i) { return (M / kConfigs[i].bm) * (N / kConfigs[i].bn); };
    int cfg = -1;
    const char* force = std::getenv("MB_GEMM_TILED_CONFIG");  // tuning/testing override
    if (force != nullptr && *force != '\0') {
        const int f = std::atoi(force);
        if (f >= 0 && f < (int)(sizeof(kConfigs) / sizeof(kConfigs[0])) && fits(f)) cfg = f;
    }
    if (cfg >= 0)
        ;
    else if (fits(0) && tiles(0) >= cus)
        cfg = 0;
    else if (fits(1))
        cfg = 1;
    else if (fits(0))
        cfg = 0;
    if (cfg < 0 || tiles(cfg) > INT32_MAX) return MB_ERR_SHAPE;
    const TiledConfig& c = kConfigs[cfg];
    plan->implementation = "gfx950_mfma32_lds_tiled";
    plan->threads = 64 * c.wgm * c.wgn;
    plan->grid = (int)tiles(cfg);
    plan->tile_m = c.bm;
    plan->tile_n = c.bn;
    plan->tile_k = (int)bk;
    plan->wave_grid_m = c.wgm;
    plan->wave_grid_n = c.wgn;
    plan->wave_tile_m = c.bm / c.wgm / 32;
    plan->wave_tile_n = c.bn / c.wgn / 32;
    plan->frag_m = 32;
    plan->frag_n = 32;
    plan->frag_k = dtype == MB_DT_FLOAT8_E4M3FN ? 64 : 16;
    plan->k_stages = 2;
    plan->split_k = 1;
    plan->tile_group_m = 4;
    plan->workspace = 0;
    plan->variant = kVariantTiled;
    plan->config = cfg;
    return MB_OK;
}

int gemm_tiled_launch(int dtype, const void* A, const void* B, void* C, int64_t M, int64_t N,
                      int64_t K, float alpha, const GemmPlan& plan, hipStream_t stream) {
    switch (dtype) {
        case MB_DT_BFLOAT16:
            return launch_dtype<MB_DT_BFLOAT16>(plan.config, A, B, C, M, N, K, alpha,
                                                plan.tile_group_m, stream);
        case MB_DT_FLOAT16:
            return launch_dtype<MB_DT_FLOAT16>(plan.config, A, B, C, M, N, K, alpha,
                                               plan.tile_group_m, stream);
        case MB_DT_FLOAT8_E4M3FN:
            return launch_dtype<MB_DT_FLOAT8_E4M3FN>(plan.config, A, B, C, M, N, K, alpha,
                                                     plan.tile_group_m, stream);
        default:
            set_error("tiled GEMM: unsupported dtype %d", dtype);
            return MB_ERR_UNSUPPORTED;
    }
}

}  // namespace mb

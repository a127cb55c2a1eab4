// HBM stream kernels for gfx950: copy (dst = b), scale (dst = s*b) and
// triad (dst = b + s*c) over 1-D contiguous arrays.
//
// Semantics follow the reference torch path (src/teamredbench/benchmarks/hbm.py:29-39):
// copy is a bit copy; scale and triad compute in fp32 (fp64 for float64) and
// round once to the element type; triad is a single fused multiply-add.
//
// Layout and schedule: the array is viewed as 16-byte chunks. Each thread
// walks a grid-stride sequence of chunks, issuing `U` independent 16-byte
// loads per operand before any arithmetic so every wave keeps U (scale/copy)
// or 2U (triad) dwordx4 requests in flight. Consecutive lanes touch
// consecutive chunks, so each wave-wide access is one contiguous 1 KiB run.
// Loads/stores carry the nontemporal hint unless one pass fits the Infinity
// Cache (default_tuning): the arrays at HBM-bound sizes are read and written
// exactly once.
#include "mb_common.hpp"

#include <cstdlib>
#include <cstring>

namespace mb {
namespace {

// ---- element arithmetic on one 16-byte chunk --------------------------------

template <int OP, int DT>
struct ChunkOp;

// Copy: dtype-agnostic bit copy.
template <int DT>
struct ChunkOp<MB_OP_COPY, DT> {
    __device__ static inline u32x4 apply(u32x4 b, u32x4, float, double) { return b; }
};

template <>
struct ChunkOp<MB_OP_SCALE, MB_DT_FLOAT32> {
    __device__ static inline u32x4 apply(u32x4 b, u32x4, float s, double) {
        f32x4 x = __builtin_bit_cast(f32x4, b);
        f32x4 r;
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = x[i] * s;
        return __builtin_bit_cast(u32x4, r);
    }
};

template <>
struct ChunkOp<MB_OP_TRIAD, MB_DT_FLOAT32> {
    __device__ static inline u32x4 apply(u32x4 b, u32x4 c, float s, double) {
        f32x4 x = __builtin_bit_cast(f32x4, b);
        f32x4 y = __builtin_bit_cast(f32x4, c);
        f32x4 r;
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = __builtin_fmaf(s, y[i], x[i]);
        return __builtin_bit_cast(u32x4, r);
    }
};

// bf16 <-> fp32: widening is exact (bits << 16); narrowing uses the
// hardware round-to-nearest-even conversion of the __bf16 type.
__device__ inline float bf16_lo(unsigned w) { return __builtin_bit_cast(float, w << 16); }
__device__ inline float bf16_hi(unsigned w) { return __builtin_bit_cast(float, w & 0xffff0000u); }
__device__ inline unsigned pack_bf16(float lo, float hi) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    bf16x2 p = __builtin_convertvector((f32x2){lo, hi}, bf16x2);
    return __builtin_bit_cast(unsigned, p);
}

template <>
struct ChunkOp<MB_OP_SCALE, MB_DT_BFLOAT16> {
    __device__ static inline u32x4 apply(u32x4 b, u32x4, float s, double) {
        u32x4 r;
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = pack_bf16(bf16_lo(b[i]) * s, bf16_hi(b[i]) * s);
        return r;
    }
};

template <>
struct ChunkOp<MB_OP_TRIAD, MB_DT_BFLOAT16> {
    __device__ static inline u32x4 apply(u32x4 b, u32x4 c, float s, double) {
        u32x4 r;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            r[i] = pack_bf16(__builtin_fmaf(s, bf16_lo(c[i]), bf16_lo(b[i])),
                             __builtin_fmaf(s, bf16_hi(c[i]), bf16_hi(b[i])));
        return r;
    }
};

template <>
struct ChunkOp<MB_OP_SCALE, MB_DT_FLOAT16> {
    __device__ static inline u32x4 apply(u32x4 b, u32x4, float s, double) {
        typedef float f32x8 __attribute__((ext_vector_type(8)));
        f32x8 x = __builtin_convertvector(__builtin_bit_cast(f16x8, b), f32x8);
        f32x8 r;
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] = x[i] * s;
        return __builtin_bit_cast(u32x4, __builtin_convertvector(r, f16x8));
    }
};

template <>
struct ChunkOp<MB_OP_TRIAD, MB_DT_FLOAT16> {
    __device__ static inline u32x4 apply(u32x4 b, u32x4 c, float s, double) {
        typedef float f32x8 __attribute__((ext_vector_type(8)));
        f32x8 x = __builtin_convertvector(__builtin_bit_cast(f16x8, b), f32x8);
        f32x8 y = __builtin_convertvector(__builtin_bit_cast(f16x8, c), f32x8);
        f32x8 r;
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] = __builtin_fmaf(s, y[i], x[i]);
        return __builtin_bit_cast(u32x4, __builtin_convertvector(r, f16x8));
    }
};

template <>
struct ChunkOp<MB_OP_SCALE, MB_DT_FLOAT64> {
    __device__ static inline u32x4 apply(u32x4 b, u32x4, float, double s) {
        typedef double f64x2 __attribute__((ext_vector_type(2)));
        f64x2 x = __builtin_bit_cast(f64x2, b);
        f64x2 r = {x[0] * s, x[1] * s};
        return __builtin_bit_cast(u32x4, r);
    }
};

template <>
struct ChunkOp<MB_OP_TRIAD, MB_DT_FLOAT64> {
    __device__ static inline u32x4 apply(u32x4 b, u32x4 c, float, double s) {
        typedef double f64x2 __attribute__((ext_vector_type(2)));
        f64x2 x = __builtin_bit_cast(f64x2, b);
        f64x2 y = __builtin_bit_cast(f64x2, c);
        f64x2 r = {__builtin_fma(s, y[0], x[0]), __builtin_fma(s, y[1], x[1])};
        return __builtin_bit_cast(u32x4, r);
    }
};

// ---- scalar element arithmetic (tails and unaligned buffers) ----------------

template <int DT>
struct Scalar;

template <>
struct Scalar<MB_DT_FLOAT32> {
    typedef float T;
    __device__ static T scale(T b, float s, double) { return b * s; }
    __device__ static T triad(T b, T c, float s, double) { return __builtin_fmaf(s, c, b); }
};
template <>
struct Scalar<MB_DT_BFLOAT16> {
    typedef unsigned short T;
    __device__ static T rne(float x) { return (T)(pack_bf16(x, 0.0f) & 0xffffu); }
    __device__ static float wide(T v) { return __builtin_bit_cast(float, (unsigned)v << 16); }
    __device__ static T scale(T b, float s, double) { return rne(wide(b) * s); }
    __device__ static T triad(T b, T c, float s, double) {
        return rne(__builtin_fmaf(s, wide(c), wide(b)));
    }
};
template <>
struct Scalar<MB_DT_FLOAT16> {
    typedef _Float16 T;
    __device__ static T scale(T b, float s, double) { return (T)((float)b * s); }
    __device__ static T triad(T b, T c, float s, double) {
        return (T)__builtin_fmaf(s, (float)c, (float)b);
    }
};
template <>
struct Scalar<MB_DT_FLOAT64> {
    typedef double T;
    __device__ static T scale(T b, float, double s) { return b * s; }
    __device__ static T triad(T b, T c, float, double s) { return __builtin_fma(s, c, b); }
};
template <>
struct Scalar<MB_DT_INT8> {
    typedef signed char T;
    __device__ static T scale(T b, float, double) { return b; }
    __device__ static T triad(T b, T, float, double) { return b; }
};

template <int BYTES>
struct BitsOf;
template <> struct BitsOf<1> { typedef uint8_t T; };
template <> struct BitsOf<2> { typedef uint16_t T; };
template <> struct BitsOf<4> { typedef uint32_t T; };
template <> struct BitsOf<8> { typedef uint64_t T; };

template <int OP, int DT>
__device__ inline void scalar_element(void* dst, const void* b, const void* c, uint64_t i,
                                      float s, double sd) {
    typedef typename Scalar<DT>::T T;
    const T* B = static_cast<const T*>(b);
    T* D = static_cast<T*>(dst);
    if (OP == MB_OP_COPY) {
        // Integer move: bit-exact for every payload, NaNs included.
        typedef typename BitsOf<sizeof(T)>::T U;
        static_cast<U*>(dst)[i] = static_cast<const U*>(b)[i];
    } else if (OP == MB_OP_SCALE) {
        D[i] = Scalar<DT>::scale(B[i], s, sd);
    } else {
        D[i] = Scalar<DT>::triad(B[i], static_cast<const T*>(c)[i], s, sd);
    }
}

// ---- kernels ---------------------------------------------------------------

template <bool NT>
__device__ inline u32x4 load_chunk(const u32x4* p) {
    if (NT) return __builtin_nontemporal_load(p);
    return *p;
}

template <bool NT>
__device__ inline void store_chunk(u32x4* p, u32x4 v) {
    if (NT) {
        __builtin_nontemporal_store(v, p);
    } else {
        *p = v;
    }
}

// Vector body over `chunks` 16-byte chunks, then the `tail` trailing elements
// (fewer than one chunk) handled by the first threads of the grid.
// span == 0: grid-stride -- consecutive trips of a thread are one grid apart.
// span  > 0: each block walks its own contiguous run of `span` chunks, the
//            block's lanes side by side, trips one block-width apart.
template <int OP, int DT, int U, bool NT>
__global__ void __launch_bounds__(1024)
stream_vec_kernel(void* __restrict__ dst, const void* __restrict__ b, const void* __restrict__ c,
                  uint64_t chunks, uint64_t tail, uint64_t span, float s, double sd) {
    const u32x4* B = static_cast<const u32x4*>(b);
    const u32x4* C = static_cast<const u32x4*>(c);
    u32x4* D = static_cast<u32x4*>(dst);
    const uint64_t tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint64_t stride, end, i;
    if (span == 0) {
        stride = (uint64_t)gridDim.x * blockDim.x;
        end = chunks;
        i = tid;
    } else {
        stride = blockDim.x;
        const uint64_t first = (uint64_t)blockIdx.x * span;
        end = first + span < chunks ? first + span : chunks;
        i = first + threadIdx.x;
    }
    // Full trips: all U chunks of this thread are in range.
    for (; i + (U - 1) * stride < end; i += U * stride) {
        u32x4 vb[U];
        u32x4 vc[U];
#pragma unroll
        for (int u = 0; u < U; ++u) vb[u] = load_chunk<NT>(B + i + u * stride);
        if (OP == MB_OP_TRIAD) {
#pragma unroll
            for (int u = 0; u < U; ++u) vc[u] = load_chunk<NT>(C + i + u * stride);
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
            store_chunk<NT>(D + i + u * stride, ChunkOp<OP, DT>::apply(vb[u], vc[u], s, sd));
    }
    // Remainder trip: fewer than U chunks left for this thread.
    for (; i < end; i += stride) {
        u32x4 vb = load_chunk<NT>(B + i);
        u32x4 vc = vb;
        if (OP == MB_OP_TRIAD) vc = load_chunk<NT>(C + i);
        store_chunk<NT>(D + i, ChunkOp<OP, DT>::apply(vb, vc, s, sd));
    }
    if (tid < tail) {
        const int esize = (DT == MB_DT_FLOAT32) ? 4 : (DT == MB_DT_FLOAT64) ? 8 : (DT == MB_DT_INT8) ? 1 : 2;
        const uint64_t first = chunks * (16 / esize);
        scalar_element<OP, DT>(dst, b, c, first + tid, s, sd);
    }
}

// Element-wise grid-stride kernel for buffers that are not 16-byte aligned.
template <int OP, int DT>
__global__ void __launch_bounds__(1024)
stream_scalar_kernel(void* __restrict__ dst, const void* __restrict__ b, const void* __restrict__ c,
                     uint64_t n, float s, double sd) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        scalar_element<OP, DT>(dst, b, c, i, s, sd);
}

// ---- dispatch --------------------------------------------------------------

typedef void (*VecKernel)(void*, const void*, const void*, uint64_t, uint64_t, uint64_t, float, double);
typedef void (*ScalarKernel)(void*, const void*, const void*, uint64_t, float, double);

template <int OP, int DT>
VecKernel pick_vec(int u, bool nt) {
    switch (u) {
        case 1: return nt ? stream_vec_kernel<OP, DT, 1, true> : stream_vec_kernel<OP, DT, 1, false>;
        case 2: return nt ? stream_vec_kernel<OP, DT, 2, true> : stream_vec_kernel<OP, DT, 2, false>;
        case 8: return nt ? stream_vec_kernel<OP, DT, 8, true> : stream_vec_kernel<OP, DT, 8, false>;
        default: return nt ? stream_vec_kernel<OP, DT, 4, true> : stream_vec_kernel<OP, DT, 4, false>;
    }
}

// Copy kernels differ only in how the scalar tail is typed.
VecKernel vec_kernel_for(int op, int dtype, int u, bool nt) {
    if (op == MB_OP_COPY) {
        switch (dtype) {
            case MB_DT_FLOAT32: return pick_vec<MB_OP_COPY, MB_DT_FLOAT32>(u, nt);
            case MB_DT_BFLOAT16: return pick_vec<MB_OP_COPY, MB_DT_BFLOAT16>(u, nt);
            case MB_DT_FLOAT16: return pick_vec<MB_OP_COPY, MB_DT_FLOAT16>(u, nt);
            case MB_DT_FLOAT64: return pick_vec<MB_OP_COPY, MB_DT_FLOAT64>(u, nt);
            case MB_DT_INT8: return pick_vec<MB_OP_COPY, MB_DT_INT8>(u, nt);
        }
        return nullptr;
    }
    if (op == MB_OP_SCALE) {
        switch (dtype) {
            case MB_DT_FLOAT32: return pick_vec<MB_OP_SCALE, MB_DT_FLOAT32>(u, nt);
            case MB_DT_BFLOAT16: return pick_vec<MB_OP_SCALE, MB_DT_BFLOAT16>(u, nt);
            case MB_DT_FLOAT16: return pick_vec<MB_OP_SCALE, MB_DT_FLOAT16>(u, nt);
            case MB_DT_FLOAT64: return pick_vec<MB_OP_SCALE, MB_DT_FLOAT64>(u, nt);
        }
        return nullptr;
    }
    if (op == MB_OP_TRIAD) {
        switch (dtype) {
            case MB_DT_FLOAT32: return pick_vec<MB_OP_TRIAD, MB_DT_FLOAT32>(u, nt);
            case MB_DT_BFLOAT16: return pick_vec<MB_OP_TRIAD, MB_DT_BFLOAT16>(u, nt);
            case MB_DT_FLOAT16: return pick_vec<MB_OP_TRIAD, MB_DT_FLOAT16>(u, nt);
            case MB_DT_FLOAT64: return pick_vec<MB_OP_TRIAD, MB_DT_FLOAT64>(u, nt);
        }
    }
    return nullptr;
}

template <int OP>
ScalarKernel scalar_for_dtype(int dtype) {
    switch (dtype) {
        case MB_DT_FLOAT32: return stream_scalar_kernel<OP, MB_DT_FLOAT32>;
        case MB_DT_BFLOAT16: return stream_scalar_kernel<OP, MB_DT_BFLOAT16>;
        case MB_DT_FLOAT16: return stream_scalar_kernel<OP, MB_DT_FLOAT16>;
        case MB_DT_FLOAT64: return stream_scalar_kernel<OP, MB_DT_FLOAT64>;
        case MB_DT_INT8: return OP == MB_OP_COPY ? stream_scalar_kernel<OP, MB_DT_INT8> : nullptr;
    }
    return nullptr;
}

ScalarKernel scalar_kernel_for(int op, int dtype) {
    if (op == MB_OP_COPY) return scalar_for_dtype<MB_OP_COPY>(dtype);
    if (op == MB_OP_SCALE) return scalar_for_dtype<MB_OP_SCALE>(dtype);
    if (op == MB_OP_TRIAD) return scalar_for_dtype<MB_OP_TRIAD>(dtype);
    return nullptr;
}

// Tuned defaults per (op, dtype): blocks per CU, threads per block, 16-byte
// chunks per thread per trip, nontemporal hint and schedule (0 grid-stride,
// 1 contiguous span per block). The MB_TUNE_STREAM_* knobs (mb_set_tuning)
// override the last four for sweeps; their values are validated when set.
struct StreamTuning {
    int blocks_per_cu;
    int threads;
    int unroll;
    bool nontemporal;
    int schedule;
};

// Measured on MI355X at 2^28 fp32 elements: one 256-thread block per CU with
// nontemporal accesses beats deeper occupancy (more requests in flight spread
// over more DRAM pages); triad (two read streams) prefers 2 chunks per trip,
// copy and scale (one read stream) 4.
//
// The nontemporal hint keeps the arrays out of the 256 MB Infinity Cache.
// When one pass touches 64..256 MiB (reads plus writes; 80..256 MiB for the
// triad's two read streams), the arrays fit in it, and a caller that makes
// repeated passes over the same arrays (a timed loop, an iterative solver)
// finds them there with ordinary accesses. On MI355X, medians of 5-9
// interleaved runs of 50 launches: without the hint fp32 / bf16 copy ran 2%
// faster at 64 MiB and 5-9% at 96..256 MiB, scale 6-11% from 64 MiB, triad
// 1-3% at 80 MiB and 3-12% at 96..224 MiB (fp32 at 192 MiB 6920 against 6467
// GB/s); below those sizes the hint was equal or better (triad by 3-5% at
// 48..64 MiB), and above 256 MiB it won by 8-10% (fp32 triad at 384 MiB 6512
// against 5875).
constexpr uint64_t kCacheFitHi = uint64_t(256) << 20;

StreamTuning default_tuning(int op, int dtype, uint64_t n) {
    const uint64_t lo = (op == MB_OP_TRIAD ? uint64_t(80) : uint64_t(64)) << 20;
    const uint64_t touched = n <= kCacheFitHi ? (op == MB_OP_TRIAD ? 3u : 2u) * n * (uint64_t)dtype_size(dtype) : 0;
    const bool nt = !(touched >= lo && touched <= kCacheFitHi);
    if (op == MB_OP_TRIAD) return {1, 256, 2, nt, 0};
    return {1, 256, 4, nt, 0};
}

int knob_or(int knob, int fallback) {
    const int64_t v = tuning(knob);
    return v < 0 ? fallback : (int)v;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

int stream_plan(int op, int dtype, const void* dst, const void* b, const void* c, uint64_t n,
                int blocks_per_cu, const DeviceProps& props, StreamPlan* plan) {
    if (op < MB_OP_COPY || op > MB_OP_TRIAD) {
        set_error("unknown stream op %d", op);
        return MB_ERR_INVALID_ARG;
    }
    const int esize = dtype_size(dtype);
    if (esize == 0 || dtype == MB_DT_FLOAT8_E4M3FN || dtype == MB_DT_FLOAT8_E5M2) {
        set_error("unsupported dtype %d for stream op", dtype);
        return MB_ERR_UNSUPPORTED;
    }
    if (dtype == MB_DT_INT8 && op != MB_OP_COPY) {
        set_error("int8 supports only copy (got op %d)", op);
        return MB_ERR_UNSUPPORTED;
    }
    StreamTuning t = default_tuning(op, dtype, n);
    const int u = knob_or(MB_TUNE_STREAM_UNROLL, t.unroll);
    const bool nt = knob_or(MB_TUNE_STREAM_NONTEMPORAL, t.nontemporal ? 1 : 0) != 0;
    const int threads = knob_or(MB_TUNE_STREAM_THREADS, t.threads);
    const int sched = knob_or(MB_TUNE_STREAM_SCHEDULE, t.schedule);
    const int bpc = blocks_per_cu > 0 ? blocks_per_cu : t.blocks_per_cu;

    plan->threads = threads;
    plan->blocks_per_cu = bpc;
    plan->chunks_per_trip = u;
    plan->nontemporal = nt;
    const bool vec = aligned16(dst) && aligned16(b) && (op != MB_OP_TRIAD || aligned16(c));
    plan->vector_path = vec;
    const uint64_t per_chunk = 16 / (uint64_t)esize;
    uint64_t work_items;
    if (vec) {
        plan->chunks = n / per_chunk;
        plan->tail = n - plan->chunks * per_chunk;
        work_items = (plan->chunks + (uint64_t)u - 1) / (uint64_t)u;
        if (work_items < plan->tail) work_items = plan->tail;
    } else {
        plan->chunks = 0;
        plan->tail = n;
        work_items = n;
    }
    uint64_t max_blocks = (uint64_t)props.cu_count * (uint64_t)bpc;
    uint64_t by_work = (work_items + (uint64_t)threads - 1) / (uint64_t)threads;
    uint64_t blocks = by_work < max_blocks ? by_work : max_blocks;
    if (blocks < 1) blocks = 1;
    plan->blocks = (int)blocks;
    plan->span = 0;
    if (vec && sched == 1 && plan->chunks > 0) {
        // Contiguous runs, a whole number of block-wide trips each.
        const uint64_t trip = (uint64_t)threads * (uint64_t)u;
        uint64_t span = (plan->chunks + blocks - 1) / blocks;
        span = (span + trip - 1) / trip * trip;
        plan->span = span;
        plan->blocks = (int)((plan->chunks + span - 1) / span);
        if ((uint64_t)plan->blocks * threads < plan->tail) plan->blocks = (int)((plan->tail + threads - 1) / threads);
    }
    return MB_OK;
}

int stream_launch(int op, int dtype, void* dst, const void* b, const void* c, uint64_t n,
                  double s, const StreamPlan& plan, hipStream_t stream) {
    if (n == 0) return MB_OK;
    const float sf = (float)s;
    if (plan.vector_path) {
        VecKernel k = vec_kernel_for(op, dtype, plan.chunks_per_trip, plan.nontemporal);
        if (k == nullptr) {
            set_error("no vector stream kernel for op %d dtype %d", op, dtype);
            return MB_ERR_UNSUPPORTED;
        }
        hipLaunchKernelGGL(k, dim3(plan.blocks), dim3(plan.threads), 0, stream, dst, b, c,
                           plan.chunks, plan.tail, plan.span, sf, s);
    } else {
        ScalarKernel k = scalar_kernel_for(op, dtype);
        if (k == nullptr) {
            set_error("no scalar stream kernel for op %d dtype %d", op, dtype);
            return MB_ERR_UNSUPPORTED;
        }
        hipLaunchKernelGGL(k, dim3(plan.blocks), dim3(plan.threads), 0, stream, dst, b, c, n, sf, s);
    }
    MB_HIP_TRY(hipGetLastError());
    return MB_OK;
}

}  // namespace mb

/*
 * mi355bench.h -- C ABI of libmi355bench.so, the gfx950 (MI355X) stream and
 * GEMM kernels behind TeamRedBench's `backend: native` path.
 *
 * The reference crosses into native code through a subprocess: Python builds
 * argv, runs a hipcc-built executable per case and parses one JSON line from
 * its stdout (src/teamredbench/native/runtime.py:276-291,
 * src/teamredbench/benchmarks/hbm.py:95-116, src/teamredbench/benchmarks/mfu.py:106-125).
 * This library replaces that process boundary with in-process calls. Every
 * entry point below names the reference code it replaces.
 *
 * Conventions (all entry points):
 *   - Plain pointers and sizes only. Device buffers are owned by the caller;
 *     the library never allocates or frees device memory except the hipEvents
 *     used by the mb_time_* entry points and the fixed per-GPU scratch array
 *     that mb_gemm_noalloc uses (a static device variable of the library).
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *     Work is enqueued asynchronously; nothing synchronises except mb_time_*.
 *   - Return 0 on success, a negative MB_ERR_* for a rejected argument, or a
 *     positive hipError_t from the HIP runtime. On any non-zero return,
 *     mb_last_error() describes the failure (thread-local string).
 *   - Thread-safe and reentrant; per-device properties are cached once.
 */
#ifndef MI355BENCH_H
#define MI355BENCH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MB_ABI_VERSION 3

/* Status codes (negative = rejected by the library before any launch). */
#define MB_OK 0
#define MB_ERR_INVALID_ARG -1  /* null pointer, negative size, bad enum */
#define MB_ERR_UNSUPPORTED -2  /* dtype/op combination not implemented */
#define MB_ERR_SHAPE -3        /* shape the kernel family cannot take */
#define MB_ERR_WORKSPACE -4    /* workspace missing or too small */
#define MB_ERR_DEVICE -5       /* current device is not gfx950 */

/* Stream operations; semantics of src/teamredbench/benchmarks/hbm.py:29-39. */
#define MB_OP_COPY 0  /* dst = b                 (torch: dst.copy_(src))          */
#define MB_OP_SCALE 1 /* dst = s * b             (torch: torch.mul(src, s, out=dst)) */
#define MB_OP_TRIAD 2 /* dst = b + s * c         (torch: torch.add(src, aux, alpha=s, out=dst)) */

/* Element types (names follow src/teamredbench/dtypes.py:16-31). */
#define MB_DT_FLOAT32 0
#define MB_DT_BFLOAT16 1
#define MB_DT_FLOAT16 2
#define MB_DT_FLOAT64 3
#define MB_DT_INT8 4           /* copy only */
#define MB_DT_FLOAT8_E4M3FN 5  /* GEMM inputs only; output is bfloat16 */
#define MB_DT_FLOAT8_E5M2 6    /* GEMM inputs only; output is bfloat16 */

/* Kinds for mb_kernel_info. */
#define MB_KIND_STREAM 0
#define MB_KIND_GEMM 1

/*
 * mb_stream -- one launch of a stream kernel over n elements.
 *
 * Replaces the per-iteration launch in the reference executable's
 * run_kernel<T>::launch_once (native/kernels/hbm_bandwidth.hip.cpp:371-388):
 * hipMemcpyAsync for copy, scale_kernel<T> / triad_kernel<T> otherwise.
 *
 * dst, b: n elements of `dtype`; c: n elements for TRIAD, ignored (may be NULL)
 * otherwise. Any n (0 is a no-op) and any element alignment: 16-byte aligned
 * buffers take the vector kernel plus a scalar tail, others a scalar kernel.
 * Arithmetic: fp32 math with one round-to-nearest-even to the element type
 * (fp64 math for float64); TRIAD is one fused multiply-add, fma(s, c, b).
 * blocks_per_cu: grid = min(CUs * blocks_per_cu, work); <= 0 selects the
 * tuned default (the reference's --blocks-per-cu override, hbm.py:111-114).
 */
int mb_stream(int op, int dtype, void* dst, const void* b, const void* c,
              uint64_t n, double s, int blocks_per_cu, void* stream);

/*
 * mb_time_stream -- warmup + event-timed loop of mb_stream launches.
 *
 * Replaces the timing body of run_kernel<T> (hbm_bandwidth.hip.cpp:390-425):
 * `warmup` launches, a stream synchronise, then `iterations` launches between
 * two hipEvents recorded on `stream`; *elapsed_s = event time / iterations.
 * Synchronises `stream` before returning.
 */
int mb_time_stream(int op, int dtype, void* dst, const void* b, const void* c,
                   uint64_t n, double s, int blocks_per_cu, int warmup,
                   int iterations, void* stream, double* elapsed_s);

/*
 * mb_gemm -- C = A * B, row-major, fp32 accumulation.
 *
 * Replaces the launch of mfma_gemm_lowp_kernel<T>
 * (native/kernels/mfu_gemm_lowp.hip.hpp:423-445) and its untimed
 * pack_b_tiles_kernel<T> pre-pass (:396-409): B is consumed as given,
 * row-major K x N, with no re-layout outside the timed kernel.
 *
 * dtype        A (M x K)   B (K x N)   C (M x N)   accumulate / epilogue
 * BFLOAT16     bf16        bf16        bf16        fp32 / RNE(acc)
 * FLOAT16      fp16        fp16        fp16        fp32 / RNE(acc)
 * FLOAT8_E4M3FN e4m3fn     e4m3fn      bf16        fp32 / RNE(scale_a * scale_b * acc)
 * FLOAT8_E5M2  e5m2        e5m2        bf16        fp32 / RNE(scale_a * scale_b * acc)
 * FLOAT32      fp32        fp32        fp32        fp32 MFMA (full precision)
 * FLOAT64      fp64        fp64        fp64        fp64 MFMA
 * scale_a/scale_b are the fp8 per-tensor dequantisation scales (ignored for
 * the other types). Leading dimensions are K, N and N. Any M, N, K >= 1 with
 * 16-byte aligned base pointers; shapes the pipelined kernels do not divide
 * (N % 128, K % 64 bytes) run on bounds-checked kernels.
 * FLOAT32 / FLOAT64 follow the reference's high-precision path
 * (mfu_gemm_highp.hip.hpp:39-218) on v_mfma_f32_32x32x2_f32 and
 * v_mfma_f64_16x16x4_f64; FLOAT8_E5M2 is the dtype the reference declares
 * (dtypes.py:24) but does not run natively (mfu_gemm.hip.cpp:9-21).
 * workspace: device scratch of at least mb_gemm_workspace_size() bytes (may
 * be NULL when that size is 0). The kernels leave it in a state the next
 * call can use without clearing.
 */
int mb_gemm(int dtype, const void* A, const void* B, void* C, int64_t M,
            int64_t N, int64_t K, float scale_a, float scale_b, void* workspace,
            size_t workspace_bytes, void* stream);

/* Workspace bytes mb_gemm needs for this dtype and shape (0 if none). */
size_t mb_gemm_workspace_size(int dtype, int64_t M, int64_t N, int64_t K);

/*
 * mb_gemm_noalloc -- mb_gemm without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc). It has no counterpart in the reference.
 *
 * Same arguments, kernels and results as mb_gemm. The split-K / small-M
 * partial sums go to a library-owned device array of
 * MB_NOALLOC_SCRATCH_BYTES per GPU, which each GPU holds until the process
 * ends; the call itself allocates nothing. Shapes whose plan needs more
 * scratch than that return MB_ERR_WORKSPACE before any launch. The first
 * call on a device resolves that device's array address (not an
 * allocation); make it before a capture if the capture must not see it.
 * Every call on one GPU shares that GPU's array, and every call writes all
 * the partials it reads, so nothing carries over between calls; calls that
 * overlap on one GPU (concurrent streams or threads) race on the array.
 */
#define MB_NOALLOC_SCRATCH_BYTES (64u << 20)
int mb_gemm_noalloc(int dtype, const void* A, const void* B, void* C,
                    int64_t M, int64_t N, int64_t K, float scale_a,
                    float scale_b, void* stream);

/*
 * mb_time_gemm -- warmup + event-timed loop of mb_gemm launches.
 *
 * Replaces the timing body of run_low_precision_kernel<T>
 * (mfu_gemm_lowp.hip.hpp:447-485); same contract as mb_time_stream.
 */
int mb_time_gemm(int dtype, const void* A, const void* B, void* C, int64_t M,
                 int64_t N, int64_t K, float scale_a, float scale_b,
                 void* workspace, size_t workspace_bytes, int warmup,
                 int iterations, void* stream, double* elapsed_s);

/*
 * mb_time_gemm_rotating -- mb_time_gemm over `sets` operand sets: launch i
 * (warmup launches included) multiplies A[i % sets] by B[i % sets] into
 * C[i % sets], all of one shape, sharing `workspace` (the launches run in
 * order on `stream`). With sets whose operands together exceed the 256 MB
 * Infinity Cache, every launch reads its operands from HBM, so the time is
 * that of the HBM-bound case rather than of operands left in the cache by
 * the previous launch. No counterpart in the reference, whose executable
 * times one operand set (mfu_gemm_lowp.hip.hpp:447-485).
 */
int mb_time_gemm_rotating(int dtype, const void* const* A,
                          const void* const* B, void* const* C, int sets,
                          int64_t M, int64_t N, int64_t K, float scale_a,
                          float scale_b, void* workspace,
                          size_t workspace_bytes, int warmup, int iterations,
                          void* stream, double* elapsed_s);

/*
 * mb_kernel_info -- JSON object describing the kernel configuration the
 * library picks for a case, written NUL-terminated into json[0..cap).
 *
 * Replaces the "metadata" object the reference executables print
 * (hbm_bandwidth.hip.cpp:431-436; mfu_gemm_lowp.hip.hpp:492-509), keeping
 * its keys (implementation, threads_per_block, blocks_per_cu, tile_m/n/k,
 * wave_grid_*, wave_tile_*, frag_*, k_stages ...).
 * kind = MB_KIND_STREAM: a = op, b = dtype, m = n elements, n = blocks_per_cu.
 * kind = MB_KIND_GEMM:   a = dtype, m, n, k = shape (b ignored).
 * Beyond the reference's keys: "overrides" (the MB_TUNE_* knobs in force,
 * by name; {} normally) and, for GEMM, "workspace_bytes", "split_k" and
 * "fallback" (why a faster kernel family could not take the shape and a
 * bounds-checked kernel runs it instead; "" when none).
 * Returns MB_ERR_INVALID_ARG if json is NULL or cap is too small.
 */
int mb_kernel_info(int kind, int a, int b, int64_t m, int64_t n, int64_t k,
                   char* json, size_t cap);

/*
 * Plan overrides. No counterpart in the reference, whose executables fix
 * their tuning at compile time (hbm_bandwidth.hip.cpp:18-70,
 * mfu_gemm_lowp.hip.hpp:7-37) apart from --blocks-per-cu (kept above as an
 * argument of mb_stream). These knobs exist for tests and tuning sweeps that
 * must run a specific kernel configuration. Each knob is process-wide and
 * holds either -1 (the library's own choice, the default) or a forced value;
 * nothing is read from the environment. mb_kernel_info reports every knob in
 * force under "overrides", so a record shows when a non-default plan ran.
 * Set knobs before the calls they should affect: a plan is made per call, so
 * mb_gemm_workspace_size and mb_gemm must see the same settings.
 */
#define MB_TUNE_STREAM_UNROLL 0        /* 16-byte chunks per thread per trip: 1, 2, 4 or 8 */
#define MB_TUNE_STREAM_NONTEMPORAL 1   /* 0 or 1: nontemporal loads and stores */
#define MB_TUNE_STREAM_THREADS 2       /* threads per block: 64..1024, a multiple of 64 */
#define MB_TUNE_STREAM_SCHEDULE 3      /* 0 grid-stride, 1 one contiguous span per block */
#define MB_TUNE_GEMM_FORCE_GENERIC 4   /* 1: the bounds-checked generic kernel for 16-bit and fp8 */
#define MB_TUNE_GEMM_NO_SMALL_M 5      /* 1: M <= 4 stays on the MFMA kernels */
#define MB_TUNE_GEMM_TILED_CONFIG 6    /* 0: 256x256, 1: 128x256, 2: 128x128, 3: 64x128, 4: 64x64 tiles */
#define MB_TUNE_GEMM_SPLITS 7          /* K splits, 1..512 (taken when each split is whole stages; a K off
                                          the stage depth rounds every split up to whole stages) */
#define MB_TUNE_GEMM_FP8_MFMA 8        /* 16 or 32: the fp8 MFMA shape on the tiled kernel */
#define MB_TUNE_GEMM_HIGHP_STAGED 9    /* 1: fp32 / fp64 on the register-staged kernel */
#define MB_TUNE_COUNT 10

/* Force `knob` to `value`, or restore the library's choice with value -1.
 * Returns MB_ERR_INVALID_ARG for an unknown knob or a value outside the
 * range listed above. */
int mb_set_tuning(int knob, int64_t value);

/* The value `knob` holds (-1 = the library's choice); -1 for an unknown knob. */
int64_t mb_get_tuning(int knob);

/*
 * Clock stamps. No counterpart in the reference: a measurement aid that
 * tells at which clock a timed region ran (the part runs MFMA-heavy kernels
 * under its power limit, well below the clock its peak figures assume).
 * Enqueues on `stream` one kernel of MB_CLOCK_BLOCKS one-wave blocks, enough
 * for the dispatcher to place blocks on every CU; block b writes
 *   out[4b]     its CU's shader-clock counter (s_memtime),
 *   out[4b + 1] the constant MB_CLOCK_REALTIME_HZ counter (s_memrealtime),
 *   out[4b + 2] the id of the XCD it ran on (XCC_ID),
 *   out[4b + 3] its wave's HW_ID register (bits 15:8: CU, shader array and
 *               shader engine within the XCD).
 * `out` is device memory for 4 * MB_CLOCK_BLOCKS uint64_t. The shader-clock
 * counters of different CUs are not synchronised, so two stamps on the
 * stream around a region are paired CU by CU: each CU seen in both gives its
 * XCD's mean shader clock over the region,
 * (memtime_1 - memtime_0) / (memrealtime_1 - memrealtime_0) * MB_CLOCK_REALTIME_HZ.
 */
#define MB_CLOCK_BLOCKS 1024
#define MB_CLOCK_REALTIME_HZ 100000000
int mb_clock_stamp(uint64_t* out, void* stream);

/*
 * MFMA ceiling. No counterpart in the reference: a measurement aid that
 * gives the rate one MFMA instruction sustains on this part with no memory
 * traffic, under the same power limit a GEMM runs under. `blocks` blocks of
 * 256 threads (one per CU fills the part, one wave per SIMD) each run
 * `iterations` rounds of 8 independent MFMAs per wave, alternating between
 * two operand sets read from `operands` (MB_MFMA_CEILING_OPERAND_BYTES of
 * device memory holding values of the instruction's input type; 128 bytes
 * per lane), and write one float per thread to `out` (device memory for
 * 256 * blocks floats). `warmup` untimed launches, then `launches` timed on
 * `stream` between two events; *elapsed_s = seconds per launch. One launch
 * does blocks * 4 * iterations * 8 MFMAs (iterations rounded up to even).
 */
#define MB_MFMA_BF16_32X32X16 0   /* v_mfma_f32_32x32x16_bf16:          32768 FLOP per wave instruction */
#define MB_MFMA_BF16_16X16X32 1   /* v_mfma_f32_16x16x32_bf16:          16384 */
#define MB_MFMA_FP8_32X32X64 2    /* v_mfma_scale_f32_32x32x64_f8f6f4:  131072 */
#define MB_MFMA_FP8_16X16X128 3   /* v_mfma_scale_f32_16x16x128_f8f6f4: 65536 */
#define MB_MFMA_F32_32X32X2 4     /* v_mfma_f32_32x32x2_f32:            4096 */
#define MB_MFMA_CEILING_OPERAND_BYTES 8192
int mb_mfma_ceiling(int instruction, const void* operands, float* out, int blocks, int iterations, int warmup,
                    int launches, void* stream, double* elapsed_s);

/* Description of the last failure on the calling thread ("" if none). */
const char* mb_last_error(void);

/* MB_ABI_VERSION of the loaded library. */
int mb_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MI355BENCH_H */

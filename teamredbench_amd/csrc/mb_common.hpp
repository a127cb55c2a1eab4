// Internal helpers shared by the libmi355bench translation units: status and
// error-string plumbing for the C ABI, a per-device property cache, and the
// small vector types the gfx950 kernels use.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/mi355bench.h"

namespace mb {

// ---- error plumbing -------------------------------------------------------

void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

// Records `what` plus the HIP error string; returns the positive hipError_t.
int hip_fail(hipError_t err, const char* what);

#define MB_HIP_TRY(expr)                                 \
    do {                                                 \
        hipError_t mb_err_ = (expr);                     \
        if (mb_err_ != hipSuccess) {                     \
            return ::mb::hip_fail(mb_err_, #expr);       \
        }                                                \
    } while (0)

// ---- plan overrides (mb_set_tuning) -----------------------------------------

// The value a MB_TUNE_* knob holds: -1 for the library's own choice.
int64_t tuning(int knob);

// ---- device properties ----------------------------------------------------

struct DeviceProps {
    int device = -1;
    int cu_count = 0;        // multiProcessorCount (256 on MI355X)
    int max_threads_per_cu = 0;
    bool is_gfx950 = false;
    char arch[64] = {0};
};

// Properties of the current HIP device, cached per device id. Returns 0 or a
// status code (and sets the error string).
int current_device_props(const DeviceProps** out);

// ---- vector types ---------------------------------------------------------

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef double f64x2 __attribute__((ext_vector_type(2)));
typedef double f64x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

inline int dtype_size(int dtype) {
    switch (dtype) {
        case MB_DT_FLOAT32: return 4;
        case MB_DT_BFLOAT16: return 2;
        case MB_DT_FLOAT16: return 2;
        case MB_DT_FLOAT64: return 8;
        case MB_DT_INT8: return 1;
        case MB_DT_FLOAT8_E4M3FN: return 1;
        case MB_DT_FLOAT8_E5M2: return 1;
        default: return 0;
    }
}

inline const char* dtype_name(int dtype) {
    switch (dtype) {
        case MB_DT_FLOAT32: return "float32";
        case MB_DT_BFLOAT16: return "bfloat16";
        case MB_DT_FLOAT16: return "float16";
        case MB_DT_FLOAT64: return "float64";
        case MB_DT_INT8: return "int8";
        case MB_DT_FLOAT8_E4M3FN: return "float8_e4m3fn";
        case MB_DT_FLOAT8_E5M2: return "float8_e5m2";
        default: return "unknown";
    }
}

// ---- internal launch interfaces (one per translation unit) -----------------

struct StreamPlan {
    bool vector_path = false;   // 16-byte chunk kernel (else scalar kernel)
    int threads = 0;
    int blocks = 0;
    int blocks_per_cu = 0;
    int chunks_per_trip = 0;    // 16-byte chunks per thread per loop trip
    bool nontemporal = false;
    uint64_t chunks = 0;        // 16-byte chunks in the vector body
    uint64_t tail = 0;          // elements after the vector body
    uint64_t span = 0;          // chunks per block (0 = grid-stride schedule)
};

int stream_plan(int op, int dtype, const void* dst, const void* b, const void* c,
                uint64_t n, int blocks_per_cu, const DeviceProps& props, StreamPlan* plan);
int stream_launch(int op, int dtype, void* dst, const void* b, const void* c, uint64_t n,
                  double s, const StreamPlan& plan, hipStream_t stream);

struct GemmPlan {
    const char* implementation = "";
    int threads = 0;
    int grid = 0;
    int tile_m = 0, tile_n = 0, tile_k = 0;
    int wave_grid_m = 0, wave_grid_n = 0;
    int wave_tile_m = 0, wave_tile_n = 0;
    int frag_m = 0, frag_n = 0, frag_k = 0;
    int k_stages = 0;
    int split_k = 1;
    int tile_group_m = 0;
    size_t workspace = 0;
    const char* fallback = "";  // why a faster kernel family could not take the shape ("" if none)
    int variant = 0;            // kernel family selector, private to gemm*.hip
    int config = 0;             // configuration within the family
};

int gemm_plan(int dtype, int64_t M, int64_t N, int64_t K, const DeviceProps& props,
              GemmPlan* plan);

// One launch of the MFMA-only kernel of instruction `kind` (MB_MFMA_*).
int mfma_ceiling_launch(int kind, const void* operands, float* out, int blocks, int iterations, hipStream_t stream);
int gemm_launch(int dtype, const void* A, const void* B, void* C, int64_t M, int64_t N,
                int64_t K, float scale_a, float scale_b, void* workspace,
                const GemmPlan& plan, hipStream_t stream);

}  // namespace mb

// C ABI of libmi355bench.so (declared in include/mi355bench.h): argument
// validation, per-device property cache, dispatch into the stream and GEMM
// kernel families, event-timed loops and kernel metadata.
#include "mb_common.hpp"

#include <atomic>
#include <cstring>
#include <mutex>
#include <string>

namespace mb {

namespace {
thread_local std::string g_last_error;

constexpr int kMaxDevices = 64;
std::mutex g_props_mutex;
DeviceProps g_props[kMaxDevices];
bool g_props_valid[kMaxDevices] = {false};

// Plan overrides, -1 = the library's own choice. Process-wide, lock-free reads.
std::atomic<int64_t> g_tuning[MB_TUNE_COUNT] = {-1, -1, -1, -1, -1, -1, -1, -1, -1, -1};
static_assert(MB_TUNE_COUNT == 10, "initialise every knob");

struct KnobSpec {
    const char* name;
    bool (*valid)(int64_t);
};

bool is_bool(int64_t v) { return v == 0 || v == 1; }
bool is_unroll(int64_t v) { return v == 1 || v == 2 || v == 4 || v == 8; }
bool is_threads(int64_t v) { return v >= 64 && v <= 1024 && v % 64 == 0; }
bool is_config(int64_t v) { return v >= 0 && v <= 4; }
bool is_splits(int64_t v) { return v >= 1 && v <= 512; }
bool is_mfma(int64_t v) { return v == 16 || v == 32; }

const KnobSpec kKnobs[MB_TUNE_COUNT] = {
    {"stream_unroll", is_unroll},   {"stream_nontemporal", is_bool}, {"stream_threads", is_threads},
    {"stream_schedule", is_bool},   {"gemm_force_generic", is_bool}, {"gemm_no_small_m", is_bool},
    {"gemm_tiled_config", is_config}, {"gemm_splits", is_splits},    {"gemm_fp8_mfma", is_mfma},
    {"gemm_highp_staged", is_bool},
};
constexpr int kFirstGemmKnob = MB_TUNE_GEMM_FORCE_GENERIC;

}  // namespace

int64_t tuning(int knob) {
    if (knob < 0 || knob >= MB_TUNE_COUNT) return -1;
    return g_tuning[knob].load(std::memory_order_relaxed);
}

void set_error(const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

int hip_fail(hipError_t err, const char* what) {
    set_error("%s failed: %s (hipError_t %d)", what, hipGetErrorString(err), (int)err);
    return (int)err;
}

int current_device_props(const DeviceProps** out) {
    int dev = 0;
    MB_HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) {
        set_error("device id %d out of range", dev);
        return MB_ERR_INVALID_ARG;
    }
    std::lock_guard<std::mutex> lock(g_props_mutex);
    if (!g_props_valid[dev]) {
        hipDeviceProp_t p;
        MB_HIP_TRY(hipGetDeviceProperties(&p, dev));
        DeviceProps& d = g_props[dev];
        d.device = dev;
        d.cu_count = p.multiProcessorCount;
        d.max_threads_per_cu = p.maxThreadsPerMultiProcessor;
        std::strncpy(d.arch, p.gcnArchName, sizeof(d.arch) - 1);
        d.is_gfx950 = std::strncmp(p.gcnArchName, "gfx950", 6) == 0;
        g_props_valid[dev] = true;
    }
    *out = &g_props[dev];
    return MB_OK;
}

namespace {

int device_for_launch(const DeviceProps** props) {
    int rc = current_device_props(props);
    if (rc != MB_OK) return rc;
    if (!(*props)->is_gfx950) {
        set_error("libmi355bench is built for gfx950 only; current device is %s", (*props)->arch);
        return MB_ERR_DEVICE;
    }
    return MB_OK;
}

int check_stream_args(int op, void* dst, const void* b, const void* c, uint64_t n) {
    if (n == 0) return MB_OK;
    if (dst == nullptr || b == nullptr || (op == MB_OP_TRIAD && c == nullptr)) {
        set_error("null buffer pointer (dst=%p b=%p c=%p, op %d)", dst, b, c, op);
        return MB_ERR_INVALID_ARG;
    }
    return MB_OK;
}

int check_gemm_args(int dtype, const void* A, const void* B, void* C, int64_t M, int64_t N,
                    int64_t K, void* workspace, size_t workspace_bytes, const GemmPlan& plan) {
    if (A == nullptr || B == nullptr || C == nullptr) {
        set_error("null matrix pointer (A=%p B=%p C=%p)", A, B, C);
        return MB_ERR_INVALID_ARG;
    }
    const uintptr_t mis = reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B) |
                          reinterpret_cast<uintptr_t>(C);
    if ((mis & 15u) != 0) {
        set_error("GEMM operands must be 16-byte aligned (A=%p B=%p C=%p)", A, B, C);
        return MB_ERR_SHAPE;
    }
    if (plan.workspace > 0 && (workspace == nullptr || workspace_bytes < plan.workspace)) {
        set_error("GEMM %s %lldx%lldx%lld needs %zu workspace bytes (got %zu at %p)",
                  dtype_name(dtype), (long long)M, (long long)N, (long long)K, plan.workspace,
                  workspace_bytes, workspace);
        return MB_ERR_WORKSPACE;
    }
    return MB_OK;
}

// Event-timed loop shared by the mb_time_* entry points.
template <class Launch>
int timed_loop(Launch launch, int warmup, int iterations, hipStream_t stream, double* elapsed_s) {
    if (elapsed_s == nullptr || warmup < 0 || iterations < 1) {
        set_error("timed loop needs elapsed_s != NULL, warmup >= 0, iterations >= 1");
        return MB_ERR_INVALID_ARG;
    }
    for (int i = 0; i < warmup; ++i) {
        int rc = launch();
        if (rc != MB_OK) return rc;
    }
    MB_HIP_TRY(hipStreamSynchronize(stream));
    hipEvent_t start = nullptr, stop = nullptr;
    MB_HIP_TRY(hipEventCreate(&start));
    hipError_t e = hipEventCreate(&stop);
    if (e != hipSuccess) {
        (void)hipEventDestroy(start);
        return hip_fail(e, "hipEventCreate(stop)");
    }
    int rc = MB_OK;
    e = hipEventRecord(start, stream);
    if (e != hipSuccess) rc = hip_fail(e, "hipEventRecord(start)");
    for (int i = 0; rc == MB_OK && i < iterations; ++i) rc = launch();
    if (rc == MB_OK) {
        e = hipEventRecord(stop, stream);
        if (e != hipSuccess) rc = hip_fail(e, "hipEventRecord(stop)");
    }
    if (rc == MB_OK) {
        e = hipEventSynchronize(stop);
        if (e != hipSuccess) rc = hip_fail(e, "hipEventSynchronize(stop)");
    }
    float ms = 0.0f;
    if (rc == MB_OK) {
        e = hipEventElapsedTime(&ms, start, stop);
        if (e != hipSuccess) rc = hip_fail(e, "hipEventElapsedTime");
    }
    (void)hipEventDestroy(start);
    (void)hipEventDestroy(stop);
    if (rc == MB_OK) *elapsed_s = (double)ms / 1000.0 / (double)iterations;
    return rc;
}

// Minimal JSON writer into a caller buffer.
struct Json {
    std::string s = "{";
    void key(const char* k) {
        if (s.size() > 1) s += ",";
        s += "\"";
        s += k;
        s += "\":";
    }
    void str(const char* k, const char* v) {
        key(k);
        s += "\"";
        s += v;
        s += "\"";
    }
    void num(const char* k, long long v) {
        key(k);
        s += std::to_string(v);
    }
    void boolean(const char* k, bool v) {
        key(k);
        s += v ? "true" : "false";
    }
    // The knobs of [first, last) that hold an override, as a nested object.
    void overrides(int first, int last) {
        key("overrides");
        s += "{";
        bool any = false;
        for (int i = first; i < last; ++i) {
            const int64_t v = tuning(i);
            if (v < 0) continue;
            if (any) s += ",";
            s += "\"";
            s += kKnobs[i].name;
            s += "\":";
            s += std::to_string(v);
            any = true;
        }
        s += "}";
    }
    int emit(char* out, size_t cap) {
        s += "}";
        if (out == nullptr || cap < s.size() + 1) {
            set_error("kernel info needs %zu bytes (cap %zu)", s.size() + 1, cap);
            return MB_ERR_INVALID_ARG;
        }
        std::memcpy(out, s.c_str(), s.size() + 1);
        return MB_OK;
    }
};

// Scratch for mb_gemm_noalloc: the split-K and small-M partial planes
// (split_k x M x N fp32) that mb_gemm takes from a caller's workspace. One
// copy per device, held for the life of the process. Host code never uses
// the symbol's name as an address: it resolves each device's copy with
// hipGetSymbolAddress once (scratch_address) and passes that pointer.
static __device__ __align__(256) unsigned char scratch[MB_NOALLOC_SCRATCH_BYTES];

std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {nullptr};

// This device's copy of `scratch`, resolved on the first call per device
// (with that device current) and cached.
int scratch_address(int device, void** out) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[device] == nullptr) {
        void* ptr = nullptr;
        MB_HIP_TRY(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        if (ptr == nullptr) {
            set_error("hipGetSymbolAddress(scratch) returned NULL on device %d", device);
            return MB_ERR_DEVICE;
        }
        g_scratch_ptr[device] = ptr;
    }
    *out = g_scratch_ptr[device];
    return MB_OK;
}

}  // namespace
}  // namespace mb

using namespace mb;

extern "C" {

int mb_abi_version(void) { return MB_ABI_VERSION; }

int mb_set_tuning(int knob, int64_t value) {
    clear_error();
    if (knob < 0 || knob >= MB_TUNE_COUNT) {
        set_error("unknown tuning knob %d", knob);
        return MB_ERR_INVALID_ARG;
    }
    if (value != -1 && !kKnobs[knob].valid(value)) {
        set_error("tuning knob %s cannot take %lld", kKnobs[knob].name, (long long)value);
        return MB_ERR_INVALID_ARG;
    }
    g_tuning[knob].store(value, std::memory_order_relaxed);
    return MB_OK;
}

int64_t mb_get_tuning(int knob) { return tuning(knob); }


const char* mb_last_error(void) { return g_last_error.c_str(); }

namespace {

// One stamp per block from its first lane: the CU's shader-clock counter, the
// constant-rate counter, the XCD id (hardware register XCC_ID, bits 3:0) and
// the wave's HW_ID register, which names its CU within the XCD.
__global__ void __launch_bounds__(64) clock_stamp_kernel(uint64_t* out) {
    if (threadIdx.x != 0) return;
    unsigned xcc, hw;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
    const uint64_t shader = __builtin_amdgcn_s_memtime();
    const uint64_t real = __builtin_amdgcn_s_memrealtime();
    out[4 * blockIdx.x] = shader;
    out[4 * blockIdx.x + 1] = real;
    out[4 * blockIdx.x + 2] = xcc & 0xFu;
    out[4 * blockIdx.x + 3] = hw;
}

}  // namespace

int mb_mfma_ceiling(int instruction, const void* operands, float* out, int blocks, int iterations, int warmup,
                    int launches, void* stream, double* elapsed_s) {
    clear_error();
    if (operands == nullptr || out == nullptr || blocks < 1 || blocks > 65536 || iterations < 1) {
        set_error("mb_mfma_ceiling: needs operand and output buffers, 1 <= blocks <= 65536, iterations >= 1");
        return MB_ERR_INVALID_ARG;
    }
    if (instruction < MB_MFMA_BF16_32X32X16 || instruction > MB_MFMA_F32_32X32X2) {
        set_error("mb_mfma_ceiling: unknown instruction %d", instruction);
        return MB_ERR_INVALID_ARG;
    }
    const DeviceProps* props = nullptr;
    int rc = device_for_launch(&props);
    if (rc != MB_OK) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int rounds = (iterations + 1) / 2 * 2;
    return timed_loop([&]() { return mfma_ceiling_launch(instruction, operands, out, blocks, rounds, st); }, warmup,
                      launches, st, elapsed_s);
}

int mb_clock_stamp(uint64_t* out, void* stream) {
    clear_error();
    if (out == nullptr) {
        set_error("mb_clock_stamp: null output pointer");
        return MB_ERR_INVALID_ARG;
    }
    const DeviceProps* props = nullptr;
    int rc = device_for_launch(&props);
    if (rc != MB_OK) return rc;
    hipLaunchKernelGGL(clock_stamp_kernel, dim3(MB_CLOCK_BLOCKS), dim3(64), 0, static_cast<hipStream_t>(stream), out);
    MB_HIP_TRY(hipGetLastError());
    return MB_OK;
}

int mb_stream(int op, int dtype, void* dst, const void* b, const void* c, uint64_t n, double s,
              int blocks_per_cu, void* stream) {
    clear_error();
    int rc = check_stream_args(op, dst, b, c, n);
    if (rc != MB_OK) return rc;
    const DeviceProps* props = nullptr;
    if ((rc = device_for_launch(&props)) != MB_OK) return rc;
    StreamPlan plan;
    if ((rc = stream_plan(op, dtype, dst, b, c, n, blocks_per_cu, *props, &plan)) != MB_OK) return rc;
    return stream_launch(op, dtype, dst, b, c, n, s, plan, static_cast<hipStream_t>(stream));
}

int mb_time_stream(int op, int dtype, void* dst, const void* b, const void* c, uint64_t n, double s,
                   int blocks_per_cu, int warmup, int iterations, void* stream, double* elapsed_s) {
    clear_error();
    int rc = check_stream_args(op, dst, b, c, n);
    if (rc != MB_OK) return rc;
    const DeviceProps* props = nullptr;
    if ((rc = device_for_launch(&props)) != MB_OK) return rc;
    StreamPlan plan;
    if ((rc = stream_plan(op, dtype, dst, b, c, n, blocks_per_cu, *props, &plan)) != MB_OK) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    return timed_loop([&]() { return stream_launch(op, dtype, dst, b, c, n, s, plan, st); }, warmup,
                      iterations, st, elapsed_s);
}

size_t mb_gemm_workspace_size(int dtype, int64_t M, int64_t N, int64_t K) {
    const DeviceProps* props = nullptr;
    if (current_device_props(&props) != MB_OK) return 0;
    GemmPlan plan;
    if (gemm_plan(dtype, M, N, K, *props, &plan) != MB_OK) return 0;
    return plan.workspace;
}

int mb_gemm(int dtype, const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
            float scale_a, float scale_b, void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    const DeviceProps* props = nullptr;
    int rc = device_for_launch(&props);
    if (rc != MB_OK) return rc;
    GemmPlan plan;
    if ((rc = gemm_plan(dtype, M, N, K, *props, &plan)) != MB_OK) return rc;
    if ((rc = check_gemm_args(dtype, A, B, C, M, N, K, workspace, workspace_bytes, plan)) != MB_OK)
        return rc;
    return gemm_launch(dtype, A, B, C, M, N, K, scale_a, scale_b, workspace, plan,
                       static_cast<hipStream_t>(stream));
}

int mb_gemm_noalloc(int dtype, const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
                    float scale_a, float scale_b, void* stream) {
    clear_error();
    const DeviceProps* props = nullptr;
    int rc = device_for_launch(&props);
    if (rc != MB_OK) return rc;
    GemmPlan plan;
    if ((rc = gemm_plan(dtype, M, N, K, *props, &plan)) != MB_OK) return rc;
    if (plan.workspace > (size_t)MB_NOALLOC_SCRATCH_BYTES) {
        set_error("GEMM %s %lldx%lldx%lld needs %zu scratch bytes; mb_gemm_noalloc holds %zu "
                  "(use mb_gemm with a caller workspace)",
                  dtype_name(dtype), (long long)M, (long long)N, (long long)K, plan.workspace,
                  (size_t)MB_NOALLOC_SCRATCH_BYTES);
        return MB_ERR_WORKSPACE;
    }
    void* ws = nullptr;
    if (plan.workspace > 0 && (rc = scratch_address(props->device, &ws)) != MB_OK) return rc;
    if ((rc = check_gemm_args(dtype, A, B, C, M, N, K, ws, plan.workspace, plan)) != MB_OK) return rc;
    return gemm_launch(dtype, A, B, C, M, N, K, scale_a, scale_b, ws, plan, static_cast<hipStream_t>(stream));
}

int mb_time_gemm(int dtype, const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
                 float scale_a, float scale_b, void* workspace, size_t workspace_bytes, int warmup,
                 int iterations, void* stream, double* elapsed_s) {
    clear_error();
    const DeviceProps* props = nullptr;
    int rc = device_for_launch(&props);
    if (rc != MB_OK) return rc;
    GemmPlan plan;
    if ((rc = gemm_plan(dtype, M, N, K, *props, &plan)) != MB_OK) return rc;
    if ((rc = check_gemm_args(dtype, A, B, C, M, N, K, workspace, workspace_bytes, plan)) != MB_OK)
        return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    return timed_loop(
        [&]() {
            return gemm_launch(dtype, A, B, C, M, N, K, scale_a, scale_b, workspace, plan, st);
        },
        warmup, iterations, st, elapsed_s);
}

int mb_time_gemm_rotating(int dtype, const void* const* A, const void* const* B, void* const* C, int sets,
                          int64_t M, int64_t N, int64_t K, float scale_a, float scale_b, void* workspace,
                          size_t workspace_bytes, int warmup, int iterations, void* stream, double* elapsed_s) {
    clear_error();
    if (A == nullptr || B == nullptr || C == nullptr || sets < 1) {
        set_error("rotating GEMM timing needs operand arrays and sets >= 1 (sets=%d)", sets);
        return MB_ERR_INVALID_ARG;
    }
    const DeviceProps* props = nullptr;
    int rc = device_for_launch(&props);
    if (rc != MB_OK) return rc;
    GemmPlan plan;
    if ((rc = gemm_plan(dtype, M, N, K, *props, &plan)) != MB_OK) return rc;
    for (int i = 0; i < sets; ++i)
        if ((rc = check_gemm_args(dtype, A[i], B[i], C[i], M, N, K, workspace, workspace_bytes, plan)) != MB_OK)
            return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    int next = 0;
    return timed_loop(
        [&]() {
            const int i = next;
            next = next + 1 == sets ? 0 : next + 1;
            return gemm_launch(dtype, A[i], B[i], C[i], M, N, K, scale_a, scale_b, workspace, plan, st);
        },
        warmup, iterations, st, elapsed_s);
}

int mb_kernel_info(int kind, int a, int b, int64_t m, int64_t n, int64_t k, char* json, size_t cap) {
    clear_error();
    const DeviceProps* props = nullptr;
    int rc = current_device_props(&props);
    if (rc != MB_OK) return rc;
    Json j;
    if (kind == MB_KIND_STREAM) {
        const int op = a, dtype = b;
        // Plan against 16-byte aligned buffers: the layout torch allocations have.
        alignas(16) static char dummy[16];
        StreamPlan plan;
        if ((rc = stream_plan(op, dtype, dummy, dummy, dummy, (uint64_t)m, (int)n, *props, &plan)) !=
            MB_OK)
            return rc;
        j.str("implementation", plan.vector_path ? "gfx950_stream_dwordx4" : "gfx950_stream_scalar");
        j.num("threads_per_block", plan.threads);
        j.num("vector_unroll", plan.chunks_per_trip);
        j.num("blocks_per_cu", plan.blocks_per_cu);
        j.num("grid_blocks", plan.blocks);
        j.str("schedule", plan.span ? "block_span" : "grid_stride");
        j.num("vector_bytes", 16);
        j.boolean("nontemporal", plan.nontemporal);
        j.str("arch", props->arch);
        j.overrides(0, kFirstGemmKnob);
        return j.emit(json, cap);
    }
    if (kind == MB_KIND_GEMM) {
        GemmPlan plan;
        if ((rc = gemm_plan(a, m, n, k, *props, &plan)) != MB_OK) return rc;
        j.str("implementation", plan.implementation);
        j.num("threads_per_block", plan.threads);
        j.num("grid_blocks", plan.grid);
        j.num("tile_m", plan.tile_m);
        j.num("tile_n", plan.tile_n);
        j.num("tile_k", plan.tile_k);
        j.num("wave_grid_m", plan.wave_grid_m);
        j.num("wave_grid_n", plan.wave_grid_n);
        j.num("wave_tile_m", plan.wave_tile_m);
        j.num("wave_tile_n", plan.wave_tile_n);
        j.num("frag_m", plan.frag_m);
        j.num("frag_n", plan.frag_n);
        j.num("frag_k", plan.frag_k);
        j.num("k_stages", plan.k_stages);
        j.num("split_k", plan.split_k);
        j.num("tile_group_m", plan.tile_group_m);
        j.num("workspace_bytes", (long long)plan.workspace);
        j.str("fallback", plan.fallback);
        j.str("arch", props->arch);
        j.overrides(kFirstGemmKnob, MB_TUNE_COUNT);
        return j.emit(json, cap);
    }
    set_error("unknown kernel info kind %d", kind);
    return MB_ERR_INVALID_ARG;
}

}  // extern "C"

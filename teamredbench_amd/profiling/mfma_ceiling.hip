// Sustained MFMA throughput of gfx950 under its power limit, with no memory
// traffic: the ceiling a GEMM kernel's MFMA work can reach on this part with
// random operands. One 256-thread block per CU (one wave per SIMD); each wave
// keeps kSets random operand registers per input and rotates them so that every
// MFMA sees different data (operand toggling sets the power draw), over enough
// independent accumulator chains to keep the matrix pipe full. Each kind runs
// warm-up launches until the clock has settled at the power limit, then a
// timed batch; one JSON line per kind reports the sustained TFLOP/s.
//
//   mfma_ceiling [iteration scale (default 1)]
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

#define CHECK(x)                                                                            \
    do {                                                                                    \
        hipError_t e_ = (x);                                                                \
        if (e_ != hipSuccess) {                                                             \
            std::fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
            return 1;                                                                       \
        }                                                                                   \
    } while (0)

constexpr int kSets = 4;      // random operand sets per input, rotated across MFMAs
constexpr int kThreads = 256;

enum Kind { kFp8x32, kFp8x16, kBf16x32, kBf16x16, kF32x32, kNumKinds };

__device__ __forceinline__ bf16x8 as_bf16(const i32x8& v) {
    const i32x4 h = {v[0], v[1], v[2], v[3]};
    return __builtin_bit_cast(bf16x8, h);
}

// Every thread reads 2 * kSets operand vectors of 32 bytes: data holds
// gridDim.x * kThreads * 2 * kSets of them.
template <int KIND>
__global__ void __launch_bounds__(kThreads) ceiling_kernel(const i32x8* __restrict__ data, float* __restrict__ out,
                                                           int iters) {
    const int tid = blockIdx.x * kThreads + threadIdx.x;
    i32x8 a[kSets], b[kSets];
#pragma unroll
    for (int s = 0; s < kSets; ++s) {
        a[s] = data[tid * 2 * kSets + s];
        b[s] = data[tid * 2 * kSets + kSets + s];
    }
    float r = 0.f;
    if constexpr (KIND == kFp8x32) {  // 8 chains of 32x32 fp32 accumulators
        f32x16 acc[8] = {};
        for (int i = 0; i < iters; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j)
                acc[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[j % kSets], b[(j / kSets + j) % kSets],
                                                                          acc[j], 0, 0, 0, 0, 0, 0);
        for (int j = 0; j < 8; ++j) r += acc[j][0];
    } else if constexpr (KIND == kFp8x16) {  // 16 chains of 16x16
        f32x4 acc[16] = {};
        for (int i = 0; i < iters; ++i)
#pragma unroll
            for (int j = 0; j < 16; ++j)
                acc[j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[j % kSets], b[(j / kSets + j) % kSets],
                                                                           acc[j], 0, 0, 0, 0, 0, 0);
        for (int j = 0; j < 16; ++j) r += acc[j][0];
    } else if constexpr (KIND == kBf16x32) {
        f32x16 acc[8] = {};
        for (int i = 0; i < iters; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j)
                acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16(a[j % kSets]), as_bf16(b[(j / kSets + j) % kSets]),
                                                                 acc[j], 0, 0, 0);
        for (int j = 0; j < 8; ++j) r += acc[j][0];
    } else if constexpr (KIND == kBf16x16) {
        f32x4 acc[16] = {};
        for (int i = 0; i < iters; ++i)
#pragma unroll
            for (int j = 0; j < 16; ++j)
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16(a[j % kSets]), as_bf16(b[(j / kSets + j) % kSets]),
                                                                 acc[j], 0, 0, 0);
        for (int j = 0; j < 16; ++j) r += acc[j][0];
    } else {
        f32x16 acc[8] = {};
        // whole float vectors (a bit_cast of one integer vector element is not used)
        f32x8 fa[kSets], fb[kSets];
#pragma unroll
        for (int s = 0; s < kSets; ++s) {
            fa[s] = __builtin_bit_cast(f32x8, a[s]);
            fb[s] = __builtin_bit_cast(f32x8, b[s]);
        }
        for (int i = 0; i < iters; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j)
                acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[j % kSets][j], fb[(j / kSets + j) % kSets][j], acc[j], 0, 0, 0);
        for (int j = 0; j < 8; ++j) r += acc[j][0];
    }
    out[tid] = r;
}

struct KindInfo {
    const char* name;
    const char* dtype;
    int data;              // operand bytes: 0 fp8 codes, 1 bf16 pairs, 2 fp32 values
    void (*kernel)(const i32x8*, float*, int);
    double flop_per_iter;  // per wave
    int iters;             // per launch at scale 1 (~5 ms)
    double peak_tflops;    // MI355X dense peak of the dtype
};

int main(int argc, char** argv) {
    const double scale = argc > 1 ? std::atof(argv[1]) : 1.0;
    int dev = 0;
    CHECK(hipGetDevice(&dev));
    hipDeviceProp_t props;
    CHECK(hipGetDeviceProperties(&props, dev));
    const int blocks = props.multiProcessorCount;
    const size_t vecs = (size_t)blocks * kThreads * 2 * kSets;
    const size_t words = vecs * 8;

    // Operand bytes: fp8 codes drawn below the e4m3 NaN code with random sign;
    // 16-bit halves of normal(0, 1) floats for bf16; normal(0, 1) floats for
    // fp32.
    std::mt19937 rng(1);
    std::normal_distribution<float> nd(0.f, 1.f);
    std::vector<int> h8(words), h16(words), h32(words);
    for (size_t i = 0; i < words; ++i) {
        unsigned w8 = 0, w16 = 0;
        for (int byte = 0; byte < 4; ++byte) w8 |= ((rng() & 0x7e) | ((rng() & 1) << 7)) << (8 * byte);
        for (int half = 0; half < 2; ++half) {
            const float f = nd(rng);
            unsigned u;
            std::memcpy(&u, &f, 4);
            w16 |= (u >> 16) << (16 * half);
        }
        const float f = nd(rng);
        std::memcpy(&h32[i], &f, 4);
        h8[i] = (int)w8;
        h16[i] = (int)w16;
    }
    i32x8 *d8 = nullptr, *d16 = nullptr, *d32 = nullptr;
    float* out = nullptr;
    CHECK(hipMalloc(&d8, words * 4));
    CHECK(hipMalloc(&d16, words * 4));
    CHECK(hipMalloc(&d32, words * 4));
    CHECK(hipMalloc(&out, (size_t)blocks * kThreads * sizeof(float)));
    CHECK(hipMemcpy(d8, h8.data(), words * 4, hipMemcpyHostToDevice));
    CHECK(hipMemcpy(d16, h16.data(), words * 4, hipMemcpyHostToDevice));
    CHECK(hipMemcpy(d32, h32.data(), words * 4, hipMemcpyHostToDevice));

    const KindInfo kinds[kNumKinds] = {
        {"v_mfma_scale_f32_32x32x64_f8f6f4", "float8_e4m3fn", 0, ceiling_kernel<kFp8x32>, 8 * 131072.0, 20000, 5000.0},
        {"v_mfma_scale_f32_16x16x128_f8f6f4", "float8_e4m3fn", 0, ceiling_kernel<kFp8x16>, 16 * 65536.0, 20000, 5000.0},
        {"v_mfma_f32_32x32x16_bf16", "bfloat16", 1, ceiling_kernel<kBf16x32>, 8 * 32768.0, 40000, 2500.0},
        {"v_mfma_f32_16x16x32_bf16", "bfloat16", 1, ceiling_kernel<kBf16x16>, 16 * 16384.0, 40000, 2500.0},
        {"v_mfma_f32_32x32x2_f32", "float32", 2, ceiling_kernel<kF32x32>, 8 * 4096.0, 20000, 157.3},
    };
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    constexpr int kWarm = 3, kTimed = 5;
    for (const KindInfo& k : kinds) {
        const int iters = (int)(k.iters * scale) > 0 ? (int)(k.iters * scale) : 1;
        const i32x8* data = k.data == 0 ? d8 : k.data == 1 ? d16 : d32;
        for (int w = 0; w < kWarm; ++w) hipLaunchKernelGGL(k.kernel, dim3(blocks), dim3(kThreads), 0, 0, data, out, iters);
        CHECK(hipGetLastError());
        CHECK(hipDeviceSynchronize());
        CHECK(hipEventRecord(e0));
        for (int w = 0; w < kTimed; ++w) hipLaunchKernelGGL(k.kernel, dim3(blocks), dim3(kThreads), 0, 0, data, out, iters);
        CHECK(hipEventRecord(e1));
        CHECK(hipEventSynchronize(e1));
        float ms = 0.f;
        CHECK(hipEventElapsedTime(&ms, e0, e1));
        const double flop = (double)kTimed * k.flop_per_iter * iters * blocks * (kThreads / 64);
        const double tflops = flop / (ms * 1e-3) / 1e12;
        std::printf("{\"instruction\": \"%s\", \"dtype\": \"%s\", \"sustained_tflops\": %.1f, \"peak_tflops\": %.1f, "
                    "\"fraction_of_peak\": %.4f, \"ms_per_launch\": %.3f}\n",
                    k.name, k.dtype, tflops, k.peak_tflops, tflops / k.peak_tflops, ms / kTimed);
        std::fflush(stdout);
    }
    CHECK(hipFree(d8));
    CHECK(hipFree(d16));
    CHECK(hipFree(d32));
    CHECK(hipFree(out));
    return 0;
}

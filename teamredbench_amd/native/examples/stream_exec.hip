// Example external kernel for the `hbm` benchmark's executable contract: a
// self-contained HIP program that a suite selects with
//   params.native.source: <this file>
// and that the package builds (hipcc, gfx950) and runs once per case. It
// reads the argv the benchmark passes,
//   --dtype D --mode copy|scale|triad --size-mib S --warmup W --iterations I
//   --device-id N --scale s [--blocks-per-cu B]
// times `iterations` launches with hipEvents after `warmup` untimed ones,
// and prints one JSON line: {"status", "raw_metrics": {"elapsed_s"},
// "metadata": {...}, "error"}. The benchmark fills moved_bytes and the peak
// itself. float32 only; any other dtype answers status "skipped". The
// contract is the reference's (docs/extending.md:155-175); this program is
// an example of a third-party kernel plugging into it, not the library's
// own stream path (csrc/stream.hip), which runs in-process.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

namespace {

__global__ void stream_op(float* __restrict__ dst, const float* __restrict__ b, const float* __restrict__ c,
                          size_t n, float s, int mode) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const float x = b[i];
        dst[i] = mode == 0 ? x : mode == 1 ? s * x : __builtin_fmaf(s, c[i], x);
    }
}

void emit(const char* status, double elapsed_s, const char* error, const std::string& meta) {
    if (error != nullptr) {
        std::printf("{\"status\": \"%s\", \"raw_metrics\": {}, \"metadata\": {%s}, \"error\": \"%s\"}\n", status,
                    meta.c_str(), error);
    } else {
        std::printf("{\"status\": \"%s\", \"raw_metrics\": {\"elapsed_s\": %.9e}, \"metadata\": {%s}, "
                    "\"error\": null}\n", status, elapsed_s, meta.c_str());
    }
}

}  // namespace

int main(int argc, char** argv) {
    std::string dtype = "float32", mode = "copy";
    long size_mib = 1024, warmup = 10, iterations = 50, device = 0, blocks_per_cu = 4;
    double scale = 1.0;
    for (int i = 1; i + 1 < argc; i += 2) {
        const std::string key = argv[i];
        const char* val = argv[i + 1];
        if (key == "--dtype") dtype = val;
        else if (key == "--mode") mode = val;
        else if (key == "--size-mib") size_mib = std::atol(val);
        else if (key == "--warmup") warmup = std::atol(val);
        else if (key == "--iterations") iterations = std::atol(val);
        else if (key == "--device-id") device = std::atol(val);
        else if (key == "--scale") scale = std::atof(val);
        else if (key == "--blocks-per-cu") blocks_per_cu = std::atol(val);
    }
    const std::string meta = "\"implementation\": \"example_stream_exec\", \"mode\": \"" + mode + "\"";
    const int op = mode == "copy" ? 0 : mode == "scale" ? 1 : mode == "triad" ? 2 : -1;
    if (dtype != "float32" || op < 0) {
        emit("skipped", 0.0, "the example executable runs float32 copy/scale/triad only", meta);
        return 0;
    }
    if (size_mib < 1 || iterations < 1 || warmup < 0 || blocks_per_cu < 1) {
        emit("skipped", 0.0, "invalid size, iteration or block count", meta);
        return 0;
    }
    if (hipSetDevice((int)device) != hipSuccess) {
        emit("skipped", 0.0, "hipSetDevice failed", meta);
        return 0;
    }
    hipDeviceProp_t props;
    if (hipGetDeviceProperties(&props, (int)device) != hipSuccess) {
        emit("skipped", 0.0, "hipGetDeviceProperties failed", meta);
        return 0;
    }
    const size_t n = (size_t)size_mib * 1024 * 1024 / sizeof(float);
    float *dst = nullptr, *b = nullptr, *c = nullptr;
    if (hipMalloc(&dst, n * sizeof(float)) != hipSuccess || hipMalloc(&b, n * sizeof(float)) != hipSuccess ||
        hipMalloc(&c, n * sizeof(float)) != hipSuccess) {
        emit("skipped", 0.0, "hipMalloc failed", meta);
        return 0;
    }
    (void)hipMemset(b, 0, n * sizeof(float));
    (void)hipMemset(c, 0, n * sizeof(float));
    const unsigned blocks = (unsigned)(props.multiProcessorCount * blocks_per_cu);
    for (long i = 0; i < warmup; ++i) hipLaunchKernelGGL(stream_op, dim3(blocks), dim3(256), 0, 0, dst, b, c, n,
                                                         (float)scale, op);
    hipEvent_t start, stop;
    (void)hipEventCreate(&start);
    (void)hipEventCreate(&stop);
    (void)hipDeviceSynchronize();
    (void)hipEventRecord(start, 0);
    for (long i = 0; i < iterations; ++i) hipLaunchKernelGGL(stream_op, dim3(blocks), dim3(256), 0, 0, dst, b, c,
                                                             n, (float)scale, op);
    (void)hipEventRecord(stop, 0);
    const hipError_t err = hipEventSynchronize(stop);
    float ms = 0.f;
    (void)hipEventElapsedTime(&ms, start, stop);
    (void)hipFree(dst);
    (void)hipFree(b);
    (void)hipFree(c);
    if (err != hipSuccess) {
        emit("skipped", 0.0, hipGetErrorString(err), meta);
        return 1;
    }
    emit("ok", (double)ms / 1e3 / (double)iterations, nullptr,
         meta + ", \"blocks\": " + std::to_string(blocks) + ", \"arch\": \"" + props.gcnArchName + "\"");
    return 0;
}

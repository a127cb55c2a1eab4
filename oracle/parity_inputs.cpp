// ORACLE -- test infrastructure only (see stream_oracle.c).
//
// Input generator of the reference's GEMM parity harness,
// tests/native/gemm_parity.hip.cpp:44-49: std::mt19937 seeded with `seed`,
// std::uniform_real_distribution<float>(lo, hi), one draw per element in
// row-major order. Restated with the same libstdc++ engine and distribution
// so a test can rebuild that harness's A (seed 0xA1) and B (seed 0xB2).
#include <cstdint>
#include <random>

extern "C" void oracle_fill_uniform_mt19937(float* out, uint64_t n, uint32_t seed, float lo, float hi) {
    std::mt19937 rng(seed);
    std::uniform_real_distribution<float> dist(lo, hi);
    for (uint64_t i = 0; i < n; ++i) out[i] = dist(rng);
}

/*
 * ORACLE -- test infrastructure only. Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load this library, and only as the
 * checker; the product path (teamredbench_amd) never does.
 *
 * Plain-C restatement of the arithmetic on the hot path:
 *   - stream copy / scale / triad with the reference torch path's semantics
 *     (src/teamredbench/benchmarks/hbm.py:29-39): copy is a bit copy; scale is
 *     s*b and triad b + s*c computed in fp32 (fp64 for float64) with ONE
 *     rounding to the element type (triad: correctly rounded fmaf);
 *   - the element codecs those semantics rest on, written from the format
 *     definitions (not from any library): bfloat16 and IEEE binary16 decode
 *     and round-to-nearest-even encode, and OCP FP8 E4M3FN decode
 *     (the element type of src/teamredbench/dtypes.py:23);
 *   - a float64 brute-force triple loop GEMM for tiny shapes (the reference
 *     GEMM C = A*B of src/teamredbench/benchmarks/mfu.py:229-238).
 *
 * Compile with -ffp-contract=off and SSE math (x86-64 default) so every
 * float operation below is exactly one IEEE operation.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

enum { OP_COPY = 0, OP_SCALE = 1, OP_TRIAD = 2 };
enum { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2, DT_F64 = 3, DT_I8 = 4, DT_E4M3 = 5 };

static uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* bfloat16 = the high 16 bits of a binary32. */
float oracle_bf16_decode(uint16_t h) { return bits_f32((uint32_t)h << 16); }

/* Round-to-nearest-even to bfloat16; NaN stays a (quiet) NaN with its sign. */
uint16_t oracle_bf16_encode(float f) {
    uint32_t u = f32_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* IEEE binary16: 1 sign, 5 exponent (bias 15), 10 fraction bits. */
float oracle_f16_decode(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu;
    const uint32_t frac = h & 0x3ffu;
    if (exp == 0x1fu) return bits_f32(sign | 0x7f800000u | (frac << 13)); /* inf / NaN */
    if (exp == 0) {                                                      /* zero / subnormal */
        float v = (float)frac * 0x1p-24f;                                  /* exact */
        return sign ? -v : v;
    }
    return bits_f32(sign | ((exp + 112u) << 23) | (frac << 13));
}

uint16_t oracle_f16_encode(float f) {
    const uint32_t u = f32_bits(f);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu)); /* NaN */
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    if (a < 0x38800000u) {                                  /* below 2^-14: subnormal */
        /* |f| * 2^24 is exact; rintf rounds half to even in the default mode. */
        const float q = rintf(bits_f32(a) * 0x1p24f);
        return (uint16_t)(sign | (uint16_t)q);
    }
    uint32_t r = a - (112u << 23);          /* rebias exponent 127 -> 15 */
    r += 0xfffu + ((r >> 13) & 1u);         /* round at bit 13, ties to even */
    return (uint16_t)(sign | (uint16_t)(r >> 13));
}

/*
 * OCP FP8 E4M3FN: 1 sign, 4 exponent (bias 7), 3 mantissa bits; no
 * infinities; S.1111.111 is NaN; max finite 448; min subnormal 2^-9.
 */
float oracle_e4m3_decode(uint8_t q) {
    const int sign = q >> 7;
    const int exp = (q >> 3) & 0xf;
    const int man = q & 7;
    float v;
    if (exp == 0xf && man == 7) return sign ? -NAN : NAN;
    if (exp == 0)
        v = (float)man * 0x1p-9f;
    else
        v = ldexpf(1.0f + (float)man / 8.0f, exp - 7);
    return sign ? -v : v;
}

/* OCP bf8 e5m2: 1 sign, 5 exponent (bias 15), 2 mantissa bits; IEEE-like,
 * with exponent 31 holding inf (mantissa 0) and NaN. */
float oracle_e5m2_decode(uint8_t q) {
    const int sign = q >> 7;
    const int exp = (q >> 2) & 0x1f;
    const int man = q & 3;
    float v;
    if (exp == 0x1f) {
        if (man != 0) return sign ? -NAN : NAN;
        v = INFINITY;
    } else if (exp == 0) {
        v = (float)man * 0x1p-16f;
    } else {
        v = ldexpf(1.0f + (float)man / 4.0f, exp - 15);
    }
    return sign ? -v : v;
}

void oracle_decode_bf16(const uint16_t* in, float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = oracle_bf16_decode(in[i]);
}
void oracle_encode_bf16(const float* in, uint16_t* out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = oracle_bf16_encode(in[i]);
}
void oracle_decode_f16(const uint16_t* in, float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = oracle_f16_decode(in[i]);
}
void oracle_encode_f16(const float* in, uint16_t* out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = oracle_f16_encode(in[i]);
}
void oracle_decode_e4m3(const uint8_t* in, float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = oracle_e4m3_decode(in[i]);
}
void oracle_decode_e5m2(const uint8_t* in, float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = oracle_e5m2_decode(in[i]);
}

/* Returns 0, or -1 for an unsupported (op, dtype). */
int oracle_stream(int op, int dtype, void* dst, const void* b, const void* c, uint64_t n, double s) {
    const float sf = (float)s;
    if (op == OP_COPY) {
        static const int size[] = {4, 2, 2, 8, 1};
        if (dtype < 0 || dtype > DT_I8) return -1;
        memcpy(dst, b, (size_t)n * (size_t)size[dtype]);
        return 0;
    }
    if (op != OP_SCALE && op != OP_TRIAD) return -1;
    switch (dtype) {
        case DT_F32: {
            const float* B = (const float*)b;
            const float* C = (const float*)c;
            float* D = (float*)dst;
            for (uint64_t i = 0; i < n; ++i) D[i] = op == OP_SCALE ? B[i] * sf : fmaf(sf, C[i], B[i]);
            return 0;
        }
        case DT_F64: {
            const double* B = (const double*)b;
            const double* C = (const double*)c;
            double* D = (double*)dst;
            for (uint64_t i = 0; i < n; ++i) D[i] = op == OP_SCALE ? B[i] * s : fma(s, C[i], B[i]);
            return 0;
        }
        case DT_BF16:
        case DT_F16: {
            const uint16_t* B = (const uint16_t*)b;
            const uint16_t* C = (const uint16_t*)c;
            uint16_t* D = (uint16_t*)dst;
            const int bf = dtype == DT_BF16;
            for (uint64_t i = 0; i < n; ++i) {
                const float x = bf ? oracle_bf16_decode(B[i]) : oracle_f16_decode(B[i]);
                float r;
                if (op == OP_SCALE) {
                    r = x * sf;
                } else {
                    const float y = bf ? oracle_bf16_decode(C[i]) : oracle_f16_decode(C[i]);
                    r = fmaf(sf, y, x);
                }
                D[i] = bf ? oracle_bf16_encode(r) : oracle_f16_encode(r);
            }
            return 0;
        }
        default:
            return -1;
    }
}

/* C[m][n] = sum_k A[m][k] * B[k][n] in float64, row-major, tiny shapes only. */
void oracle_gemm_f64(const float* A, const float* B, double* C, int64_t M, int64_t N, int64_t K) {
    for (int64_t i = 0; i < M; ++i)
        for (int64_t j = 0; j < N; ++j) {
            double acc = 0.0;
            for (int64_t k = 0; k < K; ++k) acc += (double)A[i * K + k] * (double)B[k * N + j];
            C[i * N + j] = acc;
        }
}

/*
 * CPU oracle for the int4-dequant GEMM/GEMV. TEST INFRASTRUCTURE ONLY: see
 * q4_oracle.h for what it restates (with reference file:line) and how each
 * function is pinned. Build with -ffp-contract=off so the fp32 generator
 * arithmetic is the reference's (no fused multiply-add).
 */
#include "q4_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

uint32_t oracle_lcg_next(uint32_t state) { return state * 1664525u + 1013904223u; }

/* test_q4gemm.cpp:58-68 */
void oracle_generate_floats(float* out, size_t n, uint32_t seed, float lo, float hi) {
    uint32_t s = seed;
    const float span = hi - lo;
    for (size_t i = 0; i < n; ++i) {
        s = oracle_lcg_next(s);
        float u = (float)(s >> 8) * (1.0f / 16777216.0f);
        float t = u * span;
        out[i] = lo + t;
    }
}

/* test_q4gemm.cpp:71-80 */
void oracle_generate_int4(int8_t* out, size_t n, uint32_t seed) {
    uint32_t s = seed;
    for (size_t i = 0; i < n; ++i) {
        s = oracle_lcg_next(s);
        out[i] = (int8_t)((int)((s >> 8) % 16u) - 8);
    }
}

void oracle_generate_normal(float* out, size_t n, uint32_t seed, float mean, float stddev) {
    const double two_pi = 6.283185307179586476925286766559;
    uint32_t s = seed;
    for (size_t i = 0; i < n; i += 2) {
        s = oracle_lcg_next(s);
        double u1 = ((double)(s >> 8) + 1.0) * (1.0 / 16777216.0);
        s = oracle_lcg_next(s);
        double u2 = (double)(s >> 8) * (1.0 / 16777216.0);
        double r = sqrt(-2.0 * log(u1));
        out[i] = (float)((double)mean + (double)stddev * r * cos(two_pi * u2));
        if (i + 1 < n) out[i + 1] = (float)((double)mean + (double)stddev * r * sin(two_pi * u2));
    }
}

/* test_q4gemm.cpp:84-99; layout q4gemm.comp:7-19 */
int oracle_pack_q4(const int8_t* b, uint32_t K, uint32_t N, uint8_t* packed) {
    if (!b || !packed || (K & 1u)) return 1;
    const size_t half = K / 2u;
    memset(packed, 0, half * (size_t)N);
    for (uint32_t n = 0; n < N; ++n) {
        for (uint32_t k = 0; k < K; ++k) {
            uint32_t nib = (uint32_t)(uint8_t)b[(size_t)k * N + n] & 0xFu;
            uint32_t shift = (k & 1u) * 4u;
            packed[(size_t)n * half + (k >> 1)] |= (uint8_t)(nib << shift);
        }
    }
    return 0;
}

static inline int sign_extend_nibble(uint32_t nib) { return nib >= 8u ? (int)nib - 16 : (int)nib; }

int oracle_unpack_q4(const uint8_t* packed, uint32_t K, uint32_t N, int8_t* b) {
    if (!b || !packed || (K & 1u)) return 1;
    const size_t half = K / 2u;
    for (uint32_t n = 0; n < N; ++n) {
        for (uint32_t k = 0; k < K; ++k) {
            uint32_t byte = packed[(size_t)n * half + (k >> 1)];
            uint32_t nib = (k & 1u) ? (byte >> 4) : (byte & 0xFu);
            b[(size_t)k * N + n] = (int8_t)sign_extend_nibble(nib);
        }
    }
    return 0;
}

/* test_q4gemm.cpp:102-119 */
int oracle_q4gemm_ref(const float* a, const int8_t* b, const float* scales,
                      uint32_t M, uint32_t N, uint32_t K, double* c) {
    if (!a || !b || !scales || !c || (K % 32u)) return 1;
    const uint32_t groups = K / 32u;
    memset(c, 0, sizeof(double) * (size_t)M * N);
    for (uint32_t m = 0; m < M; ++m) {
        for (uint32_t k = 0; k < K; ++k) {
            double av = (double)a[(size_t)m * K + k];
            for (uint32_t n = 0; n < N; ++n) {
                double bv = (double)b[(size_t)k * N + n] * (double)scales[(size_t)n * groups + k / 32u];
                c[(size_t)m * N + n] += av * bv;
            }
        }
    }
    return 0;
}

/* One output element from the packed layout, terms in ascending k. */
static double packed_dot(const float* arow, const uint8_t* col, const float* colscales, uint32_t K) {
    double acc = 0.0;
    for (uint32_t k = 0; k < K; k += 2) {
        uint32_t byte = col[k >> 1];
        double s = (double)colscales[k / 32u];
        double b0 = (double)sign_extend_nibble(byte & 0xFu) * s;
        double b1 = (double)sign_extend_nibble(byte >> 4) * s;
        acc += (double)arow[k] * b0;
        acc += (double)arow[k + 1] * b1;
    }
    return acc;
}

int oracle_q4gemm_packed_rows(const float* a, const uint8_t* packed, const float* scales,
                              uint32_t M, uint32_t N, uint32_t K,
                              uint32_t row_begin, uint32_t row_end, int threads, double* c) {
    if (!a || !packed || !scales || !c || (K % 32u) || row_begin > row_end || row_end > M) return 1;
    const uint32_t rows = row_end - row_begin;
    const uint32_t groups = K / 32u;
    const size_t half = K / 2u;
    const int64_t total = (int64_t)rows * N;
#ifdef _OPENMP
    if (threads < 1) threads = 1;
#pragma omp parallel for schedule(static) num_threads(threads)
#endif
    for (int64_t idx = 0; idx < total; ++idx) {
        uint32_t r = (uint32_t)(idx / N);
        uint32_t n = (uint32_t)(idx % N);
        const float* arow = a + (size_t)(row_begin + r) * K;
        c[idx] = packed_dot(arow, packed + (size_t)n * half, scales + (size_t)n * groups, K);
    }
    (void)threads;
    return 0;
}

int oracle_q4gemm_lora_rows(const float* a, const uint8_t* packed, const float* scales,
                            const float* la, const float* lb, uint32_t rank, double scale,
                            uint32_t M, uint32_t N, uint32_t K,
                            uint32_t row_begin, uint32_t row_end, int threads, double* c) {
    if (!la || !lb || rank == 0) return 1;
    int rc = oracle_q4gemm_packed_rows(a, packed, scales, M, N, K, row_begin, row_end, threads, c);
    if (rc) return rc;
    const uint32_t rows = row_end - row_begin;
    double* t = (double*)malloc(sizeof(double) * (size_t)rows * rank);
    if (!t) return 1;
    for (uint32_t r = 0; r < rows; ++r) {
        const float* arow = a + (size_t)(row_begin + r) * K;
        for (uint32_t q = 0; q < rank; ++q) {
            double acc = 0.0;
            for (uint32_t k = 0; k < K; ++k) acc += (double)arow[k] * (double)la[(size_t)k * rank + q];
            t[(size_t)r * rank + q] = acc;
        }
    }
    for (uint32_t r = 0; r < rows; ++r) {
        for (uint32_t n = 0; n < N; ++n) {
            double delta = 0.0;
            for (uint32_t q = 0; q < rank; ++q) delta += t[(size_t)r * rank + q] * (double)lb[(size_t)q * N + n];
            c[(size_t)r * N + n] += scale * delta;
        }
    }
    free(t);
    return 0;
}

/* test_q4gemm.cpp:376-390; parity.py:6-16 */
size_t oracle_compare(const float* actual, const double* expected, size_t n, double tol,
                      double* max_rel, double* max_abs, int64_t* first_bad, double* normwise) {
    double mr = 0.0, ma = 0.0, num = 0.0, den = 0.0;
    int64_t fb = -1;
    size_t bad = 0;
    for (size_t i = 0; i < n; ++i) {
        double ref = expected[i];
        double err = fabs((double)actual[i] - ref);
        double denom = fabs(ref) > 1.0 ? fabs(ref) : 1.0;
        double rel = err / denom;
        /* NaN in actual must fail: compare through the negation. */
        if (!(rel <= tol)) {
            if (fb < 0) fb = (int64_t)i;
            ++bad;
            if (rel != rel) rel = INFINITY;
        }
        if (err != err) err = INFINITY;
        if (err > ma) ma = err;
        if (rel > mr) mr = rel;
        num += ((double)actual[i] - ref) * ((double)actual[i] - ref);
        den += ref * ref;
    }
    if (max_rel) *max_rel = mr;
    if (max_abs) *max_abs = ma;
    if (first_bad) *first_bad = fb;
    if (normwise) *normwise = sqrt(num) / (sqrt(den) > 1e-300 ? sqrt(den) : 1e-300);
    return bad;
}

int oracle_q4_quantize(const float* w, uint32_t K, uint32_t N, uint8_t* packed, float* scales) {
    if (!w || !packed || !scales || (K % 32u) != 0u) return 1;
    const uint32_t G = K / 32u;
    const size_t half = K / 2u;
    memset(packed, 0, half * (size_t)N);
    for (uint32_t n = 0; n < N; ++n) {
        for (uint32_t g = 0; g < G; ++g) {
            float m = w[(size_t)(32u * g) * N + n];
            int finite = isfinite(m);
            for (uint32_t t = 1; t < 32u; ++t) {
                const float v = w[(size_t)(32u * g + t) * N + n];
                if (fabsf(v) > fabsf(m)) m = v;
                if (!isfinite(v)) finite = 0;
            }
            float scale = -m * 0.125f;
            if (!finite) {
                scales[(size_t)n * G + g] = NAN;
                continue;
            }
            if (scale == 0.0f) {
                scales[(size_t)n * G + g] = 0.0f;
                continue;
            }
            scales[(size_t)n * G + g] = scale;
            for (uint32_t t = 0; t < 32u; ++t) {
                const uint32_t k = 32u * g + t;
                float r = rintf(w[(size_t)k * N + n] / scale);
                if (r < -8.0f) r = -8.0f;
                if (r > 7.0f) r = 7.0f;
                const uint32_t nib = (uint32_t)(int)r & 0xFu;
                packed[(size_t)n * half + (k >> 1)] |= (uint8_t)(nib << ((k & 1u) * 4u));
            }
        }
    }
    return 0;
}

/* Drives every function of the CPU oracle (oracle/q4_oracle.c, oracle/cq4_oracle.c) on
 * small inputs, including the argument-rejection paths, so that a build with
 * -fsanitize=address,undefined checks their memory accesses and arithmetic. Test
 * infrastructure: built and run by tests/test_sanitize_cpu.py. Exits 0 when every
 * check holds; the sanitizers abort on the first error they find. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "cq4_oracle.h"
#include "q4_oracle.h"

static int failures = 0;
#define CHECK(cond)                                                   \
    do {                                                              \
        if (!(cond)) {                                                \
            fprintf(stderr, "check failed: %s (line %d)\n", #cond, __LINE__); \
            ++failures;                                               \
        }                                                             \
    } while (0)

static uint16_t f16_bits(float v) {
    /* round-to-nearest fp16 of small normal values used below (|v| in [2^-14, 65504]) */
    uint32_t u;
    memcpy(&u, &v, 4);
    const uint32_t sign = (u >> 16) & 0x8000u;
    if ((u & 0x7FFFFFFFu) == 0) return (uint16_t)sign;
    int e = (int)((u >> 23) & 0xFF) - 127 + 15;
    uint32_t m = u & 0x7FFFFFu;
    uint32_t r = m >> 13, rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1))) ++r;
    if (r == 0x400u) { r = 0; ++e; }
    return (uint16_t)(sign | ((uint32_t)e << 10) | r);
}

static void q4_paths(uint32_t M, uint32_t N, uint32_t K) {
    const size_t xs = (size_t)M * K, bs = (size_t)K * N, ss = (size_t)N * (K / 32);
    float* a = malloc(xs * sizeof(float));
    int8_t* b = malloc(bs);
    int8_t* b2 = malloc(bs);
    float* s = malloc(ss * sizeof(float));
    uint8_t* packed = malloc(bs / 2);
    double* ref = malloc((size_t)M * N * sizeof(double));
    double* rows = malloc((size_t)M * N * sizeof(double));
    double* lora = malloc((size_t)M * N * sizeof(double));
    float* y = malloc((size_t)M * N * sizeof(float));
    oracle_generate_floats(a, xs, 0x12345678u, -1.0f, 1.0f);
    oracle_generate_normal(a, xs - 1, 0x2468u, 0.0f, 1.0f); /* odd count: the last pair's tail */
    oracle_generate_int4(b, bs, 0x9ABCDEF0u);
    oracle_generate_floats(s, ss, 0x13579BDFu, 0.01f, 0.05f);
    CHECK(oracle_pack_q4(b, K, N, packed) == 0);
    CHECK(oracle_unpack_q4(packed, K, N, b2) == 0);
    CHECK(memcmp(b, b2, bs) == 0);
    CHECK(oracle_q4gemm_ref(a, b, s, M, N, K, ref) == 0);
    CHECK(oracle_q4gemm_packed_rows(a, packed, s, M, N, K, 0, M, 1, rows) == 0);
    CHECK(memcmp(ref, rows, (size_t)M * N * sizeof(double)) == 0);
    if (M > 1) {
        CHECK(oracle_q4gemm_packed_rows(a, packed, s, M, N, K, 1, M, 2, rows) == 0);
        CHECK(memcmp(ref + N, rows, (size_t)(M - 1) * N * sizeof(double)) == 0);
    }
    const uint32_t R = 3;
    float* la = malloc((size_t)K * R * sizeof(float));
    float* lb = malloc((size_t)R * N * sizeof(float));
    memset(la, 0, (size_t)K * R * sizeof(float));
    memset(lb, 0, (size_t)R * N * sizeof(float));
    CHECK(oracle_q4gemm_lora_rows(a, packed, s, la, lb, R, 2.0, M, N, K, 0, M, 1, lora) == 0);
    CHECK(memcmp(lora, ref, (size_t)M * N * sizeof(double)) == 0); /* zero adapter: the base exactly */
    oracle_generate_normal(la, (size_t)K * R, 7u, 0.0f, 0.02f);
    oracle_generate_normal(lb, (size_t)R * N, 9u, 0.0f, 0.02f);
    CHECK(oracle_q4gemm_lora_rows(a, packed, s, la, lb, R, 2.0, M, N, K, 0, M, 2, lora) == 0);
    for (size_t i = 0; i < (size_t)M * N; ++i) y[i] = (float)ref[i];
    double max_rel = 0, max_abs = 0, normwise = 0;
    int64_t first_bad = 0;
    CHECK(oracle_compare(y, ref, (size_t)M * N, 1e-5, &max_rel, &max_abs, &first_bad, &normwise) == 0);
    CHECK(first_bad == -1 && max_rel < 1e-6);
    y[0] = NAN;
    CHECK(oracle_compare(y, ref, (size_t)M * N, 1e-5, &max_rel, &max_abs, &first_bad, &normwise) == 1);
    CHECK(first_bad == 0);
    /* quantizer, with an all-zero group and a non-finite group when there is room */
    float* w = malloc((size_t)K * N * sizeof(float));
    uint8_t* qp = malloc(bs / 2);
    float* qs = malloc(ss * sizeof(float));
    oracle_generate_normal(w, (size_t)K * N, 11u, 0.0f, 1.0f);
    for (uint32_t k = 0; k < 32; ++k) w[(size_t)k * N] = 0.0f;
    if (K >= 64) w[(size_t)40 * N] = INFINITY;
    CHECK(oracle_q4_quantize(w, K, N, qp, qs) == 0);
    CHECK(qs[0] == 0.0f);
    if (K >= 64) CHECK(isnan(qs[1]));
    /* rejection paths */
    CHECK(oracle_pack_q4(b, K + 1, N, packed) == 1);
    CHECK(oracle_unpack_q4(packed, K + 1, N, b2) == 1);
    CHECK(oracle_q4gemm_ref(a, b, s, M, N, K + 2, ref) == 1);
    CHECK(oracle_q4gemm_packed_rows(a, packed, s, M, N, K, 2, 1, 1, rows) == 1);
    CHECK(oracle_q4_quantize(w, K + 1, N, qp, qs) == 1);
    free(a); free(b); free(b2); free(s); free(packed); free(ref); free(rows); free(lora); free(y);
    free(la); free(lb); free(w); free(qp); free(qs);
}

static void cq4_paths(void) {
    enum { K = 64, N = 8, GS = 32, G = 2, M = 3 };
    uint16_t codebook[16], a[M * K], norms[N * G];
    int8_t ls[GS], rs[GS];
    uint32_t perm[GS];
    float f[M * K];
    oracle_generate_floats(f, M * K, 5u, -1.0f, 1.0f);
    for (int i = 0; i < M * K; ++i) a[i] = f16_bits(f[i]);
    for (int i = 0; i < 16; ++i) codebook[i] = f16_bits((float)(i - 8) / 8.0f);
    for (int i = 0; i < N * G; ++i) norms[i] = f16_bits(0.5f + 0.01f * (float)i);
    for (int i = 0; i < GS; ++i) {
        ls[i] = (i % 3) ? 1 : -1;
        rs[i] = (i % 5) ? -1 : 1;
        perm[i] = (uint32_t)((i * 7) % GS);
    }
    double out[M * K], c[M * N];
    for (uint32_t bits = 1; bits <= 4; ++bits) {
        const uint32_t row_bytes = (GS * bits + 7) / 8;
        uint8_t* idx = malloc((size_t)N * G * row_bytes);
        for (uint32_t i = 0; i < N * G * row_bytes; ++i) idx[i] = (uint8_t)(i * 37u + bits);
        oracle_cq4_matrix W = {bits, K, N, GS, G, 0, codebook, NULL, NULL, norms, idx, ls, rs, perm, NULL, NULL, NULL};
        CHECK(oracle_cq4_transform(&W, a, M, out) == 0);
        CHECK(oracle_cq4_matmul(&W, a, M, c) == 0);
        for (uint32_t k = 0; k < GS; ++k) CHECK(oracle_cq4_index_lsb(idx, k, bits) < (1u << bits));
        W.bits = 5;
        CHECK(oracle_cq4_matmul(&W, a, M, c) == 1);
        free(idx);
    }
    /* 4-row interleaved panels, 4-bit */
    {
        const uint32_t panel_bytes = 4 * GS / 2;
        uint8_t* idx = malloc((size_t)(N / 4) * G * panel_bytes);
        for (uint32_t i = 0; i < (N / 4) * G * panel_bytes; ++i) idx[i] = (uint8_t)(i * 13u);
        oracle_cq4_matrix W = {4, K, N, GS, G, ORACLE_CQ4_FLAG_INTERLEAVED_4ROW, codebook, NULL, NULL, norms, idx,
                               NULL, NULL, NULL, NULL, NULL, NULL};
        CHECK(oracle_cq4_matmul(&W, a, M, c) == 0);
        CHECK(oracle_cq4_index_interleaved(idx, 3, GS - 1) < 16u);
        free(idx);
    }
    /* orthogonal mode: one group spanning K, rotation K x K */
    {
        uint16_t* rot = malloc((size_t)K * K * sizeof(uint16_t));
        for (int i = 0; i < K * K; ++i) rot[i] = (i % (K + 1)) ? 0 : f16_bits(1.0f);
        const uint32_t row_bytes = K * 4 / 8;
        uint8_t* idx = malloc((size_t)N * row_bytes);
        for (uint32_t i = 0; i < N * row_bytes; ++i) idx[i] = (uint8_t)(i * 29u);
        oracle_cq4_matrix W = {4, K, N, K, 1, ORACLE_CQ4_FLAG_ORTHOGONAL, codebook, NULL, NULL, norms, idx,
                               NULL, NULL, NULL, rot, NULL, NULL};
        CHECK(oracle_cq4_matmul(&W, a, M, c) == 0);
        free(idx);
        free(rot);
    }
    CHECK(oracle_f16_to_double(0x0001u) == ldexp(1.0, -24));
    CHECK(oracle_cq4_matmul(NULL, a, M, c) == 1);
}

int main(void) {
    CHECK(oracle_lcg_next(0u) == 0x3C6EF35Fu);
    q4_paths(1, 1, 32);
    q4_paths(3, 5, 96);
    q4_paths(5, 17, 256);
    cq4_paths();
    if (failures) {
        fprintf(stderr, "%d check(s) failed\n", failures);
        return 1;
    }
    printf("oracle sanitizer driver: all checks passed\n");
    return 0;
}

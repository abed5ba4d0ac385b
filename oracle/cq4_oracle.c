/*
 * CPU oracle of the CQ4 codebook matmul, double precision (test infrastructure;
 * see cq4_oracle.h for what it restates and who may use it).
 */
#include "cq4_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

double oracle_f16_to_double(uint16_t h) {
    const int sign = (h >> 15) & 1;
    const int exp = (h >> 10) & 0x1F;
    const int man = h & 0x3FF;
    double v;
    if (exp == 0) {
        v = ldexp((double)man, -24); /* subnormal: man * 2^-24 */
    } else if (exp == 31) {
        v = man ? NAN : INFINITY;
    } else {
        v = ldexp((double)(man | 0x400), exp - 25); /* (1024 + man) * 2^(exp - 15 - 10) */
    }
    return sign ? -v : v;
}

/* cactus_x86.cpp:24-43 (LSB-first; 3-bit indices may straddle a byte). */
uint32_t oracle_cq4_index_lsb(const uint8_t* packed, uint32_t k, uint32_t bits) {
    const uint32_t bit = k * bits;
    uint32_t v = packed[bit / 8] >> (bit % 8);
    if (bit % 8 + bits > 8) v |= (uint32_t)packed[bit / 8 + 1] << (8 - bit % 8);
    return v & ((1u << bits) - 1u);
}

/* cactus_x86.cpp:48-53: 16-byte chunks of 8 values; row r owns bytes 4r..4r+3 of
 * a chunk; value 8c + s sits in byte (s & 3), high nibble when s >= 4. */
uint32_t oracle_cq4_index_interleaved(const uint8_t* panel, uint32_t row, uint32_t k) {
    const uint8_t b = panel[(k / 8) * 16 + row * 4 + (k & 3)];
    return (k & 4) ? (uint32_t)(b >> 4) : (uint32_t)(b & 0xF);
}

static int valid(const oracle_cq4_matrix* W, const uint16_t* A, uint32_t M) {
    if (!W || !A || M == 0) return 0;
    if (W->bits == 0 || W->bits > 4) return 0;
    if (W->K == 0 || W->N == 0 || W->group_size == 0 || W->num_groups == 0) return 0;
    if (!W->codebook || !W->norms || !W->packed_indices) return 0;
    if (W->flags & ORACLE_CQ4_FLAG_ORTHOGONAL) return W->rotation != NULL;
    return W->K == W->group_size * W->num_groups;
}

/* cactus_x86.cpp:74-80: input_scale_recip, else 1 / input_scale, else 1. */
static double recip(const oracle_cq4_matrix* W, uint32_t k) {
    if (W->input_scale_recip) return oracle_f16_to_double(W->input_scale_recip[k]);
    if (W->input_scale) return 1.0 / oracle_f16_to_double(W->input_scale[k]);
    return 1.0;
}

/* cactus_x86.cpp:55-70: in-place butterflies over strides 1, 2, 4, ..., then 1/sqrt(n). */
static void fwht(double* x, uint32_t n) {
    for (uint32_t h = 1; h < n; h <<= 1)
        for (uint32_t i = 0; i < n; i += 2 * h)
            for (uint32_t j = i; j < i + h; ++j) {
                const double a = x[j], b = x[j + h];
                x[j] = a + b;
                x[j + h] = a - b;
            }
    const double s = 1.0 / sqrt((double)n);
    for (uint32_t i = 0; i < n; ++i) x[i] *= s;
}

int oracle_cq4_transform(const oracle_cq4_matrix* W, const uint16_t* A, uint32_t M, double* out) {
    if (!valid(W, A, M) || !out) return 1;
    const uint32_t K = W->K;
    if (W->flags & ORACLE_CQ4_FLAG_ORTHOGONAL) {
        /* cactus_x86.cpp:198-210: A_rot[m][i] = sum_k A[m][k] * recip[k] * R[k][i] */
        for (uint32_t m = 0; m < M; ++m)
            for (uint32_t i = 0; i < K; ++i) {
                double acc = 0.0;
                for (uint32_t k = 0; k < K; ++k)
                    acc += oracle_f16_to_double(A[(size_t)m * K + k]) * recip(W, k) *
                           oracle_f16_to_double(W->rotation[(size_t)k * K + i]);
                out[(size_t)m * K + i] = acc;
            }
        return 0;
    }
    /* cactus_x86.cpp:87-113: scale and left sign, FWHT, right sign, then gather by the permutation */
    const uint32_t gs = W->group_size;
    double* work = (double*)malloc(sizeof(double) * gs);
    if (!work) return 1;
    for (uint32_t m = 0; m < M; ++m)
        for (uint32_t g = 0; g < W->num_groups; ++g) {
            const uint32_t base = g * gs;
            for (uint32_t k = 0; k < gs; ++k) {
                const double sign = W->left_signs ? (double)W->left_signs[k] : 1.0;
                work[k] = oracle_f16_to_double(A[(size_t)m * K + base + k]) * recip(W, base + k) * sign;
            }
            fwht(work, gs);
            for (uint32_t k = 0; k < gs; ++k)
                if (W->right_signs) work[k] *= (double)W->right_signs[k];
            for (uint32_t j = 0; j < gs; ++j)
                out[(size_t)m * K + base + j] = work[W->permutation ? W->permutation[j] : j];
        }
    free(work);
    return 0;
}

int oracle_cq4_matmul(const oracle_cq4_matrix* W, const uint16_t* A, uint32_t M, double* C) {
    if (!valid(W, A, M) || !C) return 1;
    const uint32_t K = W->K, N = W->N, bits = W->bits;
    const int orth = (W->flags & ORACLE_CQ4_FLAG_ORTHOGONAL) != 0;
    const int inter = (W->flags & ORACLE_CQ4_FLAG_INTERLEAVED_4ROW) != 0;
    /* the orthogonal mode is one group spanning K (cactus_x86.cpp:191) */
    const uint32_t gs = orth ? K : W->group_size, ng = orth ? 1 : W->num_groups;
    const size_t pgb = ((size_t)gs * bits + 7) / 8;
    double* basis = (double*)malloc(sizeof(double) * (size_t)M * K);
    if (!basis) return 1;
    if (oracle_cq4_transform(W, A, M, basis)) {
        free(basis);
        return 1;
    }
    double cb[16];
    for (uint32_t i = 0; i < (1u << bits); ++i) cb[i] = oracle_f16_to_double(W->codebook[i]);
    for (uint32_t m = 0; m < M; ++m)
        for (uint32_t n = 0; n < N; ++n) {
            double acc = 0.0;
            for (uint32_t g = 0; g < ng; ++g) {
                /* norms: panel-major [(n/4)*ng + g]*4 + n%4 when interleaved, else [n*ng + g]
                   (cactus_x86.cpp:151-159, 229) */
                const size_t ni = inter ? ((size_t)(n / 4) * ng + g) * 4 + (n & 3) : (size_t)n * ng + g;
                const double norm = oracle_f16_to_double(W->norms[ni]);
                const double* b = basis + (size_t)m * K + (size_t)g * gs;
                double s = 0.0;
                if (inter) {
                    const uint8_t* panel = W->packed_indices + ((size_t)(n / 4) * ng + g) * 4 * pgb;
                    for (uint32_t k = 0; k < gs; ++k) s += b[k] * cb[oracle_cq4_index_interleaved(panel, n & 3, k)];
                } else {
                    const uint8_t* row = W->packed_indices + ((size_t)n * ng + g) * pgb;
                    for (uint32_t k = 0; k < gs; ++k) s += b[k] * cb[oracle_cq4_index_lsb(row, k, bits)];
                }
                acc += norm * s;
            }
            C[(size_t)m * N + n] = acc;
        }
    free(basis);
    return 0;
}

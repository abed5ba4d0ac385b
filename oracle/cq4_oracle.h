/*
 * CPU oracle of the CQ4 codebook matmul (test infrastructure: only tests/,
 * __graft_entry__.smoke() and bench.py's CPU baseline use it, as the checker).
 *
 * Restates cactus_quant_matmul of vulkan-runtime/src/cactus/cactus_x86.cpp
 * (:24-53 index extraction, :55-70 normalized FWHT, :74-113 activation
 * transform, :133-182 Hadamard-basis matmul, :189-240 orthogonal matmul,
 * :384-397 dispatch and argument checks) in double precision, reading fp16
 * inputs exactly. The struct has the field order of CactusQuantMatrixBridge
 * (vulkan-runtime/src/cactus/cactus_x86_bridge.h) so one ctypes structure
 * describes a matrix to this oracle, to the reference's compiled bridge and to
 * the product's spaceslug_cq4_matmul.
 */
#ifndef CQ4_ORACLE_H
#define CQ4_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORACLE_CQ4_FLAG_ORTHOGONAL (1u << 2)
#define ORACLE_CQ4_FLAG_INTERLEAVED_4ROW (1u << 3)

typedef struct oracle_cq4_matrix {
    uint32_t bits, K, N, group_size, num_groups, flags;
    const uint16_t* codebook;          /* fp16 [2^bits] */
    const uint16_t* input_scale;       /* fp16 [K] or NULL */
    const uint16_t* input_scale_recip; /* fp16 [K] or NULL (preferred over input_scale) */
    const uint16_t* norms;             /* fp16, [n*num_groups+g], panel-major when interleaved */
    const uint8_t* packed_indices;
    const int8_t* left_signs;          /* [group_size] or NULL */
    const int8_t* right_signs;         /* [group_size] or NULL */
    const uint32_t* permutation;       /* [group_size] or NULL */
    const uint16_t* rotation;          /* fp16 [K][K], orthogonal only */
    const int8_t* expanded;            /* unused */
    const float* norm_f32;             /* unused */
} oracle_cq4_matrix;

/* fp16 bit pattern -> double (exact, subnormals included). */
double oracle_f16_to_double(uint16_t h);

/* Index k of one row's LSB-first bit-packed group (bits 1..4). */
uint32_t oracle_cq4_index_lsb(const uint8_t* packed, uint32_t k, uint32_t bits);

/* Index k of row r (0..3) of a 4-bit INTERLEAVED_4ROW panel. */
uint32_t oracle_cq4_index_interleaved(const uint8_t* panel, uint32_t row, uint32_t k);

/* The activation in the code basis: out[m][K] (Hadamard groups, or A_rot for
 * the orthogonal mode). Returns 0, or 1 on invalid arguments. */
int oracle_cq4_transform(const oracle_cq4_matrix* W, const uint16_t* A, uint32_t M, double* out);

/* C[m][n] in double (not rounded to fp16). Returns 0, or 1 when the reference
 * would return without writing (cactus_x86.cpp:384-397). */
int oracle_cq4_matmul(const oracle_cq4_matrix* W, const uint16_t* A, uint32_t M, double* C);

#ifdef __cplusplus
}
#endif

#endif

/*
 * CPU oracle for the int4-dequant GEMM/GEMV (Spaceslug q4gemm).
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker: the parity tests,
 * __graft_entry__.smoke() and the cpu_baseline leg of bench.py load it. The
 * product library (spaceslug-main_amd) never links, loads or calls it.
 *
 * It restates, in plain C, the algorithm of the reference's CPU int4 kernel
 * and its input generators:
 *   - vulkan-runtime/tests/test_q4gemm.cpp:58-68   generate_floats (NR LCG)
 *   - vulkan-runtime/tests/test_q4gemm.cpp:71-80   generate_int4
 *   - vulkan-runtime/tests/test_q4gemm.cpp:84-99   pack_q4 (layout contract
 *     vulkan-runtime/shaders/q4gemm.comp:7-19)
 *   - vulkan-runtime/tests/test_q4gemm.cpp:102-119 cpu_reference (double,
 *     loop order m -> k -> n)
 *   - vulkan-runtime/tests/test_q4gemm.cpp:376-390 and
 *     python/spaceslug/parity.py:6-16            comparator
 *   - python/spaceslug/lora.py:21-23, vulkan-runtime/shaders/lora_delta.comp:2-21,
 *     python/spaceslug/backend.py:794-799       LoRA composition
 * The normal generator (Box-Muller on the same LCG) has no counterpart in the
 * reference; it only shapes synthetic N(mu, sigma) inputs. Neither has the
 * fp32 -> int4 quantizer (oracle_q4_quantize): it restates the rule of this
 * build's spaceslug_q4_quantize (documented in include/runtime_abi.h) so the
 * GPU quantizer can be checked bit for bit.
 *
 * Parity pins (tests/test_oracle.py): Numerical Recipes' published LCG
 * sequence; hand-derived nibble bytes from the layout comments; exhaustive
 * pack/unpack over all nibble values, positions and byte lanes; exact rational
 * arithmetic (fractions.Fraction) on small shapes; integer GEMM through numpy
 * when every scale is 1; the unit-vector, linearity and power-of-two scale
 * invariants; packed-vs-unpacked bit identity.
 */
#ifndef SPACESLUG_Q4_ORACLE_H
#define SPACESLUG_Q4_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* One step of the Numerical Recipes LCG: s' = s * 1664525 + 1013904223 (mod 2^32). */
uint32_t oracle_lcg_next(uint32_t state);

/* test_q4gemm.cpp:58-68: v[i] = lo + ((s >> 8) * 2^-24) * (hi - lo), fp32 arithmetic. */
void oracle_generate_floats(float* out, size_t n, uint32_t seed, float lo, float hi);

/* test_q4gemm.cpp:71-80: v[i] = (s >> 8) % 16 - 8. */
void oracle_generate_int4(int8_t* out, size_t n, uint32_t seed);

/* Box-Muller on the same LCG (two LCG draws per pair of outputs):
 *   u1 = ((s1 >> 8) + 1) * 2^-24 in (0, 1],  u2 = (s2 >> 8) * 2^-24 in [0, 1)
 *   r = sqrt(-2 ln u1); out[2i] = mean + stddev * r cos(2 pi u2);
 *   out[2i+1] = mean + stddev * r sin(2 pi u2)   (double math, rounded to fp32). */
void oracle_generate_normal(float* out, size_t n, uint32_t seed, float mean, float stddev);

/* test_q4gemm.cpp:84-99. b is K x N row-major int8 in [-8, 7]; packed is the
 * byte image of the reference's uint32 words: packed[n*(K/2) + k/2], even k in
 * the low nibble, odd k in the high nibble, each nibble = v & 0xF.
 * Returns 0, or 1 when K is odd. */
int oracle_pack_q4(const int8_t* b, uint32_t K, uint32_t N, uint8_t* packed);

/* Inverse of oracle_pack_q4 (sign-extends each nibble). Returns 0, or 1 when K is odd. */
int oracle_unpack_q4(const uint8_t* packed, uint32_t K, uint32_t N, int8_t* b);

/* test_q4gemm.cpp:102-119, verbatim semantics: c[m][n] += double(a[m][k]) *
 * (double(b[k][n]) * double(scales[n*(K/32) + k/32])), loops m -> k -> n.
 * Returns 0, or 1 when K % 32 != 0. */
int oracle_q4gemm_ref(const float* a, const int8_t* b, const float* scales,
                      uint32_t M, uint32_t N, uint32_t K, double* c);

/* Same arithmetic, reading the packed bytes, for rows [row_begin, row_end) only
 * (c is (row_end-row_begin) x N). Each c[m][n] sums its terms in ascending k,
 * exactly as oracle_q4gemm_ref does, and every term a*(b*s) is exact in double,
 * so the result is bit-identical to oracle_q4gemm_ref. threads > 1 splits rows
 * and columns over OpenMP threads without changing any element's summation order.
 * Returns 0, or 1 on bad arguments. */
int oracle_q4gemm_packed_rows(const float* a, const uint8_t* packed, const float* scales,
                              uint32_t M, uint32_t N, uint32_t K,
                              uint32_t row_begin, uint32_t row_end, int threads, double* c);

/* LoRA-composed projection in double (lora.py:21-23, lora_delta.comp:2-21,
 * backend.py:794-799): c[m][n] = base[m][n] + scale * sum_r t[m][r] * lb[r][n]
 * with t[m][r] = sum_k a[m][k] * la[k][r]; la is K x R, lb is R x N, row-major.
 * base is oracle_q4gemm_packed_rows over the same rows. Returns 0 or 1. */
int oracle_q4gemm_lora_rows(const float* a, const uint8_t* packed, const float* scales,
                            const float* la, const float* lb, uint32_t rank, double scale,
                            uint32_t M, uint32_t N, uint32_t K,
                            uint32_t row_begin, uint32_t row_end, int threads, double* c);

/* Comparator of test_q4gemm.cpp:376-390 / parity.py:6-16:
 * rel_i = |actual_i - expected_i| / max(1, |expected_i|). Writes max_rel, max_abs
 * and the first index whose rel exceeds tol (or -1). Also writes the normwise
 * error ||actual - expected||_2 / max(1e-300, ||expected||_2). Returns the
 * number of elements over tol. */
size_t oracle_compare(const float* actual, const double* expected, size_t n, double tol,
                      double* max_rel, double* max_abs, int64_t* first_bad, double* normwise);

/* fp32 w[k][n] -> packed int4 [n][k/2] + scales [n][k/32]: per (column, group of
 * 32) m = largest-magnitude value (first in k order), scale = -m/8, nibble =
 * clamp(rint(w/scale), -8, 7); scale 0 and zero nibbles for an all-zero group;
 * NaN scale and zero nibbles for a group holding a NaN or an infinity. Returns 1
 * unless k % 32 == 0. */
int oracle_q4_quantize(const float* w, uint32_t K, uint32_t N, uint8_t* packed, float* scales);

#ifdef __cplusplus
}
#endif

#endif

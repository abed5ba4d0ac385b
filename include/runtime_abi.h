/*
 * Spaceslug runtime C-ABI, MI355X (gfx950) native build.
 *
 * Drop-in superset of the reference's top-level C-ABI (native/runtime_abi.h:1-9)
 * and of the two symbols the reference's Python host binds unconditionally
 * (python/spaceslug/backend.py:62-67): spaceslug_vector_add and spaceslug_sgemm.
 * Everything else is the int4-dequant GEMM/GEMV the reference implements as the
 * Vulkan shader vulkan-runtime/shaders/q4gemm.comp, which has no C-ABI export in
 * the reference; its entry points below follow the export conventions of
 * vulkan-runtime/src/api/sgemm_api.h:7-9 and lora_delta_api.h:5-13.
 *
 * Conventions (reference: sgemm_api.cpp:38,63; lora_delta_api.h:7;
 * tiny_forward_persistent.h:270,312,474,556-558):
 *   - C linkage, plain pointers, uint32_t dimensions, int status.
 *   - 0 = success; 1 = invalid arguments (null pointer, zero or unsupported
 *     dimension, misaligned device pointer); 2 = device/runtime failure caught at
 *     the boundary (including "no HIP device"); -4 = capability not supported.
 *     No C++ exception crosses the boundary.
 *   - Host-pointer entry points are synchronous: inputs are copied to the GPU and
 *     the output is fully written before return. The caller owns every buffer.
 *   - *_device entry points take device pointers and a hipStream_t (passed as
 *     void*; NULL = the default stream) and only enqueue work: outputs are valid
 *     once the stream is synchronised.
 *   - Persistent state lives behind opaque handles: create returns NULL on
 *     failure, destroy accepts NULL.
 *   - Single-threaded per process like the reference (its exec engine is
 *     documented single-threaded, engine.h:37): concurrent calls from several
 *     host threads are not supported.
 *
 * Weight format (q4gemm.comp:7-19; test_q4gemm.cpp:7-17), group size fixed at 32:
 *   logical W is K x N, each value v in [-8, 7]; stored as the nibble v & 0xF.
 *   w_packed is uint8[N][K/2]: byte n*(K/2) + k/2 holds k even in bits 0..3 and
 *   k odd in bits 4..7 (byte-identical to the reference's little-endian uint32
 *   words). w_scales is float[N][K/32]; dequant(k, n) = v(k, n) * w_scales[n*(K/32) + k/32].
 *   x is float[M][K] row-major; y is float[M][N] row-major.
 *   y[m][n] = sum_k x[m][k] * dequant(k, n)   (fp32 inputs, fp32 output).
 *
 * Accuracy, as max |y - ref| / max(1, |ref|) against the double-precision
 * reference (test_q4gemm.cpp:102-119, metric of test_q4gemm.cpp:380):
 *   - m <= 32: every 32-value group sum is exact (x in 31-bit fixed point per
 *     row and group, as signed digits on integer dot products or the int8 MFMA)
 *     and the groups are summed in double. The error is the final fp32 rounding
 *     (2^-24 |y|) plus the fixed-point rounding of x, at most 2^-30 of the
 *     group's largest |x| per value: <= 2e-7 on the reference KAT's input ranges
 *     (x in [-1, 1), scales in [0.5, 1.5); test_q4gemm.cpp:168-176), asserted for
 *     m = 1..32 at K up to 8192 (the decode GEMV up to K = 32768), and on x
 *     whose groups span 1e-30..1e30.
 *   - m > 32 (bf16 MFMA on x split exactly into three bf16 limbs; every product
 *     exact, one fp32 rounding per MFMA of each 32-value group sum, groups summed
 *     in double): the error grows like sqrt(K / 32). Stated tolerance
 *     6e-6 * sqrt(K / 32) on unit-range inputs (the KAT's ranges; asserted at
 *     K = 1024, 4096 and 8192, where it is 9.6e-5), and <= 1e-5 on the
 *     reference's KAT (256^3, test_q4gemm.cpp:40-49) and on the documented
 *     workload configurations (N(0, 1) x, scales in [0.01, 0.05]) up to K = 8192.
 *   - LoRA adds the fp32 product T = x * lora_a (K-split partials summed in
 *     double) times lora_b, accumulated in double.
 *   - A non-finite x gives IEEE's result for x itself, as the reference does: every
 *     output of that row is non-finite, NaN where inf meets a zero nibble, opposite
 *     infinities meet or a NaN enters, the signed infinity otherwise.
 */
#ifndef SPACESLUG_RUNTIME_ABI_H
#define SPACESLUG_RUNTIME_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SPACESLUG_OK 0
#define SPACESLUG_ERR_INVALID 1
#define SPACESLUG_ERR_DEVICE 2
#define SPACESLUG_ERR_UNSUPPORTED (-4)

/* Largest LoRA rank the fused epilogue accepts. */
#define SPACESLUG_Q4_MAX_LORA_RANK 64u

/* native/runtime_abi.h:6 (CPU implementation native/runtime_abi.cpp:3-7):
 * output[i] = left[i] + right[i]. Returns 1 on a null pointer, else 0. */
int spaceslug_vector_add(const float* left, const float* right, float* output, size_t count);

/* vulkan-runtime/src/api/sgemm_api.h:7-9 (implementation sgemm_api.cpp:37-63):
 * fp32 row-major C[m][n] = A[m][k] * B[k][n] on the GPU. Same shape contract as
 * the reference: m % 64 == 0, n % 64 == 0, k % 32 == 0, all nonzero, else 1.
 * *max_relative_error is written as 0, as the reference does. Synchronous. */
int spaceslug_sgemm(const float* a, const float* b, float* c, uint32_t m, uint32_t n, uint32_t k,
                    float* max_relative_error);

/* Capability string of the int4 path (pattern: tiny_forward_persistent.h:557-558).
 * Static storage, never NULL. */
const char* spaceslug_q4gemm_capability(void);

/* Message of the last failing call on this thread ("" if none). */
const char* spaceslug_last_error(void);

/* Replaces q4gemm.comp:61-175 as dispatched by test_q4gemm.cpp:335-356, as a
 * C-ABI call: synchronous host pointers, any 1 <= m, n <= 2^31 - 2^16, k % 32 == 0
 * (the reference shader additionally needs m % 64 == 0 and n % 64 == 0,
 * q4gemm.comp:36-37). */
int spaceslug_q4gemm(const float* x, const uint8_t* w_packed, const float* w_scales, float* y,
                     uint32_t m, uint32_t n, uint32_t k);

/* Int4 projection with a fused LoRA epilogue, replacing the three-call composition
 * of backend.py:794-799 (spaceslug_sgemm, spaceslug_lora_delta with B pre-scaled
 * by alpha/rank, then a host add; lora_delta_api.h:5-13, lora.py:21-23):
 *   y = x * dequant(W) + scale * (x * lora_a) * lora_b
 * lora_a is float[k][rank], lora_b is float[rank][n], both row-major (the layouts
 * of lora_delta.comp:2). scale is alpha / rank. 1 <= rank <= SPACESLUG_Q4_MAX_LORA_RANK.
 * Synchronous host pointers. */
int spaceslug_q4gemm_lora(const float* x, const uint8_t* w_packed, const float* w_scales,
                          const float* lora_a, const float* lora_b, float* y,
                          uint32_t m, uint32_t n, uint32_t k, uint32_t rank, float scale);

/* Device-pointer, stream-ordered variant of spaceslug_q4gemm (no reference
 * counterpart: the reference never passes device memory across its ABI). d_x,
 * d_w_packed must be 16-byte aligned; d_w_scales, d_y 4-byte aligned.
 * Enqueues only. Without LoRA, calls of up to 32 rows use no device memory
 * beyond their arguments; above 32 rows the three bf16 limbs of x (6 * m * k
 * bytes, m rounded up to a multiple of 16 on the 128 x 128 tiles) and any
 * K-split partial sums, and in LoRA calls the T = x * lora_a partials, live
 * in a library-owned device workspace that is allocated on first use and
 * grown on demand (growth synchronises the device, steady state does not
 * allocate). Calls that share a device share that workspace; the library
 * orders them: a call on a stream other than the previous user's makes its
 * stream wait (on the GPU, hipStreamWaitEvent) for that user's kernels, and
 * host threads are serialised while enqueueing. A call that needs that
 * workspace returns SPACESLUG_ERR_UNSUPPORTED, enqueueing nothing, while
 * `stream` is being captured into a graph (the graph would keep an address a
 * later, larger call frees): capture a spaceslug_q4_chain or use
 * spaceslug_q4gemm_device_noalloc. */
int spaceslug_q4gemm_device(const float* d_x, const uint8_t* d_w_packed, const float* d_w_scales,
                            float* d_y, uint32_t m, uint32_t n, uint32_t k, void* stream);

/* Size of the fixed device scratch of spaceslug_q4gemm_device_noalloc (64 MiB per device). */
#define SPACESLUG_Q4_NOALLOC_SCRATCH_BYTES (64u << 20)

/* No counterpart in the reference: for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * arguments, contract and results as spaceslug_q4gemm_device, but the call allocates and
 * frees nothing: the scratch its kernels need (the bf16 limbs of x above 32 rows, K-split
 * partial sums) lives in one fixed array of SPACESLUG_Q4_NOALLOC_SCRATCH_BYTES per device,
 * held from module load until the process ends. A shape whose scratch would exceed it
 * returns 1 without enqueueing anything (the five workload shapes fit: 2048 x 4096 x 14336
 * needs 48 MiB). Every call on a device shares that device's array and nothing in it needs
 * to start at zero; calls that overlap on one device (other streams, or threads) race on it,
 * so callers order them, e.g. on one stream. */
int spaceslug_q4gemm_device_noalloc(const float* d_x, const uint8_t* d_w_packed, const float* d_w_scales,
                                    float* d_y, uint32_t m, uint32_t n, uint32_t k, void* stream);

/* Device-pointer, stream-ordered variant of spaceslug_q4gemm_lora. Keeps
 * T = x * lora_a (m * rank floats) and any K-split partials in the same
 * library-owned device workspace as spaceslug_q4gemm_device (and so returns
 * SPACESLUG_ERR_UNSUPPORTED under stream capture the same way). */
int spaceslug_q4gemm_lora_device(const float* d_x, const uint8_t* d_w_packed,
                                 const float* d_w_scales, const float* d_lora_a,
                                 const float* d_lora_b, float* d_y, uint32_t m, uint32_t n,
                                 uint32_t k, uint32_t rank, float scale, void* stream);

/* fp32 -> int4 group-32 quantizer writing the packed layout above (no counterpart
 * in the reference, whose int4 weights come only from its test generators,
 * test_q4gemm.cpp:71-80; it is what lets real fp32 checkpoints feed the kernels).
 * w is float[k][n] row-major, the orientation of the reference's logical B
 * (test_q4gemm.cpp:16). Per column n and 32-value group g: m = the value of
 * largest magnitude (first in k order on ties), scale = -m/8, nibble =
 * clamp(rint(w/scale), -8, 7) with IEEE division and round-to-nearest-even; an
 * all-zero group gets scale 0 and zero nibbles. Needs k % 32 == 0 and
 * k/32 <= 65535; non-finite weights return 1. Synchronous host pointers. */
int spaceslug_q4_quantize(const float* w, uint8_t* w_packed, float* w_scales, uint32_t n, uint32_t k);

/* Device-pointer, stream-ordered variant of spaceslug_q4_quantize. d_w_packed must
 * be 16-byte aligned. Enqueues only and does not reject non-finite weights: a
 * group holding a NaN or an infinity gets a NaN scale and zero nibbles. */
int spaceslug_q4_quantize_device(const float* d_w, uint8_t* d_w_packed, float* d_w_scales, uint32_t n,
                                 uint32_t k, void* stream);

/* Device-resident weights (handle pattern of tiny_forward_persistent.h:556 and
 * .cpp:4751-4800, 5373-5378): uploads w_packed/w_scales once so repeated
 * projections (backend.py:1719-1735 issues five per token) do not re-stage them. */
typedef struct spaceslug_q4_weight spaceslug_q4_weight;

spaceslug_q4_weight* spaceslug_q4_weight_create(const uint8_t* w_packed, const float* w_scales,
                                                uint32_t n, uint32_t k);
void spaceslug_q4_weight_destroy(spaceslug_q4_weight* weight);

/* Synchronous host x/y against a weight handle: y[m][n] = x[m][k] * dequant(W). */
int spaceslug_q4gemm_run(const spaceslug_q4_weight* weight, const float* x, float* y, uint32_t m);

/* Retained projection chain: a fixed sequence of device-pointer projections recorded
 * once into one HIP graph and replayed with one launch, with no host round trip and
 * no per-call planning between the steps. Replaces the reference's retained
 * command buffers (vulkan-runtime/src/exec/engine.h:85-101, recordImmutable /
 * submitImmutable: "retain fully recorded command buffers and resubmit without
 * re-recording") and the persistent tiny forward's handle pattern
 * (tiny_forward_persistent.h:556-558). A step holds the arguments of one
 * spaceslug_q4gemm_device call, or of spaceslug_q4gemm_lora_device when d_lora_a is
 * not NULL; a step may read what an earlier step wrote (steps run in order). */
typedef struct spaceslug_q4_step {
    const float* d_x;          /* [m][k], 16-byte aligned */
    const uint8_t* d_w_packed; /* [n][k/2], 16-byte aligned */
    const float* d_w_scales;   /* [n][k/32] */
    float* d_y;                /* [m][n] */
    uint32_t m, n, k;
    const float* d_lora_a;     /* [k][rank], or NULL for no LoRA term */
    const float* d_lora_b;     /* [rank][n] */
    uint32_t rank;             /* 1..SPACESLUG_Q4_MAX_LORA_RANK when d_lora_a is set */
    float lora_scale;          /* alpha / rank */
} spaceslug_q4_step;

typedef struct spaceslug_q4_chain spaceslug_q4_chain;

/* Validates every step as the device entry points do, plans each, records them on
 * the current device into one graph and instantiates it. The chain owns the
 * device workspace its steps need, so replays share no memory with other calls.
 * Addresses are fixed at creation: callers change buffer contents between runs,
 * never addresses, and must not change them while a replay is in flight
 * (engine.h:89-91 asks the same of retained command buffers). NULL on failure. */
spaceslug_q4_chain* spaceslug_q4_chain_create(const spaceslug_q4_step* steps, uint32_t count);

/* Enqueues one replay of the chain on `stream` (hipStream_t as void*, NULL = the
 * default stream). Replays of one chain must be ordered (one stream, or
 * synchronised by the caller): they share the chain's workspace. Returns 1 when the
 * current device is not the chain's. */
int spaceslug_q4_chain_run(spaceslug_q4_chain* chain, void* stream);

/* Waits for the chain's device, then releases the graph and the workspace. NULL is a no-op. */
void spaceslug_q4_chain_destroy(spaceslug_q4_chain* chain);

/* CQ4 codebook matmul (the reference's other quantized matmul, cactus_quant_matmul:
 * vulkan-runtime/src/cactus/cactus_x86.cpp:133-240, 384-397; C bridge
 * cactus_bridge_quant_matmul, cactus_x86_bridge.h). The struct has the field order of
 * CactusQuantMatrixBridge, so a caller's bridge struct can be passed as is; fp16
 * values are IEEE binary16 bit patterns in uint16_t. Per output:
 *   C[m][n] = sum_g norm(n, g) * sum_k A'[m][g*gs + k] * codebook[idx(n, g, k)]
 * where A' is the activation in the code basis: per group, A * input-scale
 * reciprocal * left sign, normalized Walsh-Hadamard transform, * right sign, then
 * gathered by the permutation (cactus_x86.cpp:87-113); with
 * SPACESLUG_CQ4_FLAG_ORTHOGONAL, one group spans K and A' = (A * recip) x rotation
 * (cactus_x86.cpp:197-210). Indices are LSB-first bit-packed per (row, group)
 * (bits 1..4), or with SPACESLUG_CQ4_FLAG_INTERLEAVED_4ROW 4-bit 4-row panels with
 * panel-major norms (cactus_x86.cpp:48-53, 151-159). Arithmetic is fp32 and C is
 * rounded to fp16 once. Returns 1, writing nothing, where the reference returns
 * without writing (null pointers, bits outside 1..4, zero sizes, K != gs * groups)
 * and also for layouts it does not define: a Hadamard group size that is not a
 * power of two up to 256 (its transform buffer holds 256), interleaved panels with
 * bits != 4, N % 4 != 0 or gs % 8 != 0, M > 65535, and K or N above 2^31 - 2^16.
 * `expanded` and `norm_f32` are ignored, as the reference ignores them. */
#define SPACESLUG_CQ4_FLAG_ORTHOGONAL (1u << 2)
#define SPACESLUG_CQ4_FLAG_INTERLEAVED_4ROW (1u << 3)

typedef struct spaceslug_cq4_matrix {
    uint32_t bits;
    uint32_t K;
    uint32_t N;
    uint32_t group_size;
    uint32_t num_groups;
    uint32_t flags;
    const uint16_t* codebook;          /* fp16 [2^bits] */
    const uint16_t* input_scale;       /* fp16 [K] or NULL */
    const uint16_t* input_scale_recip; /* fp16 [K] or NULL (used first when both are set) */
    const uint16_t* norms;             /* fp16 [N * groups] ([N] orthogonal), panel-major if interleaved */
    const uint8_t* packed_indices;     /* N * groups * ceil(gs * bits / 8) bytes */
    const int8_t* left_signs;          /* [gs] or NULL */
    const int8_t* right_signs;         /* [gs] or NULL */
    const uint32_t* permutation;       /* [gs] or NULL */
    const uint16_t* rotation;          /* fp16 [K][K], orthogonal only */
    const int8_t* expanded;            /* ignored */
    const float* norm_f32;             /* ignored */
} spaceslug_cq4_matrix;

/* Synchronous host pointers: A is fp16 [M][K], C is fp16 [M][N]. */
int spaceslug_cq4_matmul(const spaceslug_cq4_matrix* w, const uint16_t* a, uint32_t m, uint16_t* c);

/* Device-pointer, stream-ordered variant: every array of `w` (the struct itself
 * is host memory) and a, c are device pointers. The code-basis activations live in
 * the library-owned device workspace of spaceslug_q4gemm_device, ordered the same
 * way across streams; under stream capture such a call returns
 * SPACESLUG_ERR_UNSUPPORTED. Decode calls (Hadamard basis, 4-bit indices, M <= 4,
 * group size a multiple of 8, M * K <= 4096) run as one launch without the
 * workspace and may be captured. */
int spaceslug_cq4_matmul_device(const spaceslug_cq4_matrix* w, const uint16_t* d_a, uint32_t m, uint16_t* d_c,
                                void* stream);

#ifdef __cplusplus
}
#endif

#endif

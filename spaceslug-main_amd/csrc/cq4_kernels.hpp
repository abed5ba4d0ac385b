// Host-side launch interface of the CQ4 codebook matmul (cq4.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace spaceslug {

constexpr uint32_t kCq4FlagOrthogonal = 1u << 2;        // cactus_x86.h:51
constexpr uint32_t kCq4FlagInterleaved4Row = 1u << 3;  // cactus_x86.h:52

typedef float f32x4_t __attribute__((ext_vector_type(4)));

// A matrix whose arrays are all device pointers (fp16 as uint16_t bit patterns).
struct Cq4View {
    uint32_t bits, K, N, group_size, num_groups, flags;
    const uint16_t* codebook;
    const uint16_t* input_scale;
    const uint16_t* input_scale_recip;
    const uint16_t* norms;
    const uint8_t* packed;
    const int8_t* left_signs;
    const int8_t* right_signs;
    const uint32_t* permutation;
    const uint16_t* rotation;
};

// Device bytes launch_cq4_matmul needs for m rows: the code-basis activations, as m * K floats,
// or on the MFMA path as their bf16 limbs (6 * m * K bytes).
size_t cq4_workspace_bytes(const Cq4View& w, uint32_t m);

// C[m][N] (fp16) = transform(A[m][K] fp16) x decode(W). `workspace` holds
// cq4_workspace_bytes(w, m) bytes, 256-byte aligned. Arguments are validated by the caller.
hipError_t launch_cq4_matmul(const Cq4View& w, const uint16_t* a, uint32_t m, uint16_t* c, void* workspace,
                             hipStream_t stream);

}  // namespace spaceslug

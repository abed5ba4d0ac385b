// CQ4 codebook matmul on gfx950: C = transform(A) x decode(W), fp16 in and out,
// fp32 arithmetic. Semantics of cactus_quant_matmul (vulkan-runtime/src/cactus/
// cactus_x86.cpp:133-240, 384-397); the reference's GPU chain is three
// dispatches through two fp16 intermediates (transform_act -> dequant_w ->
// sgemm_f16_am, vulkan-runtime/tests/test_cq4.cpp:255-334). Here:
//   1. the activation transform writes the code-basis activations A' in fp32
//      (one workgroup per (row, group) for the Hadamard basis: scale and left
//      sign, an in-LDS normalized Walsh-Hadamard transform, right sign and
//      permutation; a direct product with the rotation for the orthogonal mode);
//   2. one GEMM kernel decodes the packed indices in registers (LSB-first bit
//      packing or 4-row interleaved panels), looks codebook values up in LDS and
//      accumulates in fp32 per group, scaling each group sum by its norm; the
//      dequantized weight matrix is never materialized, and C is rounded to fp16
//      once.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "cq4_kernels.hpp"

namespace spaceslug {
namespace {

__device__ __forceinline__ float half_bits_to_float(uint16_t h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }

__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));  // round to nearest even
}

// Per-element input scale reciprocal (cactus_x86.cpp:74-80).
__device__ __forceinline__ float input_recip(const Cq4View& w, uint32_t k) {
    if (w.input_scale_recip) return half_bits_to_float(w.input_scale_recip[k]);
    if (w.input_scale) return 1.0f / half_bits_to_float(w.input_scale[k]);
    return 1.0f;
}

// Hadamard basis: grid (num_groups, M), group_size / 2 threads; thread t owns
// elements t and t + gs/2 on load and store and butterfly t at every stage.
__global__ __launch_bounds__(128) void cq4_transform_hadamard_kernel(Cq4View w, const uint16_t* __restrict__ a,
                                                                     float* __restrict__ out) {
    __shared__ float v[256];
    const uint32_t gs = w.group_size, half = gs >> 1;
    const uint32_t g = blockIdx.x, m = blockIdx.y, t = threadIdx.x;
    const size_t row = static_cast<size_t>(m) * w.K + static_cast<size_t>(g) * gs;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const uint32_t k = t + e * half;
        const float sign = w.left_signs ? static_cast<float>(w.left_signs[k]) : 1.0f;
        v[k] = half_bits_to_float(a[row + k]) * input_recip(w, g * gs + k) * sign;
    }
    __syncthreads();
    for (uint32_t h = 1; h < gs; h <<= 1) {  // butterflies over strides 1, 2, 4, ... (cactus_x86.cpp:56-66)
        const uint32_t j = (t / h) * 2 * h + (t % h);  // each thread owns one disjoint pair per stage
        const float x = v[j], y = v[j + h];
        v[j] = x + y;
        v[j + h] = x - y;
        __syncthreads();
    }
    const float inv = 1.0f / sqrtf(static_cast<float>(gs));
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const uint32_t j = t + e * half;
        // an out-of-range entry is masked into the group (the host entry point rejects it)
        const uint32_t src = w.permutation ? (w.permutation[j] & (gs - 1)) : j;
        const float sign = w.right_signs ? static_cast<float>(w.right_signs[src]) : 1.0f;
        out[row + j] = v[src] * inv * sign;
    }
}

// Orthogonal basis: A_rot[m][i] = sum_k A[m][k] recip[k] R[k][i]; grid (ceil(K/256), M).
__global__ __launch_bounds__(256) void cq4_transform_orthogonal_kernel(Cq4View w, const uint16_t* __restrict__ a,
                                                                       float* __restrict__ out) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x, m = blockIdx.y;
    if (i >= w.K) return;
    const uint16_t* arow = a + static_cast<size_t>(m) * w.K;
    float acc = 0.0f;
    for (uint32_t k = 0; k < w.K; ++k)
        acc = fmaf(half_bits_to_float(arow[k]) * input_recip(w, k), half_bits_to_float(w.rotation[static_cast<size_t>(k) * w.K + i]),
                   acc);
    out[static_cast<size_t>(m) * w.K + i] = acc;
}

// Index k of a row's LSB-first group (cactus_x86.cpp:24-43), any bits in 1..4.
__device__ __forceinline__ uint32_t index_lsb(const uint8_t* p, uint32_t k, uint32_t bits) {
    const uint32_t bit = k * bits;
    uint32_t v = p[bit >> 3] >> (bit & 7);
    if ((bit & 7) + bits > 8) v |= static_cast<uint32_t>(p[(bit >> 3) + 1]) << (8 - (bit & 7));
    return v & ((1u << bits) - 1u);
}

// One thread per (column n, ROWS rows). Per group: 8 indices per 32-bit word of
// the row's packed group, codebook values from LDS, fp32 sums per row, then
// acc += norm(n, g) * sum.
// LAYOUT 0: 4-bit LSB-first (nibble j of word c is k = 8c + j);
// LAYOUT 1: 4-bit interleaved panels (row r's word c is bytes 16c + 4r .. +3:
//           low nibble of byte b is k = 8c + b, high nibble k = 8c + 4 + b);
// LAYOUT 2: LSB-first of any width (element by element).
template <int ROWS, int LAYOUT>
__global__ __launch_bounds__(256) void cq4_gemm_kernel(Cq4View w, const float* __restrict__ ap, uint16_t* __restrict__ c,
                                                       uint32_t M, uint32_t gs, uint32_t ng) {
    __shared__ float lut[16];
    if (threadIdx.x < (1u << w.bits)) lut[threadIdx.x] = half_bits_to_float(w.codebook[threadIdx.x]);
    __syncthreads();
    const uint32_t n = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t m0 = blockIdx.y * ROWS;
    if (n >= w.N) return;
    const bool inter = LAYOUT == 1;
    const size_t pgb = (static_cast<size_t>(gs) * w.bits + 7) / 8;
    const float* arow[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) arow[r] = ap + static_cast<size_t>(min(m0 + r, M - 1)) * w.K;
    float acc[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) acc[r] = 0.0f;
    for (uint32_t g = 0; g < ng; ++g) {
        const size_t ni = inter ? (static_cast<size_t>(n / 4) * ng + g) * 4 + (n & 3) : static_cast<size_t>(n) * ng + g;
        const float norm = half_bits_to_float(w.norms[ni]);
        float s[ROWS];
#pragma unroll
        for (int r = 0; r < ROWS; ++r) s[r] = 0.0f;
        const uint32_t kg = g * gs;
        if constexpr (LAYOUT == 2) {
            const uint8_t* p = w.packed + (static_cast<size_t>(n) * ng + g) * pgb;
            for (uint32_t k = 0; k < gs; ++k) {
                const float cv = lut[index_lsb(p, k, w.bits)];
#pragma unroll
                for (int r = 0; r < ROWS; ++r) s[r] = fmaf(arow[r][kg + k], cv, s[r]);
            }
        } else {
            const uint8_t* base = inter ? w.packed + (static_cast<size_t>(n / 4) * ng + g) * 4 * pgb + (n & 3) * 4
                                        : w.packed + (static_cast<size_t>(n) * ng + g) * pgb;
            const uint32_t stride = inter ? 16 : 4;  // bytes between consecutive 8-index words of the row
            for (uint32_t c8 = 0; c8 < gs / 8; ++c8) {
                const uint32_t word = *reinterpret_cast<const uint32_t*>(base + c8 * stride);
                float av[ROWS][8];
#pragma unroll
                for (int r = 0; r < ROWS; ++r) {
                    const f32x4_t lo = *reinterpret_cast<const f32x4_t*>(arow[r] + kg + 8 * c8);
                    const f32x4_t hi = *reinterpret_cast<const f32x4_t*>(arow[r] + kg + 8 * c8 + 4);
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        av[r][q] = lo[q];
                        av[r][4 + q] = hi[q];
                    }
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    // nibble j holds k = 8c + j (LSB) or 8c + (j >> 1) + 4 (j & 1) (interleaved)
                    const int kk = inter ? (j >> 1) + 4 * (j & 1) : j;
                    const float cv = lut[(word >> (4 * j)) & 0xFu];
#pragma unroll
                    for (int r = 0; r < ROWS; ++r) s[r] = fmaf(av[r][kk], cv, s[r]);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < ROWS; ++r) acc[r] = fmaf(norm, s[r], acc[r]);
    }
#pragma unroll
    for (int r = 0; r < ROWS; ++r)
        if (m0 + r < M) c[static_cast<size_t>(m0 + r) * w.N + n] = float_to_half_bits(acc[r]);
}

template <int ROWS>
hipError_t launch_gemm(const Cq4View& w, const float* ap, uint16_t* c, uint32_t m, uint32_t gs, uint32_t ng,
                       hipStream_t stream) {
    const dim3 grid((w.N + 255) / 256, (m + ROWS - 1) / ROWS);
    const bool inter = (w.flags & kCq4FlagInterleaved4Row) != 0;
    if (inter)
        hipLaunchKernelGGL((cq4_gemm_kernel<ROWS, 1>), grid, dim3(256), 0, stream, w, ap, c, m, gs, ng);
    else if (w.bits == 4 && gs % 8 == 0)
        hipLaunchKernelGGL((cq4_gemm_kernel<ROWS, 0>), grid, dim3(256), 0, stream, w, ap, c, m, gs, ng);
    else
        hipLaunchKernelGGL((cq4_gemm_kernel<ROWS, 2>), grid, dim3(256), 0, stream, w, ap, c, m, gs, ng);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_cq4_matmul(const Cq4View& w, const uint16_t* a, uint32_t m, uint16_t* c, float* workspace,
                             hipStream_t stream) {
    const bool orth = (w.flags & kCq4FlagOrthogonal) != 0;
    const uint32_t gs = orth ? w.K : w.group_size, ng = orth ? 1 : w.num_groups;
    if (orth) {
        hipLaunchKernelGGL(cq4_transform_orthogonal_kernel, dim3((w.K + 255) / 256, m), dim3(256), 0, stream, w, a,
                           workspace);
    } else {
        // group_size / 2 threads (one for a group of 1, whose transform is the identity)
        hipLaunchKernelGGL(cq4_transform_hadamard_kernel, dim3(w.num_groups, m), dim3(w.group_size > 1 ? w.group_size / 2 : 1),
                           0, stream, w, a, workspace);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return m >= 4 ? launch_gemm<4>(w, workspace, c, m, gs, ng, stream) : launch_gemm<1>(w, workspace, c, m, gs, ng, stream);
}

}  // namespace spaceslug

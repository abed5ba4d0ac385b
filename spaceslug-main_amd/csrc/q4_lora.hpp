// LoRA pre-pass and epilogue helpers shared by the int4 GEMM kernels (q4_gemm.hip,
// q4_small.hip). T = x * la, la row-major [K][R] (lora_delta.comp:2-21, lora.py:21-23),
// is computed as K-split partials that every GEMM epilogue sums itself.
#pragma once

#include "q4_device.hpp"
#include "q4_kernels.hpp"

namespace spaceslug {
namespace {

// T[row][r] = the sum of its t_splits partials, in double and in split order, rounded once.
__device__ __forceinline__ float lora_t_value(const float* __restrict__ tpart, int t_splits, int M, int R, int row,
                                              int r) {
    double t = 0.0;
    for (int z = 0; z < t_splits; ++z) t += static_cast<double>(tpart[(static_cast<size_t>(z) * M + row) * R + r]);
    return static_cast<float>(t);
}

// LoRA pre-pass on the MFMA: tpart[z][m][r] = sum over the kLoraGroupsPerBlock groups
// of split z of x[m][k] * la[k][r] (la is K x R row-major). One workgroup of 4
// wavefronts per 16 x 16 tile of (rows, ranks) and split; each wavefront takes
// kLoraGroupsPerWave groups with all of its operands loaded before its first MFMA,
// and the four sums are added through LDS in wavefront order. The GEMM epilogues
// add the t_splits partials of T (lora_t_value), so T needs no reduction launch.
constexpr int kLoraGroupsPerWave = 8;
constexpr int kLoraGroupsPerBlock = 4 * kLoraGroupsPerWave;

__device__ __forceinline__ void lora_t_block(const float* __restrict__ x, const float* __restrict__ la,
                                             float* __restrict__ tpart, int M, int K, int R, int bx, int by,
                                             int bz) {
    __shared__ f32x4 red[4][64];
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int j = lane & 15;
    const int q = lane >> 4;
    const int G = K >> 5;
    const int m0 = bx * 16;
    const int r0 = by * 16;
    const int g_begin = bz * kLoraGroupsPerBlock + w * kLoraGroupsPerWave;
    const int row = min(m0 + j, M - 1);
    const int r = r0 + j;
    const int rc = min(r, R - 1);
    const float* xr = x + static_cast<size_t>(row) * K + 8 * q;

    f32x4 a_lo[kLoraGroupsPerWave], a_hi[kLoraGroupsPerWave];
    float b[kLoraGroupsPerWave][8];
#pragma unroll
    for (int i = 0; i < kLoraGroupsPerWave; ++i) {
        const int g = min(g_begin + i, G - 1);
        a_lo[i] = *reinterpret_cast<const f32x4*>(xr + g * 32);
        a_hi[i] = *reinterpret_cast<const f32x4*>(xr + g * 32 + 4);
        const float* lr = la + static_cast<size_t>(g * 32 + 8 * q) * R + rc;
#pragma unroll
        for (int t = 0; t < 8; ++t) b[i][t] = lr[static_cast<size_t>(t) * R];
    }
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < kLoraGroupsPerWave; ++i) {
        if (g_begin + i < G) {  // uniform per wavefront
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const float av = t < 4 ? a_lo[i][t & 3] : a_hi[i][t & 3];
                const float bv = r < R ? b[i][t] : 0.0f;
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc, 0, 0, 0);
            }
        }
    }
    red[w][lane] = acc;
    __syncthreads();
    if (w == 0) {
        f32x4 sum = red[0][lane];
#pragma unroll
        for (int v = 1; v < 4; ++v) sum += red[v][lane];
        float* dst = tpart + static_cast<size_t>(bz) * M * R;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int rr = m0 + 4 * q + i;
            if (rr < M && r < R) dst[static_cast<size_t>(rr) * R + r] = sum[i];
        }
    }
}

}  // namespace
}  // namespace spaceslug

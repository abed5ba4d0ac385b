// LoRA pre-pass and epilogue helpers shared by the int4 GEMM kernels (q4_gemm.hip,
// q4_small.hip). T = x * la, la row-major [K][R] (lora_delta.comp:2-21, lora.py:21-23),
// is computed as K-split partials that every GEMM epilogue sums itself.
#pragma once

#include "q4_device.hpp"
#include "q4_kernels.hpp"

namespace spaceslug {
namespace {

// NV values of T for a GEMM epilogue: value v is element e = e0 + stride * v of the row-major
// block [rows][nr] of T's ranks r_lo .. r_lo + nr - 1 whose first row is row0 (rows past M - 1
// clamped to it), the sum of its t_splits partials in double and in split order, rounded once;
// for e >= count it is a value the caller drops. The loads of kLoraTRound partials of all NV values issue before the first of their sums:
// the epilogue waits for one round of loads per kLoraTRound splits, not for one load after another.
constexpr int kLoraTRound = 8;
template <int NV>
__device__ __forceinline__ void lora_t_values(const float* __restrict__ tpart, int t_splits, int M, int R, int r_lo,
                                              int nr, int row0, int e0, int stride, int count, float (&out)[NV]) {
    size_t idx[NV];
    double t[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        const int e = min(e0 + stride * v, count - 1);
        idx[v] = static_cast<size_t>(min(row0 + e / nr, M - 1)) * R + r_lo + e % nr;
        t[v] = 0.0;
    }
    // Every load unconditional and in bounds (the row clamped, a split past the last one re-reading
    // the last): a load under a branch would be waited for where the branch joins.
    const size_t plane = static_cast<size_t>(M) * R;
    for (int z0 = 0; z0 < t_splits; z0 += kLoraTRound) {
        float p[kLoraTRound][NV];
#pragma unroll
        for (int dz = 0; dz < kLoraTRound; ++dz) {
            const size_t zo = static_cast<size_t>(min(z0 + dz, t_splits - 1)) * plane;
#pragma unroll
            for (int v = 0; v < NV; ++v) p[dz][v] = tpart[zo + idx[v]];
        }
#pragma unroll
        for (int dz = 0; dz < kLoraTRound; ++dz)
            if (z0 + dz < t_splits)
#pragma unroll
                for (int v = 0; v < NV; ++v) t[v] += static_cast<double>(p[dz][v]);
    }
#pragma unroll
    for (int v = 0; v < NV; ++v) out[v] = static_cast<float>(t[v]);
}

// LoRA pre-pass on the MFMA: tpart[z][m][r] = sum over the kLoraGroupsPerBlock groups
// of split z of x[m][k] * la[k][r] (la is K x R row-major). One workgroup of 4
// wavefronts per 16 x 16 tile of (rows, ranks) and split; each wavefront takes
// kLoraGroupsPerWave groups with all of its operands loaded before its first MFMA,
// and the four sums are added through LDS in wavefront order. The GEMM epilogues
// add the t_splits partials of T (lora_t_values), so T needs no reduction launch.
constexpr int kLoraGroupsPerWave = 4;
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

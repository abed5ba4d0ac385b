// fp32 GEMM behind spaceslug_sgemm (reference: vulkan-runtime/src/api/sgemm_api.cpp:37-63,
// shader sgemm.comp): C[M][N] = A[M][K] * B[K][N], row-major, M % 64 == 0,
// N % 64 == 0, K % 32 == 0. Exported because the reference's Python host binds
// it unconditionally (backend.py:65-67); the projection callers use it for the
// fp32 layers next to the int4 ones. Built on v_mfma_f32_16x16x4_f32 with the
// same lane mapping as the int4 kernel: a 64 x 64 workgroup tile of 2 x 2 waves,
// each wave 2 x 2 MFMA tiles; lane (j, q) takes k = 8q + t at step t of every
// 32-wide K chunk, reading 8 consecutive floats of its A row and the
// matching 8 rows of its B column. fp32 accumulation across K, as the
// reference's shader does.
#include "q4_device.hpp"
#include "q4_kernels.hpp"

namespace spaceslug {
namespace {

__global__ __launch_bounds__(256) void sgemm_mfma_kernel(const float* __restrict__ a,
                                                         const float* __restrict__ b,
                                                         float* __restrict__ c, int M, int N,
                                                         int K, int tiles_m) {
    constexpr int WM = 2, WN = 2;
    const int lane = threadIdx.x & 63;
    const int wid = threadIdx.x >> 6;
    const int j = lane & 15;
    const int q = lane >> 4;
    const int tile_m = blockIdx.x % tiles_m;
    const int tile_n = blockIdx.x / tiles_m;
    const int m0 = tile_m * 64 + (wid & 1) * 32;
    const int n0 = tile_n * 64 + (wid >> 1) * 32;

    f32x4 acc[WM][WN];
#pragma unroll
    for (int tm = 0; tm < WM; ++tm)
#pragma unroll
        for (int tn = 0; tn < WN; ++tn) acc[tm][tn] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    for (int kc = 0; kc < K; kc += 32) {
        float av[WM][8];
        float bv[WN][8];
#pragma unroll
        for (int tm = 0; tm < WM; ++tm) {
            const float* src = a + static_cast<size_t>(m0 + 16 * tm + j) * K + kc + 8 * q;
            const float4 lo = *reinterpret_cast<const float4*>(src);
            const float4 hi = *reinterpret_cast<const float4*>(src + 4);
            av[tm][0] = lo.x; av[tm][1] = lo.y; av[tm][2] = lo.z; av[tm][3] = lo.w;
            av[tm][4] = hi.x; av[tm][5] = hi.y; av[tm][6] = hi.z; av[tm][7] = hi.w;
        }
#pragma unroll
        for (int tn = 0; tn < WN; ++tn) {
            const float* src = b + static_cast<size_t>(kc + 8 * q) * N + n0 + 16 * tn + j;
#pragma unroll
            for (int t = 0; t < 8; ++t) bv[tn][t] = src[static_cast<size_t>(t) * N];
        }
#pragma unroll
        for (int t = 0; t < 8; ++t)
#pragma unroll
            for (int tm = 0; tm < WM; ++tm)
#pragma unroll
                for (int tn = 0; tn < WN; ++tn)
                    acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[tm][t], bv[tn][t], acc[tm][tn], 0, 0, 0);
    }
#pragma unroll
    for (int tm = 0; tm < WM; ++tm)
#pragma unroll
        for (int tn = 0; tn < WN; ++tn)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                c[static_cast<size_t>(m0 + 16 * tm + 4 * q + i) * N + n0 + 16 * tn + j] = acc[tm][tn][i];
}

}  // namespace

hipError_t launch_sgemm(const float* a, const float* b, float* c, uint32_t m, uint32_t n,
                        uint32_t k, hipStream_t stream) {
    const int tiles_m = static_cast<int>(m / 64);
    const int tiles_n = static_cast<int>(n / 64);
    hipLaunchKernelGGL(sgemm_mfma_kernel, dim3(tiles_m * tiles_n), dim3(256), 0, stream, a, b, c,
                       static_cast<int>(m), static_cast<int>(n), static_cast<int>(k), tiles_m);
    return hipGetLastError();
}

}  // namespace spaceslug
